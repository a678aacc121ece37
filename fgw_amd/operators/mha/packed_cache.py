"""Packed K/V cache: every request's live pages, contiguous, and attention over it.

The reference's packed-cache path (benchmarks/mha/external_cache_gather.py:
14-77) rounds each request's live region up to whole pages, copies those
pages in request order into a dense cache with a TileOPs paged-cache gather
(one call for K, one for V), checks the copy row-exactly, and runs its paged
attention over the dense cache through an identity page table. Here the copy
is one launch of fgw_mha_pack_pages (K and V together, whole pages, zero pages
for ids outside the pool) and the attention is build_kernel's.

pack_paged_cache is the format step on its own; build_gather_attention keeps
the reference helper's arguments and returns a (callable, info) pair, the
callable a GatherAttention that repacks and attends on every call.
"""
from __future__ import annotations

import ctypes
from collections import namedtuple
from typing import Sequence

import torch

from fgw_amd import _lib
from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import _current_stream

PackedCache = namedtuple("PackedCache", "k v table cu_rows offsets rows")


def packed_layout(lengths: Sequence[int], page_size: int, width: int):
    """(offsets, rows, table rows) of the packed cache (external_cache_gather.py:28-35):
    offsets[i + 1] - offsets[i] = ceil(len_i / page) * page; rows = max(page, total);
    table row i maps page j to offsets[i] // page + j."""
    offsets = [0]
    for n in lengths:
        offsets.append(offsets[-1] + -(-int(n) // page_size) * page_size)
    rows = max(page_size, offsets[-1])
    table = [[offsets[i] // page_size + j for j in range(width)] for i in range(len(lengths))]
    return offsets, rows, table


def _host_lengths(lengths, batch, capacity):
    if isinstance(lengths, torch.Tensor):
        if lengths.device.type != "cpu":
            raise ValueError("pack needs host-known lengths (a sequence or a CPU tensor)")
        lengths = lengths.tolist()
    lengths = [int(n) for n in lengths]
    if len(lengths) != batch:
        raise ValueError("metadata shape mismatch")
    if any(n < 0 or n > capacity for n in lengths):
        raise ValueError("Cache lengths must be within table capacity")
    return lengths


def _check_cache(k_cache, v_cache, block_table, page_size):
    if k_cache.ndim != 3 or v_cache.shape != k_cache.shape:
        raise ValueError("K/V shape mismatch")
    if k_cache.dtype not in (torch.float16, torch.bfloat16) or v_cache.dtype != k_cache.dtype:
        raise ValueError("matching FP16/BF16 Q/K/V required")
    if block_table.ndim != 2 or block_table.shape[1] <= 0 or block_table.dtype != torch.int32:
        raise ValueError("int32 metadata required")
    if page_size <= 0 or k_cache.shape[0] <= 0 or k_cache.shape[0] % page_size:
        raise ValueError("positive page size, whole pool pages and positive table width required")
    if k_cache.device.type != "cuda" or any(x.device != k_cache.device or not x.is_contiguous()
                                            for x in (k_cache, v_cache, block_table)):
        raise ValueError("contiguous inputs on the same GPU required")


def _upload_layout(offsets, table, device):
    """(cu_rows [B + 1], identity table [B, W]) on the device from one upload:
    a pinned staging copy of both, copied asynchronously on the current stream
    (pageable uploads would block the host until the stream drains)."""
    flat = offsets + [page for row in table for page in row]
    buf = torch.tensor(flat, dtype=torch.int32).pin_memory().to(device, non_blocking=True)
    b = len(offsets) - 1
    return buf[:b + 1], buf[b + 1:].view(b, -1)


def _launch_pack(k_cache, v_cache, block_table, cu_rows, total_pages, page_size, out_k, out_v):
    n, h, d = k_cache.shape
    b, w = block_table.shape
    shape = _lib.Shape(b, 1, h, d, n, w, page_size, 0,
                       _lib.DTYPE_BFLOAT16 if k_cache.dtype == torch.bfloat16
                       else _lib.DTYPE_FLOAT16)
    t = _lib.Tensors(None, k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
                     None, None, None, None)
    lib = _lib.load()
    _lib.check(lib.fgw_mha_pack_pages(ctypes.byref(shape), ctypes.byref(t), cu_rows.data_ptr(),
                                      total_pages, out_k.data_ptr(), out_v.data_ptr(),
                                      _current_stream(k_cache.device.index)))


class _PackPlan(namedtuple("_PackPlan", "offsets rows cu_rows table total_pages")):
    """Host offsets, packed rows and the device layout (row offsets, identity
    table) of one packing of a cache."""


def _plan_pack(lengths, page_size, width, device) -> _PackPlan:
    offsets, rows, table = packed_layout(lengths, page_size, width)
    cu_rows, dense_table = _upload_layout(offsets, table, device)
    return _PackPlan(offsets, rows, cu_rows, dense_table, offsets[-1] // page_size)


def _pack(k_cache, v_cache, block_table, plan: _PackPlan, page_size):
    """Dense K/V [rows, H, D] of one packing: one launch moves every live
    page; rows past the last packed page (only when every length is 0) are
    zero."""
    h, d = k_cache.shape[1:]
    out_k = torch.empty((plan.rows, h, d), dtype=k_cache.dtype, device=k_cache.device)
    out_v = torch.empty_like(out_k)
    live = plan.offsets[-1]
    if live < plan.rows:
        out_k[live:].zero_()
        out_v[live:].zero_()
    if plan.total_pages:
        _launch_pack(k_cache, v_cache, block_table, plan.cu_rows, plan.total_pages, page_size,
                     out_k, out_v)
    return out_k, out_v


def pack_paged_cache(k_cache, v_cache, block_table, lengths, page_size) -> PackedCache:
    """Copy every request's live pages, whole and in order, into a dense cache.

    `lengths` are host-known (a sequence or a CPU tensor), as in the
    reference helper, which computes the offsets on the host. Returns the
    dense K/V [rows, H, D], the identity page table [B, W] (int32, device),
    the row offsets (int32 [B + 1], device, and as a host list) and rows.
    Rows past the last packed page (only when every length is 0) are zero.
    """
    _check_cache(k_cache, v_cache, block_table, page_size)
    b, w = block_table.shape
    lengths = _host_lengths(lengths, b, w * page_size)
    plan = _plan_pack(lengths, page_size, w, k_cache.device)
    out_k, out_v = _pack(k_cache, v_cache, block_table, plan, page_size)
    return PackedCache(out_k, out_v, plan.table, plan.cu_rows, plan.offsets, plan.rows)


class GatherAttention:
    """Attention over a packed copy of the live cache, repacked on every call.

    Holds one packing plan (host offsets, device row offsets and identity
    table, computed once from host lengths) and the launch callable of the
    attention over the packed pool. A call allocates the dense K/V, packs
    them in one launch and runs the attention on the original Q with the
    identity table: the work the reference's packed-cache path times
    (benchmarks/mha/external_cache_gather.py:66-68). pack() alone returns
    the dense K/V of a call, for inspection.
    """

    def __init__(self, q, k, v, table, device_lengths, plan: _PackPlan, page_size, attention):
        self._inputs = (q, k, v, table, device_lengths)
        self._plan = plan
        self._page = page_size
        self.attention = attention
        self.packed_rows = plan.offsets[-1]
        self.rows = plan.rows

    def pack(self):
        _, k, v, table, _ = self._inputs
        return _pack(k, v, table, self._plan, self._page)

    def __call__(self):
        q, _, _, _, device_lengths = self._inputs
        dense_k, dense_v = self.pack()
        return self.attention(q, dense_k, dense_v, self._plan.table, device_lengths)


def check_packed_rows(k_cache, v_cache, block_table, plan: _PackPlan, page_size, dense_k,
                      dense_v) -> None:
    """Row-exact check of one packing (external_cache_gather.py:55-64): the
    packed rows of request i are the pool pages table[i, :ceil(len_i / page)]
    in order, bit for bit (NaN payloads included); a page id outside the pool
    packs as a zero page. Raises AssertionError naming the first request and
    tensor that differ. Runs on the device, outside any timed call."""
    pool_pages = k_cache.shape[0] // page_size
    h, d = k_cache.shape[1:]
    bits = torch.int16  # fp16 / bf16 compared as raw 16-bit patterns
    for name, original, packed in (("K", k_cache, dense_k), ("V", v_cache, dense_v)):
        pages = original.view(pool_pages, page_size, h, d)
        for i in range(len(plan.offsets) - 1):
            count = (plan.offsets[i + 1] - plan.offsets[i]) // page_size
            if not count:
                continue
            ids = block_table[i, :count].long()
            inside = (ids >= 0) & (ids < pool_pages)
            expected = pages[ids.clamp(0, pool_pages - 1)]
            expected = torch.where(inside.view(-1, 1, 1, 1), expected, torch.zeros_like(expected))
            got = packed[plan.offsets[i]:plan.offsets[i + 1]].view(count, page_size, h, d)
            if not torch.equal(got.view(bits), expected.view(bits)):
                raise AssertionError(f"packed {name} rows of request {i} differ from its pool pages")


def build_gather_attention(case, dtype_name, inputs, cube, splits, device_index, *, check=True):
    """Plan the packing and the attention over the packed cache.

    The arguments and the (callable, info) result are those of the reference
    helper (external_cache_gather.py:14, :70-77): case = (name, B, Sq, H, D,
    page, width, lengths, causal) with host lengths, inputs = (q, k, v, table,
    device lengths), cube = a module with build_kernel (for example
    fgw_amd.operators.mha.current). The callable is a GatherAttention. As in
    the reference helper, one packing is made and checked row-exactly against
    the pool pages before the callable is returned (check_packed_rows;
    info["gather_accuracy"] = "exact_passed"); check=False skips it
    ("unchecked").
    """
    _, b, sq, h, d, page, width, lengths, causal = case
    q, k, v, table, device_lengths = inputs
    _check_cache(k, v, table, page)
    lengths = _host_lengths(lengths, b, width * page)
    plan = _plan_pack(lengths, page, width, q.device)
    attention = cube.build_kernel(b, sq, h, d, plan.rows, width, page, causal, dtype_name,
                                  device_index, num_splits=splits)
    runner = GatherAttention(q, k, v, table, device_lengths, plan, page, attention)
    if check:
        dense_k, dense_v = runner.pack()
        check_packed_rows(k, v, table, plan, page, dense_k, dense_v)
    return runner, {
        "factory": "fgw_mha_pack_pages",
        "gather_accuracy": "exact_passed" if check else "unchecked",
        "gather_calls_per_attention": 1 if plan.total_pages else 0,
        "packed_rows": plan.offsets[-1], "live_rows": sum(lengths),
        "num_splits": attention.num_splits,
        "scope": "page-granular pack of K and V in one launch + build_kernel attention",
        "timed": "K/V allocation, one pack launch, all attention/split/merge kernels; "
                 "metadata prepared outside timing",
    }
