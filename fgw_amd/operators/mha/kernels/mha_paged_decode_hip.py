"""Paged multi-head attention on MI355X: the operators/mha public entry.

Same public contract as the reference operator
(operators/mha/kernels/mha_paged_decode_ascend_v7.py:516-570, original
contract mha_paged_decode_ascend_v0.py:98-126):

  Q [B, Sq, H, D], K/V pool [N, H, D], block table [B, W] int32,
  cache lengths [B] int32, page_size -> O [B, Sq, H, D] in Q's dtype.

One route serves every supported shape: FP16/BF16, D 16..256 in steps of 16,
any positive page size with whole pool pages, ragged and empty caches,
non-causal and right-aligned causal attention, Q from 1 upwards. The work is
done by hand-written CDNA4 kernels in libfgw_mha.so (fgw_amd/csrc), reached
through its C ABI; there is no other implementation to fall back to.

build_kernel returns a launch callable with the attributes of the reference
callable (v7.py:475-487, :500-512) and its component kernels
(direct_kernel, or partial_kernel + merge_kernel), so the reference harnesses'
component timing (bench_split_breakdown.py:79-96) applies unchanged.
"""
from __future__ import annotations

import ctypes
from functools import lru_cache

import torch

from fgw_amd import _lib
from fgw_amd.operators.mha import split_cost_model

ROUTE = "hip_mfma"
PERSISTENT_DEVICE = "device"  # cap the grid at the device's resident workgroups
SPLIT_POLICIES = ("auto", "legacy", "cost_model")
_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16}
_LAYOUTS = {None: _lib.LAYOUT_AUTO, "query": _lib.LAYOUT_QUERY, "key": _lib.LAYOUT_KEY,
            "prefill": _lib.LAYOUT_PREFILL}
_LAYOUT_NAMES = {_lib.LAYOUT_QUERY: "query", _lib.LAYOUT_KEY: "key", _lib.LAYOUT_PREFILL: "prefill"}


def _dtype_name(dtype) -> str:
    name = str(dtype).replace("torch.", "")
    if name not in _DTYPES:
        raise ValueError("matching FP16/BF16 Q/K/V required")
    return name


def route(dtype, dim, page_size, sq=1, causal=False):
    """The single kernel route (cf. v7.py:20-29); raises for unsupported specs."""
    name = str(dtype).replace("torch.", "")
    if name not in _DTYPES:
        raise ValueError("matching FP16/BF16 Q/K/V required")
    if dim < 16 or dim > 256 or dim % 16:
        raise ValueError("D must be in [16, 256] and divisible by 16")
    if page_size <= 0:
        raise ValueError("positive page size, whole pool pages and positive table width required")
    return ROUTE


@lru_cache(maxsize=8)
def _device_info(index: int) -> _lib.DeviceInfo:
    return _lib.query_device(index)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(index: int) -> int:
    """Raw handle of the current HIP stream of device `index`."""
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def _persistent_request(persistent_programs) -> int:
    if persistent_programs == PERSISTENT_DEVICE:
        return -1
    if persistent_programs is None:
        return 0
    if type(persistent_programs) is not int or persistent_programs < 1:
        raise ValueError("persistent_programs supports None (uncapped grid), 'device' or a positive int")
    return persistent_programs


_launch = _lib.load_launch_module()


class _Launch(_launch.Launcher):
    """Launch callable of one static specialisation; see build_kernel.

    A call (q, k_cache, v_cache, block_table, cache_seqlens) -> O runs in C++
    (fgw_amd._launch.Launcher, fgw_amd/csrc/launch_shim.cpp): the tensor
    checks with the messages of _check_detail, the output (and split
    workspace) allocation, and fgw_mha_fwd on the current stream.
    """

    def __init__(self, shape: _lib.Shape, plan: _lib.Plan, device_index: int, dtype: torch.dtype,
                 meta: dict):
        super().__init__(bytes(shape), bytes(plan), device_index,
                         _lib.entry_address("fgw_mha_fwd"), _lib.entry_address("fgw_mha_last_error"))
        self._shape = shape
        self._plan = plan
        self._device = torch.device("cuda", device_index)
        self._dtype = dtype
        self._out_shape = (shape.batch, shape.sq, shape.heads, shape.dim)
        self._kv_shape = (shape.pool_rows, shape.heads, shape.dim)
        self._meta_shapes = ((shape.batch, shape.width), (shape.batch,))
        self._index = device_index
        self._lib = _lib.load()
        self.block_q = plan.rows_per_tile
        self.compute_grid = plan.grid
        self.task_assignment = "contiguous"
        self.compute_work = plan.work_items
        self.persistent_programs = meta["persistent_programs"]
        self.requested_split_policy = meta["requested_split_policy"]
        self.split_policy = meta["split_policy"]
        self.num_splits = plan.num_splits
        # split_keys > 0: length-balanced splits in the key layout (request b
        # takes clamp(ceil(len_b / split_keys), 1, num_splits) of the slots),
        # tile-balanced causal splits in the prefill layout (query tile t takes
        # clamp(ceil(visible keys at capacity / split_keys), 1, num_splits));
        # 0 = every task num_splits.
        self.split_keys = plan.split_keys
        self.split_balance = ("tile" if plan.layout == _LAYOUTS["prefill"] else "length") \
            if plan.split_keys else "even"
        self.query_tile_tasks = plan.query_tile_tasks
        self.execution_mode = "split_and_merge" if plan.execution_mode else "direct_single_split"
        # True: a call merges the splits inside the partial kernel (the last
        # work item of each task merges it; one launch, with per-stream
        # arrival counters), except while its stream is captured into a
        # graph, where the merge is a second launch. The output bits are the
        # same either way; partial_kernel / merge_kernel stay separate.
        self.merge_fused = plan.arrival_counters > 0
        self.execution_path = ROUTE
        self.layout = _LAYOUT_NAMES[plan.layout]
        self.dim_padded = plan.dim_padded
        # K/V stages per key group of the selected kernel: 1 = the key layout's
        # single-stage kernel (two workgroups per CU), 2 = double-stage.
        self.stages = plan.stages
        # Q is read in place as [B, Sq, H, D]; no head-major copy is needed.
        self.prepare_q = lambda q: q
        if plan.execution_mode == 0:
            self.direct_kernel = self._direct
        else:
            self.partial_kernel = self._partial
            self.merge_kernel = self._merge

    # -- helpers -----------------------------------------------------------
    def _check(self, q, k, v, table, lengths):
        """Checks of the component calls (partial); the full call makes the
        same checks in C++."""
        self._check_detail(q, k, v, table, lengths)

    def _check_detail(self, q, k, v, table, lengths):
        if (tuple(q.shape) != self._out_shape or tuple(k.shape) != self._kv_shape
                or tuple(v.shape) != self._kv_shape or tuple(table.shape) != self._meta_shapes[0]
                or tuple(lengths.shape) != self._meta_shapes[1]):
            raise ValueError("tensor shapes do not match the built kernel")
        if q.dtype != self._dtype or k.dtype != self._dtype or v.dtype != self._dtype:
            raise ValueError("matching FP16/BF16 Q/K/V required")
        if table.dtype != torch.int32 or lengths.dtype != torch.int32:
            raise ValueError("int32 metadata required")
        for x in (q, k, v, table, lengths):
            if x.device != self._device or not x.is_contiguous():
                raise ValueError("contiguous inputs on the same GPU required")

    def _tensors(self, q, k, v, table, lengths, out=None, parts=None, lse=None):
        return _lib.Tensors(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                            lengths.data_ptr(), None if out is None else out.data_ptr(),
                            None if parts is None else parts.data_ptr(),
                            None if lse is None else lse.data_ptr())

    def _stream(self):
        return _current_stream(self._index)

    def _workspace(self):
        """Partials then LSE, carved from one allocation."""
        ws = torch.empty(self._plan.parts_floats + self._plan.lse_floats, dtype=torch.float32,
                         device=self._device)
        return ws[:self._plan.parts_floats], ws[self._plan.parts_floats:]

    # -- component calls -----------------------------------------------------
    def _direct(self, q, k, v, table, lengths):
        return self(q, k, v, table, lengths)

    def _partial(self, q, k, v, table, lengths):
        """Partials [B, H, S, Sq, D] (O/l) and LSE [B, H, S, Sq]."""
        self._check(q, k, v, table, lengths)
        parts, lse = self._workspace()
        t = self._tensors(q, k, v, table, lengths, None, parts, lse)
        _lib.check(self._lib.fgw_mha_partial(ctypes.byref(self._shape), ctypes.byref(self._plan),
                                             ctypes.byref(t), self._stream()))
        s = self._shape
        return (parts.view(s.batch, s.heads, self.num_splits, s.sq, s.dim),
                lse.view(s.batch, s.heads, self.num_splits, s.sq))

    def _merge(self, parts, lse, cache_seqlens=None):
        """Output from the partials. A length-balanced plan (key layout,
        split_keys > 0) merges request b's first clamp(ceil(len_b /
        split_keys), 1, S) slots and needs the call's cache_seqlens; a
        tile-balanced plan merges each query tile's own slot count."""
        s = self._shape
        if (parts.dtype != torch.float32 or lse.dtype != torch.float32
                or parts.numel() != self._plan.parts_floats or lse.numel() != self._plan.lse_floats
                or not parts.is_contiguous() or not lse.is_contiguous()
                or parts.device != self._device or lse.device != self._device):
            raise ValueError("merge expects this kernel's contiguous fp32 partials and LSE")
        if cache_seqlens is not None and (cache_seqlens.dtype != torch.int32
                                          or tuple(cache_seqlens.shape) != self._meta_shapes[1]
                                          or cache_seqlens.device != self._device
                                          or not cache_seqlens.is_contiguous()):
            raise ValueError("cache_seqlens must be this kernel's contiguous int32 [B] lengths on its GPU")
        if self.split_balance == "length" and cache_seqlens is None:
            raise ValueError("a length-balanced plan merges by cache_seqlens")
        out = torch.empty(self._out_shape, dtype=self._dtype, device=self._device)
        t = _lib.Tensors(None, None, None, None,
                         None if cache_seqlens is None else cache_seqlens.data_ptr(),
                         out.data_ptr(), parts.data_ptr(), lse.data_ptr())
        _lib.check(self._lib.fgw_mha_merge(ctypes.byref(s), ctypes.byref(self._plan),
                                           ctypes.byref(t), self._stream()))
        return out


@lru_cache(maxsize=128)
def _planned(batch, sq, heads, dim, pool_rows, width, page_size, causal, name, device_index,
             splits, persistent, layout, meta, split_keys=0, stages=0):
    """Launch callable of one (static shape, split request, grid request,
    layout): the unit the plan depends on. Ragged lengths reach the cost model
    before this cache, so a decode step with new lengths re-plans nothing
    unless the chosen split count changes."""
    device = _device_info(device_index)
    shape = _lib.Shape(batch, sq, heads, dim, pool_rows, width, page_size, int(bool(causal)),
                       _lib.DTYPE_BFLOAT16 if name == "bfloat16" else _lib.DTYPE_FLOAT16)
    plan = _lib.plan(shape, _lib.Request(splits, persistent, _LAYOUTS[layout], split_keys, stages),
                     device)
    return _Launch(shape, plan, device_index, _DTYPES[name], dict(meta))


def build_kernel(batch, sq, heads, dim, pool_rows, width, page_size, causal, dtype,
                 device_index=None, num_splits=None, split_policy="auto", full_kv_cache=False,
                 persistent_programs=PERSISTENT_DEVICE, cache_lengths=None, layout=None,
                 split_keys=None, stages=None):
    """Plan one static specialisation and return its launch callable.

    Arguments follow the reference build_kernel (v7.py:32-47) plus
    persistent_programs (v7_experimental.py:29-30: None = uncapped grid; here
    the default caps the grid at the device's resident workgroups),
    cache_lengths (host-known lengths for the cost model,
    cube_general.py:17, :45) and layout ("query" = 4 waves split 128 query
    rows; "prefill" = 8 waves split 256 query rows in two groups that
    alternate matrix and softmax phases, D in (32, 128]; "key" = waves split
    key blocks; None: key for Sq <= 32; for D in (32, 128] and Sq > 128,
    prefill when its 256-row tiles fill the device, from Sq 1024, or from
    2^24 query-key pairs; else query), split_keys (extra; with an explicit
    num_splits >= 2: in the key layout request b takes clamp(ceil(len_b /
    split_keys), 1, num_splits) splits, in the causal prefill layout query
    tile t takes clamp(ceil(its visible keys at capacity / split_keys), 1,
    num_splits); the automatic split chooses the first for ragged host-known
    decode lengths and the second for causal plans with few tiles of very
    different lengths) and stages (extra; K/V stages per key group: None =
    the planner's choice, 1 or 2 = the key layout's single- or double-stage
    kernel at head-dim tile 128). The reference caches build_kernel on its
    static arguments (lru_cache(128), v7.py:32); here the split count is
    chosen first (the cost model reads cache_lengths only under the
    auto/cost_model policy) and the plans are cached per (shape, split count,
    grid, layout, stages).
    """
    requested_split_policy = split_policy
    if split_policy not in SPLIT_POLICIES:
        raise ValueError("split_policy must be auto, legacy or cost_model")
    if num_splits is not None and (type(num_splits) is not int or num_splits < 1
                                   or num_splits & (num_splits - 1) or num_splits > 128):
        raise ValueError("num_splits supports None (automatic) or 1/2/4/8/16/32/64/128")
    name = _dtype_name(dtype)
    route(name, dim, page_size, sq, causal)
    if page_size <= 0 or pool_rows <= 0 or pool_rows % page_size or width <= 0:
        raise ValueError("positive page size, whole pool pages and positive table width required")
    if min(batch, sq, heads) <= 0:
        raise ValueError("positive Q extents and rank-2 table required")
    if device_index is None:
        device_index = torch.cuda.current_device()
    device_index = int(device_index)
    persistent = _persistent_request(persistent_programs)
    if layout not in _LAYOUTS:
        raise ValueError("layout must be None, 'query', 'key' or 'prefill'")
    if stages is not None and stages not in (1, 2, 4):
        raise ValueError("stages supports None (the default kernel), 1 or 2 (key layout, "
                         "head-dim tile 128) or the kernel's own count")

    if split_keys is not None and (type(split_keys) is not int or split_keys < 1
                                   or num_splits is None or num_splits < 2):
        raise ValueError("split_keys needs a positive int and an explicit num_splits >= 2")
    if num_splits is not None:
        split_keys = split_keys or 0
        splits, policy = num_splits, "explicit"
    else:
        if split_policy == "auto":
            device = _device_info(device_index)
            use_model = layout is None and split_cost_model.eligible_config(
                batch, sq, heads, dim, width * page_size, page_size=page_size, causal=causal,
                full_kv_cache=full_kv_cache, num_cus=device.num_cus,
                lengths_known=cache_lengths is not None,
                wg_per_cu=split_cost_model.occupancy(device))
            split_policy = "cost_model" if use_model else "legacy"
        split_keys = 0
        if split_policy == "cost_model":
            lengths = cache_lengths
            if lengths is None:
                if not full_kv_cache:
                    raise ValueError("Cost model requires full_kv_cache or host-known cache_lengths")
                lengths = (width * page_size,) * batch
            splits = split_cost_model.select_splits(batch, sq, heads, dim, width * page_size,
                                                    tuple(lengths), _device_info(device_index))
            if cache_lengths is not None and layout is None and sq <= 32:
                # Ragged lengths: the same number of work items, balanced by length.
                balanced = split_cost_model.balanced_split_keys(tuple(lengths), splits,
                                                                width * page_size)
                if balanced is not None:
                    splits, split_keys = balanced
            if not split_keys and stages is None and layout in (None, "key"):
                # The planner's automatic move to the single-stage key kernel,
                # applied to the model's split count (the single-stage kernel
                # exists in the key layout only).
                device = _device_info(device_index)
                up = split_cost_model.single_stage_splits(
                    batch, sq, heads, dim, width * page_size, splits, device.num_cus,
                    device.wg_per_cu_key_single)
                if up:
                    splits, stages = up, 1
        else:
            splits = 0
        policy = split_policy
    meta = (("persistent_programs", persistent_programs),
            ("requested_split_policy", requested_split_policy), ("split_policy", policy))
    return _planned(batch, sq, heads, dim, pool_rows, width, page_size, bool(causal), name,
                    device_index, splits, persistent, layout, meta, split_keys, stages or 0)


def mha_paged_decode(q, k_cache, v_cache, block_table, cache_seqlens, page_size, is_causal=False,
                     *, num_splits=None, split_policy="auto", persistent_programs=PERSISTENT_DEVICE):
    """Paged attention forward; same tensor contract and checks as v7.py:516-570.

    The cache lengths are copied to the host once to check
    0 <= len <= W * page_size (the reference general route's check,
    v7_experimental.py:870-873) and to detect a full cache for the split policy.
    """
    if q.ndim != 4 or k_cache.ndim != 3:
        raise ValueError("expected Q[B,Sq,H,D], K/V[N,H,D]")
    b, sq, h, d = q.shape
    if min(b, sq, h, d) <= 0 or block_table.ndim != 2:
        raise ValueError("positive Q extents and rank-2 table required")
    if k_cache.shape[1:] != (h, d) or v_cache.shape != k_cache.shape:
        raise ValueError("K/V shape mismatch")
    if block_table.shape[0] != b or block_table.shape[1] <= 0 or cache_seqlens.shape != (b,):
        raise ValueError("metadata shape mismatch")
    if q.dtype not in (torch.float16, torch.bfloat16) or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError("matching FP16/BF16 Q/K/V required")
    if block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32:
        raise ValueError("int32 metadata required")
    inputs = (q, k_cache, v_cache, block_table, cache_seqlens)
    if q.device.type != "cuda" or any(x.device != q.device or not x.is_contiguous() for x in inputs):
        raise ValueError("contiguous inputs on the same GPU required")
    capacity = block_table.shape[1] * page_size
    lengths = cache_seqlens.cpu().tolist()
    if any(n < 0 or n > capacity for n in lengths):
        raise ValueError("Cache lengths must be within table capacity")
    full_kv_cache = all(n == capacity for n in lengths)
    with torch.cuda.device(q.device):
        kernel = build_kernel(b, sq, h, d, k_cache.shape[0], block_table.shape[1], page_size,
                              bool(is_causal), "float16" if q.dtype == torch.float16 else "bfloat16",
                              q.device.index, num_splits=num_splits, split_policy=split_policy,
                              full_kv_cache=full_kv_cache, persistent_programs=persistent_programs,
                              cache_lengths=planning_lengths(lengths, full_kv_cache, num_splits,
                                                             split_policy, is_causal))
        return kernel(*inputs)


def planning_lengths(lengths, full_kv_cache, num_splits, split_policy, is_causal):
    """The host lengths mha_paged_decode hands to build_kernel, or None.

    Ragged lengths matter only to the cost model: an explicit cost_model
    request always receives them (v7_experimental.py:885-886, causal or not);
    under 'auto' only non-causal calls, the ones the model's calibrated scope
    admits, plan with them. Full caches and explicit split counts plan without
    them."""
    wants = (not full_kv_cache and num_splits is None
             and (split_policy == "cost_model" or (split_policy == "auto" and not is_causal)))
    return tuple(lengths) if wants else None
