"""CPU oracle for the paged MHA operator -- TEST INFRASTRUCTURE ONLY.

This module restates, in torch fp32 on the CPU, the reference operator's own
CPU path and input recipes (zhangwenhao91/FGW). It is the checker of the HIP
kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import it, and never as the thing measured or shipped. The product path
(fgw_amd.operators.mha) never calls into this module and fails loudly when its
HIP library is missing.

Functions and the reference lines they follow:
  physical_rows        operators/mha/kernels/mha_paged_decode_ascend_v0.py:137
  reference            operators/mha/kernels/mha_paged_decode_ascend_v0.py:129-144
  chunked_reference    benchmarks/mha/bench_mha_mfu.py:38-60
  rounded_reference    the reference kernel's rounding points: softmax in fp32 against the
                       row maximum, row sum of the fp32 probabilities, P cast to the input
                       dtype for PV (mha_paged_decode_ascend_v7.py:120-192, the vcvt at
                       :159-162), O / l cast (:455-465)
  merge_partials       operators/mha/kernels/mha_paged_decode_ascend_v7.py:352-370
  partial_states       v7.py:305-315 (O/l, LSE = ln l + m; -1e30 when empty), over
                       the block partition of this build's kernel
  visible_keys         cube_general.py:121-126 / test_mha_paged_accuracy.py:270-272
  useful_flops         benchmarks/mha/bench_mha_mfu.py:63-66
  algorithmic_bytes    byte model of the decode roofline (live K+V, Q, O, table, lengths)
  lengths_for          tests/mha/test_mha_paged_accuracy.py:73-83
  make_inputs          tests/mha/test_mha_paged_accuracy.py:86-101
  poison_unread        tests/mha/test_mha_paged_accuracy.py:232-238
  bench_inputs         benchmarks/mha/bench_mha_mfu.py:179-188
  gather_packed        benchmarks/mha/external_cache_gather.py:55-64 (row-exact packing)
  packed_offsets       benchmarks/mha/external_cache_gather.py:28-35 (page-rounded offsets,
                       identity page table)
  pack_pages           benchmarks/mha/external_cache_gather.py:55-64 (whole-page copy)
  page_div             Granlund-Montgomery division used by the kernels' page lookup

Pinning (tests/test_oracle.py): the report vectors the reference recorded
(tests/golden/accuracy_report_vectors.json) pin lengths_for/make_inputs; a
float64 brute-force softmax attention and closed forms (single key, equal
keys, empty rows) pin reference/chunked_reference; the reference's raw
partition-merge vectors (tests/mha/test_raw_partial_state.py) and a dense
comparison pin merge_partials/partial_states; its equality with reference for
float32 inputs (where the cast is exact) and a two-key closed form of the
rounded P pin rounded_reference; the published FLOP/byte counts
pin useful_flops/algorithmic_bytes; exhaustive integer checks pin page_div;
row-by-row resolution through physical_rows (live rows) and the original
pages (page tails), plus closed forms of the offsets, pin packed_offsets and
pack_pages.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import torch

TOLERANCES = {  # test_mha_paged_accuracy.py:264
    torch.bfloat16: (1e-2, 4e-3),
    torch.float16: (2e-3, 2e-3),
}


def physical_rows(table: torch.Tensor, b: int, length: int, page_size: int) -> torch.Tensor:
    """Pool rows of positions 0..length-1 of request b (v0.py:137)."""
    pos = torch.arange(int(length))
    return table[b, pos // page_size].long() * page_size + pos % page_size


def visible_keys(length: int, sq: int, qi: int, causal: bool) -> int:
    """Keys query row qi of a request with `length` cached keys attends to."""
    return max(length - sq + qi + 1, 0) if causal else length


def reference(q, k, v, table, lengths, page_size, causal):
    """CPU fp32 attention over each request's live cache (v0.py:129-144)."""
    q, k, v, table, lengths = [x.cpu() for x in (q, k, v, table, lengths)]
    b, sq, h, d = q.shape
    out = torch.zeros_like(q)
    for bi in range(b):
        length = int(lengths[bi])
        physical = physical_rows(table, bi, length, page_size)
        kk, vv = k[physical].float(), v[physical].float()
        for qi in range(sq):
            end = visible_keys(length, sq, qi, causal)
            if end:
                scores = torch.einsum("hd,thd->ht", q[bi, qi].float(), kk[:end]) * d ** -0.5
                out[bi, qi] = torch.einsum("ht,thd->hd", scores.softmax(-1), vv[:end]).to(q.dtype)
    return out


def chunked_reference(q, k, v, table, lengths, page_size, causal, chunk=128):
    """fp32 CPU attention with a bounded score workspace (bench_mha_mfu.py:38-60)."""
    q, k, v, table, lengths = [x.cpu() for x in (q, k, v, table, lengths)]
    batch, sq, heads, dim = q.shape
    output = torch.zeros_like(q)
    for b in range(batch):
        length = int(lengths[b])
        if length == 0:
            continue
        pos = torch.arange(length)
        rows = physical_rows(table, b, length, page_size)
        kk, vv = k[rows].float().transpose(0, 1), v[rows].float().transpose(0, 1)
        for start in range(0, sq, chunk):
            stop = min(start + chunk, sq)
            query = q[b, start:stop].float().transpose(0, 1)
            scores = (query @ kk.transpose(-1, -2)) * dim ** -0.5
            if causal:
                visible = pos[None, :] <= (torch.arange(start, stop)[:, None] + length - sq)
                scores.masked_fill_(~visible[None, :, :], float("-inf"))
            probabilities = scores.softmax(-1).nan_to_num(0.0)
            output[b, start:stop] = (probabilities @ vv).transpose(0, 1).to(q.dtype)
    return output


def rounded_reference(q, k, v, table, lengths, page_size, causal):
    """CPU attention with the rounding points of the reference kernel
    (v7.py:120-192, :455-465): scores and the softmax against the row maximum
    in fp32, the row sum of the fp32 probabilities, P cast to the input dtype
    for the PV product (the vcvt at v7.py:159-162), PV in fp32, O / l cast to
    the input dtype; rows with no visible key are zero. Its error against
    `reference` is the error any kernel with these rounding points makes."""
    q, k, v, table, lengths = [x.cpu() for x in (q, k, v, table, lengths)]
    b, sq, h, d = q.shape
    out = torch.zeros_like(q)
    scale = d ** -0.5
    for bi in range(b):
        n = int(lengths[bi])
        if n == 0:
            continue
        rows = physical_rows(table, bi, n, page_size)
        kk, vv = k[rows].float(), v[rows].float()
        vis = torch.tensor([visible_keys(n, sq, qi, causal) for qi in range(sq)])
        for hi in range(h):
            s_ = (q[bi, :, hi].float() @ kk[:, hi].T) * scale
            s_ = s_.masked_fill(torch.arange(n)[None, :] >= vis[:, None], float("-inf"))
            m = s_.max(dim=1, keepdim=True).values.clamp_min(-1e30)
            p = torch.exp(s_ - m)
            l_ = p.sum(dim=1, keepdim=True)
            o = p.to(q.dtype).float() @ vv[:, hi]
            res = torch.where(l_ > 0, o / l_.clamp_min(1e-30), torch.zeros_like(o))
            out[bi, :, hi] = res.to(q.dtype)
    return out


def split_ranges(n_blocks: int, splits: int) -> List[Tuple[int, int]]:
    """Floor partition of n_blocks key blocks over splits (cube_general.py:88-90)."""
    return [(n_blocks * s // splits, n_blocks * (s + 1) // splits) for s in range(splits)]


def partial_states(q, k, v, table, lengths, page_size, causal, splits, block_keys, rows_per_tile):
    """fp32 per-split partials: parts[b,h,s,q,:] = O_s / l_s, lse[b,h,s,q] = ln l_s + m_s.

    The key range of a query tile [q0, q0 + rows_per_tile) is
    [0, max visible key of the tile), cut into block_keys-key blocks that are
    floor-partitioned over the splits. Keys a row cannot see are masked.
    Empty splits give parts 0 and lse -1e30 (v7.py:305-312).
    """
    q, k, v, table, lengths = [x.cpu() for x in (q, k, v, table, lengths)]
    batch, sq, heads, dim = q.shape
    parts = torch.zeros(batch, heads, splits, sq, dim)
    lse = torch.full((batch, heads, splits, sq), -1e30)
    for b in range(batch):
        length = int(lengths[b])
        rows = physical_rows(table, b, length, page_size)
        kk, vv = k[rows].float(), v[rows].float()
        for q0 in range(0, sq, rows_per_tile):
            last = min(q0 + rows_per_tile, sq) - 1
            tile_end = min(max(visible_keys(length, sq, last, causal), 0), length)
            n_blocks = -(-tile_end // block_keys)
            for s, (b0, b1) in enumerate(split_ranges(n_blocks, splits)):
                lo, hi = b0 * block_keys, min(b1 * block_keys, tile_end)
                for qi in range(q0, last + 1):
                    end = min(visible_keys(length, sq, qi, causal), hi)
                    if end <= lo:
                        continue
                    scores = torch.einsum("hd,thd->ht", q[b, qi].float(), kk[lo:end]) * dim ** -0.5
                    m = scores.max(-1, keepdim=True).values
                    p = (scores - m).exp()
                    total = p.sum(-1, keepdim=True)
                    parts[b, :, s, qi] = torch.einsum("ht,thd->hd", p, vv[lo:end]) / total
                    lse[b, :, s, qi] = (total.log() + m).squeeze(-1)
    return parts, lse


def merge_partials(parts: torch.Tensor, lse: torch.Tensor, dtype) -> torch.Tensor:
    """LSE merge over the split axis (v7.py:352-370), online form.

    parts [B, H, S, Sq, D], lse [B, H, S, Sq] -> out [B, Sq, H, D] in dtype.
    """
    parts, lse = parts.float(), lse.float()
    batch, heads, splits, sq, dim = parts.shape
    acc = torch.zeros(batch, heads, sq, dim)
    maximum = torch.full((batch, heads, sq), -1e30)
    total = torch.zeros(batch, heads, sq)
    for s in range(splits):
        score = lse[:, :, s]
        peak = torch.maximum(maximum, score)
        old = torch.exp(maximum - peak)
        new = torch.where(score > -1e29, torch.exp(score - peak), torch.zeros_like(score))
        acc = acc * old[..., None] + parts[:, :, s] * new[..., None]
        total = total * old + new
        maximum = peak
    out = acc / torch.clamp(total, min=1e-30)[..., None]
    return out.permute(0, 2, 1, 3).contiguous().to(dtype)


def useful_flops(lengths: Sequence[int], sq: int, heads: int, dim: int, causal: bool) -> int:
    """4*H*D*sum of visible (q, k) pairs (bench_mha_mfu.py:63-66)."""
    pairs = sum(visible_keys(int(n), sq, qi, causal) for n in lengths for qi in range(sq))
    return 4 * heads * dim * pairs


def algorithmic_bytes(lengths: Sequence[int], sq: int, heads: int, dim: int, width: int,
                      elem_bytes: int = 2) -> int:
    """Live K+V + Q + O + table + lengths, no page-tail over-read."""
    batch = len(lengths)
    return (2 * heads * dim * elem_bytes * sum(int(n) for n in lengths)
            + 2 * batch * sq * heads * dim * elem_bytes + 4 * batch * width + 4 * batch)


def lengths_for(case, pattern: str, seed: int) -> List[int]:
    """Length patterns of the accuracy suites (test_mha_paged_accuracy.py:73-83)."""
    _, b, sq, _, _, p, w = case
    capacity = p * w
    if pattern == "empty":
        return [0] * b
    if pattern == "full":
        return [capacity] * b
    choices = [0, 1, max(0, sq - 1), sq, p - 1, p, p + 1, capacity - 1, capacity]
    return [min(capacity, choices[(i + seed) % len(choices)]) for i in range(b)]


def make_inputs(case, seed: int, dtype):
    """Seeded Q/K/V and a table with a shared and a repeated page (:86-101)."""
    _, b, sq, h, d, p, w = case
    generator = torch.Generator().manual_seed(seed)
    pool_pages = max(w + 3, b * w + 1)
    table = torch.stack([torch.randperm(pool_pages - 1, generator=generator)[:w]
                         for _ in range(b)]).to(torch.int32)
    if b > 1:
        table[1:, 0] = table[0, 0]
    if w > 1:
        table[-1, -1] = table[-1, 0]
    q = torch.randn(b, sq, h, d, generator=generator).to(dtype)
    k = torch.randn(pool_pages * p, h, d, generator=generator).to(dtype)
    v = torch.randn(pool_pages * p, h, d, generator=generator).to(dtype)
    return q, k, v, table


def poison_unread(k, v, table, lengths, page_size):
    """NaN in every pool row no request reads (:232-238)."""
    live = torch.zeros(k.shape[0], dtype=torch.bool)
    for bi in range(table.shape[0]):
        live[physical_rows(table, bi, int(lengths[bi]), page_size)] = True
    k, v = k.clone(), v.clone()
    k[~live], v[~live] = float("nan"), float("nan")
    return k, v


def bench_inputs(b, sq, h, d, page_size, length, dtype, seed=7):
    """Benchmark recipe: per-request shuffled pages, full cache (:179-188)."""
    width = (length + page_size - 1) // page_size
    generator = torch.Generator().manual_seed(seed)
    table = torch.randperm(b * width, generator=generator).reshape(b, width).to(torch.int32)
    lengths = torch.full((b,), length, dtype=torch.int32)
    q = torch.randn(b, sq, h, d, generator=generator).to(dtype)
    k = torch.randn(b * width * page_size, h, d, generator=generator).to(dtype)
    v = torch.randn(b * width * page_size, h, d, generator=generator).to(dtype)
    return q, k, v, table, lengths


def imbalanced_lengths(length, batch=4, seed=7):
    """Benchmark config 4's imbalanced decode variant: per-request lengths drawn
    uniformly in [length / 8, length] from Generator().manual_seed(seed) (one
    randint draw, int32); the table width stays length / page."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(length // 8, length + 1, (batch,), generator=g).to(torch.int32)


def gather_packed(k, v, table, lengths, page_size, out_len):
    """Packed [B, out_len, H, D] copies of each request's live rows, zero past len."""
    b = table.shape[0]
    ok = torch.zeros((b, out_len) + tuple(k.shape[1:]), dtype=k.dtype)
    ov = torch.zeros_like(ok)
    for bi in range(b):
        n = min(int(lengths[bi]), out_len)
        rows = physical_rows(table, bi, n, page_size)
        ok[bi, :n] = k[rows]
        ov[bi, :n] = v[rows]
    return ok, ov


def packed_offsets(lengths: Sequence[int], page_size: int, width: int):
    """Row offsets of the packed cache and its page table
    (external_cache_gather.py:28-35): request i's live region rounded up to
    whole pages, in request order; rows = max(page, total); table row i maps
    page j to offsets[i] // page + j."""
    offsets = [0]
    for n in lengths:
        offsets.append(offsets[-1] + (int(n) + page_size - 1) // page_size * page_size)
    rows = max(page_size, offsets[-1])
    table = torch.tensor([[offsets[i] // page_size + j for j in range(width)]
                          for i in range(len(lengths))], dtype=torch.int32)
    return offsets, rows, table


def pack_pages(k, v, table, lengths, page_size):
    """Packed K/V [rows, H, D]: request i's pages table[i, :ceil(len_i / page)]
    copied whole (rows past len included) to rows [offsets[i], offsets[i + 1])
    (the expected rows of external_cache_gather.py:55-64); rows past the total
    are zero."""
    lengths = [int(n) for n in lengths]
    offsets, rows, _ = packed_offsets(lengths, page_size, table.shape[1])
    h, d = k.shape[1:]
    ok = torch.zeros((rows, h, d), dtype=k.dtype)
    ov = torch.zeros_like(ok)
    for i, n in enumerate(lengths):
        count = (n + page_size - 1) // page_size
        if count:
            ids = table[i, :count].long()
            ok[offsets[i]:offsets[i + 1]] = k.view(-1, page_size, h, d)[ids].reshape(-1, h, d)
            ov[offsets[i]:offsets[i + 1]] = v.view(-1, page_size, h, d)[ids].reshape(-1, h, d)
    return ok, ov, offsets


def page_divisor(page: int) -> Tuple[int, int]:
    """(magic, shift) of the kernels' division by page (Granlund-Montgomery 1994)."""
    if page <= 1:
        return 0, 0
    shift = (page - 1).bit_length()
    magic = ((1 << 32) * ((1 << shift) - page)) // page + 1
    return magic & 0xFFFFFFFF, shift


def page_div(n: int, magic: int, shift: int) -> int:
    """32-bit restatement of the device quotient n // page."""
    if shift == 0:
        return n
    t = (magic * n) >> 32
    return (t + ((n - t) >> 1)) >> (shift - 1)
