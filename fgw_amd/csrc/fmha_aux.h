// Split-KV LSE merge and the stand-alone paged K/V gather.
#pragma once
#include "fmha_kernel.h"

namespace fgw_mha {

// LSE merge of the split partials of output rows [q0, q0 + rows) of (b, h),
// one (row, 4 dims) pair per thread:
//   peak = max over splits with LSE > -1e29,
//   w_s  = LSE_s > -1e29 ? exp(LSE_s - peak) : 0,
//   O    = sum_s w_s * Part_s / max(sum_s w_s, 1e-30), cast to the input dtype.
// This is the reference merge (v7.py:352-370, cube_general.py:259-278):
// splits are taken in chunks of kMergeChunk whose loads are all issued before
// any is used (one memory round trip per chunk), and the running peak moves
// once per chunk. Empty splits (LSE -1e30) carry zero weight and an
// all-empty row is exactly zero.
constexpr int kMergeChunk = 16;
// One (row, 4 dims): split s's LSE at ls[s * lse_stride], its part at
// ps[s * part_stride]; the result goes to dst in the input dtype. Chunks of
// CH splits; the loads of a chunk's missing splits past `splits` are
// clamped to the last split and carry weight 0.
template <bool BF16, int CH>
__device__ __forceinline__ void merge_one_chunked(const float* ls, int64_t lse_stride,
                                                  const float* ps, int64_t part_stride,
                                                  int splits, u16* dst) {
  using E = Elem<BF16>;
  float peak = kNegBig, tot = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < splits; s0 += CH) {
    float x[CH];
    f32x4 v[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int s = s0 + i < splits ? s0 + i : splits - 1;  // clamped; weight 0 below
      x[i] = ls[(int64_t)s * lse_stride];
      v[i] = *reinterpret_cast<const f32x4*>(ps + (int64_t)s * part_stride);
    }
    float cpeak = peak;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const bool live = s0 + i < splits && x[i] > -1.0e29f;
      cpeak = live ? fmaxf(cpeak, x[i]) : cpeak;
    }
    const float keep = expf(peak - cpeak);  // 0 while nothing was live, 1 if unchanged
    tot *= keep;
    acc *= keep;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const bool live = s0 + i < splits && x[i] > -1.0e29f;
      const float wgt = live ? expf(x[i] - cpeak) : 0.0f;
      tot += wgt;
      acc += live ? v[i] * wgt : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    peak = cpeak;
  }
  const float inv = 1.0f / fmaxf(tot, 1.0e-30f);
  u32x2 w;
  w.x = E::pack2(acc[0] * inv, acc[1] * inv);
  w.y = E::pack2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2*>(dst) = w;
}

// merge_one_chunked with the smallest chunk of 2, 4, 8 or 16 that holds all
// `splits` (one chunk up to 16): a chunk of 16 for 2 splits would issue
// eight times the loads (the clamped ones), which the prefill-length merges
// of few splits feel. The live splits are summed in the same order whatever
// the chunk (a larger chunk only adds zeros for its dead splits).
template <bool BF16>
__device__ __forceinline__ void merge_one(const float* ls, int64_t lse_stride, const float* ps,
                                          int64_t part_stride, int splits, u16* dst) {
  if (splits <= 2)
    merge_one_chunked<BF16, 2>(ls, lse_stride, ps, part_stride, splits, dst);
  else if (splits <= 4)
    merge_one_chunked<BF16, 4>(ls, lse_stride, ps, part_stride, splits, dst);
  else if (splits <= 8)
    merge_one_chunked<BF16, 8>(ls, lse_stride, ps, part_stride, splits, dst);
  else
    merge_one_chunked<BF16, kMergeChunk>(ls, lse_stride, ps, part_stride, splits, dst);
}

// Splits row (b, ., q) of a merge reads: all slots, the balanced count of
// request b (balanced_splits over its clamped length), or the slots of q's
// query tile in a tile-balanced causal plan.
__device__ __forceinline__ int merge_splits(const MergeParams& p, int b, int q) {
  if (p.split_keys <= 0) return p.splits;
  if (p.rows_tile > 0)
    return tile_slots(q / p.rows_tile, p.sq, p.capacity, p.rows_tile, p.split_keys, p.splits);
  int len = p.lengths[b];
  len = len < 0 ? 0 : (len > p.capacity ? p.capacity : len);
  return balanced_splits(len, p.split_keys, p.splits);
}

// Rows [q0, q0 + rows) of (b, h): `slots` is the workspace's split dimension,
// the first `used` slots are merged.
template <bool BF16>
__device__ __forceinline__ void merge_rows(const float* parts, const float* lse, void* out, int sq,
                                           int heads, int dim, int slots, int used, int b, int h,
                                           int q0, int rows, int tid, int nthreads) {
  const int d4n = dim / 4;
  const int64_t bhs = ((int64_t)b * heads + h) * slots;
  for (int idx = tid; idx < rows * d4n; idx += nthreads) {
    const int q = q0 + idx / d4n, d0 = 4 * (idx % d4n);
    u16* dst = static_cast<u16*>(out) + (((int64_t)b * sq + q) * heads + h) * dim + d0;
    merge_one<BF16>(lse + bhs * sq + q, sq, parts + (bhs * sq + q) * dim + d0,
                    (int64_t)sq * dim, used, dst);
  }
}

// Stand-alone LSE merge: one workgroup per (b, h, group of rows_per_wg rows).
constexpr int kMergeThreads = 256;
template <bool BF16>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(MergeParams p, int rows_per_wg) {
  const int groups = (p.sq + rows_per_wg - 1) / rows_per_wg;
  const int g = blockIdx.x % groups;
  const int bh = blockIdx.x / groups;
  const int q0 = g * rows_per_wg;
  const int rows = p.sq - q0 < rows_per_wg ? p.sq - q0 : rows_per_wg;
  const int b = bh / p.heads;
  const int used = merge_splits(p, b, q0);
  if (p.skip_single && used == 1) return;  // written by the forward kernel
  merge_rows<BF16>(p.parts, p.lse, p.out, p.sq, p.heads, p.dim, p.splits, used, b,
                   bh % p.heads, q0, rows, threadIdx.x, kMergeThreads);
}

// LSE merge of one output row (b, h, q) per workgroup with the splits spread
// over the threads, for split counts above kMergeChunk (where merge_one
// would take one memory round trip per chunk). Thread (g, c), g < G =
// kMergeThreads / (D / 4), takes dims 4c .. 4c + 3 of splits g, g + G, ...
// and folds them as merge_one does (running peak per chunk of kMergeChunk,
// weights exp(LSE - peak), empty splits weight 0) without normalising; the
// G group states are then rescaled to the common peak and summed in group
// order through LDS, and O = acc / max(tot, 1e-30) is cast to the input
// dtype. An all-empty row is exactly zero.
// Group g's splits g, g + G, ... of a wide merge row (see merge_wide_kernel)
// in chunks of CH whose loads are all issued before any is used; the running
// peak moves once per chunk. Missing splits past `used` load split g again
// and carry weight 0.
template <int CH>
__device__ __forceinline__ void wide_group(const float* ls, const float* ps, int64_t lse_stride,
                                           int64_t part_stride, int g, int G, int used,
                                           float& peak, float& tot, f32x4& acc) {
  for (int s0 = g; s0 < used; s0 += CH * G) {
    float x[CH];
    f32x4 v[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int s = s0 + i * G < used ? s0 + i * G : g;  // clamped; weight 0 below
      x[i] = ls[(int64_t)s * lse_stride];
      v[i] = *reinterpret_cast<const f32x4*>(ps + (int64_t)s * part_stride);
    }
    float cpeak = peak;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const bool live = s0 + i * G < used && x[i] > -1.0e29f;
      cpeak = live ? fmaxf(cpeak, x[i]) : cpeak;
    }
    const float keep = expf(peak - cpeak);
    tot *= keep;
    acc *= keep;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const bool live = s0 + i * G < used && x[i] > -1.0e29f;
      const float wgt = live ? expf(x[i] - cpeak) : 0.0f;
      tot += wgt;
      acc += live ? v[i] * wgt : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    peak = cpeak;
  }
}

template <bool BF16>
__global__ __launch_bounds__(kMergeThreads) void merge_wide_kernel(MergeParams p) {
  using E = Elem<BF16>;
  __shared__ float speak[kMergeThreads];
  __shared__ float stot[kMergeThreads];
  __shared__ f32x4 sacc[kMergeThreads];
  const int d4n = p.dim / 4;
  const int G = kMergeThreads / d4n;
  const int t = threadIdx.x, c = t % d4n, g = t / d4n;
  const bool act = g < G;
  const int q = (int)(blockIdx.x % (unsigned)p.sq);
  const int bh = (int)(blockIdx.x / (unsigned)p.sq);
  const int b = bh / p.heads, h = bh % p.heads;
  const int64_t base = (int64_t)bh * p.splits * p.sq + q;  // (b, h, split 0, q)
  const float* ls = p.lse + base;
  const float* ps = p.parts + base * p.dim + 4 * c;
  const int64_t part_stride = (int64_t)p.sq * p.dim;
  const int used = merge_splits(p, b, q);
  if (p.skip_single && used == 1) return;  // written by the forward kernel (whole workgroup)
  float peak = kNegBig, tot = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if (act) {
    // The smallest chunk of 4, 8 or 16 that holds a group's splits (16
    // beyond): 64 splits over 8 groups are one chunk of 8, not 16 with half
    // of the loads clamped. The live splits are summed in the same order.
    const int per = (used + G - 1) / G;
    if (per <= 4)
      wide_group<4>(ls, ps, p.sq, part_stride, g, G, used, peak, tot, acc);
    else if (per <= 8)
      wide_group<8>(ls, ps, p.sq, part_stride, g, G, used, peak, tot, acc);
    else
      wide_group<kMergeChunk>(ls, ps, p.sq, part_stride, g, G, used, peak, tot, acc);
    if (c == 0) speak[g] = peak;  // the same in every thread of the group
  }
  __syncthreads();
  float top = kNegBig;
  for (int k = 0; k < G; ++k) top = fmaxf(top, speak[k]);
  if (act) {
    const float scale = expf(peak - top);  // 0 for an empty group below a live peak
    sacc[t] = acc * scale;
    if (c == 0) stot[g] = tot * scale;
  }
  __syncthreads();
  if (g == 0) {
    f32x4 a = {0.0f, 0.0f, 0.0f, 0.0f};
    float total = 0.0f;
    for (int k = 0; k < G; ++k) {
      a += sacc[k * d4n + c];
      total += stot[k];
    }
    const float inv = 1.0f / fmaxf(total, 1.0e-30f);
    u32x2 w;
    w.x = E::pack2(a[0] * inv, a[1] * inv);
    w.y = E::pack2(a[2] * inv, a[3] * inv);
    u16* dst = static_cast<u16*>(p.out) + (((int64_t)b * p.sq + q) * p.heads + h) * p.dim + 4 * c;
    *reinterpret_cast<u32x2*>(dst) = w;
  }
}

// Merge of the static schedule's split tiles: group g (task, first slot,
// slots) is merged by groups_wg workgroups, workgroup j taking rows
// [j rows_wg, (j + 1) rows_wg) of the tile; the partials of slot s are in
// parts [s, rows_tile, D]. Groups a host plan cannot produce are skipped.
template <bool BF16>
__global__ __launch_bounds__(kMergeThreads) void group_merge_kernel(GroupMergeParams p) {
  const int32_t* gr = p.groups + 3 * (int64_t)(blockIdx.x / (unsigned)p.wg_per_group);
  const int task = gr[0], first = gr[1], count = gr[2];
  if (task < 0 || task >= p.tasks || first < 0 || count < 1 || first + count > p.slots) return;
  const int qt = task % p.q_tiles;
  const int bh = task / p.q_tiles;
  const int h = bh % p.heads, b = bh / p.heads;
  const int q0 = qt * p.rows_tile;
  const int tile_rows = p.sq - q0 < p.rows_tile ? p.sq - q0 : p.rows_tile;
  const int r0 = (int)(blockIdx.x % (unsigned)p.wg_per_group) * p.rows_wg;
  const int rows = tile_rows - r0 < p.rows_wg ? tile_rows - r0 : p.rows_wg;
  const int d4n = p.dim / 4;
  const int64_t slot_rows = (int64_t)p.rows_tile;
  for (int idx = threadIdx.x; idx < rows * d4n; idx += kMergeThreads) {
    const int r = r0 + idx / d4n, d0 = 4 * (idx % d4n);
    u16* dst = static_cast<u16*>(p.out) + (((int64_t)b * p.sq + q0 + r) * p.heads + h) * p.dim + d0;
    merge_one<BF16>(p.lse + first * slot_rows + r, slot_rows,
                    p.parts + (first * slot_rows + r) * p.dim + d0, slot_rows * p.dim, count, dst);
  }
}

// Packed copy of the live cache: out[b, pos] = cache[phys_row(b, pos)] for
// pos < len[b], zero rows for len[b] <= pos < out_len. Uses the same
// position -> pool-row resolution as the attention kernel.
__global__ __launch_bounds__(256) void gather_kernel(GatherParams p) {
  const int64_t r = blockIdx.x;
  const int b = (int)(r / p.out_len);
  const int pos = (int)(r % p.out_len);
  const int capacity = p.width * p.page_size;
  int len = p.lengths[b];
  len = len < 0 ? 0 : (len > capacity ? capacity : len);
  const int chunks = p.heads * p.dim / 8;
  const int64_t row_bytes = (int64_t)p.heads * p.dim * 2;
  int64_t src = -1;
  if (pos < len) {
    src = phys_row(p.table + (int64_t)b * p.width, (u32)pos, (u32)p.page_size, p.page_magic,
                   p.page_shift, p.pool_rows);
  }
  const char* ks = static_cast<const char*>(p.k);
  const char* vs = static_cast<const char*>(p.v);
  char* ko = static_cast<char*>(p.out_k) + r * row_bytes;
  char* vo = static_cast<char*>(p.out_v) + r * row_bytes;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (src >= 0) {
      kv = load16(ks + src * row_bytes + c * 16);
      vv = load16(vs + src * row_bytes + c * 16);
    }
    *reinterpret_cast<u32x4*>(ko + c * 16) = kv;
    *reinterpret_cast<u32x4*>(vo + c * 16) = vv;
  }
}

// Page-granular packing of the live cache: packed page g (rows
// [g page, g page + page) of out) is page j of request b, where b is the
// request whose packed rows [cu_rows[b], cu_rows[b + 1]) hold row g page and
// j = (g page - cu_rows[b]) / page; its source is pool page table[b, j],
// copied whole (rows past len included), or zeros for a page id outside the
// pool. The format is the reference's packed cache
// (benchmarks/mha/external_cache_gather.py:28-35: each request's live
// region rounded up to whole pages, in request order). One workgroup moves
// kPackChunks 16-byte chunks of K and of V of one page; every thread issues
// all its loads before its stores.
constexpr int kPackThreads = 256;
constexpr int kPackPerThread = 4;
constexpr int kPackChunks = kPackThreads * kPackPerThread;
__global__ __launch_bounds__(kPackThreads) void pack_pages_kernel(PackParams p) {
  const int g = (int)(blockIdx.x / (unsigned)p.wg_per_page);
  const int part = (int)(blockIdx.x % (unsigned)p.wg_per_page);
  const int64_t row0 = (int64_t)g * p.page_size;
  // Request b: the last b with cu_rows[b] <= row0 (empty requests have
  // cu_rows[b] == cu_rows[b + 1] and are passed over).
  int lo = 0, hi = p.batch;  // cu_rows[lo] <= row0 < cu_rows[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.cu_rows[mid] <= row0) lo = mid; else hi = mid;
  }
  const int b = lo;
  const int64_t j = (row0 - p.cu_rows[b]) / p.page_size;
  int64_t src_page = -1;
  if (j >= 0 && j < p.width) {
    const int32_t id = p.table[(int64_t)b * p.width + j];
    if (id >= 0 && ((int64_t)id + 1) * p.page_size <= p.pool_rows) src_page = id;
  }
  const int64_t src = src_page >= 0 ? src_page * p.page_chunks : 0;
  const u32x4* ks = static_cast<const u32x4*>(p.k) + src;
  const u32x4* vs = static_cast<const u32x4*>(p.v) + src;
  u32x4* ko = static_cast<u32x4*>(p.out_k) + (int64_t)g * p.page_chunks;
  u32x4* vo = static_cast<u32x4*>(p.out_v) + (int64_t)g * p.page_chunks;
  const int c0 = part * kPackChunks + (int)threadIdx.x;
  u32x4 kx[kPackPerThread], vx[kPackPerThread];
#pragma unroll
  for (int i = 0; i < kPackPerThread; ++i) {
    const int c = c0 + i * kPackThreads;
    kx[i] = u32x4{0u, 0u, 0u, 0u};
    vx[i] = u32x4{0u, 0u, 0u, 0u};
    if (src_page >= 0 && c < p.page_chunks) {
      kx[i] = ks[c];
      vx[i] = vs[c];
    }
  }
#pragma unroll
  for (int i = 0; i < kPackPerThread; ++i) {
    const int c = c0 + i * kPackThreads;
    if (c < p.page_chunks) {
      ko[c] = kx[i];
      vo[c] = vx[i];
    }
  }
}

}  // namespace fgw_mha
