// Split-KV LSE merge and the stand-alone paged K/V gather.
#pragma once
#include "fmha_kernel.h"

namespace fgw_mha {

// Stand-alone LSE merge: one workgroup per (b, h, group of rows_per_wg rows).
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

template <bool BF16>
__global__ __launch_bounds__(kMergeThreads) void merge_wide_kernel(MergeParams p) {
  __shared__ float speak[kMergeThreads];
  __shared__ float stot[kMergeThreads];
  __shared__ f32x4 sacc[kMergeThreads];
  const int q = (int)(blockIdx.x % (unsigned)p.sq);
  const int bh = (int)(blockIdx.x / (unsigned)p.sq);
  const int b = bh / p.heads, h = bh % p.heads;
  const int used = merge_splits(p, b, q);
  if (p.skip_single && used == 1) return;  // written by the forward kernel (whole workgroup)
  merge_wide_row<BF16>(p.parts, p.lse, p.out, p.sq, p.heads, p.dim, p.splits, used, b, h, q,
                       threadIdx.x, speak, stot, sacc);
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
