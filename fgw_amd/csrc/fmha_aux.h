// Split-KV LSE merge and the stand-alone paged K/V gather.
#pragma once
#include "fmha_kernel.h"

namespace fgw_mha {

// Combine the split partials of one output row (b, q, h) per wave:
//   peak = max over splits with LSE > -1e29,
//   w_s  = LSE_s > -1e29 ? exp(LSE_s - peak) : 0,
//   O    = sum_s w_s * Part_s / max(sum_s w_s, 1e-30), cast to the input dtype.
// This is the reference merge (v7.py:352-370, cube_general.py:259-278) with
// the running peak taken in a first pass over the LSE values; empty splits
// (LSE -1e30) carry zero weight and an all-empty row is exactly zero.
template <bool BF16>
__global__ __launch_bounds__(256) void merge_kernel(MergeParams p) {
  using E = Elem<BF16>;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t rows = (int64_t)p.batch * p.sq * p.heads;
  if (row >= rows) return;
  const int h = (int)(row % p.heads);
  const int64_t bq = row / p.heads;
  const int q = (int)(bq % p.sq);
  const int b = (int)(bq / p.sq);
  const int64_t bhs = ((int64_t)b * p.heads + h) * p.splits;

  float peak = kNegBig;
  for (int s = 0; s < p.splits; ++s) {
    const float x = p.lse[(bhs + s) * p.sq + q];
    if (x > -1.0e29f) peak = fmaxf(peak, x);
  }
  const int d0 = lane * 4;
  float tot = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < p.splits; ++s) {
    const float x = p.lse[(bhs + s) * p.sq + q];
    const float wgt = x > -1.0e29f ? expf(x - peak) : 0.0f;
    tot += wgt;
    if (wgt != 0.0f && d0 < p.dim) {
      acc += *reinterpret_cast<const f32x4*>(p.parts + ((bhs + s) * p.sq + q) * p.dim + d0) * wgt;
    }
  }
  if (d0 < p.dim) {
    const float inv = 1.0f / fmaxf(tot, 1.0e-30f);
    u32x2 w;
    w.x = E::pack2(acc[0] * inv, acc[1] * inv);
    w.y = E::pack2(acc[2] * inv, acc[3] * inv);
    u16* dst = static_cast<u16*>(p.out) + (((int64_t)b * p.sq + q) * p.heads + h) * p.dim + d0;
    *reinterpret_cast<u32x2*>(dst) = w;
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

}  // namespace fgw_mha
