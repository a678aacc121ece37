// Paged multi-head attention forward for CDNA4 (gfx950).
//
// One templated kernel covers decode and long-Q prefill, FP16/BF16 and
// head dims 16..256. It computes, per (request b, head h, query tile,
// KV split), the online-softmax attention of the tile's query rows against
// the visible keys of the split, reading K/V rows through the block table.
//
// Math follows the reference operator (operators/mha/kernels/
// mha_paged_decode_ascend_v7.py:120-205, :305-315; cube_general.py:88-157):
//   s = q.k * D^-0.5, running max m, p = exp(s - m) rounded to the input dtype
//   for the PV product, l = l*alpha + sum(p) in fp32, O = alpha*O + P.V,
//   output O / max(l, 1e-30); partial mode stores O/l and LSE = ln(l) + m.
// The exponentials run as exp2 on log2(e)-prescaled scores.
//
// Matrix-core formulation (v_mfma_f32_32x32x16_{bf16,f16}, wave64):
//   S^T = K . Q^T   A = K tile rows (keys) from LDS, B = Q^T held in VGPRs.
//                   The 32x32 accumulator gives each lane one query column
//                   (lane % 32) and 16 key rows.
//   O^T = V^T . P^T A = V^T rows (head dim) from LDS, B = P^T straight from
//                   the S^T accumulator registers after the softmax: the
//                   16 keys a lane holds are exactly the k-slots of its B
//                   operand once V^T is stored with 4-key groups 1 and 2 of
//                   every 16-key group swapped.
// So every lane owns one query row in both products: the softmax needs one
// cross-half (lane ^ 32) exchange per block for the max and the rescale of O
// is lane-local.
//
// Layouts (template parameter LAYOUT):
//   kLayoutQuery: 4 waves x 32 query rows share each 64-key K/V tile staged
//                 in double-buffered LDS (prefill, Sq > 32).
//   kLayoutKey:   4 waves each stream their own 32-key blocks of the same 32
//                 query rows (decode); the four partial softmax states are
//                 combined through LDS before the epilogue.
// Work items (b, h, q_tile, split) are spread over a persistent grid with
// contiguous ranges per program (v7.py:260-264), after an XCD-aware remap of
// the program id so that neighbouring items share an XCD's L2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmha_params.h"

namespace fgw_mha {

typedef uint32_t u32;
typedef uint16_t u16;
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegBig = -1.0e30f;  // running-max floor and empty-split LSE
constexpr int kNumXcd = 8;

template <bool BF16>
struct Elem;

template <>
struct Elem<true> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ u32 pack2(float lo, float hi) {
    bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(u32, v);
  }
};

template <>
struct Elem<false> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ u32 pack2(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(u32, v);
  }
};

// Quotient of a position by the page size (Granlund & Montgomery 1994,
// "Division by invariant integers using multiplication", fig. 4.1):
// shift = ceil(log2 page), magic = floor(2^32 (2^shift - page) / page) + 1.
// shift == 0 encodes page == 1.
__device__ __forceinline__ u32 div_page(u32 n, u32 magic, u32 shift) {
  if (shift == 0) return n;
  const u32 t = __umulhi(magic, n);
  return (t + ((n - t) >> 1)) >> (shift - 1);
}

// Pool row of logical position `pos` of one request:
//   table[b, pos // page] * page + pos % page        (v0.py:137)
// or -1 when the page id points outside the pool (such rows read as zeros
// instead of faulting).
__device__ __forceinline__ int64_t phys_row(const int32_t* table_b, u32 pos, u32 page, u32 magic,
                                            u32 shift, int64_t pool_rows) {
  const u32 pg = div_page(pos, magic, shift);
  const int64_t row = (int64_t)table_b[pg] * page + (pos - pg * page);
  return (row >= 0 && row < pool_rows) ? row : -1;
}

__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Contiguous program ids per XCD: hardware places workgroup i on XCD i % 8.
__device__ __forceinline__ int xcd_remap(int bid, int grid) {
  const int xcd = bid % kNumXcd, local = bid / kNumXcd;
  const int q = grid / kNumXcd, r = grid % kNumXcd;
  return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// 4-key group order inside a 16-key group of the V^T tile: 0,2,1,3.
__device__ __forceinline__ constexpr int swap12(int x) { return ((x & 1) << 1) | ((x >> 1) & 1); }

template <int A, int B>
struct CMax {
  static constexpr int value = A > B ? A : B;
};

template <bool BF16_, int DPAD_, int LAYOUT_>
struct Cfg {
  static constexpr bool BF16 = BF16_;
  static constexpr int DPAD = DPAD_;  // head dim rounded up to 32
  static constexpr int LAYOUT = LAYOUT_;
  static constexpr int NWQ = LAYOUT == kLayoutQuery ? 4 : 1;  // waves along queries
  static constexpr int NWK = LAYOUT == kLayoutQuery ? 1 : 4;  // waves along keys
  static constexpr int BN = LAYOUT == kLayoutQuery ? 64 : 32; // keys per block
  static constexpr int QG = 1;                                // 32-row groups per wave
  static constexpr int WAVES = NWQ * NWK;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS_WAVE = 32 * QG;
  static constexpr int ROWS_TILE = ROWS_WAVE * NWQ;
  static constexpr int KK = DPAD / 16;  // QK k-steps
  static constexpr int DT = DPAD / 32;  // O^T row tiles
  static constexpr int ST = BN / 32;    // S^T tiles per block
  static constexpr int KS = BN / 16;    // PV k-steps
  static constexpr int KSTRIDE = DPAD + 8;  // K tile row stride (elements)
  static constexpr int VSTRIDE = BN + 8;    // V^T tile row stride (elements)
  static constexpr int K_ELEMS = BN * KSTRIDE;
  static constexpr int V_ELEMS = DPAD * VSTRIDE;
  static constexpr int NBUF = NWK == 1 ? 2 : 1;
  static constexpr int GROUP_ELEMS = NBUF * (K_ELEMS + V_ELEMS);
  static constexpr int TILE_BYTES = NWK * GROUP_ELEMS * 2;
  static constexpr int OSTRIDE = DPAD + 4;  // combine buffer row stride (floats)
  static constexpr int COMB_BYTES =
      NWK > 1 ? (2 * NWK * ROWS_WAVE + NWK * ROWS_WAVE * OSTRIDE) * 4 : 0;
  static constexpr int LDS_BYTES = CMax<TILE_BYTES, COMB_BYTES>::value;
  // Loader: the 64 * NWQ threads of a key group fill its tiles.
  static constexpr int LT = 64 * NWQ;
  static constexpr int CPR = DPAD / 8;          // 16-byte chunks per key row
  static constexpr int K_CHUNKS = BN * CPR;     // K: one 16-byte chunk per task
  static constexpr int K_PER_T = (K_CHUNKS + LT - 1) / LT;
  static constexpr int V_SUBS = (BN / 4) * CPR; // V: 4 keys x 8 dims per task
  static constexpr int V_PER_T = (V_SUBS + LT - 1) / LT;
  static_assert(NWQ == 1 || NWK == 1, "tiles are shared by all waves or by none");
  static_assert(DPAD % 32 == 0 && DPAD >= 32 && DPAD <= 256, "head dim tile");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of one CU");
};

template <class C>
struct KVFetch {
  u32x4 k[C::K_PER_T];
  u32x4 v[C::V_PER_T][4];
};

// Synchronise the waves that share one key group's tiles.
template <class C>
__device__ __forceinline__ void group_sync() {
  if constexpr (C::NWQ == 1) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();
  }
}

// Global -> registers: the K and V rows of keys [pos0, pos0 + BN) of (b, h).
// Keys at or beyond `len`, dims at or beyond `dim` and rows whose page id is
// outside the pool are zero; nothing outside the live cache is read, so NaN
// in unused pool rows cannot reach the products (cube_general.py:97-109).
template <class C>
__device__ __forceinline__ void fetch_block(KVFetch<C>& f, const FwdParams& p,
                                            const int32_t* table_b, int h, int pos0, int len,
                                            int lt) {
  const int64_t row_bytes = (int64_t)p.heads * p.dim * 2;
  const char* kb = static_cast<const char*>(p.k) + (int64_t)h * p.dim * 2;
  const char* vb = static_cast<const char*>(p.v) + (int64_t)h * p.dim * 2;
  const u32 page = (u32)p.page_size;
  const u32 pg0 = div_page((u32)pos0, p.page_magic, p.page_shift);
  const u32 off0 = (u32)pos0 - pg0 * page;
  const bool one_page = off0 + C::BN <= page;
  const int64_t row0 = one_page ? (int64_t)table_b[pg0] * page + off0 : 0;

#pragma unroll
  for (int r = 0; r < C::K_PER_T; ++r) {
    const int c = lt + C::LT * r;
    const int j = c / C::CPR, dc = c % C::CPR;
    u32x4 val = {0u, 0u, 0u, 0u};
    const int pos = pos0 + j;
    if ((C::K_CHUNKS % C::LT == 0 || c < C::K_CHUNKS) && pos < len && dc * 8 < p.dim) {
      int64_t row;
      if (one_page) {
        row = row0 + j;
        row = (row >= 0 && row < p.pool_rows) ? row : -1;
      } else {
        row = phys_row(table_b, (u32)pos, page, p.page_magic, p.page_shift, p.pool_rows);
      }
      if (row >= 0) val = load16(kb + row * row_bytes + dc * 16);
    }
    f.k[r] = val;
  }
#pragma unroll
  for (int r = 0; r < C::V_PER_T; ++r) {
    const int sidx = lt + C::LT * r;
    const int jg = sidx / C::CPR, dc = sidx % C::CPR;
    const bool task = (C::V_SUBS % C::LT == 0 || sidx < C::V_SUBS) && dc * 8 < p.dim;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      u32x4 val = {0u, 0u, 0u, 0u};
      const int pos = pos0 + 4 * jg + x;
      if (task && pos < len) {
        int64_t row;
        if (one_page) {
          row = row0 + 4 * jg + x;
          row = (row >= 0 && row < p.pool_rows) ? row : -1;
        } else {
          row = phys_row(table_b, (u32)pos, page, p.page_magic, p.page_shift, p.pool_rows);
        }
        if (row >= 0) val = load16(vb + row * row_bytes + dc * 16);
      }
      f.v[r][x] = val;
    }
  }
}

// Registers -> LDS. K rows as they are; V transposed to V^T[d][key] with
// the 4-key group swap, via byte permutes (4 keys x 8 dims per task).
template <class C>
__device__ __forceinline__ void store_block(const KVFetch<C>& f, u16* ks, u16* vts, int lt) {
#pragma unroll
  for (int r = 0; r < C::K_PER_T; ++r) {
    const int c = lt + C::LT * r;
    if (C::K_CHUNKS % C::LT == 0 || c < C::K_CHUNKS) {
      const int j = c / C::CPR, dc = c % C::CPR;
      *reinterpret_cast<u32x4*>(ks + j * C::KSTRIDE + dc * 8) = f.k[r];
    }
  }
#pragma unroll
  for (int r = 0; r < C::V_PER_T; ++r) {
    const int sidx = lt + C::LT * r;
    if (C::V_SUBS % C::LT == 0 || sidx < C::V_SUBS) {
      const int jg = sidx / C::CPR, dc = sidx % C::CPR;
      const int col = 16 * (jg >> 2) + 4 * swap12(jg & 3);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int xx = 0; xx < 2; ++xx) {
          const u32 sel = xx ? 0x07060302u : 0x05040100u;
          u32x2 w;
          w.x = __builtin_amdgcn_perm(f.v[r][1][e], f.v[r][0][e], sel);
          w.y = __builtin_amdgcn_perm(f.v[r][3][e], f.v[r][2][e], sel);
          *reinterpret_cast<u32x2*>(vts + (8 * dc + 2 * e + xx) * C::VSTRIDE + col) = w;
        }
      }
    }
  }
}

// One BN-key block for one wave: S^T = K Q^T, online softmax, O^T += V^T P^T.
template <class C>
__device__ __forceinline__ void compute_block(const u16* ks, const u16* vts,
                                              const u32x4 (&qf)[C::QG][C::KK],
                                              f32x16 (&o)[C::QG][C::DT], float (&m)[C::QG],
                                              float (&l)[C::QG], const int (&vis)[C::QG], int pos0,
                                              bool need_mask, float scale_log2, int kk_live,
                                              int il, int hh) {
  using E = Elem<C::BF16>;
  f32x16 s[C::QG][C::ST];
#pragma unroll
  for (int g = 0; g < C::QG; ++g)
#pragma unroll
    for (int t = 0; t < C::ST; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[g][t][v] = 0.0f;

#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) {
    if (kk < kk_live) {
      u32x4 a[C::ST];
#pragma unroll
      for (int t = 0; t < C::ST; ++t)
        a[t] = *reinterpret_cast<const u32x4*>(ks + (32 * t + il) * C::KSTRIDE + 16 * kk + 8 * hh);
#pragma unroll
      for (int g = 0; g < C::QG; ++g)
#pragma unroll
        for (int t = 0; t < C::ST; ++t) s[g][t] = E::mma(a[t], qf[g][kk], s[g][t]);
    }
  }

  u32x4 pf[C::QG][C::KS];
#pragma unroll
  for (int g = 0; g < C::QG; ++g) {
    if (need_mask) {
#pragma unroll
      for (int t = 0; t < C::ST; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = pos0 + 32 * t + 8 * (v >> 2) + 4 * hh + (v & 3);
          if (key >= vis[g]) s[g][t][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < C::ST; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[g][t][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m[g], mx * scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(m[g] - mn);
    float rs = 0.0f;
#pragma unroll
    for (int t = 0; t < C::ST; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][t][v], scale_log2, -mn));
        s[g][t][v] = e;
        rs += e;
      }
    l[g] = l[g] * alpha + rs;
    m[g] = mn;
    if (__ballot(alpha != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) o[g][dt] *= alpha;
    }
#pragma unroll
    for (int t = 0; t < C::ST; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        u32x4 w;
        w.x = E::pack2(s[g][t][8 * u + 0], s[g][t][8 * u + 1]);
        w.y = E::pack2(s[g][t][8 * u + 2], s[g][t][8 * u + 3]);
        w.z = E::pack2(s[g][t][8 * u + 4], s[g][t][8 * u + 5]);
        w.w = E::pack2(s[g][t][8 * u + 6], s[g][t][8 * u + 7]);
        pf[g][2 * t + u] = w;
      }
  }

#pragma unroll
  for (int k2 = 0; k2 < C::KS; ++k2)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
      const u32x4 a =
          *reinterpret_cast<const u32x4*>(vts + (32 * dt + il) * C::VSTRIDE + 16 * k2 + 8 * hh);
#pragma unroll
      for (int g = 0; g < C::QG; ++g) o[g][dt] = E::mma(a, pf[g][k2], o[g][dt]);
    }
}

template <class C>
__device__ __forceinline__ void store_row(const FwdParams& p, int b, int h, int split, int qrow,
                                          int d0, f32x4 val, float inv) {
  using E = Elem<C::BF16>;
  if (p.mode == 0) {
    u16* dst = static_cast<u16*>(p.out) + (((int64_t)b * p.sq + qrow) * p.heads + h) * p.dim + d0;
    u32x2 w;
    w.x = E::pack2(val[0] * inv, val[1] * inv);
    w.y = E::pack2(val[2] * inv, val[3] * inv);
    *reinterpret_cast<u32x2*>(dst) = w;
  } else {
    float* dst = p.parts +
                 ((((int64_t)b * p.heads + h) * p.splits + split) * p.sq + qrow) * p.dim + d0;
    *reinterpret_cast<f32x4*>(dst) = val * inv;
  }
}

__device__ __forceinline__ float lse_of(float m_log2, float total) {
  return total > 0.0f ? (m_log2 + log2f(total)) * kLn2 : kNegBig;
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void fwd_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::LDS_BYTES];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int il = lane & 31, hh = lane >> 5;
  const int wq = C::NWQ > 1 ? wave : 0;
  const int wk = C::NWK > 1 ? wave : 0;
  const int lt = C::NWQ > 1 ? tid : lane;
  u16* const group_base = reinterpret_cast<u16*>(smem) + wk * C::GROUP_ELEMS;

  const int grid = gridDim.x;
  const int prog = xcd_remap(blockIdx.x, grid);
  const int per = p.work / grid, rem = p.work % grid;
  const int first = prog * per + (prog < rem ? prog : rem);
  const int count = per + (prog < rem ? 1 : 0);
  const int capacity = p.width * p.page_size;
  const int kk_live = (p.dim + 15) >> 4;

  for (int it = 0; it < count; ++it) {
    int w = first + it;
    const int split = w % p.splits;
    w /= p.splits;
    const int qt = w % p.q_tiles;
    w /= p.q_tiles;
    const int h = w % p.heads;
    const int b = w / p.heads;
    const int32_t* table_b = p.table + (int64_t)b * p.width;

    int len = p.lengths[b];
    len = len < 0 ? 0 : (len > capacity ? capacity : len);
    const int q0 = qt * C::ROWS_TILE;
    const int tile_last = (q0 + C::ROWS_TILE < p.sq ? q0 + C::ROWS_TILE : p.sq) - 1;
    int max_vis = p.causal ? len - p.sq + tile_last + 1 : len;
    max_vis = max_vis < 0 ? 0 : (max_vis > len ? len : max_vis);
    const int nblk = (max_vis + C::BN - 1) / C::BN;
    const int blk_begin = (int)((int64_t)nblk * split / p.splits);
    const int blk_end = (int)((int64_t)nblk * (split + 1) / p.splits);
    const int cnt = blk_end - blk_begin;
    const int my_n = cnt > wk ? (cnt - wk + C::NWK - 1) / C::NWK : 0;

    const int row_base = q0 + wq * C::ROWS_WAVE;
    const bool wave_active = row_base < p.sq;
    const int wave_last = (row_base + C::ROWS_WAVE < p.sq ? row_base + C::ROWS_WAVE : p.sq) - 1;
    int wmin = p.causal ? len - p.sq + row_base + 1 : len;
    wmin = wmin < 0 ? 0 : (wmin > len ? len : wmin);
    int wmax = p.causal ? len - p.sq + wave_last + 1 : len;
    wmax = wmax < 0 ? 0 : (wmax > len ? len : wmax);

    u32x4 qf[C::QG][C::KK];
    int vis[C::QG];
    float m[C::QG], l[C::QG];
    f32x16 o[C::QG][C::DT];
#pragma unroll
    for (int g = 0; g < C::QG; ++g) {
      const int qrow = row_base + 32 * g + il;
      int vv = p.causal ? len - p.sq + qrow + 1 : len;
      vis[g] = vv < 0 ? 0 : (vv > len ? len : vv);
      const u16* qp =
          static_cast<const u16*>(p.q) + (((int64_t)b * p.sq + qrow) * p.heads + h) * p.dim;
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) {
        const int d = 16 * kk + 8 * hh;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (qrow < p.sq && d < p.dim) val = load16(qp + d);
        qf[g][kk] = val;
      }
      m[g] = kNegBig;
      l[g] = 0.0f;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[g][dt][v] = 0.0f;
    }

    __syncthreads();  // LDS of the previous work item is no longer read
    KVFetch<C> f;
    if (my_n > 0) {
      fetch_block<C>(f, p, table_b, h, (blk_begin + wk) * C::BN, len, lt);
      store_block<C>(f, group_base, group_base + C::K_ELEMS, lt);
      group_sync<C>();
    }
    for (int n = 0; n < my_n; ++n) {
      const int pos0 = (blk_begin + wk + C::NWK * n) * C::BN;
      const bool more = n + 1 < my_n;
      if (more) fetch_block<C>(f, p, table_b, h, pos0 + C::NWK * C::BN, len, lt);
      const u16* ks = group_base + (n % C::NBUF) * (C::K_ELEMS + C::V_ELEMS);
      if (wave_active && pos0 < wmax) {
        compute_block<C>(ks, ks + C::K_ELEMS, qf, o, m, l, vis, pos0, pos0 + C::BN > wmin,
                         p.scale_log2, kk_live, il, hh);
      }
      if (more) {
        if constexpr (C::NBUF == 1) group_sync<C>();
        u16* nk = group_base + ((n + 1) % C::NBUF) * (C::K_ELEMS + C::V_ELEMS);
        store_block<C>(f, nk, nk + C::K_ELEMS, lt);
        group_sync<C>();
      }
    }

    if constexpr (C::NWK == 1) {
#pragma unroll
      for (int g = 0; g < C::QG; ++g) {
        const float tot = l[g] + __shfl_xor(l[g], 32);
        const int qrow = row_base + 32 * g + il;
        if (qrow < p.sq) {
          const float inv = 1.0f / fmaxf(tot, 1.0e-30f);
#pragma unroll
          for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const int d0 = 32 * dt + 8 * gq + 4 * hh;
              if (d0 < p.dim) {
                f32x4 val = {o[g][dt][4 * gq], o[g][dt][4 * gq + 1], o[g][dt][4 * gq + 2],
                             o[g][dt][4 * gq + 3]};
                store_row<C>(p, b, h, split, qrow, d0, val, inv);
              }
            }
          if (p.mode == 1 && hh == 0) {
            p.lse[(((int64_t)b * p.heads + h) * p.splits + split) * p.sq + qrow] =
                lse_of(m[g], tot);
          }
        }
      }
    } else {
      // Combine the NWK key-group states of the same query rows.
      __syncthreads();
      float* cm = reinterpret_cast<float*>(smem);
      float* cl = cm + C::NWK * C::ROWS_WAVE;
      float* co = cl + C::NWK * C::ROWS_WAVE;
#pragma unroll
      for (int g = 0; g < C::QG; ++g) {
        const float tot = l[g] + __shfl_xor(l[g], 32);
        const int r = 32 * g + il;
        if (hh == 0) {
          cm[wk * C::ROWS_WAVE + r] = m[g];
          cl[wk * C::ROWS_WAVE + r] = tot;
        }
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            f32x4 val = {o[g][dt][4 * gq], o[g][dt][4 * gq + 1], o[g][dt][4 * gq + 2],
                         o[g][dt][4 * gq + 3]};
            *reinterpret_cast<f32x4*>(co + (wk * C::ROWS_WAVE + r) * C::OSTRIDE + 32 * dt +
                                      8 * gq + 4 * hh) = val;
          }
      }
      __syncthreads();
      constexpr int D4 = C::DPAD / 4;
      for (int idx = tid; idx < C::ROWS_WAVE * D4; idx += C::THREADS) {
        const int r = idx / D4, d0 = 4 * (idx % D4);
        const int qrow = q0 + r;
        if (qrow < p.sq && d0 < p.dim) {
          float mm = kNegBig;
#pragma unroll
          for (int k = 0; k < C::NWK; ++k) mm = fmaxf(mm, cm[k * C::ROWS_WAVE + r]);
          float tot = 0.0f;
          f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int k = 0; k < C::NWK; ++k) {
            const float wt = __builtin_amdgcn_exp2f(cm[k * C::ROWS_WAVE + r] - mm);
            tot += cl[k * C::ROWS_WAVE + r] * wt;
            acc += *reinterpret_cast<const f32x4*>(co + (k * C::ROWS_WAVE + r) * C::OSTRIDE + d0) *
                   wt;
          }
          store_row<C>(p, b, h, split, qrow, d0, acc, 1.0f / fmaxf(tot, 1.0e-30f));
          if (p.mode == 1 && d0 == 0) {
            p.lse[(((int64_t)b * p.heads + h) * p.splits + split) * p.sq + qrow] = lse_of(mm, tot);
          }
        }
      }
    }
  }
}

template <bool BF16, int DPAD, int LAYOUT>
hipError_t launch_fwd(const FwdParams& p, int grid, hipStream_t stream) {
  using C = Cfg<BF16, DPAD, LAYOUT>;
  fwd_kernel<C><<<dim3(grid), dim3(C::THREADS), 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace fgw_mha

namespace fgw_mha {

// Resident workgroups per CU of one instantiation (0 if the query fails).
template <bool BF16, int DPAD, int LAYOUT>
int occupancy_fwd() {
  using C = Cfg<BF16, DPAD, LAYOUT>;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fwd_kernel<C>, C::THREADS, 0) != hipSuccess)
    return 0;
  return n;
}

}  // namespace fgw_mha
