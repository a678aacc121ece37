// Prefill layout of the paged attention forward (long query tiles).
//
// A work item is (b, h, 256-row query tile, KV split). Eight waves own 32
// query rows each and share every K/V block (32 keys at D 128, 64 at D 64),
// which the DMA engine
// moves from HBM into two three-slot LDS rings (K and V). Per block the wave
// computes S^T = K . Q^T and O^T += V^T . P^T on v_mfma_f32_32x32x16 with the
// operand layouts of fwd_kernel (fmha_kernel.h), and the online softmax of
// the reference (operators/mha/kernels/mha_paged_decode_ascend_v7.py:120-205).
//
// Software pipeline (lag 2). Step n (n = 0 .. N for N blocks) issues, in one
// basic block:
//   MFMA  QK^T of block n + 1 into S_next    (K ring slot (n + 1) % 3)
//   VALU  softmax of block n: S_cur -> P_cur  (row max, exp2, row sum, pack)
//   MFMA  PV of block n - 1 from P_prev       (V ring slot (n - 1) % 3)
// The softmax is independent of both MFMA groups, so the matrix cores and the
// VALU run side by side. Every step runs the same code: P of block -1 is
// zero, the QK^T of steps N - 1 and N reads a clamped block that is never
// used, and the softmax of step N masks every key. When block n raises the
// exponent reference m, l is rescaled inside the softmax and O at the start
// of step n + 1: after the PV of block n - 1 (old m), before that of block n.
//
// DMA. Batch n (planned after the barrier of step n, issued spread over the
// step's MFMA slots) loads K block n + 3 into K slot n % 3 and V block n + 1
// into V slot (n + 1) % 3; both slots were last read in step n - 1. Step n needs batch
// n - 2 (K block n + 1, V block n - 1), so every load has two steps to land.
// Batch indices outside [0, N) load a clamped block into the free slot, which
// keeps the per-wave count of outstanding loads uniform, so the wait before
// step n is the constant vmcnt(one batch). The loads are issued by inline
// assembly: the compiler then neither sees them as LDS writes (it would
// otherwise wait for every outstanding DMA before each transposing LDS read)
// nor counts them; the explicit waits here are the only ones they need, and
// the compiler's own vmcnt waits stay correct because loads retire in order.
#pragma once
#include "fmha_kernel.h"

namespace fgw_mha {

template <bool BF16_, int DPAD_>
struct PCfg {
  static constexpr bool BF16 = BF16_;
  static constexpr int DPAD = DPAD_;
  static constexpr int LAYOUT = kLayoutPrefill;
  static constexpr int NWQ = 4;  // waves along query rows; all share each K/V block
  static constexpr int NWK = 1;
  static constexpr int G = 2;    // 32-row groups per wave: every LDS operand feeds G MFMAs
  static constexpr int BN = 32;  // keys per block
  static constexpr int WAVES = NWQ;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS_WAVE = 32 * G;
  static constexpr int ROWS_TILE = ROWS_WAVE * NWQ;
  static constexpr int KK = DPAD / 16;  // QK k-steps
  static constexpr int DT = DPAD / 32;  // O^T row tiles
  static constexpr int ST = BN / 32;    // S^T tiles per block
  static constexpr int KS = BN / 16;    // PV k-steps
  static constexpr int CPR = DPAD / 8;  // 16-byte chunks per LDS row
  static constexpr int ROW_BYTES = DPAD * 2;
  static constexpr int TILE_BYTES = BN * ROW_BYTES;
  static constexpr int NSLOT = 3;
  static constexpr int LDS_BYTES = 2 * NSLOT * TILE_BYTES;
  static constexpr int INSTR = TILE_BYTES / 1024;  // DMA instructions per tile
  static constexpr int INSTR_PER_WAVE = INSTR / NWQ;
  static constexpr int BATCH = 2 * INSTR_PER_WAVE;  // per wave: one K and one V tile
  static constexpr int KSW = CMin<16, CPR>::value;
  static constexpr int VSW = CPR / 4;
  static constexpr int RPI = 64 / CPR;
  static_assert(DPAD == 64 || DPAD == 128, "prefill layout head-dim tiles");
  static_assert(INSTR % NWQ == 0 && INSTR_PER_WAVE >= 1, "DMA granularity");
  static_assert(LDS_BYTES <= kLdsBudget, "LDS budget of one CU");
};

// DMA of the K (IS_V false) or V tile of keys [pos0, pos0 + BN) of (b, h).
// Instruction q of the wave fills LDS [dst + 1024 i, + 1024) with
// i = q * NWQ + wave. Fast case: the block lies in one page, below len,
// inside the pool, with D == DPAD; its instructions read a uniform tile base
// plus the wave's fixed per-lane offsets (DmaBatch::issue). Otherwise every
// key row is resolved through the table and masked chunks (key >= len,
// d >= D, page id outside the pool) read the zero chunk (issue_slow_tile).
// Pool byte offset (row * row_bytes) of the first key row of block j of a
// work item (keys key0 + j BN ..), or -1 when the block needs the per-key
// path (it straddles a page or len, leaves the pool, or D < DPAD). Blocks
// j >= N are never loaded and read -1. Evaluated per lane, one block per lane.
template <class C>
__device__ __forceinline__ int64_t block_offset(const FwdParams& p, const int32_t* table_b,
                                                int64_t row_bytes, int key0, int N, int len,
                                                int j) {
  const u32 page = (u32)p.page_size;
  const int pos0 = key0 + j * C::BN;
  const bool live = j < N;
  const u32 pg0 = live ? div_page((u32)pos0, p.page_magic, p.page_shift) : 0u;
  const u32 off0 = (u32)pos0 - pg0 * page;
  const int64_t row0 = (int64_t)table_b[pg0] * page + off0;
  const bool fast = live && off0 + C::BN <= page && pos0 + C::BN <= len && row0 >= 0 &&
                    row0 + C::BN <= p.pool_rows && p.dim == C::DPAD;
  return fast ? row0 * row_bytes : -1;
}

// Offsets of blocks [64 w, 64 w + 64) of a work item, one per lane (lane l:
// block 64 w + l); the step plan reads them with readlane.
struct BlockWindow {
  int w;
  int64_t off;
};

__device__ __forceinline__ int64_t readlane64(int64_t x, int lane) {
  const u32 lo = __builtin_amdgcn_readlane((u32)x, lane);
  const u32 hi = __builtin_amdgcn_readlane((u32)((uint64_t)x >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <class C, bool IS_V>
__device__ __forceinline__ void issue_slow_tile(const FwdParams& p, const int32_t* table_b,
                                                const char* base, int64_t row_bytes, int pos0,
                                                int len, u32 dst, int wave, int lane) {
  const u32 page = (u32)p.page_size;
  const char* zero = reinterpret_cast<const char*>(kZeroChunk);
#pragma unroll
  for (int q = 0; q < C::INSTR_PER_WAVE; ++q) {
    const int i = q * C::NWQ + wave;
    const int r = C::RPI * i + lane / C::CPR, pos_in_row = lane % C::CPR;
    const int pos = pos0 + r;
    const u32 pg = div_page((u32)pos, p.page_magic, p.page_shift);
    const int32_t id = table_b[pos < len ? pg : 0u];
    const int64_t row = (int64_t)id * page + ((u32)pos - pg * page);
    const bool live = pos < len && id >= 0 && row < p.pool_rows;
    const int c = IS_V ? pos_in_row ^ (4 * (r % C::VSW)) : pos_in_row ^ (r % C::KSW);
    const char* src = live && c * 8 < p.dim ? base + row * row_bytes + c * 16 : zero;
    dma_flat(src, dst + 1024u * i);
  }
}

// One batch of DMA instructions of a wave (the K tile, then the V tile) in
// the fast case: uniform tile bases, the wave's fixed per-lane offsets and
// uniform LDS destinations. `fast` false: the batch was issued already.
template <class C>
struct DmaBatch {
  static constexpr int NI = C::BATCH;
  bool fast;
  const char* kbase;
  const char* vbase;
  u32 kdst, vdst;  // LDS byte address of the K / V slot
  // Instruction i of the batch (K tile first); the row offset of the
  // instruction joins the uniform base, the lane's offset is fixed.
  __device__ __forceinline__ void issue(int i, const DmaLanes<C>& dl, int wave,
                                        int64_t row_bytes) const {
    constexpr int IPW = C::INSTR_PER_WAVE;
    const int q = i % IPW;
    const int ii = q * C::NWQ + wave;
    const int64_t rows = (int64_t)(C::RPI * ii) * row_bytes;
    if (i < IPW) {
      dma_saddr(kbase + rows, dl.kq(q, wave), kdst + 1024u * (u32)ii);
    } else {
      dma_saddr(vbase + rows, dl.vq(q, wave), vdst + 1024u * (u32)ii);
    }
  }
};

// Keeps the computation of x inside the scheduling region where it is
// pinned: the empty volatile assembly reads x, so x cannot be sunk past it,
// and volatile assembly keeps its place between the region's fences.
__device__ __forceinline__ void pin(float x) { asm volatile("" ::"v"(x)); }
__device__ __forceinline__ void pin(u32 x) { asm volatile("" ::"v"(x)); }

// Softmax state of one wave: per 32-row group g, the exponent reference m
// (log2 units), the row sum l and the rescale factor of the last step.
template <class C>
struct RowState {
  float m[C::G], l[C::G], alpha[C::G];
  bool rescale;
};

// Body of one pipeline step, one basic block: QK^T of the next block into
// s_next from K slot `ks`, softmax of the current block (s_cur -> pf_cur),
// PV of the previous block from pf_prev and V slot `vs`. Sets st.rescale and
// st.alpha when an exponent reference moved; the caller rescales O before the
// next step's PV.
//
// The issue order is fixed by hand in NM slots (NM = K or V operands per
// block): slot j issues the LDS reads of operand j + AHEAD of each product,
// the G QK^T MFMAs of K operand j, one softmax part, the G PV MFMAs of V
// operand j and the next softmax part; the step's DMA instructions go out
// one per NM / BATCH slots, so that the waves of a workgroup do not queue a
// whole batch at the same moment. Scheduling fences between slots keep each
// read AHEAD slots before its MFMAs and the softmax spread over the MFMAs.
// The 2 NM softmax parts: the row max of group g in part g, the new
// references in part G, then exp2, row sum and pack of the scores.
template <class C>
__device__ __forceinline__ void step_body(const unsigned char* ks, const unsigned char* vs,
                                          const DmaBatch<C>& dma, const DmaLanes<C>& dl,
                                          int wave, int64_t row_bytes, const Lanes<C>& ln,
                                          const u32x4 (&qf)[C::G][C::KK],
                                          f32x16 (&s_next)[C::G][C::ST],
                                          const f32x16 (&s_cur)[C::G][C::ST],
                                          const u32x4 (&pf_prev)[C::G][C::KS],
                                          u32x4 (&pf_cur)[C::G][C::KS], f32x16 (&o)[C::G][C::DT],
                                          RowState<C>& st, float scale_log2) {
  using E = Elem<C::BF16>;
  constexpr int G = C::G;
  constexpr int NM = C::KK * C::ST;
  static_assert(NM == C::KS * C::DT, "QK^T and PV have equal operand counts");
  constexpr int NVG = 16 * C::ST;      // scores per lane and group
  constexpr int NV = G * NVG;          // scores per lane
  constexpr int NP = 2 * NM;           // softmax parts
  constexpr int EP = NP - G - 1;       // exp2 / sum / pack parts
  static_assert(EP >= 1, "softmax part split");

  auto rk = [&](int j) { return read_k<C>(ks, ln, j % C::ST, j / C::ST); };
  auto rv = [&](int j) { return read_vt<C>(vs, ln, j % C::DT, j / C::DT); };
  auto sc = [&](int k) { return s_cur[k / NVG][(k % NVG) / 16][k % 16]; };

  float mx[G], mn[G], neg_m[G], rs[G];
#pragma unroll
  for (int g = 0; g < G; ++g) rs[g] = 0.0f;
  float ev[NV];
  auto softmax_part = [&](int part) {
    if (part < G) {
      const int g = part;
      float x = sc(g * NVG);
#pragma unroll
      for (int k = 1; k < NVG; ++k) x = fmaxf(x, sc(g * NVG + k));
      mx[g] = x;
      pin(mx[g]);
    } else if (part == G) {
      bool any = false;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx[g]),
                                                         __float_as_uint(mx[g]), false, false);
        mx[g] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale_log2;
        any = any || mx[g] > st.m[g] + kRescaleSlack;
      }
      st.rescale = __ballot(any) != 0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        mn[g] = st.rescale ? fmaxf(st.m[g], mx[g]) : st.m[g];
        st.alpha[g] = __builtin_amdgcn_exp2f(st.m[g] - mn[g]);
        neg_m[g] = -mn[g];
        pin(neg_m[g]);
      }
    } else {
      const int q = part - G - 1;
      const int k_begin = q * NV / EP, k_end = (q + 1) * NV / EP;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (k >= k_begin && k < k_end) {
          const int g = k / NVG, kg = k % NVG;
          ev[k] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc(k), scale_log2, neg_m[g]));
          rs[g] += ev[k];
          if (kg & 1) {
            const u32 w = E::pack2(ev[k - 1], ev[k]);
            pin(w);
            u32x4& dst = pf_cur[g][kg / 8];
            const int c = (kg % 8) / 2;
            if (c == 0) dst.x = w;
            if (c == 1) dst.y = w;
            if (c == 2) dst.z = w;
            if (c == 3) dst.w = w;
          }
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) pin(rs[g]);
    }
  };

#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < C::ST; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) s_next[g][t][v] = 0.0f;
  constexpr int AHEAD = 2;  // slots between an operand read and its MFMAs
  u32x4 ka[AHEAD + 1], va[AHEAD + 1];
#pragma unroll
  for (int j = 0; j < AHEAD; ++j) {
    ka[j] = rk(j);
    va[j] = rv(j);
  }
  static_assert(NM % C::BATCH == 0, "DMA slots");
#pragma unroll
  for (int j = 0; j < NM; ++j) {
    if (j % (NM / C::BATCH) == 0 && dma.fast) dma.issue(j / (NM / C::BATCH), dl, wave, row_bytes);
    if (j + AHEAD < NM) {
      ka[(j + AHEAD) % (AHEAD + 1)] = rk(j + AHEAD);
      va[(j + AHEAD) % (AHEAD + 1)] = rv(j + AHEAD);
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
      s_next[g][j % C::ST] = E::mma(ka[j % (AHEAD + 1)], qf[g][j / C::ST], s_next[g][j % C::ST]);
    softmax_part(2 * j);
#pragma unroll
    for (int g = 0; g < G; ++g)
      o[g][j % C::DT] = E::mma(va[j % (AHEAD + 1)], pf_prev[g][j / C::DT], o[g][j % C::DT]);
    softmax_part(2 * j + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    st.m[g] = mn[g];
    st.l[g] = st.l[g] * st.alpha[g] + rs[g];
  }
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void prefill_kernel(FwdParams p,
                                                             const int32_t* __restrict__ table,
                                                             const int32_t* __restrict__ lengths) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::LDS_BYTES];
  unsigned char* const kring = smem;
  unsigned char* const vring = smem + C::NSLOT * C::TILE_BYTES;
  const u32 kring_lds = lds_address(kring), vring_lds = lds_address(vring);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int il = lane & 31, hh = lane >> 5;
  const Lanes<C> ln(lane);
  const int64_t row_bytes = (int64_t)p.heads * p.dim * 2;
  const DmaLanes<C> dl(lane, wave, row_bytes);

  const int grid = gridDim.x;
  const int prog = xcd_remap(blockIdx.x, grid);
  const int per = p.work / grid, rem = p.work % grid;
  const int first = prog * per + (prog < rem ? prog : rem);
  const int count = per + (prog < rem ? 1 : 0);
  const int capacity = p.width * p.page_size;

  for (int it = 0; it < count; ++it) {
    int w = first + it;
    const int split = w % p.splits;
    w /= p.splits;
    const int qt = w % p.q_tiles;
    w /= p.q_tiles;
    const int h = w % p.heads;
    const int b = w / p.heads;
    const int32_t* table_b = table + (int64_t)b * p.width;
    const char* kb = static_cast<const char*>(p.k) + (int64_t)h * p.dim * 2;
    const char* vb = static_cast<const char*>(p.v) + (int64_t)h * p.dim * 2;

    int len = lengths[b];
    len = len < 0 ? 0 : (len > capacity ? capacity : len);
    const int q0 = qt * C::ROWS_TILE;
    const int tile_last = (q0 + C::ROWS_TILE < p.sq ? q0 + C::ROWS_TILE : p.sq) - 1;
    int max_vis = p.causal ? len - p.sq + tile_last + 1 : len;
    max_vis = max_vis < 0 ? 0 : (max_vis > len ? len : max_vis);
    const int nblk = (max_vis + C::BN - 1) / C::BN;
    const int blk_begin = (int)((int64_t)nblk * split / p.splits);
    const int blk_end = (int)((int64_t)nblk * (split + 1) / p.splits);
    const int N = blk_end - blk_begin;
    const int key0 = blk_begin * C::BN;

    // Rows of this wave (group g: rows row_base + 32 g + il) and their
    // visible key counts; blocks that end above wmin hold keys some row of
    // the wave cannot see and are masked.
    const int row_base = q0 + wave * C::ROWS_WAVE;
    int wmin = p.causal ? len - p.sq + row_base + 1 : len;
    wmin = wmin < 0 ? 0 : (wmin > len ? len : wmin);
    int vis[C::G];
#pragma unroll
    for (int g = 0; g < C::G; ++g) {
      const int qrow = row_base + 32 * g + il;
      int v = p.causal ? len - p.sq + qrow + 1 : len;
      vis[g] = v < 0 ? 0 : (v > len ? len : v);
    }

    u32x4 qf[C::G][C::KK];
#pragma unroll
    for (int g = 0; g < C::G; ++g) {
      const int qrow = row_base + 32 * g + il;
      const u16* qp =
          static_cast<const u16*>(p.q) + (((int64_t)b * p.sq + qrow) * p.heads + h) * p.dim;
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) {
        const int d = 16 * kk + 8 * hh;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (qrow < p.sq && d < p.dim) val = load16(qp + d);
        qf[g][kk] = val;
      }
    }
    RowState<C> st;
    f32x16 o[C::G][C::DT];
#pragma unroll
    for (int g = 0; g < C::G; ++g) {
      st.m[g] = kNegBig;
      st.l[g] = 0.0f;
      st.alpha[g] = 1.0f;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[g][dt][v] = 0.0f;
    }
    st.rescale = false;

    __syncthreads();  // the previous work item no longer reads the rings

    if (N > 0) {
      // Batch n: K block n + 3 -> K slot n % 3, V block n + 1 -> V slot (n + 1) % 3.
      // Tile bases come from two 64-block windows of per-lane offsets (the V
      // block's window and the next), refreshed when the V block leaves the
      // first: one table read per lane every 64 steps instead of scalar
      // page-id loads and address arithmetic on every step.
      BlockWindow win0{0, block_offset<C>(p, table_b, row_bytes, key0, N, len, lane)};
      BlockWindow win1{1, block_offset<C>(p, table_b, row_bytes, key0, N, len, 64 + lane)};
      // The V block only moves forward, one block per step, and the K block
      // is at most two blocks ahead of it: windows w(jv) and w(jv) + 1 cover both.
      auto advance = [&](int jv) {
        if ((jv >> 6) != win0.w) {  // uniform: the V block entered the next window
          win0 = win1;
          win1 = BlockWindow{win0.w + 1, block_offset<C>(p, table_b, row_bytes, key0, N, len,
                                                         64 * (win0.w + 1) + lane)};
        }
      };
      auto offset_of = [&](int j) {
        return readlane64((j >> 6) == win0.w ? win0.off : win1.off, j & 63);
      };
      auto plan_batch = [&](int n, DmaBatch<C>& db) {
        const int jv = n + C::NSLOT - 2 < 0 ? 0 : (n + C::NSLOT - 2 < N ? n + C::NSLOT - 2 : N - 1);
        const int jk = n + C::NSLOT < N ? n + C::NSLOT : N - 1;
        advance(jv);
        const int64_t ov = offset_of(jv);
        const int64_t ok = offset_of(jk);
        db.kdst = kring_lds + (u32)(((n + C::NSLOT) % C::NSLOT) * C::TILE_BYTES);
        db.vdst = vring_lds + (u32)(((n + 2 * C::NSLOT - 2) % C::NSLOT) * C::TILE_BYTES);
        db.fast = ok >= 0 && ov >= 0;
        db.kbase = kb + ok;
        db.vbase = vb + ov;
        if (!db.fast) {
          issue_slow_tile<C, false>(p, table_b, kb, row_bytes, key0 + jk * C::BN, len, db.kdst,
                                    wave, lane);
          issue_slow_tile<C, true>(p, table_b, vb, row_bytes, key0 + jv * C::BN, len, db.vdst,
                                   wave, lane);
        }
      };

      DmaBatch<C> db;
#pragma unroll
      for (int n = -C::NSLOT; n < 0; ++n) {
        plan_batch(n, db);
        if (db.fast) {
#pragma unroll
          for (int q = 0; q < C::BATCH; ++q) db.issue(q, dl, wave, row_bytes);
        }
      }
      wait_vm<2 * C::BATCH>();  // batch -3: K block 0
      __syncthreads();

      f32x16 s_a[C::G][C::ST], s_b[C::G][C::ST];
      u32x4 pf_a[C::G][C::KS], pf_b[C::G][C::KS];
      {
        using E = Elem<C::BF16>;
#pragma unroll
        for (int g = 0; g < C::G; ++g)
#pragma unroll
          for (int t = 0; t < C::ST; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) s_a[g][t][v] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk)
#pragma unroll
          for (int t = 0; t < C::ST; ++t) {
            const u32x4 a = read_k<C>(kring, ln, t, kk);
#pragma unroll
            for (int g = 0; g < C::G; ++g) s_a[g][t] = E::mma(a, qf[g][kk], s_a[g][t]);
          }
      }
      // P of block -1 is zero: the PV of step 0 adds nothing.
#pragma unroll
      for (int g = 0; g < C::G; ++g)
#pragma unroll
        for (int k2 = 0; k2 < C::KS; ++k2) pf_b[g][k2] = u32x4{0u, 0u, 0u, 0u};

      // Steps n = 0 .. N; registers alternate: even steps read s_a / pf_b and
      // write s_b / pf_a, odd steps the reverse.
      auto prologue = [&](int n, f32x16(&s)[C::G][C::ST]) {
        wait_vm<C::BATCH>();  // batch n - 2: K block n + 1, V block n - 1
        __syncthreads();      // ... for every wave; the slots of step n - 1 are free
        plan_batch(n, db);  // issued from inside the step body
        if (st.rescale) {
#pragma unroll
          for (int g = 0; g < C::G; ++g)
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt) o[g][dt] *= st.alpha[g];
        }
        const int pos0 = key0 + n * C::BN;
        if (n >= N || pos0 + C::BN > wmin) {
#pragma unroll
          for (int g = 0; g < C::G; ++g) mask_block<C>(s[g], pos0, n >= N ? 0 : vis[g], hh);
        }
      };
      int sk = 1, sv = 2;  // ring slots of K block n + 1 and V block n - 1
      for (int n = 0;; n += 2) {
        prologue(n, s_a);
        step_body<C>(kring + sk * C::TILE_BYTES, vring + sv * C::TILE_BYTES, db, dl, wave,
                     row_bytes, ln, qf, s_b, s_a, pf_b, pf_a, o, st, p.scale_log2);
        sk = sk == C::NSLOT - 1 ? 0 : sk + 1;
        sv = sv == C::NSLOT - 1 ? 0 : sv + 1;
        if (n == N) break;
        prologue(n + 1, s_b);
        step_body<C>(kring + sk * C::TILE_BYTES, vring + sv * C::TILE_BYTES, db, dl, wave,
                     row_bytes, ln, qf, s_a, s_b, pf_a, pf_b, o, st, p.scale_log2);
        sk = sk == C::NSLOT - 1 ? 0 : sk + 1;
        sv = sv == C::NSLOT - 1 ? 0 : sv + 1;
        if (n + 1 == N) break;
      }
      wait_vm<0>();  // no DMA of this work item outlives it
    }

#pragma unroll
    for (int g = 0; g < C::G; ++g) {
      const int qrow = row_base + 32 * g + il;
      const float tot = st.l[g] + __shfl_xor(st.l[g], 32);
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
        if (p.mode != 0 && hh == 0) {
          p.lse[(((int64_t)b * p.heads + h) * p.splits + split) * p.sq + qrow] =
              lse_of(st.m[g], tot);
        }
      }
    }
  }
}

template <bool BF16, int DPAD>
hipError_t launch_prefill(const FwdParams& p, int grid, hipStream_t stream) {
  using C = PCfg<BF16, DPAD>;
  prefill_kernel<C><<<dim3(grid), dim3(C::THREADS), 0, stream>>>(p, p.table, p.lengths);
  return hipGetLastError();
}

template <bool BF16, int DPAD>
int occupancy_prefill() {
  using C = PCfg<BF16, DPAD>;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<C>, C::THREADS, 0) !=
      hipSuccess)
    return 0;
  return n;
}

}  // namespace fgw_mha
