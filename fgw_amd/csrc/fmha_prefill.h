// Prefill layout of the paged attention forward (long query tiles).
//
// A work item is (b, h, 256-row query tile, KV split). Eight waves own 32
// query rows each and share every 64-key K/V block, which the DMA engine
// moves from HBM into four-slot K and V rings in LDS.
// Per block a wave computes S^T = K . Q^T and O^T += V^T . P^T on
// v_mfma_f32_32x32x16 with the operand layouts and the online softmax of
// fwd_kernel (fmha_kernel.h; reference math: operators/mha/kernels/
// mha_paged_decode_ascend_v7.py:120-205).
//
// Two wave groups, ping-pong. A workgroup of eight waves puts two waves on
// every SIMD: wave w and wave w + 4, in groups A (waves 0-3) and B (4-7).
// Each wave alternates a matrix phase M(n) (PV of block n - 1, then QK^T of
// block n: MFMAs and the LDS reads that feed them) and a vector phase S(n)
// (softmax of block n: exp2, row sum, pack of P; the row max and the O
// rescale only when the exponent reference has to move).
// Group B runs one phase behind group A, and a workgroup barrier separates
// the phases, so in every phase one wave of each SIMD issues MFMAs while
// the other runs the softmax: the matrix cores stay busy while the VALU
// works, which one wave alone cannot arrange (its instructions issue in
// order).
//
//   phase 2m:      A: M(m)        B: S(m - 1)   all: DMA batch of block m + 2
//   phase 2m + 1:  A: S(m)        B: M(m)       all: wait for block m + 1
//
// for m = 0 .. N (N blocks). M(0) has no PV (there is no block -1) and M(N)
// no QK^T (there is no block N); both loops peel them. S(n) rescales O
// after the PV of block n - 1 (in M(n)) and before that of block n (in
// M(n + 1)).
//
// DMA. Block j's K and V tiles go to K slot j % 4 and V slot j % 4; the
// batch of block j < N is issued in phase 2(j - 2) by every wave (its share
// of the tile's 1 KB instructions). Both slots held block j - 4, last read
// in phase 2j - 7 (K) and 2j - 5 (V). The wait at the end of phase 2m + 1
// leaves only the batch of block m + 2 in flight (none once m + 2 >= N), so
// block m + 1 (K read from phase 2m + 2) has landed; V of block m was
// waited for a pair earlier. The pool offset of block j comes from a
// 64-block window of per-lane offsets (one table read per lane every 64
// blocks) by readlane; the first window's page ids and Q are read before
// the item's cache length arrives (guessing a full cache for the first key).
// After M(N) no DMA is in flight and nothing reads the K ring: each wave
// stages its output rows there right away (group A's during group B's
// M(N)).
// The loads are issued by inline assembly: the compiler then neither sees
// them as LDS writes (it would otherwise wait for every outstanding DMA
// before each transposing LDS read) nor counts them; the explicit waits here
// are the only ones they need, and the compiler's own vmcnt waits stay
// correct because loads retire in order.
//
// Operand addresses. Each lane keeps the LDS address of its K operand for
// every k-step and of its V^T reads for every O^T tile (the chunks are
// XOR-swizzled per row, so they differ per lane); the main loops are unrolled
// over the four ring slots, so every other part of an address (slot, S^T
// tile, PV k-step) is an immediate offset of the LDS read.
//
// Q is loaded and O stored with non-temporal hints: each is touched once,
// while the K/V blocks of (b, h) are read again by its other query tiles
// from the L2. A program with another work item to come prefetches that
// item's Q rows into the L2 before its last blocks (after the four-block
// main loop), so that the next item's Q loads do not queue at HBM behind
// those of every other program, and stores an item's output rows once the
// next item's first block has landed (the deferred output rows below), so
// that the next item's first waits do not wait for those stores.
#pragma once
#include <utility>

#include "fmha_kernel.h"

namespace fgw_mha {

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>) in order,
// fully unrolled whatever the size of the body (a plain loop under
// "#pragma unroll" may stay a loop when the body is large, and register
// arrays indexed by its counter then move to scratch memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <bool BF16_, int DPAD_>
struct PCfg {
  static constexpr bool BF16 = BF16_;
  static constexpr int DPAD = DPAD_;
  static constexpr int LAYOUT = kLayoutPrefill;
  static constexpr int NWQ = 8;  // waves along query rows; all share each K/V block
  static constexpr int NWK = 1;
  static constexpr int BN = 64;  // keys per block
  static constexpr int WAVES = NWQ;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS_WAVE = 32;
  static constexpr int ROWS_TILE = ROWS_WAVE * NWQ;
  static constexpr int KK = DPAD / 16;  // QK k-steps
  static constexpr int DT = DPAD / 32;  // O^T row tiles
  static constexpr int ST = BN / 32;    // S^T tiles per block
  static constexpr int KS = BN / 16;    // PV k-steps
  static constexpr int CPR = DPAD / 8;  // 16-byte chunks per LDS row
  static constexpr int ROW_BYTES = DPAD * 2;
  static constexpr int TILE_BYTES = BN * ROW_BYTES;
  static constexpr int NKSLOT = 4;
  static constexpr int NVSLOT = 4;
  static constexpr int RING_BYTES = (NKSLOT + NVSLOT) * TILE_BYTES;
  // After the rings: 1 KB per wave that the L2 prefetch of the next work
  // item's Q rows writes and nothing reads.
  static constexpr int LDS_BYTES = RING_BYTES + 1024 * WAVES;
  static constexpr int INSTR = TILE_BYTES / 1024;  // DMA instructions per tile
  static constexpr int INSTR_PER_WAVE = INSTR / NWQ;
  static constexpr int BATCH = 2 * INSTR_PER_WAVE;  // per wave: its share of one K and one V tile
  static constexpr int KSW = CMin<16, CPR>::value;
  static constexpr int VSW = CPR / 4;
  static constexpr int RPI = 64 / CPR;
  static_assert(DPAD == 64 || DPAD == 128, "prefill layout head-dim tiles");
  static_assert(NKSLOT == 4 && NVSLOT == 4, "matrix phases take slots n % 4");
  static_assert(INSTR % NWQ == 0 && INSTR_PER_WAVE >= 1, "DMA granularity");
  static_assert(LDS_BYTES <= kLdsBudget, "LDS budget of one CU");
};

// Page id of the page holding the first key of block j of a work item
// (keys key0 + j BN ..), clamped to the table: the read does not depend on
// len, so it can be issued before len is known. Evaluated per lane.
template <class C>
__device__ __forceinline__ int32_t block_page_id(const FwdParams& p, const int32_t* table_b,
                                                 int key0, int j) {
  const u32 pg = div_page((u32)key0 + (u32)j * C::BN, p.page_magic, p.page_shift);
  const u32 last = (u32)p.width - 1u;
  return table_b[pg < last ? pg : last];
}

// Pool byte offset (row * row_bytes) of the first key row of block j of a
// work item, from the page id of its first key (block_page_id), or -1 when
// the block needs the per-key path (it straddles a page or len, leaves the
// pool, or D < DPAD). Blocks j >= N are never loaded and read -1.
template <class C>
__device__ __forceinline__ int64_t block_offset_of(const FwdParams& p, int32_t id,
                                                   int64_t row_bytes, int key0, int N, int len,
                                                   int j) {
  const u32 page = (u32)p.page_size;
  const u32 pos0 = (u32)key0 + (u32)j * C::BN;
  const u32 pg0 = div_page(pos0, p.page_magic, p.page_shift);
  const u32 off0 = pos0 - pg0 * page;
  const int64_t row0 = (int64_t)id * page + off0;
  const bool fast = j < N && off0 + C::BN <= page && (int64_t)pos0 + C::BN <= len && row0 >= 0 &&
                    row0 + C::BN <= p.pool_rows && p.dim == C::DPAD;
  return fast ? row0 * row_bytes : -1;
}

template <class C>
__device__ __forceinline__ int64_t block_offset(const FwdParams& p, const int32_t* table_b,
                                                int64_t row_bytes, int key0, int N, int len,
                                                int j) {
  return block_offset_of<C>(p, block_page_id<C>(p, table_b, key0, j), row_bytes, key0, N, len, j);
}

// Offsets of blocks [64 w, 64 w + 64) of a work item, one per lane (lane l:
// block 64 w + l).
struct BlockWindow {
  int w;
  int64_t off;
};

__device__ __forceinline__ int64_t readlane64(int64_t x, int lane) {
  const u32 lo = __builtin_amdgcn_readlane((u32)x, lane);
  const u32 hi = __builtin_amdgcn_readlane((u32)((uint64_t)x >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// DMA of the K (IS_V false) or V tile of keys [pos0, pos0 + BN) of (b, h)
// when the block is not in the fast case: every key row is resolved through
// the table and masked chunks (key >= len, d >= D, page id outside the
// pool) read the zero chunk. Instruction q of the wave fills LDS
// [dst + 1024 i, + 1024) with i = q * NWQ + wave.
template <class C, bool IS_V>
__device__ __forceinline__ void issue_slow_tile(const FwdParams& p, const int32_t* table_b,
                                                const char* base, int64_t row_bytes, int pos0,
                                                int len, u32 dst, int wave, int lane) {
  const u32 page = (u32)p.page_size;
  const int dim = opaque_uniform(p.dim);
  lane = opaque_lane(lane);
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
    const char* src = live && c * 8 < dim ? base + row * row_bytes + c * 16 : zero;
    dma_flat(src, dst + 1024u * i);
  }
}

// The wave's share of the K and V tiles of one block in the fast case (the
// block lies in one page, below len, inside the pool, with D == DPAD):
// uniform tile bases plus the wave's fixed per-lane offsets.
// Per-lane byte offsets of the wave's DMA instructions from a block's first
// row: the chunk offsets of DmaLanes plus the instruction's first row
// (RPI i rows), so that every instruction of a block shares one uniform base.
template <class C>
struct BlockDma {
  u32 k[C::INSTR_PER_WAVE], v[C::INSTR_PER_WAVE];
  __device__ __forceinline__ BlockDma(const DmaLanes<C>& dl, int wave, int64_t row_bytes) {
#pragma unroll
    for (int q = 0; q < C::INSTR_PER_WAVE; ++q) {
      const u32 rows = (u32)((int64_t)(C::RPI * (q * C::NWQ + wave)) * row_bytes);
      k[q] = dl.kq(q, wave) + rows;
      v[q] = dl.vq(q, wave) + rows;
    }
  }
};

template <class C>
__device__ __forceinline__ void issue_fast_block(const char* kbase, const char* vbase, u32 kdst,
                                                 u32 vdst, const BlockDma<C>& bd, int wave) {
  // Instruction q of the wave fills 1 KB number q NWQ + wave of each tile.
  const u32 kw = kdst + 1024u * (u32)wave, vw = vdst + 1024u * (u32)wave;
#pragma unroll
  for (int q = 0; q < C::INSTR_PER_WAVE; ++q) {
    dma_saddr(kbase, bd.k[q], kw + 1024u * (u32)(q * C::NWQ));
    dma_saddr(vbase, bd.v[q], vw + 1024u * (u32)(q * C::NWQ));
  }
}

// Per-lane LDS byte addresses of the MFMA A operands, ring bases included:
//   K (k-step kk):  kring + k_base + 32 (kk ^ ky)          (+ slot, + 32 t rows)
//   V (O^T tile dt): vring + v_base + 64 (dt ^ vy)         (+ slot, + 16 k2 rows)
// The row parts are compile-time constants of the matrix phase and so is the
// slot in the unrolled main loops, so there every operand read is one of
// these registers plus an immediate offset.
template <class C>
struct OperandAddr {
  u32 k[C::KK];
  u32 v[C::DT];
  __device__ __forceinline__ OperandAddr(const Lanes<C>& ln, u32 kring, u32 vring) {
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) k[kk] = kring + (u32)(ln.k_base + 32 * (kk ^ ln.ky));
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) v[dt] = vring + (u32)(ln.v_base + 64 * (dt ^ ln.vy));
  }
};

typedef __attribute__((address_space(3))) unsigned char lds_byte;

__device__ __forceinline__ lds_byte* lds_at(u32 addr) { return (lds_byte*)(uintptr_t)addr; }

// Matrix phase of one wave with block n's K tile in K slot KSLOT and block
// n - 1's V tile in V slot (KSLOT + 3) % 4: O^T += V^T P^T, then S^T = K Q^T.
// One sequence of DT KS + ST KK MFMAs, each operand read from LDS AH
// operands ahead. The MFMAs that accumulate into one tile follow each other
// (o[0] over its KS steps, then o[1], ...; s[0] over its KK steps, then
// s[1]): the matrix core takes the accumulator of a dependent MFMA of the
// same shape straight from the previous one, which leaves more of the
// register file to the softmax wave of the SIMD (a ping-pong microbenchmark:
// 1484 against 1544 cycles per phase with the tiles interleaved). Each tile
// sums its steps in the same order either way.
template <class C, bool PV, bool QK>
__device__ __forceinline__ void matrix_phase(const OperandAddr<C>& ad, u32 koff, u32 voff,
                                             const u32x4 (&qf)[C::KK],
                                             const u32x4 (&pf)[C::KS], f32x16 (&s)[C::ST],
                                             f32x16 (&o)[C::DT]) {
  using E = Elem<C::BF16>;
  // Operand i of the sequence: PV steps first (when PV), then QK^T steps (when QK).
  constexpr int NPV = PV ? C::DT * C::KS : 0, NQK = QK ? C::ST * C::KK : 0, NOP = NPV + NQK;
  constexpr int AH = NOP < 7 ? NOP : 7;
  // Operand i: PV step (dt = i / KS, k2 = i % KS) for i < NPV, else QK^T step
  // (t = (i - NPV) / KK, kk = (i - NPV) % KK).
  auto rd = [&](auto ic) -> u32x4 {
    constexpr int i = decltype(ic)::value;
    if constexpr (i < NPV) {
      constexpr int dt = i / C::KS, k2 = i % C::KS;
      lds_byte* va = lds_at(ad.v[dt]) + voff + 16 * k2 * C::ROW_BYTES;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)va);
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(va + 8 * C::ROW_BYTES));
      const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
      return u32x4{lo2.x, lo2.y, hi2.x, hi2.y};
    } else {
      constexpr int t = (i - NPV) / C::KK, kk = (i - NPV) % C::KK;
      return *(const __attribute__((address_space(3))) u32x4*)(lds_at(ad.k[kk]) + koff +
                                                               t * 32 * C::ROW_BYTES);
    }
  };
  if constexpr (QK) {
#pragma unroll
    for (int t = 0; t < C::ST; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[t][v] = 0.0f;
  }
  u32x4 a[AH + 1];
  // The wave of the SIMD that runs the softmax would otherwise take every
  // VALU issue cycle it can and hold back these MFMAs; at the higher
  // priority each MFMA issues as soon as the matrix core is free.
  __builtin_amdgcn_s_setprio(2);
  static_for<AH>([&](auto ic) { a[decltype(ic)::value] = rd(ic); });
  __builtin_amdgcn_sched_barrier(0);
  static_for<NOP>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if constexpr (i + AH < NOP) a[(i + AH) % (AH + 1)] = rd(std::integral_constant<int, i + AH>{});
    if constexpr (i < NPV) {
      o[i / C::KS] = E::mma(a[i % (AH + 1)], pf[i % C::KS], o[i / C::KS]);
    } else {
      constexpr int t = (i - NPV) / C::KK, kk = (i - NPV) % C::KK;
      s[t] = E::mma(a[i % (AH + 1)], qf[kk], s[t]);
    }
    // Fence: the machine scheduler would otherwise sink each read next to
    // its MFMA (fewer live registers) and expose the full LDS latency.
    __builtin_amdgcn_sched_barrier(0);
  });
  __builtin_amdgcn_s_setprio(0);
}

// Scores of keys at or beyond the lane's visible count become -inf: element
// (t, v) holds key pos0 + 4 (lane / 32) + 32 t + 8 (v / 4) + v % 4, masked
// when 32 t + 8 (v / 4) + v % 4 >= lim = vis - 4 (lane / 32) - pos0.
// Each compare feeds its select right away (the fence): the compiler would
// otherwise issue all 32 compares first and hold their lane masks in 64
// scalar registers, which made the kernel spill scalars around the main loop.
template <class C>
__device__ __forceinline__ void mask_from(f32x16 (&s)[C::ST], int lim) {
#pragma unroll
  for (int t = 0; t < C::ST; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int idx = 32 * t + 8 * (v >> 2) + (v & 3);
      s[t][v] = idx >= lim ? -INFINITY : s[t][v];
      __builtin_amdgcn_sched_barrier(0);
    }
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void prefill_kernel(FwdParams p_arg,
                                                             const int32_t* __restrict__ table,
                                                             const int32_t* __restrict__ lengths) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::LDS_BYTES];
  unsigned char* const kring = smem;
  // The V ring's address from the K ring's (a generic pointer would be
  // null-checked at every use).
  const u32 kring_lds = lds_address(kring);
  const u32 vring_lds = kring_lds + (u32)(C::NKSLOT * C::TILE_BYTES);

  // The parameters. The work items read them again from the kernel argument
  // segment (p_arg is its first argument, at offset 0) through a pointer the
  // compiler cannot follow: it then loads what each item and each output
  // store needs where they need it, instead of holding every parameter (and
  // what it derives from them) in scalar registers across the main loop.
  const FwdParams& p = p_arg;
  auto kernarg = []() {
    typedef const __attribute__((address_space(4))) FwdParams* KP;
    KP kp = (KP)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kp));
    return (const FwdParams*)kp;
  };
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int il = lane & 31, hh = lane >> 5;
  const Lanes<C> ln(lane);
  const int64_t row_bytes = (int64_t)p.heads * p.dim * 2;
  const DmaLanes<C> dl(lane, wave, row_bytes);
  const BlockDma<C> bd(dl, wave, row_bytes);

  // Work items: the programs of one XCD (hardware: workgroup i runs on XCD
  // i % 8) share one contiguous range of the items, interleaved: program
  // `local` of the XCD takes items a + local, a + local + nx, ... So at any
  // time the XCD's CUs work on neighbouring items (the query tiles of one
  // (b, h)), whose K/V its L2 then holds once. With one item per program
  // this is the plain contiguous assignment.
  const int grid = gridDim.x;
  const int xcd = (int)blockIdx.x % kNumXcd, local = (int)blockIdx.x / kNumXcd;
  const int q8 = grid / kNumXcd, r8 = grid % kNumXcd;
  const int nx = q8 + (xcd < r8 ? 1 : 0);           // programs on this XCD
  const int sx = xcd * q8 + (xcd < r8 ? xcd : r8);  // first of them in program order
  const int per = p.work / grid, rem = p.work % grid;
  const int a = sx * per + (sx < rem ? sx : rem);
  const int end = (sx + nx) * per + (sx + nx < rem ? sx + nx : rem);
  const int count = local < end - a ? (end - a - local + nx - 1) / nx : 0;
  const int capacity = p.width * p.page_size;

  // Work item w: (b, h, query tile qt, split of nsplit).
  auto decode = [&](const FwdParams& p, int w, int& b, int& h, int& qt, int& split,
                    int& nsplit) {
    nsplit = p.splits;
    if (p.split_keys > 0) {
      // Tile-balanced causal plan: the items of one (b, h) are contiguous
      // (a program's range, and with the XCD remap one XCD's, shares its K/V
      // in L2), its tiles from the last (heaviest) one, tile t in
      // tile_slots(t) splits.
      int per_bh = 0;
      for (int t = 0; t < p.q_tiles; ++t)
        per_bh += tile_slots(t, p.sq, capacity, C::ROWS_TILE, p.split_keys, p.splits);
      const int bh = w / per_bh;
      int r = w - bh * per_bh, t = p.q_tiles - 1, n = 1;
      for (;; --t) {
        n = tile_slots(t, p.sq, capacity, C::ROWS_TILE, p.split_keys, p.splits);
        if (r < n || t == 0) break;
        r -= n;
      }
      split = r;
      nsplit = n;
      qt = t;
      h = bh % p.heads;
      b = bh / p.heads;
    } else {
      split = w % p.splits;
      w /= p.splits;
      // Causal tiles: the last (heaviest) first, so that a dispatcher or a
      // persistent program starts the long work items early.
      qt = p.causal ? p.q_tiles - 1 - w % p.q_tiles : w % p.q_tiles;
      w /= p.q_tiles;
      h = w % p.heads;
      b = w / p.heads;
    }
  };

  // Deferred output rows. A wave's last stores of an item would sit in the
  // vector memory counter ahead of the next item's loads and DMA (the
  // counter retires loads and stores in issue order), so the next item's
  // first waits would wait for them too. When another item follows, a wave
  // with all 32 of its rows in bf16/fp16 output stages them, keeps them in
  // dfr and stores them once the next item's Q and block 0 have landed,
  // ahead of the DMA of its block 2; the wait for block 1 leaves them in
  // flight, and the wait for block 2 (or the last one) covers them. The
  // stores name the global address space: as flat stores they would also
  // count in the LDS counter, which every barrier waits for. The address and
  // step are held per lane, and a zero step means nothing pending.
  constexpr int kRowChunks = C::DPAD * 2 / 16, kRowsPerStore = 64 / kRowChunks;
  constexpr int kDefer = kStagedChunks<C>;  // stores per lane
  u32x4 dfr[kDefer];
  uint64_t dfr_addr = 0;
  int dfr_step = 0;
  typedef __attribute__((address_space(1))) u32x4 GlobalChunk;
  auto store_deferred = [&]() {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < kDefer; ++k)
      __builtin_nontemporal_store(
          dfr[k], (GlobalChunk*)(dfr_addr + (uint64_t)(int64_t)(k * dfr_step)));
    asm volatile("" ::: "memory");
    dfr_step = 0;
  };
  auto dfr_pending = [&]() { return __builtin_amdgcn_readfirstlane(dfr_step) != 0; };

  for (int it = 0; it < count; ++it) {
    const FwdParams p = *kernarg();  // this item's copy (shadows the prologue's reference)
    const bool group_a = opaque_uniform(wave) < C::WAVES / 2;
    int split, nsplit, qt, h, b;
    decode(p, a + local + nx * it, b, h, qt, split, nsplit);
    const int32_t* table_b = table + (int64_t)b * p.width;
    const char* kb = static_cast<const char*>(p.k) + (int64_t)h * p.dim * 2;
    const char* vb = static_cast<const char*>(p.v) + (int64_t)h * p.dim * 2;
    const int q0 = qt * C::ROWS_TILE;
    const int row_base = q0 + wave * C::ROWS_WAVE;
    const int qrow = row_base + il;

    const int tile_last = (q0 + C::ROWS_TILE < p.sq ? q0 + C::ROWS_TILE : p.sq) - 1;
    // The item's first key block, given its cache length.
    auto first_block = [&](int n) {
      int mv = p.causal ? n - p.sq + tile_last + 1 : n;
      mv = mv < 0 ? 0 : (mv > n ? n : mv);
      return (int)((int64_t)((mv + C::BN - 1) / C::BN) * split / nsplit);
    };
    // Issued before len is known, so that the round trips overlap: the page
    // ids of the first 64-block window for a full cache (read again below if
    // len moves the item's first key; split 0 always starts at key 0), then
    // Q^T (B of the QK^T product). Q is read once: non-temporal loads, which
    // leave the L2 to the K/V blocks that the other query tiles of (b, h)
    // read again.
    const int key0_full = first_block(capacity) * C::BN;
    int32_t id_first = block_page_id<C>(p, table_b, key0_full, lane);
    u32x4 qf[C::KK];
    // A program's first item, a whole query tile at D == DPAD, reads Q
    // through LDS (below, after the item-top barrier); the others load their
    // rows straight into registers (from the L2, after the prefetch).
    const bool q_lds = it == 0 && q0 + C::ROWS_TILE <= p.sq && p.dim == C::DPAD;
    if (!q_lds) {
      const int dim = opaque_uniform(p.dim), hq = opaque_lane(hh);
      const u16* qp =
          static_cast<const u16*>(p.q) + (((int64_t)b * p.sq + qrow) * p.heads + h) * p.dim;
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) {
        const int d = 16 * kk + 8 * hq;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (qrow < p.sq && d < dim)
          val = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(qp + d));
        qf[kk] = val;
      }
    }

    int len = lengths[b];
    len = len < 0 ? 0 : (len > capacity ? capacity : len);
    int max_vis = p.causal ? len - p.sq + tile_last + 1 : len;
    max_vis = max_vis < 0 ? 0 : (max_vis > len ? len : max_vis);
    const int nblk = (max_vis + C::BN - 1) / C::BN;
    const int blk_begin = (int)((int64_t)nblk * split / nsplit);
    const int blk_end = (int)((int64_t)nblk * (split + 1) / nsplit);
    const int N = blk_end - blk_begin;
    const int key0 = blk_begin * C::BN;

    // Rows of this wave and their visible key counts; blocks that end above
    // wmin hold keys some row of the wave cannot see and are masked.
    int wmin = p.causal ? len - p.sq + row_base + 1 : len;
    wmin = wmin < 0 ? 0 : (wmin > len ? len : wmin);
    int vis = p.causal ? len - p.sq + qrow + 1 : len;
    vis = vis < 0 ? 0 : (vis > len ? len : vis);

    float m = kNegBig, l = 0.0f;
    f32x16 o[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[dt][v] = 0.0f;

    // Output of this wave's rows: O/l of the work item, or the partial
    // (O/l, LSE) of its split. With D == DPAD the rows go out through LDS,
    // each wave through its own 32 * kStagedRowBytes bytes from the start of
    // the rings; the caller guarantees that no DMA writes and no wave reads
    // that region meanwhile. kStageInK: the eight regions lie in the K ring
    // (head-dim tile 128; at 64 the upper four reach into the V ring).
    constexpr bool kStageInK = C::WAVES * 32 * kStagedRowBytes<C> <= C::NKSLOT * C::TILE_BYTES;
    auto store_output = [&]() {
      // The output's parameters come from the kernel arguments again here,
      // so that none of them is held in a register across the main loop.
      const FwdParams po = *kernarg();
      // Partials, unless a one-split tile of a tile-balanced whole call
      // writes its output rows directly.
      const bool to_parts = po.mode == 1 && !(po.split_direct && nsplit == 1);
      const int ho = opaque_lane(hh), qr = row_base + opaque_lane(il);
      const float tot = pair_sum(l);
      if (po.dim == C::DPAD) {
        static_assert(C::WAVES * 32 * kStagedRowBytes<C> <= C::RING_BYTES, "staged rows fit");
        const bool f32 = to_parts;
        float* fdst = f32 ? po.parts + ((((int64_t)b * po.heads + h) * po.splits + split) * po.sq +
                                        row_base) *
                                           C::DPAD
                          : nullptr;
        unsigned char* bdst =
            f32 ? nullptr
                : static_cast<unsigned char*>(po.out) +
                      (((int64_t)b * po.sq + row_base) * po.heads + h) * C::DPAD * 2;
        if (!f32 && it + 1 < count && po.sq - row_base >= 32) {
          // All 32 rows of the wave, and another item follows: stored by
          // that item once its Q and block 0 have landed.
          unsigned char* st = smem + wave * 32 * kStagedRowBytes<C>;
          write_staged_bf16<C>(st, opaque_lane(il), ho, o, 1.0f / fmaxf(tot, 1.0e-30f));
          const int ln = opaque_lane(lane);
#pragma unroll
          for (int k = 0; k < kDefer; ++k) dfr[k] = read_staged_bf16<C>(st, ln, k);
          const int stride = po.heads * C::DPAD * 2;
          dfr_addr = (uint64_t)(uintptr_t)bdst +
                     (uint64_t)(int64_t)((ln / kRowChunks) * stride) + 16u * (ln % kRowChunks);
          dfr_step = opaque_lane(kRowsPerStore * stride);
        } else {
          store_rows_staged<C>(smem + wave * 32 * kStagedRowBytes<C>, lane, o,
                               1.0f / fmaxf(tot, 1.0e-30f), f32, fdst, bdst,
                               (int64_t)po.heads * C::DPAD * 2, po.sq - row_base);
        }
        if (to_parts && ho == 0 && qr < po.sq)
          po.lse[(((int64_t)b * po.heads + h) * po.splits + split) * po.sq + qr] = lse_of(m, tot);
      } else if (qr < po.sq) {
        const float inv = 1.0f / fmaxf(tot, 1.0e-30f);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int d0 = 32 * dt + 8 * gq + 4 * ho;
            if (d0 < po.dim) {
              f32x4 val = {o[dt][4 * gq], o[dt][4 * gq + 1], o[dt][4 * gq + 2], o[dt][4 * gq + 3]};
              store_row<C>(po, b, h, split, qr, d0, val, inv, -1, 0, to_parts ? 1 : 0);
            }
          }
        if (to_parts && ho == 0) {
          po.lse[(((int64_t)b * po.heads + h) * po.splits + split) * po.sq + qr] = lse_of(m, tot);
        }
      }
    };

    __syncthreads();  // the previous work item no longer reads or stages in the rings

    if (N > 0) {
      // Window of 64 block offsets holding the next batch's block; the
      // following window is read one window ahead.
      // Each branch consumes its own page-id load, so the common one (the
      // guess held) waits only for that load and not for Q behind it.
      const OperandAddr<C> ad_q(ln, kring_lds, vring_lds);
      BlockWindow win0{0, 0};
      if (key0 == key0_full)
        win0.off = block_offset_of<C>(p, id_first, row_bytes, key0, N, len, lane);
      else
        win0.off = block_offset<C>(p, table_b, row_bytes, key0, N, len, lane);
      BlockWindow win1{1, 0};
      // K and V of block j < N into K slot j % 4, V slot j % 4 (jslot: an
      // int, or a compile-time constant in the unrolled loops).
      auto issue_block = [&](int j, auto jslot) {
        if ((j >> 6) != win0.w) {  // uniform: the block entered the next window
          win0 = win1;
          win1 = BlockWindow{win0.w + 1, block_offset<C>(p, table_b, row_bytes, key0, N, len,
                                                         64 * (win0.w + 1) + lane)};
        }
        const int64_t off = readlane64(win0.off, j & 63);
        const u32 kdst = kring_lds + (u32)((int)jslot * C::TILE_BYTES);
        const u32 vdst = vring_lds + (u32)((int)jslot * C::TILE_BYTES);
        if ((int32_t)((uint64_t)off >> 32) >= 0) {  // off >= 0 as a scalar compare
          issue_fast_block<C>(kb + off, vb + off, kdst, vdst, bd, wave);
        } else {
          int pos0 = key0 + j * C::BN;
          asm volatile("" : "+s"(pos0));  // no per-block induction variables for the rare path
          issue_slow_tile<C, false>(p, table_b, kb, row_bytes, pos0, len, kdst, wave, lane);
          issue_slow_tile<C, true>(p, table_b, vb, row_bytes, pos0, len, vdst, wave, lane);
        }
      };
      // Wait until block j has landed, the batch of block j + 1 (issued
      // after it when j + 1 < N) possibly still in flight.
      auto wait_block = [&](int j) {
        if (j + 1 < N)
          wait_vm<C::BATCH>();
        else
          wait_vm<0>();
      };
      // L2 prefetch of the next item's Q rows, issued by every wave after the
      // four-block main loop, before the remaining blocks: one LDS DMA per
      // wave (into its scratch kilobyte after the rings) whose 64 lanes touch
      // the 64 lines of the wave's next Q rows, so that the next item's Q
      // loads hit L2 instead of queueing at HBM behind those of every other
      // program. The first remaining body's wait leaves it in flight behind
      // that body's batch; the next wait covers it.
      const bool pf_on = it + 1 < count;
      auto prefetch = [&]() {
        const FwdParams& p = *kernarg();
        int bn, hn, qtn, splitn, nsplitn;
        decode(p, a + local + nx * (it + 1), bn, hn, qtn, splitn, nsplitn);
        const int row = qtn * C::ROWS_TILE + wave * C::ROWS_WAVE + il;
        const int rc = row < p.sq ? row : p.sq - 1;
        const char* addr = static_cast<const char*>(p.q) +
                           (((int64_t)bn * p.sq + rc) * p.heads + hn) * p.dim * 2 +
                           (hh * 128 < p.dim * 2 ? hh * 128 : 0);
        dma_flat(addr, kring_lds + (u32)(C::RING_BYTES + 1024 * wave));
      };
      // The wait at the end of body(n): block n + 1 has landed. After the
      // prefetch (pf_wait) the batch of block n + 2, when there is one, and
      // the prefetch may stay in flight.
      auto wait_body = [&](int n, bool pf_wait) {
        if (!pf_wait)
          wait_block(n + 1);
        else if (n + 2 < N)
          wait_vm<C::BATCH + 1>();
        else
          wait_vm<1>();
      };
      constexpr std::integral_constant<int, 0> s0{};
      constexpr std::integral_constant<int, 1> s1{};
      constexpr std::integral_constant<int, 2> s2{};
      constexpr std::integral_constant<int, 3> s3{};
      // Q through LDS: its four 64-row tiles in the way of K tiles (the rows
      // of Q and of the pool have the same stride, H D elements: 4 full rows
      // per instruction instead of 32 B of 32 rows), into K slots 2, 3 and V
      // slots 2, 3, which blocks 2 and 3 fill only after the barrier before
      // M(0); each wave then reads its 32 rows with the K operand addresses.
      if (q_lds) {
        // (opaque copies: nothing of this once-per-program path is held
        // across the main loop)
        const int wv = opaque_uniform(wave);
        int64_t rb = row_bytes;
        asm volatile("" : "+s"(rb));
        const int64_t tile_q = 64 * rb;
        const char* qb = static_cast<const char*>(p.q) +
                         (((int64_t)b * p.sq + q0) * p.heads + h) * p.dim * 2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32 dst = (j < 2 ? kring_lds : vring_lds) + (u32)((2 + (j & 1)) * C::TILE_BYTES) +
                          1024u * (u32)wv;
#pragma unroll
          for (int q = 0; q < C::INSTR_PER_WAVE; ++q)
            dma_saddr(qb + j * tile_q, bd.k[q], dst + 1024u * (u32)(q * C::NWQ));
        }
      }
      issue_block(0, s0);
      if (1 < N) issue_block(1, s1);
      const bool dfr_now = dfr_pending();
      if (q_lds) {
        // Q has landed (its loads are older than blocks 0 and 1), in every
        // wave.
        if (1 < N)
          wait_vm<2 * C::BATCH>();
        else
          wait_vm<C::BATCH>();
        __syncthreads();
        const int wv = opaque_uniform(wave), j = wv >> 1, t = wv & 1;
        const u32 off = (u32)((j < 2 ? 2 + j : 6 + (j - 2)) * C::TILE_BYTES + t * 32 * C::ROW_BYTES);
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk)
          qf[kk] = *(const __attribute__((address_space(3))) u32x4*)(lds_at(ad_q.k[kk]) + off);
      }

      win1.off = block_offset<C>(p, table_b, row_bytes, key0, N, len, 64 + lane);
      // The wait for block 1, with the deferred stores (issued after block
      // 0's wait) in flight behind it.
      auto wait_block1 = [&]() {
        asm volatile("" ::: "memory");
        if (!dfr_now)
          wait_block(1);
        else if (2 < N)
          wait_vm<C::BATCH + kDefer>();
        else
          wait_vm<kDefer>();
      };
      wait_block(0);
      // Q has landed too (its register loads are older than block 0's; its
      // LDS reads, on the LDS path, complete here). The empty assembly makes
      // the compiler wait for them here, once, instead of
      // before the first QK^T MFMA of every matrix phase, where its vmcnt(0)
      // would also wait for the DMA batch in flight.
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) asm volatile("" ::"v"(qf[kk]));
      // The deferred stores go out after the compiler's wait for Q (above),
      // which would otherwise cover them too.
      if (dfr_now) store_deferred();
      __syncthreads();

      f32x16 s[C::ST];
      u32x4 pf[C::KS];

      // M(n): PV of block n - 1 (V slot (n + 3) % 4), QK^T of block n (K slot
      // n % 4); M(0) skips the PV and M(N) the QK^T. slot = n % 4.
      const OperandAddr<C> ad(ln, kring_lds, vring_lds);
      auto mphase = [&](auto slot, auto pv, auto qk) {
        const u32 ks = (u32)((int)slot * C::TILE_BYTES);
        const u32 vs = (u32)((((int)slot + 3) & 3) * C::TILE_BYTES);
        matrix_phase<C, decltype(pv)::value, decltype(qk)::value>(ad, ks, vs, qf, pf, s, o);
      };
      constexpr std::true_type on{};
      constexpr std::false_type off{};
      const int vis4 = vis - 4 * hh;
      // S(n): softmax of block n.
      auto sphase = [&](int n) {
        int pos0 = key0 + n * C::BN;
        if (pos0 + C::BN > wmin) {
          asm volatile("" : "+s"(pos0));  // no per-block induction variables for the rare mask
          mask_from<C>(s, vis4 - pos0);
        }
        online_softmax<C>(s, m, l, o, p.scale_log2, pf);
      };
      // Group A: M(n) in phase 2n, S(n) in phase 2n + 1. Group B: S(n - 1)
      // in phase 2n, M(n) in phase 2n + 1. Every wave issues its share of
      // block n + 2 (when it exists) at the start of phase 2n and, at the
      // end of phase 2n + 1, waits until block n + 1 has landed. After the
      // barrier that ends phase 2N - 1 no DMA is in flight and no wave reads
      // the K ring any more (M(N) reads V only): each wave then stages its
      // output rows in its region of the K ring right after its last matrix
      // phase, group A's during group B's M(N) (when the regions lie in the
      // K ring; else after one more barrier). Straight-line loops per group
      // keep the register assignment of O, S and P fixed across phases; both
      // groups pass the same number of barriers. The main loops run four
      // blocks per iteration (n = 1 mod 4 at its top), so that the ring slots
      // of every LDS read and DMA are compile-time constants; the remaining
      // blocks take the general body.
      if (group_a) {
        auto body = [&](int n, auto slot, bool pf_wait = false) {
          if (n + 2 < N) issue_block(n + 2, ((int)slot + 2) & 3);
          mphase(slot, on, on);
          __syncthreads();
          sphase(n);
          wait_body(n, pf_wait);
          __syncthreads();
        };
        if (2 < N) issue_block(2, s2);
        mphase(s0, off, on);
        __syncthreads();
        sphase(0);
        wait_block1();
        __syncthreads();
        int n = 1;
        for (; n + 4 <= N; n += 4) {
          body(n, s1);
          body(n + 1, s2);
          body(n + 2, s3);
          body(n + 3, s0);
        }
        if (pf_on) prefetch();
        const int n_rem = n;
        for (; n < N; ++n) body(n, n & 3, pf_on && n == n_rem);
        mphase(N & 3, on, off);
        __syncthreads();
        if constexpr (!kStageInK) __syncthreads();  // group B no longer reads the V ring
        store_output();
      } else {
        auto body = [&](int n, auto slot, bool pf_wait = false) {
          if (n + 2 < N) issue_block(n + 2, ((int)slot + 2) & 3);
          sphase(n - 1);
          __syncthreads();
          mphase(slot, on, on);
          wait_body(n, pf_wait);
          __syncthreads();
        };
        if (2 < N) issue_block(2, s2);
        __syncthreads();
        mphase(s0, off, on);
        wait_block1();
        __syncthreads();
        int n = 1;
        for (; n + 4 <= N; n += 4) {
          body(n, s1);
          body(n + 1, s2);
          body(n + 2, s3);
          body(n + 3, s0);
        }
        if (pf_on) prefetch();
        const int n_rem = n;
        for (; n < N; ++n) body(n, n & 3, pf_on && n == n_rem);
        sphase(N - 1);
        __syncthreads();
        mphase(N & 3, on, off);
        if constexpr (!kStageInK) __syncthreads();  // every wave's V reads are done
        store_output();
      }
    } else {
      if (dfr_pending()) store_deferred();
      store_output();
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
