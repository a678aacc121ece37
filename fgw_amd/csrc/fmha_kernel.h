// Paged multi-head attention forward for CDNA4 (gfx950).
//
// One templated kernel covers decode and long-Q prefill, FP16/BF16 and head
// dims 16..256. It computes, per work item (request b, head h, query tile,
// KV split), the online-softmax attention of the tile's query rows against
// the split's visible keys, reading K/V rows through the block table.
//
// Math follows the reference operator (operators/mha/kernels/
// mha_paged_decode_ascend_v7.py:120-205, :305-315; cube_general.py:88-157):
//   s = q.k * D^-0.5, running max m, p = exp(s - m) rounded to the input dtype
//   for the PV product, l = l*alpha + sum(p) in fp32, O = alpha*O + P.V,
//   output O / max(l, 1e-30); partial mode stores O/l and LSE = ln(l) + m.
// Static-schedule mode (query layout only) takes the work items from a host
// plan instead: each program runs its segments (task, key-block range, slot)
// and writes whole tiles to the output, cut tiles to their partial slot
// (operators/mha/static_schedule.py:8-16).
// The exponentials run as exp2 on log2(e)-prescaled scores, against an
// exponent reference m that moves only when a block's row sums leave a bound
// (online_softmax): mathematically the same O/l and LSE. The head dim is
// padded with zeros to a power of two >= 32 (as cube_general.py:31 does);
// the scale uses the true D.
//
// Data path per 64-key (prefill) or 32-key (decode) block:
//   HBM -> LDS by global_load_lds_dwordx4 (DMA, no staging registers). K and
//   V tiles are row-major [key][d] with XOR-swizzled 16-byte chunks. Lanes
//   whose chunk is masked (key >= len, d >= D, page id outside the pool) load
//   a global zero chunk instead, so loads are branch-free and unread cache
//   rows (possibly NaN) never reach the products (cube_general.py:97-109).
//   LDS -> MFMA operands by ds_read_b128 (K) and ds_read_b64_tr_b16 (V: the
//   transposing read yields V^T operand columns straight from row-major V).
//
// Matrix-core formulation (v_mfma_f32_32x32x16_{bf16,f16}, wave64):
//   S^T = K . Q^T   A = K rows from LDS, B = Q^T held in VGPRs. The 32x32
//                   accumulator gives each lane one query column (lane % 32)
//                   and 16 key rows.
//   O^T = V^T . P^T A = V^T via transposing reads, B = P^T straight from the
//                   S^T accumulator after the softmax: the 16 keys a lane
//                   holds are its B-operand k-slots once the A operand reads
//                   keys (16ks + 4*(lane/32) + 0..3) and (... + 8 + 0..3).
// Every lane owns one query row in both products: the row maximum (taken only
// when the exponent reference moves) needs one cross-half (lane ^ 32)
// exchange, and the rescale of O is lane-local.
//
// Layouts (template parameter LAYOUT):
//   kLayoutQuery: 4 waves x 32 query rows share each 64-key K/V tile in
//                 double-buffered LDS (prefill).
//   kLayoutKey:   4 waves each stream their own 32-key blocks of the same 32
//                 query rows (decode); the four partial softmax states are
//                 combined through LDS before the epilogue.
// Stages (template parameter STAGES, 0 = the default): K/V stages per key
// group. Two keep the next block's DMA in flight while a block is computed;
// the key layout's single-stage variant (head-dim tile 128) halves its LDS so
// that two workgroups share a CU, one streaming while the other waits for its
// DMA or runs its prologue and epilogue. The arithmetic is the same, so both
// variants give the same bits.
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
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

#define FGW_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegBig = -1.0e30f;  // running-max floor and empty-split LSE
constexpr float kSoftmaxSumBound = 8192.0f;  // lane row-sum bound before O/l are rescaled
constexpr int kNumXcd = 8;
constexpr int kLdsBudget = 160 * 1024;
// Largest batch of a length-balanced split plan (FwdParams::split_keys > 0):
// the per-request split prefix sums live in LDS.
constexpr int kMaxBalancedBatch = 1024;

// Source of every masked 16-byte chunk: read-only zeros in device memory.
static __device__ __attribute__((aligned(64))) const u32 kZeroChunk[16] = {0};

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
// shift == 0 encodes page == 1. Branch-free: both forms are computed and one
// is selected.
__device__ __forceinline__ u32 div_page(u32 n, u32 magic, u32 shift) {
  const u32 t = __umulhi(magic, n);
  const u32 q = (t + ((n - t) >> 1)) >> ((shift - 1u) & 31u);
  return shift ? q : n;
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

template <int A, int B>
struct CMax {
  static constexpr int value = A > B ? A : B;
};
template <int A, int B>
struct CMin {
  static constexpr int value = A < B ? A : B;
};

template <bool BF16_, int DPAD_, int LAYOUT_, int STAGES_ = 0>
struct Cfg {
  static constexpr bool BF16 = BF16_;
  static constexpr int DPAD = DPAD_;  // head dim padded to a power of two >= 32
  static constexpr int LAYOUT = LAYOUT_;
  static constexpr int NWQ = LAYOUT == kLayoutQuery ? 4 : 1;  // waves along queries
  static constexpr int NWK = LAYOUT == kLayoutQuery ? 1 : 4;  // waves along keys
  static constexpr int BN = LAYOUT == kLayoutQuery ? 64 : 32; // keys per block
  static constexpr int WAVES = NWQ * NWK;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS_WAVE = 32;
  static constexpr int ROWS_TILE = ROWS_WAVE * NWQ;
  static constexpr int KK = DPAD / 16;  // QK k-steps
  static constexpr int DT = DPAD / 32;  // O^T row tiles
  static constexpr int ST = BN / 32;    // S^T tiles per block
  static constexpr int KS = BN / 16;    // PV k-steps
  static constexpr int CPR = DPAD / 8;  // 16-byte chunks per LDS row
  static constexpr int ROW_BYTES = DPAD * 2;
  static constexpr int TILE_BYTES = BN * ROW_BYTES;  // one K or V tile
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES;
  static constexpr int NBUF =
      STAGES_ > 0 ? STAGES_ : (NWK * 2 * STAGE_BYTES <= 128 * 1024 ? 2 : 1);
  static constexpr int GROUP_BYTES = NBUF * STAGE_BYTES;
  static constexpr int TILES_BYTES = NWK * GROUP_BYTES;
  static constexpr int OSTRIDE = DPAD + 4;  // combine buffer row stride (floats)
  static constexpr int COMB_BYTES =
      NWK > 1 ? (2 * NWK * ROWS_WAVE + NWK * ROWS_WAVE * OSTRIDE) * 4 : 0;
  // Key layout: per-request split prefix sums of a length-balanced plan,
  // after the tiles and the combine buffer.
  static constexpr int PREFIX_OFF = CMax<TILES_BYTES, COMB_BYTES>::value;
  static constexpr int PREFIX_BYTES = LAYOUT == kLayoutKey ? (kMaxBalancedBatch + 1) * 4 : 0;
  static constexpr int LDS_BYTES = PREFIX_OFF + PREFIX_BYTES;
  // DMA: one wave instruction fills 1 KB (64 lanes x 16 bytes) of a tile.
  static constexpr int INSTR = TILE_BYTES / 1024;
  static constexpr int INSTR_PER_WAVE = INSTR / NWQ;
  // Chunk swizzles: row r keeps chunk c at slot c ^ x(r). K rows are read 16
  // rows at a time at one chunk column, so x spreads 16 rows over 16 slots;
  // V rows are read 4 rows x 64 bytes at a time, so x moves 64-byte spans.
  static constexpr int KSW = CMin<16, CPR>::value;  // K: x = r % KSW
  static constexpr int VSW = CPR / 4;               // V: x = 4 * (r % VSW)
  static constexpr int RPI = 64 / CPR;              // key rows per DMA instruction
  static_assert(NWQ == 1 || NWK == 1, "tiles are shared by all waves or by none");
  static_assert((DPAD & (DPAD - 1)) == 0 && DPAD >= 32 && DPAD <= 256, "head dim tile");
  static_assert(TILE_BYTES % 1024 == 0 && INSTR % NWQ == 0 && 64 % CPR == 0, "DMA granularity");
  static_assert(NBUF == 1 || NBUF == 2, "one or two K/V stages per key group");
  static_assert(LDS_BYTES <= kLdsBudget, "LDS budget of one CU");
  static_assert(kMaxBalancedBatch % 64 == 0, "balanced-split prefix scan: whole lanes");
};

// LDS DMA (global_load_lds_dwordx4) for kernels that place their own waits
// (fmha_prefill.h) is issued by inline assembly: the compiler then neither
// counts these loads nor treats them as LDS writes (it would otherwise wait
// for every outstanding DMA before each transposing LDS read), and the
// kernels wait for them explicitly with wait_vm. The compiler's own vmcnt
// waits stay correct: loads retire in order, so extra loads it does not know
// of can only make its waits stricter. fwd_kernel uses the compiler builtin.
// Byte address of a shared-memory pointer within the workgroup's LDS.
__device__ __forceinline__ u32 lds_address(const void* p) {
  return (u32)(uintptr_t)FGW_LDS(const void, p);
}

// One DMA instruction: 64 lanes x 16 bytes into LDS [lds, lds + 1024).
// `base` and `lds` are uniform across the wave; readfirstlane places them in
// SGPRs where the compiler cannot prove that by itself. The hazards the
// compiler cannot see inside the assembly are covered by nops: one wait
// state between the M0 write and the LDS DMA, and five between a VALU write
// of the base SGPRs (readfirstlane) and the load that reads them.
// The assembly clobbers M0, which the compiler uses for nothing else in these
// kernels (it does not preserve M0 across inline assembly).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ u32 uniform_u32(u32 x) { return __builtin_amdgcn_readfirstlane(x); }

// Values the compiler cannot see through (uniform, and per lane): code derived
// from them stays where it is written, in a cold branch or once per work item,
// instead of being hoisted out of the work-item loop and held in registers
// across the main loop.
__device__ __forceinline__ int opaque_uniform(int x) {
  asm volatile("" : "+s"(x));
  return x;
}
__device__ __forceinline__ int opaque_lane(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
// Uniform global base + per-lane 32-bit offset (saddr form).
__device__ __forceinline__ void dma_saddr(const void* base, u32 voff, u32 lds) {
  const uint64_t b = (uint64_t)base;
  const uint64_t ub = ((uint64_t)uniform_u32((u32)(b >> 32)) << 32) | uniform_u32((u32)b);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(ub), "s"(uniform_u32(lds))
               : "memory", "m0");
}
// Per-lane 64-bit global address.
__device__ __forceinline__ void dma_flat(const void* addr, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(addr), "s"(uniform_u32(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N vector-memory loads of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

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

// Wait for this wave's outstanding DMA loads (vmcnt = 0; lgkm and exp untouched).
__device__ __forceinline__ void wait_dma() { wait_vm<0>(); }

// Per-lane DMA offsets. Instruction i of a stage fills slots 64 i + lane:
// key row RPI i + lr (lr = lane / CPR), position pos = lane % CPR, which
// holds chunk pos ^ x(row). Because RPI i % KSW is a multiple of RPI and
// lr < RPI, x(row) = (RPI i % KSW) | lr, so the chunk is (pos ^ lr) ^ c_i with
// c_i = RPI i % KSW; likewise for V with 4 (row % VSW). Offsets are
// precomputed per instruction when a wave issues few of them, otherwise
// derived with one XOR each.
template <class C>
struct DmaLanes {
  static constexpr bool PRE = C::INSTR_PER_WAVE <= 4;
  static constexpr int NPRE = PRE ? C::INSTR_PER_WAVE : 1;
  u32 row_off;  // lr * row_bytes
  u32 kx, vx;   // 16 (pos ^ lr), 16 (pos ^ 4 (lr % VSW)), pre-XOR chunk bytes
  u32 koff[NPRE];
  u32 voff[NPRE];
  __device__ __forceinline__ DmaLanes(int lane, int wq, int64_t row_bytes) {
    const int lr = lane / C::CPR, pos = lane % C::CPR;
    row_off = (u32)(lr * row_bytes);
    kx = 16u * (u32)(pos ^ (lr % C::KSW));
    vx = 16u * (u32)(pos ^ (4 * (lr % C::VSW)));
#pragma unroll
    for (int q = 0; q < NPRE; ++q) {
      koff[q] = k(q, wq);
      voff[q] = v(q, wq);
    }
  }
  __device__ __forceinline__ u32 k(int q, int wq) const {
    const int i = q * C::NWQ + wq;
    return row_off + (kx ^ (16u * (u32)((C::RPI * i) % C::KSW)));
  }
  __device__ __forceinline__ u32 v(int q, int wq) const {
    const int i = q * C::NWQ + wq;
    return row_off + (vx ^ (64u * (u32)((C::RPI * i) % C::VSW)));
  }
  __device__ __forceinline__ u32 kq(int q, int wq) const { return PRE ? koff[PRE ? q : 0] : k(q, wq); }
  __device__ __forceinline__ u32 vq(int q, int wq) const { return PRE ? voff[PRE ? q : 0] : v(q, wq); }
};

// Issue the DMA loads of the K (IS_V false) or V tile of keys
// [pos0, pos0 + BN) of (b, h) into LDS at `dst`. Wave `wq` of the key group
// issues the instructions i = q * NWQ + wq. `id0` is the page id of the page
// holding pos0 (read ahead by the caller). A block inside one page, below
// len, with no padded dims takes the fast path: uniform row base + per-lane
// offset. Otherwise every key is resolved through the table and masked
// chunks read the zero chunk.
template <class C, bool IS_V>
__device__ __forceinline__ void issue_tile(const FwdParams& p, const DmaLanes<C>& dl,
                                           const int32_t* table_b, const char* base,
                                           int64_t row_bytes, int pos0, int32_t id0, int len,
                                           unsigned char* dst_ptr, int wq, int lane) {
  // The LDS destination through an opaque copy: the compiler would otherwise
  // precompute every instruction's destination for every stage once and
  // hold them all in scalar registers across the work-item loop.
  const u32 dst = (u32)opaque_uniform((int)lds_address(dst_ptr));
  const u32 page = (u32)p.page_size;
  const u32 pg0 = div_page((u32)pos0, p.page_magic, p.page_shift);
  const u32 off0 = (u32)pos0 - pg0 * page;
  const int64_t row0 = (int64_t)id0 * page + off0;
  const bool fast = off0 + C::BN <= page && pos0 + C::BN <= len && row0 >= 0 &&
                    row0 + C::BN <= p.pool_rows && p.dim == C::DPAD;
  if (fast) {
#pragma unroll
    for (int q = 0; q < C::INSTR_PER_WAVE; ++q) {
      const int i = q * C::NWQ + wq;
      const int64_t rb = (row0 + C::RPI * i) * row_bytes;
      const u32 off = IS_V ? dl.vq(q, wq) : dl.kq(q, wq);
      __builtin_amdgcn_global_load_lds(base + rb + off, FGW_LDS(void, (uintptr_t)(dst + 1024u * i)),
                                       16, 0, 0);
    }
    return;
  }
  const int dim = opaque_uniform(p.dim);
  lane = opaque_lane(lane);
  const char* zero = reinterpret_cast<const char*>(kZeroChunk);
  int32_t ids[C::INSTR_PER_WAVE];
#pragma unroll
  for (int q = 0; q < C::INSTR_PER_WAVE; ++q) {
    const int pos = pos0 + C::RPI * (q * C::NWQ + wq) + lane / C::CPR;
    const u32 pg = pos < len ? div_page((u32)pos, p.page_magic, p.page_shift) : 0u;
    ids[q] = table_b[pg];
  }
#pragma unroll
  for (int q = 0; q < C::INSTR_PER_WAVE; ++q) {
    const int i = q * C::NWQ + wq;
    const int r = C::RPI * i + lane / C::CPR, pos_in_row = lane % C::CPR;
    const int pos = pos0 + r;
    const u32 pg = div_page((u32)pos, p.page_magic, p.page_shift);
    const int64_t row = (int64_t)ids[q] * page + ((u32)pos - pg * page);
    const bool live = pos < len && row >= 0 && row < p.pool_rows;
    const int c = IS_V ? pos_in_row ^ (4 * (r % C::VSW)) : pos_in_row ^ (r % C::KSW);
    const char* src = live && c * 8 < dim ? base + row * row_bytes + c * 16 : zero;
    __builtin_amdgcn_global_load_lds(src, FGW_LDS(void, (uintptr_t)(dst + 1024u * i)), 16, 0, 0);
  }
}

// Per-lane LDS byte offsets of the MFMA A operands (see issue_block):
//   K: row il (+32 t), chunk 2 kk + hh at slot (2 kk + hh) ^ x, x = il % KSW
//      -> il*ROW + 16 (hh ^ (x & 1)) + 32 (kk ^ (x >> 1))
//   V: transposing read of group g = lane / 16, lane j = lane % 16:
//      row (16 ks + 8 half) + 4 (g / 2) + j / 4, dims 32 dt + 16 (g % 2) + 4 (j % 4)
//      -> vbase + (16 ks + 8 half) * ROW + 64 (dt ^ vy), vy = (4 (g / 2) + j / 4) % VSW
template <class C>
struct Lanes {
  int k_base;  // + t * 32 * ROW_BYTES + 32 * (kk ^ ky)
  int ky;      // (il % KSW) >> 1
  int v_base;  // + (16 ks + 8 half) * ROW_BYTES + 64 * (dt ^ vy)
  int vy;
  __device__ __forceinline__ explicit Lanes(int lane) {
    const int il = lane & 31, hh = lane >> 5;
    const int x = il % C::KSW;
    ky = x >> 1;
    k_base = il * C::ROW_BYTES + 16 * (hh ^ (x & 1));
    const int g = lane >> 4, j = lane & 15;
    const int vrow = 4 * (g >> 1) + (j >> 2);
    vy = vrow % C::VSW;
    v_base = vrow * C::ROW_BYTES + 32 * (g & 1) + 8 * (j & 3);
  }
};

// A operand of S^T tile t, k-step kk: 8 K elements of key row 32 t + il.
template <class C>
__device__ __forceinline__ u32x4 read_k(const unsigned char* kt, const Lanes<C>& ln, int t,
                                        int kk) {
  return *reinterpret_cast<const u32x4*>(kt + ln.k_base + 32 * (kk ^ ln.ky) +
                                         t * 32 * C::ROW_BYTES);
}

// A operand of O^T tile dt, PV k-step k2: V[16 k2 + 4 (lane/32) + {0..3, 8..11}][32 dt + lane%32]
// from two transposing reads of row-major V.
template <class C>
__device__ __forceinline__ u32x4 read_vt(const unsigned char* vt, const Lanes<C>& ln, int dt,
                                         int k2) {
  const unsigned char* va = vt + ln.v_base + 64 * (dt ^ ln.vy) + (16 * k2) * C::ROW_BYTES;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(FGW_LDS(i16x4, va));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(FGW_LDS(i16x4, va + 8 * C::ROW_BYTES));
  const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{lo2.x, lo2.y, hi2.x, hi2.y};
}

// S^T tiles of one BN-key block: s[t] = K[32 t .. 32 t + 31] . Q^T, with the
// K operands read one k-step ahead of the MFMAs that consume them.
template <class C>
__device__ __forceinline__ void qk_block(const unsigned char* kt, const Lanes<C>& ln,
                                         const u32x4 (&qf)[C::KK], f32x16 (&s)[C::ST]) {
  using E = Elem<C::BF16>;
#pragma unroll
  for (int t = 0; t < C::ST; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) s[t][v] = 0.0f;
  u32x4 a[2][C::ST];
#pragma unroll
  for (int t = 0; t < C::ST; ++t) a[0][t] = read_k<C>(kt, ln, t, 0);
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) {
    if (kk + 1 < C::KK) {
#pragma unroll
      for (int t = 0; t < C::ST; ++t) a[(kk + 1) & 1][t] = read_k<C>(kt, ln, t, kk + 1);
    }
#pragma unroll
    for (int t = 0; t < C::ST; ++t) s[t] = E::mma(a[kk & 1][t], qf[kk], s[t]);
  }
}

// Scores of keys at or beyond the lane's visible count become -inf. Each
// compare feeds its select right away (the fence), so that the compiler does
// not hold 32 lane masks in scalar registers at once.
template <class C>
__device__ __forceinline__ void mask_block(f32x16 (&s)[C::ST], int pos0, int vis, int hh) {
#pragma unroll
  for (int t = 0; t < C::ST; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = pos0 + 32 * t + 8 * (v >> 2) + 4 * hh + (v & 3);
      s[t][v] = key >= vis ? -INFINITY : s[t][v];
      __builtin_amdgcn_sched_barrier(0);
    }
}

// max / sum of x over the lane pair (lane, lane ^ 32) by v_permlane32_swap:
// a VALU exchange of the wave's halves, where a lane shuffle would go
// through the LDS crossbar and queue behind the operand reads of the wave
// that shares the SIMD. Both lanes of a pair get bit-identical results.
__device__ __forceinline__ float pair_max(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Row maximum of the block, in log2 units, over the lane pair (lane, lane ^ 32).
// Four independent chains (scores k = c mod 4; the compiler fuses pairs of
// steps into v_max3_f32), so that one wave does not wait out the latency of
// every step of a single chain. The maxima stay compiler-visible VALU
// operations: the scores are read straight from MFMA accumulators, and the
// compiler inserts the wait states that reading them requires.
template <class C>
__device__ __forceinline__ float row_max(const f32x16 (&s)[C::ST], float scale_log2) {
  constexpr int NV = 16 * C::ST;
  float acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float x = s[0][c];
#pragma unroll
    for (int k = c + 4; k < NV; k += 4) x = fmaxf(x, s[k / 16][k % 16]);
    acc[c] = x;
  }
  const float mx = fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3]));
  return pair_max(mx) * scale_log2;
}

// p = exp2(s * scale_log2 - m) packed to the input dtype as the B operands of
// the PV product (k-step 2 t + u = s[t][8 u .. 8 u + 7]); returns the lane's
// part of the row sum (fp32, four independent partial sums).
template <class C>
__device__ __forceinline__ float softmax_exp(const f32x16 (&s)[C::ST], float m, float scale_log2,
                                             u32x4 (&pf)[C::KS]) {
  using E = Elem<C::BF16>;
  const float neg_m = -m;
  float e[C::ST][16];
  float rs[4];
#pragma unroll
  for (int t = 0; t < C::ST; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      e[t][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][v], scale_log2, neg_m));
      rs[v % 4] = t == 0 && v < 4 ? e[t][v] : rs[v % 4] + e[t][v];
    }
#pragma unroll
  for (int t = 0; t < C::ST; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4 w;
      w.x = E::pack2(e[t][8 * u + 0], e[t][8 * u + 1]);
      w.y = E::pack2(e[t][8 * u + 2], e[t][8 * u + 3]);
      w.z = E::pack2(e[t][8 * u + 4], e[t][8 * u + 5]);
      w.w = E::pack2(e[t][8 * u + 6], e[t][8 * u + 7]);
      pf[2 * t + u] = w;
    }
  return (rs[0] + rs[1]) + (rs[2] + rs[3]);
}

// Online softmax of one block: P against the current exponent reference m,
// l += row sum. The reference m moves (to the block's row maximum, with O and
// l rescaled and P recomputed) only when some lane's sum exceeds
// kSoftmaxSumBound: on the first block of a row (m = -1e30) and when a block
// raises the maximum by about 8 (log2 units) or more. Otherwise no row
// maximum is taken at all. Every p <= sum <= kSoftmaxSumBound, within FP16's
// range; O/l and the LSE do not depend on m, and m never exceeds the running
// maximum, so no p underflows earlier than with m at the running maximum.
template <class C>
__device__ __forceinline__ void online_softmax(const f32x16 (&s)[C::ST], float& m, float& l,
                                               f32x16 (&o)[C::DT], float scale_log2,
                                               u32x4 (&pf)[C::KS]) {
  float rs = softmax_exp<C>(s, m, scale_log2, pf);
  if (__ballot(!(rs <= kSoftmaxSumBound))) {
    const float mn = fmaxf(m, row_max<C>(s, scale_log2));
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) o[dt] *= alpha;
    m = mn;
    rs = softmax_exp<C>(s, m, scale_log2, pf);
  }
  l += rs;
}

// O^T += V^T P^T for one block, V^T operands read one step ahead.
template <class C>
__device__ __forceinline__ void pv_block(const unsigned char* vt, const Lanes<C>& ln,
                                         const u32x4 (&pf)[C::KS], f32x16 (&o)[C::DT]) {
  using E = Elem<C::BF16>;
  constexpr int NSTEP = C::DT * C::KS;  // step j: k2 = j / DT, dt = j % DT
  u32x4 va[2];
  va[0] = read_vt<C>(vt, ln, 0, 0);
#pragma unroll
  for (int j = 0; j < NSTEP; ++j) {
    if (j + 1 < NSTEP) va[(j + 1) & 1] = read_vt<C>(vt, ln, (j + 1) % C::DT, (j + 1) / C::DT);
    o[j % C::DT] = E::mma(va[j & 1], pf[j / C::DT], o[j % C::DT]);
  }
}

// Output of one (row, 4 dims): the normalised output in mode 0 and for a
// static-schedule segment without a slot; O/l in the partial layout of mode 1
// or in the slot rows of mode 2 otherwise.
template <class C>
__device__ __forceinline__ void store_row(const FwdParams& p, int b, int h, int split, int qrow,
                                          int d0, f32x4 val, float inv, int slot = -1,
                                          int q0 = 0, int mode = -1) {
  using E = Elem<C::BF16>;
  if (mode < 0) mode = p.mode;
  if (mode == 2 && slot >= 0) {
    float* dst = p.parts + ((int64_t)slot * C::ROWS_TILE + (qrow - q0)) * p.dim + d0;
    *reinterpret_cast<f32x4*>(dst) = val * inv;
  } else if (mode != 1) {
    u16* dst = static_cast<u16*>(p.out) + (((int64_t)b * p.sq + qrow) * p.heads + h) * p.dim + d0;
    u32x2 w;
    w.x = E::pack2(val[0] * inv, val[1] * inv);
    w.y = E::pack2(val[2] * inv, val[3] * inv);
    *reinterpret_cast<u32x2*>(dst) = w;
  } else {
    float* dst = p.parts +
                 ((((int64_t)b * p.heads + h) * p.splits + split) * p.sq + qrow) * p.dim + d0;
    const f32x4 x = val * inv;
    if (p.arrivals != nullptr) {  // fused merge: coherent at the device (arrive_and_merge)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __hip_atomic_store(dst + i, x[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      *reinterpret_cast<f32x4*>(dst) = x;
    }
  }
}

// Output rows of one wave through LDS (D == DPAD >= 64). Lane (il, hh) holds
// row il's dims 32 dt + 8 gq + 4 hh + i in o[dt][4 gq + i]; stored directly,
// each store instruction scatters 8-16 bytes per lane over 32 rows. The wave
// instead writes its 32 rows into `st` (its own 32 * kStagedRowBytes<C> bytes
// of LDS, which no other wave touches meanwhile), reads them back as 16-byte
// chunks of whole rows and stores 2-8 full rows per instruction. The 16-byte
// chunk c of staged row r sits at chunk c ^ (r % chunks per row), so both
// the column writes of 32 rows and the row reads spread over all banks.
// bf16/fp16 rows (f32 false) go to bdst + r * brow_stride bytes, all DPAD
// dims in one pass, with non-temporal stores (the final output: nothing in
// the kernel reads it again); fp32 rows (f32 true, split partials that the
// merge reads back) to fdst + r * DPAD floats, 64 dims (256 bytes per row)
// per pass. Rows r >= rows are not stored.
template <class C>
constexpr int kStagedRowBytes = 2 * C::DPAD > 256 ? 2 * C::DPAD : 256;

// bf16/fp16 staging (D == DPAD): lane (il, hh) writes its part of row il,
// scaled by inv, into the wave's region `st`.
template <class C>
__device__ __forceinline__ void write_staged_bf16(unsigned char* st, int il, int hh,
                                                  const f32x16 (&o)[C::DT], float inv) {
  using E = Elem<C::BF16>;
  constexpr int RB = C::DPAD * 2, NCH = RB / 16;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int c = 4 * dt + gq;
      u32x2 w;
      w.x = E::pack2(o[dt][4 * gq] * inv, o[dt][4 * gq + 1] * inv);
      w.y = E::pack2(o[dt][4 * gq + 2] * inv, o[dt][4 * gq + 3] * inv);
      *reinterpret_cast<u32x2*>(st + il * RB + 16 * (c ^ (il % NCH)) + 8 * hh) = w;
    }
  __builtin_amdgcn_wave_barrier();
}

// 16-byte read-backs per lane for the wave's 32 staged bf16/fp16 rows.
template <class C>
constexpr int kStagedChunks = C::DPAD / 16;

// Read-back k (0 <= k < kStagedChunks) of a lane: 16-byte chunk lane % NCH
// of staged bf16/fp16 row RPI k + lane / NCH (NCH = DPAD / 8 chunks per
// row, RPI = 64 / NCH rows per instruction).
template <class C>
__device__ __forceinline__ u32x4 read_staged_bf16(const unsigned char* st, int lane, int k) {
  constexpr int RB = C::DPAD * 2, NCH = RB / 16, RPI = 64 / NCH;
  static_assert(32 / RPI == kStagedChunks<C>, "read-backs per lane");
  const int r = RPI * k + lane / NCH, c = lane % NCH;
  return *reinterpret_cast<const u32x4*>(st + r * RB + 16 * (c ^ (r % NCH)));
}

template <class C>
__device__ __forceinline__ void store_rows_staged(unsigned char* st, int lane,
                                                  const f32x16 (&o)[C::DT], float inv, bool f32,
                                                  float* fdst, unsigned char* bdst,
                                                  int64_t brow_stride, int rows) {
  static_assert(C::DPAD >= 64 && C::DPAD % 64 == 0, "staged rows need D tiles of 64k");
  // The lane id passes through an opaque copy so that the compiler cannot
  // hoist the staging addresses (functions of the lane alone) out of the
  // work-item loop, where they would stay live across the main loop.
  asm volatile("v_mov_b32 %0, %1" : "=v"(lane) : "v"(lane));
  const int il = lane & 31, hh = lane >> 5;
  if (f32) {
    constexpr int RB = 256, NCH = RB / 16, RPI = 64 / NCH;
#pragma unroll
    for (int pass = 0; pass < C::DPAD / 64; ++pass) {
#pragma unroll
      for (int dt2 = 0; dt2 < 2; ++dt2)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int dt = 2 * pass + dt2, c = 8 * dt2 + 2 * gq + hh;
          f32x4 val = {o[dt][4 * gq], o[dt][4 * gq + 1], o[dt][4 * gq + 2], o[dt][4 * gq + 3]};
          *reinterpret_cast<f32x4*>(st + il * RB + 16 * (c ^ (il % NCH))) = val * inv;
        }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int k = 0; k < 32 / RPI; ++k) {
        const int r = RPI * k + lane / NCH, c = lane % NCH;
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RB + 16 * (c ^ (r % NCH)));
        if (r < rows)
          *reinterpret_cast<u32x4*>(fdst + (int64_t)r * C::DPAD + 64 * pass + 4 * c) = v;
      }
      __builtin_amdgcn_wave_barrier();  // the next pass rewrites the region
    }
  } else {
    constexpr int NCH = C::DPAD * 2 / 16, RPI = 64 / NCH;
    write_staged_bf16<C>(st, il, hh, o, inv);
#pragma unroll
    for (int k = 0; k < kStagedChunks<C>; ++k) {
      const int r = RPI * k + lane / NCH, c = lane % NCH;
      const u32x4 v = read_staged_bf16<C>(st, lane, k);
      if (r < rows)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(bdst + r * brow_stride + 16 * c));
    }
  }
}

__device__ __forceinline__ float lse_of(float m_log2, float total) {
  return total > 0.0f ? (m_log2 + log2f(total)) * kLn2 : kNegBig;
}

// floor(nblk * s / splits): the first key block of split s (0 <= s <= splits
// <= 128). 32-bit arithmetic whenever the product fits, which avoids the
// 64-bit division routine.
__device__ __forceinline__ int split_bound(int nblk, int s, int splits) {
  if (nblk < (1 << 24)) return (int)(((u32)nblk * (u32)s) / (u32)splits);
  return (int)((int64_t)nblk * s / splits);
}

// Splits of a request of len live keys in a length-balanced plan: enough
// that none holds more than split_keys keys, at least 1, at most splits.
// Tile-balanced causal splits (prefill layout, causal, split_keys > 0): the
// key slots of query tile t are its visible keys at full table capacity
// split_keys per slot, at least one and at most `splits`, so that a long tile
// of a causal prefill is cut into work items of similar size while the short
// ones stay whole. Shared by the planner, the kernel and the merge.
__host__ __device__ __forceinline__ int tile_slots(int t, int sq, int capacity, int rows_tile,
                                                   int split_keys, int splits) {
  const int end = (t + 1) * rows_tile < sq ? (t + 1) * rows_tile : sq;
  int vis = capacity - sq + end;
  vis = vis < 0 ? 0 : (vis > capacity ? capacity : vis);
  const int n = vis > 0 ? (vis - 1) / split_keys + 1 : 1;
  return n < splits ? n : splits;
}

__device__ __forceinline__ int balanced_splits(int len, int split_keys, int splits) {
  const int s = len > 0 ? (len - 1) / split_keys + 1 : 1;
  return s < splits ? s : splits;
}

// Exclusive prefix sums of the balanced split counts over the batch, into
// pre[0 .. B] (pre[B] = total), by the first wave of the workgroup: lane l
// takes requests [16 l, 16 l + 16) (B <= 1024), the lane sums are scanned
// across the wave with shuffles, then every lane writes its requests' prefix
// sums. Every thread of the workgroup calls it (it ends with a barrier).
template <class C>
__device__ void balanced_prefix(const FwdParams& p, const int32_t* lengths, int capacity,
                                int32_t* pre, int wave, int lane) {
  if (wave == 0) {
    constexpr int kPer = kMaxBalancedBatch / 64;
    const int b0 = lane * kPer;
    int cnt[kPer];
    int local = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int b = b0 + i;
      int c = 0;
      if (b < p.batch) {
        int len = lengths[b];
        len = len < 0 ? 0 : (len > capacity ? capacity : len);
        c = balanced_splits(len, p.split_keys, p.splits);
      }
      cnt[i] = c;
      local += c;
    }
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int up = __shfl_up(incl, off, 64);
      incl += lane >= off ? up : 0;
    }
    int run = incl - local;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (b0 + i < p.batch) {
        pre[b0 + i] = run;
        run += cnt[i];
      }
    }
    if (lane == 63) pre[p.batch] = incl;
  }
  __syncthreads();
}

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
// Split state loads of a merge. COH (the fused merge): agent-scope relaxed
// atomic loads, which read the partials other XCDs' workgroups wrote with
// agent-scope stores without any cache write-back or invalidation; else
// plain loads (a separate launch sees everything the forward kernel wrote).
template <bool COH>
__device__ __forceinline__ float merge_ld1(const float* p) {
  if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}
template <bool COH>
__device__ __forceinline__ f32x4 merge_ld4(const float* p) {
  if constexpr (COH)
    return f32x4{merge_ld1<true>(p), merge_ld1<true>(p + 1), merge_ld1<true>(p + 2),
                 merge_ld1<true>(p + 3)};
  return *reinterpret_cast<const f32x4*>(p);
}

template <bool BF16, int CH, bool COH = false>
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
      x[i] = merge_ld1<COH>(ls + (int64_t)s * lse_stride);
      v[i] = merge_ld4<COH>(ps + (int64_t)s * part_stride);
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
// MAXCH < kMergeChunk leaves the 16-split chunk out (fewer registers); the
// caller then never merges more than 8 splits this way.
template <bool BF16, int MAXCH = kMergeChunk, bool COH = false>
__device__ __forceinline__ void merge_one(const float* ls, int64_t lse_stride, const float* ps,
                                          int64_t part_stride, int splits, u16* dst) {
  if (splits <= 2)
    merge_one_chunked<BF16, 2, COH>(ls, lse_stride, ps, part_stride, splits, dst);
  else if (splits <= 4)
    merge_one_chunked<BF16, 4, COH>(ls, lse_stride, ps, part_stride, splits, dst);
  else if (MAXCH <= 8 || splits <= 8)
    merge_one_chunked<BF16, 8, COH>(ls, lse_stride, ps, part_stride, splits, dst);
  else
    merge_one_chunked<BF16, kMergeChunk, COH>(ls, lse_stride, ps, part_stride, splits, dst);
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
template <bool BF16, int MAXCH = kMergeChunk, bool COH = false>
__device__ __forceinline__ void merge_rows(const float* parts, const float* lse, void* out, int sq,
                                           int heads, int dim, int slots, int used, int b, int h,
                                           int q0, int rows, int tid, int nthreads) {
  const int d4n = dim / 4;
  const int64_t bhs = ((int64_t)b * heads + h) * slots;
  for (int idx = tid; idx < rows * d4n; idx += nthreads) {
    const int q = q0 + idx / d4n, d0 = 4 * (idx % d4n);
    u16* dst = static_cast<u16*>(out) + (((int64_t)b * sq + q) * heads + h) * dim + d0;
    merge_one<BF16, MAXCH, COH>(lse + bhs * sq + q, sq, parts + (bhs * sq + q) * dim + d0,
                    (int64_t)sq * dim, used, dst);
  }
}

constexpr int kMergeThreads = 256;

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
template <int CH, bool COH = false>
__device__ __forceinline__ void wide_group(const float* ls, const float* ps, int64_t lse_stride,
                                           int64_t part_stride, int g, int G, int used,
                                           float& peak, float& tot, f32x4& acc) {
  for (int s0 = g; s0 < used; s0 += CH * G) {
    float x[CH];
    f32x4 v[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int s = s0 + i * G < used ? s0 + i * G : g;  // clamped; weight 0 below
      x[i] = merge_ld1<COH>(ls + (int64_t)s * lse_stride);
      v[i] = merge_ld4<COH>(ps + (int64_t)s * part_stride);
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

// One output row (b, h, q) of a wide merge by all kMergeThreads threads of
// a workgroup (it holds two workgroup barriers): thread t = g (D / 4) + c
// takes dims 4c .. 4c + 3 of group g's splits; speak, stot and sacc are
// kMergeThreads entries of LDS each. MAXCH as in merge_one: with 8 the
// caller never has more than 8 splits per group.
template <bool BF16, int MAXCH = kMergeChunk, bool COH = false>
__device__ __forceinline__ void merge_wide_row(const float* parts, const float* lse, void* out,
                                               int sq, int heads, int dim, int slots, int used,
                                               int b, int h, int q, int t, float* speak,
                                               float* stot, f32x4* sacc) {
  using E = Elem<BF16>;
  const int d4n = dim / 4;
  const int G = kMergeThreads / d4n;
  const int c = t % d4n, g = t / d4n;
  const bool act = g < G;
  const int64_t base = ((int64_t)b * heads + h) * slots * sq + q;  // (b, h, split 0, q)
  const float* ls = lse + base;
  const float* ps = parts + base * dim + 4 * c;
  const int64_t part_stride = (int64_t)sq * dim;
  float peak = kNegBig, tot = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if (act) {
    // The smallest chunk of 4, 8 or 16 that holds a group's splits (16
    // beyond): 64 splits over 8 groups are one chunk of 8, not 16 with half
    // of the loads clamped. The live splits are summed in the same order.
    const int per = (used + G - 1) / G;
    if (per <= 4)
      wide_group<4, COH>(ls, ps, sq, part_stride, g, G, used, peak, tot, acc);
    else if (MAXCH <= 8 || per <= 8)
      wide_group<8, COH>(ls, ps, sq, part_stride, g, G, used, peak, tot, acc);
    else
      wide_group<kMergeChunk, COH>(ls, ps, sq, part_stride, g, G, used, peak, tot, acc);
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
    u16* dst = static_cast<u16*>(out) + (((int64_t)b * sq + q) * heads + h) * dim + 4 * c;
    *reinterpret_cast<u32x2*>(dst) = w;
  }
  __syncthreads();  // the LDS entries may be written again
}

// Fused split merge of fgw_mha_fwd (FwdParams::arrivals set, mode 1, key
// layout, at most kMergeChunk splits). Once a work item of task (b, h, q
// tile) has written its partial rows and LSE, its workgroup counts itself in
// at the task's counter; the one that arrives last (the task's `used` work
// items counted) merges the task's rows into the output with the stand-alone
// merge's arithmetic (merge_rows: one (row, 4 dims) per thread), so the
// output has the bits of the two-launch call, and sets the counter back to
// zero for the next call. Visibility across XCDs without any L2 write-back
// or invalidation (a release of the whole L2 per work item measured slower
// than the second launch it saves): the partial rows and LSE are
// agent-scope atomic stores (store_row, coherent at the device), every wave
// waits until its stores are complete before the count, the count is a
// vector global atomic at agent scope, and the merge reads the partials with
// agent-scope atomic loads (merge_ld1), issued after the count has returned.
// Every thread of the workgroup calls it; it uses 4 bytes of `lds`.
// MAXCH 8 (head-dim tile 32, whose kernels would lose a workgroup per CU to
// the 16-split chunk's registers) leaves that chunk out; the planner then
// fuses no plan that needs it (fused_merge_counters).
// Counters per task in the arrival buffer: one 128-byte line each, so that
// the atomics of different tasks do not queue on one line.
constexpr int kArrivalStride = 32;
template <int DPAD>
constexpr int kFusedMergeMaxChunk = DPAD == 32 ? 8 : kMergeChunk;
template <bool BF16, int THREADS, int ROWS_TILE, int MAXCH>
__device__ void arrive_and_merge(const FwdParams& p, int b, int h, int qt, int used,
                                 unsigned char* lds, int tid) {
  static_assert(THREADS == kMergeThreads, "the merge runs on one kMergeThreads workgroup");
  wait_vm<0>();     // this wave's partial rows and LSE are complete at the device
  __syncthreads();  // ... and every wave's
  int* flag = reinterpret_cast<int*>(lds);
  int32_t* ctr = p.arrivals + (((int64_t)b * p.heads + h) * p.q_tiles + qt) * kArrivalStride;
  if (opaque_lane(tid) == 0) {
    const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = prev == used - 1;
  }
  __syncthreads();
  if (!*flag) return;  // uniform: another work item of the task arrives later
  // The merge's inputs pass through opaque copies, so that the compiler
  // keeps the address and chunk arithmetic derived from them here instead
  // of hoisting it out of the work-item loop, where it would stay live
  // across the main loop (and cost the kernel its second workgroup per CU).
  int sq = p.sq, heads = p.heads, dim = p.dim, slots = p.splits;
  asm volatile("" : "+s"(sq), "+s"(heads), "+s"(dim), "+s"(slots), "+s"(used), "+s"(b), "+s"(h),
               "+s"(qt));
  asm volatile("" : "+v"(tid));
  const int q0 = qt * ROWS_TILE;
  const int rows = sq - q0 < ROWS_TILE ? sq - q0 : ROWS_TILE;
  merge_rows<BF16, MAXCH, true>(p.parts, p.lse, p.out, sq, heads, dim, slots, used, b, h, q0,
                                rows, tid, kMergeThreads);
  if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Page id of the page holding logical position pos.
__device__ __forceinline__ int32_t page_id(const FwdParams& p, const int32_t* table_b, int pos) {
  return table_b[div_page((u32)pos, p.page_magic, p.page_shift)];
}

// table and lengths come as separate read-only, non-aliasing arguments so
// that uniform reads of them can use the scalar cache.
template <class C>
__global__ __launch_bounds__(C::THREADS) void fwd_kernel(FwdParams p_arg,
                                                         const int32_t* __restrict__ table,
                                                         const int32_t* __restrict__ lengths) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::LDS_BYTES];
  // The parameters. Each work item reads them again from the kernel argument
  // segment (p_arg is its first argument, at offset 0) through a pointer the
  // compiler cannot follow, once for its set-up and main loop and once for
  // its output: it then loads what each part needs where it needs it,
  // instead of holding every parameter (and what it derives from them) in
  // scalar registers across the main loop.
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
  const int wq = C::NWQ > 1 ? wave : 0;
  const int wk = C::NWK > 1 ? wave : 0;
  unsigned char* const group_base = smem + wk * C::GROUP_BYTES;
  const Lanes<C> ln(lane);
  const int64_t row_bytes = (int64_t)p.heads * p.dim * 2;
  const DmaLanes<C> dl(lane, wq, row_bytes);

  const int grid = gridDim.x;
  const int prog = xcd_remap(blockIdx.x, grid);
  const int capacity = p.width * p.page_size;
  // Length-balanced splits (key layout, partial mode): request b takes
  // pre[b + 1] - pre[b] splits; its work items are [pre[b], pre[b + 1]) x
  // H x q_tiles, split-major (see the decode of w below).
  const bool balanced = C::LAYOUT == kLayoutKey && p.mode == 1 && p.split_keys > 0;
  const int32_t* const pre = reinterpret_cast<const int32_t*>(smem + C::PREFIX_OFF);
  int work = p.work;
  if constexpr (C::LAYOUT == kLayoutKey) {
    if (balanced) {
      balanced_prefix<C>(p, lengths, capacity, reinterpret_cast<int32_t*>(smem + C::PREFIX_OFF),
                         wave, lane);
      work = __builtin_amdgcn_readfirstlane(pre[p.batch]) * p.heads * p.q_tiles;
    }
  }
  int first, count;
  if (p.mode == 2) {  // static schedule: this program's segments
    first = p.seg_offsets[prog];
    count = p.seg_offsets[prog + 1] - first;
  } else if (work < grid && (int)blockIdx.x >= work) {
    first = count = 0;  // a balanced plan with fewer live items than programs
  } else {
    // Contiguous ranges over the programs that have work: all of them, or,
    // when a balanced plan has fewer live items than programs, the first
    // `work` ones, which the hardware spreads over every XCD (i % 8).
    const int active = work < grid ? work : grid;
    const int aprog = active == grid ? prog : xcd_remap(blockIdx.x, active);
    const int per = work / active, rem = work % active;
    first = aprog * per + (aprog < rem ? aprog : rem);
    count = per + (aprog < rem ? 1 : 0);
  }

  for (int it = 0; it < count; ++it) {
    // This item's copy of the parameters and of the values derived from them
    // above (they shadow the set-up's).
    FwdParams p = *kernarg();
    const int capacity = p.width * p.page_size;
    const int tasks = p.batch * p.heads * p.q_tiles;
    const bool balanced = C::LAYOUT == kLayoutKey && p.mode == 1 && p.split_keys > 0;
    int w = first + it, split = 0, slot = -1, seg_lo = 0, seg_hi = 0, nsplit = p.splits;
    if (p.mode == 2) {
      const int32_t* sg = p.segs + 4 * (int64_t)w;
      w = sg[0];
      seg_lo = sg[1] * p.seg_scale;
      seg_hi = (sg[1] + sg[2]) * p.seg_scale;
      slot = sg[3];
      // Segments a host plan cannot produce are skipped whole (uniform).
      if (w < 0 || w >= tasks || slot >= p.slots || sg[1] < 0 || sg[2] < 0) continue;
    } else if (balanced) {
      // g = w / (H q_tiles) = pre[b] + split for the request b with
      // pre[b] <= g < pre[b + 1] (pre is strictly increasing: every request
      // has at least one split); the rest of w is (h, q tile).
      const int hq = p.heads * p.q_tiles;
      const int g = w / hq;
      int lo = 0, hi = p.batch;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (__builtin_amdgcn_readfirstlane(pre[mid]) <= g) lo = mid; else hi = mid;
      }
      const int pb = __builtin_amdgcn_readfirstlane(pre[lo]);
      split = g - pb;
      nsplit = __builtin_amdgcn_readfirstlane(pre[lo + 1]) - pb;
      w = lo * hq + w % hq;
    } else {
      split = w % p.splits;
      w /= p.splits;
    }
    // Causal tiles outside a static schedule: the last (heaviest) first, so
    // that a dispatcher or a persistent program starts the long items early.
    const int qt = p.causal && p.mode != 2 ? p.q_tiles - 1 - w % p.q_tiles : w % p.q_tiles;
    w /= p.q_tiles;
    const int h = w % p.heads;
    const int b = w / p.heads;
    const int32_t* table_b = table + (int64_t)b * p.width;
    const char* kb = static_cast<const char*>(p.k) + (int64_t)h * p.dim * 2;
    const char* vb = static_cast<const char*>(p.v) + (int64_t)h * p.dim * 2;

    // Page ids of this wave's first two key blocks for a full cache, read
    // together with the length instead of after it; a shorter length moves
    // the block range and they are read again below.
    constexpr int kStep = C::NWK * C::BN;
    int spec_pos = -1;
    int32_t spec0 = 0, spec1 = 0;
    if (p.mode != 2 && !p.causal && !balanced) {
      const int nfull = (capacity + C::BN - 1) / C::BN;
      spec_pos = (split_bound(nfull, split, p.splits) + wk) * C::BN;
      if (spec_pos < capacity) spec0 = page_id(p, table_b, spec_pos);
      if (spec_pos + kStep < capacity) spec1 = page_id(p, table_b, spec_pos + kStep);
    }
    int len = lengths[b];
    len = len < 0 ? 0 : (len > capacity ? capacity : len);
    const int q0 = qt * C::ROWS_TILE;
    const int tile_last = (q0 + C::ROWS_TILE < p.sq ? q0 + C::ROWS_TILE : p.sq) - 1;
    int max_vis = p.causal ? len - p.sq + tile_last + 1 : len;
    max_vis = max_vis < 0 ? 0 : (max_vis > len ? len : max_vis);
    const int nblk = (max_vis + C::BN - 1) / C::BN;
    int blk_begin, blk_end;
    if (p.mode == 2) {  // the segment's blocks that hold visible keys
      blk_end = seg_hi < nblk ? seg_hi : nblk;
      blk_begin = seg_lo < blk_end ? seg_lo : blk_end;
    } else {
      blk_begin = split_bound(nblk, split, nsplit);
      blk_end = split_bound(nblk, split + 1, nsplit);
    }
    const int cnt = blk_end - blk_begin;
    const int my_n = cnt > wk ? (cnt - wk + C::NWK - 1) / C::NWK : 0;

    // Rows of this wave and their visible key counts; blocks that end above
    // wmin hold keys some row of the wave cannot see and are masked.
    const int row_base = q0 + wq * C::ROWS_WAVE;
    int wmin = p.causal ? len - p.sq + row_base + 1 : len;
    wmin = wmin < 0 ? 0 : (wmin > len ? len : wmin);
    const int qrow = row_base + il;
    int vis = p.causal ? len - p.sq + qrow + 1 : len;
    vis = vis < 0 ? 0 : (vis > len ? len : vis);

    float m = kNegBig, l = 0.0f;
    f32x16 o[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[dt][v] = 0.0f;

    const int first_pos = (blk_begin + wk) * C::BN;
    const bool spec = first_pos == spec_pos;
    if (it > 0) __syncthreads();  // LDS of the previous work item is no longer read
    // Every key group streams its blocks n = 0, 1, ... at key
    // (blk_begin + wk + NWK n) * BN through its own LDS stages; the DMA of
    // block n + 1 is in flight while block n is computed.
    int32_t next_id = my_n > 1 ? (spec ? spec1 : page_id(p, table_b, first_pos + kStep)) : 0;
    if (my_n > 0) {
      const int32_t id0 = spec ? spec0 : page_id(p, table_b, first_pos);
      issue_tile<C, false>(p, dl, table_b, kb, row_bytes, first_pos, id0, len, group_base, wq,
                           lane);
      issue_tile<C, true>(p, dl, table_b, vb, row_bytes, first_pos, id0, len,
                          group_base + C::TILE_BYTES, wq, lane);
    }
    // Q after the first DMA: its loads overlap the tile's.
    u32x4 qf[C::KK];
    {
      const int dim = opaque_uniform(p.dim), hq = opaque_lane(hh);
      const u16* qp =
          static_cast<const u16*>(p.q) + (((int64_t)b * p.sq + qrow) * p.heads + h) * p.dim;
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) {
        const int d = 16 * kk + 8 * hq;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (qrow < p.sq && d < dim) val = load16(qp + d);
        qf[kk] = val;
      }
    }
    for (int n = 0; n < my_n; ++n) {
      const int pos0 = first_pos + kStep * n;
      unsigned char* stage = group_base + (n % C::NBUF) * C::STAGE_BYTES;
      wait_dma();
      group_sync<C>();  // stage n is in LDS; everyone is done with stage n - 1
      const int32_t id1 = next_id;
      if (n + 2 < my_n) next_id = page_id(p, table_b, pos0 + 2 * kStep);
      if (n + 1 < my_n && C::NBUF == 2) {
        unsigned char* next = group_base + ((n + 1) % C::NBUF) * C::STAGE_BYTES;
        issue_tile<C, false>(p, dl, table_b, kb, row_bytes, pos0 + kStep, id1, len, next, wq,
                             lane);
        issue_tile<C, true>(p, dl, table_b, vb, row_bytes, pos0 + kStep, id1, len,
                            next + C::TILE_BYTES, wq, lane);
      }
      f32x16 s[C::ST];
      u32x4 pf[C::KS];
      qk_block<C>(stage, ln, qf, s);
      if (pos0 + C::BN > wmin) mask_block<C>(s, pos0, vis, hh);
      online_softmax<C>(s, m, l, o, p.scale_log2, pf);
      pv_block<C>(stage + C::TILE_BYTES, ln, pf, o);
      if (n + 1 < my_n && C::NBUF == 1) {
        group_sync<C>();  // single stage: refill only after every wave has read it
        issue_tile<C, false>(p, dl, table_b, kb, row_bytes, pos0 + kStep, id1, len, stage, wq,
                             lane);
        issue_tile<C, true>(p, dl, table_b, vb, row_bytes, pos0 + kStep, id1, len,
                            stage + C::TILE_BYTES, wq, lane);
      }
    }

    wait_dma();  // no DMA of this work item outlives it
    p = *kernarg();  // the output's parameters, not held across the main loop
    if constexpr (C::NWK == 1) {
      const float tot = pair_sum(l);
      // Direct stores: D < DPAD, or D tiles below 128 (staged, D tile 64
      // measured 1.3% slower on two query-layout shapes).
      auto store_direct = [&]() {
        if (qrow >= p.sq) return;
        const float inv = 1.0f / fmaxf(tot, 1.0e-30f);
        const int ho = opaque_lane(hh);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int d0 = 32 * dt + 8 * gq + 4 * ho;
            if (d0 < p.dim) {
              f32x4 val = {o[dt][4 * gq], o[dt][4 * gq + 1], o[dt][4 * gq + 2], o[dt][4 * gq + 3]};
              store_row<C>(p, b, h, split, qrow, d0, val, inv, slot, q0);
            }
          }
      };
      if constexpr (C::DPAD >= 128) {
        if (p.dim == C::DPAD) {
          // Every wave's DMA into the stages has landed (each waited for its
          // own above) and no wave reads them any more: they stage the output.
          __syncthreads();
          static_assert(C::NWQ * 32 * kStagedRowBytes<C> <= C::TILES_BYTES,
                        "staged rows fit the K/V stages");
          const bool f32 = p.mode == 1 || (p.mode == 2 && slot >= 0);
          float* fdst = nullptr;
          if (p.mode == 1)
            fdst = p.parts +
                   ((((int64_t)b * p.heads + h) * p.splits + split) * p.sq + row_base) * C::DPAD;
          else if (f32)
            fdst = p.parts + ((int64_t)slot * C::ROWS_TILE + (row_base - q0)) * C::DPAD;
          unsigned char* bdst =
              f32 ? nullptr
                  : static_cast<unsigned char*>(p.out) +
                        (((int64_t)b * p.sq + row_base) * p.heads + h) * C::DPAD * 2;
          store_rows_staged<C>(smem + wq * 32 * kStagedRowBytes<C>, lane, o,
                               1.0f / fmaxf(tot, 1.0e-30f), f32, fdst, bdst,
                               (int64_t)p.heads * C::DPAD * 2, p.sq - row_base);
        } else {
          store_direct();
        }
      } else {
        store_direct();
      }
      if (qrow < p.sq && hh == 0) {
        if (p.mode == 1)
          p.lse[(((int64_t)b * p.heads + h) * p.splits + split) * p.sq + qrow] = lse_of(m, tot);
        else if (p.mode == 2 && slot >= 0)
          p.lse[(int64_t)slot * C::ROWS_TILE + (qrow - q0)] = lse_of(m, tot);
      }
    } else {
      // Combine the NWK key-group states of the same query rows.
      __syncthreads();
      float* cm = reinterpret_cast<float*>(smem);
      float* cl = cm + C::NWK * C::ROWS_WAVE;
      float* co = cl + C::NWK * C::ROWS_WAVE;
      const float tot = pair_sum(l);
      if (hh == 0) {
        cm[wk * C::ROWS_WAVE + il] = m;
        cl[wk * C::ROWS_WAVE + il] = tot;
      }
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          f32x4 val = {o[dt][4 * gq], o[dt][4 * gq + 1], o[dt][4 * gq + 2], o[dt][4 * gq + 3]};
          *reinterpret_cast<f32x4*>(co + (wk * C::ROWS_WAVE + il) * C::OSTRIDE + 32 * dt +
                                    8 * gq + 4 * hh) = val;
        }
      __syncthreads();
      constexpr int D4 = C::DPAD / 4;
      for (int idx = tid; idx < C::ROWS_WAVE * D4; idx += C::THREADS) {
        const int r = idx / D4, d0 = 4 * (idx % D4);
        const int row = q0 + r;
        if (row < p.sq && d0 < p.dim) {
          float mm = kNegBig;
#pragma unroll
          for (int k = 0; k < C::NWK; ++k) mm = fmaxf(mm, cm[k * C::ROWS_WAVE + r]);
          float t2 = 0.0f;
          f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int k = 0; k < C::NWK; ++k) {
            const float wt = __builtin_amdgcn_exp2f(cm[k * C::ROWS_WAVE + r] - mm);
            t2 += cl[k * C::ROWS_WAVE + r] * wt;
            acc += *reinterpret_cast<const f32x4*>(co + (k * C::ROWS_WAVE + r) * C::OSTRIDE + d0) *
                   wt;
          }
          store_row<C>(p, b, h, split, row, d0, acc, 1.0f / fmaxf(t2, 1.0e-30f));
          if (p.mode == 1 && d0 == 0) {
            float* lp = p.lse + (((int64_t)b * p.heads + h) * p.splits + split) * p.sq + row;
            if (p.arrivals != nullptr)
              __hip_atomic_store(lp, lse_of(mm, t2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
              *lp = lse_of(mm, t2);
          }
        }
      }
    }
    if (C::LAYOUT == kLayoutKey && p.mode == 1 && p.arrivals != nullptr) {
      arrive_and_merge<C::BF16, C::THREADS, C::ROWS_TILE, kFusedMergeMaxChunk<C::DPAD>>(
          p, b, h, qt, nsplit, smem, tid);
    }
  }
}

template <bool BF16, int DPAD, int LAYOUT, int STAGES = 0>
hipError_t launch_fwd(const FwdParams& p, int grid, hipStream_t stream) {
  using C = Cfg<BF16, DPAD, LAYOUT, STAGES>;
  fwd_kernel<C><<<dim3(grid), dim3(C::THREADS), 0, stream>>>(p, p.table, p.lengths);
  return hipGetLastError();
}

// Resident workgroups per CU of one instantiation (0 if the query fails).
template <bool BF16, int DPAD, int LAYOUT, int STAGES = 0>
int occupancy_fwd() {
  using C = Cfg<BF16, DPAD, LAYOUT, STAGES>;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fwd_kernel<C>, C::THREADS, 0) != hipSuccess)
    return 0;
  return n;
}

}  // namespace fgw_mha
