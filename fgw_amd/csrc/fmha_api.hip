// C ABI of the paged MHA operator: validation, planning and dispatch.
// Declarations and reference citations: include/fgw_mha.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/fgw_mha.h"
#include "fmha_aux.h"
#include "fmha_kernel.h"
#include "fmha_prefill.h"
#include "fmha_registry.h"

namespace fgw_mha {

FGW_MHA_FOR_DPAD_LO(FGW_MHA_EXTERN, true)
FGW_MHA_FOR_DPAD_HI(FGW_MHA_EXTERN, true)
FGW_MHA_FOR_DPAD_LO(FGW_MHA_EXTERN, false)
FGW_MHA_FOR_DPAD_HI(FGW_MHA_EXTERN, false)
FGW_MHA_EXTERN_KEY_SINGLE(true)
FGW_MHA_EXTERN_KEY_SINGLE(false)
FGW_MHA_FOR_PREFILL_LO(FGW_MHA_EXTERN_PREFILL, true)
FGW_MHA_FOR_PREFILL_HI(FGW_MHA_EXTERN_PREFILL, true)
FGW_MHA_FOR_PREFILL_LO(FGW_MHA_EXTERN_PREFILL, false)
FGW_MHA_FOR_PREFILL_HI(FGW_MHA_EXTERN_PREFILL, false)

#define FGW_ENTRY(BF, DP, LY) \
  if (bf16 == BF && dpad == DP && layout == LY) return FwdEntry{&launch_fwd<BF, DP, LY>, &occupancy_fwd<BF, DP, LY>};
#define FGW_ENTRIES(BF, DP) FGW_ENTRY(BF, DP, kLayoutQuery) FGW_ENTRY(BF, DP, kLayoutKey)
#define FGW_PREFILL_ENTRY(BF, DP) \
  if (bf16 == BF && dpad == DP && layout == kLayoutPrefill) return FwdEntry{&launch_prefill<BF, DP>, &occupancy_prefill<BF, DP>};

FwdEntry fwd_entry(bool bf16, int dpad, int layout, int stages) {
  if (stages == 1 && layout == kLayoutKey && dpad == 128)
    return bf16 ? FwdEntry{&launch_fwd<true, 128, kLayoutKey, 1>,
                           &occupancy_fwd<true, 128, kLayoutKey, 1>}
                : FwdEntry{&launch_fwd<false, 128, kLayoutKey, 1>,
                           &occupancy_fwd<false, 128, kLayoutKey, 1>};
  FGW_MHA_FOR_DPAD_LO(FGW_ENTRIES, true)
  FGW_MHA_FOR_DPAD_HI(FGW_ENTRIES, true)
  FGW_MHA_FOR_DPAD_LO(FGW_ENTRIES, false)
  FGW_MHA_FOR_DPAD_HI(FGW_ENTRIES, false)
  FGW_MHA_FOR_PREFILL_LO(FGW_PREFILL_ENTRY, true)
  FGW_MHA_FOR_PREFILL_HI(FGW_PREFILL_ENTRY, true)
  FGW_MHA_FOR_PREFILL_LO(FGW_PREFILL_ENTRY, false)
  FGW_MHA_FOR_PREFILL_HI(FGW_PREFILL_ENTRY, false)
  return FwdEntry{nullptr, nullptr};
}

hipError_t launch_merge(bool bf16, const MergeParams& p, hipStream_t stream) {
  if (p.splits > kMergeChunk) {  // splits spread over a workgroup per row
    const dim3 grid((unsigned)((int64_t)p.batch * p.heads * p.sq));
    if (bf16) {
      merge_wide_kernel<true><<<grid, dim3(kMergeThreads), 0, stream>>>(p);
    } else {
      merge_wide_kernel<false><<<grid, dim3(kMergeThreads), 0, stream>>>(p);
    }
    return hipGetLastError();
  }
  // One (row, 4 dims) pair per thread: a workgroup covers whole rows.
  int rows_per_wg = (4 * kMergeThreads) / p.dim > 0 ? (4 * kMergeThreads) / p.dim : 1;
  // Tile-balanced plans merge a query tile's rows by its own slot count: a
  // power-of-two row group never straddles two 256-row tiles.
  if (p.rows_tile > 0)
    while (rows_per_wg & (rows_per_wg - 1)) rows_per_wg &= rows_per_wg - 1;
  const int64_t groups = (p.sq + rows_per_wg - 1) / rows_per_wg;
  const dim3 grid((unsigned)((int64_t)p.batch * p.heads * groups));
  if (bf16) {
    merge_kernel<true><<<grid, dim3(kMergeThreads), 0, stream>>>(p, rows_per_wg);
  } else {
    merge_kernel<false><<<grid, dim3(kMergeThreads), 0, stream>>>(p, rows_per_wg);
  }
  return hipGetLastError();
}

hipError_t launch_gather(const GatherParams& p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.batch * p.out_len;
  gather_kernel<<<dim3((unsigned)rows), dim3(256), 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_group_merge(bool bf16, const GroupMergeParams& p, int groups,
                              hipStream_t stream) {
  if (bf16)
    group_merge_kernel<true><<<dim3((unsigned)groups), dim3(kMergeThreads), 0, stream>>>(p);
  else
    group_merge_kernel<false><<<dim3((unsigned)groups), dim3(kMergeThreads), 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_pack(const PackParams& p, int total_pages, hipStream_t stream) {
  const int64_t wgs = (int64_t)total_pages * p.wg_per_page;
  pack_pages_kernel<<<dim3((unsigned)wgs), dim3(kPackThreads), 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace fgw_mha

using namespace fgw_mha;

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FGW_MHA_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxSplits = 128;
static_assert(kMaxBalancedBatch == FGW_MHA_MAX_BALANCED_BATCH, "balanced-split batch cap");
constexpr int kAutoMaxSplits = 64;
// Fewest key rounds per automatic split: two, and four in the prefill layout,
// whose work items carry a 256-row Q tile, a two-block pipeline fill and
// 256 partial rows each (measured on B1H1 long-Q shapes: Q1024/KV4096 runs
// in 24.4 us at 16 splits against 28.0 us at 32).
constexpr int kMinRoundsPerSplit = 2;
constexpr int kMinRoundsPerSplitPrefill = 4;

// Split workspace of fgw_mha_fwd_noalloc: partials then LSE of one call, in
// a device array the code object brings (each GPU that loads the library
// holds its own copy until the process ends). Host code never passes the
// array's name to a kernel: that is a host-side stand-in, not a device
// address. It uses the address hipGetSymbolAddress returns on each device.
constexpr int64_t kScratchFloats = FGW_MHA_NOALLOC_SCRATCH_BYTES / 4;
static __device__ __align__(256) float scratch[kScratchFloats];
// Its fused-merge arrival counters (one per task): zero when the code object
// is loaded, and every call returns the counters it used to zero.
constexpr int kScratchArrivals = FGW_MHA_NOALLOC_ARRIVALS;
static __device__ __align__(256) int32_t arrival_scratch[kScratchArrivals] = {};

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};
int32_t* g_arrival_ptr[kMaxDevices] = {};

// This device's addresses of `scratch` and `arrival_scratch`, looked up once
// per device with that device current (the caller's current device is
// restored).
int scratch_address(int device, float** out, int32_t** arrivals) {
  if (device < 0 || device >= kMaxDevices)
    return fail(FGW_MHA_EUNSUPPORTED, "device %d is outside the scratch table", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    int current = 0;
    hipError_t err = hipGetDevice(&current);
    if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
    if (current != device && (err = hipSetDevice(device)) != hipSuccess)
      return hip_fail(err, "hipSetDevice");
    void* ptr = nullptr;
    void* aptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err == hipSuccess) err = hipGetSymbolAddress(&aptr, HIP_SYMBOL(arrival_scratch));
    if (current != device) (void)hipSetDevice(current);
    if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(scratch)");
    if (!ptr || !aptr) return fail(FGW_MHA_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_arrival_ptr[device] = static_cast<int32_t*>(aptr);
    g_scratch_ptr[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[device];
  *arrivals = g_arrival_ptr[device];
  return FGW_MHA_OK;
}

// K/V stages per key group of the default kernel of (layout, head-dim tile);
// the prefill layout's rings have four slots.
template <int LY>
int cfg_stages(int dpad) {
  switch (dpad) {
    case 32: return Cfg<true, 32, LY>::NBUF;
    case 64: return Cfg<true, 64, LY>::NBUF;
    case 128: return Cfg<true, 128, LY>::NBUF;
    default: return Cfg<true, 256, LY>::NBUF;
  }
}
int default_stages(int layout, int dpad) {
  if (layout == kLayoutPrefill) return 4;
  return layout == kLayoutKey ? cfg_stages<kLayoutKey>(dpad) : cfg_stages<kLayoutQuery>(dpad);
}
// The key layout's single-stage variant exists for head-dim tile 128.
bool has_key_single(int layout, int dpad) { return layout == kLayoutKey && dpad == 128; }

// Automatic plans of short decode (Sq <= 16) on the key layout at head-dim
// tile 128 whose even splits number 16 or more and give each CU at most one
// work item move to the single-stage kernel with more splits: for Sq <= 4,
// 4x the splits (each keeping >= 512 keys), else 2x (>= 256 keys); for
// 4 < Sq <= 16, 2x (>= 256 keys). Returns that split count, or 0 to keep
// the plan. Two workgroups per CU then overlap one's prologue and epilogue
// with the other's stream. Measured (single-call median, same box, A/B):
// B2 H8 KV 32768 0.962-0.965x (BF16 and FP16), KV 65536 0.975x, KV 16384
// 0.981x, KV 8192 0.972x, B1 H8 / B2 H4 KV 32768 0.993x, B1 H16 Q4 0.987x;
// B2 H8 Q8 / Q16 at 2x (32 splits): KV 32768 0.976x / 0.975x, KV 8192
// 0.969x / 0.966x, where 4x (64 splits) lost at Q16 (1.03x); below 16
// splits (B2 H16 or B8 H8, 4-8 splits) it measured 1.00-1.05x, so those
// plans stay.
int single_stage_splits(const fgw_mha_shape* s, const fgw_mha_device_info* dev, int layout,
                        int dpad, int64_t tasks, int splits, int64_t capacity) {
  if (!has_key_single(layout, dpad) || s->sq > 16 || splits < 16 ||
      dev->wg_per_cu_key_single < 2 || tasks * splits > dev->num_cus)
    return 0;
  if (s->sq <= 4 && 4 * splits <= kMaxSplits && capacity / (4 * splits) >= 512) return 4 * splits;
  if (2 * splits <= kMaxSplits && capacity / (2 * splits) >= 256) return 2 * splits;
  return 0;
}
bool stages_valid(int layout, int dpad, int stages) {
  return stages == default_stages(layout, dpad) ||
         (has_key_single(layout, dpad) && (stages == 1 || stages == 2));
}

// Keys one program consumes per loop round, and query rows per work item,
// per layout.
int keys_per_round(int layout) { return layout == kLayoutKey ? 4 * 32 : 64; }
int rows_per_tile(int layout) {
  return layout == kLayoutKey ? 32 : (layout == kLayoutPrefill ? 256 : 128);
}
// Head-dim tiles with a prefill-layout kernel.
bool has_prefill(int dpad) { return dpad == 64 || dpad == 128; }

// Largest split chunk of the fused merge in the kernels of a head-dim tile.
int fused_max_chunk(int dpad) {
  switch (dpad) {
    case 32: return kFusedMergeMaxChunk<32>;
    case 64: return kFusedMergeMaxChunk<64>;
    case 128: return kFusedMergeMaxChunk<128>;
    default: return kFusedMergeMaxChunk<256>;
  }
}

// Arrival counter buffer (int32 elements: kArrivalStride per task) of a split
// plan whose merge fgw_mha_fwd fuses into the partial kernel (the last work
// item of each task merges the task's rows, arrive_and_merge in
// fmha_kernel.h), or 0 to merge in a second launch. Fused for key-layout
// plans of Sq <= 2 with at most kMergeChunk splits (one round of the
// per-thread merge), where it measured level with or faster than the second
// launch (B2 H8 D128 BF16, KV 2048-32768, 4-16 splits of either key kernel,
// 36 plans: single-call median 0.990x on geometric mean, 0.963-1.071x;
// back to back 0.970x). Elsewhere it lost: every work item waits for its
// partial stores to complete and for the count before its workgroup ends,
// and the last one merges alone; with more splits per task (32-128 splits:
// 1.158x, 1.01-1.51x) or more rows to merge (Sq 4-16: 1.074x, 0.97-1.47x)
// that tail exceeds the second launch. Kernels whose fused merge leaves out
// the 16-split chunk (kFusedMergeMaxChunk) fuse at most 8 splits.
int64_t fused_merge_counters(const fgw_mha_shape* s, int layout, int splits, int rows,
                             int64_t tasks) {
  (void)rows;
  if (splits < 2 || layout != kLayoutKey || s->sq > 2 || splits > kMergeChunk) return 0;
  if (splits > fused_max_chunk(dim_tile(s->dim))) return 0;
  // The count travels as int32 (fgw_mha_plan_t.arrival_counters).
  if (tasks > INT32_MAX / kArrivalStride) return 0;
  return tasks * kArrivalStride;
}

// split_keys > 0 means length-balanced splits in the key layout and
// tile-balanced causal splits in the prefill layout.
bool tile_balanced(int layout, int causal, int split_keys) {
  return split_keys > 0 && layout == kLayoutPrefill && causal;
}
bool split_keys_valid(const fgw_mha_shape* s, int layout, int splits, int split_keys) {
  if (split_keys == 0) return true;
  if (split_keys < 0 || splits < 2) return false;
  return (layout == kLayoutKey && s->batch <= kMaxBalancedBatch) ||
         tile_balanced(layout, s->causal, split_keys);
}
// Automatic tile-balanced causal splits (prefill layout): with few query
// tiles (at most half the device's programs) of very different lengths (the
// longest sees >= 2048 keys and >= 1.5x the mean), the long tiles are cut so
// that each work item takes at most about 1.5x an even share of all keys per
// CU. Returns split_keys (num_splits in *splits), or 0 to keep the plan.
// Measured against the automatic even splits (causal self-attention, BF16,
// back to back): B1 H8 S2048-4096 0.92-0.97x, B2 H8 / B1 H16 S2048
// 0.94x, B1 H4 S8192 0.89x, B2 H4 S4096 0.91x, B1 H2 S16384 0.82x, D64
// 0.92-0.97x; left alone because they lost: prefix-cached shapes (Sq < KV,
// tiles of similar lengths, 1.06-1.07x), B1 H32 S1024 (longest tile 1024
// keys, 1.13x), and 256 tiles (B1 H16 S4096, 1.09x).
int auto_tile_balanced(const fgw_mha_shape* s, const fgw_mha_device_info* dev, int64_t capacity,
                       int* splits) {
  const int rows = 256;
  const int q_tiles = (s->sq + rows - 1) / rows;
  const int64_t tiles = (int64_t)s->batch * s->heads * q_tiles;
  const int wg = dev->wg_per_cu[kLayoutPrefill] > 0 ? dev->wg_per_cu[kLayoutPrefill] : 1;
  if (!s->causal || 2 * tiles > (int64_t)dev->num_cus * wg) return 0;
  int64_t sum = 0, longest = 0;
  for (int t = 0; t < q_tiles; ++t) {
    const int64_t end = (int64_t)(t + 1) * rows < s->sq ? (int64_t)(t + 1) * rows : s->sq;
    int64_t vis = capacity - s->sq + end;
    vis = vis < 0 ? 0 : (vis > capacity ? capacity : vis);
    sum += vis;
    longest = vis > longest ? vis : longest;
  }
  if (longest < 2048 || 2 * longest * q_tiles < 3 * sum) return 0;
  const int64_t total = sum * s->batch * s->heads;
  int64_t keys = (3 * total + 2 * (int64_t)dev->num_cus * 64 - 1) / (2 * (int64_t)dev->num_cus * 64) * 64;
  keys = keys < 256 ? 256 : keys;
  const int64_t slots_needed = (longest + keys - 1) / keys;
  if (slots_needed < 2 || keys > INT32_MAX) return 0;
  int n = 2;
  while (n < slots_needed && n < kAutoMaxSplits) n *= 2;
  *splits = n;
  return (int)keys;
}

// Work items of a tile-balanced causal plan: every (b, h) takes
// tile_slots(t) items of each 256-row query tile t.
int64_t tile_balanced_work(const fgw_mha_shape* s, int splits, int split_keys) {
  const int rows = 256;
  const int q_tiles = (s->sq + rows - 1) / rows;
  const int capacity = s->width * s->page_size;
  int64_t per_bh = 0;
  for (int t = 0; t < q_tiles; ++t)
    per_bh += tile_slots(t, s->sq, capacity, rows, split_keys, splits);
  return (int64_t)s->batch * s->heads * per_bh;
}
// The automatic layout choice takes the prefill layout for Q longer than one
// query-layout tile (Sq > 128) when its 256-row query tiles alone give every
// resident program of the device a work item, when Sq >= 1024, or when the
// work B * H * Sq * capacity reaches 2^24 query-key pairs. Measured over 250 seeded shapes (B 1-16, H 8-32, head-dim tiles 64 and
// 128, Sq 64-2048, capacity 1024-16384, causal or not), each layout at its
// best split count, as the query layout's time over the prefill layout's:
// Sq > 128 from 2^24 pairs on 0.996-1.54 (1.24 geometric mean, 173
// shapes); 2^23-2^24 pairs 0.90-1.07 (even); below 2^23 pairs 0.89-1.0
// (the query layout's shorter work items win); Sq <= 128, where a 256-row
// tile is at least half padding, 0.76-1.05 (0.94).
bool auto_prefill(const fgw_mha_shape* s, const fgw_mha_device_info* dev, int dpad) {
  if (!has_prefill(dpad) || s->sq <= 128) return false;
  const int rows = 256;
  const int64_t tiles = (int64_t)s->batch * s->heads * ((s->sq + rows - 1) / rows);
  const int wg = dev->wg_per_cu[kLayoutPrefill] > 0 ? dev->wg_per_cu[kLayoutPrefill] : 1;
  const int64_t pairs = (int64_t)s->batch * s->heads * s->sq * ((int64_t)s->width * s->page_size);
  return tiles >= (int64_t)dev->num_cus * wg || s->sq >= 1024 || pairs >= (int64_t(1) << 24);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Granlund-Montgomery constants for the division of positions by page_size.
void page_divisor(uint32_t page, uint32_t* magic, uint32_t* shift) {
  if (page <= 1) {
    *magic = 0;
    *shift = 0;
    return;
  }
  uint32_t l = 0;
  while ((1ull << l) < page) ++l;
  const uint64_t m = (((1ull << 32) * ((1ull << l) - page)) / page) + 1;
  *magic = (uint32_t)m;
  *shift = l;
}

int check_shape(const fgw_mha_shape* s) {
  if (!s) return fail(FGW_MHA_EINVAL, "shape is NULL");
  if (s->batch <= 0 || s->sq <= 0 || s->heads <= 0 || s->dim <= 0)
    return fail(FGW_MHA_EINVAL, "positive Q extents and rank-2 table required");
  if (s->page_size <= 0 || s->pool_rows <= 0 || s->pool_rows % s->page_size || s->width <= 0)
    return fail(FGW_MHA_EINVAL,
                "positive page size, whole pool pages and positive table width required");
  if (s->dtype != FGW_MHA_FLOAT16 && s->dtype != FGW_MHA_BFLOAT16)
    return fail(FGW_MHA_EINVAL, "matching FP16/BF16 Q/K/V required");
  if (s->dim < 16 || s->dim > 256 || s->dim % 16)
    return fail(FGW_MHA_EUNSUPPORTED, "D must be in [16, 256] and divisible by 16");
  if ((int64_t)s->width * s->page_size > INT32_MAX)
    return fail(FGW_MHA_EUNSUPPORTED, "table capacity exceeds 2^31 tokens");
  if ((int64_t)s->batch * s->sq * s->heads > INT32_MAX)
    return fail(FGW_MHA_EUNSUPPORTED, "B*Sq*H exceeds 2^31 rows");
  return FGW_MHA_OK;
}

int check_plan(const fgw_mha_shape* s, const fgw_mha_plan_t* p) {
  if (!p) return fail(FGW_MHA_EINVAL, "plan is NULL");
  if (p->layout != kLayoutQuery && p->layout != kLayoutKey && p->layout != kLayoutPrefill)
    return fail(FGW_MHA_EINVAL, "plan layout %d is not a kernel layout", p->layout);
  if (p->layout == kLayoutPrefill && !has_prefill(dim_tile(s->dim)))
    return fail(FGW_MHA_EINVAL, "the prefill layout needs D in (32, 128]");
  const int rows = rows_per_tile(p->layout);
  const int q_tiles = (s->sq + rows - 1) / rows;
  const int64_t tasks = (int64_t)s->batch * s->heads * q_tiles;
  const int64_t work = tile_balanced(p->layout, s->causal, p->split_keys)
                           ? tile_balanced_work(s, p->num_splits, p->split_keys)
                           : tasks * p->num_splits;
  if (p->rows_per_tile != rows || p->q_tiles != q_tiles || p->query_tile_tasks != tasks ||
      p->num_splits < 1 || p->num_splits > kMaxSplits || p->work_items != work ||
      p->grid < 1 || p->grid > p->work_items ||
      p->dim_padded != dim_tile(s->dim) || p->execution_mode != (p->num_splits > 1 ? 1 : 0) ||
      !split_keys_valid(s, p->layout, p->num_splits, p->split_keys) ||
      !stages_valid(p->layout, p->dim_padded, p->stages) ||
      (p->arrival_counters != 0 &&
       p->arrival_counters != fused_merge_counters(s, p->layout, p->num_splits, rows, tasks)))
    return fail(FGW_MHA_EINVAL, "plan does not match the shape; call fgw_mha_plan");
  return FGW_MHA_OK;
}

int check_tensors(const fgw_mha_tensors* t, bool need_inputs, bool need_out, bool need_ws) {
  if (!t) return fail(FGW_MHA_EINVAL, "tensors is NULL");
  if (need_inputs) {
    if (!t->q || !t->k_cache || !t->v_cache || !t->block_table || !t->cache_seqlens)
      return fail(FGW_MHA_EINVAL, "input pointer is NULL");
    if (!aligned16(t->q) || !aligned16(t->k_cache) || !aligned16(t->v_cache))
      return fail(FGW_MHA_EINVAL, "Q/K/V must be 16-byte aligned");
  }
  if (need_out && (!t->out || !aligned16(t->out)))
    return fail(FGW_MHA_EINVAL, "output must be a 16-byte aligned buffer");
  if (need_ws && (!t->parts || !t->lse || !aligned16(t->parts)))
    return fail(FGW_MHA_EINVAL, "split workspace (parts, lse) required, parts 16-byte aligned");
  return FGW_MHA_OK;
}

FwdParams make_params(const fgw_mha_shape* s, const fgw_mha_plan_t* p, const fgw_mha_tensors* t,
                      int mode) {
  FwdParams f;
  f.q = t->q;
  f.k = t->k_cache;
  f.v = t->v_cache;
  f.table = t->block_table;
  f.lengths = t->cache_seqlens;
  f.out = t->out;
  f.parts = t->parts;
  f.lse = t->lse;
  f.pool_rows = s->pool_rows;
  f.batch = s->batch;
  f.sq = s->sq;
  f.heads = s->heads;
  f.dim = s->dim;
  f.width = s->width;
  f.page_size = s->page_size;
  f.causal = s->causal ? 1 : 0;
  f.splits = p->num_splits;
  f.q_tiles = p->q_tiles;
  f.work = p->work_items;
  f.mode = mode;
  f.split_keys = mode == 1 ? p->split_keys : 0;
  f.split_direct = 0;
  page_divisor((uint32_t)s->page_size, &f.page_magic, &f.page_shift);
  f.scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)s->dim));
  f.segs = nullptr;
  f.seg_offsets = nullptr;
  f.slots = 0;
  f.seg_scale = 1;
  f.arrivals = nullptr;
  return f;
}

// Checks shared by the static-schedule entries.
int check_schedule(const fgw_mha_shape* s, const fgw_mha_schedule* sc) {
  int rc = check_shape(s);
  if (rc) return rc;
  if (!sc) return fail(FGW_MHA_EINVAL, "schedule is NULL");
  const int bn = Cfg<true, 128, kLayoutQuery>::BN;
  if (sc->block_keys <= 0 || sc->block_keys % bn)
    return fail(FGW_MHA_EINVAL, "schedule block_keys must be a positive multiple of %d", bn);
  if (sc->programs < 1 || !sc->seg_offsets || !sc->segments)
    return fail(FGW_MHA_EINVAL, "schedule needs programs >= 1, segments and seg_offsets");
  if (sc->slots < 0 || sc->n_merges < 0 || (sc->n_merges > 0 && !sc->merges))
    return fail(FGW_MHA_EINVAL, "schedule slots and merges must be consistent");
  const int rows = rows_per_tile(kLayoutQuery);
  const int64_t tasks = (int64_t)s->batch * s->heads * ((s->sq + rows - 1) / rows);
  if (tasks > INT32_MAX || (int64_t)sc->slots * rows > INT32_MAX)
    return fail(FGW_MHA_EUNSUPPORTED, "schedule exceeds 2^31 tasks or partial rows");
  return FGW_MHA_OK;
}

// `whole`: the partial kernel of a full call, whose merge follows (a
// tile-balanced plan's one-split tiles then write their output directly).
int launch_partial_kernel(const fgw_mha_shape* s, const fgw_mha_plan_t* p,
                          const fgw_mha_tensors* t, int mode, hipStream_t stream,
                          bool whole = false, int32_t* arrivals = nullptr) {
  const int stages = p->stages == default_stages(p->layout, p->dim_padded) ? 0 : p->stages;
  const FwdEntry e = fwd_entry(s->dtype == FGW_MHA_BFLOAT16, p->dim_padded, p->layout, stages);
  if (!e.launch) return fail(FGW_MHA_EUNSUPPORTED, "no kernel for dim tile %d", p->dim_padded);
  FwdParams f = make_params(s, p, t, mode);
  f.split_direct = whole && mode == 1 && tile_balanced(p->layout, s->causal, p->split_keys);
  f.arrivals = mode == 1 ? arrivals : nullptr;
  const hipError_t err = e.launch(f, p->grid, stream);
  return err == hipSuccess ? FGW_MHA_OK : hip_fail(err, "forward kernel launch");
}

int launch_merge_kernel(const fgw_mha_shape* s, const fgw_mha_plan_t* p, const fgw_mha_tensors* t,
                        hipStream_t stream, bool whole = false) {
  MergeParams m;
  m.parts = t->parts;
  m.lse = t->lse;
  m.out = t->out;
  m.batch = s->batch;
  m.sq = s->sq;
  m.heads = s->heads;
  m.dim = s->dim;
  m.splits = p->num_splits;
  m.lengths = t->cache_seqlens;
  m.split_keys = p->split_keys;
  m.capacity = s->width * s->page_size;
  m.rows_tile = tile_balanced(p->layout, s->causal, p->split_keys) ? 256 : 0;
  m.skip_single = whole && m.rows_tile > 0;
  const hipError_t err = launch_merge(s->dtype == FGW_MHA_BFLOAT16, m, stream);
  return err == hipSuccess ? FGW_MHA_OK : hip_fail(err, "merge kernel launch");
}

}  // namespace

extern "C" {

int fgw_mha_abi_version(void) { return FGW_MHA_ABI_VERSION; }

const char* fgw_mha_last_error(void) { return g_error; }

int fgw_mha_query_device(int device, fgw_mha_device_info* info) {
  if (!info) return fail(FGW_MHA_EINVAL, "info is NULL");
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDeviceProperties");
  int current = 0;
  err = hipGetDevice(&current);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  if (current != device && (err = hipSetDevice(device)) != hipSuccess)
    return hip_fail(err, "hipSetDevice");
  info->num_cus = prop.multiProcessorCount;
  info->arch_gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  for (int layout = 0; layout < FGW_MHA_NUM_LAYOUTS; ++layout) {
    const int n = fwd_entry(true, 128, layout).occupancy();
    info->wg_per_cu[layout] = n > 0 ? n : 1;
  }
  const int single = fwd_entry(true, 128, kLayoutKey, 1).occupancy();
  info->wg_per_cu_key_single = single > 0 ? single : 1;
  if (current != device) (void)hipSetDevice(current);
  return FGW_MHA_OK;
}

int fgw_mha_plan(const fgw_mha_shape* s, const fgw_mha_request* req,
                 const fgw_mha_device_info* dev, fgw_mha_plan_t* out) {
  int rc = check_shape(s);
  if (rc) return rc;
  if (!req || !dev || !out) return fail(FGW_MHA_EINVAL, "request/device/plan is NULL");
  if (dev->num_cus <= 0) return fail(FGW_MHA_EINVAL, "device info has no compute units");
  const int dpad = dim_tile(s->dim);
  int layout = req->layout;
  if (layout == FGW_MHA_LAYOUT_AUTO) {
    layout = s->sq <= 32 ? kLayoutKey
                         : (auto_prefill(s, dev, dpad) ? kLayoutPrefill : kLayoutQuery);
  }
  if (layout != kLayoutQuery && layout != kLayoutKey && layout != kLayoutPrefill)
    return fail(FGW_MHA_EINVAL, "layout must be -1 (auto), 0 (query), 1 (key) or 2 (prefill)");
  if (layout == kLayoutPrefill && !has_prefill(dpad))
    return fail(FGW_MHA_EINVAL, "the prefill layout needs D in (32, 128]");
  const int rows = rows_per_tile(layout);
  const int q_tiles = (s->sq + rows - 1) / rows;
  const int64_t tasks = (int64_t)s->batch * s->heads * q_tiles;
  const int64_t capacity = (int64_t)s->width * s->page_size;
  // KV tiles of 32 tokens, as the reference general route counts them
  // (cube_general.py:36); more splits than blocks leave empty splits.
  const int64_t kv_blocks = (capacity + 31) / 32;
  if (req->stages != 0 && !stages_valid(layout, dpad, req->stages))
    return fail(FGW_MHA_EINVAL,
                "stages must be 0 (the default kernel), 1 or 2 for the key layout with head-dim "
                "tile 128, else 0 or %d", default_stages(layout, dpad));
  const int wg_default = dev->wg_per_cu[layout] > 0 ? dev->wg_per_cu[layout] : 1;

  int splits = req->num_splits;
  int split_keys = req->split_keys;  // automatic prefill plans may set it
  bool auto_single = false;  // automatic splits moved to the single-stage kernel
  if (splits != 0) {
    if (splits < 1 || splits > kMaxSplits || (splits & (splits - 1)))
      return fail(FGW_MHA_EINVAL, "num_splits supports None (automatic) or 1/2/4/.../%d",
                  kMaxSplits);
    if (splits > kv_blocks)
      return fail(FGW_MHA_EINVAL,
                  "num_splits must not exceed the number of KV tiles in table capacity");
  } else {
    const int rounds = layout == kLayoutPrefill ? kMinRoundsPerSplitPrefill : kMinRoundsPerSplit;
    int64_t min_keys = (int64_t)keys_per_round(layout) * rounds;
    // Prefill layout: a split also takes at least 8 keys per query tile task.
    // Each doubling adds a partial row per task row to write and merge, while
    // the keys of a split shrink; with many tasks the merge outweighs the
    // shorter items (B1 H16 Q1536 KV 1024, 96 tasks: 32.5 us unsplit against
    // 39.6 us at 2 splits). Measured over 160 seeded shapes: 1.006x the best
    // split count on geometric mean, against 1.012x with 256 keys alone.
    if (layout == kLayoutPrefill && 8 * tasks > min_keys) min_keys = 8 * tasks;
    // Query layout: four rounds (256 keys) once B * H * Sq * capacity reaches
    // 2^22 pairs. Over 84 seeded multi-head shapes of the query layout's range
    // (Sq 48-1023, causal or not, head-dim tiles 64 and 128) this is 1.009x
    // the best split count on geometric mean for D 128 and 1.020x otherwise,
    // against 1.040x and 1.057x at two rounds (B2 H8 Q96 KV4096 D64: 26.1 us
    // at 32 splits, 17.7 us at 16); single-head B1 shapes below 2^22 pairs keep
    // two rounds (four cost them 1.15x).
    const int64_t pairs = (int64_t)s->batch * s->heads * s->sq * capacity;
    if (layout == kLayoutQuery && pairs >= (int64_t(1) << 22) && min_keys < 4 * 64)
      min_keys = 4 * 64;
    // Double while the doubled work items still fit the resident slots: one
    // doubling past them makes a second wave of items (B1H1 Q3712/KV4096:
    // 15 tiles x 32 splits = 480 items on 256 slots, 55.8 us, against 31.2 us
    // at 16 splits).
    const int64_t slots = (int64_t)dev->num_cus * wg_default;
    splits = 1;
    while (splits < kAutoMaxSplits && tasks * splits * 2 <= slots &&
           (int64_t)(splits * 2) * min_keys <= capacity)
      splits *= 2;
    if (req->stages == 0 && req->split_keys == 0) {
      const int up = single_stage_splits(s, dev, layout, dpad, tasks, splits, capacity);
      if (up > 0) {
        splits = up;
        auto_single = true;
      }
    }
    if (layout == kLayoutPrefill && req->split_keys == 0) {
      int tb_splits = 0;
      const int keys = auto_tile_balanced(s, dev, capacity, &tb_splits);
      if (keys > 0) {
        splits = tb_splits;
        split_keys = keys;
      }
    }
  }
  if (split_keys < 0) return fail(FGW_MHA_EINVAL, "split_keys must be 0 or positive");
  if (!split_keys_valid(s, layout, splits, split_keys))
    return fail(FGW_MHA_EINVAL,
                "split_keys needs num_splits >= 2 and either the key layout with B <= %d "
                "(length-balanced splits) or the causal prefill layout (tile-balanced splits)",
                kMaxBalancedBatch);
  const int64_t work = tile_balanced(layout, s->causal, split_keys)
                           ? tile_balanced_work(s, splits, split_keys)
                           : tasks * splits;
  if (work > INT32_MAX) return fail(FGW_MHA_EUNSUPPORTED, "work items exceed 2^31");

  // Stages: the layout's default kernel unless the request names one or the
  // automatic splits moved to the key layout's single-stage kernel (head-dim
  // tile 128, two workgroups per CU; single_stage_splits). Elsewhere that
  // kernel measured slower: where a workgroup is alone on its CU (B2 H8
  // KV 32768, 8 splits: 56.9 us against 47.7 us) and for large batches split a
  // few ways (B8 H32 KV 4096, 2 splits: 115.9 us against 101.7 us at 1 split).
  const int stages =
      req->stages != 0 ? req->stages : (auto_single ? 1 : default_stages(layout, dpad));
  const int wg_kernel = stages == 1 && has_key_single(layout, dpad)
                            ? (dev->wg_per_cu_key_single > 0 ? dev->wg_per_cu_key_single : 1)
                            : wg_default;

  int64_t grid = work;
  if (req->persistent_programs < -1)
    return fail(FGW_MHA_EINVAL, "persistent_programs must be -1, 0 or positive");
  if (req->persistent_programs == -1 && !s->causal) {
    // Device cap: the resident workgroups of all CUs loop over contiguous
    // ranges of work items. Causal work items differ in size (and with
    // Sq > len many are empty), so causal plans keep one workgroup per work
    // item and let the hardware dispatcher balance them: measured 1.06-2.5x
    // faster than the cap for causal prefill with more tiles than programs.
    const int64_t cap = (int64_t)dev->num_cus * wg_kernel;
    grid = work < cap ? work : cap;
  } else if (req->persistent_programs > 0) {
    grid = work < req->persistent_programs ? work : req->persistent_programs;
  }

  out->layout = layout;
  out->rows_per_tile = rows;
  out->q_tiles = q_tiles;
  out->num_splits = splits;
  out->query_tile_tasks = (int32_t)tasks;
  out->work_items = (int32_t)work;
  out->grid = (int32_t)grid;
  out->threads = layout == kLayoutPrefill ? 512 : 256;
  out->execution_mode = splits > 1 ? 1 : 0;
  out->dim_padded = dpad;
  out->parts_floats = splits > 1 ? (int64_t)s->batch * s->heads * splits * s->sq * s->dim : 0;
  out->lse_floats = splits > 1 ? (int64_t)s->batch * s->heads * splits * s->sq : 0;
  out->split_keys = split_keys;
  out->stages = stages;
  out->arrival_counters = (int32_t)fused_merge_counters(s, layout, splits, rows, tasks);
  return FGW_MHA_OK;
}

int fgw_mha_fwd(const fgw_mha_shape* s, const fgw_mha_plan_t* p, const fgw_mha_tensors* t,
                hipStream_t stream) {
  int rc = check_shape(s);
  if (!rc) rc = check_plan(s, p);
  if (!rc) rc = check_tensors(t, true, true, p->num_splits > 1);
  if (rc) return rc;
  if (p->num_splits == 1) return launch_partial_kernel(s, p, t, 0, stream);
  if (t->arrivals && p->arrival_counters > 0)  // one launch: the last work item merges
    return launch_partial_kernel(s, p, t, 1, stream, true, t->arrivals);
  rc = launch_partial_kernel(s, p, t, 1, stream, true);
  if (rc) return rc;
  return launch_merge_kernel(s, p, t, stream, true);
}

int fgw_mha_fwd_noalloc(const fgw_mha_shape* s, const fgw_mha_plan_t* p,
                        const fgw_mha_tensors* t, hipStream_t stream) {
  int rc = check_shape(s);
  if (!rc) rc = check_plan(s, p);
  if (!rc) rc = check_tensors(t, true, true, false);
  if (rc) return rc;
  if (p->num_splits == 1) return launch_partial_kernel(s, p, t, 0, stream);
  const int64_t need = p->parts_floats + p->lse_floats;
  if (need > kScratchFloats)
    return fail(FGW_MHA_EUNSUPPORTED,
                "split workspace of %lld bytes exceeds the %lld-byte static scratch of "
                "fgw_mha_fwd_noalloc; use fgw_mha_fwd with a caller workspace",
                (long long)need * 4, (long long)kScratchFloats * 4);
  int device = 0;
  hipError_t err = stream ? hipStreamGetDevice(stream, &device) : hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(err, "stream device");
  float* base = nullptr;
  int32_t* arrivals = nullptr;
  rc = scratch_address(device, &base, &arrivals);
  if (rc) return rc;
  fgw_mha_tensors w = *t;
  w.parts = base;  // 256-byte aligned
  w.lse = base + p->parts_floats;
  if (p->arrival_counters > 0 && p->arrival_counters <= kScratchArrivals)
    return launch_partial_kernel(s, p, &w, 1, stream, true, arrivals);
  rc = launch_partial_kernel(s, p, &w, 1, stream, true);
  if (rc) return rc;
  return launch_merge_kernel(s, p, &w, stream, true);
}

int fgw_mha_partial(const fgw_mha_shape* s, const fgw_mha_plan_t* p, const fgw_mha_tensors* t,
                    hipStream_t stream) {
  int rc = check_shape(s);
  if (!rc) rc = check_plan(s, p);
  if (!rc) rc = check_tensors(t, true, false, true);
  if (rc) return rc;
  return launch_partial_kernel(s, p, t, 1, stream);
}

int fgw_mha_merge(const fgw_mha_shape* s, const fgw_mha_plan_t* p, const fgw_mha_tensors* t,
                  hipStream_t stream) {
  int rc = check_shape(s);
  if (!rc) rc = check_plan(s, p);
  if (!rc) rc = check_tensors(t, false, true, true);
  if (!rc && p->split_keys > 0 && p->layout == kLayoutKey && !t->cache_seqlens)
    rc = fail(FGW_MHA_EINVAL, "a length-balanced plan merges by cache_seqlens; it is NULL");
  if (rc) return rc;
  return launch_merge_kernel(s, p, t, stream);
}

int fgw_mha_gather_kv(const fgw_mha_shape* s, const fgw_mha_tensors* t, void* out_k, void* out_v,
                      int32_t out_len, hipStream_t stream) {
  int rc = check_shape(s);
  if (rc) return rc;
  if (!t || !t->k_cache || !t->v_cache || !t->block_table || !t->cache_seqlens || !out_k ||
      !out_v)
    return fail(FGW_MHA_EINVAL, "gather needs K/V, table, lengths and two outputs");
  if (!aligned16(t->k_cache) || !aligned16(t->v_cache) || !aligned16(out_k) || !aligned16(out_v))
    return fail(FGW_MHA_EINVAL, "gather buffers must be 16-byte aligned");
  if (out_len <= 0) return fail(FGW_MHA_EINVAL, "out_len must be positive");
  if ((int64_t)s->batch * out_len > INT32_MAX)
    return fail(FGW_MHA_EUNSUPPORTED, "B*out_len exceeds 2^31 rows");
  GatherParams g;
  g.k = t->k_cache;
  g.v = t->v_cache;
  g.table = t->block_table;
  g.lengths = t->cache_seqlens;
  g.out_k = out_k;
  g.out_v = out_v;
  g.pool_rows = s->pool_rows;
  g.batch = s->batch;
  g.heads = s->heads;
  g.dim = s->dim;
  g.width = s->width;
  g.page_size = s->page_size;
  g.out_len = out_len;
  page_divisor((uint32_t)s->page_size, &g.page_magic, &g.page_shift);
  const hipError_t err = launch_gather(g, stream);
  return err == hipSuccess ? FGW_MHA_OK : hip_fail(err, "gather kernel launch");
}

int fgw_mha_static_local(const fgw_mha_shape* s, const fgw_mha_tensors* t,
                         const fgw_mha_schedule* sc, hipStream_t stream) {
  int rc = check_schedule(s, sc);
  if (!rc) rc = check_tensors(t, true, true, sc->slots > 0);
  if (rc) return rc;
  const int dpad = dim_tile(s->dim);
  const FwdEntry e = fwd_entry(s->dtype == FGW_MHA_BFLOAT16, dpad, kLayoutQuery);
  if (!e.launch) return fail(FGW_MHA_EUNSUPPORTED, "no kernel for dim tile %d", dpad);
  fgw_mha_plan_t p;
  std::memset(&p, 0, sizeof(p));
  p.layout = kLayoutQuery;
  p.rows_per_tile = rows_per_tile(kLayoutQuery);
  p.q_tiles = (s->sq + p.rows_per_tile - 1) / p.rows_per_tile;
  p.num_splits = 1;
  p.work_items = 0;
  p.dim_padded = dpad;
  FwdParams f = make_params(s, &p, t, 2);
  f.segs = sc->segments;
  f.seg_offsets = sc->seg_offsets;
  f.slots = sc->slots;
  f.seg_scale = sc->block_keys / Cfg<true, 128, kLayoutQuery>::BN;
  const hipError_t err = e.launch(f, sc->programs, stream);
  return err == hipSuccess ? FGW_MHA_OK : hip_fail(err, "static schedule kernel launch");
}

int fgw_mha_static_merge(const fgw_mha_shape* s, const fgw_mha_tensors* t,
                         const fgw_mha_schedule* sc, hipStream_t stream) {
  int rc = check_schedule(s, sc);
  if (rc) return rc;
  if (sc->n_merges == 0) return FGW_MHA_OK;
  if (!t || !t->out || !aligned16(t->out) || !t->parts || !t->lse || !aligned16(t->parts))
    return fail(FGW_MHA_EINVAL, "merge needs out, parts and lse; out and parts 16-byte aligned");
  GroupMergeParams g;
  g.parts = t->parts;
  g.lse = t->lse;
  g.groups = sc->merges;
  g.out = t->out;
  g.sq = s->sq;
  g.heads = s->heads;
  g.dim = s->dim;
  g.rows_tile = rows_per_tile(kLayoutQuery);
  g.q_tiles = (s->sq + g.rows_tile - 1) / g.rows_tile;
  g.slots = sc->slots;
  g.tasks = s->batch * s->heads * g.q_tiles;
  // One (row, 4 dims) per thread: kMergeThreads / (D / 4) rows per workgroup.
  g.rows_wg = kMergeThreads / (s->dim / 4) > 0 ? kMergeThreads / (s->dim / 4) : 1;
  g.wg_per_group = (g.rows_tile + g.rows_wg - 1) / g.rows_wg;
  if ((int64_t)sc->n_merges * g.wg_per_group > INT32_MAX)
    return fail(FGW_MHA_EUNSUPPORTED, "merge groups exceed the grid");
  const hipError_t err = launch_group_merge(s->dtype == FGW_MHA_BFLOAT16, g,
                                            sc->n_merges * g.wg_per_group, stream);
  return err == hipSuccess ? FGW_MHA_OK : hip_fail(err, "group merge kernel launch");
}

int fgw_mha_pack_pages(const fgw_mha_shape* s, const fgw_mha_tensors* t, const int32_t* cu_rows,
                       int32_t total_pages, void* out_k, void* out_v, hipStream_t stream) {
  int rc = check_shape(s);
  if (rc) return rc;
  if (!t || !t->k_cache || !t->v_cache || !t->block_table || !cu_rows || !out_k || !out_v)
    return fail(FGW_MHA_EINVAL, "pack needs K/V, table, cu_rows and two outputs");
  if (!aligned16(t->k_cache) || !aligned16(t->v_cache) || !aligned16(out_k) || !aligned16(out_v))
    return fail(FGW_MHA_EINVAL, "pack buffers must be 16-byte aligned");
  if (total_pages < 0) return fail(FGW_MHA_EINVAL, "total_pages must not be negative");
  const int64_t page_bytes = (int64_t)s->page_size * s->heads * s->dim * 2;
  if (page_bytes % 16) return fail(FGW_MHA_EINVAL, "a page must hold whole 16-byte chunks");
  const int64_t page_chunks = page_bytes / 16;
  const int64_t wpp = (page_chunks + kPackChunks - 1) / kPackChunks;
  if (page_chunks > INT32_MAX || (int64_t)total_pages * wpp > INT32_MAX ||
      (int64_t)total_pages * s->page_size > INT32_MAX)
    return fail(FGW_MHA_EUNSUPPORTED, "packed cache exceeds 2^31 rows or workgroups");
  if (total_pages == 0) return FGW_MHA_OK;
  PackParams p;
  p.k = t->k_cache;
  p.v = t->v_cache;
  p.table = t->block_table;
  p.cu_rows = cu_rows;
  p.out_k = out_k;
  p.out_v = out_v;
  p.pool_rows = s->pool_rows;
  p.batch = s->batch;
  p.width = s->width;
  p.page_size = s->page_size;
  p.page_chunks = (int32_t)page_chunks;
  p.wg_per_page = (int32_t)wpp;
  const hipError_t err = launch_pack(p, total_pages, stream);
  return err == hipSuccess ? FGW_MHA_OK : hip_fail(err, "pack kernel launch");
}

}  // extern "C"
