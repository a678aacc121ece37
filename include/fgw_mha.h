/*
 * fgw_mha.h -- C ABI of the MI355X (gfx950) paged multi-head attention operator.
 *
 * Drop-in boundary for the reference operator entry `operators/mha/current.py`
 * (zhangwenhao91/FGW), which re-exports
 * `operators/mha/kernels/mha_paged_decode_ascend_v7.py`:
 *   mha_paged_decode(q, k_cache, v_cache, block_table, cache_seqlens, page_size,
 *                    is_causal=False, *, num_splits=None, split_policy="auto")
 *   build_kernel(batch, sq, heads, dim, pool_rows, width, page_size, causal, dtype, ...)
 * The reference has no native FFI of its own: its kernels are TileLang JIT
 * adapters. Every entry point below replaces one piece of that Python path,
 * cited per declaration. The Python mirror of the reference interface
 * (fgw_amd/operators/mha/current.py) binds these symbols through ctypes.
 *
 * Tensor contract (v0.py:107-122, v7.py:529-544):
 *   Q, O      [B, Sq, H, D]   fp16 or bf16, contiguous
 *   K, V      [N, H, D]       same dtype, N = pool rows (whole pages)
 *   table     [B, W]          int32 page ids
 *   lengths   [B]             int32 live cache length per request
 * Query row q of request b sees keys [0, len_b) (non-causal) or
 * [0, max(len_b - Sq + q + 1, 0)) (right-aligned causal, cube_general.py:121-126).
 * Rows with no visible key are exactly zero.
 *
 * All functions return 0 on success or a negative fgw_mha_status; the message
 * of the last failure on the calling thread is in fgw_mha_last_error().
 * No function allocates, frees or synchronises device memory; launches are
 * asynchronous on the given stream. Functions are reentrant.
 */
#ifndef FGW_MHA_H_
#define FGW_MHA_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGW_MHA_ABI_VERSION 6

typedef enum {
  FGW_MHA_OK = 0,
  FGW_MHA_EINVAL = -1,      /* invalid argument (Python: ValueError) */
  FGW_MHA_EUNSUPPORTED = -2, /* shape/dtype outside the kernel family (ValueError) */
  FGW_MHA_EHIP = -3          /* HIP runtime error (RuntimeError) */
} fgw_mha_status;

typedef enum { FGW_MHA_FLOAT16 = 0, FGW_MHA_BFLOAT16 = 1 } fgw_mha_dtype;

typedef enum {
  FGW_MHA_LAYOUT_AUTO = -1,
  FGW_MHA_LAYOUT_QUERY = 0, /* 4 waves x 32 query rows share 64-key K/V tiles (prefill) */
  FGW_MHA_LAYOUT_KEY = 1,   /* 4 waves split the keys of 32 query rows (decode) */
  FGW_MHA_LAYOUT_PREFILL = 2 /* 8 waves x 32 query rows in two groups that alternate MFMA and
                                softmax phases over shared 64-key K/V rings; D in (32, 128] */
} fgw_mha_layout;

#define FGW_MHA_NUM_LAYOUTS 3

/* Static shape of one operator instance: the arguments of the reference
 * build_kernel (v7.py:32-47) that fix a specialisation. */
typedef struct {
  int32_t batch;     /* B */
  int32_t sq;        /* queries per request */
  int32_t heads;     /* H */
  int32_t dim;       /* D, 16..256, multiple of 16 */
  int64_t pool_rows; /* N = pool pages * page_size */
  int32_t width;     /* W, page-table width */
  int32_t page_size; /* tokens per page, >= 1, N % page_size == 0 */
  int32_t causal;    /* 0 / 1 */
  int32_t dtype;     /* fgw_mha_dtype */
} fgw_mha_shape;

/* Planning request: the reference's split and persistent-grid controls
 * (v7.py:43-46, :94-113; v7_experimental.py:29-30 persistent_programs). */
typedef struct {
  int32_t num_splits;          /* 0 = automatic; else 1,2,4,...,128 */
  int32_t persistent_programs; /* -1 = CU-derived cap (uncapped for causal), 0 = uncapped grid, n > 0 = cap */
  int32_t layout;              /* fgw_mha_layout */
  int32_t split_keys;          /* 0 = every request's keys split evenly into num_splits; > 0 =
                                  splits balanced by length (key layout, num_splits > 1, B <=
                                  FGW_MHA_MAX_BALANCED_BATCH): request b takes
                                  clamp(ceil(len_b / split_keys), 1, num_splits) splits, so
                                  ragged requests get work items of similar size; in the
                                  causal prefill layout (num_splits > 1), tile-balanced
                                  splits: query tile t takes clamp(ceil(its visible keys at
                                  table capacity / split_keys), 1, num_splits) work items
                                  (fgw_mha_plan may choose these itself for causal plans
                                  with few tiles of very different lengths and reports them
                                  in fgw_mha_plan_t.split_keys). No reference counterpart
                                  (the reference splits every request evenly). */
  int32_t stages;              /* K/V stages per key group: 0 = the layout's default kernel
                                  (double-stage for the key layout at head-dim tile 128),
                                  except that automatic short-decode plans (Sq <= 4, 16+
                                  even splits, at most one work item per CU) move to the
                                  single-stage kernel with 4x (or 2x) the splits;
                                  1 or 2 selects the key layout's single-stage (two
                                  workgroups per CU) or double-stage kernel where both exist
                                  (head-dim tile 128); elsewhere only the kernel's own count
                                  is accepted. No reference counterpart (a kernel-variant
                                  choice). */
} fgw_mha_request;

/* Largest batch of a length-balanced split plan (split_keys > 0). */
#define FGW_MHA_MAX_BALANCED_BATCH 1024

/* Device facts the planner needs; filled by fgw_mha_query_device. */
typedef struct {
  int32_t num_cus;          /* compute units */
  int32_t wg_per_cu[FGW_MHA_NUM_LAYOUTS]; /* resident workgroups per CU, per layout, dim 128 */
  int32_t arch_gfx950;      /* 1 when the device is gfx950 */
  int32_t wg_per_cu_key_single; /* the same for the key layout's single-stage kernel */
} fgw_mha_device_info;

/* Resolved launch plan: the attributes the reference launch callable
 * exposes (v7.py:475-487, :500-512) plus workspace sizes. */
typedef struct {
  int32_t layout;          /* fgw_mha_layout actually used */
  int32_t rows_per_tile;   /* query rows per work item (reference block_q) */
  int32_t q_tiles;         /* ceil(Sq / rows_per_tile) */
  int32_t num_splits;      /* KV splits per (b, h, q tile) */
  int32_t query_tile_tasks;/* B * H * q_tiles */
  int32_t work_items;      /* query_tile_tasks * num_splits (compute_work) */
  int32_t grid;            /* launched programs (compute_grid) */
  int32_t threads;         /* threads per program */
  int32_t execution_mode;  /* 0 = direct single split, 1 = split and merge */
  int32_t dim_padded;      /* head-dim tile of the selected kernel */
  int64_t parts_floats;    /* fp32 elements of the partial-output workspace (0 if direct) */
  int64_t lse_floats;      /* fp32 elements of the LSE workspace (0 if direct) */
  int32_t split_keys;      /* request.split_keys of a split plan (0: even splits); work_items and
                              the workspaces are then upper bounds, slot s of request b is used
                              for s < clamp(ceil(len_b / split_keys), 1, num_splits) */
  int32_t stages;          /* K/V stages per key group of the selected kernel (query and key
                              layouts; the prefill layout's rings have 4 slots: 4) */
  int32_t arrival_counters; /* > 0: fgw_mha_fwd can fuse this split plan's merge into the
                              partial kernel when the call supplies an arrival buffer of this
                              many int32 (fgw_mha_tensors.arrivals; one 128-byte counter line
                              per query-tile task: 32 x query_tile_tasks); 0: the merge is
                              always a second launch (direct plans, the query and prefill
                              layouts, and tasks whose merge takes more than two rounds) */
} fgw_mha_plan_t;

/* Device buffers of one call. Workspaces are owned by the caller and sized
 * from the plan; they are unused (may be NULL) for execution_mode 0. */
typedef struct {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_table;
  const int32_t* cache_seqlens;
  void* out;
  float* parts; /* [B, H, S, Sq, D] */
  float* lse;   /* [B, H, S, Sq]    natural-log sum-exp, -1e30 for an empty split */
  int32_t* arrivals; /* NULL, or plan.arrival_counters int32, all zero on entry, for
                        fgw_mha_fwd's fused merge: each task's last work item merges the
                        task's rows and returns its counter to zero, so the buffer is zero
                        again when the call completes and can serve the next call on the
                        same stream. Calls that overlap (other streams) need their own
                        counters. Ignored by the other entry points. */
} fgw_mha_tensors;

/* ABI version of the loaded library (FGW_MHA_ABI_VERSION). No reference
 * counterpart. */
int fgw_mha_abi_version(void);

/* Message of the last failure on this thread ("" if none). No reference
 * counterpart (the reference raises Python exceptions). */
const char* fgw_mha_last_error(void);

/* CU count and per-layout occupancy of a device. Replaces the reference's
 * torch.npu.get_device_properties(...).cube_core_num reads (v7.py:64-68, :104-108). */
int fgw_mha_query_device(int device, fgw_mha_device_info* info);

/* Validate a shape and resolve layout, split count, kernel stages and grid.
 * Pure host function (no HIP calls). Replaces the split selection and
 * persistent-grid arithmetic of build_kernel (v7.py:48-113;
 * general_split_policy.py:9-21): automatic splits double while
 * B*H*q_tiles*(2 splits) still fits the device's resident workgroup slots
 * and every split keeps at least two rounds of key blocks (four in the
 * prefill layout, four in the query layout from 2^22 query-key pairs).
 * Stages: the layout's default kernel unless requested or the automatic
 * short-decode rule selects the key layout's single-stage kernel; the
 * persistent grid is capped at the selected kernel's resident slots. Errors
 * mirror the reference ValueErrors (v7.py:49-55, :97-99). */
int fgw_mha_plan(const fgw_mha_shape* shape, const fgw_mha_request* request,
                 const fgw_mha_device_info* device, fgw_mha_plan_t* plan);

/* Full forward: the direct kernel with the fused normalise/cast/store
 * epilogue when num_splits == 1, else partial + merge: one launch when the
 * plan has arrival_counters and t->arrivals is set (the last work item of
 * each (b, h, q tile) merges its splits, with the same arithmetic and so the
 * same output bits as the separate merge), two launches otherwise. Replaces
 * the compiled launch callable returned by build_kernel (v7.py:471-473,
 * :495-498; the reference always launches its merge separately,
 * v7.py:488-493). */
int fgw_mha_fwd(const fgw_mha_shape* shape, const fgw_mha_plan_t* plan,
                const fgw_mha_tensors* t, hipStream_t stream);

/* Bytes of the static device scratch that fgw_mha_fwd_noalloc uses as its
 * split workspace (partials then LSE, parts_floats + lse_floats fp32). */
#define FGW_MHA_NOALLOC_SCRATCH_BYTES (32ll << 20)
/* Its static arrival buffer (int32): plans whose arrival_counters fit fuse
 * their merge there, larger ones merge in a second launch. */
#define FGW_MHA_NOALLOC_ARRIVALS 65536

/* fgw_mha_fwd without a caller workspace and without any allocation: the
 * split workspace (t->parts / t->lse are ignored and may be NULL) is a static
 * device array of FGW_MHA_NOALLOC_SCRATCH_BYTES that the library holds on
 * every GPU it runs on until the process ends; its device address is looked
 * up once per device (on the device of `stream`). No reference counterpart:
 * for callers that cannot allocate device memory (HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). Plans whose parts_floats +
 * lse_floats exceed the scratch are rejected (FGW_MHA_EUNSUPPORTED). Direct
 * plans (num_splits == 1) need no scratch. Plans with arrival_counters (up
 * to FGW_MHA_NOALLOC_ARRIVALS) fuse their merge, with static counters that
 * every completed call leaves at zero (t->arrivals is ignored). Every call on
 * one GPU shares that GPU's scratch and counters: calls that overlap on one
 * GPU (other streams, other host threads) race on them. Nothing in the
 * scratch needs clearing: the partial kernel writes every row the merge
 * reads. */
int fgw_mha_fwd_noalloc(const fgw_mha_shape* shape, const fgw_mha_plan_t* plan,
                        const fgw_mha_tensors* t, hipStream_t stream);

/* Partial kernel only: writes parts[b,h,s,q,:] = O_s / l_s and lse[b,h,s,q].
 * Replaces launch.partial_kernel (v7.py:225-315, :488-490), the component the
 * reference's split breakdown times as "local" (bench_split_breakdown.py:79-96). */
int fgw_mha_partial(const fgw_mha_shape* shape, const fgw_mha_plan_t* plan,
                    const fgw_mha_tensors* t, hipStream_t stream);

/* LSE merge only: reads parts/lse, writes out. Replaces launch.merge_kernel
 * (v7.py:317-371, :491-493). */
int fgw_mha_merge(const fgw_mha_shape* shape, const fgw_mha_plan_t* plan,
                  const fgw_mha_tensors* t, hipStream_t stream);

/* Gather the live K/V rows of every request into packed [B, out_len, H, D]
 * buffers (zero rows past len). Uses the attention kernel's page resolution
 * table[b, pos // page] * page + pos % page (v0.py:137); replaces the paged
 * cache gather the reference validates row-exactly
 * (benchmarks/mha/external_cache_gather.py:55-64). */
int fgw_mha_gather_kv(const fgw_mha_shape* shape, const fgw_mha_tensors* t, void* out_k,
                      void* out_v, int32_t out_len, hipStream_t stream);

/* Static KV-block schedule over the query layout's 128-row tiles: a host
 * plan assigns every (task, key block) unit to one program as contiguous
 * segments; tiles cut across programs get a partial slot each and are merged
 * afterwards. task = (b H + h) ceil(Sq / 128) + q tile. Mirrors the plan the
 * reference's static host path consumes (operators/mha/static_schedule.py:
 * 8-16: segments (Q tile, first KV block, KV blocks, slot), merges (Q tile,
 * first slot, slots), slot -1 = written directly). */
typedef struct fgw_mha_schedule {
  const int32_t* segments;    /* device [n_segments, 4]: task, first block, blocks, slot (-1: direct) */
  const int32_t* seg_offsets; /* device [programs + 1]: segments of program p */
  const int32_t* merges;      /* device [n_merges, 3]: task, first slot, slots */
  int32_t programs;           /* grid of the local kernel */
  int32_t n_merges;
  int32_t slots;              /* partial slots: parts [slots, 128, D], lse [slots, 128] fp32 */
  int32_t block_keys;         /* keys per schedule block, a multiple of 64 (the reference: 128) */
} fgw_mha_schedule;

/* Local phase of a static schedule: every program runs its segments; direct
 * segments write the normalised output rows of their tile, the others O/l
 * and LSE into their slot. Segments and merges a valid plan cannot contain
 * (task or slot out of range, negative blocks) are skipped; key blocks past
 * a request's length are clamped. Replaces the static host candidate's
 * local kernel (operators/mha/kernels/mha_static_host_candidate.py:457-460,
 * :511-519). */
int fgw_mha_static_local(const fgw_mha_shape* shape, const fgw_mha_tensors* t,
                         const fgw_mha_schedule* schedule, hipStream_t stream);

/* Merge phase: one workgroup per merge group combines its slots into the
 * output rows of its tile (the LSE merge of fgw_mha_merge). Replaces the
 * static host candidate's merge kernel (mha_static_host_candidate.py:
 * 476-480, :521-525). No launch when n_merges is 0. */
int fgw_mha_static_merge(const fgw_mha_shape* shape, const fgw_mha_tensors* t,
                         const fgw_mha_schedule* schedule, hipStream_t stream);

/* Pack the live cache page by page: for request b, pool pages
 * table[b, 0 .. ceil(len_b / page) - 1] are copied whole, in order, to rows
 * [cu_rows[b], cu_rows[b + 1]) of out_k / out_v ([cu_rows[B], H, D]); a page
 * id outside the pool packs as zeros. cu_rows ([B + 1] int32, device) holds
 * the row offsets (multiples of page_size, cu_rows[0] = 0) and
 * total_pages = cu_rows[B] / page_size; the caller computes both from
 * host-known lengths. Replaces the paged-cache gather of the reference's
 * packed-cache path (benchmarks/mha/external_cache_gather.py:22-49: live
 * regions rounded up to whole pages, one gather call for K and one for V,
 * checked row-exactly at :55-64); K and V move in one launch here. */
int fgw_mha_pack_pages(const fgw_mha_shape* shape, const fgw_mha_tensors* t,
                       const int32_t* cu_rows, int32_t total_pages, void* out_k, void* out_v,
                       hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FGW_MHA_H_ */
