// Kernel-side parameter blocks shared by the host dispatcher and the device
// templates. Plain integers and pointers only; passed to kernels by value.
#pragma once
#include <stdint.h>

namespace fgw_mha {

// Work-item layouts of the forward kernel (see fmha_kernel.h).
enum Layout : int {
  kLayoutQuery = 0,  // 4 waves split the query rows of a tile and share K/V tiles
  kLayoutKey = 1,    // 4 waves split the key blocks of a work item (decode)
  kLayoutPrefill = 2,  // 8 waves x 32 query rows, pipelined K/V rings (fmha_prefill.h)
};

struct FwdParams {
  const void* q;          // [B, Sq, H, D]  fp16/bf16
  const void* k;          // [N, H, D]
  const void* v;          // [N, H, D]
  const int32_t* table;   // [B, W]
  const int32_t* lengths; // [B]
  void* out;              // [B, Sq, H, D]           (direct mode)
  float* parts;           // [B, H, S, Sq, D] fp32   (partial mode)
  float* lse;             // [B, H, S, Sq]    fp32   (partial mode)
  int64_t pool_rows;      // N
  int32_t batch, sq, heads, dim, width, page_size;
  int32_t causal;
  int32_t splits;
  int32_t q_tiles;        // ceil(Sq / rows per tile)
  int32_t work;           // B * H * q_tiles * splits
  int32_t mode;           // 0: normalised output, 1: partial (O/l, LSE), 2: static schedule
  uint32_t page_magic;    // division of positions by page_size
  uint32_t page_shift;
  float scale_log2;       // dim^-0.5 * log2(e)
  // Static schedule (mode 2, query layout): program p runs segments
  // [seg_offsets[p], seg_offsets[p + 1]) of segs, each (task, first key
  // block, key blocks, slot) with task = (b H + h) q_tiles + q tile and key
  // blocks of the kernel's BN keys. slot < 0 writes the normalised output;
  // slot >= 0 writes O/l to parts [slot, rows per tile, D] and the LSE to
  // lse [slot, rows per tile].
  const int32_t* segs;
  const int32_t* seg_offsets;
  int32_t slots;
  int32_t seg_scale;  // kernel key blocks per schedule key block
  // Length-balanced splits (key layout, mode 1): request b takes
  // balanced_splits(len_b, split_keys, splits) splits; tile-balanced causal
  // splits (prefill layout, causal, mode 1): query tile t takes
  // tile_slots(t, ...) splits; 0 = even splits.
  int32_t split_keys;
  // Tile-balanced plans in a whole call: a tile of one split writes its
  // normalised output rows directly (the merge skips them).
  int32_t split_direct;
  // Fused split merge (mode 1, query and key layouts): one counter per task
  // (b H + h) q_tiles + q tile, zero on entry; every work item counts itself
  // in once its partial rows are written, the last one of a task merges the
  // task's rows into `out` and sets the counter back to zero. nullptr: the
  // merge is a separate launch.
  int32_t* arrivals;
};

struct MergeParams {
  const float* parts;     // [B, H, S, Sq, D]
  const float* lse;       // [B, H, S, Sq]
  void* out;              // [B, Sq, H, D]
  int32_t batch, sq, heads, dim, splits;
  // Length-balanced splits: row (b, ., .) merges the first
  // balanced_splits(len_b, split_keys, splits) slots; 0 = all slots.
  const int32_t* lengths;  // [B], read only when split_keys > 0 and rows_tile == 0
  int32_t split_keys, capacity;
  // Tile-balanced causal splits: rows of query tile t merge the first
  // tile_slots(t, ...) slots; rows per query tile, 0 = not such a plan.
  int32_t rows_tile;
  int32_t skip_single;  // 1: rows of one-slot tiles were written directly; skip them
};

// Merge of the static schedule's split tiles: group g = (task, first slot,
// slots) merges parts [first .. first + slots) of one query tile.
struct GroupMergeParams {
  const float* parts;     // [slots, rows per tile, D]
  const float* lse;       // [slots, rows per tile]
  const int32_t* groups;  // [G, 3]
  void* out;              // [B, Sq, H, D]
  int32_t sq, heads, dim, q_tiles, rows_tile, slots, tasks;
  int32_t rows_wg, wg_per_group;  // rows per workgroup, workgroups per group
};

struct GatherParams {
  const void* k;
  const void* v;
  const int32_t* table;
  const int32_t* lengths;
  void* out_k;            // [B, out_len, H, D]
  void* out_v;
  int64_t pool_rows;
  int32_t batch, heads, dim, width, page_size, out_len;
  uint32_t page_magic, page_shift;
};

// Page-granular packing of the live cache (see pack_pages_kernel).
struct PackParams {
  const void* k;
  const void* v;
  const int32_t* table;
  const int32_t* cu_rows;  // [B + 1] packed row offsets, multiples of page_size
  void* out_k;             // [cu_rows[B], H, D]
  void* out_v;
  int64_t pool_rows;
  int32_t batch, width, page_size;
  int32_t page_chunks;  // 16-byte chunks of one page (page_size * H * D * 2 / 16)
  int32_t wg_per_page;
};

}  // namespace fgw_mha
