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
  int32_t mode;           // 0: normalised output, 1: partial (O/l, LSE)
  uint32_t page_magic;    // division of positions by page_size
  uint32_t page_shift;
  float scale_log2;       // dim^-0.5 * log2(e)
};

struct MergeParams {
  const float* parts;     // [B, H, S, Sq, D]
  const float* lse;       // [B, H, S, Sq]
  void* out;              // [B, Sq, H, D]
  int32_t batch, sq, heads, dim, splits;
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
