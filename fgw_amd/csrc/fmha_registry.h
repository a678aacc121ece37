// Host-side table of the compiled kernel instantiations.
#pragma once
#include <hip/hip_runtime.h>

#include "fmha_params.h"

namespace fgw_mha {

typedef hipError_t (*FwdLaunchFn)(const FwdParams&, int, hipStream_t);
typedef int (*OccupancyFn)();

struct FwdEntry {
  FwdLaunchFn launch;
  OccupancyFn occupancy;
};

// Head-dim tiles with a compiled kernel: 32, 64, 128, 256 (D padded to a
// power of two, cube_general.py:31).
inline int dim_tile(int dim) {
  int t = 32;
  while (t < dim) t *= 2;
  return t;
}

// The kernel of (dtype, head-dim tile, layout, stages); stages 0 is the
// instantiation's default, 1 the key layout's single-stage variant (tile 128).
FwdEntry fwd_entry(bool bf16, int dpad, int layout, int stages = 0);
hipError_t launch_merge(bool bf16, const MergeParams& p, hipStream_t stream);
hipError_t launch_gather(const GatherParams& p, hipStream_t stream);
hipError_t launch_pack(const PackParams& p, int total_pages, hipStream_t stream);
hipError_t launch_group_merge(bool bf16, const GroupMergeParams& p, int groups, hipStream_t stream);

}  // namespace fgw_mha

// Explicit instantiation lists, expanded once per translation unit.
#define FGW_MHA_FOR_DPAD_LO(X, BF) X(BF, 32) X(BF, 64)
#define FGW_MHA_FOR_DPAD_HI(X, BF) X(BF, 128) X(BF, 256)
#define FGW_MHA_INSTANTIATE(BF, DP)                                                         \
  template hipError_t launch_fwd<BF, DP, kLayoutQuery>(const FwdParams&, int, hipStream_t); \
  template hipError_t launch_fwd<BF, DP, kLayoutKey>(const FwdParams&, int, hipStream_t);   \
  template int occupancy_fwd<BF, DP, kLayoutQuery>();                                       \
  template int occupancy_fwd<BF, DP, kLayoutKey>();
// The key layout's single-stage variant: head-dim tile 128 (two workgroups per CU).
#define FGW_MHA_INSTANTIATE_KEY_SINGLE(BF)                                                  \
  template hipError_t launch_fwd<BF, 128, kLayoutKey, 1>(const FwdParams&, int, hipStream_t); \
  template int occupancy_fwd<BF, 128, kLayoutKey, 1>();
#define FGW_MHA_EXTERN_KEY_SINGLE(BF)                                                              \
  extern template hipError_t launch_fwd<BF, 128, kLayoutKey, 1>(const FwdParams&, int, hipStream_t); \
  extern template int occupancy_fwd<BF, 128, kLayoutKey, 1>();
// The prefill layout exists for head-dim tiles 64 and 128.
#define FGW_MHA_FOR_PREFILL_LO(X, BF) X(BF, 64)
#define FGW_MHA_FOR_PREFILL_HI(X, BF) X(BF, 128)
#define FGW_MHA_INSTANTIATE_PREFILL(BF, DP)                                   \
  template hipError_t launch_prefill<BF, DP>(const FwdParams&, int, hipStream_t); \
  template int occupancy_prefill<BF, DP>();
#define FGW_MHA_EXTERN_PREFILL(BF, DP)                                               \
  extern template hipError_t launch_prefill<BF, DP>(const FwdParams&, int, hipStream_t); \
  extern template int occupancy_prefill<BF, DP>();
#define FGW_MHA_EXTERN(BF, DP)                                                                     \
  extern template hipError_t launch_fwd<BF, DP, kLayoutQuery>(const FwdParams&, int, hipStream_t); \
  extern template hipError_t launch_fwd<BF, DP, kLayoutKey>(const FwdParams&, int, hipStream_t);   \
  extern template int occupancy_fwd<BF, DP, kLayoutQuery>();                                       \
  extern template int occupancy_fwd<BF, DP, kLayoutKey>();
