// Forward-kernel instantiations: f16, head-dim tiles of the hi half.
#include "fmha_kernel.h"
#include "fmha_prefill.h"
#include "fmha_registry.h"

namespace fgw_mha {
FGW_MHA_FOR_DPAD_HI(FGW_MHA_INSTANTIATE, false)
FGW_MHA_INSTANTIATE_KEY_SINGLE(false)
FGW_MHA_FOR_PREFILL_HI(FGW_MHA_INSTANTIATE_PREFILL, false)
}  // namespace fgw_mha
