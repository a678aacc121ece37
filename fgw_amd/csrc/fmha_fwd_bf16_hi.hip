// Forward-kernel instantiations: bf16, head-dim tiles of the hi half.
#include "fmha_kernel.h"
#include "fmha_registry.h"

namespace fgw_mha {
FGW_MHA_FOR_DPAD_HI(FGW_MHA_INSTANTIATE, true)
}  // namespace fgw_mha
