// Instantiations and launcher of the fused LNCC kernel for k = 7 (halo 3).
#include "lncc_fused_kernel.h"
#include "lncc_launch.h"

namespace fl {

hipError_t launch_fused_h3(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st) {
    return launch_fused<3>(mode, bf16, a, nblocks, st);
}

}  // namespace fl
