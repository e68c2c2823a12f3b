// Instantiations and launcher of the fused LNCC kernel for k = 9 (halo 4).
#include "lncc_fused_kernel.h"
#include "lncc_launch.h"

namespace fl {

hipError_t launch_fused_h4(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st) {
    return launch_fused<4>(mode, bf16, a, nblocks, st);
}

}  // namespace fl
