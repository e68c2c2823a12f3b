// Instantiations and launcher of the fused LNCC kernel for k = 5 (halo 2).
#include "lncc_fused_kernel.h"
#include "lncc_launch.h"

namespace fl {

hipError_t launch_fused_h2(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st) {
    return launch_fused<2>(mode, bf16, a, nblocks, st);
}

}  // namespace fl
