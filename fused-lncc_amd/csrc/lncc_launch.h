// Host-side view of the kernel launchers (argument blocks and per-halo entry points).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lncc_geometry.h"

namespace fl {

// LOSS: partial sums only; GRAD: and the pred gradient; MAPS: the reference's four maps; DUAL:
// the partial sums and both gradients (the marching kernel only)
enum Mode { MODE_LOSS = 0, MODE_GRAD = 1, MODE_MAPS = 2, MODE_DUAL = 3 };

struct FusedArgs {
    const void* pred;
    const void* target;
    void* grad;       // MODE_GRAD, MODE_DUAL: gradient wrt pred, pred dtype
    void* grad_t;     // MODE_DUAL: gradient wrt target, the same dtype
    float* ncc_map;   // MODE_MAPS: fp32 maps ncc, A, Bc, Cc (reference definitions)
    float* a_map;
    float* b_map;
    float* c_map;
    double* partials; // one ncc partial sum per workgroup
    int dimD, dimH, dimW;
    int ntx, nty, nzc, dchunk;
    float inv_n, nf, ndr;     // 1/n, n = k^3 and n * smooth_dr as float32
    float gscale;             // (2 n / M) s, s = range_scale(k) (the kernel's adjoints carry 1/s)
};

struct BoxArgs {
    const float* f0;  // fields to box-sum (f1, f2 only for the three-field combine)
    const float* f1;
    const float* f2;
    const void* pred;   // combine: p, t in the pred dtype
    const void* target;
    void* out;          // box3d: fp32 sum; combine: gradient in the pred dtype
    int dimD, dimH, dimW;
    int ntx, nty;
    float scale;
};

hipError_t launch_fused_h1(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st);
hipError_t launch_fused_h2(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st);
hipError_t launch_fused_h3(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st);
hipError_t launch_fused_h4(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st);

// The small-volume kernel (lncc_small.hip): volumes whose D, H and W are all at most kSmallEdge
// (lncc_geometry.h), one workgroup of kSmallLanes lanes per volume (FusedArgs' tile and chunk
// fields unused).
hipError_t launch_small(int halo, int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st);

// box3d (nfields = 1, fp32 out) and the reference backward combine (nfields = 3): workgroups of
// kBoxLanes lanes, one per 16 x 16 tile of one volume
constexpr int kBoxLanes = 256;
hipError_t launch_box(int halo, int nfields, bool bf16, const BoxArgs& a, uint32_t nblocks, hipStream_t st);
hipError_t launch_finalize(const double* partials, int nparts, double inv_m, float* loss, hipStream_t st);
hipError_t launch_scale(void* grad, bool bf16, int64_t n, const float* grad_out, hipStream_t st);

}  // namespace fl
