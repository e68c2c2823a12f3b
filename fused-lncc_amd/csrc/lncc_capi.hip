// C ABI of libfused_lncc_hip.so (declared in include/fused_lncc.h): host-side validation, launch
// planning (tiles, D-chunks), and the launches. No allocation and no host synchronization.
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <string>

#include "../../include/fused_lncc.h"
#include "lncc_common.h"
#include "lncc_launch.h"

namespace {

thread_local std::string g_err;
thread_local int64_t t_dchunk_override = 0;  // fl_test_set_dchunk; 0 = the planner's choice

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return FL_E_DEVICE;
}

constexpr int64_t kMaxPlaneBytes = 0x7fffffffLL;  // per-plane buffer offsets are 31-bit

struct Plan {
    int ntx, nty, nzc, dchunk;
    int64_t nblocks;
    bool small;   // the small-volume kernel: one workgroup per volume
};

// Compute units of the current device, read once per device (256 on an MI355X in its
// single-partition mode, fewer in a partitioned one); 256 when no device is visible, so that
// host-only callers (the workspace-size query in a build environment) still get a plan.
int device_cus() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Workgroups: B volumes x (W/TX) x (H/TY) tiles x D-chunks. A chunk of d output planes costs
// d + 4h + 3 pipeline steps (it recomputes the halo planes of its neighbours), so D is split only
// where that shortens the launch: small volumes, whose tiles alone leave CUs idle, get short chunks.
// fl_test_set_dchunk fixes the chunk length for the calling thread (tests of chunk seams and of
// long unsplit marches).
Plan plan_fused(int64_t B, int64_t D, int64_t H, int64_t W, int halo) {
    Plan p;
    // Volumes of at most 16 x 16 x 16 go to the small-volume kernel (whole volume in LDS, one
    // workgroup each), unless a test fixes the plane-marching kernel's chunk length.
    p.small = D <= fl::kSmallEdge && H <= fl::kSmallEdge && W <= fl::kSmallEdge && t_dchunk_override == 0;
    if (p.small) {
        p.ntx = p.nty = p.nzc = 1;
        p.dchunk = (int)D;
        p.nblocks = B;
        return p;
    }
    const int ty = fl::tile_rows(halo);
    p.ntx = (int)((W + fl::TX - 1) / fl::TX);
    p.nty = (int)((H + ty - 1) / ty);
    // callers pass shapes that passed check_grid, so base < 2^32 / NT; a forced chunk length can
    // multiply it by up to D <= 2^30, which still fits int64
    const int64_t base = B * p.ntx * p.nty;
    // Split D into nzc chunks. A chunk of d planes costs d + 4h + 3 pipeline steps, and the
    // workgroups run in rounds of one per CU: pick the split with the fewest rounds x steps (ties:
    // fewer workgroups).
    const int64_t kCUs = device_cus();
    int64_t best_cost = -1, dchunk = D;
    for (int64_t nzc = 1; nzc <= D; ++nzc) {
        const int64_t d = (D + nzc - 1) / nzc;
        const int64_t blocks = base * ((D + d - 1) / d);
        const int64_t cost = ((blocks + kCUs - 1) / kCUs) * (d + 4 * halo + 3);
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            dchunk = d;
        }
        if (blocks >= 8 * kCUs) break;
    }
    if (t_dchunk_override > 0) dchunk = t_dchunk_override < D ? t_dchunk_override : D;
    p.dchunk = (int)dchunk;
    p.nzc = (int)((D + dchunk - 1) / dchunk);
    p.nblocks = base * p.nzc;
    return p;
}

// A launch of n workgroups of `lanes` lanes: the grid in lanes must fit in 32 bits.
bool grid_fits(int64_t n, int lanes) { return n >= 1 && n <= (int64_t)0xffffffffLL / lanes; }

// elem = bytes per element of the volumes; callers that do not know the dtype (workspace size,
// finalize) pass the smallest, 2, and the launch that reads the volumes checks its own dtype.
int check_shape(int64_t B, int64_t D, int64_t H, int64_t W, int elem) {
    if (B < 1 || D < 1 || H < 1 || W < 1) return fail(FL_E_SHAPE, "fused_lncc: empty volume (B, D, H, W must be >= 1)");
    if (H > kMaxPlaneBytes || W > kMaxPlaneBytes || H * W * elem > kMaxPlaneBytes)
        return fail(FL_E_SHAPE, "fused_lncc: one (H, W) plane exceeds 2 GiB");
    if (D > (1 << 30) || B > (1LL << 40))
        return fail(FL_E_SHAPE, "fused_lncc: too many planes or volumes (D <= 2^30, B <= 2^40)");
    return FL_OK;
}

// B x ntx x nty workgroups, or -1 if the product does not fit int64 (check_shape allows B up to
// 2^40 and planes of up to 2^30 columns, whose product can exceed 2^63).
int64_t workgroups(int64_t B, int64_t ntx, int64_t nty) {
    int64_t plane = 0, n = 0;
    if (__builtin_mul_overflow(ntx, nty, &plane) || __builtin_mul_overflow(plane, B, &n)) return -1;
    return n;
}

// Tiles of the fused kernel: B x (W/TX) x (H/TY).
int64_t tile_count(int64_t B, int64_t H, int64_t W, int halo) {
    return workgroups(B, (W + fl::TX - 1) / fl::TX, (H + fl::tile_rows(halo) - 1) / fl::tile_rows(halo));
}

// The fused kernel's smallest plan (one workgroup per tile and volume, D unsplit) must fit one
// launch.
int check_grid(int64_t B, int64_t H, int64_t W, int halo) {
    if (!grid_fits(tile_count(B, H, W, halo), fl::NT))
        return fail(FL_E_SHAPE, "fused_lncc: too many volumes/tiles for one launch");
    return FL_OK;
}

int check_k(int k) {
    if (k < 3 || k > 9 || (k % 2) == 0)
        return fail(FL_E_KSIZE, "fused_lncc: kernel_size must be odd and in 3..9, got " + std::to_string(k));
    return FL_OK;
}

int check_dtype(int dtype) {
    if (dtype != FL_F32 && dtype != FL_BF16)
        return fail(FL_E_DTYPE, "fused_lncc: float32 or bfloat16 only (dtype code " + std::to_string(dtype) + ")");
    return FL_OK;
}

hipError_t launch_fused(int halo, int mode, bool bf16, const fl::FusedArgs& a, const Plan& p, hipStream_t st) {
    const uint32_t nb = (uint32_t)p.nblocks;
    if (p.small) return fl::launch_small(halo, mode, bf16, a, nb, st);
    switch (halo) {
        case 1: return fl::launch_fused_h1(mode, bf16, a, nb, st);
        case 2: return fl::launch_fused_h2(mode, bf16, a, nb, st);
        case 3: return fl::launch_fused_h3(mode, bf16, a, nb, st);
        case 4: return fl::launch_fused_h4(mode, bf16, a, nb, st);
        default: return hipErrorInvalidValue;
    }
}

// Kernel arguments shared by every mode of the fused kernel; mode-specific outputs are set by the
// caller.
fl::FusedArgs fused_args(const void* pred, const void* target, int64_t B, int64_t D, int64_t H, int64_t W,
                         int kernel_size, float smooth_dr, const Plan& p) {
    const double M = (double)B * (double)D * (double)H * (double)W;
    const double n = (double)kernel_size * kernel_size * kernel_size;
    fl::FusedArgs a = {};
    a.pred = pred;
    a.target = target;
    a.dimD = (int)D;
    a.dimH = (int)H;
    a.dimW = (int)W;
    a.ntx = p.ntx;
    a.nty = p.nty;
    a.nzc = p.nzc;
    a.dchunk = p.dchunk;
    a.inv_n = (float)(1.0 / n);
    a.nf = (float)n;
    a.ndr = (float)n * smooth_dr;
    a.gscale = (float)(2.0 * n / M) * fl::range_scale(kernel_size);   // a power of two: exact
    return a;
}

// The fused kernel's plan for this call, checked against the 32-bit grid limit (a forced short
// chunk can multiply the workgroups of a plan).
int planned(int64_t B, int64_t D, int64_t H, int64_t W, int halo, Plan& p, const char* who) {
    p = plan_fused(B, D, H, W, halo);
    if (!grid_fits(p.nblocks, fl::NT)) return fail(FL_E_SHAPE, std::string(who) + ": too many workgroups for one launch");
    return FL_OK;
}

// Scratch of the allocation-free entry point: the per-workgroup ncc partial sums of one launch of
// the fused kernel, in the library's own device memory. Every call on a device shares that
// device's copy (calls that overlap on one GPU race); each launch writes the slots it reads, so
// nothing needs clearing between calls.
constexpr int64_t kScratchPartials = 65536;  // 512 KiB of float64 per device
static __device__ __align__(256) double scratch[kScratchPartials];

// The device address of `scratch` on each device, looked up once per device with that device
// current (each GPU holds its own copy at its own address). Host code uses this address, never the
// array's name, which on the host is only a stand-in.
constexpr int kMaxScratchDevices = 64;
std::atomic<double*> g_scratch_ptr[kMaxScratchDevices];

int scratch_on_current_device(double** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_loss_grad_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(FL_E_DEVICE, "fl_lncc_loss_grad_noalloc: device index " + std::to_string(dev) + " out of range");
    double* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* addr = nullptr;
        e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || addr == nullptr) return hip_fail(e, "fl_lncc_loss_grad_noalloc: hipGetSymbolAddress(scratch)");
        p = static_cast<double*>(addr);
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return FL_OK;
}

}  // namespace

extern "C" {

int fl_version(void) { return (0 << 16) | (2 << 8) | 0; }

int fl_test_set_dchunk(int planes) {
    if (planes < 0) return fail(FL_E_SHAPE, "fl_test_set_dchunk: negative chunk length");
    t_dchunk_override = planes;
    return FL_OK;
}

const char* fl_last_error(void) { return g_err.c_str(); }

int fl_validate(int dtype, int kernel_size, int64_t B, int64_t D, int64_t H, int64_t W) {
    int rc = check_dtype(dtype);
    if (rc) return rc;
    rc = check_k(kernel_size);
    if (rc) return rc;
    rc = check_shape(B, D, H, W, dtype == FL_BF16 ? 2 : 4);
    if (rc) return rc;
    return check_grid(B, H, W, kernel_size / 2);
}

size_t fl_lds_bytes(int kernel_size, int dtype) {
    if (check_k(kernel_size) || check_dtype(dtype)) return 0;
    // the static LDS of the gradient kernels: the plane-marching kernel's five z-sum and x-sum
    // planes, the adjoint planes at each pass (five fields for both gradients, the larger), and the
    // per-wave partials of the loss (the same for both dtypes); the small-volume kernel's five 16^3
    // fields (the first three reused for the adjoints), three more for the adjoint pass, and its
    // per-wave partials. The largest of them.
    size_t floats = 0;
    switch (kernel_size / 2) {
        case 1: floats = fl::Geo<1, 5>::LDS_FLOATS; break;
        case 2: floats = fl::Geo<2, 5>::LDS_FLOATS; break;
        case 3: floats = fl::Geo<3, 5>::LDS_FLOATS; break;
        default: floats = fl::Geo<4, 5>::LDS_FLOATS; break;
    }
    const size_t marching = floats * sizeof(float) + (fl::NT / 64) * sizeof(double);
    const size_t small = (size_t)8 * fl::kSmallEdge * fl::kSmallEdge * fl::kSmallEdge * sizeof(float) +
                         (fl::kSmallLanes / 64) * sizeof(double);
    return marching > small ? marching : small;
}

size_t fl_workspace_bytes(int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size) {
    if (check_k(kernel_size) || check_shape(B, D, H, W, 2) || check_grid(B, H, W, kernel_size / 2)) return 0;
    Plan p;
    if (planned(B, D, H, W, kernel_size / 2, p, "fl_workspace_bytes")) return 0;
    return (size_t)p.nblocks * sizeof(double);
}

int fl_lncc_fused_partials(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                           int64_t W, int kernel_size, float smooth_dr, void* grad, void* workspace,
                           size_t workspace_bytes, void* stream) {
    int rc = fl_validate(dtype, kernel_size, B, D, H, W);
    if (rc) return rc;
    if (!pred || !target || !workspace) return fail(FL_E_NULL, "fl_lncc_fused_partials: NULL pointer argument");
    const int halo = kernel_size / 2;
    Plan p;
    rc = planned(B, D, H, W, halo, p, "fl_lncc_fused_partials");
    if (rc) return rc;
    if (workspace_bytes < (size_t)p.nblocks * sizeof(double))
        return fail(FL_E_WORKSPACE, "fl_lncc_fused_partials: workspace needs " +
                                        std::to_string((size_t)p.nblocks * sizeof(double)) + " bytes");
    fl::FusedArgs a = fused_args(pred, target, B, D, H, W, kernel_size, smooth_dr, p);
    a.grad = grad;
    a.partials = static_cast<double*>(workspace);
    hipError_t e = launch_fused(halo, grad ? fl::MODE_GRAD : fl::MODE_LOSS, dtype == FL_BF16, a, p,
                                static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_fused_partials: fused kernel launch");
    return FL_OK;
}

int fl_lncc_finalize(const void* workspace, int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size,
                     float* loss, void* stream) {
    int rc = check_k(kernel_size);
    if (!rc) rc = check_shape(B, D, H, W, 2);
    if (!rc) rc = check_grid(B, H, W, kernel_size / 2);
    if (rc) return rc;
    if (!workspace || !loss) return fail(FL_E_NULL, "fl_lncc_finalize: NULL pointer argument");
    Plan p;
    rc = planned(B, D, H, W, kernel_size / 2, p, "fl_lncc_finalize");
    if (rc) return rc;
    const double M = (double)B * (double)D * (double)H * (double)W;
    hipError_t e = fl::launch_finalize(static_cast<const double*>(workspace), (int)p.nblocks, 1.0 / M, loss,
                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_finalize: launch");
    return FL_OK;
}

int fl_lncc_loss_grad(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                      int64_t W, int kernel_size, float smooth_dr, float* loss, void* grad, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (!loss) {
        int rc = fl_validate(dtype, kernel_size, B, D, H, W);
        return rc ? rc : fail(FL_E_NULL, "fl_lncc_loss_grad: NULL pointer argument");
    }
    int rc = fl_lncc_fused_partials(pred, target, dtype, B, D, H, W, kernel_size, smooth_dr, grad, workspace,
                                    workspace_bytes, stream);
    if (rc) return rc;
    return fl_lncc_finalize(workspace, B, D, H, W, kernel_size, loss, stream);
}

int fl_lncc_loss_grad_noalloc(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                              int64_t W, int kernel_size, float smooth_dr, float* loss, void* grad, void* stream) {
    int rc = fl_validate(dtype, kernel_size, B, D, H, W);
    if (rc) return rc;
    if (!pred || !target || !loss) return fail(FL_E_NULL, "fl_lncc_loss_grad_noalloc: NULL pointer argument");
    const int halo = kernel_size / 2;
    Plan p;
    rc = planned(B, D, H, W, halo, p, "fl_lncc_loss_grad_noalloc");
    if (rc) return rc;
    if (p.nblocks > kScratchPartials)
        return fail(FL_E_WORKSPACE, "fl_lncc_loss_grad_noalloc: the launch needs " + std::to_string(p.nblocks) +
                                        " partial sums, the library's scratch holds " + std::to_string(kScratchPartials) +
                                        "; use fl_lncc_loss_grad with a workspace");
    double* part = nullptr;
    rc = scratch_on_current_device(&part);
    if (rc) return rc;
    fl::FusedArgs a = fused_args(pred, target, B, D, H, W, kernel_size, smooth_dr, p);
    a.grad = grad;
    a.partials = part;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = launch_fused(halo, grad ? fl::MODE_GRAD : fl::MODE_LOSS, dtype == FL_BF16, a, p, st);
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_loss_grad_noalloc: fused kernel launch");
    const double M = (double)B * (double)D * (double)H * (double)W;
    e = fl::launch_finalize(part, (int)p.nblocks, 1.0 / M, loss, st);
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_loss_grad_noalloc: finalize launch");
    return FL_OK;
}

int fl_lncc_loss_grad_pt(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                         int64_t W, int kernel_size, float smooth_dr, float* loss, void* grad_pred,
                         void* grad_target, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = fl_validate(dtype, kernel_size, B, D, H, W);
    if (rc) return rc;
    if (!pred || !target || !loss || !grad_pred || !grad_target || !workspace)
        return fail(FL_E_NULL, "fl_lncc_loss_grad_pt: NULL pointer argument");
    const int halo = kernel_size / 2;
    Plan p;
    rc = planned(B, D, H, W, halo, p, "fl_lncc_loss_grad_pt");
    if (rc) return rc;
    if (!p.small) {
        // one launch of the plane-marching kernel for both gradients
        if (workspace_bytes < (size_t)p.nblocks * sizeof(double))
            return fail(FL_E_WORKSPACE, "fl_lncc_loss_grad_pt: workspace needs " +
                                            std::to_string((size_t)p.nblocks * sizeof(double)) + " bytes");
        fl::FusedArgs a = fused_args(pred, target, B, D, H, W, kernel_size, smooth_dr, p);
        a.grad = grad_pred;
        a.grad_t = grad_target;
        a.partials = static_cast<double*>(workspace);
        hipError_t e = launch_fused(halo, fl::MODE_DUAL, dtype == FL_BF16, a, p, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "fl_lncc_loss_grad_pt: fused kernel launch");
        return fl_lncc_finalize(workspace, B, D, H, W, kernel_size, loss, stream);
    }
    // small volumes: the pred pass with the loss, then the same kernel with pred and target
    // swapped (the loss is symmetric in its inputs); the second pass's partials are not reduced
    rc = fl_lncc_loss_grad(pred, target, dtype, B, D, H, W, kernel_size, smooth_dr, loss, grad_pred, workspace,
                           workspace_bytes, stream);
    if (rc) return rc;
    return fl_lncc_fused_partials(target, pred, dtype, B, D, H, W, kernel_size, smooth_dr, grad_target, workspace,
                                  workspace_bytes, stream);
}

int fl_scale_grad(void* grad, int dtype, int64_t n, const float* grad_out, void* stream) {
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if (n < 0) return fail(FL_E_SHAPE, "fl_scale_grad: negative element count");
    if (n == 0) return FL_OK;
    if (!grad || !grad_out) return fail(FL_E_NULL, "fl_scale_grad: NULL pointer argument");
    hipError_t e = fl::launch_scale(grad, dtype == FL_BF16, n, grad_out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fl_scale_grad: launch");
    return FL_OK;
}

int fl_lncc_maps(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H, int64_t W,
                 int kernel_size, float smooth_dr, float* ncc, float* A, float* Bc, float* Cc, void* stream) {
    int rc = fl_validate(dtype, kernel_size, B, D, H, W);
    if (rc) return rc;
    const bool adjoint_maps = A || Bc || Cc;
    if (!pred || !target || !ncc || (adjoint_maps && !(A && Bc && Cc)))
        return fail(FL_E_NULL, "fl_lncc_maps: NULL pointer argument (A, Bc, Cc are all given or all NULL)");
    const int halo = kernel_size / 2;
    Plan p;
    rc = planned(B, D, H, W, halo, p, "fl_lncc_maps");
    if (rc) return rc;
    fl::FusedArgs a = fused_args(pred, target, B, D, H, W, kernel_size, smooth_dr, p);
    a.ncc_map = ncc;
    a.a_map = A;
    a.b_map = Bc;
    a.c_map = Cc;
    hipError_t e = launch_fused(halo, fl::MODE_MAPS, dtype == FL_BF16, a, p,
                                static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_maps: launch");
    return FL_OK;
}

int fl_lncc_backward(const float* A, const float* Bc, const float* Cc, const void* pred, const void* target,
                     int dtype, int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size, float scale,
                     void* grad, void* stream) {
    int rc = fl_validate(dtype, kernel_size, B, D, H, W);
    if (rc) return rc;
    if (!A || !Bc || !Cc || !pred || !target || !grad) return fail(FL_E_NULL, "fl_lncc_backward: NULL pointer argument");
    fl::BoxArgs a = {};
    a.f0 = A;
    a.f1 = Bc;
    a.f2 = Cc;
    a.pred = pred;
    a.target = target;
    a.out = grad;
    a.dimD = (int)D;
    a.dimH = (int)H;
    a.dimW = (int)W;
    a.ntx = (int)((W + 15) / 16);
    a.nty = (int)((H + 15) / 16);
    a.scale = scale;
    if (!grid_fits(workgroups(B, a.ntx, a.nty), fl::kBoxLanes))
        return fail(FL_E_SHAPE, "fl_lncc_backward: too many volumes/tiles for one launch");
    const uint32_t nb = (uint32_t)(B * a.ntx * a.nty);
    hipError_t e = fl::launch_box(kernel_size / 2, 3, dtype == FL_BF16, a, nb, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fl_lncc_backward: launch");
    return FL_OK;
}

int fl_box3d(const float* x, float* y, int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size, void* stream) {
    int rc = fl_validate(FL_F32, kernel_size, B, D, H, W);
    if (rc) return rc;
    if (!x || !y) return fail(FL_E_NULL, "fl_box3d: NULL pointer argument");
    fl::BoxArgs a = {};
    a.f0 = x;
    a.out = y;
    a.dimD = (int)D;
    a.dimH = (int)H;
    a.dimW = (int)W;
    a.ntx = (int)((W + 15) / 16);
    a.nty = (int)((H + 15) / 16);
    a.scale = 1.f;
    if (!grid_fits(workgroups(B, a.ntx, a.nty), fl::kBoxLanes))
        return fail(FL_E_SHAPE, "fl_box3d: too many volumes/tiles for one launch");
    const uint32_t nb = (uint32_t)(B * a.ntx * a.nty);
    hipError_t e = fl::launch_box(kernel_size / 2, 1, false, a, nb, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "fl_box3d: launch");
    return FL_OK;
}

}  // extern "C"
