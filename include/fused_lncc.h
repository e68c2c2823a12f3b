/*
 * fused_lncc — C ABI of the MI355X (gfx950) fused 3D LNCC loss library, libfused_lncc_hip.so.
 *
 * Plain pointers and sizes only. All device pointers are HIP device memory of the current
 * device; every call is asynchronous on `stream` (a hipStream_t, NULL = the default stream) and
 * never synchronizes with the host. Volumes are laid out contiguously as (B, D, H, W) with
 * B = N*C independent volumes and W the fastest axis; `dtype` is FL_F32 or FL_BF16.
 *
 * Return value: FL_OK (0) or a negative FL_E* code; fl_last_error() gives a message for the last
 * failing call on the calling thread. Argument errors are detected on the host before any device
 * work is queued.
 */
#ifndef FUSED_LNCC_H
#define FUSED_LNCC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fl_dtype { FL_F32 = 0, FL_BF16 = 1 };

enum fl_status {
    FL_OK = 0,
    FL_E_DTYPE = -1,     /* dtype is not FL_F32 / FL_BF16 */
    FL_E_KSIZE = -2,     /* kernel_size not odd in [3, 9] */
    FL_E_SHAPE = -3,     /* empty or too large a volume */
    FL_E_NULL = -4,      /* a required pointer is NULL */
    FL_E_WORKSPACE = -5, /* workspace smaller than fl_workspace_bytes() */
    FL_E_DEVICE = -6     /* HIP runtime or launch error */
};

/* Library version, (major << 16) | (minor << 8) | patch. */
int fl_version(void);

/* Message of the last failing call on this thread ("" if none). The text is owned by the library
 * and stays valid until the next failing call on the same thread: copy it to keep it. */
const char* fl_last_error(void);

/*
 * Host-only argument check shared by every entry point (no device access).
 * Replaces the input checks of lncc_forward / lncc_backward, fused_lncc/csrc/lncc3d.cu:128-129,
 * 145-148, 158, 255-260, 281, and the asserts of fused_lncc_loss, fused_lncc/__init__.py:81-82.
 */
int fl_validate(int dtype, int kernel_size, int64_t B, int64_t D, int64_t H, int64_t W);

/*
 * Bytes of LDS one workgroup of the gradient kernels uses for this kernel size, the largest of the
 * plane-marching kernel's (with both gradients, its larger form) and the small-volume kernel's
 * (static; 0 for an invalid k or dtype), for
 * callers that check a device's limit before launching. Replaces the
 * per-call shared-memory cap check of lncc_forward / lncc_backward, fused_lncc/csrc/lncc3d.cu:144-147,
 * 268-270 (MI355X: 160 KB per workgroup; every kernel size fits).
 */
size_t fl_lds_bytes(int kernel_size, int dtype);

/* Device bytes of the workspace fl_lncc_loss_grad needs for this shape (per-workgroup partials),
 * for the current device: the launch plan follows the device's compute-unit count. */
size_t fl_workspace_bytes(int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size);

/*
 * The hot path: one fused kernel reads pred and target once and writes
 *   *loss = 1 - mean(ncc)                       (float32, device pointer)
 *   grad  = d loss / d pred                     (pred dtype; skipped when grad == NULL)
 * where ncc is the zero-padded k^3 local squared NCC clamped to 1, followed by a one-workgroup
 * kernel that reduces the per-workgroup partial sums in a fixed order. No intermediate volume is
 * written to HBM. Replaces the pair lncc_forward (fused_lncc/csrc/lncc3d.cu:127-161) +
 * ncc.mean() (fused_lncc/__init__.py:62) and lncc_backward with scale -1/M
 * (lncc3d.cu:253-284, fused_lncc/__init__.py:73).
 */
int fl_lncc_loss_grad(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                      int64_t W, int kernel_size, float smooth_dr, float* loss, void* grad, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * fl_lncc_loss_grad without the workspace argument and without any allocation: the per-workgroup
 * partial sums go to a scratch array in the library's own device memory (512 KiB per GPU, held
 * until the process ends), so the call makes no hipMalloc/hipFree and no allocating library call.
 * No counterpart in the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). Limit: launches of at most
 * 65536 workgroups, i.e. fl_workspace_bytes(...) <= 512 KiB on the target device (e.g. up to 256
 * volumes of 512^3 at k = 7; the workgroup count of small volumes follows the device's compute-unit
 * count, so check fl_workspace_bytes rather than a rule of thumb); larger ones return
 * FL_E_WORKSPACE. The first call on each device looks up the scratch array's device address
 * (hipGetSymbolAddress), which must not happen inside a HIP graph capture: make one call on each
 * device before capturing. Every call on one GPU shares that GPU's scratch: calls that overlap on
 * one GPU (other streams, other threads) race and must be serialized by the caller. Results are
 * bit-identical to fl_lncc_loss_grad's.
 */
int fl_lncc_loss_grad_noalloc(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                              int64_t W, int kernel_size, float smooth_dr, float* loss, void* grad, void* stream);

/*
 * The two launches of fl_lncc_loss_grad, for callers that time or schedule them separately:
 * fl_lncc_fused_partials runs the fused kernel alone (gradient when grad != NULL, one float64 ncc
 * partial sum per workgroup into `workspace`); fl_lncc_finalize reduces those partials in a fixed
 * order into *loss = 1 - sum/M. Same shape arguments as fl_lncc_loss_grad. Both re-plan the launch
 * from the shape, so call them from the same host thread when fl_test_set_dchunk is in effect (its
 * chunk override is per thread; a finalize planned without it would read a different number of
 * partials).
 */
int fl_lncc_fused_partials(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                           int64_t W, int kernel_size, float smooth_dr, void* grad, void* workspace,
                           size_t workspace_bytes, void* stream);
int fl_lncc_finalize(const void* workspace, int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size,
                     float* loss, void* stream);

/*
 * Both gradients: *loss as fl_lncc_loss_grad, grad_pred = d loss / d pred and grad_target =
 * d loss / d target (each in the input dtype, already multiplied by -1/M), all required. No
 * counterpart in the reference, whose gradient goes to pred only (its README.md:116-121); it is
 * the target-side gradient that FireANTs computes for symmetric registration. The loss is symmetric
 * in its two inputs, so the target gradient is the pred gradient with the two swapped. One launch
 * forms both (five adjoint fields instead of three); for volumes of at most 16^3 it is two passes
 * of the pred-gradient kernel. Either way both gradients equal those of two such passes bit for
 * bit. Same workspace as fl_lncc_loss_grad.
 */
int fl_lncc_loss_grad_pt(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H,
                         int64_t W, int kernel_size, float smooth_dr, float* loss, void* grad_pred,
                         void* grad_target, void* workspace, size_t workspace_bytes, void* stream);

/*
 * grad *= *grad_out (device scalar), done on the device and skipped there when *grad_out == 1, so
 * the common loss.backward() path costs one tiny launch and no host sync. Replaces the tensor
 * multiply by -grad_out/M of _FusedLNCC.backward, fused_lncc/__init__.py:73.
 */
int fl_scale_grad(void* grad, int dtype, int64_t n, const float* grad_out, void* stream);

/*
 * Per-voxel maps ncc (clamped), A = dncc/dSp, Bc = dncc/dvar_p, Cc = dncc/dcross as float32,
 * each (B,D,H,W) — the outputs of lncc_forward, fused_lncc/csrc/lncc3d.cu:127-161. A, Bc and Cc
 * may all be NULL: then only the ncc map is written (4 B per voxel; the per-voxel similarity of
 * the evaluation path, examples/registration_demo.py:59-63, and the map checked in
 * tests/verify_fwd.py:21-34).
 */
int fl_lncc_maps(const void* pred, const void* target, int dtype, int64_t B, int64_t D, int64_t H, int64_t W,
                 int kernel_size, float smooth_dr, float* ncc, float* A, float* Bc, float* Cc, void* stream);

/*
 * grad = scale * (box(A) + 2 pred box(Bc) + target box(Cc)) in the pred dtype from float32 maps —
 * lncc_backward, fused_lncc/csrc/lncc3d.cu:253-284. Debug/test path.
 */
int fl_lncc_backward(const float* A, const float* Bc, const float* Cc, const void* pred, const void* target,
                     int dtype, int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size, float scale,
                     void* grad, void* stream);

/* y = zero-padded k^3 box-sum of x, float32 — box3d_sep_forward, fused_lncc/csrc/lncc3d.cu:329-344. */
int fl_box3d(const float* x, float* y, int64_t B, int64_t D, int64_t H, int64_t W, int kernel_size, void* stream);

/*
 * Test hook, no counterpart in the reference: makes every launch planned afterwards on the calling
 * thread split D into chunks of `planes` output planes (clamped to D; 0 restores the launch
 * planner, which picks the split for the device's compute-unit count). Tests use it to put chunk
 * seams into small volumes and to march long volumes unsplit. Thread-local: other threads keep
 * the planner. Returns FL_OK, or FL_E_SHAPE for a negative length.
 */
int fl_test_set_dchunk(int planes);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_LNCC_H */
