"""Tensor-level entry points over the C ABI (PyTorch supplies device memory and the stream).

The first three mirror the reference's pybind module ``fused_lncc_cuda``
(fused_lncc/csrc/lncc3d.cu:346-350) — same names, arguments and outputs — for callers and tests
that use it directly. ``loss_grad`` and ``scale_grad_`` are the hot path used by the autograd
function. All of them take contiguous (B, D, H, W) device tensors and launch on the current stream
of the tensors' device.
"""
import torch

from . import _lib

_DTYPES = {torch.float32: _lib.FL_F32, torch.bfloat16: _lib.FL_BF16}


def _dtype_code(t):
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise RuntimeError(f"fused_lncc: float32 or bfloat16 only, got {t.dtype}")
    return code


def _check4d(name, t, like=None, dtype=None):
    if not (t.is_cuda and t.is_contiguous() and t.dim() == 4):
        raise RuntimeError(f"{name} must be a contiguous 4D GPU tensor")
    if like is not None and (t.shape != like.shape or t.device != like.device):
        raise RuntimeError(f"{name} must match the shape and device of the other inputs")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev):
    """Handle of the current stream of `dev` (torch's raw accessor skips building a Stream object,
    ~2 us per call)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


class _on_device:
    """Makes `dev` the current device for the C ABI call (its stream must belong to it); a no-op,
    without the cost of torch.cuda.device's context switch, when it already is."""

    __slots__ = ("dev", "prev")

    def __init__(self, dev):
        self.dev = dev.index if dev.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.dev:
            self.prev = cur
            torch.cuda.set_device(self.dev)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _check_vols(name, t, like=None, dtype=None):
    """A contiguous (B, D, H, W) or (N, C, D, H, W) GPU tensor: volumes of the last three dims."""
    if not (t.is_cuda and t.is_contiguous() and t.dim() in (4, 5)):
        raise RuntimeError(f"{name} must be a contiguous 4D or 5D GPU tensor")
    if like is not None and (t.shape != like.shape or t.device != like.device):
        raise RuntimeError(f"{name} must match the shape and device of the other inputs")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}")


def workspace_bytes(shape, kernel_size):
    B, D, H, W = shape
    return int(_lib.load().fl_workspace_bytes(B, D, H, W, int(kernel_size)))


def loss_grad(pf, tf, kernel_size, smooth_dr, need_grad=True):
    """Fused forward (+ gradient wrt pf, already multiplied by -1/M). Returns (loss, grad|None).
    pf, tf: (B, D, H, W) or (N, C, D, H, W) with B = N*C volumes; grad has the shape of pf.
    Shape, k and dtype are validated by the C ABI before any device work."""
    code = _dtype_code(pf)
    _check_vols("pred", pf)
    _check_vols("target", tf, like=pf, dtype=pf.dtype)
    lib = _lib.load()
    if pf.dim() == 5:
        N, C, D, H, W = pf.shape
        B = N * C
    else:
        B, D, H, W = pf.shape
    k = int(kernel_size)
    with _on_device(pf.device):
        nbytes = lib.fl_workspace_bytes(B, D, H, W, k)
        if nbytes == 0:  # an invalid k or shape: let fl_validate name it
            _lib.check(lib.fl_validate(code, k, B, D, H, W))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=pf.device)
        loss = torch.empty((), dtype=torch.float32, device=pf.device)
        grad = torch.empty_like(pf) if need_grad else None
        _lib.check(lib.fl_lncc_loss_grad(
            pf.data_ptr(), tf.data_ptr(), code, B, D, H, W, k, float(smooth_dr),
            loss.data_ptr(), grad.data_ptr() if grad is not None else None, ws.data_ptr(), nbytes,
            _stream(pf.device)))
    return loss, grad


def loss_grad_pt(pf, tf, kernel_size, smooth_dr):
    """The loss and both gradients (wrt pf and wrt tf, each already multiplied by -1/M) from one
    call: one launch that forms both (the loss is symmetric in its inputs; volumes of at most 16^3
    take the pred-gradient kernel twice, the second time with the inputs swapped). Bit for bit the
    gradients of those two passes. Returns (loss, grad_pred, grad_target)."""
    code = _dtype_code(pf)
    _check_vols("pred", pf)
    _check_vols("target", tf, like=pf, dtype=pf.dtype)
    lib = _lib.load()
    if pf.dim() == 5:
        N, C, D, H, W = pf.shape
        B = N * C
    else:
        B, D, H, W = pf.shape
    k = int(kernel_size)
    with _on_device(pf.device):
        nbytes = lib.fl_workspace_bytes(B, D, H, W, k)
        if nbytes == 0:
            _lib.check(lib.fl_validate(code, k, B, D, H, W))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=pf.device)
        loss = torch.empty((), dtype=torch.float32, device=pf.device)
        gp = torch.empty_like(pf)
        gt = torch.empty_like(tf)
        _lib.check(lib.fl_lncc_loss_grad_pt(
            pf.data_ptr(), tf.data_ptr(), code, B, D, H, W, k, float(smooth_dr), loss.data_ptr(), gp.data_ptr(),
            gt.data_ptr(), ws.data_ptr(), nbytes, _stream(pf.device)))
    return loss, gp, gt


def grad_only(pf, tf, kernel_size, smooth_dr):
    """The gradient of the loss with respect to pf alone (already multiplied by -1/M): the fused
    kernel without the loss reduction. With pf and tf swapped it is the target-side gradient, the
    loss being symmetric in its two inputs."""
    code = _dtype_code(pf)
    _check_vols("pred", pf)
    _check_vols("target", tf, like=pf, dtype=pf.dtype)
    lib = _lib.load()
    if pf.dim() == 5:
        N, C, D, H, W = pf.shape
        B = N * C
    else:
        B, D, H, W = pf.shape
    k = int(kernel_size)
    with _on_device(pf.device):
        nbytes = lib.fl_workspace_bytes(B, D, H, W, k)
        if nbytes == 0:
            _lib.check(lib.fl_validate(code, k, B, D, H, W))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=pf.device)
        grad = torch.empty_like(pf)
        _lib.check(lib.fl_lncc_fused_partials(
            pf.data_ptr(), tf.data_ptr(), code, B, D, H, W, k, float(smooth_dr), grad.data_ptr(),
            ws.data_ptr(), nbytes, _stream(pf.device)))
    return grad


def scale_grad_(grad, grad_out):
    """In place: grad *= grad_out (0-d float32 device tensor), skipped on the device when it is 1."""
    code = _dtype_code(grad)
    go = grad_out.detach()
    if go.dtype != torch.float32 or go.device != grad.device:
        go = go.to(device=grad.device, dtype=torch.float32)
    with _on_device(grad.device):
        _lib.check(_lib.load().fl_scale_grad(grad.data_ptr(), code, grad.numel(), go.data_ptr(),
                                             _stream(grad.device)))
    return grad


def lncc_forward(P, T, kernel_size, dr):
    """[ncc, A, Bc, Cc] float32 maps of (B,D,H,W) inputs — fused_lncc/csrc/lncc3d.cu:127-161."""
    code = _dtype_code(P)
    _check4d("P", P)
    _check4d("T", T, like=P, dtype=P.dtype)
    lib = _lib.load()
    B, D, H, W = P.shape
    _lib.check(lib.fl_validate(code, int(kernel_size), B, D, H, W))
    outs = [torch.empty(P.shape, dtype=torch.float32, device=P.device) for _ in range(4)]
    with torch.cuda.device(P.device):
        _lib.check(lib.fl_lncc_maps(P.data_ptr(), T.data_ptr(), code, B, D, H, W, int(kernel_size),
                                    float(dr), *[o.data_ptr() for o in outs], _stream(P.device)))
    return outs


def ncc_map(P, T, kernel_size, dr):
    """The per-voxel (clamped) squared local NCC of (B,D,H,W) inputs, float32 — the first output of
    lncc_forward without the three adjoint maps."""
    code = _dtype_code(P)
    _check4d("P", P)
    _check4d("T", T, like=P, dtype=P.dtype)
    lib = _lib.load()
    B, D, H, W = P.shape
    _lib.check(lib.fl_validate(code, int(kernel_size), B, D, H, W))
    out = torch.empty(P.shape, dtype=torch.float32, device=P.device)
    with _on_device(P.device):
        _lib.check(lib.fl_lncc_maps(P.data_ptr(), T.data_ptr(), code, B, D, H, W, int(kernel_size),
                                    float(dr), out.data_ptr(), None, None, None, _stream(P.device)))
    return out


def lncc_backward(A, Bc, Cc, P, T, kernel_size, scale):
    """scale * (box A + 2P box Bc + T box Cc) in P's dtype — fused_lncc/csrc/lncc3d.cu:253-284."""
    _check4d("A", A, dtype=torch.float32)
    _check4d("B", Bc, like=A, dtype=torch.float32)
    _check4d("C", Cc, like=A, dtype=torch.float32)
    code = _dtype_code(P)
    _check4d("P", P, like=A)
    _check4d("T", T, like=A, dtype=P.dtype)
    lib = _lib.load()
    B, D, H, W = A.shape
    _lib.check(lib.fl_validate(code, int(kernel_size), B, D, H, W))
    gp = torch.empty_like(P)
    with torch.cuda.device(P.device):
        _lib.check(lib.fl_lncc_backward(A.data_ptr(), Bc.data_ptr(), Cc.data_ptr(), P.data_ptr(),
                                        T.data_ptr(), code, B, D, H, W, int(kernel_size), float(scale),
                                        gp.data_ptr(), _stream(P.device)))
    return gp


def box3d_sep_forward(x, kernel_size):
    """Zero-padded k^3 box-sum of a float32 (B,D,H,W) tensor — fused_lncc/csrc/lncc3d.cu:329-344."""
    _check4d("x", x, dtype=torch.float32)
    lib = _lib.load()
    B, D, H, W = x.shape
    _lib.check(lib.fl_validate(_lib.FL_F32, int(kernel_size), B, D, H, W))
    y = torch.empty_like(x)
    with torch.cuda.device(x.device):
        _lib.check(lib.fl_box3d(x.data_ptr(), y.data_ptr(), B, D, H, W, int(kernel_size), _stream(x.device)))
    return y
