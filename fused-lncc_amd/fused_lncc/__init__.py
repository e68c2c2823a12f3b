"""Fused 3D local (squared) normalized cross-correlation loss for AMD MI355X (gfx950).

Drop-in for the reference's ``fused_lncc`` package (fused_lncc/__init__.py:77-83):

    from fused_lncc import fused_lncc_loss
    loss = fused_lncc_loss(pred, target, kernel_size=7, smooth_dr=1e-5)   # 1 - mean(ncc)
    loss.backward()                                                        # grad to pred only

``pred``/``target`` are (N, C, D, H, W) float32 or bfloat16 tensors on a ROCm device; the loss is a
0-d float32 tensor, the gradient has the pred dtype. The forward runs one hand-written HIP kernel
that reads pred and target once and writes the gradient (already scaled by -1/M) together with
per-workgroup partial sums of ncc; a one-workgroup kernel turns those into the loss. The backward
only multiplies by ``grad_out`` on the device, skipping the work when it is 1, so a
``loss.backward()`` moves 12 bytes per fp32 voxel through HBM and never synchronizes with the host.
"""
import torch

from . import _lib, ext

__all__ = ["fused_lncc_loss", "lncc_map", "ext"]


# Custom ops keep the loss traceable by torch.compile (fused_lncc/__init__.py:22-46). Fake kernels
# give the loss as float32 whatever the input dtype, and the gradient in the input dtype.
@torch.library.custom_op("fused_lncc::loss_grad", mutates_args=())
def _loss_grad_op(pf: torch.Tensor, tf: torch.Tensor, kernel_size: int, smooth_dr: float,
                  need_grad: bool) -> tuple[torch.Tensor, torch.Tensor]:
    loss, grad = ext.loss_grad(pf, tf, kernel_size, smooth_dr, need_grad)
    if grad is None:
        grad = pf.new_empty((0,))
    return loss, grad


@_loss_grad_op.register_fake
def _(pf, tf, kernel_size, smooth_dr, need_grad):
    loss = pf.new_empty((), dtype=torch.float32)
    return loss, (torch.empty_like(pf) if need_grad else pf.new_empty((0,)))


# Both gradients from one launch (target_grad=True): the loss, the pred gradient and the target
# gradient, each gradient in the input dtype.
@torch.library.custom_op("fused_lncc::loss_grad_pt", mutates_args=())
def _loss_grad_pt_op(pf: torch.Tensor, tf: torch.Tensor, kernel_size: int,
                     smooth_dr: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return ext.loss_grad_pt(pf, tf, kernel_size, smooth_dr)


@_loss_grad_pt_op.register_fake
def _(pf, tf, kernel_size, smooth_dr):
    return pf.new_empty((), dtype=torch.float32), torch.empty_like(pf), torch.empty_like(tf)


@torch.library.custom_op("fused_lncc::scale_grad_", mutates_args=("grad",))
def _scale_grad_op(grad: torch.Tensor, grad_out: torch.Tensor) -> None:
    ext.scale_grad_(grad, grad_out)


@_scale_grad_op.register_fake
def _(grad, grad_out):
    return None


# The reference's two building-block ops, same names and signatures (fused_lncc/__init__.py:26-46).
@torch.library.custom_op("fused_lncc::forward", mutates_args=())
def _lncc_forward_op(pf: torch.Tensor, tf: torch.Tensor, kernel_size: int, smooth_dr: float) -> list[torch.Tensor]:
    return ext.lncc_forward(pf, tf, kernel_size, smooth_dr)


@_lncc_forward_op.register_fake
def _(pf, tf, kernel_size, smooth_dr):
    return [torch.empty_like(pf, dtype=torch.float32) for _ in range(4)]


@torch.library.custom_op("fused_lncc::backward", mutates_args=())
def _lncc_backward_op(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, pf: torch.Tensor,
                      tf: torch.Tensor, kernel_size: int, scale: float) -> torch.Tensor:
    return ext.lncc_backward(A, B, C, pf, tf, kernel_size, scale)


@_lncc_backward_op.register_fake
def _(A, B, C, pf, tf, kernel_size, scale):
    return torch.empty_like(pf)


def _compiling():
    try:
        return torch.compiler.is_compiling()
    except AttributeError:  # pragma: no cover
        return False


def _traced(t):
    """True under torch.compile, any dispatch-mode trace (fake tensors, make_fx) or a fake-tensor
    input: the custom ops (with their fake kernels) then stand in for the library calls, so that
    the trace records them. Eager calls on plain tensors skip the op dispatch (~20 us each) and the
    fake-mode search (~5 us)."""
    if _compiling() or torch._C._len_torch_dispatch_stack() > 0:
        return True
    return type(t) is not torch.Tensor and torch._guards.detect_fake_mode((t,)) is not None


class _FusedLNCC(torch.autograd.Function):
    """Autograd wrapper: the gradient is produced in forward by the fused kernel and handed out in
    backward (fused_lncc/__init__.py:49-74 computes it in backward from four saved fp32 maps).
    The optional target-side gradient uses the symmetry of the loss in its two inputs: it is the
    pred-side gradient with pred and target swapped, which one launch forms together with the
    pred-side one (ext.loss_grad_pt)."""

    @staticmethod
    def forward(ctx, pred, target, kernel_size, smooth_dr, need_grad, need_tgrad):
        need = bool(need_grad and ctx.needs_input_grad[0])
        need_t = bool(need_tgrad and ctx.needs_input_grad[1])
        traced = _traced(pred)
        gt = None
        if traced:
            # the registered op takes (B, D, H, W) volumes
            N, C = pred.shape[:2]
            S = pred.shape[2:]
            pf = pred.reshape(N * C, *S)
            tf = target.reshape(N * C, *S)
            if need and need_t:
                loss, grad, gt = torch.ops.fused_lncc.loss_grad_pt(pf, tf, kernel_size, smooth_dr)
            else:
                loss, grad = torch.ops.fused_lncc.loss_grad(pf, tf, kernel_size, smooth_dr, need)
                if need_t:
                    _, gt = torch.ops.fused_lncc.loss_grad(tf, pf, kernel_size, smooth_dr, True)
        else:
            # the library reads (N, C, D, H, W) as N*C volumes; grad comes back in pred's shape
            pf, tf = pred, target
            if need and need_t:  # both gradients from one launch
                loss, grad, gt = ext.loss_grad_pt(pf, tf, kernel_size, smooth_dr)
            else:
                loss, grad = ext.loss_grad(pf, tf, kernel_size, smooth_dr, need)
                if need_t:
                    gt = ext.grad_only(tf, pf, kernel_size, smooth_dr)
        ctx.k = kernel_size
        ctx.dr = smooth_dr
        ctx.shape = pred.shape
        ctx.grad = None
        ctx.tgrad = None
        ctx.need = need
        ctx.need_t = need_t
        ctx.traced = traced
        if need or need_t:
            if _compiling():
                ctx.save_for_backward(pf, tf, grad if need else None, gt)
            else:
                # kept outside save_for_backward so the first backward can scale them in place and
                # hand them to AccumulateGrad without a copy
                ctx.grad = grad if need else None
                ctx.tgrad = gt
                ctx.save_for_backward(pf, tf)
        return loss

    @staticmethod
    def backward(ctx, grad_out):
        g, gt = ctx.grad, ctx.tgrad
        ctx.grad = None
        ctx.tgrad = None
        if not ctx.traced:
            if (ctx.need and g is None) or (ctx.need_t and gt is None):
                # second backward through a retained graph: recompute
                pf, tf = ctx.saved_tensors
                if ctx.need and ctx.need_t:
                    _, g, gt = ext.loss_grad_pt(pf, tf, ctx.k, ctx.dr)
                elif ctx.need:
                    _, g = ext.loss_grad(pf, tf, ctx.k, ctx.dr, True)
                else:
                    gt = ext.grad_only(tf, pf, ctx.k, ctx.dr)
            if g is not None:
                ext.scale_grad_(g, grad_out)
            if gt is not None:
                ext.scale_grad_(gt, grad_out)
            return g, gt, None, None, None, None
        saved = ctx.saved_tensors
        if len(saved) == 4:  # compiled: functional form
            # multiplied in float32 and rounded once, as the eager scale_grad_ kernel does (a bf16
            # grad_out would be rounded before the product)
            sg, sgt = saved[2], saved[3]
            go = grad_out.float()
            g = (sg.float() * go).to(sg.dtype).reshape(ctx.shape) if ctx.need else None
            gt = (sgt.float() * go).to(sgt.dtype).reshape(ctx.shape) if ctx.need_t else None
            return g, gt, None, None, None, None
        pf, tf = saved
        if ctx.need and ctx.need_t and g is None and gt is None:
            _, g, gt = torch.ops.fused_lncc.loss_grad_pt(pf, tf, ctx.k, ctx.dr)
        if ctx.need and g is None:
            _, g = torch.ops.fused_lncc.loss_grad(pf, tf, ctx.k, ctx.dr, True)
        if ctx.need_t and gt is None:
            _, gt = torch.ops.fused_lncc.loss_grad(tf, pf, ctx.k, ctx.dr, True)
        if g is not None:
            torch.ops.fused_lncc.scale_grad_(g, grad_out.detach())
            g = g.reshape(ctx.shape)
        if gt is not None:
            torch.ops.fused_lncc.scale_grad_(gt, grad_out.detach())
            gt = gt.reshape(ctx.shape)
        return g, gt, None, None, None, None


def fused_lncc_loss(pred, target, kernel_size=7, smooth_dr=1e-5, *, target_grad=False):
    """1 - mean(squared local NCC) over all voxels. Gradient flows through ``pred`` only, as in the
    reference, unless ``target_grad=True``.

    pred, target: (N, C, D, H, W) float32 or bfloat16 ROCm tensors; kernel_size odd in 3..9.
    Returns a 0-d float32 loss in [0, 1] (fused_lncc/__init__.py:77-83).

    target_grad (keyword only, not in the reference): also propagate the exact gradient to
    ``target`` when it requires grad, as symmetric registration (both images warped) needs. One
    launch of the fused kernel writes both gradients (about 1.2x the pred-only step at
    (2,16,128^3) k=7); volumes of at most 16^3 take a second pass with pred and target swapped."""
    assert pred.dim() == 5 and pred.shape == target.shape, "expect matching (N,C,D,H,W)"
    assert kernel_size % 2 == 1, "kernel_size must be odd"
    # The gradient is computed in the forward kernel only when autograd will ask for it; under
    # no_grad or for a pred without requires_grad the kernel reads 8 B/voxel and writes nothing.
    grad_on = torch.is_grad_enabled()
    need_grad = grad_on and pred.requires_grad
    need_tgrad = bool(target_grad) and grad_on and target.requires_grad
    return _FusedLNCC.apply(pred.contiguous(), target.contiguous(), kernel_size, smooth_dr, need_grad, need_tgrad)


def lncc_map(pred, target, kernel_size=7, smooth_dr=1e-5):
    """Per-voxel squared local NCC (clamped to 1), float32, shape of ``pred``: the similarity map
    whose mean is ``1 - fused_lncc_loss`` (the evaluation output of the reference's roadmap,
    reduction='none'). Forward only: the map is not differentiable through this call."""
    assert pred.dim() == 5 and pred.shape == target.shape, "expect matching (N,C,D,H,W)"
    assert kernel_size % 2 == 1, "kernel_size must be odd"
    N, C = pred.shape[:2]
    S = pred.shape[2:]
    pf = pred.detach().contiguous().reshape(N * C, *S)
    tf = target.detach().contiguous().reshape(N * C, *S)
    return ext.ncc_map(pf, tf, kernel_size, smooth_dr).reshape(pred.shape)
