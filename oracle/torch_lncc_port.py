"""The reference's naive PyTorch LNCC restated (dense box-sum + autograd) — TEST/BASELINE ONLY.

Follows baselines/torch_lncc.py:12-37 (``_box_dense``: one grouped ``F.conv3d`` with a ones
kernel and zero padding k//2; ``_lncc``: cross, var_p, var_t with dr, ncc clamped at 1,
loss 1 - mean). It is the CPU baseline leg of bench.py and is pinned to the reference by the
golden vectors in tests/test_oracle.py. The product path never imports it.
"""
import torch
import torch.nn.functional as F


def box_dense(x, k):
    c = x.shape[1]
    return F.conv3d(x, x.new_ones(c, 1, k, k, k), padding=k // 2, groups=c)


def lncc_dense(pred, target, kernel_size=7, smooth_dr=1e-5):
    n = kernel_size ** 3
    sp, st = box_dense(pred, kernel_size), box_dense(target, kernel_size)
    cross = box_dense(pred * target, kernel_size) - sp * st / n
    vp = box_dense(pred * pred, kernel_size) - sp * sp / n + smooth_dr
    vt = box_dense(target * target, kernel_size) - st * st / n + smooth_dr
    ncc = ((cross * cross) / (vp * vt)).clamp(max=1.0)
    return 1.0 - ncc.mean()


def loss_and_grad(pred, target, kernel_size=7, smooth_dr=1e-5):
    p = pred.detach().clone().requires_grad_(True)
    loss = lncc_dense(p, target, kernel_size, smooth_dr)
    loss.backward()
    return loss.detach(), p.grad
