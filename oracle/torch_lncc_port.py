"""The reference's naive PyTorch LNCC restated (dense box-sum + autograd) — TEST/BASELINE ONLY.

Follows baselines/torch_lncc.py:12-42: zero-padded k^3 box sums from a dense grouped convolution
with a kernel of ones (padding k//2), or from three 1-D ones convolutions (the separable variant),
cross = Spt - Sp St/n, variances with dr added and no clamp,
ncc clamped at 1, loss 1 - mean. One convolution per field, as in the reference (a single
convolution over the five stacked fields takes a grouped path that is several times slower on the
CPU, which would misstate the baseline). It is the CPU baseline leg of bench.py and is pinned to
the reference by the golden vectors in tests/test_oracle.py. The product path never imports it.
"""
import torch
import torch.nn.functional as F


def box_dense(x, k):
    """Zero-padded k^3 box sum of every channel of an (N, C, D, H, W) tensor."""
    ones = torch.ones((x.shape[1], 1, k, k, k), dtype=x.dtype, device=x.device)
    return F.conv3d(x, ones, padding=k // 2, groups=x.shape[1])


def box_separable(x, k):
    """The same box sum as three 1-D grouped convolutions of ones, along D, then H, then W, with
    'same' (zero) padding (baselines/torch_lncc.py:17-22)."""
    c = x.shape[1]
    for shape in ((c, 1, k, 1, 1), (c, 1, 1, k, 1), (c, 1, 1, 1, k)):
        x = F.conv3d(x, torch.ones(shape, dtype=x.dtype, device=x.device), padding="same", groups=c)
    return x


def _lncc(pred, target, kernel_size, smooth_dr, box):
    n = kernel_size ** 3
    fields = (pred, target, pred * target, pred * pred, target * target)
    s_p, s_t, s_pt, s_pp, s_tt = (box(f, kernel_size) for f in fields)
    cov = s_pt - s_p * s_t / n
    var_p = s_pp - s_p * s_p / n + smooth_dr
    var_t = s_tt - s_t * s_t / n + smooth_dr
    ncc = torch.clamp(cov * cov / (var_p * var_t), max=1.0)
    return 1.0 - ncc.mean()


def lncc_dense(pred, target, kernel_size=7, smooth_dr=1e-5):
    """1 - mean(squared local NCC) with autograd to both inputs (baselines/torch_lncc.py:35-37)."""
    return _lncc(pred, target, kernel_size, smooth_dr, box_dense)


def lncc_separable(pred, target, kernel_size=7, smooth_dr=1e-5):
    """The same loss over the separable box sum (baselines/torch_lncc.py:40-42)."""
    return _lncc(pred, target, kernel_size, smooth_dr, box_separable)


def loss_and_grad(pred, target, kernel_size=7, smooth_dr=1e-5):
    """The loss and its gradient with respect to pred (target held fixed)."""
    p = pred.detach().clone().requires_grad_(True)
    loss = lncc_dense(p, target, kernel_size, smooth_dr)
    (grad,) = torch.autograd.grad(loss, p)
    return loss.detach(), grad
