"""Dense 3D image registration with the fused LNCC loss as the optimized similarity.

The consumer of the loss that the reference demonstrates end to end
(examples/registration_demo.py:19-64): a displacement field is optimized with Adam so that
``warp(moving, disp)`` matches ``fixed`` under ``loss = lncc(warped, fixed) + lam * diffusion(disp)``.
The warp is trilinear ``grid_sample``; the regularizer is the mean squared finite difference of
the field along each axis. Nothing here is specific to the GPU beyond the loss.

    python fused-lncc_amd/examples/registration.py --size 96 --iters 150 [--graph]

prints ms per iteration, peak memory, and the MSE and LNCC similarity (1 - loss) before and after.
"""
import argparse
import os
import sys
import time

import torch
import torch.nn.functional as F

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from fused_lncc import fused_lncc_loss  # noqa: E402


def identity_grid(shape, device):
    """(1, D, H, W, 3) sampling grid of the identity map in grid_sample's (x, y, z) order."""
    theta = torch.tensor([[[1.0, 0, 0, 0], [0, 1.0, 0, 0], [0, 0, 1.0, 0]]], device=device)
    return F.affine_grid(theta, (1, 1, *shape), align_corners=True)


def warp(vol, disp, grid):
    """vol (1,1,D,H,W) sampled at grid + disp; disp (1,3,D,H,W) in normalized units."""
    return F.grid_sample(vol, grid + disp.permute(0, 2, 3, 4, 1), mode="bilinear",
                         padding_mode="border", align_corners=True)


def box_blur(x, r, passes=3):
    """Edge-replicated box filter of radius r along the last three axes, applied `passes` times
    (close to a Gaussian of sigma ~ r * sqrt(passes / 3)); cumulative sums, no convolution."""
    for _ in range(passes):
        for dim in (-3, -2, -1):
            n = x.shape[dim]
            lo = x.narrow(dim, 0, 1).expand(*x.shape[:dim % x.dim()], r + 1, *x.shape[dim % x.dim() + 1:])
            hi = x.narrow(dim, n - 1, 1).expand(*x.shape[:dim % x.dim()], r, *x.shape[dim % x.dim() + 1:])
            c = torch.cat([lo, x, hi], dim).cumsum(dim)
            x = (c.narrow(dim, 2 * r + 1, n) - c.narrow(dim, 0, n)) / (2 * r + 1)
    return x


def smooth_random_field(shape, amp, r, generator, device):
    f = torch.randn(shape, generator=generator).to(device)
    f = box_blur(f, r)
    return amp * f / (f.std() + 1e-6)


def diffusion(disp):
    """Mean squared forward difference of the field along D, H and W."""
    return sum((disp.diff(dim=d) ** 2).mean() for d in (2, 3, 4))


def make_pair(size, device, seed=0, amp=0.06):
    """A structured fixed volume in [0, 1] and a moving volume = fixed warped by a known smooth
    displacement."""
    g = torch.Generator().manual_seed(seed)
    fixed = smooth_random_field((1, 1, size, size, size), 1.0, max(1, size // 32), g, device)
    fixed = (fixed - fixed.min()) / (fixed.max() - fixed.min())
    grid = identity_grid((size, size, size), device)
    true_disp = smooth_random_field((1, 3, size, size, size), amp, max(2, size // 12), g, device)
    moving = warp(fixed, true_disp, grid).detach()
    return fixed, moving, grid


def objective(disp, fixed, moving, grid, k=7, lam=0.5):
    return fused_lncc_loss(warp(moving, disp, grid), fixed, k) + lam * diffusion(disp)


def register(fixed, moving, grid, iters=150, lr=0.02, lam=0.5, k=7, capturable=False):
    """Adam on the displacement field; returns the field and ms per iteration (timed from the
    second iteration on: the first one carries one-time initialization of the backward kernels
    and the optimizer state). capturable selects Adam's graph-safe implementation (the one
    register_graph must use; its arithmetic differs from the default one in the last bits)."""
    disp = torch.zeros(1, 3, *fixed.shape[2:], device=fixed.device, requires_grad=True)
    opt = torch.optim.Adam([disp], lr=lr, capturable=capturable)
    t0 = None
    for i in range(iters):
        if i == 1:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        opt.zero_grad(set_to_none=True)
        objective(disp, fixed, moving, grid, k, lam).backward()
        opt.step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / (iters - 1) * 1e3 if t0 is not None else float("nan")
    return disp.detach(), ms


def register_graph(fixed, moving, grid, iters=150, lr=0.02, lam=0.5, k=7):
    """The same optimization with one iteration (objective, backward, Adam step) captured in a HIP
    graph and replayed: the host's per-iteration work (autograd, dozens of small launches) is gone,
    which is most of an iteration at 96^3. Returns the field and ms per iteration (replays only)."""
    disp = torch.zeros(1, 3, *fixed.shape[2:], device=fixed.device, requires_grad=True)
    opt = torch.optim.Adam([disp], lr=lr, capturable=True)
    # warm up on a side stream (allocates Adam's state), then start from zero again
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            opt.zero_grad(set_to_none=False)
            objective(disp, fixed, moving, grid, k, lam).backward()
            opt.step()
    torch.cuda.current_stream().wait_stream(s)
    with torch.no_grad():
        disp.zero_()
        for st in opt.state[disp].values():
            st.zero_()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        opt.zero_grad(set_to_none=False)  # a fill kernel, replayed with the rest
        objective(disp, fixed, moving, grid, k, lam).backward()
        opt.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        g.replay()
    torch.cuda.synchronize()
    return disp.detach().clone(), (time.perf_counter() - t0) / iters * 1e3


@torch.no_grad()
def quality(fixed, moving, disp, grid, k=7):
    """(MSE, LNCC similarity = 1 - loss) of the warped moving volume against fixed."""
    w = warp(moving, disp, grid)
    return F.mse_loss(w, fixed).item(), 1.0 - fused_lncc_loss(w, fixed, k).item()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--size", type=int, default=96)
    ap.add_argument("--iters", type=int, default=150)
    ap.add_argument("--k", type=int, default=7)
    ap.add_argument("--graph", action="store_true", help="replay one captured iteration (HIP graph)")
    a = ap.parse_args()
    fixed, moving, grid = make_pair(a.size, "cuda")
    zero = torch.zeros(1, 3, a.size, a.size, a.size, device="cuda")
    mse0, sim0 = quality(fixed, moving, zero, grid, a.k)
    torch.cuda.reset_peak_memory_stats()
    disp, ms = (register_graph if a.graph else register)(fixed, moving, grid, a.iters, k=a.k)
    peak = torch.cuda.max_memory_allocated() / 1e9
    mse1, sim1 = quality(fixed, moving, disp, grid, a.k)
    mode = "graph replay" if a.graph else "eager"
    print(f"{a.size}^3, {a.iters} Adam iterations ({mode}), k={a.k}: {ms:.2f} ms/iter, peak {peak:.2f} GB")
    print(f"  before: MSE {mse0:.4e}  LNCC similarity {sim0:.4f}")
    print(f"  after:  MSE {mse1:.4e}  LNCC similarity {sim1:.4f}")


if __name__ == "__main__":
    main()
