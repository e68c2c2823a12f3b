"""The registration consumer of the loss (fused-lncc_amd/examples/registration.py, after the
reference's examples/registration_demo.py:19-64): its gradient with respect to the displacement
field, through grid_sample, matches the same objective built on the oracle in float64 on the CPU,
and a short Adam run improves the alignment."""
import os
import sys

import pytest
import torch

import torch_lncc_port

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fused-lncc_amd", "examples"))
import registration as R  # noqa: E402

pytestmark = pytest.mark.gpu


def test_displacement_gradient_matches_oracle():
    size, k, lam = 20, 5, 0.5
    fixed, moving, grid = R.make_pair(size, "cuda", seed=1)
    g = torch.Generator().manual_seed(2)
    d0 = 0.02 * torch.randn(1, 3, size, size, size, generator=g)

    disp = d0.to("cuda").requires_grad_(True)
    R.objective(disp, fixed, moving, grid, k, lam).backward()
    got = disp.grad.double().cpu()

    dc = d0.double().requires_grad_(True)
    fc, mc, gc = fixed.double().cpu(), moving.double().cpu(), grid.double().cpu()
    ref = torch_lncc_port.lncc_dense(R.warp(mc, dc, gc), fc, k) + lam * R.diffusion(dc)
    ref.backward()
    want = dc.grad
    cos = float((got * want).sum() / (got.norm() * want.norm()))
    rel = float((got - want).norm() / want.norm())
    assert cos > 0.9999 and rel < 1e-3, f"cos={cos:.8f} relL2={rel:.3e}"


def test_short_registration_improves_alignment():
    size = 48
    fixed, moving, grid = R.make_pair(size, "cuda", seed=0)
    zero = torch.zeros(1, 3, size, size, size, device="cuda")
    mse0, sim0 = R.quality(fixed, moving, zero, grid)
    disp, _ = R.register(fixed, moving, grid, iters=60)
    mse1, sim1 = R.quality(fixed, moving, disp, grid)
    assert torch.isfinite(disp).all()
    assert sim1 > sim0 + 0.02 and mse1 < 0.8 * mse0, (mse0, sim0, mse1, sim1)


@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")
def test_graph_replayed_registration_matches_eager():
    """One Adam iteration captured in a HIP graph and replayed gives the field of the same
    optimization run eagerly (both with Adam's graph-safe implementation)."""
    size = 32
    fixed, moving, grid = R.make_pair(size, "cuda", seed=3)
    d_eager, _ = R.register(fixed, moving, grid, iters=20, capturable=True)
    d_graph, _ = R.register_graph(fixed, moving, grid, iters=20)
    rel = float((d_graph - d_eager).norm() / d_eager.norm())
    assert rel < 1e-5, rel
