"""torch.compile on ROCm: a training step that calls the loss compiles whole (fullgraph) and gives
the eager results; the custom ops pass torch.library's own consistency checks.

The reference registers its two ops with fake kernels so that compiled training steps can call
the loss (fused_lncc/__init__.py:22-46); this build keeps that contract for its fused op.
"""
import pytest
import torch

from fused_lncc import fused_lncc_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(dt, shape=(1, 2, 20, 24, 28)):
    g = torch.Generator().manual_seed(3)
    t = torch.rand(shape, generator=g)
    p = 0.7 * t + 0.3 * torch.rand(shape, generator=g)
    return p.to(dt).to(DEV), t.to(dt).to(DEV)


def _step(p, t):
    # the loss as one term of a larger objective, as in a registration or training step
    return fused_lncc_loss(p, t, 7) + 0.1 * (p.float() ** 2).mean()


def _run(fn, p0, t):
    p = p0.clone().requires_grad_(True)
    loss = fn(p, t)
    loss.backward()
    torch.cuda.synchronize()
    return loss.detach(), p.grad


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_step_matches_eager(dt, backend):
    torch._dynamo.reset()
    p0, t = _inputs(dt)
    le, ge = _run(_step, p0, t)
    lc, gc = _run(torch.compile(_step, backend=backend, fullgraph=True), p0, t)
    assert gc.dtype == dt and lc.dtype == torch.float32
    # the fused kernel is the same call in both; only the glue around it may be fused differently
    assert torch.allclose(lc, le, rtol=1e-6, atol=0)
    tol = 1e-6 if dt == torch.float32 else 1e-2
    assert torch.allclose(gc.float(), ge.float(), rtol=tol, atol=tol * ge.float().abs().max().item())


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_compiled_scaled_loss_matches_eager_bitwise(dt):
    """grad_out = 3 (the loss weighted in a larger objective): the compiled backward multiplies the
    stored gradient by grad_out in float32 and rounds once, as the eager in-place scaling kernel
    does, so the two gradients are equal bit for bit, in bf16 as in fp32."""
    torch._dynamo.reset()
    p0, t = _inputs(dt)

    def step(p, t):
        return 3.0 * fused_lncc_loss(p, t, 7)

    le, ge = _run(step, p0, t)
    lc, gc = _run(torch.compile(step, backend="aot_eager", fullgraph=True), p0, t)
    assert gc.dtype == dt
    assert torch.equal(lc, le) and torch.equal(gc, ge)


def test_compiled_step_second_call_and_new_shape():
    torch._dynamo.reset()
    f = torch.compile(_step, backend="aot_eager", fullgraph=True)
    for shape in [(1, 2, 20, 24, 28), (1, 2, 20, 24, 28), (2, 1, 12, 16, 18)]:
        p0, t = _inputs(torch.float32, shape)
        le, ge = _run(_step, p0, t)
        lc, gc = _run(f, p0, t)
        assert torch.allclose(lc, le, rtol=1e-6, atol=0)
        assert torch.allclose(gc, ge, rtol=1e-6, atol=1e-6 * ge.abs().max().item())


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_opcheck_custom_ops(dt):
    p, t = _inputs(dt, (2, 10, 12, 14))
    torch.library.opcheck(torch.ops.fused_lncc.loss_grad.default, (p, t, 5, 1e-5, True))
    torch.library.opcheck(torch.ops.fused_lncc.loss_grad.default, (p, t, 3, 1e-5, False))
    torch.library.opcheck(torch.ops.fused_lncc.forward.default, (p, t, 5, 1e-5))
    torch.library.opcheck(torch.ops.fused_lncc.loss_grad_pt.default, (p, t, 5, 1e-5))
