"""The optional target-side gradient (fused_lncc_loss(..., target_grad=True)), outside the
reference's own scope (its README.md:116-121: pred-only gradient) and what symmetric registration
needs. Checked against the oracle's float64 PyTorch port, where autograd differentiates the loss
with respect to target directly (not through the symmetry the kernel path uses)."""
import pytest
import torch

import torch_lncc_port
import workloads as wl
from checks import assert_grad_bf16
from fused_lncc import fused_lncc_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ref_grads(p, t, k):
    pr = p.double().requires_grad_(True)
    tr = t.double().requires_grad_(True)
    torch_lncc_port.lncc_dense(pr, tr, k).backward()
    return pr.grad, tr.grad


def _cos_rel(g, r):
    g, r = g.double().cpu().ravel(), r.double().cpu().ravel()
    return float(g @ r / (g.norm() * r.norm())), float((g - r).norm() / r.norm())


@pytest.mark.parametrize("k", [3, 7, 9])
def test_target_grad_matches_autograd(k):
    p, t = wl.randn_pair((1, 2, 18, 21, 23), 90 + k)
    p = 0.7 * t + 0.3 * p
    gp_ref, gt_ref = _ref_grads(p, t, k)
    pd = p.to(DEV).requires_grad_(True)
    td = t.to(DEV).requires_grad_(True)
    fused_lncc_loss(pd, td, k, target_grad=True).backward()
    for g, r in ((pd.grad, gp_ref), (td.grad, gt_ref)):
        c, rel = _cos_rel(g, r)
        assert c > 0.9999 and rel < 1e-3, (c, rel)


def test_default_is_pred_only_like_the_reference():
    p, t = wl.randn_pair((1, 1, 12, 14, 16), 95)
    pd = p.to(DEV).requires_grad_(True)
    td = t.to(DEV).requires_grad_(True)
    fused_lncc_loss(pd, td, 5).backward()
    assert pd.grad is not None and td.grad is None


def test_target_grad_alone_bf16_and_retained_graph():
    p, t = wl.randn_pair((1, 2, 16, 20, 24), 96)
    _, gt_ref = _ref_grads(p.bfloat16().float(), t.bfloat16().float(), 7)
    pd = p.bfloat16().to(DEV)                       # pred without requires_grad
    td = t.bfloat16().to(DEV).requires_grad_(True)
    loss = fused_lncc_loss(pd, td, 7, target_grad=True)
    (2.0 * loss).backward(retain_graph=True)
    g1 = td.grad.clone()
    td.grad = None
    loss.backward()                                 # second backward through the retained graph
    assert g1.dtype == torch.bfloat16 and pd.grad is None
    # float32 arithmetic rounded once to bf16 (the scale by 2 is exact): within one bf16 ulp of
    # the rounded float64 gradient, as for the pred gradient
    assert_grad_bf16(g1.double().cpu().numpy(), (2.0 * gt_ref).numpy())
    assert_grad_bf16(td.grad.double().cpu().numpy(), gt_ref.numpy())


def test_target_grad_compiled_matches_eager():
    torch._dynamo.reset()
    p, t = wl.randn_pair((1, 2, 20, 24, 28), 97)

    def step(a, b):
        return fused_lncc_loss(a, b, 7, target_grad=True) + 0.1 * (a * b).mean()

    def run(fn):
        a = p.to(DEV).requires_grad_(True)
        b = t.to(DEV).requires_grad_(True)
        fn(a, b).backward()
        torch.cuda.synchronize()
        return a.grad, b.grad

    ge = run(step)
    gc = run(torch.compile(step, backend="aot_eager", fullgraph=True))
    for x, y in zip(ge, gc):
        assert torch.allclose(x, y, rtol=1e-6, atol=1e-6 * x.abs().max().item())


@pytest.mark.parametrize("k", [3, 5, 7, 9])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dchunk", [None, 3])
def test_dual_kernel_against_single_passes(k, dt, dchunk, force_dchunk):
    """The entry point for both gradients gives the pred gradient of the pred-only kernel bit for
    bit and the target gradient of that kernel run with the inputs swapped, on a ragged shape with
    D-chunk seams."""
    from fused_lncc import ext

    if dchunk is not None:
        force_dchunk(dchunk)
    p, t = wl.randn_pair((2, 1, 19, 37, 45), 120 + k)
    pf = p.reshape(2, 19, 37, 45).to(dt).to(DEV)
    tf = t.reshape(2, 19, 37, 45).to(dt).to(DEV)
    loss, gp, gt = ext.loss_grad_pt(pf, tf, k, 1e-5)
    loss1, gp1 = ext.loss_grad(pf, tf, k, 1e-5, True)
    gt1 = ext.grad_only(tf, pf, k, 1e-5)
    torch.cuda.synchronize()
    assert gp.dtype == dt and gt.dtype == dt
    assert torch.equal(gp, gp1)
    assert loss.item() == loss1.item()
    # the same kernel on the same (swapped) inputs and the same plan: bit for bit
    assert torch.equal(gt, gt1)


@pytest.mark.parametrize("name", ["headline", "bf16"])
def test_dual_kernel_bitwise_at_full_size(name):
    """At the headline workload (2,16,128^3) fp32 k=7 and its bf16 k=5 variant, the one-launch
    kernel's two gradients equal the pred-gradient kernel's and the swapped pass's bit for bit, and
    its loss equals the pred pass's."""
    from fused_lncc import ext

    p, t = wl.make_inputs(name)
    k = wl.WORKLOADS[name]["k"]
    pf, tf = p.to(DEV), t.to(DEV)
    print(f"dual at {name} {tuple(p.shape)} {p.dtype} k={k}", flush=True)
    loss, gp, gt = ext.loss_grad_pt(pf, tf, k, 1e-5)
    loss1, gp1 = ext.loss_grad(pf, tf, k, 1e-5, True)
    assert torch.equal(gp, gp1)
    del gp1
    gt1 = ext.grad_only(tf, pf, k, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(gt, gt1) and loss.item() == loss1.item()
