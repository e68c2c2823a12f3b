"""The small-volume kernel (volumes whose D, H and W are all at most 16: one workgroup holds a
whole volume in LDS), against the float64 oracle and against the plane-marching kernel on the same
inputs. The library picks it for such shapes on its own; a forced D-chunk length (force_dchunk)
sends the same shapes to the plane-marching kernel instead.

Covers the reference's many-channel benchmark shape (1,256,16^3) (bench.py:52), ragged shapes down
to single planes, rows and columns, every k (k = 9 windows wider than half the volume), both
dtypes, both gradients, the ncc and adjoint maps, and the exactness properties of the reference's
direct sums (zero and constant slabs after signal, lncc3d.cu:57-92)."""
import numpy as np
import pytest
import torch

import oracle as O
import workloads as wl
from checks import assert_grad_bf16, check_against_oracle, cos_rel
from fused_lncc import ext, fused_lncc_loss, lncc_map

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [(1, 1, 16, 16, 16), (2, 3, 16, 16, 16), (1, 2, 5, 9, 16), (1, 2, 16, 1, 7), (2, 1, 3, 16, 2),
          (1, 1, 8, 8, 8), (1, 4, 13, 11, 15), (1, 1, 16, 5, 1), (1, 3, 1, 2, 2)]


def _run(p, t, k, dtype=torch.float32, dr=1e-5):
    pd = p.to(dtype).to(DEV).requires_grad_(True)
    td = t.to(dtype).to(DEV)
    loss = fused_lncc_loss(pd, td, k, dr)
    loss.backward()
    m = lncc_map(pd, td, k, dr)
    torch.cuda.synchronize()
    return float(loss.item()), pd.grad, m


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_small_matches_oracle(shape, k):
    """Loss, ncc map and gradient against the float64 oracle: the parity bar, or four times the
    reference's own float32 error where that is larger (a single-voxel volume is almost perfectly
    correlated with itself, and the reference's float32 gradient there is off by up to 5e-3)."""
    p, t = wl.randn_pair(shape, 40 + k)
    p = 0.6 * t + 0.8 * p
    print(f"small case {shape} k={k}", flush=True)
    check_against_oracle(p, t, k)


@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_single_voxel_volumes(k, force_dchunk):
    """Volumes of one voxel: every window sum is that voxel's value exactly, so both kernels evaluate
    the same per-voxel formula on the same numbers and must agree bit for bit; the loss matches the
    oracle. (The gradient of a one-voxel volume is a small difference of large terms, as the
    volume is almost perfectly correlated with itself: float32 evaluations of the formula, the
    reference's included, are off by 1e-4 to 1e-2 relative there.)"""
    shape = (2, 5, 1, 1, 1)
    p, t = wl.randn_pair(shape, 30 + k)
    l_small, g_small, m_small = _run(p, t, k)
    force_dchunk(1)
    l_march, g_march, m_march = _run(p, t, k)
    assert l_small == l_march and torch.equal(g_small, g_march) and torch.equal(m_small, m_march)
    l64, g64 = O.lncc(p.numpy(), t.numpy(), k)
    # ncc is within ~2e-4 of 1 here, which float32 resolves to about 6e-8: the loss 1 - mean(ncc)
    # is known to a few float32 ulps of 1.0 absolute, not to 1e-5 relative
    assert abs(l_small - l64) <= 1e-5 * abs(l64) + 4 * 2.0 ** -24, (l_small, l64)
    assert np.all(np.sign(g_small.double().cpu().numpy()) == np.sign(g64))


@pytest.mark.parametrize("shape", [(1, 2, 16, 16, 16), (1, 3, 7, 13, 10)], ids=["16^3", "7x13x10"])
@pytest.mark.parametrize("k", [3, 7, 9])
def test_small_bf16(shape, k):
    p, t = wl.randn_pair(shape, 60 + k)
    p = (0.6 * t + 0.8 * p).bfloat16().float()
    t = t.bfloat16().float()
    loss, g, _ = _run(p, t, k, torch.bfloat16)
    assert g.dtype == torch.bfloat16
    l64, g64 = O.lncc(p.numpy(), t.numpy(), k)
    assert abs(loss - l64) <= 1e-5 * abs(l64), (loss, l64)
    assert_grad_bf16(g.double().cpu().numpy(), g64)


@pytest.mark.parametrize("k", [3, 5, 7, 9])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_small_against_marching_kernel(k, dt, force_dchunk):
    """The same inputs through both kernels: equal losses and gradients up to float32 rounding
    (their sums run in different orders), the bf16 gradients within one bf16 ulp of each other."""
    shape = (2, 3, 16, 15, 16)
    p, t = wl.randn_pair(shape, 80 + k)
    p = 0.5 * t + 0.9 * p
    l_small, g_small, m_small = _run(p, t, k, dt)
    force_dchunk(shape[2])    # one chunk: the plane-marching kernel, unsplit
    l_march, g_march, m_march = _run(p, t, k, dt)
    assert abs(l_small - l_march) <= 2e-6 * abs(l_march), (l_small, l_march)
    assert (m_small - m_march).abs().max().item() < 1e-5
    a, b = g_small.double().cpu().numpy().ravel(), g_march.double().cpu().numpy().ravel()
    if dt == torch.float32:
        c, rel = cos_rel(a, b)
        assert c > 1 - 1e-10 and rel < 1e-5, (c, rel)
    else:
        tol = O.bf16_ulp(b) + 1e-6 * np.abs(b).max()
        assert (np.abs(a - b) <= tol).all()


@pytest.mark.parametrize("k", [5, 7, 9])
@pytest.mark.parametrize("axis", [2, 3, 4], ids=["D", "H", "W"])
@pytest.mark.parametrize("fill", [0.0, 128.0], ids=["zero", "const"])
def test_small_exact_after_signal(k, axis, fill):
    """[0, 255] integer data with a zero or constant (128) slab after signal along each axis: exact
    zeros of the ncc map and the gradient wherever the float64 oracle and the reference's float32
    arithmetic have them."""
    shape = (1, 2, 16, 16, 16)
    p, t = wl.structured_pair(shape, "byte", 90 + k + axis, axis=axis, start=7, fill=fill)
    loss, g, m = _run(p, t, k)
    l64, g64, maps = O.lncc(p.numpy(), t.numpy(), k, grad=True, maps=True)
    _, g32, m32 = O.lncc_ref32(p.numpy(), t.numpy(), k, grad=True, ncc_map=True)
    gn, mn = g.double().cpu().numpy(), m.double().cpu().numpy()
    zm = (maps["ncc"] == 0) & (m32 == 0)
    zg = (g64 == 0) & (g32 == 0)
    # a constant slab runs into the volume's edge, where the zero padding makes the windows of its
    # last planes non-constant: exact-zero gradients only come with a zero slab
    assert zm.sum() > 0 and (zg.sum() > 0 or fill != 0.0)
    assert np.count_nonzero(mn[zm]) == 0 and np.count_nonzero(gn[zg]) == 0
    assert abs(loss - l64) <= 1e-5 * abs(l64)
    c, rel = cos_rel(gn, g64)
    assert c > 0.9999 and rel < 1e-3, (c, rel)


def test_small_maps_and_loss_only():
    """lncc_forward's four maps and the forward-only kernel (no_grad) on small volumes."""
    shape = (2, 2, 11, 16, 9)
    p, t = wl.randn_pair(shape, 97)
    B = shape[0] * shape[1]
    pf = p.reshape(B, *shape[2:]).to(DEV)
    tf = t.reshape(B, *shape[2:]).to(DEV)
    maps = [x.double().cpu().numpy().reshape(shape) for x in ext.lncc_forward(pf, tf, 7, 1e-5)]
    l64, _, om = O.lncc(p.numpy(), t.numpy(), 7, grad=False, maps=True)
    assert np.abs(maps[0] - om["ncc"]).max() < 1e-4
    for got, key in zip(maps[1:], ("A", "B", "C")):
        assert np.linalg.norm(got - om[key]) / np.linalg.norm(om[key]) < 1e-4, key
    with torch.no_grad():
        loss = fused_lncc_loss(p.to(DEV), t.to(DEV), 7)
    assert abs(loss.item() - l64) <= 1e-5 * abs(l64)


def test_small_nan_and_target_grad():
    """A NaN voxel makes the loss NaN; the target-side gradient on small volumes equals the
    float64 autograd gradient of the oracle's PyTorch port."""
    import torch_lncc_port
    shape = (1, 2, 12, 16, 14)
    p, t = wl.randn_pair(shape, 98)
    p = 0.7 * t + 0.5 * p
    pn = p.clone()
    pn[0, 1, 5, 6, 7] = float("nan")
    assert np.isnan(fused_lncc_loss(pn.to(DEV), t.to(DEV), 5).item())
    pr, tr = p.double().requires_grad_(True), t.double().requires_grad_(True)
    torch_lncc_port.lncc_dense(pr, tr, 5).backward()
    pd, td = p.to(DEV).requires_grad_(True), t.to(DEV).requires_grad_(True)
    fused_lncc_loss(pd, td, 5, target_grad=True).backward()
    for g, r in ((pd.grad, pr.grad), (td.grad, tr.grad)):
        c, rel = cos_rel(g.double().cpu().numpy(), r.numpy())
        assert c > 0.9999 and rel < 1e-3, (c, rel)


def test_feat16_workload():
    """The reference's many-channel benchmark shape (1,256,16^3) k=7 in one launch: the loss and the
    gradient of every volume against the float64 oracle."""
    p, t = wl.make_inputs("feat16")
    loss, g, _ = _run(p, t, 7)
    l64, g64 = O.lncc(p.numpy(), t.numpy(), 7)
    assert abs(loss - l64) <= 1e-5 * abs(l64), (loss, l64)
    c, rel = cos_rel(g.double().cpu().numpy(), g64)
    assert c > 0.9999 and rel < 1e-3, (c, rel)
