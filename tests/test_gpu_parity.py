"""GPU parity of the HIP path against the reference's golden vectors and the CPU oracle.

Mirrors the reference's own tests (tests/test_pytest.py, test_fixes.py, test_robust.py,
test_bf16.py, verify_fwd.py, verify_bwd.py) with the parity bar:
  fp32 loss relative error <= 1e-5, bf16 loss relative error <= 1e-2,
  gradient cosine > 0.9999 and relative L2 error < 1e-3.
Inputs are generated on the CPU (seeded), so every run sees the same bytes.
"""
import glob
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
import workloads as wl
from checks import assert_grad_bf16, cos_rel
from fused_lncc import ext, fused_lncc_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FULL = sorted(f for f in glob.glob(os.path.join(GOLDEN, "*.npz")) if not os.path.basename(f).startswith("stats_"))
PARITY = [f for f in FULL if not os.path.basename(f).startswith("degen_")]

LOSS_RTOL_F32 = 1e-5
LOSS_RTOL_BF16 = 1e-2
GRAD_COS = 0.9999
GRAD_REL_L2 = 1e-3


def fused(p, t, k, dr=1e-5, dtype=None):
    """fused_lncc_loss + backward on the GPU; returns (loss, grad as float64 numpy, grad dtype)."""
    p = torch.as_tensor(p)
    t = torch.as_tensor(t)
    if dtype is not None:
        p, t = p.to(dtype), t.to(dtype)
    pd = p.to(DEV).requires_grad_(True)
    loss = fused_lncc_loss(pd, t.to(DEV), k, dr)
    loss.backward()
    torch.cuda.synchronize()
    return float(loss.item()), pd.grad.double().cpu().numpy(), pd.grad.dtype


def assert_grad(g, gr, cos_min=GRAD_COS, rel_max=GRAD_REL_L2):
    c, r = cos_rel(g, gr)
    assert c > cos_min and r < rel_max, f"cos={c:.8f} relL2={r:.3e}"


def assert_loss(l, lr, rtol):
    assert abs(l - lr) <= rtol * abs(lr), f"loss {l:.9f} vs {lr:.9f} (rel {abs(l - lr) / abs(lr):.2e})"


# ---------------------------------------------------------------- golden vectors (reference outputs)
@pytest.mark.parametrize("path", PARITY, ids=[os.path.basename(p)[:-4] for p in PARITY])
def test_golden_vectors(path):
    d = np.load(path)
    loss, g, _ = fused(d["pred"], d["target"], int(d["k"]), float(d["smooth_dr"]))
    assert_loss(loss, float(d["loss"]), LOSS_RTOL_F32)
    assert_grad(g, d["grad"])


def test_golden_bf16_values():
    d = np.load(os.path.join(GOLDEN, "bf16vals_k7.npz"))
    loss, g, gdt = fused(d["pred"], d["target"], 7, dtype=torch.bfloat16)
    assert gdt == torch.bfloat16
    assert_loss(loss, float(d["loss"]), LOSS_RTOL_BF16)
    assert_grad(g, d["grad"], 0.999, 1e-2)   # the reference's own bar
    assert_grad_bf16(g, d["grad"])


# ---------------------------------------------------------------- reference tests, restated
@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_forward_matches_reference(k):
    p, t = wl.randn_pair((2, 4, 32, 32, 32), 0)
    loss, _, _ = fused(p, t, k)
    lr, _ = O.lncc(p.numpy(), t.numpy(), k, grad=False)
    assert abs(loss - lr) < 1e-4
    assert_loss(loss, lr, LOSS_RTOL_F32)


@pytest.mark.parametrize("shape", [(2, 4, 32, 32, 32), (1, 8, 24, 40, 32)])
@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_backward_matches_reference(k, shape):
    p, t = wl.randn_pair(shape, 1)
    loss, g, _ = fused(p, t, k)
    lr, gr = O.lncc(p.numpy(), t.numpy(), k)
    assert_loss(loss, lr, LOSS_RTOL_F32)
    assert_grad(g, gr)
    assert np.abs(g - gr).mean() / np.abs(gr).mean() < 1e-3


def test_bf16_runs():
    p, t = wl.randn_pair((1, 2, 16, 16, 16), 2, dtype=torch.bfloat16)
    _, g, gdt = fused(p, t, 7)
    assert gdt == torch.bfloat16 and np.isfinite(g).all()


@pytest.mark.parametrize("k", [3, 7])
def test_bf16_matches_fp32_of_same_values(k):
    p, t = wl.randn_pair((2, 4, 40, 40, 40), 3, dtype=torch.bfloat16)
    lb, gb, _ = fused(p, t, k)
    lf, gf, _ = fused(p.float(), t.float(), k)
    assert abs(lb - lf) < 1e-3
    assert_loss(lb, lf, LOSS_RTOL_BF16)
    assert np.abs(gb - gf).mean() / np.abs(gf).mean() < 2e-2   # the reference's own bar
    assert_grad_bf16(gb, gf)


@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_fused_backward_matches_scatter(k):
    """Reference-API path: maps -> box-sum scatter formula == lncc_backward (tests/test_pytest.py:38-51),
    and the fused hot-path gradient equals that unfused path. The extension is imported by the
    reference's module name, as its test does."""
    import fused_lncc_cuda as ext
    p, t = wl.randn_pair((2, 3, 24, 20, 28), 4)
    pf = p.reshape(6, 24, 20, 28).contiguous().to(DEV)
    tf = t.reshape(6, 24, 20, 28).contiguous().to(DEV)
    ncc, A, Bc, Cc = ext.lncc_forward(pf, tf, k, 1e-5)
    sc = -1.0 / ncc.numel()
    box = lambda x: ext.box3d_sep_forward(x.contiguous(), k)  # noqa: E731
    ref = sc * (box(A) + 2.0 * pf * box(Bc) + tf * box(Cc))
    got = ext.lncc_backward(A, Bc, Cc, pf, tf, k, sc)
    assert (ref - got).abs().max().item() < 1e-8
    _, g, _ = fused(p, t, k)
    assert_grad(g.reshape(6, 24, 20, 28), got.double().cpu().numpy(), 0.99999, 1e-4)
    assert abs((1.0 - ncc.double().mean().item()) - fused(p, t, k)[0]) < 1e-6


@pytest.mark.parametrize("shape", [(2, 4, 24, 24, 24), (1, 8, 32, 40, 48)])
@pytest.mark.parametrize("k", [3, 5, 7])
def test_maps_match_oracle(k, shape):
    """Per-voxel ncc map (tests/verify_fwd.py:27-34) and the adjoint maps A, Bc, Cc."""
    p, t = wl.randn_pair(shape, 5)
    B = shape[0] * shape[1]
    pf = p.reshape(B, *shape[2:]).contiguous().to(DEV)
    tf = t.reshape(B, *shape[2:]).contiguous().to(DEV)
    maps = [m.double().cpu().numpy().reshape(shape) for m in ext.lncc_forward(pf, tf, k, 1e-5)]
    _, _, om = O.lncc(p.numpy(), t.numpy(), k, grad=False, maps=True)
    assert np.abs(maps[0] - om["ncc"]).max() < 1e-3
    assert maps[0].min() >= 0 and maps[0].max() <= 1
    for got, key in zip(maps[1:], ("A", "B", "C")):
        assert np.linalg.norm(got - om[key]) / np.linalg.norm(om[key]) < 1e-3, key


@pytest.mark.parametrize("k", [3, 7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lncc_map(k, dtype):
    """The ncc map alone (no adjoint maps): equal to lncc_forward's first output, close to the
    oracle's map, and its mean is 1 - loss."""
    from fused_lncc import lncc_map
    shape = (2, 3, 18, 21, 26)
    p, t = wl.randn_pair(shape, 70 + k)
    pd, td = p.to(dtype).to(DEV), t.to(dtype).to(DEV)
    m = lncc_map(pd, td, k)
    assert m.shape == shape and m.dtype == torch.float32
    ref = ext.lncc_forward(pd.reshape(6, *shape[2:]), td.reshape(6, *shape[2:]), k, 1e-5)[0]
    assert torch.equal(m.reshape(ref.shape), ref)
    loss = fused_lncc_loss(pd, td, k)
    assert abs((1.0 - m.double().mean().item()) - loss.item()) <= 1e-5 * abs(loss.item())
    if dtype == torch.float32:
        _, _, om = O.lncc(p.numpy(), t.numpy(), k, grad=False, maps=True)
        assert np.abs(m.double().cpu().numpy() - om["ncc"]).max() < 1e-3


def _pure_windows(x, fill, k):
    """Voxels whose zero-padded k^3 window holds no in-volume value other than ``fill``."""
    return O.box3d((np.asarray(x) != fill).astype(np.float64), k) == 0


@pytest.mark.parametrize("k", [3, 5, 7, 9])
@pytest.mark.parametrize("fill", [0.0, 0.5])
def test_box3d_exact_after_signal(k, fill):
    """box3d_sep_forward on U[0,1) signal followed by a zero or constant slab along D (the box
    kernel marches all of D) and one along W: a window that holds only the fill value sums to
    exactly what the reference's direct k-tap sums give, 0 or (number of in-volume voxels) * 0.5
    (every partial sum of up to 729 halves is a float), so it equals the float64 oracle bit for
    bit; elsewhere within float32 rounding (lncc3d.cu:203-230, 308-325)."""
    x = torch.rand(2, 60, 21, 37, generator=torch.Generator().manual_seed(40 + k))
    x[:, 30:] = fill
    x[:, :, :, 25:] = fill
    y = ext.box3d_sep_forward(x.to(DEV), k).double().cpu().numpy()
    yr = O.box3d(x.numpy(), k)
    pure = _pure_windows(x.numpy(), fill, k)
    assert pure.sum() > 1000
    bad = y[pure] != yr[pure]
    assert not bad.any(), f"{bad.sum()} of {pure.sum()} single-valued windows differ (max {np.abs(y[pure] - yr[pure]).max():.3e})"
    assert np.abs(y - yr).max() < 1e-4 * np.abs(yr).max()


@pytest.mark.parametrize("k", [3, 5, 7, 9])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_backward_exact_after_signal(k, dtype):
    """The reference's two-kernel path, lncc_forward then lncc_backward with scale -1/M
    (fused_lncc/__init__.py:62-73), on [0, 255] integer data with a zero slab along D and a
    constant slab (128) along W after signal: the gradient is exactly zero wherever the float64
    oracle's is (deep inside either slab every window is single-valued, so cross = 0, var = 0 and
    the adjoints vanish, as with the reference's direct sums), and within the parity bar (bf16:
    one ulp of the rounded oracle) everywhere."""
    shape = (1, 2, 40, 22, 36)
    p, t = wl.structured_pair(shape, "byte", 60 + k, axis=2, start=24, fill=0.0)
    p[..., 28:] = 128.0
    t[..., 28:] = 128.0
    B = shape[0] * shape[1]
    pf = p.reshape(B, *shape[2:]).to(dtype).to(DEV)
    tf = t.reshape(B, *shape[2:]).to(dtype).to(DEV)
    _, A, Bc, Cc = ext.lncc_forward(pf, tf, k, 1e-5)
    got = ext.lncc_backward(A, Bc, Cc, pf, tf, k, -1.0 / p.numel())
    assert got.dtype == dtype
    g = got.double().cpu().numpy().reshape(shape)
    _, g64 = O.lncc(p.numpy(), t.numpy(), k)
    g64 = g64.astype(np.float64).reshape(shape)
    zero = g64 == 0
    assert zero.sum() > 1000
    assert np.count_nonzero(g[zero]) == 0, f"{np.count_nonzero(g[zero])} of {zero.sum()} exact-zero gradient voxels are not zero"
    if dtype == torch.float32:
        assert_grad(g, g64)
    else:
        assert_grad_bf16(g, g64)


@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_box3d_matches_oracle(k):
    x = torch.randn(3, 13, 17, 11, generator=torch.Generator().manual_seed(k))
    y = ext.box3d_sep_forward(x.to(DEV), k).double().cpu().numpy()
    yr = O.box3d(x.numpy(), k)
    assert np.abs(y - yr).max() < 1e-4 * np.abs(yr).max()


def test_degenerate_in_range():
    z = torch.zeros(1, 1, 16, 16, 16)
    loss, g, _ = fused(z, z, 7)
    assert loss == 1.0 and np.all(g == 0)


@pytest.mark.parametrize("name", ["all-zero", "constant=5", "constant hi=1e4", "near-const"])
def test_degenerate_battery(name):
    gen = torch.Generator().manual_seed(6)
    if name == "all-zero":
        p = t = torch.zeros(2, 2, 32, 32, 32)
    elif name == "constant=5":
        p = t = torch.full((2, 2, 32, 32, 32), 5.0)
    elif name == "constant hi=1e4":
        p = t = torch.full((1, 1, 32, 32, 32), 1e4)
    else:
        p = torch.full((1, 2, 24, 24, 24), 3.0) + 1e-3 * torch.randn(1, 2, 24, 24, 24, generator=gen)
        t = torch.full((1, 2, 24, 24, 24), 3.0)
    loss, g, _ = fused(p, t, 7)
    assert np.isfinite(loss) and 0.0 <= loss <= 1.0001 and np.isfinite(g).all()


@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_nonfinite_input_gives_nonfinite_loss(bad):
    p, t = wl.randn_pair((1, 1, 16, 16, 16), 7)
    p[0, 0, 8, 8, 8] = bad
    loss = fused_lncc_loss(p.to(DEV), t.to(DEV), 7)
    assert not torch.isfinite(loss).item()


def test_plan_follows_device_cus():
    """The D-chunk plan is made for the device's compute units: the MRI-shaped volume (56 tiles of
    32 x 24 per plane at k = 9) is split into as many chunks as fill the CUs in one round."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nblocks = ext.workspace_bytes((1, 160, 192, 224), 9) // 8
    assert nblocks % 56 == 0 and nblocks <= cus < nblocks + 56, (nblocks, cus)


def test_many_volumes():
    """N*C = 2080 volumes of (128, 8, 8) (tests/test_fixes.py:9-17)."""
    p, t = wl.randn_pair((2080, 1, 128, 8, 8), 8)
    loss, g, _ = fused(p, t, 7)
    lr, gr = O.lncc(p.numpy(), t.numpy(), 7)
    assert_loss(loss, lr, LOSS_RTOL_F32)
    assert_grad(g, gr)


@pytest.mark.parametrize("k", [3, 7, 9])
@pytest.mark.parametrize("dchunk", [1, 3, 8])
def test_d_chunk_seams(k, dchunk, force_dchunk):
    """Workgroups that own short D chunks restart their z-sums at every chunk: forcing the chunk
    length (the library's test hook) puts many seams into one volume."""
    force_dchunk(dchunk)
    p, t = wl.randn_pair((1, 2, 37, 30, 41), 40 + k)
    loss, g, _ = fused(p, t, k)
    lr, gr = O.lncc(p.numpy(), t.numpy(), k)
    assert_loss(loss, lr, LOSS_RTOL_F32)
    assert_grad(g, gr)


@pytest.mark.parametrize("shape,k,corr", [
    ((1, 1, 100, 97, 131), 7, False),   # 240 workgroups: 20 partial tiles x 12 D-chunks of 9 planes
    ((1, 1, 64, 200, 50), 9, True),     # 224 workgroups: 16 chunks of 4 planes, k = 9
    ((2, 1, 70, 70, 70), 5, False),     # 252 workgroups (not a multiple of the 8 XCDs)
    ((1, 3, 40, 65, 33), 3, True),      # 252 workgroups, 14 chunks of 3 planes
])
def test_medium_shapes_against_oracle(shape, k, corr):
    """Volumes of about a million voxels, planned the way real launches are (short D-chunks for
    small volumes, grids that are not multiples of 8, partial edge tiles), against the oracle."""
    p, t = wl.randn_pair(shape, 70 + k)
    if corr:  # high local correlation: ncc near 1, where the clamp and its masking matter
        p = 0.9 * t + 0.1 * p
    loss, g, _ = fused(p, t, k)
    lr, gr = O.lncc(p.numpy(), t.numpy(), k)
    assert_loss(loss, lr, LOSS_RTOL_F32)
    assert_grad(g, gr)


def test_non_contiguous_inputs():
    """Strided and transposed views are made contiguous by the API (fused_lncc/__init__.py:83 does
    the same); the gradient reaches the original view through that copy."""
    p, t = wl.randn_pair((1, 2, 20, 28, 24), 77)
    base = p.transpose(3, 4).contiguous().to(DEV).requires_grad_(True)   # storage (.., 24, 28)
    pv = base.transpose(3, 4)                                             # view (.., 28, 24)
    tv = t.to(DEV)[..., :]
    assert not pv.is_contiguous()
    loss = fused_lncc_loss(pv, tv, 5)
    loss.backward()
    lr, gr = O.lncc(p.numpy(), t.numpy(), 5)
    assert_loss(loss.item(), lr, LOSS_RTOL_F32)
    assert_grad(base.grad.transpose(3, 4).double().cpu().numpy(), gr)
    big = torch.randn(1, 2, 20, 28, 48, generator=torch.Generator().manual_seed(78))
    ps, ts = big[..., ::2], big[..., 1::2]                                # strided slices
    ls = fused_lncc_loss(ps.to(DEV), ts.to(DEV), 3)
    lr2, _ = O.lncc(ps.contiguous().numpy(), ts.contiguous().numpy(), 3)
    assert_loss(ls.item(), lr2, LOSS_RTOL_F32)


def test_unsupported_dtype_raises():
    p = torch.randn(1, 1, 16, 16, 16, device=DEV, dtype=torch.float64)
    with pytest.raises(RuntimeError):
        fused_lncc_loss(p, p, 7)


# ---------------------------------------------------------------- autograd contract
def test_grad_out_scaling_and_retain_graph():
    p, t = wl.randn_pair((1, 2, 20, 24, 28), 9)
    _, g1, _ = fused(p, t, 5)
    pd = p.to(DEV).requires_grad_(True)
    (3.0 * fused_lncc_loss(pd, t.to(DEV), 5)).backward()
    assert np.array_equal(pd.grad.double().cpu().numpy(), (torch.from_numpy(g1).float() * 3.0).double().numpy())
    pd.grad = None
    (0.0 * fused_lncc_loss(pd, t.to(DEV), 5)).backward()
    assert torch.count_nonzero(pd.grad).item() == 0
    pd.grad = None
    loss = fused_lncc_loss(pd, t.to(DEV), 5)
    loss.backward(retain_graph=True)
    loss.backward()
    assert np.array_equal(pd.grad.double().cpu().numpy(), 2.0 * g1)


def test_no_grad_and_target_grad():
    p, t = wl.randn_pair((2, 2, 16, 24, 20), 10)
    l1, _, _ = fused(p, t, 7)
    with torch.no_grad():
        l0 = fused_lncc_loss(p.to(DEV).requires_grad_(True), t.to(DEV), 7).item()
    assert l0 == l1
    td = t.to(DEV).requires_grad_(True)
    pd = p.to(DEV).requires_grad_(True)
    fused_lncc_loss(pd, td, 7).backward()
    assert td.grad is None and pd.grad is not None


@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_regression_2x8x40(k):
    """The reference's regression at (2,8,40^3) fp32 (tests/test_fixes.py:26-35,
    tests/test_bf16.py:22-29: |dl| < 1e-4, cosine > 0.9999, loss in [0, 1]), with the parity bar."""
    p, t = wl.randn_pair((2, 8, 40, 40, 40), 12 + k)
    loss, g, _ = fused(p, t, k)
    lr, gr = O.lncc(p.numpy(), t.numpy(), k)
    assert abs(loss - lr) < 1e-4 and 0.0 <= loss <= 1.0
    assert_loss(loss, lr, LOSS_RTOL_F32)
    assert_grad(g, gr)


def test_large_shape_finite():
    """The reference's large-shape run (tests/test_robust.py:52-59): (2,32,128^3) forward + backward
    gives a finite loss in [0, 1] and a finite gradient."""
    gen = torch.Generator(device=DEV).manual_seed(13)
    t = torch.randn(2, 32, 128, 128, 128, device=DEV, generator=gen)
    p = (0.8 * t + 0.6 * torch.randn(t.shape, device=DEV, generator=gen)).requires_grad_(True)
    loss = fused_lncc_loss(p, t, 7)
    loss.backward()
    assert 0.0 <= loss.item() <= 1.0
    assert torch.isfinite(p.grad).all().item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_maximum_plane_size(dtype):
    """Planes just under the 2 GiB limit of the per-plane (31-bit) offsets: 16384 x 32767 float32 or
    32768 x 32767 bfloat16, two planes, all zero but a random patch in the far corner (the highest
    offsets). Zero data and zero padding are the same to the box sums, so the corner holds exactly
    the problem of a small volume with the patch and a 2h+2 zero margin: its gradient equals the
    small volume's scaled by the voxel-count ratio (the oracle pins the small one), and every other
    gradient voxel of the plane is exactly zero."""
    k, h = 7, 3
    H, W, D = (16384, 32767, 2) if dtype == torch.float32 else (32768, 32767, 2)
    assert H * W * (4 if dtype == torch.float32 else 2) < 2 ** 31
    ph, pw, m = 24, 40, 2 * h + 2
    p, t = wl.randn_pair((1, 1, D, ph, pw), 77)
    p, t = p.to(dtype), t.to(dtype)
    ps = torch.zeros(1, D, ph + m, pw + m, dtype=dtype)
    ts = torch.zeros_like(ps)
    ps[0, :, m:, m:], ts[0, :, m:, m:] = p[0, 0], t[0, 0]
    loss_s, g_s = ext.loss_grad(ps.to(DEV), ts.to(DEV), k, 1e-5)
    lr, gr = O.lncc(ps.float().numpy(), ts.float().numpy(), k)
    assert abs(loss_s.item() - lr) <= (1e-5 if dtype == torch.float32 else 1e-2) * abs(lr)
    if dtype == torch.float32:
        assert_grad(g_s.double().cpu().numpy(), gr)
    else:
        assert_grad_bf16(g_s.double().cpu().numpy(), gr)

    print(f"max plane: {dtype} ({D}, {H}, {W})", flush=True)
    pb = torch.zeros(1, D, H, W, dtype=dtype, device=DEV)
    tb = torch.zeros_like(pb)
    pb[0, :, H - ph:, W - pw:] = p[0, 0].to(DEV)
    tb[0, :, H - ph:, W - pw:] = t[0, 0].to(DEV)
    loss_b, g_b = ext.loss_grad(pb, tb, k, 1e-5)
    del pb, tb
    corner = g_b[0, :, H - ph - m:, W - pw - m:].double().cpu().numpy()
    scale = (D * H * W) / float(D * (ph + m) * (pw + m))
    ref = g_s[0].double().cpu().numpy() / scale
    cos = float((corner * ref).sum() / (np.linalg.norm(corner) * np.linalg.norm(ref)))
    rel = float(np.linalg.norm(corner - ref) / np.linalg.norm(ref))
    if dtype == torch.float32:
        assert cos > 0.99999 and rel < 1e-4, (cos, rel)
    else:  # both gradients are rounded to bf16 once, at different scales: two roundings
        assert cos > 0.9999 and rel < 4e-3, (cos, rel)
    g_b[0, :, H - ph - m:, W - pw - m:] = 0
    assert g_b.abs().max().item() == 0.0
    # the ncc sum of the plane is the small volume's; the float32 loss 1 - sum/M is within one
    # rounding step (2^-24 below 1) of its value, which at this M is worth 2^-24 M in the sum
    s_b = (1.0 - loss_b.item()) * D * H * W
    s_s = (1.0 - loss_s.item()) * D * (ph + m) * (pw + m)
    assert abs(s_b - s_s) <= 2.0 ** -24 * D * H * W + 1e-3 * abs(s_s), (s_b, s_s)


def test_concurrent_host_threads():
    """Re-entrancy of the C ABI: four host threads, each on its own stream with its own inputs,
    workspace and outputs, call the library at the same time (ctypes releases the GIL during the
    call); every result is bitwise the one the same call gives alone."""
    import threading
    cases = [(wl.randn_pair((1, 2, 20 + 3 * i, 30, 26 + i), 40 + i), 3 + 2 * (i % 4)) for i in range(4)]
    inputs = [(p.to(DEV).reshape(-1, *p.shape[2:]), t.to(DEV).reshape(-1, *t.shape[2:]), k) for (p, t), k in cases]
    alone = []
    for pf, tf, k in inputs:
        loss, grad = ext.loss_grad(pf, tf, k, 1e-5)
        alone.append((loss.item(), grad.cpu()))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in inputs]
    got = [None] * len(inputs)
    start = threading.Barrier(len(inputs))

    def work(i):
        pf, tf, k = inputs[i]
        with torch.cuda.stream(streams[i]):
            start.wait()
            for _ in range(20):
                loss, grad = ext.loss_grad(pf, tf, k, 1e-5)
            streams[i].synchronize()
            got[i] = (loss.item(), grad.cpu())

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(inputs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert all(not th.is_alive() for th in threads)
    for (l0, g0), (l1, g1) in zip(alone, got):
        assert l0 == l1 and torch.equal(g0, g1)


def test_side_stream_and_determinism():
    p, t = wl.randn_pair((2, 3, 40, 36, 44), 11)
    l1, g1, _ = fused(p, t, 7)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pd = p.to(DEV).requires_grad_(True)
        loss = fused_lncc_loss(pd, t.to(DEV), 7)
        loss.backward()
    s.synchronize()
    assert loss.item() == l1 and np.array_equal(pd.grad.double().cpu().numpy(), g1)


# ---------------------------------------------------------------- the five workloads
def test_workload_cpu():
    d = np.load(os.path.join(GOLDEN, "cpu_k3.npz"))
    p, t = wl.make_inputs("cpu")
    assert np.array_equal(p.numpy(), d["pred"]) and np.array_equal(t.numpy(), d["target"])
    loss, g, _ = fused(p, t, 3)
    assert_loss(loss, float(d["loss"]), LOSS_RTOL_F32)
    assert_grad(g, d["grad"])


@pytest.mark.parametrize("name", ["mri", "headline"])
def test_workload_fp32(name):
    st = np.load(os.path.join(GOLDEN, f"stats_{name}.npz"))
    p, t = wl.make_inputs(name)
    k = int(st["k"])
    loss, g, _ = fused(p, t, k)
    assert_loss(loss, float(st["loss"]), LOSS_RTOL_F32)
    assert abs(np.linalg.norm(g) - float(st["grad_l2"])) < 1e-3 * float(st["grad_l2"])
    lr, gr = O.lncc(p.numpy(), t.numpy(), k)
    assert_loss(loss, lr, LOSS_RTOL_F32)
    assert_grad(g, gr)


def test_workload_bf16():
    st = np.load(os.path.join(GOLDEN, "stats_bf16.npz"))
    p, t = wl.make_inputs("bf16")
    loss, g, gdt = fused(p, t, 5)
    assert gdt == torch.bfloat16
    assert_loss(loss, float(st["loss"]), LOSS_RTOL_BF16)
    lr, gr = O.lncc(p.float().numpy(), t.float().numpy(), 5)
    assert_grad(g, gr, 0.999, 1e-2)   # the reference's own bar
    assert_grad_bf16(g, gr)


def test_workload_large_properties():
    """(2,16,256^3) fp32 k=7: fits with no intermediate volume; size-independent properties:
    the loss is the mean of per-volume-group losses and each group's gradient is the full
    gradient rescaled by the group's share of voxels; repeated runs are bitwise identical."""
    p, t = wl.make_inputs("large")
    pd = p.to(DEV)
    td = t.to(DEV)
    del p, t
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    pd.requires_grad_(True)
    loss = fused_lncc_loss(pd, td, 7)
    loss.backward()
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    vol_bytes = pd.numel() * 4
    assert extra <= vol_bytes + (64 << 20), f"extra HBM {extra / 1e9:.2f} GB"
    L = loss.item()
    assert np.isfinite(L) and 0.0 <= L <= 1.0
    g = pd.grad.detach().clone()
    pd.grad = None
    fused_lncc_loss(pd, td, 7).backward()
    assert torch.equal(g, pd.grad)
    pd.grad = None
    parts = []
    for lo in range(0, 2, 1):
        ps = pd.detach()[lo:lo + 1].clone().requires_grad_(True)
        ls = fused_lncc_loss(ps, td[lo:lo + 1], 7)
        ls.backward()
        parts.append(ls.item())
        gs = ps.grad * 0.5
        rel = ((gs - g[lo:lo + 1]).norm() / g[lo:lo + 1].norm()).item()
        assert rel < 1e-6
        del ps, gs
    assert abs(np.mean(parts) - L) <= 1e-6 * L


def test_bf16_rounding_is_round_to_nearest_even():
    """The bf16 gradient store rounds like torch's float32 -> bfloat16 (round to nearest, ties to
    even; NaN stays NaN; the reference's store_g, fused_lncc/csrc/lncc3d.cu:21), checked bit for bit
    through the bf16 grad *= grad_out kernel on a million random products, exact half-way cases,
    infinities and NaN."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(1 << 20, generator=g) * torch.exp(8 * torch.randn(1 << 20, generator=g))).to(torch.bfloat16)
    special = torch.tensor([1.0, -1.0, 2.0, 0.5, float("inf"), float("-inf"), float("nan"), 0.0, -0.0],
                           dtype=torch.bfloat16)
    x[: special.numel()] = special
    for s in (0.7310586, 1.0 + 2.0 ** -8, -3.25):  # 1 + 2^-8 puts powers of two exactly half-way
        out = x.to(DEV).clone()
        ext.scale_grad_(out, torch.tensor(s, device=DEV))
        torch.cuda.synchronize()
        want = (x.float() * torch.tensor(s, dtype=torch.float32)).to(torch.bfloat16)
        got = out.cpu()
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(got), nan)
        # products in the float32 denormal range are left out (the device's float32 mode decides them)
        tiny = want.float().abs() < 2.0 ** -126
        keep = ~nan & ~tiny
        assert torch.equal(got[keep].view(torch.int16), want[keep].view(torch.int16))


def test_under_bf16_autocast():
    """As the reference's README notes: under bf16 autocast the loss takes the bf16 activations
    directly and the gradient reaches the model's parameters; float16 is refused (cast first)."""
    torch.manual_seed(0)
    net = torch.nn.Conv3d(1, 1, 3, padding=1).to(DEV)
    x = torch.randn(1, 1, 16, 18, 20, device=DEV)
    t = torch.randn(1, 1, 16, 18, 20, device=DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = net(x)
        assert y.dtype == torch.bfloat16
        loss = fused_lncc_loss(y, t.bfloat16(), 5)
    loss.backward()
    assert loss.dtype == torch.float32 and torch.isfinite(loss)
    assert net.weight.grad is not None and torch.isfinite(net.weight.grad).all()
    assert net.weight.grad.abs().sum() > 0
    with pytest.raises(RuntimeError, match="float32 or bfloat16"):
        fused_lncc_loss(y.detach().half(), t.half(), 5)
