"""Pins the CPU oracle (oracle/lncc_oracle.c) before the GPU results are compared with it.

* golden vectors written from the reference's own torch LNCC (baselines/torch_lncc.py:12-42):
  loss and autograd gradient on full small tensors, loss plus gradient checksums at the
  MRI-shaped, headline and bf16 workloads;
* box-sum against brute force, the constant-field closed form and scipy's uniform_filter;
* gradient against float64 central finite differences of the oracle's own loss, and the
  self-adjoint identity <box a, b> = <a, box b> that the backward relies on;
* closed-form special cases (all-zero, constant pred, affine pred, NaN);
* sensitivity: a wrong k, a wrong dr or a wrong clamp policy fails the golden comparison;
* the float32 restatement of the reference kernel (lncc_ref32, the error yardstick of the GPU
  numerics tests): the golden vectors to float32 accuracy, exact zeros in zero and constant
  windows, float32-sized errors on offset intensities, and a wrong dr told apart.
"""
import glob
import os

import numpy as np
import pytest
import scipy.ndimage as ndi
import torch

import oracle as O
import workloads as wl

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FULL = sorted(f for f in glob.glob(os.path.join(GOLDEN, "*.npz")) if not os.path.basename(f).startswith("stats_"))
PARITY = [f for f in FULL if not os.path.basename(f).startswith("degen_")]


def _cos_rel(g, gr):
    g = np.asarray(g, np.float64).ravel()
    gr = np.asarray(gr, np.float64).ravel()
    n = np.linalg.norm(gr)
    return float(g @ gr / (np.linalg.norm(g) * n)), float(np.linalg.norm(g - gr) / n)


def test_fixture_set_present():
    names = {os.path.basename(f) for f in FULL}
    assert "cpu_k3.npz" in names and len(FULL) >= 15
    for n in ("mri", "headline", "bf16"):
        assert os.path.exists(os.path.join(GOLDEN, f"stats_{n}.npz"))


@pytest.mark.parametrize("path", PARITY, ids=[os.path.basename(p)[:-4] for p in PARITY])
@pytest.mark.parametrize("policy", [O.POLICY_TORCH, O.POLICY_KERNEL])
def test_oracle_matches_golden(path, policy):
    d = np.load(path)
    loss, g = O.lncc(d["pred"], d["target"], int(d["k"]), float(d["smooth_dr"]), policy=policy)
    ref = float(d["loss"])
    assert abs(loss - ref) <= 2e-6 * max(abs(ref), 1e-3)
    cos, rel = _cos_rel(g, d["grad"])
    assert cos > 0.999999 and rel < 1e-5


def test_oracle_degenerate_losses():
    for name, expect in (("degen_zero", 1.0), ("degen_const5", None)):
        d = np.load(os.path.join(GOLDEN, name + ".npz"))
        loss, g = O.lncc(d["pred"], d["target"], int(d["k"]))
        ref = float(d["loss"])
        assert abs(loss - ref) < 1e-6
        if expect is not None:
            assert loss == expect and np.all(g == 0)


@pytest.mark.parametrize("name", ["mri", "bf16", "headline"])
def test_oracle_matches_golden_stats(name):
    if name != "mri" and os.environ.get("FUSED_LNCC_FULL_CPU") != "1":
        pytest.skip("headline-size oracle run (set FUSED_LNCC_FULL_CPU=1)")
    st = np.load(os.path.join(GOLDEN, f"stats_{name}.npz"))
    p, t = wl.make_inputs(name)
    assert wl.checksum(p) == list(st["pred"]) and wl.checksum(t) == list(st["target"])
    loss, g = O.lncc(p.float().numpy(), t.float().numpy(), int(st["k"]))
    assert abs(loss - float(st["loss"])) <= 2e-6 * float(st["loss"])
    cks = wl.checksum(torch.from_numpy(g))
    assert abs(cks[1] - st["grad"][1]) <= 1e-5 * st["grad"][1]           # sum of squares
    assert abs(np.sqrt(cks[1]) - float(st["grad_l2"])) <= 1e-5 * float(st["grad_l2"])


def _brute_box(x, k):
    h = k // 2
    D, H, W = x.shape
    y = np.zeros_like(x, dtype=np.float64)
    for z in range(D):
        for yy in range(H):
            for xx in range(W):
                y[z, yy, xx] = x[max(z - h, 0):z + h + 1, max(yy - h, 0):yy + h + 1,
                                 max(xx - h, 0):xx + h + 1].sum()
    return y


@pytest.mark.parametrize("k", [3, 5, 7, 9])
def test_box_brute_force(k):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((1, 5, 6, 7))
    assert np.allclose(O.box3d(x, k)[0], _brute_box(x[0], k), rtol=0, atol=1e-12)


@pytest.mark.parametrize("k", [3, 7, 9])
def test_box_constant_closed_form(k):
    D, H, W, c, h = 11, 4, 13, 2.5, k // 2
    y = O.box3d(np.full((1, D, H, W), c), k)[0]
    cnt = [np.array([min(i + h, n - 1) - max(i - h, 0) + 1 for i in range(n)]) for n in (D, H, W)]
    expect = c * cnt[0][:, None, None] * cnt[1][None, :, None] * cnt[2][None, None, :]
    assert np.array_equal(y, expect)


@pytest.mark.parametrize("k", [3, 5, 7])
def test_box_uniform_filter(k):
    rng = np.random.default_rng(10 + k)
    x = rng.standard_normal((2, 9, 10, 12))
    ref = np.stack([ndi.uniform_filter(v, size=k, mode="constant", cval=0.0) * k ** 3 for v in x])
    assert np.allclose(O.box3d(x, k), ref, rtol=1e-10, atol=1e-10)


def test_box_self_adjoint():
    rng = np.random.default_rng(3)
    a, b = rng.standard_normal((2, 1, 7, 8, 9))
    lhs = np.sum(O.box3d(a, 5) * b)
    rhs = np.sum(a * O.box3d(b, 5))
    assert abs(lhs - rhs) < 1e-9 * abs(lhs)


@pytest.mark.parametrize("k,policy", [(3, O.POLICY_KERNEL), (5, O.POLICY_TORCH)])
def test_grad_finite_differences(k, policy):
    rng = np.random.default_rng(7)
    p = rng.standard_normal((1, 1, 5, 6, 4)).astype(np.float32)
    t = (0.5 * p + rng.standard_normal(p.shape)).astype(np.float32)
    _, g = O.lncc(p, t, k, 1e-2, policy=policy)
    eps = 1e-3
    worst = 0.0
    for idx in [(0, 0, 0, 0, 0), (0, 0, 2, 3, 1), (0, 0, 4, 5, 3), (0, 0, 1, 0, 2), (0, 0, 3, 2, 0)]:
        # central difference on values exactly representable in float32
        pp, pm = p.copy(), p.copy()
        pp[idx] += eps
        pm[idx] -= eps
        step = float(pp[idx]) - float(pm[idx])
        lp, _ = O.lncc(pp, t, k, 1e-2, policy=policy, grad=False)
        lm, _ = O.lncc(pm, t, k, 1e-2, policy=policy, grad=False)
        fd = (lp - lm) / step
        worst = max(worst, abs(fd - g[idx]) / max(abs(g[idx]), 1e-6))
    assert worst < 2e-3


def test_special_cases():
    rng = np.random.default_rng(5)
    t = rng.standard_normal((1, 1, 9, 9, 9)).astype(np.float32)
    # constant pred: windows inside the volume have cross = 0 -> ncc = 0 (the zero padding makes
    # border windows non-constant)
    _, _, maps = O.lncc(np.full_like(t, 3.0), t, 5, maps=True)
    assert np.all(np.abs(maps["ncc"][0, 0, 2:-2, 2:-2, 2:-2]) < 1e-12)
    assert np.all(maps["ncc"][0, 0, 0] > 0)
    # affine pred: interior windows have |corr| = 1 -> ncc ~ 1 (only dr keeps it below)
    _, _, maps = O.lncc(2.0 * t + 1.0, t, 3, 0.0, maps=True)
    assert np.allclose(maps["ncc"][0, 0, 1:-1, 1:-1, 1:-1], 1.0, atol=1e-9)
    # NaN anywhere -> NaN loss (fused_lncc/csrc/lncc3d.cu:105-107)
    p = rng.standard_normal(t.shape).astype(np.float32)
    p[0, 0, 4, 4, 4] = np.nan
    loss, _ = O.lncc(p, t, 3)
    assert np.isnan(loss)
    # pearson: an interior ncc equals the squared correlation coefficient of the window (dr = 0)
    p = rng.standard_normal(t.shape).astype(np.float32)
    _, _, maps = O.lncc(p, t, 5, 0.0, maps=True)
    win = (slice(2, 7), slice(1, 6), slice(3, 8))
    r = np.corrcoef(p[0, 0][win].astype(np.float64).ravel(), t[0, 0][win].astype(np.float64).ravel())[0, 1]
    assert abs(maps["ncc"][0, 0, 4, 3, 5] - r * r) < 1e-12


def test_golden_comparison_is_sensitive():
    """Plausible mistakes in the oracle's parameters fail the golden comparison."""
    d = np.load(os.path.join(GOLDEN, "dr1_k3.npz"))
    p, t, ref = d["pred"], d["target"], float(d["loss"])
    ok, _ = O.lncc(p, t, 3, 1.0)
    assert abs(ok - ref) < 1e-6
    wrong_dr, _ = O.lncc(p, t, 3, 1e-5)
    wrong_k, _ = O.lncc(p, t, 5, 1.0)
    assert abs(wrong_dr - ref) > 1e-3 and abs(wrong_k - ref) > 1e-3
    # swapping pred and target changes the gradient wrt pred
    _, g = O.lncc(p, t, 3, 1.0)
    _, gs = O.lncc(t, p, 3, 1.0)
    assert _cos_rel(gs, d["grad"])[1] > 1e-2 and _cos_rel(g, d["grad"])[1] < 1e-5


def test_policies_differ_only_where_clamped():
    rng = np.random.default_rng(9)
    t = rng.standard_normal((1, 1, 8, 8, 8)).astype(np.float32)
    p = (t + 1e-4 * rng.standard_normal(t.shape)).astype(np.float32)
    lk, gk = O.lncc(p, t, 3, 1e-5, policy=O.POLICY_KERNEL)
    lt, gt = O.lncc(p, t, 3, 1e-5, policy=O.POLICY_TORCH)
    assert abs(lk - lt) < 1e-12 and np.allclose(gk, gt)


def test_round_bf16_matches_torch():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.14159, 65504.0, 1e-30, np.inf, -np.inf], np.float32)
    ours = O.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, ref)
    assert np.isnan(O.round_bf16(np.array([np.nan], np.float32))[0])


def test_round_bf16_array_form():
    """The vectorized rounding the bf16 gradient checks use agrees with the C routine and with
    torch's float32 -> bfloat16 cast on a million values spanning the exponent range, exact ties
    included; bf16_ulp is the spacing of bfloat16 numbers (2^-7 at 1, halved below each power of
    two)."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(1 << 20, generator=g) * torch.exp(10 * torch.randn(1 << 20, generator=g))).numpy()
    ties = (np.arange(1, 2001, dtype=np.uint32) << 16 | np.uint32(0x8000)).view(np.float32)
    x = np.concatenate([x, ties, -ties]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.round_bf16_np(x), ref)
    assert np.array_equal(O.round_bf16_np(x[:512]), O.round_bf16(x[:512]))
    assert O.bf16_ulp(np.array([1.0]))[0] == 2.0 ** -7 and O.bf16_ulp(np.array([0.75]))[0] == 2.0 ** -8
    # the next bf16 number away from zero is one unit up in the magnitude bits
    v = ref[:4096][(ref[:4096] != 0) & np.isfinite(ref[:4096])]
    nxt = (v.view(np.uint32) + np.uint32(1 << 16)).view(np.float32)
    ok = np.isfinite(nxt)
    gap = np.abs(nxt[ok].astype(np.float64) - v[ok].astype(np.float64))
    assert np.array_equal(gap, O.bf16_ulp(v[ok]))


@pytest.mark.parametrize("path", FULL, ids=[os.path.basename(p)[:-4] for p in FULL])
def test_separable_loss_of_the_fixtures(path):
    """Every fixture also holds the loss of the reference's separable box-sum path
    (baselines/torch_lncc.py:17-22,40-42, three 1-D convolutions). The float64 oracle matches it at
    the parity bar, and the restated separable path reproduces it (the degenerate constant fields
    are rounding noise in the reference: range only)."""
    import torch_lncc_port as port
    d = np.load(path)
    k, dr = int(d["k"]), float(d["smooth_dr"])
    lsep = float(d["loss_separable"])
    p, t = torch.from_numpy(d["pred"]), torch.from_numpy(d["target"])
    ls = float(port.lncc_separable(p, t, k, dr))
    if os.path.basename(path).startswith("degen_"):
        assert 0.0 <= lsep <= 1.0 and 0.0 <= ls <= 1.0
        return
    lo, _ = O.lncc(d["pred"], d["target"], k, dr, grad=False)
    assert abs(lo - lsep) <= 1e-5 * abs(lsep), (lo, lsep)
    assert abs(ls - lsep) <= 1e-6 * abs(lsep), (ls, lsep)


def test_separable_box_is_the_dense_box():
    import torch_lncc_port as port
    x = torch.randn(2, 3, 9, 11, 13, dtype=torch.float64)
    for k in (3, 5, 7, 9):
        a = port.box_separable(x, k)
        assert torch.allclose(a, port.box_dense(x, k), rtol=1e-12, atol=1e-12)
        assert np.allclose(a.numpy(), O.box3d(x.numpy(), k), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", ["cpu_k3", "nc_k5", "dr1_k3", "edge_k7_1x3x7x9x11"])
def test_torch_port_matches_golden(name):
    """The CPU baseline (the reference's naive torch path, restated) reproduces the golden vectors."""
    import torch_lncc_port
    d = np.load(os.path.join(GOLDEN, name + ".npz"))
    loss, g = torch_lncc_port.loss_and_grad(torch.from_numpy(d["pred"]), torch.from_numpy(d["target"]),
                                            int(d["k"]), float(d["smooth_dr"]))
    assert abs(float(loss) - float(d["loss"])) <= 1e-6 * max(abs(float(d["loss"])), 1e-3)
    cos, rel = _cos_rel(g.numpy(), d["grad"])
    assert cos > 0.999999 and rel < 1e-5


# ---- the float32 restatement of the reference kernel (lncc_oracle_ref32), the yardstick of the
# GPU numerics tests: pinned here to the reference's own outputs and to exact cases

@pytest.mark.parametrize("path", PARITY, ids=[os.path.basename(p)[:-4] for p in PARITY])
def test_ref32_matches_golden(path):
    """Same loss and gradient as the reference's torch path, to float32 accuracy."""
    d = np.load(path)
    loss, g = O.lncc_ref32(d["pred"], d["target"], int(d["k"]), float(d["smooth_dr"]))
    ref = float(d["loss"])
    assert abs(loss - ref) <= 5e-6 * max(abs(ref), 1e-3)
    cos, rel = _cos_rel(g, d["grad"])
    assert cos > 1 - 1e-10 and rel < 1e-5


def test_ref32_exact_in_zero_and_constant_windows():
    """Direct float32 window sums: a window of exact zeros, or of one representable constant per
    input, sums exactly, so ncc and the adjoints there are exactly 0, as in float64."""
    rng = np.random.default_rng(17)
    p = rng.random((1, 1, 20, 11, 13)).astype(np.float32)
    t = (0.6 * p + 0.4 * rng.random(p.shape)).astype(np.float32)
    p[0, 0, 8:], t[0, 0, 8:] = 0.0, 0.0          # zero slab after the signal
    p[0, 0, :, :, 7:], t[0, 0, :, :, 7:] = 0.5, 7.0   # constant block along W
    for k in (3, 5):
        l64, g64, maps = O.lncc(p, t, k, maps=True)
        l32, g32, m32 = O.lncc_ref32(p, t, k, ncc_map=True)
        zero = maps["ncc"] == 0
        assert zero.sum() > 200 and np.all(m32[zero] == 0)
        gz = g64 == 0
        assert gz.sum() > 200 and np.all(g32[gz] == 0)
        assert abs(l32 - l64) < 1e-6


def test_ref32_rounds_in_float32():
    """On offset intensities (100 + N(0,1)) the restatement's error against float64 is that of
    float32 cancellation (far above float64 rounding), and a wrong dr is still told apart."""
    rng = np.random.default_rng(3)
    t = rng.standard_normal((1, 1, 10, 12, 12)).astype(np.float32)
    p = (0.8 * t + 0.6 * rng.standard_normal(t.shape)).astype(np.float32)
    l64, g64 = O.lncc(p + 100, t + 100, 5)
    l32, g32 = O.lncc_ref32(p + 100, t + 100, 5)
    assert 1e-6 < abs(l32 - l64) < 1e-3
    assert 1e-5 < _cos_rel(g32, g64)[1] < 1e-2
    d = np.load(os.path.join(GOLDEN, "dr1_k3.npz"))
    wrong, _ = O.lncc_ref32(d["pred"], d["target"], 3, 1e-5)
    assert abs(wrong - float(d["loss"])) > 1e-3
