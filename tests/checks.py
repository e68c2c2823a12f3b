"""Shared checks of the GPU parity tests (imported by the test modules)."""
import numpy as np

import oracle as O

RATIO = 4.0   # the HIP path may be at most this many times further from float64 than the reference


def cos_rel(g, gr):
    """Cosine similarity and relative L2 error of g against the reference gradient gr."""
    g = np.asarray(g, np.float64).ravel()
    gr = np.asarray(gr, np.float64).ravel()
    n = np.linalg.norm(gr)
    return float(g @ gr / (np.linalg.norm(g) * n)), float(np.linalg.norm(g - gr) / n)


def assert_grad_bf16(g, gr):
    """A bfloat16 gradient against the float32 oracle gradient of the same (bf16-representable)
    inputs: the kernel accumulates in float32 and rounds once to nearest even, so the gradient is
    the oracle's rounded to bf16 up to the float32 error: within one bf16 ulp of round_bf16(oracle)
    everywhere (plus 1e-5 of the gradient's scale for elements near zero), relative L2 error <=
    3e-3 (one rounding to 8 significant bits costs ~1.1e-3) and cosine > 0.9999. The reference's
    own bf16 checks are looser (tests/test_bf16.py:10-21)."""
    g = np.asarray(g, np.float64).ravel()
    gr = np.asarray(gr, np.float64).ravel()
    c, r = cos_rel(g, gr)
    assert c > 0.9999 and r <= 3e-3, f"bf16 gradient cos={c:.8f} relL2={r:.3e}"
    rb = O.round_bf16_np(gr).astype(np.float64)
    tol = O.bf16_ulp(rb) + 1e-5 * np.abs(gr).max()
    bad = np.abs(g - rb) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} bf16 gradient elements more than one ulp from the rounded oracle"


def gpu_loss_grad_map(p, t, k, dr=1e-5, dtype=None):
    """fused_lncc_loss + backward and lncc_map on the GPU: (loss, gradient, ncc map) as float64."""
    import torch
    from fused_lncc import fused_lncc_loss, lncc_map
    dtype = dtype or torch.float32
    pd = p.to(dtype).to("cuda").requires_grad_(True)
    td = t.to(dtype).to("cuda")
    loss = fused_lncc_loss(pd, td, k, dr)
    loss.backward()
    m = lncc_map(pd, td, k, dr)
    torch.cuda.synchronize()
    return float(loss.item()), pd.grad.double().cpu().numpy(), m.double().cpu().numpy()


def rel_l2(g, ref):
    n = np.linalg.norm(ref)
    return float(np.linalg.norm(g - ref) / n) if n > 0 else float(np.linalg.norm(g))


def cosine(g, ref):
    return float(np.dot(g.ravel(), ref.ravel()) / (np.linalg.norm(g) * np.linalg.norm(ref)))


def check_against_oracle(p, t, k, dr=1e-5, dtype=None):
    """The HIP loss, ncc map and gradient against the float64 oracle, bounded by the parity bar or
    by RATIO times the error of the reference's own float32 arithmetic. With dtype bfloat16 the
    kernel reads the inputs rounded to bf16 (the oracle gets the same values) and rounds its
    gradient once to bf16, which adds at most 2^-8 of each element (the gradient bound grows by
    4e-3); the loss and the ncc map are float32 and keep their bounds."""
    import torch
    dtype = dtype or torch.float32
    if dtype == torch.bfloat16:
        p, t = p.bfloat16().float(), t.bfloat16().float()
    loss, g, m = gpu_loss_grad_map(p, t, k, dr, dtype)
    pn, tn = p.numpy(), t.numpy()
    l64, g64, maps = O.lncc(pn, tn, k, dr, grad=True, maps=True)
    m64 = maps["ncc"]
    l32, g32, m32 = O.lncc_ref32(pn, tn, k, dr, grad=True, ncc_map=True)
    g64 = g64.astype(np.float64)
    g32 = g32.astype(np.float64)
    m32 = m32.astype(np.float64)
    tag = f"k={k} shape={tuple(p.shape)} {str(dtype)[6:]}"

    # The loss is the mean of the ncc map, so its error is the mean of the per-voxel errors: its
    # scale is the reference's RMS map error over sqrt(N / k^3) (errors are correlated over a
    # window), of which the reference's own loss error is one sample.
    e32 = m32 - m64
    rms32 = float(np.sqrt(np.mean(e32 * e32)))
    scale = rms32 * np.sqrt(k ** 3 / e32.size)
    err_l, err_l32 = abs(loss - l64), abs(l32 - l64)
    assert err_l <= max(RATIO * max(err_l32, scale), 1e-5 * abs(l64)), \
        f"{tag}: loss {loss:.9f} oracle {l64:.9f} ref32 {l32:.9f} (error scale {scale:.2e})"

    # exact zeros where the reference's direct sums are exact
    zm = (m64 == 0) & (m32 == 0)
    assert np.count_nonzero(m[zm]) == 0, f"{tag}: {np.count_nonzero(m[zm])} of {zm.sum()} exact-zero ncc voxels are not zero (max {np.abs(m[zm]).max():.3e})"
    zg = (g64 == 0) & (g32 == 0)
    assert np.count_nonzero(g[zg]) == 0, f"{tag}: {np.count_nonzero(g[zg])} of {zg.sum()} exact-zero gradient voxels are not zero (max {np.abs(g[zg]).max():.3e})"

    err_m, err_m32 = np.abs(m - m64).max(), np.abs(e32).max()
    assert err_m <= max(RATIO * err_m32, 1e-4), f"{tag}: ncc map max error {err_m:.3e} (reference {err_m32:.3e})"
    rms = float(np.sqrt(np.mean((m - m64) ** 2)))
    assert rms <= max(2.0 * rms32, 1e-6), f"{tag}: ncc map RMS error {rms:.3e} (reference {rms32:.3e})"

    if np.linalg.norm(g64) > 0:
        rel, rel32 = rel_l2(g, g64), rel_l2(g32, g64)
        c = cosine(g, g64)
        rounding = 4e-3 if dtype == torch.bfloat16 else 0.0
        assert rel <= max(RATIO * rel32, 1e-3) + rounding and c > 1 - max(RATIO * (1 - cosine(g32, g64)), 1e-4), \
            f"{tag}: gradient relL2 {rel:.3e} cos {c:.8f} (reference relL2 {rel32:.3e})"
    return zm.sum(), zg.sum()
