"""Shared gradient checks of the GPU parity tests (imported by the test modules)."""
import numpy as np

import oracle as O


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
