"""Randomized parity sweep: many small shapes (edges smaller than the halo, one-plane volumes,
ragged tiles), every kernel size, both dtypes, against the CPU oracle with the parity bar.
The second sweep asks for both gradients (target_grad=True: the pred-gradient kernel, then the
same kernel with the inputs swapped) and forces short D-chunks on some cases, so chunk seams land
inside the volume.
Seeded, so every run draws the same cases; each case prints its parameters on failure."""
import random

import numpy as np
import pytest
import torch

import oracle as O
import workloads as wl
from fused_lncc import fused_lncc_loss

pytestmark = pytest.mark.gpu


def _cases(n=60, seed=11):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        k = rng.choice([3, 5, 7, 9])
        shape = (rng.randint(1, 2), rng.randint(1, 2), rng.randint(1, 36), rng.randint(1, 66), rng.randint(1, 66))
        dt = rng.choice(["f32", "f32", "bf16"])
        corr = rng.random() < 0.3
        out.append((i, k, shape, dt, corr))
    return out


def _check_grad(g, gr, dt):
    g = g.double().cpu().numpy().ravel()
    gr = np.asarray(gr, np.float64).ravel()
    n = np.linalg.norm(gr)
    if n == 0:
        assert np.linalg.norm(g) == 0
        return
    cos = float(g @ gr / (np.linalg.norm(g) * n))
    rel = float(np.linalg.norm(g - gr) / n)
    if dt == "f32":
        assert cos > 0.9999 and rel < 1e-3, (cos, rel)
    else:  # the gradient is rounded once to bf16 (8 significant bits): within one ulp of the
        # rounded oracle gradient, up to float32 error near zero
        assert cos > 0.9999 and rel <= 3e-3, (cos, rel)
        rb = O.round_bf16_np(gr).astype(np.float64)
        bad = np.abs(g - rb) > O.bf16_ulp(rb) + 1e-5 * np.abs(gr).max()
        assert not bad.any(), f"{bad.sum()} of {bad.size} elements beyond one bf16 ulp"


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}-k{c[1]}-{'x'.join(map(str, c[2]))}-{c[3]}")
def test_random_shapes(case):
    i, k, shape, dt, corr = case
    p, t = wl.randn_pair(shape, 500 + i)
    if corr:
        p = 0.8 * t + 0.2 * p
    dtype = torch.float32 if dt == "f32" else torch.bfloat16
    pq, tq = p.to(dtype), t.to(dtype)
    pd = pq.to("cuda").requires_grad_(True)
    loss = fused_lncc_loss(pd, tq.to("cuda"), k)
    loss.backward()
    torch.cuda.synchronize()
    lr, gr = O.lncc(pq.float().numpy(), tq.float().numpy(), k)
    assert pd.grad.dtype == dtype
    assert abs(loss.item() - lr) <= (1e-5 if dt == "f32" else 1e-2) * abs(lr)
    _check_grad(pd.grad, gr, dt)


def _cases_both(n=40, seed=23):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        k = rng.choice([3, 5, 7, 9])
        shape = (rng.randint(1, 2), rng.randint(1, 2), rng.randint(1, 40), rng.randint(1, 72), rng.randint(1, 72))
        dt = rng.choice(["f32", "f32", "bf16"])
        corr = rng.random() < 0.3
        dchunk = rng.choice([0, 0, 1, 2, 5, 11])   # 0: the planner's own chunking
        out.append((i, k, shape, dt, corr, dchunk))
    return out


@pytest.mark.parametrize("case", _cases_both(),
                         ids=lambda c: f"{c[0]}-k{c[1]}-{'x'.join(map(str, c[2]))}-{c[3]}-dc{c[5]}")
def test_random_shapes_both_gradients(case, force_dchunk):
    i, k, shape, dt, corr, dchunk = case
    if dchunk:
        force_dchunk(dchunk)
    p, t = wl.randn_pair(shape, 900 + i)
    if corr:
        p = 0.85 * t + 0.15 * p
    dtype = torch.float32 if dt == "f32" else torch.bfloat16
    pq, tq = p.to(dtype), t.to(dtype)
    pd = pq.to("cuda").requires_grad_(True)
    td = tq.to("cuda").requires_grad_(True)
    loss = fused_lncc_loss(pd, td, k, target_grad=True)
    loss.backward()
    torch.cuda.synchronize()
    lr, gr = O.lncc(pq.float().numpy(), tq.float().numpy(), k)
    _, grt = O.lncc(tq.float().numpy(), pq.float().numpy(), k)   # the loss is symmetric in its inputs
    assert pd.grad.dtype == dtype and td.grad.dtype == dtype
    assert abs(loss.item() - lr) <= (1e-5 if dt == "f32" else 1e-2) * abs(lr)
    _check_grad(pd.grad, gr, dt)
    _check_grad(td.grad, grt, dt)
