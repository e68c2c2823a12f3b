"""Large seeded parity sweep of fused_lncc_loss against the oracle, on the GPU: random shapes up to
(2,2,48,80,80), every k, fp32 and bf16, 30% with both gradients, forced D-chunks of 1-17 planes,
correlated inputs and zero slabs after signal; the parity bar of tests/test_gpu_sweep.py.
Not collected by pytest (minutes per 10,000 cases); prints one line per failing case.
usage: python tests/gpu_sweep_large.py N SEED"""
import os
import random
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("fused-lncc_amd", "oracle", os.path.join("tests", "golden")):
    sys.path.insert(0, os.path.join(ROOT, sub))
import oracle as O
import workloads as wl
from fused_lncc import fused_lncc_loss, _lib

def check_grad(g, gr, dt):
    g = g.double().cpu().numpy().ravel(); gr = np.asarray(gr, np.float64).ravel()
    n = np.linalg.norm(gr)
    if n == 0:
        return np.linalg.norm(g) == 0, "zero"
    cos = float(g @ gr / (np.linalg.norm(g) * n)); rel = float(np.linalg.norm(g - gr) / n)
    if dt == "f32":
        return cos > 0.9999 and rel < 1e-3, (cos, rel)
    rb = O.round_bf16_np(gr).astype(np.float64)
    bad = np.abs(g - rb) > O.bf16_ulp(rb) + 1e-5 * np.abs(gr).max()
    return cos > 0.9999 and rel <= 3e-3 and not bad.any(), (cos, rel, int(bad.sum()))

N = int(sys.argv[1]); seed = int(sys.argv[2])
rng = random.Random(seed)
lib = _lib.load()
fails = 0; t0 = time.time()
for i in range(N):
    k = rng.choice([3, 5, 7, 9])
    shape = (rng.randint(1, 2), rng.randint(1, 2), rng.randint(1, 48), rng.randint(1, 80), rng.randint(1, 80))
    dt = rng.choice(["f32", "f32", "bf16"])
    both = rng.random() < 0.3
    dchunk = rng.choice([0, 0, 0, 1, 2, 3, 5, 11, 17])
    mode = rng.random()
    p, t = wl.randn_pair(shape, seed * 100000 + i)
    if mode < 0.2:
        p = 0.8 * t + 0.2 * p
    elif mode < 0.3:   # a zero slab after signal along D
        z = shape[2] // 2
        p[:, :, z:] = 0; t[:, :, z:] = 0
    dtype = torch.float32 if dt == "f32" else torch.bfloat16
    pq, tq = p.to(dtype), t.to(dtype)
    lib.fl_test_set_dchunk(dchunk)
    pd = pq.to("cuda").requires_grad_(True); td = tq.to("cuda").requires_grad_(both)
    loss = fused_lncc_loss(pd, td, k, target_grad=both)
    loss.backward()
    torch.cuda.synchronize()
    lib.fl_test_set_dchunk(0)
    lr, gr = O.lncc(pq.float().numpy(), tq.float().numpy(), k)
    okl = abs(loss.item() - lr) <= (1e-5 if dt == "f32" else 1e-2) * max(abs(lr), 1e-6)
    okg, info = check_grad(pd.grad, gr, dt)
    okt, infot = True, None
    if both:
        _, grt = O.lncc(tq.float().numpy(), pq.float().numpy(), k)
        okt, infot = check_grad(td.grad, grt, dt)
    if not (okl and okg and okt):
        fails += 1
        print("FAIL", i, k, shape, dt, "both" if both else "", "dchunk", dchunk, "mode", round(mode, 2), "loss", loss.item(), lr, info, infot, flush=True)
    if (i + 1) % 250 == 0:
        print(f"{i + 1} cases, {fails} failures, {time.time() - t0:.0f} s", flush=True)
print("done", N, "cases,", fails, "failures")
