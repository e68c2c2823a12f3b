"""Synthetic input recipes for the LNCC workloads (CPU-generated, bit-identical across machines).

Every tensor is drawn on the CPU from a seeded ``torch.Generator`` and only then moved to a
device, so the GPU tests, the fixtures and the benchmark all see the same bytes.

Workloads (pred, target are (N, C, D, H, W)):

* ``cpu``      (1,1,32,32,32) fp32, k=3: target ~ U[0,1) seed 0, pred = 0.7*target + 0.3*U[0,1) seed 1.
* ``mri``      (1,1,160,192,224) fp32, k=9: target = N(0,1) seed 0, Gaussian-smoothed (sigma 2 voxels,
  separable, truncated at 4 sigma, reflect padding, float64), min-max scaled to [0,1];
  pred = roll(target, +2 along W) + 0.05*N(0,1) seed 1.
* ``headline`` (2,16,128,128,128) fp32, k=7: target ~ N(0,1) seed 0, pred = 0.8*target + 0.6*N(0,1) seed 1.
* ``bf16``     the headline recipe at (2,16,128,128,128) built in fp32, cast to bf16, k=5.
* ``large``    the headline recipe at (2,16,256,256,256) fp32, k=7.
* ``feat16``   (1,256,16,16,16) fp32, k=7, and ``feat64`` (2,64,64,64,64) fp32, k=7: the reference's other
  two benchmark shapes (bench.py:52, BENCHMARKS.md:17-18), many channels of small feature volumes;
  pred, target ~ N(0,1) independent (seeds 0 and 1), as the reference's benchmark draws them.
"""
import math

import numpy as np
import torch

WORKLOADS = {
    "cpu": dict(shape=(1, 1, 32, 32, 32), k=3, dtype="float32"),
    "mri": dict(shape=(1, 1, 160, 192, 224), k=9, dtype="float32"),
    "headline": dict(shape=(2, 16, 128, 128, 128), k=7, dtype="float32"),
    "bf16": dict(shape=(2, 16, 128, 128, 128), k=5, dtype="bfloat16"),
    "large": dict(shape=(2, 16, 256, 256, 256), k=7, dtype="float32"),
    "feat16": dict(shape=(1, 256, 16, 16, 16), k=7, dtype="float32"),
    "feat64": dict(shape=(2, 64, 64, 64, 64), k=7, dtype="float32"),
}


def _gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _gauss_smooth_f64(x, sigma=2.0):
    """Separable Gaussian (truncated at 4 sigma, reflect padding) over the last three axes, float64."""
    r = int(math.ceil(4 * sigma))
    taps = np.exp(-0.5 * (np.arange(-r, r + 1) / sigma) ** 2)
    taps /= taps.sum()
    y = x.astype(np.float64)
    for ax in (-3, -2, -1):
        pad = [(0, 0)] * y.ndim
        pad[ax] = (r, r)
        yp = np.pad(y, pad, mode="reflect")
        n = y.shape[ax]
        acc = np.zeros_like(y)
        for i, w in enumerate(taps):
            acc += w * np.take(yp, np.arange(i, i + n), axis=ax)
        y = acc
    return y


def make_inputs(name, shape=None):
    """Return (pred, target) as CPU tensors for workload ``name`` (optionally at another shape)."""
    spec = WORKLOADS[name]
    shape = tuple(shape or spec["shape"])
    if name == "cpu":
        t = torch.rand(shape, generator=_gen(0))
        p = 0.7 * t + 0.3 * torch.rand(shape, generator=_gen(1))
    elif name == "mri":
        noise = torch.randn(shape, generator=_gen(0)).numpy()
        sm = _gauss_smooth_f64(noise)
        sm = (sm - sm.min()) / (sm.max() - sm.min())
        t = torch.from_numpy(sm.astype(np.float32))
        p = torch.roll(t, shifts=2, dims=-1) + 0.05 * torch.randn(shape, generator=_gen(1))
    elif name in ("headline", "bf16", "large"):
        t = torch.randn(shape, generator=_gen(0))
        p = 0.8 * t + 0.6 * torch.randn(shape, generator=_gen(1))
        if name == "bf16":
            t, p = t.to(torch.bfloat16), p.to(torch.bfloat16)
    elif name in ("feat16", "feat64"):
        p = torch.randn(shape, generator=_gen(0))
        t = torch.randn(shape, generator=_gen(1))
    else:
        raise KeyError(name)
    return p.contiguous(), t.contiguous()


def randn_pair(shape, seed, dtype=torch.float32):
    """Independent N(0,1) pred/target pair, the input style of the reference's own tests."""
    g = _gen(seed)
    p = torch.randn(shape, generator=g)
    t = torch.randn(shape, generator=g)
    return p.to(dtype).contiguous(), t.to(dtype).contiguous()


def structured_pair(shape, kind, seed, axis=None, start=0, fill=0.0):
    """Pred/target pairs with the structure real volumes have, float32 on the CPU:

    * ``unit``   target ~ U[0,1), pred = 0.7*target + 0.3*U[0,1) (intensities scaled to [0,1]);
    * ``byte``   integer intensities: target ~ U{0..255}, pred = clip(target + U{-24..24}, 0, 255);
    * ``offset`` target = 100 + N(0,1), pred = 100 + 0.8*(target - 100) + 0.6*N(0,1): unit
      contrast on a large offset, where the variances cancel most digits of the box-sums.

    With ``axis`` (2 = D, 3 = H, 4 = W of the (N,C,D,H,W) shape) both volumes are set to ``fill``
    from index ``start`` on along that axis: an exactly zero background, or a constant one, after
    the signal, as in skull-stripped or padded scans."""
    g = _gen(seed)
    if kind == "unit":
        t = torch.rand(shape, generator=g)
        p = 0.7 * t + 0.3 * torch.rand(shape, generator=g)
    elif kind == "byte":
        t = torch.randint(0, 256, shape, generator=g).float()
        p = (t + torch.randint(-24, 25, shape, generator=g).float()).clamp(0, 255)
    elif kind == "offset":
        n = torch.randn(shape, generator=g)
        t = 100.0 + n
        p = 100.0 + 0.8 * n + 0.6 * torch.randn(shape, generator=g)
    else:
        raise KeyError(kind)
    if axis is not None:
        idx = [slice(None)] * len(shape)
        idx[axis] = slice(start, None)
        t[tuple(idx)] = fill
        p[tuple(idx)] = fill
    return p.contiguous(), t.contiguous()


def checksum(x):
    """Order-fixed float64 digest of a tensor: (sum, sum of squares, weighted sum)."""
    a = x.detach().to(torch.float64).reshape(-1).cpu().numpy()
    w = np.cos(np.arange(a.size, dtype=np.float64) * 0.001)
    return [float(np.sum(a)), float(np.sum(a * a)), float(np.dot(a, w))]
