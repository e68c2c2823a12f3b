"""ctypes front-end of the CPU oracle (``liblncc_oracle.so``) — TEST INFRASTRUCTURE ONLY.

Only the tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` import this
module, as the reference the results are compared with. The product path (the ``fused_lncc``
package) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liblncc_oracle.so")
POLICY_TORCH = 0   # baselines/torch_lncc.py:25-32 semantics (no variance clamp, grad where ncc <= 1)
POLICY_KERNEL = 1  # fused_lncc/csrc/lncc3d.cu:93-107 semantics (variance clamp, adjoints 0 where ncc >= 1)

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        dp = ctypes.POINTER(ctypes.c_double)
        fp = ctypes.POINTER(ctypes.c_float)
        L.lncc_oracle.argtypes = [fp, fp] + [ctypes.c_int] * 5 + [ctypes.c_double, ctypes.c_int, dp,
                                                                   fp, dp, dp, dp, dp]
        L.lncc_oracle.restype = ctypes.c_int
        L.lncc_oracle_box3d.argtypes = [dp, dp] + [ctypes.c_int] * 5
        L.lncc_oracle_box3d.restype = None
        L.lncc_oracle_ref32.argtypes = [fp, fp] + [ctypes.c_int] * 5 + [ctypes.c_float, dp, fp, fp]
        L.lncc_oracle_ref32.restype = ctypes.c_int
        L.lncc_oracle_round_bf16.argtypes = [ctypes.c_float]
        L.lncc_oracle_round_bf16.restype = ctypes.c_float
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct)) if a is not None else None


def _bdhw(shape):
    if len(shape) == 5:
        return shape[0] * shape[1], shape[2], shape[3], shape[4]
    if len(shape) == 4:
        return tuple(shape)
    raise ValueError("expect (N,C,D,H,W) or (B,D,H,W)")


def lncc(pred, target, k, smooth_dr=1e-5, policy=POLICY_KERNEL, grad=True, maps=False):
    """Loss (float), gradient wrt pred (float32 array, or None) and optional float64 maps."""
    p, t = _f32(pred), _f32(target)
    assert p.shape == t.shape
    B, D, H, W = _bdhw(p.shape)
    loss = ctypes.c_double(0.0)
    g = np.empty(p.shape, np.float32) if grad else None
    mp = [np.empty(p.shape, np.float64) for _ in range(4)] if maps else [None] * 4
    rc = lib().lncc_oracle(_ptr(p, ctypes.c_float), _ptr(t, ctypes.c_float), B, D, H, W, int(k),
                           float(smooth_dr), int(policy), ctypes.byref(loss), _ptr(g, ctypes.c_float),
                           *[_ptr(m, ctypes.c_double) for m in mp])
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    if maps:
        return loss.value, g, dict(zip(("ncc", "A", "B", "C"), mp))
    return loss.value, g


def lncc_ref32(pred, target, k, smooth_dr=1e-5, grad=True, ncc_map=False):
    """What the reference kernel itself returns in float32 for these inputs (its direct k-tap
    float32 box-sums and IEEE divisions, fused_lncc/csrc/lncc3d.cu): loss (float), gradient wrt pred
    (float32 array or None) and, with ncc_map=True, the float32 ncc map. Used to bound the GPU
    path's error on ill-conditioned inputs by the reference's own error against the float64
    oracle."""
    p, t = _f32(pred), _f32(target)
    assert p.shape == t.shape
    B, D, H, W = _bdhw(p.shape)
    loss = ctypes.c_double(0.0)
    g = np.empty(p.shape, np.float32) if grad else None
    m = np.empty(p.shape, np.float32) if ncc_map else None
    rc = lib().lncc_oracle_ref32(_ptr(p, ctypes.c_float), _ptr(t, ctypes.c_float), B, D, H, W, int(k),
                                 float(smooth_dr), ctypes.byref(loss), _ptr(g, ctypes.c_float),
                                 _ptr(m, ctypes.c_float))
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    if ncc_map:
        return loss.value, g, m
    return loss.value, g


def box3d(x, k):
    """Zero-padded k^3 box-sum in float64 of an (N,C,D,H,W) or (B,D,H,W) array."""
    a = np.ascontiguousarray(x, dtype=np.float64)
    B, D, H, W = _bdhw(a.shape)
    y = np.empty_like(a)
    lib().lncc_oracle_box3d(_ptr(a, ctypes.c_double), _ptr(y, ctypes.c_double), B, D, H, W, int(k))
    return y


def round_bf16_np(x):
    """round_bf16 for whole arrays (finite values): float32 -> bfloat16 bits by round to nearest,
    ties to even, back to float32."""
    u = _f32(x).view(np.uint32)
    u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return u.view(np.float32)


def bf16_ulp(x):
    """The spacing of bfloat16 numbers (8 significant bits) at |x|, elementwise, float64."""
    a = np.abs(np.asarray(x, np.float64))
    _, e = np.frexp(a)
    return np.where(a > 0, np.ldexp(1.0, e - 8), 0.0)


def round_bf16(x):
    """float32 -> bfloat16 (round to nearest even) -> float32, elementwise, via the C routine."""
    f = lib().lncc_oracle_round_bf16
    a = _f32(x)
    return np.vectorize(lambda v: f(float(v)), otypes=[np.float32])(a)
