"""Write golden vectors for the LNCC loss from the reference's own pure-PyTorch implementation.

Run once, in a container that holds the reference checkout, with
``python tests/golden/make_golden.py [--large]``. It loads ``baselines/torch_lncc.py`` of the
reference (``lncc_dense``/``lncc_separable``: grouped ``F.conv3d`` box-sums, zero padding,
``torch_lncc.py:12-42``), evaluates the loss and the autograd gradient with respect to ``pred`` on
the CPU in float32, and stores inputs and outputs as ``.npz`` data under this directory. Nothing
here runs at test time: the tests read only the ``.npz`` files.

Small cases keep full tensors. ``--large`` adds the big workloads (MRI-shaped k=9, the
(2,16,128^3) k=7 headline and its bf16/k=5 variant) as loss values plus order-fixed float64
checksums of the inputs and of the gradient.
"""
import argparse
import importlib.util
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import workloads as wl  # noqa: E402

REF_FILE = "/root/reference/baselines/torch_lncc.py"


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_torch_lncc", REF_FILE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def run_ref(ref, p, t, k, dr=1e-5, separable=False):
    p = p.detach().float().clone().requires_grad_(True)
    t = t.detach().float()
    fn = ref.lncc_separable if separable else ref.lncc_dense
    loss = fn(p, t, k, dr)
    loss.backward()
    return float(loss.item()), p.grad.detach().clone()


def save_full(ref, name, p, t, k, dr=1e-5, note=""):
    loss, grad = run_ref(ref, p, t, k, dr)
    loss_sep, _ = run_ref(ref, p, t, k, dr, separable=True)
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(
        path, pred=p.float().numpy(), target=t.float().numpy(), k=np.int32(k),
        smooth_dr=np.float64(dr), loss=np.float64(loss), loss_separable=np.float64(loss_sep),
        grad=grad.numpy(), note=np.str_(note))
    print(f"{name}: shape={tuple(p.shape)} k={k} dr={dr} loss={loss:.9f} sep={loss_sep:.9f}")


def small_cases(ref):
    p, t = wl.make_inputs("cpu")
    save_full(ref, "cpu_k3", p, t, 3, note="workload cpu (1,1,32^3) k=3")
    edge = [(1, 1, 2, 2, 2), (1, 1, 2, 40, 40), (1, 3, 7, 9, 11), (3, 5, 13, 17, 19), (1, 1, 128, 1, 1)]
    for i, shp in enumerate(edge):
        p, t = wl.randn_pair(shp, 100 + i)
        save_full(ref, "edge_k7_" + "x".join(map(str, shp)), p, t, 7, note="edge shape, randn")
    for k in (3, 5, 7, 9):
        p, t = wl.randn_pair((1, 2, 12, 10, 14), 200 + k)
        save_full(ref, f"nc_k{k}", p, t, k, note="non-cubic (1,2,12,10,14), randn")
    shp = (1, 1, 10, 10, 10)
    z = torch.zeros(shp)
    save_full(ref, "degen_zero", z, z, 7, note="all zero")
    c5 = torch.full(shp, 5.0)
    save_full(ref, "degen_const5", c5, c5, 7, note="constant 5")
    p, t = wl.randn_pair((1, 1, 9, 8, 7), 400)
    save_full(ref, "dr1_k3", p, t, 3, dr=1.0, note="smooth_dr=1")
    save_full(ref, "dr0p1_k5", p, t, 5, dr=0.1, note="smooth_dr=0.1")
    p, t = wl.randn_pair((1, 1, 12, 12, 12), 500)
    save_full(ref, "affine_k5", 2.0 * t + 1.0, t, 5, note="pred = 2*target + 1 (ncc saturates)")
    p, t = wl.randn_pair((1, 2, 16, 16, 16), 600, dtype=torch.bfloat16)
    save_full(ref, "bf16vals_k7", p, t, 7, note="bf16-representable values, fp32 reference")


def large_cases(ref):
    out = {}
    for name in ("mri", "bf16", "headline"):
        spec = wl.WORKLOADS[name]
        t0 = time.time()
        p, t = wl.make_inputs(name)
        loss, grad = run_ref(ref, p.float(), t.float(), spec["k"])
        out[name] = dict(loss=loss, pred=wl.checksum(p), target=wl.checksum(t), grad=wl.checksum(grad),
                         grad_l2=float(grad.double().norm()), k=spec["k"], shape=list(spec["shape"]))
        print(f"{name}: loss={loss:.9f} ({time.time() - t0:.1f}s)", flush=True)
        del p, t, grad
        np.savez(os.path.join(HERE, f"stats_{name}.npz"), **{
            key: np.asarray(val) for key, val in out[name].items()})


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--large", action="store_true")
    a = ap.parse_args()
    torch.set_num_threads(os.cpu_count())
    ref = load_reference()
    if a.large:
        large_cases(ref)
    else:
        small_cases(ref)
