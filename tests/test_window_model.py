"""The window sums of the fused kernel (fused-lncc_amd/csrc/lncc_window.h), checked on the host by
tests/window_model.cpp: exact on integer data, exactly zero on zero windows and exactly K*c on
windows of one constant inside random data, within the direct-sum error bound everywhere, for the
x/y segment lengths and the D-march (with zero and constant slabs after signal) of every k, with
each split of the previous block's suffix kept as a partial sum. These are the properties of the
reference's direct k-tap sums (fused_lncc/csrc/lncc3d.cu:57-92) that the kernel's sums must share.
Planted mistakes (running sums along D, a dropped term, a damaged suffix chain) must be reported."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "window_model.cpp")
INC = os.path.join(ROOT, "fused-lncc_amd", "csrc")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = str(tmp_path_factory.mktemp("win") / "window_model")
    # -ffp-contract=off: fused multiply-adds only where the code asks for them, as on the GPU
    subprocess.run([cxx, "-std=c++17", "-O2", "-Wall", "-Werror", "-ffp-contract=off", "-I", INC, SRC, "-o", exe],
                   check=True)
    return exe


def test_window_sums_are_window_local(model):
    r = subprocess.run([model], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "all ok"
    # 13 segment checks, and the march for every k = 3..9 and every chain split M = 0..k-1
    assert len([ln for ln in lines if ln.endswith(": ok")]) == 13 + 3 + 5 + 7 + 9


@pytest.mark.parametrize("plant,what", [(1, "march K=7 chain M=0: FAILED"), (2, "box_sums h=3 S=20 (x): FAILED"),
                                        (3, "march K=7 chain M=4: FAILED")])
def test_planted_mistakes_are_reported(model, plant, what):
    r = subprocess.run([model, str(plant)], capture_output=True, text=True)
    assert r.returncode == 1 and what in r.stdout, r.stdout
