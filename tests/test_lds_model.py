"""The fused kernel's LDS accesses, checked on the host (tests/lds_model.cpp): bounds, write
collisions within a phase, arrays read and written in one phase, and that every read feeding a
used output reads what the producing stage wrote, for every kernel size and both adjoint layouts
(three fields for the pred gradient, five for both gradients), from the lane maps the kernel
itself uses (fused-lncc_amd/csrc/lncc_geometry.h).

This is the stand-in for the reference's compute-sanitizer workloads (tests/_sanitize*.py): GPU
address sanitizers are not available for LDS and ROCm has no LDS race checker. Each planted
mistake (a model-side perturbation of one lane map) must be reported, so the model is known to
see the kinds of error it is for."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "lds_model.cpp")
INC = os.path.join(ROOT, "fused-lncc_amd", "csrc")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = str(tmp_path_factory.mktemp("lds") / "lds_model")
    subprocess.run([cxx, "-std=c++17", "-O2", "-Wall", "-Werror", "-I", INC, SRC, "-o", exe], check=True)
    return exe


def test_kernel_lane_maps_pass(model):
    r = subprocess.run([model], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "all ok"
    # h = 1..4 with three adjoint fields and with five (both gradients)
    assert len([ln for ln in lines if ln.endswith(", ok")]) == 8
    assert len([ln for ln in lines if "5 adjoint fields" in ln]) == 4


@pytest.mark.parametrize("plant,kind", [(1, "used read of unwritten Zs"), (2, "Y window past the row read"),
                                        (3, "used read of unwritten GY"), (4, "read out of Zs")])
def test_planted_mistakes_are_reported(model, plant, kind):
    r = subprocess.run([model, str(plant)], capture_output=True, text=True)
    assert r.returncode == 1 and kind in r.stdout, r.stdout
