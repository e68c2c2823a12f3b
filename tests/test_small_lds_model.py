"""The small-volume kernel's LDS accesses, checked on the host (tests/small_lds_model.cpp) from the
index functions the kernel itself uses (fused-lncc_amd/csrc/lncc_geometry.h): a one-to-one layout,
no bank conflicts in any access instruction of any phase, line reads inside the volume's 16
positions except those the lane quarter's code class skips, no LDS float read and written between
two barriers, and every read finding what an earlier phase wrote. Planted mistakes (unrotated
rows, a wrong code class, the last buffer aliased onto the one being read) must be reported."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "small_lds_model.cpp")
INC = os.path.join(ROOT, "fused-lncc_amd", "csrc")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = str(tmp_path_factory.mktemp("slds") / "small_lds_model")
    subprocess.run([cxx, "-std=c++17", "-O2", "-Wall", "-Werror", "-I", INC, SRC, "-o", exe], check=True)
    return exe


def test_small_kernel_lds_accesses(model):
    r = subprocess.run([model], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "all ok" and len([ln for ln in lines if ln.endswith(": ok")]) == 4


@pytest.mark.parametrize("plant,kind", [(1, "lanes on bank"), (2, "quarter 0 reads position -1"),
                                        (3, "reads and writes LDS float")])
def test_planted_mistakes_are_reported(model, plant, kind):
    r = subprocess.run([model, str(plant)], capture_output=True, text=True)
    assert r.returncode == 1 and kind in r.stdout, r.stdout
