"""The C ABI from a non-Python host: include/fused_lncc.h compiles as strict C99 and as C++17, and a
C program links against the built library and gets the host-side answers (validation, workspace
size, error text) without touching a GPU. This is the binding surface a C, C++ or cgo caller uses.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "fused-lncc_amd", "fused_lncc")

C_SRC = r"""
#include <stdio.h>
#include <string.h>
#include "fused_lncc.h"

int main(void) {
    int ok = fl_validate(FL_F32, 7, 32, 128, 128, 128);
    int bad_k = fl_validate(FL_F32, 8, 32, 128, 128, 128);
    char msg[256];  /* the returned text lives until the next failing call on this thread */
    strncpy(msg, fl_last_error(), sizeof msg - 1);
    msg[sizeof msg - 1] = '\0';
    int bad_t = fl_validate(7, 7, 1, 8, 8, 8);
    size_t ws = fl_workspace_bytes(32, 128, 128, 128, 7);
    int null_rc = fl_lncc_loss_grad(NULL, NULL, FL_F32, 1, 8, 8, 8, 7, 1e-5f, NULL, NULL, NULL, 0, NULL);
    printf("%d %d %d %d %zu %d|%s\n", fl_version(), ok, bad_k, bad_t, ws, null_rc, msg);
    return !(ok == FL_OK && bad_k == FL_E_KSIZE && bad_t == FL_E_DTYPE && ws > 0 && ws % 8 == 0 &&
             null_rc == FL_E_NULL && strstr(msg, "kernel_size") != NULL);
}
"""


def _compiler(name):
    path = shutil.which(name)
    if path is None:
        pytest.skip(f"{name} not available")
    return path


def test_header_compiles_as_c99_and_cxx17(tmp_path):
    src = tmp_path / "inc.c"
    src.write_text('#include "fused_lncc.h"\nint main(void) { return fl_version() < 0; }\n')
    subprocess.run([_compiler("gcc"), "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                    f"-I{INC}", str(src)], check=True)
    cpp = tmp_path / "inc.cpp"
    cpp.write_text(src.read_text())
    subprocess.run([_compiler("g++"), "-std=c++17", "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                    f"-I{INC}", str(cpp)], check=True)


def test_c_program_links_and_calls_the_library(tmp_path):
    if not os.path.exists(os.path.join(LIBDIR, "libfused_lncc_hip.so")):
        pytest.skip("library not built")
    src = tmp_path / "client.c"
    src.write_text(C_SRC)
    exe = tmp_path / "client"
    subprocess.run([_compiler("gcc"), "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{INC}", str(src),
                    f"-L{LIBDIR}", "-lfused_lncc_hip", f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    head, msg = r.stdout.strip().split("|", 1)
    version, ok, bad_k, bad_t, ws, null_rc = map(int, head.split())
    assert version >= (0 << 16) | (1 << 8) and ok == 0 and bad_k == -2 and bad_t == -1 and null_rc == -4
    assert ws > 0 and "kernel_size" in msg
