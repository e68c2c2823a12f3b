"""The C ABI end to end from a plain C99 host on the GPU, the way a C, C++, cgo or JNI caller uses it:
the program allocates device buffers with the HIP runtime, copies the inputs up, calls
fl_lncc_loss_grad (and fl_lncc_loss_grad_pt for both gradients) on the default stream, copies the
loss and the gradients back, and the test compares them with the oracle. No Python tensor or
torch stream is involved on the device side."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "fused-lncc_amd", "fused_lncc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

C_SRC = r"""
#include <stdio.h>
#include <stdlib.h>
#include <hip/hip_runtime_api.h>
#include "fused_lncc.h"

static int read_all(const char* path, void* buf, size_t n) {
    FILE* f = fopen(path, "rb");
    if (!f) return 1;
    size_t got = fread(buf, 1, n, f);
    fclose(f);
    return got != n;
}

static int write_all(const char* path, const void* buf, size_t n) {
    FILE* f = fopen(path, "wb");
    if (!f) return 1;
    size_t put = fwrite(buf, 1, n, f);
    fclose(f);
    return put != n;
}

#define HIP_OK(x) do { if ((x) != hipSuccess) { fprintf(stderr, "HIP error at %d\n", __LINE__); return 2; } } while (0)

/* usage: client B D H W k dir  (dir holds p.bin, t.bin; receives gp.bin, gp2.bin, gt.bin) */
int main(int argc, char** argv) {
    if (argc != 7) return 1;
    const long long B = atoll(argv[1]), D = atoll(argv[2]), H = atoll(argv[3]), W = atoll(argv[4]);
    const int k = atoi(argv[5]);
    const char* dir = argv[6];
    const size_t n = (size_t)(B * D * H * W), bytes = n * sizeof(float);
    char path[4096];
    float* hp = malloc(bytes); float* ht = malloc(bytes); float* hg = malloc(bytes);
    if (!hp || !ht || !hg) return 1;
    snprintf(path, sizeof path, "%s/p.bin", dir); if (read_all(path, hp, bytes)) return 1;
    snprintf(path, sizeof path, "%s/t.bin", dir); if (read_all(path, ht, bytes)) return 1;

    void *dp, *dt, *dg, *dg2, *dws; float* dloss;
    const size_t ws = fl_workspace_bytes(B, D, H, W, k);
    HIP_OK(hipMalloc(&dp, bytes)); HIP_OK(hipMalloc(&dt, bytes)); HIP_OK(hipMalloc(&dg, bytes));
    HIP_OK(hipMalloc(&dg2, bytes)); HIP_OK(hipMalloc(&dws, ws)); HIP_OK(hipMalloc((void**)&dloss, sizeof(float)));
    HIP_OK(hipMemcpy(dp, hp, bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dt, ht, bytes, hipMemcpyHostToDevice));

    float loss = 0.f, loss2 = 0.f;
    int rc = fl_lncc_loss_grad(dp, dt, FL_F32, B, D, H, W, k, 1e-5f, dloss, dg, dws, ws, NULL);
    if (rc != FL_OK) { fprintf(stderr, "%s\n", fl_last_error()); return 3; }
    HIP_OK(hipMemcpy(&loss, dloss, sizeof(float), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hg, dg, bytes, hipMemcpyDeviceToHost));
    snprintf(path, sizeof path, "%s/gp.bin", dir); if (write_all(path, hg, bytes)) return 1;

    rc = fl_lncc_loss_grad_pt(dp, dt, FL_F32, B, D, H, W, k, 1e-5f, dloss, dg, dg2, dws, ws, NULL);
    if (rc != FL_OK) { fprintf(stderr, "%s\n", fl_last_error()); return 3; }
    HIP_OK(hipMemcpy(&loss2, dloss, sizeof(float), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hg, dg, bytes, hipMemcpyDeviceToHost));
    snprintf(path, sizeof path, "%s/gp2.bin", dir); if (write_all(path, hg, bytes)) return 1;
    HIP_OK(hipMemcpy(hg, dg2, bytes, hipMemcpyDeviceToHost));
    snprintf(path, sizeof path, "%s/gt.bin", dir); if (write_all(path, hg, bytes)) return 1;

    /* a workspace one double short is refused before any launch */
    rc = fl_lncc_loss_grad(dp, dt, FL_F32, B, D, H, W, k, 1e-5f, dloss, dg, dws, ws - 8, NULL);
    printf("%.9g %.9g %d\n", loss, loss2, rc);
    hipFree(dp); hipFree(dt); hipFree(dg); hipFree(dg2); hipFree(dws); hipFree(dloss);
    free(hp); free(ht); free(hg);
    return 0;
}
"""


@pytest.fixture(scope="module")
def client(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    if not os.path.exists(os.path.join(LIBDIR, "libfused_lncc_hip.so")):
        pytest.fail("library not built: run `python fused-lncc_amd/build.py`")
    d = tmp_path_factory.mktemp("cclient")
    src = d / "client.c"
    src.write_text(C_SRC)
    exe = d / "client"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{INC}",
                    f"-I{ROCM}/include", str(src), f"-L{LIBDIR}", "-lfused_lncc_hip", f"-L{ROCM}/lib", "-lamdhip64",
                    f"-Wl,-rpath,{LIBDIR}", f"-Wl,-rpath,{ROCM}/lib", "-o", str(exe)], check=True)
    return str(exe)


def _cos_rel(g, r):
    g, r = g.ravel().astype(np.float64), r.ravel().astype(np.float64)
    return float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r))), float(np.linalg.norm(g - r) / np.linalg.norm(r))


@pytest.mark.parametrize("shape,k", [((2, 20, 37, 45), 7), ((1, 9, 64, 33), 3), ((3, 12, 30, 40), 9)])
def test_c_host_end_to_end(client, tmp_path, shape, k):
    print(f"C host: shape={shape} k={k}", flush=True)
    rng = np.random.default_rng(sum(shape) + k)
    t = rng.standard_normal(shape).astype(np.float32)
    p = (0.8 * t + 0.6 * rng.standard_normal(shape)).astype(np.float32)
    p.tofile(tmp_path / "p.bin")
    t.tofile(tmp_path / "t.bin")
    r = subprocess.run([client, *map(str, shape), str(k), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    loss, loss2, short_rc = r.stdout.split()
    loss, loss2 = float(loss), float(loss2)
    gp = np.fromfile(tmp_path / "gp.bin", np.float32).reshape(shape)
    gp2 = np.fromfile(tmp_path / "gp2.bin", np.float32).reshape(shape)
    gt = np.fromfile(tmp_path / "gt.bin", np.float32).reshape(shape)
    lr, gr = O.lncc(p, t, k)
    _, grt = O.lncc(t, p, k)   # the loss is symmetric in its inputs
    assert abs(loss - lr) <= 1e-5 * abs(lr) and abs(loss2 - lr) <= 1e-5 * abs(lr)
    for got, ref in ((gp, gr), (gp2, gr), (gt, grt)):
        cos, rel = _cos_rel(got, np.asarray(ref))
        assert cos > 0.9999 and rel < 1e-3, (cos, rel)
    assert int(short_rc) == -5   # FL_E_WORKSPACE
