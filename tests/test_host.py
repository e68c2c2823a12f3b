"""CPU-side checks of the C ABI and the Python boundary: no kernel is launched here.

* the built library loads and exports every symbol include/fused_lncc.h declares;
* fl_validate rejects what the reference rejects (fused_lncc/csrc/lncc3d.cu:123,128-129,158,
  255-260,281; fused_lncc/__init__.py:81-82) before any device work;
* the Python API raises the reference's exception types;
* the fake (meta) kernels give torch.compile the right dtypes, and the loss with its backward
  traces on fake tensors;
* the product package never imports the oracle, and refuses to run without the built library.
"""
import ast
import os
import re

import pytest
import torch

import fused_lncc
from fused_lncc import _lib, ext, fused_lncc_loss

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fused_lncc.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fl_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.fl_version() >= (0 << 16) | (1 << 8)


@pytest.mark.parametrize("dtype,k,shape,code", [
    (0, 7, (2, 8, 8, 8), _lib.FL_OK),
    (1, 3, (1, 1, 1, 1), _lib.FL_OK),
    (2, 7, (2, 8, 8, 8), _lib.FL_E_DTYPE),      # float64 / anything else
    (0, 11, (2, 8, 8, 8), _lib.FL_E_KSIZE),
    (0, 6, (2, 8, 8, 8), _lib.FL_E_KSIZE),
    (0, 1, (2, 8, 8, 8), _lib.FL_E_KSIZE),
    (0, 7, (0, 8, 8, 8), _lib.FL_E_SHAPE),
    (0, 7, (1, 8, 0, 8), _lib.FL_E_SHAPE),
    (0, 7, (1, 2, 1 << 16, 1 << 14), _lib.FL_E_SHAPE),   # one plane > 2 GiB
])
def test_validate(dtype, k, shape, code):
    lib = _lib.load()
    assert lib.fl_validate(dtype, k, *shape) == code
    if code != _lib.FL_OK:
        assert lib.fl_last_error().decode()


def test_errors_before_device_work():
    lib = _lib.load()
    # NULL pointers are refused on the host, with a message, and nothing is launched
    rc = lib.fl_lncc_loss_grad(None, None, 0, 1, 8, 8, 8, 7, 1e-5, None, None, None, 0, None)
    assert rc == _lib.FL_E_NULL and "NULL" in lib.fl_last_error().decode()
    rc = lib.fl_box3d(None, None, 1, 8, 8, 8, 4, None)
    assert rc == _lib.FL_E_KSIZE
    rc = lib.fl_scale_grad(None, 5, 10, None, None)
    assert rc == _lib.FL_E_DTYPE
    # a workspace that is too small is refused
    rc = lib.fl_lncc_loss_grad(8, 8, 0, 1, 8, 8, 8, 7, 1e-5, 8, None, 8, 0, None)
    assert rc == _lib.FL_E_WORKSPACE
    # the adjoint maps are all given or all omitted
    rc = lib.fl_lncc_maps(8, 8, 0, 1, 8, 8, 8, 7, 1e-5, 8, 8, None, 8, None)
    assert rc == _lib.FL_E_NULL and "all NULL" in lib.fl_last_error().decode()
    # both gradients: every pointer is required, the workspace is checked for every k, and the
    # shape before either
    for k in (3, 7, 9):
        rc = lib.fl_lncc_loss_grad_pt(8, 8, 0, 1, 8, 8, 8, k, 1e-5, 8, 8, None, 8, 64, None)
        assert rc == _lib.FL_E_NULL and "NULL" in lib.fl_last_error().decode()
        rc = lib.fl_lncc_loss_grad_pt(8, 8, 0, 1, 8, 8, 8, k, 1e-5, 8, 8, 8, 8, 0, None)
        assert rc == _lib.FL_E_WORKSPACE and "workspace needs" in lib.fl_last_error().decode()
    assert lib.fl_lncc_loss_grad_pt(8, 8, 0, 1, 0, 8, 8, 7, 1e-5, 8, 8, 8, 8, 64, None) == _lib.FL_E_SHAPE
    assert lib.fl_lncc_loss_grad_pt(8, 8, 2, 1, 8, 8, 8, 7, 1e-5, 8, 8, 8, 8, 64, None) == _lib.FL_E_DTYPE


def test_workspace_bytes():
    lib = _lib.load()
    n = lib.fl_workspace_bytes(32, 128, 128, 128, 7)
    assert n > 0 and n % 8 == 0
    assert lib.fl_workspace_bytes(32, 128, 128, 128, 8) == 0
    assert ext.workspace_bytes((1, 1, 1, 1), 3) == 8
    # a 30000 x 30000 plane is 1.8e9 B in bf16 (allowed) and 3.6e9 B in float32 (refused): the
    # workspace size does not depend on the dtype, the launch checks its own
    assert lib.fl_workspace_bytes(1, 8, 30000, 30000, 7) > 0
    assert lib.fl_validate(_lib.FL_BF16, 7, 1, 8, 30000, 30000) == _lib.FL_OK
    assert lib.fl_validate(_lib.FL_F32, 7, 1, 8, 30000, 30000) == _lib.FL_E_SHAPE


def test_lds_bytes():
    lib = _lib.load()
    sizes = [lib.fl_lds_bytes(k, _lib.FL_F32) for k in (3, 5, 7, 9)]
    # the largest of the kernels: at k = 7 the plane-marching kernel with both gradients, whose
    # 161184 B the profiler reports as its 512-byte-granular allocation of 161280 B; every size
    # at least the small-volume kernel's eight 16^3 float fields and 16 float64 partials
    # (131200 B) and within the CU's 160 KiB
    assert sizes[2] == 161184 and -(-sizes[2] // 512) * 512 == 161280
    assert all(8 * 16 ** 3 * 4 + 16 * 8 <= b <= 160 * 1024 for b in sizes)
    assert lib.fl_lds_bytes(7, _lib.FL_BF16) == sizes[2]
    assert lib.fl_lds_bytes(8, _lib.FL_F32) == 0 and lib.fl_lds_bytes(7, 5) == 0


def test_shape_limits_without_overflow():
    lib = _lib.load()
    # H*W*4 would overflow int64: refused by the per-dimension bound first
    assert lib.fl_validate(_lib.FL_F32, 7, 1, 1, 2 ** 40, 2 ** 40) == _lib.FL_E_SHAPE
    assert "2 GiB" in lib.fl_last_error().decode()
    # B x tiles x D would overflow int64
    assert lib.fl_validate(_lib.FL_F32, 7, 2 ** 62, 2 ** 30, 64, 64) == _lib.FL_E_SHAPE
    assert "too many" in lib.fl_last_error().decode()
    # B x tiles alone can exceed int64: bf16 planes of 1 x 1073740448 columns hold 33554389 tiles
    # of 32 columns, and 549756518401 (< 2^40) such volumes make 2^64 + 3260373 tiles, which a plain
    # int64 product wraps to a small positive count that would pass the grid limit
    assert lib.fl_validate(_lib.FL_BF16, 7, 549756518401, 1, 1, 1073740448) == _lib.FL_E_SHAPE
    assert "too many" in lib.fl_last_error().decode()
    assert lib.fl_workspace_bytes(549756518401, 1, 1, 1073740448, 7) == 0
    # the box kernels' 16-column tiles: 67108778 per such plane of 1073740448 / 2 columns (fp32)
    assert lib.fl_box3d(8, 8, 549756518401, 1, 1, 536870224, 7, None) == _lib.FL_E_SHAPE
    # the debug box-sum path has 16 x 16 tiles: a grid of 2^26 x 8 x 8 workgroups is refused on the
    # host (nothing is launched)
    assert lib.fl_box3d(8, 8, 2 ** 26, 1, 128, 128, 7, None) == _lib.FL_E_SHAPE
    assert "too many" in lib.fl_last_error().decode()


def test_grid_in_lanes_fits_32_bits():
    """A launch's grid counted in lanes must fit in 32 bits: 1024 lanes per workgroup of the fused
    kernel (one workgroup per 32 x 32 tile and volume at least), 256 per box-kernel workgroup (one
    per 16 x 16 tile). The boundary is exact on both sides, and the error comes from the host."""
    lib = _lib.load()
    # 1024 x 1024 planes: 32 x 32 = 1024 fused tiles per volume; 4096 volumes = 2^22 tiles = 2^32 lanes
    assert lib.fl_validate(_lib.FL_F32, 7, 4095, 1, 1024, 1024) == _lib.FL_OK
    assert lib.fl_validate(_lib.FL_F32, 7, 4096, 1, 1024, 1024) == _lib.FL_E_SHAPE
    assert "too many" in lib.fl_last_error().decode()
    assert lib.fl_workspace_bytes(4096, 1, 1024, 1024, 7) == 0
    rc = lib.fl_lncc_loss_grad(8, 8, _lib.FL_F32, 4096, 1, 1024, 1024, 7, 1e-5, 8, 8, 8, 1 << 40, None)
    assert rc == _lib.FL_E_SHAPE
    # box kernel: 64 x 64 = 4096 tiles of 16 x 16 per 1024^2 plane; 2^12 volumes = 2^24 tiles = 2^32 lanes
    assert lib.fl_box3d(8, 8, 4096, 1, 1024, 1024, 7, None) == _lib.FL_E_SHAPE
    assert "too many" in lib.fl_last_error().decode()
    assert lib.fl_lncc_backward(8, 8, 8, 8, 8, _lib.FL_F32, 4096, 1, 1024, 1024, 7, 1.0, 8, None) == _lib.FL_E_SHAPE


def test_no_alloc_entry_point_limits():
    """The allocation-free entry point refuses, on the host and with a clear message, a launch
    larger than its static scratch (65536 workgroups), and a missing output pointer."""
    lib = _lib.load()
    # 300 volumes of 512 x 512 planes: 300 x 256 tiles of 32 x 32 > 65536 workgroups
    rc = lib.fl_lncc_loss_grad_noalloc(8, 8, _lib.FL_F32, 300, 4, 512, 512, 7, 1e-5, 8, 8, None)
    assert rc == _lib.FL_E_WORKSPACE and "scratch holds 65536" in lib.fl_last_error().decode()
    rc = lib.fl_lncc_loss_grad_noalloc(8, 8, _lib.FL_F32, 1, 4, 8, 8, 7, 1e-5, None, 8, None)
    assert rc == _lib.FL_E_NULL
    assert lib.fl_lncc_loss_grad_noalloc(8, 8, _lib.FL_F32, 1, 4, 8, 8, 8, 1e-5, 8, 8, None) == _lib.FL_E_KSIZE


def test_reference_module_name():
    """`import fused_lncc_cuda` gives the reference's three extension entry points
    (fused_lncc/csrc/lncc3d.cu:346-350), the same functions as fused_lncc.ext's."""
    import fused_lncc_cuda
    for name in ("lncc_forward", "lncc_backward", "box3d_sep_forward"):
        assert getattr(fused_lncc_cuda, name) is getattr(ext, name)


def test_python_api_errors():
    p = torch.randn(1, 1, 8, 8, 8)
    with pytest.raises(AssertionError):
        fused_lncc_loss(p, p, 6)                      # even k
    with pytest.raises(AssertionError):
        fused_lncc_loss(p, p[:, :, :4], 7)            # shape mismatch
    with pytest.raises(AssertionError):
        fused_lncc_loss(p[0], p[0], 7)                # not 5-D
    with pytest.raises(RuntimeError, match="float32 or bfloat16"):
        fused_lncc_loss(p.double(), p.double(), 7)    # float64
    with pytest.raises(RuntimeError, match="GPU tensor"):
        fused_lncc_loss(p, p, 7)                      # CPU tensors: refused, no CPU fallback
    with pytest.raises(RuntimeError, match="kernel_size"):
        _lib.check(_lib.load().fl_validate(0, 11, 1, 8, 8, 8))


def test_fake_kernels_dtypes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        for dt in (torch.float32, torch.bfloat16):
            pf = torch.empty(6, 24, 20, 28, dtype=dt, device="cuda" if torch.cuda.is_available() else "cpu")
            loss, grad = torch.ops.fused_lncc.loss_grad(pf, pf, 7, 1e-5, True)
            assert loss.dtype == torch.float32 and loss.shape == ()
            assert grad.dtype == dt and grad.shape == pf.shape
            outs = torch.ops.fused_lncc.forward(pf, pf, 7, 1e-5)
            assert len(outs) == 4 and all(o.dtype == torch.float32 for o in outs)
            g = torch.ops.fused_lncc.backward(outs[1], outs[2], outs[3], pf, pf, 7, 1.0)
            assert g.dtype == dt


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_fake_trace_of_loss_and_backward(dt):
    """The autograd function traces end to end on fake tensors (what torch.compile does before any
    kernel runs): a float32 0-d loss, a gradient in the pred dtype, and the custom ops in the graph."""
    from torch.fx.experimental.proxy_tensor import make_fx

    def step(p, t):
        loss = fused_lncc_loss(p, t, 5)
        (g,) = torch.autograd.grad(2.0 * loss, p)
        return loss, g

    p = torch.randn(1, 2, 8, 9, 10, dtype=dt, requires_grad=True)
    t = torch.randn(1, 2, 8, 9, 10, dtype=dt)
    gm = make_fx(step, tracing_mode="fake")(p, t)
    ops = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
    assert any("fused_lncc.loss_grad" in o for o in ops), ops
    assert any("fused_lncc.scale_grad_" in o for o in ops), ops
    outs = [n for n in gm.graph.nodes if n.op == "output"][0].args[0]
    loss_meta, g_meta = outs[0].meta["val"], outs[1].meta["val"]
    assert loss_meta.dtype == torch.float32 and loss_meta.shape == ()
    assert g_meta.dtype == dt and g_meta.shape == p.shape


def test_fake_trace_with_target_grad():
    """With target_grad=True the trace holds one call of the both-gradients op and both
    gradients come out in the input dtype and shape."""
    from torch.fx.experimental.proxy_tensor import make_fx

    def step(p, t):
        loss = fused_lncc_loss(p, t, 7, target_grad=True)
        gp, gt = torch.autograd.grad(loss, (p, t))
        return loss, gp, gt

    p = torch.randn(1, 2, 8, 9, 10, dtype=torch.bfloat16, requires_grad=True)
    t = torch.randn(1, 2, 8, 9, 10, dtype=torch.bfloat16, requires_grad=True)
    gm = make_fx(step, tracing_mode="fake")(p, t)
    calls = [str(n.target) for n in gm.graph.nodes if n.op == "call_function" and "fused_lncc.loss_grad" in str(n.target)]
    assert len(calls) == 1 and "loss_grad_pt" in calls[0], calls
    outs = [n for n in gm.graph.nodes if n.op == "output"][0].args[0]
    for o in outs[1:]:
        assert o.meta["val"].dtype == torch.bfloat16 and o.meta["val"].shape == p.shape


def test_traced_detection():
    """Eager calls on plain tensors take the direct library path; under a dispatch-mode trace
    (real-mode make_fx, a fake-tensor mode) or for a fake-tensor input the custom ops stand in."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.proxy_tensor import make_fx

    x = torch.ones(2, 3)
    assert not fused_lncc._traced(x)
    assert not fused_lncc._traced(torch.nn.Parameter(x))
    seen = []

    def f(a):
        seen.append(fused_lncc._traced(a))
        return a * 2

    make_fx(f)(x)
    make_fx(f, tracing_mode="fake")(x)
    assert seen == [True, True]
    mode = FakeTensorMode()
    fx = mode.from_tensor(x)
    assert fused_lncc._traced(fx)
    with mode:
        assert fused_lncc._traced(fx)


def test_product_never_imports_the_oracle():
    pkg = os.path.dirname(fused_lncc.__file__)
    for fn in os.listdir(pkg):
        if fn.endswith(".py"):
            tree = ast.parse(open(os.path.join(pkg, fn)).read())
            for node in ast.walk(tree):
                if isinstance(node, (ast.Import, ast.ImportFrom)):
                    names = [a.name for a in node.names] + [getattr(node, "module", None) or ""]
                    assert not any("oracle" in n for n in names), fn


def test_missing_library_fails_loudly():
    """Without the built library the package refuses to run (no CPU fallback): a fresh
    interpreter whose loader points at a path that does not exist gets an ImportError that says
    how to build, on the first call that needs the library."""
    import subprocess
    import sys
    code = ("import fused_lncc._lib as L\n"
            "L.LIB_PATH = '/nonexistent/libfused_lncc_hip.so'\n"
            "L._lib = None\n"
            "try:\n"
            "    L.load()\n"
            "except ImportError as e:\n"
            "    print('ImportError:', e)\n")
    env = dict(os.environ, PYTHONPATH=os.path.join(ROOT, "fused-lncc_amd"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert out.returncode == 0, out.stderr
    assert "ImportError:" in out.stdout and "no CPU fallback" in out.stdout


def _package_copy(tmp_path):
    """The package, its build script and HIP sources, and the C-ABI header they include, copied
    without any built file."""
    import shutil
    src = os.path.join(ROOT, "fused-lncc_amd")
    dst = tmp_path / "fused-lncc_amd"
    shutil.copytree(src, dst, ignore=shutil.ignore_patterns("_build", "*.so", "*.so.tmp", "*.lock", "__pycache__"))
    shutil.copytree(os.path.join(ROOT, "include"), tmp_path / "include")
    return dst


def test_first_use_builds_missing_library(tmp_path):
    """A package without its library builds it on the first call that needs it (as the reference
    compiles its extension on first import), and the result exports every symbol of the C ABI;
    with FUSED_LNCC_NO_BUILD=1 the same call fails loudly instead."""
    import subprocess
    import sys
    pkg = _package_copy(tmp_path)
    code = ("import fused_lncc._lib as L\n"
            "lib = L.load()\n"
            "print('loaded', L.LIB_PATH, all(hasattr(lib, n) for n in L.SIGNATURES))\n")
    env = dict(os.environ, PYTHONPATH=str(pkg))
    env.pop("FUSED_LNCC_NO_BUILD", None)
    off = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         env=dict(env, FUSED_LNCC_NO_BUILD="1"), timeout=300)
    assert off.returncode != 0 and "no CPU fallback" in off.stderr
    assert not (pkg / "fused_lncc" / "libfused_lncc_hip.so").exists()
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=900)
    assert out.returncode == 0, out.stderr[-3000:]
    assert "building it" in out.stderr
    assert out.stdout.strip() == f"loaded {pkg / 'fused_lncc' / 'libfused_lncc_hip.so'} True"


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with status 2 and says so, before touching a
    device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2 and "one GPU only" in r.stderr, (r.returncode, r.stderr)
