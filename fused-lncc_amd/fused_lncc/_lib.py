"""ctypes binding of libfused_lncc_hip.so (C ABI in include/fused_lncc.h).

On first use a missing library is built from the package's HIP sources (hipcc, gfx950), as the
reference compiles its extension on first import (fused_lncc/__init__.py:10-19); set
FUSED_LNCC_NO_BUILD=1 to turn that off. Loading fails loudly when the library is neither built
nor buildable: there is no CPU fallback.
"""
import ctypes
import os
import subprocess
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfused_lncc_hip.so")
_DEFAULT_LIB = LIB_PATH
_BUILD_SCRIPT = os.path.join(os.path.dirname(_HERE), "build.py")

FL_F32 = 0
FL_BF16 = 1
FL_OK = 0
FL_E_DTYPE = -1
FL_E_KSIZE = -2
FL_E_SHAPE = -3
FL_E_NULL = -4
FL_E_WORKSPACE = -5
FL_E_DEVICE = -6

# symbol -> (restype, argtypes); every symbol declared in include/fused_lncc.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_size_t
SIGNATURES = {
    "fl_version": (_I, []),
    "fl_last_error": (ctypes.c_char_p, []),
    "fl_validate": (_I, [_I, _I, _L, _L, _L, _L]),
    "fl_workspace_bytes": (_S, [_L, _L, _L, _L, _I]),
    "fl_lds_bytes": (_S, [_I, _I]),
    "fl_lncc_loss_grad": (_I, [_P, _P, _I, _L, _L, _L, _L, _I, _F, _P, _P, _P, _S, _P]),
    "fl_lncc_fused_partials": (_I, [_P, _P, _I, _L, _L, _L, _L, _I, _F, _P, _P, _S, _P]),
    "fl_lncc_loss_grad_noalloc": (_I, [_P, _P, _I, _L, _L, _L, _L, _I, _F, _P, _P, _P]),
    "fl_lncc_loss_grad_pt": (_I, [_P, _P, _I, _L, _L, _L, _L, _I, _F, _P, _P, _P, _P, _S, _P]),
    "fl_lncc_finalize": (_I, [_P, _L, _L, _L, _L, _I, _P, _P]),
    "fl_scale_grad": (_I, [_P, _I, _L, _P, _P]),
    "fl_lncc_maps": (_I, [_P, _P, _I, _L, _L, _L, _L, _I, _F, _P, _P, _P, _P, _P]),
    "fl_lncc_backward": (_I, [_P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _I, _F, _P, _P]),
    "fl_box3d": (_I, [_P, _P, _L, _L, _L, _L, _I, _P]),
    "fl_test_set_dchunk": (_I, [_I]),
}

_lib = None


class FusedLNCCError(RuntimeError):
    """A C-ABI call returned an error code; the message comes from fl_last_error()."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


def _build_missing_library():
    """Build the in-package library with build.py, once per machine: concurrent first uses wait
    on a lock file, and the one that finds the library built on waking does nothing. Raises
    ImportError with the compiler's messages when the build fails."""
    import fcntl
    try:
        lock = open(LIB_PATH + ".lock", "w")
    except OSError as e:   # a read-only install: nothing can be built here
        raise ImportError(f"fused_lncc: {LIB_PATH} is not built and cannot be built in place ({e}); run "
                          "`python fused-lncc_amd/build.py` where the package is writable. There is no CPU "
                          "fallback.") from e
    with lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if os.path.exists(LIB_PATH):
            return
        print(f"fused_lncc: {LIB_PATH} is missing; building it (hipcc, gfx950) ...", file=sys.stderr, flush=True)
        r = subprocess.run([sys.executable, _BUILD_SCRIPT], capture_output=True, text=True)
        if r.returncode != 0 or not os.path.exists(LIB_PATH):
            tail = "\n".join((r.stdout + r.stderr).strip().splitlines()[-20:])
            raise ImportError(f"fused_lncc: building {LIB_PATH} failed:\n{tail}\nThere is no CPU fallback.")


def load():
    """Load the library once (the HIP runtime it links is the one torch already loaded), building
    it first when it is missing (module docstring)."""
    global _lib
    if _lib is None:
        if (not os.path.exists(LIB_PATH) and LIB_PATH == _DEFAULT_LIB and os.path.exists(_BUILD_SCRIPT)
                and os.environ.get("FUSED_LNCC_NO_BUILD") != "1"):
            _build_missing_library()
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"fused_lncc: {LIB_PATH} is not built; run `python fused-lncc_amd/build.py` "
                "(hipcc, gfx950). There is no CPU fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class dchunk:
    """Test hook: launches on this thread inside the block split D into chunks of `planes` output
    planes (clamped to D); the launch planner decides again on exit."""

    def __init__(self, planes):
        self.planes = int(planes)

    def __enter__(self):
        check(load().fl_test_set_dchunk(self.planes))
        return self

    def __exit__(self, *exc):
        load().fl_test_set_dchunk(0)
        return False


def check(rc):
    if rc != FL_OK:
        msg = load().fl_last_error().decode(errors="replace")
        raise FusedLNCCError(rc, msg)
