"""ctypes binding of libfused_lncc_hip.so (C ABI in include/fused_lncc.h).

Loading fails loudly when the library has not been built: there is no CPU fallback.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfused_lncc_hip.so")

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


def load():
    """Load the library once (the HIP runtime it links is the one torch already loaded)."""
    global _lib
    if _lib is None:
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
