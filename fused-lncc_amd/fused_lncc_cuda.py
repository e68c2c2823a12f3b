"""The reference's extension module name, for callers that import it directly.

The reference builds its CUDA kernels as the pybind11 module ``fused_lncc_cuda`` with three entry
points (fused_lncc/csrc/lncc3d.cu:346-350), which its CI test imports by that name
(tests/test_pytest.py:42). This module exposes the same three names, with the same arguments and
outputs, over this package's HIP library (``fused_lncc.ext``):

* ``lncc_forward(P, T, kernel_size, dr) -> [ncc, A, Bc, Cc]``
* ``lncc_backward(A, Bc, Cc, P, T, kernel_size, scale) -> grad``
* ``box3d_sep_forward(x, kernel_size) -> box-sum``
"""
from fused_lncc.ext import box3d_sep_forward, lncc_backward, lncc_forward

__all__ = ["lncc_forward", "lncc_backward", "box3d_sep_forward"]
