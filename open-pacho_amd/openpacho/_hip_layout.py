"""Products of private 2-D transposes without materializing them (hip backend).

Counterpart of the reference's provider layout plans: ``prepare_layout_matmul``
(_opencl.py:260-285) and ``TransposedGemm`` (_matmul_layout.py:8-48), used for
"layout_matmul" plan steps (_compiler.py:103-156). Instead of a vendor BLAS
call with transpose flags, ``run`` issues one hp_gemm_layout, whose MFMA
kernels read a transposed operand in place (the slice loader that serves B
serves a transposed A and vice versa). A plan stores metadata and the backend
only; the operands stay dynamic, so a prepared call can be rebound.
"""

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _hip_lib as lib_

_FLOATS = (np.dtype("float32"), np.dtype("float64"))


@dataclass(frozen=True)
class HIPTransposedGemm:
    backend: object
    ashape: tuple
    bshape: tuple
    shape: tuple
    dtype: np.dtype
    transpose_a: bool
    transpose_b: bool

    def run(self, a, b):
        m, n = self.shape
        k = self.ashape[0] if self.transpose_a else self.ashape[1]
        out = self.backend.empty(self.shape, self.dtype)
        with self.backend._active():
            self.backend._call(
                "hp_gemm_layout",
                lib_.DTYPE_CODES[self.dtype],
                ctypes.c_void_p(a._data.ptr),
                ctypes.c_void_p(b._data.ptr),
                ctypes.c_void_p(out.ptr),
                m,
                n,
                k,
                int(self.transpose_a),
                int(self.transpose_b),
            )
        return out

    def explain(self):
        return {
            "provider": "hip",
            "transpose_a": self.transpose_a,
            "transpose_b": self.transpose_b,
            "stored_shapes": (self.ashape, self.bshape),
            "leading_dimensions": (self.ashape[1], self.bshape[1], self.shape[1]),
            # Operands, not distinct gathers: one private transpose may feed
            # both sides of a product.
            "transpose_operand_bytes": self.dtype.itemsize
            * sum(
                rows * columns
                for (rows, columns), transposed in ((self.ashape, self.transpose_a), (self.bshape, self.transpose_b))
                if transposed
            ),
        }


def prepare(backend, ashape, bshape, shape, dtype, *, transpose_a=False, transpose_b=False):
    """A layout plan, or None to keep the materialized transpose (_opencl.py:263-285)."""
    dtype = np.dtype(dtype)
    if dtype not in _FLOATS or len(ashape) != 2 or len(bshape) != 2 or not (transpose_a or transpose_b):
        return None
    left = tuple(ashape[::-1]) if transpose_a else tuple(ashape)
    right = tuple(bshape[::-1]) if transpose_b else tuple(bshape)
    if not all((*left, *right)):
        return None
    if left[1] != right[0] or tuple(shape) != (left[0], right[1]):
        return None
    return HIPTransposedGemm(
        backend, tuple(ashape), tuple(bshape), tuple(shape), dtype, bool(transpose_a), bool(transpose_b)
    )
