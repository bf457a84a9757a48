"""Fused GEMV residual ``b - A @ x`` for compiled plans on the hip backend.

Counterpart of the reference's custom-provider epilogue (_gemv.py:10-75,
``residual_matvec_data``), reached from "residual_matvec" plan steps
(_compiler.py:157-176, executed at :306-307). Contract kept from the
reference: the matrix product is rounded in the array dtype before the
subtraction, so the result equals the eager ``b - a @ x`` bit for bit (here
because hp_gemv_residual runs hp_gemv's own reduction and only replaces its
store); no intermediate is downloaded; the output is a new buffer; zero rows
give an empty result and zero columns a copy of ``b``. Errors follow the
reference: ValueError for operands outside the contract, NotImplementedError
when a vendor BLAS provider owns matrix products.
"""

import ctypes

import numpy as np

from . import _hip_lib as lib_

_FLOATS = (np.dtype("float32"), np.dtype("float64"))


def check_residual(backend, a, x, b):
    """Validate (matrix, vector, rhs) for the residual; mirrors _gemv.py:11-22."""
    if a.ndim != 2 or x.ndim != 1 or b.ndim != 1:
        raise ValueError("Residual GEMV requires a matrix and two vectors")
    rows, columns = a.shape
    if x.shape != (columns,) or b.shape != (rows,):
        raise ValueError("Residual GEMV dimensions do not match")
    if a.dtype != x.dtype or a.dtype != b.dtype or a.dtype not in _FLOATS:
        raise ValueError("Residual GEMV requires matching float32/float64 dtypes")
    if any(value._backend is not backend for value in (a, x, b)):
        raise ValueError("Residual GEMV inputs must belong to the same backend")
    if getattr(backend, "blas", "custom") not in (None, "custom"):
        raise NotImplementedError("Residual GEMV requires the custom hip provider")


def residual_matvec_data(backend, a, x, b):
    """Storage of ``b - a @ x`` computed by one hp_gemv_residual launch."""
    check_residual(backend, a, x, b)
    rows, columns = a.shape
    out = backend.empty((rows,), a.dtype)
    if rows:
        with backend._active():
            backend._call(
                "hp_gemv_residual",
                lib_.DTYPE_CODES[a.dtype],
                *(ctypes.c_void_p(v._data.ptr) for v in (a, x, b)),
                ctypes.c_void_p(out.ptr),
                rows,
                columns,
            )
    return out
