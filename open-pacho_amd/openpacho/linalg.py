"""Euclidean vector and Frobenius matrix norms (reference linalg.py:8-38).

Other norm orders are deliberately unsupported. Non-floating inputs are
promoted to float64 before the backend's scaled reduction.
"""

import numpy as np

from . import _array as xp


def _accepted_order(ord, ndim, axis):
    if ord is None:
        return True
    matrix = (ndim == 2 and axis is None) or (isinstance(axis, tuple) and len(axis) == 2)
    vector = (ndim == 1 and axis is None) or isinstance(axis, (int, np.integer))
    return (ord == "fro" and matrix) or (ord == 2 and vector)


@xp._implements(np.linalg.norm)
def norm(x, ord=None, axis=None, keepdims=False):
    x = xp.asarray(x)
    if isinstance(axis, tuple) and len(axis) not in (1, 2):
        raise ValueError("norm requires one vector axis or two matrix axes")
    if x.ndim == 0 and axis is not None:
        raise ValueError("axis out of bounds for scalar norm")
    if not _accepted_order(ord, x.ndim, axis):
        raise NotImplementedError("Only Euclidean vector and Frobenius matrix norms are supported")
    if x.dtype.kind != "f":
        x = x.astype(np.float64)
    axes = xp._axes(axis, x.ndim)
    shape = xp._reduced_shape(x.shape, axes, keepdims)
    data = x._backend.norm(x, axes, keepdims, x.dtype)
    return xp.ndarray._wrap(data, shape, x.dtype, x._backend)

