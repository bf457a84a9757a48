"""Extrema with the library's NaN and signed-zero contract, on the host.

Contract (reference _reductions.py:1-6, :149-163): NaN propagates; when the
extreme value is zero, min returns -0 if any reduced zero is negative and max
returns +0 if any reduced zero is positive. The hip backend implements the
same rule in its reduction kernels.
"""

import numpy as np


def numpy_extreme(value, axes, keepdims, operation):
    if operation not in ("min", "max"):
        raise ValueError(f"Unknown extreme reduction operation: {operation}")
    reducer = np.min if operation == "min" else np.max
    result = np.asarray(reducer(value, axis=axes, keepdims=keepdims))
    if value.dtype.kind == "f" and np.any(result == 0):
        zeros = value == 0
        negative = np.signbit(value)
        if operation == "min":
            want_negative = np.any(zeros & negative, axis=axes, keepdims=keepdims)
        else:
            want_negative = ~np.any(zeros & ~negative, axis=axes, keepdims=keepdims)
        signed = np.where(want_negative, -0.0, 0.0).astype(value.dtype)
        result = np.where(result == 0, signed, result)
    return np.asarray(result, dtype=value.dtype).reshape(-1)
