"""Host (NumPy backend) Euclidean norm with two-pass max scaling.

Semantics (reference _norm.py:39-52): scale = max|x| over the reduced axes;
total = sum((x / scale)^2) in the requested dtype, with 0 where scale == 0;
result = scale * sqrt(total), and an infinite scale gives inf (a NaN scale
stays NaN). Empty reductions give 0.
"""

import numpy as np


def two_pass_norm(value, axes, dtype):
    dtype = np.dtype(dtype)
    outer = int(np.prod([d for i, d in enumerate(value.shape) if i not in axes], dtype=np.int64))
    reduced = int(np.prod([value.shape[i] for i in axes], dtype=np.int64))
    if not outer or not reduced:
        return np.zeros(outer, dtype=dtype)
    scale = np.max(np.abs(value), axis=axes, keepdims=True)
    with np.errstate(all="ignore"):
        ratio = np.zeros_like(value)
        np.divide(value, scale, out=ratio, where=scale != 0)
        total = np.sum(ratio * ratio, axis=axes, keepdims=True, dtype=dtype)
        result = scale * np.sqrt(total)
    result = np.where(np.isinf(scale), scale, result)
    return np.asarray(result, dtype=dtype).reshape(-1)
