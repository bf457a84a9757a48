"""TEST INFRASTRUCTURE ONLY - the reference NumPy backend's hot-path algorithms.

This is the CPU baseline that bench.py times (kind "port") and the tolerance
reference of the reference's own conformance tests:
- matmul:   reference backends.py:139-142 (``np.asarray(a @ b, dtype)``).
- norm:     reference _norm.py:44-52 (scale = max|x|; sum((x/scale)^2) in the
            output dtype, 0 where scale == 0; scale*sqrt(total); inf scale
            gives inf).
- random:   reference _random.py:34-58 (_numpy_data), via oracle.philox.
Pinned by tests/test_oracle_kernels.py and tests/test_oracle_philox.py: golden samples and norms written
from the reference NumPy backend (tests/golden/), closed forms (Pythagorean
triples, constant vectors), and the special-value table of reference
tests/test_stable_norm.py:60-66.
"""

import numpy as np

from . import philox


def matmul(a, b, dtype=None):
    dtype = dtype or np.result_type(a.dtype, b.dtype)
    return np.asarray(a @ b, dtype=dtype)


def norm(x, axis=None, keepdims=False, dtype=None):
    x = np.asarray(x)
    dtype = np.dtype(dtype or (x.dtype if x.dtype.kind == "f" else np.float64))
    axes = tuple(range(x.ndim)) if axis is None else (axis if isinstance(axis, tuple) else (axis,))
    axes = tuple(a % max(1, x.ndim) for a in axes)
    out_shape = tuple(1 if i in axes else d for i, d in enumerate(x.shape))
    if not x.size:
        result = np.zeros(out_shape, dtype)
    else:
        scale = np.max(np.abs(x), axis=axes, keepdims=True)
        with np.errstate(all="ignore"):
            ratio = np.divide(x, scale, out=np.zeros_like(x), where=scale != 0)
            total = np.sum(ratio * ratio, axis=axes, keepdims=True, dtype=dtype)
            result = scale * np.sqrt(total)
        result = np.where(np.isinf(scale), scale, result).astype(dtype)
    if not keepdims:
        result = result.reshape(tuple(d for i, d in enumerate(x.shape) if i not in axes))
    return result


def random(distribution, dtype, shape, seed, start=0, first=0.0, second=1.0):
    count = int(np.prod(shape, dtype=np.int64))
    out = np.empty(count, np.dtype(dtype))
    for base in range(0, count, 65536):
        n = min(65536, count - base)
        out[base : base + n] = philox.samples(distribution, dtype, n, seed, start + base, first, second)
    return out.reshape(shape)
