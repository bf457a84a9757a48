"""Opt-in physical padding hint for GEMM (reference _padding.py:13-22).

``padding`` must be a boolean. A backend that can pad exposes
``prepare_padded_matmul(ashape, bshape, shape, dtype)`` returning a plan with
``run(a, b)``, ``explain()`` and ``dispatch_count``, or None to decline (then
ordinary matmul runs). An absent capability declines the hint; preparation
failures propagate. The hip backend's plan is openpacho._hip_padding.
"""

import numpy as np


def validate_padding(value):
    if not isinstance(value, (bool, np.bool_)):
        raise TypeError("padding must be a boolean")
    return bool(value)


def prepare_padding(backend, ashape, bshape, shape, dtype):
    factory = getattr(backend, "prepare_padded_matmul", None)
    return None if factory is None else factory(ashape, bshape, shape, dtype)
