"""Elementwise operation table and NumPy-2 type resolution.

The supported ufunc set and the promotion rule follow the reference
(_ops.py:5-76): Python scalars are "weak" (they adopt the array's dtype),
resolution is delegated to ``ufunc.resolve_dtypes``, and integer ``power`` is
rejected. ``where`` resolves its branches with ``np.result_type``.
"""

from functools import lru_cache

import numpy as np

_NAMES = (
    "add",
    "subtract",
    "multiply",
    "true_divide",
    "power",
    "negative",
    "positive",
    "absolute",
    "sqrt",
    "exp",
    "log",
    "sin",
    "cos",
    "tanh",
    "equal",
    "not_equal",
    "less",
    "less_equal",
    "greater",
    "greater_equal",
    "isfinite",
)

UFUNCS = {name: getattr(np, name) for name in _NAMES}

_PYTHON_SCALARS = (int, float, complex)


class HostScalar:
    """A scalar operand passed by value to a kernel (never uploaded).

    Backends recognise it through the ``_host_scalar`` marker; ``_data`` holds
    the value already converted to ``dtype``.
    """

    _host_scalar = True
    shape = ()

    def __init__(self, value, dtype):
        self.dtype = np.dtype(dtype)
        self._data = np.asarray(value, dtype=self.dtype)[()]

    def __repr__(self):
        return f"HostScalar({self._data!r}, {self.dtype})"


def _operand_type(value):
    weak = getattr(value, "weak_type", None)
    if weak is not None:
        return weak
    if type(value) in _PYTHON_SCALARS:
        return type(value)
    if hasattr(value, "dtype"):
        return value.dtype
    return np.asarray(value).dtype


def _operand_shape(value):
    if hasattr(value, "shape"):
        return value.shape
    return np.shape(value)


def broadcast_shape(shapes):
    """np.broadcast_shapes, with the common all-equal case answered directly."""
    shapes = [tuple(shape) for shape in shapes if shape != ()]  # scalars broadcast to anything
    if not shapes:
        return ()
    if all(shape == shapes[0] for shape in shapes[1:]):
        return shapes[0]
    return np.broadcast_shapes(*shapes)


@lru_cache(maxsize=4096)
def _resolved_dtypes(ufunc, types):
    # NumPy's loop resolution depends only on the operand types (dtypes, or
    # Python scalar types under weak promotion), so it is memoized by them.
    return tuple(np.dtype(d) for d in ufunc.resolve_dtypes(types + (None,)))


def resolve_elementwise(ufunc, inputs):
    """Return ``(resolved dtypes, broadcast shape)`` for one elementwise call.

    ``resolved`` lists the operand dtypes followed by the output dtype.
    """
    shape = broadcast_shape([_operand_shape(v) for v in inputs])
    if ufunc is np.where:
        samples = []
        for value in inputs[1:]:
            if getattr(value, "weak_type", None) is not None:
                samples.append(value.sample)
            elif type(value) in (bool, *_PYTHON_SCALARS):
                samples.append(value)
            else:
                samples.append(_operand_type(value))
        branch = np.result_type(*samples)
        return (np.dtype(bool), branch, branch, branch), shape
    if ufunc not in UFUNCS.values():
        raise NotImplementedError(f"Unsupported elementwise operation {ufunc.__name__}")
    resolved = _resolved_dtypes(ufunc, tuple(_operand_type(v) for v in inputs))
    if ufunc is np.power and resolved[-1].kind in "iu":
        raise NotImplementedError("Integer power is not supported; cast to float or multiply explicitly")
    return resolved, shape
