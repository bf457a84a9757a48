"""Elementwise operation table and NumPy-2 type resolution.

The supported ufunc set and the promotion rule follow the reference
(_ops.py:5-76): Python scalars are "weak" (they adopt the array's dtype),
resolution is delegated to ``ufunc.resolve_dtypes``, and integer ``power`` is
rejected. ``where`` resolves its branches with ``np.result_type``.
"""

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


def resolve_elementwise(ufunc, inputs):
    """Return ``(resolved dtypes, broadcast shape)`` for one elementwise call.

    ``resolved`` lists the operand dtypes followed by the output dtype.
    """
    shape = np.broadcast_shapes(*(_operand_shape(v) for v in inputs))
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
    resolved = ufunc.resolve_dtypes(tuple(_operand_type(v) for v in inputs) + (None,))
    if ufunc is np.power and resolved[-1].kind in "iu":
        raise NotImplementedError("Integer power is not supported; cast to float or multiply explicitly")
    return tuple(np.dtype(d) for d in resolved), shape
