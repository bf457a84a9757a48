"""Typed operation capture shared by ``fuse`` and ``compile``.

While a function is captured, the default backend is a TraceBackend: every
array operation records an Expression node instead of running. Node fields
(``op``, ``inputs``, ``value``, ``resolved``, ``attrs``, ``shape``, ``dtype``)
are the lowering protocol's view of the graph (reference _fusion.py:86-253).
Host scalars passed as arguments become ScalarExpression values that are
re-evaluated from the bindings of every call, so cached plans never freeze
them. Host observations, synchronisation, uninitialised arrays and random
generation are rejected during capture.
"""

import operator
from dataclasses import dataclass
from functools import wraps
from types import SimpleNamespace

import numpy as np
from numpy.lib.mixins import NDArrayOperatorsMixin

from ._array import ndarray
from ._ops import HostScalar, resolve_elementwise
from .exceptions import BackendMismatchError


@dataclass(frozen=True)
class InputRef:
    """Position of a captured array argument in the call bindings."""

    index: int


class ScalarExpression(NDArrayOperatorsMixin):
    """Host scalar arithmetic captured symbolically and re-evaluated per call."""

    __array_priority__ = 1500
    shape = ()

    def __init__(self, evaluate, sample):
        self.evaluate = evaluate
        self.sample = sample
        self.weak_type = type(sample) if type(sample) in (int, float, complex) else None
        self.dtype = np.asarray(sample).dtype

    def __bool__(self):
        raise TypeError("Data-dependent control flow is not captured; declare static_argnames")

    def __index__(self):
        raise TypeError("Shape/axis/loop arguments must be declared in static_argnames")

    def __array__(self, dtype=None, copy=None):
        raise TypeError("Cannot convert a captured scalar to a host array")

    def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
        if method != "__call__" or kwargs:
            raise NotImplementedError("Only plain scalar ufunc calls can be captured")
        if any(isinstance(v, Expression) for v in inputs):
            return trace_op(ufunc, *inputs)
        return ScalarExpression.combine(ufunc, inputs)

    @staticmethod
    def combine(function, inputs):
        if any(isinstance(v, ndarray) for v in inputs):
            return NotImplemented

        def resolve(bindings):
            values = [v.evaluate(bindings) if isinstance(v, ScalarExpression) else v for v in inputs]
            with np.errstate(all="ignore"):
                return function(*values)

        samples = [v.sample if isinstance(v, ScalarExpression) else v for v in inputs]
        with np.errstate(all="ignore"):
            sample = function(*samples)
        return ScalarExpression(resolve, sample)


def _binary(function, reflected):
    if reflected:
        return lambda self, other: ScalarExpression.combine(function, (other, self))
    return lambda self, other: ScalarExpression.combine(function, (self, other))


for _dunder, _function in (
    ("add", operator.add),
    ("sub", operator.sub),
    ("mul", operator.mul),
    ("truediv", operator.truediv),
):
    setattr(ScalarExpression, f"__{_dunder}__", _binary(_function, False))
    setattr(ScalarExpression, f"__r{_dunder}__", _binary(_function, True))
ScalarExpression.__neg__ = lambda self: ScalarExpression.combine(operator.neg, (self,))
ScalarExpression.__pos__ = lambda self: ScalarExpression.combine(operator.pos, (self,))


class Expression(ndarray):
    """A node of a captured graph; behaves as an array during capture."""

    __array_priority__ = 2000

    def __init__(self, backend, shape, dtype, *, op="input", inputs=(), value=None, resolved=(), attrs=None):
        self._shape = tuple(shape)
        self._dtype = np.dtype(dtype)
        self._backend = backend
        self._data = self
        self.op = op
        self.inputs = tuple(inputs)
        self.value = value
        self.resolved = tuple(resolved)
        self.attrs = dict(attrs or {})

    def __repr__(self):
        return f"Expression(op={self.op!r}, shape={self.shape}, dtype={self.dtype})"

    def __bool__(self):
        raise TypeError("Captured functions do not support data-dependent Python control flow")

    def __array__(self, dtype=None, copy=None):
        raise TypeError("Host conversion is forbidden during capture")

    def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
        if method != "__call__" or kwargs.get("out") is not None:
            raise NotImplementedError("Only plain ufunc calls can be captured")
        kwargs.pop("out", None)
        if kwargs:
            raise NotImplementedError("ufunc options are not captured")
        if ufunc is np.matmul:
            from ._array import matmul

            return matmul(*inputs)
        return trace_op(ufunc, *inputs)


def _reduced(shape, axes, keepdims):
    if keepdims:
        return tuple(1 if i in axes else d for i, d in enumerate(shape))
    return tuple(d for i, d in enumerate(shape) if i not in axes)


class TraceBackend:
    """Backend stand-in that records operations of one capture."""

    _is_tracing = True

    def __init__(self, target, *, elementwise_only=False):
        self.target = target
        self.name = target.name
        self.device = target.device
        self.elementwise_only = elementwise_only

    def _require_general(self, what):
        if self.elementwise_only:
            raise NotImplementedError(f"fuse supports elementwise expressions only, not {what}; use compile")

    def validate_dtype(self, dtype):
        return self.target.validate_dtype(dtype)

    def wrap(self, data, shape, dtype):
        if not isinstance(data, Expression):
            raise TypeError("Invalid captured storage")
        if data.shape == tuple(shape) and data.dtype == np.dtype(dtype):
            return data
        self._require_general("reshape")
        return Expression(self, shape, dtype, op="reshape", inputs=(data,))

    def upload(self, value):
        value = np.asarray(value)
        if value.ndim:
            raise TypeError("Pass host arrays as explicit OpenPacho arguments before capture")
        return Expression(self, (), value.dtype, op="scalar", value=HostScalar(value, value.dtype))

    def download(self, value):
        raise TypeError("Host observations are forbidden during capture; observe the returned array")

    def synchronize(self):
        raise TypeError("Explicit synchronization is not captured")

    def empty(self, shape, dtype):
        raise NotImplementedError("Uninitialized arrays are not captured")

    def full(self, shape, value, dtype):
        self._require_general("full")
        return Expression(self, shape, dtype, op="full", attrs={"value": value})

    def elementwise(self, name, args, shape, dtype):
        if name == "cast":
            return Expression(self, shape, dtype, op="cast", inputs=tuple(args), resolved=(args[0].dtype, dtype))
        return trace_op(getattr(np, name), *args)

    def gather(self, a, shape, offset, strides):
        self._require_general("gather")
        attrs = {"offset": offset, "strides": tuple(strides)}
        return Expression(self, shape, a.dtype, op="gather", inputs=(a,), attrs=attrs)

    def reduce(self, a, axes, keepdims, dtype, *, operation="sum"):
        self._require_general("reduce")
        attrs = {"axes": tuple(axes), "keepdims": keepdims}
        if operation != "sum":
            attrs["operation"] = operation
        return Expression(self, _reduced(a.shape, axes, keepdims), dtype, op="reduce", inputs=(a,), attrs=attrs)

    def matmul(self, a, b, shape, dtype):
        self._require_general("matmul")
        return Expression(self, shape, dtype, op="matmul", inputs=(a, b))

    def prepare_padded_matmul(self, ashape, bshape, shape, dtype):
        self._require_general("matmul")

        def run(a, b):
            return Expression(self, shape, dtype, op="matmul", inputs=(a, b), attrs={"padding": True})

        return SimpleNamespace(run=run)

    def norm(self, a, axes, keepdims, dtype):
        self._require_general("norm")
        attrs = {"axes": tuple(axes), "keepdims": keepdims}
        return Expression(self, _reduced(a.shape, axes, keepdims), dtype, op="norm", inputs=(a,), attrs=attrs)


def trace_op(ufunc, *inputs):
    """Record one elementwise operation whose operands include a captured node."""
    backend = next(v for v in inputs if isinstance(v, Expression))._backend
    for value in inputs:
        if isinstance(value, ndarray) and value._backend is not backend:
            raise BackendMismatchError("Captured arrays must be explicit arguments on the same backend")
    resolved, shape = resolve_elementwise(ufunc, inputs)
    for dtype in resolved:
        backend.validate_dtype(dtype)
    operands = []
    for value, dtype in zip(inputs, resolved):
        if isinstance(value, Expression):
            operands.append(value)
        elif isinstance(value, ScalarExpression):
            operands.append(Expression(backend, (), dtype, op="scalar", value=value))
        elif np.isscalar(value):
            operands.append(Expression(backend, (), dtype, op="scalar", value=HostScalar(value, dtype)))
        else:
            raise TypeError("Captured operands must be arrays or numeric scalars")
    return Expression(backend, shape, resolved[-1], op=ufunc.__name__, inputs=operands, resolved=resolved)


def fuse(function):
    """Capture one pure elementwise result; use compile for persistent plans."""

    @wraps(function)
    def wrapped(*args, **kwargs):
        from ._compiler import capture_call

        plan, bindings = capture_call(function, args, kwargs, elementwise_only=True)
        return plan.execute(bindings)

    return wrapped
