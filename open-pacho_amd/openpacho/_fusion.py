"""Typed operation capture shared by ``fuse`` and ``compile``.

While a function is captured, the default backend is a TraceBackend: every
array operation records an Expression node instead of running. Node fields
(``op``, ``inputs``, ``value``, ``resolved``, ``attrs``, ``shape``, ``dtype``)
are the lowering protocol's view of the graph (reference _fusion.py:86-253).
Host scalars passed as arguments become ScalarExpression terms that are
re-evaluated from the bindings of every call, so cached plans never freeze
them. Host observations, synchronisation, uninitialised arrays and random
generation are rejected during capture.

Two kinds of captured value live here:
- ScalarExpression, a tree of host arithmetic over scalar arguments. A leaf
  reads one call binding; an inner term applies a Python/NumPy function to
  its operands. Evaluation walks the tree for each call.
- Expression, a graph node that stands in for an array. TraceBackend
  answers the backend protocol by recording nodes; ``fuse`` allows only the
  elementwise part of the protocol.
"""

import operator
from dataclasses import dataclass
from functools import wraps
from types import SimpleNamespace

import numpy as np
from numpy.lib.mixins import NDArrayOperatorsMixin

from ._array import _reduced_shape, ndarray
from ._ops import HostScalar, resolve_elementwise
from .exceptions import BackendMismatchError


@dataclass(frozen=True)
class InputRef:
    """Position of a captured array argument in the call bindings."""

    index: int


# ---- host scalar terms ---------------------------------------------------------


class ScalarExpression(NDArrayOperatorsMixin):
    """Host scalar arithmetic captured symbolically and re-evaluated per call.

    ``sample`` is the value at capture time (it fixes the dtype and NumPy's
    weak-scalar promotion); ``evaluate(bindings)`` recomputes the value for
    the bindings of a later call.
    """

    __array_priority__ = 1500
    shape = ()

    def __init__(self, function, operands, sample, position=None):
        self._function = function  # None for a leaf
        self._operands = tuple(operands)
        self._position = position  # leaf: index into the bindings
        self.sample = sample
        self.weak_type = type(sample) if type(sample) in (int, float, complex) else None
        self.dtype = np.asarray(sample).dtype

    @classmethod
    def argument(cls, position, sample):
        """The scalar bound at ``position`` of each call."""
        return cls(None, (), sample, position)

    def evaluate(self, bindings):
        if self._function is None:
            return bindings[self._position]
        values = [v.evaluate(bindings) if isinstance(v, ScalarExpression) else v for v in self._operands]
        with np.errstate(all="ignore"):
            return self._function(*values)

    @classmethod
    def apply(cls, function, operands):
        """A term applying ``function``; NotImplemented next to an array."""
        if any(isinstance(v, ndarray) for v in operands):
            return NotImplemented
        samples = [v.sample if isinstance(v, ScalarExpression) else v for v in operands]
        with np.errstate(all="ignore"):
            sample = function(*samples)
        return cls(function, operands, sample)

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
        return self.apply(ufunc, inputs)

    # Python operators on a captured scalar (NumPy's operators come through
    # __array_ufunc__; these cover the cases where the other side is a plain
    # Python number).
    def __add__(self, other):
        return self.apply(operator.add, (self, other))

    def __radd__(self, other):
        return self.apply(operator.add, (other, self))

    def __sub__(self, other):
        return self.apply(operator.sub, (self, other))

    def __rsub__(self, other):
        return self.apply(operator.sub, (other, self))

    def __mul__(self, other):
        return self.apply(operator.mul, (self, other))

    def __rmul__(self, other):
        return self.apply(operator.mul, (other, self))

    def __truediv__(self, other):
        return self.apply(operator.truediv, (self, other))

    def __rtruediv__(self, other):
        return self.apply(operator.truediv, (other, self))

    def __neg__(self):
        return self.apply(operator.neg, (self,))

    def __pos__(self):
        return self.apply(operator.pos, (self,))


# ---- graph nodes ---------------------------------------------------------------


class Expression(ndarray):
    """A node of a captured graph; behaves as an array during capture."""

    __array_priority__ = 2000

    def __init__(self, backend, shape, dtype, *, op="input", inputs=(), value=None, resolved=(), attrs=None):
        # Storage of a node is the node itself: protocol code that passes
        # ``array._data`` around keeps working on the graph.
        self._data, self._backend = self, backend
        self._shape, self._dtype = tuple(shape), np.dtype(dtype)
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
        plain = method == "__call__" and kwargs.pop("out", None) is None
        if not plain:
            raise NotImplementedError("Only plain ufunc calls can be captured")
        if kwargs:
            raise NotImplementedError("ufunc options are not captured")
        if ufunc is np.matmul:
            from ._array import matmul

            return matmul(*inputs)
        return trace_op(ufunc, *inputs)


def _compile_only(capability):
    """Mark a TraceBackend method as unavailable to ``fuse`` captures."""

    def decorate(method):
        @wraps(method)
        def checked(self, *args, **kwargs):
            if self.elementwise_only:
                raise NotImplementedError(f"fuse supports elementwise expressions only, not {capability}; use compile")
            return method(self, *args, **kwargs)

        return checked

    return decorate


class TraceBackend:
    """Backend stand-in that records operations of one capture."""

    _is_tracing = True

    def __init__(self, target, *, elementwise_only=False):
        self.target = target
        self.name, self.device = target.name, target.device
        self.elementwise_only = elementwise_only

    def _record(self, op, shape, dtype, inputs=(), **fields):
        return Expression(self, shape, dtype, op=op, inputs=inputs, **fields)

    def validate_dtype(self, dtype):
        return self.target.validate_dtype(dtype)

    def wrap(self, data, shape, dtype):
        if not isinstance(data, Expression):
            raise TypeError("Invalid captured storage")
        if data.shape != tuple(shape) or data.dtype != np.dtype(dtype):
            return self._reshape(data, shape, dtype)
        return data

    @_compile_only("reshape")
    def _reshape(self, data, shape, dtype):
        return self._record("reshape", shape, dtype, (data,))

    # Host traffic and uninitialised storage have no place in a plan.
    def upload(self, value):
        value = np.asarray(value)
        if value.ndim:
            raise TypeError("Pass host arrays as explicit OpenPacho arguments before capture")
        return self._record("scalar", (), value.dtype, value=HostScalar(value, value.dtype))

    def download(self, value):
        raise TypeError("Host observations are forbidden during capture; observe the returned array")

    def synchronize(self):
        raise TypeError("Explicit synchronization is not captured")

    def empty(self, shape, dtype):
        raise NotImplementedError("Uninitialized arrays are not captured")

    def elementwise(self, name, args, shape, dtype):
        if name == "cast":
            return self._record("cast", shape, dtype, tuple(args), resolved=(args[0].dtype, dtype))
        return trace_op(getattr(np, name), *args)

    @_compile_only("full")
    def full(self, shape, value, dtype):
        return self._record("full", shape, dtype, attrs={"value": value})

    @_compile_only("gather")
    def gather(self, a, shape, offset, strides):
        return self._record("gather", shape, a.dtype, (a,), attrs={"offset": offset, "strides": tuple(strides)})

    @_compile_only("reduce")
    def reduce(self, a, axes, keepdims, dtype, *, operation="sum"):
        attrs = {"axes": tuple(axes), "keepdims": keepdims}
        if operation != "sum":
            attrs["operation"] = operation
        return self._record("reduce", _reduced_shape(a.shape, axes, keepdims), dtype, (a,), attrs=attrs)

    @_compile_only("matmul")
    def matmul(self, a, b, shape, dtype):
        return self._record("matmul", shape, dtype, (a, b))

    @_compile_only("matmul")
    def prepare_padded_matmul(self, ashape, bshape, shape, dtype):
        return SimpleNamespace(run=lambda a, b: self._record("matmul", shape, dtype, (a, b), attrs={"padding": True}))

    @_compile_only("norm")
    def norm(self, a, axes, keepdims, dtype):
        attrs = {"axes": tuple(axes), "keepdims": keepdims}
        return self._record("norm", _reduced_shape(a.shape, axes, keepdims), dtype, (a,), attrs=attrs)


def _operand_node(value, dtype, backend):
    """An elementwise operand as a node of ``backend``'s graph."""
    if isinstance(value, Expression):
        return value
    if isinstance(value, ScalarExpression):
        return backend._record("scalar", (), dtype, value=value)
    if np.isscalar(value):
        return backend._record("scalar", (), dtype, value=HostScalar(value, dtype))
    raise TypeError("Captured operands must be arrays or numeric scalars")


def trace_op(ufunc, *inputs):
    """Record one elementwise operation whose operands include a captured node."""
    backend = next(v._backend for v in inputs if isinstance(v, Expression))
    if any(isinstance(v, ndarray) and v._backend is not backend for v in inputs):
        raise BackendMismatchError("Captured arrays must be explicit arguments on the same backend")
    dtypes, shape = resolve_elementwise(ufunc, inputs)
    for dtype in dtypes:
        backend.validate_dtype(dtype)
    nodes = [_operand_node(v, d, backend) for v, d in zip(inputs, dtypes)]
    return backend._record(ufunc.__name__, shape, dtypes[-1], tuple(nodes), resolved=dtypes)


def fuse(function):
    """Capture one pure elementwise result; use compile for persistent plans."""

    @wraps(function)
    def wrapped(*args, **kwargs):
        from ._compiler import capture_call

        plan, bindings = capture_call(function, args, kwargs, elementwise_only=True)
        return plan.execute(bindings)

    return wrapped
