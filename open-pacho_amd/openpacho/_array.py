"""Resident, C-contiguous arrays owned by one backend, with explicit transfers.

Public behaviour follows the reference array facade (_array.py:31-522):
- arrays are created by array()/asarray()/constructors and never converted to
  host implicitly (``__array__`` raises; use asnumpy()/to_host());
- NumPy's ufunc and function protocols route ``np.*`` calls here;
- slicing and transposes return independent arrays (backend gathers), while
  reshape shares storage;
- matmul promotes with ``np.result_type``, broadcasts batch dimensions and
  may take the opt-in ``padding=True`` plan of the backend.
"""

import builtins
import operator
from math import prod

import numpy as np
from numpy.lib.mixins import NDArrayOperatorsMixin

from ._ops import UFUNCS as _UFUNCS
from ._ops import HostScalar, resolve_elementwise
from .backends import get_backend
from .exceptions import BackendMismatchError

_FUNCTIONS = {}
_UNSET = object()
_NATIVE_SCALAR_BACKENDS = ("hip",)


def _shape(value):
    if isinstance(value, (int, np.integer)):
        value = (value,)
    dims = tuple(operator.index(d) for d in value)
    if any(d < 0 for d in dims):
        raise ValueError("negative dimensions are not allowed")
    return dims


def _strides(shape):
    """C-order element strides of ``shape``."""
    out, step = [], 1
    for dim in reversed(shape):
        out.append(step)
        step *= dim
    return tuple(reversed(out))


def _reduced_shape(shape, axes, keepdims):
    if keepdims:
        return tuple(1 if i in axes else d for i, d in enumerate(shape))
    return tuple(d for i, d in enumerate(shape) if i not in axes)


class ndarray(NDArrayOperatorsMixin):
    """C-contiguous array owned by one backend; construct with array()/asarray().

    Slicing and transpose produce independent arrays, unlike NumPy views.
    Reshape shares storage; item assignment is not supported.
    """

    __array_priority__ = 1000

    def __init__(self, *args, **kwargs):
        raise TypeError("Use openpacho.array(), asarray(), zeros(), or ones()")

    @classmethod
    def _wrap(cls, data, shape, dtype, backend):
        """Attach shape/dtype metadata to backend storage (no copy)."""
        if getattr(backend, "_is_tracing", False):
            return backend.wrap(data, shape, dtype)
        obj = object.__new__(cls)
        obj._data = data
        obj._shape = tuple(shape)
        obj._dtype = np.dtype(dtype)
        obj._backend = backend
        return obj

    shape = property(lambda self: self._shape)
    dtype = property(lambda self: self._dtype)
    ndim = property(lambda self: len(self._shape))
    size = property(lambda self: prod(self._shape))
    nbytes = property(lambda self: prod(self._shape) * self._dtype.itemsize)
    backend = property(lambda self: self._backend.name)
    device = property(lambda self: self._backend.device)

    @property
    def T(self):
        return transpose(self)

    def __repr__(self):
        return (
            f"openpacho.ndarray(shape={self.shape}, dtype={self.dtype}, "
            f"backend={self.backend!r}, device={self.device!r})"
        )

    def __len__(self):
        if not self._shape:
            raise TypeError("len() of unsized object")
        return self._shape[0]

    def __bool__(self):
        raise ValueError("Array truth is ambiguous; transfer a scalar explicitly with .item()")

    def __array__(self, dtype=None, copy=None):
        raise TypeError("Implicit host conversion is disabled. Use openpacho.asnumpy(a) or a.to_host()")

    def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
        if method != "__call__" or kwargs.get("out") is not None:
            return NotImplemented
        kwargs.pop("out", None)
        if ufunc is np.matmul:
            return matmul(*inputs, **kwargs)
        if ufunc not in _UFUNCS.values():
            return NotImplemented
        if kwargs:
            raise NotImplementedError(f"ufunc options {tuple(kwargs)} are not supported")
        return _elementwise(ufunc, *inputs)

    def __array_function__(self, func, types, args, kwargs):
        handler = _FUNCTIONS.get(func)
        if handler is None or not all(issubclass(t, (ndarray, np.ndarray)) for t in types):
            return NotImplemented
        return handler(*args, **kwargs)

    def to_host(self):
        """Synchronize and return an independent NumPy array."""
        return self._backend.download(self)

    def item(self):
        if self.size != 1:
            raise ValueError("item() requires exactly one element")
        return self.to_host().item()

    def copy(self):
        return self.astype(self.dtype, copy=True)

    def astype(self, dtype, *, copy=True):
        dtype = self._backend.validate_dtype(dtype)
        if dtype == self.dtype and not copy:
            return self
        data = self._backend.elementwise("cast", [self], self.shape, dtype)
        return self._wrap(data, self.shape, dtype, self._backend)

    def reshape(self, *shape, order="C"):
        if len(shape) == 1 and not isinstance(shape[0], (int, np.integer)):
            shape = shape[0]
        return reshape(self, shape, order=order)

    def transpose(self, *axes):
        if len(axes) == 1 and (axes[0] is None or isinstance(axes[0], (tuple, list))):
            axes = axes[0]
        return transpose(self, axes or None)

    def sum(self, axis=None, dtype=None, out=None, keepdims=False):
        return sum(self, axis=axis, dtype=dtype, out=out, keepdims=keepdims)

    def mean(self, axis=None, dtype=None, out=None, keepdims=False):
        return mean(self, axis=axis, dtype=dtype, out=out, keepdims=keepdims)

    def min(self, axis=None, out=None, keepdims=False, initial=_UNSET, where=_UNSET):
        return amin(self, axis, out, keepdims, initial, where)

    def max(self, axis=None, out=None, keepdims=False, initial=_UNSET, where=_UNSET):
        return amax(self, axis, out, keepdims, initial, where)

    def __getitem__(self, key):
        key = key if isinstance(key, tuple) else (key,)
        if builtins.sum(k is Ellipsis for k in key) > 1:
            raise IndexError("an index can only have a single ellipsis")
        consumed = builtins.sum(k is not None and k is not Ellipsis for k in key)
        if consumed > self.ndim:
            raise IndexError("too many indices")
        fill = [slice(None)] * (self.ndim - consumed)
        if any(k is Ellipsis for k in key):
            expanded = []
            for k in key:
                expanded.extend(fill if k is Ellipsis else [k])
        else:
            expanded = list(key) + fill
        source = _strides(self.shape)
        out_shape, out_strides, offset, axis = [], [], 0, 0
        for k in expanded:
            if k is None:
                out_shape.append(1)
                out_strides.append(0)
                continue
            extent, step = self.shape[axis], source[axis]
            axis += 1
            if isinstance(k, slice):
                begin, end, stride = k.indices(extent)
                out_shape.append(len(range(begin, end, stride)))
                out_strides.append(step * stride)
                offset += begin * step
            elif isinstance(k, (int, np.integer)) and not isinstance(k, (bool, np.bool_)):
                position = operator.index(k)
                if not -extent <= position < extent:
                    raise IndexError("index out of bounds")
                offset += (position % extent) * step
            else:
                raise NotImplementedError("Only integer, slice, ellipsis and newaxis indexing are supported")
        data = self._backend.gather(self, tuple(out_shape), offset, tuple(out_strides))
        return self._wrap(data, out_shape, self.dtype, self._backend)


# ---- construction and transfer ------------------------------------------


def array(obj, dtype=None, *, copy=True, order="C", backend=None):
    if order != "C":
        raise NotImplementedError("Only C order is supported")
    if isinstance(obj, ndarray):
        target = obj._backend if backend is None else get_backend(backend)
        if target is not obj._backend:
            raise BackendMismatchError("Use to_backend(a, backend) to transfer explicitly")
        return obj.astype(dtype or obj.dtype, copy=copy)
    target = get_backend(backend)
    host = np.asarray(obj, dtype=dtype, order="C")
    target.validate_dtype(host.dtype)
    return ndarray._wrap(target.upload(host), host.shape, host.dtype, target)


def asarray(obj, dtype=None, *, order="C", backend=None):
    return array(obj, dtype=dtype, copy=False, order=order, backend=backend)


def asnumpy(a):
    if isinstance(a, ndarray):
        return a.to_host()
    return np.array(a, copy=True)


def to_backend(a, backend, *, device=None):
    target = get_backend(backend, device=device)
    if isinstance(a, ndarray) and a._backend is target:
        return a
    return asarray(asnumpy(a), backend=target)


def _common_backend(values):
    owners = [v._backend for v in values if isinstance(v, ndarray)]
    if not owners:
        return get_backend()
    if any(o is not owners[0] for o in owners[1:]):
        raise BackendMismatchError("Arrays belong to different backends/devices; use to_backend()")
    return owners[0]


# ---- elementwise -----------------------------------------------------------


def _elementwise(ufunc, *inputs):
    if any(isinstance(v, Expression) for v in inputs):
        return trace_op(ufunc, *inputs)
    backend = _common_backend(inputs)
    resolved, shape = resolve_elementwise(ufunc, inputs)
    for dtype in resolved:
        backend.validate_dtype(dtype)
    by_value = backend.name in _NATIVE_SCALAR_BACKENDS
    operands = []
    for value, dtype in zip(inputs, resolved):
        if by_value and not isinstance(value, ndarray) and np.isscalar(value):
            operands.append(HostScalar(value, dtype))
        else:
            operands.append(asarray(value, dtype=dtype, backend=backend))
    data = backend.elementwise(ufunc.__name__, operands, shape, resolved[-1])
    return ndarray._wrap(data, shape, resolved[-1], backend)


def _make_ufunc(ufunc):
    def call(*args):
        return _elementwise(ufunc, *args)

    call.__name__ = ufunc.__name__
    call.__qualname__ = ufunc.__name__
    call.__doc__ = f"Elementwise {ufunc.__name__} on the arrays' backend."
    return call


for _name, _ufunc in _UFUNCS.items():
    globals()[_name] = _make_ufunc(_ufunc)

_MISSING = object()


def where(condition, x=_MISSING, y=_MISSING):
    """Select broadcasted values on the chosen backend; both branches are evaluated."""
    if x is _MISSING and y is _MISSING:
        raise NotImplementedError("One-argument where (nonzero indices) is not supported")
    if x is _MISSING or y is _MISSING:
        raise TypeError("where requires both x and y")
    return _elementwise(np.where, condition, x, y)


# ---- constructors -----------------------------------------------------------


def empty(shape, dtype=float, *, order="C", backend=None):
    if order != "C":
        raise NotImplementedError("Only C order is supported")
    shape = _shape(shape)
    target = get_backend(backend)
    dtype = target.validate_dtype(dtype)
    return ndarray._wrap(target.empty(shape, dtype), shape, dtype, target)


def full(shape, fill_value, dtype=None, *, order="C", backend=None):
    if np.ndim(fill_value) != 0:
        raise NotImplementedError("full() supports scalar fill values")
    if order != "C":
        raise NotImplementedError("Only C order is supported")
    shape = _shape(shape)
    target = get_backend(backend)
    dtype = target.validate_dtype(dtype or np.asarray(fill_value).dtype)
    return ndarray._wrap(target.full(shape, fill_value, dtype), shape, dtype, target)


def zeros(shape, dtype=float, *, order="C", backend=None):
    return full(shape, 0, dtype=dtype, order=order, backend=backend)


def ones(shape, dtype=float, *, order="C", backend=None):
    return full(shape, 1, dtype=dtype, order=order, backend=backend)


def zeros_like(a, dtype=None):
    a = asarray(a)
    return zeros(a.shape, dtype=dtype or a.dtype, backend=a._backend)


def ones_like(a, dtype=None):
    a = asarray(a)
    return ones(a.shape, dtype=dtype or a.dtype, backend=a._backend)


def arange(start, stop=None, step=1, dtype=None, *, backend=None):
    """Host-evaluated sequence, uploaded once (constructors may run on host)."""
    return asarray(np.arange(start, stop, step, dtype=dtype), backend=backend)


def linspace(start, stop, num=50, endpoint=True, dtype=None, *, backend=None):
    return asarray(np.linspace(start, stop, num=num, endpoint=endpoint, dtype=dtype), backend=backend)


def eye(N, M=None, k=0, dtype=float, *, backend=None):
    return asarray(np.eye(N, M=M, k=k, dtype=dtype), backend=backend)


# ---- shape manipulation -----------------------------------------------------


def reshape(a, shape, order="C"):
    a = asarray(a)
    if order != "C":
        raise NotImplementedError("Only C order is supported")
    dims = (shape,) if isinstance(shape, (int, np.integer)) else tuple(shape)
    dims = tuple(operator.index(d) for d in dims)
    if builtins.sum(d == -1 for d in dims) > 1 or any(d < -1 for d in dims):
        raise ValueError("Invalid reshape dimensions")
    if -1 in dims:
        known = prod(d for d in dims if d != -1)
        if known == 0 or a.size % known:
            raise ValueError("Cannot infer reshape dimension")
        dims = tuple(a.size // known if d == -1 else d for d in dims)
    if prod(dims) != a.size:
        raise ValueError("Cannot reshape array to requested shape")
    return ndarray._wrap(a._data, dims, a.dtype, a._backend)


def _axis(axis, ndim):
    axis = operator.index(axis)
    if not -ndim <= axis < ndim:
        raise ValueError(f"axis {axis} out of bounds for array of dimension {ndim}")
    return axis % ndim


def _axes(axis, ndim):
    if axis is None:
        return tuple(range(ndim))
    # NumPy accepts axis=0/-1 (not tuples) on scalar reductions.
    if ndim == 0 and not isinstance(axis, tuple) and axis in (0, -1):
        return ()
    values = tuple(_axis(i, ndim) for i in (axis if isinstance(axis, tuple) else (axis,)))
    if len(set(values)) != len(values):
        raise ValueError("duplicate reduction axis")
    return tuple(sorted(values))


def transpose(a, axes=None):
    a = asarray(a)
    order = tuple(reversed(range(a.ndim))) if axes is None else tuple(axes)
    if len(order) != a.ndim:
        raise ValueError("axes don't match array")
    order = tuple(_axis(i, a.ndim) for i in order)
    if len(set(order)) != a.ndim:
        raise ValueError("repeated axis in transpose")
    source = _strides(a.shape)
    shape = tuple(a.shape[i] for i in order)
    data = a._backend.gather(a, shape, 0, tuple(source[i] for i in order))
    return ndarray._wrap(data, shape, a.dtype, a._backend)


def diag(a, k=0):
    a = asarray(a)
    k = operator.index(k)
    if a.ndim != 2:
        raise NotImplementedError("diag currently extracts matrix diagonals only")
    rows, cols = a.shape
    row0, col0 = max(0, -k), max(0, k)
    length = max(0, min(rows - row0, cols - col0))
    data = a._backend.gather(a, (length,), row0 * cols + col0, (cols + 1,))
    return ndarray._wrap(data, (length,), a.dtype, a._backend)


# ---- reductions ---------------------------------------------------------------


def sum(a, axis=None, dtype=None, out=None, keepdims=False):
    if out is not None:
        raise NotImplementedError("out= is not supported")
    a = asarray(a)
    axes = _axes(axis, a.ndim)
    if dtype is None:
        kind = a.dtype.kind
        dtype = np.dtype("int64") if kind in "bi" else np.dtype("uint64") if kind == "u" else a.dtype
    dtype = a._backend.validate_dtype(dtype)
    data = a._backend.reduce(a, axes, keepdims, dtype)
    return ndarray._wrap(data, _reduced_shape(a.shape, axes, keepdims), dtype, a._backend)


def _extreme(a, axis, out, keepdims, initial, where, operation):
    if out is not None:
        raise NotImplementedError("out= is not supported")
    if initial is not _UNSET:
        raise NotImplementedError("initial= is not supported")
    if where is not _UNSET:
        raise NotImplementedError("where= is not supported")
    a = asarray(a)
    axes = _axes(axis, a.ndim)
    if prod(a.shape[i] for i in axes) == 0:
        raise ValueError(f"zero-size array to reduction operation {operation} which has no identity")
    data = a._backend.reduce(a, axes, keepdims, a.dtype, operation=operation)
    return ndarray._wrap(data, _reduced_shape(a.shape, axes, keepdims), a.dtype, a._backend)


def amin(a, axis=None, out=None, keepdims=False, initial=_UNSET, where=_UNSET):
    """Minimum preserving dtype, propagating NaNs and preferring negative zero ties."""
    return _extreme(a, axis, out, keepdims, initial, where, "min")


def amax(a, axis=None, out=None, keepdims=False, initial=_UNSET, where=_UNSET):
    """Maximum preserving dtype, propagating NaNs and preferring positive zero ties."""
    return _extreme(a, axis, out, keepdims, initial, where, "max")


def mean(a, axis=None, dtype=None, out=None, keepdims=False):
    a = asarray(a)
    if a.ndim == 0 and axis is not None and not isinstance(axis, tuple):
        raise ValueError("axis out of bounds for scalar mean")
    dtype = np.dtype(dtype or (a.dtype if a.dtype.kind == "f" else np.float64))
    if dtype.kind != "f":
        raise NotImplementedError("mean supports floating point accumulation only")
    count = prod(a.shape[i] for i in _axes(axis, a.ndim))
    return sum(a, axis=axis, dtype=dtype, out=out, keepdims=keepdims) / count


# ---- products -----------------------------------------------------------------


def matmul(a, b, *, padding=False):
    """Matrix product; ``padding`` is an opt-in hint for the GPU GEMM kernels."""
    if (
        padding is False
        and type(a) is ndarray
        and type(b) is ndarray
        and a._backend is b._backend
        and a._dtype == b._dtype
        and 0 < len(a._shape) <= 2
        and 0 < len(b._shape) <= 2
    ):
        # Same backend and dtype, no batch axes: the general path below would
        # convert nothing and broadcast nothing; skip straight to the product.
        backend, dtype = a._backend, a._dtype
        if a._shape[-1] != b._shape[0]:
            raise ValueError("matmul inner dimensions do not match")
        if dtype.kind == "b":
            raise NotImplementedError("Boolean matmul is not supported")
        shape = a._shape[:-1] + b._shape[1:]
        return ndarray._wrap(backend.matmul(a, b, shape, dtype), shape, dtype, backend)
    if padding is not False:
        from ._padding import validate_padding

        padding = validate_padding(padding)
    backend = _common_backend((a, b))
    a, b = asarray(a, backend=backend), asarray(b, backend=backend)
    if a.ndim == 0 or b.ndim == 0:
        raise ValueError("matmul requires arrays with at least one dimension")
    if a.shape[-1] != b.shape[-2 if b.ndim > 1 else 0]:
        raise ValueError("matmul inner dimensions do not match")
    dtype = backend.validate_dtype(np.result_type(a.dtype, b.dtype))
    if dtype.kind == "b":
        raise NotImplementedError("Boolean matmul is not supported")
    a, b = a.astype(dtype, copy=False), b.astype(dtype, copy=False)
    batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    rows = () if a.ndim == 1 else (a.shape[-2],)
    cols = () if b.ndim == 1 else (b.shape[-1],)
    shape = batch + rows + cols
    plan = None
    if padding:
        from ._padding import prepare_padding

        plan = prepare_padding(backend, a.shape, b.shape, shape, dtype)
    data = backend.matmul(a, b, shape, dtype) if plan is None else plan.run(a, b)
    return ndarray._wrap(data, shape, dtype, backend)


def _rank(value):
    return value.ndim if isinstance(value, ndarray) else np.ndim(value)


def dot(a, b):
    if _rank(a) == 0 or _rank(b) == 0:
        return _elementwise(np.multiply, a, b)
    if _rank(a) > 2 or _rank(b) > 2:
        raise NotImplementedError("Higher-rank dot differs from batched matmul; use @ for batches")
    return matmul(a, b)


for _fn in (sum, amin, amax, mean, reshape, transpose, dot, diag, zeros_like, ones_like, where):
    _FUNCTIONS[getattr(np, _fn.__name__)] = _fn
_FUNCTIONS[np.min] = amin
_FUNCTIONS[np.max] = amax

# Imported last: _fusion builds on ndarray (import cycle), and a function-level
# import would run on every eager elementwise call.
from ._fusion import Expression, trace_op  # noqa: E402
