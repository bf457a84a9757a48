"""Resident, C-contiguous arrays owned by one backend, with explicit transfers.

Public behaviour follows the reference array facade (_array.py:31-522):
- arrays are created by array()/asarray()/constructors and never converted to
  host implicitly (``__array__`` raises; use asnumpy()/to_host());
- NumPy's ufunc and function protocols route ``np.*`` calls here;
- slicing and transposes return independent arrays (backend gathers), while
  reshape shares storage;
- matmul promotes with ``np.result_type``, broadcasts batch dimensions and
  may take the opt-in ``padding=True`` plan of the backend.

Every operation ends in one backend protocol call on storage; what this module
adds is the metadata arithmetic around it: index geometry for gathers, axis
normalisation and result shapes for reductions, operand promotion and batch
broadcasting for products.
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

_UNSET = object()
# Backends whose elementwise kernels take Python scalars as kernel arguments
# (no upload of a 0-d array per scalar).
_NATIVE_SCALAR_BACKENDS = ("hip",)

# NumPy function -> implementation, for __array_function__.
_HANDLERS = {}


def _implements(*functions):
    def register(implementation):
        for function in functions:
            _HANDLERS[function] = implementation
        return implementation

    return register


# ---- shape arithmetic ----------------------------------------------------------


def _shape(value):
    """A shape argument (an int or a sequence of ints) as a tuple."""
    dims = (operator.index(value),) if isinstance(value, (int, np.integer)) else tuple(map(operator.index, value))
    if min(dims, default=0) < 0:
        raise ValueError("negative dimensions are not allowed")
    return dims


def _strides(shape):
    """C-order element strides of ``shape``."""
    strides = [1] * len(shape)
    for axis in range(len(shape) - 2, -1, -1):
        strides[axis] = strides[axis + 1] * shape[axis + 1]
    return tuple(strides)


def _axis(axis, ndim):
    axis = operator.index(axis)
    if axis < -ndim or axis >= ndim:
        raise ValueError(f"axis {axis} out of bounds for array of dimension {ndim}")
    return axis + ndim if axis < 0 else axis


def _axes(axis, ndim):
    """Sorted, validated reduction axes (None: all of them)."""
    if axis is None:
        return tuple(range(ndim))
    grouped = isinstance(axis, tuple)
    # NumPy accepts axis=0/-1 (not tuples) on reductions of a 0-d array.
    if ndim == 0 and not grouped and axis in (0, -1):
        return ()
    normalised = [_axis(a, ndim) for a in (axis if grouped else (axis,))]
    if len(set(normalised)) < len(normalised):
        raise ValueError("duplicate reduction axis")
    return tuple(sorted(normalised))


def _reduced_shape(shape, axes, keepdims):
    kept = ((1 if i in axes else d) for i, d in enumerate(shape)) if keepdims else (
        d for i, d in enumerate(shape) if i not in axes)
    return tuple(kept)


def _index_terms(key, ndim):
    """The index as one term per output-producing position: None (new axis),
    a slice, or an int; an Ellipsis becomes the full slices it stands for."""
    key = key if isinstance(key, tuple) else (key,)
    ellipses = [i for i, k in enumerate(key) if k is Ellipsis]
    if len(ellipses) > 1:
        raise IndexError("an index can only have a single ellipsis")
    consuming = len(key) - len(ellipses) - builtins.sum(k is None for k in key)
    if consuming > ndim:
        raise IndexError("too many indices")
    fill = [slice(None)] * (ndim - consuming)
    if ellipses:
        at = ellipses[0]
        return list(key[:at]) + fill + list(key[at + 1 :])
    return list(key) + fill


def _index_geometry(shape, key):
    """(shape, element offset, element strides) that a basic index selects
    from a C-contiguous array of ``shape``."""
    source = iter(zip(shape, _strides(shape)))
    out_shape, out_strides, offset = [], [], 0
    for term in _index_terms(key, len(shape)):
        if term is None:
            out_shape.append(1)
            out_strides.append(0)
            continue
        extent, stride = next(source)
        if isinstance(term, slice):
            first, stop, step = term.indices(extent)
            out_shape.append(len(range(first, stop, step)))
            out_strides.append(stride * step)
            offset += first * stride
        elif isinstance(term, (int, np.integer)) and not isinstance(term, (bool, np.bool_)):
            position = operator.index(term)
            if not -extent <= position < extent:
                raise IndexError("index out of bounds")
            offset += (position % extent) * stride
        else:
            raise NotImplementedError("Only integer, slice, ellipsis and newaxis indexing are supported")
    return tuple(out_shape), offset, tuple(out_strides)


# ---- the array -----------------------------------------------------------------


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
        array = object.__new__(cls)
        array._data, array._shape, array._dtype, array._backend = data, tuple(shape), np.dtype(dtype), backend
        return array

    @property
    def shape(self):
        return self._shape

    @property
    def dtype(self):
        return self._dtype

    @property
    def ndim(self):
        return len(self._shape)

    @property
    def size(self):
        return prod(self._shape)

    @property
    def nbytes(self):
        return self.size * self._dtype.itemsize

    @property
    def backend(self):
        return self._backend.name

    @property
    def device(self):
        return self._backend.device

    @property
    def T(self):
        return transpose(self)

    def __repr__(self):
        return (
            f"openpacho.ndarray(shape={self.shape}, dtype={self.dtype}, "
            f"backend={self.backend!r}, device={self.device!r})"
        )

    def __len__(self):
        if self._shape:
            return self._shape[0]
        raise TypeError("len() of unsized object")

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
        if ufunc not in _UFUNC_SET:
            return NotImplemented
        if kwargs:
            raise NotImplementedError(f"ufunc options {tuple(kwargs)} are not supported")
        return _elementwise(ufunc, *inputs)

    def __array_function__(self, func, types, args, kwargs):
        handler = _HANDLERS.get(func)
        if handler is not None and all(issubclass(t, (ndarray, np.ndarray)) for t in types):
            return handler(*args, **kwargs)
        return NotImplemented

    def to_host(self):
        """Synchronize and return an independent NumPy array."""
        return self._backend.download(self)

    def item(self):
        if self.size == 1:
            return self.to_host().item()
        raise ValueError("item() requires exactly one element")

    def copy(self):
        return self.astype(self.dtype, copy=True)

    def astype(self, dtype, *, copy=True):
        dtype = self._backend.validate_dtype(dtype)
        if dtype == self._dtype and not copy:
            return self
        return _result(self._backend.elementwise("cast", [self], self._shape, dtype), self._shape, dtype, self._backend)

    def reshape(self, *shape, order="C"):
        single = len(shape) == 1 and not isinstance(shape[0], (int, np.integer))
        return reshape(self, shape[0] if single else shape, order=order)

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
        shape, offset, strides = _index_geometry(self._shape, key)
        return _result(self._backend.gather(self, shape, offset, strides), shape, self._dtype, self._backend)


def _result(data, shape, dtype, backend):
    return ndarray._wrap(data, shape, dtype, backend)


# ---- construction and transfer -------------------------------------------------


def _c_order(order):
    if order != "C":
        raise NotImplementedError("Only C order is supported")


def array(obj, dtype=None, *, copy=True, order="C", backend=None):
    _c_order(order)
    if isinstance(obj, ndarray):
        if backend is not None and get_backend(backend) is not obj._backend:
            raise BackendMismatchError("Use to_backend(a, backend) to transfer explicitly")
        return obj.astype(dtype or obj.dtype, copy=copy)
    target = get_backend(backend)
    host = np.asarray(obj, dtype=dtype, order="C")
    target.validate_dtype(host.dtype)
    return _result(target.upload(host), host.shape, host.dtype, target)


def asarray(obj, dtype=None, *, order="C", backend=None):
    return array(obj, dtype=dtype, copy=False, order=order, backend=backend)


def asnumpy(a):
    return a.to_host() if isinstance(a, ndarray) else np.array(a, copy=True)


def to_backend(a, backend, *, device=None):
    target = get_backend(backend, device=device)
    if isinstance(a, ndarray) and a._backend is target:
        return a
    return asarray(asnumpy(a), backend=target)


def _common_backend(values):
    """The one backend that owns every array among ``values`` (default if none)."""
    owner = None
    for value in values:
        if isinstance(value, ndarray):
            if owner is None:
                owner = value._backend
            elif value._backend is not owner:
                raise BackendMismatchError("Arrays belong to different backends/devices; use to_backend()")
    return get_backend() if owner is None else owner


# ---- elementwise ---------------------------------------------------------------

_UFUNC_SET = frozenset(_UFUNCS.values())


def _elementwise(ufunc, *inputs):
    if any(isinstance(v, Expression) for v in inputs):
        return trace_op(ufunc, *inputs)
    backend = _common_backend(inputs)
    dtypes, shape = resolve_elementwise(ufunc, inputs)
    for dtype in dtypes:
        backend.validate_dtype(dtype)
    scalars_by_value = backend.name in _NATIVE_SCALAR_BACKENDS

    def operand(value, dtype):
        if scalars_by_value and not isinstance(value, ndarray) and np.isscalar(value):
            return HostScalar(value, dtype)
        return asarray(value, dtype=dtype, backend=backend)

    operands = [operand(v, d) for v, d in zip(inputs, dtypes)]
    out_dtype = dtypes[-1]
    return _result(backend.elementwise(ufunc.__name__, operands, shape, out_dtype), shape, out_dtype, backend)


def _ufunc_function(ufunc):
    name = ufunc.__name__

    def function(*args):
        return _elementwise(ufunc, *args)

    function.__name__ = function.__qualname__ = name
    function.__doc__ = f"Elementwise {name} on the arrays' backend."
    return function


globals().update({name: _ufunc_function(ufunc) for name, ufunc in _UFUNCS.items()})

_MISSING = object()


@_implements(np.where)
def where(condition, x=_MISSING, y=_MISSING):
    """Select broadcasted values on the chosen backend; both branches are evaluated."""
    given = (x is not _MISSING) + (y is not _MISSING)
    if given == 0:
        raise NotImplementedError("One-argument where (nonzero indices) is not supported")
    if given == 1:
        raise TypeError("where requires both x and y")
    return _elementwise(np.where, condition, x, y)


# ---- constructors --------------------------------------------------------------


def empty(shape, dtype=float, *, order="C", backend=None):
    _c_order(order)
    shape, target = _shape(shape), get_backend(backend)
    dtype = target.validate_dtype(dtype)
    return _result(target.empty(shape, dtype), shape, dtype, target)


def full(shape, fill_value, dtype=None, *, order="C", backend=None):
    if np.ndim(fill_value) != 0:
        raise NotImplementedError("full() supports scalar fill values")
    _c_order(order)
    shape, target = _shape(shape), get_backend(backend)
    dtype = target.validate_dtype(np.asarray(fill_value).dtype if dtype is None else dtype)
    return _result(target.full(shape, fill_value, dtype), shape, dtype, target)


def zeros(shape, dtype=float, *, order="C", backend=None):
    return full(shape, 0, dtype=dtype, order=order, backend=backend)


def ones(shape, dtype=float, *, order="C", backend=None):
    return full(shape, 1, dtype=dtype, order=order, backend=backend)


def _filled_like(a, value, dtype):
    a = asarray(a)
    return full(a.shape, value, dtype=a.dtype if dtype is None else dtype, backend=a._backend)


@_implements(np.zeros_like)
def zeros_like(a, dtype=None):
    return _filled_like(a, 0, dtype)


@_implements(np.ones_like)
def ones_like(a, dtype=None):
    return _filled_like(a, 1, dtype)


# Sequences are computed once on the host and uploaded; arithmetic never is.


def arange(start, stop=None, step=1, dtype=None, *, backend=None):
    """Host-evaluated sequence, uploaded once (constructors may run on host)."""
    return asarray(np.arange(start, stop, step, dtype=dtype), backend=backend)


def linspace(start, stop, num=50, endpoint=True, dtype=None, *, backend=None):
    return asarray(np.linspace(start, stop, num=num, endpoint=endpoint, dtype=dtype), backend=backend)


def eye(N, M=None, k=0, dtype=float, *, backend=None):
    return asarray(np.eye(N, M=M, k=k, dtype=dtype), backend=backend)


# ---- shape manipulation --------------------------------------------------------


@_implements(np.reshape)
def reshape(a, shape, order="C"):
    a = asarray(a)
    _c_order(order)
    dims = [operator.index(d) for d in ((shape,) if isinstance(shape, (int, np.integer)) else shape)]
    unknown = [i for i, d in enumerate(dims) if d == -1]
    if len(unknown) > 1 or any(d < -1 for d in dims):
        raise ValueError("Invalid reshape dimensions")
    if unknown:
        known = prod(d for d in dims if d != -1)
        if known == 0 or a.size % known:
            raise ValueError("Cannot infer reshape dimension")
        dims[unknown[0]] = a.size // known
    if prod(dims) != a.size:
        raise ValueError("Cannot reshape array to requested shape")
    return _result(a._data, tuple(dims), a.dtype, a._backend)


@_implements(np.transpose)
def transpose(a, axes=None):
    a = asarray(a)
    order = tuple(range(a.ndim - 1, -1, -1)) if axes is None else tuple(axes)
    if len(order) != a.ndim:
        raise ValueError("axes don't match array")
    order = tuple(_axis(i, a.ndim) for i in order)
    if len(set(order)) != a.ndim:
        raise ValueError("repeated axis in transpose")
    strides = _strides(a.shape)
    shape = tuple(a.shape[i] for i in order)
    return _result(a._backend.gather(a, shape, 0, tuple(strides[i] for i in order)), shape, a.dtype, a._backend)


@_implements(np.diag)
def diag(a, k=0):
    a = asarray(a)
    k = operator.index(k)
    if a.ndim != 2:
        raise NotImplementedError("diag currently extracts matrix diagonals only")
    rows, cols = a.shape
    first_row, first_col = (0, k) if k >= 0 else (-k, 0)
    length = max(0, min(rows - first_row, cols - first_col))
    data = a._backend.gather(a, (length,), first_row * cols + first_col, (cols + 1,))
    return _result(data, (length,), a.dtype, a._backend)


# ---- reductions ----------------------------------------------------------------


def _unsupported_options(out=None, **options):
    if out is not None:
        raise NotImplementedError("out= is not supported")
    for name, value in options.items():
        if value is not _UNSET:
            raise NotImplementedError(f"{name}= is not supported")


def _sum_dtype(dtype):
    """NumPy's default accumulator: 64-bit for bool and integers."""
    if dtype.kind in "bi":
        return np.dtype(np.int64)
    if dtype.kind == "u":
        return np.dtype(np.uint64)
    return dtype


def _reduction(a, axes, keepdims, dtype, **operation):
    data = a._backend.reduce(a, axes, keepdims, dtype, **operation)
    return _result(data, _reduced_shape(a.shape, axes, keepdims), dtype, a._backend)


@_implements(np.sum)
def sum(a, axis=None, dtype=None, out=None, keepdims=False):
    _unsupported_options(out)
    a = asarray(a)
    axes = _axes(axis, a.ndim)
    dtype = a._backend.validate_dtype(_sum_dtype(a.dtype) if dtype is None else dtype)
    return _reduction(a, axes, keepdims, dtype)


def _extreme(operation, a, axis, out, keepdims, initial, where):
    _unsupported_options(out, initial=initial, where=where)
    a = asarray(a)
    axes = _axes(axis, a.ndim)
    if any(a.shape[i] == 0 for i in axes):
        raise ValueError(f"zero-size array to reduction operation {operation} which has no identity")
    return _reduction(a, axes, keepdims, a.dtype, operation=operation)


@_implements(np.amin, np.min)
def amin(a, axis=None, out=None, keepdims=False, initial=_UNSET, where=_UNSET):
    """Minimum preserving dtype, propagating NaNs and preferring negative zero ties."""
    return _extreme("min", a, axis, out, keepdims, initial, where)


@_implements(np.amax, np.max)
def amax(a, axis=None, out=None, keepdims=False, initial=_UNSET, where=_UNSET):
    """Maximum preserving dtype, propagating NaNs and preferring positive zero ties."""
    return _extreme("max", a, axis, out, keepdims, initial, where)


@_implements(np.mean)
def mean(a, axis=None, dtype=None, out=None, keepdims=False):
    a = asarray(a)
    if a.ndim == 0 and axis is not None and not isinstance(axis, tuple):
        raise ValueError("axis out of bounds for scalar mean")
    dtype = np.dtype(dtype or (a.dtype if a.dtype.kind == "f" else np.float64))
    if dtype.kind != "f":
        raise NotImplementedError("mean supports floating point accumulation only")
    count = prod(a.shape[i] for i in _axes(axis, a.ndim))
    return sum(a, axis=axis, dtype=dtype, out=out, keepdims=keepdims) / count


# ---- products ------------------------------------------------------------------


def _product_shape(a_shape, b_shape):
    """Broadcast batch, then the rows of a matrix left operand and the columns
    of a matrix right operand (a vector operand contributes neither)."""
    batch = np.broadcast_shapes(a_shape[:-2], b_shape[:-2])
    rows = a_shape[-2:-1]  # empty for a vector
    cols = b_shape[-1:] if len(b_shape) > 1 else ()
    return batch + rows + cols


def _simple_operands(a, b):
    """Two arrays of one backend and dtype, each a vector or a matrix."""
    return (
        type(a) is ndarray
        and type(b) is ndarray
        and a._backend is b._backend
        and a._dtype == b._dtype
        and 0 < len(a._shape) <= 2
        and 0 < len(b._shape) <= 2
    )


def matmul(a, b, *, padding=False):
    """Matrix product; ``padding`` is an opt-in hint for the GPU GEMM kernels."""
    if padding is False and _simple_operands(a, b):
        # Nothing to convert or broadcast: straight to the backend product.
        if a._shape[-1] != b._shape[0]:
            raise ValueError("matmul inner dimensions do not match")
        if a._dtype.kind == "b":
            raise NotImplementedError("Boolean matmul is not supported")
        shape = a._shape[:-1] + b._shape[1:]
        return _result(a._backend.matmul(a, b, shape, a._dtype), shape, a._dtype, a._backend)
    if padding is not False:
        from ._padding import validate_padding

        padding = validate_padding(padding)
    backend = _common_backend((a, b))
    a, b = asarray(a, backend=backend), asarray(b, backend=backend)
    if not a.ndim or not b.ndim:
        raise ValueError("matmul requires arrays with at least one dimension")
    if a.shape[-1] != b.shape[-2 if b.ndim > 1 else 0]:
        raise ValueError("matmul inner dimensions do not match")
    dtype = backend.validate_dtype(np.result_type(a.dtype, b.dtype))
    if dtype.kind == "b":
        raise NotImplementedError("Boolean matmul is not supported")
    a, b = a.astype(dtype, copy=False), b.astype(dtype, copy=False)
    shape = _product_shape(a.shape, b.shape)
    plan = None
    if padding:
        from ._padding import prepare_padding

        plan = prepare_padding(backend, a.shape, b.shape, shape, dtype)
    data = plan.run(a, b) if plan is not None else backend.matmul(a, b, shape, dtype)
    return _result(data, shape, dtype, backend)


@_implements(np.dot)
def dot(a, b):
    if type(a) is ndarray and type(b) is ndarray and len(a._shape) == 1 == len(b._shape):
        # Two vectors of one backend, dtype and length: a backend that offers
        # a one-call vector dot skips the product dispatch (the same 0-d
        # result as the matmul below).
        fast = getattr(a._backend, "vector_dot", None)
        if fast is not None and a._backend is b._backend and a._dtype == b._dtype and a._dtype.kind == "f":
            if a._shape == b._shape and a._shape[0]:
                result = object.__new__(ndarray)
                result._data, result._shape, result._dtype, result._backend = fast(a, b), (), a._dtype, a._backend
                return result
    ranks = [v.ndim if isinstance(v, ndarray) else np.ndim(v) for v in (a, b)]
    if 0 in ranks:
        return _elementwise(np.multiply, a, b)
    if max(ranks) > 2:
        raise NotImplementedError("Higher-rank dot differs from batched matmul; use @ for batches")
    return matmul(a, b)


# Imported last: _fusion builds on ndarray (import cycle), and a function-level
# import would run on every eager elementwise call.
from ._fusion import Expression, trace_op  # noqa: E402
