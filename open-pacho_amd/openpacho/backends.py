"""Backend selection and the NumPy (CPU) backend.

Selection semantics follow the reference (backends.py:153-235): a
ContextVar holds the default backend per thread/task, ``set_backend`` changes
it for the current context and ``use_backend`` scopes it. Importing the
package initialises no GPU runtime; the ``hip`` backend loads its native
library on first selection.

This build provides two backends: ``numpy`` (the CPU reference) and ``hip``
(MI355X, libpacho_hip.so). Requests for the reference's ``opencl``,
``vulkan`` or ``cuda`` runtimes raise BackendUnavailableError.
"""

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
from functools import lru_cache

import numpy as np

from .exceptions import BackendUnavailableError, UnsupportedDtypeError

SUPPORTED_DTYPES = tuple(
    np.dtype(name) for name in ("bool", "int32", "int64", "uint32", "uint64", "float32", "float64")
)

_FOREIGN_RUNTIMES = ("opencl", "vulkan", "cuda")


def check_dtype(dtype):
    """Normalise ``dtype`` and reject types outside the supported set."""
    dtype = np.dtype(dtype)
    if not dtype.isnative or dtype not in SUPPORTED_DTYPES:
        raise UnsupportedDtypeError(f"Unsupported dtype {dtype}; supported: {SUPPORTED_DTYPES}")
    return dtype


@dataclass(frozen=True)
class DeviceInfo:
    id: str
    name: str
    vendor: str
    kind: str
    fp64: bool
    memory_bytes: int
    driver: str


def _foreign(name):
    return BackendUnavailableError(
        f"The {name!r} runtime is not part of this build; it provides 'numpy' and 'hip' (MI355X)"
    )


def devices(backend="hip"):
    """List the devices of an explicitly selected GPU API."""
    if backend == "hip":
        from ._hip import hip_devices

        return hip_devices()
    if backend in _FOREIGN_RUNTIMES:
        raise _foreign(backend)
    raise ValueError("Device discovery requires backend='hip'")


class NumpyBackend:
    """CPU reference backend: every operation is a NumPy call on host arrays.

    Storage is a flat C-order NumPy array; the array facade keeps the shape.
    """

    _is_tracing = False

    name = "numpy"
    device = "CPU (NumPy)"
    fp64 = True

    def validate_dtype(self, dtype):
        return check_dtype(dtype)

    def random_distributions(self, dtype):
        return ("random", "uniform", "normal", "exponential")

    def random_data(self, shape, dtype, distribution, seed, start, first, second):
        from ._philox import generate

        return generate(shape, dtype, distribution, seed, start, first, second)

    def upload(self, host):
        return np.array(host, copy=True, order="C").reshape(-1)

    def download(self, a):
        return a._data.reshape(a.shape).copy()

    def empty(self, shape, dtype):
        return np.empty(int(np.prod(shape, dtype=np.int64)), dtype=dtype)

    def full(self, shape, value, dtype):
        return np.full(int(np.prod(shape, dtype=np.int64)), value, dtype=dtype)

    def elementwise(self, name, args, shape, dtype):
        operands = [a._data.reshape(a.shape) for a in args]
        if name == "cast":
            result = operands[0].astype(dtype)
        else:
            with np.errstate(all="ignore"):
                result = getattr(np, name)(*operands)
        return np.array(np.broadcast_to(np.asarray(result, dtype=dtype), shape), copy=True).reshape(-1)

    def gather(self, a, shape, offset, strides):
        if not int(np.prod(shape, dtype=np.int64)):
            return np.empty(0, dtype=a.dtype)
        itemsize = a.dtype.itemsize
        view = np.lib.stride_tricks.as_strided(
            a._data[offset:], shape=shape, strides=tuple(s * itemsize for s in strides), writeable=False
        )
        return np.array(view, copy=True).reshape(-1)

    def reduce(self, a, axes, keepdims, dtype, *, operation="sum"):
        value = a._data.reshape(a.shape)
        if operation == "sum":
            result = np.sum(value, axis=axes, keepdims=keepdims, dtype=dtype)
            return np.asarray(result).reshape(-1)
        from ._reductions import numpy_extreme

        return numpy_extreme(value, axes, keepdims, operation)

    def matmul(self, a, b, shape, dtype):
        product = a._data.reshape(a.shape) @ b._data.reshape(b.shape)
        return np.asarray(product, dtype=dtype).reshape(-1)

    def norm(self, a, axes, keepdims, dtype):
        from ._norm_host import two_pass_norm

        return two_pass_norm(a._data.reshape(a.shape), axes, dtype)

    def synchronize(self):
        return None


_NUMPY = NumpyBackend()
_DEFAULT = ContextVar("openpacho_backend", default=_NUMPY)


@lru_cache(maxsize=8)
def _hip_backend(device):
    from ._hip import HIPBackend

    return HIPBackend(device)


class _Selection:
    """One get_backend request. resolve() tries each step in turn; a step
    returns the backend, raises, or returns None to pass the request on.

    Semantics follow reference backends.py:190-214 for the names this build
    provides ('numpy', 'hip'); the reference's other runtimes are reported as
    unavailable rather than unknown.
    """

    def __init__(self, target, device, blas, clblast_library):
        self.target, self.device, self.blas, self.clblast = target, device, blas, clblast_library

    def _configured(self):
        return any(option is not None for option in (self.device, self.blas, self.clblast))

    def resolve(self):
        for step in (self._owner, self._provider_options, self._default, self._instance, self._named):
            found = step()
            if found is not None:
                return found
        raise ValueError("backend must be 'numpy', 'hip', or a backend object")

    def _owner(self):
        """An array's backend, or a capture's trace backend, as they are."""
        from ._array import ndarray

        if isinstance(self.target, ndarray):
            owner, refusal = self.target._backend, "An array's backend cannot be reconfigured"
        elif getattr(self.target, "_is_tracing", False):
            owner, refusal = self.target, "Captured backend does not accept reconfiguration"
        else:
            return None
        if self._configured():
            raise ValueError(refusal)
        return owner

    def _provider_options(self):
        """BLAS options belong to 'hip' selected by name; a CLBlast library to
        a runtime this build does not have."""
        target = self.target
        if self.clblast is None and (self.blas is None or target == "hip"):
            return None
        if isinstance(target, str) and target in _FOREIGN_RUNTIMES:
            raise _foreign(target)
        if self.clblast is not None:
            raise ValueError("clblast_library requires backend='opencl'")
        raise ValueError("BLAS configuration requires backend='hip'")

    def _default(self):
        if self.target is not None:
            return None
        if self.device is not None:
            raise ValueError("device requires backend='hip'")
        return _DEFAULT.get()

    def _instance(self):
        if not (isinstance(self.target, NumpyBackend) or getattr(self.target, "name", None) == "hip"):
            return None
        if self.device is not None:
            raise ValueError("device cannot accompany an existing backend")
        return self.target

    def _named(self):
        if not isinstance(self.target, str):
            return None
        if self.target in _FOREIGN_RUNTIMES:
            raise _foreign(self.target)
        if self.target == "hip":
            if self.blas not in (None, "custom"):
                raise ValueError("The hip backend has one matrix provider, blas='custom'")
            return _hip_backend(None if self.device is None else str(self.device))
        if self.target == "numpy" and self.device is None:
            return _NUMPY
        return None


def get_backend(backend=None, *, device=None, blas=None, clblast_library=None):
    """Resolve a backend selection, or return an array's own backend."""
    return _Selection(backend, device, blas, clblast_library).resolve()


def set_backend(backend, *, device=None, blas=None, clblast_library=None):
    """Select the backend for new arrays in this execution context."""
    selected = get_backend(backend, device=device, blas=blas, clblast_library=clblast_library)
    _DEFAULT.set(selected)
    return selected


@contextmanager
def use_backend(backend, *, device=None, blas=None, clblast_library=None):
    selected = get_backend(backend, device=device, blas=blas, clblast_library=clblast_library)
    token = _DEFAULT.set(selected)
    try:
        yield selected
    finally:
        _DEFAULT.reset(token)


def synchronize(backend=None):
    get_backend(backend).synchronize()
