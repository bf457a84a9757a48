"""MI355X backend: the OpenPacho backend protocol on libpacho_hip.so.

Protocol (reference backends.py:82-150 and _cuda.py:129-679): ``name``,
``device``, ``fp64``, ``validate_dtype``, ``empty``, ``full``, ``upload``,
``download``, ``elementwise``, ``gather``, ``reduce``, ``matmul``, ``norm``,
``synchronize``, ``random_distributions``, ``random_data``, plus the optional
``create_lowering``, ``prepare_padded_matmul``, ``prepare_layout_matmul``,
``residual_matvec``,
``execution_scope``, ``release_cached_memory`` and ``close``.

Storage is an _Allocation (device pointer + capacity) from the library's
stream-ordered pool. All work of a backend runs on its single stream, so an
allocation may be returned while kernels that read it are still queued.
Returned blocks of the pool's smallest size class (0-d results, short
vectors) wait in a short host-side list for the next small request instead
of crossing into the library twice; pool statistics, releases and close()
hand that list back first. Operations never download or fall back
to the CPU: a missing library or device raises BackendUnavailableError and a
failing call raises.
"""

import ctypes
from collections import OrderedDict
from math import prod
from threading import RLock
import weakref

import numpy as np

from . import _hip_lib as lib_
from ._hip_lowering import BLOCK, HIPLowering, eager_source
from .backends import DeviceInfo, check_dtype
from .exceptions import BackendUnavailableError, UnsupportedDtypeError

_MAX_ELEMENTS = 2**31 - 1
_KERNEL_CACHE = 256
# Blocks up to the library pool's smallest size class (runtime.hip
# size_class: every request <= 512 bytes gets a 512-byte block) are
# interchangeable; at most _SMALL_KEPT of them wait on the host for reuse.
_SMALL_BLOCK = 512
_SMALL_KEPT = 64
_C_SCALARS = {
    np.dtype("bool"): ctypes.c_uint8,
    np.dtype("int32"): ctypes.c_int32,
    np.dtype("int64"): ctypes.c_int64,
    np.dtype("uint32"): ctypes.c_uint32,
    np.dtype("uint64"): ctypes.c_uint64,
    np.dtype("float32"): ctypes.c_float,
    np.dtype("float64"): ctypes.c_double,
}


def hip_devices():
    """DeviceInfo for every visible HIP device."""
    lib = lib_.load()
    count = ctypes.c_int(0)
    lib_.check(lib, lib.hp_device_count(ctypes.byref(count)), "hp_device_count")
    found = []
    for index in range(count.value):
        name = ctypes.create_string_buffer(256)
        arch = ctypes.create_string_buffer(256)
        total = ctypes.c_int64(0)
        units = ctypes.c_int(0)
        fp64 = ctypes.c_int(0)
        status = lib.hp_device_info(
            index, name, 256, arch, 256, ctypes.byref(total), ctypes.byref(units), ctypes.byref(fp64)
        )
        lib_.check(lib, status, "hp_device_info")
        found.append(
            DeviceInfo(
                str(index),
                name.value.decode(errors="replace"),
                "AMD",
                "GPU",
                bool(fp64.value),
                int(total.value),
                f"{arch.value.decode(errors='replace')} / {lib.hp_version().decode()}",
            )
        )
    return found


class _Allocation:
    """Device storage owned by one backend; returned to the pool when dropped."""

    __slots__ = ("backend", "ptr", "capacity", "__weakref__")

    def __init__(self, backend, ptr, capacity):
        self.backend = backend
        self.ptr = int(ptr)
        self.capacity = capacity
        backend._lease(self)

    def __del__(self):
        try:
            if self.ptr:
                ptr, self.ptr = self.ptr, 0
                self.backend._release(ptr, self.capacity)
        except Exception:  # noqa: BLE001 - interpreter shutdown only
            pass


def _collapse(shape, strides):
    """Merge adjacent axes that are contiguous with each other (for gathers)."""
    dims = [(d, s) for d, s in zip(shape, strides) if d != 1]
    if not dims:
        return (1,), (0,)
    merged = [list(dims[0])]
    for d, s in dims[1:]:
        if merged[-1][1] == s * d:
            merged[-1][0] *= d
            merged[-1][1] = s
        else:
            merged.append([d, s])
    return tuple(m[0] for m in merged), tuple(m[1] for m in merged)


class _Active:
    """The backend lock, refused once the backend is closed.

    A plain context manager: entering it costs a lock acquire, where a
    generator-based one costs a generator per operation on the dispatch path.
    """

    __slots__ = ("_backend",)

    def __init__(self, backend):
        self._backend = backend

    def __enter__(self):
        backend = self._backend
        backend._lock.acquire()
        if backend._closed:
            backend._lock.release()
            raise RuntimeError("hip backend is closed")

    def __exit__(self, *exc):
        self._backend._lock.release()
        return False


class HIPBackend:
    name = "hip"
    blas = "custom"
    fp64 = True
    _is_tracing = False  # a class attribute: the facade probes it on every result
    # One fused step cannot amortise entering a scope; plans of >= 2 launches do.
    execution_scope_min_steps = 2

    def __init__(self, device=None):
        self._lib = lib_.load()
        self._lock = RLock()
        self._guard = _Active(self)
        # Weak references to the live allocations, zeroed by close(): plain
        # references in a list (a WeakSet entry costs a callback per
        # allocation), dead ones dropped whenever the list doubles.
        self._leases = []
        self._lease_prune_at = 1024
        self._small = []  # returned blocks of <= _SMALL_BLOCK bytes, still live in the library
        self._kernels = OrderedDict()
        self._ctx = None
        self._closed = False
        identifier = "0" if device is None else str(device)
        found = hip_devices()
        matches = [d for d in found if d.id == identifier]
        if not matches:
            raise BackendUnavailableError(f"HIP device {device!r} not found; call devices('hip')")
        self.device = matches[0].name
        self.device_info = matches[0]
        self._ordinal = int(identifier)
        ctx = ctypes.c_void_p()
        status = self._lib.hp_init(self._ordinal, ctypes.byref(ctx))
        if status:
            raise BackendUnavailableError(f"HIP initialization failed: {lib_.last_error(self._lib)}")
        self._ctx = ctx
        self._pool_limit = self.device_info.memory_bytes // 4  # hp_init's default
        # Bound once: the calls of the shortest operations are their cost.
        self._free = self._lib.hp_free
        self._dot = self._lib.hp_dot
        self._dot_new = self._lib.hp_dot_new

    # ---- plumbing ---------------------------------------------------------------

    def _call(self, name, *args):
        if self._closed:
            raise RuntimeError("hip backend is closed")
        status = getattr(self._lib, name)(self._ctx, *args)
        lib_.check(self._lib, status, name)

    def _active(self):
        return self._guard

    def execution_scope(self):
        """Hold the backend lock for one plan execution."""
        return self._active()

    def _lease(self, allocation):
        """Record a new allocation (called with the backend lock held)."""
        leases = self._leases
        leases.append(weakref.ref(allocation))
        if len(leases) >= self._lease_prune_at:
            self._leases = [ref for ref in leases if ref() is not None]
            self._lease_prune_at = max(1024, 2 * len(self._leases))

    def _release(self, ptr, capacity):
        with self._lock:
            if self._closed:
                return
            if capacity <= _SMALL_BLOCK and len(self._small) < _SMALL_KEPT:
                self._small.append(ptr)
            else:
                self._free(self._ctx, ptr)

    def _return_small(self):
        """Hand the host-side small blocks back to the library pool (called
        with the backend lock held)."""
        small, self._small = self._small, []
        for ptr in small:
            lib_.check(self._lib, self._free(self._ctx, ptr), "hp_free")

    def _launch(self, source, name, grid, operands, out):
        """Compile (cached) and launch an RTC kernel over operands + out."""
        with self._active():
            kernel = self._kernels.get(source)
            if kernel is None:
                handle = ctypes.c_void_p()
                self._call("hp_rtc_compile", source.encode(), name.encode(), ctypes.byref(handle))
                if len(self._kernels) >= _KERNEL_CACHE:
                    _, old = self._kernels.popitem(last=False)
                    self._lib.hp_rtc_release(self._ctx, old)
                kernel = self._kernels[source] = handle
            else:
                self._kernels.move_to_end(source)
            values = []
            for operand in operands:
                if getattr(operand, "_host_scalar", False):
                    values.append(_C_SCALARS[operand.dtype](operand._data.item()))
                else:
                    values.append(ctypes.c_void_p(operand._data.ptr))
            values.append(ctypes.c_void_p(out.ptr))
            pointers = (ctypes.c_void_p * len(values))(*(ctypes.addressof(v) for v in values))
            self._call("hp_rtc_launch", kernel, grid, BLOCK, 0, pointers)

    # ---- protocol: dtypes, storage, transfers --------------------------------------

    def validate_dtype(self, dtype):
        if isinstance(dtype, np.dtype) and dtype in lib_.DTYPE_CODES:
            return dtype  # already a supported, native-order dtype
        dtype = check_dtype(dtype)
        if dtype not in lib_.DTYPE_CODES:
            raise UnsupportedDtypeError(f"hip backend does not support {dtype}")
        return dtype

    def empty(self, shape, dtype):
        dtype = self.validate_dtype(dtype)
        count = prod(shape)
        if count > _MAX_ELEMENTS:
            raise ValueError("Array exceeds GPU indexing limits")
        capacity = max(1, count * dtype.itemsize)
        with self._active():
            if capacity <= _SMALL_BLOCK and self._small:
                return _Allocation(self, self._small.pop(), capacity)
            ptr = ctypes.c_void_p()
            self._call("hp_alloc", capacity, ctypes.byref(ptr))
            return _Allocation(self, ptr.value, capacity)

    def full(self, shape, value, dtype):
        dtype = self.validate_dtype(dtype)
        out = self.empty(shape, dtype)
        count = prod(shape)
        if count:
            bits = np.asarray(value, dtype=dtype).tobytes().ljust(8, b"\0")
            pattern = int.from_bytes(bits[:8], "little")
            with self._active():
                self._call("hp_fill", ctypes.c_void_p(out.ptr), count, dtype.itemsize, pattern)
        return out

    def upload(self, host):
        host = np.ascontiguousarray(host) if np.ndim(host) else np.asarray(host)
        out = self.empty(host.shape, host.dtype)
        if host.size:
            with self._active():
                self._call("hp_h2d", ctypes.c_void_p(out.ptr), ctypes.c_void_p(host.ctypes.data), host.nbytes)
        return out

    def download(self, a):
        out = np.empty(a.shape, a.dtype)
        with self._active():
            if not a._data.ptr:
                raise RuntimeError("array storage was released when its hip backend closed")
            self._call("hp_d2h", ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(a._data.ptr), out.nbytes)
        return out

    def synchronize(self):
        with self._active():
            self._call("hp_sync")

    def release_cached_memory(self):
        with self._active():
            self._return_small()
            self._call("hp_release_cached")

    @property
    def pool_limit(self):
        """Bytes of freed blocks the pool keeps for reuse (a quarter of device
        memory by default). Blocks larger than the limit are freed at once;
        lowering it frees cached blocks until the cache fits."""
        return self._pool_limit

    @pool_limit.setter
    def pool_limit(self, value):
        value = int(value)
        if value < 0:
            raise ValueError("pool limit must be non-negative")
        with self._active():
            self._return_small()
            self._call("hp_set_pool_limit", value)
        self._pool_limit = value

    def pool_stats(self):
        values = [ctypes.c_int64(0) for _ in range(4)]
        with self._active():
            self._return_small()
            self._call("hp_pool_stats", *(ctypes.byref(v) for v in values))
        keys = ("cached_bytes", "cached_items", "live_bytes", "live_items")
        return dict(zip(keys, (v.value for v in values)))

    # ---- protocol: elementwise and layout ------------------------------------------

    def elementwise(self, name, args, shape, dtype):
        dtype = self.validate_dtype(dtype)
        out = self.empty(shape, dtype)
        if prod(shape):
            source, grid = eager_source(name, args, shape, dtype)
            self._launch(source, "pacho_elementwise", grid, args, out)
        return out

    def gather(self, a, shape, offset, strides):
        out = self.empty(shape, a.dtype)
        if not prod(shape):
            return out
        dims, steps = _collapse(tuple(shape), tuple(strides))
        if len(dims) > 8:
            raise NotImplementedError("gather supports at most 8 non-contiguous axes")
        with self._active():
            self._call(
                "hp_gather",
                a.dtype.itemsize,
                ctypes.c_void_p(a._data.ptr),
                ctypes.c_void_p(out.ptr),
                offset,
                len(dims),
                lib_.int64_array(dims),
                lib_.int64_array(steps),
            )
        return out

    def _rows_view(self, a, axes):
        """(source ndarray, outer, reduced, inner) with ``axes`` as one middle block."""
        from ._array import ndarray

        shape = a.shape
        axes = tuple(axes)
        if not axes:
            return a, prod(shape), 1, 1
        if axes == tuple(range(axes[0], axes[-1] + 1)):
            outer = prod(shape[: axes[0]])
            reduced = prod(shape[axes[0] : axes[-1] + 1])
            inner = prod(shape[axes[-1] + 1 :])
            return a, outer, reduced, inner
        # Non-adjacent axes: gather the kept axes first and the reduced last.
        kept = tuple(i for i in range(len(shape)) if i not in axes)
        order = kept + axes
        strides = [prod(shape[i + 1 :]) for i in range(len(shape))]
        new_shape = tuple(shape[i] for i in order)
        data = self.gather(a, new_shape, 0, tuple(strides[i] for i in order))
        moved = ndarray._wrap(data, new_shape, a.dtype, self)
        return moved, prod(shape[i] for i in kept), prod(shape[i] for i in axes), 1

    def reduce(self, a, axes, keepdims, dtype, *, operation="sum"):
        from ._array import ndarray

        dtype = self.validate_dtype(dtype)
        if operation not in lib_.REDUCTIONS:
            raise ValueError(f"Unknown reduction operation: {operation}")
        boolean_sum = dtype.kind == "b" and operation == "sum"
        if boolean_sum:
            # NumPy's sum in bool is a logical or (so are the reference's OpenCL
            # kernels, _opencl.py:340-341): max over 0/1 bytes, False if empty.
            operation = "max"
        if a.dtype != dtype:
            cast = self.elementwise("cast", [a], a.shape, dtype)
            a = ndarray._wrap(cast, a.shape, dtype, self)
        source, outer, reduced, inner = self._rows_view(a, axes)
        if boolean_sum and not reduced:
            return self.full((outer * inner,), False, dtype)
        out = self.empty((outer * inner,), dtype)
        if outer * inner:
            with self._active():
                self._call(
                    "hp_reduce",
                    lib_.DTYPE_CODES[dtype],
                    lib_.REDUCTIONS[operation],
                    ctypes.c_void_p(source._data.ptr),
                    ctypes.c_void_p(out.ptr),
                    outer,
                    reduced,
                    inner,
                )
        return out

    # ---- protocol: products ---------------------------------------------------------

    def matmul(self, a, b, shape, dtype):
        dtype = np.dtype(dtype)
        code = lib_.DTYPE_CODES[dtype]
        k = a.shape[-1]
        out = self.empty(shape, dtype)
        if not prod(shape):
            return out
        if dtype.kind != "f":
            # Integer and bool products (hp_gemm's integer kernel): vectors are
            # 1-row / 1-column matrices of the same storage.
            m = 1 if a.ndim == 1 else a.shape[-2]
            n = 1 if b.ndim == 1 else b.shape[-1]
            a_batch = a.shape[:-2] if a.ndim > 1 else ()
            b_batch = b.shape[:-2] if b.ndim > 1 else ()
            self._gemm(code, a, b, out, m, n, k, np.broadcast_shapes(a_batch, b_batch), a_batch, b_batch)
            return out
        if b.ndim == 1:
            with self._active():
                if a.ndim == 1:
                    self._call("hp_dot", code, *self._ptrs(a, b, out), k)
                else:
                    rows = prod(a.shape[:-1])
                    self._call("hp_gemv", code, *self._ptrs(a, b, out), rows, k)
            return out
        m = 1 if a.ndim == 1 else a.shape[-2]
        n = b.shape[-1]
        batch = tuple(shape[: len(shape) - (1 if a.ndim == 1 else 2)])
        a_batch = a.shape[:-2] if a.ndim > 1 else ()
        self._gemm(code, a, b, out, m, n, k, batch, a_batch, b.shape[:-2])
        return out

    def vector_dot(self, a, b):
        """Storage of the 0-d a . b of two non-empty 1-D float vectors of one
        dtype and length. The result takes a small block waiting on the host
        when there is one (one library call: the launch), else the allocation
        and the launch are one call. A short dot costs its host calls, not its
        kernel."""
        dtype = a._dtype
        with self._lock:
            if self._closed:
                raise RuntimeError("hip backend is closed")
            small = self._small
            if small:
                block = small.pop()
                status = self._dot(self._ctx, lib_.DTYPE_CODES[dtype], a._data.ptr, b._data.ptr, block, a._shape[0])
                if status:
                    small.append(block)
                    lib_.check(self._lib, status, "hp_dot")
                return _Allocation(self, block, dtype.itemsize)
            ptr = ctypes.c_void_p()
            status = self._dot_new(self._ctx, lib_.DTYPE_CODES[dtype], a._data.ptr, b._data.ptr, a._shape[0], ptr)
            if status:
                lib_.check(self._lib, status, "hp_dot_new")
            return _Allocation(self, ptr.value, dtype.itemsize)

    def _gemm(self, code, a, b, out, m, n, k, batch, a_batch, b_batch):
        dims, a_strides, b_strides = self._batch_strides(batch, a_batch, m * k, b_batch, k * n)
        with self._active():
            self._call(
                "hp_gemm",
                code,
                *self._ptrs(a, b, out),
                m,
                n,
                k,
                len(dims),
                lib_.int64_array(dims),
                lib_.int64_array(a_strides),
                lib_.int64_array(b_strides),
            )

    @staticmethod
    def _ptrs(*arrays):
        return [ctypes.c_void_p(x.ptr if hasattr(x, "ptr") else x._data.ptr) for x in arrays]

    @staticmethod
    def _batch_strides(batch, a_batch, a_matrix, b_batch, b_matrix):
        """Per-dimension operand strides of the output batch (0 = broadcast)."""

        def strides(source, matrix):
            lead = len(batch) - len(source)
            result = []
            for axis in range(len(batch)):
                if axis < lead or source[axis - lead] == 1:
                    result.append(0)
                else:
                    result.append(prod(source[axis - lead + 1 :]) * matrix)
            return result

        sa, sb = strides(a_batch, a_matrix), strides(b_batch, b_matrix)
        # Merge adjacent batch axes that stay affine for both operands.
        dims, ra, rb = [], [], []
        for d, x, y in zip(batch, sa, sb):
            if d == 1:
                continue
            if dims and ra[-1] == x * d and rb[-1] == y * d:
                dims[-1] *= d
                ra[-1], rb[-1] = x, y
            else:
                dims.append(d)
                ra.append(x)
                rb.append(y)
        if len(dims) > 6:
            raise NotImplementedError("matmul supports at most 6 independent batch axes")
        return dims, ra, rb

    def residual_matvec(self, a, x, b):
        """``b - a @ x`` in one launch (plan step "residual_matvec")."""
        from ._hip_gemv import residual_matvec_data

        return residual_matvec_data(self, a, x, b)

    def prepare_layout_matmul(self, ashape, bshape, shape, dtype, *, transpose_a=False, transpose_b=False):
        """Plan for a product of private 2-D transposes (plan step "layout_matmul")."""
        from ._hip_layout import prepare

        return prepare(self, ashape, bshape, shape, dtype, transpose_a=transpose_a, transpose_b=transpose_b)

    def prepare_padded_matmul(self, ashape, bshape, shape, dtype):
        from ._hip_padding import prepare

        return prepare(self, ashape, bshape, shape, dtype)

    def pad_copy(self, array, shape):
        """Pad (with +0 words) or crop ``array`` into a new buffer of ``shape``."""
        shape = tuple(shape)
        if len(shape) != array.ndim or shape[:-2] != array.shape[:-2]:
            raise ValueError("padding copies keep the batch prefix and rank")
        if array.dtype.itemsize not in (4, 8):
            raise TypeError("padding copies move 4- or 8-byte words")
        out = self.empty(shape, array.dtype)
        if prod(shape):
            with self._active():
                self._call(
                    "hp_pad_copy",
                    array.dtype.itemsize,
                    ctypes.c_void_p(array._data.ptr),
                    ctypes.c_void_p(out.ptr),
                    prod(shape[:-2]),
                    array.shape[-2],
                    array.shape[-1],
                    shape[-2],
                    shape[-1],
                )
        return out

    def norm(self, a, axes, keepdims, dtype):
        dtype = self.validate_dtype(dtype)
        if dtype.kind != "f":
            raise UnsupportedDtypeError("norm requires float32 or float64")
        count = prod(d for i, d in enumerate(a.shape) if i not in axes)
        out = self.empty((count,), dtype)
        if not count:
            return out
        source, outer, reduced, inner = self._rows_view(a, axes)
        with self._active():
            self._call(
                "hp_norm",
                lib_.DTYPE_CODES[dtype],
                ctypes.c_void_p(source._data.ptr),
                ctypes.c_void_p(out.ptr),
                outer,
                reduced,
                inner,
            )
        return out

    # ---- protocol: random numbers ---------------------------------------------------

    def random_distributions(self, dtype):
        return ("random", "uniform", "normal", "exponential")

    def random_data(self, shape, dtype, distribution, seed, start, first, second):
        dtype = self.validate_dtype(dtype)
        out = self.empty(shape, dtype)
        count = prod(shape)
        if not count:
            return out
        first, second = dtype.type(first), dtype.type(second)
        upper = np.nextafter(second, first) if distribution == "uniform" else dtype.type(1)
        with self._active():
            self._call(
                "hp_philox",
                lib_.DTYPE_CODES[dtype],
                lib_.DISTRIBUTIONS[distribution],
                ctypes.c_void_p(out.ptr),
                count,
                seed,
                start,
                float(first),
                float(second),
                float(upper),
            )
        return out

    # ---- protocol: compilation and lifetime -------------------------------------------

    def create_lowering(self):
        return HIPLowering(self)

    def close(self):
        with self._lock:
            if self._closed:
                return
            for ref in self._leases:
                lease = ref()
                if lease is not None:
                    lease.ptr = 0
            self._leases = []
            self._small = []  # still live in the library: hp_destroy frees them
            for kernel in self._kernels.values():
                self._lib.hp_rtc_release(self._ctx, kernel)
            self._kernels.clear()
            if self._ctx is not None:
                self._lib.hp_destroy(self._ctx)
                self._ctx = None
            self._closed = True

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown only
            pass
