"""TEST INFRASTRUCTURE ONLY - Philox4x32-10 stream oracle (NumPy + C).

Restates reference src/openpacho/_random.py:19-31 (block function) and
:34-58 (_numpy_data: per-element counters, unit conversion, transforms).
Pinned by: the Random123 known-answer vectors (reference tests/test_random.py:
27-41), agreement of the NumPy and C restatements, the counter-carry cases of
test_random.py:93-103, and golden samples written from the reference NumPy
backend (tests/golden/).
"""

import ctypes
from pathlib import Path

import numpy as np

_MULT = (0xD2511F53, 0xCD9E8D57)
_WEYL = (0x9E3779B9, 0xBB67AE85)
_MASK = 0xFFFFFFFF


def block_int(counter, key):
    """Pure-Python block function on ints (small cases; _random.py:19-31)."""
    c0, c1, c2, c3 = (int(w) & _MASK for w in counter)
    k0, k1 = (int(w) & _MASK for w in key)
    for _ in range(10):
        p0, p1 = c0 * _MULT[0], c2 * _MULT[1]
        c0, c1, c2, c3 = (p1 >> 32) ^ c1 ^ k0, p1 & _MASK, (p0 >> 32) ^ c3 ^ k1, p0 & _MASK
        k0, k1 = (k0 + _WEYL[0]) & _MASK, (k1 + _WEYL[1]) & _MASK
    return c0, c1, c2, c3


def words(count, seed, start):
    """(count, 4) uint32 words for counters start..start+count-1 (NumPy)."""
    idx = np.arange(count, dtype=np.uint64) + np.uint64(start)
    c = [idx & np.uint64(_MASK), idx >> np.uint64(32), np.zeros(count, np.uint64), np.zeros(count, np.uint64)]
    k0, k1 = seed & _MASK, seed >> 32
    m0, m1 = np.uint64(_MULT[0]), np.uint64(_MULT[1])
    for _ in range(10):
        p0, p1 = c[0] * m0, c[2] * m1
        c = [
            (p1 >> np.uint64(32)) ^ c[1] ^ np.uint64(k0),
            p1 & np.uint64(_MASK),
            (p0 >> np.uint64(32)) ^ c[3] ^ np.uint64(k1),
            p0 & np.uint64(_MASK),
        ]
        k0, k1 = (k0 + _WEYL[0]) & _MASK, (k1 + _WEYL[1]) & _MASK
    return np.stack(c, axis=1).astype(np.uint32)


def unit(dtype, w_a, w_b):
    """_random.py:43-45 unit conversion from two uint32 word arrays."""
    a, b = np.asarray(w_a, np.uint64), np.asarray(w_b, np.uint64)
    if np.dtype(dtype) == np.float32:
        return (a >> np.uint64(8)).astype(np.float32) * np.float32(2.0**-24)
    return ((a >> np.uint64(5)).astype(np.float64) * 67108864.0 + (b >> np.uint64(6)).astype(np.float64)) * 2.0**-53


def samples(distribution, dtype, count, seed, start, first, second):
    """_random.py:34-58: one distribution's samples (NumPy, float transforms)."""
    dtype = np.dtype(dtype)
    first, second = dtype.type(first), dtype.type(second)
    w = words(count, seed, start)
    u = unit(dtype, w[:, 0], w[:, 1])
    with np.errstate(all="ignore"):
        if distribution == "random":
            return u
        if distribution == "uniform":
            return np.clip(first + (second - first) * u, first, np.nextafter(second, first))
        nl = -np.log1p(-u)
        if distribution == "exponential":
            return second * nl
        angle = dtype.type(2 * np.pi) * unit(dtype, w[:, 2], w[:, 3])
        return first + second * (np.sqrt(dtype.type(-2) * np.log1p(-u)) * np.cos(angle))


# ---- C restatement (fast, for full-size bit-exact checks) -------------------------

_LIB = None


def c_library():
    """Load oracle/_build/libphilox_oracle.so (built by oracle/Makefile)."""
    global _LIB
    if _LIB is None:
        path = Path(__file__).resolve().parent / "_build" / "libphilox_oracle.so"
        if not path.exists():
            raise FileNotFoundError(f"{path} missing; run `make -C oracle`")
        lib = ctypes.CDLL(str(path))
        u32p = ctypes.POINTER(ctypes.c_uint32)
        lib.oracle_philox_block.argtypes = [u32p, u32p, u32p]
        lib.oracle_philox_words.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64]
        for name, real in (("oracle_uniform_f32", ctypes.c_float), ("oracle_uniform_f64", ctypes.c_double)):
            getattr(lib, name).argtypes = [
                ctypes.c_void_p,
                ctypes.c_int64,
                ctypes.c_uint64,
                ctypes.c_uint64,
                ctypes.c_int,
                real,
                real,
                real,
            ]
        _LIB = lib
    return _LIB


def c_block(counter, key):
    lib = c_library()
    c = (ctypes.c_uint32 * 4)(*counter)
    k = (ctypes.c_uint32 * 2)(*key)
    out = (ctypes.c_uint32 * 4)()
    lib.oracle_philox_block(c, k, out)
    return tuple(out)


def c_words(count, seed, start):
    out = np.empty((count, 4), np.uint32)
    c_library().oracle_philox_words(out.ctypes.data, count, seed, start)
    return out


def c_uniform(dtype, count, seed, start, distribution="random", low=0.0, high=1.0):
    """Bit-exact 'random'/'uniform' samples from the C restatement."""
    dtype = np.dtype(dtype)
    low, high = dtype.type(low), dtype.type(high)
    upper = np.nextafter(high, low)
    out = np.empty(count, dtype)
    dist = 0 if distribution == "random" else 1
    fn = c_library().oracle_uniform_f32 if dtype == np.float32 else c_library().oracle_uniform_f64
    fn(out.ctypes.data, count, seed, start, dist, float(low), float(high), float(upper))
    return out
