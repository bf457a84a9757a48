"""Philox4x32-10 on the host, for the NumPy backend's random arrays.

Algorithm: Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
1, 2, 3" (SC11), four 32-bit words, ten rounds, multipliers 0xD2511F53 and
0xCD9E8D57, Weyl key increments 0x9E3779B9 and 0xBB67AE85.

Stream contract (reference _random.py:19-58): output element i uses the
counter block (lo32(start+i), hi32(start+i), 0, 0) under the key
(lo32(seed), hi32(seed)); the unit value is (w0 >> 8) * 2^-24 for float32 and
((w0 >> 5) * 2^26 + (w1 >> 6)) * 2^-53 for float64, and the distributions
transform it exactly as the device kernels do.
"""

import numpy as np

_M0 = np.uint64(0xD2511F53)
_M1 = np.uint64(0xCD9E8D57)
_LOW = np.uint64(0xFFFFFFFF)
_SHIFT = np.uint64(32)
_WEYL = (0x9E3779B9, 0xBB67AE85)
_CHUNK = 1 << 16


def philox_blocks(counter_lo, counter_hi, key_lo, key_hi):
    """Ten rounds on arrays of 32-bit counter words (c2 = c3 = 0)."""
    x0 = np.asarray(counter_lo, dtype=np.uint64)
    x1 = np.asarray(counter_hi, dtype=np.uint64)
    x2 = np.zeros_like(x0)
    x3 = np.zeros_like(x0)
    k0, k1 = int(key_lo), int(key_hi)
    for _ in range(10):
        left = x0 * _M0
        right = x2 * _M1
        x0, x1, x2, x3 = (
            (right >> _SHIFT) ^ x1 ^ np.uint64(k0),
            right & _LOW,
            (left >> _SHIFT) ^ x3 ^ np.uint64(k1),
            left & _LOW,
        )
        k0 = (k0 + _WEYL[0]) & 0xFFFFFFFF
        k1 = (k1 + _WEYL[1]) & 0xFFFFFFFF
    return x0, x1, x2, x3


def _unit(dtype, hi_word, lo_word):
    if dtype == np.float32:
        return (hi_word >> np.uint64(8)).astype(np.float32) * np.float32(2.0**-24)
    mantissa = (hi_word >> np.uint64(5)).astype(np.float64) * 67108864.0 + (lo_word >> np.uint64(6)).astype(
        np.float64
    )
    return mantissa * 2.0**-53


def generate(shape, dtype, distribution, seed, start, first, second):
    """Host samples for one generator call (flat C-order storage)."""
    dtype = np.dtype(dtype)
    count = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    out = np.empty(count, dtype)
    first, second = dtype.type(first), dtype.type(second)
    if distribution == "uniform":
        upper = np.nextafter(second, first)
    key_lo, key_hi = seed & 0xFFFFFFFF, seed >> 32
    for base in range(0, count, _CHUNK):
        n = min(_CHUNK, count - base)
        counters = np.arange(n, dtype=np.uint64) + np.uint64(start + base)
        w0, w1, w2, w3 = philox_blocks(counters & _LOW, counters >> _SHIFT, key_lo, key_hi)
        u = _unit(dtype, w0, w1)
        if distribution == "random":
            values = u
        elif distribution == "uniform":
            values = np.minimum(np.maximum(first + (second - first) * u, first), upper)
        else:
            with np.errstate(all="ignore"):
                nl = -np.log1p(-u)
                if distribution == "exponential":
                    values = second * nl
                else:
                    angle = dtype.type(2 * np.pi) * _unit(dtype, w2, w3)
                    values = first + second * (np.sqrt(dtype.type(2) * nl) * np.cos(angle))
        out[base : base + n] = values
    return out
