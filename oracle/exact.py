"""TEST INFRASTRUCTURE ONLY - exact and extended-precision references.

- exact_dot: the exact value of sum(a_i * b_i) for finite binary floats, as a
  Fraction (every float is a dyadic rational; integer arithmetic is exact).
  Follows the method of reference benchmarks/gemm_precision_oracle.py:27-93
  (exact dyadic sums), re-derived here with Python integers.
- float64_matmul_rows: fp64 recomputation from the rounded fp32 inputs (the
  "higher precision" oracle of reference benchmarks/numerical_metrics.py:45-96).
- product_bound_ratio: the same recomputation over every output of a 2-D
  product in row blocks, against the elementwise forward-error bound of a
  K-term sum (used for full-output checks of config-size products).
- norm_extended: the Euclidean norm in x86 80-bit long double with two-pass
  power-of-two scaling (64-bit significand, exponent range covers squares of
  1e+-300), used for full-size fp64 norms.
- norm_exact: exact sum of squares with integers, square root rounded once.
Pinned by tests/test_oracle_kernels.py (closed forms, Pythagorean triples,
cancellation cases whose exact value is known, agreement with math.fsum).
"""

import math
from fractions import Fraction

import numpy as np


def _ratio(value):
    num, den = float(value).as_integer_ratio()
    return num, den


def exact_dot(a, b):
    """Exact sum(a[i] * b[i]) as a Fraction (a, b finite 1-D float arrays)."""
    # Common denominator: products of two binary64 values are multiples of
    # 2**-2148; scale every product to that unit and add integers.
    unit = 2**2148
    total = 0
    for x, y in zip(np.asarray(a, dtype=np.float64).tolist(), np.asarray(b, dtype=np.float64).tolist()):
        nx, dx = _ratio(x)
        ny, dy = _ratio(y)
        total += nx * ny * (unit // (dx * dy))
    return Fraction(total, unit)


def relative_error(value, exact):
    """|value - exact| / |exact| (exact a Fraction); inf/nan aware."""
    value = float(value)
    if not math.isfinite(value):
        return math.inf
    if exact == 0:
        return 0.0 if value == 0 else math.inf
    return float(abs(Fraction(value) - exact) / abs(exact))


def float64_matmul_rows(a, b, rows):
    """float64 product rows a[rows] @ b from the rounded inputs."""
    return np.asarray(a[rows], dtype=np.float64) @ np.asarray(b, dtype=np.float64)


def product_bound_ratio(a, b, got, unit, block=1024):
    """Largest |got - a @ b| / (unit * sqrt(k) * 4 * (|a| @ |b|)) over EVERY
    output of a 2-D product, with a @ b and |a| @ |b| in float64 from the
    rounded inputs, computed in row blocks of `block` (8192^3 needs two
    float64 products, not a float64 copy of C). A value <= 1 means every
    output lies within the elementwise forward-error bound of a K-term sum in
    the working precision (unit = 4e-7 for float32, 8e-16 for float64); an
    output that is NaN, infinite or wrong by O(1) gives inf or >> 1.
    """
    a = np.asarray(a)
    b64 = np.asarray(b, dtype=np.float64)
    babs = np.abs(b64)
    got = np.asarray(got)
    k = a.shape[1]
    worst = 0.0
    for r0 in range(0, a.shape[0], block):
        rows = np.asarray(a[r0 : r0 + block], dtype=np.float64)
        want = rows @ b64
        scale = np.abs(rows) @ babs
        bound = unit * math.sqrt(k) * 4 * scale + 1e-30
        err = np.abs(np.asarray(got[r0 : r0 + block], dtype=np.float64) - want)
        if not np.all(np.isfinite(err)):
            return math.inf
        worst = max(worst, float(np.max(err / bound)) if err.size else 0.0)
    return worst


def norm_extended(x, axis=None):
    """Two-pass power-of-two scaled norm in np.longdouble (chunked when flat)."""
    x = np.asarray(x)
    ld = np.longdouble
    if axis is None:
        scale = np.max(np.abs(x)) if x.size else 0
        if np.isnan(scale):
            return np.array(np.nan, ld)
        if np.isinf(scale):
            return np.array(np.inf, ld)
        if scale == 0:
            return np.array(0, ld)
        exponent = int(np.floor(np.log2(float(scale))))
        total = ld(0)
        flat = x.reshape(-1)
        for base in range(0, flat.size, 1 << 22):
            part = np.ldexp(flat[base : base + (1 << 22)].astype(ld), -exponent)
            total += np.sum(part * part, dtype=ld)
        return np.array(np.ldexp(np.sqrt(total), exponent), ld)
    scale = np.max(np.abs(x), axis=axis, keepdims=True).astype(ld)
    with np.errstate(all="ignore"):
        finite = (scale > 0) & np.isfinite(scale)
        exponent = np.where(finite, np.floor(np.log2(np.where(finite, scale, 1))), 0).astype(np.int64)
        scaled = np.ldexp(x.astype(ld), -exponent)
        total = np.sum(scaled * scaled, axis=axis, keepdims=True, dtype=ld)
        result = np.ldexp(np.sqrt(total), exponent)
    result = np.where(np.isinf(scale), np.inf, result)
    return np.where(np.isnan(scale), np.nan, result)


def sum_of_squares_exact(x):
    """Exact sum(x_i^2) of a finite 1-D float array, as a Fraction."""
    unit = 2**2148
    acc = 0
    for v in np.asarray(x, dtype=np.float64).tolist():
        n, d = _ratio(v)
        acc += n * n * (unit // (d * d))
    return Fraction(acc, unit)


def sqrt_fraction(total):
    """sqrt of a nonnegative Fraction, rounded once to binary64 (via 80+ exact bits)."""
    if total == 0:
        return 0.0
    num, den = total.numerator, total.denominator
    magnitude = num.bit_length() - den.bit_length()
    shift = 80 - magnitude // 2  # root keeps about 80 significant bits
    if shift >= 0:
        root = math.isqrt((num << (2 * shift)) // den)
        return float(Fraction(root, 1 << shift))
    root = math.isqrt(num // (den << (-2 * shift)))
    return float(root << -shift)


def norm_exact(x):
    """Exact-squares Euclidean norm of a finite 1-D array, as a float64."""
    return sqrt_fraction(sum_of_squares_exact(x))
