"""Pinning the restatements of the reference custom kernels and the exact oracles."""

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import exact, kernels, padding
from oracle import numpy_backend as nb

GOLDEN_NORM = Path(__file__).parent / "golden" / "reference_norm.npz"


# ---- exact oracles -----------------------------------------------------------------


def test_exact_dot_closed_forms():
    assert exact.exact_dot([1.0, 2.0, 3.0], [4.0, 5.0, 6.0]) == 32
    # Catastrophic cancellation: float arithmetic returns 0, the exact value is 1.
    a = np.array([2.0**60, 1.0, -(2.0**60)])
    b = np.array([1.0, 1.0, 1.0])
    assert float(np.dot(a, b)) == 0.0
    assert exact.exact_dot(a, b) == 1
    # Extreme binary exponents stay exact.
    assert exact.exact_dot([2.0**-1074, 2.0**1000], [2.0**1000, 2.0**-1074]) == Fraction(2, 2**74)
    x = np.float32(0.1)
    assert exact.exact_dot([x], [x]) == Fraction(*float(x).as_integer_ratio()) ** 2


def test_exact_norm_known_values_and_fsum_agreement():
    assert exact.norm_exact([3.0, 4.0]) == 5.0
    assert exact.norm_exact([5.0, 12.0]) == 13.0
    assert exact.norm_exact([1e300, 1e300]) == pytest.approx(1e300 * math.sqrt(2), rel=1e-16)
    assert exact.norm_exact([1e-300] * 4) == pytest.approx(2e-300, rel=1e-16)
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, 1000).astype(np.float32)
    # float32 squares are exact in float64; fsum is correctly rounded.
    fsum = math.sqrt(math.fsum(float(v) * float(v) for v in x))
    assert exact.norm_exact(x) == pytest.approx(fsum, rel=2e-16)


def test_product_bound_ratio_accepts_float_sums_and_rejects_planted_mistakes():
    rng = np.random.default_rng(12)
    for dtype, unit in ((np.float32, 4e-7), (np.float64, 8e-16)):
        a = rng.uniform(-1, 1, (37, 300)).astype(dtype)
        b = rng.uniform(-1, 1, (300, 23)).astype(dtype)
        # The sequential working-precision loop (the reference kernel's order)
        # and the working-precision BLAS product lie inside the bound.
        assert exact.product_bound_ratio(a, b, kernels.gemm_sequential_rows(a, b), unit, block=8) <= 1
        assert exact.product_bound_ratio(a, b, a @ b, unit, block=5) <= 1
        good = (a.astype(np.float64) @ b.astype(np.float64)).astype(dtype)
        # One output off in its last few bits of float32 stays inside; one
        # dropped term, a transposed operand or a NaN falls out.
        dropped = good.copy()
        dropped[36, 22] -= a[36, 299] * b[299, 22]
        assert exact.product_bound_ratio(a, b, dropped, unit, block=8) > 1
        square = rng.uniform(-1, 1, (40, 40)).astype(dtype)
        assert exact.product_bound_ratio(square, square, square.T @ square, unit) > 1
        poisoned = good.copy()
        poisoned[0, 0] = np.nan
        assert exact.product_bound_ratio(a, b, poisoned, unit) == math.inf


def test_extended_norm_matches_exact_on_extreme_inputs():
    rng = np.random.default_rng(11)
    x = 10.0 ** rng.uniform(-300, 300, 2000) * (rng.integers(0, 2, 2000) * 2 - 1)
    assert float(exact.norm_extended(x)) == pytest.approx(exact.norm_exact(x), rel=1e-18)
    rows = rng.uniform(-1, 1, (4, 300))
    got = exact.norm_extended(rows, axis=1).reshape(-1)
    for r in range(4):
        assert float(got[r]) == pytest.approx(exact.norm_exact(rows[r]), rel=1e-18)


# ---- reference custom-kernel restatements -----------------------------------------------


def test_gemm_sequential_is_the_sequential_float32_loop():
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (5, 37)).astype(np.float32)
    b = rng.uniform(-1, 1, (37, 6)).astype(np.float32)
    rows, cols = np.meshgrid(range(5), range(6), indexing="ij")
    got = kernels.gemm_sequential(a, b, rows.ravel(), cols.ravel()).reshape(5, 6)
    for i in range(5):
        for j in range(6):
            acc = np.float32(0)
            for k in range(37):
                acc = np.float32(acc + np.float32(a[i, k] * b[k, j]))
            assert got[i, j] == acc
    # Exactly representable terms: any order gives the exact integer result.
    ints = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert kernels.gemm_sequential(ints, ints.T.copy(), [2], [1])[0] == float(ints[2] @ ints[1])


def test_gemm_sequential_rows_is_the_sampled_order_on_every_coordinate():
    rng = np.random.default_rng(2)
    for dtype in (np.float32, np.float64):
        a = rng.uniform(-1, 1, (7, 129)).astype(dtype)
        b = rng.uniform(-1, 1, (129, 11)).astype(dtype)
        rows, cols = np.meshgrid(range(7), range(11), indexing="ij")
        sampled = kernels.gemm_sequential(a, b, rows.ravel(), cols.ravel()).reshape(7, 11)
        block = kernels.gemm_sequential_rows(a, b)
        assert block.dtype == dtype
        np.testing.assert_array_equal(block.view(np.uint8), sampled.view(np.uint8))
    # A transposed operand or a dropped product would change the exact
    # integer result of a non-symmetric case.
    left = np.arange(6, dtype=np.float32).reshape(2, 3)
    right = np.arange(12, dtype=np.float32).reshape(3, 4) - 5
    np.testing.assert_array_equal(kernels.gemm_sequential_rows(left, right), left.astype(np.float64) @ right)


def test_gemv_lanes_order_and_exact_cases():
    x = np.arange(1, 301, dtype=np.float64)
    assert kernels.gemv_lanes(x, np.ones(300)) == 300 * 301 / 2
    a = np.zeros((5, 257), np.float32)
    v = np.zeros(257, np.float32)
    a[0, :4] = [4096, -4096, 3, -3]
    v[:4] = 1
    a[1, 20], v[20] = 2.0**60, 2.0**-60
    got = kernels.gemv_lanes(a, v)
    assert got[0] == 0 and got[1] == 1
    # Brute force of the documented order on a small vector: lane sums then tree.
    rng = np.random.default_rng(3)
    y = rng.uniform(-1, 1, 300).astype(np.float32)
    lanes = [np.float32(0)] * 128
    for j in range(300):
        lanes[j % 128] = np.float32(lanes[j % 128] + np.float32(y[j] * y[j]))
    step = 64
    while step:
        for lane in range(step):
            lanes[lane] = np.float32(lanes[lane] + lanes[lane + step])
        step //= 2
    assert kernels.gemv_lanes(y, y) == lanes[0]


def test_long_dot_uses_1024_term_chunks_then_reduce():
    rng = np.random.default_rng(9)
    x = rng.uniform(-1, 1, 9001).astype(np.float32)
    chunks = [kernels.gemv_lanes(x[i : i + 1024], x[i : i + 1024]) for i in range(0, 9001, 1024)]
    assert kernels.gemv_lanes(x, x) == kernels.reduce_lanes(np.array(chunks, np.float32))
    assert kernels.gemv_lanes(x, x) == pytest.approx(float(x.astype(np.float64) @ x), rel=1e-5)


@pytest.mark.parametrize(
    "values,expected",
    [([0.0, 0.0], 0.0), ([np.inf, 1.0], np.inf), ([np.nan, np.inf], np.nan), ([-3.0, 4.0], 5.0)],
)
def test_pair_merge_special_values(values, expected):
    got = kernels.norm_pair_merge(np.asarray(values, np.float64))
    assert math.isnan(got) if math.isnan(expected) else got == expected


@pytest.mark.parametrize("dtype,small,large", [(np.float32, 1e-25, 1e25), (np.float64, 1e-200, 1e200)])
@pytest.mark.parametrize("length", [2, 4099, 8193])
def test_pair_merge_extreme_constants_and_chunk_passes(dtype, small, large, length):
    for scale in (small, large):
        x = np.full(length, scale, dtype)
        got = kernels.norm_pair_merge(x)
        want = abs(float(dtype(scale))) * math.sqrt(length)
        assert float(got) == pytest.approx(want, rel=2e-6)


def test_pair_merge_error_against_exact_is_small():
    rng = np.random.default_rng(2)
    x = (10.0 ** rng.uniform(-30, 30, 5000) * (rng.integers(0, 2, 5000) * 2 - 1)).astype(np.float32)
    ref = exact.norm_exact(x)
    assert abs(float(kernels.norm_pair_merge(x)) - ref) / ref < 2e-6


def test_reduce_lanes_matches_sum_for_exact_terms():
    assert kernels.reduce_lanes(np.ones(10000, np.float32)) == 10000
    assert kernels.reduce_lanes(np.arange(5000, dtype=np.float64)) == 5000 * 4999 / 2


# ---- NumPy-backend norm against the reference's own outputs ------------------------------


def test_numpy_backend_norm_reproduces_reference_golden():
    with np.load(GOLDEN_NORM) as data:
        golden = {k: data[k] for k in data.files}
    for dtype in ("float32", "float64"):
        x = golden[f"loguniform|{dtype}|input"]
        np.testing.assert_allclose(nb.norm(x), golden[f"loguniform|{dtype}|norm"], rtol=1e-6 if dtype == "float32" else 1e-15)
        cube = golden[f"cube|{dtype}|input"]
        for axis in ((2, 0), 1, None):
            key = "none" if axis is None else str(axis)
            np.testing.assert_allclose(
                nb.norm(cube, axis=axis, keepdims=True), golden[f"cube|{dtype}|axis={key}"], rtol=1e-6
            )
        rows = golden[f"rows|{dtype}|input"]
        np.testing.assert_allclose(nb.norm(rows, axis=1), golden[f"rows|{dtype}|norm"], rtol=1e-6)
        # The reference values themselves sit within float rounding of the exact norm.
        ref = exact.norm_exact(x)
        assert abs(float(golden[f"loguniform|{dtype}|norm"]) - ref) / ref < (2e-6 if dtype == "float32" else 1e-14)


# ---- padding plan closed form ----------------------------------------------------------


def test_padding_closed_form_matches_reference_worked_values():
    p = padding.plan((33, 17), (17, 65))
    assert p["padded_input_shapes"] == ((64, 32), (32, 96))
    assert p["padded_output_shape"] == (64, 96)
    assert p["scratch_bytes"] == 45056 and p["copy_dispatches"] == 3 and p["dispatch_count"] == 4
    p = padding.plan((2, 1, 33, 17), (1, 3, 17, 65))
    assert p["padded_input_shapes"] == ((2, 1, 64, 32), (1, 3, 32, 96))
    assert p["padded_output_shape"] == (2, 3, 64, 96)
    p = padding.plan((64, 32), (32, 96))
    assert p["scratch_bytes"] == 0 and p["dispatch_count"] == 1
    assert padding.plan((4097, 3001), (3001, 2049))["scratch_bytes"] == 109_039_616
    for a, b in [((31, 16), (16, 32)), ((0, 32), (32, 96))]:
        assert padding.plan(a, b) is None
    assert padding.plan((33, 17), (17, 65), "float64") is None


# ---- brute-force scalar restatements of the reference kernels' loops -------------------
# These walk lanes, chunks and tree steps one scalar at a time, in the order
# of reference _norm.py:62-118 (with _merge :28-36) and _cuda.py:466-485, with
# NumPy scalars of the kernel's dtype (every operation rounds once). The
# vectorised oracles must reproduce them bit for bit.


def _scalar_merge(dt, s, t, v, w):
    if np.isnan(s) or np.isnan(v):
        s = dt(s + v)
        return s, s
    if np.isinf(v):
        return v, dt(1)
    if not np.isinf(s) and v > dt(0):
        if s < v:
            z = dt(s / v)
            return v, dt(w + dt(dt(t * z) * z))
        z = dt(v / s)
        return s, dt(t + dt(dt(w * z) * z))
    return s, t


def _scalar_norm_kernel(values):
    dt = values.dtype.type
    current = [(abs(v), dt(1)) for v in values]
    while True:
        reduced = len(current)
        chunks = (reduced + 4095) // 4096
        out = []
        for chunk in range(chunks):
            scales, sums = [dt(0)] * 128, [dt(0)] * 128
            for lane in range(128):
                s, t = dt(0), dt(0)
                for j in range(lane, min(4096, reduced - chunk * 4096), 128):
                    v, w = current[chunk * 4096 + j]
                    s, t = _scalar_merge(dt, s, t, v, w)
                scales[lane], sums[lane] = s, t
            step = 64
            while step:
                for lane in range(step):
                    scales[lane], sums[lane] = _scalar_merge(dt, scales[lane], sums[lane], scales[lane + step], sums[lane + step])
                step //= 2
            out.append((scales[0], sums[0]))
        if chunks == 1:
            return out[0]
        current = out


def _scalar_reduce_kernel(values):
    dt = values.dtype.type
    current = list(values)
    while True:
        reduced = len(current)
        chunks = (reduced + 4095) // 4096
        partial = []
        for chunk in range(chunks):
            sums = []
            for lane in range(128):
                acc = dt(0)
                for r in range(chunk * 4096 + lane, min((chunk + 1) * 4096, reduced), 128):
                    acc = dt(acc + current[r])
                sums.append(acc)
            step = 64
            while step:
                for lane in range(step):
                    sums[lane] = dt(sums[lane] + sums[lane + step])
                step //= 2
            partial.append(sums[0])
        if chunks == 1:
            return partial[0]
        current = partial


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_pair_merge_matches_the_scalar_kernel_loop(dtype):
    rng = np.random.default_rng(31)
    cases = [
        rng.uniform(-1, 1, 300),
        10.0 ** rng.uniform(-30, 30, 300) * rng.choice([-1, 1], 300),
        np.concatenate([np.zeros(40), rng.normal(size=200), [0.0] * 7]),
        rng.normal(size=2 * 4096 + 77),  # two chunks, then a second pass over the pairs
        10.0 ** rng.uniform(-20, 20, 3 * 4096 + 1),
    ]
    for values in cases:
        values = values.astype(dtype)
        want_s, want_t = _scalar_norm_kernel(values)
        got_s, got_t = kernels.norm_pair_state(values)
        assert got_s.dtype == dtype and got_t.dtype == dtype
        assert (got_s.tobytes(), got_t.tobytes()) == (dtype(want_s).tobytes(), dtype(want_t).tobytes())
        with np.errstate(all="ignore"):
            assert kernels.norm_pair_merge(values).tobytes() == dtype(want_s * dtype(np.sqrt(want_t))).tobytes()
    special = np.ones(300, dtype)
    special[17], special[250] = np.inf, np.nan
    assert np.isnan(kernels.norm_pair_merge(special)) and np.isnan(_scalar_norm_kernel(special)[0])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_reduce_lanes_matches_the_scalar_kernel_loop(dtype):
    rng = np.random.default_rng(32)
    for n in (1, 127, 300, 4096, 4097, 2 * 4096 + 300, 3 * 4096 * 2 + 5):
        values = (rng.normal(size=n) * 10.0 ** rng.uniform(-3, 3, n)).astype(dtype)
        want = _scalar_reduce_kernel(values)
        got = kernels.reduce_lanes(values)
        assert np.asarray(got).tobytes() == dtype(want).tobytes(), n
