"""GPU parity of GEMV/DOT (hp_gemv / hp_dot) against fp64 and exact oracles.

Shapes and tolerances follow reference tests/test_cuda_gemv.py:133-222; the
full-size case is BASELINE.json config 2 (16384^2 float32, x ~ N(0,1), seed 1)
with the hip error bounded by 2x the error of the reference cooperative
kernel's arithmetic order (oracle.kernels.gemv_lanes).
"""

from fractions import Fraction

import numpy as np
import pytest

import openpacho as p
from oracle import exact, kernels

pytestmark = pytest.mark.gpu

SHAPES = [(33, 17), (129, 67), (33, 255), (33, 256), (33, 257), (513, 1023), (3, 4099), (2, 3, 257), (2, 1, 513), (7, 1024), (5, 2047)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemv_irregular_rows_batches_and_boundaries(hip, dtype, shape):
    rng = np.random.default_rng(9101 + len(shape) + shape[-1])
    left = rng.uniform(-1, 1, shape).astype(dtype)
    right = rng.uniform(-1, 1, shape[-1]).astype(dtype)
    actual = p.asarray(left, backend=hip) @ p.asarray(right, backend=hip)
    expected = np.matmul(left.astype(np.float64), right.astype(np.float64))
    tol = (5e-5, 5e-6) if dtype == np.float32 else (5e-12, 5e-13)
    np.testing.assert_allclose(p.asnumpy(actual), expected, rtol=tol[0], atol=tol[1])


def test_long_rows_cancellation_regression(hip):
    rng = np.random.default_rng(941)
    left = rng.uniform(-0.5, 0.5, (129, 8193)).astype(np.float32)
    right = rng.uniform(-0.5, 0.5, 8193).astype(np.float32)
    actual = p.asarray(left, backend=hip) @ p.asarray(right, backend=hip)
    np.testing.assert_allclose(p.asnumpy(actual), left.astype(np.float64) @ right.astype(np.float64), rtol=5e-5, atol=5e-6)


@pytest.mark.parametrize("length", [1, 63, 64, 65, 4096, 4097, 9001, 16384, 16385, 100003])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_dot_tails_boundaries_and_long_partials(hip, length, dtype):
    rng = np.random.default_rng(9102 + length)
    left = rng.uniform(-1, 1, length).astype(dtype)
    right = rng.uniform(-1, 1, length).astype(dtype)
    actual = p.dot(p.asarray(left, backend=hip), p.asarray(right, backend=hip))
    assert actual.shape == ()
    want = float(exact.exact_dot(left, right))
    tol = (5e-5, 5e-6) if dtype == np.float32 else (5e-12, 5e-13)
    np.testing.assert_allclose(p.asnumpy(actual), want, rtol=tol[0], atol=tol[1])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gemv_cancellation_large_finite_signed_and_nonfinite(hip, dtype):
    left = np.zeros((5, 257), dtype=dtype)
    right = np.zeros(257, dtype=dtype)
    left[0, :4] = [4096, -4096, 3, -3]
    right[:4] = 1
    left[1, 20], right[20] = 2.0**60, 2.0**-60
    left[2, 10], right[10] = -0.0, 1.0
    left[2, 11], right[11] = 0.0, 1.0
    left[3, 60], right[60] = np.inf, 0.0
    left[4, 61], right[61] = -np.inf, 1.0
    values = p.asnumpy(p.asarray(left, backend=hip) @ p.asarray(right, backend=hip))
    assert values[0] == 0 and values[1] == 1
    assert values[2] == 0 and not np.signbit(values[2])
    assert np.isnan(values[3]) and np.isneginf(values[4])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("poison", [np.nan, np.inf])
def test_dot_result_block_is_written_not_read(hip, dtype, poison):
    """p.dot's 0-d result is a new pool block that the kernel only writes
    (reference tests/test_cuda.py:345-391 for products): the block it reuses
    is poisoned first, and every call gets a fresh one."""
    x = p.asarray(np.arange(1, 4097, dtype=dtype) / 4096, backend=hip)
    want = float(exact.exact_dot(p.asnumpy(x), p.asnumpy(x)))
    hip.release_cached_memory()  # the poisoned block is then the only cached one of its size
    block = p.full((), poison, dtype=dtype, backend=hip)
    address = block._data.ptr
    del block
    first = p.dot(x, x)
    assert first._data.ptr == address
    assert first.shape == () and first.dtype == dtype
    assert float(p.asnumpy(first)) == pytest.approx(want, rel=1e-6)
    second = p.dot(x, x)
    assert second._data is not first._data and second._data.ptr != first._data.ptr
    assert p.asnumpy(second).tobytes() == p.asnumpy(first).tobytes()


def test_empty_and_zero_inner(hip):
    for dtype in (np.float32, np.float64):
        empty = p.asarray(np.zeros((0, 64), dtype), backend=hip) @ p.asarray(np.zeros(64, dtype), backend=hip)
        assert empty.shape == (0,)
        zero = p.asarray(np.zeros((3, 0), dtype), backend=hip) @ p.asarray(np.zeros(0, dtype), backend=hip)
        np.testing.assert_array_equal(p.asnumpy(zero), np.zeros(3))
        assert p.dot(p.asarray(np.zeros(0, dtype), backend=hip), p.asarray(np.zeros(0, dtype), backend=hip)).item() == 0


def _rel_l2(value, reference):
    return float(np.linalg.norm(value - reference) / np.linalg.norm(reference))


def test_config2_gemv_16384_squared_within_2x_reference_kernel_error(hip):
    n = 16384
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    y = p.asnumpy(p.asarray(a, backend=hip) @ p.asarray(x, backend=hip))
    assert y.shape == (n,) and np.isfinite(y).all()
    oracle = np.empty(n)
    for r in range(0, n, 2048):
        oracle[r : r + 2048] = a[r : r + 2048].astype(np.float64) @ x.astype(np.float64)
    hip_error = _rel_l2(y, oracle)
    rows = np.arange(0, n, 64)  # 256 sampled rows for the reference-order restatement
    ref = kernels.gemv_lanes(a[rows], x)
    ref_error = _rel_l2(ref, oracle[rows])
    assert _rel_l2(y[rows], oracle[rows]) <= 2 * ref_error
    assert hip_error < 1e-6
    dot = p.dot(p.asarray(x, backend=hip), p.asarray(x, backend=hip)).item()
    assert dot == pytest.approx(float(exact.exact_dot(x, x)), rel=1e-6)


def test_config2_dot_within_2x_reference_kernel_error(hip):
    """dot(x, x) of config 2 (16384 N(0, 1) float32, seed 1) and 63 more
    vectors of that distribution: the RMS relative error of hip against the
    exact value is at most 2x that of the reference kernel's order (1024-term
    chunks of 128 lanes, tree, then the reduce kernel: kernels.gemv_lanes).
    One vector alone is too noisy a bar: the reference order's error spans
    an order of magnitude between vectors."""
    n = 16384
    rng = np.random.default_rng(1)
    rng.uniform(-1, 1, (n, n)).astype(np.float32)  # config 2 draws A first
    vectors = [rng.standard_normal(n).astype(np.float32)]
    vectors += [np.random.default_rng(7000 + i).standard_normal(n).astype(np.float32) for i in range(63)]
    hip_err, ref_err = [], []
    for x in vectors:
        truth = float(exact.exact_dot(x, x))
        got = p.dot(p.asarray(x, backend=hip), p.asarray(x, backend=hip)).item()
        hip_err.append((got - truth) / truth)
        ref_err.append((float(kernels.gemv_lanes(x, x)) - truth) / truth)
    hip_rms, ref_rms = np.sqrt(np.mean(np.square(hip_err))), np.sqrt(np.mean(np.square(ref_err)))
    assert hip_rms <= 2 * ref_rms, f"{hip_rms} > 2 x {ref_rms}"


# ---- fused residual b - A @ x (hp_gemv_residual), reference tests/test_residual_matvec.py:25-83

RESIDUAL_SHAPES = [(0, 5), (3, 0), (7, 3), (5, 63), (9, 64), (3, 129), (19, 513), (1, 4097), (33, 1024), (6, 2051)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", RESIDUAL_SHAPES)
def test_residual_matches_eager_rounding_bit_for_bit(hip, dtype, shape, monkeypatch):
    from openpacho._array import ndarray
    from openpacho._hip_gemv import residual_matvec_data

    rng = np.random.default_rng(814)
    a = p.asarray(rng.uniform(-1, 1, shape).astype(dtype), backend=hip)
    x = p.asarray(rng.uniform(-1, 1, shape[1]).astype(dtype), backend=hip)
    product = p.asnumpy(a @ x)
    # One ulp above the product: any change of the product's rounding shows.
    host_b = np.nextafter(product, np.full_like(product, np.inf)) if shape[1] else np.ones_like(product)
    b = p.asarray(host_b, backend=hip)
    expected = p.asnumpy(b - a @ x)

    def forbidden_download(*args):
        pytest.fail("residual downloaded an intermediate")

    with monkeypatch.context() as patch:
        patch.setattr(hip, "download", forbidden_download)
        out = residual_matvec_data(hip, a, x, b)
    actual = p.asnumpy(ndarray._wrap(out, b.shape, b.dtype, hip))
    np.testing.assert_array_equal(actual, expected)
    assert out is not b._data
    # The same bits as NumPy's subtraction of the downloaded product: one
    # rounding of the product, then one of the difference.
    np.testing.assert_array_equal(actual, host_b - product)
    # Against the exact residual b - A x of the same inputs: the product's
    # error (k terms, each rounding at most once per add) plus one rounding.
    if shape[0] and shape[1]:
        host_a, host_x = p.asnumpy(a), p.asnumpy(x)
        eps = float(np.finfo(dtype).eps)
        for r in range(shape[0]):
            exact_r = Fraction(float(host_b[r])) - exact.exact_dot(host_a[r], host_x)
            scale = float(exact.exact_dot(np.abs(host_a[r]), np.abs(host_x)))
            bound = (shape[1] + 1) * eps * scale + eps * abs(float(exact_r))
            assert abs(float(Fraction(float(actual[r])) - exact_r)) <= bound, r


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_residual_nonfinite_and_cancellation(hip, dtype):
    from openpacho._array import ndarray
    from openpacho._hip_gemv import residual_matvec_data

    a = np.zeros((5, 128), dtype=dtype)
    a[0, 0], a[1, 0], a[2, 0] = np.inf, -np.inf, np.nan
    a[3, :4] = np.asarray([1e6, 1, -1e6, 2], dtype=dtype)
    a[4, :2] = [3, -3]
    host_b = np.asarray([np.inf, 1, 2, 3, 0], dtype=dtype)
    a, x, b = [p.asarray(v, backend=hip) for v in (a, np.ones(128, dtype), host_b)]
    expected = p.asnumpy(b - a @ x)
    out = residual_matvec_data(hip, a, x, b)
    np.testing.assert_array_equal(p.asnumpy(ndarray._wrap(out, b.shape, b.dtype, hip)), expected)


def test_compiler_fuses_private_product_but_preserves_shared_outputs(hip):
    a = p.asarray(np.arange(3 * 129, dtype=np.float32).reshape(3, 129) / 100, backend=hip)
    x = p.asarray(np.ones(129, dtype=np.float32), backend=hip)
    b = p.asarray(np.ones(3, dtype=np.float32), backend=hip)
    operation = p.compile(lambda a, x, b: b - a @ x)
    assert [s["kind"] for s in operation.explain(a, x, b)["steps"]] == ["residual_matvec"]
    np.testing.assert_array_equal(p.asnumpy(operation(a, x, b)), p.asnumpy(b - a @ x))

    @p.compile
    def shared(a, x, b):
        product = a @ x
        return product, b - product

    assert "residual_matvec" not in [s["kind"] for s in shared.explain(a, x, b)["steps"]]
    product, residual = shared(a, x, b)
    np.testing.assert_array_equal(p.asnumpy(product), p.asnumpy(a @ x))
    np.testing.assert_array_equal(p.asnumpy(residual), p.asnumpy(b - a @ x))
