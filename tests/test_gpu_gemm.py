"""GPU parity of the MFMA GEMM (hp_gemm) against fp64/exact oracles.

Cases follow reference tests/test_cuda.py:280-441 (vector/irregular/empty/K=0
products, NaN/Inf-poisoned destinations, batched broadcasting),
tests/test_padding.py:374-527 (padded plans, special values, signed zeros)
and BASELINE.json config 4 (8192^3 fp32, 4096^3 fp64, 4097x3001x2049 padded,
64x(512x1024)@(1024x768)). The error bar: hip error against the exact/fp64
oracle <= 2x the error of the reference kernel's sequential-K order
(oracle.kernels.gemm_sequential) on the same sampled outputs.
"""

import ctypes

import numpy as np
import pytest

import openpacho as p
from oracle import exact, kernels
from oracle import padding as pad_oracle

pytestmark = pytest.mark.gpu

MATMUL_CASES = (
    ("vector", np.asarray([1.25, -2.0, 0.5, 3.0, -1.0, 2.5, 4.0]), np.asarray([-2.0, 3.0, 1.5, -0.5, 2.0, 0.25, -1.0])),
    ("gemv", np.arange(15, dtype=np.float64).reshape(3, 5) / 11, np.asarray([1.0, -2.0, 0.5, 3.0, -1.5])),
    ("vecmat", np.asarray([1.0, -2.0, 0.5, 3.0, -1.5]), np.arange(20, dtype=np.float64).reshape(5, 4) / 13),
    ("irregular_gemm", np.arange(35, dtype=np.float64).reshape(5, 7) / 17, np.arange(21, dtype=np.float64).reshape(7, 3) / 19),
    ("odd_tile_gemm", np.arange(33 * 17, dtype=np.float64).reshape(33, 17) / 101, np.arange(17 * 65, dtype=np.float64).reshape(17, 65) / 103),
    ("large_odd_gemm", np.arange(65 * 63, dtype=np.float64).reshape(65, 63) / 107, np.arange(63 * 97, dtype=np.float64).reshape(63, 97) / 109),
)


def _tol(dtype):
    return (3e-5, 3e-6) if np.dtype(dtype) == np.float32 else (2e-11, 2e-12)


def test_vector_and_irregular_products(hip):
    for dtype in (np.float32, np.float64):
        for name, left, right in MATMUL_CASES:
            left, right = left.astype(dtype), right.astype(dtype)
            actual = p.matmul(p.asarray(left, backend=hip), p.asarray(right, backend=hip))
            rtol, atol = _tol(dtype)
            np.testing.assert_allclose(p.asnumpy(actual), np.matmul(left, right), rtol=rtol, atol=atol, err_msg=name)
            assert p.asnumpy(actual).dtype == dtype


@pytest.mark.parametrize("left_shape,right_shape", [((0, 5), (5, 3)), ((2, 0), (0, 3)), ((1, 0), (0, 7)), ((4, 3), (3, 0)), ((0,), (0,))])
def test_empty_and_k0_products(hip, left_shape, right_shape):
    for dtype in (np.float32, np.float64):
        left, right = np.zeros(left_shape, dtype), np.zeros(right_shape, dtype)
        actual = p.asnumpy(p.matmul(p.asarray(left, backend=hip), p.asarray(right, backend=hip)))
        np.testing.assert_array_equal(actual, np.matmul(left, right))


def _poisoned(backend, left, right, dtype, poison, monkeypatch):
    left, right = left.astype(dtype), right.astype(dtype)
    expected = np.matmul(left, right)
    a, b = p.asarray(left, backend=backend), p.asarray(right, backend=backend)
    destination = p.full(expected.shape, poison, dtype=dtype, backend=backend)
    original = backend.empty

    def poisoned_empty(shape, requested):
        if tuple(shape) == expected.shape and np.dtype(requested) == np.dtype(dtype):
            return destination._data
        return original(shape, requested)

    monkeypatch.setattr(backend, "empty", poisoned_empty)
    actual = p.matmul(a, b)
    monkeypatch.undo()
    assert actual._data is destination._data
    return actual, expected


def test_products_overwrite_nan_and_inf_destinations(hip, monkeypatch):
    for dtype in (np.float32, np.float64):
        for poison in (np.nan, np.inf):
            for name, left, right in MATMUL_CASES[:4]:
                actual, expected = _poisoned(hip, left, right, dtype, poison, monkeypatch)
                rtol, atol = _tol(dtype)
                np.testing.assert_allclose(p.asnumpy(actual), expected, rtol=rtol, atol=atol, err_msg=name)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize(
    "shapes",
    [
        ((3, 33, 17), (3, 17, 65)),
        ((2, 1, 33, 17), (1, 3, 17, 65)),
        ((2, 5, 7), (7, 3)),
        ((5, 7), (2, 7, 3)),
        ((2, 5, 7), (7,)),
        ((7,), (2, 7, 3)),
        ((2, 5, 0), (2, 0, 3)),
        ((0, 5, 7), (1, 7, 3)),
        ((2, 3, 1, 40, 24), (3, 4, 24, 72)),
    ],
)
def test_batched_broadcast_products(hip, dtype, shapes):
    rng = np.random.default_rng(830)
    left, right = (rng.normal(size=s).astype(dtype) for s in shapes)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    operation = p.compile(lambda x, y: x @ y)
    rtol, atol = (3e-5, 3e-5) if dtype == np.float32 else (2e-11, 2e-12)
    for result in (a @ b, operation(a, b)):
        np.testing.assert_allclose(p.asnumpy(result), left @ right, rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize(
    "m,n,k",
    [
        (256, 128, 16),  # one tile, M/N edge (clamped loads)
        (512, 256, 64),  # interior, several tiles and slices
        (257, 129, 17),  # every edge, K odd (zero-filled K edge slice)
        (300, 200, 100),  # K edge with K % 4 == 0
        (1, 1, 1),
        (31, 33, 4099),  # long K, partial tiles
        (640, 384, 48),  # M/N edges with K whole: edge tiles moved inside
        (777, 300, 64),  # moved edge tiles that own 9 rows / 44 columns
        (257, 257, 32),  # moved edge tiles that own a single row / column
        (513, 1023, 16),  # one K slice; edges of 1 row and 255 columns
        (4096, 4096, 1024),  # whole rounds of interior tiles, no stream-K
    ],
)
def test_kernel_modes_against_float64(hip, dtype, m, n, k):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    got = p.asnumpy(p.asarray(a, backend=hip) @ p.asarray(b, backend=hip))
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    bound = (4e-7 if dtype == np.float32 else 8e-16) * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)


# Tile counts that leave the last round of resident workgroups partly
# filled, so their K slices are cut into stream-K runs and summed by the fixup
# kernel: runs that cross tile boundaries (extra > 0), single-tile problems
# cut over many workers, batched tiles, every load mode. Products of at most
# 256 K slices take the 128 x 128 tiles (three workgroups per compute unit),
# longer ones the 256 x 256 tiles (one per compute unit): both are covered.
STREAM_K_CASES = [
    (np.float32, (), 512, 256, 8192),  # 256 x 256 tiles: interior, 2 tiles x 512 slices
    (np.float32, (), 1000, 700, 4100),  # 256 x 256 tiles: edges, K % 16 == 4
    (np.float32, (2,), 600, 300, 4112),  # 256 x 256 tiles: batched, moved edge tiles
    (np.float32, (), 512, 256, 1552),  # interior, 2 tiles x 97 slices
    (np.float32, (), 31, 33, 4099),  # one tile cut over 32 workers
    (np.float32, (), 1000, 700, 2000),  # M/N edges, 12 tiles
    (np.float32, (), 777, 555, 1111),  # K odd
    (np.float32, (3,), 300, 200, 700),  # batched: 6 tiles
    (np.float32, (2,), 600, 300, 512),  # batched, moved edge tiles summed by the fixup
    (np.float32, (), 257, 257, 4096),  # single-row/column moved tiles cut over many workers
    (np.float64, (), 1000, 1000, 2100),  # 32 tiles over 256 workers, extra > 0
    (np.float64, (2,), 256, 384, 1024),  # interior fp64, batched
    (np.float64, (), 129, 65, 3001),  # K odd, fp64
]


@pytest.mark.parametrize("dtype,batch,m,n,k", STREAM_K_CASES)
def test_stream_k_splits_against_float64_and_deterministic(hip, dtype, batch, m, n, k):
    rng = np.random.default_rng(m + 3 * n + 7 * k)
    a = rng.uniform(-1, 1, batch + (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    got = p.asnumpy(A @ B)
    again = p.asnumpy(A @ B)
    np.testing.assert_array_equal(got, again)  # fixed K order: bitwise repeatable
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    bound = (4e-7 if dtype == np.float32 else 8e-16) * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("m,n,k", [(300, 260, 64), (512, 256, 48), (129, 70, 37)])
def test_operands_at_element_alignment(hip, dtype, m, n, k):
    """hp_gemm with A, B and C at an odd element offset (rows not 16-byte aligned)."""
    rng = np.random.default_rng(m + n + k)
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    size = np.dtype(dtype).itemsize
    pad = np.zeros(1, dtype)
    A = hip.upload(np.concatenate([pad, a.ravel()]))
    B = hip.upload(np.concatenate([pad, b.ravel()]))
    C = hip.upload(np.full(m * n + 1, np.nan, dtype))
    code = 5 if dtype == np.float32 else 6
    with hip._active():
        hip._call("hp_gemm", code, ctypes.c_void_p(A.ptr + size), ctypes.c_void_p(B.ptr + size),
                  ctypes.c_void_p(C.ptr + size), m, n, k, 0, None, None, None)
        out = np.empty(m * n + 1, dtype)
        hip._call("hp_d2h", ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(C.ptr), out.nbytes)
    assert np.isnan(out[0])  # the element before C is untouched
    got = out[1:].reshape(m, n)
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    bound = (4e-7 if dtype == np.float32 else 8e-16) * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)


def _sampled_error_ratio(a, b, got, samples, seed):
    """(hip error, reference-order error) over sampled outputs, exact oracle."""
    rng = np.random.default_rng(seed)
    rows = rng.integers(0, a.shape[0], samples)
    cols = rng.integers(0, b.shape[1], samples)
    ref = kernels.gemm_sequential(a, b, rows, cols)
    hip_err, ref_err = [], []
    for i, (r, c) in enumerate(zip(rows, cols)):
        truth = exact.exact_dot(a[r, :], b[:, c])
        scale = float(exact.exact_dot(np.abs(a[r, :]), np.abs(b[:, c])))
        hip_err.append(abs(float(got[i] if got.ndim == 1 else got[r, c]) - float(truth)) / scale)
        ref_err.append(abs(float(ref[i]) - float(truth)) / scale)
    return float(np.sqrt(np.mean(np.square(hip_err)))), float(np.sqrt(np.mean(np.square(ref_err))))


def test_config1_shape_1024_cubed_within_2x_reference_kernel_error(hip):
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    b = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    got = p.asnumpy(p.asarray(a, backend=hip) @ p.asarray(b, backend=hip))
    hip_err, ref_err = _sampled_error_ratio(a, b, got, 256, 5)
    assert hip_err <= 2 * ref_err
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


def test_config4_fp32_8192_cubed(hip):
    n = 8192
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    c = A @ B
    got_rows = p.asnumpy(c[4095:4096])  # gather of one row
    assert got_rows.shape == (1, n)
    full = p.asnumpy(c)
    # Every output (the whole-tile kernel of the headline: a wrong fragment
    # block in any tile fails), then the product repeated bit for bit.
    assert exact.product_bound_ratio(a, b, full, 4e-7) <= 1
    np.testing.assert_array_equal(p.asnumpy(A @ B), full)
    np.testing.assert_array_equal(full[4095], got_rows[0])
    hip_err, ref_err = _sampled_error_ratio(a, b, full, 48, 6)
    assert hip_err <= 2 * ref_err


def test_config4_fp64_4096_cubed(hip):
    n = 4096
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (n, n))
    b = rng.uniform(-1, 1, (n, n))
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    full = p.asnumpy(A @ B)
    assert exact.product_bound_ratio(a, b, full, 8e-16) <= 1
    np.testing.assert_array_equal(p.asnumpy(A @ B), full)
    hip_err, ref_err = _sampled_error_ratio(a, b, full, 48, 7)
    assert hip_err <= 2 * ref_err
    np.testing.assert_allclose(full[[0, 2047, 4095]], a[[0, 2047, 4095]] @ b, rtol=0, atol=1e-11)


def test_config4_padded_odd_shape(hip):
    m, k, n = 4097, 3001, 2049
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    compiled = p.compile(lambda x, y: p.matmul(x, y), padding=True)
    step = [s for s in compiled.explain(A, B)["steps"] if s["kind"] == "padded_matmul"]
    assert len(step) == 1
    info = step[0]["padding"]
    expected = pad_oracle.plan((m, k), (k, n))
    # The reference's padded problem, computed without its copies.
    assert info["padded_input_shapes"] == expected["padded_input_shapes"]
    assert info["padded_output_shape"] == expected["padded_output_shape"]
    assert expected["scratch_bytes"] == 109_039_616 and info["scratch_bytes"] == 0
    assert info["copy_dispatches"] == 0 and info["alignment"] == (32, 16, 32)
    first = None
    for result in (p.matmul(A, B, padding=True), compiled(A, B)):
        got = p.asnumpy(result)
        assert got.shape == (m, n)
        if first is None:
            first = got
            assert exact.product_bound_ratio(a, b, got, 4e-7) <= 1  # every output
        else:
            np.testing.assert_array_equal(got, first)  # eager and compiled, bit for bit
        hip_err, ref_err = _sampled_error_ratio(a, b, got, 32, 8)
        assert hip_err <= 2 * ref_err
    np.testing.assert_array_equal(p.asnumpy(A @ B), first)  # the unpadded product too
    np.testing.assert_array_equal(p.asnumpy(A), a)


def test_config4_batched_broadcast(hip):
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (64, 512, 1024)).astype(np.float32)
    b = rng.uniform(-1, 1, (1024, 768)).astype(np.float32)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    got = p.asnumpy(A @ B)
    assert got.shape == (64, 512, 768)
    # Every batch against float32 BLAS (a wrong fragment block in any tile
    # shows as errors of order 1), then repeated bit for bit: several
    # workgroups share each compute unit here, which once exposed an LDS
    # read/write race that hit different tiles on each run.
    np.testing.assert_allclose(got, np.matmul(a, b), rtol=0, atol=1e-3)
    np.testing.assert_array_equal(p.asnumpy(A @ B), got)
    for batch in (0, 31, 63):
        want = a[batch].astype(np.float64) @ b.astype(np.float64)
        np.testing.assert_allclose(got[batch], want, rtol=0, atol=2e-4)
        hip_err, ref_err = _sampled_error_ratio(a[batch], b, got[batch], 32, 9 + batch)
        assert hip_err <= 2 * ref_err, f"batch {batch}: {hip_err} > 2 x {ref_err}"


@pytest.mark.parametrize("shapes", [((33, 17), (17, 65)), ((65, 47), (47, 67)), ((64, 32), (32, 96)), ((2, 1, 33, 17), (1, 3, 17, 65))])
def test_padding_rounds_to_tiles_and_preserves_logical_results(hip, shapes):
    rng = np.random.default_rng(8301)
    left, right = (rng.uniform(-0.5, 0.5, size=s).astype(np.float32) for s in shapes)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    compiled = p.compile(lambda x, y: p.matmul(x, y), padding=True)
    details = compiled.explain(a, b)
    step = [s for s in details["steps"] if s["kind"] == "padded_matmul"][0]["padding"]
    plan = pad_oracle.plan(*shapes)
    assert tuple(step["padded_input_shapes"]) == plan["padded_input_shapes"]
    assert tuple(step["padded_output_shape"]) == plan["padded_output_shape"]
    assert step["scratch_bytes"] == 0 and step["copy_dispatches"] == 0
    expected = left.astype(np.float64) @ right.astype(np.float64)
    prepared = compiled.prepare(a, b)
    first = compiled(a, b)
    for result in (p.matmul(a, b, padding=True), first, prepared(a, b)):
        np.testing.assert_allclose(p.asnumpy(result), expected, rtol=5e-4, atol=5e-4)
    snapshot = p.asnumpy(first)
    again = prepared(a, b)
    assert first._data is not again._data
    np.testing.assert_array_equal(p.asnumpy(a), left)
    np.testing.assert_array_equal(p.asnumpy(first), snapshot)
    changed = prepared(p.asarray(left + np.float32(0.25), backend=hip), p.asarray(right - np.float32(0.125), backend=hip))
    want = (left + np.float32(0.25)).astype(np.float64) @ (right - np.float32(0.125)).astype(np.float64)
    np.testing.assert_allclose(p.asnumpy(changed), want, rtol=5e-4, atol=5e-4)


def test_padding_declines_float64_and_small(hip):
    rng = np.random.default_rng(8303)
    for rows, dtype in ((33, np.float64), (31, np.float32)):
        left = rng.normal(size=(rows, 17)).astype(dtype)
        right = rng.normal(size=(17, 65)).astype(dtype)
        compiled = p.compile(lambda x, y: p.matmul(x, y), padding=True)
        a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
        assert not any(s["kind"] == "padded_matmul" for s in compiled.explain(a, b)["steps"])
        np.testing.assert_allclose(p.asnumpy(compiled(a, b)), left @ right, rtol=5e-4, atol=5e-4)


def test_padding_preserves_special_values_and_signed_zero(hip):
    left = np.zeros((33, 17), np.float32)
    right = np.zeros((17, 65), np.float32)
    left[0, 0], right[0, 0] = np.nan, 1.0
    left[1, 1], right[1, 1], right[1, 2] = np.inf, 0.0, 1.0
    left[2, 2], right[2, 3] = -np.inf, 1.0
    left[3, 3], right[3, 4] = -np.float32(0.0), 1.0
    left[4, 4], right[4, 5] = np.float32(0.0), -1.0
    left[5, 5], right[5, 6] = np.nextafter(np.float32(0), np.float32(1)), 1.0
    left[6, 6], right[6, 7] = np.finfo(np.float32).tiny, 1.0
    left[7, 7], right[7, 8] = np.finfo(np.float32).max, 1.0
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    padded = p.asnumpy(p.matmul(a, b, padding=True))
    ordinary = p.asnumpy(p.matmul(a, b))
    for predicate in (np.isnan, np.isinf, np.isfinite):
        np.testing.assert_array_equal(predicate(padded), predicate(ordinary))
    for index in ((3, 4), (4, 5), (5, 6), (6, 7), (7, 8)):
        assert np.signbit(padded[index]) == np.signbit(ordinary[index])
        np.testing.assert_array_equal(padded[index], ordinary[index])
    np.testing.assert_array_equal(p.asnumpy(a), left)


# ---- narrow 64 x 64 tiles: short products with M, N multiples of 64 and K
# of 16 that give one to four such tiles per compute unit (256 to 1024 on
# MI355X) and at most 2^23 multiply-adds per compute unit. Each tile is one
# workgroup whose waves (eight at one tile per compute unit, else four) take
# every eighth (fourth) K slice and add their tiles in wave order, so a wave
# may own one slice or none.

NARROW_CASES = [
    ((), 1024, 1024, 16),  # one slice: seven of eight waves own none
    ((), 1024, 1024, 48),  # three slices: five waves own none
    ((), 1024, 1024, 1024),
    ((), 2048, 512, 2048),  # long K: 32 slices per wave
    ((), 1024, 2048, 80),  # two tiles per compute unit
    ((), 2048, 2048, 512),  # four tiles per compute unit
    ((4,), 512, 512, 144),  # batched
]


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("batch,m,n,k", NARROW_CASES)
def test_narrow_tiles_against_float64_and_deterministic(hip, ta, tb, batch, m, n, k):
    if batch and (ta or tb):
        pytest.skip("transposed operands are 2-D")
    rng = np.random.default_rng(m + 5 * n + 11 * k + 2 * ta + tb)
    left = rng.uniform(-1, 1, batch + ((k, m) if ta else (m, k))).astype(np.float32)
    right = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    product = p.compile(lambda x, y: (x.T if ta else x) @ (y.T if tb else y))
    got = p.asnumpy(product(a, b))
    np.testing.assert_array_equal(got, p.asnumpy(product(a, b)))  # fixed wave order: repeatable
    op_a = (left.T if ta else left).astype(np.float64)
    op_b = (right.T if tb else right).astype(np.float64)
    want = op_a @ op_b
    scale = np.abs(op_a) @ np.abs(op_b)
    bound = 4e-7 * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)
    if ta or tb:
        # The materialized transposes give the same bits (same tiles, same K order).
        eager = p.asnumpy(p.asarray(np.ascontiguousarray(op_a.astype(np.float32)), backend=hip)
                          @ p.asarray(np.ascontiguousarray(op_b.astype(np.float32)), backend=hip))
        np.testing.assert_array_equal(got, eager)


# ---- 256 x 192 tiles: products whose 256 x 256 tiles would fill part of
# one round of the 256 compute units (and be cut into stream-K runs) while
# the 192-wide tiles fill at least 7/8 of it whole. One launch, both operands
# by 4-byte LDS-DMA with descriptor-range edges.

WIDE_CASES = [
    ((), 4096, 3072, 512),  # 192 -> 256 tiles, interior
    ((), 4000, 2900, 333),  # M, N and K edges
    ((2,), 2048, 3072, 160),  # batched
    ((), 2048, 6000, 64),  # short K, N edge of 48 columns
    ((240,), 100, 100, 50),  # matrices smaller than a tile: every slice by 4-byte DMA
    ((14,), 4096, 150, 64),  # N below the tile width
]


LAYOUTS = [(False, False), (True, False), (False, True), (True, True)]


@pytest.mark.parametrize(
    "ta,tb,batch,m,n,k",
    [(ta, tb) + case for case in WIDE_CASES for ta, tb in LAYOUTS if not (case[0] and (ta or tb))],
)  # transposed operands are 2-D
def test_wide_tiles_against_float64_and_deterministic(hip, ta, tb, batch, m, n, k):
    rng = np.random.default_rng(3 * m + n + 13 * k + 2 * ta + tb)
    left = rng.uniform(-1, 1, batch + ((k, m) if ta else (m, k))).astype(np.float32)
    right = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    product = p.compile(lambda x, y: (x.T if ta else x) @ (y.T if tb else y))
    got = p.asnumpy(product(a, b))
    np.testing.assert_array_equal(got, p.asnumpy(product(a, b)))  # fixed K order: repeatable
    op_a = (left.T if ta else left).astype(np.float64)
    op_b = (right.T if tb else right).astype(np.float64)
    want = op_a @ op_b
    scale = np.abs(op_a) @ np.abs(op_b)
    bound = 4e-7 * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)
    if ta or tb:
        # The materialized transposes give the same bits (same tiles, same K order).
        eager = p.asnumpy(p.asarray(np.ascontiguousarray(op_a.astype(np.float32)), backend=hip)
                          @ p.asarray(np.ascontiguousarray(op_b.astype(np.float32)), backend=hip))
        np.testing.assert_array_equal(got, eager)


# ---- 256 x 128 tiles (eight waves of 64 x 64): products whose 256 x 256
# tiles would fill part of one round (and be cut by stream-K) while these
# fill it whole, with more than 64 K slices. Modes 0 (whole tiles), 1 (M/N
# edges: edge tiles moved inside) and 2 (a K edge), every operand layout,
# and one batched product.

HALF_CASES = [
    ((), 4096, 2048, 1088),
    ((), 4000, 1900, 1088),
    ((), 4096, 2048, 1090),
    ((2,), 2048, 2048, 1088),
]


@pytest.mark.parametrize(
    "ta,tb,batch,m,n,k",
    [(ta, tb) + case for case in HALF_CASES for ta, tb in LAYOUTS if not (case[0] and (ta or tb))],
)  # transposed operands are 2-D
def test_half_tiles_against_float64_and_deterministic(hip, ta, tb, batch, m, n, k):
    rng = np.random.default_rng(5 * m + 3 * n + k + 2 * ta + tb)
    left = rng.uniform(-1, 1, batch + ((k, m) if ta else (m, k))).astype(np.float32)
    right = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    product = p.compile(lambda x, y: (x.T if ta else x) @ (y.T if tb else y))
    got = p.asnumpy(product(a, b))
    np.testing.assert_array_equal(got, p.asnumpy(product(a, b)))
    op_a = np.swapaxes(left, -1, -2) if ta else left
    op_b = right.T if tb else right
    if ta or tb:  # the materialized transposes give the same bits
        plain_a = p.asarray(np.ascontiguousarray(op_a), backend=hip)
        plain = plain_a @ p.asarray(np.ascontiguousarray(op_b), backend=hip)
        np.testing.assert_array_equal(got, p.asnumpy(plain))
    want = op_a.astype(np.float64) @ op_b.astype(np.float64)
    scale = np.abs(op_a).astype(np.float64) @ np.abs(op_b).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4e-7 * np.sqrt(k) * 4 * scale + 1e-30)


# ---- odd K (a K-edge slice): the whole K slices of products at least one
# tile tall and wide load by 16-byte LDS-DMA from 4-byte aligned addresses,
# the K-edge slice by 4-byte LDS-DMA that zero-fills past K. 256 x 256 tiles
# in one whole round, 256 x 256 tiles cut by stream-K, 128 x 128 tiles.

ODD_K_CASES = [(4096, 4096, 161), (1024, 1024, 4097), (520, 300, 2049)]


@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("m,n,k", ODD_K_CASES)
def test_odd_k_products_against_float64_and_deterministic(hip, ta, tb, m, n, k):
    rng = np.random.default_rng(m + 7 * n + 3 * k + 2 * ta + tb)
    left = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
    right = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    product = p.compile(lambda x, y: (x.T if ta else x) @ (y.T if tb else y))
    got = p.asnumpy(product(a, b))
    np.testing.assert_array_equal(got, p.asnumpy(product(a, b)))
    op_a = (left.T if ta else left).astype(np.float64)
    op_b = (right.T if tb else right).astype(np.float64)
    want = op_a @ op_b
    scale = np.abs(op_a) @ np.abs(op_b)
    bound = 4e-7 * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)


# ---- products of private transposes (hp_gemm_layout), reference
# tests/test_clblast.py:410-440 and tests/test_compiled_layout.py:43-80

LAYOUT_SHAPES = [(35, 33, 39), (300, 257, 129), (512, 1024, 768), (700, 2001, 517), (700, 1024, 517)]  # m, k, n


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,k,n", LAYOUT_SHAPES)
def test_compiled_transpose_products_read_operands_in_place(hip, monkeypatch, dtype, ta, tb, m, k, n):
    rng = np.random.default_rng(395 + m + k + n)
    left = rng.uniform(-0.5, 0.5, (k, m) if ta else (m, k)).astype(dtype)
    right = rng.uniform(-0.5, 0.5, (n, k) if tb else (k, n)).astype(dtype)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    replacement = p.asarray(left * 2, backend=hip)
    compiled = p.compile(lambda a, b: (a.T if ta else a) @ (b.T if tb else b))
    prepared = compiled.prepare(a, b)
    steps = prepared.explain()["steps"]
    assert [s["kind"] for s in steps] == ["layout_matmul"]
    assert steps[0]["layout"]["provider"] == "hip"

    def forbidden(*args, **kwargs):
        raise AssertionError("private transpose product must not gather or download")

    with monkeypatch.context() as context:
        context.setattr(hip, "gather", forbidden)
        context.setattr(hip, "download", forbidden)
        result = prepared(a, b)
        rebound = prepared(replacement, b)
        hip.synchronize()
    # Same tiles, K order and MFMA sequence as the materialized transposes.
    eager = p.asnumpy((a.T if ta else a) @ (b.T if tb else b))
    np.testing.assert_array_equal(p.asnumpy(result), eager)
    op_a = (left.T if ta else left).astype(np.float64)
    op_b = (right.T if tb else right).astype(np.float64)
    scale = np.abs(op_a) @ np.abs(op_b)
    bound = (4e-7 if dtype == np.float32 else 8e-16) * np.sqrt(k) * 4
    assert np.all(np.abs(p.asnumpy(result) - op_a @ op_b) <= bound * scale + 1e-30)
    assert np.all(np.abs(p.asnumpy(rebound) - 2 * (op_a @ op_b)) <= 2 * bound * scale + 1e-30)


# ---- exactly representable accumulation and special values, reference
# tests/test_rectangular_gemm.py:62-104


@pytest.mark.parametrize("m,k,n", [(33, 4081, 257), (65, 4095, 1023), (95, 8191, 2051)])
def test_dyadic_products_are_exact_and_rebinding_is_copy_free(hip, monkeypatch, m, k, n):
    rng = np.random.default_rng(613)
    # Multiples of 1/256 with |sum| < 2^7: every partial sum is exact in fp32,
    # so any K order gives the float64 result bit for bit.
    host = [rng.integers(-2, 3, shape).astype("float32") / 16 for shape in ((m, k), (k, n))]
    a, b = (p.asarray(h, backend=hip) for h in host)
    twice_a = p.asarray(host[0] * 2, backend=hip)
    baseline = p.asnumpy(a @ b)
    compiled = p.compile(lambda a, b: a @ b).prepare(a, b)
    with monkeypatch.context() as guard:
        guard.setattr(hip, "download", lambda *args: pytest.fail("Hidden download"))
        guard.setattr(hip, "gather", lambda *args: pytest.fail("Unexpected packing/crop"))
        first, second = compiled(a, b), compiled(twice_a, b)
    np.testing.assert_array_equal(p.asnumpy(first).view("uint32"), baseline.view("uint32"))
    np.testing.assert_array_equal(p.asnumpy(first), host[0].astype("float64") @ host[1])
    np.testing.assert_array_equal(p.asnumpy(second), baseline * 2)
    assert first._data is not second._data


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_special_values_and_subnormals_propagate(hip, dtype):
    left = np.zeros((33, 4081), dtype=dtype)
    right = np.zeros((4081, 257), dtype=dtype)
    tiny = np.nextafter(dtype(0), dtype(1))
    left[0, 0], left[1, 0], left[2, 0] = np.inf, np.nan, tiny
    left[3, 0], left[3, 1] = np.finfo(dtype).max, np.finfo(dtype).max  # overflow to inf
    right[0, :3] = [0, 1, -1]
    right[1, :3] = [0, 1, 1]
    got = p.asnumpy(p.asarray(left, backend=hip) @ p.asarray(right, backend=hip))
    with np.errstate(all="ignore"):
        want = left.astype(np.float64) @ right.astype(np.float64)
    want = want.astype(dtype)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    finite = ~np.isnan(want)
    np.testing.assert_array_equal(got[finite], want[finite])
    assert got[2, 1] == tiny and got[2, 2] == -tiny  # subnormals are not flushed


INTEGER_SHAPES = [
    ((37, 129), (129,)),  # reference tests/test_matrix_optimization.py:33-40 shapes
    ((1, 4097), (4097,)),
    ((3, 1025), (1025,)),
    ((1, 4096), (4096,)),
    ((4097,), (4097,)),
    ((7,), (7, 5)),
    ((33, 70), (70, 45)),
    ((2, 1, 5, 7), (3, 7, 4)),
    ((4, 0), (0, 3)),
]


@pytest.mark.parametrize("dtype", [np.int32, np.int64, np.uint32, np.uint64])
@pytest.mark.parametrize("shapes", INTEGER_SHAPES)
def test_integer_products_wrap_like_numpy_bit_for_bit(hip, dtype, shapes):
    # Integer products sum in the operand type modulo 2^bits (NumPy and the
    # reference OpenCL backend's generic product): small values check the
    # indexing, full-range values the wraparound.
    rng = np.random.default_rng(48)
    info = np.iinfo(dtype)
    for low, high in ((-3, 4), (info.min, info.max)):
        low = max(low, info.min)
        a, b = (rng.integers(low, high, size=s, dtype=dtype, endpoint=True) for s in shapes)
        with np.errstate(over="ignore"):
            want = a @ b
        got = p.asarray(a, backend=hip) @ p.asarray(b, backend=hip)
        assert got.dtype == want.dtype and got.shape == want.shape
        np.testing.assert_array_equal(p.asnumpy(got), want)


def test_mixed_integer_promotion_and_compiled_product(hip):
    a = np.arange(-6, 6, dtype=np.int32).reshape(3, 4)
    b = np.arange(8, dtype=np.int64).reshape(4, 2) * (2**40)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    np.testing.assert_array_equal(p.asnumpy(A @ B), a @ b)
    np.testing.assert_array_equal(p.asnumpy(p.compile(lambda x, y: x @ y + 1)(A, B)), a @ b + 1)
    with pytest.raises(NotImplementedError, match="Boolean matmul"):
        p.asarray(a > 0, backend=hip) @ p.asarray(b > 0, backend=hip)


def test_bool_gemm_abi_is_or_of_ands(hip):
    # The facade rejects bool products (reference _array.py:471); the C-ABI
    # computes them as NumPy does: any(a[i, :] & b[:, j]).
    rng = np.random.default_rng(7)
    a = rng.random((19, 33)) < 0.05
    b = rng.random((33, 21)) < 0.05
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    out = p.empty((19, 21), dtype=np.bool_, backend=hip)
    with hip._active():
        hip._call("hp_gemm", 0, *hip._ptrs(A, B, out), 19, 21, 33, 0, None, None, None)
    np.testing.assert_array_equal(p.asnumpy(out), a @ b)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_batch_strides_off_the_16_byte_grid(hip, dtype):
    """hp_gemm with an A batch stride of m*k + 1 elements: every other batch
    matrix starts off a 16-byte boundary, so the product must take the 4-byte
    LDS-DMA of mode 2, not the 16-byte form (M, N, K would otherwise allow
    it)."""
    from openpacho import _hip_lib

    m, n, k, batch = 256, 256, 32, 3
    stride = m * k + 1
    rng = np.random.default_rng(stride)
    a_host = rng.uniform(-1, 1, stride * batch).astype(dtype)
    b_host = rng.uniform(-1, 1, (k, n)).astype(dtype)
    A, B = hip.upload(a_host), hip.upload(b_host)
    C = hip.upload(np.full(batch * m * n, np.nan, dtype))
    code = _hip_lib.DTYPE_CODES[np.dtype(dtype)]
    with hip._active():
        hip._call("hp_gemm", code, *hip._ptrs(A, B, C), m, n, k, 1, _hip_lib.int64_array([batch]),
                  _hip_lib.int64_array([stride]), _hip_lib.int64_array([0]))
    got = p.asnumpy(p.ndarray._wrap(C, (batch, m, n), dtype, hip))
    bound = (4e-7 if dtype == np.float32 else 8e-16) * np.sqrt(k) * 4
    for i in range(batch):
        a_i = a_host[i * stride : i * stride + m * k].reshape(m, k).astype(np.float64)
        want = a_i @ b_host.astype(np.float64)
        scale = np.abs(a_i) @ np.abs(b_host.astype(np.float64))
        assert np.all(np.abs(got[i] - want) <= bound * scale + 1e-30), i


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("batch,m,n,k", [(3, 300, 280, 77), (2, 256, 256, 1001), (4, 129, 513, 33), (2, 520, 260, 3)])
def test_k_edge_of_adjacent_batch_matrices_contracts_zeros(hip, dtype, batch, m, n, k):
    """Batched A and B with K off the 16-wide slice grid: in memory each
    batch matrix's K edge is followed by the next matrix's data (A's next row,
    B's next batch), which must not enter the contraction; rows and columns
    past M and N of one batch matrix may hold the next one's data but reach
    no stored output. Results against float64, bitwise repeatable."""
    rng = np.random.default_rng(batch * 1000 + k)
    a = rng.uniform(-1, 1, (batch, m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (batch, k, n)).astype(dtype)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    got = p.asnumpy(A @ B)
    np.testing.assert_array_equal(got, p.asnumpy(A @ B))
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    bound = (4e-7 if dtype == np.float32 else 8e-16) * np.sqrt(k) * 4
    assert np.all(np.abs(got - want) <= bound * scale + 1e-30)


# Products whose last tile row or column holds at most 8 rows or columns run
# as whole 256 x 256 tiles plus edge strips (the few-rows kernel reads B once
# with K cut into chunks, the few-columns kernel streams A rows).
EDGE_CASES = [
    (257, 300, 512),  # one edge row; 44 edge columns stay in tiles
    (520, 264, 1000),  # 8 rows
    (263, 1031, 77),  # 7 rows, odd K: two K chunks of the rows strip
    (1280, 513, 3001),  # one edge column, odd K
    (4097, 4097, 16),  # one row and one column, one K slice (rows strip written directly)
    (300, 2305, 4096),  # one edge column beside 44 rows in tiles
]


def test_edge_strips_are_ordered_before_the_next_work_on_the_stream(hip):
    """The strips of a 4097 x 2049 x 1025 product (one edge row, one edge
    column) run on the context's second stream; the next calls on the main
    stream, queued without a host wait, must see their outputs (a copy of C)
    and must not overwrite their inputs before they have read them (a fill
    of A). C starts as NaN, so a strip output read too early shows."""
    m, k, n = 4097, 2049, 1025
    rng = np.random.default_rng(11)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    bound = 4e-7 * np.sqrt(k) * 4
    A, B = hip.upload(a.ravel()), hip.upload(b.ravel())
    C, D = hip.upload(np.zeros(m * n, np.float32)), hip.upload(np.zeros(m * n, np.float32))
    nan_bits = int(np.array(np.nan, np.float32).view(np.uint32))
    with hip._active():
        for _ in range(3):
            hip._call("hp_h2d", ctypes.c_void_p(A.ptr), ctypes.c_void_p(a.ctypes.data), a.nbytes)
            hip._call("hp_fill", ctypes.c_void_p(C.ptr), m * n, 4, ctypes.c_uint64(nan_bits))
            hip._call("hp_gemm", 5, ctypes.c_void_p(A.ptr), ctypes.c_void_p(B.ptr), ctypes.c_void_p(C.ptr), m, n, k,
                      0, None, None, None)
            hip._call("hp_d2d", ctypes.c_void_p(D.ptr), ctypes.c_void_p(C.ptr), m * n * 4)
            hip._call("hp_fill", ctypes.c_void_p(A.ptr), m * k, 4, ctypes.c_uint64(0))
            got = np.empty(m * n, np.float32)
            hip._call("hp_d2h", ctypes.c_void_p(got.ctypes.data), ctypes.c_void_p(D.ptr), got.nbytes)
            got = got.reshape(m, n).astype(np.float64)
            assert np.all(np.abs(got - want) <= bound * scale + 1e-30)


@pytest.mark.parametrize("m,k,n", EDGE_CASES)
def test_edge_strips_against_float64_and_repeatable(hip, m, k, n):
    rng = np.random.default_rng(m * 5 + k + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    A, B = p.asarray(a, backend=hip), p.asarray(b, backend=hip)
    got = p.asnumpy(A @ B)
    np.testing.assert_array_equal(got, p.asnumpy(A @ B))
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4e-7 * np.sqrt(k) * 4 * scale + 1e-30)
    edge_rows = m % 256 if m > 256 and m % 256 <= 8 else 0
    edge_cols = n % 256 if n > 256 and n % 256 <= 8 else 0
    rows = np.r_[0:4, m - edge_rows - 1 : m]  # the last tile row and the strip
    cols = np.r_[0:4, n - edge_cols - 1 : n]
    hip_err, ref_err = _sampled_error_ratio(a, b, got, 64, m + n)
    assert hip_err <= 2 * ref_err
    strip = [(r, c) for r in rows for c in cols if r >= m - edge_rows or c >= n - edge_cols]
    if strip:
        rr, cc = np.array(strip).T
        ref = kernels.gemm_sequential(a, b, rr, cc)
        truth = np.array([float(exact.exact_dot(a[r], b[:, c])) for r, c in strip])
        mag = np.array([float(exact.exact_dot(np.abs(a[r]), np.abs(b[:, c]))) for r, c in strip])
        hip_strip = np.sqrt(np.mean(((got[rr, cc] - truth) / mag) ** 2))
        ref_strip = np.sqrt(np.mean(((ref - truth) / mag) ** 2))
        assert hip_strip <= 2 * ref_strip + 2.0**-24


# Strips in every operand layout: one code path over strides, one sum order,
# so a product of transposed operands equals the product of the materialized
# transposes bit for bit. (m, k, n): 7 rows and 7 columns; 8 and 8 over
# several K chunks of the rows strip; 2 columns with a K tail of 4 and no
# rows strip.
STRIP_LAYOUT_CASES = [(263, 1031, 263), (520, 2600, 1032), (1290, 4100, 770)]


@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("m,k,n", STRIP_LAYOUT_CASES)
def test_edge_strips_in_every_layout_match_materialized_transposes(hip, ta, tb, m, k, n):
    rng = np.random.default_rng(7 * m + k + 3 * n + 2 * ta + tb)
    left = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
    right = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    product = p.compile(lambda x, y: (x.T if ta else x) @ (y.T if tb else y))
    got = p.asnumpy(product(a, b))
    np.testing.assert_array_equal(got, p.asnumpy(product(a, b)))
    op_a, op_b = (left.T if ta else left), (right.T if tb else right)
    plain_a = p.asarray(np.ascontiguousarray(op_a), backend=hip)
    plain = p.asnumpy(plain_a @ p.asarray(np.ascontiguousarray(op_b), backend=hip))
    np.testing.assert_array_equal(got, plain)
    want = op_a.astype(np.float64) @ op_b.astype(np.float64)
    scale = np.abs(op_a).astype(np.float64) @ np.abs(op_b).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4e-7 * np.sqrt(k) * 4 * scale + 1e-30)


def _tile_rows_ratio(A, C, b, r0, r1):
    """Bound ratio of C[r0:r1] against float64 from A's rows (device gathers)."""
    return exact.product_bound_ratio(p.asnumpy(A[r0:r1]), b, p.asnumpy(C[r0:r1]), 4e-7)


def test_k_contiguous_operand_over_4_gib(hip):
    """Odd K with A of 4.4 GB: the 4-byte LDS-DMA descriptor of a tile spans
    that tile's own rows. A range through the end of the operand wrapped its
    32 bits here: the tile at row 7936 saw 1.83 MB of its 4.2 MB and loaded
    the rest as zeros."""
    m, k, n = 270000, 4099, 256
    rng = p.random.default_rng(17, backend=hip)
    A = rng.uniform(-1, 1, (m, k), dtype="float32")
    b = np.random.default_rng(18).uniform(-1, 1, (k, n)).astype(np.float32)
    C = A @ p.asarray(b, backend=hip)
    for r0 in (0, 7936, 8192, 134912, 269824):
        ratio = _tile_rows_ratio(A, C, b, r0, min(r0 + 256, m))
        assert ratio <= 1, f"rows from {r0}: {ratio}"


def test_k_edge_lanes_of_a_2_to_4_gib_operand_read_zero(hip):
    """Odd K with A of 2.46 GB whose rows from 131072 on are +inf. The lanes
    past K in the K-edge slice take an offset of 2^31 bytes that must lie
    outside the descriptor's range; with a range above 2^31 they read rows
    about 131000 further on (inf, times the +0 of B past K: NaN outputs)."""
    m, k, n = 150000, 4099, 256
    rng = p.random.default_rng(19, backend=hip)
    A = rng.uniform(-1, 1, (m, k), dtype="float32")
    first_inf = 131072
    with hip._active():
        hip._call("hp_fill", ctypes.c_void_p(A._data.ptr + first_inf * k * 4), (m - first_inf) * k, 4, 0x7F800000)
    b = np.random.default_rng(20).uniform(-1, 1, (k, n)).astype(np.float32)
    C = A @ p.asarray(b, backend=hip)
    for r0 in (0, 256, 4096, 16384, first_inf - 256):
        ratio = _tile_rows_ratio(A, C, b, r0, r0 + 256)
        assert ratio <= 1, f"rows from {r0}: {ratio}"
    assert not np.isfinite(p.asnumpy(C[first_inf : first_inf + 4])).any()
