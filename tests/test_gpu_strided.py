"""GPU parity of reductions and norms over a strided axis (inner > 1).

The reference splits any reduced axis into fixed chunks, one block each
(reference _cuda.py:449-491; norms through _norm.py:53-118). Here the axis
is split into row chunks across workgroups with lanes on adjacent columns,
then per-chunk partials merge in a fixed order. Checked against NumPy (exact
for integers, extrema and special values), against float64 for sums, and
against the extended-precision norm oracle; repeated calls must agree bit for
bit. Shapes cover wide axes (16-byte loads), narrow ones (several rows per
workgroup step), odd widths (one element per lane), outer > 1, axes short
enough for the one-thread-per-output path, and the 1 GiB case.
"""

import ctypes

import numpy as np
import pytest

import openpacho as p
from oracle import exact

pytestmark = pytest.mark.gpu

SHAPES = [
    (8192, 1024),  # wide: 16-byte loads, one row per workgroup step
    (1000, 4),  # narrow: 64 rows per step of a 256-thread workgroup
    (100003, 3),  # odd width: one element per lane, 85 rows per step
    (5000, 1000),  # width not a multiple of 4 (scalar loads), 4 column blocks
    (777, 2),  # short axis: one thread per output
    (40, 600),  # short axis, wide
]


def _host(shape, dtype, seed):
    rng = np.random.default_rng(seed)
    if np.dtype(dtype).kind == "f":
        return rng.normal(size=shape).astype(dtype)
    info = np.iinfo(dtype)
    return rng.integers(max(info.min, -1000), min(info.max, 1000), shape, dtype=dtype, endpoint=True)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.int64, np.uint32, np.uint64])
def test_axis0_sum_min_max(hip, shape, dtype):
    host = _host(shape, dtype, shape[0] + shape[1])
    a = p.asarray(host, backend=hip)
    got = p.asnumpy(p.sum(a, axis=0))
    if np.dtype(dtype).kind == "f":
        want = host.astype(np.float64).sum(axis=0)
        scale = np.abs(host).astype(np.float64).sum(axis=0)
        eps = np.finfo(dtype).eps
        # A blocked sum's error is at most ~(log-depth + rows per thread) ulps of
        # the sum of magnitudes; 64 eps covers every plan here.
        assert np.all(np.abs(got - want) <= 64 * eps * scale)
    else:
        np.testing.assert_array_equal(got, host.sum(axis=0, dtype=dtype))
    np.testing.assert_array_equal(p.asnumpy(p.min(a, axis=0)), host.min(axis=0))
    np.testing.assert_array_equal(p.asnumpy(p.max(a, axis=0)), host.max(axis=0))
    again = p.asnumpy(p.sum(a, axis=0))
    assert again.tobytes() == got.tobytes()


@pytest.mark.parametrize("shape,axis", [((6, 3000, 40), 1), ((3, 50, 7, 20), 1), ((2, 4096, 257), 1), ((64, 9, 33), 0)])
def test_middle_axes_with_outer(hip, shape, axis):
    host = _host(shape, np.float32, 11)
    a = p.asarray(host, backend=hip)
    got = p.asnumpy(p.sum(a, axis=axis))
    want = host.astype(np.float64).sum(axis=axis)
    scale = np.abs(host).astype(np.float64).sum(axis=axis)
    assert np.all(np.abs(got - want) <= 64 * np.finfo(np.float32).eps * scale)
    np.testing.assert_array_equal(p.asnumpy(p.max(a, axis=axis)), host.max(axis=axis))
    norm = p.asnumpy(p.linalg.norm(a, axis=axis))
    ref = np.sqrt(np.sum(np.square(host.astype(np.float64)), axis=axis))
    np.testing.assert_allclose(norm, ref, rtol=4e-6, atol=0)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_infinities_and_overflow_sum_like_numpy(hip, dtype):
    big = np.finfo(dtype).max / 2 * 1.5
    host = np.zeros((5, 6), dtype)
    host[:, 0] = [1, np.inf, 2, 0, 0]
    host[:, 1] = [1, -np.inf, 2, 0, 0]
    host[:, 2] = [np.inf, 1, -np.inf, 0, 0]
    host[:, 3] = [big, big, 0, 0, 0]  # overflows to +inf
    host[:, 4] = [-big, -big, 0, 0, 0]
    host[:, 5] = [np.nan, 1, np.inf, 0, 0]
    for rows in (5, 700):  # one-thread-per-output path and the chunked path
        tall = np.zeros((rows, 6), dtype)
        tall[:5] = host
        a = p.asarray(tall, backend=hip)
        with np.errstate(all="ignore"):
            want = np.sum(tall, axis=0)
        got = p.asnumpy(p.sum(a, axis=0))
        np.testing.assert_array_equal(got, want)
        assert np.isposinf(got[0]) and np.isneginf(got[1]) and np.isnan(got[2])
        assert np.isposinf(got[3]) and np.isneginf(got[4]) and np.isnan(got[5])


def test_int64_sum_wraps_like_numpy(hip):
    host = np.full((3000, 5), np.iinfo(np.int64).max // 1000, np.int64)
    host[:, 1] = np.iinfo(np.int64).min // 999
    a = p.asarray(host, backend=hip)
    with np.errstate(over="ignore"):
        want = host.sum(axis=0)
    np.testing.assert_array_equal(p.asnumpy(p.sum(a, axis=0)), want)
    flat = p.asarray(host.ravel(), backend=hip)  # contiguous-row path
    np.testing.assert_array_equal(p.asnumpy(p.sum(flat)), host.ravel().sum())


def test_extrema_nan_signed_zero_and_bool_columns(hip):
    host = np.zeros((3000, 4), np.float32)
    host[:, 0] = -0.0
    host[1234, 1] = -0.0
    host[:, 2] = np.arange(3000)
    host[2999, 2] = np.nan
    host[:, 3] = -np.arange(3000)
    a = p.asarray(host, backend=hip)
    mins, maxs = p.asnumpy(p.min(a, axis=0)), p.asnumpy(p.max(a, axis=0))
    assert np.signbit(mins[0]) and np.signbit(maxs[0])  # all -0: both -0
    assert np.signbit(mins[1]) and not np.signbit(maxs[1])  # mixed zeros
    assert np.isnan(mins[2]) and np.isnan(maxs[2])
    assert mins[3] == -2999 and maxs[3] == 0
    flags = np.zeros((5000, 3), bool)
    flags[:, 1] = True
    flags[4321, 2] = True
    b = p.asarray(flags, backend=hip)
    np.testing.assert_array_equal(p.asnumpy(p.min(b, axis=0)), flags.min(axis=0))
    np.testing.assert_array_equal(p.asnumpy(p.max(b, axis=0)), flags.max(axis=0))


@pytest.mark.parametrize("shape", [(8192, 1024), (100003, 3), (5000, 1000), (777, 2), (300, 5)])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_axis0_norm_one_read_matches_extended_oracle(hip, shape, dtype):
    rng = np.random.default_rng(17)
    decades = 30 if dtype == np.float32 else 300
    host = (10.0 ** rng.uniform(-decades, decades, shape) * rng.choice([-1, 1], shape)).astype(dtype)
    a = p.asarray(host, backend=hip)
    got = p.asnumpy(p.linalg.norm(a, axis=0))
    want = exact.norm_extended(host, axis=0)
    rel = np.abs(got.astype(np.longdouble) - want) / want
    assert float(rel.max()) < 8 * np.finfo(dtype).eps
    again = p.asnumpy(p.linalg.norm(a, axis=0))
    assert again.tobytes() == got.tobytes()


def test_norm_columns_special_values(hip):
    host = np.ones((3000, 6), np.float32)
    host[:, 0] = 0.0
    host[7, 1] = np.inf
    host[7, 2], host[9, 2] = np.inf, np.nan  # NaN beats Inf
    host[:, 3] = 1e-45  # subnormals, no underflow to 0
    host[:, 4] = 3e36  # squares overflow float32; the norm does not
    host[2999, 5] = np.nan
    a = p.asarray(host, backend=hip)
    got = p.asnumpy(p.linalg.norm(a, axis=0))
    assert got[0] == 0 and not np.signbit(got[0])
    assert np.isposinf(got[1]) and np.isnan(got[2]) and np.isnan(got[5])
    np.testing.assert_allclose(got[3], np.sqrt(3000) * 1.4e-45, rtol=0.01)
    np.testing.assert_allclose(got[4], np.sqrt(3000.0) * np.float32(3e36), rtol=1e-6)


def test_one_gib_axis0_reductions(hip):
    rows, cols = 262144, 1024
    data = p.random.default_rng(3, backend=hip).uniform(-1, 1, (rows, cols), dtype="float32")
    host = p.asnumpy(data)
    got = p.asnumpy(p.sum(data, axis=0))
    want = host.astype(np.float64).sum(axis=0)
    scale = np.abs(host).astype(np.float64).sum(axis=0)
    assert np.all(np.abs(got - want) <= 64 * np.finfo(np.float32).eps * scale)
    np.testing.assert_array_equal(p.asnumpy(p.max(data, axis=0)), host.max(axis=0))
    np.testing.assert_array_equal(p.asnumpy(p.min(data, axis=0)), host.min(axis=0))
    norm = p.asnumpy(p.linalg.norm(data, axis=0))
    ref = np.sqrt(np.einsum("ij,ij->j", host.astype(np.float64), host.astype(np.float64)))
    np.testing.assert_allclose(norm, ref, rtol=2e-6, atol=0)


def test_noalloc_strided_norm_matches_hp_norm(hip):
    from openpacho import _hip_lib

    rng = np.random.default_rng(8)
    for shape in ((262144, 1024), (5000, 1000), (777, 2)):  # the largest plans its partials below 8 MiB
        host = rng.uniform(-1, 1, shape).astype(np.float32)
        x = p.asarray(host, backend=hip)
        outs = [p.empty((shape[1],), dtype=np.float32, backend=hip) for _ in range(2)]
        with hip._active():
            for entry, out in zip(("hp_norm", "hp_norm_noalloc"), outs):
                hip._call(entry, _hip_lib.DTYPE_CODES[np.dtype(np.float32)], *hip._ptrs(x, out), 1, shape[0], shape[1])
        first, second = (p.asnumpy(o) for o in outs)
        assert first.tobytes() == second.tobytes()
        del x
