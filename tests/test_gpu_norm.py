"""GPU parity of the scaled Euclidean norms (hp_norm) against the oracles.

Cases follow reference tests/test_stable_norm.py:30-66 and test_cuda.py:442-465
(extreme constants, axes, chunk boundaries, NaN-over-Inf precedence, +0 for
zeros) plus the reference NumPy backend's golden outputs, and BASELINE.json
config 3 at full size (2^28 log-uniform elements; 65536x4096 rows) with the
hip error bounded by 2x the reference kernel's (oracle.kernels.norm_pair_merge).
"""

import math
from pathlib import Path

import numpy as np
import pytest

import openpacho as p
from oracle import exact, kernels

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden" / "reference_norm.npz"


@pytest.mark.parametrize("dtype,small,large", [(np.float32, 1e-25, 1e25), (np.float64, 1e-200, 1e200)])
@pytest.mark.parametrize("shape,axis", [((2,), None), ((3, 5, 7), (2, 0)), ((4099,), None), ((2, 0, 5), 1), ((), None), ((5, 9000), 1), ((9000, 3), 0)])
def test_scaled_norm_extreme_constants(hip, dtype, small, large, shape, axis):
    for scale in (small, large, 0.0):
        host = np.full(shape, scale, dtype=dtype)
        a = p.asarray(host, backend=hip)
        axes = tuple(range(len(shape))) if axis is None else (axis,) if isinstance(axis, int) else axis
        count = math.prod(shape[i] for i in axes)
        outshape = tuple(1 if i in axes else d for i, d in enumerate(shape))
        expected = np.full(outshape, abs(float(dtype(scale))) * math.sqrt(count), dtype=dtype)
        calculate = p.compile(lambda x: p.linalg.norm(x, axis=axis, keepdims=True))
        for result in (p.linalg.norm(a, axis=axis, keepdims=True), calculate(a)):
            assert result.dtype == np.dtype(dtype) and result.shape == expected.shape
            np.testing.assert_allclose(p.asnumpy(result), expected, rtol=2e-6, atol=0)


@pytest.mark.parametrize("values,expected", [([0.0, 0.0], 0.0), ([np.inf, 1.0], np.inf), ([np.nan, np.inf], np.nan), ([-3.0, 4.0], 5.0)])
def test_norm_special(hip, values, expected):
    actual = p.linalg.norm(p.asarray(values, backend=hip)).item()
    assert math.isnan(actual) if math.isnan(expected) else actual == expected


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("length", [4096, 4097, 8193, 20000])
def test_chunk_boundaries_and_nonfinite_precedence(hip, dtype, length):
    small, large = (1e-25, 1e25) if dtype == np.float32 else (1e-200, 1e200)
    host = np.zeros((6, length), dtype=dtype)
    host[0, [0, -1]] = large
    host[1, [0, -1]] = small
    host[2, -1] = np.inf
    host[3, 0], host[3, -1] = np.nan, np.inf
    host[4, 0], host[4, -1] = np.inf, np.nan
    host[5, [0, -1]] = -0.0
    value = p.asarray(host, backend=hip)
    expected = np.array([large * np.sqrt(2), small * np.sqrt(2), np.inf, np.nan, np.nan, 0.0], dtype=dtype).reshape(6, 1)
    calculate = p.compile(lambda a: p.linalg.norm(a, axis=1, keepdims=True))
    for result in (p.linalg.norm(value, axis=1, keepdims=True), calculate(value)):
        np.testing.assert_allclose(p.asnumpy(result), expected, rtol=2e-6, atol=0)
        assert not np.signbit(p.asnumpy(result)[5, 0])
    flat = p.asnumpy(p.linalg.norm(p.asarray(host[3], backend=hip)))
    assert np.isnan(flat)


def test_matches_reference_numpy_backend_golden(hip):
    with np.load(GOLDEN) as data:
        golden = {k: data[k] for k in data.files}
    for dtype in ("float32", "float64"):
        tol = 2e-6 if dtype == "float32" else 1e-14
        x = golden[f"loguniform|{dtype}|input"]
        np.testing.assert_allclose(p.asnumpy(p.linalg.norm(p.asarray(x, backend=hip))), golden[f"loguniform|{dtype}|norm"], rtol=tol)
        cube = golden[f"cube|{dtype}|input"]
        for axis in ((2, 0), 1, None):
            key = "none" if axis is None else str(axis)
            got = p.linalg.norm(p.asarray(cube, backend=hip), axis=axis, keepdims=True)
            np.testing.assert_allclose(p.asnumpy(got), golden[f"cube|{dtype}|axis={key}"], rtol=tol)
        rows = golden[f"rows|{dtype}|input"]
        np.testing.assert_allclose(p.asnumpy(p.linalg.norm(p.asarray(rows, backend=hip), axis=1)), golden[f"rows|{dtype}|norm"], rtol=tol)


def test_integer_input_promotes_to_float64(hip):
    result = p.linalg.norm(p.asarray(np.array([3, 4], np.int64), backend=hip))
    assert result.dtype == np.float64 and result.item() == 5.0


def _loguniform(n, decades, dtype, seed=2):
    rng = np.random.default_rng(seed)
    out = np.empty(n, dtype)
    for base in range(0, n, 1 << 24):
        m = min(1 << 24, n - base)
        mags = 10.0 ** rng.uniform(-decades, decades, m)
        signs = rng.integers(0, 2, m) * 2 - 1
        out[base : base + m] = (mags * signs).astype(dtype)
    return out


@pytest.mark.parametrize("dtype,decades,n", [(np.float32, 30, 1 << 28), (np.float64, 300, 1 << 28)])
def test_config3_flat_norm_full_size(hip, dtype, decades, n):
    x = _loguniform(n, decades, dtype)
    got = float(p.linalg.norm(p.asarray(x, backend=hip)).item())
    oracle = float(exact.norm_extended(x))
    hip_error = abs(got - oracle) / oracle
    # The reference pair-merge kernel's error on the same full vector (its
    # three passes over 65,536 chunk pairs, then 16, then 1), with one ulp
    # of the output as the floor: both results are rounded to dtype, and a
    # correctly rounded value is already up to half an ulp off.
    ref_error = abs(float(kernels.norm_pair_merge(x)) - oracle) / oracle
    assert hip_error <= max(2 * ref_error, np.finfo(dtype).eps), f"{hip_error} > 2 x {ref_error}"
    assert hip_error < 8 * np.finfo(dtype).eps


def test_config3_row_norms_full_size(hip):
    rows, cols = 65536, 4096
    rng = np.random.default_rng(2)
    x = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    got = p.asnumpy(p.linalg.norm(p.asarray(x, backend=hip), axis=1))
    assert got.shape == (rows,) and np.isfinite(got).all()
    oracle = np.empty(rows)
    for r in range(0, rows, 8192):
        block = x[r : r + 8192].astype(np.float64)
        oracle[r : r + 8192] = np.sqrt(np.einsum("ij,ij->i", block, block))
    rel = np.abs(got - oracle) / oracle
    sample = np.arange(0, rows, 1024)
    ref = np.array([kernels.norm_pair_merge(x[r]) for r in sample])
    ref_rel = np.abs(ref - oracle[sample]) / oracle[sample]
    assert np.sqrt(np.mean(rel[sample] ** 2)) <= 2 * np.sqrt(np.mean(ref_rel**2)) + 1e-9
    assert rel.max() < 1e-6


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_flat_norm_single_pass_repeats_across_grid_sizes(hip, dtype):
    # A flat norm is a row pass that writes one (exponent, sum) pair per
    # wave plus a merge launch over those pairs: calls of different grid
    # sizes in a row reuse the partial buffer and repeats are bitwise
    # identical.
    rng = np.random.default_rng(17)
    sizes = [1 << 22, 5000, 3 * 4096 + 1, 1 << 20, 2, (1 << 24) + 7]
    hosts = [rng.uniform(-1, 1, n).astype(dtype) for n in sizes]
    arrays = [p.asarray(h, backend=hip) for h in hosts]
    first = [p.asnumpy(p.linalg.norm(a)) for a in arrays]
    for _ in range(2):
        for a, want, host in zip(arrays, first, hosts):
            got = p.asnumpy(p.linalg.norm(a))
            assert got.tobytes() == want.tobytes()
            exact_norm = np.sqrt(np.sum(host.astype(np.float64) ** 2))
            assert abs(float(got) - exact_norm) <= 4 * np.finfo(dtype).eps * exact_norm
