"""GPU parity of the Philox generator (hp_philox / hp_philox_words) against the oracle.

Integer stream and the random/uniform transforms: bit-exact. Normal and
exponential: the reference's tolerance (3e-6 float32, 1e-13 float64;
reference tests/test_random.py:75-80). Inputs mirror the reference tests
(seeds 0 / 42 / 2^64-1, counters across the 2^32 carry and the end of the
2^64 space) plus BASELINE.json config 5 (2^28 samples from seed 42).
"""

import ctypes
from pathlib import Path

import numpy as np
import pytest

import openpacho as p
from oracle import philox
from oracle import numpy_backend as nb

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden" / "reference_rng.npz"
PARAMS = {"random": {}, "uniform": {"low": -3, "high": 7}, "normal": {"loc": 2, "scale": 3}, "exponential": {"scale": 2}}
ORACLE_ARGS = {"random": (0, 1), "uniform": (-3, 7), "normal": (2, 3), "exponential": (0, 2)}


def _words(backend, count, seed, start):
    out = backend.empty((count, 4), np.uint32)
    backend._call("hp_philox_words", ctypes.c_void_p(out.ptr), count, seed, start)
    host = np.empty((count, 4), np.uint32)
    backend._call("hp_d2h", ctypes.c_void_p(host.ctypes.data), ctypes.c_void_p(out.ptr), host.nbytes)
    return host


@pytest.mark.parametrize("seed", [0, 42, 2**64 - 1])
@pytest.mark.parametrize("start,count", [(0, 4097), (2**32 - 3, 1000), (2**32 - 300, 600), (2**64 - 7, 7)])
def test_integer_stream_is_bit_exact(hip, seed, start, count):
    np.testing.assert_array_equal(_words(hip, count, seed, start), philox.c_words(count, seed, start))


@pytest.mark.parametrize("dtype", ["float32", "float64"])
@pytest.mark.parametrize("start", [0, 2**32 - 3, 2**32 - 700, 2**32 - 2053, 2**64 - 1029])
@pytest.mark.parametrize("count", [1, 3, 1029, 4096, 2058])
def test_random_and_uniform_are_bit_exact(hip, dtype, start, count):
    # Counts below, at and past one workgroup's 2048 samples; start
    # 2^32 - 2053 with count 2058 puts the 2^32 carry inside the last,
    # partial workgroup.
    if start + count > 2**64:
        pytest.skip("past the counter space")
    for dist, kwargs in (("random", {}), ("uniform", {"low": -3, "high": 7})):
        rng = p.random.default_rng(2**64 - 1, backend=hip)
        rng._counter = start
        got = p.asnumpy(getattr(rng, dist)(size=count, dtype=dtype, **kwargs))
        want = philox.c_uniform(dtype, count, 2**64 - 1, start, dist, kwargs.get("low", 0), kwargs.get("high", 1))
        np.testing.assert_array_equal(got, want, err_msg=f"{dist} {dtype} start={start}")


@pytest.mark.parametrize("dtype", ["float32", "float64"])
@pytest.mark.parametrize("dist", ["normal", "exponential"])
def test_transcendental_transforms_within_reference_tolerance(hip, dtype, dist):
    tol = 3e-6 if dtype == "float32" else 1e-13
    for seed, start in ((2**64 - 1, 0), (42, 2**32 - 3)):
        rng = p.random.default_rng(seed, backend=hip)
        rng._counter = start
        got = p.asnumpy(getattr(rng, dist)(size=(33, 17), dtype=dtype, **PARAMS[dist]))
        first, second = ORACLE_ARGS[dist]
        want = nb.random(dist, dtype, (33, 17), seed, start, first, second)
        np.testing.assert_allclose(got, want, rtol=tol, atol=tol)


# Seed 42 draws the float32 unit u = 0 (word0 >> 8 == 0) at these counters,
# where -log1p(-0) = +0: exponential gives +0 and normal gives loc + scale * (+0 * cos).
ZERO_UNIT_COUNTERS = (25077234, 26967075)


@pytest.mark.parametrize("dist,first,second", [("exponential", 0.0, 2.0), ("normal", -0.0, 3.0), ("normal", 0.0, 3.0)])
def test_zero_unit_sample_has_the_reference_signed_zero(hip, dist, first, second):
    for counter in ZERO_UNIT_COUNTERS:
        assert philox.c_words(1, 42, counter)[0, 0] >> 8 == 0
        rng = p.random.default_rng(42, backend=hip)
        rng._counter = counter - 2
        kwargs = {"scale": second} if dist == "exponential" else {"loc": first, "scale": second}
        got = p.asnumpy(getattr(rng, dist)(size=5, dtype="float32", **kwargs))
        want = nb.random(dist, "float32", (5,), 42, counter - 2, first, second)
        assert got[2] == 0 and want[2] == 0
        np.testing.assert_array_equal(np.signbit(got), np.signbit(want), err_msg=f"{dist} counter={counter}")
        np.testing.assert_allclose(got, want, rtol=3e-6, atol=3e-6)


# Bounds that select each uniform kernel: a pre-scaled width with a median
# clamp where width * 2^-24 (2^-53) is exact and no bound is -0, the plain
# first + width * u with comparisons otherwise (signed zeros, subnormal widths).
UNIFORM_BOUNDS = [
    (-3.0, 7.0),
    (0.0, 1.0),
    (-0.0, 1.0),
    (0.0, 0.0),
    (-0.0, 0.0),
    (0.0, -0.0),
    (1.0, 1.0 + 2.0**-23),
    (1e-38, 3e-38),
    (-1.5e38, 1.5e38),
    (5e-324, 1e-322),
    (-2.0**-126, 2.0**-126),
    # low == 0 with a positive width: the kernel without offset or clamp
    (0.0, 3.7),
    (0.0, 1e30),
    (0.0, 3.4e38),
    (0.0, 2.0**-100),
    (-0.0, 5.5),
]


@pytest.mark.parametrize("dtype", ["float32", "float64"])
@pytest.mark.parametrize("low,high", UNIFORM_BOUNDS)
def test_uniform_bounds_are_bit_exact_on_both_kernels(hip, dtype, low, high):
    rng = p.random.default_rng(7, backend=hip)
    rng._counter = 2**32 - 1000
    got = p.asnumpy(rng.uniform(low, high, size=4099, dtype=dtype))
    want = philox.c_uniform(dtype, 4099, 7, 2**32 - 1000, "uniform", low, high)
    np.testing.assert_array_equal(got.view(f"u{got.itemsize}"), want.view(f"u{want.itemsize}"))


def test_matches_reference_numpy_backend_golden_samples(hip):
    with np.load(GOLDEN) as data:
        golden = {k: data[k] for k in data.files}
    for key, expected in golden.items():
        dist, dtype, seed, start = key.split("|")
        rng = p.random.default_rng(int(seed), backend=hip)
        rng._counter = int(start)
        got = p.asnumpy(getattr(rng, dist)(size=expected.shape[0], dtype=dtype, **PARAMS[dist]))
        if dist in ("random", "uniform"):
            np.testing.assert_array_equal(got, expected, err_msg=key)
        else:
            tol = 3e-6 if dtype == "float32" else 1e-13
            np.testing.assert_allclose(got, expected, rtol=tol, atol=tol, err_msg=key)


def test_split_calls_replay_the_same_stream(hip):
    for dist, kwargs in PARAMS.items():
        whole = p.asnumpy(getattr(p.random.default_rng(7, backend=hip), dist)(size=(33, 17), dtype="float32", **kwargs))
        replay = p.random.default_rng(7, backend=hip)
        parts = np.concatenate(
            [p.asnumpy(getattr(replay, dist)(size=n, dtype="float32", **kwargs)) for n in (1, 127, 0, 433)]
        )
        np.testing.assert_array_equal(parts, whole.ravel())


def test_carry_exhaustion_and_empty(hip):
    rng = p.random.default_rng(0, backend=hip)
    ref = p.random.default_rng(0, backend="numpy")
    for start in (2**32 - 3, 2**64 - 7):
        rng._counter = ref._counter = start
        np.testing.assert_array_equal(p.asnumpy(rng.random(7, dtype="float32")), p.asnumpy(ref.random(7, dtype="float32")))
    with pytest.raises(OverflowError):
        rng.random(1, dtype="float32")
    assert rng.random((0, 17), dtype="float32").shape == (0, 17)


def test_ranges_scalars_and_no_host_upload(hip, monkeypatch):
    def forbidden(*args, **kwargs):
        raise AssertionError("RNG must not upload a host-generated matrix")

    monkeypatch.setattr(hip, "upload", forbidden)
    rng = p.random.default_rng(17, backend=hip)
    assert rng.random(dtype="float32").shape == ()
    for low, high in [(-3, 7), (1, np.nextafter(np.float32(1), np.float32(2))), (2, 2)]:
        values = p.asnumpy(rng.uniform(low, high, (17, 33), dtype="float32"))
        assert (values >= low).all()
        assert (values < high).all() if high > low else (values == low).all()
    np.testing.assert_array_equal(p.asnumpy(rng.normal(3, 0, 65, dtype="float32")), 3)
    np.testing.assert_array_equal(p.asnumpy(rng.exponential(0, 65, dtype="float32")), 0)


@pytest.mark.parametrize("distribution", ["random", "uniform", "normal", "exponential"])
def test_statistical_smoke(hip, distribution):
    values = p.asnumpy(getattr(p.random.default_rng(47, backend=hip), distribution)(size=(513, 513), dtype="float32"))
    values = values.astype(float).ravel()
    assert np.all(np.isfinite(values))
    mean, variance = (0.5, 1 / 12) if distribution in ("random", "uniform") else ((0, 1) if distribution == "normal" else (1, 1))
    assert abs(values.mean() - mean) < 0.015
    assert abs(values.var() - variance) < 0.025
    assert abs(np.corrcoef(values[:-1], values[1:])[0, 1]) < 0.015


def test_config5_full_stream_2_28_random_is_bit_exact(hip):
    """2^28 samples from seed 42, whole stream compared."""
    n = 1 << 28
    got = p.asnumpy(p.random.default_rng(42, backend=hip).random(n, dtype="float32"))
    want = philox.c_uniform("float32", n, 42, 0)
    assert np.array_equal(got, want)
    # Chained calls continue the stream (counter n onwards).
    rng = p.random.default_rng(42, backend=hip)
    rng._counter = n
    tail = p.asnumpy(rng.uniform(size=4096, dtype="float32"))
    np.testing.assert_array_equal(tail, philox.c_uniform("float32", 4096, 42, n, "uniform", 0, 1))


@pytest.mark.parametrize("high", [1.0, 3.7])
def test_config5_full_size_uniform_from_zero_is_bit_exact(hip, high):
    # 2^28 samples reach every 24-bit unit numerator, including the largest,
    # so the unclamped uniform(0, w) kernel is checked where a clamp could bind.
    n = 1 << 28
    got = p.asnumpy(p.random.default_rng(42, backend=hip).uniform(0.0, high, n, dtype="float32"))
    want = philox.c_uniform("float32", n, 42, 0, "uniform", 0.0, high)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got.max() < np.float32(high)


def test_config5_full_size_normal_and_exponential_properties(hip):
    n = 1 << 28
    rng = p.random.default_rng(42, backend=hip)
    normal = rng.normal(0, 1, n, dtype="float32")
    expo = rng.exponential(1, n, dtype="float32")
    head = p.asnumpy(normal[:65536])
    want = nb.random("normal", "float32", (65536,), 42, 0, 0, 1)
    np.testing.assert_allclose(head, want, rtol=3e-6, atol=3e-6)
    for values, mean, var in ((normal, 0.0, 1.0), (expo, 1.0, 1.0)):
        total = float(p.sum(values.astype(np.float64)).item())
        square = float(p.sum((values * values).astype(np.float64)).item())
        m = total / n
        assert abs(m - mean) < 1e-3 and abs(square / n - m * m - var) < 2e-3
    tail = p.asnumpy(expo[n - 65536 :])
    want = nb.random("exponential", "float32", (65536,), 42, 2 * n - 65536, 0, 1)
    np.testing.assert_allclose(tail, want, rtol=3e-6, atol=3e-6)
