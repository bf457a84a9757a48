"""GPU parity of the rest of the backend protocol: elementwise (hipRTC), gathers,
reductions, compiled plans (fused / map_reduce), residency and lifetime.

Integer, bool and index work is bit-exact against NumPy; floating results are
compared with the reference tests' tolerances (tests/test_cuda.py:55-64).
"""

import gc

import numpy as np
import pytest

import openpacho as p

pytestmark = pytest.mark.gpu

DTYPES = ["bool", "int32", "int64", "uint32", "uint64", "float32", "float64"]


@pytest.mark.parametrize("dtype", DTYPES)
def test_roundtrip_full_and_cast(hip, dtype):
    host = (np.arange(37) % 5).astype(dtype)
    value = p.asarray(host, backend=hip)
    assert value.backend == "hip" and value._data.ptr
    np.testing.assert_array_equal(p.asnumpy(value), host)
    np.testing.assert_array_equal(p.asnumpy(p.full((3, 4), 1, dtype=dtype, backend=hip)), np.ones((3, 4), dtype))
    for target in DTYPES:
        np.testing.assert_array_equal(p.asnumpy(value.astype(target)), host.astype(target))


BINARY = ["add", "subtract", "multiply", "true_divide", "power", "equal", "not_equal", "less", "less_equal", "greater", "greater_equal"]
UNARY = ["negative", "positive", "absolute", "sqrt", "exp", "log", "sin", "cos", "tanh", "isfinite"]


@pytest.mark.parametrize("dtype", ["int32", "int64", "uint32", "float32", "float64"])
def test_every_ufunc_matches_numpy(hip, dtype):
    rng = np.random.default_rng(4)
    if dtype.startswith("float"):
        x = rng.uniform(0.1, 3, (7, 9)).astype(dtype)
        y = rng.uniform(0.1, 3, (9,)).astype(dtype)
    else:
        x = rng.integers(1, 50, (7, 9)).astype(dtype)
        y = rng.integers(1, 50, (9,)).astype(dtype)
    a, b = p.asarray(x, backend=hip), p.asarray(y, backend=hip)
    for name in BINARY + UNARY:
        fn = getattr(np, name)
        if name == "power" and dtype[0] in "iu":
            with pytest.raises(NotImplementedError):
                fn(a, b)
            continue
        if name == "negative" and dtype[0] == "u":
            continue
        args = (a, b) if name in BINARY else (a,)
        host = (x, y) if name in BINARY else (x,)
        with np.errstate(all="ignore"):
            want = fn(*host)
        got = p.asnumpy(fn(*args))
        assert got.dtype == want.dtype, name
        if want.dtype.kind == "f":
            np.testing.assert_allclose(got, want, rtol=2e-6 if want.dtype == np.float32 else 1e-14, err_msg=name)
        else:
            np.testing.assert_array_equal(got, want, err_msg=name)


def test_integer_wraparound_and_scalars(hip):
    x = np.array([2**31 - 1, -(2**31), 5], np.int32)
    a = p.asarray(x, backend=hip)
    np.testing.assert_array_equal(p.asnumpy(a + 1), x + np.int32(1))
    np.testing.assert_array_equal(p.asnumpy(np.absolute(a)), np.absolute(x))
    np.testing.assert_array_equal(p.asnumpy(a * 3), x * np.int32(3))
    u = p.asarray(np.array([0, 1], np.uint64), backend=hip)
    np.testing.assert_array_equal(p.asnumpy(np.negative(u)), np.negative(np.array([0, 1], np.uint64)))
    w = p.where(a > 0, a, -1)
    np.testing.assert_array_equal(p.asnumpy(w), np.where(x > 0, x, -1))


def test_float_special_values(hip):
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, 3.4e38], np.float32)
    a = p.asarray(x, backend=hip)
    with np.errstate(all="ignore"):
        for fn in (np.negative, np.absolute, np.isfinite, np.sqrt, np.tanh):
            np.testing.assert_array_equal(p.asnumpy(fn(a)), fn(x))
        np.testing.assert_array_equal(p.asnumpy(a * 2), x * np.float32(2))
        np.testing.assert_array_equal(np.signbit(p.asnumpy(-a)), np.signbit(-x))


def test_gathers_are_bit_exact(hip):
    host = np.arange(2 * 3 * 4 * 5, dtype=np.float64).reshape(2, 3, 4, 5)
    host[0, 0, 0, 0] = -0.0
    a = p.asarray(host, backend=hip)
    for key in [(1, slice(None, None, -1)), (Ellipsis, 2), (slice(None), None, 1, slice(1, 4, 2)), (0, 0, 0, 0)]:
        np.testing.assert_array_equal(p.asnumpy(a[key]), host[key])
    np.testing.assert_array_equal(p.asnumpy(a.transpose(3, 1, 0, 2)), host.transpose(3, 1, 0, 2))
    np.testing.assert_array_equal(p.asnumpy(a.T), host.T)
    m = p.asarray(np.arange(20.0).reshape(4, 5), backend=hip)
    np.testing.assert_array_equal(p.asnumpy(p.diag(m, -1)), np.diag(np.arange(20.0).reshape(4, 5), -1))
    assert np.signbit(p.asnumpy(a[0, 0, 0, 0]))


@pytest.mark.parametrize("dtype", ["int32", "int64", "uint64", "float32", "float64"])
def test_reductions(hip, dtype):
    rng = np.random.default_rng(5)
    host = rng.integers(-50, 50, (6, 7, 300)).astype(dtype) if dtype[0] != "f" else rng.normal(size=(6, 7, 300)).astype(dtype)
    a = p.asarray(host, backend=hip)
    for axis in (None, 0, 1, 2, (0, 2), (1, 2)):
        got = p.asnumpy(p.sum(a, axis=axis))
        want = np.sum(host, axis=axis)
        if dtype[0] == "f":
            np.testing.assert_allclose(got, want, rtol=1e-5 if dtype == "float32" else 1e-12, atol=1e-4)
        else:
            np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(p.asnumpy(p.max(a, axis=axis)), np.max(host, axis=axis))
        np.testing.assert_array_equal(p.asnumpy(p.min(a, axis=axis)), np.min(host, axis=axis))
    long = rng.normal(size=50000).astype(np.float32) if dtype[0] == "f" else np.ones(50000, dtype)
    got = p.asnumpy(p.sum(p.asarray(long, backend=hip)))
    np.testing.assert_allclose(got, np.sum(long.astype(np.float64)), rtol=1e-5)


def test_extrema_nan_and_signed_zero_contract(hip):
    host = np.array([[0.0, -0.0, 3.0], [np.nan, 1.0, -2.0], [-0.0, 0.0, -0.0]], np.float32)
    a = p.asarray(host, backend=hip)
    mins, maxs = p.asnumpy(p.min(a, axis=1)), p.asnumpy(p.max(a, axis=1))
    assert mins[0] == 0 and np.signbit(mins[0]) and np.isnan(mins[1]) and np.signbit(mins[2])
    assert maxs[0] == 3 and np.isnan(maxs[1]) and maxs[2] == 0 and not np.signbit(maxs[2])
    b = p.asarray(np.array([True, False, True]), backend=hip)
    assert p.min(b).item() is False and p.max(b).item() is True
    assert p.sum(b, dtype=np.float32).item() == 2.0


def test_compile_fuses_rebinds_scalars_and_keeps_outputs(hip, monkeypatch):
    calls = []
    original = hip.elementwise

    def track(name, args, shape, dtype):
        calls.append(name)
        return original(name, args, shape, dtype)

    monkeypatch.setattr(hip, "elementwise", track)

    @p.compile
    def affine(value, scale):
        shifted = value * scale
        return shifted, shifted + 1.0

    host = np.arange(12, dtype=np.float32).reshape(3, 4)
    value = p.asarray(host, backend=hip)
    first, first_shifted = affine(value, 2.0)
    second, second_shifted = affine(value, 3.5)
    np.testing.assert_array_equal(p.asnumpy(first), host * 2)
    np.testing.assert_array_equal(p.asnumpy(first_shifted), host * 2 + 1)
    np.testing.assert_array_equal(p.asnumpy(second), host * 3.5)
    np.testing.assert_array_equal(p.asnumpy(second_shifted), host * 3.5 + 1)
    assert affine.cache_info()["misses"] == 1 and affine.cache_info()["hits"] >= 1
    assert not calls
    assert [s["kind"] for s in affine.explain(value, 4.0)["steps"]] == ["fused", "fused"]


def test_compiled_map_reduce_and_mean(hip):
    host = np.arange(8, dtype=np.float32)
    value = p.asarray(host, backend=hip)
    compiled = p.compile(lambda x: ((x + 1) * (x - 2)).sum())
    for _ in range(3):
        assert compiled(value).item() == 96.0
    assert [s["kind"] for s in compiled.explain(value)["steps"]] == ["map_reduce"]
    big = np.random.default_rng(1).normal(size=(3, 20000)).astype(np.float32)
    mr = p.compile(lambda x: p.mean(p.tanh(x * 0.5), axis=1))
    np.testing.assert_allclose(p.asnumpy(mr(p.asarray(big, backend=hip))), np.mean(np.tanh(big * np.float32(0.5)), axis=1), rtol=1e-5, atol=1e-6)
    ext = p.compile(lambda x: (p.max(x, axis=0), p.min(x * 2, axis=1)))
    arr = np.random.default_rng(2).normal(size=(5, 6)).astype(np.float32)
    got = ext(p.asarray(arr, backend=hip))
    np.testing.assert_array_equal(p.asnumpy(got[0]), arr.max(axis=0))
    np.testing.assert_array_equal(p.asnumpy(got[1]), (arr * 2).min(axis=1))


def test_mlp_forward_small_against_float64(hip):
    rng = p.random.default_rng(42, backend=hip)
    x = rng.uniform(-1, 1, (64, 96), dtype="float32")
    widths = (96, 128, 128, 32)
    params = []
    for fan_in, fan_out in zip(widths[:-1], widths[1:]):
        params += [rng.normal(0, (1 / fan_in) ** 0.5, (fan_in, fan_out), dtype="float32"), p.zeros(fan_out, dtype=np.float32, backend=hip)]

    @p.compile
    def mlp(x, w1, b1, w2, b2, w3, b3):
        h = p.tanh(x @ w1 + b1)
        h = p.tanh(h @ w2 + b2)
        out = p.tanh(h @ w3 + b3)
        return p.mean(out, axis=1)

    got = p.asnumpy(mlp(x, *params))
    kinds = [s["kind"] for s in mlp.explain(x, *params)["steps"]]
    assert kinds == ["matmul", "fused", "matmul", "fused", "matmul", "map_reduce", "fused"]
    h = p.asnumpy(x).astype(np.float64)
    hosts = [p.asnumpy(v).astype(np.float64) for v in params]
    for w, b in zip(hosts[0::2], hosts[1::2]):
        h = np.tanh(h @ w + b)
    np.testing.assert_allclose(got, h.mean(axis=1), rtol=1e-5, atol=1e-6)


def test_operations_do_not_download_or_fall_back(hip, monkeypatch):
    host = np.arange(12, dtype=np.float32).reshape(3, 4) / 5
    value = p.asarray(host, backend=hip)
    original = np.asarray

    def forbid(candidate, *args, **kwargs):
        if isinstance(candidate, p.ndarray):
            raise TypeError("implicit NumPy conversion")
        return original(candidate, *args, **kwargs)

    def forbid_download(*args, **kwargs):
        raise AssertionError("host download")

    monkeypatch.setattr(np, "asarray", forbid)
    monkeypatch.setattr(hip, "download", forbid_download)
    results = (
        value + 1.0,
        np.add(value, 2.0),
        p.sum(value, axis=0),
        p.mean(value, axis=1),
        value[::-1, ::2],
        value.T,
        value @ value.T,
        p.linalg.norm(value),
        p.compile(lambda a: p.linalg.norm(a, axis=1))(value),
        p.random.default_rng(1, backend=hip).normal(size=4, dtype="float32"),
    )
    assert all(r._backend is hip for r in results)


def test_pool_recycles_and_release_keeps_live_arrays(hip):
    hip.synchronize()
    live = p.asarray(np.arange(16, dtype=np.float32), backend=hip)
    temporary = p.asarray(np.arange(16, dtype=np.float32) + 1, backend=hip)
    del temporary
    gc.collect()
    stats = hip.pool_stats()
    assert stats["cached_items"] >= 1
    hip.release_cached_memory()
    assert hip.pool_stats()["cached_items"] == 0
    np.testing.assert_array_equal(p.asnumpy(live), np.arange(16, dtype=np.float32))


def test_small_blocks_wait_on_host_and_return_to_the_pool(hip):
    """Returned blocks of <= 512 bytes (one pool size class) are reused from
    the host without a library call; at most 64 wait there, the rest go back
    to the pool, and statistics and releases see the pool after the host list
    is handed back."""
    from openpacho import _hip

    gc.collect()
    hip.synchronize()
    hip.release_cached_memory()
    base = hip.pool_stats()
    arrays = [p.full((7,), float(i), dtype=np.float32, backend=hip) for i in range(_hip._SMALL_KEPT + 8)]
    addresses = {a._data.ptr for a in arrays}
    assert len(addresses) == len(arrays)
    del arrays
    gc.collect()
    kept = list(hip._small)
    assert len(kept) == _hip._SMALL_KEPT and set(kept) <= addresses
    reused = p.full((), 2.5, dtype=np.float64, backend=hip)  # a 0-d float64 takes a float32 vector's block
    assert reused._data.ptr == kept[-1]
    assert float(p.asnumpy(reused)) == 2.5
    x = p.asarray(np.arange(1, 65, dtype=np.float32), backend=hip)
    dots = [p.dot(x, x) for _ in range(3)]
    assert len({d._data.ptr for d in dots}) == 3
    assert all(float(p.asnumpy(d)) == float(np.dot(np.arange(1, 65.0), np.arange(1, 65.0))) for d in dots)
    del dots, reused, x
    gc.collect()
    stats = hip.pool_stats()
    assert not hip._small
    assert stats["live_items"] == base["live_items"]
    assert stats["cached_items"] == base["cached_items"] + len(addresses)
    hip.release_cached_memory()
    assert hip.pool_stats()["cached_items"] == 0


def test_inflight_free_is_stream_ordered(hip):
    # Free an input right after launching its consumer; the next allocation of
    # the same size may reuse the block but runs after the consumer.
    for _ in range(20):
        a = p.asarray(np.full(1 << 20, 3.0, np.float32), backend=hip)
        b = a * 2.0
        del a
        c = p.full(1 << 20, 7.0, dtype=np.float32, backend=hip)
        np.testing.assert_array_equal(p.asnumpy(b)[:4], 6.0)
        np.testing.assert_array_equal(p.asnumpy(c)[-4:], 7.0)


def test_fault_injection_raises_and_burns_rng_range(hip):
    rng = p.random.default_rng(5, backend=hip)
    hip._lib.hp_debug_fail_next(hip._ctx, 1)
    with pytest.raises(RuntimeError, match="injected"):
        rng.random(10, dtype="float32")
    assert rng._counter == 10
    reference = p.random.default_rng(5, backend="numpy")
    reference.random(10, dtype="float32")
    np.testing.assert_array_equal(p.asnumpy(rng.random(33, dtype="float32")), p.asnumpy(reference.random(33, dtype="float32")))


def test_invalid_arguments_are_errors_not_faults(hip):
    with pytest.raises(ValueError):
        hip._call("hp_gemm", 5, None, None, None, -1, 1, 1, 0, None, None, None)
    with pytest.raises(ValueError):
        hip._call("hp_philox", 5, 0, None, 10, 0, 2**64 - 5, 0.0, 1.0, 1.0)
    with pytest.raises(ValueError):
        p.empty(2**31, dtype=np.float32, backend=hip)


def test_close_is_idempotent_and_invalidates_arrays():
    from openpacho._hip import HIPBackend

    owned = HIPBackend()
    live = p.asarray([1.0, 2.0, 3.0], dtype=np.float32, backend=owned)
    assert p.asnumpy(live + 1.0).tolist() == [2.0, 3.0, 4.0]
    owned.close()
    owned.close()
    assert live._data.ptr == 0
    with pytest.raises(RuntimeError):
        p.asnumpy(live)
    with pytest.raises(RuntimeError):
        live + 1.0


def test_pool_respects_byte_limit(hip):
    # Reference tests/test_cuda.py:598-612: freed blocks stay cached only
    # within the pool's byte limit.
    previous = hip.pool_limit
    try:
        hip.release_cached_memory()
        hip.pool_limit = 1024
        for _ in range(12):
            temporary = p.empty((128,), dtype=np.float32, backend=hip)
            del temporary
        gc.collect()
        hip.synchronize()
        stats = hip.pool_stats()
        assert stats["cached_bytes"] <= hip.pool_limit and stats["cached_items"] <= 128
        large = p.full(4096, 2.0, dtype=np.float32, backend=hip)  # above the limit: freed, not cached
        del large
        gc.collect()
        assert hip.pool_stats()["cached_bytes"] <= 1024
        with pytest.raises(ValueError):
            hip.pool_limit = -1
    finally:
        hip.pool_limit = previous
        hip.release_cached_memory()


def test_bool_fill_rebinds_without_changing_previous_output(hip):
    # Reference tests/test_cuda.py:530-534.
    first = p.full(33, True, dtype=np.bool_, backend=hip)
    second = p.full(33, False, dtype=np.bool_, backend=hip)
    np.testing.assert_array_equal(p.asnumpy(first), np.ones(33, dtype=np.bool_))
    np.testing.assert_array_equal(p.asnumpy(second), np.zeros(33, dtype=np.bool_))
