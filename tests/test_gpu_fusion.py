"""Compiled/fused plans on hip keep public semantics, precision and lifetimes.

Contracts (reference tests/test_cuda_fusion.py:28-175), for the hip lowering
(hipRTC sources of _hip_lowering.py):
1. a reduction of a private elementwise producer is one map_reduce step and
   is exact over any axes, tails and empty shapes (small integers, so every
   order gives the same sum);
2. dynamic scalars rebind without retracing, including through broadcasting
   and a float64 result;
3. float32 rounding happens before float64 accumulation;
4. plans upload nothing and retain no input; outputs shared between steps are
   computed once;
5. IEEE special values and signed zeros pass through fused transcendentals;
6. no hidden FMA contraction, and a compiled sum rounds like the eager one;
7. one plan replays correctly from several threads;
8. (hip) a product read by a fused group stays a matmul step;
9. (hip) a sum with a bool accumulator is a logical or, eager and compiled.
"""

import gc
import weakref
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import openpacho as p

pytestmark = pytest.mark.gpu


def _kinds(compiled, *args):
    return [step["kind"] for step in compiled.explain(*args)["steps"]]


# ---- 1 ---------------------------------------------------------------------------

REDUCTIONS = [
    ((8193,), None),
    ((7, 40), (1,)),
    ((4, 3, 31), (0, 2)),
    ((11, 5, 13), (1, 2)),
    ((65, 2, 70), (0,)),
    ((3, 4), ()),
    ((), None),
    ((3, 0, 2), (1,)),
    ((0, 5000), (1,)),
    ((2, 30001), (1,)),
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape,axes", REDUCTIONS)
def test_map_reduce_is_exact_over_axes_tails_and_empty_shapes(hip, dtype, shape, axes):
    host = ((np.arange(int(np.prod(shape))) % 5) - 2).astype(dtype).reshape(shape)
    compiled = p.compile(lambda a: np.sum(a * a - a + 1, axis=axes, keepdims=True))
    x = p.asarray(host, backend=hip)
    got = compiled(x)
    assert got.dtype == dtype
    np.testing.assert_array_equal(p.asnumpy(got), np.sum(host * host - host + 1, axis=axes, keepdims=True))
    assert _kinds(compiled, x) == ["map_reduce"]


# ---- 2, 3 ------------------------------------------------------------------------


def test_scalars_rebind_through_broadcast_and_promotion(hip):
    host = (np.arange(3 * 50 * 6, dtype=np.float32).reshape(3, 50, 6) - 400) / 512
    offsets = np.linspace(-1, 1, 6)  # float64: the result is float64
    compiled = p.compile(lambda a, b, scale: np.mean((a - b) * scale, axis=(0, 1)))
    a, b = p.asarray(host, backend=hip), p.asarray(offsets, backend=hip)
    for scale in (0.25, -3.0, 7.5):
        got = compiled(a, b, scale)
        assert got.dtype == np.float64 and got.shape == (6,)
        np.testing.assert_allclose(p.asnumpy(got), np.mean((host - offsets) * scale, axis=(0, 1)), rtol=1e-13, atol=1e-15)
    assert compiled.cache_info()["misses"] == 1 and compiled.cache_info()["hits"] == 2


def test_float32_products_round_before_a_float64_sum(hip):
    host = np.linspace(-2.5, 4.1, 12345, dtype=np.float32)
    compiled = p.compile(lambda a: np.sum(a * a, dtype=np.float64))
    want = np.sum((host * host).astype(np.float64))  # rounded in float32 first
    np.testing.assert_allclose(p.asnumpy(compiled(p.asarray(host, backend=hip))), want, rtol=1e-14)
    # A float64 -> float32 -> float64 round trip keeps exactly the float32 rounding.
    values = np.array([1 + 2**-30, -(1 + 2**-24 + 2**-40), 3e-46, 1e39], np.float64)
    narrowed = p.compile(lambda a: a.astype(np.float32).astype(np.float64))
    with np.errstate(over="ignore"):
        want = values.astype(np.float32).astype(np.float64)
    np.testing.assert_array_equal(p.asnumpy(narrowed(p.asarray(values, backend=hip))), want)


# ---- 4 ---------------------------------------------------------------------------


def test_plans_upload_nothing_keep_nothing_and_share_outputs(hip, monkeypatch):
    host = (np.arange(8191, dtype=np.float32) - 4000) / 256
    x = p.asarray(host, backend=hip)
    monkeypatch.setattr(hip, "upload", lambda *args: pytest.fail("a plan uploaded data"))

    @p.compile
    def several(a, shift):
        moved = a - shift
        return moved, np.sum(moved * moved), moved * 0.5

    assert _kinds(several, x, 1.0) == ["fused", "map_reduce", "fused"]
    for shift in (1.0, -2.0):
        moved = host - np.float32(shift)
        for got, want in zip(several(x, shift), (moved, np.sum(moved.astype(np.float64) ** 2), moved * 0.5)):
            np.testing.assert_allclose(p.asnumpy(got), want, rtol=2e-6)
    storage = weakref.ref(x._data)
    del x, got
    hip.synchronize()
    gc.collect()
    assert storage() is None


# ---- 5, 6 ------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_special_values_and_signed_zeros_through_fused_transcendentals(hip, dtype):
    host = np.array([0.0, -0.0, 1.5, -2.25, np.inf, -np.inf, np.nan, 1e-300 if dtype == np.float64 else 1e-40], dtype)
    x = p.asarray(host, backend=hip)
    with np.errstate(all="ignore"):
        def damped(a):
            return np.cos(a) - np.exp(-(a * a)) * np.sin(a)

        np.testing.assert_allclose(p.asnumpy(p.fuse(damped)(x)), damped(host), rtol=2e-6, equal_nan=True)
        predicate = p.fuse(lambda a: np.isfinite(a) != (a < 0))
        np.testing.assert_array_equal(p.asnumpy(predicate(x)), np.isfinite(host) != (host < 0))
    negated = p.asnumpy(p.fuse(lambda a: -a * dtype(2))(x))
    np.testing.assert_array_equal(np.signbit(negated[:2]), [True, False])
    assert p.asnumpy(p.fuse(lambda a: np.isfinite(a >= 0))(x)).all()


def test_no_contraction_and_eager_rounding_of_compiled_sums(hip):
    eps = 2.0**-23
    a = p.asarray(np.array([1 + eps, 1 + 2 * eps], np.float32), backend=hip)
    b = p.asarray(np.array([1 - eps, 1 - 2 * eps], np.float32), backend=hip)
    compiled = p.compile(lambda a, b: a * b - 1)
    got = p.asnumpy(compiled(a, b))
    # (1+e)(1-e) = 1 - e^2 rounds to 1 (and 1 - 4e^2 to 1) before the
    # subtraction; a fused multiply-add would keep -e^2.
    np.testing.assert_array_equal(got, [0, 0])
    np.testing.assert_array_equal(got, p.asnumpy(a * b - 1))
    host = np.tile(np.array([3e19, 2, -3e19, 5, 7e-39, -1], np.float32), 1501)
    x = p.asarray(host, backend=hip)
    total = p.compile(lambda x: np.sum(x * 0.25 + 1))
    np.testing.assert_array_equal(p.asnumpy(total(x)), p.asnumpy(np.sum(x * 0.25 + 1)))


# ---- 7, 8 ------------------------------------------------------------------------


def test_a_product_read_by_a_fused_group_is_a_matmul_and_threads_replay(hip, monkeypatch):
    rng = np.random.default_rng(15)
    host_a = rng.uniform(-1, 1, (41, 19)).astype(np.float32)
    host_x = rng.uniform(-1, 1, 19).astype(np.float32)
    host_b = rng.uniform(-1, 1, 41).astype(np.float32)
    a, x, b = (p.asarray(v, backend=hip) for v in (host_a, host_x, host_b))
    products = []
    real = hip.matmul
    monkeypatch.setattr(hip, "matmul", lambda *args: (products.append(args), real(*args))[1])
    # The subtraction is inlined into the fused multiply, so the product is
    # a leaf of that group (a plain matmul step), as in the reference plans.
    compiled = p.compile(lambda a, x, b, rate: (b - a @ x) * rate)
    assert _kinds(compiled, a, x, b, 1.0) == ["matmul", "fused"]
    rates = (0.5, -1.0, 2.0, 3.5, 4.25, -0.75)
    with ThreadPoolExecutor(max_workers=3) as pool:
        results = list(pool.map(lambda r: p.asnumpy(compiled(a, x, b, r)), rates))
    for got, rate in zip(results, rates):
        want = (host_b.astype(np.float64) - host_a.astype(np.float64) @ host_x) * rate
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    assert len(products) == len(rates)


# ---- 9 ---------------------------------------------------------------------------


@pytest.mark.parametrize("shape,axis", [((6,), None), ((4, 20001), 1), ((20001, 4), 0), ((3, 0), 1), ((0, 3), 0)])
def test_a_bool_accumulator_sums_as_a_logical_or(hip, shape, axis):
    host = np.random.default_rng(9).choice(np.array([0, 0, 0, 3, -2, np.nan], np.float32), size=shape)
    if host.size and host.ndim == 2:
        host[(0, slice(None)) if axis == 1 else (slice(None), 0)] = 0  # one all-false line
    x = p.asarray(host, backend=hip)
    want = np.sum(host > 0, axis=axis, dtype=np.bool_)
    for got in (p.sum(x > 0, axis=axis, dtype=np.bool_), p.compile(lambda a: np.sum(a > 0, axis=axis, dtype=np.bool_))(x)):
        assert got.dtype == np.bool_ and got.shape == want.shape
        np.testing.assert_array_equal(p.asnumpy(got), want)
    truthy = p.compile(lambda a: np.sum(a, axis=axis, dtype=np.bool_))(x)  # NaN is true
    np.testing.assert_array_equal(p.asnumpy(truthy), np.sum(host, axis=axis, dtype=np.bool_))
    counted = p.compile(lambda a: np.sum(a > 0, axis=axis))(x)  # a numeric accumulator counts
    np.testing.assert_array_equal(p.asnumpy(counted), np.sum(host > 0, axis=axis))
    assert counted.dtype == np.sum(host > 0, axis=axis).dtype
