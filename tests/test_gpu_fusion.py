"""Compiled/fused plans on hip keep public semantics, precision and lifetimes.

Restates the contracts of reference tests/test_cuda_fusion.py:28-175 for the
hip lowering (hipRTC sources of _hip_lowering.py): exact reductions over axes,
tails and empty shapes; dynamic scalar rebinding without retracing; float32
rounding before float64 accumulation; no uploads and no retained inputs; IEEE
special values and signed zeros through fused transcendentals; no hidden FMA
contraction and the eager reduction order; thread-safe replays of one plan.
Where hip differs from the reference's initial CUDA backend it says so: a
``b - a @ x`` that is not itself inlined into a fused group is one
residual_matvec step (tests/test_gpu_gemv.py).
"""

import gc
import weakref
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import openpacho as p

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize(
    "shape,axes",
    [
        ((9001,), None),
        ((5, 32), (-1,)),
        ((3, 2, 33), (1, 2)),
        ((9, 7, 39), (0, 2)),
        ((67, 3, 69), (0, 2)),
        ((2, 3), ()),
        ((), None),
        ((2, 0, 3), (1,)),
        ((0, 4097), (1,)),
        ((3, 20000), (1,)),
    ],
)
def test_axes_tails_and_empty_reductions(hip, dtype, shape, axes):
    host = (np.arange(int(np.prod(shape))) % 7).astype(dtype).reshape(shape)
    operation = p.compile(lambda a: np.sum(a * a + 2, axis=axes, keepdims=True))
    a = p.asarray(host, backend=hip)
    actual = operation(a)
    assert actual.dtype == host.dtype
    np.testing.assert_array_equal(p.asnumpy(actual), np.sum(host * host + 2, axis=axes, keepdims=True))
    assert [step["kind"] for step in operation.explain(a)["steps"]] == ["map_reduce"]


def test_broadcast_mean_rebinds_scalars_and_dtypes(hip):
    host = np.arange(4 * 67 * 9, dtype=np.float32).reshape(4, 67, 9) / 1000
    bias = np.arange(9, dtype=np.float64)
    operation = p.compile(lambda a, b, rate: np.mean((a + b) * rate, axis=(0, 2)))
    a, b = [p.asarray(x, backend=hip) for x in (host, bias)]
    for rate in (0.5, 1.75):
        actual = operation(a, b, rate)
        assert actual.dtype == np.float64
        np.testing.assert_allclose(p.asnumpy(actual), np.mean((host + bias) * rate, axis=(0, 2)), rtol=1e-13)
    assert operation.cache_info()["misses"] == 1


def test_float32_rounding_precedes_float64_accumulation(hip):
    host = np.linspace(0.7, 3.3, 9001, dtype=np.float32)
    operation = p.compile(lambda a: np.sum(a * a, dtype=np.float64))
    actual = operation(p.asarray(host, backend=hip))
    np.testing.assert_allclose(p.asnumpy(actual), np.sum(host * host, dtype=np.float64), rtol=1e-14)
    x = np.array([1 + 2**-25, 1 - 2**-25, 2**-150], np.float64)
    narrow = p.compile(lambda a: a.astype(np.float32).astype(np.float64) - a)
    np.testing.assert_array_equal(
        p.asnumpy(narrow(p.asarray(x, backend=hip))), x.astype(np.float32).astype(np.float64) - x
    )


def test_shared_outputs_no_upload_and_no_retained_inputs(hip, monkeypatch):
    host = np.arange(9001, dtype=np.float32) / 1000
    a = p.asarray(host, backend=hip)
    monkeypatch.setattr(hip, "upload", lambda *args: pytest.fail("unexpected upload"))
    total = p.compile(lambda a, rate: np.sum((a + rate) * (a + rate)))
    np.testing.assert_allclose(p.asnumpy(total(a, 2.0)), np.sum((host + 2) ** 2), rtol=2e-6)
    assert [s["kind"] for s in total.explain(a, 2.0)["steps"]] == ["map_reduce"]

    @p.compile
    def shared(a, rate):
        shifted = a + rate
        return shifted, np.sum(shifted * shifted), shifted - 1

    first = shared(a, 2.0)
    second = shared(a, 3.0)
    for values, offset in ((first, 2), (second, 3)):
        for actual, expected in zip(values, (host + offset, np.sum((host + offset) ** 2), host + offset - 1)):
            np.testing.assert_allclose(p.asnumpy(actual), expected, rtol=2e-6)
    ref = weakref.ref(a._data)
    del a, first, second, values, actual
    hip.synchronize()
    gc.collect()
    assert ref() is None


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fuse_transcendentals_nonfinite_and_signed_zero(hip, dtype):
    host = np.array([-0.0, 0.0, 0.3, -0.7, np.nan, np.inf, -np.inf], dtype=dtype)
    a = p.asarray(host, backend=hip)
    f = p.fuse(lambda a: np.isfinite(a) == (a > 0))
    np.testing.assert_array_equal(p.asnumpy(f(a)), np.isfinite(host) == (host > 0))
    with np.errstate(all="ignore"):

        def op(a):
            return np.sin(a) * np.exp(-a * a) + np.cos(a)

        np.testing.assert_allclose(p.asnumpy(p.fuse(op)(a)), op(host), rtol=2e-6, equal_nan=True)
    zero = p.asnumpy(p.fuse(lambda a: a * dtype(1))(a))
    np.testing.assert_array_equal(np.signbit(zero[:2]), np.signbit(host[:2]))
    boolean = p.fuse(lambda a: np.isfinite(a > 0))
    np.testing.assert_array_equal(p.asnumpy(boolean(a)), np.ones(host.shape, bool))


def test_no_hidden_fma_and_same_reduction_order(hip):
    a = p.asarray([1 + 2**-23], dtype=p.float32, backend=hip)
    b = p.asarray([1 - 2**-23], dtype=p.float32, backend=hip)
    fused = p.compile(lambda a, b: a * b - 1)
    np.testing.assert_array_equal(p.asnumpy(fused(a, b)), p.asnumpy(a * b - 1))
    assert p.asnumpy(fused(a, b))[0] == 0  # (1 + e)(1 - e) rounds to 1 before the subtraction
    host = np.tile(np.array([1e20, 1, -1e20, 3, 1e-38], np.float32), 2001)
    x = p.asarray(host, backend=hip)
    total = p.compile(lambda x: np.sum((x + 1) * 0.5))
    np.testing.assert_array_equal(p.asnumpy(total(x)), p.asnumpy(np.sum((x + 1) * 0.5)))


def test_inlined_product_stays_a_matmul_and_threads_rebind(hip, monkeypatch):
    # The subtraction is inlined into the fused multiply, so the product is a
    # leaf of that group (a plain matmul step), as in the reference plans.
    host = np.arange(33 * 17, dtype=np.float32).reshape(33, 17) / 1000
    a, x, b = [p.asarray(v, backend=hip) for v in (host, np.ones(17, np.float32), np.ones(33, np.float32))]
    original = hip.matmul
    calls = []
    monkeypatch.setattr(hip, "matmul", lambda *args: (calls.append(1), original(*args))[1])
    operation = p.compile(lambda a, x, b, rate: (b - a @ x) * rate)
    operation(a, x, b, 1.0)
    kinds = [step["kind"] for step in operation.explain(a, x, b, 1.0)["steps"]]
    assert kinds == ["matmul", "fused"]

    def work(rate):
        return p.asnumpy(operation(a, x, b, rate))

    with ThreadPoolExecutor(max_workers=3) as executor:
        results = list(executor.map(work, (0.5, 1.5, 2.5)))
    for value, rate in zip(results, (0.5, 1.5, 2.5)):
        np.testing.assert_allclose(value, (1 - host @ np.ones(17, np.float32)) * rate, rtol=2e-6, atol=1e-6)
    assert len(calls) == 4


@pytest.mark.parametrize("shape,axis", [((5,), None), ((3, 20001), 1), ((20001, 3), 0), ((4, 0), 1), ((0, 4), 0)])
def test_boolean_accumulator_is_a_logical_or(hip, shape, axis):
    # NumPy sums in bool as a logical or, as the reference's OpenCL kernels do
    # (its initial CUDA backend rejects the case); eager and compiled agree.
    host = np.random.default_rng(3).choice(np.array([0, 0, 0, 2, -1, np.nan], np.float32), size=shape)
    if host.size and axis == 1:
        host[0, :] = 0  # an all-false row
    if host.size and axis == 0:
        host[:, 0] = 0
    a = p.asarray(host, backend=hip)
    want = np.sum(host > 0, axis=axis, dtype=np.bool_)
    eager = p.sum(a > 0, axis=axis, dtype=np.bool_)
    compiled = p.compile(lambda a: np.sum(a > 0, axis=axis, dtype=np.bool_))
    for got in (eager, compiled(a)):
        assert got.dtype == np.bool_ and got.shape == want.shape
        np.testing.assert_array_equal(p.asnumpy(got), want)
    nonzero = p.compile(lambda a: np.sum(a, axis=axis, dtype=np.bool_))(a)  # NaN counts as true
    np.testing.assert_array_equal(p.asnumpy(nonzero), np.sum(host, axis=axis, dtype=np.bool_))
    counted = p.compile(lambda a: np.sum(a > 0, axis=axis))(a)  # numeric accumulator
    np.testing.assert_array_equal(p.asnumpy(counted), np.sum(host > 0, axis=axis))
    assert counted.dtype == np.sum(host > 0, axis=axis).dtype
