"""compile()/fuse() and prepared-plan contracts, run on the NumPy backend and on hip.

Restates the backend-parametrised contracts of the reference's
tests/test_compiler.py:35-400 (public forms, cache keys and bounds, static
arguments, explain without host observations, no transfers, no retained
inputs, thread sharing, rejected mutation and nesting), tests/test_fusion.py:7-106
(broadcast/dtype, transcendentals, non-finite comparisons, scalars as kernel
arguments, one launch per fused group, rejected control flow, scalar overflow,
intermediate rounding, a pool that keeps queued inputs), tests/test_prepared.py:25-70
(rebinding, specialization checks) and tests/test_irregular_workloads.py:41-95
(odd and rectangular tile boundaries, GEMV residual with axis reductions) and
tests/test_compiler_optimization.py:19-90 (mapped reductions over every dtype,
axes and empty shapes; a bool accumulator; shared intermediates). The same
body runs on the NumPy backend (CPU tier) and on hip (``gpu``).
"""

import gc
import weakref
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import openpacho as p


@pytest.fixture(params=["numpy", pytest.param("hip", marks=pytest.mark.gpu)])
def backend(request):
    if request.param == "numpy":
        return p.get_backend("numpy")
    return request.getfixturevalue("hip")


def _array(value, backend, dtype=None):
    return p.asarray(value, dtype=dtype, backend=backend)


def _result(actual, expected, *, rtol=2e-5, atol=2e-6):
    expected = np.asarray(expected)
    assert actual.shape == expected.shape
    assert actual.dtype == expected.dtype, (actual.dtype, expected.dtype)
    host = p.asnumpy(actual)
    if expected.dtype.kind in "fc":
        np.testing.assert_allclose(host, expected, rtol=rtol, atol=atol, equal_nan=True)
    else:
        np.testing.assert_array_equal(host, expected)


# ---- compile (reference tests/test_compiler.py) ---------------------------------------


def test_compile_public_forms(backend):
    def source(a):
        return 2 * a + 1

    @p.compile
    def decorated(a):
        return 2 * a + 1

    @p.compile()
    def factory_decorated(a):
        return 2 * a + 1

    value = np.arange(7, dtype=np.float32)
    for compiled, name in ((p.compile(source), "source"), (decorated, "decorated"), (factory_decorated, "factory_decorated")):
        assert compiled.__name__ == name
        _result(compiled(_array(value, backend)), 2 * value + 1)


def test_compile_retraces_only_on_cache_miss(backend):
    traces = []

    def source(a):
        traces.append("capture")
        return a * 3 - 1

    compiled = p.compile(source)
    value = np.arange(9, dtype=np.float32)
    array = _array(value, backend)
    _result(compiled(array), value * 3 - 1)
    _result(compiled(array), value * 3 - 1)
    assert traces == ["capture"]
    assert (compiled.cache_info()["misses"], compiled.cache_info()["hits"]) == (1, 1)


def test_compile_rebinds_dynamic_scalars_with_weak_promotion(backend):
    compiled = p.compile(lambda a, b, rate: (1 - rate) * a + rate * b)
    left, right = np.linspace(-2, 2, 11, dtype=np.float32), np.linspace(3, -1, 11, dtype=np.float32)
    a, b = _array(left, backend), _array(right, backend)
    for rate in (0.25, 0.75):
        actual = compiled(a, b, rate)
        assert actual.dtype == np.float32
        _result(actual, (1 - rate) * left + rate * right)
    assert (compiled.cache_info()["misses"], compiled.cache_info()["hits"]) == (1, 1)


def test_compile_shared_ndarray_dispatch_and_tuple_outputs(backend):
    def mixed(x, matrix):
        return (
            np.sum(x, axis=1),
            np.mean(x, axis=0, keepdims=True),
            np.matmul(matrix, matrix.T),
            np.reshape(x, (6,)),
            np.transpose(x),
            np.diag(matrix, k=1),
            np.linalg.norm(x),
        )

    x = np.arange(6, dtype=np.float32).reshape(2, 3) - 1
    matrix = np.arange(9, dtype=np.float32).reshape(3, 3)
    outputs = p.compile(mixed)(_array(x, backend), _array(matrix, backend))
    assert isinstance(outputs, tuple)
    for actual, expected in zip(outputs, mixed(x, matrix), strict=True):
        _result(actual, expected)


@pytest.mark.parametrize("operation", ["reshape", "reduce"])
def test_compile_zero_dim_asarray_flows_through_non_elementwise(backend, operation):
    def scalar_flow(_):
        scalar = p.asarray(2, dtype=np.float32)
        return np.reshape(scalar, (1,)) if operation == "reshape" else np.sum(scalar)

    expected = np.asarray(2, dtype=np.float32)
    expected = expected.reshape(1) if operation == "reshape" else np.sum(expected)
    _result(p.compile(scalar_flow)(_array(np.zeros(1, dtype=np.float32), backend)), expected)
    zero = p.compile(lambda _: np.sum(p.zeros_like(p.asarray(2, dtype=np.float32))))
    _result(zero(_array(np.zeros(1, dtype=np.float32), backend)), np.asarray(0, dtype=np.float32))


def test_compile_tuple_outputs_reuse_an_input(backend):
    def pair(a, b):
        shared = a + b
        return shared, shared * shared, np.sum(shared)

    left = np.arange(12, dtype=np.float32).reshape(3, 4)
    right = np.full((3, 4), 2, dtype=np.float32)
    outputs = p.compile(pair)(_array(left, backend), _array(right, backend))
    for actual, expected in zip(outputs, pair(left, right), strict=True):
        _result(actual, expected)


def test_compile_cache_tracks_shape_dtype_and_is_bounded(backend):
    compiled = p.compile(lambda a: a + 1)
    values = np.arange(6, dtype=np.float32)
    for value in (values, values.copy(), values.reshape(2, 3), values.astype(np.int32)):
        _result(compiled(_array(value, backend)), value + 1)
    info = compiled.cache_info()
    assert (info["misses"], info["hits"], info["size"]) == (3, 1, 3)
    bounded = p.compile(lambda a: a + 1, cache_size=2)
    for length in (3, 4, 5, 3):
        value = np.arange(length, dtype=np.float32)
        _result(bounded(_array(value, backend)), value + 1)
    info = bounded.cache_info()
    assert (info["max_size"], info["size"], info["misses"]) == (2, 2, 4)
    bounded.clear_cache()
    assert bounded.cache_info() == {"hits": 0, "misses": 0, "size": 0, "max_size": 2}


def test_compile_static_arguments_create_specialized_plans(backend):
    value = np.arange(12, dtype=np.float32).reshape(3, 4)
    array = _array(value, backend)
    reshape_to = p.compile(lambda a, shape: np.reshape(a, shape), static_argnames=("shape",))
    _result(reshape_to(array, (2, 6)), value.reshape(2, 6))
    _result(reshape_to(array, (6, 2)), value.reshape(6, 2))
    assert (reshape_to.cache_info()["misses"], reshape_to.cache_info()["hits"]) == (2, 0)
    reduce_axis = p.compile(lambda a, axis: np.sum(a, axis=axis), static_argnames="axis")
    for axis in (0, 1, 0):
        _result(reduce_axis(array, axis), np.sum(value, axis=axis))
    assert (reduce_axis.cache_info()["misses"], reduce_axis.cache_info()["hits"]) == (2, 1)
    with pytest.raises(TypeError, match="static_argnames"):
        p.compile(lambda a, shape: np.reshape(a, shape))(array, (2, 6))


def test_compile_explain_reports_plan_without_host_observations(backend):
    traces = []

    def source(a):
        traces.append("capture")
        return np.sum(a, axis=0) + 1

    compiled = p.compile(source)
    array = _array(np.arange(6, dtype=np.float32).reshape(2, 3), backend)
    details = compiled.explain(array)
    assert details["backend"] == backend.name and details["device"] == backend.device
    assert details["outputs"] == 1 and details["steps"]
    assert details["host_observations"] == 0 and details["python_retrace_on_cache_hit"] is False
    compiled(array)
    assert traces == ["capture"]


def test_compile_does_not_transfer_during_capture_or_execution(backend, monkeypatch):
    array = _array(np.arange(17, dtype=np.float32), backend)
    compiled = p.compile(lambda a: np.sqrt(a * a + 1))
    if backend.name != "numpy":
        with monkeypatch.context() as patch:
            for name in ("upload", "download"):
                patch.setattr(backend, name, lambda *args, **kwargs: pytest.fail("implicit host transfer"))
            result = compiled(array)
            assert result.backend == backend.name
    else:
        result = compiled(array)
    _result(result, np.sqrt(np.arange(17, dtype=np.float32) ** 2 + 1))


def test_compile_plan_does_not_retain_input_arrays(backend):
    compiled = p.compile(lambda a: a * 2 + 1)
    source = _array(np.arange(13, dtype=np.float32), backend)
    ref = weakref.ref(source)
    result = compiled(source)
    del source
    gc.collect()
    assert ref() is None
    _result(result, np.arange(13, dtype=np.float32) * 2 + 1)


def test_compile_concurrent_calls_share_one_plan(backend):
    traces = []

    def source(a, scale):
        traces.append("capture")
        return a * scale + 1

    compiled = p.compile(source)
    values = [np.arange(23, dtype=np.float32) + i for i in range(8)]
    arrays = [_array(v, backend) for v in values]
    with ThreadPoolExecutor(max_workers=4) as pool:
        results = list(pool.map(lambda a: compiled(a, 0.5), arrays))
    for actual, value in zip(results, values):
        _result(actual, value * 0.5 + 1)
    assert traces == ["capture"]
    assert (compiled.cache_info()["misses"], compiled.cache_info()["hits"]) == (1, len(values) - 1)


def test_compile_rejects_input_mutation_and_nesting(backend):
    def mutating(a):
        a += 1
        return a

    array = _array(np.arange(4, dtype=np.float32), backend)
    with pytest.raises((TypeError, NotImplementedError)):
        p.compile(mutating)(array)
    inner = p.compile(lambda a: a * 2)
    with pytest.raises(TypeError, match="Nested compiled"):
        p.compile(lambda a: inner(a) + 1)(array)


def test_compile_native_numpy_passthrough():
    calls = []

    def source(a):
        calls.append("python")
        return np.sin(a) + 2

    value = np.arange(5, dtype=np.float32)
    result = p.compile(source)(value)
    assert isinstance(result, np.ndarray) and calls == ["python"]
    np.testing.assert_allclose(result, np.sin(value) + 2)


@pytest.mark.gpu
def test_compile_cache_separates_backends_and_rejects_mixing(hip):
    numpy_array = _array(np.arange(5, dtype=np.float32), "numpy")
    hip_array = _array(np.arange(5, dtype=np.float32), hip)
    compiled = p.compile(lambda a: a * 2)
    _result(compiled(numpy_array), np.arange(5, dtype=np.float32) * 2)
    on_hip = compiled(hip_array)
    assert on_hip.backend == "hip"
    _result(on_hip, np.arange(5, dtype=np.float32) * 2)
    assert (compiled.cache_info()["misses"], compiled.cache_info()["size"]) == (2, 2)
    with pytest.raises(p.BackendMismatchError):
        p.compile(lambda a, b: a + b)(numpy_array, hip_array)
    with pytest.raises(p.BackendMismatchError):
        p.fuse(lambda a: a + hip_array)(numpy_array)


# ---- mapped reductions (reference tests/test_compiler_optimization.py) ------------------


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.uint32, np.bool_])
@pytest.mark.parametrize(
    "shape,axes",
    [
        ((4099,), None),
        ((5, 32), (-1,)),
        ((3, 2, 33), (1, 2)),
        ((9, 7, 39), (0, 2)),
        ((67, 3, 69), (0, 2)),
        ((2, 3), ()),
        ((), None),
        ((2, 0, 3), (1,)),
        ((0, 4097), (1,)),
    ],
)
def test_compiled_mapped_reduction(backend, dtype, shape, axes):
    host = (np.arange(int(np.prod(shape))) % 7).astype(dtype).reshape(shape)

    @p.compile
    def total(a):
        mapped = a == 1 if dtype is np.bool_ else a * a + 2
        return np.sum(mapped, axis=axes, keepdims=True)

    mapped = host == 1 if dtype is np.bool_ else host * host + 2
    _result(total(_array(host, backend)), np.sum(mapped, axis=axes, keepdims=True), rtol=3e-5, atol=3e-5)


def test_map_boolean_accumulator_and_shared_intermediate(backend):
    host = np.zeros(9001, dtype=np.int32)
    host[-1] = 1
    compiled = p.compile(lambda a: np.sum(a > 0, dtype=np.bool_))
    _result(compiled(_array(host, backend)), np.sum(host > 0, dtype=np.bool_))
    values = np.arange(4133, dtype=np.float32) / 1000

    @p.compile
    def shared(a):
        x = a + 2
        return x, np.sum(x * x), x - 1

    for actual, expected in zip(shared(_array(values, backend)), (values + 2, np.sum((values + 2) ** 2), values + 1)):
        _result(actual, expected, rtol=3e-5, atol=3e-5)


# ---- fuse (reference tests/test_fusion.py) ---------------------------------------------


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.int64])
@pytest.mark.parametrize("shape", [(17, 3), (0, 3), ()])
def test_fused_broadcast_and_dtype(backend, dtype, shape):
    a, b = np.full(shape, 2, dtype=dtype), np.asarray(3, dtype=dtype)
    result = p.fuse(lambda a, b: (a + b) * (a - 1))(_array(a, backend), _array(b, backend))
    _result(result, (a + b) * (a - 1))


def test_fused_transcendentals_and_shared_expression(backend):
    a = np.linspace(-2, 2, 35, dtype=np.float32).reshape(5, 7)
    b = np.linspace(0, 1, 7, dtype=np.float64)

    @p.fuse
    def f(a, b, scale=0.25):
        t = p.sin(a) * np.exp(-a * a)
        return (t + t) * scale + p.cos(b)

    result = f(_array(a, backend), _array(b, backend))
    t = np.sin(a) * np.exp(-a * a)
    assert result.dtype == np.float64
    np.testing.assert_allclose(p.asnumpy(result), (t + t) * 0.25 + np.cos(b), rtol=2e-6)


def test_fused_comparison_with_nonfinite_values(backend):
    host = np.asarray([np.nan, np.inf, -np.inf, -1, 0, 2], dtype=np.float32)
    f = p.fuse(lambda a: p.isfinite(a) == (a > 0))
    _result(f(_array(host, backend)), np.isfinite(host) == (host > 0))


@pytest.mark.gpu
def test_fused_scalars_are_arguments_and_one_launch_without_uploads(hip, monkeypatch):
    a = _array(np.asarray([1, 2, 3], dtype=np.float32), hip)
    f = p.fuse(lambda a, scale: a * scale + 7.125)
    f(a, 0.25)
    kernels = len(hip._kernels)
    np.testing.assert_allclose(p.asnumpy(f(a, 0.5)), [7.625, 8.125, 8.625])
    assert len(hip._kernels) == kernels  # the new scalar is not baked into a new program
    ones = p.ones((257,), backend=hip, dtype=np.float32)
    calls = []
    launch = hip._launch
    monkeypatch.setattr(hip, "_launch", lambda *args: (calls.append(args[1]), launch(*args))[1])
    monkeypatch.setattr(hip, "upload", lambda *args: pytest.fail("unexpected upload"))
    np.testing.assert_allclose(p.asnumpy(p.fuse(lambda a: 0.99 * a + 0.01 * a)(ones)), 1)
    assert len(calls) == 1
    np.testing.assert_allclose(p.asnumpy(0.5 * ones + 1), 1.5)
    assert len(calls) == 3  # eager: one launch per operation


def test_fusion_rejects_control_flow_reductions_and_tuples(backend):
    a = p.ones((3,), backend=backend)
    with pytest.raises(TypeError, match="control flow"):
        p.fuse(lambda a: a if a > 0 else -a)(a)
    with pytest.raises((TypeError, NotImplementedError)):
        p.fuse(lambda a: np.sum(a))(a)
    with pytest.raises((TypeError, NotImplementedError)):
        p.fuse(lambda a: a @ a)(a)
    with pytest.raises(TypeError, match="one elementwise"):
        p.fuse(lambda a: (a, a))(a)


def test_fused_scalar_overflow_and_intermediate_rounding(backend):
    with pytest.raises(OverflowError):
        p.fuse(lambda a: a + 2**40)(_array([1], backend, np.int32))
    a = _array([2**24], backend, np.float32)
    np.testing.assert_array_equal(p.asnumpy(p.fuse(lambda a: (a + 1) - a)(a)), [0])


@pytest.mark.gpu
def test_pool_preserves_queued_inputs_and_releases_cache(hip):
    a = p.ones(513, dtype=np.float32, backend=hip)
    for _ in range(100):
        a = a + 1
    np.testing.assert_array_equal(p.asnumpy(a), np.full(513, 101, dtype=np.float32))
    hip.release_cached_memory()
    assert hip.pool_stats()["cached_items"] == 0
    np.testing.assert_array_equal(p.asnumpy(a), 101)


# ---- prepared plans (reference tests/test_prepared.py) ---------------------------------


def test_prepared_rebinds_and_does_not_retain_examples(backend):
    @p.compile
    def affine(a, factor=2.0):
        return a * factor + 1

    a = _array(np.arange(12, dtype=np.float32), backend)
    ref = weakref.ref(a)
    run = affine.prepare(a)
    del a
    gc.collect()
    assert ref() is None
    b = p.ones(12, dtype=np.float32, backend=backend)
    first, second = run(b, 3.0), run(a=b, factor=7.0)
    affine.clear_cache()
    third = run(b)
    for result, expected in ((first, 4), (second, 8), (third, 3)):
        np.testing.assert_array_equal(p.asnumpy(result), np.full(12, expected, np.float32))
    assert affine.cache_info()["size"] == 0
    assert run.explain()["binding_validation"]


def test_prepared_rejects_specialization_changes(backend):
    @p.compile(static_argnames="axis")
    def total(a, factor=2.0, *, axis=0):
        return p.sum(a * factor, axis=axis)

    a = p.ones((3, 4), dtype=np.float32, backend=backend)
    run = total.prepare(a)
    np.testing.assert_array_equal(p.asnumpy(run(a)), np.full(4, 6, np.float32))
    for args, kwargs in (
        ((p.ones((4, 3), dtype=np.float32, backend=backend),), {}),
        ((a.astype(np.float64),), {}),
        ((np.ones((3, 4), np.float32),), {}),
        ((a, 2), {}),
        ((a,), {"axis": 1}),
    ):
        with pytest.raises(ValueError, match="specialization"):
            run(*args, **kwargs)
    with pytest.raises(TypeError):
        run()
    with pytest.raises(TypeError):
        run(a, 2.0, 3)


# ---- odd shapes (reference tests/test_irregular_workloads.py) --------------------------


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize(
    "shapes",
    [
        ((31, 15), (15, 33)),
        ((33, 17), (17, 65)),
        ((65, 63), (63, 97)),
        ((127, 65), (65, 35)),
        ((45, 30), (30, 70)),
        ((3, 1, 33, 17), (1, 5, 17, 35)),
        ((257, 129), (129, 513)),
    ],
)
def test_rectangular_tile_boundaries_eager_compiled_and_rebound(backend, dtype, shapes):
    rng = np.random.default_rng(831)
    host = [rng.uniform(-1, 1, shape).astype(dtype) for shape in shapes]
    a, b = [_array(x, backend) for x in host]
    operation = p.compile(lambda left, right: left @ right)
    expected = host[0].astype(np.float64) @ host[1].astype(np.float64)
    tol = 3e-5 if dtype == np.float32 else 5e-13
    for result in (a @ b, operation(a, b)):
        assert result.shape == expected.shape and result.dtype == dtype
        np.testing.assert_allclose(p.asnumpy(result), expected, rtol=tol, atol=tol)
    later = operation(-a, b)  # same plan, new values, while an earlier result lives
    np.testing.assert_allclose(p.asnumpy(later), -expected, rtol=tol, atol=tol)
    np.testing.assert_allclose(p.asnumpy(result), expected, rtol=tol, atol=tol)
    assert operation.cache_info()["misses"] == 1
    np.testing.assert_array_equal(p.asnumpy(a), host[0])
    np.testing.assert_array_equal(p.asnumpy(b), host[1])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", [(31, 63), (65, 129), (127, 257), (1, 5000)])
def test_rectangular_gemv_residual_and_axis_reductions(backend, dtype, shape):
    rng = np.random.default_rng(832)
    ah, xh, bh = (rng.uniform(-1, 1, s).astype(dtype) for s in (shape, shape[1], shape[0]))
    a, x, b = [_array(v, backend) for v in (ah, xh, bh)]

    @p.compile
    def operation(a, x, b):
        return b - a @ x, np.sum(a * a, axis=0), np.sum(a * a, axis=1)

    wide = [v.astype(np.float64) for v in (ah, xh, bh)]
    reference = (wide[2] - wide[0] @ wide[1], np.sum(wide[0] ** 2, axis=0), np.sum(wide[0] ** 2, axis=1))
    tol = 3e-5 if dtype == np.float32 else 5e-13
    for result, expected in zip(operation(a, x, b), reference, strict=True):
        assert result.shape == expected.shape and result.dtype == dtype
        np.testing.assert_allclose(p.asnumpy(result), expected, rtol=tol, atol=tol)
    if backend.name != "numpy":
        assert "residual_matvec" in [s["kind"] for s in operation.explain(a, x, b)["steps"]]
