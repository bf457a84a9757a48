"""API behaviour on the NumPy backend (CPU): the contracts the hip backend plugs into.

Expectations follow the reference's own tests: test_random.py (stream
ownership, validation, burn-on-failure, splitting), test_compiler.py /
test_cuda.py (plan caching, explain step kinds), test_padding_metadata.py.
"""

import json
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import pytest

import openpacho as p
from openpacho import _hip_padding
from openpacho.backends import NumpyBackend
from openpacho.exceptions import BackendMismatchError, BackendUnavailableError, UnsupportedDtypeError

GOLDEN_PLANS = Path(__file__).parent / "golden" / "reference_plans.json"


# ---- selection and dtypes ----------------------------------------------------------


def test_selection_and_foreign_runtimes():
    assert p.get_backend("numpy").name == "numpy"
    with pytest.raises(BackendUnavailableError):
        p.get_backend("cuda")
    with pytest.raises(ValueError):
        p.get_backend("numpy", blas="custom")
    with pytest.raises(ValueError):
        p.get_backend("hip", blas="cublas")
    with pytest.raises(ValueError):
        p.get_backend("bogus")
    with p.use_backend("numpy") as selected:
        assert p.get_backend() is selected


def test_dtype_whitelist():
    for bad in (np.float16, np.int8, np.complex64):
        with pytest.raises(UnsupportedDtypeError):
            p.asarray(np.zeros(2, bad))


def test_no_implicit_host_conversion_and_mismatch():
    a = p.asarray([1.0, 2.0])
    with pytest.raises(TypeError):
        np.asarray(a)
    with pytest.raises(ValueError):
        bool(a)
    other = NumpyBackend()
    b = p.asarray([1.0, 2.0], backend=other)
    with pytest.raises(BackendMismatchError):
        a + b


def test_elementwise_promotion_and_broadcast():
    x = p.asarray(np.arange(6, dtype=np.float32).reshape(2, 3))
    y = x + 1.5
    assert y.dtype == np.float32 and p.asnumpy(y)[1, 2] == 6.5
    z = np.add(x, p.asarray(np.ones(3, np.float64)))
    assert z.dtype == np.float64 and z.shape == (2, 3)
    w = p.where(x > 2, x, 0)
    assert p.asnumpy(w).tolist() == [[0, 0, 0], [3, 4, 5]]
    with pytest.raises(NotImplementedError):
        p.power(p.asarray([2, 3]), 2)


def test_indexing_transpose_reshape_diag():
    host = np.arange(24, dtype=np.int64).reshape(2, 3, 4)
    a = p.asarray(host)
    np.testing.assert_array_equal(p.asnumpy(a[1, ::-1, 1:3]), host[1, ::-1, 1:3])
    np.testing.assert_array_equal(p.asnumpy(a[..., None, 2]), host[..., None, 2])
    np.testing.assert_array_equal(p.asnumpy(a.transpose(2, 0, 1)), host.transpose(2, 0, 1))
    np.testing.assert_array_equal(p.asnumpy(a.reshape(4, -1)), host.reshape(4, -1))
    np.testing.assert_array_equal(p.asnumpy(p.diag(a[0], 1)), np.diag(host[0], 1))
    with pytest.raises(IndexError):
        a[2]


def test_reductions_and_extrema_contract():
    host = np.array([[0.0, -0.0, 3.0], [np.nan, 1.0, -2.0]], np.float32)
    a = p.asarray(host)
    assert np.signbit(p.asnumpy(p.min(a[0:1, 0:2]))) and not np.signbit(p.asnumpy(p.max(a[0:1, 0:2])))
    assert np.isnan(p.asnumpy(p.max(a, axis=1))[1])
    assert p.sum(p.asarray([True, True, False])).dtype == np.int64
    np.testing.assert_allclose(p.asnumpy(p.mean(p.asarray(np.arange(6.0).reshape(2, 3)), axis=1)), [1, 4])
    with pytest.raises(ValueError):
        p.amax(p.asarray(np.zeros((0, 3))), axis=0)


def test_matmul_shapes_dot_and_errors():
    a = p.asarray(np.ones((2, 5, 7), np.float32))
    b = p.asarray(np.ones((7, 3), np.float32))
    assert (a @ b).shape == (2, 5, 3)
    assert p.dot(p.asarray([1.0, 2.0]), p.asarray([3.0, 4.0])).item() == 11.0
    assert p.dot(2.0, p.asarray([1.0])).shape == (1,)
    with pytest.raises(NotImplementedError):
        p.dot(a, a)
    with pytest.raises(ValueError):
        p.matmul(p.asarray([1.0, 2.0]), p.asarray([1.0]))
    with pytest.raises(TypeError):
        p.matmul(a, b, padding="yes")


def test_linalg_norm_order_rules():
    x = p.asarray(np.arange(6.0).reshape(2, 3))
    assert p.linalg.norm(x, "fro").shape == ()
    assert p.linalg.norm(p.asarray([3, 4])).dtype == np.float64
    with pytest.raises(NotImplementedError):
        p.linalg.norm(x, 1)
    np.testing.assert_allclose(p.asnumpy(np.linalg.norm(x, axis=1)), np.linalg.norm(np.arange(6.0).reshape(2, 3), axis=1))


# ---- random generator contract ------------------------------------------------------


def test_rng_split_and_reproducible():
    rng = p.random.default_rng(2**64 - 1)
    whole = p.asnumpy(rng.normal(2, 3, (33, 17), dtype="float32"))
    replay = p.random.default_rng(2**64 - 1)
    parts = np.concatenate([p.asnumpy(replay.normal(2, 3, n, dtype="float32")) for n in (1, 127, 0, 433)])
    np.testing.assert_array_equal(parts, whole.ravel())


def test_rng_counter_carry_exhaustion_and_empty():
    rng = p.random.default_rng(0)
    rng._counter = 2**64 - 7
    assert rng.random(7, dtype="float32").shape == (7,)
    with pytest.raises(OverflowError):
        rng.random(1, dtype="float32")
    assert rng.random((0, 17), dtype="float32").shape == (0, 17)


@pytest.mark.parametrize("seed", [-1, 2**64, True, 1.5, [1, 2]])
def test_invalid_seed(seed):
    with pytest.raises((ValueError, TypeError)):
        p.random.default_rng(seed)


def test_invalid_parameters_do_not_consume_stream():
    rng = p.random.default_rng(0, backend="numpy")
    for method, kwargs in [
        (rng.random, {"size": -1}),
        (rng.random, {"size": 2**31}),
        (rng.random, {"dtype": "int32"}),
        (rng.uniform, {"low": 3, "high": 2}),
        (rng.uniform, {"high": float("inf")}),
        (rng.normal, {"scale": -1}),
        (rng.exponential, {"scale": float("nan")}),
        (rng.normal, {"loc": [1, 2]}),
        (rng.uniform, {"low": -3e38, "high": 3e38, "dtype": "float32"}),
        (rng.normal, {"scale": -1e-50, "dtype": "float32"}),
        (rng.exponential, {"scale": -1e-50, "dtype": "float32"}),
        (rng.uniform, {"low": 1e-50, "high": 0, "dtype": "float32"}),
        (rng.normal, {"loc": 10**1000}),
    ]:
        with pytest.raises((ValueError, TypeError)):
            method(**kwargs)
    assert rng._counter == 0


def test_concurrent_calls_reserve_distinct_complete_ranges():
    rng = p.random.default_rng(12, backend="numpy")
    with ThreadPoolExecutor(max_workers=4) as pool:
        chunks = list(pool.map(lambda _: p.asnumpy(rng.random(129)), range(8)))
    expected = p.asnumpy(p.random.default_rng(12, backend="numpy").random(129 * 8)).reshape(8, 129)
    assert sorted(c.tobytes() for c in chunks) == sorted(c.tobytes() for c in expected)


def test_launch_failure_burns_reserved_range(monkeypatch):
    first = NumpyBackend()
    with p.use_backend(first):
        rng = p.random.default_rng(47)
    assert p.get_backend(rng.random(3)) is first

    def fail(*args):
        raise RuntimeError("uncertain dispatch")

    monkeypatch.setattr(first, "random_data", fail)
    with pytest.raises(RuntimeError, match="uncertain dispatch"):
        rng.random(7)
    assert rng._counter == 10
    monkeypatch.undo()
    reference = p.random.default_rng(47, backend="numpy")
    reference.random(10)
    np.testing.assert_array_equal(p.asnumpy(rng.random(33)), p.asnumpy(reference.random(33)))


def test_capture_rejects_generation():
    rng = p.random.default_rng(0, backend="numpy")
    for decorator in (p.compile, p.fuse):

        @decorator
        def sample(a):
            return a + rng.random(a.shape)

        with pytest.raises(NotImplementedError, match="not captured"):
            sample(p.ones(3, backend="numpy"))
        assert rng._counter == 0


# ---- compiled plans --------------------------------------------------------------------


class _RecordingLowering:
    """Grouping-only lowerer, same as the golden writer's (GPU-style grouping)."""

    def can_residual_matvec(self, matrix, vector, rhs, node):
        return False

    def can_reduce_materialized(self, node):
        return node.dtype.kind == "f" and node.dtype.itemsize == 4 and node.attrs.get("operation") in ("min", "max")

    def prepare_fused(self, node, group, leaves):
        return tuple(leaves), [g.op for g in group]

    def prepare_map_reduce(self, node, group, leaves):
        return tuple(leaves), [g.op for g in group]


class _GroupingBackend(NumpyBackend):
    def create_lowering(self):
        return _RecordingLowering()


def _plan_cases(backend):
    def arr(*shape):
        return p.asarray(np.ones(shape, np.float32), backend=backend)

    def mlp(x, w1, b1, w2, b2, w3, b3):
        h = p.tanh(x @ w1 + b1)
        h = p.tanh(h @ w2 + b2)
        out = p.tanh(h @ w3 + b3)
        return p.mean(out, axis=1)

    def affine(value, scale):
        shifted = value * scale
        return shifted, shifted + 1.0

    def products(a, b):
        product = p.matmul(a, b)
        return product, p.sum(product), p.mean(product)

    return {
        "mlp": (mlp, (arr(8, 16), arr(16, 16), arr(16), arr(16, 16), arr(16), arr(16, 4), arr(4))),
        "affine": (affine, (arr(3, 4), 2.0)),
        "product_reductions": (products, (arr(33, 17), arr(17, 65))),
        "norm_rows": (lambda a: p.linalg.norm(a, axis=1, keepdims=True), (arr(6, 4097),)),
        "sum_of_squares_shift": (lambda x: ((x + 1) * (x - 2)).sum(), (arr(8),)),
        "extrema": (lambda x: (p.max(x, axis=0), p.min(x * 2, axis=1)), (arr(5, 6),)),
    }


def test_plan_grouping_matches_reference_golden():
    golden = json.loads(GOLDEN_PLANS.read_text())
    for name, (fn, args) in _plan_cases(_GroupingBackend()).items():
        steps = p.compile(fn).explain(*args)["steps"]
        got = [{k: (list(v) if isinstance(v, tuple) else v) for k, v in s.items() if k != "padding"} for s in steps]
        assert got == golden[name], name


def test_compile_cache_rebinding_and_prepare():
    calls = []

    @p.compile
    def affine(value, scale):
        calls.append(1)
        shifted = value * scale
        return shifted, shifted + 1.0

    host = np.arange(12, dtype=np.float32).reshape(3, 4)
    value = p.asarray(host)
    first, _ = affine(value, 2.0)
    second, second_shifted = affine(value, 3.5)
    np.testing.assert_array_equal(p.asnumpy(first), host * 2)
    np.testing.assert_array_equal(p.asnumpy(second_shifted), host * 3.5 + 1)
    assert affine.cache_info()["misses"] == 1 and affine.cache_info()["hits"] >= 1 and len(calls) == 1
    prepared = affine.prepare(value, 2.0)
    with pytest.raises(ValueError):
        prepared(p.asarray(host[:2]), 2.0)
    assert affine(host, 2.0)[0].shape == (3, 4)  # NumPy inputs run the Python function


# ---- padding plan metadata -------------------------------------------------------------------


class _NoAlloc:
    def empty(self, shape, dtype):
        raise AssertionError("metadata preparation must not allocate")


def _plan(ashape, bshape, shape, dtype=np.float32, **kw):
    return _hip_padding.prepare(_NoAlloc(), ashape, bshape, shape, dtype, **kw)


def test_padding_metadata():
    # The padded problem is the reference's (oracle.padding.plan pins its
    # worked values); hip computes it without copies, and says so.
    plan = _plan((33, 17), (17, 65), (33, 65))
    assert plan.padded_input_shapes == ((64, 32), (32, 96)) and plan.padded_output_shape == (64, 96)
    info = plan.explain()
    assert info["scratch_bytes"] == 0 and info["copy_dispatches"] == 0 and plan.dispatch_count == 1
    assert info["alignment"] == (32, 16, 32)
    assert _plan((64, 32), (32, 96), (64, 96)).dispatch_count == 1
    assert _plan((17,), (17, 65), (65,)) is None
    assert _plan((31, 16), (16, 32), (31, 32)) is None
    assert _plan((33, 17), (17, 65), (33, 65), np.float64) is None
    assert _plan((2**31, 16), (16, 32), (2**31, 32)) is None
    assert _plan((33, 17), (17, 65), (33, 65), max_buffer_bytes=24575) is None
    big = _plan((4097, 3001), (3001, 2049), (4097, 2049))
    assert big.padded_input_shapes == ((4128, 3008), (3008, 2080)) and big.padded_output_shape == (4128, 2080)
    assert big.explain()["scratch_bytes"] == 0
    assert big.explain()["bounds_checks_removed"] is False
    assert _plan((512, 64), (64, 256), (512, 256)).explain()["bounds_checks_removed"] is True


# ---- residual GEMV contract (host side), reference tests/test_residual_matvec.py:86-102


def test_residual_rejects_incompatible_contracts_without_driver():
    from types import SimpleNamespace

    from openpacho._hip_gemv import check_residual

    backend = SimpleNamespace(name="hip", blas="custom")

    def value(shape, dtype="float32", owner=backend):
        return SimpleNamespace(shape=shape, ndim=len(shape), dtype=np.dtype(dtype), _backend=owner)

    valid = (value((3, 4)), value((4,)), value((3,)))
    check_residual(backend, *valid)
    for args in (
        (value((4,)), valid[1], valid[2]),
        (valid[0], value((5,)), valid[2]),
        (valid[0], valid[1], value((3,), "float64")),
        tuple(value(v.shape, "int32") for v in valid),
        (valid[0], valid[1], value((3,), owner=object())),
    ):
        with pytest.raises(ValueError):
            check_residual(backend, *args)
    backend.blas = "clblast"
    with pytest.raises(NotImplementedError, match="custom"):
        check_residual(backend, *valid)


def test_hip_lowering_residual_capability():
    from types import SimpleNamespace

    from openpacho._hip_lowering import HIPLowering

    backend = SimpleNamespace(blas="custom")
    lowering = HIPLowering(backend)
    f32, f64 = np.dtype("float32"), np.dtype("float64")
    matrix = SimpleNamespace(ndim=2, shape=(1, 4097), dtype=f32)
    vector = SimpleNamespace(ndim=1, shape=(4097,), dtype=f32)
    rhs = SimpleNamespace(ndim=1, shape=(1,), dtype=f32)
    node = SimpleNamespace(inputs=(rhs, rhs), shape=(1,), dtype=f32)
    # Unlike the reference Vulkan lowerer, no shape is excluded: the fused
    # kernel is the eager GEMV with another store.
    assert lowering.can_residual_matvec(matrix, vector, rhs, node)
    mixed = SimpleNamespace(inputs=(rhs, SimpleNamespace(shape=(1,), dtype=f64)), shape=(1,), dtype=f32)
    assert not lowering.can_residual_matvec(matrix, vector, rhs, mixed)
    batched = SimpleNamespace(ndim=3, shape=(2, 1, 4097), dtype=f32)
    assert not lowering.can_residual_matvec(batched, vector, rhs, node)
    backend.blas = "clblast"
    assert not lowering.can_residual_matvec(matrix, vector, rhs, node)


# ---- layout plans for private transposes, reference tests/test_compiled_layout.py


class _LayoutBackend(NumpyBackend):
    """CPU backend offering hip layout plans, executed with NumPy."""

    name = "test-layout"

    def __init__(self):
        self.gathers = 0
        self.calls = []

    def gather(self, *args):
        self.gathers += 1
        return super().gather(*args)

    def download(self, array):
        raise AssertionError("execution must not transfer to host")

    def prepare_layout_matmul(self, ashape, bshape, shape, dtype, *, transpose_a=False, transpose_b=False):
        from openpacho._hip_layout import prepare

        plan = prepare(self, ashape, bshape, shape, dtype, transpose_a=transpose_a, transpose_b=transpose_b)
        if plan is None:
            return None
        backend = self

        class _NumpyRun:
            explain = plan.explain

            def run(self, a, b):
                backend.calls.append((a.shape, b.shape, plan.transpose_a, plan.transpose_b))
                left, right = a._data.reshape(a.shape), b._data.reshape(b.shape)
                return ((left.T if plan.transpose_a else left) @ (right.T if plan.transpose_b else right)).ravel()

        return _NumpyRun()


@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_private_transpose_becomes_layout_step(ta, tb, dtype):
    backend = _LayoutBackend()
    rng = np.random.default_rng(42)
    left = rng.normal(size=(7, 5) if ta else (5, 7)).astype(dtype)
    right = rng.normal(size=(9, 7) if tb else (7, 9)).astype(dtype)
    a, b = p.array(left, backend=backend), p.array(right, backend=backend)

    @p.compile
    def product(a, b):
        return (a.T if ta else a) @ (b.T if tb else b)

    prepared = product.prepare(a, b)
    steps = prepared.explain()["steps"]
    assert [s["kind"] for s in steps] == ["layout_matmul"]
    layout = steps[0]["layout"]
    assert layout["provider"] == "hip"
    assert layout["leading_dimensions"] == (left.shape[1], right.shape[1], 9)
    assert layout["transpose_operand_bytes"] == np.dtype(dtype).itemsize * (left.size * ta + right.size * tb)
    for scale in (1, 2):
        current = p.array(left * scale, backend=backend)
        result = prepared(current, b)
        expected = ((left * scale).T if ta else left * scale) @ (right.T if tb else right)
        np.testing.assert_allclose(result._data.reshape(result.shape), expected, rtol=1e-6)
    assert backend.gathers == 0
    assert backend.calls == [(left.shape, right.shape, ta, tb)] * 2


@pytest.mark.parametrize("public", [False, True])
def test_shared_or_public_transpose_remains_materialized(public):
    backend = _LayoutBackend()
    host = np.arange(35, dtype=np.float32).reshape(7, 5)
    a, b = p.array(host, backend=backend), p.array(host, backend=backend)

    def source(a, b):
        t = a.T
        return (t @ b, t) if public else (t @ b, t + 1)

    fn = p.compile(source)
    actual = fn(a, b)
    assert [s["kind"] for s in fn.explain(a, b)["steps"]].count("gather") == 1
    assert not backend.calls and backend.gathers == 1
    for result, reference in zip(actual, source(host, host)):
        np.testing.assert_array_equal(result._data.reshape(result.shape), reference)


@pytest.mark.parametrize("ashape,bshape", [((0, 5), (0, 9)), ((7, 0), (7, 9)), ((7, 5), (7, 0))])
def test_layout_declines_empty_dimensions(ashape, bshape):
    backend = _LayoutBackend()
    a = p.array(np.zeros(ashape, dtype=np.float32), backend=backend)
    b = p.array(np.zeros(bshape, dtype=np.float32), backend=backend)
    result = p.compile(lambda a, b: a.T @ b)(a, b)
    assert not backend.calls
    np.testing.assert_array_equal(result._data.reshape(result.shape), np.zeros(ashape).T @ np.zeros(bshape))


def test_layout_keeps_conversions_and_padding_precedence():
    backend = _LayoutBackend()
    a = p.array(np.arange(35, dtype=np.float32).reshape(7, 5), backend=backend)
    b = p.array(np.arange(63, dtype=np.float64).reshape(7, 9), backend=backend)
    fn = p.compile(lambda a, b: a.T @ b)
    assert [s["kind"] for s in fn.explain(a, b)["steps"]] == ["gather", "cast", "matmul"]
    one = p.array(np.ones((7, 5), dtype=np.float32), backend=backend)
    square = p.compile(lambda a: a.T @ a)
    assert [s["kind"] for s in square.explain(one)["steps"]] == ["layout_matmul"]  # one transpose, both sides
    calls = []

    class Padded:
        def run(self, x, y):
            calls.append("padding")
            return backend.matmul(x, y, (5, 5), x.dtype)

        def explain(self):
            return {}

    backend.prepare_padded_matmul = lambda *args: Padded()
    p.compile(lambda a: a.T @ a, padding=True)(one)
    assert calls == ["padding"] and not backend.calls


def test_non_full_transpose_gather_is_not_folded():
    from openpacho._compiler import ExecutionPlan
    from openpacho._fusion import Expression, InputRef, TraceBackend

    backend = _LayoutBackend()
    for offset, strides, shape in [(1, (1, 5), (5, 7)), (0, (7, 1), (5, 7)), (0, (1, 5), (4, 7))]:
        trace = TraceBackend(backend)
        original = Expression(trace, (7, 5), np.float32, value=InputRef(0))
        gather = trace.gather(original, shape, offset, strides)
        right = Expression(trace, (7, 9), np.float32, value=InputRef(1))
        product = trace.matmul(gather, right, (shape[0], 9), np.float32)
        plan = ExecutionPlan(backend, (product,), False)
        assert [s[1] for s in plan.steps] == ["gather", "matmul"]


def test_import_and_numpy_backend_load_nothing_native():
    # Reference tests/test_cuda.py:682-704: importing the package and using
    # the NumPy backend must not load the optional device runtimes.
    import subprocess
    import sys
    import textwrap

    package = Path(p.__file__).resolve().parents[1]
    script = textwrap.dedent(
        f"""
        import sys
        sys.path.insert(0, {str(package)!r})
        import openpacho
        assert openpacho.get_backend("numpy").name == "numpy"
        maps = open("/proc/self/maps").read()
        for library in ("libpacho_hip", "libamdhip64", "libhiprtc"):
            assert library not in maps, library + " loaded without the hip backend"
        assert "openpacho._hip_lib" not in sys.modules and "torch" not in sys.modules
        """
    )
    completed = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120)
    assert completed.returncode == 0, completed.stderr or completed.stdout
