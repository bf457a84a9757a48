"""The opt-in padding seam of ``matmul(padding=...)`` and ``compile(padding=...)``.

Restates the backend-independent contracts of the reference's
tests/test_padding.py:62-327 and the crop-before-reduction case of :444-474:
- the flag is a strict boolean (Python or NumPy bool; ints, None, strings and
  arrays raise TypeError naming padding);
- plain NumPy inputs keep the native path, and on the NumPy backend padding
  is a no-op (no padded step; float64 keeps the ordinary route);
- routing goes through the backend's ``prepare_padded_matmul`` capability,
  whatever the backend's name: a None plan falls back to ``backend.matmul``,
  a plan is prepared once per compiled specialisation and rebinds without
  retaining inputs, explicit ``padding=True`` inside a default compile is
  captured, default padding never calls the factory and factory failures
  propagate;
- the execution scope counts the padded plan's dispatches, not logical steps;
- on hip, sums and means of a padded product see only the logical result.
"""

from __future__ import annotations

import gc
import weakref
from contextlib import contextmanager

import numpy as np
import pytest

import openpacho as pacho
from openpacho.backends import NumpyBackend


def _array(value, backend="numpy", dtype=None):
    return pacho.asarray(value, dtype=dtype, backend=backend)


def _padded_steps(details):
    return [step for step in details["steps"] if step["kind"] == "padded_matmul"]


class DecliningBackend(NumpyBackend):
    """Offers the padding capability and declines every request."""

    name = "declining-padding"

    def __init__(self):
        self.requests = 0
        self.products = 0

    def prepare_padded_matmul(self, ashape, bshape, shape, dtype):
        self.requests += 1
        return None

    def matmul(self, a, b, shape, dtype):
        self.products += 1
        return super().matmul(a, b, shape, dtype)


class HostPlan:
    """A padded plan that multiplies on the host and counts its runs."""

    def __init__(self, output_shape, dtype):
        self.output_shape = tuple(output_shape)
        self.dtype = np.dtype(dtype)
        self.runs = 0

    def run(self, left, right):
        self.runs += 1
        product = left._data.reshape(left.shape) @ right._data.reshape(right.shape)
        return np.asarray(product, dtype=self.dtype).reshape(-1).copy()

    def explain(self):
        return {
            "input_shapes": (),
            "padded_input_shapes": (),
            "output_shape": self.output_shape,
            "padded_output_shape": self.output_shape,
            "scratch_bytes": 0,
            "alignment": (32, 16, 32),
            "bounds_checks_removed": True,
        }


class PlanningBackend(NumpyBackend):
    """A backend of arbitrary name that always prepares a HostPlan."""

    name = "some-accelerator"

    def __init__(self):
        self.requests = []
        self.plans = []

    def prepare_padded_matmul(self, ashape, bshape, shape, dtype):
        self.requests.append((tuple(ashape), tuple(bshape), tuple(shape), np.dtype(dtype)))
        self.plans.append(HostPlan(shape, dtype))
        return self.plans[-1]


@pytest.mark.parametrize("flag", [1, 0, np.int64(1), np.int32(0), None, "true", np.array(True)])
def test_padding_flag_must_be_a_boolean(flag):
    left = _array(np.ones((2, 2), dtype=np.float32))
    right = _array(np.ones((2, 2), dtype=np.float32))
    with pytest.raises(TypeError, match="padding"):
        pacho.matmul(left, right, padding=flag)
    with pytest.raises(TypeError, match="padding"):
        pacho.compile(lambda a, b: a + b, padding=flag)


@pytest.mark.parametrize("flag", [False, True, np.bool_(False), np.bool_(True)])
def test_python_and_numpy_booleans_are_accepted(flag):
    left_host = np.arange(4, dtype=np.float32).reshape(2, 2)
    right_host = np.eye(2, dtype=np.float32)
    left, right = _array(left_host), _array(right_host)
    np.testing.assert_array_equal(pacho.asnumpy(pacho.matmul(left, right, padding=flag)), left_host @ right_host)
    compiled = pacho.compile(lambda a, b: pacho.matmul(a, b), padding=flag)
    np.testing.assert_array_equal(pacho.asnumpy(compiled(left, right)), left_host @ right_host)


def test_plain_numpy_inputs_run_the_python_function():
    calls = []

    @pacho.compile(padding=True)
    def native(left, right):
        calls.append("python")
        return np.matmul(left, right)

    left = np.arange(6, dtype=np.float32).reshape(2, 3)
    right = np.arange(12, dtype=np.float32).reshape(3, 4)
    result = native(left, right)
    assert isinstance(result, np.ndarray) and calls == ["python"]
    np.testing.assert_array_equal(result, left @ right)


@pytest.mark.parametrize(
    "shapes",
    [((33, 17), (17, 65)), ((31, 16), (16, 31)), ((0, 17), (17, 65)), ((33, 17), (17, 0)), ((17,), (17, 65)), ((33, 17), (17,))],
)
def test_numpy_backend_padding_is_a_no_op(shapes):
    rng = np.random.default_rng(1201)
    left_host, right_host = (rng.normal(size=shape).astype(np.float32) for shape in shapes)
    left, right = _array(left_host), _array(right_host)
    expected = left_host @ right_host
    for result in (pacho.matmul(left, right), pacho.matmul(left, right, padding=True)):
        assert result._backend is left._backend
        np.testing.assert_array_equal(pacho.asnumpy(result), expected)
    compiled = pacho.compile(lambda a, b: pacho.matmul(a, b), padding=True)
    details = compiled.explain(left, right)
    assert details["padding"] is True and not _padded_steps(details)
    np.testing.assert_array_equal(pacho.asnumpy(compiled(left, right)), expected)


def test_numpy_backend_float64_keeps_the_ordinary_route():
    rng = np.random.default_rng(1202)
    left_host, right_host = rng.normal(size=(33, 17)), rng.normal(size=(17, 65))
    left, right = _array(left_host), _array(right_host)
    compiled = pacho.compile(lambda a, b: pacho.matmul(a, b), padding=True)
    details = compiled.explain(left, right)
    assert details["padding"] is True and not _padded_steps(details)
    result = compiled(left, right)
    assert result.dtype == np.float64
    np.testing.assert_allclose(pacho.asnumpy(result), left_host @ right_host)


def test_declined_plan_falls_back_to_the_backend_product():
    backend = DecliningBackend()
    left_host = np.arange(33 * 17, dtype=np.float32).reshape(33, 17) / 13
    right_host = np.arange(17 * 65, dtype=np.float32).reshape(17, 65) / 17
    result = pacho.matmul(_array(left_host, backend), _array(right_host, backend), padding=True)
    assert backend.requests == 1 and backend.products == 1
    np.testing.assert_allclose(pacho.asnumpy(result), left_host @ right_host)


@pytest.mark.parametrize("dispatches", [1, 2, 4])
def test_execution_scope_counts_padded_dispatches(dispatches):
    class Scoped(PlanningBackend):
        execution_scope_min_steps = 2
        entered = 0

        @contextmanager
        def execution_scope(self):
            self.entered += 1
            yield

        def prepare_padded_matmul(self, *args):
            plan = super().prepare_padded_matmul(*args)
            plan.dispatch_count = dispatches
            return plan

    backend = Scoped()
    a = _array(np.ones((33, 17), dtype=np.float32), backend)
    b = _array(np.ones((17, 65), dtype=np.float32), backend)
    call = pacho.compile(lambda a, b: a @ b, padding=True).prepare(a, b)
    np.testing.assert_array_equal(pacho.asnumpy(call(a, b)), np.full((33, 65), 17))
    assert backend.entered == int(dispatches >= 2)


def test_plan_is_prepared_once_and_rebinds_without_retaining_inputs():
    backend = PlanningBackend()
    left_host = np.arange(33 * 17, dtype=np.float32).reshape(33, 17) / 19
    right_host = np.arange(17 * 65, dtype=np.float32).reshape(17, 65) / 23
    left, right = _array(left_host, backend), _array(right_host, backend)
    compiled = pacho.compile(lambda a, b: pacho.matmul(a, b), padding=True)
    refs = weakref.ref(left), weakref.ref(right)
    prepared = compiled.prepare(left, right)
    assert len(backend.requests) == 1 and backend.requests[0][:3] == ((33, 17), (17, 65), (33, 65))
    del left, right
    gc.collect()
    assert all(ref() is None for ref in refs)

    first_inputs = _array(left_host, backend), _array(right_host, backend)
    first = prepared(*first_inputs)
    first_host = pacho.asnumpy(first)
    second = prepared(_array(left_host + 1, backend), _array(right_host - 1, backend))
    assert len(backend.requests) == 1 and backend.plans[0].runs == 2
    assert first._data is not second._data
    np.testing.assert_array_equal(pacho.asnumpy(first), first_host)
    np.testing.assert_allclose(first_host, left_host @ right_host)
    np.testing.assert_allclose(pacho.asnumpy(second), (left_host + 1) @ (right_host - 1))
    compiled(*first_inputs)  # the ordinary entry point hits the prepared plan
    assert compiled.cache_info()["misses"] == 1 and compiled.cache_info()["hits"] == 1
    details = prepared.explain()
    assert details["padding"] is True and len(_padded_steps(details)) == 1


def test_explicit_padding_inside_a_default_compile_is_captured():
    backend = PlanningBackend()
    left_host, right_host = np.ones((33, 17), dtype=np.float32), np.ones((17, 65), dtype=np.float32)
    left, right = _array(left_host, backend), _array(right_host, backend)

    @pacho.compile
    def product(a, b):
        return pacho.matmul(a, b, padding=True)

    details = product.explain(left, right)
    assert details["padding"] is False and len(_padded_steps(details)) == 1
    assert len(backend.requests) == 1
    np.testing.assert_array_equal(pacho.asnumpy(product(left, right)), left_host @ right_host)


def test_default_padding_never_asks_and_factory_failures_propagate(monkeypatch):
    backend = PlanningBackend()
    left = _array(np.ones((33, 17), dtype=np.float32), backend)
    right = _array(np.ones((17, 65), dtype=np.float32), backend)

    def broken(*args):
        raise RuntimeError("padding preparation failed")

    monkeypatch.setattr(backend, "prepare_padded_matmul", broken)
    pacho.matmul(left, right)
    pacho.compile(lambda a, b: a @ b)(left, right)
    with pytest.raises(RuntimeError, match="padding preparation failed"):
        pacho.matmul(left, right, padding=True)
    with pytest.raises(RuntimeError, match="padding preparation failed"):
        pacho.compile(lambda a, b: a @ b, padding=True)(left, right)


@pytest.mark.gpu
@pytest.mark.parametrize("shapes", [((65, 47), (47, 67)), ((2, 1, 33, 17), (1, 3, 17, 65))])
def test_hip_padding_crops_before_sum_and_mean(hip, shapes):
    rng = np.random.default_rng(1204)
    left_host = (rng.normal(size=shapes[0]) + 2).astype(np.float32)
    right_host = (rng.normal(size=shapes[1]) + 1).astype(np.float32)
    left, right = pacho.asarray(left_host, backend=hip), pacho.asarray(right_host, backend=hip)

    def summaries(a, b):
        product = pacho.matmul(a, b, padding=True)
        return product.sum(axis=-1), product.mean(axis=(-2, -1))

    compiled = pacho.compile(summaries, padding=True)
    assert len(_padded_steps(compiled.explain(left, right))) == 1
    product = left_host.astype(np.float64) @ right_host.astype(np.float64)
    for sums, means in (summaries(left, right), compiled(left, right)):
        assert sums.shape == product.shape[:-1] and means.shape == product.shape[:-2]
        np.testing.assert_allclose(pacho.asnumpy(sums), product.sum(axis=-1), rtol=2e-5, atol=1e-3)
        np.testing.assert_allclose(pacho.asnumpy(means), product.mean(axis=(-2, -1)), rtol=2e-5, atol=1e-4)
