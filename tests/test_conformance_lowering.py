"""Backend extension contracts of compiled plans, without a GPU.

Restates the reference's tests/test_lowering.py:21-145 for this package, whose
plans read ``create_lowering`` from the backend object:
- a backend's name never selects a lowering, and a failing factory's error
  propagates;
- the execution scope is bound when the plan is built, entered once per
  call, and exited when execution fails;
- an independently written lowerer rebinds inputs and scalars without
  retracing, receives float32 host scalars for float32 work, keeps shared
  outputs apart and retains nothing;
- a backend without a lowerer keeps the ordinary primitive steps.
"""

import gc
import weakref
from contextlib import contextmanager

import numpy as np
import pytest

import openpacho as pacho
from openpacho._array import ndarray
from openpacho.backends import NumpyBackend


class Device(NumpyBackend):
    name = "example-device"


class NumpyLowerer:
    """Runs fused and map-reduce groups through the backend's elementwise and
    reduce primitives, recording host scalar dtypes and its outputs."""

    def __init__(self, backend):
        self.backend = backend
        self.outputs = []
        self.scalar_dtypes = []

    def can_residual_matvec(self, matrix, vector, rhs, node):
        return False

    def prepare_fused(self, node, group, leaves):
        return tuple(leaves), tuple(group)

    prepare_map_reduce = prepare_fused

    def _evaluate(self, group, arguments, operands):
        known = {id(a): o for a, o in zip(arguments, operands)}
        self.scalar_dtypes += [o.dtype for o in operands if getattr(o, "_host_scalar", False)]
        for expression in group:
            inputs = []
            for child, dtype in zip(expression.inputs, expression.resolved):
                value = known[id(child)]
                data = np.asarray(value._data, dtype=dtype).reshape(-1)
                inputs.append(ndarray._wrap(data, value.shape, dtype, self.backend))
            data = self.backend.elementwise(expression.op, inputs, expression.shape, expression.dtype)
            known[id(expression)] = ndarray._wrap(data, expression.shape, expression.dtype, self.backend)
        return known[id(group[-1])]

    def run_fused(self, node, payload, arguments, operands):
        data = self._evaluate(payload, arguments, operands)._data
        self.outputs.append(weakref.ref(data))
        return data

    def run_map_reduce(self, node, payload, arguments, operands):
        mapped = self._evaluate(payload, arguments, operands)
        return self.backend.reduce(mapped, node.attrs["axes"], node.attrs["keepdims"], node.dtype)


def _kinds(compiled, *args):
    return [step["kind"] for step in compiled.explain(*args)["steps"]]


@pytest.mark.parametrize("name", ["opencl", "cuda", "hip"])
def test_names_do_not_select_a_lowering_and_factory_errors_propagate(name):
    named = type("Named", (NumpyBackend,), {"name": name})()
    array = pacho.asarray(np.arange(4, dtype=np.float32), backend=named)
    compiled = pacho.compile(lambda a: (a + 1) * 2)
    np.testing.assert_array_equal(pacho.asnumpy(compiled(array)), (np.arange(4) + 1) * 2)
    assert next(iter(compiled._plans.values())).lowering is None

    class Broken(NumpyBackend):
        def create_lowering(self):
            raise RuntimeError("lowering preparation failed")

    with pytest.raises(RuntimeError, match="preparation failed"):
        pacho.compile(lambda a: a + 1)(pacho.asarray(np.arange(3, dtype=np.float32), backend=Broken()))


def test_execution_scope_is_bound_once_and_exits_on_failure():
    events = []

    class Scoped(Device):
        @contextmanager
        def execution_scope(self):
            events.append("enter")
            try:
                yield
            finally:
                events.append("exit")

    backend = Scoped()
    array = pacho.asarray(np.arange(3, dtype=np.float32), backend=backend)
    compiled = pacho.compile(lambda a: a + 1)
    np.testing.assert_array_equal(pacho.asnumpy(compiled(array)), [1, 2, 3])
    backend.execution_scope = lambda: pytest.fail("the scope is bound when the plan is built")
    compiled(array)

    def fail(*args):
        raise RuntimeError("execution failed")

    backend.elementwise = fail
    with pytest.raises(RuntimeError, match="execution failed"):
        compiled(array)
    assert events == ["enter", "exit"] * 3


def test_independent_lowerer_rebinds_and_keeps_shared_outputs(monkeypatch):
    monkeypatch.setattr(Device, "create_lowering", lambda self: NumpyLowerer(self), raising=False)
    backend = Device()

    @pacho.compile
    def operation(a, rate):
        shared = a + rate
        return shared, np.sum(shared * shared), shared - 1

    host = np.arange(12, dtype=np.float32).reshape(3, 4)
    array = pacho.asarray(host, backend=backend)
    array_ref = weakref.ref(array)
    first = operation(array, 2.0)
    plan = next(iter(operation._plans.values()))
    assert [step["kind"] for step in plan.explain()["steps"]] == ["fused", "map_reduce", "fused"]
    second = operation(pacho.asarray(host + 5, backend=backend), 3.0)
    for actual, expected in zip(first, (host + 2, np.sum((host + 2) ** 2), host + 1)):
        np.testing.assert_array_equal(pacho.asnumpy(actual), expected)
    for actual, expected in zip(second, (host + 8, np.sum((host + 8) ** 2), host + 7)):
        np.testing.assert_array_equal(pacho.asnumpy(actual), expected)
    assert operation.cache_info()["misses"] == 1
    assert plan.lowering.scalar_dtypes and all(d == np.float32 for d in plan.lowering.scalar_dtypes)
    del array, first, second, actual
    gc.collect()
    assert array_ref() is None
    assert all(output() is None for output in plan.lowering.outputs)


def test_backend_without_lowerer_keeps_ordinary_primitives():
    backend = Device()
    array = pacho.asarray(np.arange(5, dtype=np.float32), backend=backend)
    compiled = pacho.compile(lambda a: np.sum((a + 2) * a))
    np.testing.assert_array_equal(pacho.asnumpy(compiled(array)), 50)
    assert next(iter(compiled._plans.values())).lowering is None
    assert _kinds(compiled, array) == ["add", "multiply", "reduce"]
