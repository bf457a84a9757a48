"""Planning of reductions over materialized inputs (``can_reduce_materialized``).

Restates the reference's tests/test_materialized_extrema.py:83-216 without a
GPU: a lowering implemented on NumPy stands in for the device, and the hip
lowering's own capability (float32 min/max) is the native policy.
- The hook is optional and read from the lowering, never from a backend name.
- The native capability routes a bare float32 min/max over an array to one
  map_reduce step with no mapped group; other dtypes and sums stay plain
  reductions; an elementwise producer still fuses into the map_reduce.
- A producer shared by two reductions and an elementwise output is computed
  once per call, rebinds with prepared plans, and nothing is retained.
- A gather input keeps its own step ahead of the map_reduce.
- The hip source generator accepts a materialized leaf without a group.
"""

import gc
import weakref
from contextlib import contextmanager
from types import SimpleNamespace

import numpy as np
import pytest

import openpacho as p
from openpacho._array import ndarray
from openpacho._hip_lowering import HIPLowering
from openpacho.backends import NumpyBackend


class NumpyLowering:
    """A lowering that runs every fused and map-reduce group on NumPy and
    records what the compiler asks of it."""

    def __init__(self, backend):
        self.backend = backend
        self.requests = []  # (node, group, leaves) of each prepare_map_reduce
        self.outputs = []  # weak references to every mapped array it made
        self.reduced_inputs = []  # id of the array each reduction read

    def can_residual_matvec(self, *args):
        return False

    def prepare_fused(self, node, group, leaves):
        return tuple(leaves), tuple(group)

    def prepare_map_reduce(self, node, group, leaves):
        self.requests.append((node, tuple(group), tuple(leaves)))
        return tuple(leaves), tuple(group)

    def _evaluate(self, target, group, arguments, operands):
        known = {id(a): o for a, o in zip(arguments, operands)}
        for expression in group:
            inputs = []
            for child, dtype in zip(expression.inputs, expression.resolved):
                value = known[id(child)]
                data = np.asarray(value._data, dtype=dtype).reshape(-1)
                inputs.append(ndarray._wrap(data, value.shape, dtype, self.backend))
            data = self.backend.elementwise(expression.op, inputs, expression.shape, expression.dtype)
            self.outputs.append(weakref.ref(data))
            known[id(expression)] = ndarray._wrap(data, expression.shape, expression.dtype, self.backend)
        return known[id(target)]

    def run_fused(self, node, payload, arguments, operands):
        return self._evaluate(node, payload, arguments, operands)._data

    def run_map_reduce(self, node, payload, arguments, operands):
        mapped = self._evaluate(node.inputs[0], payload, arguments, operands)
        self.reduced_inputs.append(id(mapped._data))
        return self.backend.reduce(
            mapped, node.attrs["axes"], node.attrs["keepdims"], node.dtype, operation=node.attrs.get("operation", "sum")
        )


def numpy_device(policy=None, *, name="external"):
    """A NumPy backend whose lowering optionally offers ``policy`` as its
    ``can_reduce_materialized`` hook."""
    attributes = {} if policy is None else {"can_reduce_materialized": policy}
    lowering = type("Lowering", (NumpyLowering,), attributes)

    class Device(NumpyBackend):
        def create_lowering(self):
            return lowering(self)

    backend = Device()
    backend.name = name
    return backend


def _kinds(compiled, *args):
    return [step["kind"] for step in compiled.explain(*args)["steps"]]


@pytest.mark.parametrize("name", ("hip", "opencl", "cuda", "external"))
@pytest.mark.parametrize("opt_in", (False, True))
def test_capability_is_optional_and_independent_of_the_backend_name(name, opt_in):
    backend = numpy_device((lambda self, node: True) if opt_in else None, name=name)
    host = np.arange(15, dtype=np.float64).reshape(3, 5)
    array = p.asarray(host, backend=backend)
    calculate = p.compile(lambda x: p.max(x, axis=1))
    np.testing.assert_array_equal(p.asnumpy(calculate(array)), host.max(axis=1))
    assert _kinds(calculate, array) == ["map_reduce" if opt_in else "reduce"]


@pytest.mark.parametrize(
    "dtype,operation,kind",
    [
        (np.float32, "min", "map_reduce"),
        (np.float32, "max", "map_reduce"),
        (np.float64, "min", "reduce"),
        (np.float64, "max", "reduce"),
        (np.int32, "max", "reduce"),
        (np.bool_, "min", "reduce"),
        (np.float32, "sum", "reduce"),
    ],
)
def test_hip_capability_limits_the_bare_route_and_keeps_fusion(dtype, operation, kind):
    backend = numpy_device(HIPLowering.can_reduce_materialized)
    host = np.arange(15).reshape(3, 5).astype(dtype)
    array = p.asarray(host, backend=backend)
    function = getattr(p, operation)
    bare = p.compile(lambda x: function(x, axis=1))
    mapped = p.compile(lambda x: function(p.where(x == 0, x, x), axis=1))
    expected = getattr(np, operation)(host, axis=1, **({"dtype": dtype} if operation == "sum" else {}))
    for calculate, expected_kind in ((bare, kind), (mapped, "map_reduce")):
        np.testing.assert_array_equal(p.asnumpy(calculate(array)), expected)
        assert _kinds(calculate, array) == [expected_kind]
    if kind == "map_reduce":
        node, group, leaves = next(iter(bare._plans.values())).lowering.requests[0]
        assert group == () and leaves == node.inputs
    assert next(iter(mapped._plans.values())).lowering.requests[0][1]  # a non-empty mapped group


@pytest.mark.parametrize("returned", (False, True))
def test_shared_producer_is_computed_once_rebound_and_not_retained(returned):
    backend = numpy_device(HIPLowering.can_reduce_materialized)
    events, traces = [], []

    @contextmanager
    def scope():
        events.append("enter")
        try:
            yield
        finally:
            events.append("exit")

    backend.execution_scope = scope
    backend.execution_scope_min_steps = 4

    @p.compile
    def calculate(x, rate):
        traces.append("trace")
        shared = x + rate
        results = (p.min(shared, axis=0), p.max(shared, axis=1), shared * 2)
        return (shared, *results) if returned else results

    host = np.arange(15, dtype=np.float32).reshape(3, 5)
    first_input = p.asarray(host, backend=backend)
    first_ref = weakref.ref(first_input)
    prepared = calculate.prepare(first_input, 2.0)
    plan = prepared._plan
    assert [step[1] for step in plan.steps] == ["fused", "map_reduce", "map_reduce", "fused"]
    for node, group, leaves in plan.lowering.requests:
        assert not group and leaves == node.inputs
        assert leaves[0] is plan.steps[0][0]  # both reductions read the materialized sum
    backend.execution_scope = lambda: pytest.fail("the plan keeps the scope it was built with")

    first = calculate(first_input, 2.0)
    replacement = p.asarray(host * -3, backend=backend)
    second = prepared(x=replacement, rate=4.0)
    for actual, shared in ((first, host + 2), (second, host * -3 + 4)):
        expected = (shared.min(axis=0), shared.max(axis=1), shared * 2)
        if returned:
            expected = (shared, *expected)
        for result, want in zip(actual, expected):
            np.testing.assert_array_equal(p.asnumpy(result), want)
    assert traces == ["trace"] and calculate.cache_info()["misses"] == 1
    assert events == ["enter", "exit"] * 2
    read = plan.lowering.reduced_inputs
    assert len(read) == 4 and read[0] == read[1] and read[2] == read[3]
    assert len(plan.lowering.outputs) == 4  # one add and one multiply per call
    del first_input, replacement, first, second, actual, result
    gc.collect()
    assert first_ref() is None
    assert all(output() is None for output in plan.lowering.outputs)


def test_gather_input_keeps_its_own_step():
    backend = numpy_device(HIPLowering.can_reduce_materialized)
    host = np.arange(15, dtype=np.float32).reshape(3, 5)
    array = p.asarray(host, backend=backend)
    calculate = p.compile(lambda x: p.max(x.T, axis=1, keepdims=True))
    np.testing.assert_array_equal(p.asnumpy(calculate(array)), host.T.max(axis=1, keepdims=True))
    plan = next(iter(calculate._plans.values()))
    assert [step[1] for step in plan.steps] == ["gather", "map_reduce"]
    node, group, leaves = plan.lowering.requests[0]
    assert group == () and leaves == node.inputs and leaves[0] is plan.steps[0][0]


def test_hip_source_accepts_a_materialized_leaf_without_a_mapped_group():
    backend = numpy_device(HIPLowering.can_reduce_materialized)
    array = p.asarray(np.zeros((3, 8193), dtype=np.float32), backend=backend)
    prepared = p.compile(lambda x: p.max(x, axis=1)).prepare(array)
    node = prepared._plan.outputs[0]
    lowering = HIPLowering(SimpleNamespace())
    assert lowering.can_reduce_materialized(node)
    arguments, (source, count, chunks) = lowering.prepare_map_reduce(node, (), node.inputs)
    assert arguments == node.inputs
    assert "pacho_map_reduce" in source
    # 3 rows of 8193 elements: 8192-element chunks, two per row.
    assert (count, chunks) == (3, 2)
