"""Planning of reductions over materialized inputs (``can_reduce_materialized``).

Contracts (reference tests/test_materialized_extrema.py:83-216), checked
without a GPU: a lowering that evaluates its groups with NumPy stands in for
the device, and the hip lowering's own capability (float32 min/max) is the
native policy.
1. The hook is optional and read from the lowering, never from a backend name.
2. With the hip policy, a bare float32 min/max over an array is one map_reduce
   step with no mapped group; other dtypes and sums stay plain reductions; an
   elementwise producer still fuses into a map_reduce.
3. A producer shared by two reductions and an elementwise output is computed
   once per call, rebinds through prepared plans, and nothing is retained.
4. A gather input keeps its own step ahead of the map_reduce.
5. The hip source generator accepts a materialized leaf without a group.
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


def _hip_policy(node):
    return HIPLowering.can_reduce_materialized(None, node)


class HostLowering:
    """A lowering whose groups run as NumPy ufuncs on the backend's host
    storage. It logs each map_reduce request and every array it creates."""

    def __init__(self, backend, policy):
        self.backend = backend
        if policy is not None:
            self.can_reduce_materialized = policy  # an optional hook
        self.map_reduce_requests = []  # (node, group, leaves)
        self.created = []  # weak references to mapped results
        self.reduced_storage = []  # id of the storage each reduction read

    def can_residual_matvec(self, *args):
        return False

    def prepare_fused(self, node, group, leaves):
        return tuple(leaves), tuple(group)

    def prepare_map_reduce(self, node, group, leaves):
        self.map_reduce_requests.append((node, tuple(group), tuple(leaves)))
        return tuple(leaves), tuple(group)

    def _value(self, root, group, arguments, operands):
        """Host array of ``root`` after evaluating the group in order."""
        table = {id(a): np.asarray(o._data).reshape(o.shape) for a, o in zip(arguments, operands)}
        for node in group:
            values = [table[id(c)].astype(d, copy=False) for c, d in zip(node.inputs, node.resolved)]
            with np.errstate(all="ignore"):
                table[id(node)] = np.asarray(getattr(np, node.op)(*values), dtype=node.dtype)
        result = np.ascontiguousarray(np.broadcast_to(table[id(root)], root.shape)).reshape(-1)
        if group:
            self.created.append(weakref.ref(result))
        return result

    def run_fused(self, node, payload, arguments, operands):
        return self._value(node, payload, arguments, operands)

    def run_map_reduce(self, node, payload, arguments, operands):
        source = node.inputs[0]
        data = self._value(source, payload, arguments, operands)
        self.reduced_storage.append(id(data) if payload else id(operands[0]._data))
        mapped = ndarray._wrap(data, source.shape, source.dtype, self.backend)
        operation = node.attrs.get("operation", "sum")
        return self.backend.reduce(mapped, node.attrs["axes"], node.attrs["keepdims"], node.dtype, operation=operation)


def _device(policy, name="external"):
    class Device(NumpyBackend):
        def create_lowering(self):
            return HostLowering(self, policy)

    device = Device()
    device.name = name
    return device


def _plan(compiled):
    (plan,) = compiled._plans.values()
    return plan


def _kinds(plan):
    return [step.kind for step in plan.steps]


# ---- 1 -----------------------------------------------------------------------------


@pytest.mark.parametrize("hook", [None, lambda node: True])
@pytest.mark.parametrize("name", ["hip", "cuda", "opencl", "somewhere"])
def test_the_hook_alone_decides_not_the_backend_name(name, hook):
    device = _device(hook, name)
    host = np.linspace(-3, 3, 24).reshape(4, 6)
    largest = p.compile(lambda x: p.max(x, axis=0))
    np.testing.assert_array_equal(p.asnumpy(largest(p.asarray(host, backend=device))), host.max(axis=0))
    assert _kinds(_plan(largest)) == (["reduce"] if hook is None else ["map_reduce"])


# ---- 2 -----------------------------------------------------------------------------

NATIVE = [
    (np.float32, "min", True),
    (np.float32, "max", True),
    (np.float64, "max", False),
    (np.float64, "min", False),
    (np.int64, "min", False),
    (np.bool_, "max", False),
    (np.float32, "sum", False),
]


@pytest.mark.parametrize("dtype,operation,native", NATIVE)
def test_hip_policy_routes_bare_float32_extrema_only(dtype, operation, native):
    device = _device(_hip_policy)
    host = (np.arange(24).reshape(4, 6) % 7).astype(dtype)
    reduce = getattr(p, operation)
    bare = p.compile(lambda x: reduce(x, axis=0))
    produced = p.compile(lambda x: reduce(p.where(x > 2, x, x), axis=0))
    want = getattr(np, operation)(host, axis=0, **({"dtype": dtype} if operation == "sum" else {}))
    x = p.asarray(host, backend=device)
    for compiled in (bare, produced):
        np.testing.assert_array_equal(p.asnumpy(compiled(x)), want)
    assert _kinds(_plan(bare)) == (["map_reduce"] if native else ["reduce"])
    assert _kinds(_plan(produced)) == ["map_reduce"]
    node, group, leaves = _plan(produced).lowering.map_reduce_requests[0]
    assert group and node.inputs[0] is group[-1]
    if native:
        node, group, leaves = _plan(bare).lowering.map_reduce_requests[0]
        assert group == () and leaves == node.inputs


# ---- 3 -----------------------------------------------------------------------------


@pytest.mark.parametrize("return_producer", [False, True])
def test_a_shared_producer_runs_once_per_call_and_is_released(return_producer):
    device = _device(_hip_policy)
    scopes, captures = [], []

    @contextmanager
    def scope():
        scopes.append("enter")
        yield
        scopes.append("exit")

    device.execution_scope = scope
    device.execution_scope_min_steps = 4

    @p.compile
    def statistics(x, offset):
        captures.append(1)
        shifted = x + offset
        outputs = (p.min(shifted, axis=1), p.max(shifted, axis=0), shifted * 3)
        return (shifted, *outputs) if return_producer else outputs

    host = np.arange(20, dtype=np.float32).reshape(4, 5)
    first_input = p.asarray(host, backend=device)
    first_input_ref = weakref.ref(first_input)
    prepared = statistics.prepare(first_input, 1.0)
    plan = prepared._plan
    assert _kinds(plan) == ["fused", "map_reduce", "map_reduce", "fused"]
    producer = plan.steps[0].node
    for node, group, leaves in plan.lowering.map_reduce_requests:
        assert group == () and leaves == (producer,)  # both read the materialized sum
    device.execution_scope = lambda: pytest.fail("a built plan keeps its scope")

    results = [statistics(first_input, 1.0), prepared(x=p.asarray(host - 10, backend=device), offset=-2.0)]
    for result, shifted in zip(results, (host + 1, host - 12)):
        want = (shifted.min(axis=1), shifted.max(axis=0), shifted * 3)
        for got, expected in zip(result, ((shifted, *want) if return_producer else want)):
            np.testing.assert_array_equal(p.asnumpy(got), expected)
    assert len(captures) == 1 and statistics.cache_info()["misses"] == 1
    assert scopes == ["enter", "exit"] * 2
    read = plan.lowering.reduced_storage
    assert len(read) == 4 and read[0] == read[1] and read[2] == read[3]  # one producer per call
    assert len(plan.lowering.created) == 4  # the producer and the product, twice
    del first_input, results, result, got
    gc.collect()
    assert first_input_ref() is None
    assert not any(ref() is not None for ref in plan.lowering.created)


# ---- 4 -----------------------------------------------------------------------------


def test_a_gather_is_its_own_step_before_the_reduction():
    device = _device(_hip_policy)
    host = np.arange(20, dtype=np.float32).reshape(4, 5)
    compiled = p.compile(lambda x: p.min(x.T, axis=1, keepdims=True))
    np.testing.assert_array_equal(p.asnumpy(compiled(p.asarray(host, backend=device))), host.T.min(axis=1, keepdims=True))
    plan = _plan(compiled)
    assert _kinds(plan) == ["gather", "map_reduce"]
    (node, group, leaves), = plan.lowering.map_reduce_requests
    assert group == () and leaves == (plan.steps[0].node,)


# ---- 5 -----------------------------------------------------------------------------


@pytest.mark.parametrize("rows,width,chunks", [(3, 8193, 2), (2, 100, 1), (1, 3 * 8192, 3)])
def test_hip_source_for_a_materialized_leaf(rows, width, chunks):
    device = _device(_hip_policy)
    prepared = p.compile(lambda x: p.max(x, axis=1)).prepare(p.asarray(np.zeros((rows, width), np.float32), backend=device))
    node = prepared._plan.outputs[0]
    lowering = HIPLowering(SimpleNamespace())
    assert lowering.can_reduce_materialized(node)
    arguments, (source, count, per_row) = lowering.prepare_map_reduce(node, (), node.inputs)
    assert arguments == node.inputs and "pacho_map_reduce" in source
    assert (count, per_row) == (rows, chunks)  # 8192-element chunks per output row
