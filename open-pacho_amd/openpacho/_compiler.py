"""Cached, bounded function capture and backend-independent execution plans.

A CompiledFunction captures its Python body once per specialisation key
(argument shapes, dtypes, backends, scalar types and static values) into an
ExecutionPlan, then replays the plan on every call with fresh bindings.

Grouping rules (reference _compiler.py:87-238), which decide what
``explain()["steps"]`` reports:
- a matmul is its own step; with padding enabled and a backend padding plan it
  becomes one ``padded_matmul`` step; a matmul reading a private, full 2-D
  transpose becomes one ``layout_matmul`` step on the untransposed operand
  when the backend offers ``prepare_layout_matmul`` (reference :103-156);
- ``b - A @ x`` with a private product becomes ``residual_matvec`` when the
  lowerer accepts it (reference :157-176);
- an elementwise node starts a ``fused`` group that inlines every elementwise
  producer used only by that group and not returned by the function;
- a reduction of such a private elementwise producer becomes ``map_reduce``;
- everything else (reductions of materialised arrays, norms, gathers, fills,
  reshapes) is executed as its own primitive step.
Intermediates are released as soon as their last consumer has run.

Structure: binding helpers; capture (a traced call of the function on
Expression stand-ins); _Graph (consumer counts and the private/transposed
tests on a captured graph); _Planner (the rules above, tried in order for
each node, dependencies planned first); ExecutionPlan (runs the steps, one
executor per step kind); CompiledFunction and PreparedCall (caching and
rebinding, both keyed by the same per-argument specs).
"""

import inspect
from collections import Counter, OrderedDict
from functools import update_wrapper
from threading import RLock
from typing import Any, NamedTuple

import numpy as np

from ._array import ndarray
from ._fusion import Expression, InputRef, ScalarExpression, TraceBackend
from ._ops import UFUNCS, HostScalar
from ._padding import prepare_padding, validate_padding
from .backends import use_backend
from .exceptions import BackendMismatchError

ELEMENTWISE = frozenset({f.__name__ for f in UFUNCS.values()} | {"cast", "where"})
_DYNAMIC_SCALARS = (int, float, bool, np.generic)


# ---- binding ---------------------------------------------------------------------

# NumPy functions implemented in C expose no signature on some NumPy releases
# (np.where on 2.2); compile/fuse bind them by their documented parameters.
_BUILTIN_SIGNATURES = {
    np.where: inspect.Signature(
        [inspect.Parameter(name, inspect.Parameter.POSITIONAL_ONLY) for name in ("condition", "x", "y")]
    ),
}


def _signature_of(function):
    try:
        return inspect.signature(function)
    except ValueError:
        pass
    try:
        return _BUILTIN_SIGNATURES[function]
    except (KeyError, TypeError):
        raise TypeError(f"compile cannot bind the arguments of {function!r}") from None


def _bind(function, args, kwargs, signature=None):
    """Bound arguments (defaults applied) of a call; no variadic parameters."""
    signature = signature or _signature_of(function)
    variadic = (inspect.Parameter.VAR_KEYWORD, inspect.Parameter.VAR_POSITIONAL)
    if any(p.kind in variadic for p in signature.parameters.values()):
        raise TypeError("compile requires named parameters, without *args or **kwargs")
    bound = signature.bind(*args, **kwargs)
    bound.apply_defaults()
    return bound


def _all_positional(signature):
    """Every parameter can be passed by position: a full positional call needs
    no binding at all."""
    allowed = (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)
    return all(p.kind in allowed for p in signature.parameters.values())


def _bindings(function, signature, positional, args, kwargs):
    """Argument values in parameter order, binding only when needed."""
    if positional and not kwargs and len(args) == len(signature.parameters):
        return tuple(args)
    return tuple(_bind(function, args, kwargs, signature).arguments.values())


# ---- capture ---------------------------------------------------------------------


def _stand_in(trace, name, position, value, static_argnames):
    """The capture-time value of one argument."""
    if name in static_argnames:
        return value
    if isinstance(value, ndarray):
        return Expression(trace, value.shape, value.dtype, value=InputRef(position))
    if isinstance(value, _DYNAMIC_SCALARS):
        return ScalarExpression.argument(position, value)
    raise TypeError(
        f"Argument {name!r} must be an OpenPacho array or numeric scalar; "
        "declare shape/axis options in static_argnames"
    )


def _trace_target(values):
    """The backend that every array argument lives on: the trace's target.

    Refuses a call without arrays, a capture inside a running capture (the
    arrays would be the outer trace's stand-ins) and arrays of two backends.
    """
    homes = [value._backend for value in values if isinstance(value, ndarray)]
    if not homes:
        raise TypeError("Capture requires at least one OpenPacho array argument")
    if getattr(homes[0], "_is_tracing", False):
        raise TypeError("Nested compile/fuse calls are not supported; wrap the outer plain function")
    if len({id(home) for home in homes}) > 1:
        raise BackendMismatchError("Captured arguments belong to different backends/devices")
    return homes[0]


def _plan_outputs(result, elementwise_only):
    """(outputs, multiple): a tuple result names several outputs, anything
    else one; every output must be a traced array expression, and fuse()
    plans have exactly one."""
    multiple = isinstance(result, tuple)
    outputs = result if multiple else (result,)
    if not outputs or not all(isinstance(value, Expression) for value in outputs):
        raise TypeError("Captured functions must return array expressions")
    if elementwise_only and multiple:
        raise TypeError("fuse must return one elementwise array expression")
    return outputs, multiple


def capture_call(function, args, kwargs, *, elementwise_only=False, static_argnames=(), padding=False):
    """Run ``function`` once on stand-ins of its arguments and return
    ``(plan, bindings)``: the plan of the expression graph it built on a
    recording backend, and the bound argument values (defaults applied) in
    parameter order, which the plan's InputRef/argument positions index.

    Capture contract (reference _compiler.py:30-68): arrays become
    expressions of their shape and dtype, numeric scalars become scalar
    arguments, names in ``static_argnames`` keep their values (they may shape
    the graph), and anything else is refused.
    """
    bound = _bind(function, args, kwargs)
    bindings = tuple(bound.arguments.values())
    target = _trace_target(bindings)
    trace = TraceBackend(target, elementwise_only=elementwise_only)
    stand_ins = {
        name: _stand_in(trace, name, position, value, static_argnames)
        for position, (name, value) in enumerate(bound.arguments.items())
    }
    call = inspect.BoundArguments(bound.signature, stand_ins)
    with use_backend(trace):
        result = function(*call.args, **call.kwargs)
    outputs, multiple = _plan_outputs(result, elementwise_only)
    return ExecutionPlan(target, outputs, multiple, padding=padding), bindings


# ---- graph analysis ----------------------------------------------------------------


class _Graph:
    """Consumers of each node of a captured graph, and the two structural
    tests the grouping rules ask."""

    def __init__(self, outputs):
        self.outputs = {id(o) for o in outputs}
        self.consumers = Counter()
        seen, pending = set(), list(outputs)
        while pending:
            node = pending.pop()
            if id(node) in seen:
                continue
            seen.add(id(node))
            # x * x reads x once for its consumer.
            self.consumers.update({id(child) for child in node.inputs})
            pending.extend(node.inputs)

    def private(self, node):
        """Read by at most one node and not returned: it can be inlined."""
        return self.consumers[id(node)] <= 1 and id(node) not in self.outputs

    def private_full_transpose(self, node):
        """A private gather that is exactly the transpose of a whole 2-D array."""
        if node.op != "gather" or len(node.inputs) != 1 or len(node.shape) != 2 or not self.private(node):
            return False
        source = node.inputs[0]
        rows_cols = tuple(source.shape)
        return (
            len(rows_cols) == 2
            and tuple(node.shape) == rows_cols[::-1]
            and node.dtype == source.dtype
            and node.attrs.get("offset") == 0
            and tuple(node.attrs.get("strides", ())) == (1, rows_cols[1])
        )


class Step(NamedTuple):
    node: Any
    kind: str
    args: tuple
    payload: Any = None


class _Planner:
    """Turns a captured graph into steps. For each node the rules are tried in
    order; the first that applies emits the node's step after planning the
    nodes it reads."""

    def __init__(self, backend, lowering, padding, graph):
        self.backend, self.lowering, self.padding, self.graph = backend, lowering, padding, graph
        self.steps = []
        self._done = set()
        self._rules = (
            self._padded_product,
            self._layout_product,
            self._residual,
            self._fused,
            self._mapped_reduction,
            self._materialized_reduction,
        )

    def plan(self, node):
        if id(node) in self._done:
            return
        if node.op in ("input", "scalar"):
            self._done.add(id(node))
            return
        for rule in self._rules:
            if rule(node):
                return
        self._emit(node, node.op, node.inputs)

    def _emit(self, node, kind, args, payload=None, *, planned=False):
        if not planned:
            for arg in args:
                self.plan(arg)
        self.steps.append(Step(node, kind, tuple(args), payload))
        self._done.add(id(node))
        return True

    def _group(self, root):
        """Inline ``root`` and every private elementwise producer under it:
        (group in dependency order, leaves read by the group). Leaves are
        planned as they are met."""
        group, leaves, visited = [], [], set()

        def visit(node, is_root):
            if id(node) in visited:
                return
            visited.add(id(node))
            if node.op in ELEMENTWISE and (is_root or self.graph.private(node)):
                for child in node.inputs:
                    visit(child, False)
                group.append(node)
            else:
                self.plan(node)
                leaves.append(node)

        visit(root, True)
        return group, leaves

    # Rules. Each returns True when it emitted the node's step.

    def _padded_product(self, node):
        if node.op != "matmul" or not (self.padding or node.attrs.get("padding", False)):
            return False
        left, right = node.inputs
        plan = prepare_padding(self.backend, left.shape, right.shape, node.shape, node.dtype)
        return plan is not None and self._emit(node, "padded_matmul", node.inputs, plan)

    def _layout_product(self, node):
        prepare = getattr(self.backend, "prepare_layout_matmul", None)
        if node.op != "matmul" or prepare is None:
            return False
        flags = tuple(self.graph.private_full_transpose(arg) for arg in node.inputs)
        if not any(flags):
            return False
        stored = tuple(arg.inputs[0] if flag else arg for arg, flag in zip(node.inputs, flags))
        layout = prepare(stored[0].shape, stored[1].shape, node.shape, node.dtype,
                         transpose_a=flags[0], transpose_b=flags[1])
        return layout is not None and self._emit(node, "layout_matmul", stored, layout)

    def _residual(self, node):
        if self.lowering is None or node.op != "subtract" or node.inputs[1].op != "matmul":
            return False
        rhs, product = node.inputs
        matrix, vector = product.inputs
        if not self.graph.private(product) or not self.lowering.can_residual_matvec(matrix, vector, rhs, node):
            return False
        return self._emit(node, "residual_matvec", (matrix, vector, rhs))

    def _fused(self, node):
        if self.lowering is None or node.op not in ELEMENTWISE:
            return False
        group, leaves = self._group(node)
        arguments, payload = self.lowering.prepare_fused(node, group, leaves)
        return self._emit(node, "fused", arguments, payload, planned=True)

    def _mapped_reduction(self, node):
        if self.lowering is None or node.op != "reduce":
            return False
        source = node.inputs[0]
        if source.op not in ELEMENTWISE or not self.graph.private(source):
            return False
        group, leaves = self._group(source)
        arguments, payload = self.lowering.prepare_map_reduce(node, group, leaves)
        return self._emit(node, "map_reduce", arguments, payload, planned=True)

    def _materialized_reduction(self, node):
        accepts = getattr(self.lowering, "can_reduce_materialized", None)
        if node.op != "reduce" or accepts is None or not accepts(node):
            return False
        for arg in node.inputs:
            self.plan(arg)
        arguments, payload = self.lowering.prepare_map_reduce(node, (), node.inputs)
        return self._emit(node, "map_reduce", arguments, payload, planned=True)


# ---- execution ---------------------------------------------------------------------


class ExecutionPlan:
    """The steps of one captured specialisation, run on fresh bindings."""

    def __init__(self, backend, outputs, multiple, *, padding=False):
        self.backend = backend
        self.outputs = outputs
        self.multiple = multiple
        self.padding = validate_padding(padding)
        factory = getattr(backend, "create_lowering", None)
        self.lowering = factory() if factory is not None else None
        planner = _Planner(backend, self.lowering, self.padding, _Graph(outputs))
        for output in outputs:
            planner.plan(output)
        self.steps = planner.steps
        # A backend scope (a lock held for the whole plan) only pays for plans
        # of at least its minimum number of launches.
        scope = getattr(backend, "execution_scope", None)
        launches = sum(getattr(s.payload, "dispatch_count", 1) if s.kind == "padded_matmul" else 1 for s in self.steps)
        self._execution_scope = scope if launches >= getattr(backend, "execution_scope_min_steps", 0) else None
        # Reads of each value by later steps and by the result: a value is
        # released when the count reaches zero.
        self._reads = Counter(id(arg) for step in self.steps for arg in step.args)
        self._reads.update(id(o) for o in outputs)
        self._executors = {
            "fused": self._run_fused,
            "map_reduce": self._run_map_reduce,
            "reduce": self._run_reduce,
            "matmul": lambda node, payload, operands: backend.matmul(*operands, node.shape, node.dtype),
            "padded_matmul": lambda node, payload, operands: payload.run(*operands),
            "layout_matmul": lambda node, payload, operands: payload.run(*operands),
            "norm": lambda node, payload, operands: backend.norm(
                operands[0], node.attrs["axes"], node.attrs["keepdims"], node.dtype),
            "residual_matvec": lambda node, payload, operands: backend.residual_matvec(*operands),
            "gather": lambda node, payload, operands: backend.gather(
                operands[0], node.shape, node.attrs["offset"], node.attrs["strides"]),
            "reshape": lambda node, payload, operands: operands[0]._data,
            "full": lambda node, payload, operands: backend.full(node.shape, node.attrs["value"], node.dtype),
        }

    def execute(self, bindings):
        if self._execution_scope is None:
            return self._run(bindings)
        with self._execution_scope():
            return self._run(bindings)

    def _leaf(self, node, bindings):
        if node.op == "input":
            return bindings[node.value.index]
        if node.op == "scalar":
            value = node.value
            if isinstance(value, ScalarExpression):
                return HostScalar(value.evaluate(bindings), node.dtype)
            return value
        raise RuntimeError(f"Missing plan dependency {node.op}")

    def _materialized(self, value):
        """A host scalar operand as a 0-d array (primitive steps take arrays)."""
        if isinstance(value, HostScalar):
            return ndarray._wrap(self.backend.full((), value._data, value.dtype), (), value.dtype, self.backend)
        return value

    def _run(self, bindings):
        values, reads = {}, self._reads.copy()

        def value_of(node):
            if id(node) not in values:
                values[id(node)] = self._leaf(node, bindings)
            return values[id(node)]

        for node, kind, args, payload in self.steps:
            operands = [value_of(a) for a in args]
            if kind in ELEMENTWISE:
                data = self._run_elementwise(node, kind, operands)
            elif kind in ("fused", "map_reduce"):
                data = self._executors[kind](node, payload, args, operands)
            else:
                executor = self._executors.get(kind)
                if executor is None:
                    raise NotImplementedError(f"No execution rule for {kind}")
                data = executor(node, payload, [self._materialized(v) for v in operands])
            values[id(node)] = ndarray._wrap(data, node.shape, node.dtype, self.backend)
            for arg in args:
                reads[id(arg)] -= 1
                if not reads[id(arg)]:
                    values.pop(id(arg), None)
        results = tuple(self._materialized(value_of(o)) for o in self.outputs)
        return results if self.multiple else results[0]

    def _run_fused(self, node, payload, args, operands):
        return self.lowering.run_fused(node, payload, args, operands)

    def _run_map_reduce(self, node, payload, args, operands):
        return self.lowering.run_map_reduce(node, payload, args, operands)

    def _run_reduce(self, node, payload, operands):
        extra = {"operation": node.attrs["operation"]} if "operation" in node.attrs else {}
        return self.backend.reduce(operands[0], node.attrs["axes"], node.attrs["keepdims"], node.dtype, **extra)

    def _run_elementwise(self, node, kind, operands):
        """An elementwise node run alone (no lowering): operands in the node's
        resolved dtypes, scalars by value."""
        converted = []
        for value, dtype in zip(operands, node.resolved):
            if isinstance(value, HostScalar):
                converted.append(HostScalar(value._data, dtype))
            else:
                converted.append(value.astype(dtype, copy=False) if value.dtype != dtype else value)
        return self.backend.elementwise(kind, converted, node.shape, node.dtype)

    def explain(self):
        def describe(step):
            entry = {"kind": step.kind, "shape": step.node.shape, "dtype": str(step.node.dtype)}
            if step.kind in ("reduce", "map_reduce"):
                entry["operation"] = step.node.attrs.get("operation", "sum")
            if step.kind == "padded_matmul":
                entry["padding"] = step.payload.explain()
            elif step.kind == "layout_matmul":
                entry["layout"] = step.payload.explain()
            return entry

        return {
            "backend": self.backend.name,
            "device": self.backend.device,
            "blas": getattr(self.backend, "blas", None),
            "padding": self.padding,
            "outputs": len(self.outputs),
            "steps": [describe(step) for step in self.steps],
            "host_observations": 0,
            "python_retrace_on_cache_hit": False,
        }


# ---- caching and rebinding -----------------------------------------------------------


def _static_key(value):
    if isinstance(value, tuple):
        return (tuple, tuple(_static_key(v) for v in value))
    if value is None or isinstance(value, (str, int, float, bool, np.dtype)):
        return (type(value), value)
    raise TypeError("Static arguments must be immutable scalar values, dtypes or tuples")


def _argument_spec(name, value, static):
    """What a plan depends on in one argument: the whole value of a static
    argument; shape, dtype and backend of an array; type and dtype of a
    dynamic scalar."""
    if static:
        return ("static", _static_key(value))
    if isinstance(value, ndarray):
        if getattr(value._backend, "_is_tracing", False):
            raise TypeError("Nested compiled calls are not supported")
        return ("array", value.shape, value.dtype.str, value._backend)
    if isinstance(value, _DYNAMIC_SCALARS):
        return ("scalar", type(value), np.asarray(value).dtype.str)
    raise TypeError(f"Unsupported dynamic argument {name!r}; use static_argnames for metadata")


class CompiledFunction:
    def __init__(self, function, static_argnames=(), cache_size=32, *, padding=False):
        self._padding = validate_padding(padding)
        self.static_argnames = (static_argnames,) if isinstance(static_argnames, str) else tuple(static_argnames)
        signature = _signature_of(function)
        if not set(self.static_argnames) <= set(signature.parameters):
            raise ValueError("static_argnames contains an unknown parameter")
        if not isinstance(cache_size, int) or cache_size < 1:
            raise ValueError("cache_size must be a positive integer")
        self.python_function = function
        self._signature = signature
        self._names = tuple(signature.parameters)
        self._positional = _all_positional(signature)
        self.max_size = cache_size
        self._plans = OrderedDict()
        self._lock = RLock()
        self._hits = self._misses = 0
        update_wrapper(self, function)

    @property
    def padding(self):
        return self._padding

    def _specs(self, bindings):
        return tuple(
            (name, *_argument_spec(name, value, name in self.static_argnames))
            for name, value in zip(self._names, bindings)
        )

    def _plan(self, args, kwargs):
        bindings = _bindings(self.python_function, self._signature, self._positional, args, kwargs)
        key = self._specs(bindings)
        with self._lock:
            plan = self._plans.get(key)
            if plan is not None:
                self._hits += 1
                self._plans.move_to_end(key)
                return plan, bindings
            plan, bindings = capture_call(
                self.python_function, args, kwargs, static_argnames=self.static_argnames, padding=self.padding
            )
            self._misses += 1
            self._plans[key] = plan
            if len(self._plans) > self.max_size:
                self._plans.popitem(last=False)
            return plan, bindings

    def __call__(self, *args, **kwargs):
        # Plain NumPy inputs run the original Python function unchanged.
        if not any(isinstance(v, ndarray) for v in (*args, *kwargs.values())):
            return self.python_function(*args, **kwargs)
        plan, bindings = self._plan(args, kwargs)
        return plan.execute(bindings)

    def explain(self, *args, **kwargs):
        return self._plan(args, kwargs)[0].explain()

    def prepare(self, *args, **kwargs):
        """Specialise once; the returned callable validates every later binding."""
        plan, bindings = self._plan(args, kwargs)
        return PreparedCall(self, plan, bindings)

    def cache_info(self):
        with self._lock:
            return {"hits": self._hits, "misses": self._misses, "size": len(self._plans), "max_size": self.max_size}

    def clear_cache(self):
        with self._lock:
            self._plans.clear()
            self._hits = self._misses = 0


class PreparedCall:
    """A compiled specialisation that checks each call's arguments against it."""

    def __init__(self, compiled, plan, bindings):
        self._plan = plan
        self._compiled = compiled
        self._expected = compiled._specs(bindings)
        update_wrapper(self, compiled.python_function)

    def __call__(self, *args, **kwargs):
        compiled = self._compiled
        bindings = _bindings(self.__wrapped__, compiled._signature, compiled._positional, args, kwargs)
        for value, (name, *spec) in zip(bindings, self._expected):
            try:
                actual = _argument_spec(name, value, name in compiled.static_argnames)
            except TypeError:
                actual = None
            if actual is None or list(actual) != spec:
                raise ValueError(f"Prepared argument {name!r} does not match its specialization")
        return self._plan.execute(bindings)

    def explain(self):
        return dict(self._plan.explain(), prepared=True, binding_validation=True)


def compile(function=None, *, static_argnames=(), cache_size=32, padding=False):
    """Compile a pure array function; supports compile(f), @compile and @compile().

    NumPy inputs run the original function. OpenPacho inputs select their
    backend. Cache hits rebind arrays and dynamic scalars without tracing.
    Shape/axis options must be static; no host reads, mutation or dynamic
    Python control flow; no CPU fallback on capture or execution failure.
    ``padding`` allows private tile-aligned buffers for the GPU GEMM.
    """
    padding = validate_padding(padding)

    def decorate(fn):
        return CompiledFunction(fn, static_argnames, cache_size, padding=padding)

    return decorate if function is None else decorate(function)
