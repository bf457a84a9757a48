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
"""

import inspect
from collections import Counter, OrderedDict
from functools import update_wrapper
from threading import RLock

import numpy as np

from ._array import ndarray
from ._fusion import Expression, InputRef, ScalarExpression, TraceBackend
from ._ops import UFUNCS, HostScalar
from ._padding import prepare_padding, validate_padding
from .backends import use_backend
from .exceptions import BackendMismatchError

ELEMENTWISE = frozenset({f.__name__ for f in UFUNCS.values()} | {"cast", "where"})
_DYNAMIC_SCALARS = (int, float, bool, np.generic)


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
        try:
            return _BUILTIN_SIGNATURES[function]
        except (KeyError, TypeError):
            raise TypeError(f"compile cannot bind the arguments of {function!r}") from None


def _bind(function, args, kwargs, signature=None):
    signature = signature or _signature_of(function)
    if any(p.kind in (p.VAR_KEYWORD, p.VAR_POSITIONAL) for p in signature.parameters.values()):
        raise TypeError("compile requires named parameters, without *args or **kwargs")
    bound = signature.bind(*args, **kwargs)
    bound.apply_defaults()
    return bound


def capture_call(function, args, kwargs, *, elementwise_only=False, static_argnames=(), padding=False):
    """Trace ``function`` once and return ``(plan, bindings)``."""
    bound = _bind(function, args, kwargs)
    bindings = tuple(bound.arguments.values())
    arrays = [v for v in bindings if isinstance(v, ndarray)]
    if not arrays:
        raise TypeError("Capture requires at least one OpenPacho array argument")
    target = arrays[0]._backend
    if getattr(target, "_is_tracing", False):
        raise TypeError("Nested compile/fuse calls are not supported; wrap the outer plain function")
    if any(v._backend is not target for v in arrays):
        raise BackendMismatchError("Captured arguments belong to different backends/devices")
    trace = TraceBackend(target, elementwise_only=elementwise_only)
    for position, (name, value) in enumerate(tuple(bound.arguments.items())):
        if name in static_argnames:
            continue
        if isinstance(value, ndarray):
            bound.arguments[name] = Expression(trace, value.shape, value.dtype, value=InputRef(position))
        elif isinstance(value, _DYNAMIC_SCALARS):
            bound.arguments[name] = ScalarExpression(lambda b, i=position: b[i], value)
        else:
            raise TypeError(
                f"Argument {name!r} must be an OpenPacho array or numeric scalar; "
                "declare shape/axis options in static_argnames"
            )
    with use_backend(trace):
        result = function(*bound.args, **bound.kwargs)
    multiple = isinstance(result, tuple)
    outputs = result if multiple else (result,)
    if not outputs or any(not isinstance(v, Expression) for v in outputs):
        raise TypeError("Captured functions must return array expressions")
    if elementwise_only and multiple:
        raise TypeError("fuse must return one elementwise array expression")
    return ExecutionPlan(target, outputs, multiple, padding=padding), bindings


def _post_order(outputs):
    order, seen = [], set()
    stack = [(node, False) for node in reversed(outputs)]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            order.append(node)
            continue
        if id(node) in seen:
            continue
        seen.add(id(node))
        stack.append((node, True))
        for child in reversed(node.inputs):
            if id(child) not in seen:
                stack.append((child, False))
    return order


class ExecutionPlan:
    def __init__(self, backend, outputs, multiple, *, padding=False):
        self.backend = backend
        self.outputs = outputs
        self.multiple = multiple
        self.padding = validate_padding(padding)
        factory = getattr(backend, "create_lowering", None)
        self.lowering = None if factory is None else factory()
        self._execution_scope = getattr(backend, "execution_scope", None)
        self.nodes = _post_order(outputs)
        # A consumer that reads a node twice (x*x) counts once.
        self.uses = Counter(child for node in self.nodes for child in {id(c) for c in node.inputs})
        self.output_ids = {id(o) for o in outputs}
        self.steps = []
        self._built = set()
        for output in outputs:
            self._ensure(output)
        launches = sum(
            getattr(payload, "dispatch_count", 1) if kind == "padded_matmul" else 1
            for _, kind, _, payload in self.steps
        )
        if launches < getattr(backend, "execution_scope_min_steps", 0):
            self._execution_scope = None
        self.live_uses = Counter(id(a) for _, _, args, _ in self.steps for a in args)
        self.live_uses.update(id(o) for o in outputs)

    # ---- grouping ---------------------------------------------------------------

    def _private(self, node):
        return self.uses[id(node)] <= 1 and id(node) not in self.output_ids

    def _private_transpose(self, node):
        """A gather that is exactly the full transpose of a 2-D array, used once."""
        if node.op != "gather" or len(node.inputs) != 1 or len(node.shape) != 2 or not self._private(node):
            return False
        original = node.inputs[0]
        return (
            len(original.shape) == 2
            and tuple(node.shape) == tuple(original.shape[::-1])
            and node.dtype == original.dtype
            and node.attrs.get("offset") == 0
            and tuple(node.attrs.get("strides", ())) == (1, original.shape[1])
        )

    def _add(self, node, kind, args, payload=None):
        self.steps.append((node, kind, tuple(args), payload))
        self._built.add(id(node))

    def _ensure_all(self, nodes):
        for child in nodes:
            self._ensure(child)

    def _collect(self, root):
        """Inline private elementwise producers under ``root``; return (group, leaves)."""
        group, leaves, visited = [], [], set()

        def visit(current, is_root):
            if id(current) in visited:
                return
            visited.add(id(current))
            if current.op in ELEMENTWISE and (is_root or self._private(current)):
                for child in current.inputs:
                    visit(child, False)
                group.append(current)
            else:
                self._ensure(current)
                leaves.append(current)

        visit(root, True)
        return group, leaves

    def _ensure(self, node):
        if id(node) in self._built:
            return
        if node.op in ("input", "scalar"):
            self._built.add(id(node))
            return
        lowering = self.lowering
        if node.op == "matmul" and (self.padding or node.attrs.get("padding", False)):
            left, right = node.inputs
            plan = prepare_padding(self.backend, left.shape, right.shape, node.shape, node.dtype)
            if plan is not None:
                self._ensure_all(node.inputs)
                return self._add(node, "padded_matmul", node.inputs, plan)
        prepare_layout = getattr(self.backend, "prepare_layout_matmul", None)
        if node.op == "matmul" and prepare_layout is not None:
            transposed = tuple(self._private_transpose(arg) for arg in node.inputs)
            if any(transposed):
                args = tuple(arg.inputs[0] if t else arg for arg, t in zip(node.inputs, transposed))
                layout = prepare_layout(
                    args[0].shape,
                    args[1].shape,
                    node.shape,
                    node.dtype,
                    transpose_a=transposed[0],
                    transpose_b=transposed[1],
                )
                if layout is not None:
                    self._ensure_all(args)
                    return self._add(node, "layout_matmul", args, layout)
        if lowering is not None and node.op == "subtract" and node.inputs[1].op == "matmul":
            rhs, product = node.inputs
            matrix, vector = product.inputs
            if self._private(product) and lowering.can_residual_matvec(matrix, vector, rhs, node):
                args = (matrix, vector, rhs)
                self._ensure_all(args)
                return self._add(node, "residual_matvec", args)
        if lowering is not None and node.op in ELEMENTWISE:
            group, leaves = self._collect(node)
            arguments, payload = lowering.prepare_fused(node, group, leaves)
            return self._add(node, "fused", arguments, payload)
        if (
            lowering is not None
            and node.op == "reduce"
            and node.inputs[0].op in ELEMENTWISE
            and self._private(node.inputs[0])
        ):
            group, leaves = self._collect(node.inputs[0])
            arguments, payload = lowering.prepare_map_reduce(node, group, leaves)
            return self._add(node, "map_reduce", arguments, payload)
        materialized = getattr(lowering, "can_reduce_materialized", None)
        if node.op == "reduce" and materialized is not None and materialized(node):
            self._ensure_all(node.inputs)
            arguments, payload = lowering.prepare_map_reduce(node, (), node.inputs)
            return self._add(node, "map_reduce", arguments, payload)
        self._ensure_all(node.inputs)
        self._add(node, node.op, node.inputs)

    # ---- execution ----------------------------------------------------------------

    def execute(self, bindings):
        if self._execution_scope is not None:
            with self._execution_scope():
                return self._run(bindings)
        return self._run(bindings)

    def _run(self, bindings):
        backend = self.backend
        values = {}
        remaining = self.live_uses.copy()

        def fetch(node):
            key = id(node)
            if key in values:
                return values[key]
            if node.op == "input":
                value = bindings[node.value.index]
            elif node.op == "scalar":
                value = node.value
                if isinstance(value, ScalarExpression):
                    value = HostScalar(value.evaluate(bindings), node.dtype)
            else:
                raise RuntimeError(f"Missing plan dependency {node.op}")
            values[key] = value
            return value

        def as_array(value):
            if isinstance(value, HostScalar):
                return ndarray._wrap(backend.full((), value._data, value.dtype), (), value.dtype, backend)
            return value

        for node, kind, args, payload in self.steps:
            operands = [fetch(a) for a in args]
            if kind == "fused":
                data = self.lowering.run_fused(node, payload, args, operands)
            elif kind == "map_reduce":
                data = self.lowering.run_map_reduce(node, payload, args, operands)
            elif kind in ELEMENTWISE:
                converted = []
                for value, dtype in zip(operands, node.resolved):
                    if isinstance(value, HostScalar):
                        converted.append(HostScalar(value._data, dtype))
                    else:
                        converted.append(value if value.dtype == dtype else value.astype(dtype, copy=False))
                data = backend.elementwise(kind, converted, node.shape, node.dtype)
            else:
                operands = [as_array(v) for v in operands]
                data = self._primitive(node, kind, payload, operands)
            values[id(node)] = ndarray._wrap(data, node.shape, node.dtype, backend)
            for arg in args:
                remaining[id(arg)] -= 1
                if remaining[id(arg)] == 0:
                    values.pop(id(arg), None)
        results = [as_array(fetch(node)) for node in self.outputs]
        return tuple(results) if self.multiple else results[0]

    def _primitive(self, node, kind, payload, operands):
        backend = self.backend
        if kind == "reduce":
            options = {"operation": node.attrs["operation"]} if "operation" in node.attrs else {}
            return backend.reduce(operands[0], node.attrs["axes"], node.attrs["keepdims"], node.dtype, **options)
        if kind == "matmul":
            return backend.matmul(*operands, node.shape, node.dtype)
        if kind in ("padded_matmul", "layout_matmul"):
            return payload.run(*operands)
        if kind == "norm":
            return backend.norm(operands[0], node.attrs["axes"], node.attrs["keepdims"], node.dtype)
        if kind == "residual_matvec":
            return backend.residual_matvec(*operands)
        if kind == "gather":
            return backend.gather(operands[0], node.shape, node.attrs["offset"], node.attrs["strides"])
        if kind == "reshape":
            return operands[0]._data
        if kind == "full":
            return backend.full(node.shape, node.attrs["value"], node.dtype)
        raise NotImplementedError(f"No execution rule for {kind}")

    def explain(self):
        steps = []
        for node, kind, _, payload in self.steps:
            step = {"kind": kind, "shape": node.shape, "dtype": str(node.dtype)}
            if kind in ("reduce", "map_reduce"):
                step["operation"] = node.attrs.get("operation", "sum")
            if kind == "padded_matmul":
                step["padding"] = payload.explain()
            if kind == "layout_matmul":
                step["layout"] = payload.explain()
            steps.append(step)
        return {
            "backend": self.backend.name,
            "device": self.backend.device,
            "blas": getattr(self.backend, "blas", None),
            "padding": self.padding,
            "outputs": len(self.outputs),
            "steps": steps,
            "host_observations": 0,
            "python_retrace_on_cache_hit": False,
        }


# ---- cached compiled functions -----------------------------------------------------


def _static_key(value):
    if isinstance(value, tuple):
        return (tuple, tuple(_static_key(v) for v in value))
    if value is None or isinstance(value, (str, int, float, bool, np.dtype)):
        return (type(value), value)
    raise TypeError("Static arguments must be immutable scalar values, dtypes or tuples")


def _positional_only_signature(signature):
    return all(p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD) for p in signature.parameters.values())


class CompiledFunction:
    def __init__(self, function, static_argnames=(), cache_size=32, *, padding=False):
        self._padding = validate_padding(padding)
        if isinstance(static_argnames, str):
            static_argnames = (static_argnames,)
        self.static_argnames = tuple(static_argnames)
        signature = _signature_of(function)
        if not set(self.static_argnames) <= set(signature.parameters):
            raise ValueError("static_argnames contains an unknown parameter")
        if not isinstance(cache_size, int) or cache_size < 1:
            raise ValueError("cache_size must be a positive integer")
        self.python_function = function
        self._signature = signature
        self._names = tuple(signature.parameters)
        self._fast = _positional_only_signature(signature)
        self.max_size = cache_size
        self._plans = OrderedDict()
        self._lock = RLock()
        self._hits = 0
        self._misses = 0
        update_wrapper(self, function)

    @property
    def padding(self):
        return self._padding

    def _key_part(self, name, value):
        if name in self.static_argnames:
            return (name, "static", _static_key(value))
        if isinstance(value, ndarray):
            if getattr(value._backend, "_is_tracing", False):
                raise TypeError("Nested compiled calls are not supported")
            return (name, "array", value.shape, value.dtype.str, value._backend)
        if isinstance(value, _DYNAMIC_SCALARS):
            return (name, "scalar", type(value), np.asarray(value).dtype.str)
        raise TypeError(f"Unsupported dynamic argument {name!r}; use static_argnames for metadata")

    def _plan(self, args, kwargs):
        if self._fast and not kwargs and len(args) == len(self._names):
            bindings = args
            items = zip(self._names, bindings)
        else:
            bound = _bind(self.python_function, args, kwargs, self._signature)
            bindings = tuple(bound.arguments.values())
            items = bound.arguments.items()
        key = tuple(self._key_part(name, value) for name, value in items)
        with self._lock:
            plan = self._plans.get(key)
            if plan is not None:
                self._hits += 1
                self._plans.move_to_end(key)
                return plan, bindings
            plan, bindings = capture_call(
                self.python_function, args, kwargs, static_argnames=self.static_argnames, padding=self.padding
            )
            self._plans[key] = plan
            self._misses += 1
            while len(self._plans) > self.max_size:
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
        self._signature = compiled._signature
        self._fast = _positional_only_signature(self._signature)
        self._specs = []
        for name, value in zip(self._signature.parameters, bindings):
            if name in compiled.static_argnames:
                spec = ("static", _static_key(value))
            elif isinstance(value, ndarray):
                spec = ("array", value.shape, value.dtype, value._backend)
            else:
                spec = ("scalar", type(value), np.asarray(value).dtype)
            self._specs.append((name, spec))
        update_wrapper(self, compiled.python_function)

    @staticmethod
    def _matches(value, spec):
        kind = spec[0]
        if kind == "array":
            return (
                isinstance(value, ndarray)
                and value.shape == spec[1]
                and value.dtype == spec[2]
                and value._backend is spec[3]
            )
        if kind == "static":
            return _static_key(value) == spec[1]
        return type(value) is spec[1] and np.asarray(value).dtype == spec[2]

    def __call__(self, *args, **kwargs):
        if not kwargs and self._fast and len(args) == len(self._specs):
            bindings = args
        else:
            bindings = tuple(_bind(self.__wrapped__, args, kwargs, self._signature).arguments.values())
        for value, (name, spec) in zip(bindings, self._specs):
            if not self._matches(value, spec):
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
