"""hipRTC lowering of elementwise groups and mapped reductions for ``hip``.

The compiler owns grouping; this module turns one group into HIP source that
hp_rtc_compile builds for gfx950 with contraction off. Payloads hold source
text and launch geometry only, never runtime arrays or scalar values, so a
cached plan rebinds fresh operands on every call.

Numerics follow the reference lowering (_cuda_lowering.py:13-41): every node
converts each operand to its resolved dtype before the operation and rounds
its result to the node dtype, so a fused chain rounds exactly like the eager
sequence of NumPy-typed operations. Booleans are stored as one byte.
Integer add/subtract/multiply/negate wrap modulo 2^bits as in NumPy.
Mapped reductions use the extrema contract of the reduction kernels
(NaN propagates, min prefers -0, max prefers +0).
"""

from functools import lru_cache
from math import prod

import numpy as np

from ._array import ndarray

_CTYPE = {
    np.dtype("bool"): "unsigned char",
    np.dtype("int32"): "int",
    np.dtype("int64"): "long long",
    np.dtype("uint32"): "unsigned int",
    np.dtype("uint64"): "unsigned long long",
    np.dtype("float32"): "float",
    np.dtype("float64"): "double",
}
_UNSIGNED = {np.dtype("int32"): "unsigned int", np.dtype("int64"): "unsigned long long"}

BLOCK = 256
ELEMENTS_PER_THREAD = 4  # groups of VECTOR consecutive elements per thread
VECTOR = 4
REDUCE_CHUNK = 8192

_PRELUDE = r"""
// Four consecutive elements at p, aligned to four elements (one vector access).
template <typename T> __device__ __forceinline__ void pacho_load4(const T* __restrict__ p, T (&v)[4]) {
  typedef T V __attribute__((ext_vector_type(4)));
  const V x = *reinterpret_cast<const V*>(p);
  v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
}
template <typename T> __device__ __forceinline__ void pacho_store4(T* __restrict__ p, const T (&v)[4]) {
  typedef T V __attribute__((ext_vector_type(4)));
  V x;
  x[0] = v[0]; x[1] = v[1]; x[2] = v[2]; x[3] = v[3];
  *reinterpret_cast<V*>(p) = x;
}
template <typename T> __device__ __forceinline__ T pacho_min(T a, T b) { return a < b ? a : b; }
template <typename T> __device__ __forceinline__ T pacho_max(T a, T b) { return a > b ? a : b; }
__device__ __forceinline__ float pacho_min(float a, float b) {
  if (isnan(a)) return a; if (isnan(b)) return b;
  if (a == 0.0f && b == 0.0f) return signbit(a) ? a : b;
  return a < b ? a : b;
}
__device__ __forceinline__ float pacho_max(float a, float b) {
  if (isnan(a)) return a; if (isnan(b)) return b;
  if (a == 0.0f && b == 0.0f) return signbit(a) ? b : a;
  return a > b ? a : b;
}
__device__ __forceinline__ double pacho_min(double a, double b) {
  if (isnan(a)) return a; if (isnan(b)) return b;
  if (a == 0.0 && b == 0.0) return signbit(a) ? a : b;
  return a < b ? a : b;
}
__device__ __forceinline__ double pacho_max(double a, double b) {
  if (isnan(a)) return a; if (isnan(b)) return b;
  if (a == 0.0 && b == 0.0) return signbit(a) ? b : a;
  return a > b ? a : b;
}
"""


def ctype(dtype):
    return _CTYPE[np.dtype(dtype)]


def _operation(op, resolved, out_dtype):
    """C expression of ``op`` over operands ``a``, ``b``, ``c`` of the resolved dtypes."""
    kind = resolved[0].kind if resolved else "f"
    dt = resolved[0] if resolved else out_dtype
    wrap = dt in _UNSIGNED and op in ("add", "subtract", "multiply", "negative")
    if wrap:
        u, t = _UNSIGNED[dt], ctype(dt)
        return {
            "add": f"({t})(({u})a + ({u})b)",
            "subtract": f"({t})(({u})a - ({u})b)",
            "multiply": f"({t})(({u})a * ({u})b)",
            "negative": f"({t})(({u})0 - ({u})a)",
        }[op]
    if op == "absolute":
        if kind == "f":
            return "fabs(a)"
        if kind == "i":
            u, t = _UNSIGNED[dt], ctype(dt)
            return f"(a < 0 ? ({t})(({u})0 - ({u})a) : a)"
        return "a"
    if op == "isfinite":
        return "isfinite(a)" if kind == "f" else "1"
    table = {
        "add": "a + b",
        "subtract": "a - b",
        "multiply": "a * b",
        "true_divide": "a / b",
        "divide": "a / b",
        "power": "pow(a, b)",
        "negative": "-a",
        "positive": "a",
        "sqrt": "sqrt(a)",
        "exp": "exp(a)",
        "log": "log(a)",
        "sin": "sin(a)",
        "cos": "cos(a)",
        "tanh": "tanh(a)",
        "equal": "a == b",
        "not_equal": "a != b",
        "less": "a < b",
        "less_equal": "a <= b",
        "greater": "a > b",
        "greater_equal": "a >= b",
        "cast": "a",
        "where": "(a != 0) ? b : c",
    }
    if op not in table:
        raise NotImplementedError(f"hip lowering has no rule for {op}")
    return table[op]


def _broadcast_offset(root_shape, leaf_shape, var, suffix="LL"):
    """Element offset of ``leaf`` (right-aligned broadcast) at flat root index
    ``var``; constants carry ``suffix`` (``LL`` for 64-bit index math, ``U``
    for 32-bit)."""
    if tuple(leaf_shape) == tuple(root_shape):
        return var
    lead = len(root_shape) - len(leaf_shape)
    terms = []
    for axis, extent in enumerate(leaf_shape):
        if extent == 1:
            continue
        outer = prod(root_shape[lead + axis + 1 :])
        inner = prod(leaf_shape[axis + 1 :])
        terms.append(f"(({var} / {max(1, outer)}{suffix}) % {extent}{suffix}) * {inner}{suffix}")
    return " + ".join(terms) or f"0{suffix}"


def _rows_of_four(root_shape, leaf_shape):
    """True when four consecutive root elements starting at a multiple of
    four read four consecutive leaf elements: the leaf equals the root or is
    broadcast over leading axes only, and the root's last axis holds whole
    groups of four."""
    if tuple(leaf_shape) == tuple(root_shape):
        return True
    if not leaf_shape or not root_shape or root_shape[-1] % VECTOR != 0:
        return False
    return leaf_shape[-1] == root_shape[-1]


class _Leaf:
    __slots__ = ("scalar", "dtype", "shape")

    def __init__(self, scalar, dtype, shape):
        self.scalar, self.dtype, self.shape = scalar, np.dtype(dtype), tuple(shape)


def _body(root_shape, leaves, nodes, var="i", leaf_value=None, suffix="LL"):
    """Source lines computing each node; returns (params, lines, result symbol).

    ``leaves`` is a list of _Leaf; ``nodes`` a list of (op, input refs,
    resolved dtypes, out dtype) where refs index leaves (0..L-1) then nodes.
    ``leaf_value(k)``, when given, is the expression of array leaf k's value
    (else its load at flat index ``var``).
    """
    params, lines, names = [], [], []
    for k, leaf in enumerate(leaves):
        t = ctype(leaf.dtype)
        if leaf.scalar:
            params.append(f"{t} x{k}")
            lines.append(f"const {t} v{k} = x{k};")
        else:
            params.append(f"const {t}* __restrict__ x{k}")
            value = leaf_value(k) if leaf_value else f"x{k}[{_broadcast_offset(root_shape, leaf.shape, var, suffix)}]"
            lines.append(f"const {t} v{k} = {value};")
        names.append(f"v{k}")
    for j, (op, refs, resolved, out_dtype) in enumerate(nodes):
        symbol = f"v{len(leaves) + j}"
        lines.append(f"{ctype(out_dtype)} {symbol};")
        lines.append("{")
        for label, ref, dt in zip("abc", refs, resolved):
            source = names[ref]
            if dt.kind == "b":
                source = f"({source} != 0)"
            lines.append(f"  const {ctype(dt)} {label} = ({ctype(dt)})({source});")
        expression = _operation(op, resolved, out_dtype)
        if out_dtype.kind == "b":
            expression = f"(({expression}) != 0)"
        lines.append(f"  {symbol} = ({ctype(out_dtype)})({expression});")
        lines.append("}")
        names.append(symbol)
    return params, lines, names[-1]


def elementwise_source(root_shape, leaves, nodes, out_dtype):
    """One thread per VECTOR consecutive elements in each of
    ELEMENTS_PER_THREAD groups (a wave's group is 256 consecutive elements).
    A group whose operands all sit at 4-element alignment reads leaves that
    equal the root or repeat along leading axes (a bias) and writes the
    output with one vector access each (16 bytes for 4-byte types); other
    leaves, the tail and misaligned operands go element by element. Every
    element computes the same expression as in the element-by-element form,
    so the bits do not depend on the path."""
    count = prod(root_shape)
    span = BLOCK * ELEMENTS_PER_THREAD * VECTOR
    small = count + span < 2**32
    idx, suffix = ("unsigned", "U") if small else ("long long", "LL")
    t_out = ctype(out_dtype)
    params, lines, result = _body(root_shape, leaves, nodes, "i", suffix=suffix)
    params.append(f"{t_out}* __restrict__ out")
    scalar_body = "\n          ".join(lines)
    rows = [k for k, leaf in enumerate(leaves) if not leaf.scalar and _rows_of_four(root_shape, leaf.shape)]
    aligned = " && ".join(
        [f"((unsigned long long)x{k} % {VECTOR * leaves[k].dtype.itemsize}U == 0)" for k in rows]
        + [f"((unsigned long long)out % {VECTOR * out_dtype.itemsize}U == 0)"]
    )
    loads = "\n        ".join(
        f"{ctype(leaves[k].dtype)} l{k}[{VECTOR}]; pacho_load4(x{k} + "
        f"({_broadcast_offset(root_shape, leaves[k].shape, 'i0', suffix)}), l{k});"
        for k in rows
    )
    per_element = []
    for e in range(VECTOR):
        def leaf_value(k, e=e):
            if k in rows:
                return f"l{k}[{e}]"
            return f"x{k}[{_broadcast_offset(root_shape, leaves[k].shape, f'(i0 + {e}{suffix})', suffix)}]"

        _, element_lines, element_result = _body(root_shape, leaves, nodes, leaf_value=leaf_value, suffix=suffix)
        per_element.append("{\n          " + "\n          ".join(element_lines) + f"\n          r[{e}] = {element_result};\n        }}")
    vector_body = "\n        ".join(per_element)
    source = f"""{_PRELUDE}
extern "C" __global__ __launch_bounds__({BLOCK}) void pacho_elementwise({", ".join(params)}) {{
  const bool aligned = {aligned};
#pragma unroll
  for (int u = 0; u < {ELEMENTS_PER_THREAD}; ++u) {{
    const {idx} i0 = (({idx})(blockIdx.x * {ELEMENTS_PER_THREAD}U + u) * {BLOCK}U + threadIdx.x) * {VECTOR}U;
    if (aligned && i0 + {VECTOR}{suffix} <= {count}{suffix}) {{
        {loads}
        {t_out} r[{VECTOR}];
        {vector_body}
        pacho_store4(out + i0, r);
    }} else {{
#pragma unroll
      for (int e = 0; e < {VECTOR}; ++e) {{
        const {idx} i = i0 + e;
        if (i < {count}{suffix}) {{
          {scalar_body}
          out[i] = {result};
        }}
      }}
    }}
  }}
}}
"""
    grid = max(1, -(-count // span))
    return source, grid


def _identity(operation, dtype):
    t = ctype(dtype)
    if operation == "sum":
        return f"({t})0"
    if dtype.kind == "b":
        return "1" if operation == "min" else "0"
    if dtype.kind == "f":
        huge = "__builtin_huge_valf()" if dtype.itemsize == 4 else "__builtin_huge_val()"
        return f"({t})(-{huge})" if operation == "max" else f"({t})({huge})"
    info = np.iinfo(dtype)
    value = info.max if operation == "min" else info.min
    if dtype.kind == "i" and value == info.min:
        return f"(({t})({value + 1}LL) - ({t})1)"
    suffix = "ULL" if dtype.kind == "u" else "LL"
    return f"({t})({value}{suffix})"


def _combine(operation, dtype, left, right):
    if operation == "sum":
        return f"({left}) + ({right})"
    if dtype.kind == "b":
        op = "&&" if operation == "min" else "||"
        return f"(unsigned char)((({left}) != 0) {op} (({right}) != 0))"
    return f"pacho_{operation}({left}, {right})"


def _reduction_index(shape, axes):
    """Index of element (o, r) of ``shape`` with ``axes`` reduced, plus counts."""
    out_dims = [d for i, d in enumerate(shape) if i not in axes]
    red_dims = [shape[i] for i in axes]
    terms, oi, ri = [], 0, 0
    for axis, extent in enumerate(shape):
        stride = prod(shape[axis + 1 :])
        if axis in axes:
            step = prod(red_dims[ri + 1 :])
            terms.append(f"((r / {max(1, step)}LL) % {max(1, extent)}LL) * {stride}LL")
            ri += 1
        else:
            step = prod(out_dims[oi + 1 :])
            terms.append(f"((o / {max(1, step)}LL) % {max(1, extent)}LL) * {stride}LL")
            oi += 1
    return " + ".join(terms) or "0LL", prod(out_dims), prod(red_dims)


def map_reduce_source(mapped_shape, axes, leaves, nodes, operation, acc_dtype):
    index, count, reduced = _reduction_index(mapped_shape, axes)
    chunks = max(1, -(-reduced // REDUCE_CHUNK))
    if nodes:
        params, lines, result = _body(mapped_shape, leaves, nodes)
    else:  # reduction of a materialised array: the single leaf is the value
        params, lines, result = _body(mapped_shape, leaves, [])
    acc = ctype(acc_dtype)
    value = f"({result} != 0)" if (nodes and nodes[-1][3].kind == "b") else result
    params.append(f"{acc}* __restrict__ out")
    body = "\n      ".join(lines)
    waves = BLOCK // 64
    source = f"""{_PRELUDE}
extern "C" __global__ __launch_bounds__({BLOCK}) void pacho_map_reduce({", ".join(params)}) {{
  __shared__ {acc} partial[{waves}];
  const long long g = blockIdx.x;
  const long long o = g / {chunks}LL, chunk = g % {chunks}LL;
  const long long begin = chunk * {REDUCE_CHUNK}LL;
  const long long end = begin + {REDUCE_CHUNK}LL < {reduced}LL ? begin + {REDUCE_CHUNK}LL : {reduced}LL;
  {acc} acc = {_identity(operation, acc_dtype)};
  for (long long r = begin + threadIdx.x; r < end; r += {BLOCK}LL) {{
    const long long i = {index};
    {{
      {body}
      acc = {_combine(operation, acc_dtype, "acc", f"({acc})({value})")};
    }}
  }}
#pragma unroll
  for (int offset = 1; offset < 64; offset <<= 1) {{
    const {acc} other = __shfl_xor(acc, offset, 64);
    acc = {_combine(operation, acc_dtype, "acc", "other")};
  }}
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {{
    {acc} total = partial[0];
    for (int w = 1; w < {waves}; ++w) total = {_combine(operation, acc_dtype, "total", "partial[w]")};
    out[g] = total;
  }}
}}
"""
    return source, count, chunks


def _leaf_of(node):
    return _Leaf(node.op == "scalar", node.dtype, node.shape)


def _graph(group, leaves):
    position = {id(leaf): k for k, leaf in enumerate(leaves)}
    nodes = []
    for j, node in enumerate(group):
        position[id(node)] = len(leaves) + j
        refs = [position[id(child)] for child in node.inputs]
        nodes.append((node.op, refs, tuple(np.dtype(d) for d in node.resolved), np.dtype(node.dtype)))
    return [_leaf_of(leaf) for leaf in leaves], nodes


class HIPLowering:
    """Lowering protocol of the compiler (prepare/run for fused and map_reduce)."""

    def __init__(self, backend):
        self.backend = backend

    def can_residual_matvec(self, matrix, vector, rhs, node):
        """Fuse ``rhs - matrix @ vector`` (reference _lowering.py:20-30 rules).

        The backend's hp_gemv_residual reproduces the eager product bit for bit
        for every shape, so no shape is excluded.
        """
        product = node.inputs[1]
        return (
            getattr(self.backend, "blas", "custom") in (None, "custom")
            and matrix.ndim == 2
            and vector.ndim == rhs.ndim == 1
            and rhs.shape == product.shape == node.shape
            and node.dtype.kind == "f"
            and node.dtype == matrix.dtype == vector.dtype == rhs.dtype == product.dtype
        )

    def can_reduce_materialized(self, node):
        return (
            node.dtype.kind == "f"
            and node.dtype.itemsize == 4
            and node.attrs.get("operation") in ("min", "max")
        )

    def prepare_fused(self, node, group, leaves):
        specs, nodes = _graph(group, leaves)
        source, grid = elementwise_source(node.shape, specs, nodes, np.dtype(node.dtype))
        return tuple(leaves), (source, grid)

    def run_fused(self, node, payload, arguments, operands):
        source, grid = payload
        out = self.backend.empty(node.shape, node.dtype)
        self.backend._launch(source, "pacho_elementwise", grid, operands, out)
        return out

    def prepare_map_reduce(self, node, group, leaves):
        operation = node.attrs.get("operation", "sum")
        if node.dtype.kind == "b" and operation == "sum":
            operation = "max"  # a sum in bool is a logical or (HIPBackend.reduce)
        mapped = node.inputs[0]
        if prod(mapped.shape) > 2**31 - 1:
            raise ValueError("Array exceeds GPU indexing limits")
        specs, nodes = _graph(group, leaves)
        source, count, chunks = map_reduce_source(
            mapped.shape, tuple(node.attrs["axes"]), specs, nodes, operation, np.dtype(node.dtype)
        )
        return tuple(leaves), (source, count, chunks)

    def run_map_reduce(self, node, payload, arguments, operands):
        source, count, chunks = payload
        out = self.backend.empty((count, chunks), node.dtype)
        self.backend._launch(source, "pacho_map_reduce", count * chunks, operands, out)
        if chunks == 1:
            return out
        partial = ndarray._wrap(out, (count, chunks), node.dtype, self.backend)
        options = {"operation": node.attrs["operation"]} if "operation" in node.attrs else {}
        return self.backend.reduce(partial, (1,), False, node.dtype, **options)


def eager_source(name, args, shape, dtype):
    """Source of one eager elementwise operation (a one-node fused group)."""
    operands = tuple((bool(getattr(a, "_host_scalar", False)), np.dtype(a.dtype), tuple(a.shape)) for a in args)
    return _eager_source(name, operands, tuple(shape), np.dtype(dtype))


@lru_cache(maxsize=1024)
def _eager_source(name, operands, shape, dtype):
    # Keyed by what the source depends on (operation, operand kinds, dtypes
    # and shapes): repeated eager operations skip the code generation.
    leaves = [_Leaf(scalar, leaf_dtype, leaf_shape) for scalar, leaf_dtype, leaf_shape in operands]
    resolved = tuple(leaf_dtype for _, leaf_dtype, _ in operands)
    if name == "cast":
        resolved = (resolved[0],)
    nodes = [(name, list(range(len(operands))), resolved, dtype)]
    return elementwise_source(shape, leaves, nodes, dtype)
