"""Write golden vectors from the reference's NumPy backend (run in the build container).

Usage: python tests/golden/make_golden.py [/root/reference]

The reference is imported only here, in a separate process, and only for the
functions that no published vector or closed form pins:
- the float transforms of the Philox stream (random/uniform/normal/exponential,
  float32/float64) at several seeds and counter offsets, incl. carry and the
  end of the 2^64 counter space (reference _random.py:34-58);
- the NumPy two-pass norm on crafted vectors (reference _norm.py:44-52);
- the step kinds that ExecutionPlan.explain() reports for representative
  functions under a recording GPU-style lowering (reference _compiler.py:87-238).
Outputs (data only): reference_rng.npz, reference_norm.npz, reference_plans.json.
"""

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REFERENCE = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
sys.path.insert(0, str(REFERENCE / "src"))

import openpacho as ref  # noqa: E402  (the reference package)
from openpacho.backends import NumpyBackend  # noqa: E402

PARAMS = {
    "random": {},
    "uniform": {"low": -3, "high": 7},
    "normal": {"loc": 2, "scale": 3},
    "exponential": {"scale": 2},
}
SEEDS = (42, 2**64 - 1, 0x0123456789ABCDEF)
STARTS = ((0, 512), (2**32 - 3, 512), (2**64 - 7, 7))


def rng_vectors():
    out = {}
    for dtype in ("float32", "float64"):
        for dist, kwargs in PARAMS.items():
            for seed in SEEDS:
                for start, count in STARTS:
                    gen = ref.random.default_rng(seed, backend="numpy")
                    gen._counter = start
                    values = getattr(gen, dist)(size=count, dtype=dtype, **kwargs)
                    out[f"{dist}|{dtype}|{seed}|{start}"] = ref.asnumpy(values)
    return out


def norm_vectors():
    rng = np.random.default_rng(2)
    out = {}
    for dtype, decades in (("float32", 30), ("float64", 300)):
        mags = 10.0 ** rng.uniform(-decades, decades, 4099)
        signs = rng.integers(0, 2, 4099) * 2 - 1
        x = (mags * signs).astype(dtype)
        out[f"loguniform|{dtype}|input"] = x
        out[f"loguniform|{dtype}|norm"] = ref.asnumpy(ref.linalg.norm(ref.asarray(x, backend="numpy")))
        m = rng.uniform(-1, 1, (3, 5, 7)).astype(dtype)
        out[f"cube|{dtype}|input"] = m
        for axis in ((2, 0), 1, None):
            key = "none" if axis is None else str(axis)
            value = ref.linalg.norm(ref.asarray(m, backend="numpy"), axis=axis, keepdims=True)
            out[f"cube|{dtype}|axis={key}"] = ref.asnumpy(value)
        rows = rng.uniform(-1, 1, (8, 1024)).astype(dtype)
        out[f"rows|{dtype}|input"] = rows
        out[f"rows|{dtype}|norm"] = ref.asnumpy(ref.linalg.norm(ref.asarray(rows, backend="numpy"), axis=1))
    return out


class _RecordingLowering:
    """Grouping-only lowerer: mirrors what a GPU backend's lowering reports."""

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


def plan_vectors():
    backend = _GroupingBackend()
    f32 = np.float32

    def arr(*shape):
        return ref.asarray(np.ones(shape, f32), backend=backend)

    cases = {}

    def mlp(x, w1, b1, w2, b2, w3, b3):
        h = ref.tanh(x @ w1 + b1)
        h = ref.tanh(h @ w2 + b2)
        out = ref.tanh(h @ w3 + b3)
        return ref.mean(out, axis=1)

    cases["mlp"] = (mlp, (arr(8, 16), arr(16, 16), arr(16), arr(16, 16), arr(16), arr(16, 4), arr(4)))

    def affine(value, scale):
        shifted = value * scale
        return shifted, shifted + 1.0

    cases["affine"] = (affine, (arr(3, 4), 2.0))

    def products(a, b):
        product = ref.matmul(a, b)
        return product, ref.sum(product), ref.mean(product)

    cases["product_reductions"] = (products, (arr(33, 17), arr(17, 65)))
    cases["norm_rows"] = (lambda a: ref.linalg.norm(a, axis=1, keepdims=True), (arr(6, 4097),))
    cases["sum_of_squares_shift"] = (lambda x: ((x + 1) * (x - 2)).sum(), (arr(8),))
    cases["extrema"] = (lambda x: (ref.max(x, axis=0), ref.min(x * 2, axis=1)), (arr(5, 6),))
    results = {}
    for name, (fn, args) in cases.items():
        explanation = ref.compile(fn).explain(*args)
        results[name] = [
            {k: (list(v) if isinstance(v, tuple) else v) for k, v in step.items() if k != "padding"}
            for step in explanation["steps"]
        ]
    return results


def main():
    np.savez_compressed(HERE / "reference_rng.npz", **rng_vectors())
    np.savez_compressed(HERE / "reference_norm.npz", **norm_vectors())
    (HERE / "reference_plans.json").write_text(json.dumps(plan_vectors(), indent=1, sort_keys=True) + "\n")
    print("wrote", *(p.name for p in sorted(HERE.glob("reference_*"))))


if __name__ == "__main__":
    main()
