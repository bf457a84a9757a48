"""GPU parity of BASELINE config 5's compiled dense network at its full size.

The workload of reference examples/dense_network.py:39-77 as a compiled plan
(grouping of reference _compiler.py:177-205): X (8192, 4096) U[-1, 1), layer
widths 4096 -> 4096 -> 4096 -> 1024 with weights N(0, 1/fan_in) and zero
biases, every value drawn on the device by default_rng(42, backend='hip'), then
tanh(h @ w + b) per layer and a row-wise mean.

Checked here:
- the plan's step kinds equal the reference compiler's golden list;
- each layer's product (the same hp_gemm launch the plan's matmul step makes)
  has every output within the elementwise float32 error bound of a K-term
  sum against float64, repeats bit for bit, and is within 2x the reference
  custom kernel's error (sequential K, separate rounding) against the exact
  dyadic oracle on sampled outputs;
- the compiled plan's output rows are within 2x the error of the reference
  kernel chain (sequential-K products, float32 tanh, the reference reduce
  order for the mean) against a float64 recomputation from the same weights.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import openpacho as p
from oracle import exact, kernels

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_plans.json"
WIDTHS = (4096, 4096, 4096, 1024)
BATCH = 8192


def _sampled_layer_errors(inputs, weights, product, samples, seed):
    """RMS relative error of hip and of the sequential-K order, exact oracle."""
    rng = np.random.default_rng(seed)
    rows = rng.integers(0, inputs.shape[0], samples)
    cols = rng.integers(0, weights.shape[1], samples)
    reference = kernels.gemm_sequential(inputs, weights, rows, cols)
    hip_err, ref_err = [], []
    for i, (r, c) in enumerate(zip(rows, cols)):
        truth = exact.exact_dot(inputs[r, :], weights[:, c])
        scale = float(exact.exact_dot(np.abs(inputs[r, :]), np.abs(weights[:, c])))
        hip_err.append(abs(float(product[r, c]) - float(truth)) / scale)
        ref_err.append(abs(float(reference[i]) - float(truth)) / scale)
    return float(np.sqrt(np.mean(np.square(hip_err)))), float(np.sqrt(np.mean(np.square(ref_err))))


def _reference_chain_means(x_rows, weights, biases):
    """Row means of the reference CUDA chain, restated on the host in float32."""
    h = x_rows
    for w, b in zip(weights, biases):
        h = np.tanh(kernels.gemm_sequential_rows(h, w) + b).astype(np.float32)
    count = np.float32(h.shape[1])
    return np.array([kernels.reduce_lanes(row) for row in h], dtype=np.float32) / count


def test_config5_compiled_mlp_full_size(hip):
    rng = p.random.default_rng(42, backend=hip)
    params = []
    for fan_in, fan_out in zip(WIDTHS[:-1], WIDTHS[1:]):
        params.append(rng.normal(0, (1 / fan_in) ** 0.5, (fan_in, fan_out), dtype="float32"))
        params.append(p.zeros(fan_out, dtype=np.float32, backend=hip))
    x = rng.uniform(-1, 1, (BATCH, WIDTHS[0]), dtype="float32")

    @p.compile
    def mlp(x, w1, b1, w2, b2, w3, b3):
        h = p.tanh(x @ w1 + b1)
        h = p.tanh(h @ w2 + b2)
        out = p.tanh(h @ w3 + b3)
        return p.mean(out, axis=1)

    golden = [step["kind"] for step in json.loads(GOLDEN.read_text())["mlp"]]
    assert [s["kind"] for s in mlp.explain(x, *params)["steps"]] == golden
    got = p.asnumpy(mlp(x, *params))
    assert got.shape == (BATCH,) and got.dtype == np.float32
    assert np.all(np.isfinite(got))

    weights = [p.asnumpy(w) for w in params[0::2]]
    biases = [p.asnumpy(b) for b in params[1::2]]
    assert all(not b.any() for b in biases)
    for w, fan_in in zip(weights, WIDTHS[:-1]):  # N(0, 1/fan_in) was drawn
        assert abs(float(w.std()) * fan_in**0.5 - 1) < 0.01

    # Each layer's product, from the layer input the device computed.
    layer_input = x
    for index, (w_dev, b_dev) in enumerate(zip(params[0::2], params[1::2])):
        product = layer_input @ w_dev
        host_in, host_product = p.asnumpy(layer_input), p.asnumpy(product)
        # Every output of the layer's whole-tile product, and a bitwise repeat.
        assert exact.product_bound_ratio(host_in, weights[index], host_product, 4e-7) <= 1, f"layer {index}"
        np.testing.assert_array_equal(p.asnumpy(layer_input @ w_dev), host_product)
        hip_err, ref_err = _sampled_layer_errors(host_in, weights[index], host_product, 24, 50 + index)
        assert hip_err <= 2 * ref_err, f"layer {index}: {hip_err} > 2 x {ref_err}"
        layer_input = p.tanh(product + b_dev)
    eager = p.asnumpy(p.mean(layer_input, axis=1))
    np.testing.assert_allclose(eager, got, rtol=0, atol=2e-6)

    # The compiled output against float64, beside the reference chain's error.
    rows = np.random.default_rng(5).choice(BATCH, 64, replace=False)
    x_rows = p.asnumpy(x)[rows]
    h64 = x_rows.astype(np.float64)
    for w, b in zip(weights, biases):
        h64 = np.tanh(h64 @ w.astype(np.float64) + b.astype(np.float64))
    truth = h64.mean(axis=1)
    reference = _reference_chain_means(x_rows, weights, biases)
    hip_err = float(np.sqrt(np.mean(np.square(got[rows] - truth))))
    ref_err = float(np.sqrt(np.mean(np.square(reference - truth))))
    assert hip_err <= 2 * ref_err, f"{hip_err} > 2 x {ref_err}"
    assert np.max(np.abs(got[rows] - truth)) < 1e-5
