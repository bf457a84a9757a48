"""Application clients of the hot path on the hip backend.

The reference ships two client families of this path:
a dense regression network trained by explicit SGD (reference
examples/dense_network.py:50-77: tanh layer, transposed products for the
gradients, row sums for bias gradients) and dense iterative solvers
(reference examples/solvers.py:23-60: compiled residual/norm/dot steps of CG).
These tests restate both clients with the public API and run them compiled on
hip, against the NumPy backend (CPU) and float64 closed forms. They check that
the compiled plans use the fused paths (layout_matmul for private transposes,
residual_matvec for b - A @ x) and that results match within tolerance.
"""

import numpy as np
import pytest

import openpacho as p
from openpacho.linalg import norm

pytestmark = pytest.mark.gpu


def _sgd_step(x, y, w1, b1, w2, b2, rate):
    hidden = np.tanh(x @ w1 + b1)
    prediction = hidden @ w2 + b2
    residual = prediction - y
    loss = (residual * residual).mean() / 2
    d2 = residual / (x.shape[0] * w2.shape[1])
    dw2 = hidden.T @ d2
    db2 = d2.sum(axis=0)
    d1 = (d2 @ w2.T) * (1 - hidden * hidden)
    dw1 = x.T @ d1
    db1 = d1.sum(axis=0)
    return loss, w1 - rate * dw1, b1 - rate * db1, w2 - rate * dw2, b2 - rate * db2


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_dense_network_sgd_step_compiled(hip, dtype):
    n, d, h, o = 257, 129, 65, 33
    rng = np.random.default_rng(50)
    host = [
        rng.uniform(-1, 1, (n, d)),
        rng.uniform(-1, 1, (n, o)),
        rng.normal(0, d**-0.5, (d, h)),
        np.zeros(h),
        rng.normal(0, h**-0.5, (h, o)),
        np.zeros(o),
    ]
    host = [v.astype(dtype) for v in host]
    step = p.compile(_sgd_step)
    gpu = [p.asarray(v, backend=hip) for v in host]
    kinds = [s["kind"] for s in step.explain(*gpu, 0.5)["steps"]]
    assert kinds.count("layout_matmul") == 3 and "gather" not in kinds
    cpu = [p.asarray(v, backend="numpy") for v in host]
    tol = 2e-5 if dtype == np.float32 else 1e-12
    losses = []
    for _ in range(3):
        got = step(*gpu, 0.5)
        want = _sgd_step(*cpu, 0.5)
        for g, w in zip(got, want):
            np.testing.assert_allclose(p.asnumpy(g), p.asnumpy(w), rtol=tol, atol=tol)
        losses.append(float(p.asnumpy(got[0])))
        gpu = [gpu[0], gpu[1], *got[1:]]
        cpu = [cpu[0], cpu[1], *want[1:]]
    assert losses[2] < losses[0]


@p.compile
def _residual_state(A, x, b):
    r = b - A @ x
    return r, norm(r)


@p.compile
def _cg_curvature(A, direction):
    q = A @ direction
    return q, p.dot(direction, q)


@p.compile
def _cg_update(x, r, direction, q, rr, curvature):
    alpha = rr / curvature
    x_new = x + alpha * direction
    r_new = r - alpha * q
    return x_new, r_new, p.dot(r_new, r_new)


@p.compile
def _cg_direction(r, direction, rr_new, rr):
    return r + (rr_new / rr) * direction


def _conjugate_gradient(A, b, tolerance, max_iterations):
    # Only the scalar r.r crosses to the host, once per iteration (the
    # convergence diagnostic of the reference solvers).
    x = p.zeros(b.shape, dtype=b.dtype, backend=b._backend)
    r, _ = _residual_state(A, x, b)
    direction = r
    rr = p.dot(r, r)
    target = (tolerance * float(p.asnumpy(norm(b)))) ** 2
    for iteration in range(max_iterations):
        if float(p.asnumpy(rr)) <= target:
            return x, iteration
        q, curvature = _cg_curvature(A, direction)
        x, r, rr_new = _cg_update(x, r, direction, q, rr, curvature)
        direction = _cg_direction(r, direction, rr_new, rr)
        rr = rr_new
    return x, max_iterations


@pytest.mark.parametrize("dtype,tolerance", [(np.float64, 1e-10), (np.float32, 1e-5)])
def test_conjugate_gradient_on_resident_operands(hip, dtype, tolerance):
    n = 300
    rng = np.random.default_rng(60)
    m = rng.uniform(-1, 1, (n, n))
    host_a = (m.T @ m / n + np.eye(n)).astype(dtype)  # SPD, condition number ~ 5
    host_b = rng.uniform(-1, 1, n).astype(dtype)
    A, b = p.asarray(host_a, backend=hip), p.asarray(host_b, backend=hip)
    kinds = [s["kind"] for s in _residual_state.explain(A, b, b)["steps"]]
    assert kinds[0] == "residual_matvec"
    x, iterations = _conjugate_gradient(A, b, tolerance / 10, 100)
    assert iterations < 100
    r, r_norm = _residual_state(A, x, b)
    exact = np.linalg.solve(host_a.astype(np.float64), host_b.astype(np.float64))
    relative = float(p.asnumpy(r_norm)) / np.linalg.norm(host_b)
    assert relative < tolerance
    np.testing.assert_allclose(p.asnumpy(x), exact, rtol=50 * tolerance, atol=50 * tolerance)
    true_residual = host_b.astype(np.float64) - host_a.astype(np.float64) @ p.asnumpy(x).astype(np.float64)
    assert np.linalg.norm(true_residual) / np.linalg.norm(host_b) < 10 * tolerance


def test_solver_downloads_only_scalar_diagnostics(hip, monkeypatch):
    # Reference tests/test_residency.py:30-46: during the solve only the
    # one-element convergence diagnostics cross to the host.
    A = p.asarray([[4.0, 1.0], [1.0, 3.0]], dtype=p.float32, backend=hip)
    b = p.asarray([1.0, 2.0], dtype=p.float32, backend=hip)
    original = hip.download
    sizes = []

    def track_download(a):
        sizes.append(a.size)
        assert a.size == 1, "Solver transferred a vector or matrix during iteration"
        return original(a)

    with monkeypatch.context() as patch:
        patch.setattr(hip, "download", track_download)
        x, iterations = _conjugate_gradient(A, b, 1e-6, 50)
    assert sizes and iterations < 50
    np.testing.assert_allclose(p.asnumpy(x), [1 / 11, 7 / 11], rtol=1e-5)
