"""The product's own CPU paths against the reference NumPy backend's outputs.

NumpyBackend.random_data (openpacho/_philox.py) and NumpyBackend.norm
(openpacho/_norm_host.py) are the package's CPU backend, separate from the
oracle under oracle/. Here they run through the public API (default_rng with
backend='numpy', linalg.norm) and are compared with the fixtures that the
reference NumPy backend wrote (tests/golden/make_golden.py): random and
uniform bit for bit, normal and exponential within the tolerance of reference
tests/test_random.py:75-80, norms bit for bit (the same NumPy operations in
the same order as reference _norm.py:44-52).
"""

from pathlib import Path

import numpy as np
import pytest

import openpacho as p

GOLDEN = Path(__file__).parent / "golden"
PARAMS = {"random": (0, 1), "uniform": (-3, 7), "normal": (2, 3), "exponential": (0, 2)}


def _load(name):
    with np.load(GOLDEN / name) as data:
        return {key: data[key] for key in data.files}


def _draw(rng, dist, size, dtype):
    first, second = PARAMS[dist]
    if dist == "random":
        return rng.random(size, dtype=dtype)
    if dist == "uniform":
        return rng.uniform(first, second, size, dtype=dtype)
    if dist == "normal":
        return rng.normal(first, second, size, dtype=dtype)
    return rng.exponential(second, size, dtype=dtype)


def test_numpy_backend_random_streams_match_reference_fixtures():
    golden = _load("reference_rng.npz")
    assert len(golden) == 72
    for key, expected in golden.items():
        dist, dtype, seed, start = key.split("|")
        rng = p.random.default_rng(int(seed), backend="numpy")
        rng._counter = int(start)
        got = p.asnumpy(_draw(rng, dist, expected.shape, dtype))
        assert got.dtype == expected.dtype, key
        if dist in ("random", "uniform"):
            np.testing.assert_array_equal(got.view(np.uint8), expected.view(np.uint8), err_msg=key)
        else:
            tol = 3e-6 if dtype == "float32" else 1e-13
            np.testing.assert_allclose(got, expected, rtol=tol, atol=tol, err_msg=key)
        assert rng._counter == int(start) + expected.size  # one counter per element


def test_numpy_backend_random_data_protocol_matches_fixtures():
    """The backend method itself, as the hip generator's callers invoke it."""
    golden = _load("reference_rng.npz")
    backend = p.get_backend("numpy")
    for key in ("uniform|float32|42|4294967293", "random|float64|18446744073709551615|18446744073709551609",
                "normal|float64|81985529216486895|0", "exponential|float32|42|4294967293"):
        dist, dtype, seed, start = key.split("|")
        expected = golden[key]
        first, second = PARAMS[dist]  # exponential: (0, scale), as Generator passes it
        got = backend.random_data(expected.shape, np.dtype(dtype), dist, int(seed), int(start), first, second)
        got = np.asarray(got).reshape(expected.shape)
        tol = 0 if dist in ("random", "uniform") else (3e-6 if dtype == "float32" else 1e-13)
        np.testing.assert_allclose(got, expected, rtol=tol, atol=tol, err_msg=key)


@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_numpy_backend_norm_matches_reference_fixtures(dtype):
    golden = _load("reference_norm.npz")
    x = golden[f"loguniform|{dtype}|input"]
    got = p.asnumpy(p.linalg.norm(p.asarray(x, backend="numpy")))
    np.testing.assert_array_equal(got, golden[f"loguniform|{dtype}|norm"])
    cube = p.asarray(golden[f"cube|{dtype}|input"], backend="numpy")
    for axis in ((2, 0), 1, None):
        key = "none" if axis is None else str(axis)
        got = p.asnumpy(p.linalg.norm(cube, axis=axis, keepdims=True))
        np.testing.assert_array_equal(got, golden[f"cube|{dtype}|axis={key}"], err_msg=key)
    rows = p.asarray(golden[f"rows|{dtype}|input"], backend="numpy")
    np.testing.assert_array_equal(p.asnumpy(p.linalg.norm(rows, axis=1)), golden[f"rows|{dtype}|norm"])
