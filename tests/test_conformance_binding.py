"""Compiled-call binding, residency and generator routing, on NumPy and on hip.

Contracts (reference tests/test_compiled_binding.py:19-156,
tests/test_residency.py:9-27, tests/test_random_routing.py:12-19):
1. a cache hit whose arguments are all positional builds its bindings without
   signature binding;
2. keyword and default arguments rebind the same plan; positional-only and
   keyword-only parameters keep Python's own binding errors; variadic
   parameters are refused;
3. static values, array shape, dtype and backend instance are the
   specialization key, nothing else;
4. a plan keeps no input array alive;
5. the execution scope is bound once, when the plan is built, from its launch
   count against the backend's threshold (never from a backend name);
6. NumPy dispatch of elementwise, reduction, transpose-product and slicing
   work on a device array downloads nothing;
7. a Generator on a backend instance that no name selects uses that
   instance's implementation.
Contracts 1, 2, 4 and 6 run on the NumPy backend (CPU tier) and on hip
(``gpu``); 3, 5 and 7 need several NumPy backend instances and run on CPU.
"""

from __future__ import annotations

import gc
import weakref
from contextlib import contextmanager

import numpy as np
import pytest

import openpacho as pacho
import openpacho._compiler as compiler_module
from openpacho.backends import NumpyBackend


@pytest.fixture(params=["numpy", pytest.param("hip", marks=pytest.mark.gpu)])
def backend(request):
    return pacho.get_backend("numpy") if request.param == "numpy" else request.getfixturevalue("hip")


@pytest.fixture
def bind_calls(monkeypatch):
    """Every signature binding the compiler performs, recorded."""
    calls = []
    real = compiler_module._bind

    def counted(*args, **kwargs):
        calls.append(args[0])
        return real(*args, **kwargs)

    monkeypatch.setattr(compiler_module, "_bind", counted)
    return calls


def _host(n=6, dtype=np.float32):
    return np.arange(n, dtype=dtype)


# ---- 1. positional hits bind nothing -----------------------------------------------


def test_positional_hits_skip_binding(backend, bind_calls):
    def scaled(a, factor):
        return a * factor - 2

    compiled = pacho.compile(scaled)
    x = pacho.asarray(_host(), backend=backend)
    for factor in (1.5, 2.5, 3.5):
        np.testing.assert_allclose(pacho.asnumpy(compiled(x, factor)), _host() * factor - 2)
    assert len(bind_calls) == 1  # the capture of the first call only
    np.testing.assert_allclose(pacho.asnumpy(compiled(x, factor=4.0)), _host() * 4 - 2)
    assert len(bind_calls) == 2  # a keyword call binds, and hits the same plan
    assert compiled.cache_info() == {"hits": 3, "misses": 1, "size": 1, "max_size": 32}


# ---- 2. signatures -------------------------------------------------------------------


def test_keywords_and_defaults_share_one_plan(backend):
    def shifted(a, shift=1.0):
        return a + shift

    compiled = pacho.compile(shifted)
    x = pacho.asarray(_host(4), backend=backend)
    for call, want in ((lambda: compiled(x), 1.0), (lambda: compiled(x, shift=5.0), 5.0), (lambda: compiled(x, 7.0), 7.0)):
        np.testing.assert_allclose(pacho.asnumpy(call()), _host(4) + want)
    info = compiled.cache_info()
    assert info["misses"] == 1 and info["hits"] == 2


def test_python_binding_rules_are_kept(backend):
    x = pacho.asarray(_host(3), backend=backend)

    def positional_only(a, k=2.0, /):
        return a * k

    def keyword_only(a, *, k=2.0):
        return a * k

    compiled = pacho.compile(positional_only)
    np.testing.assert_allclose(pacho.asnumpy(compiled(x, 4.0)), _host(3) * 4)
    with pytest.raises(TypeError, match="positional[- ]only"):
        compiled(x, k=4.0)
    compiled = pacho.compile(keyword_only)
    np.testing.assert_allclose(pacho.asnumpy(compiled(x, k=4.0)), _host(3) * 4)
    np.testing.assert_allclose(pacho.asnumpy(compiled(x)), _host(3) * 2)
    with pytest.raises(TypeError):
        compiled(x, 4.0)


@pytest.mark.parametrize("variadic", [lambda a, *more: a, lambda a, **options: a])
def test_variadic_parameters_are_refused(backend, variadic):
    with pytest.raises(TypeError, match="without \\*args or \\*\\*kwargs"):
        pacho.compile(variadic)(pacho.asarray(_host(2), backend=backend))


# ---- 3. the specialization key --------------------------------------------------------


def test_specialization_key_is_static_values_shape_dtype_and_backend():
    compiled = pacho.compile(lambda a, shape: np.reshape(a, shape), static_argnames="shape")
    home, other = NumpyBackend(), NumpyBackend()
    base = _host(12)
    calls = [
        (base, np.float32, home, (3, 4), "miss"),
        (base + 1, np.float32, home, (3, 4), "hit"),  # new values, same key
        (base, np.float32, home, (4, 3), "miss"),  # static value
        (base, np.float64, home, (3, 4), "miss"),  # dtype
        (base, np.float32, other, (3, 4), "miss"),  # backend instance
        (np.arange(24, dtype=np.float32), np.float32, home, (6, 4), "miss"),  # shape
        (base * 2, np.float32, other, (3, 4), "hit"),
    ]
    misses = hits = 0
    for values, dtype, owner, shape, outcome in calls:
        array = pacho.asarray(values, dtype=dtype, backend=owner)
        np.testing.assert_array_equal(pacho.asnumpy(compiled(array, shape)), values.astype(dtype).reshape(shape))
        misses += outcome == "miss"
        hits += outcome == "hit"
        info = compiled.cache_info()
        assert (info["misses"], info["hits"]) == (misses, hits)


# ---- 4. no retained inputs --------------------------------------------------------------


def test_plans_hold_no_reference_to_their_inputs(backend):
    compiled = pacho.compile(lambda a, b: a * b + a)
    left = pacho.asarray(_host(9), backend=backend)
    right = pacho.asarray(_host(9) - 4, backend=backend)
    watched = [weakref.ref(left), weakref.ref(right)]
    out = compiled(left, right)
    del left, right
    gc.collect()
    assert all(ref() is None for ref in watched)
    np.testing.assert_allclose(pacho.asnumpy(out), _host(9) * (_host(9) - 4) + _host(9))


# ---- 5. the execution scope --------------------------------------------------------------


def test_execution_scope_is_chosen_when_the_plan_is_built():
    backend = NumpyBackend()
    log = []

    @contextmanager
    def scope():
        log.append("in")
        yield
        log.append("out")

    backend.execution_scope = scope
    backend.execution_scope_min_steps = 2
    x = pacho.asarray(_host(5), backend=backend)
    short = pacho.compile(lambda a: a * 3)  # one launch: below the threshold
    short(x)
    assert next(iter(short._plans.values()))._execution_scope is None and log == []
    long = pacho.compile(lambda a: (a - 1) * 3)  # two launches on a backend without a lowerer
    np.testing.assert_array_equal(pacho.asnumpy(long(x)), (_host(5) - 1) * 3)
    assert log == ["in", "out"]
    backend.execution_scope_min_steps = 50  # read once: an existing plan keeps its scope
    long(x)
    assert log == ["in", "out"] * 2


# ---- 6. residency ---------------------------------------------------------------------------


def test_numpy_protocol_calls_stay_on_the_device(backend, monkeypatch):
    host = np.linspace(-2, 2, 20, dtype=np.float32).reshape(4, 5)
    a = pacho.asarray(host, backend=backend)

    def no_download(*args, **kwargs):
        raise AssertionError("host download")

    monkeypatch.setattr(backend, "download", no_download)
    results = {
        "elementwise and reduction": np.sqrt(np.sum((a + 1) ** 2, axis=0)),
        "transpose product": np.transpose(a) @ a,
        "slice": a[1:, ::-2],
    }
    monkeypatch.undo()
    assert {r.backend for r in results.values()} == {backend.name}
    np.testing.assert_allclose(pacho.asnumpy(results["elementwise and reduction"]), np.sqrt(np.sum((host + 1) ** 2, axis=0)), rtol=2e-6)
    np.testing.assert_allclose(pacho.asnumpy(results["transpose product"]), host.T @ host, rtol=2e-6, atol=1e-6)
    np.testing.assert_array_equal(pacho.asnumpy(results["slice"]), host[1:, ::-2])


# ---- 7. generator routing ---------------------------------------------------------------------


def test_generator_uses_an_unregistered_backend_instance():
    class SideBackend(NumpyBackend):
        name = "side-device"

    side = SideBackend()
    drawn = pacho.random.default_rng(1234, backend=side).exponential(2.0, size=(4, 3))
    assert pacho.get_backend(drawn) is side
    reference = pacho.random.default_rng(1234, backend="numpy").exponential(2.0, size=(4, 3))
    np.testing.assert_array_equal(pacho.asnumpy(drawn), pacho.asnumpy(reference))
