"""Compiled products of private transposes on hip (``layout_matmul`` steps).

Restates the remaining contracts of the reference's
tests/test_compiled_layout.py:128-184 on the hip provider:
- a failing provider call propagates, with no materialized-transpose
  fallback (forced from the host with hp_debug_fail_next, so no kernel
  misbehaves);
- one private transpose used as both operands is read in place twice;
- a dtype conversion keeps its gather and cast steps;
- an eager transpose still materializes independent storage.
"""

import numpy as np
import pytest

import openpacho as p

pytestmark = pytest.mark.gpu


def _count_gathers(hip, monkeypatch):
    calls = []
    original = hip.gather
    monkeypatch.setattr(hip, "gather", lambda *args: (calls.append(1), original(*args))[1])
    return calls


def test_provider_error_propagates_without_materialized_fallback(hip, monkeypatch):
    a = p.asarray(np.ones((7, 5), dtype=np.float32), backend=hip)
    prepared = p.compile(lambda a: a.T @ a).prepare(a)
    gathers = _count_gathers(hip, monkeypatch)
    hip._lib.hp_debug_fail_next(hip._ctx, 1)
    with pytest.raises(RuntimeError, match="injected"):
        prepared(a)
    assert not gathers
    np.testing.assert_array_equal(p.asnumpy(prepared(a)), np.full((5, 5), 7, np.float32))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_one_private_transpose_used_by_both_operands(hip, monkeypatch, dtype):
    host = (np.arange(25, dtype=dtype).reshape(5, 5) - 12) / 8
    a = p.asarray(host, backend=hip)

    def source(a):
        t = a.T
        return t @ t

    compiled = p.compile(source)
    assert [s["kind"] for s in compiled.explain(a)["steps"]] == ["layout_matmul"]
    gathers = _count_gathers(hip, monkeypatch)
    np.testing.assert_array_equal(p.asnumpy(compiled(a)), host.T @ host.T)  # dyadic values: exact
    assert not gathers


def test_mixed_dtype_keeps_the_required_conversion(hip):
    left = np.arange(35, dtype=np.float32).reshape(7, 5)
    right = np.arange(63, dtype=np.float64).reshape(7, 9)
    a, b = p.asarray(left, backend=hip), p.asarray(right, backend=hip)
    compiled = p.compile(lambda a, b: a.T @ b)
    result = compiled(a, b)
    assert result.dtype == np.float64
    np.testing.assert_array_equal(p.asnumpy(result), left.T.astype(np.float64) @ right)
    # The conversion stays (on a backend with a lowering, as a fused group)
    # and the product is not turned into a layout step.
    assert [s["kind"] for s in compiled.explain(a, b)["steps"]] == ["gather", "fused", "matmul"]


def test_eager_transpose_materializes_independent_storage(hip, monkeypatch):
    a = p.asarray(np.arange(35, dtype=np.float32).reshape(7, 5), backend=hip)
    gathers = _count_gathers(hip, monkeypatch)
    t = a.T
    assert len(gathers) == 1 and t._data.ptr != a._data.ptr
    np.testing.assert_array_equal(p.asnumpy(t), np.arange(35, dtype=np.float32).reshape(7, 5).T)
