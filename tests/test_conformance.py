"""NumPy conformance of the public API, run on the NumPy backend and on hip.

Restates the backend-parametrised contracts of the reference's
tests/test_arrays.py:38-341, tests/test_edge_cases.py:42-200,
tests/test_where.py:32-140 and tests/test_extrema.py:43-230, which the
reference runs on every backend it has. Here the same test body runs on the
NumPy backend (CPU tier) and on hip (``gpu`` marker); results must equal NumPy
bit for bit for integer, bool and selection work and within the reference's
tolerances for floating arithmetic. Launch bookkeeping follows this build's
backend (hipRTC launches through ``_launch``, library kernels through
``_call``), not the reference's ``_run``.
"""

import numpy as np
import pytest

import openpacho as p
from openpacho.backends import NumpyBackend
from openpacho.exceptions import BackendMismatchError, UnsupportedDtypeError


@pytest.fixture(params=["numpy", pytest.param("hip", marks=pytest.mark.gpu)])
def backend(request):
    if request.param == "numpy":
        return p.get_backend("numpy")
    return request.getfixturevalue("hip")


def _array(value, backend, dtype=None):
    return p.array(value, dtype=dtype, backend=backend)


def _same(actual, expected, *, rtol=1e-5, atol=1e-6):
    expected = np.asarray(expected)
    result = p.asnumpy(actual)
    assert result.shape == expected.shape
    assert result.dtype == expected.dtype, (result.dtype, expected.dtype)
    if expected.dtype.kind in "fc":
        np.testing.assert_allclose(result, expected, rtol=rtol, atol=atol, equal_nan=True)
    else:
        np.testing.assert_array_equal(result, expected)


def _exact(actual, expected, backend):
    expected = np.asarray(expected)
    assert p.get_backend(actual) is backend
    assert actual.shape == expected.shape and actual.dtype == expected.dtype, (actual.dtype, expected.dtype)
    np.testing.assert_array_equal(p.asnumpy(actual), expected)


# ---- arrays (reference tests/test_arrays.py) -----------------------------------------


def test_metadata_roundtrip_and_host_copy(backend):
    source = np.arange(6, dtype=np.float32).reshape(2, 3)
    array = _array(source, backend)
    source[...] = -1  # the upload is a snapshot
    assert (array.shape, array.dtype, array.ndim, array.size) == ((2, 3), np.float32, 2, 6)
    assert array.nbytes == 24 and array.backend == backend.name and array.device == backend.device
    expected = np.arange(6, dtype=np.float32).reshape(2, 3)
    downloaded = p.asnumpy(array)
    np.testing.assert_array_equal(downloaded, expected)
    downloaded[...] = 99  # the download is a copy
    np.testing.assert_array_equal(p.asnumpy(array), expected)


def test_constructors_match_numpy(backend):
    base = np.arange(6, dtype=np.float32).reshape(2, 3)
    for actual, expected in (
        (p.zeros((2, 3), dtype=np.float32, backend=backend), np.zeros((2, 3), np.float32)),
        (p.ones((2, 3), dtype=np.float32, backend=backend), np.ones((2, 3), np.float32)),
        (p.full((2, 3), -4, dtype=np.int32, backend=backend), np.full((2, 3), -4, np.int32)),
        (p.arange(-2, 6, 2, dtype=np.int32, backend=backend), np.arange(-2, 6, 2, dtype=np.int32)),
        (p.linspace(-1, 1, num=5, dtype=np.float32, backend=backend), np.linspace(-1, 1, 5, dtype=np.float32)),
        (p.eye(3, 4, k=-1, dtype=np.float32, backend=backend), np.eye(3, 4, k=-1, dtype=np.float32)),
        (p.zeros_like(_array(base, backend)), np.zeros_like(base)),
        (p.ones_like(_array(base, backend)), np.ones_like(base)),
    ):
        _same(actual, expected)
    empty = p.empty((2, 3), dtype=np.float32, backend=backend)
    assert empty.shape == (2, 3) and empty.dtype == np.float32 and empty.nbytes == 24


@pytest.mark.parametrize(
    "dtype,values",
    [
        (np.bool_, [False, True, True]),
        (np.int32, [-3, 0, 5]),
        (np.int64, [-3, 0, 5]),
        (np.uint32, [0, 3, 5]),
        (np.uint64, [0, 3, 5]),
        (np.float32, [-3.5, 0, 5.25]),
        (np.float64, [-3.5, 0, 5.25]),
    ],
)
def test_supported_dtype_roundtrip(backend, dtype, values):
    expected = np.asarray(values, dtype=dtype)
    _exact(_array(expected, backend), expected, backend)


def test_scalar_and_empty_shapes(backend):
    scalar = _array(np.asarray(3.5, dtype=np.float32), backend)
    assert (scalar.shape, scalar.ndim, scalar.size, scalar.nbytes) == ((), 0, 1, 4)
    assert scalar.item() == 3.5
    _same(scalar + 2, np.asarray(5.5, dtype=np.float32))
    host = np.empty((0, 3), dtype=np.float32)
    empty = _array(host, backend)
    assert (empty.shape, empty.size, empty.nbytes) == ((0, 3), 0, 0)
    _same(empty + 1, host)
    _same(empty * 2, host)
    _same(p.sum(empty), np.sum(host))
    mean = p.asnumpy(p.mean(empty))
    assert mean.shape == () and np.isnan(mean)


def test_elementwise_broadcasting_and_reverse_scalars(backend):
    host = np.asarray([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    bias = np.asarray([0.5, -1, 2], dtype=np.float32)
    a, b = _array(host, backend), _array(bias, backend)
    for actual, expected in (
        (a + b, host + bias),
        (a - b, host - bias),
        (a * b, host * bias),
        (a / (b + 3), host / (bias + 3)),
        (2 + a, 2 + host),
        (2 - a, 2 - host),
        (2 * a, 2 * host),
        (2 / a, 2 / host),
        (a**2.0, host**2.0),
    ):
        _same(actual, expected)
    weak = a + 0.5
    assert weak.dtype == np.float32
    _same(weak, host + 0.5)


def test_elementwise_ufuncs_comparisons_and_dispatch(backend):
    values = np.asarray([-2.0, -0.25, 0.5, 2.0], dtype=np.float32)
    positive = np.asarray([0.25, 1, 2, 4], dtype=np.float32)
    a, pos = _array(values, backend), _array(positive, backend)
    for name in ("sqrt", "exp", "log", "sin", "cos", "tanh", "abs"):
        domain = name in ("sqrt", "log")
        _same(getattr(p, name)(pos if domain else a), getattr(np, name)(positive if domain else values))
    for actual, expected in (
        (a > 0, values > 0),
        (a <= 0, values <= 0),
        (a == 0, values == 0),
        (p.isfinite(a), np.isfinite(values)),
        (np.isfinite(a), np.isfinite(values)),
    ):
        _exact(actual, expected, backend)


def test_division_preserves_nan_and_infinity(backend):
    numerator = np.asarray([1.0, 0.0, -1.0], dtype=np.float32)
    zeros = np.zeros(3, dtype=np.float32)
    actual = p.asnumpy(_array(numerator, backend) / _array(zeros, backend))
    assert np.isposinf(actual[0]) and np.isnan(actual[1]) and np.isneginf(actual[2])


def test_noncontiguous_upload_and_basic_slicing_are_copies(backend):
    source = np.arange(24, dtype=np.float32).reshape(4, 6)[:, ::2]
    array = _array(source, backend)
    np.testing.assert_array_equal(p.asnumpy(array), source)
    sliced = array[::-1, 1:5:2]
    _same(sliced, source[::-1, 1:5:2])
    downloaded = p.asnumpy(sliced)
    downloaded[...] = -100
    _same(sliced, source[::-1, 1:5:2])
    _same(array[None, :, 0], source[None, :, 0])
    with pytest.raises(TypeError):
        array[0, 0] = 1


def test_transpose_and_reshape_match_numpy(backend):
    source = np.arange(6, dtype=np.float32).reshape(2, 3)
    array = _array(source, backend)
    _exact(array.T, source.T, backend)
    _exact(array.transpose(1, 0), source.transpose(1, 0), backend)
    _exact(array.reshape(3, 2), source.reshape(3, 2), backend)
    _exact(p.reshape(array, (6,)), source.reshape(6), backend)


def test_reductions_for_large_arrays_and_axis_tuples(backend):
    source = (np.arange(17 * 19, dtype=np.float32).reshape(17, 19) - 100) / 7
    array = _array(source, backend)
    for axis, keepdims in ((None, False), (0, False), (1, True), ((0, 1), False), ((0, 1), True)):
        _same(p.sum(array, axis=axis, keepdims=keepdims), np.sum(source, axis=axis, keepdims=keepdims))
        _same(
            p.mean(array, axis=axis, keepdims=keepdims),
            np.mean(source, axis=axis, keepdims=keepdims),
            rtol=2e-5,
            atol=2e-6,
        )


@pytest.mark.parametrize("dtype", [np.int32, np.uint32])
def test_integer_reduction_default_dtypes(backend, dtype):
    source = np.arange(17 * 19, dtype=dtype).reshape(17, 19)
    _exact(p.sum(_array(source, backend), axis=0), np.sum(source, axis=0), backend)


def test_reduction_validation(backend):
    array = _array(np.arange(6, dtype=np.float32).reshape(2, 3), backend)
    with pytest.raises(ValueError):
        p.sum(array, axis=(0, 0))
    with pytest.raises(ValueError):
        p.sum(array, axis=2)
    with pytest.raises(NotImplementedError):
        p.sum(array, out=array)


@pytest.mark.parametrize(
    "left,right",
    [
        ((3,), (3,)),
        ((2, 3), (3, 4)),
        ((2, 3), (3,)),
        ((3,), (3, 4)),
    ],
)
def test_dot_and_matmul_rank_combinations(backend, left, right):
    a = np.arange(int(np.prod(left)), dtype=np.float32).reshape(left) + 1
    b = np.arange(int(np.prod(right)), dtype=np.float32).reshape(right) - 2
    _same(p.matmul(_array(a, backend), _array(b, backend)), np.matmul(a, b), rtol=2e-5, atol=2e-6)
    _same(p.dot(_array(a, backend), _array(b, backend)), np.dot(a, b), rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("left,right", [((0, 3), (3, 2)), ((2, 0), (0, 3)), ((0,), (0,)), ((2, 0), (0,))])
def test_zero_dimension_matmul(backend, left, right):
    a, b = np.zeros(left, np.float32), np.zeros(right, np.float32)
    _exact(p.matmul(_array(a, backend), _array(b, backend)), np.matmul(a, b), backend)


def test_matmul_validation(backend):
    left = _array(np.ones((2, 3), dtype=np.float32), backend)
    with pytest.raises(ValueError):
        p.matmul(left, _array(np.ones((2, 2), dtype=np.float32), backend))
    with pytest.raises(ValueError):
        p.matmul(_array(np.ones((1, 1, 1), dtype=np.float32), backend), left)


def test_diag_extracts_two_dimensional_matrix_diagonals(backend):
    source = np.arange(12, dtype=np.float32).reshape(3, 4)
    array = _array(source, backend)
    for k in (-2, -1, 0, 1, 3):
        _exact(p.diag(array, k=k), np.diag(source, k=k), backend)
    with pytest.raises(NotImplementedError):
        p.diag(_array(np.arange(3, dtype=np.float32), backend))


def test_implicit_host_conversion_and_unsupported_dispatch_are_explicit(backend):
    array = _array(np.arange(3, dtype=np.float32), backend)
    for attempt in (
        lambda: np.asarray(array),
        lambda: np.array(array),
        lambda: np.concatenate((array, array)),
        lambda: np.stack((array, array)),
        lambda: np.add(array, array, out=np.empty(3, dtype=np.float32)),
    ):
        with pytest.raises(TypeError):
            attempt()
    with pytest.raises(ValueError):
        bool(array)
    with pytest.raises(NotImplementedError):
        p.power(_array(np.asarray([1, 2, 3], dtype=np.int32), backend), 2)


def test_backend_mismatch_and_explicit_transfer(backend):
    other = NumpyBackend()
    source = np.arange(6, dtype=np.float32).reshape(2, 3)
    mine, theirs = _array(source, backend), _array(source, other)
    with pytest.raises(BackendMismatchError):
        mine + theirs
    moved = p.to_backend(theirs, backend)
    assert moved.backend == backend.name
    _exact(p.to_backend(moved, other) + 0, source, other)


# ---- promotion and boundaries (reference tests/test_edge_cases.py) ---------------------


def test_mixed_dtype_arithmetic_uses_numpy_promotion(backend):
    ints = np.asarray([-3, 2, 7], dtype=np.int32)
    doubles = np.asarray([0.5, -2.0, 1.25], dtype=np.float64)
    for left, right in ((ints, doubles), (doubles.astype(np.float32), doubles)):
        a, b = _array(left, backend), _array(right, backend)
        for actual, expected in ((a + b, left + right), (a - b, left - right), (a * b, left * right)):
            _same(actual, expected)


def test_integer_true_division_promotes_to_float64(backend):
    left = np.asarray([1, -3, 7], dtype=np.int32)
    right = np.asarray([2, 2, -4], dtype=np.int32)
    actual = _array(left, backend) / _array(right, backend)
    assert actual.dtype == np.float64
    _same(actual, np.true_divide(left, right))


def test_boolean_arithmetic_and_large_boolean_reduction(backend):
    values = np.ones(256, dtype=bool)
    array = _array(values, backend)
    _exact(array + array, values + values, backend)
    total = p.sum(array, dtype=bool)
    _exact(total, np.sum(values, dtype=bool), backend)
    assert total.item() is True


def test_astype_bool_matches_numpy_for_nan_and_signed_values(backend):
    values = np.asarray([0.0, 2.0, -1.0, np.nan, -0.0], dtype=np.float32)
    _exact(_array(values, backend).astype(bool), values.astype(bool), backend)


@pytest.mark.parametrize(
    "dtype,values",
    [
        (np.float16, [1.0]),
        (np.int8, [1]),
        (np.uint16, [1]),
        (np.complex64, [1 + 2j]),
        (object, [1]),
        (np.dtype([("value", np.float32)]), [(1.0,)]),
        (np.dtype(">f4"), [1.0, 2.0]),
    ],
)
def test_unsupported_dtypes_fail_explicitly(backend, dtype, values):
    with pytest.raises(UnsupportedDtypeError):
        _array(np.asarray(values, dtype=dtype), backend)


def test_numpy_ndarray_left_operand_dispatches_to_array_backend(backend):
    host = np.asarray([[4, 5, 6], [7, 8, 9]], dtype=np.float32)
    right = np.asarray([[1, 2, 3], [1, 2, 3]], dtype=np.float32)
    array = _array(right, backend)
    for actual, expected in (
        (host + array, host + right),
        (host - array, host - right),
        (host * array, host * right),
        (host / array, host / right),
        (np.add(host, array), np.add(host, right)),
    ):
        assert p.get_backend(actual) is backend
        _same(actual, expected)


def test_multiple_rank_broadcasting_and_incompatible_shapes(backend):
    left = np.arange(6, dtype=np.float32).reshape(2, 1, 3)
    right = np.arange(12, dtype=np.float32).reshape(4, 3)
    a, b = _array(left, backend), _array(right, backend)
    _same(a + b, left + right)
    _same(a * _array(np.asarray(2.0, dtype=np.float32), backend), left * np.float32(2))
    with pytest.raises(ValueError):
        a + _array(np.ones((2, 2), dtype=np.float32), backend)


@pytest.mark.parametrize(
    "key",
    [
        (Ellipsis, slice(None, None, -1)),
        (slice(None, None, -1), slice(None), slice(None, None, -2)),
        (slice(1, 1), slice(None), slice(None)),
        (slice(None), slice(2, 2, -1), slice(None)),
        (-1, -1, -1),
    ],
)
def test_negative_empty_and_integer_slices_match_numpy(backend, key):
    source = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
    _exact(_array(source, backend)[key], source[key], backend)


def test_scalar_reduction_axes_follow_numpy(backend):
    source = np.asarray(7, dtype=np.int32)
    array = _array(source, backend)
    for axis in (None, 0, -1, ()):
        _exact(p.sum(array, axis=axis), np.sum(source, axis=axis), backend)
    scalar = np.asarray(2.5, dtype=np.float32)
    scalar_array = _array(scalar, backend)
    for axis in (None, ()):
        _same(p.mean(scalar_array, axis=axis), np.mean(scalar, axis=axis))
    for axis in (0, -1):
        with pytest.raises(ValueError):
            p.mean(scalar_array, axis=axis)
    with pytest.raises(ValueError):
        p.sum(array, axis=(0,))


def test_negative_and_duplicate_reduction_axes(backend):
    source = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    array = _array(source, backend)
    for axis, keepdims in ((-1, False), ((-1, 0), False), ((0, -1), True), (-2, True)):
        _same(p.sum(array, axis=axis, keepdims=keepdims), np.sum(source, axis=axis, keepdims=keepdims))
    for axis in ((-1, 2), (0, -3)):
        with pytest.raises(ValueError):
            p.sum(array, axis=axis)


def test_numpy_norm_scalar_and_supported_3d_axes(backend):
    scalar = np.asarray(-3.5, dtype=np.float32)
    _same(np.linalg.norm(_array(scalar, backend)), np.linalg.norm(scalar))
    tensor = np.arange(24, dtype=np.float32).reshape(2, 3, 4) / 5
    array = _array(tensor, backend)
    _same(np.linalg.norm(array), np.linalg.norm(tensor), rtol=2e-5, atol=2e-6)
    _same(np.linalg.norm(array, axis=(1, 2)), np.linalg.norm(tensor, axis=(1, 2)), rtol=2e-5, atol=2e-6)
    with pytest.raises(ValueError):
        np.linalg.norm(array, axis=(0, 1, 2))


def test_use_backend_restores_nested_contexts_and_exceptions(backend):
    original = p.get_backend()
    numpy_backend = p.get_backend("numpy")
    with p.use_backend(numpy_backend) as selected:
        assert selected is numpy_backend and p.get_backend() is numpy_backend
        with p.use_backend(backend) as nested:
            assert nested is backend and p.get_backend() is backend
        assert p.get_backend() is numpy_backend
        with pytest.raises(RuntimeError), p.use_backend(backend):
            raise RuntimeError("restore context")
        assert p.get_backend() is numpy_backend
    assert p.get_backend() is original


# ---- selection (reference tests/test_where.py) ------------------------------------------


def test_where_three_way_broadcast_and_numpy_dispatch(backend):
    condition = np.array([[[True, False, True]], [[False, True, False]]])
    left = np.arange(4, dtype=np.float32).reshape(1, 4, 1)
    right = np.array([-2, -3, -4], dtype=np.float32)
    arrays = [_array(a, backend) for a in (condition, left, right)]
    for operation in (p.where, np.where, p.compile(np.where), p.fuse(np.where)):
        _exact(operation(*arrays), np.where(condition, left, right), backend)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_where_numeric_truth_preserves_nonfinites_and_zero_sign(backend, dtype):
    condition = np.array([0, -0.0, 0.5, np.nan, np.inf, -np.inf], dtype=dtype)
    left = np.array([np.nan, np.nan, np.nan, -0.0, np.inf, -np.inf], dtype=dtype)
    right = np.array([0, -0.0, 42, 13, np.nan, np.nan], dtype=dtype)
    args = [_array(a, backend) for a in (condition, left, right)]
    expected = np.where(condition, left, right)
    for operation in (p.where, p.compile(lambda c, x, y: np.where(c, x, y))):
        result = operation(*args)
        _exact(result, expected, backend)
        np.testing.assert_array_equal(np.signbit(p.asnumpy(result)[[0, 1, 3]]), [False, True, True])


@pytest.mark.parametrize("other", [1, 1.0, np.float64(1), "array"])
def test_where_branch_promotion_keeps_weak_and_strong_scalars(backend, other):
    condition = np.array([0, 0.5], dtype=np.float64)
    host = np.array([2, 3], dtype=np.float32)
    c, a = _array(condition, backend), _array(host, backend)
    if isinstance(other, str):
        other = np.array(1, dtype=np.float64)
        b = _array(other, backend)
    else:
        b = other
    expected = np.where(condition, host, other)
    _exact(p.where(c, a, b), expected, backend)
    _exact(p.compile(lambda c, a, b: p.where(c, a, b))(c, a, b), expected, backend)


def test_where_nested_selection_rebinds_boolean_and_numeric_scalars(backend):
    host = np.array([-3, -1, 0, 2, 4], dtype=np.float32)
    a = _array(host, backend)

    @p.compile
    def select(a, enabled, threshold, replacement):
        return np.where(enabled, np.where(a >= threshold, a, replacement), -a)

    prepared = select.prepare(a, True, 0.0, -1.0)
    for enabled, threshold, replacement in ((True, 0.0, -1.0), (False, 3.0, 7.0), (True, 3.0, 7.0)):
        expected = np.where(enabled, np.where(host >= threshold, host, replacement), -host)
        _exact(prepared(a, enabled, threshold, replacement), expected, backend)
    assert select.cache_info()["misses"] == 1


def test_where_empty_scalar_and_boolean_outputs(backend):
    select = p.compile(lambda c, x: np.where(c, x, False))
    for shape in ((), (0, 3), (2, 0, 3)):
        condition, host = np.ones(shape, dtype=bool), np.zeros(shape, dtype=bool)
        c, a = _array(condition, backend), _array(host, backend)
        expected = np.where(condition, host, False)
        _exact(p.where(c, a, False), expected, backend)
        _exact(select(c, a), expected, backend)


def test_where_large_integer_selection_is_exact(backend):
    left = np.array([2**62 + 1, -(2**62) + 3], dtype=np.int64)
    right = np.array([2**62 + 9, -(2**62) + 17], dtype=np.int64)
    c, a, b = [_array(v, backend) for v in (np.array([True, False]), left, right)]
    for operation in (p.where, p.compile(lambda c, a, b: p.where(c, a, b))):
        _exact(operation(c, a, b), np.where([True, False], left, right), backend)


def test_where_map_reduce_stays_resident_and_fuses(backend, monkeypatch):
    host = (np.arange(9003, dtype=np.float32) % 23 - 11).reshape(3, 3001)
    a = _array(host, backend)
    select = p.compile(lambda a, cut: np.sum(np.where(a > cut, a * a, 0.0), axis=1))
    if backend.name != "numpy":
        monkeypatch.setattr(backend, "upload", lambda *args: pytest.fail("unexpected upload"))
    with monkeypatch.context() as guarded:
        guarded.setattr(backend, "download", lambda *args: pytest.fail("unexpected download"))
        results = (select(a, 0.0), select(a, 4.0))
    for result, cut in zip(results, (0, 4)):
        _exact(result, np.sum(np.where(host > cut, host * host, 0.0), axis=1), backend)
    if backend.name != "numpy":
        assert [s["kind"] for s in select.explain(a, 0.0)["steps"]] == ["map_reduce"]


def test_where_errors_are_explicit_and_unselected_branch_is_validated(backend):
    a = p.ones(3, dtype=np.float32, backend=backend)
    with pytest.raises(NotImplementedError, match="nonzero|one.argument"):
        p.where(a)
    with pytest.raises(TypeError):
        p.where(a, 1)
    with pytest.raises(ValueError):
        p.where(a, np.ones(2), np.ones(3))
    with pytest.raises(UnsupportedDtypeError):
        p.where(True, a, 1j)
    other = p.asarray([1, 2, 3], backend=NumpyBackend())
    with pytest.raises(BackendMismatchError):
        p.where(True, a, other)
    with pytest.raises(BackendMismatchError):
        p.compile(lambda a, b: np.where(True, a, b))(a, other)


# ---- extrema (reference tests/test_extrema.py) ------------------------------------------


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_extrema_axes_and_numpy_dispatch(backend, dtype):
    host = (np.arange(30).reshape(2, 3, 5) - 16).astype(dtype)
    a = _array(host, backend)
    for axis, keepdims in ((None, False), (0, True), (-1, False), ((2, 0), True), ((), False)):
        calculate = p.compile(
            lambda x: (np.min(x, axis=axis, keepdims=keepdims), np.amax(x, axis=axis, keepdims=keepdims))
        )
        expected = [f(host, axis=axis, keepdims=keepdims) for f in (np.min, np.max)]
        eager = (a.min(axis=axis, keepdims=keepdims), a.max(axis=axis, keepdims=keepdims))
        for results in (eager, calculate(a)):
            for actual, reference in zip(results, expected):
                _exact(actual, reference, backend)
    assert p.min is p.amin and p.max is p.amax
    _exact(np.amin(a), np.min(host), backend)
    _exact(np.max(a), np.max(host), backend)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_extrema_nan_infinity_and_zero_ties_across_chunks(backend, dtype):
    host = np.zeros((5, 8193), dtype=dtype)
    host[0, :4096] = -0.0
    host[1] = -0.0
    host[3, 4097] = np.nan
    host[4, 0], host[4, -1] = -np.inf, np.inf
    a = _array(host, backend)
    calculate = p.compile(lambda x: (p.min(x, axis=1), p.max(x, axis=1)))
    expected = (
        np.array([-0.0, -0.0, +0.0, np.nan, -np.inf], dtype=dtype),
        np.array([+0.0, -0.0, +0.0, np.nan, +np.inf], dtype=dtype),
    )
    for results in ((p.min(a, axis=1), p.max(a, axis=1)), calculate(a)):
        for actual, reference in zip(results, expected):
            _exact(actual, reference, backend)
            np.testing.assert_array_equal(np.signbit(p.asnumpy(actual)[:3]), np.signbit(reference[:3]))
    zero = _array(np.array(-0.0, dtype=dtype), backend)
    for function in (p.min, p.max):
        assert np.signbit(function(zero, axis=()).item())


@pytest.mark.parametrize("dtype", [np.int32, np.int64, np.uint32, np.uint64])
def test_extrema_integer_limits_stay_exact(backend, dtype):
    info = np.iinfo(dtype)
    pattern = np.array([info.min, info.min + 1, info.max - 1, info.max], dtype=dtype)
    host = np.stack([np.resize(pattern, 4101), np.full(4101, info.max, dtype=dtype)])
    a = _array(host, backend)
    calculate = p.compile(lambda x: (p.min(x, axis=1), p.max(x, axis=1)))
    for results in ((p.min(a, axis=1), p.max(a, axis=1)), calculate(a)):
        for actual, function in zip(results, (np.min, np.max)):
            _exact(actual, function(host, axis=1), backend)
    mapped = p.compile(lambda x: p.max(p.where(x >= 0, x, x), axis=1))
    _exact(mapped(a), np.max(host, axis=1), backend)


def test_extrema_boolean_identities_and_compiled_cache(backend):
    host = np.zeros((3, 4097), dtype=np.bool_)
    host[0] = True
    host[1, -1] = True
    a = _array(host, backend)
    calculate_min = p.compile(lambda x: p.min(p.equal(x, True), axis=1))
    calculate_max = p.compile(lambda x: p.max(p.equal(x, True), axis=1))
    calculate_sum = p.compile(lambda x: p.sum(p.equal(x, True), axis=1, dtype=np.float32))
    for function, expected in ((p.min, np.min), (p.max, np.max)):
        _exact(function(a, axis=1), expected(host, axis=1), backend)
    for function, expected in ((calculate_min, np.min), (calculate_max, np.max), (calculate_min, np.min)):
        _exact(function(a), expected(host, axis=1), backend)
    _exact(calculate_sum(a), np.sum(host, axis=1, dtype=np.float32), backend)


def test_materialized_extrema_preserve_shared_public_and_transposed_inputs(backend):
    @p.compile
    def calculate(x, offset):
        shared = x + offset
        return shared, p.min(shared, axis=0), p.max(shared, axis=1), p.max(shared.T, axis=1)

    host = (np.arange(3 * 257, dtype=np.float32) % 29 - 14).reshape(3, 257)
    first = _array(host, backend)
    prepared = calculate.prepare(first, 0.5)
    for array, reference, offset in ((first, host, 0.5), (_array(-host, backend), -host, -1.5)):
        shared = reference + np.float32(offset)
        expected = shared, shared.min(axis=0), shared.max(axis=1), shared.T.max(axis=1)
        for actual, want in zip(prepared(array, offset), expected):
            _exact(actual, want, backend)
    if backend.name != "numpy":
        kinds = [step["kind"] for step in prepared.explain()["steps"]]
        assert kinds.count("map_reduce") == 3 and kinds.count("gather") == 1


@pytest.mark.parametrize("operation", ["min", "max"])
def test_extrema_map_reduce_rebinds_and_stays_resident(backend, monkeypatch, operation):
    function = getattr(p, operation)
    host = (np.arange(3 * 8193, dtype=np.float32) % 41 - 20).reshape(3, 8193)
    inputs = [_array(value, backend) for value in (host, host * 0.5)]
    calculate = p.compile(lambda x, cut: function(p.where(x > cut, x, -x), axis=1, keepdims=True))
    if backend.name != "numpy":
        monkeypatch.setattr(backend, "upload", lambda *args: pytest.fail("implicit upload"))
    prepared = calculate.prepare(inputs[0], 0.0)
    with monkeypatch.context() as guarded:
        guarded.setattr(backend, "download", lambda *args: pytest.fail("implicit download"))
        results = (prepared(inputs[0], 0.0), prepared(inputs[1], 4.0))
    for result, h, cut in zip(results, (host, host * 0.5), (0, 4)):
        _exact(result, getattr(np, operation)(np.where(h > cut, h, -h), axis=1, keepdims=True), backend)
    if backend.name != "numpy":
        steps = calculate.explain(inputs[0], 0.0)["steps"]
        assert [step["kind"] for step in steps] == ["map_reduce"]
        assert steps[0]["operation"] == operation


def test_extrema_empty_scalar_and_explicit_errors(backend):
    for function in (p.min, p.max):
        for shape, axis in (((0,), None), ((0, 0), 0), ((0, 3), 0), ((3, 0), 1)):
            a = p.empty(shape, dtype=np.float32, backend=backend)
            for apply in (lambda x: function(x, axis=axis), p.compile(lambda x: function(x, axis=axis))):
                with pytest.raises(ValueError, match="zero.size|empty"):
                    apply(a)
        for shape, axis, expected_shape in (((0, 3), 1, (0,)), ((3, 0), 0, (0,)), ((0,), (), (0,))):
            a = p.empty(shape, dtype=np.float32, backend=backend)
            for result in (function(a, axis=axis), p.compile(lambda x: function(x, axis=axis))(a)):
                _exact(result, np.empty(expected_shape, dtype=np.float32), backend)
        a = _array(np.array(-4.5, dtype=np.float32), backend)
        for axis in (None, 0, -1, ()):
            assert function(a, axis=axis).item() == -4.5
        for kwargs in ({"out": a}, {"initial": 0}, {"where": True}):
            with pytest.raises(NotImplementedError):
                function(a, **kwargs)
        for axis in ((0,), 1):
            with pytest.raises(ValueError):
                function(a, axis=axis)
        with pytest.raises(ValueError, match="duplicate"):
            function(p.ones((2, 3), backend=backend), axis=(0, 0))
        with pytest.raises(NotImplementedError, match="elementwise"):
            p.fuse(lambda x: function(x))(a)


def _softmax(x):
    shifted = x - p.max(x, axis=1, keepdims=True)
    weights = p.exp(shifted)
    return weights / p.sum(weights, axis=1, keepdims=True)


def _logsumexp(x):
    top = p.max(x, axis=1, keepdims=True)
    return top + p.log(p.sum(p.exp(x - top), axis=1, keepdims=True))


def test_stable_normalization(backend):
    host = np.array([[10000, 10001, 9999], [-10000, -10001, -9999]], dtype=np.float32)
    a = _array(host, backend)
    wide = host.astype(np.float64)
    shifted = wide - wide.max(axis=1, keepdims=True)
    want_softmax = np.exp(shifted) / np.exp(shifted).sum(axis=1, keepdims=True)
    want_lse = wide.max(axis=1, keepdims=True) + np.log(np.exp(shifted).sum(axis=1, keepdims=True))
    for calculate in (lambda x: (_softmax(x), _logsumexp(x)), p.compile(lambda x: (_softmax(x), _logsumexp(x)))):
        weights, logs = calculate(a)
        np.testing.assert_allclose(p.asnumpy(weights), want_softmax, rtol=2e-6, atol=0)
        np.testing.assert_allclose(p.asnumpy(logs), want_lse, rtol=0, atol=5e-4)
        np.testing.assert_allclose(p.asnumpy(weights).sum(axis=1), 1, rtol=2e-6)
        assert p.get_backend(weights) is backend and weights.dtype == np.float32
