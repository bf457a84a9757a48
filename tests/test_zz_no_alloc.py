"""GPU test of hp_norm_noalloc, the allocation-free variant of hp_norm.

Through the C ABI: each case runs hp_norm and hp_norm_noalloc on the same
input and requires identical bits, on two calls in a row where the second
input is smaller (the static workspace keeps the first call's contents). The
pool counters must not move across the allocation-free calls, and a shape
whose temporaries exceed the static workspace must fail before any launch.
"""

import ctypes
import math
import re
from pathlib import Path

import numpy as np
import pytest

import openpacho as p
from openpacho import _hip_lib

pytestmark = pytest.mark.gpu

HEADER = Path(__file__).resolve().parents[1] / "include" / "pacho_hip.h"
_DEFINE = re.search(r"#define HP_NORM_NOALLOC_SCRATCH_BYTES \((\d+) << (\d+)\)", HEADER.read_text())
SCRATCH_BYTES = int(_DEFINE.group(1)) << int(_DEFINE.group(2))

# (dtype, outer, reduced, inner): the first of each pair is the larger call.
CASES = [
    # one row over many chunks: running pairs + one merge pass
    (np.float32, [(1, (1 << 24) + 5, 1), (1, 70001, 1)]),
    (np.float64, [(1, (1 << 23) + 3, 1), (1, 9000, 1)]),
    # several rows of several chunks: pairs per (row, chunk), then merges;
    # 4097+ chunks per row take a second merge pass (both workspace halves)
    (np.float32, [(2, (1 << 24) + 4096 * 3, 1), (3, 40000, 1)]),
    (np.float64, [(3, 2048 * 4100, 1), (5, 2048 * 3 + 1, 1)]),
    # one chunk per row (no workspace), strided axis, empty reduced axis
    (np.float32, [(4096, 4096, 1), (17, 100, 1)]),
    (np.float32, [(64, 300, 129), (3, 7, 5)]),
    # strided axis, long: 512 chunks of pairs from the first pass, merged by
    # one narrow-block pass; the second call's plan differs in every extent
    (np.float32, [(1, 32768, 1024), (2, 20000, 640)]),
    (np.float64, [(5, 0, 3), (2, 0, 1)]),
]


def _pool(hip):
    stats = [ctypes.c_int64() for _ in range(4)]
    hip._call("hp_pool_stats", *[ctypes.byref(s) for s in stats])
    return tuple(s.value for s in stats)


def _norms(hip, entry, x, shape, dtype):
    outer, reduced, inner = shape
    out = p.empty((outer * inner,), dtype=dtype, backend=hip)
    code = _hip_lib.DTYPE_CODES[np.dtype(dtype)]
    hip._call(entry, code, *hip._ptrs(x, out), outer, reduced, inner)
    return out


@pytest.mark.parametrize("dtype,calls", CASES)
def test_noalloc_matches_hp_norm_on_two_calls(hip, dtype, calls):
    rng = np.random.default_rng(4242)
    inputs = []
    for outer, reduced, inner in calls:
        host = rng.uniform(-1, 1, outer * reduced * inner).astype(dtype)
        host[:: max(1, host.size // 7)] *= dtype(1e30) if dtype == np.float32 else 1e300
        inputs.append((host, p.asarray(host, backend=hip)))
    with hip._active():
        expected = [p.asnumpy(_norms(hip, "hp_norm", x, shape, dtype)) for (_, x), shape in zip(inputs, calls)]
        outputs = [p.empty((o * i,), dtype=dtype, backend=hip) for o, _, i in calls]
        hip.synchronize()
        before = _pool(hip)
        code = _hip_lib.DTYPE_CODES[np.dtype(dtype)]
        for (_, x), out, (outer, reduced, inner) in zip(inputs, outputs, calls):
            hip._call("hp_norm_noalloc", code, *hip._ptrs(x, out), outer, reduced, inner)
        hip.synchronize()
        assert _pool(hip) == before
    for (host, _), out, want, (outer, reduced, inner) in zip(inputs, outputs, expected, calls):
        got = p.asnumpy(out)
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
        if dtype == np.float32:
            scaled = host.reshape(outer, reduced, inner).astype(np.float64) / 1e30
            ref = np.sqrt(np.sum(np.square(scaled), axis=1)) * 1e30
            np.testing.assert_allclose(got, ref.ravel(), rtol=2e-6, atol=0)


def test_noalloc_workspace_boundary(hip):
    """Rows of 2049 doubles are two chunks of pairs: 32 bytes of workspace per
    row and no second merge buffer. SCRATCH_BYTES / 32 rows fill the static
    array exactly and run; one row more needs 256 bytes beyond it (the pair
    buffer is rounded up to 256 bytes) and is rejected on the host from the
    extents alone, before any launch and without touching the pool."""
    reduced = 2049
    rows = SCRATCH_BYTES // 32
    x = p.empty((rows * reduced,), dtype=np.float64, backend=hip)
    with hip._active():
        hip._call("hp_fill", ctypes.c_void_p(x._data.ptr), rows * reduced, 8, 0x3FF0000000000000)  # 1.0
        want = _norms(hip, "hp_norm", x, (rows, reduced, 1), np.float64)
        out = p.empty((rows,), dtype=np.float64, backend=hip)
        hip.synchronize()
        before = _pool(hip)
        hip._call("hp_norm_noalloc", 6, *hip._ptrs(x, out), rows, reduced, 1)
        hip.synchronize()
        assert _pool(hip) == before
        with pytest.raises(ValueError, match="static scratch"):
            hip._call("hp_norm_noalloc", 6, *hip._ptrs(x, out), rows + 1, reduced, 1)
        assert _pool(hip) == before
    got = p.asnumpy(out)
    np.testing.assert_array_equal(got.view(np.uint64), p.asnumpy(want).view(np.uint64))
    assert np.all(got == math.sqrt(reduced))


def test_noalloc_rejects_shapes_beyond_the_static_workspace(hip):
    # 3 rows x 2^19 chunks of 2048 doubles: 24 MiB of pairs. Rejected on the
    # host from the extents alone; the pointers are never dereferenced.
    assert 3 * (1 << 19) * 16 > SCRATCH_BYTES
    x = p.empty((8,), dtype=np.float64, backend=hip)
    out = p.empty((3,), dtype=np.float64, backend=hip)
    with hip._active():
        before = _pool(hip)
        with pytest.raises(ValueError, match="static scratch"):
            hip._call("hp_norm_noalloc", 6, *hip._ptrs(x, out), 3, 2048 << 19, 1)
        assert _pool(hip) == before
