"""TEST INFRASTRUCTURE ONLY - the reference CUDA custom kernels' arithmetic order.

These restatements reproduce, operation by operation, the rounding sequence of
the reference's custom CUDA kernels (compiled with --fmad=false: every product
and every sum rounds separately; reference _cuda.py:321-328). Their error
against an exact oracle is the "reference custom-kernel error" that the
north-star bar scales (hip error <= 2x this).

- gemm_sequential: _gemm.py:67-77 (fp32 register tile: K ascending, c += a*b)
  and _cuda.py:619-636 (direct fp64 kernel: same order in binary64).
  gemm_sequential_rows is the same order for whole rows of the product.
- gemv_lanes:      _cuda_gemv.py:35-43 (lane l sums j = l (mod 128) in order,
  then shared tree 64 -> 1), with DOT chunks of 1024 for 1-D K > 4096
  (:67-84) reduced by reduce_lanes.
- reduce_lanes:    _cuda.py:449-491 (4096-term chunks, 128-lane strided
  sequential accumulation, tree 64 -> 1, recursive on partials).
- norm_pair_merge: _norm.py:28-36 and :62-118 ((scale, ssq) merge per lane,
  tree over 128 lanes, 4096-term chunks, multi-pass, final s*sqrt(t)).

Pinned by tests/test_oracle_kernels.py: exact closed forms (sums of exactly
representable terms), agreement with np.sum-free brute-force loops on tiny
inputs, the reference's special-value table for norms, and error bounds.
"""

import numpy as np

LANES = 128


def gemm_sequential(a, b, rows, cols):
    """C[rows[i], cols[i]] of the fp32/fp64 sequential-K kernel, vectorised over samples."""
    a, b = np.asarray(a), np.asarray(b)
    dt = np.result_type(a.dtype, b.dtype)
    rows, cols = np.asarray(rows), np.asarray(cols)
    acc = np.zeros(rows.shape, dtype=dt)
    with np.errstate(all="ignore"):
        for k in range(a.shape[1]):
            product = np.multiply(a[rows, k], b[k, cols], dtype=dt)
            acc = np.add(acc, product, dtype=dt)
    return acc


def gemm_sequential_rows(a_rows, b):
    """a_rows @ b (2-D) in the sequential-K order, every row of the block.

    The same rounding sequence as gemm_sequential (c += a[:, k] * b[k, :],
    k ascending, product and sum rounded separately), vectorised over a row
    block instead of over sampled coordinates.
    """
    a_rows, b = np.asarray(a_rows), np.asarray(b)
    dt = np.result_type(a_rows.dtype, b.dtype)
    acc = np.zeros((a_rows.shape[0], b.shape[1]), dtype=dt)
    with np.errstate(all="ignore"):
        for k in range(a_rows.shape[1]):
            acc += np.multiply(a_rows[:, k, None], b[k, None, :], dtype=dt)
    return acc


def _tree(values):
    """Shared-memory tree over the last axis of length 128: sums[l] += sums[l+step]."""
    values = values.copy()
    step = LANES // 2
    while step:
        values[..., :step] = values[..., :step] + values[..., step : 2 * step]
        step //= 2
    return values[..., 0]


def _lane_sums(terms):
    """Lane-strided sequential sums: terms (..., n) -> (..., 128)."""
    n = terms.shape[-1]
    padded = -(-n // LANES) * LANES
    grid = np.zeros(terms.shape[:-1] + (padded,), terms.dtype)
    grid[..., :n] = terms
    grid = grid.reshape(terms.shape[:-1] + (padded // LANES, LANES))
    acc = np.zeros(terms.shape[:-1] + (LANES,), terms.dtype)
    for step in range(grid.shape[-2]):
        acc = acc + grid[..., step, :]
    return acc


def reduce_lanes(values):
    """Sum of a 1-D array with the reference reduce kernel's order."""
    values = np.asarray(values)
    while True:
        n = values.shape[0]
        chunks = -(-n // 4096)
        partial = np.empty(chunks, values.dtype)
        for c in range(chunks):
            partial[c] = _tree(_lane_sums(values[c * 4096 : (c + 1) * 4096]))
        if chunks == 1:
            return partial[0]
        values = partial


def gemv_lanes(a, x):
    """A @ x (A 2-D) or x . y (A 1-D) in the reference cooperative kernel's order."""
    a, x = np.asarray(a), np.asarray(x)
    dt = np.result_type(a.dtype, x.dtype)
    with np.errstate(all="ignore"):
        if a.ndim == 1 and a.shape[0] > 4096:
            n = a.shape[0]
            chunks = -(-n // 1024)
            partial = np.empty(chunks, dt)
            for c in range(chunks):
                seg = slice(c * 1024, min((c + 1) * 1024, n))
                partial[c] = _tree(_lane_sums(np.multiply(a[seg], x[seg], dtype=dt)))
            return reduce_lanes(partial)
        terms = np.multiply(a, x, dtype=dt)
        return _tree(_lane_sums(terms))


def _merge(s, t, v, w):
    """Vectorised _norm.py:28-36 merge of (v, w) into (s, t)."""
    s, t = s.copy(), t.copy()
    with np.errstate(all="ignore"):
        nan = np.isnan(s) | np.isnan(v)
        inf_v = ~nan & np.isinf(v)
        grow = ~nan & ~inf_v & ~np.isinf(s) & (v > 0)
        up = grow & (s < v)
        same = grow & ~(s < v)
        z_up = np.where(up, s / np.where(up, v, 1), 0)
        z_same = np.where(same, v / np.where(same, s, 1), 0)
        nan_s = s + v
        t = np.where(nan, nan_s, t)
        s = np.where(nan, nan_s, s)
        s = np.where(inf_v, v, s)
        t = np.where(inf_v, np.ones_like(t), t)
        t = np.where(up, w + (t * z_up) * z_up, t)
        s = np.where(up, v, s)
        t = np.where(same, t + (w * z_same) * z_same, t)
    return s, t


def norm_pair_state(x):
    """The (scale, ssq) pair the reference GPU kernel's last pass merges to.

    Vectorised across the 4096-term chunks of a pass: lanes past the end of a
    chunk hold zeros, which the merge treats as absent terms (v > 0 fails).
    """
    x = np.asarray(x)
    dt = x.dtype
    if x.shape[0] == 0:
        return dt.type(0), dt.type(0)
    values, weights = np.abs(x), np.ones_like(x)
    while True:
        n = values.shape[0]
        chunks = -(-n // 4096)
        grid_v = np.zeros(chunks * 4096, dt)
        grid_w = np.zeros(chunks * 4096, dt)
        grid_v[:n], grid_w[:n] = values, weights
        grid_v = grid_v.reshape(chunks, 4096 // LANES, LANES)
        grid_w = grid_w.reshape(chunks, 4096 // LANES, LANES)
        s = np.zeros((chunks, LANES), dt)
        t = np.zeros((chunks, LANES), dt)
        for step in range(grid_v.shape[1]):
            s, t = _merge(s, t, grid_v[:, step], grid_w[:, step])
        half = LANES // 2
        while half:
            s_lo, t_lo = _merge(s[:, :half], t[:, :half], s[:, half : 2 * half], t[:, half : 2 * half])
            s[:, :half], t[:, :half] = s_lo, t_lo
            half //= 2
        if chunks == 1:
            return s[0, 0], t[0, 0]
        values, weights = s[:, 0].copy(), t[:, 0].copy()


def norm_pair_merge(x):
    """Norm of a 1-D float array following the reference GPU kernel's passes:
    s * sqrt(t) of norm_pair_state (0 for an empty array)."""
    x = np.asarray(x)
    dt = x.dtype
    if x.shape[0] == 0:
        return dt.type(0)
    s, t = norm_pair_state(x)
    with np.errstate(all="ignore"):
        return dt.type(s * np.sqrt(t))
