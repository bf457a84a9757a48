"""TEST INFRASTRUCTURE ONLY - closed-form GEMM padding plan metadata.

Restates reference src/openpacho/_padding.py:80-109 (eligibility, rounding
M and N up to 32 and K up to 16, batch prefixes kept) and :60-77 (explain:
scratch bytes of every padded private buffer, copy dispatches, dispatch count).
Pinned by the worked values of reference tests/test_padding_metadata.py:34-92
and by the BASELINE.json config (4097x3001x2049 -> 109,039,616 scratch bytes).
"""

from math import prod


def _up(value, multiple):
    return -(-value // multiple) * multiple


def plan(ashape, bshape, dtype="float32"):
    """Return the expected padded shapes and explain() numbers, or None."""
    ashape, bshape = tuple(ashape), tuple(bshape)
    if dtype != "float32" or len(ashape) < 2 or len(bshape) < 2:
        return None
    m, k, n = ashape[-2], ashape[-1], bshape[-1]
    batch = tuple(max(x, y) for x, y in zip((1,) * (len(bshape) - len(ashape)) + ashape[:-2], (1,) * (len(ashape) - len(bshape)) + bshape[:-2]))
    shape = batch + (m, n)
    if not prod(shape) or min(m, n) < 32 or k < 16:
        return None
    ap = ashape[:-2] + (_up(m, 32), _up(k, 16))
    bp = bshape[:-2] + (_up(k, 16), _up(n, 32))
    cp = shape[:-2] + (_up(m, 32), _up(n, 32))
    scratch = [prod(p) * 4 for o, p in ((ashape, ap), (bshape, bp)) if o != p]
    if cp != shape:
        scratch.append(prod(cp) * 4)
    return {
        "padded_input_shapes": (ap, bp),
        "padded_output_shape": cp,
        "output_shape": shape,
        "scratch_bytes": sum(scratch),
        "copy_dispatches": len(scratch),
        "dispatch_count": 1 + len(scratch),
    }
