"""The hip backend's opt-in padding plan for fp32 GEMM (``matmul(padding=True)``).

Eligibility and rounding follow the reference (_padding.py:80-109): float32
operands with at least 32 output rows and columns and K >= 16 form a plan
whose padded problem rounds M and N up to 32 and K up to 16, with +0 in the
padding, and whose result is the padded product cropped to the logical shape.

The plan computes that padded problem without copying it. The MFMA kernel
already contracts the K edge against +0 (its last K slice zero-fills past K)
and stores only the rows and columns of the logical output, so the padded
buffers of the reference's plan (two +0-filled operand copies and a padded
product cropped by a third copy) would add three HBM passes and change no bit
of the result. ``explain()`` therefore reports the padded shapes and
alignment of the padded problem with the scratch and copies this plan really
uses: none (``scratch_bytes`` 0, ``copy_dispatches`` 0, ``dispatch_count``
1). ``bounds_checks_removed`` is True when the logical problem is a whole
number of the kernel's workgroup tiles (256 x 16 x 256): only then does the
product run without edge handling.
"""

from dataclasses import dataclass
from math import prod

import numpy as np

ALIGNMENT = (32, 16, 32)  # M, K, N (reference explain() field)
KERNEL_TILE = (256, 16, 256)  # M, K, N workgroup tile of the fp32 MFMA GEMM


def _round_up(value, multiple):
    return -(-value // multiple) * multiple


@dataclass(frozen=True)
class HIPPaddedGemm:
    backend: object
    input_shapes: tuple
    output_shape: tuple
    padded_input_shapes: tuple
    padded_output_shape: tuple
    dtype: np.dtype

    dispatch_count = 1  # one product call; no pad or crop copies

    def run(self, a, b):
        return self.backend.matmul(a, b, self.output_shape, self.dtype)

    def explain(self):
        (m, k), n = self.input_shapes[0][-2:], self.output_shape[-1]
        return {
            "input_shapes": self.input_shapes,
            "padded_input_shapes": self.padded_input_shapes,
            "output_shape": self.output_shape,
            "padded_output_shape": self.padded_output_shape,
            "alignment": ALIGNMENT,
            "scratch_bytes": 0,
            "copy_dispatches": 0,
            "bounds_checks_removed": all(v % t == 0 for v, t in zip((m, k, n), KERNEL_TILE)),
        }


def prepare(backend, ashape, bshape, shape, dtype, *, max_buffer_bytes=None):
    """Form a plan, or decline with None, before any allocation.

    ``max_buffer_bytes`` keeps the reference's limit on the largest padded
    buffer, so eligibility does not depend on the zero-copy execution.
    """
    ashape, bshape, shape = tuple(ashape), tuple(bshape), tuple(shape)
    if (
        np.dtype(dtype) != np.dtype("float32")
        or len(ashape) < 2
        or len(bshape) < 2
        or not prod(shape)
        or min(ashape[-2], bshape[-1]) < 32
        or ashape[-1] < 16
    ):
        return None
    m, k, n = ashape[-2], ashape[-1], bshape[-1]
    expected = np.broadcast_shapes(ashape[:-2], bshape[:-2]) + (m, n)
    if k != bshape[-2] or shape != expected:
        raise ValueError("Invalid padded matmul shapes")
    mp, kp, np_ = (_round_up(v, t) for v, t in zip((m, k, n), ALIGNMENT))
    ap, bp, cp = ashape[:-2] + (mp, kp), bshape[:-2] + (kp, np_), shape[:-2] + (mp, np_)
    largest = max(prod(s) for s in (ap, bp, cp))
    if largest > 2**31 - 1 or (max_buffer_bytes is not None and largest * 4 > max_buffer_bytes):
        return None
    return HIPPaddedGemm(backend, (ashape, bshape), shape, (ap, bp), cp, np.dtype(dtype))
