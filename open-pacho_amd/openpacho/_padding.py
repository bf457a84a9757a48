"""Opt-in physical padding for the GPU GEMM, without changing logical arrays.

Plan contract (reference _padding.py:13-109): float32 operands with at least
32 output rows and columns and K >= 16 are copied into private buffers whose
M and N are rounded up to multiples of 32 and K to a multiple of 16, filled
with +0; the GEMM runs on the padded shapes and the padded product is cropped
back. Batch prefixes are kept. Plans hold only shape metadata and backend
callables: inputs are packed anew on every call. A plan that cannot be formed
(ineligible dtype/shape, index or buffer limits) declines with ``None`` and
ordinary matmul runs instead; allocation failures later are errors.
"""

from dataclasses import dataclass
from math import prod

import numpy as np

ALIGNMENT = (32, 16, 32)  # M, K, N


def validate_padding(value):
    if not isinstance(value, (bool, np.bool_)):
        raise TypeError("padding must be a boolean")
    return bool(value)


def prepare_padding(backend, ashape, bshape, shape, dtype):
    """An absent capability declines the hint; preparation failures propagate."""
    factory = getattr(backend, "prepare_padded_matmul", None)
    return None if factory is None else factory(ashape, bshape, shape, dtype)


def _round_up(value, multiple):
    return -(-value // multiple) * multiple


@dataclass(frozen=True)
class PaddedGemm:
    backend: object
    input_shapes: tuple
    output_shape: tuple
    padded_input_shapes: tuple
    padded_output_shape: tuple
    copy: object  # copy(backend, array, shape) -> storage (pad or crop)
    gemm: object  # gemm(backend, a, b, shape) -> storage
    guard_free: bool = False

    @property
    def dispatch_count(self):
        copies = sum(a != b for a, b in zip(self.input_shapes, self.padded_input_shapes))
        return 1 + copies + (self.output_shape != self.padded_output_shape)

    def run(self, a, b):
        from ._array import ndarray

        operands = []
        for array, padded in zip((a, b), self.padded_input_shapes):
            if array.shape != padded:
                array = ndarray._wrap(self.copy(self.backend, array, padded), padded, array.dtype, self.backend)
            operands.append(array)
        data = self.gemm(self.backend, operands[0], operands[1], self.padded_output_shape)
        if self.padded_output_shape != self.output_shape:
            padded = ndarray._wrap(data, self.padded_output_shape, a.dtype, self.backend)
            data = self.copy(self.backend, padded, self.output_shape)
        return data

    def explain(self):
        scratch = [
            prod(padded) * 4 for original, padded in zip(self.input_shapes, self.padded_input_shapes) if original != padded
        ]
        if self.output_shape != self.padded_output_shape:
            scratch.append(prod(self.padded_output_shape) * 4)
        return {
            "input_shapes": self.input_shapes,
            "padded_input_shapes": self.padded_input_shapes,
            "output_shape": self.output_shape,
            "padded_output_shape": self.padded_output_shape,
            "alignment": ALIGNMENT,
            "scratch_bytes": sum(scratch),
            "copy_dispatches": len(scratch),
            # True only when the padded problem is a whole number of the
            # kernel's own tiles, so no element guard remains in the GEMM.
            "bounds_checks_removed": self.guard_free,
        }


def prepare_register_padding(
    backend, ashape, bshape, shape, dtype, copy, gemm, *, max_buffer_bytes=None, kernel_tile=None
):
    """Form a padding plan, or decline with None before any allocation."""
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
    guard_free = kernel_tile is not None and all(v % t == 0 for v, t in zip((mp, kp, np_), kernel_tile))
    return PaddedGemm(backend, (ashape, bshape), shape, (ap, bp), cp, copy, gemm, guard_free)
