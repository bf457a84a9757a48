"""The hip backend's opt-in padding plan for fp32 GEMM (``matmul(padding=True)``).

Plan semantics follow the reference (_padding.py:80-109 eligibility and
rounding, :25-77 run/explain/dispatch_count): float32 operands with at least
32 output rows and columns and K >= 16 are copied into private +0-filled
buffers with M and N rounded up to 32 and K to 16; the GEMM runs on the padded
shapes and the padded product is cropped. The plan is its own object because
the reference's PaddedGemm dispatches its GEMM by backend name; this one calls
the hip backend's own matmul and pad/crop copies (hp_pad_copy), so the module
needs only ``ndarray`` from the array facade.

On this backend padding turns an unaligned problem (e.g. odd K, which forces
scalar guarded loads) into the 16-byte vector-load path of the MFMA kernel.
``bounds_checks_removed`` is True only when the padded problem is a whole
number of the kernel's workgroup tiles (256 x 16 x 256), because only then
does the GEMM run without element guards.
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

    @property
    def dispatch_count(self):
        copies = sum(a != b for a, b in zip(self.input_shapes, self.padded_input_shapes))
        return 1 + copies + (self.output_shape != self.padded_output_shape)

    def run(self, a, b):
        from ._array import ndarray

        backend = self.backend
        operands = []
        for array, padded in zip((a, b), self.padded_input_shapes):
            if array.shape != padded:
                array = ndarray._wrap(backend.pad_copy(array, padded), padded, array.dtype, backend)
            operands.append(array)
        data = backend.matmul(operands[0], operands[1], self.padded_output_shape, a.dtype)
        if self.padded_output_shape != self.output_shape:
            padded = ndarray._wrap(data, self.padded_output_shape, a.dtype, backend)
            data = backend.pad_copy(padded, self.output_shape)
        return data

    def explain(self):
        scratch = [
            prod(padded) * 4 for original, padded in zip(self.input_shapes, self.padded_input_shapes) if original != padded
        ]
        if self.output_shape != self.padded_output_shape:
            scratch.append(prod(self.padded_output_shape) * 4)
        mp, kp = self.padded_input_shapes[0][-2:]
        np_ = self.padded_output_shape[-1]
        return {
            "input_shapes": self.input_shapes,
            "padded_input_shapes": self.padded_input_shapes,
            "output_shape": self.output_shape,
            "padded_output_shape": self.padded_output_shape,
            "alignment": ALIGNMENT,
            "scratch_bytes": sum(scratch),
            "copy_dispatches": len(scratch),
            "bounds_checks_removed": all(v % t == 0 for v, t in zip((mp, kp, np_), KERNEL_TILE)),
        }


def prepare(backend, ashape, bshape, shape, dtype, *, max_buffer_bytes=None):
    """Form a plan, or decline with None before any allocation."""
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
    return HIPPaddedGemm(backend, (ashape, bshape), shape, (ap, bp), cp)
