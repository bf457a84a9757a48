"""GPU parity of hp_pad_copy, the bit-preserving batched pad/crop copy.

The contract of reference _padding_copy.py:99-177 and docs/padding.md:85-98:
dst[b][r][c] = src[b][r][c] inside the source, all-zero words (+0, bits
0x0...0) outside it; every copied word keeps its bits (NaN payloads,
signalling NaNs, subnormals, -0). Checked bit for bit against NumPy slicing
and np.pad, through the C ABI and through HIPBackend.pad_copy.
"""

import ctypes

import numpy as np
import pytest

import openpacho as p

pytestmark = pytest.mark.gpu

SPECIAL32 = np.array([0x7FC00001, 0x7F800001, 0xFFC12345, 0x00000001, 0x807FFFFF, 0x80000000, 0x7F800000, 0xFF800000],
                     dtype=np.uint32)
SPECIAL64 = np.array([0x7FF8000000000001, 0x7FF0000000000001, 0xFFF123456789ABCD, 0x0000000000000001,
                      0x800FFFFFFFFFFFFF, 0x8000000000000000, 0x7FF0000000000000, 0xFFF0000000000000],
                     dtype=np.uint64)


def _words(rng, shape, word):
    special = SPECIAL32 if word == np.uint32 else SPECIAL64
    info = np.iinfo(word)
    src = rng.integers(0, info.max, size=shape, dtype=word, endpoint=True)
    flat = src.reshape(-1)
    where = rng.choice(flat.size, min(flat.size, 4 * special.size), replace=False)
    flat[where] = np.resize(special, where.size)
    return src


def _expected(src, dst_rows, dst_cols):
    out = np.zeros(src.shape[:-2] + (dst_rows, dst_cols), src.dtype)
    r, c = min(src.shape[-2], dst_rows), min(src.shape[-1], dst_cols)
    out[..., :r, :c] = src[..., :r, :c]
    return out


def _abi_pad(hip, src, dst_rows, dst_cols):
    batch = int(np.prod(src.shape[:-2], dtype=np.int64))
    size = src.dtype.itemsize
    d_src = hip.upload(src.reshape(-1)) if src.size else None
    count = batch * dst_rows * dst_cols
    # The destination starts as all-ones words, so an unwritten word shows.
    d_dst = hip.upload(np.full(max(count, 1), np.iinfo(src.dtype).max, src.dtype))
    with hip._active():
        hip._call("hp_pad_copy", size, ctypes.c_void_p(d_src.ptr if d_src else None), ctypes.c_void_p(d_dst.ptr),
                  batch, src.shape[-2], src.shape[-1], dst_rows, dst_cols)
        out = np.empty(max(count, 1), src.dtype)
        hip._call("hp_d2h", ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(d_dst.ptr), out.nbytes)
    return out[:count].reshape(src.shape[:-2] + (dst_rows, dst_cols))


@pytest.mark.parametrize("word", [np.uint32, np.uint64])
@pytest.mark.parametrize(
    "src_shape,dst",
    [
        ((3, 5, 7), (8, 16)),  # pad rows and columns
        ((3, 5, 7), (2, 3)),  # crop both
        ((3, 5, 7), (9, 4)),  # pad rows, crop columns
        ((3, 5, 7), (5, 7)),  # identity
        ((2, 300, 1000), (320, 1024)),  # 256-lane rows, unrolled loads
        ((1, 4097, 3001), (4128, 3008)),  # config 4's padded A
        ((4, 0, 7), (3, 9)),  # empty source: zeros only
        ((2, 6, 0), (4, 2)),
    ],
)
def test_pad_copy_is_bitwise_numpy(hip, word, src_shape, dst):
    rng = np.random.default_rng(sum(src_shape) + dst[0] * 7 + dst[1])
    src = _words(rng, src_shape, word)
    got = _abi_pad(hip, src, *dst)
    want = _expected(src, *dst)
    np.testing.assert_array_equal(got, want)
    if all(dst[i] >= src_shape[1 + i] for i in range(2)):
        pads = [(0, 0)] * (src.ndim - 2) + [(0, dst[0] - src_shape[-2]), (0, dst[1] - src_shape[-1])]
        np.testing.assert_array_equal(got, np.pad(src, pads))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_backend_pad_copy_keeps_special_values(hip, dtype):
    word = np.uint32 if dtype == np.float32 else np.uint64
    rng = np.random.default_rng(3)
    bits = _words(rng, (2, 33, 17), word)
    host = bits.view(dtype)
    out = hip.pad_copy(p.asarray(host, backend=hip), (2, 64, 32))
    got = hip.download(p.ndarray._wrap(out, (2, 64, 32), dtype, hip)).view(word)
    np.testing.assert_array_equal(got, _expected(bits, 64, 32))
    assert not got[:, 33:, :].any() and not got[:, :, 17:].any()  # +0, never -0
    crop = hip.pad_copy(p.asarray(host, backend=hip), (2, 20, 10))
    got = hip.download(p.ndarray._wrap(crop, (2, 20, 10), dtype, hip)).view(word)
    np.testing.assert_array_equal(got, bits[:, :20, :10])


def test_pad_copy_rejects_other_word_sizes(hip):
    src = hip.upload(np.zeros(16, np.uint32))
    dst = hip.upload(np.zeros(16, np.uint32))
    with hip._active(), pytest.raises(ValueError, match="4- or 8-byte"):
        hip._call("hp_pad_copy", 2, ctypes.c_void_p(src.ptr), ctypes.c_void_p(dst.ptr), 1, 4, 4, 4, 4)
