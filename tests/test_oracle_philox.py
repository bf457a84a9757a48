"""Pinning the Philox oracle: published vectors, two restatements, golden samples."""

from pathlib import Path

import numpy as np
import pytest

from oracle import philox
from oracle import numpy_backend as nb

GOLDEN = Path(__file__).parent / "golden" / "reference_rng.npz"

# Random123 kat_vectors, Philox4x32 ten rounds (reference tests/test_random.py:27-41).
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    (
        (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
        (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1),
    ),
]


@pytest.mark.parametrize("counter,key,expected", KAT)
def test_known_answers_python_and_c(counter, key, expected):
    assert philox.block_int(counter, key) == expected
    assert philox.c_block(counter, key) == expected


def test_numpy_words_match_block_function_including_carry():
    for seed, start in ((0, 0), (42, 2**32 - 3), (2**64 - 1, 2**64 - 7)):
        count = 7
        got = philox.words(count, seed, start)
        for i in range(count):
            ctr = start + i
            want = philox.block_int((ctr & 0xFFFFFFFF, ctr >> 32, 0, 0), (seed & 0xFFFFFFFF, seed >> 32))
            assert tuple(int(w) for w in got[i]) == want


def test_c_and_numpy_restatements_agree():
    for seed, start in ((7, 0), (2**63 + 5, 2**32 - 100)):
        np.testing.assert_array_equal(philox.words(4096, seed, start), philox.c_words(4096, seed, start))
        for dtype in ("float32", "float64"):
            np.testing.assert_array_equal(
                philox.samples("random", dtype, 4096, seed, start, 0, 1), philox.c_uniform(dtype, 4096, seed, start)
            )
            np.testing.assert_array_equal(
                philox.samples("uniform", dtype, 4096, seed, start, -3, 7),
                philox.c_uniform(dtype, 4096, seed, start, "uniform", -3, 7),
            )


def test_unit_values_are_exact_dyadic_grids():
    w = philox.words(1000, 3, 0)
    u32 = philox.unit("float32", w[:, 0], w[:, 1])
    assert u32.dtype == np.float32 and (u32 >= 0).all() and (u32 < 1).all()
    np.testing.assert_array_equal(u32 * np.float32(2**24), (w[:, 0] >> 8).astype(np.float32))
    u64 = philox.unit("float64", w[:, 0], w[:, 1])
    expected = ((w[:, 0].astype(np.uint64) >> 5) << np.uint64(26)) + (w[:, 1].astype(np.uint64) >> 6)
    np.testing.assert_array_equal(u64 * 2.0**53, expected.astype(np.float64))


def _golden():
    with np.load(GOLDEN) as data:
        return {key: data[key] for key in data.files}


PARAMS = {"random": (0, 1), "uniform": (-3, 7), "normal": (2, 3), "exponential": (0, 2)}


def test_oracle_reproduces_reference_numpy_backend_samples():
    golden = _golden()
    assert len(golden) == 2 * 4 * 3 * 3
    for key, expected in golden.items():
        dist, dtype, seed, start = key.split("|")
        first, second = PARAMS[dist]
        got = nb.random(dist, dtype, expected.shape, int(seed), int(start), first, second)
        if dist in ("random", "uniform"):
            np.testing.assert_array_equal(got, expected, err_msg=key)
        else:
            # Same formula, same NumPy; transcendental calls may differ only
            # across NumPy builds (tolerance of reference test_random.py:75-80).
            tol = 3e-6 if dtype == "float32" else 1e-13
            np.testing.assert_allclose(got, expected, rtol=tol, atol=tol, err_msg=key)


def test_planted_mistakes_are_caught_by_the_golden_samples():
    """A plausible slip (wrong word, sin for cos, log for log1p) fails the fixtures."""
    golden = _golden()
    key = "normal|float32|42|0"
    expected = golden[key]
    w = philox.words(expected.shape[0], 42, 0)
    u = philox.unit("float32", w[:, 0], w[:, 1])
    v = philox.unit("float32", w[:, 2], w[:, 3])
    two = np.float32(2)
    variants = {
        "sin": 2 + 3 * (np.sqrt(two * -np.log1p(-u)) * np.sin(np.float32(2 * np.pi) * v)),
        "swap_words": 2 + 3 * (np.sqrt(two * -np.log1p(-v)) * np.cos(np.float32(2 * np.pi) * u)),
        "log": 2 + 3 * (np.sqrt(two * -np.log(u + np.float32(1e-30))) * np.cos(np.float32(2 * np.pi) * v)),
    }
    for name, value in variants.items():
        assert not np.allclose(value, expected, rtol=3e-6, atol=3e-6), name
