"""Register budgets of the built kernels (CPU tier).

``open-pacho_amd/build.py`` records the compiler's per-kernel resource
remarks (registers, scratch, occupancy) in ``_build/resources.json``. A
register spill in a hot kernel goes to scratch memory and costs far more
than any test of results shows (a spilling fp64 GEMM loader once cost
4096^2 x 4095 fp64 12 points of peak with every test green), so the budgets
are checked here: no fp32 GEMM, GEMV, norm, reduction or RNG kernel spills,
fp64 GEMM kernels stay within their known spills, and the GEMMs keep two
waves per SIMD. Skipped when the library has not been built in this tree.
"""

import json
from pathlib import Path

import pytest

RESOURCES = Path(__file__).resolve().parents[1] / "open-pacho_amd" / "_build" / "resources.json"

# Known fp64 GEMM spills (VGPRs), by translation unit: the kernels run at the
# 256-VGPR limit of two waves per SIMD; the stream-K and any-K variants of
# the transposed-A layouts spill a little.
FP64_SPILL_LIMIT = {"gemm_f64_nn": 11, "gemm_f64_nt": 0, "gemm_f64_tn": 28, "gemm_f64_tt": 22}


@pytest.fixture(scope="module")
def resources():
    if not RESOURCES.exists():
        pytest.skip("library not built in this tree (open-pacho_amd/build.py)")
    return json.loads(RESOURCES.read_text())


def _kernels(resources, unit):
    return {name: r for name, r in resources.get(unit, {}).items() if "kernel" in name}


def test_fp32_gemm_kernels_do_not_spill_and_keep_two_waves(resources):
    for unit in ("gemm_f32_nn", "gemm_f32_tn", "gemm_f32_nt", "gemm_f32_tt"):
        kernels = _kernels(resources, unit)
        assert kernels, unit
        for name, r in kernels.items():
            assert r.get("VGPRs Spill", 0) == 0 and r.get("SGPRs Spill", 0) == 0, (unit, name, r)
            if "f326kernel" in name:
                assert r["Occupancy [waves/SIMD]"] >= 2, (unit, name, r)


def test_fp64_gemm_spills_stay_within_known_limits(resources):
    for unit, limit in FP64_SPILL_LIMIT.items():
        kernels = _kernels(resources, unit)
        assert kernels, unit
        for name, r in kernels.items():
            assert r.get("VGPRs Spill", 0) <= limit, (unit, name, r)
            if "f646kernel" in name:
                assert r["Occupancy [waves/SIMD]"] >= 2, (unit, name, r)


@pytest.mark.parametrize("unit", ["gemv", "norm", "reduce", "philox", "copy", "gemm"])
def test_streaming_kernels_do_not_spill(resources, unit):
    kernels = _kernels(resources, unit)
    assert kernels, unit
    for name, r in kernels.items():
        assert r.get("VGPRs Spill", 0) == 0 and r.get("SGPRs Spill", 0) == 0, (unit, name, r)
        assert r.get("Dynamic Stack") in (None, "False"), (unit, name, r)
