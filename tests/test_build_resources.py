"""Register budgets of the built kernels (CPU tier).

``open-pacho_amd/build.py`` records the compiler's per-kernel resource
remarks (registers, scratch, occupancy) in ``_build/resources.json``. A
register spill in a hot kernel goes to scratch memory and costs far more
than any test of results shows (a spilling fp64 GEMM loader once cost
4096^2 x 4095 fp64 12 points of peak with every test green), so the budgets
are checked here: no fp32 GEMM, GEMV, norm, reduction or RNG kernel spills,
fp64 GEMM kernels stay within their known spills, and the GEMMs keep two
waves per SIMD. Skipped when the library has not been built in this tree.
The GEMM units are also compiled to assembly here, to check the order of
their LDS reads, barriers and waits.
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


# Scalar registers that the any-alignment stream-K kernels (two pieces, each
# with the state of both LDS-DMA forms: 16-byte for whole K slices, 4-byte
# for the K edge) may spill. An SGPR spill goes to a lane of a VGPR
# (v_writelane / v_readlane, no memory traffic); the assembly test below
# checks that no spill code sits inside a loop of the tiled kernels.
FP32_SGPR_SPILL_LIMIT = 32


def test_fp32_gemm_kernels_do_not_spill_and_keep_two_waves(resources):
    for unit in ("gemm_f32_nn", "gemm_f32_tn", "gemm_f32_nt", "gemm_f32_tt"):
        kernels = _kernels(resources, unit)
        assert kernels, unit
        for name, r in kernels.items():
            assert r.get("VGPRs Spill", 0) == 0, (unit, name, r)
            assert r.get("SGPRs Spill", 0) <= FP32_SGPR_SPILL_LIMIT, (unit, name, r)
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


# Two properties of the GEMM kernels' assembly that no result test sees:
# 1. The prologue reads LDS buffer 0 between the first two barriers; the
#    second orders those reads before slice 2's LDS writes into the same
#    buffer. If the compiler sinks the reads below it (into the block that
#    first uses them), a late wave can read slice 2's data (seen as one wrong
#    16 x 64 fragment block in batched products with several workgroups per
#    compute unit).
# 2. No fragment read of the tiled kernels waits for vmcnt: the LDS-DMA in
#    flight during a slice writes the other buffer. A wait there (the
#    compiler adds one for some placements of that barrier) cost 8192^3 4% of
#    peak. (The narrow kernel waits for its DMA by design at the start of
#    each slice, before it reads the next slice; it has no such barrier.)
# 3. No scalar-register spill code (v_writelane / v_readlane) in a block that
#    the compiler marks as part of a loop (the K loops).
@pytest.mark.parametrize("unit", [f"gemm_{t}_{layout}" for t in ("f32", "f64") for layout in ("nn", "nt", "tn", "tt")])
def test_gemm_lds_reads_keep_their_barriers_and_skip_dma_waits(unit, tmp_path):
    import importlib.util
    import shutil
    import subprocess

    spec = importlib.util.spec_from_file_location("pacho_build", RESOURCES.parents[1] / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    if not (shutil.which("hipcc") or Path("/opt/rocm/bin/hipcc").exists()):
        pytest.skip("hipcc not available")
    source = build.CSRC / f"{unit}.hip"
    asm = tmp_path / f"{unit}.s"
    flags = [f for f in build.FLAGS if f != "-Wall"] + build.UNIT_FLAGS.get(unit, [])
    subprocess.run([build.hipcc(), *flags, "--cuda-device-only", "-S", str(source), "-o", str(asm)], check=True,
                   capture_output=True)
    kernel, previous, barriers, checked, in_loop = None, "", {}, set(), False
    for line in asm.read_text().splitlines():
        text = line.strip()
        if line.startswith("_Z") and ":" in line:  # a function label
            kernel = line.split(":")[0]
            barriers[kernel] = []
            in_loop = False
        if line.startswith(".LBB"):  # a block label; loop blocks carry a loop comment
            in_loop = "Loop Header" in line or "in Loop:" in line
        if kernel is None or not text or text.startswith(";"):
            continue
        if in_loop and "kernel" in kernel and "narrow" not in kernel:
            assert not text.startswith(("v_writelane", "v_readlane")), f"spill code in a loop of {kernel}"
        if text.startswith("s_barrier"):
            barriers[kernel].append(0)
        elif text.startswith("ds_read") and barriers[kernel]:
            barriers[kernel][-1] += 1  # LDS reads after the latest barrier
        if text.startswith("ds_read") and "narrow" not in kernel:
            assert not previous.startswith("s_waitcnt vmcnt"), f"fragment read waits for vmcnt in {kernel}"
        previous = text
    for kernel, reads in barriers.items():
        if "kernel" in kernel and "narrow" not in kernel and len(reads) >= 2:
            checked.add(kernel)
            assert reads[0] > 0, f"no LDS reads between the first two barriers (sunk reads) in {kernel}"
    assert checked, unit
