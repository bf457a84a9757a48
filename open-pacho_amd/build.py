"""Build libpacho_hip.so (HIP kernels + C ABI) for gfx950 with hipcc.

Objects go to open-pacho_amd/_build/; the shared library is written next to the
Python package (open-pacho_amd/openpacho/libpacho_hip.so), where the `hip`
backend loads it. Run: python open-pacho_amd/build.py [--jobs N]
"""

import argparse
import json
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIBRARY = ROOT / "openpacho" / "libpacho_hip.so"
ARCH = "gfx950"

# Numerics policy: no floating-point contraction (the reference compiles its
# kernels with --fmad=false), IEEE denormals, correctly rounded fp32 div/sqrt.
# Packed fp32 instructions are disabled for every HIP source.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def hipcc():
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; install ROCm or put /opt/rocm/bin on PATH")
    return found


REMARK = re.compile(r"remark:\s+(.+?): (\S+) \[-Rpass-analysis=kernel-resource-usage\]")


def _resources(lines):
    """Per-kernel register, scratch and occupancy figures from the compiler's
    kernel-resource-usage remarks (device functions that are not kernels are
    reported too and kept)."""
    kernels, current = {}, None
    for line in lines:
        match = REMARK.search(line)
        if not match:
            continue
        key, value = match.group(1).strip(), match.group(2)
        if key == "Function Name":
            current = kernels.setdefault(value, {})
        elif current is not None:
            current[key] = int(value) if value.isdigit() else value
    return kernels


# Per-unit flags. The fp32 GEMM units keep MFMA accumulators in VGPRs. The
# flag came with an earlier one-wave-per-SIMD form of the narrow kernel, where
# the compiler otherwise put them in AGPRs and copied them to VGPRs and back
# every slice. Now it changes only register assignment (in the four-wave
# narrow kernel and the 256 x 256 mode-2 kernel); every kernel of these units
# has been measured with it.
UNIT_FLAGS = {f"gemm_f32_{layout}": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"] for layout in ("nn", "nt", "tn", "tt")}


def _compile(source):
    obj = BUILD / (source.stem + ".o")
    command = [hipcc(), *FLAGS, *UNIT_FLAGS.get(source.stem, []), "-Rpass-analysis=kernel-resource-usage", "-c",
               str(source), "-o", str(obj)]
    result = subprocess.run(command, capture_output=True, text=True)
    lines = (result.stdout + result.stderr).splitlines()
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = ("packed-fp32-ops", "is not a recognized feature for this target", "kernel-resource-usage")
    log = "\n".join(line for line in lines if not any(n in line for n in noise)).strip()
    if result.returncode:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{log}")
    return obj, log, _resources(lines)


def build(jobs=None, verbose=False):
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, sources))
    resources = {}
    for obj, log, kernels in results:
        if log and verbose:
            print(f"[{obj.name}] {log}")
        resources[obj.stem] = kernels
    # Read by tests/test_build_resources.py (register spills, occupancy).
    (BUILD / "resources.json").write_text(json.dumps(resources, indent=1, sort_keys=True) + "\n")
    tmp = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)]
    command += [str(obj) for obj, _, _ in results] + ["-lhiprtc"]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"link failed:\n{result.stdout}{result.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("-v", "--verbose", action="store_true")
    args = parser.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(path)


if __name__ == "__main__":
    sys.exit(main())
