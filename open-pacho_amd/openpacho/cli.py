"""The ``pacho`` command: device discovery and a checked resident benchmark.

Interface of reference cli.py:20-143 (the ``pacho`` console script of
pyproject.toml:27-28):

- ``pacho devices [--backend hip] [--json]`` lists the devices of one GPU API.
  This build provides ``hip``; naming another runtime exits with status 2 and
  the backend's BackendUnavailableError text.
- ``pacho benchmark [--backend {numpy,hip}] [--device ID] [--size N]
  [--repeat R] [--dtype float32|float64] [--seed S] [--output PATH]`` times
  three resident operations (add, matmul, sum) on two size x size U[-1, 1)
  matrices, checks every result against NumPy on the host, and prints the
  report as strict JSON (schema_version 1; non-finite numbers are refused,
  reference cli.py:135). Exit status: 0 when every case is valid, 1 when one
  is not, 2 for an unavailable backend, an unsupported dtype or a bad value.

Timings are synchronized wall-clock seconds around the Python call, so they
include dispatch and allocation (reference cli.py:22-25): ``cold_seconds`` is
the first call, ``resident_seconds`` the ``repeat`` calls after it, and
``download_seconds`` the copy of the first result to the host.
"""

import argparse
import importlib.metadata
import json
import platform
import statistics
import sys
import time
from dataclasses import asdict
from pathlib import Path

import numpy as np

from ._array import asarray, asnumpy
from .backends import devices, get_backend
from .exceptions import BackendUnavailableError, UnsupportedDtypeError

SCHEMA_VERSION = 1
GPU_APIS = ("hip", "opencl", "vulkan", "cuda")
BENCH_BACKENDS = ("numpy",) + GPU_APIS
# One callable per case serves both sides: it is applied to the two resident
# device arrays and to the two host arrays they were uploaded from. Python
# functions, not operator.add: called with a tuple's arrays as its only
# references, NumPy's temporary elision would add into the host input in place
# (arrays of 256 KiB or more), corrupting the inputs of the later checks.
CASES = (
    ("add", lambda a, b: a + b),
    ("matmul", lambda a, b: a @ b),
    ("sum", lambda a, b: a.sum()),
)
TOLERANCE = {"float32": 5e-4, "float64": 1e-10}


def _seconds(engine, call):
    """(result, synchronized wall seconds) of one call on ``engine``."""
    engine.synchronize()
    begin = time.perf_counter()
    result = call()
    engine.synchronize()
    return result, time.perf_counter() - begin


def _host_seconds(call):
    begin = time.perf_counter()
    call()
    return time.perf_counter() - begin


def _versions(engine):
    found = {"numpy": np.__version__, "python": platform.python_version()}
    if engine.name == "hip":
        from . import _hip_lib

        found["pacho_hip"] = _hip_lib.load().hp_version().decode()
    try:
        found["open-pacho-amd"] = importlib.metadata.version("open-pacho-amd")
    except importlib.metadata.PackageNotFoundError:
        pass  # run from the source tree, not installed
    return found


def _case(engine, name, operation, device_args, host_args, repeat, tolerance):
    first, cold = _seconds(engine, lambda: operation(*device_args))
    begin = time.perf_counter()
    host = np.asarray(asnumpy(first))
    download = time.perf_counter() - begin
    expected = np.asarray(operation(*host_args))
    resident, reference = [], []
    for _ in range(repeat):
        resident.append(_seconds(engine, lambda: operation(*device_args))[1])
        reference.append(_host_seconds(lambda: operation(*host_args)))
    return {
        "operation": name,
        "valid": bool(host.shape == expected.shape and np.allclose(host, expected, rtol=tolerance, atol=tolerance)),
        "max_abs_error": float(np.max(np.abs(host - expected))) if host.size else 0.0,
        "cold_seconds": cold,
        "download_seconds": download,
        "resident_seconds": resident,
        "resident_median_seconds": statistics.median(resident),
        "numpy_seconds": reference,
        "numpy_median_seconds": statistics.median(reference),
    }


def benchmark(*, size=128, repeat=5, dtype="float32", backend="hip", device=None, seed=47):
    """Checked timings of add, matmul and sum on resident size x size inputs.

    Raises ValueError for a non-positive size or repeat or a dtype other than
    float32/float64, and the backend's own errors when it cannot be created.
    """
    if size < 1 or repeat < 1:
        raise ValueError("size and repeat must be positive")
    if dtype not in TOLERANCE:
        raise ValueError("benchmark dtype must be float32 or float64")
    engine = get_backend(backend, device=device)
    draw = np.random.default_rng(seed)
    host_args = tuple(draw.uniform(-1, 1, (size, size)).astype(dtype) for _ in range(2))
    device_args, upload = _seconds(engine, lambda: tuple(asarray(h, backend=engine) for h in host_args))
    cases = [_case(engine, name, op, device_args, host_args, repeat, TOLERANCE[dtype]) for name, op in CASES]
    return {
        "schema_version": SCHEMA_VERSION,
        "backend": engine.name,
        "device": engine.device,
        "os": platform.platform(),
        "versions": _versions(engine),
        "dtype": dtype,
        "size": size,
        "seed": seed,
        "repeat": repeat,
        "upload_seconds": upload,
        "cases": cases,
        "all_valid": all(case["valid"] for case in cases),
    }


def _parser():
    parser = argparse.ArgumentParser(prog="pacho", description="OpenPacho device discovery and checked benchmarks")
    commands = parser.add_subparsers(dest="command", required=True)
    listing = commands.add_parser("devices", help="List the devices of one GPU API (no interactive selection)")
    listing.add_argument("--backend", choices=GPU_APIS, default="hip")
    listing.add_argument("--json", action="store_true")
    bench = commands.add_parser("benchmark", help="Time resident operations, each checked against NumPy")
    bench.add_argument("--backend", choices=BENCH_BACKENDS, default="hip")
    bench.add_argument("--device", help="Device ID from 'pacho devices'")
    bench.add_argument("--size", type=int, default=128)
    bench.add_argument("--repeat", type=int, default=5)
    bench.add_argument("--dtype", choices=tuple(TOLERANCE), default="float32")
    bench.add_argument("--seed", type=int, default=47)
    bench.add_argument("--output", type=Path)
    return parser


def _list_devices(backend, as_json):
    found = devices(backend)
    if as_json:
        print(json.dumps([asdict(info) for info in found], indent=2))
        return
    for info in found:
        print(f"{info.id}  {info.kind}  {info.name}  ({info.vendor})  float64={info.fp64}")
    if not found:
        print(f"No {backend} devices found.")


def main(argv=None):
    """Entry point of the ``pacho`` script; returns the exit status."""
    args = _parser().parse_args(argv)
    try:
        if args.command == "devices":
            _list_devices(args.backend, args.json)
            return 0
        report = benchmark(size=args.size, repeat=args.repeat, dtype=args.dtype, backend=args.backend,
                           device=args.device, seed=args.seed)
        text = json.dumps(report, indent=2, allow_nan=False)
        if args.output:
            args.output.parent.mkdir(parents=True, exist_ok=True)
            args.output.write_text(text + "\n", encoding="utf-8")
        print(text)
        return 0 if report["all_valid"] else 1
    except (BackendUnavailableError, UnsupportedDtypeError, ValueError) as exc:
        print(f"pacho: {exc}", file=sys.stderr)
        return 2


if __name__ == "__main__":
    raise SystemExit(main())
