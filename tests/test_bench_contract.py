"""bench.py's command-line contract on the CPU (no GPU is touched).

One GPU only: ``--gpus`` above 1 exits with status 2 and a message before
any backend is created. The roofline helper reports the fraction against
MI355X's published peaks, and the PMC traffic and VALU tables it reads name
kernels that exist in the built library. Every timed workload is preceded by
at least a minimum number of untimed calls and a minimum span of untimed work.
"""

import json
import subprocess
import sys
import types
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_exits_with_a_message(gpus):
    done = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", gpus], capture_output=True, text=True, timeout=120
    )
    assert done.returncode == 2
    assert "one MI355X" in done.stderr and not done.stdout


def test_roofline_fractions_use_published_peaks():
    gemm = bench.roofline("mfma", 2 * 8192**3, 7.8)
    assert gemm["peak"] == 157.3 and gemm["unit"] == "TFLOP/s"
    assert gemm["frac"] == pytest.approx(2 * 8192**3 / 7.8e-3 / 1e12 / 157.3, rel=1e-3)
    hbm = bench.roofline("hbm", 2**30, 0.157)
    assert hbm["peak"] == 8000.0 and hbm["unit"] == "GB/s"
    assert hbm["frac"] == pytest.approx(2**30 / 0.157e-3 / 1e9 / 8000.0, rel=1e-3)


def test_profile_tables_name_built_kernels():
    resources = ROOT / "open-pacho_amd" / "_build" / "resources.json"
    if not resources.exists():
        pytest.skip("library not built in this tree")
    built = json.dumps(json.loads(resources.read_text()))
    traffic = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    valu = json.loads((ROOT / "profiles" / "valu.json").read_text())
    for table in (traffic, valu):
        for name, entry in table.items():
            if name.startswith("_"):
                continue
            kernel = entry["kernel"]  # e.g. "philox_kernel<float, 5>", "f32::kernel<0, false, false, false>"
            base = kernel.split("<")[0].split("::")[-1]
            assert base in built, (name, kernel)


def test_warm_up_runs_the_minimum_calls_and_the_minimum_time(monkeypatch):
    """At least `calls` calls and WARM_MS of time; after the first call the
    calls are queued in batches of about 5 ms of work, synchronized between
    batches only (a sync after every call left the device idle)."""
    monkeypatch.setattr(bench, "WARM_MS", 30.0)
    clock = types.SimpleNamespace(now=0.0)
    monkeypatch.setattr(bench, "time", types.SimpleNamespace(perf_counter=lambda: clock.now))
    events = []

    def call():
        events.append("c")
        clock.now += 0.00125  # 1.25 ms of "device work" per call: batches of 4

    bench.warm(call, lambda: events.append("s"), 3)
    assert clock.now * 1e3 >= 30.0 and events[:2] == ["c", "s"] and events[-1] == "s"
    batches = "".join(events[2:]).split("s")[:-1]
    assert batches and all(b == "cccc" for b in batches)
    assert events.count("c") >= 3 and events.count("s") < events.count("c")
    monkeypatch.setattr(bench, "WARM_MS", 0.0)
    events.clear()
    bench.warm(call, lambda: events.append("s"), 5)
    assert events.count("c") >= 5


def test_cpu_baseline_protocol_warms_then_takes_the_median_of_seven():
    calls = []
    start = bench.time.perf_counter()
    seconds, timed = bench.cpu_timed(lambda: calls.append(bench.time.perf_counter()))
    elapsed = bench.time.perf_counter() - start
    assert timed >= 7 and len(calls) >= timed + 3
    warm_calls = [t for t in calls if t - start < 0.25]
    assert len(warm_calls) >= 3 and elapsed >= 0.25
    assert seconds >= 0


def test_cpu_blas_legs_report_affinity_cores_and_one_thread():
    import numpy as np

    a = np.ones((64, 64), np.float32)
    leg = bench.cpu_blas(lambda: a @ a, 2.0 * 64**3, "GFLOP/s", "64^3")
    assert leg["cores"] == bench.cpu_threads() and leg["kind"] == "port"
    assert leg["one_thread"]["cores"] == 1 and leg["one_thread"]["value"] > 0
    assert "median of" in leg["sample"]


def test_strict_json_writes_non_finite_numbers_as_strings():
    line = bench.strict_json({"a": float("inf"), "b": [float("nan"), 1.5], "c": {"d": -float("inf")}, "e": 2})
    assert line == {"a": "inf", "b": ["nan", 1.5], "c": {"d": "-inf"}, "e": 2}
    json.loads(json.dumps(line, allow_nan=False))
