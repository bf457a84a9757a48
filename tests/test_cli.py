"""The ``pacho`` command on the NumPy backend (reference tests/test_cli.py).

Report contract of reference cli.py:20-143: schema_version 1, one case per
operation with its timings, ``all_valid``, strict JSON, exit status 0 / 1
(an invalid case) / 2 (bad arguments or an unavailable backend).
"""

import json
import subprocess
import sys
from pathlib import Path

import pytest

from openpacho import cli

ROOT = Path(__file__).resolve().parents[1]
CASE_KEYS = {"operation", "valid", "max_abs_error", "cold_seconds", "download_seconds", "resident_seconds",
             "resident_median_seconds", "numpy_seconds", "numpy_median_seconds"}
REPORT_KEYS = {"schema_version", "backend", "device", "os", "versions", "dtype", "size", "seed", "repeat",
               "upload_seconds", "cases", "all_valid"}


def test_benchmark_json(tmp_path, capsys):
    path = tmp_path / "out" / "bench.json"
    argv = ["benchmark", "--backend", "numpy", "--size", "4", "--repeat", "2", "--output", str(path)]
    assert cli.main(argv) == 0
    report = json.loads(path.read_text())
    assert set(report) == REPORT_KEYS
    assert report["schema_version"] == 1 and report["backend"] == "numpy" and report["all_valid"]
    assert [case["operation"] for case in report["cases"]] == ["add", "matmul", "sum"]
    for case in report["cases"]:
        assert set(case) == CASE_KEYS
        assert len(case["resident_seconds"]) == 2 and case["resident_median_seconds"] > 0
        assert case["valid"] and case["max_abs_error"] < 5e-4
    assert json.loads(capsys.readouterr().out) == report


@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_benchmark_report_fields(dtype):
    report = cli.benchmark(size=9, repeat=3, dtype=dtype, backend="numpy", seed=5)
    assert report["dtype"] == dtype and report["size"] == 9 and report["seed"] == 5 and report["repeat"] == 3
    assert report["versions"]["numpy"] and report["versions"]["python"]
    assert report["upload_seconds"] >= 0 and report["all_valid"]
    json.dumps(report, allow_nan=False)  # strict JSON


def test_invalid_benchmark(capsys):
    assert cli.main(["benchmark", "--backend", "numpy", "--size", "0"]) == 2
    assert "positive" in capsys.readouterr().err
    assert cli.main(["benchmark", "--backend", "numpy", "--repeat", "0"]) == 2
    assert "positive" in capsys.readouterr().err


def test_an_invalid_case_exits_with_status_1(monkeypatch, capsys):
    """A device result that differs from NumPy's makes the report invalid."""
    calls = []

    def wrong_on_device(a, b):
        calls.append(type(a).__name__)
        return a - b if type(a).__module__.startswith("openpacho") else a + b

    monkeypatch.setattr(cli, "CASES", (("add", wrong_on_device),) + cli.CASES[1:])
    assert cli.main(["benchmark", "--backend", "numpy", "--size", "3", "--repeat", "1"]) == 1
    report = json.loads(capsys.readouterr().out)
    assert not report["all_valid"] and not report["cases"][0]["valid"] and report["cases"][1]["valid"]
    assert "ndarray" in calls


@pytest.mark.parametrize("api", ["cuda", "opencl", "vulkan"])
def test_foreign_runtimes_are_refused(api, capsys):
    assert cli.main(["devices", "--backend", api]) == 2
    assert "not part of this build" in capsys.readouterr().err
    assert cli.main(["benchmark", "--backend", api]) == 2
    assert "pacho:" in capsys.readouterr().err


def test_unknown_choices_are_argparse_errors():
    with pytest.raises(SystemExit) as exc:
        cli.main(["benchmark", "--dtype", "float16"])
    assert exc.value.code == 2


def test_module_entry_point():
    env_path = str(ROOT / "open-pacho_amd")
    out = subprocess.run(
        [sys.executable, "-m", "openpacho", "benchmark", "--backend", "numpy", "--size", "5", "--repeat", "1",
         "--dtype", "float64"],
        capture_output=True, text=True, cwd=env_path, timeout=120, check=False,
    )
    assert out.returncode == 0, out.stderr
    assert json.loads(out.stdout)["all_valid"]


def test_console_script_is_declared():
    tomli = pytest.importorskip("tomli")
    project = tomli.loads((ROOT / "open-pacho_amd" / "pyproject.toml").read_text())["project"]
    assert project["scripts"]["pacho"] == "openpacho.cli:main"


def test_host_inputs_survive_every_case():
    """float64 257 x 257 inputs (above NumPy's 256 KiB temporary-elision
    threshold) stay unchanged through every case, on both sides."""
    report = cli.benchmark(size=257, repeat=2, dtype="float64", backend="numpy")
    assert report["all_valid"], [(c["operation"], c["max_abs_error"]) for c in report["cases"]]
    assert all(case["max_abs_error"] == 0 for case in report["cases"][:2])
