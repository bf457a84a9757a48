"""The ``pacho`` command on the hip backend (reference cli.py:20-143)."""

import json

import pytest

from openpacho import cli

pytestmark = pytest.mark.gpu


def test_devices_lists_the_mi355x(hip, capsys):
    assert cli.main(["devices", "--backend", "hip", "--json"]) == 0
    found = json.loads(capsys.readouterr().out)
    assert found and {"id", "name", "vendor", "kind", "fp64", "memory_bytes", "driver"} <= set(found[0])
    assert found[0]["kind"] == "GPU" and found[0]["fp64"] is True and "gfx950" in found[0]["driver"]
    assert cli.main(["devices"]) == 0  # hip is the default API; plain text
    assert "GPU" in capsys.readouterr().out


@pytest.mark.parametrize("dtype,size", [("float32", 128), ("float64", 257)])
def test_benchmark_report_on_hip(hip, tmp_path, capsys, dtype, size):
    path = tmp_path / "report.json"
    argv = ["benchmark", "--backend", "hip", "--size", str(size), "--repeat", "3", "--dtype", dtype,
            "--output", str(path)]
    assert cli.main(argv) == 0
    report = json.loads(path.read_text())
    assert json.loads(capsys.readouterr().out) == report
    assert report["schema_version"] == 1 and report["backend"] == "hip" and report["all_valid"]
    assert report["device"] == hip.device and report["versions"]["pacho_hip"].startswith("pacho_hip")
    for case in report["cases"]:
        assert case["valid"] and len(case["resident_seconds"]) == 3 and case["resident_median_seconds"] > 0
