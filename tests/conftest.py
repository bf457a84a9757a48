"""Shared fixtures. Tiers:

- default (CPU): oracle pinning against published/golden vectors, facade and
  plan behaviour on the NumPy backend, C-ABI symbol exports, RTC source checks;
- ``-m gpu``: parity of the hip backend (libpacho_hip.so on an MI355X) against
  the oracles, through the C ABI. On a GPU run a hip backend that cannot be
  created FAILS the test (no silent skip), unless PACHO_REQUIRE_HIP=0.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "open-pacho_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libpacho_hip.so")


@pytest.fixture(scope="session")
def hip():
    import openpacho as pacho
    from openpacho.exceptions import BackendUnavailableError

    try:
        backend = pacho.get_backend("hip", device=os.environ.get("PACHO_HIP_DEVICE") or None)
    except (BackendUnavailableError, ImportError, OSError) as exc:
        if os.environ.get("PACHO_REQUIRE_HIP", "1") == "0":
            pytest.skip(f"hip unavailable: {exc}")
        pytest.fail(f"hip backend unavailable on a GPU test run: {exc}")
    yield backend
    backend.synchronize()


@pytest.fixture
def numpy_backend():
    import openpacho as pacho

    return pacho.get_backend("numpy")
