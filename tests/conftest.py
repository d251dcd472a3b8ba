import json
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

# Load torch's HIP runtime before libgollek_hip.so (same SONAME): the tests
# then run against the runtime bench.py uses, which imports torch first.
try:
    import torch  # noqa: F401
except Exception:  # pragma: no cover - torch is optional for the CPU suite
    torch = None

GOLDEN = REPO / "tests" / "golden" / "reference_fixtures.json"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    return json.loads(GOLDEN.read_text())


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False
