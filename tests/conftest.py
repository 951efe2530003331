import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "astc-kv_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs HIP kernels)")


@pytest.fixture(scope="session")
def golden():
    return GOLDEN


def pytest_report_header(config):
    return [f"astc-kv repo root: {ROOT}"]
