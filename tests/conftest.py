import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "suzuqu-engine-4exp_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def oracle():
    import oracle_ffi

    return oracle_ffi.Oracle()


@pytest.fixture(scope="session")
def rt():
    import q4kv

    r = q4kv.Runtime()
    yield r
    r.free_all()
