import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def native_lib():
    """The built HIP library (built here only if nothing is built yet)."""
    from welder_typical_chain_amd import _lib
    if not _lib.LIB_PATH.exists():
        from welder_typical_chain_amd import build
        build.build()
    return _lib.lib()
