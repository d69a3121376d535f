import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run on the GPU box")


@pytest.fixture(scope="session")
def ctx():
    """One library context for the whole GPU session (one process, one GPU)."""
    from ingot_amd._lib import Context

    c = Context(0)
    yield c
    c.close()
