import os
import sys

import pytest

try:
    # torch (used by the decode-driver tests) loads its own HIP runtime; a
    # process can use only one, so torch comes first, before any test loads
    # libarm_ai_amd.so, which then binds to the same runtime.
    import torch  # noqa: F401
except ImportError:  # pragma: no cover
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def ctx():
    """One library context on device 0 for the whole GPU session."""
    import arm_ai_amd as A

    c = A.Context(0)
    yield c
    c.close()
