import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built library")


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def torch():
    """The 'hip' package, initialised on device 0 (GPU tests only)."""
    import __graft_entry__ as ge
    t = ge.load_package()
    t.init(0)
    return t


@pytest.fixture(scope="session")
def pkg():
    """The package without device init (CPU tests)."""
    import __graft_entry__ as ge
    return ge.load_package()
