import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def pkg():
    """The product package (``sparse-attention-vggt_amd``), loaded under its import name."""
    import __graft_entry__
    return __graft_entry__.package()


@pytest.fixture(scope="session", autouse=True)
def fixed_walk_order(pkg):
    """Tests run the attention kernel in the fixed key-walk order (run-to-run identical output);
    tests of the paced order ask for it explicitly."""
    from importlib import import_module
    ops = import_module(pkg.__name__ + ".ops")
    ops.set_walk_order("fixed")
    yield
    ops.set_walk_order("paced")
