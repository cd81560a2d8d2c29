import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libzkh.so on cuda:0)")


def load_zkh():
    """Import the zk-hillclimb_amd package (hyphenated directory) as module `zkh`."""
    if "zkh" in sys.modules:
        return sys.modules["zkh"]
    path = os.path.join(ROOT, "zk-hillclimb_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location("zkh", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["zkh"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def zkh():
    return load_zkh()


@pytest.fixture(scope="session")
def ctx(zkh):
    c = zkh.Context(0)
    yield c
    c.close()
