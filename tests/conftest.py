import importlib.util
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "kimi-k3-for-me_amd")
sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long CPU test")


def load_k3x():
    """The package's Python binding (the package directory name is not importable)."""
    spec = importlib.util.spec_from_file_location("k3x", os.path.join(PKG, "k3x.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def k3x():
    return load_k3x()


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle_lib as ol
    ol.oracle()
    return ol


@pytest.fixture(scope="session")
def ref_lib():
    import oracle_lib as ol
    r = ol.ref()
    if r is None:
        pytest.skip("compiled reference (oracle/_ref) not built: reference tree absent")
    return r


@pytest.fixture(scope="session")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU visible"
    return t
