import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen3.8-27b-mi50-cpp-engine_amd")
sys.path.insert(0, ROOT)


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


q27x = _load("q27x", os.path.join(PKG, "q27x.py"))
q27o = _load("q27o", os.path.join(ROOT, "oracle", "q27o.py"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI of libq27x.so)")


@pytest.fixture(scope="session")
def X():
    return q27x


@pytest.fixture(scope="session")
def O():
    q27o.lib()
    return q27o


@pytest.fixture(scope="session")
def gpu():
    if q27x.gpu_count() < 1:
        pytest.fail("no GPU visible to libq27x.so")
    q27x.call("q27x_set_device", 0)
    return q27x
