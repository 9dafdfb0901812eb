import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "continuous-batching-inference-server_amd")
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


def load_cbis():
    if "cbis" in sys.modules:
        return sys.modules["cbis"]
    spec = importlib.util.spec_from_file_location("cbis", os.path.join(PKG, "cbis.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["cbis"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def cbis():
    return load_cbis()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a GPU")
    torch.cuda.init()
    return torch.device("cuda:0")
