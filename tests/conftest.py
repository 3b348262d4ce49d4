"""pytest configuration: the `gpu` marker and loaders for the package (whose
directory name is not an importable identifier) and the oracle."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "qwen3.8-flash-next_amd")
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def load_pkg():
    if "qmoe_amd" in sys.modules:
        return sys.modules["qmoe_amd"]
    spec = importlib.util.spec_from_file_location(
        "qmoe_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qmoe_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    from oracle import oracle as orc  # noqa: E402
    return orc


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    return load_oracle()


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.skip("no HIP device")
    import torch
    torch.cuda.init()
    return torch.device("cuda:0")
