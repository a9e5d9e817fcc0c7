"""Shared fixtures.  CPU tests (`-m "not gpu"`) cover the oracle, the golden vectors, the
host-side validation and the library's exported symbols; GPU tests (`-m gpu`) compare the
HIP path, called through the C ABI, with the oracle."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_pkg():
    """Import moe-680m_amd/ (a directory name that is not an identifier) by path."""
    if "moe680m_amd" in sys.modules:
        return sys.modules["moe680m_amd"]
    pkg_dir = os.path.join(ROOT, "moe-680m_amd")
    spec = importlib.util.spec_from_file_location(
        "moe680m_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["moe680m_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def gpu(pkg):
    """The package with a usable GPU.  A GPU test on a machine whose library is missing
    or whose GPU is absent fails (it is never silently skipped on the GPU box)."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    pkg.lib()
    return pkg
