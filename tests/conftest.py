"""Test configuration: the ``gpu`` marker and package loading.

The package directory ``hetero-cp-ringattn_amd`` is not a valid Python identifier, so it
is loaded under the module name ``hcp_ring_amd``.
"""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "hetero-cp-ringattn_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def _load_pkg():
    if "hcp_ring_amd" in sys.modules:
        return sys.modules["hcp_ring_amd"]
    spec = importlib.util.spec_from_file_location(
        "hcp_ring_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["hcp_ring_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


_load_pkg()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def hcp():
    mod = _load_pkg()
    if not os.path.exists(mod.LIB_PATH):
        spec = importlib.util.spec_from_file_location("hcp_build", os.path.join(PKG_DIR, "build.py"))
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build()
    return mod


@pytest.fixture(scope="session")
def gpu(hcp):
    """The HIP library with a usable device (tests marked gpu only)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    torch.cuda.init()
    return hcp
