import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "vllm-lite_amd")
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def load_package():
    """Imports the vllm-lite_amd directory as the package `vllm_lite_amd`."""
    if "vllm_lite_amd" in sys.modules:
        return sys.modules["vllm_lite_amd"]
    spec = importlib.util.spec_from_file_location(
        "vllm_lite_amd", os.path.join(PKG_DIR, "__init__.py"),
        submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["vllm_lite_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libpa.so on cuda:0)")


@pytest.fixture(scope="session")
def pa():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.load()
    return o
