"""Shared pytest setup: the `gpu` marker, package/oracle loaders and fixtures.

`-m "not gpu"` tests run anywhere (they never touch a GPU); `-m gpu` tests need
an MI355X and the prebuilt libcmk_iq2.so.
"""

import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "candelora-metal-kernels_amd")
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


def load_package():
    name = "candelora_metal_kernels_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def inputs():
    return load_package().inputs


@pytest.fixture(scope="session")
def cabi():
    return load_package().cabi


@pytest.fixture(scope="session")
def pkg():
    return load_package()
