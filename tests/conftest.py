"""Shared test setup.

- Registers the `gpu` marker: tests that need an MI355X (gfx950) GPU.
- Loads the package directory `cuvs-silicon_amd/` as module `cuvs_silicon_amd`
  (the directory name is not an importable identifier).
"""
from __future__ import annotations

import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "cuvs-silicon_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_package():
    name = "cuvs_silicon_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def cvs():
    return load_package()


@pytest.fixture(scope="session")
def ctx(cvs):
    c = cvs.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    return o
