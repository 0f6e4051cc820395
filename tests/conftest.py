"""Shared fixtures. CPU tests run anywhere; tests marked `gpu` need a gfx950 device."""
from __future__ import annotations

import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

PKG_NAME = "qgemm_perf_framework_ng_amd"
PKG_DIR = os.path.join(REPO, "qgemm-perf-framework-ng_amd")


def load_package():
    """Import the package directory (its name carries hyphens) as qgemm_perf_framework_ng_amd."""
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(
        PKG_NAME, os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run on the MI355X box)")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="session")
def hip(pkg, torch_gpu):
    """The HIP library on a verified gfx950 device."""
    arch, cus = pkg.device_check()
    print(f"\n[pfng] device {arch} with {cus} CUs, {pkg.version()}", flush=True)
    return pkg
