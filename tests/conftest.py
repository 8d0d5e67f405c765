"""Shared fixtures: the product package (remora-lab_amd/, loaded by path since
the directory name is not an identifier), the CPU oracle, and a device
context for tests marked `gpu`."""
from __future__ import annotations

import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_rkv():
    name = "remora_lab_amd"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "remora-lab_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def rkv():
    return load_rkv()


@pytest.fixture(scope="session")
def rko():
    from oracle import rko as mod
    mod.lib()
    return mod


@pytest.fixture(scope="session")
def ctx(rkv):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test collected on a host without a GPU")
    c = rkv.Ctx(0)
    yield c
    c.close()
