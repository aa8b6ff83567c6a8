"""pytest configuration: markers, import paths and shared fixtures.

`gpu` tests need a gfx950 device and the built libt0hip.so; everything else runs
on the CPU (the oracle, the host-side codec/container/export code, and the
C-ABI symbol checks)."""
import os
import sys

import numpy as np
import pytest
# torch carries its own HIP/HSA runtime beside the system ROCm one libt0hip.so
# links; both coexist in one process when torch's libraries are loaded and its
# runtime initialized before libt0hip.so initializes HIP (the engine fixture
# below asks for torch_cuda first), the order bench.py uses too.
import torch  # noqa: F401

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "t0-web_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libt0hip.so")


@pytest.fixture(scope="session")
def oracle():
    import t0ref
    t0ref.lib()
    return t0ref


@pytest.fixture(scope="session")
def t0hip():
    import t0hip as m
    m.lib()
    return m


@pytest.fixture(scope="session")
def engine(t0hip, torch_cuda):
    return t0hip.Engine(0)


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible GPU")
    return torch


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
