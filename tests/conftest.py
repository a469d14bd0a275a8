"""Shared pytest setup: the `gpu` marker, import paths, and lazily-built fixtures.

`-m "not gpu"` tests run on any host (oracle vs golden vectors, host logic, the C-ABI exports);
`-m gpu` tests call the HIP backend through the C ABI on a gfx950 device and compare with the
oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "e2.c_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP backend")


@pytest.fixture(scope="session")
def oracle():
    from oracle.binding import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.binding import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built (the reference tree is absent on this host)")
    return Ref()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import e2mi
    e2mi.load()  # raises if the HIP backend is missing: no silent fallback
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)


def assert_f32_close(got, want, rtol=1e-4, atol=1e-6, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want) / (np.abs(want) + atol / rtol)
    worst = float(err.max()) if err.size else 0.0
    assert worst <= rtol, f"{what}: max rel err {worst:.3g} > {rtol}"


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
