"""Shared test fixtures.

`oracle` is the CPU checker (oracle/oracle.py over oracle/liboracle.so);
`qw` is the ctypes binding of the HIP library under test.  GPU tests are
marked `gpu` and run only on the MI355X box.
"""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen3.5_0.8b_deploy_amd")
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def qw():
    return _load("qw", os.path.join(PKG, "qw.py"))


@pytest.fixture(scope="session")
def ctx(qw):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = qw.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def rel_err(got, ref):
    """Normwise max relative error: max|got-ref| / max|ref|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def relerr():
    return rel_err
