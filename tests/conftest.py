"""Shared test plumbing: the `gpu` marker, the FP32 parity criterion, device helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# FP32 parity bar: |gpu - ref| <= ATOL + RTOL * |ref| elementwise (relative 1e-4,
# absolute 1e-5 near zero), against the oracle's restatement of the reference kernels.
RTOL = 1e-4
ATOL = 1e-5


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu)")


def fp32_violations(got, ref, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    bad = d > atol + rtol * np.abs(ref)
    return int(bad.sum()), float(d.max(initial=0.0))


def assert_fp32_close(got, ref, what="", rtol=RTOL, atol=ATOL):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    assert np.isfinite(got).all() == np.isfinite(ref).all() or np.array_equal(np.isnan(got), np.isnan(ref)), what
    nbad, dmax = fp32_violations(got, ref, rtol, atol)
    assert nbad == 0, (f"{what}: {nbad} of {got.size} elements outside |d| <= {atol} + {rtol}*|ref| "
                       f"(max |d| = {dmax:.3e})")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from onnxsharp_amd import native
    info = native.DeviceInfo()
    native.call("osh_init", 0, info)
    return torch.device("cuda", 0)
