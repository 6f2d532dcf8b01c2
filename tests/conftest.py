"""Shared test setup.

Markers: ``gpu`` = needs an MI355X (runs the HIP kernels through the C ABI).
CPU tests cover the oracle against the reference's golden vectors, the host
logic, and that the C-ABI library loads and exports every declared symbol.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "ref_ops.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the gfx950 kernels")


def close(got, ref, atol, rtol):
    """The reference's GPU parity gate (tests/test_cuda.c:17-26):
    max|got - ref| <= atol + rtol * max|ref|. Returns (ok, maxdiff, threshold)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    md = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    thr = atol + rtol * (float(np.max(np.abs(ref))) if ref.size else 0.0)
    return md <= thr, md, thr


def assert_close(got, ref, atol, rtol, what=""):
    ok, md, thr = close(got, ref, atol, rtol)
    assert ok, f"{what}: maxdiff {md:.3e} > threshold {thr:.3e}"


def relerr_max(got, ref):
    """max|got - ref| / max|ref| (tests/test_quant.c:30-35)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    mr = float(np.max(np.abs(ref)))
    md = float(np.max(np.abs(got - ref)))
    return md / mr if mr > 0 else md


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def port():
    import oracle
    return oracle.port()


@pytest.fixture(scope="session")
def ref():
    import oracle
    return oracle.ref()


@pytest.fixture(scope="session")
def hip():
    """The HIP backend; a gpu test fails (never skips) when the library or device is missing."""
    import aria_amd
    L = aria_amd.lib()
    assert L.aria_cuda_available() == 1, f"no HIP device: {aria_amd.last_error()}"
    print(f"[gpu] {aria_amd.device_info()}", flush=True)
    return aria_amd


def rng(seed):
    return np.random.default_rng(seed)


def randn(r, shape, sigma=1.0):
    return (sigma * r.standard_normal(shape)).astype(np.float32)
