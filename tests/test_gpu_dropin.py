"""GPU: the reference's own device parity program, tests/test_cuda.c, unchanged, linked
against libaria_hip.so in place of the CUDA backend (oracle/Makefile `dropin`), run on the
MI355X. It compares every op of the reference GPU ABI (src/aria_gpu.h:38-61: linear,
matmul, rmsnorm, gemma_rmsnorm, dynamic_tanh, softcap, silu, gelu_tanh, silu_gate, softmax
with mask, rope_apply, attention, conv1d) with the reference's CPU ops at its own
tolerances (tests/test_cuda.c:17-26, 35-112) and exits non-zero on any failure."""
from __future__ import annotations

import os
import subprocess

import pytest

import oracle

pytestmark = pytest.mark.gpu


def test_reference_test_cuda_passes_on_backend(hip):
    exe = os.path.join(oracle.DROPIN, "test_cuda_hip")
    assert os.path.exists(exe), "oracle/_ref/dropin/test_cuda_hip missing: build() where the reference is present"
    print("[gpu] running the reference's tests/test_cuda.c against libaria_hip.so", flush=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(out.stdout, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    lines = [ln for ln in out.stdout.splitlines() if ln.startswith(("ok", "FAIL"))]
    assert len(lines) == 17 and all(ln.startswith("ok") for ln in lines), out.stdout
    assert "test_cuda: OK" in out.stdout
