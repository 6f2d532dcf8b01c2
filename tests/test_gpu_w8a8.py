"""GPU parity of the W8A8 path (k_gemm_i8.hip: per-row int8 activation quantisation and the
int8 MFMA GEMM) through the C ABI.

Gate: bit-identical to the oracle's or_linear_q8a8 / or_quant_act_q8, which tests/test_oracle.py
pins bit for bit to the compiled reference aria_linear_q8a8 (src/aria_quant.c:253-345) on the
reference's own W8A8 shapes (tests/test_quant.c:146). Shapes cover every tile configuration
(N <= 1024, <= 3072, <= 4096 and wider), ragged M / N edges, the SIMT form (K % 64 != 0, K % 4 != 0),
zero rows (amax == 0) and the full config-3 sizes (checked on a subset of rows: the
quantisation is per row).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import randn, rng

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ops(hip):
    from aria_amd import ops as O
    return O


SHAPES = [(1, 32, 1), (3, 64, 2), (4, 96, 3), (5, 100, 4), (7, 1030, 7), (9, 1024, 13), (12, 256, 6),
          (1, 64, 4), (33, 128, 260), (64, 64, 256), (130, 1024, 1000), (200, 1024, 3072), (64, 4096, 1024),
          (97, 512, 512), (197, 256, 4100), (197, 256, 3500)]


@pytest.mark.parametrize("MKN", SHAPES)
@pytest.mark.parametrize("bias", [False, True])
def test_w8a8_shapes(ops, port, MKN, bias):
    M, K, N = MKN
    print(f"w8a8 M={M} K={K} N={N} bias={bias}", flush=True)
    r = rng(M * 131 + K * 7 + N)
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.1); b = randn(r, N) if bias else None
    if M > 2:
        x[M // 2] = 0.0                                   # amax == 0: sx = 0, xq = 0
    q, s = port.q8_quant(W)
    y = ops.linear_q8a8(x, q, s, b)
    want = port.linear_q8a8(x, q, s, b)
    bad = np.flatnonzero(bits(y) != bits(want))
    assert bad.size == 0, (bad.size, y.ravel()[bad[:4]], want.ravel()[bad[:4]])


@pytest.mark.parametrize("KN", [(1024, 4096), (4096, 1024), (1024, 3072)])
def test_w8a8_config3_full(ops, port, KN):
    """Config-3 sizes, M = 2592 rows (the largest tile height): every row against the int64
    sums' closed form is too slow on the host, so a row subset against the oracle."""
    K, N = KN
    M = 2592
    print(f"w8a8 full M={M} K={K} N={N}", flush=True)
    r = rng(0xA8A80000 + K + N)
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.02); b = randn(r, N, 0.02)
    q, s = port.q8_quant(W)
    y = ops.linear_q8a8(x, q, s, b)
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 63, 64, 95, 96, 127, 128, M - 1],
                                     r.choice(M, 40, replace=False)]))
    want = port.linear_q8a8(np.ascontiguousarray(x[rows]), q, s, b)
    assert np.array_equal(bits(y[rows]), bits(want))


@pytest.mark.parametrize("K", [256, 1024, 1031, 2048, 3072, 4096, 5000, 8192])
@pytest.mark.parametrize("f16", [0, 1])
def test_quant_act_q8_rows(hip, port, K, f16):
    """The activation quantiser on both of its row mappings (one wave per row; one workgroup
    per row for 2048 <= K <= 8192, K % 1024 == 0) and its scalar forms, fp32 and fp16 input:
    int8 rows and scales bit-identical to or_quant_act_q8, with a zero row and rows whose
    maximum sits in the first or the last element."""
    from aria_amd.device import DeviceArray, sync
    L = hip.lib()
    r = rng(4000 + K + f16)
    M = 37
    x = randn(r, (M, K))
    x[3] = 0.0
    x[5, 0] = 50.0
    x[6, K - 1] = -60.0
    xin = x.astype(np.float16) if f16 else x
    xq_want, sx_want = port.quant_act_q8(np.ascontiguousarray(xin, np.float32))
    dx = DeviceArray.from_host(xin)
    dxq, dsx = DeviceArray((M, K), np.int8), DeviceArray((M,), np.float32)
    hip.check(L.aria_hip_quant_act_q8_dev(dxq.p, dsx.p, dx.p, f16, M, K, None))
    sync()
    assert np.array_equal(dxq.to_host(), xq_want)
    assert np.array_equal(bits(dsx.to_host()), bits(sx_want))


def test_w8a8_device_api(hip, port):
    """fp16 activations (what the fused norms emit), fp16 outputs, and the composite entry
    with caller workspace, through the device-pointer ABI."""
    from aria_amd.device import DeviceArray, sync
    L = hip.lib()
    r = rng(91)
    M, K, N = 300, 1024, 768
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.1); b = randn(r, N)
    x[7] = 0.0
    q, s = port.q8_quant(W)
    x16 = x.astype(np.float16)
    xr = x16.astype(np.float32)                            # the half's exact value
    xq_want, sx_want = port.quant_act_q8(xr)
    dx16, dq, ds, db = (DeviceArray.from_host(a) for a in (x16, q, s, b))
    dxq = DeviceArray((M, K), np.int8)
    dsx = DeviceArray((M,), np.float32)
    hip.check(L.aria_hip_quant_act_q8_dev(dxq.p, dsx.p, dx16.p, 1, M, K, None))
    sync()
    assert np.array_equal(dxq.to_host(), xq_want) and np.array_equal(bits(dsx.to_host()), bits(sx_want))
    want = port.linear_q8a8(xr, q, s, b)
    dy = DeviceArray((M, N), np.float32)
    dy16 = DeviceArray((M, N), np.float16)
    hip.check(L.aria_hip_gemm_i8_dev(dy.p, 0, dxq.p, dsx.p, dq.p, ds.p, db.p, M, K, N, None))
    hip.check(L.aria_hip_gemm_i8_dev(dy16.p, 1, dxq.p, dsx.p, dq.p, ds.p, db.p, M, K, N, None))
    sync()
    assert np.array_equal(bits(dy.to_host()), bits(want))
    assert np.array_equal(dy16.to_host().view(np.uint16), want.astype(np.float16).view(np.uint16))
    # composite with workspace, fp32 activations, no bias (+ 0.0f)
    ws = int(L.aria_hip_q8a8_ws_bytes(M, K))
    assert ws >= M * K + 4 * M
    dws = DeviceArray((ws,), np.uint8)
    dx = DeviceArray.from_host(x)
    hip.check(L.aria_hip_linear_q8a8_dev(dy.p, dx.p, 0, dq.p, ds.p, None, M, K, N, dws.p, None))
    sync()
    assert np.array_equal(bits(dy.to_host()), bits(port.linear_q8a8(x, q, s, None)))
    # empty shapes are no-ops
    hip.check(L.aria_hip_linear_q8a8_dev(dy.p, dx.p, 0, dq.p, ds.p, None, 0, K, N, dws.p, None))
    hip.check(L.aria_hip_gemm_i8_dev(dy.p, 0, dxq.p, dsx.p, dq.p, ds.p, None, M, K, 0, None))


def test_rmsnorm_q8_fused(hip, port):
    """The W8A8 producers: RMSNorm(w) (-> adaLN, per-batch modulation) quantised in registers,
    against the oracle's fp32 norm composition then or_quant_act_q8. The fp32 norm matches the
    oracle to the last bit on nearly every element (test_gpu_ops), so the int8 rows and scales
    agree except where a 1-ulp difference crosses a rounding boundary or moves the row max."""
    from aria_amd.device import DeviceArray, sync
    L = hip.lib()
    r = rng(41)
    B, S, D = 2, 75, 1024
    x = randn(r, (B * S, D)); w = (1 + randn(r, D, 0.02)).astype(np.float32)
    sc = randn(r, (B, D), 0.1); sh = randn(r, (B, D), 0.1)
    x[3] = 0.0                                             # zero row: sx 0, xq 0
    dx, dw, dsc, dsh = (DeviceArray.from_host(a) for a in (x, w, sc, sh))
    dq = DeviceArray((B * S, D), np.int8)
    ds = DeviceArray((B * S,), np.float32)
    for mod in (True, False):
        hip.check(L.aria_hip_rmsnorm_adaln_q8_dev(dq.p, ds.p, dx.p, dw.p, dsc.p if mod else None,
                                                  dsh.p if mod else None, B * S, D, S, 1e-5, None))
        sync()
        y = np.concatenate([port.adaln_modulate(port.rmsnorm(x[b * S:(b + 1) * S], w, 1e-5), sc[b], sh[b])
                            if mod else port.rmsnorm(x[b * S:(b + 1) * S], w, 1e-5) for b in range(B)])
        xq, sx = port.quant_act_q8(np.ascontiguousarray(y, np.float32))
        gq, gs = dq.to_host(), ds.to_host()
        assert np.mean(gq == xq) > 0.9999 and np.abs(gq.astype(np.int32) - xq).max() <= 1, mod
        assert np.mean(bits(gs) == bits(sx)) > 0.97 and np.allclose(gs, sx, rtol=1e-6, atol=0), mod
        if not mod:                                        # (with adaLN the zero row becomes shift)
            assert gs[3] == 0.0 and np.all(gq[3] == 0)
    assert L.aria_hip_rmsnorm_adaln_q8_dev(dq.p, ds.p, dx.p, dw.p, None, None, B * S, 100, 0, 1e-5, None) == -1
