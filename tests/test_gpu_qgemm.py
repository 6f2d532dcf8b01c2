"""GPU parity of the Q8/Q4 dequant-on-use GEMM (k_qgemm.hip) through the C ABI.

Gate: max|y_gpu - y_ref| <= 1e-3 * max|y_ref| against the reference's own
dequantized fp32 GEMM (aria_linear_q8 / aria_linear_q4 outputs in the golden file, or the
oracle restatement of them). At the full config-3 shapes the check is against a float64 matmul
with the dequantized weights (size-independent: same gate), plus an oracle subset of rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import randn, relerr_max, rng

pytestmark = pytest.mark.gpu

GATE = 1e-3


@pytest.fixture(scope="module")
def ops(hip):
    from aria_amd import ops as O
    return O


@pytest.mark.parametrize("name", ["a", "b", "c", "d"])
def test_qgemm_golden(ops, golden, name):
    g = golden
    x, b = g[f"qw{name}_x"], g[f"qw{name}_b"]
    e8 = relerr_max(ops.linear_q8(x, g[f"qw{name}_q8"], g[f"qw{name}_s8"], b), g[f"qw{name}_y8"])
    e4 = relerr_max(ops.linear_q4(x, g[f"qw{name}_q4"], g[f"qw{name}_s4"], b), g[f"qw{name}_y4"])
    print(f"golden {name}: q8 relerr {e8:.2e}  q4 relerr {e4:.2e}")
    assert e8 <= GATE and e4 <= GATE


@pytest.mark.parametrize("MKN", [(1, 64, 32), (33, 64, 100), (129, 96, 257), (200, 1024, 3072), (64, 4096, 1024),
                                 (130, 768, 2048), (7, 1031, 40), (3, 33, 5)])
@pytest.mark.parametrize("bias", [False, True])
def test_qgemm_shapes(ops, port, MKN, bias):
    M, K, N = MKN
    r = rng(M * 31 + K * 7 + N)
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.02); b = randn(r, N, 0.02) if bias else None
    q8, s8 = port.q8_quant(W)
    q4, s4 = port.q4_quant(W)
    e8 = relerr_max(ops.linear_q8(x, q8, s8, b), port.linear_q8(x, q8, s8, b))
    e4 = relerr_max(ops.linear_q4(x, q4, s4, b), port.linear_q4(x, q4, s4, b))
    assert e8 <= GATE and e4 <= GATE, (e8, e4)


@pytest.mark.parametrize("KN", [(1024, 4096), (4096, 1024)])
def test_qgemm_config3_full(ops, port, KN):
    """Config 3 at its full size: X [2592,K] ~N(0,1), W [N,K] ~N(0,0.02)."""
    K, N = KN
    M = 2592
    r = rng(0xA21A0000 + K)
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.02)
    q8, s8 = ops.q8_quant(W)                       # device pack (bit-exact tested elsewhere)
    q4, s4 = ops.q4_quant(W)
    y8 = ops.linear_q8(x, q8, s8)
    y4 = ops.linear_q4(x, q4, s4)
    x64 = x.astype(np.float64)
    ref8 = x64 @ (q8.astype(np.float64) * s8[:, None].astype(np.float64)).T
    ref4 = x64 @ port.q4_dequant(q4, s4, K).astype(np.float64).T
    e8, e4 = relerr_max(y8, ref8), relerr_max(y4, ref4)
    rows = np.sort(r.choice(M, 24, replace=False))
    o8 = relerr_max(y8[rows], port.linear_q8(np.ascontiguousarray(x[rows]), q8, s8))
    o4 = relerr_max(y4[rows], port.linear_q4(np.ascontiguousarray(x[rows]), q4, s4))
    print(f"K={K} N={N}: q8 {e8:.2e} (oracle rows {o8:.2e})  q4 {e4:.2e} (oracle rows {o4:.2e})")
    assert max(e8, e4, o8, o4) <= GATE


def test_qgemm_f16_activations_and_outputs(hip, port):
    """fp16 activations (what the fused norm emits) and fp16 outputs through the device API."""
    from aria_amd.device import DeviceArray, sync
    r = rng(77)
    M, K, N = 300, 1024, 768
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.02); b = randn(r, N, 0.02)
    x16 = x.astype(np.float16)
    xr = x16.astype(np.float32)
    L = hip.lib()
    for wtype, (q, s) in ((0, port.q8_quant(W)), (1, port.q4_quant(W))):
        want = port.linear_q8(xr, q, s, b) if wtype == 0 else port.linear_q4(xr, q, s, b)
        dx, dq, ds, db = (DeviceArray.from_host(a) for a in (x16, q, s, b))
        dy = DeviceArray((M, N), np.float32)
        dy16 = DeviceArray((M, N), np.float16)
        hip.check(L.aria_hip_qlinear_dev(dy.p, 0, dx.p, 1, wtype, dq.p, ds.p, db.p, M, K, N, None))
        hip.check(L.aria_hip_qlinear_dev(dy16.p, 1, dx.p, 1, wtype, dq.p, ds.p, db.p, M, K, N, None))
        sync()
        assert relerr_max(dy.to_host(), want) <= GATE
        assert relerr_max(dy16.to_host().astype(np.float32), want) <= 2e-3
    # fp16 weights (the unquantized projections)
    W16 = W.astype(np.float16)
    want = xr.astype(np.float64) @ W16.astype(np.float64).T + b
    dx, dw, db = DeviceArray.from_host(x16), DeviceArray.from_host(W16), DeviceArray.from_host(b)
    dy = DeviceArray((M, N), np.float32)
    hip.check(L.aria_hip_qlinear_dev(dy.p, 0, dx.p, 1, 2, dw.p, None, db.p, M, K, N, None))
    sync()
    assert relerr_max(dy.to_host(), want) <= 1e-5


def test_qgemm_identity_weights(ops, port):
    """Identity weights pin the operand order and the per-row scale: y = x * 127*scale."""
    r = rng(78)
    K = 256
    x = randn(r, (70, K))
    I = (np.eye(K, dtype=np.float32) * 0.5)
    q8, s8 = port.q8_quant(I)
    y = ops.linear_q8(x, q8, s8)
    assert np.allclose(y, x * np.float32(127 * s8[0]), rtol=2e-3, atol=1e-3)
    # a permutation matrix: y[:, n] = x[:, perm[n]] (transposed operands would fail this)
    perm = r.permutation(K)
    P = np.zeros((K, K), np.float32); P[np.arange(K), perm] = 1.0
    q4, s4 = port.q4_quant(P)
    y = ops.linear_q4(x, q4, s4)
    assert relerr_max(y, x[:, perm]) <= GATE


@pytest.mark.parametrize("tiles", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12])
@pytest.mark.parametrize("wtype", [0, 1])
def test_qgemm_every_tile_shape(hip, port, tiles, wtype):
    """Each workgroup tile shape, with ragged M and N edges, fp32 and fp16 activations."""
    from aria_amd.device import DeviceArray, sync
    r = rng(90 + tiles * 2 + wtype)
    M, K, N = 197, 384, 136
    x = randn(r, (M, K)); W = randn(r, (N, K), 0.02); b = randn(r, N, 0.02)
    q, s = port.q8_quant(W) if wtype == 0 else port.q4_quant(W)
    L = hip.lib()
    for xf16 in (0, 1):
        xin = x.astype(np.float16) if xf16 else x
        xr = xin.astype(np.float32)
        want = port.linear_q8(xr, q, s, b) if wtype == 0 else port.linear_q4(xr, q, s, b)
        dx, dq, ds, db = (DeviceArray.from_host(a) for a in (xin, q, s, b))
        dy = DeviceArray((M, N), np.float32)
        hip.check(L.aria_hip_qlinear_ex_dev(dy.p, 0, dx.p, xf16, wtype, dq.p, ds.p, db.p, M, K, N, tiles, None))
        sync()
        assert relerr_max(dy.to_host(), want) <= GATE, (tiles, wtype, xf16)


@pytest.mark.parametrize("wtype,tiles", [(w, t) for w in (0, 1) for t in range(13, 22)] +
                         [(2, t) for t in range(13, 18)])
def test_qgemm_lds_dma_tiles(hip, port, tiles, wtype):
    """The LDS-DMA kernel's tile configurations (tiles 13.. = configuration tiles - 13; nine
    for Q8/Q4, two with the K range split inside the workgroup and the last two with 8 waves
    over 256 or 512 weight rows, and five for fp16 weights, some in two pipeline stages) with
    ragged M and N edges, fp16 activations; fp16 weights against the float64 product of the
    same fp16 values."""
    from aria_amd.device import DeviceArray, sync
    r = rng(140 + tiles * 3 + wtype)
    M, K, N = 197, 384, 136
    x = randn(r, (M, K)).astype(np.float16); W = randn(r, (N, K), 0.05); b = randn(r, N, 0.02)
    if wtype == 2:
        q, s = W.astype(np.float16), None
        want = (x.astype(np.float64) @ q.astype(np.float64).T + b).astype(np.float32)
    else:
        q, s = port.q8_quant(W) if wtype == 0 else port.q4_quant(W)
        xr = x.astype(np.float32)
        want = port.linear_q8(xr, q, s, b) if wtype == 0 else port.linear_q4(xr, q, s, b)
    L = hip.lib()
    dx, dq, db = (DeviceArray.from_host(a) for a in (x, q, b))
    ds = DeviceArray.from_host(s) if s is not None else None
    dy = DeviceArray((M, N), np.float32)
    hip.check(L.aria_hip_qlinear_ex_dev(dy.p, 0, dx.p, 1, wtype, dq.p, ds.p if ds else None, db.p, M, K, N,
                                        tiles, None))
    sync()
    assert relerr_max(dy.to_host(), want) <= GATE, (tiles, wtype)


@pytest.mark.parametrize("wtype,tiles,MKN", [(2, 13, (5000, 768, 4608)), (0, 13, (2592, 1024, 1024)),
                                             (1, 14, (2592, 1024, 3072)), (1, 16, (2592, 1024, 4096)),
                                             (0, 17, (2592, 1024, 8192)), (1, 18, (2592, 4096, 1024)),
                                             (1, 20, (2592, 1024, 4096)), (0, 21, (2592, 1024, 3072))])
def test_qgemm_lds_dma_repeatable(hip, port, wtype, tiles, MKN):
    """Repeated launches of the LDS-DMA kernel on the same inputs give the same bits. Its
    pipeline overwrites a stage by DMA one step after the stage was read, so an LDS read still
    in flight at the step's barrier would let the next DMA change a fragment under it: seen as
    one 32 x 32 block wrong in about one launch in four at the first shape before every
    fragment read was waited for ahead of the barrier."""
    from aria_amd.device import DeviceArray, sync
    M, K, N = MKN
    r = rng(170 + wtype)
    x = randn(r, (M, K)).astype(np.float16); W = randn(r, (N, K), 1.0 / np.sqrt(K))
    if wtype == 2:
        q, s = W.astype(np.float16), None
    else:
        q, s = port.q8_quant(W) if wtype == 0 else port.q4_quant(W)
    L = hip.lib()
    dx, dq = DeviceArray.from_host(x), DeviceArray.from_host(q)
    ds = DeviceArray.from_host(s) if s is not None else None
    dy = DeviceArray((M, N), np.float32)
    first = None
    for rep in range(6):
        hip.check(L.aria_hip_qlinear_ex_dev(dy.p, 0, dx.p, 1, wtype, dq.p, ds.p if ds else None, None, M, K, N,
                                            tiles, None))
        sync()
        y = dy.to_host()
        if first is None:
            first = y
            if wtype == 2:
                rows = np.arange(0, M, 97)
                want = x[rows].astype(np.float64) @ q.astype(np.float64).T
                assert relerr_max(y[rows], want) <= GATE
        else:
            assert np.array_equal(y, first), (rep, int((y != first).sum()))
