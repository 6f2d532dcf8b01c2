"""Element-wise GPU checks of the decoder's two fused GEMM epilogues (qgemm_dev.h), called
through the library's internal launcher aria_k_qgemm_e with fp16 weights:

* DYT_ROPE (the to_qkv projection of the small-music decoder, src/aria_taae.c:120-127): the
  output columns are five sections of heads x 64 (q | k | v | qd | kd); q and qd become
  tanh(alpha_q y) * g_q[d] + b_q[d], k and kd tanh(alpha_k y) * g_k[d] + b_k[d] (d the dim within
  the head), then rotate-half RoPE over the first `rot` dims at position m % S; v is stored as it
  is. Checked at rot 0, 8, 16 and 32, a ragged M, and a sequence length S that does not divide M.
* ADD_DYT (to_out / ff_out): y += x W^T + b in place, and dst = half(tanh(alpha y) * g[c] + b2[c])
  of the new y.

The reference is a float64 restatement on the same fp16 operands (numpy matmul, numpy tanh,
the rotation of aria_rope_apply, src/aria_cpu.c:790-809). A wrong rotation partner, table
row or section kind moves values by O(1); the gates below are four orders tighter.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import randn, rng

pytestmark = pytest.mark.gpu

ARIA_WF16, EPI_ADD_DYT, EPI_DYT_ROPE = 2, 5, 6


class Epi(C.Structure):
    """aria_qgemm_epi (aria_amd/csrc/aria_hip_kernels.h)"""
    _fields_ = [("mode", C.c_int), ("rows_per_batch", C.c_int),
                ("gate", C.c_void_p), ("add2", C.c_void_p), ("gate2", C.c_void_p),
                ("gate_bs", C.c_int), ("gate2_bs", C.c_int),
                ("heads", C.c_int), ("nsec", C.c_int), ("kind", C.c_int * 3),
                ("dst", C.c_void_p * 3), ("w", C.c_void_p * 4),
                ("cos_t", C.c_void_p), ("sin_t", C.c_void_p),
                ("rot", C.c_int), ("eps", C.c_float), ("eps2", C.c_float)]


def _launcher(hip):
    f = hip.lib().aria_k_qgemm_e
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                  C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(Epi), C.c_void_p]
    return f


def _rope_tables(S, rot):
    rh = max(rot // 2, 1)
    inv = 1.0 / (10000.0 ** (np.arange(rh) * 2.0 / max(rot, 2)))
    ang = np.arange(S)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _dyt_rope_ref(y, S, heads, rot, aq, gq, bq, ak, gk, bk, cos_t, sin_t):
    """float64 restatement of the DYT_ROPE epilogue on y = x W^T [M, 5 heads 64]"""
    M = y.shape[0]
    out = y.copy()
    pos = np.arange(M) % S
    for sec in range(5):
        if sec == 2:
            continue
        a, g, b = (aq, gq, bq) if sec in (0, 3) else (ak, gk, bk)
        for h in range(heads):
            c0 = (sec * heads + h) * 64
            t = np.tanh(a * y[:, c0:c0 + 64]) * g[None, :] + b[None, :]
            if rot > 0:
                rh = rot // 2
                cs, sn = cos_t[pos].astype(np.float64), sin_t[pos].astype(np.float64)
                x1, x2 = t[:, :rh].copy(), t[:, rh:rot].copy()
                t[:, :rh] = x1 * cs - x2 * sn
                t[:, rh:rot] = x2 * cs + x1 * sn
            out[:, c0:c0 + 64] = t
    return out


@pytest.mark.parametrize("rot", [0, 8, 16, 32])
@pytest.mark.parametrize("tiles", [0, 13, 4])
def test_dyt_rope_epilogue(hip, rot, tiles):
    """tiles 0: the configuration picked for the shape (the LDS-DMA kernel), 13: its 64 x 128
    tile, 4: the LDS-operand kernel's 96 x 128"""
    from aria_amd.device import DeviceArray
    L = hip.lib()
    st = L.aria_hip_default_stream()
    r = rng(700 + rot + tiles)
    M, K, heads, S = 197, 128, 2, 34         # 197 = 5 x 34 + 27: positions wrap inside tiles
    N = 5 * heads * 64
    x = randn(r, (M, K)).astype(np.float16)
    W = randn(r, (N, K), 1.0 / np.sqrt(K)).astype(np.float16)
    aq, ak = 0.7, 1.3
    gq, bq = (1.0 + 0.2 * randn(r, 64)), 0.1 * randn(r, 64)
    gk, bk = (1.0 + 0.2 * randn(r, 64)), 0.1 * randn(r, 64)
    cos_t, sin_t = _rope_tables(S, rot)
    dx, dW = DeviceArray.from_host(x), DeviceArray.from_host(W)
    dgq, dbq, dgk, dbk = (DeviceArray.from_host(v.astype(np.float32)) for v in (gq, bq, gk, bk))
    dc, ds = DeviceArray.from_host(cos_t), DeviceArray.from_host(sin_t)
    dy = DeviceArray((M, N), np.float32)
    e = Epi()
    e.mode, e.rows_per_batch, e.heads = EPI_DYT_ROPE, S, heads
    e.w[0], e.w[1], e.w[2], e.w[3] = dgq.p, dbq.p, dgk.p, dbk.p
    e.eps, e.eps2 = aq, ak
    e.cos_t, e.sin_t, e.rot = dc.p, ds.p, rot
    hip.check(_launcher(hip)(dy.p, 0, dx.p, 1, ARIA_WF16, dW.p, None, None, M, K, N, tiles, 0, C.byref(e), st))
    hip.check(L.aria_hip_stream_sync(st))
    got = dy.to_host().astype(np.float64)
    y = x.astype(np.float64) @ W.astype(np.float64).T
    want = _dyt_rope_ref(y, S, heads, rot, aq, gq.astype(np.float32).astype(np.float64),
                         bq.astype(np.float32).astype(np.float64), ak, gk.astype(np.float32).astype(np.float64),
                         bk.astype(np.float32).astype(np.float64), cos_t, sin_t)
    err = np.max(np.abs(got - want))
    assert err <= 2e-5 + 2e-5 * np.max(np.abs(want)), (rot, tiles, err)


@pytest.mark.parametrize("tiles", [0, 13, 4])
def test_add_dyt_epilogue(hip, tiles):
    from aria_amd.device import DeviceArray
    L = hip.lib()
    st = L.aria_hip_default_stream()
    r = rng(800 + tiles)
    M, K, N = 197, 192, 200                  # ragged M and N
    x = randn(r, (M, K)).astype(np.float16)
    W = randn(r, (N, K), 1.0 / np.sqrt(K)).astype(np.float16)
    bias = 0.1 * randn(r, N)
    y0 = randn(r, (M, N))
    alpha = 0.8
    g, b2 = (1.0 + 0.2 * randn(r, N)), 0.1 * randn(r, N)
    dx, dW, db = DeviceArray.from_host(x), DeviceArray.from_host(W), DeviceArray.from_host(bias)
    dy = DeviceArray.from_host(y0)
    dg, db2 = DeviceArray.from_host(g), DeviceArray.from_host(b2)
    dh = DeviceArray((M, N), np.float16)
    e = Epi()
    e.mode, e.rows_per_batch = EPI_ADD_DYT, M
    e.dst[0] = dh.p
    e.w[0], e.w[1] = dg.p, db2.p
    e.eps = alpha
    hip.check(_launcher(hip)(dy.p, 0, dx.p, 1, ARIA_WF16, dW.p, None, db.p, M, K, N, tiles, 0, C.byref(e), st))
    hip.check(L.aria_hip_stream_sync(st))
    ynew = y0.astype(np.float64) + (x.astype(np.float64) @ W.astype(np.float64).T + bias.astype(np.float64))
    got_y = dy.to_host().astype(np.float64)
    assert np.max(np.abs(got_y - ynew)) <= 1e-5 + 1e-5 * np.max(np.abs(ynew)), tiles
    href = np.tanh(alpha * got_y) * g.astype(np.float64) + b2.astype(np.float64)
    got_h = dh.to_host().astype(np.float64)
    # fp16 output: within one half-precision rounding (2^-11 relative) plus tanh's few 1e-7
    assert np.all(np.abs(got_h - href) <= 2.0 ** -11 * np.abs(href) + 1e-6), tiles
