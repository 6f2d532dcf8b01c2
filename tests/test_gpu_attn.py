"""GPU parity of the DiT attention pieces (k_attn.hip) through the C ABI.

* fused attention vs the oracle's aria_attention restatement (fp32 scores, softmax, PV) on
  the same fp16-rounded q/k/v, gate of the reference's tests/test_cuda.c:112
  (1e-3 + 1e-3*max|ref|); shapes cover the config-4 self (S = 1296) and cross (256 keys)
  attention, ragged query/key counts and the test_cuda.c shape;
* head preparation (q/k RMSNorm + RoPE, v copy) vs the oracle composition, to fp16 rounding.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, randn, rng

pytestmark = pytest.mark.gpu


def f16r(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("B,H,Nq,Nk", [(1, 8, 48, 48), (2, 16, 1296, 1296), (2, 16, 1296, 256), (1, 2, 130, 77),
                                       (2, 1, 1, 1), (1, 3, 200, 1300), (4, 16, 1024, 1024), (4, 16, 1024, 300),
                                       (1, 24, 1296, 1296)])
def test_flash_attention(hip, port, B, H, Nq, Nk):
    """Every workgroup form: the keys split in two halves (Nk >= 512) with 4 query waves per
    half (1024 x 64 heads, the small cases), 5 (1296 x 24) or 6 (1296 x 32), or one half with
    3 query waves (1296 x 32, the small cases) or 4 (1024 x 64); ragged query and key counts."""
    r = rng(B * 1000 + Nq + Nk)
    q = f16r(randn(r, (B * H, Nq, 64))); k = f16r(randn(r, (B * H, Nk, 64))); v = f16r(randn(r, (B * H, Nk, 64)))
    out = np.empty((B, Nq, H * 64), np.float32)
    hip.check(hip.lib().aria_hip_attention_f16(out.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                               B, H, Nq, Nk, 64))
    if Nq * Nk * B * H > 20_000_000:    # full-size: oracle on a subset of heads
        heads = [0, B * H - 1]
    else:
        heads = list(range(B * H))
    for bh in heads:
        want = port.attention(q[bh:bh + 1].copy(), k[bh:bh + 1].copy(), v[bh:bh + 1].copy())[0]
        b, h = divmod(bh, H)
        got = out[b, :, h * 64:(h + 1) * 64]
        assert_close(got, want, 1e-3, 1e-3, f"head {bh}")


def test_flash_attention_golden(hip, golden):
    """The reference's own aria_attention output (golden), inputs rounded to fp16 first."""
    g = golden
    for key in ("att", "attx"):
        q, k, v = (f16r(g[f"{key}_{n}"]) for n in "qkv")
        H, Nq, _ = q.shape
        Nk = k.shape[1]
        out = np.empty((1, Nq, H * 64), np.float32)
        hip.check(hip.lib().aria_hip_attention_f16(out.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                                   1, H, Nq, Nk, 64))
        got = out[0].reshape(Nq, H, 64).transpose(1, 0, 2)
        # inputs were rounded, the golden used the unrounded ones: fp16 input rounding is the budget
        assert_close(got, g[f"{key}_y"], 2e-3, 2e-3, key)


@pytest.mark.parametrize("rot", [32, 64, 0])
def test_qkv_prep(hip, port, rot):
    from aria_amd.device import DeviceArray, sync
    import ctypes as C
    r = rng(300 + rot)
    B, S, H = 2, 70, 16
    src = randn(r, (B * S, 3 * H * 64))
    wq = (1 + randn(r, 64, 0.1)).astype(np.float32); wk = (1 + randn(r, 64, 0.1)).astype(np.float32)
    c, s = port.rope_freqs(S, max(rot, 2), 10000.0)
    dsrc = DeviceArray.from_host(src)
    dq, dk, dv = (DeviceArray((B, H, S, 64), np.float16) for _ in range(3))
    dwq, dwk = DeviceArray.from_host(wq), DeviceArray.from_host(wk)
    dc, ds = DeviceArray.from_host(c), DeviceArray.from_host(s)
    kind = (C.c_int * 3)(0, 1, 2)
    dst = (C.c_void_p * 3)(dq.p, dk.p, dv.p)
    ws = (C.c_void_p * 3)(dwq.p, dwk.p, None)
    hip.check(hip.lib().aria_hip_qkv_prep_dev(dsrc.p, 3 * H * 64, B, S, H, 3, kind, dst, ws, dc.p, ds.p, rot, 1e-6,
                                              None))
    sync()
    x = src.reshape(B, S, 3, H, 64)
    for sec, (d, w) in enumerate(((dq, wq), (dk, wk), (dv, None))):
        got = d.to_host().astype(np.float32)
        heads = np.ascontiguousarray(x[:, :, sec].transpose(0, 2, 1, 3))    # [B, H, S, 64]
        if sec < 2:
            want = port.rmsnorm(heads.reshape(-1, 64), w, 1e-6).reshape(B * H, S, 64)
            if rot:
                want = port.rope_apply(want, c, s, rot)
            want = want.reshape(B, H, S, 64)
        else:
            want = heads
        assert_close(got, f16r(want), 0.0, 2 ** -10, f"section {sec}")


def test_cross_prep_q_only(hip, port):
    """Cross-attention query: RMSNorm, no RoPE, one section."""
    from aria_amd.device import DeviceArray, sync
    import ctypes as C
    r = rng(333)
    B, S, H = 2, 33, 16
    src = randn(r, (B * S, H * 64)); w = (1 + randn(r, 64, 0.1)).astype(np.float32)
    dsrc, dw = DeviceArray.from_host(src), DeviceArray.from_host(w)
    dq = DeviceArray((B, H, S, 64), np.float16)
    hip.check(hip.lib().aria_hip_qkv_prep_dev(dsrc.p, H * 64, B, S, H, 1, (C.c_int * 1)(0), (C.c_void_p * 1)(dq.p),
                                              (C.c_void_p * 1)(dw.p), None, None, 0, 1e-6, None))
    sync()
    heads = np.ascontiguousarray(src.reshape(B, S, H, 64).transpose(0, 2, 1, 3))
    want = port.rmsnorm(heads.reshape(-1, 64), w, 1e-6).reshape(B, H, S, 64)
    assert_close(dq.to_host().astype(np.float32), f16r(want), 0.0, 2 ** -10, "q-norm")
