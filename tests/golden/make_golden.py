"""Writes tests/golden/ref_ops.npz: inputs and outputs of the reference's own CPU
path (oracle/_ref/libaria_ref.so, compiled from the reference's src/aria_cpu.c and
src/aria_quant.c by oracle/Makefile) at small shapes.

The fixture is data only (arrays, no code): every test can check against the
reference's outputs even where the compiled reference is absent.

Run from the repository root after `make -C oracle`:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_ops.npz")


def main() -> None:
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libaria_ref.so is missing: run make -C oracle")
    rng = np.random.default_rng(0xA21A0000)
    g = {}

    def randn(shape, sigma=1.0):
        return (sigma * rng.standard_normal(shape)).astype(np.float32)

    # row norms (src/aria_cpu.c:643-733); eps 1e-6 as the config, 1e-5 as the DiT sub-layers
    x = randn((64, 1024)); w = (1.0 + randn(1024, 0.1)).astype(np.float32)
    g["rms_x"], g["rms_w"] = x, w
    g["rms_y_eps1e-6"] = R.rmsnorm(x, w, 1e-6)
    g["rms_y_now_eps1e-5"] = R.rmsnorm(x, None, 1e-5)
    gw = randn(1024, 0.1)
    g["gemma_w"] = gw
    g["gemma_y"] = R.gemma_rmsnorm(x, gw, 1e-6)
    xq = randn((96, 64))                           # q/k-norm rows (hd = 64)
    wq = (1.0 + randn(64, 0.1)).astype(np.float32)
    g["qk_x"], g["qk_w"], g["qk_y"] = xq, wq, R.rmsnorm(xq, wq, 1e-6)

    # activations (src/aria_cpu.c:735-756), test_cuda.c scaling x4
    a = randn(4099, 2.0)
    g["act_x"] = a
    g["gelu_y"] = R.gelu_tanh(a)
    g["silu_y"] = R.silu(a)
    up = randn(4099)
    g["silu_gate_up"] = up
    g["silu_gate_y"] = R.silu_gate(a, up)
    b2 = randn(4099)
    g["add_b"] = b2
    g["add_y"] = R.add(a, b2)

    # softmax (src/aria_cpu.c:758-776): the config's N(0,2) scores at both widths, plus a mask
    s1 = randn((32, 1296), 2.0); s2 = randn((48, 216), 2.0); s3 = randn((64, 80))
    m3 = np.zeros((64, 80), np.float32); m3[:, 73:] = -3.4e38
    s4 = randn((7, 1297), 2.0)
    g["sm1_x"], g["sm1_y"] = s1, R.softmax(s1)
    g["sm2_x"], g["sm2_y"] = s2, R.softmax(s2)
    g["sm3_x"], g["sm3_m"], g["sm3_y"] = s3, m3, R.softmax(s3, m3)
    g["sm4_x"], g["sm4_y"] = s4, R.softmax(s4)

    # rotary (src/aria_cpu.c:778-809): tables + apply, rot 32 (the DiT) and 64 (the config)
    for rot in (32, 64):
        c, s = R.rope_freqs(80, rot, 10000.0)
        xr = randn((4, 80, 64))
        g[f"rope{rot}_cos"], g[f"rope{rot}_sin"], g[f"rope{rot}_x"] = c, s, xr
        g[f"rope{rot}_y"] = R.rope_apply(xr, c, s, rot)

    # Q8 / Q4 pack and the dequant-on-use GEMMs (src/aria_quant.c:78-145, 353-380, 469-538)
    for name, (N, K) in {"a": (64, 1024), "b": (37, 1031), "c": (5, 31), "d": (96, 130)}.items():
        W = randn((N, K), 0.02)
        W[1, :] = 0.0                        # zero row: scale 0, q 0
        if K >= 64:
            W[2, 32:64] = 0.0125             # constant Q4 block: step 0, nibbles 0
        q8, s8 = R.q8_quant(W)
        q4, s4_ = R.q4_quant(W)
        g[f"qw{name}_W"], g[f"qw{name}_q8"], g[f"qw{name}_s8"] = W, q8, s8
        g[f"qw{name}_q4"], g[f"qw{name}_s4"] = q4, s4_
        X = randn((37, K))
        bias = randn(N, 0.02)
        g[f"qw{name}_x"], g[f"qw{name}_b"] = X, bias
        g[f"qw{name}_y8"] = R.linear_q8(X, q8, s8, bias)
        g[f"qw{name}_y4"] = R.linear_q4(X, q4, s4_, bias)

    # attention (src/aria_cpu.c:811-849) at the test_cuda.c shape and a cross-attention shape
    q = randn((8, 48, 64)); k = randn((8, 48, 64)); v = randn((8, 48, 64))
    g["att_q"], g["att_k"], g["att_v"], g["att_y"] = q, k, v, R.attention(q, k, v)
    q2 = randn((2, 40, 64)); k2 = randn((2, 24, 64)); v2 = randn((2, 24, 64))
    g["attx_q"], g["attx_k"], g["attx_v"], g["attx_y"] = q2, k2, v2, R.attention(q2, k2, v2)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
