"""TEST INFRASTRUCTURE ONLY: the DiT block as a CPU composition of the reference's ops.

Follows dit_block_core (src/aria_sa3_dit.c:141-312) step by step for one sequence
(the reference is batch 1), with each projection dispatched like aria_linear_qw
(src/aria_quant.c:419-430): Q8 -> aria_linear_q8 (aria_linear_q8a8 with int8
activations), Q4 -> aria_linear_q4, F32 -> aria_linear. ``ops`` is the compiled
reference (oracle.ref()) or the restatement
(oracle.port()); the block's static glue (adaln_modulate, gate_sigmoid, the GLU
combine, extract/merge heads) comes from the restatement.

The composition is pinned against the reference's own aria_dit_block_forward
(tests/test_oracle.py); the FFN may also be the config's tanh-GELU MLP, which the
reference does not have (same GEMMs, GELU instead of the GLU combine).
"""
from __future__ import annotations

import numpy as np

FFN_GLU, FFN_GELU = 0, 1


def heads(a, off, H, hd=64):
    """extract_heads (src/aria_sa3_dit.c:44-57): [S, stride] -> [H, S, hd] at column off."""
    S = a.shape[0]
    return np.ascontiguousarray(a[:, off:off + H * hd].reshape(S, H, hd).transpose(1, 0, 2))


def merge(a):
    """merge_heads (src/aria_sa3_dit.c:59-69): [H, S, hd] -> [S, H*hd]."""
    H, S, hd = a.shape
    return np.ascontiguousarray(a.transpose(1, 0, 2).reshape(S, H * hd))


def pack_weights(ops, W, precision="q4"):
    """Per-projection packed form, the reference recipe (src/aria_sa3_dit.c:473-506):
    q4 -> attention Q8 + FFN Q4; q8 -> all Q8; q8a8 -> all Q8 with int8 activations
    (aria_qweight.a8, src/aria_quant.c:384, dispatched to aria_linear_q8a8); f32 -> fp32."""
    out = {}
    for name in ("sa_to_qkv", "sa_to_out", "ca_to_q", "ca_to_out", "ff_in_w", "ff_out_w"):
        ffn = name.startswith("ff_")
        if precision == "f32":
            out[name] = ("f32", np.ascontiguousarray(W[name], np.float32))
        elif precision == "q4" and ffn:
            q, s = ops.q4_quant(np.ascontiguousarray(W[name], np.float32))
            out[name] = ("q4", q, s)
        else:
            q, s = ops.q8_quant(np.ascontiguousarray(W[name], np.float32))
            out[name] = ("q8a8" if precision == "q8a8" else "q8", q, s)
    return out


def dequantized(P, W, packed):
    """W with every packed projection replaced by its dequantized fp32 value, so the
    reference's fp32 block forward computes what the dequant-on-use path computes."""
    Wd = dict(W)
    for name, pk in packed.items():
        if pk[0] in ("q8", "q8a8"):
            Wd[name] = P.q8_dequant(pk[1], pk[2])
        elif pk[0] == "q4":
            Wd[name] = P.q4_dequant(pk[1], pk[2], W[name].shape[1])
    return Wd


def cross_kv(ops, ctx, W, H, ca_kv=None):
    """Per-request cross K/V (src/aria_sa3_dit.c:327-338): kv = ctx ca_to_kv^T, k = k-norm."""
    kv = ops.linear(np.ascontiguousarray(ctx, np.float32), ca_kv if ca_kv is not None else W["ca_to_kv"])
    dim = kv.shape[1] // 2
    k = heads(kv, 0, H)
    v = heads(kv, dim, H)
    k = ops.rmsnorm(k.reshape(-1, 64), W["ca_k_norm"], 1e-6).reshape(k.shape)
    return k, v


def block_forward(ops, P, x, kc, vc, gcond, W, packed, cos_t, sin_t, rot, H, ffn=FFN_GLU, local=None):
    """One block on one sequence: x [S, dim] -> new x. kc/vc [H, Sc, 64] from cross_kv.
    local: the inpaint local-additive cond [S, dim] added after the cross-attention
    residual (src/aria_sa3_dit.c:247-252), or None."""
    S, dim = x.shape

    def lin(name, h, bias=None):
        pk = packed[name]
        h = np.ascontiguousarray(h, np.float32)
        if pk[0] == "q8":
            return ops.linear_q8(h, pk[1], pk[2], bias)
        if pk[0] == "q8a8":
            return ops.linear_q8a8(h, pk[1], pk[2], bias)
        if pk[0] == "q4":
            return ops.linear_q4(h, pk[1], pk[2], bias)
        return ops.linear(h, pk[1], bias)

    mod = (W["to_scale_shift_gate"] + gcond).astype(np.float32)
    sc_s, sh_s, g_s, sc_f, sh_f, g_f = (np.ascontiguousarray(c) for c in np.split(mod, 6))
    x = np.ascontiguousarray(x, np.float32)
    # self-attention
    h = ops.rmsnorm(x, W["pre_norm"], 1e-5)
    h = P.adaln_modulate(h, sc_s, sh_s)
    qkv = lin("sa_to_qkv", h)
    q, k, v = heads(qkv, 0, H), heads(qkv, dim, H), heads(qkv, 2 * dim, H)
    q = ops.rmsnorm(q.reshape(-1, 64), W["sa_q_norm"], 1e-6).reshape(q.shape)
    k = ops.rmsnorm(k.reshape(-1, 64), W["sa_k_norm"], 1e-6).reshape(k.shape)
    if rot:
        q = ops.rope_apply(q, cos_t, sin_t, rot)
        k = ops.rope_apply(k, cos_t, sin_t, rot)
    o = lin("sa_to_out", merge(ops.attention(q, k, v)))
    x = ops.add(x, P.gate_sigmoid(o, g_s))
    # cross-attention
    h = ops.rmsnorm(x, W["cross_norm"], 1e-5)
    qc = heads(lin("ca_to_q", h), 0, H)
    qc = ops.rmsnorm(qc.reshape(-1, 64), W["ca_q_norm"], 1e-6).reshape(qc.shape)
    o = lin("ca_to_out", merge(ops.attention(qc, kc, vc)))
    x = ops.add(x, o)
    if local is not None:
        x = ops.add(x, np.ascontiguousarray(local, np.float32))
    # feed-forward
    h = ops.rmsnorm(x, W["ff_norm"], 1e-5)
    h = P.adaln_modulate(h, sc_f, sh_f)
    if ffn == FFN_GLU:
        g = P.glu_combine(lin("ff_in_w", h, W["ff_in_b"]))
    else:
        g = ops.gelu_tanh(lin("ff_in_w", h, W["ff_in_b"]))
    o = lin("ff_out_w", g, W["ff_out_b"])
    return ops.add(x, P.gate_sigmoid(o, g_f))
