"""GPU parity: each hot-path op of the HIP backend, called through the C ABI, against the
reference's golden vectors and the oracle on the same seeded inputs.

Gates:
  * integer / byte work (Q8/Q4 pack, unpack, indexing), modulate, add, pingpong: bit-exact;
  * fp32 norms / activations / softmax / RoPE / fused chain: max|d| <= 1e-5 * max|ref|
    (the 1e-5 relative fp32 gate; transcendental ops differ from glibc by ulps);
  * op-level ABI tolerances of the reference's tests/test_cuda.c (linear 1e-3 + 2e-4*max,
    rmsnorm 1e-4 + 1e-4*max, elementwise/softmax/rope 1e-5 + 1e-5*max, attention 1e-3 + 1e-3*max).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, randn, rng

pytestmark = pytest.mark.gpu

FP32_RTOL = 1e-5


def rel_close(got, want, rtol=FP32_RTOL, what=""):
    assert_close(got, want, 0.0, rtol, what)


@pytest.fixture(scope="module")
def ops(hip):
    from aria_amd import ops as O
    return O


# ------------------------------------------------------------------ norms

def test_rmsnorm_golden(ops, golden):
    g = golden
    rel_close(ops.rmsnorm(g["rms_x"], g["rms_w"], 1e-6), g["rms_y_eps1e-6"], what="rms w")
    rel_close(ops.rmsnorm(g["rms_x"], None, 1e-5), g["rms_y_now_eps1e-5"], what="rms no-w")
    rel_close(ops.gemma_rmsnorm(g["rms_x"], g["gemma_w"], 1e-6), g["gemma_y"], what="gemma")
    rel_close(ops.rmsnorm(g["qk_x"], g["qk_w"], 1e-6), g["qk_y"], what="qk-norm dim 64")
    # the double-accumulated statistic reproduces the reference nearly bit for bit
    y = ops.rmsnorm(g["rms_x"], g["rms_w"], 1e-6)
    assert np.mean(y == g["rms_y_eps1e-6"]) > 0.999


@pytest.mark.parametrize("dim", [64, 128, 256, 768, 1024, 2048, 80, 1000, 3])
def test_rmsnorm_shapes(ops, port, dim):
    r = rng(100 + dim)
    x = randn(r, (37, dim)); w = randn(r, dim)
    rel_close(ops.rmsnorm(x, w, 1e-6), port.rmsnorm(x, w, 1e-6), what=f"rms {dim}")
    rel_close(ops.gemma_rmsnorm(x, w, 1e-6), port.gemma_rmsnorm(x, w, 1e-6), what=f"gemma {dim}")


def test_rmsnorm_test_cuda_contract(ops, port):
    """tests/test_cuda.c:60-66: R=300, D=1024, x,w uniform [-1,1), gate 1e-4 + 1e-4*max."""
    r = rng(7)
    x = r.uniform(-1, 1, (300, 1024)).astype(np.float32); w = r.uniform(-1, 1, 1024).astype(np.float32)
    assert_close(ops.rmsnorm(x, w, 1e-6), port.rmsnorm(x, w, 1e-6), 1e-4, 1e-4, "rmsnorm")
    assert_close(ops.gemma_rmsnorm(x, w, 1e-6), port.gemma_rmsnorm(x, w, 1e-6), 1e-4, 1e-4, "gemma")


@pytest.mark.parametrize("dim", [1024, 768, 64, 100])
def test_layernorm(ops, port, dim):
    r = rng(200 + dim)
    x = randn(r, (41, dim), 2.0) + 1.5
    g = (1 + randn(r, dim, 0.1)).astype(np.float32); b = randn(r, dim, 0.1)
    rel_close(ops.layernorm(x, g, b, 1e-6), port.layernorm(x, g, b, 1e-6), what="ln g,b")
    rel_close(ops.layernorm(x, None, None, 1e-6), port.layernorm(x, None, None, 1e-6), what="ln plain")
    # constant rows -> beta exactly
    y = ops.layernorm(np.full((3, dim), 2.5, np.float32), g, b, 1e-6)
    assert np.array_equal(y, np.broadcast_to(b, y.shape))


def test_rmsnorm_adaln(ops, port):
    r = rng(9)
    B, S, D = 2, 53, 1024
    x = randn(r, (B * S, D)); w = (1 + randn(r, D, 0.02)).astype(np.float32)
    sc = randn(r, (B, D), 0.1); sh = randn(r, (B, D), 0.1)
    got = ops.rmsnorm_adaln(x, w, sc, sh, 1e-5, rows_per_batch=S)
    want = np.concatenate([port.adaln_modulate(port.rmsnorm(x[b * S:(b + 1) * S], w, 1e-5), sc[b], sh[b])
                           for b in range(B)])
    rel_close(got, want, what="rmsnorm+adaln")


@pytest.mark.parametrize("shape", [(2, 216, 1024), (2, 1296, 1024), (1, 7, 100)])
def test_fused_chain(ops, port, shape):
    """Config 1 / config 2 chain: gelu(LN(x)*(1+scale)+shift) + x, one HBM pass."""
    r = rng(shape[1])
    B, S, D = shape
    x = randn(r, shape); sc = randn(r, (B, D), 0.1); sh = randn(r, (B, D), 0.1)
    g = np.ones(D, np.float32); b = np.zeros(D, np.float32)
    rel_close(ops.ln_mod_gelu_res(x, g, b, sc, sh, 1e-6), port.fused_chain(x, g, b, sc, sh, 1e-6),
              what="chain gamma=1,beta=0")
    g = (1 + randn(r, D, 0.1)).astype(np.float32); b = randn(r, D, 0.1)
    rel_close(ops.ln_mod_gelu_res(x, g, b, sc, sh, 1e-6), port.fused_chain(x, g, b, sc, sh, 1e-6),
              what="chain gamma,beta")


# ------------------------------------------------------------------ elementwise

def test_activations_golden(ops, golden):
    g = golden
    rel_close(ops.gelu_tanh(g["act_x"]), g["gelu_y"], what="gelu")
    rel_close(ops.silu(g["act_x"]), g["silu_y"], what="silu")
    rel_close(ops.silu_gate(g["act_x"], g["silu_gate_up"]), g["silu_gate_y"], what="silu_gate")
    assert np.array_equal(ops.add(g["act_x"], g["add_b"]), g["add_y"])


def test_test_cuda_elementwise(ops, port):
    """tests/test_cuda.c:69-86 shapes and gates (1e-5 + 1e-5*max)."""
    r = rng(12)
    x = r.uniform(-1, 1, 4096).astype(np.float32)
    assert_close(ops.softcap(x * 30, 50.0), 50.0 * np.tanh((x * 30).astype(np.float64) / 50.0), 1e-5, 1e-5, "softcap")
    assert_close(ops.silu(x * 4), port.silu(x * 4), 1e-5, 1e-5, "silu")
    assert_close(ops.gelu_tanh(x * 4), port.gelu_tanh(x * 4), 1e-5, 1e-5, "gelu")
    up = r.uniform(-1, 1, 4096).astype(np.float32)
    assert_close(ops.silu_gate(x, up), port.silu_gate(x, up), 1e-5, 1e-5, "silu_gate")
    xd = r.uniform(-1, 1, (256, 64)).astype(np.float32)
    w = r.uniform(-1, 1, 64).astype(np.float32); b = r.uniform(-1, 1, 64).astype(np.float32)
    want = np.tanh(0.7 * xd.astype(np.float64)) * w + b
    assert_close(ops.dynamic_tanh(xd, 0.7, w, b), want, 1e-5, 1e-5, "dynamic_tanh")


def test_modulate_gate_glu_pingpong(ops, port):
    r = rng(13)
    B, S, D = 2, 40, 1024
    x = randn(r, (B * S, D)); sc = randn(r, (B, D), 0.1); sh = randn(r, (B, D), 0.1)
    want = np.concatenate([port.adaln_modulate(x[b * S:(b + 1) * S], sc[b], sh[b]) for b in range(B)])
    assert np.array_equal(ops.modulate(x, sc, sh, rows_per_batch=S), want)
    o = randn(r, (B * S, D)); gate = randn(r, (B, D), 0.5); bias = randn(r, D, 0.02)
    for bb in (None, bias):
        got = ops.gate_residual(x, o, gate, bb, rows_per_batch=S)
        want = np.concatenate([port.gate_residual(x[b * S:(b + 1) * S], o[b * S:(b + 1) * S], gate[b], bb)
                               for b in range(B)])
        rel_close(got, want, what=f"gate_residual bias={bb is not None}")
    proj = randn(r, (S, 2 * 512)); pb = randn(r, 1024, 0.02)
    rel_close(ops.glu_combine(proj), port.glu_combine(proj), what="glu")
    rel_close(ops.glu_combine(proj, pb), port.glu_combine(proj, pb), what="glu+bias")
    xs = randn(r, 64 * 2592); v = randn(r, 64 * 2592); n = randn(r, 64 * 2592)
    assert np.array_equal(ops.pingpong(xs, v, n, 0.8125, 0.6), port.pingpong(xs, v, n, 0.8125, 0.6))
    assert np.array_equal(ops.pingpong(xs[:1001], v[:1001], n[:1001], 0.3, 0.1),
                          port.pingpong(xs[:1001], v[:1001], n[:1001], 0.3, 0.1))


# ------------------------------------------------------------------ softmax / rope

def test_softmax_golden(ops, golden):
    g = golden
    for k in ("sm1", "sm2", "sm4"):
        assert_close(ops.softmax(g[k + "_x"]), g[k + "_y"], 1e-5, 1e-5, k)
    assert_close(ops.softmax(g["sm3_x"], g["sm3_m"]), g["sm3_y"], 1e-5, 1e-5, "masked")
    assert np.all(ops.softmax(g["sm3_x"], g["sm3_m"])[:, 73:] == 0)


@pytest.mark.parametrize("cols", [1, 3, 63, 64, 216, 256, 1296, 1297, 4096, 5000])
def test_softmax_shapes(ops, port, cols):
    r = rng(cols)
    s = randn(r, (19, cols), 2.0)
    assert_close(ops.softmax(s), port.softmax(s), 1e-5, 1e-5, f"softmax {cols}")


def test_rope_golden(ops, golden):
    g = golden
    for rot in (32, 64):
        assert_close(ops.rope_apply(g[f"rope{rot}_x"], g[f"rope{rot}_cos"], g[f"rope{rot}_sin"], rot),
                     g[f"rope{rot}_y"], 1e-5, 1e-5, f"rope{rot}")


def test_rope_shapes(ops, port):
    r = rng(15)
    # the vector kernel rotates 4, 2 or 1 head rows per thread as H allows (4 | H, 2 | H, odd H);
    # rot 24 leaves lanes of each workgroup idle (3 lanes per position), rot 128 takes 16
    for (H, N, D, rot) in [(4, 60, 64, 32), (32, 1296, 64, 32), (32, 1296, 64, 64), (3, 17, 20, 6),
                           (2, 33, 64, 32), (5, 41, 64, 64), (6, 20, 72, 16), (8, 70, 64, 24), (4, 50, 128, 128)]:
        c, s = port.rope_freqs(N, rot, 10000.0)
        x = randn(r, (H, N, D))
        got = ops.rope_apply(x, c, s, rot)
        assert_close(got, port.rope_apply(x, c, s, rot), 1e-5, 1e-5, f"rope {H},{N},{D},{rot}")
        assert np.array_equal(got[..., rot:], x[..., rot:])


# ------------------------------------------------------------------ quantisation

@pytest.mark.parametrize("name", ["a", "b", "c", "d"])
def test_quant_pack_golden(ops, golden, name):
    g = golden
    W = g[f"qw{name}_W"]
    q8, s8 = ops.q8_quant(W)
    assert np.array_equal(q8, g[f"qw{name}_q8"]) and np.array_equal(s8, g[f"qw{name}_s8"])
    q4, s4 = ops.q4_quant(W)
    assert np.array_equal(q4, g[f"qw{name}_q4"]) and np.array_equal(s4, g[f"qw{name}_s4"])


@pytest.mark.parametrize("NK", [(4096, 1024), (1024, 4096), (3, 1), (7, 31), (9, 33), (5, 1031), (2, 64)])
def test_quant_pack_unpack(ops, port, NK):
    N, K = NK
    r = rng(N * 7 + K)
    W = randn(r, (N, K), 0.02)
    if N > 2:
        W[1] = 0.0
    q8, s8 = ops.q8_quant(W)
    p8, ps8 = port.q8_quant(W)
    assert np.array_equal(q8, p8) and np.array_equal(s8, ps8)
    q4, s4 = ops.q4_quant(W)
    p4, ps4 = port.q4_quant(W)
    assert np.array_equal(q4, p4) and np.array_equal(s4, ps4)
    assert np.array_equal(ops.q8_dequant(q8, s8), port.q8_dequant(q8, s8))
    assert np.array_equal(ops.q4_dequant(q4, s4, K), port.q4_dequant(q4, s4, K))


# ------------------------------------------------------------------ op-level dense ABI

@pytest.mark.parametrize("MKN", [(279, 1024, 3072), (33, 100, 17), (1, 1024, 1024), (256, 2048, 768)])
def test_linear(ops, port, MKN):
    """tests/test_cuda.c:28-47 shapes, gate 1e-3 + 2e-4*max."""
    M, K, N = MKN
    r = rng(M + K + N)
    x = r.uniform(-1, 1, (M, K)).astype(np.float32); W = r.uniform(-1, 1, (N, K)).astype(np.float32)
    b = r.uniform(-1, 1, N).astype(np.float32)
    assert_close(ops.linear(x, W, b), port.linear(x, W, b), 1e-3, 2e-4, f"linear {MKN}")


def test_matmul_attention_conv(ops, port):
    r = rng(21)
    A = r.uniform(-1, 1, (200, 128)).astype(np.float32); B = r.uniform(-1, 1, (128, 96)).astype(np.float32)
    assert_close(ops.matmul(A, B), port.matmul(A, B), 1e-3, 2e-4, "matmul")
    q, k, v = (r.uniform(-1, 1, (8, 48, 64)).astype(np.float32) for _ in range(3))
    assert_close(ops.attention(q, k, v), port.attention(q, k, v), 1e-3, 1e-3, "attention")
    k2, v2 = (r.uniform(-1, 1, (8, 30, 64)).astype(np.float32) for _ in range(2))
    m = np.zeros((48, 30), np.float32); m[:, 25:] = -3.4e38
    assert_close(ops.attention(q, k2, v2, m), port.attention(q, k2, v2, m), 1e-3, 1e-3, "attention mask")
    inp = r.uniform(-1, 1, (16, 120)).astype(np.float32)
    w = r.uniform(-1, 1, (32, 16, 3)).astype(np.float32); bb = r.uniform(-1, 1, 32).astype(np.float32)
    # conv1d by float64 brute force
    pad = 1
    xp = np.pad(inp.astype(np.float64), ((0, 0), (pad, pad)))
    want = sum(w[:, :, kk].astype(np.float64) @ xp[:, kk:kk + 120] for kk in range(3)) + bb[:, None]
    assert_close(ops.conv1d(inp, w, bb, pad), want, 1e-4, 1e-4, "conv1d")


def test_golden_attention(ops, golden):
    g = golden
    assert_close(ops.attention(g["att_q"], g["att_k"], g["att_v"]), g["att_y"], 1e-3, 1e-3, "self")
    assert_close(ops.attention(g["attx_q"], g["attx_k"], g["attx_v"]), g["attx_y"], 1e-3, 1e-3, "cross")


# ------------------------------------------------------------------ device-pointer API

def test_device_chain_f16(hip, port):
    """rmsnorm_adaln with fp16 output (the GEMM operand) through device pointers."""
    from aria_amd.device import DeviceArray, sync
    r = rng(31)
    S, D = 96, 1024
    x = randn(r, (S, D)); w = (1 + randn(r, D, 0.02)).astype(np.float32)
    sc = randn(r, D, 0.1); sh = randn(r, D, 0.1)
    dx, dw, dsc, dsh = (DeviceArray.from_host(a) for a in (x, w, sc, sh))
    dy = DeviceArray((S, D), np.float16)
    hip.check(hip.lib().aria_hip_rmsnorm_adaln_dev(dy.p, 1, dx.p, dw.p, dsc.p, dsh.p, S, D, 0, 1e-5, None))
    sync()
    want = port.adaln_modulate(port.rmsnorm(x, w, 1e-5), sc, sh).astype(np.float16)
    got = dy.to_host()
    assert np.mean(got == want) > 0.999 and np.max(np.abs(got.astype(np.float32) - want.astype(np.float32))) <= \
        np.float32(2 ** -10) * np.max(np.abs(want.astype(np.float32)))


def test_argument_errors(hip):
    L = hip.lib()
    assert L.aria_hip_rmsnorm_adaln_dev(None, 0, None, None, None, None, 4, 8, 3, 1e-5, None) == -1
    assert L.aria_hip_rope_apply_dev(None, None, None, 1, 1, 8, 10, None) == -1
    assert "invalid argument" in hip.last_error()


def test_rope_two_tensors_one_launch(hip, port):
    """aria_hip_rope_apply2_dev rotates q and k exactly as two single-tensor calls."""
    from aria_amd.device import DeviceArray, sync
    r = rng(41)
    for rot in (32, 64, 6):
        H, N, D = 8, 100, 64
        c, s = port.rope_freqs(N, rot, 10000.0)
        q = randn(r, (H, N, D)); k = randn(r, (H, N, D))
        dq, dk, dc, ds = (DeviceArray.from_host(a) for a in (q, k, c, s))
        hip.check(hip.lib().aria_hip_rope_apply2_dev(dq.p, dk.p, dc.p, ds.p, H, N, D, rot, None))
        sync()
        assert_close(dq.to_host(), port.rope_apply(q, c, s, rot), 1e-5, 1e-5, f"q rot {rot}")
        assert_close(dk.to_host(), port.rope_apply(k, c, s, rot), 1e-5, 1e-5, f"k rot {rot}")


def test_softmax_fully_masked_rows(ops, port):
    """Rows whose every column carries the -3.4e38 padding mask stay finite, as in the reference."""
    r = rng(42)
    s = randn(r, (8, 1296), 2.0)
    m = np.full_like(s, -3.4e38)
    got = ops.softmax(s, m)
    assert np.all(np.isfinite(got))
    assert_close(got, port.softmax(s, m), 1e-5, 1e-5, "all-masked")


@pytest.mark.parametrize("n", [1, 4099, 1 << 20])
def test_axpy_scale_addto(ops, port, ref, n):
    """aria_hip_axpy_dev / aria_hip_scale_dev / aria_hip_add_dev with y aliasing its first input
    (aria_addto), against the reference's aria_axpy / aria_scale / aria_addto
    (src/aria_cpu.c:989-1000): bit-exact, ragged sizes included."""
    r = rng(77 + n)
    x = randn(r, n); y = randn(r, n)
    for s_ in (0.7071, -3.25):
        assert np.array_equal(ops.scale(x, s_).view(np.uint32), port.scale(x, s_).view(np.uint32))
        assert np.array_equal(ops.axpy(y, x, s_).view(np.uint32), port.axpy(y, x, s_).view(np.uint32))
    assert np.array_equal(ops.addto(y, x).view(np.uint32), port.addto(y, x).view(np.uint32))
    if ref is not None:
        assert np.array_equal(ops.axpy(y, x, -3.25).view(np.uint32), ref.axpy(y, x, -3.25).view(np.uint32))
        assert np.array_equal(ops.scale(x, 0.7071).view(np.uint32), ref.scale(x, 0.7071).view(np.uint32))
        assert np.array_equal(ops.addto(y, x).view(np.uint32), ref.addto(y, x).view(np.uint32))


# ------------------------------------------------------------------ fp32 -> fp16 staging

@pytest.mark.parametrize("n", [4, 1020, 4096, 4100, 75648, 4097, 7])
def test_f32_to_f16_bits(hip, n):
    """aria_k_f32_to_f16 (the GEMMs' staging of fp32 activations, the weights' and K/V's
    conversion at set-up) against numpy's round-to-nearest-even float16, bit for bit: the
    streamed four-vectors-per-lane form (n % 4 == 0, ragged last wave at 4100 and 75648), the
    scalar form (4097, 7), and values at every rounding case (ties, subnormals, overflow to
    inf, signed zeros, inf, NaN)."""
    import ctypes as C
    from aria_amd.device import DeviceArray, sync
    r = rng(900 + n)
    x = (r.standard_normal(n) * np.exp2(r.integers(-26, 18, n))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 65519.996, 6.1e-5, 5.96e-8,
                        2.98e-8, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -(1.0 + 2.0 ** -11)], np.float32)
    k = min(n, special.size)
    x[:k] = special[:k]
    f = hip.lib().aria_k_f32_to_f16
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
    dx, dy = DeviceArray.from_host(x), DeviceArray(n, np.float16)
    hip.check(f(dy.p, dx.p, n, None))
    sync()
    got, want = dy.to_host().view(np.uint16), x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(np.isnan(dy.to_host()), nan)
    bad = np.flatnonzero((got != want) & ~nan)
    assert bad.size == 0, (bad[:4], x[bad[:4]], got[bad[:4]], want[bad[:4]])
