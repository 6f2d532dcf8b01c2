"""Host-pointer op surface of the MI355X backend, mirroring the reference's
src/aria_ops.h and src/aria_quant.h names and argument meaning (numpy in, numpy
out). Each call goes through the C ABI (aria_cuda_* of include/aria_gpu.h or
aria_hip_* of include/aria_hip.h): copy in, run the gfx950 kernel, copy out.

In-place ops of the reference (silu, gelu_tanh, softcap, softmax, rope_apply)
return a new array and leave the argument untouched here.
"""
from __future__ import annotations

import numpy as np

from . import check, lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


# ---- aria_gpu.h wrappers (src/aria_gpu.h:38-61) ----

def rmsnorm(x, w, eps):
    x = _f32(x); w = _f32(w)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().aria_cuda_rmsnorm(_p(y), _p(x), _p(w), x.size // dim, dim, eps)
    return y


def gemma_rmsnorm(x, w, eps):
    x = _f32(x); w = _f32(w)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().aria_cuda_gemma_rmsnorm(_p(y), _p(x), _p(w), x.size // dim, dim, eps)
    return y


def dynamic_tanh(x, alpha, w, b):
    x = _f32(x); w = _f32(w); b = _f32(b)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().aria_cuda_dynamic_tanh(_p(y), _p(x), alpha, _p(w), _p(b), x.size // dim, dim)
    return y


def softcap(x, cap):
    y = _f32(x).copy()
    lib().aria_cuda_softcap(_p(y), y.size, cap)
    return y


def silu(x):
    y = _f32(x).copy()
    lib().aria_cuda_silu(_p(y), y.size)
    return y


def gelu_tanh(x):
    y = _f32(x).copy()
    lib().aria_cuda_gelu_tanh(_p(y), y.size)
    return y


def silu_gate(gate, up):
    gate = _f32(gate); up = _f32(up)
    out = np.empty_like(gate)
    lib().aria_cuda_silu_gate(_p(out), _p(gate), _p(up), gate.size)
    return out


def softmax(x, mask=None):
    y = _f32(x).copy()
    mask = _f32(mask)
    cols = y.shape[-1]
    lib().aria_cuda_softmax(_p(y), y.size // cols, cols, _p(mask))
    return y


def rope_apply(x, cos_t, sin_t, rot_dim):
    y = _f32(x).copy()
    cos_t = _f32(cos_t); sin_t = _f32(sin_t)
    N, D = y.shape[-2], y.shape[-1]
    lib().aria_cuda_rope_apply(_p(y), _p(cos_t), _p(sin_t), y.size // (N * D), N, D, rot_dim)
    return y


def linear(x, W, b=None):
    x = _f32(x); W = _f32(W); b = _f32(b)
    M, K = x.shape
    N = W.shape[0]
    y = np.empty((M, N), np.float32)
    lib().aria_cuda_linear(_p(y), _p(x), _p(W), _p(b), M, K, N)
    return y


def matmul(A, B):
    A = _f32(A); B = _f32(B)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    lib().aria_cuda_matmul(_p(Cm), _p(A), _p(B), M, K, N)
    return Cm


def attention(q, k, v, mask=None):
    q = _f32(q); k = _f32(k); v = _f32(v); mask = _f32(mask)
    H, Nq, D = q.shape
    Nk = k.shape[1]
    out = np.empty_like(q)
    lib().aria_cuda_attention(_p(out), _p(q), _p(k), _p(v), H, Nq, Nk, D, _p(mask))
    return out


def conv1d(inp, w, bias, pad):
    inp = _f32(inp); w = _f32(w); bias = _f32(bias)
    Cout, Cin, K = w.shape
    L = inp.shape[1]
    out = np.empty((Cout, L), np.float32)
    lib().aria_cuda_conv1d(_p(out), _p(inp), _p(w), _p(bias), Cin, Cout, K, pad, L)
    return out


# ---- aria_hip.h host-pointer forms ----

def layernorm(x, gamma, beta, eps):
    x = _f32(x); gamma = _f32(gamma); beta = _f32(beta)
    dim = x.shape[-1]
    y = np.empty_like(x)
    check(lib().aria_hip_layernorm(_p(y), _p(x), _p(gamma), _p(beta), x.size // dim, dim, eps),
          "aria_hip_layernorm")
    return y


def rmsnorm_adaln(x, w, scale, shift, eps, rows_per_batch=0):
    x = _f32(x); w = _f32(w); scale = _f32(scale); shift = _f32(shift)
    dim = x.shape[-1]
    y = np.empty_like(x)
    check(lib().aria_hip_rmsnorm_adaln(_p(y), _p(x), _p(w), _p(scale), _p(shift), x.size // dim, dim,
                                       rows_per_batch, eps), "aria_hip_rmsnorm_adaln")
    return y


def ln_mod_gelu_res(x, gamma, beta, scale, shift, eps):
    """x [B, S, D], scale/shift [B, D]: gelu(LN(x)*(1+scale)+shift) + x, one pass."""
    x = _f32(x); gamma = _f32(gamma); beta = _f32(beta); scale = _f32(scale); shift = _f32(shift)
    B, S, D = x.shape
    out = np.empty_like(x)
    check(lib().aria_hip_ln_mod_gelu_res(_p(out), _p(x), _p(gamma), _p(beta), _p(scale), _p(shift),
                                         B * S, D, S, eps), "aria_hip_ln_mod_gelu_res")
    return out


def modulate(x, scale, shift, rows_per_batch=0):
    x = _f32(x); scale = _f32(scale); shift = _f32(shift)
    dim = x.shape[-1]
    y = np.empty_like(x)
    check(lib().aria_hip_modulate(_p(y), _p(x), _p(scale), _p(shift), x.size // dim, dim, rows_per_batch),
          "aria_hip_modulate")
    return y


def gate_residual(res, o, gate, bias=None, rows_per_batch=0):
    res = _f32(res); o = _f32(o); gate = _f32(gate); bias = _f32(bias)
    dim = res.shape[-1]
    out = np.empty_like(res)
    check(lib().aria_hip_gate_residual(_p(out), _p(res), _p(o), _p(gate), _p(bias), res.size // dim, dim,
                                       rows_per_batch), "aria_hip_gate_residual")
    return out


def glu_combine(proj, bias=None):
    proj = _f32(proj); bias = _f32(bias)
    inner = proj.shape[-1] // 2
    rows = proj.size // proj.shape[-1]
    out = np.empty(proj.shape[:-1] + (inner,), np.float32)
    check(lib().aria_hip_glu_combine(_p(out), _p(proj), _p(bias), rows, inner), "aria_hip_glu_combine")
    return out


def add(a, b):
    a = _f32(a); b = _f32(b)
    y = np.empty_like(a)
    check(lib().aria_hip_add(_p(y), _p(a), _p(b), a.size), "aria_hip_add")
    return y


def addto(y, a):
    """aria_addto (src/aria_ops.h:167): y += a, as aria_hip_add_dev with y aliasing its first input"""
    from .device import DeviceArray
    dy = DeviceArray.from_host(_f32(y)); da = DeviceArray.from_host(_f32(a))
    try:
        check(lib().aria_hip_add_dev(dy.p, dy.p, da.p, dy.nbytes // 4, None), "aria_hip_add_dev")
        check(lib().aria_hip_stream_sync(None), "aria_hip_add_dev")
        return dy.to_host()
    finally:
        dy.free(); da.free()


def scale(x, s):
    """aria_scale (src/aria_ops.h:168): y = x * s (returns y)"""
    from .device import DeviceArray
    dx = DeviceArray.from_host(_f32(x)); dy = DeviceArray(dx.shape)
    try:
        check(lib().aria_hip_scale_dev(dy.p, dx.p, s, dx.nbytes // 4, None), "aria_hip_scale_dev")
        check(lib().aria_hip_stream_sync(None), "aria_hip_scale_dev")
        return dy.to_host()
    finally:
        dx.free(); dy.free()


def axpy(y, x, s):
    """aria_axpy (src/aria_ops.h:169): y += s * x (returns the new y)"""
    from .device import DeviceArray
    dy = DeviceArray.from_host(_f32(y)); dx = DeviceArray.from_host(_f32(x))
    try:
        check(lib().aria_hip_axpy_dev(dy.p, dx.p, s, dy.nbytes // 4, None), "aria_hip_axpy_dev")
        check(lib().aria_hip_stream_sync(None), "aria_hip_axpy_dev")
        return dy.to_host()
    finally:
        dy.free(); dx.free()


def pingpong(x, v, noise, tc, tn):
    y = _f32(x).copy()
    v = _f32(v); noise = _f32(noise)
    check(lib().aria_hip_pingpong(_p(y), _p(v), _p(noise), tc, tn, y.size), "aria_hip_pingpong")
    return y


def q8_quant(W):
    W = _f32(W)
    N, K = W.shape
    q = np.empty((N, K), np.int8); s = np.empty(N, np.float32)
    check(lib().aria_hip_q8_quant(_p(q), _p(s), _p(W), N, K), "aria_hip_q8_quant")
    return q, s


def q4_quant(W):
    W = _f32(W)
    N, K = W.shape
    q = np.empty((N, (K + 1) // 2), np.uint8); s = np.empty((N, 2 * ((K + 31) // 32)), np.float32)
    check(lib().aria_hip_q4_quant(_p(q), _p(s), _p(W), N, K), "aria_hip_q4_quant")
    return q, s


def linear_q8(x, q, s, b=None):
    """aria_linear_q8 (src/aria_quant.h:45): y = x dequant(q, s)^T + b, on MFMA."""
    x = _f32(x); b = _f32(b)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float32)
    check(lib().aria_hip_linear_q8(_p(y), _p(x), _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(s)),
                                   _p(b), M, K, N), "aria_hip_linear_q8")
    return y


def linear_q4(x, q, s, b=None):
    """aria_linear_q4 (src/aria_quant.h:65): y = x dequant(q, s)^T + b, on MFMA."""
    x = _f32(x); b = _f32(b)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float32)
    check(lib().aria_hip_linear_q4(_p(y), _p(x), _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(s)),
                                   _p(b), M, K, N), "aria_hip_linear_q4")
    return y


def linear_q8a8(x, q, s, b=None):
    """aria_linear_q8a8 (src/aria_quant.h:50): per-row int8 activations, exact int32 dot
    products on the int8 MFMA, y = acc * sx[m] * s[n] + b (bit-identical to the reference)."""
    x = _f32(x); b = _f32(b)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float32)
    check(lib().aria_hip_linear_q8a8(_p(y), _p(x), _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(s)),
                                     _p(b), M, K, N), "aria_hip_linear_q8a8")
    return y


def q8_dequant(q, s):
    N, K = q.shape
    W = np.empty((N, K), np.float32)
    check(lib().aria_hip_q8_dequant(_p(W), _p(q), _p(s), N, K), "aria_hip_q8_dequant")
    return W


def q4_dequant(q, s, K):
    N = q.shape[0]
    W = np.empty((N, K), np.float32)
    check(lib().aria_hip_q4_dequant(_p(W), _p(q), _p(s), N, K), "aria_hip_q4_dequant")
    return W
