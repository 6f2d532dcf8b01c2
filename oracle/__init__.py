"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU checkers.

* ``port()``  -> this repository's scalar restatement (oracle/liboracle.so,
  built from oracle/aria_oracle.c).
* ``ref()``   -> the reference's own CPU path (oracle/_ref/libaria_ref.so,
  compiled from the reference's src/aria_cpu.c + src/aria_quant.c), or None
  when that prebuilt file is absent.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may
import this package, and only to check or time the CPU side. The product
library (aria_amd) never calls it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libaria_ref.so")

_F = C.POINTER(C.c_float)
_I8 = C.POINTER(C.c_int8)
_U8 = C.POINTER(C.c_uint8)
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t


DROPIN = os.path.join(HERE, "_ref", "dropin")


def build(ref: bool = True) -> None:
    """Compile the checkers (make -C oracle). The reference part is skipped by the
    Makefile when the reference tree is absent. With ref, the drop-in link check
    (the reference's -DARIA_CUDA objects, CLI and tests/test_cuda.c linked against
    libaria_hip.so) is built too, when the backend library exists."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "all" if ref else "oracle"], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "-B", "-j8", "dropin"], check=True)


def _fp(a):
    return None if a is None else a.ctypes.data_as(_F)


def _chk(a, dt):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.dtype == dt and a.flags.c_contiguous, (a.dtype, dt)
    return a


class _Lib:
    """Thin numpy-facing wrapper; the same method names for the port and the reference
    (the reference side exposes the functions it has under the same argument order)."""

    def __init__(self, path: str, prefix: str):
        self.path = path
        self.lib = C.CDLL(path)
        self.p = prefix

    def _fn(self, name):
        return getattr(self.lib, self.p + name)

    # ---- norms ----
    def rmsnorm(self, x, w, eps):
        x = _chk(x, np.float32); _chk(w, np.float32)
        rows, dim = x.shape[0], x.shape[-1]
        rows = x.size // dim
        y = np.empty_like(x)
        self._fn("rmsnorm")(_fp(y), _fp(x), _fp(w), _i(rows), _i(dim), _f(eps))
        return y

    def gemma_rmsnorm(self, x, w, eps):
        x = _chk(x, np.float32); _chk(w, np.float32)
        dim = x.shape[-1]
        y = np.empty_like(x)
        self._fn("gemma_rmsnorm")(_fp(y), _fp(x), _fp(w), _i(x.size // dim), _i(dim), _f(eps))
        return y

    def gelu_tanh(self, x):
        y = _chk(x, np.float32).copy()
        self._fn("gelu_tanh")(_fp(y), self._n(y.size))
        return y

    def silu(self, x):
        y = _chk(x, np.float32).copy()
        self._fn("silu")(_fp(y), self._n(y.size))
        return y

    def silu_gate(self, gate, up):
        _chk(gate, np.float32); _chk(up, np.float32)
        out = np.empty_like(gate)
        self._fn("silu_gate")(_fp(out), _fp(gate), _fp(up), self._n(gate.size))
        return out

    def add(self, a, b):
        _chk(a, np.float32); _chk(b, np.float32)
        y = np.empty_like(a)
        self._fn("add")(_fp(y), _fp(a), _fp(b), self._n(a.size))
        return y

    def addto(self, y, a):
        """y + a as aria_addto does in place (returns the new y)"""
        y = _chk(y, np.float32).copy(); _chk(a, np.float32)
        self._fn("addto")(_fp(y), _fp(a), self._n(a.size))
        return y

    def scale(self, x, s):
        _chk(x, np.float32)
        y = np.empty_like(x)
        self._fn("scale")(_fp(y), _fp(x), _f(s), self._n(x.size))
        return y

    def axpy(self, y, x, s):
        """y + s*x as aria_axpy does in place (returns the new y)"""
        y = _chk(y, np.float32).copy(); _chk(x, np.float32)
        self._fn("axpy")(_fp(y), _fp(x), _f(s), self._n(x.size))
        return y

    def softmax(self, x, mask=None):
        y = _chk(x, np.float32).copy()
        cols = y.shape[-1]
        self._fn("softmax" if self.p == "or_" else "softmax_inplace")(
            _fp(y), _i(y.size // cols), _i(cols), _fp(_chk(mask, np.float32)))
        return y

    def rope_freqs(self, n, rot, base):
        rh = rot // 2
        c = np.empty((n, rh), np.float32); s = np.empty((n, rh), np.float32)
        self._fn("rope_freqs")(_fp(c), _fp(s), _i(n), _i(rot), _f(base))
        return c, s

    def rope_apply(self, x, cos_t, sin_t, rot):
        y = _chk(x, np.float32).copy()
        N, D = y.shape[-2], y.shape[-1]
        H = y.size // (N * D)
        self._fn("rope_apply")(_fp(y), _fp(cos_t), _fp(sin_t), _i(H), _i(N), _i(D), _i(rot))
        return y

    # ---- quant ----
    def q8_quant(self, W):
        _chk(W, np.float32)
        N, K = W.shape
        q = np.empty((N, K), np.int8); s = np.empty(N, np.float32)
        self._fn("q8_quant")(q.ctypes.data_as(_I8), _fp(s), _fp(W), _i(N), _i(K))
        return q, s

    def q4_quant(self, W):
        _chk(W, np.float32)
        N, K = W.shape
        nblk = (K + 31) // 32
        q = np.empty((N, (K + 1) // 2), np.uint8); s = np.empty((N, 2 * nblk), np.float32)
        self._fn("q4_quant")(q.ctypes.data_as(_U8), _fp(s), _fp(W), _i(N), _i(K))
        return q, s

    def linear_q8(self, x, q, s, b=None):
        _chk(x, np.float32)
        M, K = x.shape
        N = q.shape[0]
        y = np.empty((M, N), np.float32)
        self._fn("linear_q8")(_fp(y), _fp(x), q.ctypes.data_as(_I8), _fp(s), _fp(b),
                              _i(M), _i(K), _i(N))
        return y

    def linear_q8a8(self, x, q, s, b=None):
        _chk(x, np.float32)
        M, K = x.shape
        N = q.shape[0]
        y = np.empty((M, N), np.float32)
        self._fn("linear_q8a8")(_fp(y), _fp(x), q.ctypes.data_as(_I8), _fp(s), _fp(b),
                                _i(M), _i(K), _i(N))
        return y

    def quant_act_q8(self, x):
        """port only (the reference quantises inside aria_linear_q8a8)"""
        _chk(x, np.float32)
        M, K = x.shape
        xq = np.empty((M, K), np.int8); sx = np.empty(M, np.float32)
        self._fn("quant_act_q8")(xq.ctypes.data_as(_I8), _fp(sx), _fp(x), _i(M), _i(K))
        return xq, sx

    def linear_q4(self, x, q, s, b=None):
        _chk(x, np.float32)
        M, K = x.shape
        N = q.shape[0]
        y = np.empty((M, N), np.float32)
        self._fn("linear_q4")(_fp(y), _fp(x), q.ctypes.data_as(_U8), _fp(s), _fp(b),
                              _i(M), _i(K), _i(N))
        return y

    def linear(self, x, W, b=None):
        _chk(x, np.float32); _chk(W, np.float32)
        M, K = x.shape
        N = W.shape[0]
        y = np.empty((M, N), np.float32)
        self._fn("linear")(_fp(y), _fp(x), _fp(W), _fp(b), _i(M), _i(K), _i(N))
        return y

    def matmul(self, A, B):
        M, K = A.shape
        N = B.shape[1]
        Cm = np.empty((M, N), np.float32)
        self._fn("matmul")(_fp(Cm), _fp(A), _fp(B), _i(M), _i(K), _i(N))
        return Cm

    def attention(self, q, k, v, mask=None):
        H, Nq, D = q.shape
        Nk = k.shape[1]
        out = np.empty_like(q)
        if self.p == "or_":
            self._fn("attention")(_fp(out), _fp(q), _fp(k), _fp(v), _i(H), _i(Nq), _i(Nk), _i(D),
                                  _fp(mask))
        else:
            self._fn("attention")(_fp(out), _fp(q), _fp(k), _fp(v), _i(H), _i(Nq), _i(Nk), _i(D),
                                  _fp(mask), None)
        return out

    # ---- sampler (reference only: src/aria_sampler.c) ----
    def build_schedule(self, steps, sigma_max=1.0, shift=1, seq_len=1296):
        """aria_build_schedule (src/aria_sampler.c:167-200) with the reference class defaults
        of the shift type (aria_dist_shift_defaults); shift 1 = LOGSNR. steps + 1 sigmas."""
        cfg = DistShift()
        self.lib.aria_dist_shift_defaults(C.byref(cfg), _i(shift))
        out = np.empty(steps + 1, np.float32)
        self.lib.aria_build_schedule(_fp(out), _i(steps), _f(sigma_max), C.byref(cfg), _i(seq_len))
        return out

    def pingpong_cb(self, x, sigmas, velocity, injected_noise):
        """aria_pingpong_cb (src/aria_sampler.c:203-229) with injected noise [steps, n]:
        velocity(step, x, t) -> v is called through the reference's denoiser callback
        (aria_denoiser_fn, src/aria_sampler.h:61). Returns the final x."""
        x = np.ascontiguousarray(x, np.float32).copy()
        n = x.size
        steps = len(sigmas) - 1
        sig = np.ascontiguousarray(sigmas, np.float32)
        nz = np.ascontiguousarray(injected_noise, np.float32).reshape(steps, n)
        calls = [0]

        def cb(ctx, xp, t, vout, nn):
            xa = np.ctypeslib.as_array(xp, shape=(nn,)).copy()
            v = np.ascontiguousarray(velocity(calls[0], xa, t), np.float32).reshape(nn)
            C.memmove(vout, v.ctypes.data, nn * 4)
            calls[0] += 1

        fn = DENOISE_FN(cb)
        self.lib.aria_pingpong_cb(_fp(x), _i(n), _fp(sig), _i(steps), fn, None, None, _fp(nz),
                                  None, None, None, None)
        assert calls[0] == steps
        return x

    def _n(self, n):
        # the reference's elementwise ops take int n; the port takes size_t
        return _sz(n) if self.p == "or_" else _i(n)

    def dit_block_forward(self, x, ctx, gcond, cos_t, sin_t, rot, W, num_heads, inner):
        """The reference's own fp32 block forward, aria_dit_block_forward
        (src/aria_sa3_dit.c:316-349 -> dit_block_core :141-312), batch 1, SiLU-GLU FFN.
        x [S, dim] (not modified; returns the new residual stream), ctx [Sc, dim_ctx],
        gcond [6*dim], W: dict of the aria_dit_block_w fields (fp32)."""
        if self.p != "aria_":
            raise RuntimeError("dit_block_forward exists only in the compiled reference")
        S, dim = x.shape
        Sc, dim_ctx = ctx.shape
        keep = {k: np.ascontiguousarray(v, np.float32) for k, v in W.items() if v is not None}
        w = BlockW()
        for f in BLOCK_FIELDS:
            a = keep.get(f)
            setattr(w, f, a.ctypes.data if a is not None else None)
        y = np.ascontiguousarray(x, np.float32).copy()
        ctx = np.ascontiguousarray(ctx, np.float32)
        gcond = np.ascontiguousarray(gcond, np.float32)
        self.lib.aria_dit_block_forward(_fp(y), _i(S), _i(dim), _i(num_heads), _i(dim // num_heads), _i(inner),
                                        _fp(ctx), _i(Sc), _i(dim_ctx), _fp(gcond), _fp(cos_t), _fp(sin_t),
                                        _i(rot), C.byref(w), _i(0))
        return y


# aria_denoiser_fn (src/aria_sampler.h:61): void (*)(void *ctx, const float *x, float t, float *v, int n)
DENOISE_FN = C.CFUNCTYPE(None, C.c_void_p, _F, C.c_float, _F, C.c_int)


class DistShift(C.Structure):
    """aria_dist_shift (src/aria_sampler.h:44-50)"""
    _fields_ = [("type", C.c_int), ("anchor_length", C.c_float), ("anchor_logsnr", C.c_float),
                ("rate", C.c_float), ("logsnr_end", C.c_float), ("base_shift", C.c_float),
                ("max_shift", C.c_float), ("use_sine", C.c_int), ("alpha_min", C.c_float),
                ("alpha_max", C.c_float), ("min_length", C.c_float), ("max_length", C.c_float)]


# aria_dit_block_w, src/aria_sa3_dit.h:40-48 (21 pointers in this order)
BLOCK_FIELDS = ("pre_norm", "cross_norm", "ff_norm", "sa_to_qkv", "sa_q_norm", "sa_k_norm", "sa_to_out",
                "ca_to_q", "ca_to_kv", "ca_q_norm", "ca_k_norm", "ca_to_out", "ff_in_w", "ff_in_b",
                "ff_out_w", "ff_out_b", "to_scale_shift_gate", "to_local0_w", "to_local0_b", "to_local2_w",
                "to_local2_b")


class BlockW(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in BLOCK_FIELDS]


class Port(_Lib):
    """The restatement: extra functions that the reference has only as static glue."""

    def __init__(self):
        super().__init__(PORT_SO, "or_")

    def layernorm(self, x, gamma, beta, eps):
        _chk(x, np.float32)
        dim = x.shape[-1]
        y = np.empty_like(x)
        self.lib.or_layernorm(_fp(y), _fp(x), _fp(gamma), _fp(beta), _i(x.size // dim), _i(dim),
                              _f(eps))
        return y

    def adaln_modulate(self, y, scale, shift):
        y = _chk(y, np.float32).copy()
        dim = y.shape[-1]
        self.lib.or_adaln_modulate(_fp(y), _fp(scale), _fp(shift), _i(y.size // dim), _i(dim))
        return y

    def gate_residual(self, res, o, gate, bias=None):
        dim = res.shape[-1]
        out = np.empty_like(res)
        self.lib.or_gate_residual(_fp(out), _fp(res), _fp(o), _fp(gate), _fp(bias),
                                  _i(res.size // dim), _i(dim))
        return out

    def gate_sigmoid(self, y, gate):
        y = y.copy()
        dim = y.shape[-1]
        self.lib.or_gate_sigmoid(_fp(y), _fp(gate), _i(y.size // dim), _i(dim))
        return y

    def glu_combine(self, proj, bias=None):
        rows, two_inner = proj.size // proj.shape[-1], proj.shape[-1]
        inner = two_inner // 2
        out = np.empty(proj.shape[:-1] + (inner,), np.float32)
        self.lib.or_glu_combine(_fp(out), _fp(proj), _fp(bias), _i(rows), _i(inner))
        return out

    def pingpong(self, x, v, noise, tc, tn):
        x = x.copy()
        self.lib.or_pingpong(_fp(x), _fp(v), _fp(noise), _f(tc), _f(tn), _sz(x.size))
        return x

    def fused_chain(self, x, gamma, beta, scale, shift, eps):
        """x [B, S, D]; scale/shift [B, D]."""
        B, S, D = x.shape
        out = np.empty_like(x)
        self.lib.or_fused_chain(_fp(out), _fp(x), _fp(gamma), _fp(beta), _fp(scale), _fp(shift),
                                _i(B), _i(S), _i(D), _f(eps))
        return out

    def q8_dequant(self, q, s):
        N, K = q.shape
        W = np.empty((N, K), np.float32)
        self.lib.or_q8_dequant(_fp(W), q.ctypes.data_as(_I8), _fp(s), _i(N), _i(K))
        return W

    def q4_dequant(self, q, s, K):
        N = q.shape[0]
        W = np.empty((N, K), np.float32)
        self.lib.or_q4_dequant(_fp(W), q.ctypes.data_as(_U8), _fp(s), _i(N), _i(K))
        return W


_port = None
_ref = None


def port() -> Port:
    global _port
    if _port is None:
        if not os.path.exists(PORT_SO):
            build(ref=False)
        _port = Port()
    return _port


def ref():
    """The compiled reference CPU path, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        _ref = _Lib(REF_SO, "aria_")
    return _ref
