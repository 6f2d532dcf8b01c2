"""Python host side of the small-music taae_v2 decoder on the MI355X backend
(include/aria_dit.h: aria_cuda_dec_create / _free / _forward, aria_hip_dec_forward_dev).

``Decoder`` uploads a weight view once and decodes latent [256, T] -> audio
[2, T * 4096] on the device. The view is the reference's aria_sa3_dec_view
(src/aria_sa3_dec.h:75-85): filled by the reference's own loader
(aria_sa3_dec_get_view) when the caller has one, or by ``view_from_tensors`` from a
checkpoint's fp32 tensors under the reference's names.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import HipError, check, last_error, lib

PFX = "pretransform.model."
BLK = PFX + "decoder.layers.3.transformers.%d."


D, HD, INNER, QKV = 768, 64, 2304, 3840


def tensor_shapes():
    """name -> shape of every tensor aria_sa3_dec_load reads (src/aria_sa3_dec.c:242-266)."""
    sh = {PFX + "bottleneck.running_std": (1,),
          PFX + "decoder.layers.1.weight": (D, 256), PFX + "decoder.layers.1.bias": (D,),
          PFX + "decoder.layers.3.new_tokens": (D,),
          PFX + "decoder.layers.3.mapping.weight_g": (512, 1, 1),
          PFX + "decoder.layers.3.mapping.weight_v": (512, D, 3),
          PFX + "decoder.layers.3.mapping.bias": (512,)}
    for i in range(6):
        for n in ("pre_norm", "self_attn.q_norm", "self_attn.k_norm", "ff_norm"):
            dim = HD if "attn" in n else D
            sh[BLK % i + n + ".alpha"] = (1,)
            sh[BLK % i + n + ".gamma"] = (dim,)
            sh[BLK % i + n + ".beta"] = (dim,)
        sh[BLK % i + "self_attn.to_qkv.weight"] = (QKV, D)
        sh[BLK % i + "self_attn.to_out.weight"] = (D, D)
        sh[BLK % i + "ff.ff.0.proj.weight"] = (2 * INNER, D)
        sh[BLK % i + "ff.ff.0.proj.bias"] = (2 * INNER,)
        sh[BLK % i + "ff.ff.2.weight"] = (D, INNER)
        sh[BLK % i + "ff.ff.2.bias"] = (D,)
    return sh


def random_tensors(rng, qk_gain=2.0):
    """A synthetic checkpoint (random init; no trained weights are available): the decoder's
    tensors under the reference's names, scaled so activations stay O(1) through the six
    blocks: Linear weights ~ N(0, 1/fan_in) (residual outputs halved), DyT alpha in
    [0.5, 1.5], gamma ~ 1, beta small; the q/k norm gains qk_gain make the attention peaked
    enough that position (RoPE) and chunking matter."""
    t = {}
    for name, shape in tensor_shapes().items():
        if name.endswith(".alpha"):
            a = rng.uniform(0.5, 1.5, shape)
        elif name.endswith(".gamma"):
            g = qk_gain if "attn" in name else 1.0
            a = g * (1.0 + 0.1 * rng.standard_normal(shape))
        elif name.endswith(".beta") or name.endswith(".bias"):
            a = 0.05 * rng.standard_normal(shape)
        elif name.endswith("running_std"):
            a = np.array([0.9])
        elif name.endswith("new_tokens"):
            a = 0.5 * rng.standard_normal(shape)
        elif name.endswith("weight_g"):
            a = rng.uniform(0.5, 1.5, shape)
        elif name.endswith("weight_v"):
            a = rng.standard_normal(shape)
        else:   # Linear [out, in]
            s = 1.0 / np.sqrt(shape[1])
            if "to_out" in name or "ff.ff.2" in name:
                s *= 0.5
            a = s * rng.standard_normal(shape)
        t[name] = np.ascontiguousarray(a, np.float32)
    return t


class TaaeBlockView(C.Structure):
    """aria_taae_block_view, src/aria_sa3_dec.h:75-79 (same fields, same order)"""
    _fields_ = [(f, C.c_float) for f in ("pre_alpha", "qn_alpha", "kn_alpha", "ff_alpha")] + \
               [(f, C.c_void_p) for f in ("pre_gamma", "pre_beta", "qn_gamma", "qn_beta", "kn_gamma", "kn_beta",
                                          "ff_gamma", "ff_beta", "to_qkv", "to_out", "ff_in_w", "ff_in_b",
                                          "ff_out_w", "ff_out_b")]


class DecView(C.Structure):
    """aria_sa3_dec_view, src/aria_sa3_dec.h:80-84"""
    _fields_ = [("running_std", C.c_float)] + \
               [(f, C.c_void_p) for f in ("proj_w", "proj_b", "new_tokens", "mapping_w", "mapping_b")] + \
               [("blocks", TaaeBlockView * 6)]


def fold_mapping(g, v):
    """The weight-normalised mapping conv folded as the reference's loader folds it
    (src/aria_sa3_dec.c:268-282): per output row, scale = (float)(g / sqrt(sum v^2)) with the
    sum and quotient in double, then v * scale in float. Returns [512, 768 * 3]."""
    v2 = np.ascontiguousarray(v, np.float32).reshape(v.shape[0], -1)
    ss = np.sum(v2.astype(np.float64) ** 2, axis=1)
    sc = (np.asarray(g, np.float64).reshape(-1) / np.sqrt(ss)).astype(np.float32)
    return np.ascontiguousarray(v2 * sc[:, None], np.float32)


def view_from_tensors(t):
    """(view, keep): a DecView over fp32 arrays taken from the checkpoint tensors ``t``
    (name -> array, the names aria_sa3_dec_load reads, src/aria_sa3_dec.c:242-266); ``keep``
    holds the arrays the view points into and must outlive the create call."""
    keep = []

    def arr(name):
        a = np.ascontiguousarray(t[name], np.float32)
        keep.append(a)
        return a.ctypes.data

    def sca(name):
        return float(np.asarray(t[name], np.float32).reshape(-1)[0])

    v = DecView()
    v.running_std = sca(PFX + "bottleneck.running_std")
    v.proj_w = arr(PFX + "decoder.layers.1.weight")
    v.proj_b = arr(PFX + "decoder.layers.1.bias")
    v.new_tokens = arr(PFX + "decoder.layers.3.new_tokens")
    fw = fold_mapping(t[PFX + "decoder.layers.3.mapping.weight_g"], t[PFX + "decoder.layers.3.mapping.weight_v"])
    keep.append(fw)
    v.mapping_w = fw.ctypes.data
    v.mapping_b = arr(PFX + "decoder.layers.3.mapping.bias")
    for i in range(6):
        b, p = v.blocks[i], BLK % i
        b.pre_alpha, b.qn_alpha = sca(p + "pre_norm.alpha"), sca(p + "self_attn.q_norm.alpha")
        b.kn_alpha, b.ff_alpha = sca(p + "self_attn.k_norm.alpha"), sca(p + "ff_norm.alpha")
        b.pre_gamma, b.pre_beta = arr(p + "pre_norm.gamma"), arr(p + "pre_norm.beta")
        b.qn_gamma, b.qn_beta = arr(p + "self_attn.q_norm.gamma"), arr(p + "self_attn.q_norm.beta")
        b.kn_gamma, b.kn_beta = arr(p + "self_attn.k_norm.gamma"), arr(p + "self_attn.k_norm.beta")
        b.ff_gamma, b.ff_beta = arr(p + "ff_norm.gamma"), arr(p + "ff_norm.beta")
        b.to_qkv, b.to_out = arr(p + "self_attn.to_qkv.weight"), arr(p + "self_attn.to_out.weight")
        b.ff_in_w, b.ff_in_b = arr(p + "ff.ff.0.proj.weight"), arr(p + "ff.ff.0.proj.bias")
        b.ff_out_w, b.ff_out_b = arr(p + "ff.ff.2.weight"), arr(p + "ff.ff.2.bias")
    return v, keep


class Decoder:
    """The small-music decoder resident on the device (aria_cuda_dec)."""

    def __init__(self, view):
        self.h = lib().aria_cuda_dec_create(C.byref(view))
        if not self.h:
            raise HipError(f"aria_cuda_dec_create failed: {last_error()}")

    @classmethod
    def from_tensors(cls, t):
        v, keep = view_from_tensors(t)
        d = cls(v)
        del keep
        return d

    def forward(self, latent):
        """audio [2, T * 4096] from latent [256, T] (host arrays; synchronous)."""
        lat = np.ascontiguousarray(latent, np.float32)
        assert lat.ndim == 2 and lat.shape[0] == 256, lat.shape
        T = lat.shape[1]
        # the entry point returns nothing (src/aria_sa3_dec.h:109): a failed call leaves the
        # buffer as it was, so it starts as NaN and a failure shows as NaN left in it
        out = np.full((2, T * 4096), np.nan, np.float32)
        lib().aria_cuda_dec_forward(self.h, out.ctypes.data, lat.ctypes.data, T)
        if np.isnan(out[:, :1]).any() or np.isnan(out[:, -1:]).any():
            raise HipError(f"aria_cuda_dec_forward failed: {last_error()}")
        return out

    def forward_dev(self, daudio, dlatent, T):
        """the decode on device pointers, enqueued on ``self.stream`` (not waited for)"""
        check(lib().aria_hip_dec_forward_dev(self.h, daudio, dlatent, T), "aria_hip_dec_forward_dev")

    @property
    def stream(self):
        return lib().aria_hip_dec_stream(self.h)

    def workspace_bytes(self):
        return int(lib().aria_hip_dec_workspace_bytes(self.h))

    def free(self):
        if self.h:
            lib().aria_cuda_dec_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
