"""TEST INFRASTRUCTURE ONLY: the small-music taae_v2 decoder's CPU checkers.

* ``RefDecoder``  the reference's own CPU decoder (src/aria_sa3_dec.c, src/aria_taae.c)
  from oracle/_ref/libaria_ref.so, loaded by the reference's loader
  (aria_sa3_dec_load, src/aria_sa3_dec.c:238-285) from a safetensors file that
  ``write_safetensors`` writes; ``view()`` is its aria_sa3_dec_get_view
  (src/aria_sa3_dec.c:299-318), the struct the device decoder is created from.
* ``decode_np``   a numpy restatement of aria_sa3_dec_forward (src/aria_sa3_dec.c:47-128)
  and taae_block_forward / taae_chunk_pass (src/aria_taae.c:93-205), pinned against
  RefDecoder in tests/test_oracle.py; its stage outputs (``stages=True``) locate a
  device mismatch.
The synthetic checkpoints come from aria_amd.dec.random_tensors (the reference's tensor
names and shapes; no checkpoint is available here).

Only tests/ and bench.py's cpu_baseline leg use this module.
"""
from __future__ import annotations

import ctypes as C
import json
import struct

import numpy as np

D, H, HD, ROT, INNER, QKV, S = 768, 12, 64, 32, 2304, 3840, 34
PFX = "pretransform.model."
BLK = PFX + "decoder.layers.3.transformers.%d."


def write_safetensors(path, tensors):
    """F32 safetensors: 8-byte little-endian header length, JSON header (padded with
    spaces so the data starts 64-byte aligned), then the tensors back to back."""
    hdr, off, blobs = {}, 0, []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, np.float32)
        hdr[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(hdr).encode()
    h += b" " * ((-(8 + len(h))) % 64)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


# ---- the reference's view structs (src/aria_sa3_dec.h:75-85), for aria_sa3_dec_get_view ----
class TaaeBlockView(C.Structure):
    _fields_ = [(f, C.c_float) for f in ("pre_alpha", "qn_alpha", "kn_alpha", "ff_alpha")] + \
               [(f, C.c_void_p) for f in ("pre_gamma", "pre_beta", "qn_gamma", "qn_beta", "kn_gamma", "kn_beta",
                                          "ff_gamma", "ff_beta", "to_qkv", "to_out", "ff_in_w", "ff_in_b",
                                          "ff_out_w", "ff_out_b")]


class DecView(C.Structure):
    _fields_ = [("running_std", C.c_float)] + \
               [(f, C.c_void_p) for f in ("proj_w", "proj_b", "new_tokens", "mapping_w", "mapping_b")] + \
               [("blocks", TaaeBlockView * 6)]


class RefDecoder:
    """The reference's CPU decoder over a safetensors file (kept open while in use: the
    loader borrows the weights from the file's mapping, src/aria_sa3_dec.c:224-231)."""

    def __init__(self, lib, path):
        self.L = lib
        L = lib
        L.safetensors_open.restype = C.c_void_p
        L.safetensors_open.argtypes = [C.c_char_p]
        L.safetensors_close.argtypes = [C.c_void_p]
        L.aria_sa3_dec_load.restype = C.c_void_p
        L.aria_sa3_dec_load.argtypes = [C.c_void_p]
        L.aria_sa3_dec_free.argtypes = [C.c_void_p]
        L.aria_sa3_dec_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.aria_sa3_dec_get_view.argtypes = [C.c_void_p, C.c_void_p]
        self.sf = L.safetensors_open(path.encode())
        if not self.sf:
            raise RuntimeError(f"safetensors_open({path}) failed")
        self.m = L.aria_sa3_dec_load(self.sf)
        if not self.m:
            L.safetensors_close(self.sf)
            raise RuntimeError("aria_sa3_dec_load failed")

    def forward(self, latent):
        """audio [2, T * 4096] from latent [256, T] (aria_sa3_dec_forward)."""
        lat = np.ascontiguousarray(latent, np.float32)
        T = lat.shape[1]
        out = np.empty((2, T * 4096), np.float32)
        self.L.aria_sa3_dec_forward(self.m, out.ctypes.data, lat.ctypes.data, T)
        return out

    def view(self):
        v = DecView()
        self.L.aria_sa3_dec_get_view(self.m, C.byref(v))
        return v

    def close(self):
        if self.m:
            self.L.aria_sa3_dec_free(self.m)
            self.m = None
        if self.sf:
            self.L.safetensors_close(self.sf)
            self.sf = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ---- numpy restatement ----
def fold_mapping(g, v):
    """Weight-norm fold of the mapping conv (src/aria_sa3_dec.c:268-282): per output row,
    scale = (float)(g / sqrt(sum v^2)) in double, then v * scale in float."""
    v2 = v.reshape(512, -1)
    ss = np.sum(v2.astype(np.float64) ** 2, axis=1)
    sc = (g.reshape(512).astype(np.float64) / np.sqrt(ss)).astype(np.float32)
    return (v2 * sc[:, None]).astype(np.float32)


def _dyt(x, a, g, b):
    return (np.tanh(np.float32(a) * x) * g + b).astype(np.float32)


def rope_tables(n=S):
    """aria_rope_freqs(n, 32, 10000) (src/aria_cpu.c:778-788): [n, 16] each."""
    i = np.arange(ROT // 2, dtype=np.float64)
    inv = 1.0 / np.power(10000.0, 2 * i / ROT)
    ang = np.arange(n, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _rope(x, c, s):
    """rotate-half on the first 32 dims of x [..., S, 64] (src/aria_cpu.c:790-809)"""
    y = x.copy()
    a, b = x[..., :16], x[..., 16:32]
    y[..., :16] = a * c - b * s
    y[..., 16:32] = b * c + a * s
    return y


def _softmax(x):
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def block_np(x, t, i):
    """taae_block_forward (src/aria_taae.c:93-162) on x [nch * 34, 768]; returns the new x."""
    p = BLK % i
    N = x.shape[0]
    nch = N // S
    sc = lambda n: float(t[p + n][0])
    h = _dyt(x, sc("pre_norm.alpha"), t[p + "pre_norm.gamma"], t[p + "pre_norm.beta"])
    qkv = h @ t[p + "self_attn.to_qkv.weight"].T
    heads = qkv.reshape(nch, S, 5, H, HD).transpose(2, 0, 3, 1, 4)   # [5, nch, H, S, 64]
    q, k, v, qd, kd = heads
    qa, ka = sc("self_attn.q_norm.alpha"), sc("self_attn.k_norm.alpha")
    qg, qb = t[p + "self_attn.q_norm.gamma"], t[p + "self_attn.q_norm.beta"]
    kg, kb = t[p + "self_attn.k_norm.gamma"], t[p + "self_attn.k_norm.beta"]
    c, s = rope_tables()
    q, qd = _rope(_dyt(q, qa, qg, qb), c, s), _rope(_dyt(qd, qa, qg, qb), c, s)
    k, kd = _rope(_dyt(k, ka, kg, kb), c, s), _rope(_dyt(kd, ka, kg, kb), c, s)
    ob = _softmax(q @ k.transpose(0, 1, 3, 2) * np.float32(0.125)) @ v
    od = _softmax(qd @ kd.transpose(0, 1, 3, 2) * np.float32(0.125)) @ v
    merged = (ob - od).transpose(0, 2, 1, 3).reshape(N, D)
    x = x + merged @ t[p + "self_attn.to_out.weight"].T
    h = _dyt(x, sc("ff_norm.alpha"), t[p + "ff_norm.gamma"], t[p + "ff_norm.beta"])
    proj = h @ t[p + "ff.ff.0.proj.weight"].T + t[p + "ff.ff.0.proj.bias"]
    val, gate = proj[:, :INNER], proj[:, INNER:]
    gated = val * (gate / (np.float32(1) + np.exp(-gate)))
    return (x + (gated @ t[p + "ff.ff.2.weight"].T + t[p + "ff.ff.2.bias"])).astype(np.float32)


def decode_np(t, latent, stages=False):
    """aria_sa3_dec_forward: latent [256, T] -> audio [2, T * 4096]; with stages, also a
    dict of the intermediates (x [T, 768], seq after each pass [L, 768], mapped [T*16, 512])."""
    T = latent.shape[1]
    st = {}
    z = latent.astype(np.float32) * np.float32(t[PFX + "bottleneck.running_std"][0])
    x = z.T @ t[PFX + "decoder.layers.1.weight"].T + t[PFX + "decoder.layers.1.bias"]
    st["x"] = x
    Tp = T + (T & 1)
    L = 17 * Tp
    seq = np.empty((L, D), np.float32)
    seq[:] = t[PFX + "decoder.layers.3.new_tokens"]
    seq[0::17] = 0.0
    seq[0:17 * T:17] = x
    for i in range(3):
        seq = block_np(seq, t, i)
    st["pass1"] = seq
    pad = np.concatenate([seq[:17], seq, seq[-17:]])
    for i in range(3, 6):
        pad = block_np(pad, t, i)
    seq = pad[17:17 + L]
    st["pass2"] = seq
    Lout, Lt = 16 * Tp, 16 * T
    pos = np.arange(Lout)
    feat = seq[(pos // 16) * 17 + 1 + pos % 16]                      # [Lout, 768]
    fz = np.concatenate([np.zeros((1, D), np.float32), feat, np.zeros((1, D), np.float32)])
    xc = np.stack([fz[0:Lout], fz[1:Lout + 1], fz[2:Lout + 2]], axis=2).reshape(Lout, 3 * D)
    W = fold_mapping(t[PFX + "decoder.layers.3.mapping.weight_g"], t[PFX + "decoder.layers.3.mapping.weight_v"])
    mapped = (xc @ W.T + t[PFX + "decoder.layers.3.mapping.bias"])[:Lt]
    st["mapped"] = mapped
    audio = mapped.reshape(Lt, 2, 256).transpose(1, 0, 2).reshape(2, Lt * 256)
    return (audio, st) if stages else audio
