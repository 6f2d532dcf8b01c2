"""Python host side of the DiT block on the MI355X backend (include/aria_dit.h).

``DitBlock`` packs one block's fp32 weights on the device (the reference's
aria_dit_block_w fields, PyTorch Linear layout) and runs the per-request cross K/V
projection and the block forward over B sequences through the C ABI. Buffers are
``aria_amd.device.DeviceArray``; the forward allocates nothing per call (one
workspace sized at construction).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import HipError, check, lib
from .device import DeviceArray

# src/aria_sa3_dit.h:40-48, same order
BLOCK_FIELDS = ("pre_norm", "cross_norm", "ff_norm", "sa_to_qkv", "sa_q_norm", "sa_k_norm", "sa_to_out",
                "ca_to_q", "ca_to_kv", "ca_q_norm", "ca_k_norm", "ca_to_out", "ff_in_w", "ff_in_b",
                "ff_out_w", "ff_out_b", "to_scale_shift_gate", "to_local0_w", "to_local0_b", "to_local2_w",
                "to_local2_b")


class BlockW(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in BLOCK_FIELDS]


# src/aria_quant.h:27-35
F32, F16, BF16, Q8, Q4, Q8A8, AUTO = range(7)
FFN_GLU, FFN_GELU = 0, 1

class DitBlock:
    """One DiT block resident on the device.

    weights: dict of float32 numpy arrays keyed by BLOCK_FIELDS (missing local-cond
    fields are fine). precision: Q4 (attention Q8 + FFN Q4), Q8, or F32/F16 (fp16).
    """

    def __init__(self, weights, dim, num_heads, inner, dim_ctx, ffn=FFN_GLU, precision=Q4, head_dim=64):
        L = lib()
        self._keep = {k: np.ascontiguousarray(v, np.float32) for k, v in weights.items() if v is not None}
        w = BlockW()
        for f in BLOCK_FIELDS:
            a = self._keep.get(f)
            setattr(w, f, a.ctypes.data if a is not None else None)
        self.h = L.aria_hip_dit_block_create(C.addressof(w), dim, num_heads, head_dim, inner, ffn, dim_ctx,
                                             precision)
        self._keep = None   # the device holds packed copies
        if not self.h:
            from . import last_error
            raise HipError(f"aria_hip_dit_block_create failed: {last_error()}")
        self.dim, self.H, self.inner, self.dim_ctx, self.ffn = dim, num_heads, inner, dim_ctx, ffn
        self.ws = None
        self.ws_key = None

    @property
    def weight_bytes(self):
        return int(lib().aria_hip_dit_block_weight_bytes(self.h))

    def workspace(self, B, S, Sc):
        n = int(lib().aria_hip_dit_block_workspace_bytes(self.h, B, S, Sc))
        if self.ws is None or self.ws.nbytes < n:
            self.ws = DeviceArray(n, np.uint8)
        return self.ws

    def cross_kv(self, dctx: DeviceArray, B, Sc, stream=None):
        dk = DeviceArray((B, self.H, Sc, 64), np.float16)
        dv = DeviceArray((B, self.H, Sc, 64), np.float16)
        ws = self.workspace(B, 0, Sc)
        check(lib().aria_hip_dit_block_cross_kv_dev(self.h, dctx.p, B, Sc, dk.p, dv.p, ws.p, ws.nbytes, stream),
              "aria_hip_dit_block_cross_kv_dev")
        return dk, dv

    def forward(self, dx: DeviceArray, B, S, dgcond, dk, dv, Sc, dcos, dsin, rot, ws=None, stream=None):
        ws = ws or self.workspace(B, S, Sc)
        check(lib().aria_hip_dit_block_forward_dev(self.h, dx.p, B, S, dgcond.p if dgcond is not None else None,
                                                   dk.p, dv.p, Sc, dcos.p if dcos is not None else None,
                                                   dsin.p if dsin is not None else None, rot, ws.p, ws.nbytes,
                                                   stream), "aria_hip_dit_block_forward_dev")

    def free(self):
        if self.h:
            lib().aria_hip_dit_block_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def random_block_weights(rng, dim, inner, dim_ctx, ffn=FFN_GLU, w_sigma=0.02, gain_sigma=0.02):
    """Config-4 synthetic weights: projections ~N(0, w_sigma), norm gains 1 + N(0, gain_sigma),
    biases N(0, w_sigma), to_scale_shift_gate zero (the modulation comes from gcond)."""
    def n(shape, s=w_sigma):
        return (s * rng.standard_normal(shape)).astype(np.float32)
    ffrows = 2 * inner if ffn == FFN_GLU else inner
    return {
        "pre_norm": (1 + n(dim, gain_sigma)), "cross_norm": (1 + n(dim, gain_sigma)),
        "ff_norm": (1 + n(dim, gain_sigma)),
        "sa_to_qkv": n((3 * dim, dim)), "sa_q_norm": (1 + n(64, gain_sigma)), "sa_k_norm": (1 + n(64, gain_sigma)),
        "sa_to_out": n((dim, dim)), "ca_to_q": n((dim, dim)), "ca_to_kv": n((2 * dim, dim_ctx)),
        "ca_q_norm": (1 + n(64, gain_sigma)), "ca_k_norm": (1 + n(64, gain_sigma)), "ca_to_out": n((dim, dim)),
        "ff_in_w": n((ffrows, dim)), "ff_in_b": n(ffrows), "ff_out_w": n((dim, inner)), "ff_out_b": n(dim),
        "to_scale_shift_gate": np.zeros(6 * dim, np.float32),
    }
