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
    fields are fine). precision: Q4 (attention Q8 + FFN Q4), Q8, Q8A8 (all Q8 with int8
    activations, W8A8), or F32/F16 (fp16).
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


# ---------------------------------------------------------------------------
# the whole denoiser: the reference's aria_cuda_dit_* ABI (src/aria_sa3_dit.h:127-171)
# ---------------------------------------------------------------------------

class DitView(C.Structure):
    """aria_sa3_dit_view, src/aria_sa3_dit.h:128-133"""
    _fields_ = [(f, C.c_int) for f in ("depth", "ed", "num_heads", "head_dim", "inner", "io_ch", "n_mem",
                                       "rot_dim", "differential")] + \
               [(f, C.c_void_p) for f in ("preprocess", "postprocess", "project_in", "project_out",
                                          "memory_tokens", "blocks")]


class ReqView(C.Structure):
    """aria_sa3_dit_req_view, src/aria_sa3_dit.h:136-145"""
    _fields_ = [(f, C.c_int) for f in ("T", "S", "n_cond", "depth")] + \
               [(f, C.c_void_p) for f in ("global_seconds", "rope_cos", "rope_sin", "cross_k", "cross_v",
                                          "cross_kd", "cross_ed", "local_emb")] + \
               [("has_local", C.c_int), ("steer", C.c_void_p)]


NOISE_FN = C.CFUNCTYPE(None, C.POINTER(C.c_float), C.c_int, C.c_void_p)
PROGRESS_FN = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)


def _ptr_array(arrs):
    a = (C.c_void_p * len(arrs))(*[x.ctypes.data for x in arrs])
    return a


class Dit:
    """The SA3 diffusion transformer resident on the device (aria_cuda_dit).

    model: dict with 'preprocess' [C,C], 'postprocess' [C,C], 'project_in' [ed,C],
    'project_out' [C,ed], 'memory_tokens' [n_mem, ed] (fp32) and 'blocks' (a list of
    block weight dicts keyed by BLOCK_FIELDS, SiLU-GLU FFN, ca_to_kv [2*ed, ed]).
    """

    def __init__(self, model, depth, ed, num_heads, inner, io_ch, n_mem, rot_dim, precision=Q4, ffn=FFN_GLU):
        L = lib()
        keep = {k: np.ascontiguousarray(model[k], np.float32) for k in
                ("preprocess", "postprocess", "project_in", "project_out", "memory_tokens") if model.get(k) is not None}
        bw = (BlockW * depth)()
        bkeep = []
        for b in range(depth):
            kb = {k: np.ascontiguousarray(v, np.float32) for k, v in model["blocks"][b].items() if v is not None}
            bkeep.append(kb)
            for f in BLOCK_FIELDS:
                a = kb.get(f)
                setattr(bw[b], f, a.ctypes.data if a is not None else None)
        v = DitView(depth=depth, ed=ed, num_heads=num_heads, head_dim=64, inner=inner, io_ch=io_ch, n_mem=n_mem,
                    rot_dim=rot_dim, differential=0, blocks=C.addressof(bw))
        for k, a in keep.items():
            setattr(v, k, a.ctypes.data)
        if ffn == FFN_GLU:
            self.h = L.aria_cuda_dit_create(C.byref(v), precision)
        else:
            self.h = L.aria_hip_dit_create_ex(C.byref(v), precision, ffn)
        if not self.h:
            from . import last_error
            raise HipError(f"aria_cuda_dit_create failed: {last_error()}")
        self.depth, self.ed, self.H, self.io_ch, self.n_mem, self.rot = depth, ed, num_heads, io_ch, n_mem, rot_dim
        self.B = self.T = 0

    def _views(self, T, cross_ed, rope_cos, rope_sin, local, cross_kv):
        S = self.n_mem + T
        views = (ReqView * len(cross_ed))()
        self._req_keep = []
        for i, ced in enumerate(cross_ed):
            rv = views[i]
            rv.T, rv.S, rv.depth = T, S, self.depth
            if rope_cos is not None:
                c = np.ascontiguousarray(rope_cos, np.float32)
                s = np.ascontiguousarray(rope_sin, np.float32)
                rv.rope_cos, rv.rope_sin = c.ctypes.data, s.ctypes.data
                self._req_keep += [c, s]
            if ced is not None:
                e = np.ascontiguousarray(ced, np.float32)
                rv.n_cond, rv.cross_ed = e.shape[0], e.ctypes.data
                self._req_keep.append(e)
            else:
                ks = [np.ascontiguousarray(k, np.float32) for k in cross_kv[i][0]]
                vs = [np.ascontiguousarray(v, np.float32) for v in cross_kv[i][1]]
                pk, pv = _ptr_array(ks), _ptr_array(vs)
                rv.n_cond = ks[0].shape[1]
                rv.cross_k, rv.cross_v = C.addressof(pk), C.addressof(pv)
                self._req_keep += ks + vs + [pk, pv]
            if local is not None and local[i] is not None:
                ls = [np.ascontiguousarray(a, np.float32) for a in local[i]]
                pl = _ptr_array(ls)
                rv.local_emb, rv.has_local = C.addressof(pl), 1
                self._req_keep += ls + [pl]
        self._req_keep.append(views)
        return views

    def set_request(self, T, cross_ed, rope_cos=None, rope_sin=None, local=None, cross_kv=None):
        """cross_ed: list of B context embeddings [n_cond, ed] (None -> cross_kv[i] = (K list, V list),
        host-projected [H, n_cond, 64] per block); local: list of B per-block [S, ed] lists or None."""
        views = self._views(T, cross_ed, rope_cos, rope_sin, local, cross_kv)
        B = len(views)
        if B == 1:
            from . import last_error
            lib().aria_cuda_dit_set_request(self.h, C.byref(views[0]))
            err = last_error()
            buf = C.c_void_p()
            if lib().aria_hip_dit_device_buffers(self.h, C.byref(buf), None, None) != 0:
                raise HipError(f"aria_cuda_dit_set_request failed: {err}")
        else:
            check(lib().aria_hip_dit_set_request_batch(self.h, views, B), "aria_hip_dit_set_request_batch")
        self.B, self.T = B, T
        self._req_keep = None

    def step(self, x, gcond):
        """x [B, io_ch, T], gcond [B, 6*ed] -> velocity [B, io_ch, T]"""
        x = np.ascontiguousarray(x, np.float32)
        g = np.ascontiguousarray(gcond, np.float32)
        v = np.empty_like(x)
        if self.B == 1:
            lib().aria_cuda_dit_step(self.h, v.ctypes.data, x.ctypes.data, g.ctypes.data)
        else:
            check(lib().aria_hip_dit_step_batch(self.h, v.ctypes.data, x.ctypes.data, g.ctypes.data),
                  "aria_hip_dit_step_batch")
        return v

    def sample(self, x, sched, gcond_all, noise, progress=None):
        """the device pingpong loop; noise(n) -> float32 [n] called once per step, in order"""
        x = np.ascontiguousarray(x, np.float32).copy()
        sched = np.ascontiguousarray(sched, np.float32)
        g = np.ascontiguousarray(gcond_all, np.float32)

        def _nz(buf, n, _user):
            np.ctypeslib.as_array(buf, (n,))[:] = noise(n)

        def _pg(i, n, _user):
            if progress:
                progress(i, n)
        nz, pg = NOISE_FN(_nz), PROGRESS_FN(_pg)
        rc = lib().aria_cuda_dit_sample(self.h, x.ctypes.data, sched.ctypes.data, len(sched) - 1, g.ctypes.data,
                                        C.cast(nz, C.c_void_p), None, C.cast(pg, C.c_void_p) if progress else None,
                                        None)
        if rc != 0:
            raise HipError("aria_cuda_dit_sample failed")
        return x

    def device_buffers(self):
        dx, dv, dg = C.c_void_p(), C.c_void_p(), C.c_void_p()
        check(lib().aria_hip_dit_device_buffers(self.h, C.byref(dx), C.byref(dv), C.byref(dg)),
              "aria_hip_dit_device_buffers")
        return dx.value, dv.value, dg.value

    def run(self, stream=None):
        check(lib().aria_hip_dit_run(self.h, stream), "aria_hip_dit_run")

    @property
    def graph_active(self):
        return bool(lib().aria_hip_dit_graph_active(self.h))

    def load_overlay(self, path):
        """Take the block GEMM weights from the reference's packed .aria overlay
        (aria_sa3_dit_quant_save's file) instead of quantising them at create."""
        check(lib().aria_hip_dit_load_overlay(self.h, str(path).encode()), "aria_hip_dit_load_overlay")

    def free(self):
        if self.h:
            lib().aria_cuda_dit_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def random_dit(rng, depth, ed, inner, io_ch, n_mem, w_sigma=0.02, ffn=FFN_GLU):
    """Synthetic SA3-shaped weights (random init; no checkpoint is available)."""
    def n(shape, s=w_sigma):
        return (s * rng.standard_normal(shape)).astype(np.float32)
    return {
        "preprocess": n((io_ch, io_ch), 0.05), "postprocess": n((io_ch, io_ch), 0.05),
        "project_in": n((ed, io_ch), 0.1), "project_out": n((io_ch, ed), 0.05),
        "memory_tokens": n((n_mem, ed), 1.0),
        "blocks": [random_block_weights(rng, ed, inner, ed, ffn=ffn) for _ in range(depth)],
    }
