"""aria_amd - MI355X (gfx950) backend for aria's DiT tensor-op hot path.

The product is the C-ABI shared library ``aria_amd/libaria_hip.so`` (C host code
``csrc/aria_hip.c`` + hand-written gfx950 kernels ``csrc/*.hip``), declared in
``include/aria_gpu.h`` (the reference's GPU ABI) and ``include/aria_hip.h``
(device-pointer extension). This package is the Python host side above that
ABI: it loads the library with ctypes (``lib()``), and ``aria_amd.ops`` /
``aria_amd.device`` give numpy-facing calls that mirror the reference's
``aria_ops.h`` / ``aria_quant.h`` names.

There is no CPU fallback: when the library is missing every call raises.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaria_hip.so")
CSRC = os.path.join(HERE, "csrc")

_P = C.c_void_p
_F = C.POINTER(C.c_float)
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t

# name -> (restype, argtypes); every symbol declared in include/aria_gpu.h and include/aria_hip.h
SIGNATURES = {
    # include/aria_gpu.h
    "aria_cuda_available": (_i, []),
    "aria_cuda_recommended": (_i, []),
    "aria_cuda_int8_tc": (_i, []),
    "aria_cuda_device_info": (None, [C.c_char_p, _sz]),
    "aria_cuda_meminfo": (None, [C.POINTER(_sz), C.POINTER(_sz)]),
    "aria_cuda_malloc": (_P, [_sz]),
    "aria_cuda_free": (None, [_P]),
    "aria_cuda_memcpy_h2d": (None, [_P, _P, _sz]),
    "aria_cuda_memcpy_d2h": (None, [_P, _P, _sz]),
    "aria_cuda_sync": (None, []),
    "aria_cuda_linear_dev": (None, [_P, _P, _P, _P, _i, _i, _i]),
    "aria_cuda_linear": (None, [_P, _P, _P, _P, _i, _i, _i]),
    "aria_cuda_matmul": (None, [_P, _P, _P, _i, _i, _i]),
    "aria_cuda_rmsnorm": (None, [_P, _P, _P, _i, _i, _f]),
    "aria_cuda_gemma_rmsnorm": (None, [_P, _P, _P, _i, _i, _f]),
    "aria_cuda_dynamic_tanh": (None, [_P, _P, _f, _P, _P, _i, _i]),
    "aria_cuda_softcap": (None, [_P, _i, _f]),
    "aria_cuda_silu": (None, [_P, _i]),
    "aria_cuda_gelu_tanh": (None, [_P, _i]),
    "aria_cuda_silu_gate": (None, [_P, _P, _P, _i]),
    "aria_cuda_softmax": (None, [_P, _i, _i, _P]),
    "aria_cuda_rope_apply": (None, [_P, _P, _P, _i, _i, _i, _i]),
    "aria_cuda_attention": (None, [_P, _P, _P, _P, _i, _i, _i, _i, _P]),
    "aria_cuda_conv1d": (None, [_P, _P, _P, _P, _i, _i, _i, _i, _i]),
    # include/aria_hip.h: runtime
    "aria_hip_init": (_i, []),
    "aria_hip_last_error": (C.c_char_p, []),
    "aria_hip_default_stream": (_P, []),
    "aria_hip_stream_sync": (_i, [_P]),
    "aria_hip_stream_create": (_P, []),
    "aria_hip_stream_destroy": (None, [_P]),
    "aria_hip_event_create": (_P, []),
    "aria_hip_event_destroy": (None, [_P]),
    "aria_hip_event_record": (_i, [_P, _P]),
    "aria_hip_event_elapsed_ms": (_f, [_P, _P]),
    "aria_hip_memcpy_h2d_async": (_i, [_P, _P, _sz, _P]),
    "aria_hip_memcpy_d2h_async": (_i, [_P, _P, _sz, _P]),
    "aria_hip_memcpy_d2d_async": (_i, [_P, _P, _sz, _P]),
    "aria_hip_cu_count": (_i, []),
    "aria_hip_arch": (_i, [C.c_char_p, _sz]),
    # include/aria_hip.h: device-pointer ops
    "aria_hip_rmsnorm_dev": (_i, [_P, _P, _P, _i, _i, _f, _P]),
    "aria_hip_gemma_rmsnorm_dev": (_i, [_P, _P, _P, _i, _i, _f, _P]),
    "aria_hip_layernorm_dev": (_i, [_P, _P, _P, _P, _i, _i, _f, _P]),
    "aria_hip_rmsnorm_adaln_dev": (_i, [_P, _i, _P, _P, _P, _P, _i, _i, _i, _f, _P]),
    "aria_hip_ln_mod_gelu_res_dev": (_i, [_P, _P, _P, _P, _P, _P, _i, _i, _i, _f, _P]),
    "aria_hip_add_dev": (_i, [_P, _P, _P, _sz, _P]),
    "aria_hip_axpy_dev": (_i, [_P, _P, _f, _sz, _P]),
    "aria_hip_scale_dev": (_i, [_P, _P, _f, _sz, _P]),
    "aria_hip_gelu_tanh_dev": (_i, [_P, _P, _sz, _P]),
    "aria_hip_silu_dev": (_i, [_P, _P, _sz, _P]),
    "aria_hip_silu_gate_dev": (_i, [_P, _P, _P, _sz, _P]),
    "aria_hip_modulate_dev": (_i, [_P, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_gate_residual_dev": (_i, [_P, _P, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_glu_combine_dev": (_i, [_P, _i, _P, _P, _i, _i, _P]),
    "aria_hip_pingpong_dev": (_i, [_P, _P, _P, _f, _f, _sz, _P]),
    "aria_hip_softmax_dev": (_i, [_P, _i, _i, _P, _P]),
    "aria_hip_rope_apply_dev": (_i, [_P, _P, _P, _i, _i, _i, _i, _P]),
    "aria_hip_rope_apply2_dev": (_i, [_P, _P, _P, _P, _i, _i, _i, _i, _P]),
    "aria_hip_q8_quant_dev": (_i, [_P, _P, _P, _i, _i, _P]),
    "aria_hip_q4_quant_dev": (_i, [_P, _P, _P, _i, _i, _P]),
    "aria_hip_q8_dequant_dev": (_i, [_P, _P, _P, _i, _i, _P]),
    "aria_hip_q4_dequant_dev": (_i, [_P, _P, _P, _i, _i, _P]),
    "aria_hip_qlinear_dev": (_i, [_P, _i, _P, _i, _i, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_rmsnorm_adaln_q8_dev": (_i, [_P, _P, _P, _P, _P, _P, _i, _i, _i, _f, _P]),
    "aria_hip_quant_act_q8_dev": (_i, [_P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_gemm_i8_dev": (_i, [_P, _i, _P, _P, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_q8a8_ws_bytes": (_sz, [_i, _i]),
    "aria_hip_linear_q8a8_dev": (_i, [_P, _P, _i, _P, _P, _P, _i, _i, _i, _P, _P]),
    "aria_hip_qlinear_ex_dev": (_i, [_P, _i, _P, _i, _i, _P, _P, _P, _i, _i, _i, _i, _P]),
    "aria_hip_linear_q8_dev": (_i, [_P, _P, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_qlinear_noalloc_dev": (_i, [_P, _i, _P, _i, _i, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_linear_q4_dev": (_i, [_P, _P, _P, _P, _P, _i, _i, _i, _P]),
    "aria_hip_qkv_prep_dev": (_i, [_P, _i, _i, _i, _i, _i, _P, _P, _P, _P, _P, _i, _f, _P]),
    "aria_hip_flash_attention_dev": (_i, [_P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _P]),
    "aria_hip_attention_f16": (_i, [_P, _P, _P, _P, _i, _i, _i, _i, _i]),
    # include/aria_dit.h
    "aria_hip_dit_block_create": (_P, [_P, _i, _i, _i, _i, _i, _i, _i]),
    "aria_hip_dit_block_free": (None, [_P]),
    "aria_hip_dit_block_weight_bytes": (_sz, [_P]),
    "aria_hip_dit_block_workspace_bytes": (_sz, [_P, _i, _i, _i]),
    "aria_hip_dit_block_cross_kv_dev": (_i, [_P, _P, _i, _i, _P, _P, _P, _sz, _P]),
    "aria_hip_dit_block_forward_dev": (_i, [_P, _P, _i, _i, _P, _P, _P, _i, _P, _P, _i, _P, _sz, _P]),
    "aria_cuda_dit_create": (_P, [_P, _i]),
    "aria_cuda_dit_free": (None, [_P]),
    "aria_cuda_dit_set_request": (None, [_P, _P]),
    "aria_cuda_dit_set_step": (None, [_P, _i]),
    "aria_cuda_dit_step": (None, [_P, _P, _P, _P]),
    "aria_cuda_dit_sample": (_i, [_P, _P, _P, _i, _P, _P, _P, _P, _P]),
    "aria_hip_dit_create_ex": (_P, [_P, _i, _i]),
    "aria_hip_dit_set_request_batch": (_i, [_P, _P, _i]),
    "aria_hip_dit_step_batch": (_i, [_P, _P, _P, _P]),
    "aria_hip_dit_device_buffers": (_i, [_P, _P, _P, _P]),
    "aria_hip_dit_run": (_i, [_P, _P]),
    "aria_hip_dit_graph_active": (_i, [_P]),
    "aria_hip_dit_load_overlay": (_i, [_P, C.c_char_p]),
    "aria_cuda_dec_create": (_P, [_P]),
    "aria_cuda_dec_free": (None, [_P]),
    "aria_cuda_dec_forward": (None, [_P, _P, _P, _i]),
    "aria_cuda_dec_medium_create": (_P, [_P]),
    "aria_cuda_dec_medium_free": (None, [_P]),
    "aria_cuda_dec_medium_forward": (None, [_P, _P, _P, _i]),
    "aria_hip_dec_forward_dev": (_i, [_P, _P, _P, _i]),
    "aria_hip_dec_stream": (_P, [_P]),
    "aria_hip_dec_workspace_bytes": (_sz, [_P]),
    # include/aria_hip.h: host-pointer forms
    "aria_hip_linear_q8": (_i, [_P, _P, _P, _P, _P, _i, _i, _i]),
    "aria_hip_linear_q8a8": (_i, [_P, _P, _P, _P, _P, _i, _i, _i]),
    "aria_hip_linear_q4": (_i, [_P, _P, _P, _P, _P, _i, _i, _i]),
    "aria_hip_q8_quant": (_i, [_P, _P, _P, _i, _i]),
    "aria_hip_q4_quant": (_i, [_P, _P, _P, _i, _i]),
    "aria_hip_q8_dequant": (_i, [_P, _P, _P, _i, _i]),
    "aria_hip_q4_dequant": (_i, [_P, _P, _P, _i, _i]),
    "aria_hip_layernorm": (_i, [_P, _P, _P, _P, _i, _i, _f]),
    "aria_hip_rmsnorm_adaln": (_i, [_P, _P, _P, _P, _P, _i, _i, _i, _f]),
    "aria_hip_ln_mod_gelu_res": (_i, [_P, _P, _P, _P, _P, _P, _i, _i, _i, _f]),
    "aria_hip_modulate": (_i, [_P, _P, _P, _P, _i, _i, _i]),
    "aria_hip_gate_residual": (_i, [_P, _P, _P, _P, _P, _i, _i, _i]),
    "aria_hip_glu_combine": (_i, [_P, _P, _P, _i, _i]),
    "aria_hip_add": (_i, [_P, _P, _P, _sz]),
    "aria_hip_pingpong": (_i, [_P, _P, _P, _f, _f, _sz]),
}

_lib = None


class HipError(RuntimeError):
    pass


def build(clean: bool = True) -> None:
    """Compile every HIP kernel for gfx950 plus the C host backend into libaria_hip.so."""
    global _lib
    if clean:
        subprocess.run(["make", "-s", "-C", CSRC, "clean"], check=True)
    jobs = str(min(16, os.cpu_count() or 4))
    subprocess.run(["make", "-s", "-C", CSRC, "-j" + jobs], check=True)
    _lib = None


def lib() -> C.CDLL:
    """The loaded backend; raises when it has not been built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def available() -> bool:
    """True when the library loads and a HIP device is usable."""
    try:
        return bool(lib().aria_cuda_available())
    except (HipError, OSError):
        return False


def last_error() -> str:
    s = lib().aria_hip_last_error()
    return s.decode() if s else ""


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise HipError(f"{what or 'aria_hip call'} failed ({rc}): {last_error()}")


def device_info() -> str:
    buf = C.create_string_buffer(256)
    lib().aria_cuda_device_info(buf, 256)
    return buf.value.decode()
