"""CPU: the C-ABI library builds, loads, exports every symbol include/*.h declares, and
behaves as the reference's backend does without a device (no compute call is made)."""
from __future__ import annotations

import glob
import os
import re
import subprocess

import pytest

from conftest import ROOT

HDRS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for h in HDRS:
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\b(aria_\w+)\s*\(", src):
            # skip typedef'd callback parameter names and macro uses
            names.add(m.group(1))
    return names


def exported_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True)
    return {ln.split()[-1] for ln in out.stdout.splitlines() if " T " in ln}


@pytest.fixture(scope="module")
def libpath():
    import aria_amd
    assert os.path.exists(aria_amd.LIB_PATH), "libaria_hip.so missing: __graft_entry__.build()"
    return aria_amd.LIB_PATH


def test_headers_found():
    names = {os.path.basename(h) for h in HDRS}
    assert {"aria_gpu.h", "aria_hip.h"} <= names


def test_every_declared_symbol_is_exported(libpath):
    decl = declared_functions()
    exp = exported_symbols(libpath)
    missing = sorted(decl - exp)
    assert not missing, f"declared in include/*.h but not exported: {missing}"


def test_reference_gpu_abi_complete(libpath):
    """Every function of the reference's src/aria_gpu.h:19-61 is served."""
    ref_abi = """aria_cuda_available aria_cuda_recommended aria_cuda_int8_tc aria_cuda_device_info
    aria_cuda_meminfo aria_cuda_malloc aria_cuda_free aria_cuda_memcpy_h2d aria_cuda_memcpy_d2h
    aria_cuda_sync aria_cuda_linear_dev aria_cuda_linear aria_cuda_matmul aria_cuda_rmsnorm
    aria_cuda_gemma_rmsnorm aria_cuda_dynamic_tanh aria_cuda_softcap aria_cuda_silu
    aria_cuda_gelu_tanh aria_cuda_silu_gate aria_cuda_softmax aria_cuda_rope_apply
    aria_cuda_attention aria_cuda_conv1d""".split()
    exp = exported_symbols(libpath)
    assert not [s for s in ref_abi if s not in exp]


def test_python_signatures_cover_headers(libpath):
    import aria_amd
    assert declared_functions() <= set(aria_amd.SIGNATURES), \
        sorted(declared_functions() - set(aria_amd.SIGNATURES))
    aria_amd.lib()   # every signature resolves


def test_no_device_behaviour(libpath):
    """Without a GPU (this container) the backend reports absence instead of failing hard:
    available()=0 (src/aria_gpu.h:20), malloc -> NULL, extension calls -> ENODEV."""
    import aria_amd
    L = aria_amd.lib()
    if L.aria_cuda_available():
        pytest.skip("a HIP device is present")
    assert L.aria_cuda_recommended() == 0
    assert L.aria_cuda_int8_tc() == 0
    assert L.aria_hip_init() == -2
    assert not L.aria_cuda_malloc(1024)
    assert L.aria_hip_rmsnorm_dev(None, None, None, 1, 8, 1e-6, None) == -2
    assert "no HIP device" in aria_amd.last_error()
    assert aria_amd.device_info() == "no HIP device"
    # the DiT and decoder handles: NULL, so the reference's caller keeps its CPU path
    assert not L.aria_cuda_dit_create(None, 4)
    assert not L.aria_cuda_dec_create(None)
    assert not L.aria_cuda_dec_medium_create(None)
    assert L.aria_hip_dit_set_request_batch(None, None, 2) == -2


def test_oracle_is_not_linked_into_product(libpath):
    """The product library must not depend on the oracle or the compiled reference."""
    out = subprocess.run(["ldd", libpath], capture_output=True, text=True).stdout
    assert "oracle" not in out and "aria_ref" not in out
    exp = exported_symbols(libpath)
    assert not [s for s in exp if s.startswith("or_")]


# every field of each restated type (include/aria_dit.h), in declaration order
LAYOUT_FIELDS = {
    "aria_dit_block_w": ["pre_norm", "cross_norm", "ff_norm", "sa_to_qkv", "sa_q_norm", "sa_k_norm", "sa_to_out",
                         "ca_to_q", "ca_to_kv", "ca_q_norm", "ca_k_norm", "ca_to_out", "ff_in_w", "ff_in_b",
                         "ff_out_w", "ff_out_b", "to_scale_shift_gate", "to_local0_w", "to_local0_b",
                         "to_local2_w", "to_local2_b"],
    "aria_sa3_dit_view": ["depth", "ed", "num_heads", "head_dim", "inner", "io_ch", "n_mem", "rot_dim",
                          "differential", "preprocess", "postprocess", "project_in", "project_out",
                          "memory_tokens", "blocks"],
    "aria_sa3_dit_req_view": ["T", "S", "n_cond", "depth", "global_seconds", "rope_cos", "rope_sin", "cross_k",
                              "cross_v", "cross_kd", "cross_ed", "local_emb", "has_local", "steer"],
    "aria_steer": ["site", "op", "layer", "dir", "dim", "dir_norm2", "scale", "step_lo", "step_hi"],
    "aria_steer_set": ["items", "n"],
    "aria_taae_block_view": ["pre_alpha", "qn_alpha", "kn_alpha", "ff_alpha", "pre_gamma", "pre_beta", "qn_gamma",
                             "qn_beta", "kn_gamma", "kn_beta", "ff_gamma", "ff_beta", "to_qkv", "to_out", "ff_in_w",
                             "ff_in_b", "ff_out_w", "ff_out_b"],
    "aria_sa3_dec_view": ["running_std", "proj_w", "proj_b", "new_tokens", "mapping_w", "mapping_b", "blocks"],
}
DTYPE_VALUES = ["ARIA_F32", "ARIA_F16", "ARIA_BF16", "ARIA_Q8", "ARIA_Q4", "ARIA_Q8A8", "ARIA_DTYPE_AUTO"]


def _layout_program(includes):
    lines = ["#include <stdio.h>", "#include <stddef.h>"] + [f'#include "{h}"' for h in includes] + ["int main(void) {"]
    for t, fields in LAYOUT_FIELDS.items():
        lines.append(f'    printf("{t} %zu\\n", sizeof({t}));')
        for f in fields:
            lines.append(f'    printf("{t}.{f} %zu %zu\\n", offsetof({t}, {f}), sizeof((({t} *)0)->{f}));')
    lines.append('    printf("aria_dtype %zu\\n", sizeof(aria_dtype));')
    for v in DTYPE_VALUES:
        lines.append(f'    printf("{v} %d\\n", (int){v});')
    lines += ["    return 0;", "}"]
    return "\n".join(lines) + "\n"


def _layout(tmp_path, tag, includes, incdir):
    src = tmp_path / f"layout_{tag}.c"
    src.write_text(_layout_program(includes))
    exe = tmp_path / f"layout_{tag}"
    subprocess.run(["gcc", "-std=c11", "-D_GNU_SOURCE", "-w", "-I", incdir, str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()


REF_SRC = "/root/reference/src"


def test_struct_layouts(tmp_path):
    """The restated reference types are byte-compatible: every field's offset and size, each
    type's size and the aria_dtype values, compiled from include/aria_dit.h and from the
    reference's own headers (src/aria_sa3_dit.h:40-48, 128-145, src/aria_steer.h:26-38,
    src/aria_quant.h:27-35, src/aria_sa3_dec.h:75-84) by the same program. Where the reference
    tree is absent (the GPU box) the sizes measured from it are checked instead."""
    mine = _layout(tmp_path, "mine", ["aria_dit.h"], os.path.join(ROOT, "include"))
    if os.path.exists(os.path.join(REF_SRC, "aria_sa3_dit.h")):
        theirs = _layout(tmp_path, "ref", ["aria_sa3_dit.h", "aria_sa3_dec.h"], REF_SRC)
        assert mine == theirs, [(a, b) for a, b in zip(mine, theirs) if a != b]
    got = dict(ln.rsplit(" ", 1) if ln.count(" ") == 1 else (ln, "") for ln in mine)
    assert [int(got[t]) for t in ("aria_dit_block_w", "aria_sa3_dit_view", "aria_sa3_dit_req_view", "aria_steer",
                                  "aria_steer_set", "aria_taae_block_view", "aria_sa3_dec_view", "aria_dtype")] \
        == [168, 88, 96, 48, 16, 128, 816, 4]


def test_reference_callers_link_against_backend(libpath):
    """The drop-in: the reference's own library sources and CLI (src/main.c), compiled with
    -DARIA_CUDA as its `cuda` target does (Makefile:175-191), and its device parity program
    tests/test_cuda.c link against libaria_hip.so with --no-undefined in place of
    aria_cuda.o -lcudart -lcublas (oracle/Makefile `dropin`). Every device symbol those
    callers use is one the backend exports, and test_cuda skips cleanly without a device."""
    import oracle
    if os.path.exists(os.path.join(REF_SRC, "aria_model_sa3.c")):
        subprocess.run(["make", "-s", "-C", os.path.dirname(oracle.__file__), "-j8", "dropin"], check=True)
    cli = os.path.join(oracle.DROPIN, "aria")
    tc = os.path.join(oracle.DROPIN, "test_cuda_hip")
    if not (os.path.exists(cli) and os.path.exists(tc)):
        pytest.skip("drop-in binaries not built (reference tree absent)")
    exp = exported_symbols(libpath)
    for exe in (cli, tc):
        und = subprocess.run(["nm", "-u", exe], capture_output=True, text=True, check=True).stdout.split()
        dev = {s for s in und if s.startswith("aria_cuda_")}
        assert dev and not (dev - exp), sorted(dev - exp)
        ldd = subprocess.run(["ldd", exe], capture_output=True, text=True).stdout
        assert "libaria_hip.so" in ldd and "not found" not in ldd, ldd
    cli_und = set(subprocess.run(["nm", "-u", cli], capture_output=True, text=True).stdout.split())
    # the DiT/decoder seam of src/aria_model_sa3.c:487-510, 569-601, 634-656
    assert {"aria_cuda_dit_create", "aria_cuda_dit_set_request", "aria_cuda_dit_step", "aria_cuda_dit_sample",
            "aria_cuda_dec_create", "aria_cuda_int8_tc", "aria_cuda_recommended"} <= cli_und
    import aria_amd
    if aria_amd.lib().aria_cuda_available():
        pytest.skip("a HIP device is present (tests/test_gpu_dropin.py runs test_cuda there)")
    out = subprocess.run([tc], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "SKIP" in out.stdout, out.stdout
