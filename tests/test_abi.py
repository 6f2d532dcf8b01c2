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


def test_struct_layouts(tmp_path):
    """The restated reference types are byte-compatible: sizes and offsets as the reference
    headers give them on x86-64 (src/aria_sa3_dit.h:40-48, 128-145, src/aria_steer.h:26-38)."""
    src = tmp_path / "layout.c"
    src.write_text("""
#include <stdio.h>
#include <stddef.h>
#include "aria_dit.h"
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n",
           sizeof(aria_dit_block_w), sizeof(aria_sa3_dit_view), offsetof(aria_sa3_dit_view, blocks),
           sizeof(aria_sa3_dit_req_view), offsetof(aria_sa3_dit_req_view, cross_ed),
           offsetof(aria_sa3_dit_req_view, steer), sizeof(aria_steer), sizeof(aria_steer_set),
           offsetof(aria_sa3_dit_req_view, has_local), sizeof(aria_dtype));
    return 0;
}
""")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [168, 88, 80, 96, 64, 88, 48, 16, 80, 4]
