"""GPU parity of the device-resident DiT (the reference's aria_cuda_dit_* ABI, include/aria_dit.h).

Oracle, per sequence: the reference's own step composition (src/aria_sa3_dit.c:734-777) on the
CPU -- transpose, preprocess_conv + x, memory tokens + project_in, the depth blocks through the
compiled reference's aria_dit_block_forward on the dequantized weights (what dequant-on-use
computes), project_out, postprocess_conv + out, transpose -- with the reference's linear.
Gate: the reference's full-DiT gate, max|d| <= 2e-3 + 5e-3 * max|ref| (tests/test_dit_full.c:61).

The sampler is checked bit-exact against aria_cuda_dit_step + the host pingpong update, the
reference's own contract for aria_cuda_dit_sample (src/aria_sa3_dit.h:163-166); the captured
graph bit-exact against the inline step, over several replays with host work in between.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, randn, rng

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 5e-3
PNAME = {4: "q4", 3: "q8", 0: "f32", 5: "q8a8"}


@pytest.fixture
def R(ref):
    if ref is None:
        pytest.skip("oracle/_ref not built: the DiT oracle needs the compiled reference")
    return ref


def model(seed, depth=2, ed=128, inner=256, io_ch=16, n_mem=3):
    from aria_amd.dit import random_dit
    return random_dit(rng(seed), depth, ed, inner, io_ch, n_mem)


def make_dit(M, precision, H=2, rot=32):
    from aria_amd.dit import Dit
    ed = M["project_in"].shape[0]
    return Dit(M, len(M["blocks"]), ed, H, M["blocks"][0]["ff_out_w"].shape[1], M["project_in"].shape[1],
               M["memory_tokens"].shape[0], rot, precision=precision)


def ref_step(R, port, M, precision, x_CT, ced, gcond, c, s, rot, H, local=None, ffn=0):
    """velocity of one sequence on the CPU, src/aria_sa3_dit.c:734-777. SiLU-GLU blocks run the
    reference's aria_dit_block_forward; tanh-GELU blocks the pinned composition of reference ops,
    both on the dequantized weights with the reference's fp32 linear."""
    from oracle import dit_block as DB
    n_mem, ed = M["memory_tokens"].shape
    inner = M["blocks"][0]["ff_out_w"].shape[1]
    xtc = np.ascontiguousarray(x_CT.T)
    xtc = xtc + R.linear(xtc, M["preprocess"])
    seq = np.concatenate([M["memory_tokens"], R.linear(xtc, M["project_in"])]).astype(np.float32)
    for b, W in enumerate(M["blocks"]):
        packed = DB.pack_weights(R, W, PNAME[precision])
        if ffn == DB.FFN_GELU:
            Wd = DB.dequantized(port, W, packed)
            kc, vc = DB.cross_kv(R, ced, W, H)
            seq = DB.block_forward(R, port, seq, kc, vc, gcond, Wd, DB.pack_weights(R, Wd, "f32"), c, s, rot, H,
                                   DB.FFN_GELU)
        elif local is None and PNAME[precision] != "q8a8":
            seq = R.dit_block_forward(seq, ced, gcond, c, s, rot, DB.dequantized(port, W, packed), H, inner)
        else:
            kc, vc = DB.cross_kv(R, ced, W, H)
            seq = DB.block_forward(R, port, seq, kc, vc, gcond, W, packed, c, s, rot, H, DB.FFN_GLU,
                                   None if local is None else local[b])
    out = R.linear(np.ascontiguousarray(seq[n_mem:]), M["project_out"])
    out = out + R.linear(out, M["postprocess"])
    return np.ascontiguousarray(out.T)


def inputs(seed, B, io_ch, T, n_cond, ed):
    r = rng(seed)
    return randn(r, (B, io_ch, T)), randn(r, (B, n_cond, ed)), randn(r, (B, 6 * ed), 0.1)


@pytest.mark.parametrize("precision", [4, 3, 0])        # ARIA_Q4, ARIA_Q8, ARIA_F32 (fp16 storage)
def test_dit_step_parity(hip, port, R, precision):
    """aria_cuda_dit_step, batch 1, two teacher-forced steps on one request."""
    M = model(11 + precision)
    T, n_cond, H, rot = 40, 12, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    dit = make_dit(M, precision, H, rot)
    _, ced, _ = inputs(1, 1, io_ch, T, n_cond, ed)
    dit.set_request(T, [ced[0]], c, s)
    for k in range(2):
        x, _, g = inputs(100 + k, 1, io_ch, T, n_cond, ed)
        got = dit.step(x, g)
        want = ref_step(R, port, M, precision, x[0], ced[0], g[0], c, s, rot, H)
        assert_close(got[0], want, ATOL, RTOL, f"dit step {k} {PNAME[precision]}")
    dit.free()


def test_dit_step_parity_w8a8(hip, port, R):
    """aria_cuda_dit_step with ARIA_Q8A8 (int8 activations on every Q8 projection; at ed 256 the
    norms quantise in registers): against the composition of reference ops with aria_linear_q8a8."""
    M = model(17, ed=256, inner=512)
    T, n_cond, H, rot = 40, 12, 4, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    dit = make_dit(M, 5, H, rot)
    _, ced, _ = inputs(3, 1, io_ch, T, n_cond, ed)
    dit.set_request(T, [ced[0]], c, s)
    for k in range(2):
        x, _, g = inputs(200 + k, 1, io_ch, T, n_cond, ed)
        got = dit.step(x, g)
        want = ref_step(R, port, M, 5, x[0], ced[0], g[0], c, s, rot, H)
        assert_close(got[0], want, ATOL, RTOL, f"dit step {k} q8a8")
    dit.free()


def test_dit_batch_cfg_pair(hip, port, R):
    """aria_hip_dit_set_request_batch / step_batch: the CFG pair (two contexts) in one pass."""
    M = model(21)
    T, n_cond, H, rot = 33, 9, 2, 64
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    dit = make_dit(M, 4, H, rot)
    x, ced, g = inputs(2, 2, io_ch, T, n_cond, ed)
    dit.set_request(T, [ced[0], ced[1]], c, s)
    got = dit.step(x, g)
    for b in range(2):
        want = ref_step(R, port, M, 4, x[b], ced[b], g[b], c, s, rot, H)
        assert_close(got[b], want, ATOL, RTOL, f"cfg pair seq {b}")
    dit.free()


def test_dit_local_cond(hip, port, R):
    """inpaint local-additive cond: added per block after the cross-attention residual."""
    M = model(31)
    T, n_cond, H, rot = 24, 8, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    n_mem = M["memory_tokens"].shape[0]
    S = n_mem + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    r = rng(5)
    local = []
    for _ in M["blocks"]:
        a = np.zeros((S, ed), np.float32)
        a[n_mem:] = randn(r, (T, ed), 0.5)    # zeros at the memory-token rows, as the reference pads
        local.append(a)
    dit = make_dit(M, 4, H, rot)
    x, ced, g = inputs(3, 1, io_ch, T, n_cond, ed)
    dit.set_request(T, [ced[0]], c, s, local=[local])
    got = dit.step(x, g)
    want = ref_step(R, port, M, 4, x[0], ced[0], g[0], c, s, rot, H, local=local)
    assert_close(got[0], want, ATOL, RTOL, "dit local cond")
    # planted check: the same step without the local cond must differ beyond the gate
    plain = ref_step(R, port, M, 4, x[0], ced[0], g[0], c, s, rot, H)
    assert np.abs(plain - want).max() > ATOL + RTOL * np.abs(want).max()
    dit.free()


def test_dit_host_projected_kv(hip, port, R):
    """legacy request form: no cross_ed, per-block host K/V [H, n_cond, 64] (fp32 -> fp16 on upload)."""
    from oracle import dit_block as DB
    M = model(41)
    T, n_cond, H, rot = 20, 10, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    x, ced, g = inputs(4, 1, io_ch, T, n_cond, ed)
    ks, vs = [], []
    for W in M["blocks"]:
        k, v = DB.cross_kv(R, ced[0], W, H)
        ks.append(k); vs.append(v)
    dit = make_dit(M, 4, H, rot)
    dit.set_request(T, [None], c, s, cross_kv=[(ks, vs)])
    got = dit.step(x, g)
    want = ref_step(R, port, M, 4, x[0], ced[0], g[0], c, s, rot, H)
    assert_close(got[0], want, ATOL, RTOL, "dit host K/V")
    dit.free()


def test_dit_graph_matches_inline(hip, port, monkeypatch):
    """the captured step replays bit-identically to the inline step (ARIA_NO_GRAPH=1), across
    several replays with fresh inputs and host work in between; a warm-hit set_request
    (same context) keeps the graph."""
    M = model(51)
    T, n_cond, H, rot = 36, 8, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = port.rope_freqs(S, rot, 10000.0)
    _, ced, _ = inputs(6, 2, io_ch, T, n_cond, ed)
    monkeypatch.setenv("ARIA_NO_GRAPH", "1")
    inline = make_dit(M, 4, H, rot)
    inline.set_request(T, [ced[0], ced[1]], c, s)
    monkeypatch.delenv("ARIA_NO_GRAPH")
    graph = make_dit(M, 4, H, rot)
    graph.set_request(T, [ced[0], ced[1]], c, s)
    for k in range(3):
        x, _, g = inputs(200 + k, 2, io_ch, T, n_cond, ed)
        a = inline.step(x, g)
        b = graph.step(x, g)
        assert not inline.graph_active
        assert graph.graph_active, "the step was not captured"
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {k} differs from inline"
        np.sum(a * 1.0001)   # host work between replays
    graph.set_request(T, [ced[0], ced[1]], c, s)   # warm hit
    assert graph.graph_active
    x, _, g = inputs(300, 2, io_ch, T, n_cond, ed)
    assert np.array_equal(inline.step(x, g).view(np.uint32), graph.step(x, g).view(np.uint32))
    inline.free(); graph.free()


def test_dit_graph_capture_failure_falls_back(hip, port, monkeypatch):
    """A capture that fails (forced by ARIA_GRAPH_FAIL at create: the failure branch drops the
    captured graph, whose work never ran) leaves the handle on inline launches for good, with
    results bit-identical to ARIA_NO_GRAPH, over repeated steps and a new request."""
    M = model(52)
    T, n_cond, H, rot = 30, 8, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = port.rope_freqs(S, rot, 10000.0)
    _, ced, _ = inputs(9, 2, io_ch, T, n_cond, ed)
    monkeypatch.setenv("ARIA_NO_GRAPH", "1")
    inline = make_dit(M, 4, H, rot)
    monkeypatch.delenv("ARIA_NO_GRAPH")
    monkeypatch.setenv("ARIA_GRAPH_FAIL", "1")
    failing = make_dit(M, 4, H, rot)
    monkeypatch.delenv("ARIA_GRAPH_FAIL")
    for d in (inline, failing):
        d.set_request(T, [ced[0], ced[1]], c, s)
    for k in range(3):
        x, _, g = inputs(400 + k, 2, io_ch, T, n_cond, ed)
        a, b = inline.step(x, g), failing.step(x, g)
        assert not failing.graph_active
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {k} differs from inline"
    T2 = 22
    S2 = M["memory_tokens"].shape[0] + T2
    c2, s2 = port.rope_freqs(S2, rot, 10000.0)
    for d in (inline, failing):
        d.set_request(T2, [ced[0]], c2, s2)
    x, _, g = inputs(410, 1, io_ch, T2, n_cond, ed)
    assert np.array_equal(inline.step(x, g).view(np.uint32), failing.step(x, g).view(np.uint32))
    assert not failing.graph_active
    inline.free(); failing.free()


def test_dit_device_buffers_run(hip, port):
    """aria_hip_dit_device_buffers + aria_hip_dit_run: the step on HBM-resident buffers equals
    the host-buffer step bit for bit."""
    from aria_amd import lib
    M = model(61)
    T, n_cond, H, rot = 28, 8, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = port.rope_freqs(S, rot, 10000.0)
    x, ced, g = inputs(7, 1, io_ch, T, n_cond, ed)
    dit = make_dit(M, 4, H, rot)
    dit.set_request(T, [ced[0]], c, s)
    want = dit.step(x, g)
    dx, dv, dg = dit.device_buffers()
    L = lib()
    L.aria_cuda_memcpy_h2d(dx, x.ctypes.data, x.nbytes)
    L.aria_cuda_memcpy_h2d(dg, g.ctypes.data, g.nbytes)
    dit.run()
    L.aria_cuda_sync()
    got = np.empty_like(x)
    L.aria_cuda_memcpy_d2h(got.ctypes.data, dv, got.nbytes)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    dit.free()


def test_dit_sample_bitexact(hip, port):
    """aria_cuda_dit_sample == aria_cuda_dit_step + the host pingpong update, bit for bit,
    with the noise drawn in the same order."""
    M = model(71)
    T, n_cond, H, rot, steps = 30, 8, 2, 32, 5
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = port.rope_freqs(S, rot, 10000.0)
    x0, ced, _ = inputs(8, 1, io_ch, T, n_cond, ed)
    gall = randn(rng(9), (steps, 6 * ed), 0.1)
    sched = np.linspace(1.0, 0.0, steps + 1).astype(np.float32)
    dit = make_dit(M, 4, H, rot)
    dit.set_request(T, [ced[0]], c, s)

    def noise_stream(seed):
        r = rng(seed)
        return lambda n: r.standard_normal(n).astype(np.float32)

    seen = []
    got = dit.sample(x0[0], sched, gall, noise_stream(10), progress=lambda i, n: seen.append(i))
    assert seen == list(range(1, steps + 1))
    draw = noise_stream(10)
    x = x0[0].copy()
    for i in range(steps):
        v = dit.step(x[None], gall[i][None])[0]
        x = port.pingpong(x, v, draw(x.size).reshape(x.shape), sched[i], sched[i + 1])
    assert np.array_equal(got.view(np.uint32), x.view(np.uint32))
    dit.free()


def test_dit_sample_staging_failure(hip, port):
    """aria_cuda_dit_sample returns -1 without running when its staging cannot be reserved (the
    reference's caller then runs its host loop, src/aria_model_sa3.c:579-587): a schedule whose
    per-step gcond table would need terabytes fails the device reservation; no noise is drawn, x
    is untouched, and the handle samples normally afterwards."""
    import ctypes as C
    from aria_amd.dit import NOISE_FN
    M = model(72)
    T, n_cond, H, rot = 20, 8, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = port.rope_freqs(S, rot, 10000.0)
    x0, ced, _ = inputs(12, 1, io_ch, T, n_cond, ed)
    dit = make_dit(M, 4, H, rot)
    dit.set_request(T, [ced[0]], c, s)
    calls = []
    nz = NOISE_FN(lambda buf, n, user: calls.append(n))
    x = x0[0].copy()
    sched = np.linspace(1.0, 0.0, 3).astype(np.float32)
    g = randn(rng(13), (2, 6 * ed), 0.1)
    rc = hip.lib().aria_cuda_dit_sample(dit.h, x.ctypes.data, sched.ctypes.data, 1 << 30, g.ctypes.data,
                                        C.cast(nz, C.c_void_p), None, None, None)
    assert rc == -1 and not calls and np.array_equal(x, x0[0])
    draw = rng(14)
    got = dit.sample(x0[0], sched, g, lambda n: draw.standard_normal(n).astype(np.float32))
    assert np.isfinite(got).all() and not np.array_equal(got, x0[0])
    dit.free()


def test_dit_create_rejects(hip):
    """unsupported shapes return NULL with an error (the caller falls back to the CPU DiT)."""
    from aria_amd import HipError
    from aria_amd.dit import Dit
    M = model(81)
    with pytest.raises(HipError):
        Dit(M, 2, 128, 4, 256, 16, 3, 32)     # head_dim 32


def test_dit_config5_steps(hip, port, R):
    """Config 5 shape: 24 q4 blocks (config-4 block, tanh-GELU 4x FFN), T = 1296, batch 2,
    latent [2, 64, 1296], context [2, 256, 1024], 8 pingpong steps on the reference's LogSNR
    schedule (aria_build_schedule, src/aria_sampler.c:167-200) with per-step gcond and noise.
    The device step runs every step (graph replay) and the latent advances by the host
    pingpong update on the device velocity; at steps 0, 4 and 7 (the last) the CPU computes the
    velocity from the same step input (teacher forcing, tests/test_quant_dit.c:1-7), ~48 block
    forwards per checked step."""
    from aria_amd.dit import Dit, random_dit, FFN_GELU
    depth, ed, H, inner, C, T, Sc, rot, steps = 24, 1024, 16, 4096, 64, 1296, 256, 32, 8
    M = random_dit(rng(0xC5), depth, ed, inner, C, 0, ffn=FFN_GELU)
    c, s = R.rope_freqs(T, rot, 10000.0)
    x, ced, _ = inputs(0xC50, 2, C, T, Sc, ed)
    r = rng(0xC51)
    gall = randn(r, (steps, 2, 6 * ed), 0.1)
    noise = randn(r, (steps,) + x.shape)
    sched = R.build_schedule(steps)
    dit = Dit(M, depth, ed, H, inner, C, 0, rot, precision=4, ffn=FFN_GELU)
    dit.set_request(T, [ced[0], ced[1]], c, s)
    for i in range(steps):
        v = dit.step(x, gall[i])
        assert dit.graph_active
        if i in (0, 4, 7):
            for b in range(2):
                want = ref_step(R, port, M, 4, x[b], ced[b], gall[i][b], c, s, rot, H, ffn=FFN_GELU)
                d = np.abs(v[b] - want)
                print(f"config-5 step {i} seq {b}: max|d| {d.max():.3e} max|ref| {np.abs(want).max():.3f}", flush=True)
                assert_close(v[b], want, ATOL, RTOL, f"config-5 step {i} seq {b}")
        x = port.pingpong(x, v, noise[i], float(sched[i]), float(sched[i + 1]))
    dit.free()


def write_overlay(R, M, path, precision="q4"):
    """The reference's packed overlay file: the header as aria_sa3_dit_quant_save writes it
    (src/aria_sa3_dit.c:521-523), every record by the reference's own aria_qweight_write
    (src/aria_quant.c:439-449) on the reference quantizer's output, in the recipe's types."""
    import ctypes as C
    libc = C.CDLL(None)
    libc.fopen.restype = C.c_void_p
    libc.fopen.argtypes = [C.c_char_p, C.c_char_p]
    libc.fwrite.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
    libc.fclose.argtypes = [C.c_void_p]

    class QW(C.Structure):   # aria_qweight (src/aria_quant.h:76-83)
        _fields_ = [("dt", C.c_int), ("N", C.c_int), ("K", C.c_int), ("f32", C.c_void_p), ("q", C.c_void_p),
                    ("scale", C.c_void_p), ("a8", C.c_int)]
    R.lib.aria_qweight_write.argtypes = [C.c_void_p, C.c_void_p]
    R.lib.aria_qweight_write.restype = C.c_int
    blocks = M["blocks"]
    ed, inner = M["project_in"].shape[0], blocks[0]["ff_out_w"].shape[1]
    f = libc.fopen(str(path).encode(), b"wb")
    assert f
    keep = []
    try:
        libc.fwrite(b"ARIAQNT1", 1, 8, f)
        hdr = (C.c_int32 * 4)(4 if precision == "q4" else 3, len(blocks), ed, inner)
        libc.fwrite(hdr, 4, 4, f)
        for W in blocks:
            for name in ("sa_to_qkv", "sa_to_out", "ca_to_q", "ca_to_out", "ff_in_w", "ff_out_w"):
                w = np.ascontiguousarray(W[name], np.float32)
                if precision == "q4" and name.startswith("ff_"):
                    q, sc = R.q4_quant(w); dt = 4
                else:
                    q, sc = R.q8_quant(w); dt = 3
                keep += [q, sc]
                rec = QW(dt, w.shape[0], w.shape[1], None, q.ctypes.data, sc.ctypes.data, 0)
                assert R.lib.aria_qweight_write(f, C.byref(rec)) == 0
    finally:
        libc.fclose(f)


def test_dit_packed_overlay(hip, port, R, tmp_path):
    """aria_hip_dit_load_overlay (F3): the reference's .aria overlay loaded into the device model
    gives steps bit-identical to the model that packs the same f32 weights on the device (whose
    pack is bit-exact with the reference quantizer), with the captured step re-made; files that
    do not fit the model are refused and leave it working."""
    M = model(19)
    T, n_cond, H, rot = 24, 8, 2, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    path = tmp_path / "dit.aria"
    write_overlay(R, M, path)
    a, b = make_dit(M, 4, H, rot), make_dit(M, 4, H, rot)
    _, ced, _ = inputs(5, 1, io_ch, T, n_cond, ed)
    x, _, g = inputs(300, 1, io_ch, T, n_cond, ed)
    for d in (a, b):
        d.set_request(T, [ced[0]], c, s)
    y0 = b.step(x, g)                                      # captures b's step
    b.load_overlay(path)
    ya, yb = a.step(x, g), b.step(x, g)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)) and np.array_equal(ya.view(np.uint32), y0.view(np.uint32))
    # another model's file (depth differs) and a Q4 file for a W8A8 model are refused
    M3 = model(20, depth=3)
    bad = tmp_path / "depth3.aria"
    write_overlay(R, M3, bad)
    L = hip.lib()
    assert L.aria_hip_dit_load_overlay(b.h, str(bad).encode()) == -1
    assert np.array_equal(b.step(x, g).view(np.uint32), yb.view(np.uint32))
    M8 = model(21, ed=256, inner=512)
    w8 = make_dit(M8, 5, 4, rot)
    q4file = tmp_path / "q4.aria"
    write_overlay(R, M8, q4file)
    assert L.aria_hip_dit_load_overlay(w8.h, str(q4file).encode()) == -1
    q8file = tmp_path / "q8.aria"
    write_overlay(R, M8, q8file, "q8")
    # the W8A8 model that loads int8 weights from the file (GLU rows interleaved on load, per-row
    # scales, the captured step re-made) steps bit-identically to one that packs them on the device
    w8b = make_dit(M8, 5, 4, rot)
    T8 = 20
    S8 = M8["memory_tokens"].shape[0] + T8
    c8, s8 = R.rope_freqs(S8, rot, 10000.0)
    _, ced8, _ = inputs(6, 1, M8["project_in"].shape[1], T8, n_cond, 256)
    x8, _, g8 = inputs(301, 1, M8["project_in"].shape[1], T8, n_cond, 256)
    for d in (w8, w8b):
        d.set_request(T8, [ced8[0]], c8, s8)
    y8 = w8.step(x8, g8)                                   # captures w8's step on its own weights
    assert L.aria_hip_dit_load_overlay(w8.h, str(q8file).encode()) == 0
    z8, zb = w8.step(x8, g8), w8b.step(x8, g8)
    assert np.array_equal(z8.view(np.uint32), zb.view(np.uint32))
    assert np.array_equal(z8.view(np.uint32), y8.view(np.uint32))
    for d in (a, b, w8, w8b):
        d.free()


def test_dit_w8a8_env_knob(hip, R, monkeypatch):
    """ARIA_W8A8 set turns an ARIA_Q8 model into the W8A8 path at create, as the reference's
    aria_cuda_dit_create does (src/aria_cuda.cu:1186): its steps are bit-identical to an
    ARIA_Q8A8 model's and differ from a plain Q8 model's."""
    M = model(23, ed=256, inner=512)
    T, n_cond, H, rot = 24, 8, 4, 32
    io_ch, ed = M["project_in"].shape[1], M["project_in"].shape[0]
    S = M["memory_tokens"].shape[0] + T
    c, s = R.rope_freqs(S, rot, 10000.0)
    monkeypatch.delenv("ARIA_W8A8", raising=False)
    q8 = make_dit(M, 3, H, rot)
    a8 = make_dit(M, 5, H, rot)
    monkeypatch.setenv("ARIA_W8A8", "1")
    env = make_dit(M, 3, H, rot)
    monkeypatch.delenv("ARIA_W8A8")
    _, ced, _ = inputs(7, 1, io_ch, T, n_cond, ed)
    x, _, g = inputs(302, 1, io_ch, T, n_cond, ed)
    ys = []
    for d in (q8, a8, env):
        d.set_request(T, [ced[0]], c, s)
        ys.append(d.step(x, g))
    assert np.array_equal(ys[2].view(np.uint32), ys[1].view(np.uint32))
    assert not np.array_equal(ys[0], ys[1])
    for d in (q8, a8, env):
        d.free()
