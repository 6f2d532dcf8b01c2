"""GPU: aria_hip_qlinear_noalloc_dev, the allocation-free GEMM entry point, through the C ABI.

Its results must equal aria_hip_qlinear_dev's (the entry point it varies) bit for bit, on two
calls in a row where the second has a smaller input (the static scratch keeps the first call's
contents); fp16 activations need no staging; a staging size past the scratch is refused with an
error and no launch; calls enqueued on two streams without a host synchronisation between them
run one after another on the device (each result still equals its own reference); the call
captured into a HIP graph (what callers that cannot allocate do with it) gives, on every replay,
the eager entry point's result for the activations in place at that replay."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import randn, rng

pytestmark = pytest.mark.gpu


def _run(hip, fn, y, x, x_f16, wt, q, s, b, M, K, N):
    L = hip.lib()
    rc = getattr(L, fn)(y.p, 0, x.p, x_f16, wt, q.p, s.p, None if b is None else b.p, M, K, N, None)
    assert rc == 0, f"{fn}: {hip.last_error()}"
    assert L.aria_hip_stream_sync(None) == 0
    return y.to_host()


@pytest.mark.parametrize("wt", [0, 1])      # Q8, Q4
def test_noalloc_matches_qlinear(hip, port, wt):
    from aria_amd.device import DeviceArray as DA
    print(f"[gpu] noalloc GEMM wtype {wt}", flush=True)
    r = rng(900 + wt)
    # first call: config-3 GEMM2 shape (fp16 staging 21 MB), then a smaller one
    for (M, K, N, bias) in ((2592, 4096, 1024, True), (333, 1024, 768, False)):
        W = randn(r, (N, K), 0.02)
        q, s = port.q8_quant(W) if wt == 0 else port.q4_quant(W)
        x = randn(r, (M, K))
        b = randn(r, N, 0.02) if bias else None
        dq, ds, dx = DA.from_host(q), DA.from_host(s), DA.from_host(x)
        db = DA.from_host(b) if bias else None
        ya, yb = DA((M, N)), DA((M, N))
        want = _run(hip, "aria_hip_qlinear_dev", ya, dx, 0, wt, dq, ds, db, M, K, N)
        got = _run(hip, "aria_hip_qlinear_noalloc_dev", yb, dx, 0, wt, dq, ds, db, M, K, N)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (M, K, N)
        # fp16 activations: no staging at all
        xh = DA.from_host(x.astype(np.float16))
        want16 = _run(hip, "aria_hip_qlinear_dev", ya, xh, 1, wt, dq, ds, db, M, K, N)
        got16 = _run(hip, "aria_hip_qlinear_noalloc_dev", yb, xh, 1, wt, dq, ds, db, M, K, N)
        assert np.array_equal(got16.view(np.uint32), want16.view(np.uint32)), (M, K, N)
        for d in (dq, ds, dx, ya, yb, xh) + ((db,) if bias else ()):
            d.free()


@pytest.mark.parametrize("wt", [0, 1])      # Q8, Q4
def test_noalloc_two_streams(hip, port, wt):
    from aria_amd.device import DeviceArray as DA
    print(f"[gpu] noalloc GEMM on two streams, wtype {wt}", flush=True)
    L = hip.lib()
    r = rng(930 + wt)
    K, N = 1024, 1024
    W = randn(r, (N, K), 0.02)
    q, s = port.q8_quant(W) if wt == 0 else port.q4_quant(W)
    dq, ds = DA.from_host(q), DA.from_host(s)
    # a large staging first (its GEMM runs long), then a smaller one from the other stream,
    # then the first stream again
    xs = [randn(r, (M, K)) for M in (2592, 700, 2592)]
    dxs = [DA.from_host(x) for x in xs]
    want = [_run(hip, "aria_hip_qlinear_dev", DA((x.shape[0], N)), dx, 0, wt, dq, ds, None, x.shape[0], K, N)
            for x, dx in zip(xs, dxs)]
    ys = [DA((x.shape[0], N)) for x in xs]
    s1, s2 = L.aria_hip_stream_create(), L.aria_hip_stream_create()
    assert s1 and s2, hip.last_error()
    try:
        for i, st in enumerate((s1, s2, s1)):
            M = xs[i].shape[0]
            rc = L.aria_hip_qlinear_noalloc_dev(ys[i].p, 0, dxs[i].p, 0, wt, dq.p, ds.p, None, M, K, N, st)
            assert rc == 0, hip.last_error()
        assert L.aria_hip_stream_sync(s1) == 0 and L.aria_hip_stream_sync(s2) == 0
    finally:
        L.aria_hip_stream_destroy(s1)
        L.aria_hip_stream_destroy(s2)
    for i in range(3):
        got = ys[i].to_host()
        assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), i
    for d in [dq, ds] + dxs + ys:
        d.free()


@pytest.mark.parametrize("wt", [0, 1])      # Q8, Q4
def test_noalloc_graph_replays(hip, port, wt):
    """Capture (the bench-only libaria_probe.so's capture helpers, thread-local mode) of one
    no-alloc call with fp32 activations: the graph holds the staging into the static scratch
    and the GEMM, with no event of the cross-stream ordering. Three replays, each after eager
    work on the stream (new activations copied in, an eager no-alloc call of another shape on a
    second stream) and a synchronisation, each checked bit for bit against aria_hip_qlinear_dev."""
    import ctypes as C
    import os
    from aria_amd.device import DeviceArray as DA
    print(f"[gpu] noalloc GEMM under graph capture, wtype {wt}", flush=True)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    P = C.CDLL(os.path.join(root, "aria_amd", "libaria_probe.so"))
    for name, args in (("aria_probe_capture_begin", [C.c_void_p]),
                       ("aria_probe_capture_end", [C.c_void_p, C.POINTER(C.c_void_p)]),
                       ("aria_probe_graph_launch", [C.c_void_p, C.c_void_p]),
                       ("aria_probe_graph_free", [C.c_void_p])):
        getattr(P, name).restype, getattr(P, name).argtypes = C.c_int, args
    L = hip.lib()
    r = rng(950 + wt)
    M, K, N = 700, 1024, 768
    W = randn(r, (N, K), 0.02)
    q, s = port.q8_quant(W) if wt == 0 else port.q4_quant(W)
    dq, ds = DA.from_host(q), DA.from_host(s)
    xs = [randn(r, (M, K)) for _ in range(3)]
    want = []
    for x in xs:
        dxe = DA.from_host(x)
        want.append(_run(hip, "aria_hip_qlinear_dev", DA((M, N)), dxe, 0, wt, dq, ds, None, M, K, N))
        dxe.free()
    dx, dy = DA((M, K)), DA((M, N))
    x2 = randn(r, (333, K))
    dx2, dy2 = DA.from_host(x2), DA((333, N))
    want2 = _run(hip, "aria_hip_qlinear_dev", DA((333, N)), dx2, 0, wt, dq, ds, None, 333, K, N)
    st, st2 = L.aria_hip_stream_create(), L.aria_hip_stream_create()
    assert st and st2, hip.last_error()
    ex = C.c_void_p()
    try:
        assert P.aria_probe_capture_begin(st) == 0
        rc = L.aria_hip_qlinear_noalloc_dev(dy.p, 0, dx.p, 0, wt, dq.p, ds.p, None, M, K, N, st)
        assert P.aria_probe_capture_end(st, C.byref(ex)) == 0 and ex.value
        assert rc == 0, hip.last_error()
        for i, x in enumerate(xs):
            assert L.aria_hip_memcpy_h2d_async(dx.p, x.ctypes.data, x.nbytes, st) == 0
            assert L.aria_hip_qlinear_noalloc_dev(dy2.p, 0, dx2.p, 0, wt, dq.p, ds.p, None, 333, K, N, st2) == 0
            assert L.aria_hip_stream_sync(st) == 0 and L.aria_hip_stream_sync(st2) == 0
            assert P.aria_probe_graph_launch(ex, st) == 0
            assert L.aria_hip_stream_sync(st) == 0
            assert np.array_equal(dy.to_host().view(np.uint32), want[i].view(np.uint32)), f"replay {i}"
            assert np.array_equal(dy2.to_host().view(np.uint32), want2.view(np.uint32)), f"eager {i}"
    finally:
        if ex.value:
            P.aria_probe_graph_free(ex)
        L.aria_hip_stream_destroy(st)
        L.aria_hip_stream_destroy(st2)
    for d in (dq, ds, dx, dy, dx2, dy2):
        d.free()


def test_noalloc_refuses_oversize(hip):
    from aria_amd.device import DeviceArray as DA
    L = hip.lib()
    M, K, N = 4097, 4096, 64          # 4097 * 4096 * 2 B > 32 MiB of scratch
    x, y = DA((M, K)), DA((M, N))
    q, s = DA((N, K), np.int8), DA(N)
    rc = L.aria_hip_qlinear_noalloc_dev(y.p, 0, x.p, 0, 0, q.p, s.p, None, M, K, N, None)
    assert rc == -1 and "scratch" in hip.last_error()
    for d in (x, y, q, s):
        d.free()
