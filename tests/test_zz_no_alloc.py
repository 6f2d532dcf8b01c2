"""GPU: aria_hip_qlinear_noalloc_dev, the allocation-free GEMM entry point, through the C ABI.

Its results must equal aria_hip_qlinear_dev's (the entry point it varies) bit for bit, on two
calls in a row where the second has a smaller input (the static scratch keeps the first call's
contents); fp16 activations need no staging; a staging size past the scratch is refused with an
error and no launch; calls enqueued on two streams without a host synchronisation between them
run one after another on the device (each result still equals its own reference)."""
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
