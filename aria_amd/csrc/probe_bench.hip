/*
 * probe_bench.hip - timing helpers for bench.py, built into the bench-only
 * aria_amd/libaria_probe.so (not the product library):
 *
 *   aria_probe_copy      a streaming device copy, the bandwidth ceiling the row ops and the
 *                        softmax are compared with. Same access shape as those kernels: each
 *                        wave moves one contiguous 4 KB run (a [*, 1024] fp32 row), each lane
 *                        4 float4 with every load issued before the first store, 256-lane
 *                        workgroups over a one-shot grid (no grid-stride loop), non-temporal
 *                        loads and stores (nt = 1) or plain ones (nt = 0).
 *   aria_probe_capture_* capture the work a caller enqueues on a stream into a hipGraph and
 *                        replay it, so a loop of back-to-back launches is timed without the
 *                        host's launch cadence (a Python call per launch takes ~4 us, as long
 *                        as the 21 MB row ops themselves).
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4_p __attribute__((ext_vector_type(4)));

template <int V, bool NT>
__global__ __launch_bounds__(256) void k_probe_copy(f32x4_p *__restrict__ dst, const f32x4_p *__restrict__ src,
                                                    size_t n4) {
    /* each wave moves one contiguous run of 64 V float4 (V KB), lane l the float4s
     * l, l + 64, ...: the layout of a row kernel's wave over a [*, 1024] fp32 row */
    const size_t base = ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 * V) + (threadIdx.x & 63);
    /* the loads are unconditional (an index past the end re-reads the last float4), so all V
     * are in flight at once: a guarded load compiles to a branch with a vmcnt(0) wait in front
     * of the next load */
    f32x4_p v[V];
#pragma unroll
    for (int j = 0; j < V; j++) {
        const size_t i = base + (size_t)j * 64, ic = i < n4 ? i : n4 - 1;
        v[j] = NT ? __builtin_nontemporal_load(src + ic) : src[ic];
    }
#pragma unroll
    for (int j = 0; j < V; j++) {
        const size_t i = base + (size_t)j * 64;
        if (i < n4) {
            if (NT) __builtin_nontemporal_store(v[j], dst + i);
            else dst[i] = v[j];
        }
    }
}

/* dst <- src, bytes a multiple of 16 and both pointers 16-byte aligned. Returns a hipError_t. */
extern "C" int aria_probe_copy(void *dst, const void *src, size_t bytes, int nt, void *stream) {
    if ((bytes & 15u) || (((uintptr_t)dst | (uintptr_t)src) & 15u)) return hipErrorInvalidValue;
    if (!bytes) return hipSuccess;
    const size_t n4 = bytes / 16;
    constexpr int V = 4;
    const dim3 grid((unsigned)((n4 + 256 * V - 1) / (256 * V)));
    hipStream_t s = (hipStream_t)stream;
    if (nt) hipLaunchKernelGGL((k_probe_copy<V, true>), grid, dim3(256), 0, s, (f32x4_p *)dst, (const f32x4_p *)src, n4);
    else hipLaunchKernelGGL((k_probe_copy<V, false>), grid, dim3(256), 0, s, (f32x4_p *)dst, (const f32x4_p *)src, n4);
    return (int)hipGetLastError();
}

/* Start capturing `stream` (thread-local mode: other threads' work is not pulled in). */
extern "C" int aria_probe_capture_begin(void *stream) {
    return (int)hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
}

/* End the capture and instantiate it; *exec receives the executable graph (NULL on failure). */
extern "C" int aria_probe_capture_end(void *stream, void **exec) {
    *exec = NULL;
    hipGraph_t g = NULL;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (e != hipSuccess) return (int)e;
    hipGraphExec_t x = NULL;
    e = hipGraphInstantiate(&x, g, NULL, NULL, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return (int)e;
    *exec = (void *)x;
    return 0;
}

extern "C" int aria_probe_graph_launch(void *exec, void *stream) {
    return (int)hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream);
}

extern "C" int aria_probe_graph_free(void *exec) {
    return exec ? (int)hipGraphExecDestroy((hipGraphExec_t)exec) : 0;
}
