/*
 * k_noalloc.hip - the allocation-free form of the dequant-on-use GEMM entry point.
 *
 * aria_hip_qlinear_dev with fp32 activations stages them as fp16 in device memory it
 * allocates per call (stream-ordered pool) before the MFMA kernel runs. Callers that must
 * not allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc) call aria_hip_qlinear_noalloc_dev instead: the staging lives in `scratch`,
 * a file-scope device array of ARIA_HIP_NOALLOC_SCRATCH bytes that each GPU holds for the
 * life of the process. Its device address is resolved once per device with
 * hipGetSymbolAddress (host code sees only a stand-in for the array's name), at library init
 * for the library's device and on the first call on any other, and kept per device; every
 * kernel argument and copy uses that address.
 *
 * Every call on one GPU shares that GPU's array and the array keeps the last call's
 * contents. The staging is fully written before the GEMM reads it, so nothing needs
 * clearing. Calls from several streams are ordered on the device: each staging call records
 * an event after its GEMM, and a call on another stream than the previous one first makes its
 * stream wait for that event (one mutex covers the wait, the launches and the record, so two
 * host threads cannot interleave them). A stream under capture records and waits for nothing
 * (an event from outside a capture cannot join its graph): there the graph orders the calls.
 */
#include <hip/hip_runtime.h>

#include <mutex>

extern "C" {
#include "aria_hip.h"
#include "aria_hip_internal.h"
#include "aria_hip_kernels.h"
}

#define ARIA_WQ8 0
#define ARIA_WQ4 1
#define ARIA_WF16 2

static __device__ __align__(256) unsigned char scratch[ARIA_HIP_NOALLOC_SCRATCH];

#define NOALLOC_MAX_DEV 64
static std::mutex g_mu;
static void *g_ptr[NOALLOC_MAX_DEV];   /* device address of `scratch`, per device */
static hipEvent_t g_done[NOALLOC_MAX_DEV];   /* recorded after the last staging call's GEMM */
static hipStream_t g_last[NOALLOC_MAX_DEV];  /* that call's stream */
static bool g_used[NOALLOC_MAX_DEV];

/* the current device's scratch address and ordering event, set up at library init (the
 * library's device) or on the first call on another device; called with g_mu held */
static int scratch_addr(void **out, int *devp) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return aria_hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= NOALLOC_MAX_DEV) {
        aria_hip_set_error("aria_hip_qlinear_noalloc_dev: device %d beyond the %d the scratch table holds", dev,
                           NOALLOC_MAX_DEV);
        return ARIA_HIP_EINVAL;
    }
    if (!g_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return aria_hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                        "hipGetSymbolAddress (scratch)");
        /* no system-scope fence at the record: only streams of this device wait for it (the
         * fence's cache writeback made every staging call ~3 us slower) */
        if ((e = hipEventCreateWithFlags(&g_done[dev], hipEventDisableTiming | hipEventDisableSystemFence)) != hipSuccess)
            return aria_hip_fail(e, "hipEventCreateWithFlags (no-alloc ordering)");
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    *devp = dev;
    return 0;
}

extern "C" int aria_noalloc_setup(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    void *p = nullptr;
    int dev = 0;
    return scratch_addr(&p, &dev);
}

extern "C" int aria_hip_qlinear_noalloc_dev(void *dy, int y_f16, const void *dx, int x_f16, int wtype,
                                            const void *dq, const float *dscale, const float *db, int M, int K,
                                            int N, void *stream) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (M < 0 || K <= 0 || N < 0 || (wtype != ARIA_WQ8 && wtype != ARIA_WQ4 && wtype != ARIA_WF16) ||
        (M && N && (!dy || !dx || !dq || (wtype != ARIA_WF16 && !dscale)))) {
        aria_hip_set_error("aria_hip_qlinear_noalloc_dev: invalid argument (M %d, K %d, N %d, wtype %d)", M, K, N,
                           wtype);
        return ARIA_HIP_EINVAL;
    }
    if (M == 0 || N == 0) return 0;
    hipStream_t s = aria_hip_stream(stream);
    const void *xa = dx;
    int xh = x_f16;
    if (!x_f16 && K % 32 == 0 && ((uintptr_t)dx & 15u) == 0) {
        /* the fp16 staging of aria_hip_qlinear_dev, in the static scratch */
        const size_t need = (size_t)M * K * 2;
        if (need > ARIA_HIP_NOALLOC_SCRATCH) {
            aria_hip_set_error("aria_hip_qlinear_noalloc_dev: fp16 staging of %d x %d activations needs %zu bytes, "
                               "above the %zu-byte scratch; split M or pass fp16 activations",
                               M, K, need, (size_t)ARIA_HIP_NOALLOC_SCRATCH);
            return ARIA_HIP_EINVAL;
        }
        std::lock_guard<std::mutex> lk(g_mu);
        void *p = nullptr;
        int dev = 0;
        if ((rc = scratch_addr(&p, &dev))) return rc;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(s, &cs);
        if (e != hipSuccess) return aria_hip_fail(e, "hipStreamIsCapturing");
        const bool order = cs == hipStreamCaptureStatusNone;
        if (order && g_used[dev] && g_last[dev] != s && (e = hipStreamWaitEvent(s, g_done[dev], 0)) != hipSuccess)
            return aria_hip_fail(e, "hipStreamWaitEvent (no-alloc ordering)");
        if ((e = aria_k_f32_to_f16((uint16_t *)p, (const float *)dx, (size_t)M * K, s)) != hipSuccess)
            return aria_hip_fail(e, "k_f32_to_f16 (scratch staging)");
        if ((e = aria_k_qgemm_t(dy, y_f16, p, 1, wtype, dq, dscale, db, M, K, N, 0, 0, s)) != hipSuccess)
            return aria_hip_fail(e, "k_qgemm (no-alloc)");
        if (order) {
            if ((e = hipEventRecord(g_done[dev], s)) != hipSuccess)
                return aria_hip_fail(e, "hipEventRecord (no-alloc ordering)");
            g_last[dev] = s;
            g_used[dev] = true;
        }
        return 0;
    }
    hipError_t e = aria_k_qgemm_t(dy, y_f16, xa, xh, wtype, dq, dscale, db, M, K, N, 0, 0, s);
    if (e != hipSuccess) return aria_hip_fail(e, "k_qgemm (no-alloc)");
    return 0;
}
