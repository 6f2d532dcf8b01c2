/*
 * aria_hip.c - the MI355X (gfx950) GPU backend host code, in C11.
 *
 * Serves the reference's GPU C ABI (include/aria_gpu.h = the reference's
 * src/aria_gpu.h) and the device-pointer extension (include/aria_hip.h). It
 * owns device selection, the library stream, error reporting and the
 * host-pointer wrappers; the arithmetic lives in the .hip kernels, reached
 * through the launchers of aria_hip_kernels.h.
 *
 * Host wrappers follow the reference's contract (src/aria_cuda.cu:115-131):
 * allocate device buffers, copy inputs in, launch on the library stream, copy
 * outputs back, free, and return only when the result is in host memory.
 * In-place ops (silu, gelu, softcap, softmax, rope) update the host buffer.
 *
 * Threading: one library stream created at first use (default priority,
 * non-blocking); calls from several host threads serialise on it. The last
 * error text is kept per thread.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include "aria_gpu.h"
#include "aria_hip.h"
#include "aria_hip_internal.h"
#include "aria_hip_kernels.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* runtime state                                                             */
/* ------------------------------------------------------------------------- */

static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static int g_ok = 0;
static int g_dev = 0;
static hipStream_t g_stream = NULL;
static hipDeviceProp_t g_prop;
static char g_init_err[256] = "not initialised";
static __thread char t_err[512];

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
}

static int hip_fail(hipError_t e, const char *what) {
    set_err("%s: %s", what, hipGetErrorString(e));
    fprintf(stderr, "[aria-hip] %s\n", t_err);
    return (int)e;
}

#define HCK(call)                                        \
    do {                                                 \
        hipError_t e_ = (call);                          \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

static void init_once(void) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        snprintf(g_init_err, sizeof g_init_err, "no HIP device (%s)",
                 e != hipSuccess ? hipGetErrorString(e) : "count 0");
        return;
    }
    g_dev = 0;
    if ((e = hipSetDevice(g_dev)) != hipSuccess ||
        (e = hipGetDeviceProperties(&g_prop, g_dev)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking)) != hipSuccess) {
        snprintf(g_init_err, sizeof g_init_err, "HIP init: %s", hipGetErrorString(e));
        return;
    }
    g_ok = 1;
    /* the allocation-free GEMM's scratch address and ordering event; a failure here is
     * reported by that entry point, which retries the set-up on its first call */
    if (aria_noalloc_setup()) hipGetLastError();
}

/* make the library device current on the calling thread; 0 or ENODEV */
static int ensure(void) {
    pthread_once(&g_once, init_once);
    if (!g_ok) {
        set_err("%s", g_init_err);
        return ARIA_HIP_ENODEV;
    }
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != g_dev) hipSetDevice(g_dev);
    return 0;
}

static hipStream_t pick(void *stream) { return stream ? (hipStream_t)stream : g_stream; }

#define ENSURE()                 \
    do {                         \
        int r_ = ensure();       \
        if (r_) return r_;       \
    } while (0)

#define KCK(call, name)                                   \
    do {                                                  \
        hipError_t e_ = (call);                           \
        if (e_ != hipSuccess) return hip_fail(e_, name);  \
    } while (0)

/* shared with the other host files (aria_hip_internal.h) */
int aria_hip_ensure(void) { return ensure(); }
int aria_hip_fail(hipError_t e, const char *what) { return hip_fail(e, what); }
void aria_hip_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
}
hipStream_t aria_hip_stream(void *stream) { return pick(stream); }

int aria_hip_init(void) { return ensure(); }
const char *aria_hip_last_error(void) { return t_err; }
void *aria_hip_default_stream(void) { return ensure() ? NULL : (void *)g_stream; }

int aria_hip_stream_sync(void *stream) {
    ENSURE();
    HCK(hipStreamSynchronize(pick(stream)));
    return 0;
}

void *aria_hip_stream_create(void) {
    if (ensure()) return NULL;
    hipStream_t st = NULL;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return NULL;
    return (void *)st;
}
void aria_hip_stream_destroy(void *stream) {
    if (stream && stream != (void *)g_stream) hipStreamDestroy((hipStream_t)stream);
}

void *aria_hip_event_create(void) {
    if (ensure()) return NULL;
    hipEvent_t ev = NULL;
    if (hipEventCreate(&ev) != hipSuccess) return NULL;
    return (void *)ev;
}
void aria_hip_event_destroy(void *ev) {
    if (ev) hipEventDestroy((hipEvent_t)ev);
}
int aria_hip_event_record(void *ev, void *stream) {
    ENSURE();
    HCK(hipEventRecord((hipEvent_t)ev, pick(stream)));
    return 0;
}
float aria_hip_event_elapsed_ms(void *ev0, void *ev1) {
    float ms = -1.0f;
    if (hipEventSynchronize((hipEvent_t)ev1) != hipSuccess) return -1.0f;
    if (hipEventElapsedTime(&ms, (hipEvent_t)ev0, (hipEvent_t)ev1) != hipSuccess) return -1.0f;
    return ms;
}
int aria_hip_memcpy_h2d_async(void *d, const void *h, size_t bytes, void *stream) {
    ENSURE();
    HCK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, pick(stream)));
    return 0;
}
int aria_hip_memcpy_d2h_async(void *h, const void *d, size_t bytes, void *stream) {
    ENSURE();
    HCK(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, pick(stream)));
    return 0;
}
int aria_hip_memcpy_d2d_async(void *d, const void *s, size_t bytes, void *stream) {
    ENSURE();
    HCK(hipMemcpyAsync(d, s, bytes, hipMemcpyDeviceToDevice, pick(stream)));
    return 0;
}
int aria_hip_cu_count(void) { return ensure() ? 0 : g_prop.multiProcessorCount; }
int aria_hip_arch(char *buf, size_t buflen) {
    ENSURE();
    if (buf && buflen) {
        snprintf(buf, buflen, "%s", g_prop.gcnArchName);
        char *colon = strchr(buf, ':');   /* "gfx950:sramecc+:xnack-" -> "gfx950" */
        if (colon) *colon = '\0';
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* reference ABI: device query and raw memory (src/aria_gpu.h:19-36)         */
/* ------------------------------------------------------------------------- */

int aria_cuda_available(void) { return ensure() == 0; }

int aria_cuda_recommended(void) {
    if (ensure()) return 0;
    return strncmp(g_prop.gcnArchName, "gfx950", 6) == 0 || strncmp(g_prop.gcnArchName, "gfx942", 6) == 0;
}

/* the W8A8 path (k_gemm_i8.hip) runs on gfx950's int8 MFMA (v_mfma_i32_32x32x32_i8) */
int aria_cuda_int8_tc(void) {
    if (ensure()) return 0;
    return strncmp(g_prop.gcnArchName, "gfx950", 6) == 0;
}

void aria_cuda_device_info(char *buf, size_t buflen) {
    if (!buf || !buflen) return;
    if (ensure()) { snprintf(buf, buflen, "no HIP device"); return; }
    char arch[64];
    aria_hip_arch(arch, sizeof arch);
    snprintf(buf, buflen, "%s (%s, %d CUs, %.1f GB)", g_prop.name, arch, g_prop.multiProcessorCount,
             (double)g_prop.totalGlobalMem / 1e9);
}

void aria_cuda_meminfo(size_t *used, size_t *total) {
    size_t fr = 0, tot = 0;
    if (ensure() == 0) hipMemGetInfo(&fr, &tot);
    if (used) *used = tot - fr;
    if (total) *total = tot;
}

void *aria_cuda_malloc(size_t bytes) {
    if (ensure()) return NULL;
    void *p = NULL;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) { hip_fail(e, "hipMalloc"); return NULL; }
    return p;
}
void aria_cuda_free(void *d) {
    if (d && ensure() == 0) hipFree(d);
}
void aria_cuda_memcpy_h2d(void *d, const void *h, size_t bytes) {
    if (ensure() || !bytes) return;
    hipError_t e = hipMemcpy(d, h, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) hip_fail(e, "hipMemcpy h2d");
}
void aria_cuda_memcpy_d2h(void *h, const void *d, size_t bytes) {
    if (ensure() || !bytes) return;
    hipError_t e = hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) hip_fail(e, "hipMemcpy d2h");
}
void aria_cuda_sync(void) {
    if (ensure()) return;
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) hip_fail(e, "sync");
}

/* ------------------------------------------------------------------------- */
/* host-wrapper scratch: device staging buffers for one synchronous call     */
/* ------------------------------------------------------------------------- */

#define STAGE_MAX 8
typedef struct {
    void *p[STAGE_MAX];
    int n;
    int err;
} stage_t;

static void *st_alloc(stage_t *st, size_t bytes) {
    if (st->err || st->n >= STAGE_MAX) { st->err = st->err ? st->err : ARIA_HIP_EINVAL; return NULL; }
    void *p = NULL;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 4);
    if (e != hipSuccess) { st->err = hip_fail(e, "hipMalloc (staging)"); return NULL; }
    st->p[st->n++] = p;
    return p;
}
/* device copy of a host input (NULL stays NULL) */
static void *st_in(stage_t *st, const void *h, size_t bytes) {
    if (!h) return NULL;
    void *d = st_alloc(st, bytes);
    if (!d) return NULL;
    hipError_t e = hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, g_stream);
    if (e != hipSuccess) st->err = hip_fail(e, "hipMemcpyAsync h2d");
    return d;
}
static int st_out(stage_t *st, void *h, const void *d, size_t bytes) {
    if (st->err) return st->err;
    hipError_t e = hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, g_stream);
    if (e != hipSuccess) st->err = hip_fail(e, "hipMemcpyAsync d2h");
    return st->err;
}
static int st_finish(stage_t *st) {
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess && !st->err) st->err = hip_fail(e, "hipStreamSynchronize");
    for (int i = 0; i < st->n; i++) hipFree(st->p[i]);
    st->n = 0;
    return st->err;
}
static void st_kernel(stage_t *st, hipError_t e, const char *name) {
    if (!st->err && e != hipSuccess) st->err = hip_fail(e, name);
}

#define FB(n) ((size_t)(n) * sizeof(float))

/* ------------------------------------------------------------------------- */
/* device-pointer entry points (aria_hip.h)                                  */
/* ------------------------------------------------------------------------- */

#define REQ(cond)                                                   \
    do {                                                            \
        if (!(cond)) { set_err("invalid argument: %s", #cond); return ARIA_HIP_EINVAL; } \
    } while (0)

int aria_hip_rmsnorm_dev(float *dy, const float *dx, const float *dw, int rows, int dim, float eps,
                         void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dy && dx)));
    KCK(aria_k_rownorm_nt(dy, 0, dx, dw, NULL, NULL, NULL, 0, 0, 0, ARIA_NORM_RMS, rows, dim, eps, 1, pick(stream)),
        "k_rownorm(rms)");
    return 0;
}
int aria_hip_gemma_rmsnorm_dev(float *dy, const float *dx, const float *dw, int rows, int dim, float eps,
                               void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dy && dx && dw)));
    KCK(aria_k_rownorm(dy, 0, dx, dw, NULL, NULL, NULL, 0, 0, 0, ARIA_NORM_GEMMA, rows, dim, eps,
                       pick(stream)), "k_rownorm(gemma)");
    return 0;
}
int aria_hip_layernorm_dev(float *dy, const float *dx, const float *dg, const float *db, int rows, int dim,
                           float eps, void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dy && dx)));
    KCK(aria_k_rownorm_nt(dy, 0, dx, dg, db, NULL, NULL, 0, 0, 0, ARIA_NORM_LAYER, rows, dim, eps, 1, pick(stream)),
        "k_rownorm(layer)");
    return 0;
}
int aria_hip_rmsnorm_adaln_dev(void *dy, int out_f16, const float *dx, const float *dw, const float *dsc,
                               const float *dsh, int rows, int dim, int rpb, float eps, void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dy && dx && dsc && dsh)));
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    KCK(aria_k_rownorm(dy, out_f16, dx, dw, NULL, dsc, dsh, rpb, 0, 0, ARIA_NORM_RMS, rows, dim, eps,
                       pick(stream)), "k_rownorm(rms+adaln)");
    return 0;
}
int aria_hip_ln_mod_gelu_res_dev(float *dout, const float *dx, const float *dg, const float *db,
                                 const float *dsc, const float *dsh, int rows, int dim, int rpb, float eps,
                                 void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dout && dx && dsc && dsh)));
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    REQ(dout != dx);
    KCK(aria_k_rownorm_nt(dout, 0, dx, dg, db, dsc, dsh, rpb, 1, 1, ARIA_NORM_LAYER, rows, dim, eps, 1,
                          pick(stream)), "k_rownorm(ln+mod+gelu+res)");
    return 0;
}

int aria_hip_add_dev(float *dy, const float *da, const float *db, size_t n, void *stream) {
    ENSURE();
    REQ(n == 0 || (dy && da && db));
    KCK(aria_k_add(dy, da, db, n, pick(stream)), "k_add");
    return 0;
}
int aria_hip_axpy_dev(float *dy, const float *dx, float a, size_t n, void *stream) {
    ENSURE();
    REQ(n == 0 || (dy && dx));
    KCK(aria_k_axpy(dy, dx, a, n, pick(stream)), "k_axpy");
    return 0;
}
int aria_hip_scale_dev(float *dy, const float *dx, float a, size_t n, void *stream) {
    ENSURE();
    REQ(n == 0 || (dy && dx));
    KCK(aria_k_scale(dy, dx, a, n, pick(stream)), "k_scale");
    return 0;
}
int aria_hip_gelu_tanh_dev(float *dy, const float *dx, size_t n, void *stream) {
    ENSURE();
    REQ(n == 0 || (dy && dx));
    KCK(aria_k_gelu_tanh(dy, dx, n, pick(stream)), "k_gelu");
    return 0;
}
int aria_hip_silu_dev(float *dy, const float *dx, size_t n, void *stream) {
    ENSURE();
    REQ(n == 0 || (dy && dx));
    KCK(aria_k_silu(dy, dx, n, pick(stream)), "k_silu");
    return 0;
}
int aria_hip_silu_gate_dev(float *dout, const float *dgate, const float *dup, size_t n, void *stream) {
    ENSURE();
    REQ(n == 0 || (dout && dgate && dup));
    KCK(aria_k_silu_gate(dout, dgate, dup, n, pick(stream)), "k_silu_gate");
    return 0;
}
int aria_hip_modulate_dev(float *dy, const float *dx, const float *dsc, const float *dsh, int rows, int dim,
                          int rpb, void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dy && dx && dsc && dsh)));
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    KCK(aria_k_modulate(dy, dx, dsc, dsh, rows, dim, rpb, pick(stream)), "k_modulate");
    return 0;
}
int aria_hip_gate_residual_dev(float *dout, const float *dres, const float *do_, const float *dgate,
                               const float *dbias, int rows, int dim, int rpb, void *stream) {
    ENSURE();
    REQ(rows >= 0 && dim > 0 && (rows == 0 || (dout && dres && do_ && dgate)));
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    KCK(aria_k_gate_residual(dout, dres, do_, dgate, dbias, rows, dim, rpb, pick(stream)), "k_gate_residual");
    return 0;
}
int aria_hip_glu_combine_dev(void *dout, int out_f16, const float *dproj, const float *dbias, int rows,
                             int inner, void *stream) {
    ENSURE();
    REQ(rows >= 0 && inner > 0 && (rows == 0 || (dout && dproj)));
    KCK(aria_k_glu_combine(dout, out_f16, dproj, dbias, rows, inner, pick(stream)), "k_glu");
    return 0;
}
int aria_hip_pingpong_dev(float *dx, const float *dv, const float *dz, float tc, float tn, size_t n,
                          void *stream) {
    ENSURE();
    REQ(n == 0 || (dx && dv && dz));
    KCK(aria_k_pingpong(dx, dv, dz, tc, tn, n, pick(stream)), "k_pingpong");
    return 0;
}
int aria_hip_softmax_dev(float *dx, int rows, int cols, const float *dmask, void *stream) {
    ENSURE();
    REQ(rows >= 0 && cols > 0 && (rows == 0 || dx));
    KCK(aria_k_softmax(dx, rows, cols, dmask, pick(stream)), "k_softmax");
    return 0;
}
int aria_hip_rope_apply_dev(float *dx, const float *dc, const float *ds, int H, int N, int D, int rot,
                            void *stream) {
    ENSURE();
    REQ(H >= 0 && N >= 0 && D > 0 && rot >= 0 && rot <= D && rot % 2 == 0);
    REQ(H == 0 || N == 0 || rot == 0 || (dx && dc && ds));
    KCK(aria_k_rope(dx, dc, ds, H, N, D, rot, pick(stream)), "k_rope");
    return 0;
}
int aria_hip_rope_apply2_dev(float *dq, float *dk, const float *dc, const float *ds, int H, int N, int D,
                             int rot, void *stream) {
    ENSURE();
    REQ(H >= 0 && N >= 0 && D > 0 && rot >= 0 && rot <= D && rot % 2 == 0);
    REQ(H == 0 || N == 0 || rot == 0 || (dq && dk && dc && ds && dq != dk));
    KCK(aria_k_rope2(dq, dk, dc, ds, H, N, D, rot, pick(stream)), "k_rope2");
    return 0;
}
int aria_hip_q8_quant_dev(int8_t *dq, float *dscale, const float *dW, int N, int K, void *stream) {
    ENSURE();
    REQ(N >= 0 && K > 0 && (N == 0 || (dq && dscale && dW)));
    KCK(aria_k_q8_quant(dq, dscale, dW, N, K, pick(stream)), "k_q8_quant");
    return 0;
}
int aria_hip_q4_quant_dev(uint8_t *dq, float *dscale, const float *dW, int N, int K, void *stream) {
    ENSURE();
    REQ(N >= 0 && K > 0 && (N == 0 || (dq && dscale && dW)));
    REQ(((uintptr_t)dscale & 7u) == 0);
    KCK(aria_k_q4_quant(dq, dscale, dW, N, K, pick(stream)), "k_q4_quant");
    return 0;
}
int aria_hip_q8_dequant_dev(float *dW, const int8_t *dq, const float *dscale, int N, int K, void *stream) {
    ENSURE();
    REQ(N >= 0 && K > 0 && (N == 0 || (dq && dscale && dW)));
    KCK(aria_k_q8_dequant(dW, dq, dscale, N, K, pick(stream)), "k_q8_dequant");
    return 0;
}
int aria_hip_q4_dequant_dev(float *dW, const uint8_t *dq, const float *dscale, int N, int K, void *stream) {
    ENSURE();
    REQ(N >= 0 && K > 0 && (N == 0 || (dq && dscale && dW)));
    KCK(aria_k_q4_dequant(dW, dq, dscale, N, K, pick(stream)), "k_q4_dequant");
    return 0;
}

int aria_hip_qlinear_ex_dev(void *dy, int y_f16, const void *dx, int x_f16, int wtype, const void *dq,
                            const float *dscale, const float *db, int M, int K, int N, int tiles, void *stream) {
    ENSURE();
    REQ(M >= 0 && K > 0 && N >= 0 && tiles >= 0 && tiles <= 32);
    REQ(wtype == ARIA_WQ8 || wtype == ARIA_WQ4 || wtype == ARIA_WF16);
    REQ(M == 0 || N == 0 || (dy && dx && dq && (wtype == ARIA_WF16 || dscale)));
    if (M == 0 || N == 0) return 0;
    hipStream_t s = pick(stream);
    /* fp32 activations: one conversion pass to fp16 (stream-ordered pool memory), then the
     * fp16-operand kernel, which stages half the bytes per slice; the value rounded is the
     * same RTNE half the in-kernel staging would produce */
    void *x16 = NULL;
    if (!x_f16 && K % 32 == 0 && ((uintptr_t)dx & 15u) == 0 &&
        hipMallocAsync(&x16, (size_t)M * K * 2, s) == hipSuccess) {
        hipError_t e = aria_k_f32_to_f16((uint16_t *)x16, (const float *)dx, (size_t)M * K, s);
        if (e == hipSuccess) e = aria_k_qgemm_t(dy, y_f16, x16, 1, wtype, dq, dscale, db, M, K, N, tiles, 0, s);
        hipError_t ef = hipFreeAsync(x16, s);
        if (e == hipSuccess) e = ef;
        KCK(e, "k_qgemm (fp16-staged activations)");
        return 0;
    }
    hipGetLastError();   /* a refused pool allocation leaves no sticky error: take the direct path */
    KCK(aria_k_qgemm_t(dy, y_f16, dx, x_f16, wtype, dq, dscale, db, M, K, N, tiles, 0, s), "k_qgemm");
    return 0;
}
int aria_hip_qlinear_dev(void *dy, int y_f16, const void *dx, int x_f16, int wtype, const void *dq,
                         const float *dscale, const float *db, int M, int K, int N, void *stream) {
    return aria_hip_qlinear_ex_dev(dy, y_f16, dx, x_f16, wtype, dq, dscale, db, M, K, N, 0, stream);
}
int aria_hip_qkv_prep_dev(const float *dsrc, int ld, int B, int S, int H, int nsec, const int *kind,
                          uint16_t *const *ddst, const float *const *dw, const float *dcos, const float *dsin,
                          int rot, float eps, void *stream) {
    ENSURE();
    REQ(B >= 0 && S >= 0 && H > 0 && nsec >= 1 && nsec <= 3 && kind && ddst);
    REQ(ld >= nsec * H * 64 && ld % 4 == 0 && (rot == 0 || rot == 32 || rot == 64));
    REQ(B == 0 || S == 0 || (dsrc && ((uintptr_t)dsrc & 15u) == 0));
    for (int i = 0; i < nsec; i++) {
        REQ(kind[i] >= 0 && kind[i] <= 2 && ddst[i] && ((uintptr_t)ddst[i] & 7u) == 0);
        if (kind[i] != 2 && rot) REQ(dcos && dsin);
    }
    KCK(aria_k_qkv_prep(dsrc, ld, B, S, H, nsec, kind, ddst, dw, dcos, dsin, rot, eps, pick(stream)),
        "k_qkv_prep");
    return 0;
}
int aria_hip_flash_attention_dev(const uint16_t *dq, const uint16_t *dk, const uint16_t *dv, void *dout,
                                 int out_f16, int B, int H, int Nq, int Nk, int D, void *stream) {
    ENSURE();
    REQ(D == 64 && B >= 0 && H > 0 && Nq >= 0 && Nk > 0);
    REQ(B == 0 || Nq == 0 || (dq && dk && dv && dout));
    REQ((((uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv) & 15u) == 0 && ((uintptr_t)dout & 15u) == 0);
    KCK(aria_k_flash_attn(dq, dk, dv, dout, out_f16, B * H, H, Nq, Nk, pick(stream)), "k_flash_attn");
    return 0;
}
int aria_hip_linear_q8_dev(float *dy, const float *dx, const int8_t *dq, const float *dscale, const float *db,
                           int M, int K, int N, void *stream) {
    return aria_hip_qlinear_dev(dy, 0, dx, 0, ARIA_WQ8, dq, dscale, db, M, K, N, stream);
}
int aria_hip_linear_q4_dev(float *dy, const float *dx, const uint8_t *dq, const float *dscale, const float *db,
                           int M, int K, int N, void *stream) {
    return aria_hip_qlinear_dev(dy, 0, dx, 0, ARIA_WQ4, dq, dscale, db, M, K, N, stream);
}

/* W8A8 (k_gemm_i8.hip, the int8-output norms of k_rownorm.hip) */
int aria_hip_rmsnorm_adaln_q8_dev(int8_t *dyq, float *dsx, const float *dx, const float *dw, const float *dsc,
                                  const float *dsh, int rows, int dim, int rpb, float eps, void *stream) {
    ENSURE();
    REQ(rows >= 0 && (dim == 256 || dim == 512 || dim == 768 || dim == 1024 || dim == 2048));
    REQ(rows == 0 || (dyq && dsx && dx && !dsc == !dsh));
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    REQ((((uintptr_t)dyq & 3u) | ((uintptr_t)dx & 15u) | ((uintptr_t)dw & 15u) | ((uintptr_t)dsc & 15u) |
         ((uintptr_t)dsh & 15u)) == 0);
    KCK(aria_k_rownorm_q8(dyq, dsx, dx, dw, dsc, dsh, rpb, rows, dim, eps, pick(stream)), "k_rownorm_q8");
    return 0;
}
int aria_hip_quant_act_q8_dev(int8_t *dxq, float *dsx, const void *dx, int x_f16, int M, int K, void *stream) {
    ENSURE();
    REQ(M >= 0 && K > 0 && (M == 0 || (dxq && dsx && dx)));
    REQ(K % 4 || (((uintptr_t)dxq & 3u) == 0 && ((uintptr_t)dx & (x_f16 ? 7u : 15u)) == 0));
    KCK(aria_k_quant_act_q8(dxq, dsx, dx, x_f16, M, K, pick(stream)), "k_quant_act_q8");
    return 0;
}
int aria_hip_gemm_i8_dev(void *dy, int y_f16, const int8_t *dxq, const float *dsx, const int8_t *dq,
                         const float *dscale, const float *db, int M, int K, int N, void *stream) {
    ENSURE();
    REQ(M >= 0 && K > 0 && N >= 0 && (M == 0 || N == 0 || (dy && dxq && dsx && dq && dscale)));
    KCK(aria_k_gemm_i8(dy, y_f16, dxq, dsx, dq, dscale, db, M, K, N, 0, NULL, pick(stream)), "k_gemm_i8");
    return 0;
}
size_t aria_hip_q8a8_ws_bytes(int M, int K) {
    if (M <= 0 || K <= 0) return 0;
    return (((size_t)M * K + 255) & ~(size_t)255) + (size_t)M * sizeof(float);
}
int aria_hip_linear_q8a8_dev(float *dy, const void *dx, int x_f16, const int8_t *dq, const float *dscale,
                             const float *db, int M, int K, int N, void *dws, void *stream) {
    ENSURE();
    REQ(M >= 0 && K > 0 && N >= 0);
    if (M == 0 || N == 0) return 0;
    REQ(dy && dx && dq && dscale && dws && ((uintptr_t)dws & 255u) == 0);
    int8_t *xq = (int8_t *)dws;
    float *sx = (float *)(void *)((char *)dws + (((size_t)M * K + 255) & ~(size_t)255));
    int r = aria_hip_quant_act_q8_dev(xq, sx, dx, x_f16, M, K, stream);
    if (r) return r;
    return aria_hip_gemm_i8_dev(dy, 0, xq, sx, dq, dscale, db, M, K, N, stream);
}

/* ------------------------------------------------------------------------- */
/* host-pointer forms (aria_hip.h) - one synchronous staged call each        */
/* ------------------------------------------------------------------------- */

#define HOST_BEGIN() stage_t st_ = {{0}, 0, 0}; ENSURE()
#define HOST_END() return st_finish(&st_)

static int host_qlinear(float *y, const float *x, int wtype, const void *q, const float *scale, const float *b,
                        int M, int K, int N) {
    HOST_BEGIN();
    REQ(M >= 0 && K > 0 && N >= 0 && y && x && q && scale);
    if (M == 0 || N == 0) return 0;
    size_t qb = wtype == ARIA_WQ8 ? (size_t)N * K : (size_t)N * ((K + 1) / 2);
    size_t ns = wtype == ARIA_WQ8 ? (size_t)N : (size_t)N * 2 * ((K + 31) / 32);
    float *dx = st_in(&st_, x, FB((size_t)M * K));
    void *dq = st_in(&st_, q, qb);
    float *ds = st_in(&st_, scale, FB(ns));
    float *db = st_in(&st_, b, FB(N));
    float *dy = st_alloc(&st_, FB((size_t)M * N));
    if (!st_.err)
        st_.err = aria_hip_qlinear_dev(dy, 0, dx, 0, wtype, dq, ds, db, M, K, N, g_stream);
    st_out(&st_, y, dy, FB((size_t)M * N));
    HOST_END();
}
int aria_hip_attention_f16(float *out, const float *q, const float *k, const float *v, int B, int H, int Nq,
                           int Nk, int D) {
    HOST_BEGIN();
    REQ(out && q && k && v && B > 0 && H > 0 && Nq > 0 && Nk > 0 && D == 64);
    size_t nq = (size_t)B * H * Nq * D, nk = (size_t)B * H * Nk * D;
    float *dq32 = st_in(&st_, q, FB(nq));
    float *dk32 = st_in(&st_, k, FB(nk));
    float *dv32 = st_in(&st_, v, FB(nk));
    uint16_t *dq = st_alloc(&st_, nq * 2), *dk = st_alloc(&st_, nk * 2), *dv = st_alloc(&st_, nk * 2);
    float *dout = st_alloc(&st_, FB(nq));
    if (!st_.err) st_kernel(&st_, aria_k_f32_to_f16(dq, dq32, nq, g_stream), "k_f2h");
    if (!st_.err) st_kernel(&st_, aria_k_f32_to_f16(dk, dk32, nk, g_stream), "k_f2h");
    if (!st_.err) st_kernel(&st_, aria_k_f32_to_f16(dv, dv32, nk, g_stream), "k_f2h");
    if (!st_.err) st_kernel(&st_, aria_k_flash_attn(dq, dk, dv, dout, 0, B * H, H, Nq, Nk, g_stream), "k_flash_attn");
    st_out(&st_, out, dout, FB(nq));
    HOST_END();
}
int aria_hip_linear_q8(float *y, const float *x, const int8_t *q, const float *scale, const float *b, int M,
                       int K, int N) {
    return host_qlinear(y, x, ARIA_WQ8, q, scale, b, M, K, N);
}
int aria_hip_linear_q4(float *y, const float *x, const uint8_t *q, const float *scale, const float *b, int M,
                       int K, int N) {
    return host_qlinear(y, x, ARIA_WQ4, q, scale, b, M, K, N);
}
int aria_hip_linear_q8a8(float *y, const float *x, const int8_t *q, const float *scale, const float *b, int M,
                         int K, int N) {
    HOST_BEGIN();
    REQ(M >= 0 && K > 0 && N >= 0 && y && x && q && scale);
    if (M == 0 || N == 0) return 0;
    float *dx = st_in(&st_, x, FB((size_t)M * K));
    void *dq = st_in(&st_, q, (size_t)N * K);
    float *ds = st_in(&st_, scale, FB(N));
    float *db = st_in(&st_, b, FB(N));
    float *dy = st_alloc(&st_, FB((size_t)M * N));
    int8_t *xq = st_alloc(&st_, (size_t)M * K);
    float *sx = st_alloc(&st_, FB(M));
    if (!st_.err) st_kernel(&st_, aria_k_quant_act_q8(xq, sx, dx, 0, M, K, g_stream), "k_quant_act_q8");
    if (!st_.err) st_kernel(&st_, aria_k_gemm_i8(dy, 0, xq, sx, dq, ds, db, M, K, N, 0, NULL, g_stream), "k_gemm_i8");
    st_out(&st_, y, dy, FB((size_t)M * N));
    HOST_END();
}


int aria_hip_q8_quant(int8_t *q, float *scale, const float *W, int N, int K) {
    HOST_BEGIN();
    REQ(N >= 0 && K > 0 && q && scale && W);
    if (N == 0) return 0;
    float *dW = st_in(&st_, W, FB((size_t)N * K));
    int8_t *dq = st_alloc(&st_, (size_t)N * K);
    float *ds = st_alloc(&st_, FB(N));
    if (!st_.err) st_kernel(&st_, aria_k_q8_quant(dq, ds, dW, N, K, g_stream), "k_q8_quant");
    st_out(&st_, q, dq, (size_t)N * K);
    st_out(&st_, scale, ds, FB(N));
    HOST_END();
}
int aria_hip_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K) {
    HOST_BEGIN();
    REQ(N >= 0 && K > 0 && q && scale && W);
    if (N == 0) return 0;
    size_t qb = (size_t)N * ((K + 1) / 2), ns = (size_t)N * 2 * ((K + 31) / 32);
    float *dW = st_in(&st_, W, FB((size_t)N * K));
    uint8_t *dq = st_alloc(&st_, qb);
    float *ds = st_alloc(&st_, FB(ns));
    if (!st_.err) st_kernel(&st_, aria_k_q4_quant(dq, ds, dW, N, K, g_stream), "k_q4_quant");
    st_out(&st_, q, dq, qb);
    st_out(&st_, scale, ds, FB(ns));
    HOST_END();
}
int aria_hip_q8_dequant(float *W, const int8_t *q, const float *scale, int N, int K) {
    HOST_BEGIN();
    REQ(N >= 0 && K > 0 && q && scale && W);
    if (N == 0) return 0;
    int8_t *dq = st_in(&st_, q, (size_t)N * K);
    float *ds = st_in(&st_, scale, FB(N));
    float *dW = st_alloc(&st_, FB((size_t)N * K));
    if (!st_.err) st_kernel(&st_, aria_k_q8_dequant(dW, dq, ds, N, K, g_stream), "k_q8_dequant");
    st_out(&st_, W, dW, FB((size_t)N * K));
    HOST_END();
}
int aria_hip_q4_dequant(float *W, const uint8_t *q, const float *scale, int N, int K) {
    HOST_BEGIN();
    REQ(N >= 0 && K > 0 && q && scale && W);
    if (N == 0) return 0;
    size_t qb = (size_t)N * ((K + 1) / 2), ns = (size_t)N * 2 * ((K + 31) / 32);
    uint8_t *dq = st_in(&st_, q, qb);
    float *ds = st_in(&st_, scale, FB(ns));
    float *dW = st_alloc(&st_, FB((size_t)N * K));
    if (!st_.err) st_kernel(&st_, aria_k_q4_dequant(dW, dq, ds, N, K, g_stream), "k_q4_dequant");
    st_out(&st_, W, dW, FB((size_t)N * K));
    HOST_END();
}

/* run one row-norm variant on host buffers */
static int host_rownorm(float *y, const float *x, const float *w, const float *b, const float *sc,
                        const float *sh, int rpb, int gelu, int resid, int norm, int rows, int dim, float eps,
                        int vec_len) {
    HOST_BEGIN();
    REQ(rows >= 0 && dim > 0 && y && x);
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    if (rows == 0) return 0;
    size_t n = (size_t)rows * dim;
    int nb = rpb > 0 ? rows / rpb : 1;
    float *dx = st_in(&st_, x, FB(n));
    float *dw = st_in(&st_, w, FB(vec_len));
    float *db = st_in(&st_, b, FB(vec_len));
    float *dsc = st_in(&st_, sc, FB((size_t)nb * dim));
    float *dsh = st_in(&st_, sh, FB((size_t)nb * dim));
    float *dy = st_alloc(&st_, FB(n));
    if (!st_.err)
        st_kernel(&st_, aria_k_rownorm(dy, 0, dx, dw, db, dsc, dsh, rpb, gelu, resid, norm, rows, dim, eps,
                                       g_stream), "k_rownorm");
    st_out(&st_, y, dy, FB(n));
    HOST_END();
}

int aria_hip_layernorm(float *y, const float *x, const float *g, const float *b, int rows, int dim, float eps) {
    return host_rownorm(y, x, g, b, NULL, NULL, 0, 0, 0, ARIA_NORM_LAYER, rows, dim, eps, dim);
}
int aria_hip_rmsnorm_adaln(float *y, const float *x, const float *w, const float *sc, const float *sh, int rows,
                           int dim, int rpb, float eps) {
    if (!sc || !sh) { set_err("invalid argument: scale/shift NULL"); return ARIA_HIP_EINVAL; }
    return host_rownorm(y, x, w, NULL, sc, sh, rpb, 0, 0, ARIA_NORM_RMS, rows, dim, eps, dim);
}
int aria_hip_ln_mod_gelu_res(float *out, const float *x, const float *g, const float *b, const float *sc,
                             const float *sh, int rows, int dim, int rpb, float eps) {
    if (!sc || !sh) { set_err("invalid argument: scale/shift NULL"); return ARIA_HIP_EINVAL; }
    return host_rownorm(out, x, g, b, sc, sh, rpb, 1, 1, ARIA_NORM_LAYER, rows, dim, eps, dim);
}

int aria_hip_modulate(float *y, const float *x, const float *sc, const float *sh, int rows, int dim, int rpb) {
    HOST_BEGIN();
    REQ(rows >= 0 && dim > 0 && y && x && sc && sh);
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    if (rows == 0) return 0;
    size_t n = (size_t)rows * dim;
    int nb = rpb > 0 ? rows / rpb : 1;
    float *dx = st_in(&st_, x, FB(n));
    float *dsc = st_in(&st_, sc, FB((size_t)nb * dim));
    float *dsh = st_in(&st_, sh, FB((size_t)nb * dim));
    float *dy = st_alloc(&st_, FB(n));
    if (!st_.err) st_kernel(&st_, aria_k_modulate(dy, dx, dsc, dsh, rows, dim, rpb, g_stream), "k_modulate");
    st_out(&st_, y, dy, FB(n));
    HOST_END();
}
int aria_hip_gate_residual(float *out, const float *res, const float *o, const float *gate, const float *bias,
                           int rows, int dim, int rpb) {
    HOST_BEGIN();
    REQ(rows >= 0 && dim > 0 && out && res && o && gate);
    REQ(rpb >= 0 && (rpb == 0 || rows % rpb == 0));
    if (rows == 0) return 0;
    size_t n = (size_t)rows * dim;
    int nb = rpb > 0 ? rows / rpb : 1;
    float *dr = st_in(&st_, res, FB(n));
    float *dov = st_in(&st_, o, FB(n));
    float *dg = st_in(&st_, gate, FB((size_t)nb * dim));
    float *db = st_in(&st_, bias, FB(dim));
    float *dout = st_alloc(&st_, FB(n));
    if (!st_.err)
        st_kernel(&st_, aria_k_gate_residual(dout, dr, dov, dg, db, rows, dim, rpb, g_stream), "k_gate_residual");
    st_out(&st_, out, dout, FB(n));
    HOST_END();
}
int aria_hip_glu_combine(float *out, const float *proj, const float *bias, int rows, int inner) {
    HOST_BEGIN();
    REQ(rows >= 0 && inner > 0 && out && proj);
    if (rows == 0) return 0;
    float *dp = st_in(&st_, proj, FB((size_t)rows * 2 * inner));
    float *db = st_in(&st_, bias, FB((size_t)2 * inner));
    float *dout = st_alloc(&st_, FB((size_t)rows * inner));
    if (!st_.err) st_kernel(&st_, aria_k_glu_combine(dout, 0, dp, db, rows, inner, g_stream), "k_glu");
    st_out(&st_, out, dout, FB((size_t)rows * inner));
    HOST_END();
}
int aria_hip_add(float *y, const float *a, const float *b, size_t n) {
    HOST_BEGIN();
    REQ(y && a && b);
    if (n == 0) return 0;
    float *da = st_in(&st_, a, FB(n));
    float *db = st_in(&st_, b, FB(n));
    float *dy = st_alloc(&st_, FB(n));
    if (!st_.err) st_kernel(&st_, aria_k_add(dy, da, db, n, g_stream), "k_add");
    st_out(&st_, y, dy, FB(n));
    HOST_END();
}
int aria_hip_pingpong(float *x, const float *v, const float *noise, float tc, float tn, size_t n) {
    HOST_BEGIN();
    REQ(x && v && noise);
    if (n == 0) return 0;
    float *dx = st_in(&st_, x, FB(n));
    float *dv = st_in(&st_, v, FB(n));
    float *dz = st_in(&st_, noise, FB(n));
    if (!st_.err) st_kernel(&st_, aria_k_pingpong(dx, dv, dz, tc, tn, n, g_stream), "k_pingpong");
    st_out(&st_, x, dx, FB(n));
    HOST_END();
}

/* ------------------------------------------------------------------------- */
/* reference op-level host wrappers (src/aria_gpu.h:38-61)                   */
/* ------------------------------------------------------------------------- */

void aria_cuda_linear_dev(float *dy, const float *dx, const float *dW, const float *db, int M, int K, int N) {
    if (ensure() || M <= 0 || N <= 0) return;
    hipError_t e = aria_k_sgemm(dy, dx, dW, db, M, N, K, 1, 1.0f, 1, 0, 0, 0, g_stream);
    if (e != hipSuccess) hip_fail(e, "k_sgemm");
}

void aria_cuda_linear(float *y, const float *x, const float *W, const float *b, int M, int K, int N) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || M <= 0 || N <= 0) return;
    float *dx = st_in(&st, x, FB((size_t)M * K));
    float *dW = st_in(&st, W, FB((size_t)N * K));
    float *db = st_in(&st, b, FB(N));
    float *dy = st_alloc(&st, FB((size_t)M * N));
    if (!st.err) st_kernel(&st, aria_k_sgemm(dy, dx, dW, db, M, N, K, 1, 1.0f, 1, 0, 0, 0, g_stream), "k_sgemm");
    st_out(&st, y, dy, FB((size_t)M * N));
    st_finish(&st);
}

void aria_cuda_matmul(float *Cm, const float *A, const float *B, int M, int K, int N) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || M <= 0 || N <= 0) return;
    float *dA = st_in(&st, A, FB((size_t)M * K));
    float *dB = st_in(&st, B, FB((size_t)K * N));
    float *dC = st_alloc(&st, FB((size_t)M * N));
    if (!st.err) st_kernel(&st, aria_k_sgemm(dC, dA, dB, NULL, M, N, K, 0, 1.0f, 1, 0, 0, 0, g_stream), "k_sgemm");
    st_out(&st, Cm, dC, FB((size_t)M * N));
    st_finish(&st);
}

static void host_norm_void(float *y, const float *x, const float *w, int rows, int dim, float eps, int norm) {
    host_rownorm(y, x, w, NULL, NULL, NULL, 0, 0, 0, norm, rows, dim, eps, dim);
}
void aria_cuda_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps) {
    host_norm_void(y, x, w, rows, dim, eps, ARIA_NORM_RMS);
}
void aria_cuda_gemma_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps) {
    host_norm_void(y, x, w, rows, dim, eps, ARIA_NORM_GEMMA);
}

void aria_cuda_dynamic_tanh(float *y, const float *x, float alpha, const float *w, const float *b, int rows,
                            int dim) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || rows <= 0 || dim <= 0) return;
    size_t n = (size_t)rows * dim;
    float *dx = st_in(&st, x, FB(n));
    float *dw = st_in(&st, w, FB(dim));
    float *db = st_in(&st, b, FB(dim));
    float *dy = st_alloc(&st, FB(n));
    if (!st.err) st_kernel(&st, aria_k_dynamic_tanh(dy, dx, alpha, dw, db, rows, dim, g_stream), "k_dyt");
    st_out(&st, y, dy, FB(n));
    st_finish(&st);
}

/* in-place unary op on a host buffer */
static void host_inplace(float *x, size_t n, int op, float a) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || n == 0 || !x) return;
    float *dx = st_in(&st, x, FB(n));
    if (!st.err) {
        hipError_t e = op == 0 ? aria_k_silu(dx, dx, n, g_stream)
                     : op == 1 ? aria_k_gelu_tanh(dx, dx, n, g_stream)
                               : aria_k_softcap(dx, dx, a, n, g_stream);
        st_kernel(&st, e, "k_unary");
    }
    st_out(&st, x, dx, FB(n));
    st_finish(&st);
}
void aria_cuda_silu(float *x, int n) { if (n > 0) host_inplace(x, (size_t)n, 0, 0.0f); }
void aria_cuda_gelu_tanh(float *x, int n) { if (n > 0) host_inplace(x, (size_t)n, 1, 0.0f); }
void aria_cuda_softcap(float *s, int n, float cap) { if (n > 0) host_inplace(s, (size_t)n, 2, cap); }

void aria_cuda_silu_gate(float *out, const float *gate, const float *up, int n) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || n <= 0) return;
    float *dg = st_in(&st, gate, FB(n));
    float *du = st_in(&st, up, FB(n));
    float *dout = st_alloc(&st, FB(n));
    if (!st.err) st_kernel(&st, aria_k_silu_gate(dout, dg, du, (size_t)n, g_stream), "k_silu_gate");
    st_out(&st, out, dout, FB(n));
    st_finish(&st);
}

void aria_cuda_softmax(float *x, int rows, int cols, const float *mask) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || rows <= 0 || cols <= 0) return;
    size_t n = (size_t)rows * cols;
    float *dx = st_in(&st, x, FB(n));
    float *dm = st_in(&st, mask, FB(n));
    if (!st.err) st_kernel(&st, aria_k_softmax(dx, rows, cols, dm, g_stream), "k_softmax");
    st_out(&st, x, dx, FB(n));
    st_finish(&st);
}

void aria_cuda_rope_apply(float *x, const float *cos_t, const float *sin_t, int H, int N, int D, int rot_dim) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || H <= 0 || N <= 0 || D <= 0 || rot_dim <= 0 || rot_dim > D) return;
    size_t n = (size_t)H * N * D, nt = (size_t)N * (rot_dim / 2);
    float *dx = st_in(&st, x, FB(n));
    float *dc = st_in(&st, cos_t, FB(nt));
    float *ds = st_in(&st, sin_t, FB(nt));
    if (!st.err) st_kernel(&st, aria_k_rope(dx, dc, ds, H, N, D, rot_dim, g_stream), "k_rope");
    st_out(&st, x, dx, FB(n));
    st_finish(&st);
}

/* attention (src/aria_cpu.c:811-849): per head scores = (q k^T) * 1/sqrtf(D),
 * softmax(+mask), out = P V; the two contractions in fp32. */
void aria_cuda_attention(float *out, const float *q, const float *k, const float *v, int H, int Nq, int Nk, int D,
                         const float *mask) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || H <= 0 || Nq <= 0 || Nk <= 0 || D <= 0) return;
    size_t nq = (size_t)H * Nq * D, nk = (size_t)H * Nk * D, ns = (size_t)H * Nq * Nk;
    float *dq = st_in(&st, q, FB(nq));
    float *dk = st_in(&st, k, FB(nk));
    float *dv = st_in(&st, v, FB(nk));
    float *dm = st_in(&st, mask, FB((size_t)Nq * Nk));
    float *dsc = st_alloc(&st, FB(ns));
    float *dout = st_alloc(&st, FB(nq));
    float scale = 1.0f / sqrtf((float)D);
    if (!st.err)
        st_kernel(&st, aria_k_sgemm(dsc, dq, dk, NULL, Nq, Nk, D, 1, scale, H, (long long)Nq * D,
                                    (long long)Nk * D, (long long)Nq * Nk, g_stream), "k_sgemm(qk)");
    if (!st.err) {
        if (dm) {   /* the mask is [Nq, Nk], shared by every head */
            for (int h = 0; h < H && !st.err; h++)
                st_kernel(&st, aria_k_softmax(dsc + (size_t)h * Nq * Nk, Nq, Nk, dm, g_stream), "k_softmax");
        } else {
            st_kernel(&st, aria_k_softmax(dsc, H * Nq, Nk, NULL, g_stream), "k_softmax");
        }
    }
    if (!st.err)
        st_kernel(&st, aria_k_sgemm(dout, dsc, dv, NULL, Nq, D, Nk, 0, 1.0f, H, (long long)Nq * Nk,
                                    (long long)Nk * D, (long long)Nq * D, g_stream), "k_sgemm(pv)");
    st_out(&st, out, dout, FB(nq));
    st_finish(&st);
}

void aria_cuda_conv1d(float *out, const float *in, const float *w, const float *bias, int Cin, int Cout, int K,
                      int pad, int L) {
    stage_t st = {{0}, 0, 0};
    if (ensure() || Cin <= 0 || Cout <= 0 || K <= 0 || L <= 0) return;
    float *din = st_in(&st, in, FB((size_t)Cin * L));
    float *dw = st_in(&st, w, FB((size_t)Cout * Cin * K));
    float *db = st_in(&st, bias, FB(Cout));
    float *dout = st_alloc(&st, FB((size_t)Cout * L));
    if (!st.err) st_kernel(&st, aria_k_conv1d(dout, din, dw, db, Cin, Cout, K, pad, L, g_stream), "k_conv1d");
    st_out(&st, out, dout, FB((size_t)Cout * L));
    st_finish(&st);
}
