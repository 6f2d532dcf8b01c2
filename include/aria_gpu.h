/*
 * aria_gpu.h - the GPU backend C ABI, served by the MI355X (gfx950) HIP backend
 * libaria_hip.so. Drop-in for the reference's src/aria_gpu.h: the same symbol
 * names (the aria_cuda_* prefix is kept because the reference's callers,
 * src/aria_model_sa3.c and tests/test_cuda.c, call these names unchanged), the
 * same argument order and meaning, the same ownership (host wrappers allocate,
 * copy in, launch, copy out and free; all are synchronous on return).
 *
 * Errors: as in the reference, the void functions report a HIP failure on
 * stderr ("[aria-hip] ...") and return; aria_cuda_malloc returns NULL.
 * aria_hip_last_error() (aria_hip.h) exposes the last failure as text.
 *
 * Each declaration names the reference line it replaces.
 */
#ifndef ARIA_GPU_H
#define ARIA_GPU_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/aria_gpu.h:20 - 1 if a HIP device is usable, else 0. */
int aria_cuda_available(void);
/* src/aria_gpu.h:24 - 1 when the device beats the CPU path (CDNA3/CDNA4: gfx942, gfx950). */
int aria_cuda_recommended(void);
/* src/aria_gpu.h:25 - 1 when the W8A8 int8 path is served: on gfx950 (int8 MFMA), where
 * aria_cuda_dit_create with ARIA_Q8A8 (and ARIA_DTYPE_AUTO) runs the int8 projections. */
int aria_cuda_int8_tc(void);
/* src/aria_gpu.h:27 - "name (gfxNNN, CUs, VRAM)" into buf. */
void aria_cuda_device_info(char *buf, size_t buflen);
/* src/aria_gpu.h:29 - device memory in use and total, bytes. */
void aria_cuda_meminfo(size_t *used, size_t *total);

/* src/aria_gpu.h:32-36 - raw device memory. */
void *aria_cuda_malloc(size_t bytes);
void  aria_cuda_free(void *dptr);
void  aria_cuda_memcpy_h2d(void *ddst, const void *hsrc, size_t bytes);
void  aria_cuda_memcpy_d2h(void *hdst, const void *dsrc, size_t bytes);
void  aria_cuda_sync(void);

/* src/aria_gpu.h:40-43 - y[M,N] = x[M,K] W[N,K]^T + b (b may be NULL);
 * _dev takes device pointers, the plain form host pointers. */
void aria_cuda_linear_dev(float *dy, const float *dx, const float *dW, const float *db,
                          int M, int K, int N);
void aria_cuda_linear(float *y, const float *x, const float *W, const float *b,
                      int M, int K, int N);

/* src/aria_gpu.h:46-60 - host-pointer wrappers mirroring src/aria_ops.h. */
void aria_cuda_matmul(float *C, const float *A, const float *B, int M, int K, int N);
void aria_cuda_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps);
void aria_cuda_gemma_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps);
void aria_cuda_dynamic_tanh(float *y, const float *x, float alpha,
                            const float *w, const float *b, int rows, int dim);
void aria_cuda_softcap(float *s, int n, float cap);
void aria_cuda_silu(float *x, int n);
void aria_cuda_gelu_tanh(float *x, int n);
void aria_cuda_silu_gate(float *out, const float *gate, const float *up, int n);
void aria_cuda_softmax(float *x, int rows, int cols, const float *mask);
void aria_cuda_rope_apply(float *x, const float *cos_t, const float *sin_t,
                          int H, int N, int D, int rot_dim);
void aria_cuda_attention(float *out, const float *q, const float *k, const float *v,
                         int H, int Nq, int Nk, int D, const float *mask);
void aria_cuda_conv1d(float *out, const float *in, const float *w, const float *bias,
                      int Cin, int Cout, int K, int pad, int L);

#ifdef __cplusplus
}
#endif
#endif /* ARIA_GPU_H */
