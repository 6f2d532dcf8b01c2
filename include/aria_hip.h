/*
 * aria_hip.h - device-pointer, stream-ordered entry points of the MI355X backend
 * (libaria_hip.so), beside the reference-compatible ABI in aria_gpu.h.
 *
 * These are the hot-path operations the reference's device DiT composes inside
 * src/aria_cuda.cu (fused norm+modulate, gate+residual, GLU, softmax, RoPE, Q8/Q4
 * dequant-on-use GEMM, pingpong), exposed one by one so that a caller holding
 * device buffers can chain them on one stream with no host round trip, and the
 * host-pointer forms of the quantizer/GEMM interfaces of src/aria_quant.h.
 *
 * Conventions:
 *   - Pointers named d* or taking "device" in the comment are device memory;
 *     all others are host memory.
 *   - stream: a hipStream_t passed as void*; NULL means the library's own stream
 *     (aria_hip_default_stream()). Device-pointer calls only enqueue work.
 *   - Return value: 0 on success, a negative ARIA_HIP_E* code on a rejected
 *     argument, or the positive hipError_t of a failed HIP call.
 *     aria_hip_last_error() describes the last failure.
 *   - Shapes are row-major fp32 unless stated; weights are PyTorch Linear
 *     [N = out, K = in] (src/aria_ops.h:10).
 *   - rows_per_batch: per-batch broadcast vectors (adaLN scale/shift/gate) are
 *     [rows / rows_per_batch, dim]; row r uses vector r / rows_per_batch.
 */
#ifndef ARIA_HIP_H
#define ARIA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARIA_HIP_EINVAL  (-1)   /* bad shape, NULL where a buffer is required */
#define ARIA_HIP_ENODEV  (-2)   /* no usable HIP device */
#define ARIA_HIP_ENOMEM  (-3)   /* device allocation failed */

/* ---- runtime ---- */
/* Select device 0 and create the library stream; idempotent, thread-safe.
 * Returns 0, or ARIA_HIP_ENODEV. Every other call initialises on demand. */
int aria_hip_init(void);
const char *aria_hip_last_error(void);
void *aria_hip_default_stream(void);
int aria_hip_stream_sync(void *stream);
/* A further stream (non-blocking, default priority) for callers that run work side by side, or
 * NULL; aria_hip_stream_destroy ignores NULL and the library's own stream. */
void *aria_hip_stream_create(void);
void aria_hip_stream_destroy(void *stream);
/* HIP events for stream-ordered timing (bench harness). */
void *aria_hip_event_create(void);
void aria_hip_event_destroy(void *ev);
int aria_hip_event_record(void *ev, void *stream);
/* milliseconds between two recorded events (synchronises on the second), or -1 */
float aria_hip_event_elapsed_ms(void *ev0, void *ev1);
int aria_hip_memcpy_h2d_async(void *ddst, const void *hsrc, size_t bytes, void *stream);
int aria_hip_memcpy_d2h_async(void *hdst, const void *dsrc, size_t bytes, void *stream);
int aria_hip_memcpy_d2d_async(void *ddst, const void *dsrc, size_t bytes, void *stream);
/* device properties: number of CUs, and the gfx target name ("gfx950") */
int aria_hip_cu_count(void);
int aria_hip_arch(char *buf, size_t buflen);

/* ---- row normalisations (device pointers) ----
 * Replace aria_rmsnorm / aria_gemma_rmsnorm (src/aria_ops.h:91-108,
 * src/aria_cpu.c:643-733). LayerNorm has no reference op: biased variance,
 * y = (x - mean)/sqrt(var + eps) * gamma + beta, gamma/beta may be NULL. */
int aria_hip_rmsnorm_dev(float *dy, const float *dx, const float *dw, int rows, int dim,
                         float eps, void *stream);
int aria_hip_gemma_rmsnorm_dev(float *dy, const float *dx, const float *dw, int rows, int dim,
                               float eps, void *stream);
int aria_hip_layernorm_dev(float *dy, const float *dx, const float *dgamma, const float *dbeta,
                           int rows, int dim, float eps, void *stream);
/* Fused RMSNorm(w) -> adaLN modulate, one pass: y = (x*inv*w)*(1+scale)+shift.
 * The reference runs aria_rmsnorm then adaln_modulate (src/aria_sa3_dit.c:175-176,
 * 255-256); its device twin is k_rmsnorm_adaln(_h) (src/aria_cuda.cu:199-249).
 * out_f16 != 0 writes IEEE half (the GEMM operand) into dy. */
int aria_hip_rmsnorm_adaln_dev(void *dy, int out_f16, const float *dx, const float *dw,
                               const float *dscale, const float *dshift, int rows, int dim,
                               int rows_per_batch, float eps, void *stream);
/* Config 1/2 chain fused into one pass:
 * out = gelu_tanh(LayerNorm(x)*gamma+beta)*(1+scale)+shift) + x. */
int aria_hip_ln_mod_gelu_res_dev(float *dout, const float *dx, const float *dgamma,
                                 const float *dbeta, const float *dscale, const float *dshift,
                                 int rows, int dim, int rows_per_batch, float eps, void *stream);

/* ---- elementwise / broadcast (device pointers; n counts floats) ----
 * aria_add/addto/scale/axpy, aria_silu, aria_gelu_tanh, aria_silu_gate
 * (src/aria_ops.h:111-117,166-170); y may alias x. */
int aria_hip_add_dev(float *dy, const float *da, const float *db, size_t n, void *stream);
int aria_hip_axpy_dev(float *dy, const float *dx, float a, size_t n, void *stream);
int aria_hip_scale_dev(float *dy, const float *dx, float a, size_t n, void *stream);
int aria_hip_gelu_tanh_dev(float *dy, const float *dx, size_t n, void *stream);
int aria_hip_silu_dev(float *dy, const float *dx, size_t n, void *stream);
int aria_hip_silu_gate_dev(float *dout, const float *dgate, const float *dup, size_t n,
                           void *stream);
/* adaln_modulate (src/aria_sa3_dit.c:71-82): y = x*(1+scale)+shift. */
int aria_hip_modulate_dev(float *dy, const float *dx, const float *dscale, const float *dshift,
                          int rows, int dim, int rows_per_batch, void *stream);
/* gate_sigmoid + residual (src/aria_sa3_dit.c:85-97, 211-215) as one pass:
 * out = res + (o [+ bias]) * sigmoid(1 - gate); out may alias res. */
int aria_hip_gate_residual_dev(float *dout, const float *dres, const float *do_,
                               const float *dgate, const float *dbias, int rows, int dim,
                               int rows_per_batch, void *stream);
/* GLU combine (src/aria_sa3_dit.c:108-121): proj [rows, 2*inner] = [value | gate],
 * out[r,i] = silu(gate (+b)) * (value (+b)); out_f16 writes half. */
int aria_hip_glu_combine_dev(void *dout, int out_f16, const float *dproj, const float *dbias,
                             int rows, int inner, void *stream);
/* pingpong (src/aria_sampler.c:216-220): x = (1-tn)*(x - tc*v) + tn*noise,
 * each operation rounded on its own: bit-identical to the host loop. */
int aria_hip_pingpong_dev(float *dx, const float *dv, const float *dnoise, float tc, float tn,
                          size_t n, void *stream);

/* ---- softmax / rotary (device pointers) ---- */
/* aria_softmax_inplace (src/aria_ops.h:164), mask [rows, cols] or NULL. */
int aria_hip_softmax_dev(float *dx, int rows, int cols, const float *dmask, void *stream);
/* aria_rope_apply (src/aria_ops.h:126): x [H, N, D] in place, tables [N, rot/2]. */
int aria_hip_rope_apply_dev(float *dx, const float *dcos, const float *dsin, int H, int N, int D,
                            int rot_dim, void *stream);
/* The same rotation on q and k (same shape, distinct buffers) in one launch, as the
 * DiT applies it (src/aria_sa3_dit.c:193-194). */
int aria_hip_rope_apply2_dev(float *dq, float *dk, const float *dcos, const float *dsin, int H, int N,
                             int D, int rot_dim, void *stream);

/* ---- quantisation (src/aria_quant.h layouts) ---- */
/* Device pack: bit-exact with aria_q8_quant / aria_q4_quant (src/aria_quant.c:78, 353). */
int aria_hip_q8_quant_dev(int8_t *dq, float *dscale, const float *dW, int N, int K, void *stream);
int aria_hip_q4_quant_dev(uint8_t *dq, float *dscale, const float *dW, int N, int K, void *stream);
/* Device unpack to fp32 (the per-weight value the dequant GEMM uses). */
int aria_hip_q8_dequant_dev(float *dW, const int8_t *dq, const float *dscale, int N, int K,
                            void *stream);
int aria_hip_q4_dequant_dev(float *dW, const uint8_t *dq, const float *dscale, int N, int K,
                            void *stream);

/* Dequant-on-use GEMM on MFMA, y[M,N] = x[M,K] W[N,K]^T (+ b[N]); b may be NULL.
 * Replaces aria_linear_q8 / aria_linear_q4 (src/aria_quant.h:45, 65;
 * src/aria_quant.c:98-145, 469-538) and the reference's dequantize-to-fp16 +
 * cublasGemmEx device path (src/aria_cuda.cu:1009-1035). Weights stay packed in HBM.
 * wtype 0 = Q8 (dq int8 [N,K], dscale [N]), 1 = Q4 (dq u8 [N,ceil(K/2)], dscale
 * [N, 2*ceil(K/32)] [min,step] pairs), 2 = fp16 weights (dq = half [N,K], dscale unused).
 * x_f16 / y_f16 select IEEE-half activations / outputs instead of fp32. */
int aria_hip_qlinear_dev(void *dy, int y_f16, const void *dx, int x_f16, int wtype, const void *dq,
                         const float *dscale, const float *db, int M, int K, int N, void *stream);
/* As aria_hip_qlinear_dev with an explicit workgroup tile (M x N): 1 = 192x128,
 * 2 = 128x128, 3 = 96x256, 4 = 96x128, 5 = 128x256, 6 = 64x128, 7 = 128x64, 8 = 64x64
 * (both operands staged through LDS); 9..12 = 32x256, 64x256, 96x256, 128x256 with the
 * weights loaded straight into registers (Q8/Q4 with K % 64 == 0, else the 128x128 LDS
 * kernel); 0 = chosen from the shape (tuning knob; fp32 activations without an fp16
 * staging buffer always run 128x128). */
int aria_hip_qlinear_ex_dev(void *dy, int y_f16, const void *dx, int x_f16, int wtype, const void *dq,
                            const float *dscale, const float *db, int M, int K, int N, int tiles,
                            void *stream);
int aria_hip_linear_q8_dev(float *dy, const float *dx, const int8_t *dq, const float *dscale,
                           const float *db, int M, int K, int N, void *stream);
/* aria_hip_qlinear_dev that allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results, bit for bit; the
 * fp16 staging of fp32 activations goes to a static device array of
 * ARIA_HIP_NOALLOC_SCRATCH bytes per GPU instead of per-call pool memory, so M * K * 2 must
 * not exceed it (ARIA_HIP_EINVAL otherwise; fp16 activations need no staging). Every call
 * on one GPU shares that array. A staging call on another stream than the GPU's previous one
 * first waits (hipStreamWaitEvent) for that call's GEMM, so calls from several streams or
 * threads run one after another on the device. Under stream capture the call records no
 * event and waits for none: inside a graph the caller orders the calls. */
#define ARIA_HIP_NOALLOC_SCRATCH ((size_t)32 << 20)
int aria_hip_qlinear_noalloc_dev(void *dy, int y_f16, const void *dx, int x_f16, int wtype, const void *dq,
                                 const float *dscale, const float *db, int M, int K, int N, void *stream);
int aria_hip_linear_q4_dev(float *dy, const float *dx, const uint8_t *dq, const float *dscale,
                           const float *db, int M, int K, int N, void *stream);

/* ---- W8A8: int8 activations x int8 weights on the int8 MFMA ----
 * Replaces the reference's gemm_w8a8 / gemm_w8a8_h (src/aria_cuda.cu:934-1004: per-token
 * activation quantisation k_quant_act_q8(_h), int8 IMMA GEMM into int32, dequant k_deq_i32)
 * with the numbers of aria_linear_q8a8 (src/aria_quant.h:47-51, src/aria_quant.c:253-345),
 * bit for bit. */
/* RMSNorm(w) (-> adaLN modulate with per-batch dscale / dshift [rows / rows_per_batch, dim],
 * or both NULL) with W8A8 output, one pass: the fp32 result row (the aria_hip_rmsnorm_adaln_dev
 * value) is quantised in registers as aria_hip_quant_act_q8_dev does, dyq int8 [rows, dim] and
 * dsx [rows]. The reference's W8A8 block runs k_rmsnorm(_adaln) into fp32 then
 * k_quant_act_q8 (src/aria_cuda.cu:1075, 1094, 1133 with 934-949). dim 256, 512, 768, 1024 or
 * 2048. */
int aria_hip_rmsnorm_adaln_q8_dev(int8_t *dyq, float *dsx, const float *dx, const float *dw, const float *dscale,
                                  const float *dshift, int rows, int dim, int rows_per_batch, float eps,
                                  void *stream);
/* Per-row symmetric int8 activations: sx[m] = amax / 127 (amax = max |x[m,:]|),
 * dxq[m,k] = clamp(rint(x * 127 / amax), -127, 127), all zero when amax == 0. dx is
 * fp32 or fp16 (x_f16) [M, K]; dxq [M, K] int8, dsx [M]. */
int aria_hip_quant_act_q8_dev(int8_t *dxq, float *dsx, const void *dx, int x_f16, int M, int K,
                              void *stream);
/* dy[m,n] = (float)(sum_k dxq[m,k] dq[n,k]) * dsx[m] * dscale[n] (+ db[n], else + 0.0f),
 * exact int32 sums, fp32 (or fp16 with y_f16) output. dq / dscale are the Q8 weight
 * (aria_q8_quant layout). */
int aria_hip_gemm_i8_dev(void *dy, int y_f16, const int8_t *dxq, const float *dsx, const int8_t *dq,
                         const float *dscale, const float *db, int M, int K, int N, void *stream);
/* Both steps, as aria_linear_q8a8 on device data: dws is caller workspace of at least
 * aria_hip_q8a8_ws_bytes(M, K) bytes (the int8 rows and their scales). */
size_t aria_hip_q8a8_ws_bytes(int M, int K);
int aria_hip_linear_q8a8_dev(float *dy, const void *dx, int x_f16, const int8_t *dq, const float *dscale,
                             const float *db, int M, int K, int N, void *dws, void *stream);
/* Host-pointer form with the reference's signature (src/aria_quant.h:50). */
int aria_hip_linear_q8a8(float *y, const float *x, const int8_t *q, const float *scale, const float *b,
                         int M, int K, int N);

/* ---- attention (the DiT's, head dim 64) ----
 * Head preparation, replacing extract_heads + q/k RMSNorm + RoPE of the block
 * (src/aria_sa3_dit.c:183-194, 222-226): dsrc [B*S, ld] fp32 holds nsec sections of
 * H*64 columns (e.g. the qkv projection); section i is written to ddst[i] (a host
 * array of device pointers) as fp16 [B, H, S, 64]. kind[i]: 0 = q, 1 = k (RMSNorm
 * with dw[i] (may be NULL), eps, then RoPE over rot dims with tables [S, rot/2];
 * rot 0 = none), 2 = v (copy). kind and ddst/dw are host arrays of nsec entries. */
int aria_hip_qkv_prep_dev(const float *dsrc, int ld, int B, int S, int H, int nsec, const int *kind,
                          uint16_t *const *ddst, const float *const *dw, const float *dcos,
                          const float *dsin, int rot, float eps, void *stream);
/* Fused attention, replacing aria_attention (src/aria_ops.h:135, src/aria_cpu.c:811-849)
 * for the DiT: q [B*H, Nq, D], k/v [B*H, Nk, D] fp16 -> dout [B, Nq, H*D] with heads
 * merged (the layout the output projection reads), fp16 when out_f16 else fp32.
 * softmax(q k^T / sqrt(D)) v with scores kept on chip. D must be 64. */
int aria_hip_flash_attention_dev(const uint16_t *dq, const uint16_t *dk, const uint16_t *dv, void *dout,
                                 int out_f16, int B, int H, int Nq, int Nk, int D, void *stream);
/* Host form of the fused attention (parity entry): q/k/v fp32 [B*H, N, D] are rounded
 * to fp16 on the device; out fp32 [B, Nq, H*D]. */
int aria_hip_attention_f16(float *out, const float *q, const float *k, const float *v, int B, int H,
                           int Nq, int Nk, int D);

/* Host-pointer forms with the reference's signatures (src/aria_quant.h:43-45, 64-65):
 * allocate, copy in, run, copy out, free; synchronous. Return 0 or an error. */
int aria_hip_q8_quant(int8_t *q, float *scale, const float *W, int N, int K);
int aria_hip_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K);
int aria_hip_q8_dequant(float *W, const int8_t *q, const float *scale, int N, int K);
int aria_hip_q4_dequant(float *W, const uint8_t *q, const float *scale, int N, int K);
int aria_hip_linear_q8(float *y, const float *x, const int8_t *q, const float *scale,
                       const float *b, int M, int K, int N);
int aria_hip_linear_q4(float *y, const float *x, const uint8_t *q, const float *scale,
                       const float *b, int M, int K, int N);

/* ---- host-pointer forms of the fused ops (parity entry points) ---- */
int aria_hip_layernorm(float *y, const float *x, const float *gamma, const float *beta,
                       int rows, int dim, float eps);
int aria_hip_rmsnorm_adaln(float *y, const float *x, const float *w, const float *scale,
                           const float *shift, int rows, int dim, int rows_per_batch, float eps);
int aria_hip_ln_mod_gelu_res(float *out, const float *x, const float *gamma, const float *beta,
                             const float *scale, const float *shift, int rows, int dim,
                             int rows_per_batch, float eps);
int aria_hip_modulate(float *y, const float *x, const float *scale, const float *shift,
                      int rows, int dim, int rows_per_batch);
int aria_hip_gate_residual(float *out, const float *res, const float *o, const float *gate,
                           const float *bias, int rows, int dim, int rows_per_batch);
int aria_hip_glu_combine(float *out, const float *proj, const float *bias, int rows, int inner);
int aria_hip_add(float *y, const float *a, const float *b, size_t n);
int aria_hip_pingpong(float *x, const float *v, const float *noise, float tc, float tn, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* ARIA_HIP_H */
