/*
 * aria_hip_kernels.h - internal: C-callable launchers of the gfx950 kernels.
 *
 * The .hip translation units own the kernels and expose one launcher each; the
 * C host backend (aria_hip.c) validates shapes, then calls these. Every
 * launcher takes device pointers and a HIP stream, enqueues work and returns
 * the hipError_t of the launch (0 = success). None of them allocates.
 */
#ifndef ARIA_HIP_KERNELS_H
#define ARIA_HIP_KERNELS_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Row normalisation with optional fused epilogue (k_rownorm.hip).
 * norm: 0 RMSNorm y=(x*inv)*w, 1 Gemma y=(x*inv)*(1+w), 2 LayerNorm y=n*g+b.
 * Epilogue, in this order, each optional:
 *   scale/shift (adaLN modulate, [nbatch, dim], batch = row / rows_per_batch),
 *   gelu (tanh GELU), resid (+ x of the same row).
 * out_f16 != 0 stores IEEE half (RTNE) instead of float. */
enum { ARIA_NORM_RMS = 0, ARIA_NORM_GEMMA = 1, ARIA_NORM_LAYER = 2 };
hipError_t aria_k_rownorm(void *y, int out_f16, const float *x, const float *w, const float *b,
                          const float *scale, const float *shift, int rows_per_batch,
                          int gelu, int resid, int norm, int rows, int dim, float eps,
                          hipStream_t s);
/* the same with nt != 0: the row is loaded and the result stored with non-temporal hints
 * (for the standalone ops, whose operands are streamed once) */
hipError_t aria_k_rownorm_nt(void *y, int out_f16, const float *x, const float *w, const float *b,
                             const float *scale, const float *shift, int rows_per_batch,
                             int gelu, int resid, int norm, int rows, int dim, float eps, int nt,
                             hipStream_t s);
/* RMSNorm + adaLN with scale = scale_t[c] + scale_g[b * g_bs + c] formed in place (scale_g,
 * shift_g may be NULL); w may be NULL */
hipError_t aria_k_rownorm_ada(void *y, int out_f16, const float *x, const float *w,
                              const float *scale_t, const float *shift_t, const float *scale_g,
                              const float *shift_g, int g_bs, int rows_per_batch, int rows,
                              int dim, float eps, hipStream_t s);
/* RMSNorm (w may be NULL; scale / shift per batch [rows / rows_per_batch, dim] or NULL) and
 * RMSNorm + adaLN with the modulation formed in place, with W8A8 output: yq int8 [rows, dim]
 * with sx[row] = amax / 127, the quantisation of the fp32 result (aria_k_quant_act_q8's rule);
 * dim must be one the register path takes (256, 512, 768, 1024, 2048) */
hipError_t aria_k_rownorm_q8(int8_t *yq, float *sx, const float *x, const float *w, const float *scale,
                             const float *shift, int rows_per_batch, int rows, int dim, float eps, hipStream_t s);
hipError_t aria_k_rownorm_ada_q8(int8_t *yq, float *sx, const float *x, const float *w, const float *scale_t,
                                 const float *shift_t, const float *scale_g, const float *shift_g, int g_bs,
                                 int rows_per_batch, int rows, int dim, float eps, hipStream_t s);

/* Elementwise (k_elementwise.hip). n counts floats. */
hipError_t aria_k_add(float *y, const float *a, const float *b, size_t n, hipStream_t s);
hipError_t aria_k_scale(float *y, const float *x, float a, size_t n, hipStream_t s);
hipError_t aria_k_axpy(float *y, const float *x, float a, size_t n, hipStream_t s);
hipError_t aria_k_gelu_tanh(float *y, const float *x, size_t n, hipStream_t s);
hipError_t aria_k_silu(float *y, const float *x, size_t n, hipStream_t s);
hipError_t aria_k_softcap(float *y, const float *x, float cap, size_t n, hipStream_t s);
hipError_t aria_k_silu_gate(float *out, const float *gate, const float *up, size_t n,
                            hipStream_t s);
hipError_t aria_k_dynamic_tanh(float *y, const float *x, float alpha, const float *w,
                               const float *b, int rows, int dim, hipStream_t s);
/* y = x*(1+scale[batch])+shift[batch], [rows, dim], batch = row / rows_per_batch. */
hipError_t aria_k_modulate(float *y, const float *x, const float *scale, const float *shift,
                           int rows, int dim, int rows_per_batch, hipStream_t s);
/* out = res + (o [+ bias]) * sigmoid(1 - gate[batch]); gate [nbatch, dim]. */
hipError_t aria_k_gate_residual(float *out, const float *res, const float *o,
                                const float *gate, const float *bias, int rows, int dim,
                                int rows_per_batch, hipStream_t s);
/* out[r, i] = silu(proj[r, inner+i] (+b)) * (proj[r, i] (+b)); out_f16 stores half. */
hipError_t aria_k_glu_combine(void *out, int out_f16, const float *proj, const float *bias,
                              int rows, int inner, hipStream_t s);
/* x = (1-tn)*(x - tc*v) + tn*noise, each op rounded on its own. */
hipError_t aria_k_pingpong(float *x, const float *v, const float *noise, float tc, float tn,
                           size_t n, hipStream_t s);
/* fp32 -> fp16 (RTNE), n elements. */
hipError_t aria_k_f32_to_f16(uint16_t *y, const float *x, size_t n, hipStream_t s);
/* per batch b: dst[b] [cols, rows] = transpose of src[b] [rows, cols] */
hipError_t aria_k_transpose(float *dst, const float *src, int rows, int cols, int batch, hipStream_t s);
/* mod[c][b][i] = tssg[c*dim+i] + gcond[b*6*dim + c*dim + i] (gcond may be NULL), c < 6 */
hipError_t aria_k_mod_chunks(float *mod, const float *tssg, const float *gcond, int B, int dim,
                             hipStream_t s);

/* Row softmax in place with optional additive mask [rows, cols] (k_softmax.hip). */
hipError_t aria_k_softmax(float *x, int rows, int cols, const float *mask, hipStream_t s);

/* Rotate-half RoPE in place on x [H, N, D]; tables [N, rot/2] (k_rope.hip). */
hipError_t aria_k_rope(float *x, const float *cos_t, const float *sin_t, int H, int N, int D,
                       int rot_dim, hipStream_t s);
/* the same rotation on two tensors of one shape (q and k) in one launch; x1 may be NULL */
hipError_t aria_k_rope2(float *x0, float *x1, const float *cos_t, const float *sin_t, int H, int N,
                        int D, int rot_dim, hipStream_t s);

/* Quantisation (k_quant.hip). Layouts are the reference's aria_quant.h ones. */
hipError_t aria_k_q8_quant(int8_t *q, float *scale, const float *W, int N, int K, hipStream_t s);
hipError_t aria_k_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K,
                           hipStream_t s);
hipError_t aria_k_q8_dequant(float *W, const int8_t *q, const float *scale, int N, int K,
                             hipStream_t s);
hipError_t aria_k_q4_dequant(float *W, const uint8_t *q, const float *scale, int N, int K,
                             hipStream_t s);

/* Dequant-on-use GEMM on MFMA (k_qgemm.hip): y[M,N] = x[M,K] W^T (+ bias[N]).
 * wtype: ARIA_WQ8 (q int8 [N,K], scale [N]), ARIA_WQ4 (q u8 [N,ceil(K/2)], scale
 * [N, 2*ceil(K/32)] as [min, step] pairs), ARIA_WF16 (q = fp16 W [N,K], scale unused).
 * x is fp32 or fp16 (x_f16), y fp32 or fp16 (y_f16). */
enum { ARIA_WQ8 = 0, ARIA_WQ4 = 1, ARIA_WF16 = 2, ARIA_WI8 = 3 };
/* Fused epilogues, applied to v = acc * scale (+ bias) (GELU'd when gelu != 0):
 *   STORE     y = v (fp32 or fp16)
 *   GATE_RES  y = y + v * sigmoid(1 - g), g = gate[b * gate_bs + col]
 *             (+ gate2[b * gate2_bs + col]), b = row / rows_per_batch      (fp32, in place)
 *   ADD       y = (y + v) (+ add2)                                        (fp32, in place)
 *   HEADS     the N columns are nsec sections of heads*64: each 64-column head is
 *             RMS-normalised (w, statistic in double) and rotated (RoPE rot dims) for
 *             kinds 0/1, copied for kind 2, and written fp16 to dst[sec] as
 *             [batch, heads, rows_per_batch, 64] (y unused)
 *   GLU       columns interleave (value, gate) pairs: y[m][c/2] = silu(gate) * value,
 *             [M, N/2], fp16 or fp32 (y_f16) (the weight rows were interleaved when packed)
 *   ADD_DYT   ADD, then also dst[0][m][c] = half(tanh(eps * y) * w[0][c] + w[1][c]) of the new y
 *             (the next DynamicTanh norm's GEMM operand; eps carries alpha; fp16 weights only)
 *   DYT_ROPE  the decoder's attention operands: N = 5 sections of heads*64 columns (q | k | v |
 *             qd | kd); per head dim d, q and qd become tanh(eps x) * w[0][d] + w[1][d], k and
 *             kd tanh(eps2 x) * w[2][d] + w[3][d], then rotate-half RoPE over the first rot
 *             dims (8, 16 or 32) at position m % rows_per_batch (cos_t / sin_t
 *             [rows_per_batch, rot / 2]); v as it is; y fp32 [M, N] (fp16 weights only) */
enum { ARIA_EPI_STORE = 0, ARIA_EPI_GATE_RES = 1, ARIA_EPI_ADD = 2, ARIA_EPI_HEADS = 3, ARIA_EPI_GLU = 4,
       ARIA_EPI_ADD_DYT = 5, ARIA_EPI_DYT_ROPE = 6 };
typedef struct {
    int mode, rows_per_batch;
    const float *gate, *add2, *gate2;
    int gate_bs, gate2_bs;
    int heads, nsec, kind[3];
    uint16_t *dst[3];
    const float *w[4];
    const float *cos_t, *sin_t;
    int rot;
    float eps, eps2;
} aria_qgemm_epi;
hipError_t aria_k_qgemm(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                        const float *scale, const float *bias, int M, int K, int N, hipStream_t s);
/* the same with an explicit workgroup tile (M x N): 1..8 = the LDS-operand kernel's
 * 192x128, 128x128, 96x256, 96x128, 128x256, 64x128, 128x64, 64x64; 9..12 = the
 * weights-in-registers kernel's 32x256 .. 128x256 (Q8/Q4, K % 64 == 0); 0 = picked from
 * the shape; gelu != 0 applies tanh-GELU after bias */
hipError_t aria_k_qgemm_t(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                          const float *scale, const float *bias, int M, int K, int N, int tiles,
                          int gelu, hipStream_t s);
/* the same with a fused epilogue (epi NULL = STORE); HEADS needs N % 64 == 0 */
hipError_t aria_k_qgemm_e(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                          const float *scale, const float *bias, int M, int K, int N, int tiles,
                          int gelu, const aria_qgemm_epi *epi, hipStream_t s);

/* W8A8 (k_gemm_i8.hip), the reference's gemm_w8a8 (src/aria_cuda.cu:934-990) and
 * aria_linear_q8a8 (src/aria_quant.c:253-345).
 * aria_k_quant_act_q8: per row, amax = max |x|, sx[m] = amax / 127, xq = clamp(rint(x * 127 /
 *   amax), -127, 127) (all zero when amax == 0); x fp32 or fp16 (x_f16) [M, K].
 * aria_k_gemm_i8: y = (float)(xq . q) * sx[m] * scale[n] (+ bias[n], else + 0.0f): exact int32
 *   dot products on the int8 MFMA, the two multiplies rounded in that order, then the fused
 *   epilogue (epi NULL = STORE; gelu as in aria_k_qgemm_e). K % 64 == 0 with 16-byte aligned
 *   rows runs the MFMA kernel; other shapes a SIMT kernel (STORE only, no GELU). */
hipError_t aria_k_quant_act_q8(int8_t *xq, float *sx, const void *x, int x_f16, int M, int K, hipStream_t s);
hipError_t aria_k_gemm_i8(void *y, int y_f16, const int8_t *xq, const float *sx, const int8_t *q,
                          const float *scale, const float *bias, int M, int K, int N, int gelu,
                          const aria_qgemm_epi *epi, hipStream_t s);
/* the same with the tile height fixed: fm = 1..4 (32 fm rows x 256 columns), 0 = picked */
hipError_t aria_k_gemm_i8_t(void *y, int y_f16, const int8_t *xq, const float *sx, const int8_t *q,
                            const float *scale, const float *bias, int M, int K, int N, int fm, int gelu,
                            const aria_qgemm_epi *epi, hipStream_t s);

/* Attention (k_attn.hip). Head preparation: src [B*S, ld] fp32 holds nsec sections of
 * H*64 columns; kind[i] = 0 (q: RMSNorm w[i] + RoPE), 1 (k: same), 2 (v: copy); each
 * section is written to dst[i] as fp16 [B, H, S, 64]. rot = 0 skips RoPE. */
hipError_t aria_k_qkv_prep(const float *src, int ld, int B, int S, int H, int nsec, const int *kind,
                           uint16_t *const *dst, const float *const *w, const float *cos_t,
                           const float *sin_t, int rot, float eps, hipStream_t s);
/* fused attention, head dim 64: q [BH, Nq, 64], k/v [BH, Nk, 64] fp16 -> o [B, Nq, H*64]
 * (merged heads, fp16 when o_f16 else fp32), scale 1/8 */
hipError_t aria_k_flash_attn(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *o, int o_f16,
                             int BH, int H, int Nq, int Nk, hipStream_t s);
/* memory read (and discarded) by workgroups added to an attention launch on the CUs its own
 * workgroups leave idle, so that it passes through the memory-side cache before a later
 * kernel reads it (up to ARIA_PF_SPANS spans; bytes a multiple of 16, 16-byte aligned) */
#define ARIA_PF_SPANS 12
typedef struct {
    const void *p[ARIA_PF_SPANS];
    size_t bytes[ARIA_PF_SPANS];
    int n;
} aria_prefetch_set;
/* aria_k_flash_attn that also prefetches pf (NULL: none) on the CUs the split form leaves idle */
hipError_t aria_k_flash_attn_pf(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *o, int o_f16,
                                int BH, int H, int Nq, int Nk, const aria_prefetch_set *pf, hipStream_t s);

/* fp32 SIMT GEMM (k_sgemm.hip), batched with element strides sA/sB/sC:
 * C_b[M,N] = alpha * (A_b[M,K] op(B_b)) (+ bias[N]); op(B) = B^T for B_b [N,K]
 * (transB = 1, Linear layout) or B for B_b [K,N] (transB = 0). */
hipError_t aria_k_sgemm(float *C, const float *A, const float *B, const float *bias, int M, int N,
                        int K, int transB, float alpha, int batch, long long sA, long long sB,
                        long long sC, hipStream_t s);
/* conv1d stride 1, zero padding (k_sgemm.hip). */
hipError_t aria_k_conv1d(float *out, const float *in, const float *w, const float *bias, int Cin,
                         int Cout, int K, int pad, int L, hipStream_t s);

/* The small-music decoder's glue and attention (k_dec.hip); model dim 768, 12 heads of 64,
 * 34-token chunks, 17-token groups.
 *   dec_in:     xt fp16 [T, 256] = latent [256, T] * std, transposed
 *   dec_expand: seq [Tp * 17, 768]: group t = x[t] (zeros for t >= T), then 16 new_tokens
 *   dec_dyt:    y fp16 = tanh(alpha x) * g + b over [rows, 768]
 *   dec_attn:   merged fp16 [nch * 34, 768] = the differential attention of each chunk from
 *               qkv [nch * 34, 3840] (q | k | v | qd | kd), whose q/k sections already carry
 *               the DynamicTanh norms and RoPE (the to_qkv GEMM's DYT_ROPE epilogue)
 *   dec_im2col: xc fp32 [Lt, 2304] = the k3 mapping convolution's input rows
 *   dec_map:    audio [2, M * 256] = unpatch(xc [M, 2304] . W [512, 2304]^T + b), fp32 MFMA */
hipError_t aria_k_dec_in(uint16_t *xt, const float *lat, int T, float std, hipStream_t s);
hipError_t aria_k_dec_expand(float *seq, const float *x, const float *tok, int T, int Tp, hipStream_t s);
hipError_t aria_k_dec_dyt(uint16_t *y, const float *x, float alpha, const float *g, const float *b, int rows,
                          hipStream_t s);
hipError_t aria_k_dec_attn(uint16_t *merged, const float *qkv, int nch, hipStream_t s);
hipError_t aria_k_dec_im2col(float *xc, const float *seq, int Lt, int Lout, hipStream_t s);
hipError_t aria_k_dec_map(float *audio, const float *xc, const float *W, const float *b, int M, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif /* ARIA_HIP_KERNELS_H */
