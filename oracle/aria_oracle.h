/*
 * aria_oracle.h - TEST INFRASTRUCTURE ONLY. A scalar CPU restatement of the
 * reference's DiT tensor-op path (matteospanio/aria src/aria_cpu.c,
 * src/aria_quant.c, src/aria_sa3_dit.c, src/aria_sampler.c), used as the parity
 * checker for the HIP backend. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links it.
 *
 * Every function is single-threaded, evaluates in the reference's order and is
 * built with -ffp-contract=off (the reference's -std=c11 build does not contract
 * a*b+c into an FMA). Where the reference uses an explicit FMA or a SIMD
 * reduction order, the comment says what this restatement does instead and
 * which tolerance covers the difference.
 *
 * Pinning (what checks each function beyond restating it) is listed per function
 * in the header of oracle/aria_oracle.c.
 */
#ifndef ARIA_ORACLE_H
#define ARIA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- row normalisations ---- */
void or_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps);
void or_gemma_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps);
void or_layernorm(float *y, const float *x, const float *gamma, const float *beta,
                  int rows, int dim, float eps);

/* ---- adaLN / gate / residual (DiT block glue) ---- */
void or_adaln_modulate(float *y, const float *scale, const float *shift, int rows, int dim);
void or_gate_sigmoid(float *y, const float *gate, int rows, int dim);
void or_gate_residual(float *out, const float *res, const float *o, const float *gate,
                      const float *bias, int rows, int dim);

/* ---- elementwise ---- */
void or_add(float *y, const float *a, const float *b, size_t n);
void or_addto(float *y, const float *a, size_t n);
void or_scale(float *y, const float *x, float s, size_t n);
void or_axpy(float *y, const float *x, float s, size_t n);
void or_gelu_tanh(float *x, size_t n);
void or_silu(float *x, size_t n);
void or_silu_gate(float *out, const float *gate, const float *up, size_t n);
void or_glu_combine(float *out, const float *proj, const float *bias, int rows, int inner);
void or_pingpong(float *x, const float *v, const float *noise, float tc, float tn, size_t n);

/* ---- softmax / rotary ---- */
void or_softmax(float *x, int rows, int cols, const float *mask);
void or_rope_freqs(float *cos_t, float *sin_t, int n, int rot_dim, float base);
void or_rope_apply(float *x, const float *cos_t, const float *sin_t,
                   int H, int N, int D, int rot_dim);

/* ---- fused config-1/2 chain: out = gelu(LN(x)*(1+scale)+shift) + x ---- */
void or_fused_chain(float *out, const float *x, const float *gamma, const float *beta,
                    const float *scale, const float *shift, int batch, int rows_per_batch,
                    int dim, float eps);

/* ---- quantisation ---- */
void or_q8_quant(int8_t *q, float *scale, const float *W, int N, int K);
void or_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K);
void or_q8_dequant(float *W, const int8_t *q, const float *scale, int N, int K);
void or_q4_dequant(float *W, const uint8_t *q, const float *scale, int N, int K);
void or_linear_q8(float *y, const float *x, const int8_t *q, const float *scale,
                  const float *b, int M, int K, int N);
void or_quant_act_q8(int8_t *xq, float *sx, const float *x, int M, int K);
void or_linear_q8a8(float *y, const float *x, const int8_t *q, const float *scale,
                    const float *b, int M, int K, int N);
void or_linear_q4(float *y, const float *x, const uint8_t *q, const float *scale,
                  const float *b, int M, int K, int N);

/* ---- dense fp32 ---- */
void or_linear(float *y, const float *x, const float *W, const float *b, int M, int K, int N);
void or_matmul(float *C, const float *A, const float *B, int M, int K, int N);
void or_attention(float *out, const float *q, const float *k, const float *v,
                  int H, int Nq, int Nk, int D, const float *mask);

#ifdef __cplusplus
}
#endif
#endif /* ARIA_ORACLE_H */
