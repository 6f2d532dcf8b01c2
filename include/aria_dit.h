/*
 * aria_dit.h - the DiT block on the MI355X backend (libaria_hip.so).
 *
 * Types restated from the reference so a caller of its DiT code can pass the same
 * structures (the layout must match byte for byte; tests/test_abi.py checks it):
 *   aria_dtype        src/aria_quant.h:27-35
 *   aria_dit_block_w  src/aria_sa3_dit.h:40-48 (21 host fp32 pointers, PyTorch Linear
 *                     layout [out, in])
 *
 * aria_hip_dit_block is one block's weights resident in HBM, packed per the
 * reference's mixed-precision recipe (src/aria_sa3_dit.c:473-506, device mirror
 * src/aria_cuda.cu:1216-1229): with precision ARIA_Q4 the attention projections
 * (sa_to_qkv, sa_to_out, ca_to_q, ca_to_out) are Q8 and the FFN (ff_in, ff_out) Q4;
 * with ARIA_Q8 all six are Q8; with ARIA_F32/F16/BF16 they are fp16. ca_to_kv is
 * fp16 in every case (it runs once per request). Packing happens on the device and is
 * bit-exact with the reference host quantizer (aria_q8_quant / aria_q4_quant).
 *
 * The forward pass replaces dit_block_core (src/aria_sa3_dit.c:141-312) and the
 * reference device block dit_block_dev (src/aria_cuda.cu:1037-1157) for B independent
 * sequences (B = 2 for CFG) sharing the weights: the GEMMs run over M = B*S rows,
 * attention per (sequence, head). It allocates nothing: the caller passes a
 * workspace of aria_hip_dit_block_workspace_bytes() bytes, so the call can be
 * captured in a HIP graph.
 */
#ifndef ARIA_DIT_H
#define ARIA_DIT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef ARIA_QUANT_H
typedef enum {
    ARIA_F32 = 0,
    ARIA_F16 = 1,
    ARIA_BF16 = 2,
    ARIA_Q8 = 3,
    ARIA_Q4 = 4,
    ARIA_Q8A8 = 5,
    ARIA_DTYPE_AUTO = 6,
} aria_dtype;
#endif

#ifndef ARIA_SA3_DIT_H
typedef struct {
    const float *pre_norm, *cross_norm, *ff_norm;
    const float *sa_to_qkv, *sa_q_norm, *sa_k_norm, *sa_to_out;
    const float *ca_to_q, *ca_to_kv, *ca_q_norm, *ca_k_norm, *ca_to_out;
    const float *ff_in_w, *ff_in_b, *ff_out_w, *ff_out_b;
    const float *to_scale_shift_gate;
    const float *to_local0_w, *to_local0_b, *to_local2_w, *to_local2_b;
} aria_dit_block_w;
#endif

/* FFN form: GLU is the SA3 DiT's (ff_in_w [2*inner, dim], out = silu(gate)*value with
 * value = first half, src/aria_sa3_dit.c:108-121); GELU is a plain tanh-GELU MLP
 * (ff_in_w [inner, dim]). */
enum { ARIA_FFN_GLU = 0, ARIA_FFN_GELU = 1 };

typedef struct aria_hip_dit_block aria_hip_dit_block;

/* Upload and pack one block. dim = num_heads * head_dim (head_dim must be 64),
 * inner = FFN hidden width, dim_ctx = cross-attention context width. Host weights
 * are read, not kept. NULL on failure (aria_hip_last_error()). */
aria_hip_dit_block *aria_hip_dit_block_create(const aria_dit_block_w *w, int dim, int num_heads,
                                              int head_dim, int inner, int ffn, int dim_ctx,
                                              aria_dtype precision);
void aria_hip_dit_block_free(aria_hip_dit_block *b);
/* device bytes the block occupies (packed weights + vectors) */
size_t aria_hip_dit_block_weight_bytes(const aria_hip_dit_block *b);
/* workspace bytes for B sequences of S tokens and Sc context tokens */
size_t aria_hip_dit_block_workspace_bytes(const aria_hip_dit_block *b, int B, int S, int Sc);

/* Per request: the block's cross-attention K/V from the context (the reference
 * projects them once per request, src/aria_sa3_dit.c:644-693, src/aria_cuda.cu:1324-1353):
 * dctx [B*Sc, dim_ctx] fp32 -> dk, dv fp16 [B, H, Sc, 64] (k RMS-normalised with
 * ca_k_norm, eps 1e-6). */
int aria_hip_dit_block_cross_kv_dev(aria_hip_dit_block *b, const float *dctx, int B, int Sc,
                                    uint16_t *dk, uint16_t *dv, void *dws, size_t ws_bytes,
                                    void *stream);

/* One block forward, in place on dx [B*S, dim] fp32 (the residual stream).
 * dgcond: [B, 6*dim] per-sequence global conditioning added to to_scale_shift_gate
 * (the modulation is chunked scale_self, shift_self, gate_self, scale_ff, shift_ff,
 * gate_ff, src/aria_sa3_dit.c:152-156); NULL means zero.
 * dk/dv: cross K/V from aria_hip_dit_block_cross_kv_dev (Sc keys).
 * dcos/dsin: RoPE tables [S, rot/2] for positions 0..S-1; rot = 32 or 64 (0 = none).
 * Sub-layer norms use eps 1e-5, q/k norms 1e-6 (src/aria_sa3_dit.c:149). */
int aria_hip_dit_block_forward_dev(aria_hip_dit_block *b, float *dx, int B, int S, const float *dgcond,
                                   const uint16_t *dk, const uint16_t *dv, int Sc, const float *dcos,
                                   const float *dsin, int rot, void *dws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* ARIA_DIT_H */
