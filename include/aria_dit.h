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

/* ------------------------------------------------------------------------- */
/* The reference's device-resident DiT ABI (src/aria_sa3_dit.h:127-171)      */
/* ------------------------------------------------------------------------- */

#ifndef ARIA_STEER_H
/* src/aria_steer.h:14-38 (steering is accepted; this backend does not apply it) */
typedef enum { ARIA_STEER_RESIDUAL = 0, ARIA_STEER_LATENT, ARIA_STEER_COND } aria_steer_site;
typedef enum { ARIA_STEER_ADD = 0, ARIA_STEER_PROJECT } aria_steer_op;
typedef struct {
    aria_steer_site site;
    aria_steer_op op;
    int layer;
    const float *dir;
    int dim;
    float dir_norm2;
    float scale;
    int step_lo, step_hi;
} aria_steer;
typedef struct { const aria_steer *items; int n; } aria_steer_set;
#endif

#ifndef ARIA_SA3_DIT_H
/* src/aria_sa3_dit.h:128-133 */
typedef struct {
    int depth, ed, num_heads, head_dim, inner, io_ch, n_mem, rot_dim;
    int differential;
    const float *preprocess, *postprocess, *project_in, *project_out, *memory_tokens;
    const aria_dit_block_w *blocks;
} aria_sa3_dit_view;
/* src/aria_sa3_dit.h:136-145 */
typedef struct {
    int T, S, n_cond, depth;
    const float *global_seconds, *rope_cos, *rope_sin;
    float *const *cross_k, *const *cross_v;
    float *const *cross_kd;
    const float *cross_ed;
    float *const *local_emb;
    int has_local;
    const aria_steer_set *steer;
} aria_sa3_dit_req_view;
typedef struct aria_cuda_dit aria_cuda_dit;
#endif

/* src/aria_sa3_dit.h:155 - upload the model (SiLU-GLU blocks, ca_to_kv [2*ed, ed]) packed
 * per precision (see aria_hip_dit_block_create). NULL when there is no device, the shape
 * is unsupported (differential attention, head_dim != 64) or it does not fit; the
 * reference's caller then runs the CPU DiT (src/aria_model_sa3.c:503-509). */
aria_cuda_dit *aria_cuda_dit_create(const aria_sa3_dit_view *v, aria_dtype precision);
/* src/aria_sa3_dit.h:156 */
void aria_cuda_dit_free(aria_cuda_dit *h);
/* src/aria_sa3_dit.h:157 - per request: cross K/V of every block from cross_ed (projected on
 * the device), RoPE tables, local-additive cond; copies what it needs (steer is borrowed). */
void aria_cuda_dit_set_request(aria_cuda_dit *h, const aria_sa3_dit_req_view *rv);
/* src/aria_sa3_dit.h:159 - current denoise step (steering window; kept for the ABI) */
void aria_cuda_dit_set_step(aria_cuda_dit *h, int step);
/* src/aria_sa3_dit.h:161 - v_CT = velocity(x_CT, gcond), [io_ch, T] host buffers, gcond [6*ed];
 * synchronous. The step runs as one captured HIP graph after its first call
 * (ARIA_NO_GRAPH=1 forces the inline path). */
void aria_cuda_dit_step(aria_cuda_dit *h, float *v_CT, const float *x_CT, const float *gcond);
/* src/aria_sa3_dit.h:167-171 - the pingpong sampler with x resident on the device; gcond_all
 * [steps][6*ed], noise(buf, n, user) called once per step in order; bit-identical to
 * aria_cuda_dit_step + the host pingpong update. -1 (nothing run) if pinned staging fails. */
int aria_cuda_dit_sample(aria_cuda_dit *h, float *x_CT, const float *sched, int steps,
                         const float *gcond_all, void (*noise)(float *, int, void *), void *noise_user,
                         void (*progress)(int, int, void *), void *progress_user);

/* aria_cuda_dit_create with the FFN form chosen: ARIA_FFN_GLU (the SA3 model, what
 * aria_cuda_dit_create builds) or ARIA_FFN_GELU (a tanh-GELU MLP, ff_in_w [inner, ed]). */
aria_cuda_dit *aria_hip_dit_create_ex(const aria_sa3_dit_view *v, aria_dtype precision, int ffn);

/* ---- batched extension: B sequences (the CFG pair) per pass over the weights ---- */
/* rv: B request views with equal T and n_cond (one cross_ed each). */
int aria_hip_dit_set_request_batch(aria_cuda_dit *h, const aria_sa3_dit_req_view *rv, int B);
/* host buffers: v, x [B, io_ch, T]; gcond [B, 6*ed]; synchronous */
int aria_hip_dit_step_batch(aria_cuda_dit *h, float *v, const float *x, const float *gcond);
/* The handle's device step buffers (x [B, io_ch, T] in, v out, gcond [B, 6*ed]) and one
 * stream-ordered step on them (graph replay after the first call), for callers that keep
 * the latent in HBM; stream NULL = the handle's stream. */
int aria_hip_dit_device_buffers(aria_cuda_dit *h, float **dx, float **dv, float **dgcond);
int aria_hip_dit_run(aria_cuda_dit *h, void *stream);
/* 1 if the step runs as a captured graph, 0 if inline */
int aria_hip_dit_graph_active(const aria_cuda_dit *h);
/* Load the reference's packed block overlay (.aria: aria_sa3_dit_quant_save's file,
 * src/aria_sa3_dit.c:509-527, records of aria_qweight_write, src/aria_quant.c:439-449) into the
 * device model: the six block GEMM weights of every block are taken from the file as packed
 * (Q8 / Q4 per record) instead of being quantised from the f32 view, so the quantisation at
 * create is skipped (the reference loads it with aria_sa3_dit_quant_load, src/aria_sa3_dit.c:
 * 529-551, for its CPU path). depth / ed / inner and every record's shape must match the model;
 * a W8A8 (ARIA_Q8A8) model needs Q8 records. A captured step is dropped (re-captured on the
 * next step). 0, or an error with the model unchanged. */
int aria_hip_dit_load_overlay(aria_cuda_dit *h, const char *path);

/* ---- device decoders (src/aria_sa3_dec.h:75-109) ----
 * The small-music decoder runs on the device: aria_cuda_dec_create uploads the weight view
 * (the reference's aria_sa3_dec_get_view fills it, src/aria_sa3_dec.c:299-318), and
 * aria_cuda_dec_forward decodes latent [256, T] -> audio [2, T * 4096], host buffers,
 * synchronous, as the reference's caller uses it (src/aria_model_sa3.c:293-305, 634-647).
 * create returns NULL when there is no device or the weights do not fit (the caller keeps
 * its CPU decoder). The medium decoder is not served: its create returns NULL.
 * The two view types restate the reference's field for field (same order, same types), so
 * a view filled by the reference's loader is read as is. */
#ifndef ARIA_SA3_DEC_H
typedef struct {
    float pre_alpha, qn_alpha, kn_alpha, ff_alpha;
    const float *pre_gamma, *pre_beta, *qn_gamma, *qn_beta, *kn_gamma, *kn_beta, *ff_gamma, *ff_beta;
    const float *to_qkv, *to_out, *ff_in_w, *ff_in_b, *ff_out_w, *ff_out_b;
} aria_taae_block_view;
typedef struct {
    float running_std;
    const float *proj_w, *proj_b, *new_tokens, *mapping_w, *mapping_b;
    aria_taae_block_view blocks[6];
} aria_sa3_dec_view;
typedef struct aria_sa3_dec_medium_view aria_sa3_dec_medium_view;
typedef struct aria_cuda_dec aria_cuda_dec;
typedef struct aria_cuda_dec_medium aria_cuda_dec_medium;
aria_cuda_dec *aria_cuda_dec_create(const aria_sa3_dec_view *v);
void aria_cuda_dec_free(aria_cuda_dec *h);
void aria_cuda_dec_forward(aria_cuda_dec *h, float *audio, const float *latent, int T);
aria_cuda_dec_medium *aria_cuda_dec_medium_create(const aria_sa3_dec_medium_view *v);
void aria_cuda_dec_medium_free(aria_cuda_dec_medium *h);
void aria_cuda_dec_medium_forward(aria_cuda_dec_medium *h, float *audio, const float *latent, int T);
#endif

/* ---- decoder extension: the decode on device buffers ----
 * latent [256, T] and audio [2, T * 4096] in HBM, enqueued on the handle's stream
 * (aria_hip_dec_stream) and not waited for; 0 or a negative ARIA_HIP_E* code. */
int aria_hip_dec_forward_dev(aria_cuda_dec *h, float *daudio, const float *dlatent, int T);
void *aria_hip_dec_stream(const aria_cuda_dec *h);
/* device bytes of the decode workspace (grown to the longest T decoded so far) */
size_t aria_hip_dec_workspace_bytes(const aria_cuda_dec *h);

#ifdef __cplusplus
}
#endif
#endif /* ARIA_DIT_H */
