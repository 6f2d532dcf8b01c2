/*
 * aria_hip_dit.c - the DiT block on the MI355X backend (include/aria_dit.h), C11 host code.
 *
 * A block's weights live in HBM in the reference's packed layouts (Q8 / Q4 per the
 * mixed-precision recipe, fp16 otherwise). The forward pass is the order of
 * dit_block_core (src/aria_sa3_dit.c:141-312), each step one gfx950 kernel:
 *
 *   modulation chunks (scale, shift, gate) = to_scale_shift_gate + gcond, formed in the
 *            kernels that use them (the norm kernels and the gated-residual epilogues)
 *   self:    h16 = rmsnorm(x, pre_norm)*(1+scale)+shift  (fp16)    k_rownorm (fused adaLN)
 *            q,k,v = h16 . sa_to_qkv^T, split into heads, q/k rmsnorm + RoPE, fp16
 *            head-major                                             k_qgemm (Q8, HEADS epilogue)
 *            att = softmax(q k^T / 8) v (fp16, heads merged)        k_flash_attn
 *            x  += (att . sa_to_out^T) * sigmoid(1 - gate)          k_qgemm (GATE_RES epilogue)
 *   cross:   h16 = rmsnorm(x, cross_norm); q = h16 . ca_to_q^T + q-norm (HEADS epilogue);
 *            attention over the request's cached K/V; x += att . ca_to_out^T (+ local
 *            cond)                                                  k_qgemm (ADD epilogue)
 *   ffn:     h16 = rmsnorm(x, ff_norm)*(1+scale)+shift
 *            GLU:  g16 = silu(gate)*value of h16 . ff_in^T + b       k_qgemm (Q4, GLU epilogue)
 *            GELU: g16 = gelu(h16 . ff_in^T + b)                    k_qgemm with GELU epilogue
 *            x  += (g16 . ff_out^T + b) * sigmoid(1 - gate)         k_qgemm (Q4, GATE_RES epilogue)
 *
 * Nothing is allocated in the forward pass: every intermediate lives in the caller's
 * workspace (layout in ws_layout below).
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include "aria_dit.h"
#include "aria_gpu.h"
#include "aria_hip.h"
#include "aria_hip_internal.h"
#include "aria_hip_kernels.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int wtype, N, K;
    void *q;       /* int8 / u8 packed / fp16 */
    float *scale;  /* Q8 [N], Q4 [N, 2*ceil(K/32)], NULL for fp16 */
} dmat;

struct aria_hip_dit_block {
    int dim, H, hd, inner, ffn, dim_ctx, ffrows;
    int w8;   /* ARIA_Q8A8: every Q8 projection runs on int8 activations (W8A8) */
    aria_dtype prec;
    float *pre_norm, *cross_norm, *ff_norm, *sa_q_norm, *sa_k_norm, *ca_q_norm, *ca_k_norm;
    float *ff_in_b, *ff_out_b, *tssg;
    dmat sa_qkv, sa_out, ca_q, ca_out, ca_kv, ff_in, ff_out;
    size_t bytes;
};

#define FAIL(e, what) aria_hip_fail((e), (what))

static void dfree(void *p) {
    if (p) hipFree(p);
}

static int dalloc(void **p, size_t bytes, size_t *acc) {
    *p = NULL;
    hipError_t e = hipMalloc(p, bytes ? bytes : 4);
    if (e != hipSuccess) return FAIL(e, "hipMalloc (block weights)");
    if (acc) *acc += bytes;
    return 0;
}

/* device copy of a host vector (NULL stays NULL) */
static int upv(float **d, const float *h, size_t n, size_t *acc) {
    *d = NULL;
    if (!h) return 0;
    int rc = dalloc((void **)d, n * sizeof(float), acc);
    if (rc) return rc;
    hipError_t e = hipMemcpy(*d, h, n * sizeof(float), hipMemcpyHostToDevice);
    return e == hipSuccess ? 0 : FAIL(e, "hipMemcpy (block vector)");
}

/* upload W [N,K] fp32 and pack it on the device */
static int pack(dmat *m, const float *W, int N, int K, int wtype, hipStream_t s, size_t *acc) {
    memset(m, 0, sizeof *m);
    m->wtype = wtype; m->N = N; m->K = K;
    if (!W) { aria_hip_set_error("block weight missing (%d x %d)", N, K); return ARIA_HIP_EINVAL; }
    float *tmp = NULL;
    int rc = dalloc((void **)&tmp, (size_t)N * K * sizeof(float), NULL);
    if (rc) return rc;
    hipError_t e = hipMemcpy(tmp, W, (size_t)N * K * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        if (wtype == ARIA_WQ8) {
            if (!(rc = dalloc(&m->q, (size_t)N * K, acc)) && !(rc = dalloc((void **)&m->scale, (size_t)N * 4, acc)))
                e = aria_k_q8_quant((int8_t *)m->q, m->scale, tmp, N, K, s);
        } else if (wtype == ARIA_WQ4) {
            size_t qb = (size_t)N * ((K + 1) / 2), ns = (size_t)N * 2 * ((K + 31) / 32);
            if (!(rc = dalloc(&m->q, qb, acc)) && !(rc = dalloc((void **)&m->scale, ns * 4, acc)))
                e = aria_k_q4_quant((uint8_t *)m->q, m->scale, tmp, N, K, s);
        } else {
            if (!(rc = dalloc(&m->q, (size_t)N * K * 2, acc)))
                e = aria_k_f32_to_f16((uint16_t *)m->q, tmp, (size_t)N * K, s);
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    dfree(tmp);
    if (rc) return rc;
    return e == hipSuccess ? 0 : FAIL(e, "block weight packing");
}

/* device bytes of a packed matrix, as pack() and the overlay loader allocate them */
static size_t dm_bytes(const dmat *m) {
    if (!m->q) return 0;
    const size_t N = (size_t)m->N, K = (size_t)m->K;
    if (m->wtype == ARIA_WQ8) return N * K + N * 4;
    if (m->wtype == ARIA_WQ4) return N * ((K + 1) / 2) + N * 2 * ((K + 31) / 32) * 4;
    return N * K * 2;
}

static void dm_free(dmat *m) {
    dfree(m->q);
    dfree(m->scale);
    m->q = NULL; m->scale = NULL;
}

void aria_hip_dit_block_free(aria_hip_dit_block *b) {
    if (!b) return;
    float *vecs[] = {b->pre_norm, b->cross_norm, b->ff_norm, b->sa_q_norm, b->sa_k_norm, b->ca_q_norm,
                     b->ca_k_norm, b->ff_in_b, b->ff_out_b, b->tssg};
    for (size_t i = 0; i < sizeof vecs / sizeof *vecs; i++) dfree(vecs[i]);
    dm_free(&b->sa_qkv); dm_free(&b->sa_out); dm_free(&b->ca_q); dm_free(&b->ca_out);
    dm_free(&b->ca_kv); dm_free(&b->ff_in); dm_free(&b->ff_out);
    free(b);
}

aria_hip_dit_block *aria_hip_dit_block_create(const aria_dit_block_w *w, int dim, int num_heads, int head_dim,
                                              int inner, int ffn, int dim_ctx, aria_dtype precision) {
    if (aria_hip_ensure()) return NULL;
    if (!w || head_dim != 64 || num_heads <= 0 || dim != num_heads * head_dim || inner <= 0 || dim_ctx <= 0 ||
        (ffn != ARIA_FFN_GLU && ffn != ARIA_FFN_GELU) || dim % 64 || inner % 64 || dim_ctx % 32) {
        aria_hip_set_error("aria_hip_dit_block_create: unsupported shape (dim %d, heads %d x %d, inner %d, ctx %d)",
                           dim, num_heads, head_dim, inner, dim_ctx);
        return NULL;
    }

    aria_hip_dit_block *b = (aria_hip_dit_block *)calloc(1, sizeof *b);
    if (!b) return NULL;
    b->dim = dim; b->H = num_heads; b->hd = head_dim; b->inner = inner; b->ffn = ffn; b->dim_ctx = dim_ctx;
    b->ffrows = ffn == ARIA_FFN_GLU ? 2 * inner : inner;
    b->prec = precision;
    b->w8 = precision == ARIA_Q8A8;
    int attn_t, ffn_t;
    if (precision == ARIA_Q4) { attn_t = ARIA_WQ8; ffn_t = ARIA_WQ4; }
    else if (precision == ARIA_Q8 || precision == ARIA_Q8A8) { attn_t = ARIA_WQ8; ffn_t = ARIA_WQ8; }
    else { attn_t = ARIA_WF16; ffn_t = ARIA_WF16; }
    hipStream_t s = aria_hip_stream(NULL);
    size_t *acc = &b->bytes;
    int rc = 0;
    if (!rc) rc = upv(&b->pre_norm, w->pre_norm, dim, acc);
    if (!rc) rc = upv(&b->cross_norm, w->cross_norm, dim, acc);
    if (!rc) rc = upv(&b->ff_norm, w->ff_norm, dim, acc);
    if (!rc) rc = upv(&b->sa_q_norm, w->sa_q_norm, head_dim, acc);
    if (!rc) rc = upv(&b->sa_k_norm, w->sa_k_norm, head_dim, acc);
    if (!rc) rc = upv(&b->ca_q_norm, w->ca_q_norm, head_dim, acc);
    if (!rc) rc = upv(&b->ca_k_norm, w->ca_k_norm, head_dim, acc);
    /* GLU: ff_in rows (and bias) are stored interleaved (value_i, gate_i) so the GEMM
     * epilogue finds each pair in adjacent columns; rows are quantized independently, so
     * the packed values are the reference quantizer's */
    float *glu_w = NULL, *glu_b = NULL;
    if (ffn == ARIA_FFN_GLU && w->ff_in_w) {
        glu_w = (float *)malloc((size_t)2 * inner * dim * sizeof(float));
        glu_b = w->ff_in_b ? (float *)malloc((size_t)2 * inner * sizeof(float)) : NULL;
        if (!glu_w || (w->ff_in_b && !glu_b)) rc = ARIA_HIP_ENOMEM;
        for (int i = 0; i < inner && !rc; i++) {
            memcpy(glu_w + (size_t)(2 * i) * dim, w->ff_in_w + (size_t)i * dim, (size_t)dim * sizeof(float));
            memcpy(glu_w + (size_t)(2 * i + 1) * dim, w->ff_in_w + (size_t)(inner + i) * dim, (size_t)dim * sizeof(float));
            if (glu_b) { glu_b[2 * i] = w->ff_in_b[i]; glu_b[2 * i + 1] = w->ff_in_b[inner + i]; }
        }
    }
    if (!rc) rc = upv(&b->ff_in_b, glu_w ? glu_b : w->ff_in_b, (size_t)b->ffrows, acc);
    if (!rc) rc = upv(&b->ff_out_b, w->ff_out_b, dim, acc);
    if (!rc) rc = upv(&b->tssg, w->to_scale_shift_gate, (size_t)6 * dim, acc);
    if (!rc && !b->tssg) { aria_hip_set_error("to_scale_shift_gate missing"); rc = ARIA_HIP_EINVAL; }
    if (!rc) rc = pack(&b->sa_qkv, w->sa_to_qkv, 3 * dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->sa_out, w->sa_to_out, dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->ca_q, w->ca_to_q, dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->ca_out, w->ca_to_out, dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->ca_kv, w->ca_to_kv, 2 * dim, dim_ctx, ARIA_WF16, s, acc);
    if (!rc) rc = pack(&b->ff_in, glu_w ? glu_w : w->ff_in_w, b->ffrows, dim, ffn_t, s, acc);
    free(glu_w);
    free(glu_b);
    if (!rc) rc = pack(&b->ff_out, w->ff_out_w, dim, inner, ffn_t, s, acc);
    if (rc) {
        aria_hip_dit_block_free(b);
        return NULL;
    }
    return b;
}

size_t aria_hip_dit_block_weight_bytes(const aria_hip_dit_block *b) { return b ? b->bytes : 0; }

/* ---- workspace ---- */
typedef struct {
    uint16_t *h16, *q16, *k16, *v16, *att16, *ff16;
    float *big, *o;
    /* W8A8 only: int8 activations [M, max(dim, inner)] + row scales [M], and the fp32
     * producer output that is quantised (attention merge, FFN product) */
    int8_t *xq;
    float *sx, *f32;
} wsl;

#define WS_ALIGN 256
static size_t al(size_t n) { return (n + WS_ALIGN - 1) & ~(size_t)(WS_ALIGN - 1); }

static size_t ws_layout(const aria_hip_dit_block *b, int B, int S, int Sc, char *base, wsl *w) {
    const size_t M = (size_t)B * S, d = (size_t)b->dim;
    /* big: the per-request cross K/V projection [B*Sc, 2*dim] fp32; the block's own
     * projections write through their fused epilogues (o is kept for layout only) */
    const size_t big = (size_t)B * Sc * 2 * d * 4;
    const size_t wide = (size_t)(b->inner > b->dim ? b->inner : b->dim);
    const size_t sz[11] = {M * d * 2, big, M * d * 2, M * d * 2, M * d * 2, M * d * 2, 0,
                           M * (size_t)b->inner * 2,
                           b->w8 ? M * wide : 0, b->w8 ? M * 4 : 0, b->w8 ? M * wide * 4 : 0};
    size_t off = 0, o[11];
    for (int i = 0; i < 11; i++) { o[i] = off; off += al(sz[i]); }
    if (base && w) {
        w->xq = b->w8 ? (int8_t *)(base + o[8]) : NULL;
        w->sx = b->w8 ? (float *)(base + o[9]) : NULL;
        w->f32 = b->w8 ? (float *)(base + o[10]) : NULL;
        w->h16 = (uint16_t *)(base + o[0]);
        w->big = (float *)(base + o[1]);
        w->q16 = (uint16_t *)(base + o[2]);
        w->k16 = (uint16_t *)(base + o[3]);
        w->v16 = (uint16_t *)(base + o[4]);
        w->att16 = (uint16_t *)(base + o[5]);
        w->o = (float *)(base + o[6]);
        w->ff16 = (uint16_t *)(base + o[7]);
    }
    return off;
}

size_t aria_hip_dit_block_workspace_bytes(const aria_hip_dit_block *b, int B, int S, int Sc) {
    if (!b || B <= 0 || S < 0 || Sc < 0) return 0;
    return ws_layout(b, B, S, Sc, NULL, NULL);
}

#define STEP(call, name)                                     \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) return FAIL(e_, name);         \
    } while (0)

static hipError_t gemm(const dmat *m, void *y, int y_f16, const uint16_t *x16, const float *bias, int M, int gelu,
                       hipStream_t s) {
    return aria_k_qgemm_t(y, y_f16, x16, 1, m->wtype, m->q, m->scale, bias, M, m->K, m->N, 0, gelu, s);
}
/* the projection with a fused epilogue (residual stream updates, head preparation) */
static hipError_t gemm_e(const dmat *m, float *y, const uint16_t *x16, const float *bias, int M,
                         const aria_qgemm_epi *e, hipStream_t s) {
    return aria_k_qgemm_e(y, 0, x16, 1, m->wtype, m->q, m->scale, bias, M, m->K, m->N, 0, 0, e, s);
}
static aria_qgemm_epi epi_heads(int S, int H, int nsec, const int *kind, uint16_t *const *dst, const float *const *w,
                                const float *dcos, const float *dsin, int rot, float eps) {
    aria_qgemm_epi e;
    memset(&e, 0, sizeof e);
    e.mode = ARIA_EPI_HEADS; e.rows_per_batch = S; e.heads = H; e.nsec = nsec;
    for (int i = 0; i < nsec; i++) { e.kind[i] = kind[i]; e.dst[i] = dst[i]; e.w[i] = w[i]; }
    e.cos_t = dcos; e.sin_t = dsin; e.rot = rot; e.eps = eps;
    return e;
}
/* gate = gate_t[col] + gate_g[b * g_bs + col] (gate_g may be NULL) */
static aria_qgemm_epi epi_resid(int mode, int S, const float *gate_t, const float *gate_g, int g_bs,
                                const float *add2) {
    aria_qgemm_epi e;
    memset(&e, 0, sizeof e);
    e.mode = mode; e.rows_per_batch = S; e.gate = gate_t; e.gate_bs = 0; e.gate2 = gate_g; e.gate2_bs = g_bs;
    e.add2 = add2;
    return e;
}

int aria_hip_dit_block_cross_kv_dev(aria_hip_dit_block *b, const float *dctx, int B, int Sc, uint16_t *dk,
                                    uint16_t *dv, void *dws, size_t ws_bytes, void *stream) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (!b || B <= 0 || Sc <= 0 || !dctx || !dk || !dv || !dws) {
        aria_hip_set_error("aria_hip_dit_block_cross_kv_dev: invalid argument");
        return ARIA_HIP_EINVAL;
    }
    wsl w;
    if (ws_layout(b, B, 0, Sc, (char *)dws, &w) > ws_bytes) {
        aria_hip_set_error("aria_hip_dit_block_cross_kv_dev: workspace too small");
        return ARIA_HIP_EINVAL;
    }
    hipStream_t s = aria_hip_stream(stream);
    const int d = b->dim;
    /* kv = ctx . ca_to_kv^T, [B*Sc, 2*dim] = [k | v] (src/aria_sa3_dit.c:327-338) */
    rc = aria_hip_qlinear_dev(w.big, 0, dctx, 0, b->ca_kv.wtype, b->ca_kv.q, NULL, NULL, B * Sc, b->dim_ctx, 2 * d,
                              stream);
    if (rc) return rc;
    const int kind[2] = {1, 2};
    uint16_t *dst[2] = {dk, dv};
    const float *nw[2] = {b->ca_k_norm, NULL};
    STEP(aria_k_qkv_prep(w.big, 2 * d, B, Sc, b->H, 2, kind, dst, nw, NULL, NULL, 0, 1e-6f, s), "k_qkv_prep (cross kv)");
    return 0;
}

static int block_forward(aria_hip_dit_block *b, float *dx, int B, int S, const float *dgcond, const uint16_t *dk,
                         const uint16_t *dv, int Sc, const float *dcos, const float *dsin, int rot,
                         const float *dlocal, void *dws, size_t ws_bytes, const aria_hip_dit_block *next,
                         hipStream_t s);

int aria_hip_dit_block_forward_dev(aria_hip_dit_block *b, float *dx, int B, int S, const float *dgcond,
                                   const uint16_t *dk, const uint16_t *dv, int Sc, const float *dcos,
                                   const float *dsin, int rot, void *dws, size_t ws_bytes, void *stream) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    return block_forward(b, dx, B, S, dgcond, dk, dv, Sc, dcos, dsin, rot, NULL, dws, ws_bytes, NULL,
                         aria_hip_stream(stream));
}

/* an int8 projection on the block's current int8 activations (w->xq, w->sx) */
static hipError_t gemm_i8(const dmat *m, float *y, const wsl *w, const float *bias, int M, int gelu,
                          const aria_qgemm_epi *e, hipStream_t s) {
    return aria_k_gemm_i8(y, 0, w->xq, w->sx, (const int8_t *)m->q, m->scale, bias, M, m->K, m->N, gelu, e, s);
}

/* bytes of a packed matrix and of its scales */
static size_t dm_qbytes(const dmat *m) {
    return m->wtype == ARIA_WQ8 ? (size_t)m->N * m->K
         : m->wtype == ARIA_WQ4 ? (size_t)m->N * ((m->K + 1) / 2) : (size_t)m->N * m->K * 2;
}
static size_t dm_sbytes(const dmat *m) {
    return m->wtype == ARIA_WQ8 ? (size_t)m->N * 4 : m->wtype == ARIA_WQ4 ? (size_t)m->N * 2 * ((m->K + 31) / 32) * 4 : 0;
}

/* the next block's projection weights, read by the self-attention launch on the CUs it leaves
 * idle: inside a DiT step the 24 blocks' weights do not stay in the 256 MB Infinity Cache, and
 * each block's GEMMs would otherwise fetch theirs from HBM as they run */
static void next_weights(const aria_hip_dit_block *nb, aria_prefetch_set *pf) {
    pf->n = 0;
    if (!nb) return;
    const dmat *ms[] = {&nb->sa_qkv, &nb->sa_out, &nb->ca_q, &nb->ca_out, &nb->ff_in, &nb->ff_out};
    for (size_t i = 0; i < sizeof ms / sizeof *ms && pf->n + 2 <= ARIA_PF_SPANS; i++) {
        pf->p[pf->n] = ms[i]->q; pf->bytes[pf->n++] = dm_qbytes(ms[i]) & ~(size_t)15;
        pf->p[pf->n] = ms[i]->scale; pf->bytes[pf->n++] = dm_sbytes(ms[i]) & ~(size_t)15;
    }
}

/* The W8A8 block (precision ARIA_Q8A8: the reference's h->w8a8 path, src/aria_cuda.cu:1055-1147,
 * with aria_linear_q8a8's numbers): the same steps as block_forward with every projection on
 * int8 activations. The reference keeps its producers in fp32 and quantises that output per
 * row (gemm_w8a8); here the norms quantise their fp32 rows in registers and write int8 + row
 * scales directly, and the attention outputs and the FFN product, whose rows span many
 * workgroups, are written fp32 and quantised by aria_k_quant_act_q8. The int8 GEMMs carry the
 * same fused epilogues (heads, gated residual, residual + local cond, GLU / GELU). */
/* the widths whose rows the norm kernel holds in registers (and can quantise there) */
static int w8_fused_norm(int d) { return d == 256 || d == 512 || d == 768 || d == 1024 || d == 2048; }

static int block_forward_w8(aria_hip_dit_block *b, const wsl *w, float *dx, int B, int S, const float *const *tc,
                            const float *const *gc, int gbs, const uint16_t *dk, const uint16_t *dv, int Sc,
                            const float *dcos, const float *dsin, int rot, const float *dlocal,
                            const aria_prefetch_set *pf, hipStream_t s) {
    const int d = b->dim, H = b->H, M = B * S;
    const float eps_norm = 1e-5f, eps_qk = 1e-6f;

    const int fused = w8_fused_norm(d);   /* else: fp32 norm, then the quantiser */

    /* ---- self-attention ---- */
    if (fused) {
        STEP(aria_k_rownorm_ada_q8(w->xq, w->sx, dx, b->pre_norm, tc[0], tc[1], gc[0], gc[1], gbs, S, M, d, eps_norm, s),
             "k_rownorm_q8 (pre_norm + adaLN)");
    } else {
        STEP(aria_k_rownorm_ada(w->f32, 0, dx, b->pre_norm, tc[0], tc[1], gc[0], gc[1], gbs, S, M, d, eps_norm, s),
             "k_rownorm (pre_norm + adaLN)");
        STEP(aria_k_quant_act_q8(w->xq, w->sx, w->f32, 0, M, d, s), "k_quant_act_q8 (pre_norm)");
    }
    {
        const int kind[3] = {0, 1, 2};
        uint16_t *dst[3] = {w->q16, w->k16, w->v16};
        const float *nw[3] = {b->sa_q_norm, b->sa_k_norm, NULL};
        const aria_qgemm_epi e = epi_heads(S, H, 3, kind, dst, nw, dcos, dsin, rot, eps_qk);
        STEP(gemm_i8(&b->sa_qkv, NULL, w, NULL, M, 0, &e, s), "k_gemm_i8 (sa_to_qkv + heads)");
    }
    STEP(aria_k_flash_attn_pf(w->q16, w->k16, w->v16, w->f32, 0, B * H, H, S, S, pf, s), "k_flash_attn (self)");
    STEP(aria_k_quant_act_q8(w->xq, w->sx, w->f32, 0, M, d, s), "k_quant_act_q8 (self merge)");
    {
        const aria_qgemm_epi e = epi_resid(ARIA_EPI_GATE_RES, S, tc[2], gc[2], gbs, NULL);
        STEP(gemm_i8(&b->sa_out, dx, w, NULL, M, 0, &e, s), "k_gemm_i8 (sa_to_out + gated residual)");
    }

    /* ---- cross-attention ---- */
    if (fused) {
        STEP(aria_k_rownorm_q8(w->xq, w->sx, dx, b->cross_norm, NULL, NULL, 0, M, d, eps_norm, s),
             "k_rownorm_q8 (cross_norm)");
    } else {
        STEP(aria_k_rownorm(w->f32, 0, dx, b->cross_norm, NULL, NULL, NULL, 0, 0, 0, ARIA_NORM_RMS, M, d, eps_norm, s),
             "k_rownorm (cross_norm)");
        STEP(aria_k_quant_act_q8(w->xq, w->sx, w->f32, 0, M, d, s), "k_quant_act_q8 (cross_norm)");
    }
    {
        const int kind[1] = {0};
        uint16_t *dst[1] = {w->q16};
        const float *nw[1] = {b->ca_q_norm};
        const aria_qgemm_epi e = epi_heads(S, H, 1, kind, dst, nw, NULL, NULL, 0, eps_qk);
        STEP(gemm_i8(&b->ca_q, NULL, w, NULL, M, 0, &e, s), "k_gemm_i8 (ca_to_q + heads)");
    }
    STEP(aria_k_flash_attn(w->q16, dk, dv, w->f32, 0, B * H, H, S, Sc, s), "k_flash_attn (cross)");
    STEP(aria_k_quant_act_q8(w->xq, w->sx, w->f32, 0, M, d, s), "k_quant_act_q8 (cross merge)");
    {
        const aria_qgemm_epi e = epi_resid(ARIA_EPI_ADD, S, NULL, NULL, 0, dlocal);
        STEP(gemm_i8(&b->ca_out, dx, w, NULL, M, 0, &e, s), "k_gemm_i8 (ca_to_out + residual)");
    }

    /* ---- feed-forward ---- */
    if (fused) {
        STEP(aria_k_rownorm_ada_q8(w->xq, w->sx, dx, b->ff_norm, tc[3], tc[4], gc[3], gc[4], gbs, S, M, d, eps_norm, s),
             "k_rownorm_q8 (ff_norm + adaLN)");
    } else {
        STEP(aria_k_rownorm_ada(w->f32, 0, dx, b->ff_norm, tc[3], tc[4], gc[3], gc[4], gbs, S, M, d, eps_norm, s),
             "k_rownorm (ff_norm + adaLN)");
        STEP(aria_k_quant_act_q8(w->xq, w->sx, w->f32, 0, M, d, s), "k_quant_act_q8 (ff_norm)");
    }
    if (b->ffn == ARIA_FFN_GLU) {
        aria_qgemm_epi e;
        memset(&e, 0, sizeof e);
        e.mode = ARIA_EPI_GLU;
        STEP(gemm_i8(&b->ff_in, w->f32, w, b->ff_in_b, M, 0, &e, s), "k_gemm_i8 (ff_in + GLU)");
    } else {
        STEP(gemm_i8(&b->ff_in, w->f32, w, b->ff_in_b, M, 1, NULL, s), "k_gemm_i8 (ff_in + GELU)");
    }
    STEP(aria_k_quant_act_q8(w->xq, w->sx, w->f32, 0, M, b->inner, s), "k_quant_act_q8 (ffn product)");
    {
        const aria_qgemm_epi e = epi_resid(ARIA_EPI_GATE_RES, S, tc[5], gc[5], gbs, NULL);
        STEP(gemm_i8(&b->ff_out, dx, w, b->ff_out_b, M, 0, &e, s), "k_gemm_i8 (ff_out + gated residual)");
    }
    return 0;
}

/* dlocal: the inpaint local-additive conditioning [B*S, dim] added after the cross-attention
 * (src/aria_sa3_dit.c:248-252), or NULL; next: the block that runs after this one in a DiT
 * step (its weights are prefetched during this block's self-attention), or NULL */
static int block_forward(aria_hip_dit_block *b, float *dx, int B, int S, const float *dgcond, const uint16_t *dk,
                         const uint16_t *dv, int Sc, const float *dcos, const float *dsin, int rot,
                         const float *dlocal, void *dws, size_t ws_bytes, const aria_hip_dit_block *next,
                         hipStream_t s) {
    if (!b || B <= 0 || S <= 0 || Sc <= 0 || !dx || !dk || !dv || !dws || (rot && (!dcos || !dsin)) ||
        (rot != 0 && rot != 32 && rot != 64)) {
        aria_hip_set_error("aria_hip_dit_block_forward_dev: invalid argument");
        return ARIA_HIP_EINVAL;
    }
    wsl w;
    if (ws_layout(b, B, S, Sc, (char *)dws, &w) > ws_bytes) {
        aria_hip_set_error("aria_hip_dit_block_forward_dev: workspace too small");
        return ARIA_HIP_EINVAL;
    }
    const int d = b->dim, H = b->H, M = B * S;
    const float eps_norm = 1e-5f, eps_qk = 1e-6f;

    /* modulation chunk c (scale_self, shift_self, gate_self, scale_ff, shift_ff, gate_ff) =
     * to_scale_shift_gate[c] + gcond[b][c] (src/aria_sa3_dit.c:152-156), formed where it is
     * used: in the norm kernels and in the gated-residual epilogues */
    const float *tc[6], *gc[6];
    for (int c = 0; c < 6; c++) {
        tc[c] = b->tssg + (size_t)c * d;
        gc[c] = dgcond ? dgcond + (size_t)c * d : NULL;
    }
    const int gbs = 6 * d;
    aria_prefetch_set pf;
    next_weights(next, &pf);
    if (b->w8) return block_forward_w8(b, &w, dx, B, S, tc, gc, gbs, dk, dv, Sc, dcos, dsin, rot, dlocal, &pf, s);

    /* ---- self-attention ---- */
    STEP(aria_k_rownorm_ada(w.h16, 1, dx, b->pre_norm, tc[0], tc[1], gc[0], gc[1], gbs, S, M, d, eps_norm, s),
         "k_rownorm (pre_norm + adaLN)");
    {   /* qkv projection with q/k RMSNorm + RoPE and the head split in its epilogue */
        const int kind[3] = {0, 1, 2};
        uint16_t *dst[3] = {w.q16, w.k16, w.v16};
        const float *nw[3] = {b->sa_q_norm, b->sa_k_norm, NULL};
        const aria_qgemm_epi e = epi_heads(S, H, 3, kind, dst, nw, dcos, dsin, rot, eps_qk);
        STEP(gemm_e(&b->sa_qkv, NULL, w.h16, NULL, M, &e, s), "k_qgemm (sa_to_qkv + heads)");
    }
    STEP(aria_k_flash_attn_pf(w.q16, w.k16, w.v16, w.att16, 1, B * H, H, S, S, &pf, s), "k_flash_attn (self)");
    {   /* x += (att . sa_to_out^T) * sigmoid(1 - gate_self) */
        const aria_qgemm_epi e = epi_resid(ARIA_EPI_GATE_RES, S, tc[2], gc[2], gbs, NULL);
        STEP(gemm_e(&b->sa_out, dx, w.att16, NULL, M, &e, s), "k_qgemm (sa_to_out + gated residual)");
    }

    /* ---- cross-attention (no RoPE, no gate) ---- */
    STEP(aria_k_rownorm(w.h16, 1, dx, b->cross_norm, NULL, NULL, NULL, 0, 0, 0, ARIA_NORM_RMS, M, d, eps_norm, s),
         "k_rownorm (cross_norm)");
    {
        const int kind[1] = {0};
        uint16_t *dst[1] = {w.q16};
        const float *nw[1] = {b->ca_q_norm};
        const aria_qgemm_epi e = epi_heads(S, H, 1, kind, dst, nw, NULL, NULL, 0, eps_qk);
        STEP(gemm_e(&b->ca_q, NULL, w.h16, NULL, M, &e, s), "k_qgemm (ca_to_q + heads)");
    }
    STEP(aria_k_flash_attn(w.q16, dk, dv, w.att16, 1, B * H, H, S, Sc, s), "k_flash_attn (cross)");
    {   /* x += att . ca_to_out^T, then the local-additive cond (src/aria_sa3_dit.c:242-252) */
        const aria_qgemm_epi e = epi_resid(ARIA_EPI_ADD, S, NULL, NULL, 0, dlocal);
        STEP(gemm_e(&b->ca_out, dx, w.att16, NULL, M, &e, s), "k_qgemm (ca_to_out + residual)");
    }

    /* ---- feed-forward ---- */
    STEP(aria_k_rownorm_ada(w.h16, 1, dx, b->ff_norm, tc[3], tc[4], gc[3], gc[4], gbs, S, M, d, eps_norm, s),
         "k_rownorm (ff_norm + adaLN)");
    if (b->ffn == ARIA_FFN_GLU) {   /* g16 = silu(gate) * value in the projection's epilogue */
        aria_qgemm_epi e;
        memset(&e, 0, sizeof e);
        e.mode = ARIA_EPI_GLU;
        STEP(aria_k_qgemm_e(w.ff16, 1, w.h16, 1, b->ff_in.wtype, b->ff_in.q, b->ff_in.scale, b->ff_in_b, M,
                            b->ff_in.K, b->ff_in.N, 0, 0, &e, s), "k_qgemm (ff_in + GLU)");
    } else {
        STEP(gemm(&b->ff_in, w.ff16, 1, w.h16, b->ff_in_b, M, 1, s), "k_qgemm (ff_in + GELU)");
    }
    {   /* x += (g16 . ff_out^T + b) * sigmoid(1 - gate_ff) */
        const aria_qgemm_epi e = epi_resid(ARIA_EPI_GATE_RES, S, tc[5], gc[5], gbs, NULL);
        STEP(gemm_e(&b->ff_out, dx, w.ff16, b->ff_out_b, M, &e, s), "k_qgemm (ff_out + gated residual)");
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* device-resident DiT (the reference's aria_cuda_dit_* ABI)                 */
/* ------------------------------------------------------------------------- */

/* A growable staging buffer: device memory or pinned host memory. Its contents do not
 * survive a grow. */
typedef struct {
    void *p;
    size_t cap;
} sbuf;

static int sbuf_reserve(sbuf *b, size_t bytes, int pinned) {
    if (bytes <= b->cap) return 0;
    if (b->p) {
        if (pinned) hipHostFree(b->p); else hipFree(b->p);
    }
    b->p = NULL; b->cap = 0;
    const size_t want = bytes + bytes / 4;  /* slack, so a slightly longer request reuses it */
    hipError_t e = pinned ? hipHostMalloc(&b->p, want, 0) : hipMalloc(&b->p, want);
    if (e != hipSuccess) { hipGetLastError(); b->p = NULL; return -1; }
    b->cap = want;
    return 0;
}

static void sbuf_release(sbuf *b, int pinned) {
    if (b->p) {
        if (pinned) hipHostFree(b->p); else hipFree(b->p);
    }
    b->p = NULL; b->cap = 0;
}

enum { GRAPH_NONE = 0, GRAPH_LIVE = 1, GRAPH_OFF = 2 };
#define NZ_SLOTS 2

struct aria_cuda_dit {
    int depth, ed, H, inner, io_ch, n_mem, rot;
    aria_hip_dit_block **blk;
    uint16_t *pre, *post, *pin, *pout;      /* fp16: [C,C], [C,C], [ed,C], [C,ed] (as the reference's
                                             * device step keeps them, src/aria_cuda.cu:1197-1200) */
    float *mem;                             /* fp32 [n_mem, ed] */
    hipStream_t st;
    /* request state */
    int have_req, B, T, S, Sc, cur_step;
    uint16_t **ck, **cv;                    /* [depth] each [B, H, Sc, 64] */
    float *cos_t, *sin_t;                   /* [S, rot/2] */
    float **local;                          /* [depth] each [B*S, ed], or NULL */
    const aria_steer_set *steer;
    float *saved_ced;                       /* host copy of the B context embeddings */
    void *ws;
    size_t ws_bytes;
    float *dx, *dv, *dgcond, *dxtc, *dtmp, *dseq, *dout;
    /* the step as a HIP graph (see graph_ensure) */
    int gstate;                             /* GRAPH_NONE / GRAPH_LIVE / GRAPH_OFF */
    int no_graph;                           /* ARIA_NO_GRAPH at create: inline for good */
    int graph_fail;                         /* ARIA_GRAPH_FAIL at create: every capture is
                                               treated as failed (tests the fallback) */
    hipGraph_t graph;
    hipGraphExec_t gexec;
    /* sampler staging (see aria_cuda_dit_sample) */
    sbuf gc_tab;                            /* device: every step's gcond rows */
    sbuf nz_host, nz_dev;                   /* NZ_SLOTS noise slots, pinned host / device */
    hipStream_t up;                         /* upload stream for the noise slots */
    hipEvent_t ev_up[NZ_SLOTS], ev_used[NZ_SLOTS], ev_step;
    int have_events;
};

static int up_mat(float **d, const float *h, size_t n) {
    *d = NULL;
    if (!h) return 0;
    return upv(d, h, n, NULL);
}

/* fp16 device copy of an fp32 host matrix (NULL stays NULL), converted on the device (RTNE) */
static int up_mat16(uint16_t **d, const float *h, size_t n, hipStream_t s) {
    *d = NULL;
    if (!h) return 0;
    float *tmp = NULL;
    int rc = upv(&tmp, h, n, NULL);
    if (!rc) rc = dalloc((void **)d, n * 2, NULL);
    if (!rc) {
        hipError_t e = aria_k_f32_to_f16(*d, tmp, n, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = FAIL(e, "fp16 conversion (io projections)");
    }
    dfree(tmp);
    return rc;
}

/* forget the captured step (buffers or weights it names are about to change); the next
 * run captures again unless the handle is inline for good */
static void graph_drop(aria_cuda_dit *h) {
    if (h->gexec) hipGraphExecDestroy(h->gexec);
    if (h->graph) hipGraphDestroy(h->graph);
    h->gexec = NULL; h->graph = NULL;
    h->gstate = h->no_graph ? GRAPH_OFF : GRAPH_NONE;
}

static void req_free(aria_cuda_dit *h) {
    graph_drop(h);
    if (h->ck) for (int b = 0; b < h->depth; b++) { dfree(h->ck[b]); dfree(h->cv[b]); }
    if (h->local) for (int b = 0; b < h->depth; b++) dfree(h->local[b]);
    free(h->ck); free(h->cv); free(h->local);
    h->ck = h->cv = NULL; h->local = NULL;
    float *bufs[] = {h->cos_t, h->sin_t, h->dx, h->dv, h->dgcond, h->dxtc, h->dtmp, h->dseq, h->dout};
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; i++) dfree(bufs[i]);
    h->cos_t = h->sin_t = h->dx = h->dv = h->dgcond = h->dxtc = h->dtmp = h->dseq = h->dout = NULL;
    dfree(h->ws);
    h->ws = NULL; h->ws_bytes = 0;
    free(h->saved_ced);
    h->saved_ced = NULL;
    h->have_req = 0;
}

void aria_cuda_dit_free(aria_cuda_dit *h) {
    if (!h) return;
    if (aria_hip_ensure() == 0) hipStreamSynchronize(h->st);
    req_free(h);
    if (h->blk) for (int b = 0; b < h->depth; b++) aria_hip_dit_block_free(h->blk[b]);
    free(h->blk);
    void *w[] = {h->pre, h->post, h->pin, h->pout, h->mem};
    for (size_t i = 0; i < sizeof w / sizeof *w; i++) dfree(w[i]);
    if (h->up) hipStreamSynchronize(h->up);
    sbuf_release(&h->gc_tab, 0);
    sbuf_release(&h->nz_dev, 0);
    sbuf_release(&h->nz_host, 1);
    if (h->have_events) {
        for (int i = 0; i < NZ_SLOTS; i++) { hipEventDestroy(h->ev_up[i]); hipEventDestroy(h->ev_used[i]); }
        hipEventDestroy(h->ev_step);
    }
    if (h->up) hipStreamDestroy(h->up);
    if (h->st) hipStreamDestroy(h->st);
    free(h);
}

aria_cuda_dit *aria_hip_dit_create_ex(const aria_sa3_dit_view *v, aria_dtype precision, int ffn) {
    if (aria_hip_ensure() || !v || !v->blocks) return NULL;
    if (v->differential || v->head_dim != 64 || v->num_heads * v->head_dim != v->ed || v->depth <= 0 ||
        v->io_ch <= 0 || v->n_mem < 0 || (v->rot_dim != 0 && v->rot_dim != 32 && v->rot_dim != 64)) {
        aria_hip_set_error("aria_cuda_dit_create: unsupported model shape");
        return NULL;
    }
    /* auto: W8A8 where the int8 matrix path exists, as the reference (src/aria_model_sa3.c:500-502) */
    if (precision == ARIA_DTYPE_AUTO) precision = aria_cuda_int8_tc() ? ARIA_Q8A8 : ARIA_F32;
    /* ARIA_W8A8 set (any value) turns a Q8 model into W8A8, the reference's opt-in knob
     * (src/aria_cuda.cu:1186, and aria_linear_qw on the CPU, src/aria_quant.c:420-421) */
    if (precision == ARIA_Q8 && getenv("ARIA_W8A8") != NULL) precision = ARIA_Q8A8;
    aria_cuda_dit *h = (aria_cuda_dit *)calloc(1, sizeof *h);
    if (!h) return NULL;
    h->depth = v->depth; h->ed = v->ed; h->H = v->num_heads; h->inner = v->inner; h->io_ch = v->io_ch;
    h->n_mem = v->n_mem; h->rot = v->rot_dim;
    const char *ng = getenv("ARIA_NO_GRAPH");   /* read once per handle */
    h->no_graph = ng && ng[0] && ng[0] != '0';
    const char *gf = getenv("ARIA_GRAPH_FAIL");
    h->graph_fail = gf && gf[0] && gf[0] != '0';
    h->gstate = h->no_graph ? GRAPH_OFF : GRAPH_NONE;
    if (hipStreamCreateWithFlags(&h->st, hipStreamNonBlocking) != hipSuccess) { free(h); return NULL; }
    /* VRAM fit: packed blocks (<= fp16 size) + fp32 io projections, with margin */
    size_t fr = 0, tot = 0;
    hipMemGetInfo(&fr, &tot);
    const size_t per_block = ((size_t)10 * v->ed * v->ed + (size_t)(ffn == ARIA_FFN_GLU ? 3 : 2) * v->inner * v->ed) * 2;
    if ((size_t)v->depth * per_block + ((size_t)256 << 20) > fr) {
        aria_hip_set_error("aria_cuda_dit_create: model does not fit in device memory");
        aria_cuda_dit_free(h);
        return NULL;
    }
    h->blk = (aria_hip_dit_block **)calloc((size_t)v->depth, sizeof *h->blk);
    int rc = h->blk ? 0 : ARIA_HIP_ENOMEM;
    for (int b = 0; b < v->depth && !rc; b++) {
        h->blk[b] = aria_hip_dit_block_create(&v->blocks[b], v->ed, v->num_heads, 64, v->inner, ffn, v->ed,
                                              precision);
        if (!h->blk[b]) rc = ARIA_HIP_EINVAL;
    }
    const size_t C = (size_t)v->io_ch, E = (size_t)v->ed;
    if (!rc) rc = up_mat16(&h->pre, v->preprocess, C * C, h->st);
    if (!rc) rc = up_mat16(&h->post, v->postprocess, C * C, h->st);
    if (!rc) rc = up_mat16(&h->pin, v->project_in, E * C, h->st);
    if (!rc) rc = up_mat16(&h->pout, v->project_out, C * E, h->st);
    if (!rc && v->n_mem) rc = up_mat(&h->mem, v->memory_tokens, (size_t)v->n_mem * E);
    if (!rc && (!h->pin || !h->pout)) rc = ARIA_HIP_EINVAL;
    if (rc) {
        aria_cuda_dit_free(h);
        return NULL;
    }
    return h;
}

aria_cuda_dit *aria_cuda_dit_create(const aria_sa3_dit_view *v, aria_dtype precision) {
    return aria_hip_dit_create_ex(v, precision, ARIA_FFN_GLU);
}

/* warm hit (src/aria_cuda.cu:1268-1285): the same shapes and context embeddings as the
 * current request, no local cond and no steering -> keep the graph and K/V caches */
static int req_same(const aria_cuda_dit *h, const aria_sa3_dit_req_view *rv, int B) {
    if (!h->have_req || !h->saved_ced || h->B != B || h->local) return 0;
    for (int i = 0; i < B; i++) {
        if (!rv[i].cross_ed || rv[i].has_local || (rv[i].steer && rv[i].steer->n > 0)) return 0;
        if (rv[i].S != h->S || rv[i].T != h->T || rv[i].n_cond != h->Sc) return 0;
        if (memcmp(h->saved_ced + (size_t)i * h->Sc * h->ed, rv[i].cross_ed, (size_t)h->Sc * h->ed * sizeof(float)))
            return 0;
    }
    return 1;
}

static int req_setup(aria_cuda_dit *h, const aria_sa3_dit_req_view *rv, int B) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (!h || !rv || B <= 0) return ARIA_HIP_EINVAL;
    if (req_same(h, rv, B)) {
        h->cur_step = 0;
        h->steer = NULL;
        return 0;
    }
    const int T = rv[0].T, S = rv[0].S, Sc = rv[0].n_cond;
    for (int i = 0; i < B; i++)
        if (rv[i].T != T || rv[i].S != S || rv[i].n_cond != Sc || S != h->n_mem + T || T <= 0 || Sc <= 0 ||
            (!rv[i].cross_ed && (!rv[i].cross_k || !rv[i].cross_v)) || (h->rot && (!rv[i].rope_cos || !rv[i].rope_sin))) {
            aria_hip_set_error("aria_hip_dit_set_request: request views disagree or lack context K/V");
            return ARIA_HIP_EINVAL;
        }
    hipStreamSynchronize(h->st);
    req_free(h);
    h->B = B; h->T = T; h->S = S; h->Sc = Sc; h->steer = rv[0].steer; h->cur_step = 0;
    const int E = h->ed, C = h->io_ch, H = h->H, rh = h->rot / 2;
    size_t need = aria_hip_dit_block_workspace_bytes(h->blk[0], B, S, Sc);
    rc = dalloc(&h->ws, need, NULL);
    h->ws_bytes = need;
    const size_t nxc = (size_t)B * C * T;
    float **step_bufs[] = {&h->dx, &h->dv, &h->dxtc, &h->dtmp, &h->dout};
    for (size_t i = 0; i < sizeof step_bufs / sizeof *step_bufs && !rc; i++)
        rc = dalloc((void **)step_bufs[i], nxc * 4, NULL);
    if (!rc) rc = dalloc((void **)&h->dgcond, (size_t)B * 6 * E * 4, NULL);
    if (!rc) rc = dalloc((void **)&h->dseq, (size_t)B * S * E * 4, NULL);
    if (!rc && rh) {
        rc = upv(&h->cos_t, rv[0].rope_cos, (size_t)S * rh, NULL);
        if (!rc) rc = upv(&h->sin_t, rv[0].rope_sin, (size_t)S * rh, NULL);
    }
    h->ck = (uint16_t **)calloc((size_t)h->depth, sizeof *h->ck);
    h->cv = (uint16_t **)calloc((size_t)h->depth, sizeof *h->cv);
    if (!rc && (!h->ck || !h->cv)) rc = ARIA_HIP_ENOMEM;
    const size_t khv = (size_t)H * Sc * 64;   /* one sequence's K (or V) of one block */
    for (int b = 0; b < h->depth && !rc; b++) {
        rc = dalloc((void **)&h->ck[b], B * khv * 2, NULL);
        if (!rc) rc = dalloc((void **)&h->cv[b], B * khv * 2, NULL);
    }
    float *tmp = NULL;
    if (!rc && rv[0].cross_ed) {
        /* cross K/V of every block projected on the device from the B context embeddings
         * stacked [B*Sc, ed] (src/aria_cuda.cu:1324-1353) */
        rc = dalloc((void **)&tmp, (size_t)B * Sc * E * 4, NULL);
        for (int i = 0; i < B && !rc; i++) {
            hipError_t e = hipMemcpy(tmp + (size_t)i * Sc * E, rv[i].cross_ed, (size_t)Sc * E * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = FAIL(e, "hipMemcpy (cross_ed)");
        }
        for (int b = 0; b < h->depth && !rc; b++)
            rc = aria_hip_dit_block_cross_kv_dev(h->blk[b], tmp, B, Sc, h->ck[b], h->cv[b], h->ws, h->ws_bytes, h->st);
        if (!rc) {
            h->saved_ced = (float *)malloc((size_t)B * Sc * E * sizeof(float));
            for (int i = 0; i < B && h->saved_ced; i++)
                memcpy(h->saved_ced + (size_t)i * Sc * E, rv[i].cross_ed, (size_t)Sc * E * sizeof(float));
        }
    } else if (!rc) {
        /* legacy: host-projected fp32 K/V [H, Sc, 64] per block, converted to fp16 here */
        rc = dalloc((void **)&tmp, B * khv * 2 * 4, NULL);
        for (int b = 0; b < h->depth && !rc; b++) {
            for (int i = 0; i < B && !rc; i++) {
                hipError_t e = hipMemcpy(tmp + i * khv, rv[i].cross_k[b], khv * 4, hipMemcpyHostToDevice);
                if (e == hipSuccess)
                    e = hipMemcpy(tmp + (B + i) * khv, rv[i].cross_v[b], khv * 4, hipMemcpyHostToDevice);
                if (e != hipSuccess) rc = FAIL(e, "hipMemcpy (cross K/V)");
            }
            if (!rc) {
                hipError_t e = aria_k_f32_to_f16(h->ck[b], tmp, B * khv, h->st);
                if (e == hipSuccess) e = aria_k_f32_to_f16(h->cv[b], tmp + B * khv, B * khv, h->st);
                if (e == hipSuccess) e = hipStreamSynchronize(h->st);
                if (e != hipSuccess) rc = FAIL(e, "cross K/V upload");
            }
        }
    }
    /* inpaint local-additive cond per block, [S, ed] per sequence (zeros where absent) */
    int any_local = 0;
    for (int i = 0; i < B; i++) any_local |= rv[i].has_local && rv[i].local_emb;
    if (!rc && any_local) {
        h->local = (float **)calloc((size_t)h->depth, sizeof *h->local);
        if (!h->local) rc = ARIA_HIP_ENOMEM;
        for (int b = 0; b < h->depth && !rc; b++) {
            rc = dalloc((void **)&h->local[b], (size_t)B * S * E * 4, NULL);
            for (int i = 0; i < B && !rc; i++) {
                const float *src = rv[i].has_local && rv[i].local_emb ? rv[i].local_emb[b] : NULL;
                hipError_t e = src ? hipMemcpy(h->local[b] + (size_t)i * S * E, src, (size_t)S * E * 4,
                                               hipMemcpyHostToDevice)
                                   : hipMemset(h->local[b] + (size_t)i * S * E, 0, (size_t)S * E * 4);
                if (e != hipSuccess) rc = FAIL(e, "local cond upload");
            }
        }
    }
    if (!rc) {
        hipError_t e = hipStreamSynchronize(h->st);
        if (e != hipSuccess) rc = FAIL(e, "set_request");
    }
    dfree(tmp);
    if (!rc && h->steer && h->steer->n > 0) {
        static int warned;
        if (!warned++) fprintf(stderr, "[aria-hip] residual steering is not applied by this backend\n");
    }
    if (rc) { req_free(h); return rc; }
    h->have_req = 1;
    return 0;
}

void aria_cuda_dit_set_request(aria_cuda_dit *h, const aria_sa3_dit_req_view *rv) { req_setup(h, rv, 1); }
int aria_hip_dit_set_request_batch(aria_cuda_dit *h, const aria_sa3_dit_req_view *rv, int B) {
    return req_setup(h, rv, B);
}
void aria_cuda_dit_set_step(aria_cuda_dit *h, int step) {
    if (h) h->cur_step = step;
}

/* one velocity evaluation on the handle's buffers (src/aria_sa3_dit.c:734-777):
 * [C,T] -> [T,C]; xtc += preprocess(xtc); seq = [memory tokens | project_in(xtc)];
 * depth blocks; out = project_out(seq[n_mem:]); out += postprocess(out); -> [C,T] */
/* y [M, N] (+)= x [M, K] . W^T with fp32 x rounded to fp16 in the GEMM's staging and fp16 W,
 * fp32 accumulation and output: the reference's device step runs its four io projections so
 * (gemm_f16w, src/aria_cuda.cu:906-917). add: y += the product (the residual of the pre/post
 * convolutions, x == y), in the epilogue when the MFMA kernel takes the shape and one 128-wide
 * tile covers N (fp32 activations run 128 x 128 tiles), so each workgroup owns whole rows and has
 * read them before it writes them; otherwise through dtmp and k_add. */
static int io_gemm(aria_cuda_dit *h, float *y, const float *x, const uint16_t *W, int M, int K, int N, int add,
                   hipStream_t s) {
    const int mfma = K % 32 == 0 && N % 4 == 0;
    if (add && mfma && N <= 128) {
        aria_qgemm_epi e;
        memset(&e, 0, sizeof e);
        e.mode = ARIA_EPI_ADD;
        e.rows_per_batch = M;
        STEP(aria_k_qgemm_e(y, 0, x, 0, ARIA_WF16, W, NULL, NULL, M, K, N, 0, 0, &e, s), "k_qgemm (io projection)");
        return 0;
    }
    float *dst = add ? h->dtmp : y;
    STEP(aria_k_qgemm_e(dst, 0, x, 0, ARIA_WF16, W, NULL, NULL, M, K, N, 0, 0, NULL, s), "k_qgemm (io projection)");
    if (add) STEP(aria_k_add(y, y, dst, (size_t)M * N, s), "k_add (io projection)");
    return 0;
}

static int step_compute(aria_cuda_dit *h, hipStream_t s) {
    const int B = h->B, T = h->T, S = h->S, C = h->io_ch, E = h->ed, Mt = h->n_mem;
    int rc;
    STEP(aria_k_transpose(h->dxtc, h->dx, C, T, B, s), "k_transpose (x)");
    if (h->pre && (rc = io_gemm(h, h->dxtc, h->dxtc, h->pre, B * T, C, C, 1, s))) return rc;
    for (int b = 0; b < B && Mt; b++)
        STEP(hipMemcpyAsync(h->dseq + (size_t)b * S * E, h->mem, (size_t)Mt * E * 4, hipMemcpyDeviceToDevice, s),
             "memory tokens");
    /* project_in / project_out: one GEMM over both sequences when no memory tokens interleave */
    const int nb = Mt ? B : 1, rows = Mt ? T : B * T;
    for (int b = 0; b < nb; b++)
        if ((rc = io_gemm(h, h->dseq + ((size_t)b * S + Mt) * E, h->dxtc + (size_t)b * T * C, h->pin, rows, C, E, 0, s)))
            return rc;
    for (int b = 0; b < h->depth; b++) {
        rc = block_forward(h->blk[b], h->dseq, B, S, h->dgcond, h->ck[b], h->cv[b], h->Sc, h->cos_t, h->sin_t,
                           h->rot, h->local ? h->local[b] : NULL, h->ws, h->ws_bytes,
                           b + 1 < h->depth ? h->blk[b + 1] : NULL, s);
        if (rc) return rc;
    }
    for (int b = 0; b < nb; b++)
        if ((rc = io_gemm(h, h->dout + (size_t)b * T * C, h->dseq + ((size_t)b * S + Mt) * E, h->pout, rows, E, C, 0, s)))
            return rc;
    if (h->post && (rc = io_gemm(h, h->dout, h->dout, h->post, B * T, C, C, 1, s))) return rc;
    STEP(aria_k_transpose(h->dv, h->dout, T, C, B, s), "k_transpose (v)");
    return 0;
}

/* The step as one HIP graph, captured from the handle's stream the first time a step runs
 * on the current request's buffers and replayed from then on; set_request (for a new layout)
 * and an overlay load drop it. Capture is thread-local, so work that other threads enqueue
 * meanwhile is not pulled in. If capture or instantiation fails the handle runs the kernels
 * inline from then on, with the same results (the captured work never ran, so the step is
 * enqueued again inline). ARIA_GRAPH_FAIL set at create takes the failure branch after every
 * capture, which lets a test reach it. Returns 1 when a graph is ready. */
static int graph_ensure(aria_cuda_dit *h) {
    if (h->gstate != GRAPH_NONE) return h->gstate == GRAPH_LIVE;
    h->gstate = GRAPH_OFF;   /* unless everything below succeeds */
    if (hipStreamSynchronize(h->st) != hipSuccess ||
        hipStreamBeginCapture(h->st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        hipGetLastError();
        return 0;
    }
    const int rc = step_compute(h, h->st);
    hipGraph_t g = NULL;
    hipGraphExec_t x = NULL;
    const hipError_t ec = hipStreamEndCapture(h->st, &g);
    if (rc || ec != hipSuccess || !g || h->graph_fail || hipGraphInstantiate(&x, g, NULL, NULL, 0) != hipSuccess) {
        hipGetLastError();
        if (g) hipGraphDestroy(g);
        return 0;
    }
    h->graph = g;
    h->gexec = x;
    h->gstate = GRAPH_LIVE;
    return 1;
}

static int dit_run(aria_cuda_dit *h, hipStream_t s) {
    if (!graph_ensure(h)) return step_compute(h, s);
    const hipError_t e = hipGraphLaunch(h->gexec, s);
    return e == hipSuccess ? 0 : FAIL(e, "hipGraphLaunch");
}

int aria_hip_dit_graph_active(const aria_cuda_dit *h) { return h && h->gstate == GRAPH_LIVE; }

/* ---- the reference's packed DiT overlay (.aria) ----
 * File (aria_sa3_dit_quant_save, src/aria_sa3_dit.c:509-527): "ARIAQNT1", int32 {dt, depth, ed,
 * inner}, then per block six records in the order sa_to_qkv, sa_to_out, ca_to_q, ca_to_out,
 * ff_in_w, ff_out_w (src/aria_sa3_dit.c:512-516), each as aria_qweight_write lays it out
 * (src/aria_quant.c:439-449): int32 {dt, N, K}, u64 qbytes, the packed bytes, u64 nscale, the
 * fp32 scales. The records replace the blocks' projections as they are: no quantisation, on
 * the host or the device. */
static int ov_read(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n ? 0 : -1; }

static int ov_record(FILE *f, int N, int K, int glu_rows, int want_q8, dmat *out, size_t *acc) {
    int32_t hdr[3];
    uint64_t qb64 = 0, ns64 = 0;
    if (ov_read(f, hdr, sizeof hdr)) return -1;
    const int dt = hdr[0];
    if ((dt != ARIA_Q8 && dt != ARIA_Q4) || hdr[1] != N || hdr[2] != K || (want_q8 && dt != ARIA_Q8)) return -2;
    const size_t rb = dt == ARIA_Q8 ? (size_t)K : (size_t)(K + 1) / 2;        /* bytes per row */
    const size_t sr = dt == ARIA_Q8 ? 1 : (size_t)2 * ((K + 31) / 32);       /* scales per row */
    if (ov_read(f, &qb64, 8) || qb64 != rb * N) return -2;
    uint8_t *q = (uint8_t *)malloc(rb * N), *qi = NULL;
    float *sc = NULL, *si = NULL;
    int rc = q ? ov_read(f, q, rb * N) : -3;
    if (!rc && (ov_read(f, &ns64, 8) || ns64 != sr * N)) rc = -2;
    if (!rc) rc = (sc = (float *)malloc(sr * N * sizeof(float))) ? ov_read(f, sc, sr * N * sizeof(float)) : -3;
    if (!rc && glu_rows) {   /* GLU: rows (value_i, gate_i) interleaved, as block create packs them */
        const int inner = N / 2;
        qi = (uint8_t *)malloc(rb * N);
        si = (float *)malloc(sr * N * sizeof(float));
        if (!qi || !si) rc = -3;
        for (int i = 0; !rc && i < inner; i++) {
            memcpy(qi + (size_t)(2 * i) * rb, q + (size_t)i * rb, rb);
            memcpy(qi + (size_t)(2 * i + 1) * rb, q + (size_t)(inner + i) * rb, rb);
            memcpy(si + (size_t)(2 * i) * sr, sc + (size_t)i * sr, sr * sizeof(float));
            memcpy(si + (size_t)(2 * i + 1) * sr, sc + (size_t)(inner + i) * sr, sr * sizeof(float));
        }
    }
    memset(out, 0, sizeof *out);
    out->wtype = dt == ARIA_Q8 ? ARIA_WQ8 : ARIA_WQ4; out->N = N; out->K = K;
    if (!rc) rc = dalloc(&out->q, rb * N, acc) ? -3 : 0;
    if (!rc) rc = dalloc((void **)&out->scale, sr * N * sizeof(float), acc) ? -3 : 0;
    if (!rc && (hipMemcpy(out->q, qi ? qi : q, rb * N, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(out->scale, si ? si : sc, sr * N * sizeof(float), hipMemcpyHostToDevice) != hipSuccess))
        rc = -3;
    if (rc) dm_free(out);
    free(q); free(sc); free(qi); free(si);
    return rc;
}

int aria_hip_dit_load_overlay(aria_cuda_dit *h, const char *path) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (!h || !path) { aria_hip_set_error("aria_hip_dit_load_overlay: invalid argument"); return ARIA_HIP_EINVAL; }
    FILE *f = fopen(path, "rb");
    if (!f) { aria_hip_set_error("aria_hip_dit_load_overlay: cannot open %s", path); return ARIA_HIP_EINVAL; }
    char magic[8];
    int32_t hdr[4];
    if (ov_read(f, magic, 8) || memcmp(magic, "ARIAQNT1", 8) || ov_read(f, hdr, sizeof hdr) ||
        (hdr[0] != ARIA_Q8 && hdr[0] != ARIA_Q4) || hdr[1] != h->depth || hdr[2] != h->ed || hdr[3] != h->inner) {
        fclose(f);
        aria_hip_set_error("aria_hip_dit_load_overlay: not a packed overlay for this model (depth %d, ed %d, inner %d)",
                           h->depth, h->ed, h->inner);
        return ARIA_HIP_EINVAL;
    }
    const int ed = h->ed, inner = h->inner;
    /* read every record first, so a bad file leaves the model as it was */
    dmat *nw = (dmat *)calloc((size_t)h->depth * 6, sizeof(dmat));
    size_t *nbytes = (size_t *)calloc((size_t)h->depth, sizeof(size_t));   /* new bytes per block */
    rc = nw && nbytes ? 0 : -3;
    for (int i = 0; !rc && i < h->depth; i++) {
        aria_hip_dit_block *b = h->blk[i];
        const int glu = b->ffn == ARIA_FFN_GLU;
        const int shp[6][2] = {{3 * ed, ed}, {ed, ed}, {ed, ed}, {ed, ed}, {b->ffrows, ed}, {ed, inner}};
        for (int j = 0; !rc && j < 6; j++)
            rc = ov_record(f, shp[j][0], shp[j][1], j == 4 && glu, b->w8, &nw[i * 6 + j], &nbytes[i]);
    }
    fclose(f);
    if (rc) {
        if (nw) for (int k = 0; k < h->depth * 6; k++) dm_free(&nw[k]);
        free(nw);
        free(nbytes);
        aria_hip_set_error("aria_hip_dit_load_overlay: %s", rc == -3 ? "out of memory"
                           : rc == -2 ? "record type or shape does not match the model (W8A8 blocks need Q8)"
                                      : "truncated file");
        return rc == -3 ? ARIA_HIP_ENOMEM : ARIA_HIP_EINVAL;
    }
    /* in-flight steps use the old weights; a captured step holds their addresses */
    hipStreamSynchronize(h->st);
    graph_drop(h);
    for (int i = 0; i < h->depth; i++) {
        aria_hip_dit_block *b = h->blk[i];
        dmat *dst[6] = {&b->sa_qkv, &b->sa_out, &b->ca_q, &b->ca_out, &b->ff_in, &b->ff_out};
        for (int j = 0; j < 6; j++) {
            b->bytes -= dm_bytes(dst[j]);
            dm_free(dst[j]);
            *dst[j] = nw[i * 6 + j];
        }
        b->bytes += nbytes[i];
        b->prec = (aria_dtype)hdr[0];
    }
    free(nw);
    free(nbytes);
    return 0;
}

int aria_hip_dit_device_buffers(aria_cuda_dit *h, float **dx, float **dv, float **dgcond) {
    if (!h || !h->have_req) return ARIA_HIP_EINVAL;
    if (dx) *dx = h->dx;
    if (dv) *dv = h->dv;
    if (dgcond) *dgcond = h->dgcond;
    return 0;
}

int aria_hip_dit_run(aria_cuda_dit *h, void *stream) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (!h || !h->have_req) { aria_hip_set_error("aria_hip_dit_run: no request set"); return ARIA_HIP_EINVAL; }
    return dit_run(h, stream ? (hipStream_t)stream : h->st);
}

int aria_hip_dit_step_batch(aria_cuda_dit *h, float *v, const float *x, const float *gcond) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (!h || !h->have_req || !v || !x || !gcond) {
        aria_hip_set_error("aria_hip_dit_step_batch: no request set or NULL buffer");
        return ARIA_HIP_EINVAL;
    }
    const size_t n = (size_t)h->B * h->io_ch * h->T, ng = (size_t)h->B * 6 * h->ed;
    STEP(hipMemcpyAsync(h->dx, x, n * 4, hipMemcpyHostToDevice, h->st), "hipMemcpyAsync (x)");
    STEP(hipMemcpyAsync(h->dgcond, gcond, ng * 4, hipMemcpyHostToDevice, h->st), "hipMemcpyAsync (gcond)");
    rc = dit_run(h, h->st);
    if (rc) return rc;
    STEP(hipMemcpyAsync(v, h->dv, n * 4, hipMemcpyDeviceToHost, h->st), "hipMemcpyAsync (v)");
    STEP(hipStreamSynchronize(h->st), "hipStreamSynchronize");
    return 0;
}

void aria_cuda_dit_step(aria_cuda_dit *h, float *v_CT, const float *x_CT, const float *gcond) {
    if (h && h->B != 1) { aria_hip_set_error("aria_cuda_dit_step: request has %d sequences", h->B); return; }
    aria_hip_dit_step_batch(h, v_CT, x_CT, gcond);
}

/* Sampler staging, reserved before the first step runs: the gcond table of every step on the
 * device, NZ_SLOTS noise slots in pinned host memory and on the device, an upload stream and
 * the slot events. -1 leaves the handle as it was for the step path. */
static int sample_stage(aria_cuda_dit *h, int steps, size_t n, size_t ng) {
    if (sbuf_reserve(&h->gc_tab, (size_t)(steps > 0 ? steps : 1) * ng * sizeof(float), 0) ||
        sbuf_reserve(&h->nz_host, (size_t)NZ_SLOTS * n * sizeof(float), 1) ||
        sbuf_reserve(&h->nz_dev, (size_t)NZ_SLOTS * n * sizeof(float), 0))
        return -1;
    if (!h->up && hipStreamCreateWithFlags(&h->up, hipStreamNonBlocking) != hipSuccess) {
        hipGetLastError();
        h->up = NULL;
        return -1;
    }
    if (!h->have_events) {
        int ok = hipEventCreateWithFlags(&h->ev_step, hipEventDisableTiming) == hipSuccess;
        for (int i = 0; i < NZ_SLOTS && ok; i++)
            ok = hipEventCreateWithFlags(&h->ev_up[i], hipEventDisableTiming) == hipSuccess &&
                 hipEventCreateWithFlags(&h->ev_used[i], hipEventDisableTiming) == hipSuccess;
        if (!ok) { hipGetLastError(); return -1; }   /* (a partial set is not reused) */
        h->have_events = 1;
    }
    return 0;
}

/* The pingpong sampler with x resident in HBM (contract: src/aria_sa3_dit.h:163-171; the host
 * loop it reproduces bit for bit is src/aria_sampler.c:203-229).
 * Per step i on the handle's stream: gcond row i is copied from the device table (uploaded
 * once, before the first step), the velocity step runs (graph replay), then the update
 * x = (1 - tn)(x - tc v) + tn noise_i. The host draws noise_i while step i runs, into slot
 * i % NZ_SLOTS; the slot goes to the device on the upload stream, overlapping the step, and
 * the update waits for that upload. A slot is refilled only after the update that read its
 * previous contents (ev_used), which also orders the refill after the slot's last upload.
 * noise is called exactly once per step, in step order. */
int aria_cuda_dit_sample(aria_cuda_dit *h, float *x_CT, const float *sched, int steps, const float *gcond_all,
                         void (*noise)(float *, int, void *), void *noise_user, void (*progress)(int, int, void *),
                         void *progress_user) {
    if (aria_hip_ensure() || !h || !h->have_req || !x_CT || !sched || !gcond_all || !noise || steps < 0) return -1;
    const size_t n = (size_t)h->B * h->io_ch * h->T, ng = (size_t)h->B * 6 * h->ed;
    if (sample_stage(h, steps, n, ng)) return -1;
    hipStream_t cs = h->st;
    float *gtab = (float *)h->gc_tab.p, *hslot = (float *)h->nz_host.p, *dslot = (float *)h->nz_dev.p;
    int ok = hipMemcpyAsync(h->dx, x_CT, n * 4, hipMemcpyHostToDevice, cs) == hipSuccess &&
             (steps == 0 || hipMemcpyAsync(gtab, gcond_all, (size_t)steps * ng * 4, hipMemcpyHostToDevice, cs) ==
                                hipSuccess);
    for (int i = 0; i < steps && ok; i++) {
        const int k = i % NZ_SLOTS;
        float *hk = hslot + (size_t)k * n, *dk = dslot + (size_t)k * n;
        h->cur_step = i;
        ok = hipMemcpyAsync(h->dgcond, gtab + (size_t)i * ng, ng * 4, hipMemcpyDeviceToDevice, cs) == hipSuccess &&
             dit_run(h, cs) == 0;
        if (!ok) break;
        if (i >= NZ_SLOTS && hipEventSynchronize(h->ev_used[k]) != hipSuccess) { ok = 0; break; }
        noise(hk, (int)n, noise_user);
        ok = hipMemcpyAsync(dk, hk, n * 4, hipMemcpyHostToDevice, h->up) == hipSuccess &&
             hipEventRecord(h->ev_up[k], h->up) == hipSuccess && hipStreamWaitEvent(cs, h->ev_up[k], 0) == hipSuccess &&
             aria_k_pingpong(h->dx, h->dv, dk, sched[i], sched[i + 1], n, cs) == hipSuccess &&
             hipEventRecord(h->ev_used[k], cs) == hipSuccess;
        if (ok && progress) {
            ok = hipEventRecord(h->ev_step, cs) == hipSuccess && hipEventSynchronize(h->ev_step) == hipSuccess;
            if (ok) progress(i + 1, steps, progress_user);
        }
    }
    if (ok) ok = hipMemcpyAsync(x_CT, h->dx, n * 4, hipMemcpyDeviceToHost, cs) == hipSuccess;
    if (hipStreamSynchronize(cs) != hipSuccess) ok = 0;
    if (hipStreamSynchronize(h->up) != hipSuccess) ok = 0;
    if (!ok) hipGetLastError();
    return ok ? 0 : -1;
}

/* ------------------------------------------------------------------------- */
/* the medium device decoder is not served: NULL keeps the caller on its CPU decoder  */
/* ------------------------------------------------------------------------- */

aria_cuda_dec_medium *aria_cuda_dec_medium_create(const aria_sa3_dec_medium_view *v) {
    (void)v;
    aria_hip_set_error("aria_cuda_dec_medium_create: the device decoder is not part of this backend");
    return NULL;
}
void aria_cuda_dec_medium_free(aria_cuda_dec_medium *h) { (void)h; }
void aria_cuda_dec_medium_forward(aria_cuda_dec_medium *h, float *audio, const float *latent, int T) {
    (void)h; (void)audio; (void)latent; (void)T;
    aria_hip_set_error("aria_cuda_dec_medium_forward: no device decoder");
}
