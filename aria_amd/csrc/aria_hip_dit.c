/*
 * aria_hip_dit.c - the DiT block on the MI355X backend (include/aria_dit.h), C11 host code.
 *
 * A block's weights live in HBM in the reference's packed layouts (Q8 / Q4 per the
 * mixed-precision recipe, fp16 otherwise). The forward pass is the order of
 * dit_block_core (src/aria_sa3_dit.c:141-312), each step one gfx950 kernel:
 *
 *   mod      = to_scale_shift_gate + gcond, chunk-major            k_mod_chunks
 *   self:    h16 = rmsnorm(x, pre_norm)*(1+scale)+shift  (fp16)    k_rownorm (fused adaLN)
 *            qkv = h16 . sa_to_qkv^T                                k_qgemm (Q8)
 *            q,k,v heads, q/k rmsnorm + RoPE (fp16, head-major)     k_qkv_prep
 *            att = softmax(q k^T / 8) v (fp16, heads merged)        k_flash_attn
 *            x  += (att . sa_to_out^T) * sigmoid(1 - gate)          k_qgemm, k_gate_residual
 *   cross:   h16 = rmsnorm(x, cross_norm); q = h16 . ca_to_q^T; q-norm; attention over the
 *            request's cached K/V; x += att . ca_to_out^T           (same kernels, k_add)
 *   ffn:     h16 = rmsnorm(x, ff_norm)*(1+scale)+shift
 *            GLU:  proj = h16 . ff_in^T + b; g16 = silu(gate)*value  k_qgemm (Q4), k_glu_combine
 *            GELU: g16 = gelu(h16 . ff_in^T + b)                    k_qgemm with GELU epilogue
 *            x  += (g16 . ff_out^T + b) * sigmoid(1 - gate)         k_qgemm (Q4), k_gate_residual
 *
 * Nothing is allocated in the forward pass: every intermediate lives in the caller's
 * workspace (layout in ws_layout below).
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include "aria_dit.h"
#include "aria_hip.h"
#include "aria_hip_internal.h"
#include "aria_hip_kernels.h"

#include <stdlib.h>
#include <string.h>

typedef struct {
    int wtype, N, K;
    void *q;       /* int8 / u8 packed / fp16 */
    float *scale;  /* Q8 [N], Q4 [N, 2*ceil(K/32)], NULL for fp16 */
} dmat;

struct aria_hip_dit_block {
    int dim, H, hd, inner, ffn, dim_ctx, ffrows;
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
    if (!rc) rc = upv(&b->ff_in_b, w->ff_in_b, (size_t)b->ffrows, acc);
    if (!rc) rc = upv(&b->ff_out_b, w->ff_out_b, dim, acc);
    if (!rc) rc = upv(&b->tssg, w->to_scale_shift_gate, (size_t)6 * dim, acc);
    if (!rc && !b->tssg) { aria_hip_set_error("to_scale_shift_gate missing"); rc = ARIA_HIP_EINVAL; }
    if (!rc) rc = pack(&b->sa_qkv, w->sa_to_qkv, 3 * dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->sa_out, w->sa_to_out, dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->ca_q, w->ca_to_q, dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->ca_out, w->ca_to_out, dim, dim, attn_t, s, acc);
    if (!rc) rc = pack(&b->ca_kv, w->ca_to_kv, 2 * dim, dim_ctx, ARIA_WF16, s, acc);
    if (!rc) rc = pack(&b->ff_in, w->ff_in_w, b->ffrows, dim, ffn_t, s, acc);
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
    float *big, *o, *mod;
} wsl;

#define WS_ALIGN 256
static size_t al(size_t n) { return (n + WS_ALIGN - 1) & ~(size_t)(WS_ALIGN - 1); }

static size_t ws_layout(const aria_hip_dit_block *b, int B, int S, int Sc, char *base, wsl *w) {
    const size_t M = (size_t)B * S, d = (size_t)b->dim;
    size_t big = M * 3 * d * 4;
    if (b->ffn == ARIA_FFN_GLU && M * (size_t)b->ffrows * 4 > big) big = M * (size_t)b->ffrows * 4;
    if ((size_t)B * Sc * 2 * d * 4 > big) big = (size_t)B * Sc * 2 * d * 4;
    const size_t sz[9] = {M * d * 2, big, M * d * 2, M * d * 2, M * d * 2, M * d * 2, M * d * 4,
                          M * (size_t)b->inner * 2, (size_t)6 * B * d * 4};
    size_t off = 0, o[9];
    for (int i = 0; i < 9; i++) { o[i] = off; off += al(sz[i]); }
    if (base && w) {
        w->h16 = (uint16_t *)(base + o[0]);
        w->big = (float *)(base + o[1]);
        w->q16 = (uint16_t *)(base + o[2]);
        w->k16 = (uint16_t *)(base + o[3]);
        w->v16 = (uint16_t *)(base + o[4]);
        w->att16 = (uint16_t *)(base + o[5]);
        w->o = (float *)(base + o[6]);
        w->ff16 = (uint16_t *)(base + o[7]);
        w->mod = (float *)(base + o[8]);
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

int aria_hip_dit_block_forward_dev(aria_hip_dit_block *b, float *dx, int B, int S, const float *dgcond,
                                   const uint16_t *dk, const uint16_t *dv, int Sc, const float *dcos,
                                   const float *dsin, int rot, void *dws, size_t ws_bytes, void *stream) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
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
    hipStream_t s = aria_hip_stream(stream);
    const int d = b->dim, H = b->H, M = B * S;
    const size_t Bd = (size_t)B * d;
    const float eps_norm = 1e-5f, eps_qk = 1e-6f;

    STEP(aria_k_mod_chunks(w.mod, b->tssg, dgcond, B, d, s), "k_mod_chunks");
    const float *scale_self = w.mod, *shift_self = w.mod + Bd, *gate_self = w.mod + 2 * Bd;
    const float *scale_ff = w.mod + 3 * Bd, *shift_ff = w.mod + 4 * Bd, *gate_ff = w.mod + 5 * Bd;

    /* ---- self-attention ---- */
    STEP(aria_k_rownorm(w.h16, 1, dx, b->pre_norm, NULL, scale_self, shift_self, S, 0, 0, ARIA_NORM_RMS, M, d,
                        eps_norm, s), "k_rownorm (pre_norm + adaLN)");
    STEP(gemm(&b->sa_qkv, w.big, 0, w.h16, NULL, M, 0, s), "k_qgemm (sa_to_qkv)");
    {
        const int kind[3] = {0, 1, 2};
        uint16_t *dst[3] = {w.q16, w.k16, w.v16};
        const float *nw[3] = {b->sa_q_norm, b->sa_k_norm, NULL};
        STEP(aria_k_qkv_prep(w.big, 3 * d, B, S, H, 3, kind, dst, nw, dcos, dsin, rot, eps_qk, s), "k_qkv_prep");
    }
    STEP(aria_k_flash_attn(w.q16, w.k16, w.v16, w.att16, 1, B * H, H, S, S, s), "k_flash_attn (self)");
    STEP(gemm(&b->sa_out, w.o, 0, w.att16, NULL, M, 0, s), "k_qgemm (sa_to_out)");
    STEP(aria_k_gate_residual(dx, dx, w.o, gate_self, NULL, M, d, S, s), "k_gate_residual (self)");

    /* ---- cross-attention (no RoPE, no gate) ---- */
    STEP(aria_k_rownorm(w.h16, 1, dx, b->cross_norm, NULL, NULL, NULL, 0, 0, 0, ARIA_NORM_RMS, M, d, eps_norm, s),
         "k_rownorm (cross_norm)");
    STEP(gemm(&b->ca_q, w.big, 0, w.h16, NULL, M, 0, s), "k_qgemm (ca_to_q)");
    {
        const int kind[1] = {0};
        uint16_t *dst[1] = {w.q16};
        const float *nw[1] = {b->ca_q_norm};
        STEP(aria_k_qkv_prep(w.big, d, B, S, H, 1, kind, dst, nw, NULL, NULL, 0, eps_qk, s), "k_qkv_prep (cross q)");
    }
    STEP(aria_k_flash_attn(w.q16, dk, dv, w.att16, 1, B * H, H, S, Sc, s), "k_flash_attn (cross)");
    STEP(gemm(&b->ca_out, w.o, 0, w.att16, NULL, M, 0, s), "k_qgemm (ca_to_out)");
    STEP(aria_k_add(dx, dx, w.o, (size_t)M * d, s), "k_add (cross residual)");

    /* ---- feed-forward ---- */
    STEP(aria_k_rownorm(w.h16, 1, dx, b->ff_norm, NULL, scale_ff, shift_ff, S, 0, 0, ARIA_NORM_RMS, M, d, eps_norm, s),
         "k_rownorm (ff_norm + adaLN)");
    if (b->ffn == ARIA_FFN_GLU) {
        STEP(gemm(&b->ff_in, w.big, 0, w.h16, b->ff_in_b, M, 0, s), "k_qgemm (ff_in)");
        STEP(aria_k_glu_combine(w.ff16, 1, w.big, NULL, M, b->inner, s), "k_glu_combine");
    } else {
        STEP(gemm(&b->ff_in, w.ff16, 1, w.h16, b->ff_in_b, M, 1, s), "k_qgemm (ff_in + GELU)");
    }
    STEP(gemm(&b->ff_out, w.o, 0, w.ff16, NULL, M, 0, s), "k_qgemm (ff_out)");
    STEP(aria_k_gate_residual(dx, dx, w.o, gate_ff, b->ff_out_b, M, d, S, s), "k_gate_residual (ff)");
    return 0;
}
