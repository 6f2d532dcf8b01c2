/*
 * aria_hip_dec.c - the small-music taae_v2 decoder on the MI355X backend (C11 host code):
 * aria_cuda_dec_create / _free / _forward (src/aria_sa3_dec.h:98-109), the device form of
 * aria_sa3_dec_forward (src/aria_sa3_dec.c:47-128) behind the reference's interface.
 *
 * create uploads the view once: the four block GEMM matrices, the 256 -> 768 projection as
 * fp16 (the reference's device decoder stores them so, src/aria_cuda.cu:1832-1880); the
 * ff_in rows and bias interleaved (value_i, gate_i) for the GEMM's GLU epilogue; the
 * folded mapping convolution [512, 768 * 3] as fp32, whose row layout already is the
 * im2col operand's; norms, biases, new tokens and the 34-position RoPE tables as fp32.
 *
 * forward, latent [256, T] -> audio [2, T * 4096], one stream, every pass over all chunks:
 *   xt16 = half(latent * std)^T                        k_dec_in
 *   x    = xt16 . proj^T + b                           k_qgemm (fp16 weights)
 *   seq  = groups of 17: x[t], 16 new tokens           k_dec_expand
 *   blocks 0-2 on the 34-row chunks of seq, then the 17-row halos copied in and blocks 3-5
 *   on the chunks of the haloed sequence (the midpoint shift, src/aria_taae.c:169-205);
 *   seq sits 17 rows into a buffer of L + 34 rows, so the shifted pass runs in place and
 *   nothing is copied back. Per block (src/aria_taae.c:93-162):
 *     h16    = dyt(seq, pre_norm)                      k_dec_dyt (block 0; later blocks get it
 *                                                      from the previous ff_out's epilogue)
 *     qkv    = h16 . to_qkv^T, q/k DyT + RoPE          k_qgemm (DYT_ROPE epilogue)
 *     m16    = diff-attention per (chunk, head)        k_dec_attn
 *     seq   += m16 . to_out^T; h16 = dyt(seq, ff_norm) k_qgemm (ADD_DYT epilogue)
 *     g16    = silu(gate) * value of h16 . ff_in^T + b k_qgemm (GLU epilogue)
 *     seq   += g16 . ff_out^T + b; h16 = dyt(seq, next pre_norm)  k_qgemm (ADD_DYT / ADD)
 *   xc   = im2col of the last 16 of each group          k_dec_im2col (first T * 16 rows)
 *   audio = unpatch(xc . mapping^T + b)                 k_dec_map (fp32 MFMA)
 * The workspace is kept on the handle and grown when a longer latent arrives.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include "aria_dit.h"
#include "aria_hip.h"
#include "aria_hip_internal.h"
#include "aria_hip_kernels.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define DD 768       /* transformer dim */
#define DS 34        /* chunk (two groups of 17) */
#define DHALF 17
#define DQKV 3840
#define DINNER 2304
#define DOUT 512
#define DRH 16       /* rotated dims / 2 */
#define DMAXT (1 << 20)

typedef struct {
    float pre_alpha, qn_alpha, kn_alpha, ff_alpha;
    float *pre_g, *pre_b, *qn_g, *qn_b, *kn_g, *kn_b, *ff_g, *ff_b, *ff_in_b, *ff_out_b;
    uint16_t *to_qkv, *to_out, *ff_in, *ff_out;
} dec_blk;

struct aria_cuda_dec {
    float running_std;
    uint16_t *proj_w;
    float *proj_b, *new_tokens, *mapping_w, *mapping_b, *rcos, *rsin;
    dec_blk blk[6];
    hipStream_t st;
    void *ws;
    size_t ws_bytes;
    int ws_T;   /* the longest latent the workspace holds */
    void *pin;  /* pinned host staging of the host entry's copies (grown on demand) */
    size_t pin_bytes;
};

static int d_alloc(void **p, size_t bytes) {
    *p = NULL;
    hipError_t e = hipMalloc(p, bytes ? bytes : 4);
    return e == hipSuccess ? 0 : aria_hip_fail(e, "hipMalloc (decoder)");
}

static int up_f32(float **d, const float *h, size_t n) {
    *d = NULL;
    if (!h) { aria_hip_set_error("aria_cuda_dec_create: a decoder weight is missing from the view"); return ARIA_HIP_EINVAL; }
    int rc = d_alloc((void **)d, n * 4);
    if (rc) return rc;
    hipError_t e = hipMemcpy(*d, h, n * 4, hipMemcpyHostToDevice);
    return e == hipSuccess ? 0 : aria_hip_fail(e, "hipMemcpy (decoder vector)");
}

/* fp32 host [n] -> fp16 device, converted on the device (RTNE) */
static int up_f16(uint16_t **d, const float *h, size_t n, hipStream_t s) {
    *d = NULL;
    float *tmp = NULL;
    int rc = up_f32(&tmp, h, n);
    if (!rc) rc = d_alloc((void **)d, n * 2);
    if (!rc) {
        hipError_t e = aria_k_f32_to_f16(*d, tmp, n, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = aria_hip_fail(e, "decoder weight conversion");
    }
    if (tmp) hipFree(tmp);
    return rc;
}

static void f_free(void *p) {
    if (p) hipFree(p);
}

void aria_cuda_dec_free(aria_cuda_dec *h) {
    if (!h) return;
    if (h->st) hipStreamSynchronize(h->st);
    if (h->pin) hipHostFree(h->pin);
    f_free(h->ws);
    f_free(h->proj_w); f_free(h->proj_b); f_free(h->new_tokens); f_free(h->mapping_w); f_free(h->mapping_b);
    f_free(h->rcos); f_free(h->rsin);
    for (int i = 0; i < 6; i++) {
        dec_blk *b = &h->blk[i];
        void *p[] = {b->pre_g, b->pre_b, b->qn_g, b->qn_b, b->kn_g, b->kn_b, b->ff_g, b->ff_b, b->ff_in_b,
                     b->ff_out_b, b->to_qkv, b->to_out, b->ff_in, b->ff_out};
        for (size_t j = 0; j < sizeof p / sizeof *p; j++) f_free(p[j]);
    }
    if (h->st) hipStreamDestroy(h->st);
    free(h);
}

static int blk_create(dec_blk *d, const aria_taae_block_view *v, hipStream_t s) {
    d->pre_alpha = v->pre_alpha; d->qn_alpha = v->qn_alpha; d->kn_alpha = v->kn_alpha; d->ff_alpha = v->ff_alpha;
    int rc = up_f32(&d->pre_g, v->pre_gamma, DD);
    if (!rc) rc = up_f32(&d->pre_b, v->pre_beta, DD);
    if (!rc) rc = up_f32(&d->qn_g, v->qn_gamma, 64);
    if (!rc) rc = up_f32(&d->qn_b, v->qn_beta, 64);
    if (!rc) rc = up_f32(&d->kn_g, v->kn_gamma, 64);
    if (!rc) rc = up_f32(&d->kn_b, v->kn_beta, 64);
    if (!rc) rc = up_f32(&d->ff_g, v->ff_gamma, DD);
    if (!rc) rc = up_f32(&d->ff_b, v->ff_beta, DD);
    if (!rc) rc = up_f32(&d->ff_out_b, v->ff_out_b, DD);
    if (!rc) rc = up_f16(&d->to_qkv, v->to_qkv, (size_t)DQKV * DD, s);
    if (!rc) rc = up_f16(&d->to_out, v->to_out, (size_t)DD * DD, s);
    if (!rc) rc = up_f16(&d->ff_out, v->ff_out_w, (size_t)DD * DINNER, s);
    if (rc) return rc;
    if (!v->ff_in_w || !v->ff_in_b) {
        aria_hip_set_error("aria_cuda_dec_create: ff_in weight or bias missing from the view");
        return ARIA_HIP_EINVAL;
    }
    /* GLU: row 2i = value row i, row 2i + 1 = gate row inner + i (bias likewise) */
    float *w = (float *)malloc((size_t)2 * DINNER * DD * sizeof(float));
    float *b = (float *)malloc((size_t)2 * DINNER * sizeof(float));
    if (!w || !b) rc = ARIA_HIP_ENOMEM;
    for (int i = 0; i < DINNER && !rc; i++) {
        memcpy(w + (size_t)(2 * i) * DD, v->ff_in_w + (size_t)i * DD, DD * sizeof(float));
        memcpy(w + (size_t)(2 * i + 1) * DD, v->ff_in_w + (size_t)(DINNER + i) * DD, DD * sizeof(float));
        b[2 * i] = v->ff_in_b[i];
        b[2 * i + 1] = v->ff_in_b[DINNER + i];
    }
    if (!rc) rc = up_f16(&d->ff_in, w, (size_t)2 * DINNER * DD, s);
    if (!rc) rc = up_f32(&d->ff_in_b, b, (size_t)2 * DINNER);
    free(w);
    free(b);
    return rc;
}

aria_cuda_dec *aria_cuda_dec_create(const aria_sa3_dec_view *v) {
    if (aria_hip_ensure() || !v) {
        if (!v) aria_hip_set_error("aria_cuda_dec_create: NULL view");
        return NULL;
    }
    size_t fr = 0, tot = 0;
    hipMemGetInfo(&fr, &tot);
    /* weights: 6 blocks of (3840 + 768 + 4608 + 2304) x 768 fp16, the fp32 mapping, headroom */
    const size_t need = (size_t)6 * 11520 * DD * 2 + (size_t)DOUT * 3 * DD * 4 + ((size_t)256 << 20);
    if (need > fr) {
        aria_hip_set_error("aria_cuda_dec_create: the decoder does not fit in device memory");
        return NULL;
    }
    aria_cuda_dec *h = (aria_cuda_dec *)calloc(1, sizeof *h);
    if (!h) return NULL;
    if (hipStreamCreateWithFlags(&h->st, hipStreamNonBlocking) != hipSuccess) {
        aria_hip_set_error("aria_cuda_dec_create: hipStreamCreate failed");
        free(h);
        return NULL;
    }
    h->running_std = v->running_std;
    int rc = up_f16(&h->proj_w, v->proj_w, (size_t)DD * 256, h->st);
    if (!rc) rc = up_f32(&h->proj_b, v->proj_b, DD);
    if (!rc) rc = up_f32(&h->new_tokens, v->new_tokens, DD);
    if (!rc) rc = up_f32(&h->mapping_w, v->mapping_w, (size_t)DOUT * 3 * DD);
    if (!rc) rc = up_f32(&h->mapping_b, v->mapping_b, DOUT);
    for (int i = 0; i < 6 && !rc; i++) rc = blk_create(&h->blk[i], &v->blocks[i], h->st);
    if (!rc) {
        /* RoPE tables for the 34 chunk positions, base 10000, 32 rotated dims, as the
         * reference computes them (src/aria_cpu.c:778-788): double angle, rounded to float */
        float cs[DS * DRH], sn[DS * DRH];
        for (int i = 0; i < DRH; i++) {
            const double inv = 1.0 / pow(10000.0, (double)(2 * i) / 32.0);
            for (int p = 0; p < DS; p++) {
                cs[p * DRH + i] = (float)cos((double)p * inv);
                sn[p * DRH + i] = (float)sin((double)p * inv);
            }
        }
        rc = up_f32(&h->rcos, cs, DS * DRH);
        if (!rc) rc = up_f32(&h->rsin, sn, DS * DRH);
    }
    if (rc) {
        aria_cuda_dec_free(h);
        return NULL;
    }
    return h;
}

/* ---- workspace for a latent of T frames (all offsets 256-byte aligned) ----
 *   lat   [256, T] f32        xt16 [T, 256] f16       x [T, 768] f32
 *   seq   [L + 34, 768] f32   (the sequence at row 17; halos at rows 0-16, L + 17 ..)
 *   h16   [L + 34, 768] f16   m16 [L + 34, 768] f16
 *   qkv   [L + 34, 3840] f32  (after the blocks: xc [T * 16, 2304] f32)
 *   g16   [L + 34, 2304] f16
 *   audio [2, T * 4096] f32
 * L = 17 * Tp, Tp = T rounded up to even. */
typedef struct {
    float *lat, *x, *seq, *qkv, *xc, *audio;
    uint16_t *xt16, *h16, *m16, *g16;
} dec_ws;

static size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

static size_t ws_layout(int T, dec_ws *w, char *base) {
    const size_t Tp = (size_t)(T + (T & 1)), R = 17 * Tp + DS, Lt = (size_t)T * 16;
    size_t off = 0;
#define CARVE(field, type, bytes) do { if (w) w->field = (type *)(base + off); off += al(bytes); } while (0)
    CARVE(lat, float, (size_t)256 * T * 4);
    CARVE(xt16, uint16_t, (size_t)T * 256 * 2);
    CARVE(x, float, (size_t)T * DD * 4);
    CARVE(seq, float, R * DD * 4);
    CARVE(h16, uint16_t, R * DD * 2);
    CARVE(m16, uint16_t, R * DD * 2);
    CARVE(qkv, float, R * DQKV * 4);
    CARVE(g16, uint16_t, R * DINNER * 2);
    CARVE(audio, float, Lt * 512 * 4);
#undef CARVE
    if (w) {
        w->xc = w->qkv;                   /* Lt * 2304 * 4 <= R * 3840 * 4 */
    }
    return off;
}

#define STEP(call, what) do { hipError_t e_ = (call); if (e_ != hipSuccess) return aria_hip_fail(e_, what); } while (0)

static int gemm(void *y, int y_f16, const uint16_t *x, const uint16_t *w, const float *b, int M, int K, int N,
                int mode, hipStream_t s) {
    aria_qgemm_epi e;
    memset(&e, 0, sizeof e);
    e.mode = mode;
    e.rows_per_batch = M;
    STEP(aria_k_qgemm_e(y, y_f16, x, 1, ARIA_WF16, w, NULL, b, M, K, N, 0, 0, &e, s), "k_qgemm (decoder)");
    return 0;
}

/* x += m16 . W^T (+ b), and h16 = half(dyt(x, alpha, g, be)) of the new x, in the GEMM's
 * epilogue (the next DynamicTanh norm's operand; tanh as tanh_fast) */
static int gemm_add_dyt(float *x, const uint16_t *m16, const uint16_t *w, const float *b, int M, int K, uint16_t *h16,
                        float alpha, const float *g, const float *be, hipStream_t s) {
    aria_qgemm_epi e;
    memset(&e, 0, sizeof e);
    e.mode = ARIA_EPI_ADD_DYT;
    e.rows_per_batch = M;
    e.dst[0] = h16;
    e.w[0] = g;
    e.w[1] = be;
    e.eps = alpha;
    STEP(aria_k_qgemm_e(x, 0, m16, 1, ARIA_WF16, w, NULL, b, M, K, DD, 0, 0, &e, s), "k_qgemm (decoder + DyT)");
    return 0;
}

/* qkv = h16 . to_qkv^T with the q / k sections DynamicTanh-normed (qn, kn) and rotated at
 * their chunk position (rcos / rsin [34, 16]) in the GEMM's epilogue, the order of
 * src/aria_taae.c:120-127 */
static int gemm_qkv(const aria_cuda_dec *h, const dec_blk *b, float *qkv, const uint16_t *h16, int M,
                    hipStream_t s) {
    aria_qgemm_epi e;
    memset(&e, 0, sizeof e);
    e.mode = ARIA_EPI_DYT_ROPE;
    e.rows_per_batch = DS;
    e.heads = DD / 64;
    e.w[0] = b->qn_g; e.w[1] = b->qn_b; e.w[2] = b->kn_g; e.w[3] = b->kn_b;
    e.eps = b->qn_alpha;
    e.eps2 = b->kn_alpha;
    e.cos_t = h->rcos;
    e.sin_t = h->rsin;
    e.rot = 2 * DRH;
    STEP(aria_k_qgemm_e(qkv, 0, h16, 1, ARIA_WF16, b->to_qkv, NULL, NULL, M, DD, DQKV, 0, 0, &e, s),
         "k_qgemm (decoder to_qkv + q/k DyT + RoPE)");
    return 0;
}

/* one block on the nch chunks of 34 rows at x, in place (src/aria_taae.c:93-162). h16 (rows
 * aligned with x) holds dyt(x, pre_norm) on entry; the to_out GEMM's epilogue writes
 * dyt(x, ff_norm) into it, and ff_out's writes the next block's pre_norm DyT when `next` is given
 * (plain residual add otherwise) */
static int block(const aria_cuda_dec *h, const dec_blk *b, const dec_blk *next, const dec_ws *w, float *x,
                 uint16_t *h16, int nch, hipStream_t s) {
    const int N = nch * DS;
    int rc;
    if ((rc = gemm_qkv(h, b, w->qkv, h16, N, s))) return rc;
    STEP(aria_k_dec_attn(w->m16, w->qkv, nch, s), "k_dec_attn");
    if ((rc = gemm_add_dyt(x, w->m16, b->to_out, NULL, N, DD, h16, b->ff_alpha, b->ff_g, b->ff_b, s))) return rc;
    if ((rc = gemm(w->g16, 1, h16, b->ff_in, b->ff_in_b, N, DD, 2 * DINNER, ARIA_EPI_GLU, s))) return rc;
    if (next) return gemm_add_dyt(x, w->g16, b->ff_out, b->ff_out_b, N, DINNER, h16, next->pre_alpha, next->pre_g,
                                  next->pre_b, s);
    return gemm(x, 0, w->g16, b->ff_out, b->ff_out_b, N, DINNER, DD, ARIA_EPI_ADD, s);
}

/* the device part of the decode: latent [256, T] -> audio [2, T * 4096], device pointers. The
 * norm operands h16 are indexed like the haloed buffer (row 17 = the sequence's row 0), so the
 * DyT that block 2 writes for block 3 is already where the shifted pass reads it; only its halo
 * rows are copied, as the sequence's are. */
static int dec_run(aria_cuda_dec *h, const dec_ws *w, float *audio, const float *lat, int T, hipStream_t s) {
    const int Tp = T + (T & 1), L = 17 * Tp, Lt = 16 * T, Lout = 16 * Tp;
    float *seq = w->seq + (size_t)DHALF * DD;      /* the sequence proper */
    uint16_t *hseq = w->h16 + (size_t)DHALF * DD;  /* its norm operands */
    int rc;
    STEP(aria_k_dec_in(w->xt16, lat, T, h->running_std, s), "k_dec_in");
    STEP(aria_k_qgemm_e(w->x, 0, w->xt16, 1, ARIA_WF16, h->proj_w, NULL, h->proj_b, T, 256, DD, 0, 0, NULL, s),
         "k_qgemm (decoder proj)");
    STEP(aria_k_dec_expand(seq, w->x, h->new_tokens, T, Tp, s), "k_dec_expand");
    STEP(aria_k_dec_dyt(hseq, seq, h->blk[0].pre_alpha, h->blk[0].pre_g, h->blk[0].pre_b, L, s), "k_dec_dyt (pre_norm)");
    for (int i = 0; i < 3; i++)
        if ((rc = block(h, &h->blk[i], &h->blk[i + 1], w, seq, hseq, L / DS, s))) return rc;
    /* halos: [x[:17], x, x[-17:]] (src/aria_taae.c:176-183), for the sequence and its operands */
    STEP(hipMemcpyAsync(w->seq, seq, (size_t)DHALF * DD * 4, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (halo)");
    STEP(hipMemcpyAsync(seq + (size_t)L * DD, seq + (size_t)(L - DHALF) * DD, (size_t)DHALF * DD * 4,
                        hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (halo)");
    STEP(hipMemcpyAsync(w->h16, hseq, (size_t)DHALF * DD * 2, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (halo)");
    STEP(hipMemcpyAsync(hseq + (size_t)L * DD, hseq + (size_t)(L - DHALF) * DD, (size_t)DHALF * DD * 2,
                        hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (halo)");
    for (int i = 3; i < 6; i++)
        if ((rc = block(h, &h->blk[i], i < 5 ? &h->blk[i + 1] : NULL, w, w->seq, w->h16, L / DS + 1, s))) return rc;
    STEP(aria_k_dec_im2col(w->xc, seq, Lt, Lout, s), "k_dec_im2col");
    STEP(aria_k_dec_map(audio, w->xc, h->mapping_w, h->mapping_b, Lt, s), "k_dec_map (mapping + unpatch)");
    return 0;
}

static int ws_ensure(aria_cuda_dec *h, int T, dec_ws *w) {
    if (T > h->ws_T) {
        const size_t need = ws_layout(T, NULL, NULL);
        hipError_t e = hipStreamSynchronize(h->st);
        if (e != hipSuccess) return aria_hip_fail(e, "hipStreamSynchronize (decoder)");
        f_free(h->ws);
        h->ws = NULL;
        h->ws_T = 0;
        h->ws_bytes = 0;
        int rc = d_alloc(&h->ws, need);
        if (rc) return rc;
        h->ws_bytes = need;
        h->ws_T = T;
    }
    ws_layout(T, w, (char *)h->ws);
    return 0;
}

/* pinned host memory of at least `bytes` for the host entry's copies, or NULL when it cannot be
 * had (the copies then use the caller's pageable buffers directly) */
static void *pin_get(aria_cuda_dec *h, size_t bytes) {
    if (bytes <= h->pin_bytes) return h->pin;
    if (h->pin) hipHostFree(h->pin);
    h->pin = NULL;
    h->pin_bytes = 0;
    if (hipHostMalloc(&h->pin, bytes, 0) != hipSuccess) {
        hipGetLastError();
        h->pin = NULL;
        return NULL;
    }
    h->pin_bytes = bytes;
    return h->pin;
}

/* audio [2, T * 4096] from latent [256, T], host buffers, synchronous (src/aria_sa3_dec.h:109).
 * Both copies go through one pinned staging buffer kept on the handle: the latent is staged and
 * uploaded, the decode runs, the audio comes back into the same buffer (stream order puts the
 * download after the upload has read it) and is copied out. Warm, at T = 108 the whole call takes
 * about 0.94 ms against 0.70 ms of device work. */
void aria_cuda_dec_forward(aria_cuda_dec *h, float *audio, const float *latent, int T) {
    if (aria_hip_ensure()) return;
    if (!h || !audio || !latent || T <= 0 || T > DMAXT) {
        aria_hip_set_error("aria_cuda_dec_forward: invalid argument (T %d)", T);
        return;
    }
    dec_ws w;
    if (ws_ensure(h, T, &w)) return;
    hipStream_t s = h->st;
    const size_t lat_bytes = (size_t)256 * T * 4, aud_bytes = (size_t)2 * T * 4096 * 4;
    float *pin = (float *)pin_get(h, aud_bytes);   /* aud_bytes > lat_bytes */
    if (pin) memcpy(pin, latent, lat_bytes);
    hipError_t e = hipMemcpyAsync(w.lat, pin ? pin : latent, lat_bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) { aria_hip_fail(e, "hipMemcpyAsync (latent)"); return; }
    if (dec_run(h, &w, w.audio, w.lat, T, s)) { hipStreamSynchronize(s); return; }
    e = hipMemcpyAsync(pin ? (void *)pin : (void *)audio, w.audio, aud_bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) { aria_hip_fail(e, "decoder audio download"); return; }
    if (pin) memcpy(audio, pin, aud_bytes);
}

/* the same on device buffers, stream-ordered on the handle's stream: latent [256, T] and
 * audio [2, T * 4096] in HBM (for callers that keep the sampler's latent on the device) */
int aria_hip_dec_forward_dev(aria_cuda_dec *h, float *daudio, const float *dlatent, int T) {
    int rc = aria_hip_ensure();
    if (rc) return rc;
    if (!h || !daudio || !dlatent || T <= 0 || T > DMAXT) {
        aria_hip_set_error("aria_hip_dec_forward_dev: invalid argument (T %d)", T);
        return ARIA_HIP_EINVAL;
    }
    dec_ws w;
    if ((rc = ws_ensure(h, T, &w))) return rc;
    hipStream_t s = h->st;
    return dec_run(h, &w, daudio, dlatent, T, s);
}

/* the handle's stream (for events around aria_hip_dec_forward_dev) and its workspace size */
void *aria_hip_dec_stream(const aria_cuda_dec *h) { return h ? (void *)h->st : NULL; }
size_t aria_hip_dec_workspace_bytes(const aria_cuda_dec *h) { return h ? h->ws_bytes : 0; }
