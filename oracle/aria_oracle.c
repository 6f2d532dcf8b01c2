/*
 * aria_oracle.c - TEST INFRASTRUCTURE ONLY: scalar restatement of the reference
 * DiT op path, the checker for the HIP backend (see aria_oracle.h). Built by
 * oracle/Makefile with -ffp-contract=off, never linked into the product.
 *
 * Pinning (checks that are not a retyping of the formula; tests/test_oracle.py):
 *   or_rmsnorm        KAT [3,4] eps 0 -> [0.848528,1.131371] (tests/test_ops.c:72-79);
 *                     vs the compiled reference aria_rmsnorm; scale invariance.
 *   or_gemma_rmsnorm  vs compiled reference aria_gemma_rmsnorm; w=0 equals rmsnorm(w=NULL).
 *   or_layernorm      no reference op exists. Closed forms: constant row -> beta;
 *                     [a,-a] -> +-a/sqrt(a^2+eps); output mean 0 / var 1; long-double brute force.
 *   or_adaln_modulate scale=0,shift=0 identity; vs numpy float32 with explicit rounding.
 *   or_gate_*         gate=1 -> sigmoid(0)=0.5 exactly; vs compiled reference composition.
 *   or_gelu_tanh      KAT gelu(1)=0.841192 (tests/test_ops.c:86-91); vs compiled reference.
 *   or_silu(_gate)    KATs silu(1)=0.731059, silu_gate(1,2)=1.462118 (tests/test_ops.c:80-85,101-106).
 *   or_softmax        KAT [1,2,3] (tests/test_ops.c:93-100); rows sum to 1; masked cols -> 0.
 *   or_rope_*         p=0 identity; pair-norm preservation; R(p1)R(p2)=R(p1+p2); vs reference.
 *   or_q8/q4_quant    bit-exact vs the compiled reference aria_q8_quant/aria_q4_quant;
 *                     closed forms (zero row, constant block, +-amax -> +-127, odd-K pad nibble).
 *   or_linear_q8/q4   vs reference aria_linear_q8/q4; identity-weight brute force in double.
 *   or_quant_act_q8 / or_linear_q8a8  bit-exact vs the compiled reference aria_linear_q8a8
 *                     on the reference's own W8A8 shapes (tests/test_quant.c:141-170);
 *                     closed forms (row max -> +-127, zero row -> 0, int64 brute force of
 *                     the dot products, one-hot weights pick one column).
 *   or_linear         vs an independent float64 numpy matmul; KAT tests/test_ops.c:53-63.
 *   or_attention      vs compiled reference aria_attention; uniform-score closed form.
 *   or_add/addto/scale/axpy  bit-exact vs the compiled reference aria_add/addto/scale/axpy;
 *                     closed forms (s = 0, s = 1, x + (-x) = 0, exact small integers).
 *   or_pingpong       bit-exact vs the compiled reference sampler loop aria_pingpong_cb
 *                     (src/aria_sampler.c:203-229) over 8 LogSNR steps with injected noise;
 *                     closed forms tn=1 -> noise, tc=1,tn=0 -> x-v, tc=tn=0 identity.
 */
#include "aria_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* RMSNorm. Follows src/aria_cpu.c:643-682: sum of squares accumulated in double
 * (aria_sumsq_f, src/aria_cpu.c:57-98; each (double)x*x is exact, only the
 * summation order differs from the 8-lane AVX2 reduction), inv rounded to float
 * once, then (x*inv)*w in float. */
void or_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * dim;
        float *yr = y + (size_t)r * dim;
        double ss = 0.0;
        for (int i = 0; i < dim; i++) ss += (double)xr[i] * (double)xr[i];
        float inv = (float)(1.0 / sqrt(ss / dim + eps));
        for (int i = 0; i < dim; i++) {
            float v = xr[i] * inv;
            yr[i] = w ? v * w[i] : v;
        }
    }
}

/* Gemma RMSNorm, src/aria_cpu.c:703-733: y = (x*inv)*(1+w). */
void or_gemma_rmsnorm(float *y, const float *x, const float *w, int rows, int dim, float eps) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * dim;
        float *yr = y + (size_t)r * dim;
        double ss = 0.0;
        for (int i = 0; i < dim; i++) ss += (double)xr[i] * (double)xr[i];
        float inv = (float)(1.0 / sqrt(ss / dim + eps));
        for (int i = 0; i < dim; i++) yr[i] = (xr[i] * inv) * (1.0f + w[i]);
    }
}

/* LayerNorm: the reference has no such op (its norms are RMSNorm variants,
 * src/aria_ops.h:89-108). Textbook biased-variance LayerNorm with the statistics
 * in double, matching how the reference computes its RMS statistic:
 *   mu = sum(x)/dim, var = sum((x-mu)^2)/dim, rstd = 1/sqrt(var+eps)   (double)
 *   n  = (float)((x-mu)*rstd);  y = n*gamma + beta                      (float) */
void or_layernorm(float *y, const float *x, const float *gamma, const float *beta,
                  int rows, int dim, float eps) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * dim;
        float *yr = y + (size_t)r * dim;
        double s = 0.0;
        for (int i = 0; i < dim; i++) s += (double)xr[i];
        double mu = s / dim, v = 0.0;
        for (int i = 0; i < dim; i++) { double d = (double)xr[i] - mu; v += d * d; }
        double rstd = 1.0 / sqrt(v / dim + (double)eps);
        for (int i = 0; i < dim; i++) {
            float n = (float)(((double)xr[i] - mu) * rstd);
            if (gamma) n = n * gamma[i];
            if (beta) n = n + beta[i];
            yr[i] = n;
        }
    }
}

/* adaLN modulate, src/aria_sa3_dit.c:71-82: y = y*(1+scale)+shift, each op
 * rounded on its own (no contraction in the reference's -std=c11 build). */
void or_adaln_modulate(float *y, const float *scale, const float *shift, int rows, int dim) {
    for (int r = 0; r < rows; r++) {
        float *yr = y + (size_t)r * dim;
        for (int i = 0; i < dim; i++) {
            float t = 1.0f + scale[i];
            float p = yr[i] * t;
            yr[i] = p + shift[i];
        }
    }
}

/* gate, src/aria_sa3_dit.c:85-97: y *= sigmoid(1-gate), sigmoid per column. */
void or_gate_sigmoid(float *y, const float *gate, int rows, int dim) {
    float *sg = (float *)malloc((size_t)dim * sizeof(float));
    for (int i = 0; i < dim; i++) sg[i] = 1.0f / (1.0f + expf(-(1.0f - gate[i])));
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < dim; i++) y[(size_t)r * dim + i] *= sg[i];
    free(sg);
}

/* gate + residual as one pass: out = res + (o [+ b]) * sigmoid(1-gate).
 * With bias NULL this is src/aria_sa3_dit.c:211-215 (gate_sigmoid then x += o);
 * the bias fold follows src/aria_cuda.cu:620-628 (b binds to o first, and a
 * NULL bias adds nothing so -0.0 survives). */
void or_gate_residual(float *out, const float *res, const float *o, const float *gate,
                      const float *bias, int rows, int dim) {
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < dim; i++) {
            size_t idx = (size_t)r * dim + i;
            float sg = 1.0f / (1.0f + expf(-(1.0f - gate[i])));
            float ov = bias ? o[idx] + bias[i] : o[idx];
            float g = ov * sg;
            out[idx] = res[idx] + g;
        }
}

/* src/aria_cpu.c:989-994 */
void or_add(float *y, const float *a, const float *b, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}
void or_addto(float *y, const float *a, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] += a[i];
}
/* src/aria_cpu.c:995-1000: y = x*s and y += s*x (a product, then a sum: no contraction) */
void or_scale(float *y, const float *x, float s, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = x[i] * s;
}
void or_axpy(float *y, const float *x, float s, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] += s * x[i];
}

/* tanh GELU, src/aria_cpu.c:742-749, evaluated left to right as written:
 * inner = c*(v + ((0.044715*v)*v)*v); out = (0.5*v)*(1+tanh(inner)). */
void or_gelu_tanh(float *x, size_t n) {
    const float c = 0.7978845608028654f;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        float cube = 0.044715f * v;
        cube = cube * v;
        cube = cube * v;
        float inner = c * (v + cube);
        float h = 0.5f * v;
        x[i] = h * (1.0f + tanhf(inner));
    }
}

/* src/aria_cpu.c:735-740 */
void or_silu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) { float v = x[i]; x[i] = v / (1.0f + expf(-v)); }
}

/* src/aria_cpu.c:751-756 */
void or_silu_gate(float *out, const float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}

/* GLU combine of a projected row [value | gate] (value = first half,
 * src/aria_cpu.c:976-982 / src/aria_sa3_dit.c:108-121); an optional bias [2*inner]
 * is added to each half first, as src/aria_cuda.cu:712-731 folds the ff_in bias. */
void or_glu_combine(float *out, const float *proj, const float *bias, int rows, int inner) {
    for (int r = 0; r < rows; r++) {
        const float *pr = proj + (size_t)r * 2 * inner;
        float *orow = out + (size_t)r * inner;
        for (int i = 0; i < inner; i++) {
            float up = pr[i], g = pr[inner + i];
            if (bias) { up = up + bias[i]; g = g + bias[inner + i]; }
            float s = g / (1.0f + expf(-g));
            orow[i] = s * up;
        }
    }
}

/* pingpong update, src/aria_sampler.c:216-220: d = x - tc*v;
 * x = (1-tn)*d + tn*noise, every operation rounded on its own. */
void or_pingpong(float *x, const float *v, const float *noise, float tc, float tn, size_t n) {
    float a = 1.0f - tn;
    for (size_t i = 0; i < n; i++) {
        float tv = tc * v[i];
        float d = x[i] - tv;
        float p = a * d;
        float q = tn * noise[i];
        x[i] = p + q;
    }
}

/* row softmax with optional additive mask, src/aria_cpu.c:758-776: max, then
 * e = expf(x-max) with a sequential fp32 sum, inv = sum>0 ? 1/sum : 0, x *= inv. */
void or_softmax(float *x, int rows, int cols, const float *mask) {
    for (int r = 0; r < rows; r++) {
        float *xr = x + (size_t)r * cols;
        const float *mr = mask ? mask + (size_t)r * cols : NULL;
        float maxv = -INFINITY;
        for (int i = 0; i < cols; i++) {
            float v = xr[i] + (mr ? mr[i] : 0.0f);
            xr[i] = v;
            if (v > maxv) maxv = v;
        }
        float sum = 0.0f;
        for (int i = 0; i < cols; i++) { float e = expf(xr[i] - maxv); xr[i] = e; sum += e; }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int i = 0; i < cols; i++) xr[i] *= inv;
    }
}

/* RoPE tables, src/aria_cpu.c:778-788: inv_i = 1/base^(2i/rot) and the angles
 * in double, stored as float [n, rot/2]. */
void or_rope_freqs(float *cos_t, float *sin_t, int n, int rot_dim, float base) {
    int rh = rot_dim / 2;
    for (int i = 0; i < rh; i++) {
        double inv = 1.0 / pow((double)base, (double)(2 * i) / (double)rot_dim);
        for (int p = 0; p < n; p++) {
            double ang = (double)p * inv;
            cos_t[(size_t)p * rh + i] = (float)cos(ang);
            sin_t[(size_t)p * rh + i] = (float)sin(ang);
        }
    }
}

/* rotate-half RoPE on [H,N,D], src/aria_cpu.c:790-809:
 * a' = a*c - b*s, b' = b*c + a*s for pairs (i, i+rot/2); dims >= rot untouched. */
void or_rope_apply(float *x, const float *cos_t, const float *sin_t,
                   int H, int N, int D, int rot_dim) {
    int rh = rot_dim / 2;
    for (int h = 0; h < H; h++)
        for (int p = 0; p < N; p++) {
            float *row = x + ((size_t)h * N + p) * D;
            const float *c = cos_t + (size_t)p * rh, *s = sin_t + (size_t)p * rh;
            for (int i = 0; i < rh; i++) {
                float a = row[i], b = row[i + rh];
                float ac = a * c[i], bs = b * s[i], bc = b * c[i], as = a * s[i];
                row[i] = ac - bs;
                row[i + rh] = bc + as;
            }
        }
}

/* Config 1/2 chain: out = gelu_tanh(LN(x)*(1+scale[b])+shift[b]) + x, the
 * composition or_layernorm -> or_adaln_modulate -> or_gelu_tanh -> or_add.
 * scale/shift are [batch, dim], broadcast over each batch's rows. */
void or_fused_chain(float *out, const float *x, const float *gamma, const float *beta,
                    const float *scale, const float *shift, int batch, int rows_per_batch,
                    int dim, float eps) {
    size_t per = (size_t)rows_per_batch * dim;
    for (int b = 0; b < batch; b++) {
        float *ob = out + b * per;
        const float *xb = x + b * per;
        or_layernorm(ob, xb, gamma, beta, rows_per_batch, dim, eps);
        or_adaln_modulate(ob, scale + (size_t)b * dim, shift + (size_t)b * dim, rows_per_batch, dim);
        or_gelu_tanh(ob, per);
        or_addto(ob, xb, per);
    }
}

/* Q8 pack, src/aria_quant.c:78-96: per row amax, s = amax/127, inv = 1/s,
 * q = clamp(lrintf(w*inv), -127, 127) (round half to even), zero row -> q = 0. */
void or_q8_quant(int8_t *q, float *scale, const float *W, int N, int K) {
    for (int n = 0; n < N; n++) {
        const float *wr = W + (size_t)n * K;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) { float a = fabsf(wr[k]); if (a > amax) amax = a; }
        float s = amax / 127.0f;
        scale[n] = s;
        int8_t *qr = q + (size_t)n * K;
        if (s > 0.0f) {
            float inv = 1.0f / s;
            for (int k = 0; k < K; k++) qr[k] = (int8_t)clampi((int)lrintf(wr[k] * inv), -127, 127);
        } else {
            memset(qr, 0, (size_t)K);
        }
    }
}

/* Q4 pack, src/aria_quant.c:353-380: blocks of 32 along K (last may be short),
 * [min, (max-min)/15] per block, nib = clamp(lrintf((w-min)*inv), 0, 15),
 * even k -> low nibble, odd k -> high nibble of byte k>>1; row stride ceil(K/2). */
void or_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K) {
    int nblk = (K + 31) / 32;
    size_t rb = (size_t)(K + 1) / 2;
    for (int n = 0; n < N; n++) {
        const float *wr = W + (size_t)n * K;
        uint8_t *qr = q + (size_t)n * rb;
        float *sr = scale + (size_t)n * 2 * nblk;
        memset(qr, 0, rb);
        for (int bi = 0; bi < nblk; bi++) {
            int k0 = bi * 32, k1 = k0 + 32 < K ? k0 + 32 : K;
            float mn = wr[k0], mx = wr[k0];
            for (int k = k0 + 1; k < k1; k++) { float v = wr[k]; if (v < mn) mn = v; if (v > mx) mx = v; }
            float s = (mx - mn) / 15.0f;
            sr[2 * bi] = mn; sr[2 * bi + 1] = s;
            float inv = s > 0.0f ? 1.0f / s : 0.0f;
            for (int k = k0; k < k1; k++) {
                uint8_t nib = s > 0.0f ? (uint8_t)clampi((int)lrintf((wr[k] - mn) * inv), 0, 15) : 0;
                if (k & 1) qr[k >> 1] |= (uint8_t)(nib << 4);
                else       qr[k >> 1] |= nib;
            }
        }
    }
}

/* Q8 dequant, tests/test_quant.c:20-23 and src/aria_cuda.cu:819-823: W = q*scale[n]. */
void or_q8_dequant(float *W, const int8_t *q, const float *scale, int N, int K) {
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) W[(size_t)n * K + k] = (float)q[(size_t)n * K + k] * scale[n];
}

/* Q4 dequant, src/aria_cuda.cu:825-835: W = min + nib*scale with the pair at
 * (n*nblk + k/32)*2 and the nibble at byte n*ceil(K/2) + k/2. */
void or_q4_dequant(float *W, const uint8_t *q, const float *scale, int N, int K) {
    int nblk = (K + 31) / 32;
    size_t rb = (size_t)(K + 1) / 2;
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) {
            uint8_t byte = q[(size_t)n * rb + (k >> 1)];
            int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
            size_t si = ((size_t)n * nblk + k / 32) * 2;
            float p = (float)nib * scale[si + 1];
            W[(size_t)n * K + k] = scale[si] + p;
        }
}

/* Q8 dequant-on-use GEMM, the scalar branch of src/aria_quant.c:98-145:
 * acc = sum_k x*(float)q sequentially in fp32, y = acc*scale[n] + b[n]. (The AVX2
 * branch sums 16 lanes then reduces; the difference is far below the 1e-3 gate.) */
void or_linear_q8(float *y, const float *x, const int8_t *q, const float *scale,
                  const float *b, int M, int K, int N) {
    for (int m = 0; m < M; m++) {
        const float *xr = x + (size_t)m * K;
        for (int n = 0; n < N; n++) {
            const int8_t *qn = q + (size_t)n * K;
            float acc = 0.0f;
            for (int k = 0; k < K; k++) { float p = xr[k] * (float)qn[k]; acc += p; }
            float s = acc * scale[n];
            y[(size_t)m * N + n] = s + (b ? b[n] : 0.0f);
        }
    }
}

/* W8A8 activation quantisation, the row loop of src/aria_quant.c:258-270: amax = max |x|
 * (a strict > scan from 0), sx = amax / 127, xq = clamp(lrintf(x * (127 / amax)), -127, 127),
 * all zero when amax == 0. */
void or_quant_act_q8(int8_t *xq, float *sx, const float *x, int M, int K) {
    for (int m = 0; m < M; m++) {
        const float *xr = x + (size_t)m * K;
        int8_t *qr = xq + (size_t)m * K;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) { float a = fabsf(xr[k]); if (a > amax) amax = a; }
        sx[m] = amax / 127.0f;
        if (amax > 0.0f) {
            float inv = 127.0f / amax;
            for (int k = 0; k < K; k++) {
                long v = lrintf(xr[k] * inv);
                qr[k] = (int8_t)(v < -127 ? -127 : (v > 127 ? 127 : v));
            }
        } else {
            memset(qr, 0, (size_t)K);
        }
    }
}

/* W8A8 GEMM, the scalar branch of src/aria_quant.c:272-345: acc = sum_k xq*q in int32
 * (exact), y = (float)acc * sx[m] * scale[n] + (b ? b[n] : 0.0f), left to right. */
void or_linear_q8a8(float *y, const float *x, const int8_t *q, const float *scale,
                    const float *b, int M, int K, int N) {
    int8_t *xq = (int8_t *)malloc((size_t)M * K + 1);
    float *sx = (float *)malloc((size_t)M * sizeof(float) + 4);
    if (!xq || !sx) { free(xq); free(sx); return; }
    or_quant_act_q8(xq, sx, x, M, K);
    for (int m = 0; m < M; m++) {
        const int8_t *xr = xq + (size_t)m * K;
        for (int n = 0; n < N; n++) {
            const int8_t *qn = q + (size_t)n * K;
            int32_t acc = 0;
            for (int k = 0; k < K; k++) acc += (int32_t)xr[k] * qn[k];
            float v = (float)acc * sx[m];
            v = v * scale[n];
            y[(size_t)m * N + n] = v + (b ? b[n] : 0.0f);
        }
    }
    free(xq);
    free(sx);
}

/* Q4 dequant-on-use GEMM, src/aria_quant.c:469-538 (its x86 build is this scalar
 * loop): per block xsum = sum x, nxsum = sum x*nib, acc += mn*xsum + sc*nxsum. */
void or_linear_q4(float *y, const float *x, const uint8_t *q, const float *scale,
                  const float *b, int M, int K, int N) {
    int nblk = (K + 31) / 32;
    size_t rb = (size_t)(K + 1) / 2;
    for (int m = 0; m < M; m++) {
        const float *xr = x + (size_t)m * K;
        for (int n = 0; n < N; n++) {
            const uint8_t *qn = q + (size_t)n * rb;
            const float *sn = scale + (size_t)n * 2 * nblk;
            float acc = 0.0f;
            for (int bi = 0; bi < nblk; bi++) {
                int k0 = bi * 32, k1 = k0 + 32 < K ? k0 + 32 : K;
                float mn = sn[2 * bi], sc = sn[2 * bi + 1];
                float xsum = 0.0f, nxsum = 0.0f;
                for (int k = k0; k < k1; k++) {
                    uint8_t byte = qn[k >> 1];
                    int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                    xsum += xr[k];
                    float p = xr[k] * (float)nib;
                    nxsum += p;
                }
                float t0 = mn * xsum, t1 = sc * nxsum;
                acc += t0 + t1;
            }
            y[(size_t)m * N + n] = acc + (b ? b[n] : 0.0f);
        }
    }
}

/* fp32 linear y = x W^T + b: the per-output invariant of the reference's packed
 * GEMM (tests/test_gemm.c:1-4, 18-25): one fmaf chain from +0 over ascending k,
 * bias added last. */
void or_linear(float *y, const float *x, const float *W, const float *b, int M, int K, int N) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = fmaf(x[(size_t)m * K + k], W[(size_t)n * K + k], acc);
            y[(size_t)m * N + n] = b ? acc + b[n] : acc;
        }
}

/* C = A B, src/aria_cpu.c:626-641: c[n] += a[k]*b[k,n] over ascending k. */
void or_matmul(float *C, const float *A, const float *B, int M, int K, int N) {
    for (int m = 0; m < M; m++) {
        float *cr = C + (size_t)m * N;
        for (int n = 0; n < N; n++) cr[n] = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = A[(size_t)m * K + k];
            const float *br = B + (size_t)k * N;
            for (int n = 0; n < N; n++) { float p = a * br[n]; cr[n] += p; }
        }
    }
}

/* attention, src/aria_cpu.c:811-849: per head, scores = q k^T (fp32 linear),
 * scores *= 1/sqrtf(D), softmax with optional mask, out = P V. */
void or_attention(float *out, const float *q, const float *k, const float *v,
                  int H, int Nq, int Nk, int D, const float *mask) {
    float scale = 1.0f / sqrtf((float)D);
    float *sc = (float *)malloc((size_t)Nq * Nk * sizeof(float));
    for (int h = 0; h < H; h++) {
        const float *qh = q + (size_t)h * Nq * D, *kh = k + (size_t)h * Nk * D;
        const float *vh = v + (size_t)h * Nk * D;
        or_linear(sc, qh, kh, NULL, Nq, D, Nk);
        for (size_t i = 0; i < (size_t)Nq * Nk; i++) sc[i] *= scale;
        or_softmax(sc, Nq, Nk, mask);
        or_matmul(out + (size_t)h * Nq * D, sc, vh, Nq, Nk, D);
    }
    free(sc);
}
