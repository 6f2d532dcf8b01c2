/*
 * k_dec.hip - the small-music autoencoder decoder's glue and attention on gfx950.
 *
 * Replaces the per-op CPU loops of the reference's taae_v2 decoder (src/aria_sa3_dec.c:
 * aria_sa3_same_decode and aria_unpatch_stereo, lines 47-116; src/aria_taae.c:
 * taae_block_forward, lines 93-162) around the GEMMs, which run on the dequant GEMM
 * kernels with fp16 weights:
 *   k_dec_in      softnorm inverse and transpose: latent [256, T] * std -> fp16 [T, 256]
 *   k_dec_expand  the 17-token groups: frame t's projected token, then 16 new_tokens
 *   k_dec_dyt     DynamicTanh norm tanh(alpha x) * gamma + beta -> fp16 GEMM operand
 *   k_dec_attn    one chunk-head of the differential self-attention, fused: the q/k
 *                 DynamicTanh norms, RoPE (32 rotated dims), both softmax(q k^T / 8) v
 *                 products over the chunk's 34 tokens, their difference, merged fp16
 *   k_dec_im2col  the k = 3 mapping convolution's input rows (the last 16 of each group),
 *                 fp32: the mapping runs as an fp32 GEMM, as the reference keeps it
 *   k_dec_out     trim to T * 16 and unpatch to stereo: audio[c][l * 256 + i]
 * Arithmetic follows the reference's order (built with -ffp-contract=off); tanhf is the
 * device library's, the softmax exponential v_exp_f32 (~1 ulp).
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

#define DEC_D 768
#define DEC_S 34
#define DEC_HD 64
#define DEC_RH 16           /* rot / 2 */
#define DEC_QKV 3840

/* xt[t][c] = half(latent[c][t] * std): 64 x 4 tiles through LDS (coalesced on both sides) */
__global__ __launch_bounds__(256) void k_dec_in(uint16_t *xt, const float *lat, int T, float std) {
    __shared__ float tile[64][65];
    const int t0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int c = c0 + r, t = t0 + tx;
        tile[r][tx] = (t < T) ? lat[(size_t)c * T + t] * std : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int t = t0 + r;
        if (t < T) xt[(size_t)t * 256 + c0 + tx] = f2h_bits(tile[tx][r]);
    }
}

/* seq[r] for r < Tp * 17: group t = r / 17, slot j = r % 17; slot 0 is x[t] (zeros for the
 * padding frame t >= T), slots 1..16 the learned new_tokens (src/aria_sa3_dec.c:69-77) */
__global__ __launch_bounds__(256) void k_dec_expand(float4 *seq, const float4 *x, const float4 *tok, int T, int Tp) {
    const size_t n = (size_t)Tp * 17 * (DEC_D / 4);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const int r = (int)(i / (DEC_D / 4)), c = (int)(i % (DEC_D / 4));
        const int t = r / 17, j = r % 17;
        float4 v;
        if (j) v = tok[c];
        else v = (t < T) ? x[(size_t)t * (DEC_D / 4) + c] : make_float4(0.f, 0.f, 0.f, 0.f);
        seq[i] = v;
    }
}

/* y = half(tanhf(alpha * x) * g + b) over [rows, 768], as aria_dynamic_tanh
 * (src/aria_cpu.c:684-698) */
__global__ __launch_bounds__(256) void k_dec_dyt(uint2 *y, const float4 *x, float alpha, const float4 *g,
                                                 const float4 *b, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const int c = (int)(i % (DEC_D / 4));
        const float4 v = x[i], gg = g[c], bb = b[c];
        float o0 = tanhf(alpha * v.x), o1 = tanhf(alpha * v.y), o2 = tanhf(alpha * v.z), o3 = tanhf(alpha * v.w);
        o0 = o0 * gg.x + bb.x; o1 = o1 * gg.y + bb.y; o2 = o2 * gg.z + bb.z; o3 = o3 * gg.w + bb.w;
        y[i] = make_uint2((uint32_t)f2h_bits(o0) | ((uint32_t)f2h_bits(o1) << 16),
                          (uint32_t)f2h_bits(o2) | ((uint32_t)f2h_bits(o3) << 16));
    }
}

struct DecAttnArgs {
    uint16_t *merged;           /* [nch * 34, 768] fp16 */
    const float *qkv;           /* [nch * 34, 3840]: q | k | v | qd | kd */
    const float *qg, *qb, *kg, *kb;
    float qa, ka;
    const float *rcos, *rsin;   /* [34, 16] */
};

/* One (chunk, head) per workgroup of two waves; wave w computes the attention of pair w
 * (0: q, k; 1: qd, kd) with lane i < 34 owning query row i: its normalised, rotated q row
 * stays in registers, the chunk's k rows (normalised, rotated) and v rows sit in LDS and
 * are read as broadcasts (every lane the same address). Scores in registers, softmax per
 * lane, then o = P v. The difference ob - od goes out as the merged fp16 row
 * (src/aria_taae.c:116-133). */
__global__ __launch_bounds__(128) void k_dec_attn(DecAttnArgs a, int H) {
    __shared__ float sk[2][DEC_S][DEC_HD];
    __shared__ float sv[DEC_S][DEC_HD];
    __shared__ float sod[DEC_S][DEC_HD + 1];
    const int ch = blockIdx.x / H, h = blockIdx.x % H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float *base = a.qkv + (size_t)ch * DEC_S * DEC_QKV + h * DEC_HD;

    /* k and kd rows: DynamicTanh with the k-norm, then RoPE (pairs d, d + 16, d < 16) */
    for (int i = tid; i < 2 * DEC_S * DEC_HD; i += 128) {
        const int p = i / (DEC_S * DEC_HD), r = (i / DEC_HD) % DEC_S, d = i % DEC_HD;
        const float x = base[(size_t)r * DEC_QKV + (p ? 3072 : 768) + d];
        sk[p][r][d] = tanhf(a.ka * x) * a.kg[d] + a.kb[d];
    }
    for (int i = tid; i < DEC_S * DEC_HD; i += 128) {
        const int r = i / DEC_HD, d = i % DEC_HD;
        sv[r][d] = base[(size_t)r * DEC_QKV + 1536 + d];
    }
    __syncthreads();
    for (int i = tid; i < 2 * DEC_S * DEC_RH; i += 128) {
        const int p = i / (DEC_S * DEC_RH), r = (i / DEC_RH) % DEC_S, d = i % DEC_RH;
        const float x0 = sk[p][r][d], x1 = sk[p][r][d + DEC_RH];
        const float c = a.rcos[r * DEC_RH + d], s = a.rsin[r * DEC_RH + d];
        const float ac = x0 * c, bs = x1 * s, bc = x1 * c, as = x0 * s;
        sk[p][r][d] = ac - bs;
        sk[p][r][d + DEC_RH] = bc + as;
    }
    __syncthreads();

    const int r = lane;
    float o[DEC_HD];
    if (r < DEC_S) {
        /* this lane's query row (pair `wave`), normalised and rotated in registers */
        float q[DEC_HD];
        const float *qr = base + (size_t)r * DEC_QKV + (wave ? 2304 : 0);
#pragma unroll
        for (int d = 0; d < DEC_HD; d++) q[d] = tanhf(a.qa * qr[d]) * a.qg[d] + a.qb[d];
#pragma unroll
        for (int d = 0; d < DEC_RH; d++) {
            const float c = a.rcos[r * DEC_RH + d], s = a.rsin[r * DEC_RH + d];
            const float x0 = q[d], x1 = q[d + DEC_RH];
            const float ac = x0 * c, bs = x1 * s, bc = x1 * c, as = x0 * s;
            q[d] = ac - bs;
            q[d + DEC_RH] = bc + as;
        }
        float sc[DEC_S];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < DEC_S; j++) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < DEC_HD; d++) acc = __builtin_fmaf(q[d], sk[wave][j][d], acc);
            sc[j] = acc * 0.125f;   /* 1 / sqrt(64) */
            mx = fmaxf(mx, sc[j]);
        }
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < DEC_S; j++) {
            sc[j] = exp_fast(sc[j] - mx);
            sum += sc[j];
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
        for (int d = 0; d < DEC_HD; d++) o[d] = 0.0f;
#pragma unroll
        for (int j = 0; j < DEC_S; j++) {
            const float p = sc[j] * inv;
#pragma unroll
            for (int d = 0; d < DEC_HD; d++) o[d] = __builtin_fmaf(p, sv[j][d], o[d]);
        }
        if (wave == 1) {
#pragma unroll
            for (int d = 0; d < DEC_HD; d++) sod[r][d] = o[d];
        }
    }
    __syncthreads();
    if (wave == 0 && r < DEC_S) {
        uint32_t *dst = reinterpret_cast<uint32_t *>(a.merged + ((size_t)ch * DEC_S + r) * DEC_D + h * DEC_HD);
#pragma unroll
        for (int d = 0; d < DEC_HD; d += 2)
            dst[d >> 1] = (uint32_t)f2h_bits(o[d] - sod[r][d]) | ((uint32_t)f2h_bits(o[d + 1] - sod[r][d + 1]) << 16);
    }
}

/* xc[t][3 i + k] = seq token of feature position t + k - 1 (zero outside [0, Lout)), for the
 * first Lt positions (the trimmed output needs no more); feature position p is seq row
 * (p / 16) * 17 + 1 + p % 16, the last 16 of each group (src/aria_sa3_dec.c:85-99). The row
 * layout is the folded mapping weight's [512][768][3], so the k = 3 convolution is one GEMM. */
__global__ __launch_bounds__(256) void k_dec_im2col(float *xc, const float *seq, int Lt, int Lout) {
    const size_t n = (size_t)Lt * 3 * DEC_D;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < n; idx += (size_t)gridDim.x * 256) {
        const int t = (int)(idx / (3 * DEC_D)), j = (int)(idx % (3 * DEC_D)), i = j / 3, k = j % 3;
        const int tt = t + k - 1;
        xc[idx] = (tt >= 0 && tt < Lout) ? seq[(size_t)((tt / 16) * 17 + 1 + tt % 16) * DEC_D + i] : 0.0f;
    }
}

/* audio[c][l * 256 + i] = mapped[l][c * 256 + i], l < Lt (src/aria_sa3_dec.c:108-116, 41-46) */
__global__ __launch_bounds__(256) void k_dec_out(float4 *audio, const float4 *mapped, int Lt) {
    const size_t n = (size_t)Lt * 128;   /* float4 per channel pair row: 512 / 4 */
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const int l = (int)(i / 128), q = (int)(i % 128), c = q / 64, j = q % 64;
        audio[(size_t)c * Lt * 64 + (size_t)l * 64 + j] = mapped[i];
    }
}

static inline dim3 grid_for(size_t n) {
    size_t b = (n + 255) / 256;
    if (b > 8192) b = 8192;
    return dim3((unsigned)(b ? b : 1));
}

extern "C" hipError_t aria_k_dec_in(uint16_t *xt, const float *lat, int T, float std, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_dec_in, dim3((T + 63) / 64, 4), dim3(256), 0, s, xt, lat, T, std);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_dec_expand(float *seq, const float *x, const float *tok, int T, int Tp, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_expand, grid_for((size_t)Tp * 17 * (DEC_D / 4)), dim3(256), 0, s, (float4 *)seq,
                       (const float4 *)x, (const float4 *)tok, T, Tp);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_dec_dyt(uint16_t *y, const float *x, float alpha, const float *g, const float *b,
                                     int rows, hipStream_t s) {
    const size_t n4 = (size_t)rows * (DEC_D / 4);
    hipLaunchKernelGGL(k_dec_dyt, grid_for(n4), dim3(256), 0, s, (uint2 *)y, (const float4 *)x, alpha,
                       (const float4 *)g, (const float4 *)b, n4);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_dec_attn(uint16_t *merged, const float *qkv, float qa, const float *qg, const float *qb,
                                      float ka, const float *kg, const float *kb, const float *rcos, const float *rsin,
                                      int nch, hipStream_t s) {
    if (nch <= 0) return hipSuccess;
    DecAttnArgs a;
    a.merged = merged; a.qkv = qkv; a.qg = qg; a.qb = qb; a.kg = kg; a.kb = kb; a.qa = qa; a.ka = ka;
    a.rcos = rcos; a.rsin = rsin;
    hipLaunchKernelGGL(k_dec_attn, dim3(nch * 12), dim3(128), 0, s, a, 12);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_dec_im2col(float *xc, const float *seq, int Lt, int Lout, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_im2col, grid_for((size_t)Lt * 3 * DEC_D), dim3(256), 0, s, xc, seq, Lt, Lout);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_dec_out(float *audio, const float *mapped, int Lt, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_out, grid_for((size_t)Lt * 128), dim3(256), 0, s, (float4 *)audio,
                       (const float4 *)mapped, Lt);
    return hipGetLastError();
}
