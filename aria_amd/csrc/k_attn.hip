/*
 * k_attn.hip - the DiT's attention on gfx950: head preparation and fused MFMA attention.
 *
 * k_qkv_prep replaces the reference block's extract_heads + q/k RMSNorm + RoPE
 * (src/aria_sa3_dit.c:183-194, 222-226; device twin k_extract_normrope,
 * src/aria_cuda.cu:447-470): from a projection row [S, nsec*dim] it writes
 * head-major fp16 [B, H, S, hd] tensors, RMS-normalising (statistic in double,
 * as aria_rmsnorm) and rotating (rotate-half, rot dims) the q and k sections.
 *
 * k_flash_attn replaces aria_attention (src/aria_cpu.c:811-849: scores = q k^T,
 * x 1/sqrt(D), row softmax, P V) and the reference's unfused device path
 * (src/aria_cuda.cu:785-806: fp16 QK^T -> fp32 scores in HBM -> softmax -> PV).
 * Scores never reach HBM: each 32-query slice keeps a running max / sum (online
 * softmax) and an fp32 output accumulator.
 *
 * Formulation: S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_32x32x16_f16, so the
 * score accumulator of lane l (query column l%32, keys 8*(r/4)+4*(l/32)+r%4) is
 * directly the B operand of the P V product once rounded to fp16; the key order
 * inside each 16-key MFMA step is permuted identically for the V^T operand (sums
 * over keys do not depend on order). Lanes l and l^32 hold the same query, so the
 * softmax statistics need a single xor-32 exchange.
 *
 * Precision: Q, K, V and P are fp16, accumulation fp32, exp via v_exp_f32.
 * Workgroup: 4 waves x 32 queries = 128 queries of one (batch, head); K and V
 * tiles of 64 keys are staged in LDS (V transposed) with register prefetch of
 * the next tile.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

/* ------------------------------------------------------------------------- */
/* head preparation                                                          */
/* ------------------------------------------------------------------------- */

/* One 16-lane group per (token, section, head) row of hd = 64 (4 floats per lane).
 * src: [B*S, ld] fp32 projection output; section sec starts at column sec*dim.
 * Sections: q (norm wq, rope), k (norm wk, rope), v (copy). nsec = number present
 * in src; which[sec] says what each is (0 = q, 1 = k, 2 = v). */
struct PrepArgs {
    const float *src;
    int ld, S, H, nsec;
    int kind[3];
    uint16_t *dst[3];
    const float *w[3];
    const float *cos_t, *sin_t;
    int rot;
    float eps;
    int rows;   /* B*S*nsec*H */
};

__global__ __launch_bounds__(256) void k_qkv_prep(PrepArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * 256 + threadIdx.x) >> 4;   /* one row per 16 lanes */
    const int l = lane & 15;
    if (row >= a.rows) return;
    const int h = row % a.H;
    const int sec = (row / a.H) % a.nsec;
    const int tok = row / (a.H * a.nsec);   /* b*S + s */
    const int s = tok % a.S, b = tok / a.S;
    const float4 v = *reinterpret_cast<const float4 *>(a.src + (size_t)tok * a.ld + (size_t)sec * a.H * 64 + h * 64 + 4 * l);
    const int kind = a.kind[sec];
    float o[4] = {v.x, v.y, v.z, v.w};
    if (kind != 2) {
        double ss = ((double)v.x * v.x + (double)v.y * v.y) + ((double)v.z * v.z + (double)v.w * v.w);
        ss = grp_sum<16>(ss);
        const float inv = (float)(1.0 / sqrt(ss / 64 + (double)a.eps));
        const float *w = a.w[sec];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o[e] = o[e] * inv;
            if (w) o[e] = o[e] * w[4 * l + e];
        }
        if (a.rot > 0 && a.cos_t) {
            const int rh = a.rot >> 1, lp = rh >> 2;   /* partner lane offset */
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; e++) p[e] = __shfl(o[e], (lane & 48) | (l ^ lp), ARIA_WAVE);
            const int d0 = 4 * l;
            if (d0 < a.rot) {
                const bool first = d0 < rh;
                const int i0 = first ? d0 : d0 - rh;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float c = a.cos_t[(size_t)s * rh + i0 + e], sn = a.sin_t[(size_t)s * rh + i0 + e];
                    /* first half: a*c - b*s; second half: b*c + a*s (a = first, b = second) */
                    if (first) { float ac = o[e] * c, bs = p[e] * sn; o[e] = ac - bs; }
                    else { float bc = o[e] * c, as = p[e] * sn; o[e] = bc + as; }
                }
            }
        }
    }
    uint16_t *d = a.dst[sec] + (((size_t)b * a.H + h) * a.S + s) * 64 + 4 * l;
    *reinterpret_cast<uint2 *>(d) = make_uint2((uint32_t)f2h_bits(o[0]) | ((uint32_t)f2h_bits(o[1]) << 16),
                                               (uint32_t)f2h_bits(o[2]) | ((uint32_t)f2h_bits(o[3]) << 16));
}

extern "C" hipError_t aria_k_qkv_prep(const float *src, int ld, int B, int S, int H, int nsec, const int *kind,
                                      uint16_t *const *dst, const float *const *w, const float *cos_t,
                                      const float *sin_t, int rot, float eps, hipStream_t s) {
    if (B <= 0 || S <= 0 || H <= 0 || nsec <= 0) return hipSuccess;
    PrepArgs a;
    a.src = src; a.ld = ld; a.S = S; a.H = H; a.nsec = nsec;
    for (int i = 0; i < 3; i++) {
        a.kind[i] = i < nsec ? kind[i] : 2;
        a.dst[i] = i < nsec ? dst[i] : nullptr;
        a.w[i] = i < nsec ? w[i] : nullptr;
    }
    a.cos_t = cos_t; a.sin_t = sin_t; a.rot = rot; a.eps = eps;
    a.rows = B * S * nsec * H;
    const long threads = (long)a.rows * 16;
    hipLaunchKernelGGL(k_qkv_prep, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

/* ------------------------------------------------------------------------- */
/* fused attention                                                           */
/* ------------------------------------------------------------------------- */

#define KT 64                 /* keys per staged tile */
#define KS_STRIDE (64 + 8)    /* halves: K tile rows [key][d] */
#define VT_STRIDE (KT + 8)    /* halves: V^T tile rows [d][key] */

struct AttnArgs {
    const uint16_t *q, *k, *v;   /* [B*H, N, 64] fp16 */
    void *o;                     /* [B, Nq, H*64] merged heads */
    int H, Nq, Nk;
    float scale_log2;            /* (1/sqrt(64)) * log2(e) */
    int o_f16;
};

__device__ __forceinline__ half8_t ld_h8(const uint16_t *p) { return *reinterpret_cast<const half8_t *>(p); }

__global__ __launch_bounds__(256) void k_flash_attn(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][KT * KS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][64 * VT_STRIDE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
    const int bh = blockIdx.y;
    const int q0 = blockIdx.x * 128 + wave * 32;
    const uint16_t *Qh = a.q + (size_t)bh * a.Nq * 64;
    const uint16_t *Kh = a.k + (size_t)bh * a.Nk * 64;
    const uint16_t *Vh = a.v + (size_t)bh * a.Nk * 64;

    /* Q^T fragments (B operand of S^T = K Q^T): query q0 + l32, d = 16*ds + 8g + [0,8) */
    half8_t qf[4];
    {
        const int qi = q0 + l32;
#pragma unroll
        for (int ds = 0; ds < 4; ds++) {
            if (qi < a.Nq) qf[ds] = ld_h8(Qh + (size_t)qi * 64 + 16 * ds + 8 * g);
            else qf[ds] = (half8_t){};
        }
    }

    /* tile staging: thread t loads key t/4, d chunk 16*(t%4) of K and V */
    const int skey = tid >> 2, sd = 16 * (tid & 3);
    uint32_t rk[8], rv[8];
    auto gload = [&](int kt0) {
        const int key = kt0 + skey;
        const bool ok = key < a.Nk;
        const size_t off = (size_t)(ok ? key : 0) * 64 + sd;   /* always an in-bounds address */
        const uint4 k0 = *reinterpret_cast<const uint4 *>(Kh + off);
        const uint4 k1 = *reinterpret_cast<const uint4 *>(Kh + off + 8);
        const uint4 v0 = *reinterpret_cast<const uint4 *>(Vh + off);
        const uint4 v1 = *reinterpret_cast<const uint4 *>(Vh + off + 8);
        rk[0] = ok ? k0.x : 0u; rk[1] = ok ? k0.y : 0u; rk[2] = ok ? k0.z : 0u; rk[3] = ok ? k0.w : 0u;
        rk[4] = ok ? k1.x : 0u; rk[5] = ok ? k1.y : 0u; rk[6] = ok ? k1.z : 0u; rk[7] = ok ? k1.w : 0u;
        rv[0] = ok ? v0.x : 0u; rv[1] = ok ? v0.y : 0u; rv[2] = ok ? v0.z : 0u; rv[3] = ok ? v0.w : 0u;
        rv[4] = ok ? v1.x : 0u; rv[5] = ok ? v1.y : 0u; rv[6] = ok ? v1.z : 0u; rv[7] = ok ? v1.w : 0u;
    };
    auto sstore = [&](int buf) {
        uint4 *dk = reinterpret_cast<uint4 *>(&Ks[buf][skey * KS_STRIDE + sd]);
        dk[0] = make_uint4(rk[0], rk[1], rk[2], rk[3]);
        dk[1] = make_uint4(rk[4], rk[5], rk[6], rk[7]);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            Vt[buf][(sd + 2 * i) * VT_STRIDE + skey] = (uint16_t)(rv[i] & 0xFFFF);
            Vt[buf][(sd + 2 * i + 1) * VT_STRIDE + skey] = (uint16_t)(rv[i] >> 16);
        }
    };

    f32x16_t oacc[2];
#pragma unroll
    for (int r = 0; r < 16; r++) { oacc[0][r] = 0.0f; oacc[1][r] = 0.0f; }
    float m_run = -INFINITY, l_run = 0.0f;

    const int ntiles = (a.Nk + KT - 1) / KT;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int t = 0; t < ntiles; t++) {
        const int buf = t & 1, kt0 = t * KT;
        if (t + 1 < ntiles) gload(kt0 + KT);
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int kb = half * 32;   /* key offset inside the tile */
            /* S^T [32 keys x 32 queries] */
            f32x16_t s;
#pragma unroll
            for (int r = 0; r < 16; r++) s[r] = 0.0f;
#pragma unroll
            for (int ds = 0; ds < 4; ds++) {
                const half8_t kf = ld_h8(&Ks[buf][(kb + l32) * KS_STRIDE + 16 * ds + 8 * g]);
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ds], s, 0, 0, 0);
            }
            /* online softmax over this lane's 16 keys + the partner lane's 16 */
            float mt = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = kt0 + kb + 8 * (r >> 2) + 4 * g + (r & 3);
                s[r] = key < a.Nk ? s[r] * a.scale_log2 : -INFINITY;
                mt = fmaxf(mt, s[r]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32, ARIA_WAVE));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            float rs = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                s[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
                rs += s[r];
            }
            rs += __shfl_xor(rs, 32, ARIA_WAVE);
            l_run = l_run * alpha + rs;
            m_run = m_new;
#pragma unroll
            for (int r = 0; r < 16; r++) { oacc[0][r] *= alpha; oacc[1][r] *= alpha; }
            /* P^T fragments: MFMA step ks takes accumulator registers 8ks..8ks+7 */
            half8_t pf[2];
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int i = 0; i < 8; i++) pf[ks][i] = (_Float16)s[8 * ks + i];
            /* O^T [64 d x 32 q] += V^T [d x keys] P^T; V^T row d, keys of step ks for lane group g:
             * kb + 16ks + 4g + {0..3} and kb + 16ks + 8 + 4g + {0..3} */
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    const uint16_t *vp = &Vt[buf][(dt * 32 + l32) * VT_STRIDE + kb + 16 * ks + 4 * g];
                    const half4_t lo = *reinterpret_cast<const half4_t *>(vp);
                    const half4_t hi = *reinterpret_cast<const half4_t *>(vp + 8);
                    const half8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[ks], oacc[dt], 0, 0, 0);
                }
            }
        }
        /* buffer buf^1 was last read in iteration t-1, which ended with a barrier */
        if (t + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
    }

    /* O[q, d] = O^T[d, q] / l ; lane holds query q0 + l32, d = 32dt + 8(r/4) + 4g + r%4 */
    const int qi = q0 + l32;
    if (qi >= a.Nq) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const int b = bh / a.H, h = bh % a.H;
    const size_t orow = ((size_t)b * a.Nq + qi) * (size_t)(a.H * 64) + h * 64;
#pragma unroll
    for (int dt = 0; dt < 2; dt++) {
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d = 32 * dt + 8 * rq + 4 * g;
            const float v0 = oacc[dt][4 * rq] * inv, v1 = oacc[dt][4 * rq + 1] * inv;
            const float v2 = oacc[dt][4 * rq + 2] * inv, v3 = oacc[dt][4 * rq + 3] * inv;
            if (a.o_f16) {
                *reinterpret_cast<uint2 *>((uint16_t *)a.o + orow + d) =
                    make_uint2((uint32_t)f2h_bits(v0) | ((uint32_t)f2h_bits(v1) << 16),
                               (uint32_t)f2h_bits(v2) | ((uint32_t)f2h_bits(v3) << 16));
            } else {
                *reinterpret_cast<float4 *>((float *)a.o + orow + d) = make_float4(v0, v1, v2, v3);
            }
        }
    }
}

extern "C" hipError_t aria_k_flash_attn(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *o, int o_f16,
                                        int BH, int H, int Nq, int Nk, hipStream_t s) {
    if (BH <= 0 || Nq <= 0) return hipSuccess;
    AttnArgs a;
    a.q = q; a.k = k; a.v = v; a.o = o; a.H = H; a.Nq = Nq; a.Nk = Nk; a.o_f16 = o_f16;
    a.scale_log2 = 0.125f * ARIA_LOG2E;
    dim3 grid((Nq + 127) / 128, BH);
    hipLaunchKernelGGL(k_flash_attn, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}
