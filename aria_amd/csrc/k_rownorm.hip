/*
 * k_rownorm.hip - row normalisations with a fused epilogue, one HBM pass.
 *
 * Replaces the reference's aria_rmsnorm / aria_gemma_rmsnorm (src/aria_cpu.c:643-733),
 * the DiT's rmsnorm + adaln_modulate pair (src/aria_sa3_dit.c:71-82, 175-176,
 * 255-256) and the config chain LayerNorm -> modulate -> tanh-GELU -> + x.
 *
 * Mapping: a row is owned by LPR lanes of one wave64 (LPR = 64 for dim >= 256,
 * 16 for the 64-wide q/k-norm rows). Each lane loads VPL float4 (128-bit,
 * coalesced: lane l reads vectors l, l+LPR, ...), keeps them in registers,
 * reduces the statistic in double across its LPR lanes with xor shuffles, and
 * writes the transformed row once: HBM traffic = read x + write y. No LDS, no
 * block barrier; 4 waves per 256-thread workgroup.
 *
 * Statistics follow the reference: sum of squares accumulated in double
 * (src/aria_cpu.c:57-98), inv = (float)(1.0/sqrt(ss/dim + eps)), then the
 * per-element products in float with separate roundings. LayerNorm (which has
 * no reference op) keeps mean, variance and (x-mean)*rstd in double.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

struct NormArgs {
    void *y;
    const float *x, *w, *b, *scale, *shift;
    int rows_per_batch, rows, dim;
    float eps;
    int gelu, resid, f16;
};

template <int NORM>
__device__ __forceinline__ float norm_elem(float xv, float inv, double mu, double rstd, const float *w,
                                           const float *b, int c) {
    float n;
    if (NORM == ARIA_NORM_LAYER) {
        n = (float)(((double)xv - mu) * rstd);
        if (w) n = n * w[c];
        if (b) n = n + b[c];
    } else if (NORM == ARIA_NORM_GEMMA) {
        n = (xv * inv) * (1.0f + w[c]);
    } else {
        n = xv * inv;
        if (w) n = n * w[c];
    }
    return n;
}

__device__ __forceinline__ float epilogue(float n, float xv, const NormArgs &a, const float *sc,
                                          const float *sh, int c) {
    if (sc) {
        float t = 1.0f + sc[c];
        n = n * t;
        n = n + sh[c];
    }
    if (a.gelu) n = gelu_tanh_f(n);
    if (a.resid) n = n + xv;
    return n;
}

/* register-resident fast path: dim == VPL * 4 * LPR */
template <int NORM, int VPL, int LPR>
__global__ __launch_bounds__(256) void k_rownorm_v(NormArgs a) {
    constexpr int RPW = ARIA_WAVE / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * 4 + wave) * RPW + lane / LPR;
    const int l = lane % LPR;
    if (row >= a.rows) return;   /* whole LPR-lane groups leave together */
    const int dim = a.dim;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x + (size_t)row * dim);
    float4 v[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) v[j] = x4[j * LPR + l];

    float inv = 0.0f;
    double mu = 0.0, rstd = 0.0;
    if (NORM == ARIA_NORM_LAYER) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < VPL; j++)
            s += ((double)v[j].x + (double)v[j].y) + ((double)v[j].z + (double)v[j].w);
        s = grp_sum<LPR>(s);
        mu = s / dim;
        double q = 0.0;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            double d0 = (double)v[j].x - mu, d1 = (double)v[j].y - mu;
            double d2 = (double)v[j].z - mu, d3 = (double)v[j].w - mu;
            q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        q = grp_sum<LPR>(q);
        rstd = 1.0 / sqrt(q / dim + (double)a.eps);
    } else {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            double x0 = v[j].x, x1 = v[j].y, x2 = v[j].z, x3 = v[j].w;
            s += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
        }
        s = grp_sum<LPR>(s);
        inv = (float)(1.0 / sqrt(s / dim + (double)a.eps));
    }

    const float *sc = nullptr, *sh = nullptr;
    if (a.scale) {
        int bt = row / a.rows_per_batch;
        sc = a.scale + (size_t)bt * dim;
        sh = a.shift + (size_t)bt * dim;
    }
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const int c0 = 4 * (j * LPR + l);
        float4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float xv = f4get(v[j], e);
            float n = norm_elem<NORM>(xv, inv, mu, rstd, a.w, a.b, c0 + e);
            f4set(o, e, epilogue(n, xv, a, sc, sh, c0 + e));
        }
        if (a.f16) {
            uint2 p;
            p.x = (uint32_t)f2h_bits(o.x) | ((uint32_t)f2h_bits(o.y) << 16);
            p.y = (uint32_t)f2h_bits(o.z) | ((uint32_t)f2h_bits(o.w) << 16);
            reinterpret_cast<uint2 *>((uint16_t *)a.y + (size_t)row * dim)[j * LPR + l] = p;
        } else {
            reinterpret_cast<float4 *>((float *)a.y + (size_t)row * dim)[j * LPR + l] = o;
        }
    }
}

/* generic path: any dim, one wave per row, the row is re-read from L1/L2 */
template <int NORM>
__global__ __launch_bounds__(256) void k_rownorm_g(NormArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int dim = a.dim;
    const float *xr = a.x + (size_t)row * dim;
    float inv = 0.0f;
    double mu = 0.0, rstd = 0.0;
    if (NORM == ARIA_NORM_LAYER) {
        double s = 0.0;
        for (int c = lane; c < dim; c += 64) s += (double)xr[c];
        s = grp_sum<64>(s);
        mu = s / dim;
        double q = 0.0;
        for (int c = lane; c < dim; c += 64) { double d = (double)xr[c] - mu; q += d * d; }
        q = grp_sum<64>(q);
        rstd = 1.0 / sqrt(q / dim + (double)a.eps);
    } else {
        double s = 0.0;
        for (int c = lane; c < dim; c += 64) s += (double)xr[c] * (double)xr[c];
        s = grp_sum<64>(s);
        inv = (float)(1.0 / sqrt(s / dim + (double)a.eps));
    }
    const float *sc = nullptr, *sh = nullptr;
    if (a.scale) {
        int bt = row / a.rows_per_batch;
        sc = a.scale + (size_t)bt * dim;
        sh = a.shift + (size_t)bt * dim;
    }
    for (int c = lane; c < dim; c += 64) {
        float xv = xr[c];
        float n = epilogue(norm_elem<NORM>(xv, inv, mu, rstd, a.w, a.b, c), xv, a, sc, sh, c);
        if (a.f16) ((uint16_t *)a.y)[(size_t)row * dim + c] = f2h_bits(n);
        else ((float *)a.y)[(size_t)row * dim + c] = n;
    }
}

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

template <int NORM>
static hipError_t launch_norm(const NormArgs &a, hipStream_t s) {
    const int dim = a.dim;
    bool vec = (dim % 4 == 0) && al16(a.x) && (a.f16 ? ((uintptr_t)a.y & 7u) == 0 : al16(a.y)) &&
               (!a.w || al16(a.w)) && (!a.b || al16(a.b)) && (!a.scale || al16(a.scale)) &&
               (!a.shift || al16(a.shift));
    dim3 blk(256);
    auto grid_for = [&](int rows_per_wave) { return dim3((a.rows + 4 * rows_per_wave - 1) / (4 * rows_per_wave)); };
    if (vec && dim == 64) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 1, 16>), grid_for(4), blk, 0, s, a);
    } else if (vec && dim == 128) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 1, 32>), grid_for(2), blk, 0, s, a);
    } else if (vec && dim == 256) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 1, 64>), grid_for(1), blk, 0, s, a);
    } else if (vec && dim == 512) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 2, 64>), grid_for(1), blk, 0, s, a);
    } else if (vec && dim == 768) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 3, 64>), grid_for(1), blk, 0, s, a);
    } else if (vec && dim == 1024) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 4, 64>), grid_for(1), blk, 0, s, a);
    } else if (vec && dim == 2048) {
        hipLaunchKernelGGL((k_rownorm_v<NORM, 8, 64>), grid_for(1), blk, 0, s, a);
    } else {
        hipLaunchKernelGGL((k_rownorm_g<NORM>), grid_for(1), blk, 0, s, a);
    }
    return hipGetLastError();
}

extern "C" hipError_t aria_k_rownorm(void *y, int out_f16, const float *x, const float *w,
                                     const float *b, const float *scale, const float *shift,
                                     int rows_per_batch, int gelu, int resid, int norm, int rows,
                                     int dim, float eps, hipStream_t s) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    NormArgs a;
    a.y = y; a.x = x; a.w = w; a.b = b; a.scale = scale; a.shift = shift;
    a.rows_per_batch = rows_per_batch > 0 ? rows_per_batch : rows;
    a.rows = rows; a.dim = dim; a.eps = eps;
    a.gelu = gelu; a.resid = resid; a.f16 = out_f16;
    switch (norm) {
        case ARIA_NORM_GEMMA: return launch_norm<ARIA_NORM_GEMMA>(a, s);
        case ARIA_NORM_LAYER: return launch_norm<ARIA_NORM_LAYER>(a, s);
        default: return launch_norm<ARIA_NORM_RMS>(a, s);
    }
}
