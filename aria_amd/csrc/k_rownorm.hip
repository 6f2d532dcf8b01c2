/*
 * k_rownorm.hip - row normalisations with a fused epilogue, one HBM pass.
 *
 * Replaces the reference's aria_rmsnorm / aria_gemma_rmsnorm (src/aria_cpu.c:643-733),
 * the DiT's rmsnorm + adaln_modulate pair (src/aria_sa3_dit.c:71-82, 175-176,
 * 255-256) and the config chain LayerNorm -> modulate -> tanh-GELU -> + x.
 *
 * Mapping: a row is owned by LPR lanes of one wave64 (LPR = 64 for dim >= 256,
 * 16/32 for the 64/128-wide q/k-norm rows). Each lane loads VPL float4 (128-bit,
 * coalesced: lane l reads vectors l, l+LPR, ...), keeps them in registers,
 * reduces the statistic in double across its LPR lanes (DPP butterfly, no LDS,
 * no barrier) and writes the transformed row once: HBM traffic = read x + write y.
 * Broadcast vectors (w, b, scale, shift) are read as float4 at the same column.
 *
 * RMS statistics follow the reference: sum of squares accumulated in double
 * (src/aria_cpu.c:57-98), inv = (float)(1.0/sqrt(ss/dim + eps)), then the
 * per-element products in float with separate roundings, so the output matches
 * the reference nearly bit for bit. LayerNorm (which has no reference op) is two
 * fp32 passes over the registers: mean = sum/dim, then the centred sum of squares
 * (fma), rstd = v_rsq_f32(var + eps), y = (x - mean)*rstd. Against a double
 * statistic this differs by ~1e-7 relative; the double form cost ~10 VALU per
 * element (conversions, fp64 DPP reductions, divide and sqrt), which at 2.5 waves
 * per SIMD is about 0.6 us of issue time per launch at [2592, 1024].
 *
 * The register path is compiled per operand set (EPI mask): gain, bias, modulate,
 * second modulation term, GELU, residual, half output. With these as run-time
 * flags the optional operands cost a select and a zero fill per element (~110 of
 * the fused chain's VALU); launch_norm instantiates the combinations the callers
 * use and sends any other to the generic kernel.
 */
#include <utility>
#include "aria_dev.h"
#include "aria_hip_kernels.h"

/* EPI_NT: the row is loaded and stored with non-temporal hints (the standalone ops, whose
 * operands are streamed once; the DiT's norms feed the next GEMM and keep the default) */
enum { EPI_MOD = 1, EPI_GELU = 2, EPI_RES = 4, EPI_F16 = 8, EPI_W = 16, EPI_B = 32, EPI_MADD = 64, EPI_Q8 = 128,
       EPI_NT = 256 };

struct NormArgs {
    void *y;
    const float *x, *w, *b, *scale, *shift;
    /* modulation = scale[bt * mod_bs + c] (+ scale_add[bt * add_bs + c]), shift likewise:
     * the DiT passes the block's to_scale_shift_gate chunk (batch stride 0) plus the
     * per-request gcond chunk, so the sum is formed here instead of in a separate pass */
    const float *scale_add, *shift_add;
    int mod_bs, add_bs;
    int rows_per_batch, rows, dim;
    float eps;
    int gelu, resid, f16;
    float *sx;   /* EPI_Q8: y is int8 [rows, dim] and sx[row] its scale (W8A8 activations) */
    int nt;      /* EPI_NT */
};

template <int NORM>
__device__ __forceinline__ float norm_elem(float xv, float inv, float mu, float rstd, bool hw, float w,
                                           bool hb, float b) {
    float n;
    if (NORM == ARIA_NORM_LAYER) {
        n = (xv - mu) * rstd;
        if (hw) n = n * w;
        if (hb) n = n + b;
    } else if (NORM == ARIA_NORM_GEMMA) {
        n = (xv * inv) * (1.0f + w);
    } else {
        n = xv * inv;
        if (hw) n = n * w;
    }
    return n;
}

template <int NORM, int EPI>
__device__ __forceinline__ float norm_elem_c(float xv, float inv, float mu, float rstd, float w, float b) {
    float n;
    if (NORM == ARIA_NORM_LAYER) {
        n = (xv - mu) * rstd;
        if (EPI & EPI_W) n = n * w;
        if (EPI & EPI_B) n = n + b;
    } else if (NORM == ARIA_NORM_GEMMA) {
        n = xv * inv;
        if (EPI & EPI_W) n = n * (1.0f + w);
    } else {
        n = xv * inv;
        if (EPI & EPI_W) n = n * w;
    }
    return n;
}

/* t1 = 1 + scale, formed once per column with the broadcast vectors (the same fp32 add) */
template <int EPI>
__device__ __forceinline__ float epi_elem(float n, float xv, float t1, float sh) {
    if (EPI & EPI_MOD) {
        n = n * t1;
        n = n + sh;
    }
    if (EPI & EPI_GELU) n = gelu_tanh_f(n);
    if (EPI & EPI_RES) n = n + xv;
    return n;
}

/* register-resident fast path: dim == VPL * 4 * LPR.
 * With a full wave per row (LPR = 64) and any broadcast vector (gain, bias, scale, shift),
 * the workgroup's four rows share them (RMSNorm with its gain alone: 5.30 -> 5.14 us at
 * [2592, 1024]): the 256 lanes load each vector once into LDS
 * (forming 1 + (scale + scale_add) and shift + shift_add there, once), and every wave reads its lanes'
 * parts back from LDS. Per row that replaces 4-20 KB of L1 requests by one LDS read of the same
 * bytes (a CU reads 3x more per clock from LDS than from L1). A workgroup whose rows straddle
 * two batches of the modulation loads per lane as before. */
template <int NORM, int VPL, int LPR, int EPI>
__global__ __launch_bounds__(256) void k_rownorm_v(NormArgs a) {
    constexpr int RPW = ARIA_WAVE / LPR;
    constexpr int NVEC = ((EPI & EPI_W) ? 1 : 0) + ((EPI & EPI_B) ? 1 : 0) + ((EPI & EPI_MOD) ? 2 : 0);
    constexpr bool SHARE = LPR == 64 && NVEC >= 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * RPW + lane / LPR;
    const int l = lane % LPR;
    if (!SHARE && row0 >= a.rows) return;   /* whole LPR-lane groups leave together */
    /* SHARE: every wave stays to the barrier; a row past the end re-reads the last row and
     * stores nothing */
    const bool live = row0 < a.rows;
    const int row = live ? row0 : a.rows - 1;
    const int dim = a.dim;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x + (size_t)row * dim);
    float4 v[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) v[j] = (EPI & EPI_NT) ? ld_nt(x4 + j * LPR + l) : x4[j * LPR + l];

    /* the broadcast vectors are loaded with the row, before the reduction, so their
     * latency overlaps the row's instead of following it */
    const float4 *w4 = reinterpret_cast<const float4 *>(a.w);
    const float4 *b4 = reinterpret_cast<const float4 *>(a.b);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 wv[VPL], bv[VPL], scv[VPL], shv[VPL];
    /* the vectors of batch bt at float4 column c4; sc returns the modulation factor 1 + scale */
    auto vecs_at = [&](int bt, int c4, float4 &w, float4 &b, float4 &sc, float4 &sh) __attribute__((always_inline)) {
        w = (EPI & EPI_W) ? w4[c4] : z4;
        b = (EPI & EPI_B) ? b4[c4] : z4;
        sc = z4; sh = z4;
        if (EPI & EPI_MOD) {
            sc = reinterpret_cast<const float4 *>(a.scale + (size_t)bt * a.mod_bs)[c4];
            sh = reinterpret_cast<const float4 *>(a.shift + (size_t)bt * a.mod_bs)[c4];
            if (EPI & EPI_MADD) {
                const float4 sa = reinterpret_cast<const float4 *>(a.scale_add + (size_t)bt * a.add_bs)[c4];
                const float4 ha = reinterpret_cast<const float4 *>(a.shift_add + (size_t)bt * a.add_bs)[c4];
                sc = make_float4(sc.x + sa.x, sc.y + sa.y, sc.z + sa.z, sc.w + sa.w);
                sh = make_float4(sh.x + ha.x, sh.y + ha.y, sh.z + ha.z, sh.w + ha.w);
            }
            sc = make_float4(1.0f + sc.x, 1.0f + sc.y, 1.0f + sc.z, 1.0f + sc.w);   /* the 1 + scale factor */
        }
    };
    bool shared_done = false;
    if constexpr (SHARE) {
        /* one batch for the whole workgroup? (uniform per workgroup) */
        const int rf = blockIdx.x * 4, rl = min(rf + 3, a.rows - 1);
        const bool one = !(EPI & EPI_MOD) || rf / a.rows_per_batch == rl / a.rows_per_batch;
        if (one) {
            __shared__ float4 sv[4][VPL * 64];
            const int bt = rf / a.rows_per_batch;
            for (int c4 = threadIdx.x; c4 < VPL * 64; c4 += 256) {
                float4 w, b, sc, sh;
                vecs_at(bt, c4, w, b, sc, sh);
                sv[0][c4] = w; sv[1][c4] = b; sv[2][c4] = sc; sv[3][c4] = sh;
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < VPL; j++) {
                const int c4 = j * 64 + l;
                wv[j] = (EPI & EPI_W) ? sv[0][c4] : z4;
                bv[j] = (EPI & EPI_B) ? sv[1][c4] : z4;
                scv[j] = (EPI & EPI_MOD) ? sv[2][c4] : z4;
                shv[j] = (EPI & EPI_MOD) ? sv[3][c4] : z4;
            }
            shared_done = true;
        }
    }
    if (!shared_done) {
        const int bt = (EPI & EPI_MOD) ? row / a.rows_per_batch : 0;
#pragma unroll
        for (int j = 0; j < VPL; j++) vecs_at(bt, j * LPR + l, wv[j], bv[j], scv[j], shv[j]);
    }

    float inv = 0.0f, mu = 0.0f, rstd = 0.0f;
    if (NORM == ARIA_NORM_LAYER) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; j++) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
        s = grp_sum<LPR>(s);
        mu = s / (float)dim;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const float d0 = v[j].x - mu, d1 = v[j].y - mu, d2 = v[j].z - mu, d3 = v[j].w - mu;
            q = __builtin_fmaf(d0, d0, q); q = __builtin_fmaf(d1, d1, q);
            q = __builtin_fmaf(d2, d2, q); q = __builtin_fmaf(d3, d3, q);
        }
        q = grp_sum<LPR>(q);
        rstd = __builtin_amdgcn_rsqf(q / (float)dim + a.eps);
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

    if constexpr ((EPI & EPI_Q8) != 0) {
        /* W8A8: the fp32 row stays in registers, its absolute maximum is reduced across
         * the row's lanes, and the row is written as int8 with sx = amax / 127 (the
         * reference quantises the fp32 producer output the same way, src/aria_quant.c:258-270) */
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            v[j].x = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].x, inv, mu, rstd, wv[j].x, bv[j].x), v[j].x, scv[j].x, shv[j].x);
            v[j].y = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].y, inv, mu, rstd, wv[j].y, bv[j].y), v[j].y, scv[j].y, shv[j].y);
            v[j].z = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].z, inv, mu, rstd, wv[j].z, bv[j].z), v[j].z, scv[j].z, shv[j].z);
            v[j].w = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].w, inv, mu, rstd, wv[j].w, bv[j].w), v[j].w, scv[j].w, shv[j].w);
            mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
        }
        mx = grp_max<LPR>(mx);
        if (!live) return;
        const float qinv = mx > 0.0f ? 127.0f / mx : 0.0f;
        uint32_t *yq = reinterpret_cast<uint32_t *>((int8_t *)a.y + (size_t)row * dim);
#pragma unroll
        for (int j = 0; j < VPL; j++) yq[j * LPR + l] = q8_pack4(v[j], qinv);
        if (l == 0) a.sx[row] = mx / 127.0f;
        return;
    }
    if (!live) return;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const int c4 = j * LPR + l;
        float4 o;
        o.x = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].x, inv, mu, rstd, wv[j].x, bv[j].x), v[j].x, scv[j].x, shv[j].x);
        o.y = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].y, inv, mu, rstd, wv[j].y, bv[j].y), v[j].y, scv[j].y, shv[j].y);
        o.z = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].z, inv, mu, rstd, wv[j].z, bv[j].z), v[j].z, scv[j].z, shv[j].z);
        o.w = epi_elem<EPI>(norm_elem_c<NORM, EPI>(v[j].w, inv, mu, rstd, wv[j].w, bv[j].w), v[j].w, scv[j].w, shv[j].w);
        if (EPI & EPI_F16) {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            const u32x2_t p = {(uint32_t)f2h_bits(o.x) | ((uint32_t)f2h_bits(o.y) << 16),
                               (uint32_t)f2h_bits(o.z) | ((uint32_t)f2h_bits(o.w) << 16)};
            u32x2_t *yp = reinterpret_cast<u32x2_t *>((uint16_t *)a.y + (size_t)row * dim) + c4;
            if (EPI & EPI_NT) __builtin_nontemporal_store(p, yp);
            else *yp = p;
        } else if (EPI & EPI_NT) {
            st_nt(reinterpret_cast<float4 *>((float *)a.y + (size_t)row * dim) + c4, o);
        } else {
            reinterpret_cast<float4 *>((float *)a.y + (size_t)row * dim)[c4] = o;
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
    float inv = 0.0f, mu = 0.0f, rstd = 0.0f;
    if (NORM == ARIA_NORM_LAYER) {
        float s = 0.0f;
        for (int c = lane; c < dim; c += 64) s += xr[c];
        s = grp_sum<64>(s);
        mu = s / (float)dim;
        float q = 0.0f;
        for (int c = lane; c < dim; c += 64) { const float d = xr[c] - mu; q = __builtin_fmaf(d, d, q); }
        q = grp_sum<64>(q);
        rstd = __builtin_amdgcn_rsqf(q / (float)dim + a.eps);
    } else {
        double s = 0.0;
        for (int c = lane; c < dim; c += 64) s += (double)xr[c] * (double)xr[c];
        s = grp_sum<64>(s);
        inv = (float)(1.0 / sqrt(s / dim + (double)a.eps));
    }
    const float *sc = nullptr, *sh = nullptr;
    const float *sca = nullptr, *sha = nullptr;
    if (a.scale) {
        int bt = row / a.rows_per_batch;
        sc = a.scale + (size_t)bt * a.mod_bs;
        sh = a.shift + (size_t)bt * a.mod_bs;
        if (a.scale_add) {
            sca = a.scale_add + (size_t)bt * a.add_bs;
            sha = a.shift_add + (size_t)bt * a.add_bs;
        }
    }
    const bool hw = a.w != nullptr, hb = a.b != nullptr;
    for (int c = lane; c < dim; c += 64) {
        float xv = xr[c];
        float n = norm_elem<NORM>(xv, inv, mu, rstd, hw, hw ? a.w[c] : 0.0f, hb, hb ? a.b[c] : 0.0f);
        if (sc) {
            const float scv = sca ? sc[c] + sca[c] : sc[c], shv = sha ? sh[c] + sha[c] : sh[c];
            float t = 1.0f + scv; n = n * t; n = n + shv;
        }
        if (a.gelu) n = gelu_tanh_f(n);
        if (a.resid) n = n + xv;
        if (a.f16) ((uint16_t *)a.y)[(size_t)row * dim + c] = f2h_bits(n);
        else ((float *)a.y)[(size_t)row * dim + c] = n;
    }
}

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* the operand sets instantiated for the register path, per norm */
using EpiRms = std::integer_sequence<int, 0, EPI_W, EPI_W | EPI_NT, EPI_F16, EPI_F16 | EPI_W, EPI_MOD | EPI_W, EPI_MOD | EPI_F16 | EPI_W,
                                      EPI_MOD | EPI_MADD | EPI_W, EPI_MOD | EPI_MADD | EPI_F16 | EPI_W,
                                      EPI_Q8, EPI_Q8 | EPI_W, EPI_MOD | EPI_Q8, EPI_MOD | EPI_Q8 | EPI_W,
                                      EPI_MOD | EPI_MADD | EPI_Q8 | EPI_W>;
using EpiGemma = std::integer_sequence<int, 0, EPI_W>;
using EpiLayer = std::integer_sequence<int, 0, EPI_NT, EPI_W, EPI_B, EPI_W | EPI_B, EPI_W | EPI_B | EPI_NT,
                                        EPI_MOD | EPI_GELU | EPI_RES, EPI_MOD | EPI_GELU | EPI_RES | EPI_W | EPI_B,
                                        EPI_MOD | EPI_GELU | EPI_RES | EPI_W | EPI_B | EPI_NT>;
template <int NORM> struct EpiSet;
template <> struct EpiSet<ARIA_NORM_RMS> { using type = EpiRms; };
template <> struct EpiSet<ARIA_NORM_GEMMA> { using type = EpiGemma; };
template <> struct EpiSet<ARIA_NORM_LAYER> { using type = EpiLayer; };

template <int NORM, int VPL, int LPR, int E>
static bool launch_v1(const NormArgs &a, int epi, hipStream_t s) {
    if (epi != E) return false;
    constexpr int RPW = ARIA_WAVE / LPR;
    hipLaunchKernelGGL((k_rownorm_v<NORM, VPL, LPR, E>), dim3((a.rows + 4 * RPW - 1) / (4 * RPW)), dim3(256), 0, s, a);
    return true;
}

/* launches k_rownorm_v<NORM, VPL, LPR, epi> if epi is in the set; false otherwise */
template <int NORM, int VPL, int LPR, int... E>
static bool launch_v(const NormArgs &a, int epi, hipStream_t s, std::integer_sequence<int, E...>) {
    return (launch_v1<NORM, VPL, LPR, E>(a, epi, s) || ...);
}

template <int NORM>
static hipError_t launch_norm(const NormArgs &a, hipStream_t s) {
    const int dim = a.dim;
    /* y alignment per output form: fp32 float4 stores (16 B), fp16 (8 B), int8 (one uint32 of
     * four values per lane: 4 B) */
    const bool yal = a.sx ? ((uintptr_t)a.y & 3u) == 0 : a.f16 ? ((uintptr_t)a.y & 7u) == 0 : al16(a.y);
    const bool vec = (dim % 4 == 0) && al16(a.x) && yal &&
                     (!a.w || al16(a.w)) && (!a.b || al16(a.b)) && (!a.scale || al16(a.scale)) &&
                     (!a.shift || al16(a.shift)) && (!a.scale_add || al16(a.scale_add)) &&
                     (!a.shift_add || al16(a.shift_add)) && a.mod_bs % 4 == 0 && a.add_bs % 4 == 0;
    const int epi = (a.scale ? EPI_MOD : 0) | (a.gelu ? EPI_GELU : 0) | (a.resid ? EPI_RES : 0) |
                    (a.f16 ? EPI_F16 : 0) | (a.w ? EPI_W : 0) | (a.b ? EPI_B : 0) |
                    (a.scale && a.scale_add ? EPI_MADD : 0) | (a.sx ? EPI_Q8 : 0) | (a.nt ? EPI_NT : 0);
    using Set = typename EpiSet<NORM>::type;
    bool hit = false;
    if (vec) {
        switch (dim) {
            case 64: hit = launch_v<NORM, 1, 16>(a, epi, s, Set{}); break;
            case 128: hit = launch_v<NORM, 1, 32>(a, epi, s, Set{}); break;
            case 256: hit = launch_v<NORM, 1, 64>(a, epi, s, Set{}); break;
            case 512: hit = launch_v<NORM, 2, 64>(a, epi, s, Set{}); break;
            case 768: hit = launch_v<NORM, 3, 64>(a, epi, s, Set{}); break;
            case 1024: hit = launch_v<NORM, 4, 64>(a, epi, s, Set{}); break;
            case 2048: hit = launch_v<NORM, 8, 64>(a, epi, s, Set{}); break;
            default: break;
        }
    }
    if (!hit && vec && (epi & EPI_NT)) {   /* no streaming form of this operand set: the default one */
        const int e2 = epi & ~EPI_NT;
        switch (dim) {
            case 64: hit = launch_v<NORM, 1, 16>(a, e2, s, Set{}); break;
            case 128: hit = launch_v<NORM, 1, 32>(a, e2, s, Set{}); break;
            case 256: hit = launch_v<NORM, 1, 64>(a, e2, s, Set{}); break;
            case 512: hit = launch_v<NORM, 2, 64>(a, e2, s, Set{}); break;
            case 768: hit = launch_v<NORM, 3, 64>(a, e2, s, Set{}); break;
            case 1024: hit = launch_v<NORM, 4, 64>(a, e2, s, Set{}); break;
            case 2048: hit = launch_v<NORM, 8, 64>(a, e2, s, Set{}); break;
            default: break;
        }
    }
    if (!hit) {
        if (a.sx) return hipErrorInvalidValue;   /* int8 output: register path only */
        hipLaunchKernelGGL((k_rownorm_g<NORM>), dim3((a.rows + 3) / 4), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

extern "C" hipError_t aria_k_rownorm(void *y, int out_f16, const float *x, const float *w,
                                     const float *b, const float *scale, const float *shift,
                                     int rows_per_batch, int gelu, int resid, int norm, int rows,
                                     int dim, float eps, hipStream_t s) {
    return aria_k_rownorm_nt(y, out_f16, x, w, b, scale, shift, rows_per_batch, gelu, resid, norm, rows, dim, eps, 0, s);
}

extern "C" hipError_t aria_k_rownorm_nt(void *y, int out_f16, const float *x, const float *w,
                                        const float *b, const float *scale, const float *shift,
                                        int rows_per_batch, int gelu, int resid, int norm, int rows,
                                        int dim, float eps, int nt, hipStream_t s) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    NormArgs a;
    a.nt = nt;
    a.y = y; a.x = x; a.w = w; a.b = b; a.scale = scale; a.shift = shift;
    a.scale_add = nullptr; a.shift_add = nullptr; a.mod_bs = dim; a.add_bs = 0;
    a.rows_per_batch = rows_per_batch > 0 ? rows_per_batch : rows;
    a.rows = rows; a.dim = dim; a.eps = eps;
    a.gelu = gelu; a.resid = resid; a.f16 = out_f16; a.sx = nullptr;
    switch (norm) {
        case ARIA_NORM_GEMMA: return launch_norm<ARIA_NORM_GEMMA>(a, s);
        case ARIA_NORM_LAYER: return launch_norm<ARIA_NORM_LAYER>(a, s);
        default: return launch_norm<ARIA_NORM_RMS>(a, s);
    }
}

/* RMSNorm + adaLN modulate with the modulation formed in place: scale = scale_t[c] +
 * scale_g[b * g_bs + c] (scale_g NULL: scale_t alone), shift likewise; the result in fp16
 * or fp32. The DiT passes its to_scale_shift_gate chunks (scale_t, shift_t) and the
 * request's gcond chunks (batch stride 6 * dim). */
extern "C" hipError_t aria_k_rownorm_ada(void *y, int out_f16, const float *x, const float *w,
                                         const float *scale_t, const float *shift_t, const float *scale_g,
                                         const float *shift_g, int g_bs, int rows_per_batch, int rows,
                                         int dim, float eps, hipStream_t s) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    NormArgs a;
    a.y = y; a.x = x; a.w = w; a.b = nullptr; a.scale = scale_t; a.shift = shift_t;
    a.scale_add = scale_g; a.shift_add = shift_g; a.mod_bs = 0; a.add_bs = g_bs;
    a.rows_per_batch = rows_per_batch > 0 ? rows_per_batch : rows;
    a.rows = rows; a.dim = dim; a.eps = eps;
    a.gelu = 0; a.resid = 0; a.f16 = out_f16; a.sx = nullptr; a.nt = 0;
    return launch_norm<ARIA_NORM_RMS>(a, s);
}

/* The two RMS forms with W8A8 output: yq int8 [rows, dim] and sx [rows], the quantisation
 * of the fp32 result (dim 256..2048 in steps the register path takes). aria_k_rownorm_q8
 * takes scale / shift per batch ([rows / rows_per_batch, dim], both NULL for a plain norm). */
extern "C" hipError_t aria_k_rownorm_q8(int8_t *yq, float *sx, const float *x, const float *w, const float *scale,
                                        const float *shift, int rows_per_batch, int rows, int dim, float eps,
                                        hipStream_t s) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    NormArgs a;
    a.y = yq; a.x = x; a.w = w; a.b = nullptr; a.scale = scale; a.shift = shift;
    a.scale_add = nullptr; a.shift_add = nullptr; a.mod_bs = dim; a.add_bs = 0;
    a.rows_per_batch = rows_per_batch > 0 ? rows_per_batch : rows; a.rows = rows; a.dim = dim; a.eps = eps;
    a.gelu = 0; a.resid = 0; a.f16 = 0; a.sx = sx; a.nt = 0;
    if (!sx || ((uintptr_t)yq & 3u)) return hipErrorInvalidValue;
    return launch_norm<ARIA_NORM_RMS>(a, s);
}
extern "C" hipError_t aria_k_rownorm_ada_q8(int8_t *yq, float *sx, const float *x, const float *w,
                                            const float *scale_t, const float *shift_t, const float *scale_g,
                                            const float *shift_g, int g_bs, int rows_per_batch, int rows, int dim,
                                            float eps, hipStream_t s) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    NormArgs a;
    a.y = yq; a.x = x; a.w = w; a.b = nullptr; a.scale = scale_t; a.shift = shift_t;
    a.scale_add = scale_g; a.shift_add = shift_g; a.mod_bs = 0; a.add_bs = g_bs;
    a.rows_per_batch = rows_per_batch > 0 ? rows_per_batch : rows;
    a.rows = rows; a.dim = dim; a.eps = eps;
    a.gelu = 0; a.resid = 0; a.f16 = 0; a.sx = sx; a.nt = 0;
    if (!sx || ((uintptr_t)yq & 3u)) return hipErrorInvalidValue;
    return launch_norm<ARIA_NORM_RMS>(a, s);
}
