/*
 * k_qgemm.hip - dequantize-on-use GEMM on gfx950 MFMA:  y[M,N] = x[M,K] W[N,K]^T (+ b)
 *
 * Replaces the reference's aria_linear_q8 / aria_linear_q4 (src/aria_quant.c:98-145,
 * 469-538) and its device path (k_dequant_q8/q4 into an fp16 scratch copy of W, then
 * cublasGemmEx, src/aria_cuda.cu:1009-1035). Here the packed weights never leave
 * their quantized layout in HBM: each workgroup fetches 32-wide K slices of its
 * weight rows still packed, unpacks them in registers, and writes fp16 into LDS for
 * the MFMA.
 *
 *   Q8 (per-row symmetric): the int8 values are exact in fp16; the row scale is
 *       applied once in the epilogue, y = acc * scale[n] (+ b[n]), the reference's
 *       order (src/aria_quant.c:141).
 *   Q4 (per-32-block asymmetric): a 32-wide slice is exactly one quantization block,
 *       so each row needs one [min, step] pair per slice; the weight is rebuilt as
 *       min + nib*step in fp32 (the reference's dequant value, src/aria_cuda.cu:825-835)
 *       and rounded to fp16.
 *   F16: fp16 weights (the unquantized projections of the DiT, e.g. ca_to_kv).
 * Activations are fp32 (rounded to fp16 when staged) or already fp16 (emitted by the
 * fused norm kernels). Accumulation is fp32 in the MFMA accumulators. Error budget vs
 * the reference's fp32 dequantized GEMM: activation (and Q4 weight) rounding to fp16,
 * ~2^-11 relative per product, a few 1e-4 of max|y|.
 *
 * Tiling: 256 threads = 4 waves in a 2x2 grid; each wave owns TMW x TNW tiles of 32x32
 * computed with v_mfma_f32_32x32x16_f16 (two MFMAs per 32-wide K slice). Workgroup tile
 * BM = 64*TMW by BN = 64*TNW, picked per shape so the grid fills the 256 CUs evenly.
 * Pipeline: a ring of three register stages holds raw (still packed) slices; the
 * global loads of slice k+3 are issued while slice k is multiplied out of LDS, so each
 * load has two slice-times to land; a slice is unpacked to fp16 only when it is stored
 * to the LDS double buffer (one barrier per slice).
 * Operand layout of the 32x32x16 MFMA: lane l supplies row (l % 32) and the 8
 * consecutive k at 8*(l / 32); accumulator register r of lane l holds row
 * 8*(r/4) + 4*(l/32) + r%4, column l % 32.
 *
 * Shapes with K % 32 != 0 or unaligned operands take a SIMT fp32 kernel with the same
 * dequant values (k_qgemm_simt).
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct QArgs {
    void *y;
    const void *x;
    const void *q;
    const float *scale;
    const float *bias;
    int M, K, N;
    int y_f16;
    int nblk;
    int gelu;   /* epilogue: y = gelu_tanh(acc*scale + b) (the config FFN's activation) */
};

#define BK 32
#define LDS_STRIDE (BK + 8)   /* halves per LDS row: 80 B, conflict-free 16 B fragment reads */

__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    return (uint32_t)f2h_bits(a) | ((uint32_t)f2h_bits(b) << 16);
}

/* raw register words per 16-element chunk */
template <bool AF16> struct RawA { static constexpr int W = AF16 ? 8 : 16; };
template <int WT> struct RawB { static constexpr int W = (WT == ARIA_WQ8 || WT == ARIA_WQ4) ? 4 : 8; };

/* ---- global -> raw registers (no arithmetic, so the loads stay in flight) ---- */
template <bool AF16>
__device__ __forceinline__ void ld_a(uint32_t *r, const QArgs &a, int m, int k) {
    constexpr int W = RawA<AF16>::W;
    if (m >= a.M) {
#pragma unroll
        for (int i = 0; i < W; i++) r[i] = 0u;
        return;
    }
    const uint4 *p = AF16 ? reinterpret_cast<const uint4 *>((const uint16_t *)a.x + (size_t)m * a.K + k)
                          : reinterpret_cast<const uint4 *>((const float *)a.x + (size_t)m * a.K + k);
#pragma unroll
    for (int j = 0; j < W / 4; j++) {
        const uint4 u = p[j];
        r[4 * j] = u.x; r[4 * j + 1] = u.y; r[4 * j + 2] = u.z; r[4 * j + 3] = u.w;
    }
}

template <int WT>
__device__ __forceinline__ void ld_b(uint32_t *r, const QArgs &a, int n, int k) {
    constexpr int W = RawB<WT>::W;
    if (n >= a.N) {
#pragma unroll
        for (int i = 0; i < W; i++) r[i] = 0u;
        return;
    }
    if (WT == ARIA_WQ8) {
        const uint4 u = *reinterpret_cast<const uint4 *>((const int8_t *)a.q + (size_t)n * a.K + k);
        r[0] = u.x; r[1] = u.y; r[2] = u.z; r[3] = u.w;
    } else if (WT == ARIA_WQ4) {
        const uint2 u = *reinterpret_cast<const uint2 *>((const uint8_t *)a.q + (size_t)n * (a.K >> 1) + (k >> 1));
        const uint2 pr = *reinterpret_cast<const uint2 *>(a.scale + ((size_t)n * a.nblk + (k >> 5)) * 2);
        r[0] = u.x; r[1] = u.y; r[2] = pr.x; r[3] = pr.y;
    } else {
        const uint4 *p = reinterpret_cast<const uint4 *>((const uint16_t *)a.q + (size_t)n * a.K + k);
        const uint4 u0 = p[0], u1 = p[1];
        r[0] = u0.x; r[1] = u0.y; r[2] = u0.z; r[3] = u0.w;
        r[4] = u1.x; r[5] = u1.y; r[6] = u1.z; r[7] = u1.w;
    }
}

/* ---- raw registers -> 16 halves in LDS ---- */
__device__ __forceinline__ void st_lds8(uint16_t *dst, const uint32_t (&o)[8]) {
    uint4 *d = reinterpret_cast<uint4 *>(dst);
    d[0] = make_uint4(o[0], o[1], o[2], o[3]);
    d[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

template <bool AF16>
__device__ __forceinline__ void cv_a(uint16_t *dst, const uint32_t *r) {
    uint32_t o[8];
    if (AF16) {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = r[i];
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++)
            o[i] = pack2h(__builtin_bit_cast(float, r[2 * i]), __builtin_bit_cast(float, r[2 * i + 1]));
    }
    st_lds8(dst, o);
}

template <int WT>
__device__ __forceinline__ void cv_b(uint16_t *dst, const uint32_t *r) {
    uint32_t o[8];
    if (WT == ARIA_WQ8) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t w = r[j];
            const int b0 = (int)(int8_t)(w & 0xFF), b1 = (int)(int8_t)((w >> 8) & 0xFF);
            const int b2 = (int)(int8_t)((w >> 16) & 0xFF), b3 = (int)(int8_t)(w >> 24);
            o[2 * j] = pack2h((float)b0, (float)b1);
            o[2 * j + 1] = pack2h((float)b2, (float)b3);
        }
    } else if (WT == ARIA_WQ4) {
        const float mn = __builtin_bit_cast(float, r[2]), st = __builtin_bit_cast(float, r[3]);
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t byte = (r[j] >> (8 * e)) & 0xFF;
                const float lo = mn + (float)(byte & 0xF) * st;   /* even k: low nibble */
                const float hi = mn + (float)(byte >> 4) * st;    /* odd k: high nibble */
                o[4 * j + e] = pack2h(lo, hi);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = r[i];
    }
    st_lds8(dst, o);
}

/* Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2):
 * workgroup g runs on XCD g % 8. Tile t = (g % 8) * ceil(T/8) + g / 8 gives each
 * XCD a contiguous run of tiles in M-major order, so an XCD's L2 holds a few
 * activation row panels and the weight panels instead of every activation row. */
__device__ __forceinline__ int xcd_tile(int g, int T) {
    const int per = (T + 7) >> 3;
    return (g & 7) * per + (g >> 3);
}

template <int WT, bool AF16, int TMW, int TNW>
struct QTile {
    static constexpr int BM = 64 * TMW, BN = 64 * TNW;
    static constexpr int ACH = BM * 2, BCH = BN * 2;   /* 16-element chunks per 32-wide slice */
    static constexpr int AIT = (ACH + 255) / 256, BIT = (BCH + 255) / 256;
    static constexpr int WA = RawA<AF16>::W, WB = RawB<WT>::W;
    struct Stage {
        uint32_t a[AIT][WA];
        uint32_t b[BIT][WB];
    };

    const QArgs &q;
    int tid, m0, n0;
    uint16_t *As, *Bs;   /* [2][rows * LDS_STRIDE] */

    __device__ __forceinline__ void load(Stage &s, int kt) const {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < AIT; i++) {
            const int c = tid + i * 256;
            if (c < ACH) ld_a<AF16>(s.a[i], q, m0 + (c >> 1), k0 + 16 * (c & 1));
        }
#pragma unroll
        for (int i = 0; i < BIT; i++) {
            const int c = tid + i * 256;
            if (c < BCH) ld_b<WT>(s.b[i], q, n0 + (c >> 1), k0 + 16 * (c & 1));
        }
    }
    __device__ __forceinline__ void store(const Stage &s, int buf) const {
        uint16_t *A = As + buf * (BM * LDS_STRIDE), *B = Bs + buf * (BN * LDS_STRIDE);
#pragma unroll
        for (int i = 0; i < AIT; i++) {
            const int c = tid + i * 256;
            if (c < ACH) cv_a<AF16>(&A[(c >> 1) * LDS_STRIDE + 16 * (c & 1)], s.a[i]);
        }
#pragma unroll
        for (int i = 0; i < BIT; i++) {
            const int c = tid + i * 256;
            if (c < BCH) cv_b<WT>(&B[(c >> 1) * LDS_STRIDE + 16 * (c & 1)], s.b[i]);
        }
    }
};

template <int WT, bool AF16, int TMW, int TNW>
__global__ __launch_bounds__(256) void k_qgemm_mfma(QArgs a, int NT, int T) {
    using Q = QTile<WT, AF16, TMW, TNW>;
    constexpr int BM = Q::BM, BN = Q::BN;
    __shared__ __attribute__((aligned(16))) uint16_t As[2 * BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2 * BN * LDS_STRIDE];

    const int t = xcd_tile(blockIdx.x, T);
    if (t >= T) return;                     /* uniform per workgroup */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const Q qt{a, tid, (t / NT) * BM, (t % NT) * BN, As, Bs};
    const int KT = a.K / BK;

    f32x16_t acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; i++)
#pragma unroll
        for (int j = 0; j < TNW; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int lrow = lane & 31, lk = 8 * (lane >> 5);
    auto compute = [&](int buf) {
        const uint16_t *A = As + buf * (BM * LDS_STRIDE), *B = Bs + buf * (BN * LDS_STRIDE);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            half8_t af[TMW], bf[TNW];
#pragma unroll
            for (int i = 0; i < TMW; i++)
                af[i] = *reinterpret_cast<const half8_t *>(&A[(wm * 32 * TMW + i * 32 + lrow) * LDS_STRIDE + ks * 16 + lk]);
#pragma unroll
            for (int j = 0; j < TNW; j++)
                bf[j] = *reinterpret_cast<const half8_t *>(&B[(wn * 32 * TNW + j * 32 + lrow) * LDS_STRIDE + ks * 16 + lk]);
#pragma unroll
            for (int i = 0; i < TMW; i++)
#pragma unroll
                for (int j = 0; j < TNW; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    /* ring of three raw stages: at slice kt, stage (kt+1)%3 holds slice kt+1 and
     * stage kt%3 receives slice kt+3 */
    typename Q::Stage s0, s1, s2;
    qt.load(s0, 0);
    if (KT > 1) qt.load(s1, 1);
    if (KT > 2) qt.load(s2, 2);
    qt.store(s0, 0);
    __syncthreads();
    auto step = [&](int kt, typename Q::Stage &nxt, typename Q::Stage &fill) {
        compute(kt & 1);
        if (kt + 1 < KT) qt.store(nxt, (kt + 1) & 1);
        if (kt + 3 < KT) qt.load(fill, kt + 3);
        __syncthreads();
    };
    int kt = 0;
    for (; kt + 3 <= KT; kt += 3) {
        step(kt, s1, s0);
        step(kt + 1, s2, s1);
        step(kt + 2, s0, s2);
    }
    if (kt < KT) step(kt, s1, s0);
    if (kt + 1 < KT) step(kt + 1, s2, s1);

    /* epilogue: acc register r of lane l -> row 8*(r/4) + 4*(l/32) + r%4, column l%32 */
#pragma unroll
    for (int j = 0; j < TNW; j++) {
        const int n = qt.n0 + wn * 32 * TNW + j * 32 + (lane & 31);
        if (n >= a.N) continue;
        const float sc = (WT == ARIA_WQ8) ? a.scale[n] : 1.0f;
        const float bb = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < TMW; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = qt.m0 + wm * 32 * TMW + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= a.M) continue;
                float v = acc[i][j][r];
                if (WT == ARIA_WQ8) v = v * sc;
                if (a.bias) v = v + bb;
                if (a.gelu) v = gelu_tanh_f(v);
                if (a.y_f16) ((uint16_t *)a.y)[(size_t)m * a.N + n] = f2h_bits(v);
                else ((float *)a.y)[(size_t)m * a.N + n] = v;
            }
        }
    }
}

/* ---- SIMT fallback: any K, any alignment; fp32 FMA on the dequantized values ---- */
template <int WT>
__device__ __forceinline__ float deq_w(const QArgs &a, int n, int k) {
    if (WT == ARIA_WQ8) return (float)((const int8_t *)a.q)[(size_t)n * a.K + k];
    if (WT == ARIA_WQ4) {
        const size_t rb = (size_t)(a.K + 1) / 2;
        const uint8_t byte = ((const uint8_t *)a.q)[(size_t)n * rb + (k >> 1)];
        const int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
        const size_t si = ((size_t)n * a.nblk + k / 32) * 2;
        return a.scale[si] + (float)nib * a.scale[si + 1];
    }
    return (float)__builtin_bit_cast(_Float16, ((const uint16_t *)a.q)[(size_t)n * a.K + k]);
}

template <int WT, bool AF16>
__global__ __launch_bounds__(256) void k_qgemm_simt(QArgs a) {
    __shared__ float As[16][64 + 4];
    __shared__ float Bs[16][64 + 4];
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int tid = threadIdx.x, tr = tid / 16, tc = tid % 16;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < a.K; k0 += 16) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int idx = tid + e * 256, r = idx / 16, kk = idx % 16;
            const int gm = m0 + r, gn = n0 + r, gk = k0 + kk;
            float av = 0.0f, bv = 0.0f;
            if (gm < a.M && gk < a.K)
                av = AF16 ? (float)__builtin_bit_cast(_Float16, ((const uint16_t *)a.x)[(size_t)gm * a.K + gk])
                          : ((const float *)a.x)[(size_t)gm * a.K + gk];
            if (gn < a.N && gk < a.K) bv = deq_w<WT>(a, gn, gk);
            As[kk][r] = av;
            Bs[kk][r] = bv;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(As[kk][tr * 4 + i], Bs[kk][tc * 4 + j], acc[i][j]);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + tr * 4 + i;
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + tc * 4 + j;
            if (n >= a.N) continue;
            float v = acc[i][j];
            if (WT == ARIA_WQ8) v = v * a.scale[n];
            if (a.bias) v = v + a.bias[n];
            if (a.gelu) v = gelu_tanh_f(v);
            if (a.y_f16) ((uint16_t *)a.y)[(size_t)m * a.N + n] = f2h_bits(v);
            else ((float *)a.y)[(size_t)m * a.N + n] = v;
        }
    }
}

template <int WT, bool AF16, int TMW, int TNW>
static void launch_tiles(const QArgs &a, hipStream_t s) {
    constexpr int BM = 64 * TMW, BN = 64 * TNW;
    const int MT = (a.M + BM - 1) / BM, NT = (a.N + BN - 1) / BN, T = MT * NT;
    const int grid = ((T + 7) / 8) * 8;
    hipLaunchKernelGGL((k_qgemm_mfma<WT, AF16, TMW, TNW>), dim3(grid), dim3(256), 0, s, a, NT, T);
}

/* Tile shape: estimated time ~ rounds * per-CU tile work / tile efficiency, where a CU
 * runs `occ` workgroups at once and rounds = ceil(T / (256 * occ)). */
static int pick_tiles(int M, int N) {
    static const int cfg[4][3] = {{2, 2, 3}, {2, 1, 4}, {1, 2, 4}, {1, 1, 6}};   /* TMW, TNW, occ */
    static const double eff[4] = {1.0, 0.85, 0.85, 0.6};
    double best = 1e30;
    int bi = 0;
    for (int i = 0; i < 4; i++) {
        const int BM = 64 * cfg[i][0], BN = 64 * cfg[i][1];
        const long T = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
        const long slots = 256L * cfg[i][2];
        const long rounds = (T + slots - 1) / slots;
        const double load = (double)rounds * cfg[i][2] * (BM / 64) * (BN / 64);
        const double cost = load / eff[i];
        if (cost < best - 1e-9) { best = cost; bi = i; }
    }
    return bi;
}

template <int WT, bool AF16>
static hipError_t launch_q(const QArgs &a, int tiles, hipStream_t s) {
    const bool aligned = a.K % BK == 0 && ((uintptr_t)a.x & 15u) == 0 && ((uintptr_t)a.q & 15u) == 0 &&
                         (WT != ARIA_WQ4 || ((uintptr_t)a.scale & 7u) == 0);
    if (!aligned) {
        dim3 grid((a.N + 63) / 64, (a.M + 63) / 64);
        hipLaunchKernelGGL((k_qgemm_simt<WT, AF16>), grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const int c = (tiles >= 1 && tiles <= 4) ? tiles - 1 : pick_tiles(a.M, a.N);
    switch (c) {
        case 0: launch_tiles<WT, AF16, 2, 2>(a, s); break;
        case 1: launch_tiles<WT, AF16, 2, 1>(a, s); break;
        case 2: launch_tiles<WT, AF16, 1, 2>(a, s); break;
        default: launch_tiles<WT, AF16, 1, 1>(a, s); break;
    }
    return hipGetLastError();
}

extern "C" hipError_t aria_k_qgemm_t(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                                     const float *scale, const float *bias, int M, int K, int N, int tiles,
                                     int gelu, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    QArgs a;
    a.y = y; a.x = x; a.q = q; a.scale = scale; a.bias = bias;
    a.M = M; a.K = K; a.N = N; a.y_f16 = y_f16; a.nblk = (K + 31) / 32; a.gelu = gelu;
    if (wtype == ARIA_WQ8) return x_f16 ? launch_q<ARIA_WQ8, true>(a, tiles, s) : launch_q<ARIA_WQ8, false>(a, tiles, s);
    if (wtype == ARIA_WQ4) return x_f16 ? launch_q<ARIA_WQ4, true>(a, tiles, s) : launch_q<ARIA_WQ4, false>(a, tiles, s);
    if (wtype == ARIA_WF16)
        return x_f16 ? launch_q<ARIA_WF16, true>(a, tiles, s) : launch_q<ARIA_WF16, false>(a, tiles, s);
    return hipErrorInvalidValue;
}

extern "C" hipError_t aria_k_qgemm(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                                   const float *scale, const float *bias, int M, int K, int N, hipStream_t s) {
    return aria_k_qgemm_t(y, y_f16, x, x_f16, wtype, q, scale, bias, M, K, N, 0, 0, s);
}
