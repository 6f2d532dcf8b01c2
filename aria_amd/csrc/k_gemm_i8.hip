/*
 * k_gemm_i8.hip - the W8A8 path on gfx950: per-row int8 activation quantisation and the
 * int8 x int8 -> int32 GEMM on v_mfma_i32_32x32x32_i8 with the dequantisation fused into
 * the shared epilogue.
 *
 * Replaces the reference's gemm_w8a8 / gemm_w8a8_h (src/aria_cuda.cu:978-1004: k_quant_act_q8,
 * k_quant_act_q8_h, an IMMA cublasGemmEx into int32, then k_deq_i32 in place) and the CPU
 * aria_linear_q8a8 (src/aria_quant.c:253-345), which defines the numbers:
 *   amax = max_k |x[m,k]|, sx[m] = amax / 127, xq = clamp(lrintf(x * (127 / amax)), -127, 127)
 *   (xq = 0 when amax == 0), acc = sum_k xq[m,k] * q[n,k] in exact int32,
 *   y[m,n] = (float)acc * sx[m] * scale[n] + (b ? b[n] : 0.0f).
 * Every step is exact or one IEEE-rounded operation in the same order (the kernels are built
 * with -ffp-contract=off), so the results are bit-identical to the reference's scalar path.
 *
 * The Q8 weights are used as packed ([N, K] int8, the reference's layout): no unpacking at
 * all, and the int8 MFMA does twice the fp16 rate per cycle.
 */
#include "qgemm_dev.h"

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

/* ---- activation quantisation: one wave per row, the row held in registers ----
 * Lane l holds elements 4 (l + 64 j), j < nv = K / 256 (K % 256 == 0, up to 4096), or walks
 * the row twice (16-byte vectors when K % 4 == 0, single elements otherwise). */
#define QA_MAXV 16
template <bool F16>
__device__ __forceinline__ float4 qa_load(const void *x, size_t i) {
    if constexpr (F16) {
        const uint2 u = *reinterpret_cast<const uint2 *>((const uint16_t *)x + i);
        const half2_t a = __builtin_bit_cast(half2_t, u.x), b = __builtin_bit_cast(half2_t, u.y);
        return make_float4((float)a[0], (float)a[1], (float)b[0], (float)b[1]);
    } else {
        return *reinterpret_cast<const float4 *>((const float *)x + i);
    }
}
template <bool F16>
__global__ __launch_bounds__(256) void k_quant_act_q8(int8_t *xq, float *sx, const void *x, int M, int K) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;   /* uniform per wave */
    const size_t base = (size_t)row * K;
    uint32_t *qr = reinterpret_cast<uint32_t *>(xq + base);
    const int nv = K >> 8;
    float mx = 0.0f;
    if ((K & 255) == 0 && nv <= QA_MAXV) {
        float4 v[QA_MAXV];
#pragma unroll
        for (int j = 0; j < QA_MAXV; j++)
            if (j < nv) v[j] = qa_load<F16>(x, base + 4 * (lane + 64 * j));
#pragma unroll
        for (int j = 0; j < QA_MAXV; j++)
            if (j < nv) mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
        mx = grp_max<64>(mx);
        const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
#pragma unroll
        for (int j = 0; j < QA_MAXV; j++)
            if (j < nv) qr[lane + 64 * j] = q8_pack4(v[j], inv);
    } else if ((K & 3) == 0) {
        for (int k = 4 * lane; k < K; k += 256) {
            const float4 v = qa_load<F16>(x, base + k);
            mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
        }
        mx = grp_max<64>(mx);
        const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
        for (int k = 4 * lane; k < K; k += 256) qr[k >> 2] = q8_pack4(qa_load<F16>(x, base + k), inv);
    } else {   /* any K: one element per lane and step */
        auto ld1 = [&](int k) -> float {
            if constexpr (F16) return (float)__builtin_bit_cast(_Float16, ((const uint16_t *)x)[base + k]);
            else return ((const float *)x)[base + k];
        };
        for (int k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(ld1(k)));
        mx = grp_max<64>(mx);
        const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
        for (int k = lane; k < K; k += 64)
            xq[base + k] = (int8_t)min(max((int)__builtin_rintf(ld1(k) * inv), -127), 127);
    }
    if (lane == 0) sx[row] = mx / 127.0f;
}

/* rows of 2048 <= K <= 8192, K % 1024 == 0 (the FFN product): one 256-lane workgroup per
 * row, lane t holding elements 4 (t + 256 j), j < K / 1024, so four waves share a row's
 * latency instead of one wave walking 16 vectors per lane; the four wave maxima meet in LDS
 * (a maximum is exact in any order, so the bits equal the one-wave kernel's) */
template <bool F16>
__global__ __launch_bounds__(256) void k_quant_act_q8_row(int8_t *xq, float *sx, const void *x, int K) {
    __shared__ float wmax[4];
    const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const size_t base = (size_t)row * K;
    const int nv = K >> 10;
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < nv) v[j] = qa_load<F16>(x, base + 4 * (t + 256 * j));
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < nv) mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
    mx = grp_max<64>(mx);
    if (lane == 0) wmax[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    uint32_t *qr = reinterpret_cast<uint32_t *>(xq + base);
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < nv) qr[t + 256 * j] = q8_pack4(v[j], inv);
    if (t == 0) sx[row] = mx / 127.0f;
}

/* ---- int8 GEMM, weights in registers ----
 * 4 waves share one int8 activation tile of BM = 32 FM rows x 64 k in LDS (double
 * buffered); wave w owns weight rows n0 + 64 w .. + 63 (two 32-row MFMA blocks) and loads
 * them from the packed rows straight into MFMA operand registers. K-tile 64: lane half h
 * covers k in [32 h, 32 h + 32) of the tile and MFMA step ks (0, 1) takes its 16 k at
 * 32 h + 16 ks, for both operands, so a lane's weight bytes of a tile are 32 contiguous
 * bytes and the contraction order is the same permutation on both sides. Weights are
 * loaded two K-tiles ahead (three register stages), activations two K-tiles ahead
 * (two register sets) and stored to LDS one tile ahead: one barrier per K-tile. */
#define IBK 64
/* activation tile [BM][64] bytes: chunk c (16 B) of row r at c ^ ((r >> 2) & 3), so 16
 * lanes reading one chunk of 16 consecutive rows touch all 64 banks once */
__device__ __forceinline__ int ioff(int r, int c) { return r * IBK + ((c ^ ((r >> 2) & 3)) << 4); }
/* 128-byte rows (K-tile 128): chunk c of row r at c ^ ((r >> 1) & 7), the same property */
template <int KB>
__device__ __forceinline__ int ioffk(int r, int c) {
    if constexpr (KB == 64) return ioff(r, c);
    else return r * KB + ((c ^ ((r >> 1) & 7)) << 4);
}

/* KB: K-tile depth in bytes (64, or 128 with K % 128 == 0): lane half h covers k in
 * [KB/2 h, KB/2 (h + 1)) of the tile, MFMA step ks (KB / 32 of them) its 16 k at KB/2 h + 16 ks */
template <int FM, int MINB, int MODE, bool GELU, int KB = 64>
__global__ __launch_bounds__(256, MINB) void k_gemm_i8(QArgs a, int NTN, int T) {
    static_assert(KB == 64 || KB == 128, "K-tile");
    constexpr int NKS = KB / 32;              /* MFMA steps per K-tile */
    constexpr int FN = 2, BM = 32 * FM, BN = 256;
    constexpr int EPI_STRIDE = 32 * FN * 4 + 16;
    constexpr int TILE_BYTES = 2 * BM * KB, EPI_BYTES = 4 * 32 * EPI_STRIDE;
    constexpr int LDS_BYTES = TILE_BYTES > EPI_BYTES ? TILE_BYTES : EPI_BYTES;
    constexpr int CPR = KB / 16;              /* 16-byte chunks per row */
    constexpr int XC = BM * CPR;              /* 16-byte chunks of one activation tile */
    constexpr int XPT = (XC + 255) / 256;     /* chunks per thread */
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];

    const int t = xcd_tile(blockIdx.x, T);
    if (t >= T) return;                       /* uniform per workgroup */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lrow = lane & 31, lh = lane >> 5;
    const int m0 = (t / NTN) * BM, n0 = (t % NTN) * BN;
    const int KT = a.K / KB;
    const int8_t *xq = (const int8_t *)a.x, *wq = (const int8_t *)a.q;

    /* weight rows of this lane (rows past N re-read the last row; never stored) */
    const int8_t *wrow0 = wq + (size_t)min(n0 + wave * 64 + lrow, a.N - 1) * a.K + (KB / 2) * lh;
    const int8_t *wrow1 = wq + (size_t)min(n0 + wave * 64 + 32 + lrow, a.N - 1) * a.K + (KB / 2) * lh;
    /* [block 0: 4 NKS words, block 1: 4 NKS words] */
    typedef uint32_t ws_t __attribute__((ext_vector_type(8 * NKS)));
    auto wload = [&](ws_t &s, int kt) __attribute__((always_inline)) {
        const uint4 *p0 = reinterpret_cast<const uint4 *>(wrow0 + kt * KB);
        const uint4 *p1 = reinterpret_cast<const uint4 *>(wrow1 + kt * KB);
        uint4 u[2 * NKS];
#pragma unroll
        for (int i = 0; i < NKS; i++) { u[i] = p0[i]; u[NKS + i] = p1[i]; }
#pragma unroll
        for (int i = 0; i < 2 * NKS; i++) {
            s[4 * i] = u[i].x; s[4 * i + 1] = u[i].y; s[4 * i + 2] = u[i].z; s[4 * i + 3] = u[i].w;
        }
    };
    /* activation chunk c = tid + 256 i: row c / 4, chunk c % 4 (rows past M re-read the
     * last row; threads past the tile's last chunk re-read it and do not store) */
    typedef uint32_t xs_t __attribute__((ext_vector_type(4 * XPT)));
    auto xload = [&](xs_t &r, int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int c = (XC % 256 == 0) ? tid + 256 * i : min(tid + 256 * i, XC - 1);
            const int m = min(m0 + c / CPR, a.M - 1);
            const uint4 u = *reinterpret_cast<const uint4 *>(xq + (size_t)m * a.K + kt * KB + 16 * (c % CPR));
            r[4 * i] = u.x; r[4 * i + 1] = u.y; r[4 * i + 2] = u.z; r[4 * i + 3] = u.w;
        }
    };
    auto xstore = [&](const xs_t &r, int buf) __attribute__((always_inline)) {
        uint8_t *X = lds + buf * (BM * KB);
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int c = tid + 256 * i;
            if (XC % 256 == 0 || c < XC)
                *reinterpret_cast<uint4 *>(X + ioffk<KB>(c / CPR, c % CPR)) =
                    make_uint4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
        }
    };

    i32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    auto compute = [&](ws_t &ws, int buf) __attribute__((always_inline)) {
        const uint8_t *X = lds + buf * (BM * KB);
        i32x4_t xf[NKS][FM];
#pragma unroll
        for (int ks = 0; ks < NKS; ks++)
#pragma unroll
            for (int i = 0; i < FM; i++)
                xf[ks][i] = *reinterpret_cast<const i32x4_t *>(X + ioffk<KB>(i * 32 + lrow, NKS * lh + ks));
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            constexpr int B1 = 4 * NKS;   /* block 1's first word */
            const i32x4_t w0 = {(int)ws[4 * ks], (int)ws[4 * ks + 1], (int)ws[4 * ks + 2], (int)ws[4 * ks + 3]};
            const i32x4_t w1 = {(int)ws[B1 + 4 * ks], (int)ws[B1 + 4 * ks + 1], (int)ws[B1 + 4 * ks + 2],
                                (int)ws[B1 + 4 * ks + 3]};
#pragma unroll
            for (int i = 0; i < FM; i++) {
                acc[i][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w0, xf[ks][i], acc[i][0], 0, 0, 0);
                acc[i][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w1, xf[ks][i], acc[i][1], 0, 0, 0);
            }
        }
    };

    /* step kt (kt % 6 == P): tile kt + 2 loaded (weights into stage (P + 2) % 3, activations
     * into set P % 2), tile kt multiplied out of LDS buffer P & 1 with stage P % 3, tile
     * kt + 1 stored from set (P + 1) % 2 into the other buffer */
    ws_t w0, w1, w2;
    xs_t x0, x1;
    auto wsel = [&](auto I) __attribute__((always_inline)) -> ws_t & {
        constexpr int i = decltype(I)::value;
        if constexpr (i == 0) return w0; else if constexpr (i == 1) return w1; else return w2;
    };
    auto xsel = [&](auto I) __attribute__((always_inline)) -> xs_t & {
        if constexpr (decltype(I)::value == 0) return x0; else return x1;
    };
    xload(x0, 0);
    wload(w0, 0);
    if (KT > 1) {
        xload(x1, 1);
        wload(w1, 1);
    }
    xstore(x0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0): the loop header inherits no prologue loads */
    __syncthreads();
    auto step = [&](auto PP, auto GUARD, int kt) __attribute__((always_inline)) {
        constexpr int P = decltype(PP)::value;
        constexpr bool guard = decltype(GUARD)::value;
        if (!guard || kt + 2 < KT) {
            wload(wsel(IC<(P + 2) % 3>{}), kt + 2);
            xload(xsel(IC<P % 2>{}), kt + 2);
        }
        compute(wsel(IC<P % 3>{}), P & 1);
        if (!guard || kt + 1 < KT) xstore(xsel(IC<(P + 1) % 2>{}), (P + 1) & 1);
        __syncthreads();
    };
    using F = std::false_type;
    using G = std::true_type;
    int kt = 0;
    for (; kt + 6 + 2 <= KT; kt += 6)
        static_for<6>([&](auto PP) __attribute__((always_inline)) { step(PP, F{}, kt + decltype(PP)::value); });
    for (; kt < KT; kt += 6)
        static_for<6>([&](auto PP) __attribute__((always_inline)) {
            if (kt + decltype(PP)::value < KT) step(PP, G{}, kt + decltype(PP)::value);
        });

    /* the epilogue converts each int32 sum as it stages it ((float)acc: nearest even, as
     * the C conversion) */
    float *E = reinterpret_cast<float *>(lds) + wave * (32 * EPI_STRIDE / 4);
    epilogue<FM, FN, ARIA_WI8, MODE, GELU>(a, acc, E, lane, m0, n0 + wave * 64);
}

/* SIMT form for shapes the MFMA kernel does not take: one thread per output, plain store */
__global__ __launch_bounds__(256) void k_gemm_i8_simt(QArgs a) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)a.M * a.N) return;
    const int m = (int)(idx / a.N), n = (int)(idx % a.N);
    const int8_t *xr = (const int8_t *)a.x + (size_t)m * a.K, *wr = (const int8_t *)a.q + (size_t)n * a.K;
    int32_t acc = 0;
    for (int k = 0; k < a.K; k++) acc += (int32_t)xr[k] * (int32_t)wr[k];
    const float v = (float)acc * a.xscale[m] * a.scale[n] + (a.bias ? a.bias[n] : 0.0f);
    if (a.y_f16) ((uint16_t *)a.y)[idx] = f2h_bits(v);
    else ((float *)a.y)[idx] = v;
}

template <int FM, int MODE, bool GELU = false>
static void launch_i8_m(const QArgs &a, hipStream_t s) {
    constexpr int BM = 32 * FM, BN = 256;
    const int MT = (a.M + BM - 1) / BM, NTN = (a.N + BN - 1) / BN, T = MT * NTN;
    const int grid = ((T + 7) / 8) * 8;
    if constexpr (FM == 2) {
        if (a.K % 128 == 0) {   /* fewer barriers per MFMA where the tiles are short */
            hipLaunchKernelGGL((k_gemm_i8<FM, 2, MODE, GELU, 128>), dim3(grid), dim3(256), 0, s, a, NTN, T);
            return;
        }
    }
    hipLaunchKernelGGL((k_gemm_i8<FM, (FM <= 2 ? 2 : 1), MODE, GELU>), dim3(grid), dim3(256), 0, s, a, NTN, T);
}
template <int FM>
static void launch_i8(const QArgs &a, hipStream_t s) {
    switch (a.epi.mode) {
        case ARIA_EPI_GATE_RES: launch_i8_m<FM, ARIA_EPI_GATE_RES>(a, s); break;
        case ARIA_EPI_ADD: launch_i8_m<FM, ARIA_EPI_ADD>(a, s); break;
        case ARIA_EPI_HEADS: launch_i8_m<FM, ARIA_EPI_HEADS>(a, s); break;
        case ARIA_EPI_GLU: launch_i8_m<FM, ARIA_EPI_GLU>(a, s); break;
        default:
            if (a.gelu) launch_i8_m<FM, ARIA_EPI_STORE, true>(a, s);
            else launch_i8_m<FM, ARIA_EPI_STORE>(a, s);
            break;
    }
}

extern "C" hipError_t aria_k_quant_act_q8(int8_t *xq, float *sx, const void *x, int x_f16, int M, int K,
                                          hipStream_t s) {
    if (M <= 0) return hipSuccess;
    if (K <= 0) return hipErrorInvalidValue;
    if (K % 1024 == 0 && K >= 2048 && K <= 8192) {
        if (x_f16) hipLaunchKernelGGL(k_quant_act_q8_row<true>, dim3(M), dim3(256), 0, s, xq, sx, x, K);
        else hipLaunchKernelGGL(k_quant_act_q8_row<false>, dim3(M), dim3(256), 0, s, xq, sx, x, K);
        return hipGetLastError();
    }
    const int grid = (M + 3) / 4;
    if (x_f16) hipLaunchKernelGGL(k_quant_act_q8<true>, dim3(grid), dim3(256), 0, s, xq, sx, x, M, K);
    else hipLaunchKernelGGL(k_quant_act_q8<false>, dim3(grid), dim3(256), 0, s, xq, sx, x, M, K);
    return hipGetLastError();
}

extern "C" hipError_t aria_k_gemm_i8_t(void *y, int y_f16, const int8_t *xq, const float *sx, const int8_t *q,
                                       const float *scale, const float *bias, int M, int K, int N, int fm, int gelu,
                                       const aria_qgemm_epi *epi, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (K <= 0) return hipErrorInvalidValue;
    QArgs a;
    a.y = y; a.x = xq; a.q = q; a.scale = scale; a.bias = bias;
    a.M = M; a.K = K; a.N = N; a.y_f16 = y_f16; a.nblk = 0; a.gelu = gelu;
    a.xscale = sx;
    if (epi) a.epi = *epi;
    else { memset(&a.epi, 0, sizeof a.epi); a.epi.mode = ARIA_EPI_STORE; }
    if (a.epi.mode == ARIA_EPI_HEADS) {
        if (N % 64 || a.epi.nsec < 1 || a.epi.nsec > 3 || a.epi.heads * 64 * a.epi.nsec != N ||
            a.epi.rows_per_batch <= 0 || (a.epi.rot && (a.epi.rot > 64 || (a.epi.rot & 7)))) return hipErrorInvalidValue;
        a.y = (void *)a.epi.dst[0];
    } else if (a.epi.mode == ARIA_EPI_GLU) {
        if (N % 4 || a.gelu) return hipErrorInvalidValue;
    } else if (a.epi.mode != ARIA_EPI_GATE_RES && a.epi.mode != ARIA_EPI_ADD && a.epi.mode != ARIA_EPI_STORE) {
        return hipErrorInvalidValue;   /* ADD_DYT is the fp16-weight decoder's */
    } else if (a.epi.mode != ARIA_EPI_STORE) {
        if (y_f16 || a.epi.rows_per_batch <= 0) return hipErrorInvalidValue;
    }
    const bool mfma_ok = K % IBK == 0 && N % 4 == 0 && ((uintptr_t)xq & 15u) == 0 && ((uintptr_t)q & 15u) == 0 &&
                         ((uintptr_t)scale & 15u) == 0 && ((uintptr_t)bias & 15u) == 0 &&
                         ((uintptr_t)a.y & (y_f16 ? 7u : 15u)) == 0;
    if (!mfma_ok) {
        if (a.epi.mode != ARIA_EPI_STORE || a.gelu) return hipErrorInvalidValue;
        const size_t n = (size_t)M * N;
        hipLaunchKernelGGL(k_gemm_i8_simt, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    if (fm >= 16) return qgemm_big_i8_launch(a, fm - 16, s);   /* the LDS-DMA kernel, configuration fm - 16 */
    const bool heads = a.epi.mode == ARIA_EPI_HEADS;
    if (fm <= 0 && K % 128 == 0 && (!heads || N <= 3072)) {
        /* the LDS-DMA kernel (k_qgemm_big.hip) at every DiT shape: HEADS in 64 x 256, N <= 1024
         * in 64 x 128, N <= 3072 in 128 x 128, wider in 192 x 128 (two workgroups per CU), except
         * N = 4096 in 192 x 256 tiles of 8 waves sharing the activation tile (ff_in 24.3 -> 23.6 us
         * with GELU, the same bits); N <= 1024
         * with K >= 2048 (ff_out) in 96 x 128 tiles of 8 waves, the K range split between two
         * pipelines (23.6 -> 21.7 us at K = 4096; at K = 1024 the split measured 6 % slower);
         * HEADS with N <= 1024 (ca_q: 164 tiles, one workgroup per busy CU) in 64 x 256 tiles
         * with the split (14.0 -> 12.7 us, the same bits: int32 sums are exact) */
        return qgemm_big_i8_launch(a, heads ? ((N <= 1024 && (K / 128) % 2 == 0) ? 5 : 1) : N <= 1024 ? ((K >= 2048 && (K / 128) % 2 == 0) ? 4 : 0)
                                                    : N <= 3072 ? 2 : N <= 4096 ? 6 : 3, s);
    }
    if (fm <= 0) {
        /* tile rows, from a sweep at M = 2592 (fm: 1..4 = 32..128 rows): 128 rows when those
         * tiles fill the 256 CUs once (one workgroup per CU: 296 registers), 96 rows when
         * they give at least 1.5 workgroups per CU (two fit), else 64 rows (64 us -> 37 us at
         * N = 1024, K = 4096 against 32 rows) */
        const int NTN = (N + 255) / 256;
        const int t4 = ((M + 127) / 128) * NTN, t3 = ((M + 95) / 96) * NTN;
        fm = (t4 >= 192 && t4 <= 256) ? 4 : (t3 >= 384 ? 3 : 2);
        /* the head-preparation epilogue (RMS statistic, RoPE partner exchange) needs the
         * registers that 96- and 128-row tiles give to accumulators: the W8A8 block's qkv
         * projection measured 2.4 us faster at 64 rows than at 128, 16 us slower at 96 */
        if (a.epi.mode == ARIA_EPI_HEADS) fm = 2;
    }
    switch (fm) {
        case 1: launch_i8<1>(a, s); break;
        case 2: launch_i8<2>(a, s); break;
        case 3: launch_i8<3>(a, s); break;
        default: launch_i8<4>(a, s); break;
    }
    return hipGetLastError();
}

extern "C" hipError_t aria_k_gemm_i8(void *y, int y_f16, const int8_t *xq, const float *sx, const int8_t *q,
                                     const float *scale, const float *bias, int M, int K, int N, int gelu,
                                     const aria_qgemm_epi *epi, hipStream_t s) {
    return aria_k_gemm_i8_t(y, y_f16, xq, sx, q, scale, bias, M, K, N, 0, gelu, epi, s);
}
