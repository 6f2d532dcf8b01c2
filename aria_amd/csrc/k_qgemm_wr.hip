/*
 * k_qgemm_wr.hip - the weights-in-registers dequant-on-use GEMM (gfx950 MFMA):
 * y[M,N] = x[M,K] W[N,K]^T (+ b) for Q8 / Q4 weights and fp16 activations, K % 64 == 0.
 * Replaces the same reference functions as k_qgemm.hip (aria_linear_q8 / aria_linear_q4,
 * src/aria_quant.c:98-145, 469-538); that file holds the layouts, the error budget and the
 * tile pick. Shares the argument block and the fused epilogue (qgemm_dev.h).
 */
#include "qgemm_dev.h"

/* ---- weights-in-registers kernel (Q8 / Q4 weights, fp16 activations, K % 64 == 0) ----
 * 4 waves share one activation tile of BM = 32*FM rows in LDS; wave w owns weight rows
 * n0 + 64w .. n0 + 64w + 63 (two 32-row MFMA blocks) and loads them straight from global
 * memory into VGPRs, still packed, in the MFMA operand layout: no LDS round trip for the
 * weights, so LDS carries only the shared activations (read once per wave and per 32x64
 * block pair) and the kernel stays under the 128 B/clk LDS and 64 B/clk L1 limits.
 * K-tile = 64. The contraction order inside a tile is permuted identically for both
 * operands: lane half h = l/32 covers k in [32h, 32h + 32) of the tile, and MFMA step ks
 * takes its 8 k at 32h + 8ks. For Q4 that range is exactly one quantization block, so a
 * lane needs one [min, step] pair per tile; for Q8 it is 32 contiguous bytes.
 * Pipeline: weights three K-tiles deep in registers (loads issued two tiles ahead),
 * activations one tile ahead in registers and double-buffered in LDS, one barrier per
 * K-tile. The epilogue is the shared one (row scale, bias, GELU, fused modes). */
#define WBK 64

/* activation tile [BM][64] halves: 8 chunks of 16 B per row, logical chunk c of row r
 * stored at c ^ ((r >> 1) & 7): the producers' row-major 16 B writes and the fragment
 * reads (32 rows x one chunk per lane half) both cover all 64 banks once per 16 lanes */
__device__ __forceinline__ int xoff(int r, int c) { return r * WBK + ((c ^ ((r >> 1) & 7)) << 3); }

template <int WT>
struct WRegs {            /* one lane's raw weights for one K-tile, two 32-row blocks */
    static constexpr int NW = (WT == ARIA_WQ8) ? 8 : 6;   /* Q8: 32 B; Q4: 16 B nibbles + [min, step] */
    uint32_t w[2][NW];
};

template <int WT>
__device__ __forceinline__ void wr_load(const QArgs &a, WRegs<WT> &s, int nrow, int kt, int h) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = min(nrow + 32 * j, a.N - 1);
        if (WT == ARIA_WQ4) {
            const uint4 u = *reinterpret_cast<const uint4 *>((const uint8_t *)a.q + (size_t)n * (a.K >> 1) + kt * 32 + 16 * h);
            const uint2 p = *reinterpret_cast<const uint2 *>(a.scale + ((size_t)n * a.nblk + 2 * kt + h) * 2);
            s.w[j][0] = u.x; s.w[j][1] = u.y; s.w[j][2] = u.z; s.w[j][3] = u.w;
            s.w[j][4] = p.x; s.w[j][5] = p.y;
        } else {
            const uint4 *p = reinterpret_cast<const uint4 *>((const int8_t *)a.q + (size_t)n * a.K + kt * WBK + 32 * h);
            const uint4 u0 = p[0], u1 = p[1];
            s.w[j][0] = u0.x; s.w[j][1] = u0.y; s.w[j][2] = u0.z; s.w[j][3] = u0.w;
            s.w[j][4] = u1.x; s.w[j][5] = u1.y; s.w[j][6] = u1.z; s.w[j][7] = u1.w;
        }
    }
}

/* (w & mask) | magic in one VALU op (v_and_or_b32 takes one SGPR operand on gfx9-class
 * VOP3 encodings: mask is uniform, magic sits in a VGPR) */
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(mask), "v"(magic));
    return r;
}

/* the 8 fp16 weights of block j for MFMA step ks. Q4: a dword holds 8 nibbles, byte b =
 * (k = 2b low, k = 2b + 1 high). Each nibble is placed under the fp16 exponent of 1024
 * (0x6400 | n = 1024 + n; the high nibble of a byte lands as 1024 + 16 n) and a
 * mixed-precision FMA (fp16 operand, fp32 arithmetic, fp16 result) forms
 * (1024 + n) * step + (min - 1024 step) = min + n * step (step / 16 and min - 64 step for
 * the high nibbles): the value the reference dequantizes, rounded to fp16. The two offsets
 * are formed once per block and K-tile (off[j]), so the 1024 never has to be subtracted
 * from the nibbles (4 packed subtractions per step); the fp32 offset carries ~2e-7 absolute
 * error per weight before the fp16 rounding. */
struct Q4Off { float a, b, st, s16; };
template <int WT>
__device__ __forceinline__ Q4Off q4_off(const WRegs<WT> &s, int j) {
    Q4Off o;
    if constexpr (WT == ARIA_WQ4) {
        const float mn = __builtin_bit_cast(float, s.w[j][4]);
        o.st = __builtin_bit_cast(float, s.w[j][5]);
        o.s16 = o.st * 0.0625f;
        o.a = __builtin_fmaf(-1024.0f, o.st, mn);
        o.b = __builtin_fmaf(-64.0f, o.st, mn);
    } else {
        o.a = o.b = o.st = o.s16 = 0.0f;
    }
    return o;
}
template <int WT>
__device__ __forceinline__ half8_t wr_frag(const WRegs<WT> &s, int j, int ks, uint32_t magic, const Q4Off &f) {
    uint32_t o[4];
    if (WT == ARIA_WQ4) {
        const uint32_t w = s.w[j][ks], u = w >> 8;
        const half2_t t0 = __builtin_bit_cast(half2_t, and_or(w, 0x000F000Fu, magic));   /* 1024 + k0, k4 */
        const half2_t t1 = __builtin_bit_cast(half2_t, and_or(w, 0x00F000F0u, magic));   /* 1024 + 16 k1, 16 k5 */
        const half2_t t2 = __builtin_bit_cast(half2_t, and_or(u, 0x000F000Fu, magic));   /* 1024 + k2, k6 */
        const half2_t t3 = __builtin_bit_cast(half2_t, and_or(u, 0x00F000F0u, magic));   /* 1024 + 16 k3, 16 k7 */
        const half2_t h0 = {(_Float16)__builtin_fmaf((float)t0[0], f.st, f.a), (_Float16)__builtin_fmaf((float)t1[0], f.s16, f.b)};
        const half2_t h1 = {(_Float16)__builtin_fmaf((float)t2[0], f.st, f.a), (_Float16)__builtin_fmaf((float)t3[0], f.s16, f.b)};
        const half2_t h2 = {(_Float16)__builtin_fmaf((float)t0[1], f.st, f.a), (_Float16)__builtin_fmaf((float)t1[1], f.s16, f.b)};
        const half2_t h3 = {(_Float16)__builtin_fmaf((float)t2[1], f.st, f.a), (_Float16)__builtin_fmaf((float)t3[1], f.s16, f.b)};
        o[0] = __builtin_bit_cast(uint32_t, h0); o[1] = __builtin_bit_cast(uint32_t, h1);
        o[2] = __builtin_bit_cast(uint32_t, h2); o[3] = __builtin_bit_cast(uint32_t, h3);
    } else {
        q8x4_to_h(s.w[j][2 * ks], o[0], o[1]);
        q8x4_to_h(s.w[j][2 * ks + 1], o[2], o[3]);
    }
    return __builtin_bit_cast(half8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

template <int WT, int FM, int MINB, int MODE, bool GELU, int DP = (WT == ARIA_WQ8 && FM >= 3 ? 3 : 2)>
__global__ __launch_bounds__(256, MINB) void k_qgemm_wr(QArgs a, int NTN, int T) {
    constexpr int FN = 2, BM = 32 * FM, BN = 256;
    constexpr int EPI_STRIDE = 32 * FN * 4 + 16;
    constexpr int TILE_BYTES = 2 * BM * WBK * 2, EPI_BYTES = 4 * 32 * EPI_STRIDE;
    constexpr int LDS_BYTES = TILE_BYTES > EPI_BYTES ? TILE_BYTES : EPI_BYTES;
    __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_BYTES / 2];

    const int t = xcd_tile(blockIdx.x, T);
    if (t >= T) return;                     /* uniform per workgroup */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lrow = lane & 31, lh = lane >> 5;
    const int m0 = (t / NTN) * BM, n0 = (t % NTN) * BN;
    const int KT = a.K / WBK;
    const int nrow = n0 + wave * 64 + lrow;
    uint32_t magic = 0x64006400u;   /* fp16 1024 in both halves, kept in a VGPR */
    asm volatile("" : "+v"(magic));

    /* activation staging: thread tid moves chunk c = tid + 256 i (row c / 8, chunk c % 8);
     * rows past M re-read the last row (their results are never stored). Tile t is staged
     * in register set t % DP (xa, xb, xc), loaded DP K-tiles before it is multiplied and
     * stored to LDS one K-tile before. Weights of tile t sit in stage t % (DP + 1)
     * (s0 .. s3), also loaded DP K-tiles ahead. Sets and stages are picked by compile-time
     * constants (IC<>) so they stay in VGPRs. */
    static_assert(DP == 2 || DP == 3, "prefetch distance");
    typedef uint32_t xv_t __attribute__((ext_vector_type(4 * FM)));
    xv_t xa, xb, xc;
    WRegs<WT> s0, s1, s2, s3;
    auto xsel = [&](auto XS) __attribute__((always_inline)) -> xv_t & {
        constexpr int xs = decltype(XS)::value;
        if constexpr (xs == 0) return xa; else if constexpr (xs == 1) return xb; else return xc;
    };
    auto wsel = [&](auto ST) __attribute__((always_inline)) -> WRegs<WT> & {
        constexpr int st = decltype(ST)::value;
        if constexpr (st == 0) return s0; else if constexpr (st == 1) return s1;
        else if constexpr (st == 2) return s2; else return s3;
    };
    auto xload = [&](auto XS, int kt) __attribute__((always_inline)) {
        xv_t &xr = xsel(XS);
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int c = tid + 256 * i;
            const int m = min(m0 + (c >> 3), a.M - 1);
            const uint4 u = *reinterpret_cast<const uint4 *>((const uint16_t *)a.x + (size_t)m * a.K + kt * WBK + 8 * (c & 7));
            xr[4 * i] = u.x; xr[4 * i + 1] = u.y; xr[4 * i + 2] = u.z; xr[4 * i + 3] = u.w;
        }
    };
    auto xstore = [&](auto XS, int buf) __attribute__((always_inline)) {
        const xv_t &xr = xsel(XS);
        uint16_t *X = lds + buf * (BM * WBK);
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4 *>(&X[xoff(c >> 3, c & 7)]) = make_uint4(xr[4 * i], xr[4 * i + 1], xr[4 * i + 2], xr[4 * i + 3]);
        }
    };

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    /* The weight words are made opaque where their tile is consumed: without it the
     * compiler starts unpacking a stage right after issuing its loads, and the wait for
     * those loads then stalls every K-tile instead of landing two tiles later. */
    auto compute = [&](auto ST, int buf) __attribute__((always_inline)) {
        WRegs<WT> &ws = wsel(ST);
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < WRegs<WT>::NW; e++) asm volatile("" : "+v"(ws.w[j][e]));
        const uint16_t *X = lds + buf * (BM * WBK);
        /* FM <= 2: every activation fragment of the tile is requested first, into its own
         * registers. Left to itself the compiler reads each one into the same four VGPRs
         * right before its MFMAs and waits out the whole LDS latency 4 * FM times per
         * K-tile; issued up front, the reads overlap the unpacking below (K = 4096 GEMMs
         * 4-6 % faster). With FM = 3, 4 the same order measured 12-16 % slower (48-64 more
         * live VGPRs next to the AGPR accumulators cost the second resident workgroup), so
         * those keep the compiler's order. */
        const Q4Off f0 = q4_off<WT>(ws, 0), f1 = q4_off<WT>(ws, 1);
        if constexpr (FM <= 2) {
            half8_t xf[4][FM];
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int i = 0; i < FM; i++) xf[ks][i] = *reinterpret_cast<const half8_t *>(&X[xoff(i * 32 + lrow, 4 * lh + ks)]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const half8_t w0 = wr_frag<WT>(ws, 0, ks, magic, f0), w1 = wr_frag<WT>(ws, 1, ks, magic, f1);
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w0, xf[ks][i], acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1, xf[ks][i], acc[i][1], 0, 0, 0);
                }
            }
        } else if constexpr (WT == ARIA_WQ4) {
            /* FM >= 3, Q4: one MFMA step's fragments at a time, requested before that step's
             * unpacking (+8 VGPRs; the Q8 kernels would cross 256 registers and lose their
             * second wave per SIMD) */
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                half8_t xs[FM];
#pragma unroll
                for (int i = 0; i < FM; i++) xs[i] = *reinterpret_cast<const half8_t *>(&X[xoff(i * 32 + lrow, 4 * lh + ks)]);
                __builtin_amdgcn_sched_barrier(0);
                const half8_t w0 = wr_frag<WT>(ws, 0, ks, magic, f0), w1 = wr_frag<WT>(ws, 1, ks, magic, f1);
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w0, xs[i], acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1, xs[i], acc[i][1], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const half8_t w0 = wr_frag<WT>(ws, 0, ks, magic, f0), w1 = wr_frag<WT>(ws, 1, ks, magic, f1);
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    const half8_t x = *reinterpret_cast<const half8_t *>(&X[xoff(i * 32 + lrow, 4 * lh + ks)]);
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w0, x, acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1, x, acc[i][1], 0, 0, 0);
                }
            }
        }
    };

    xload(IC<0>{}, 0);
    wr_load<WT>(a, s0, nrow, 0, lh);
    if (KT > 1) {
        xload(IC<1>{}, 1);
        wr_load<WT>(a, s1, nrow, 1, lh);
    }
    if constexpr (DP == 3) {
        if (KT > 2) {
            xload(IC<2>{}, 2);
            wr_load<WT>(a, s2, nrow, 2, lh);
        }
    }
    xstore(IC<0>{}, 0);
    /* drain the prologue's loads: the loop header then inherits only the steady-state
     * wait counts (otherwise the merged state makes the first step of every iteration
     * wait for loads issued one step earlier) */
    __builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0) */
    __syncthreads();
    /* step kt (kt % U == P): tile kt+DP loaded (weights into stage (P+DP) % (DP+1),
     * activations into set P % DP), tile kt multiplied out of LDS buffer P & 1 with stage
     * P % (DP+1), tile kt+1 stored from set (P+1) % DP into the other buffer. GUARD: the
     * tail form. U = lcm(DP + 1, DP, 2) steps are unrolled so every index is a constant. */
    constexpr int U = DP == 2 ? 6 : 12;
    auto step = [&](auto PP, auto GUARD, int kt) __attribute__((always_inline)) {
        constexpr int P = decltype(PP)::value;
        constexpr bool guard = decltype(GUARD)::value;
        if (!guard || kt + DP < KT) {
            wr_load<WT>(a, wsel(IC<(P + DP) % (DP + 1)>{}), nrow, kt + DP, lh);
            xload(IC<P % DP>{}, kt + DP);
        }
        compute(IC<P % (DP + 1)>{}, P & 1);
        if (!guard || kt + 1 < KT) xstore(IC<(P + 1) % DP>{}, (P + 1) & 1);
        __syncthreads();
    };
    using F = std::false_type;
    using G = std::true_type;
    int kt = 0;
    for (; kt + U + DP <= KT; kt += U)
        static_for<U>([&](auto PP) __attribute__((always_inline)) { step(PP, F{}, kt + decltype(PP)::value); });
    for (; kt < KT; kt += U)
        static_for<U>([&](auto PP) __attribute__((always_inline)) {
            if (kt + decltype(PP)::value < KT) step(PP, G{}, kt + decltype(PP)::value);
        });

    float *E = reinterpret_cast<float *>(lds) + wave * (32 * EPI_STRIDE / 4);
    epilogue<FM, FN, WT, MODE, GELU>(a, acc, E, lane, m0, n0 + wave * 64);
}

template <int WT, int FM, int MODE, bool GELU = false>
static void launch_wr_m(const QArgs &a, hipStream_t s) {
    constexpr int BM = 32 * FM, BN = 256;
    const int MT = (a.M + BM - 1) / BM, NTN = (a.N + BN - 1) / BN, T = MT * NTN;
    const int grid = ((T + 7) / 8) * 8;
    hipLaunchKernelGGL((k_qgemm_wr<WT, FM, (FM <= 2 ? 2 : 1), MODE, GELU>), dim3(grid), dim3(256), 0, s, a, NTN, T);
}
/* one kernel per fused epilogue mode: a run-time mode switch inside the store loop
 * makes every store wait for the loads of the modes that read. GELU is compiled in for
 * the plain store only (the FFN input projection); the caller sends GELU with another
 * mode to the LDS-operand kernel. */
template <int WT, int FM>
static void launch_wr(const QArgs &a, hipStream_t s) {
    switch (a.epi.mode) {
        case ARIA_EPI_GATE_RES: launch_wr_m<WT, FM, ARIA_EPI_GATE_RES>(a, s); break;
        case ARIA_EPI_ADD: launch_wr_m<WT, FM, ARIA_EPI_ADD>(a, s); break;
        case ARIA_EPI_HEADS: launch_wr_m<WT, FM, ARIA_EPI_HEADS>(a, s); break;
        case ARIA_EPI_GLU: launch_wr_m<WT, FM, ARIA_EPI_GLU>(a, s); break;
        default:
            if (a.gelu) launch_wr_m<WT, FM, ARIA_EPI_STORE, true>(a, s);
            else launch_wr_m<WT, FM, ARIA_EPI_STORE>(a, s);
            break;
    }
}

hipError_t qgemm_wr_launch(const QArgs &a, int wt, int fm, hipStream_t s) {
    if (wt == ARIA_WQ8) {
        switch (fm) {
            case 1: launch_wr<ARIA_WQ8, 1>(a, s); break;
            case 2: launch_wr<ARIA_WQ8, 2>(a, s); break;
            case 3: launch_wr<ARIA_WQ8, 3>(a, s); break;
            default: launch_wr<ARIA_WQ8, 4>(a, s); break;
        }
    } else if (wt == ARIA_WQ4) {
        switch (fm) {
            case 1: launch_wr<ARIA_WQ4, 1>(a, s); break;
            case 2: launch_wr<ARIA_WQ4, 2>(a, s); break;
            case 3: launch_wr<ARIA_WQ4, 3>(a, s); break;
            default: launch_wr<ARIA_WQ4, 4>(a, s); break;
        }
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
