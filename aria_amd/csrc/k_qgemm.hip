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
 * Tiling: 256 threads = 4 waves in a WGM x WGN grid; each wave owns FM x FN blocks of
 * 32x32 computed with v_mfma_f32_32x32x16_f16 as W x^T (two MFMAs per 32-wide K slice),
 * so a lane's accumulators hold 4 consecutive n of one m. Workgroup tiles run from
 * 64x64 to 192x128 / 128x256 (m x n), picked per shape (pick_tiles).
 * Pipeline: a ring of three register stages holds raw (still packed) slices; the
 * global loads of slice k+3 are issued while slice k is multiplied out of LDS, so each
 * load has two slice-times to land; a slice is unpacked to fp16 only when it is stored
 * to the LDS double buffer (one barrier per slice). Loads past the M / N edge re-read the
 * last row, so the steady-state loop has no branches around its loads.
 * Epilogue: each wave stages 32 x 32*FN fp32 results at a time through LDS and writes
 * whole row segments (16 B per lane, coalesced), applying the Q8 scale, bias and GELU.
 * Operand layout of the 32x32x16 MFMA: lane l supplies row (l % 32) and the 8
 * consecutive k at 8*(l / 32); accumulator register r of lane l holds row
 * 8*(r/4) + 4*(l/32) + r%4, column l % 32.
 *
 * Shapes with K % 32 != 0, N % 4 != 0 or unaligned operands take a SIMT fp32 kernel with
 * the same dequant values (k_qgemm_simt).
 */
#include "qgemm_dev.h"

#define BK 32          /* k per slice */
#define LDS_STRIDE 32  /* halves per LDS row: 64 B, 4 chunks of 8 k */

/* LDS tiles are unpadded [rows][32] halves; chunk c of row r sits at position
 * c ^ ((r >> 2) & 3). The producers write one 16 B chunk per lane, four lanes per row
 * (the order that keeps their global loads coalesced), and the MFMA fragment reads take
 * 32 rows x 2 chunks per instruction: with this swizzle neither pattern has bank
 * conflicts on gfx950 (64 banks, 16 lanes per cycle for 16 B accesses). */
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * LDS_STRIDE + ((chunk ^ ((row >> 2) & 3)) << 3); }
/* producer slot c -> (row, chunk), row-major */
__device__ __forceinline__ int slot_row(int c) { return c >> 2; }
__device__ __forceinline__ int slot_chunk(int c) { return c & 3; }

/* ---- tile configuration: a 2-D grid of WGM x WGN waves, each owning FM x FN 32x32
 * blocks (FM along the activation rows m, FN along the weight rows n) ---- */
template <int FM_, int FN_, int WGM_, int WGN_>
struct Cfg {
    static constexpr int FM = FM_, FN = FN_, WGM = WGM_, WGN = WGN_;
    static constexpr int BM = 32 * FM * WGM, BN = 32 * FN * WGN, NT = 64 * WGM * WGN;
    /* workgroups per CU the register allocation must allow (two waves per SIMD, except
     * the 128-accumulator 128x256 tile, which runs one) */
    static constexpr int MINB = FM * FN >= 8 ? 1 : 2;
    /* epilogue staging: per wave 32 rows x 32*FN fp32, rows padded by 16 B */
    static constexpr int EPI_STRIDE = 32 * FN * 4 + 16;
    static constexpr int TILE_BYTES = 2 * (BM + BN) * LDS_STRIDE * 2, EPI_BYTES = 4 * 32 * EPI_STRIDE;
    static constexpr int LDS_BYTES = TILE_BYTES > EPI_BYTES ? TILE_BYTES : EPI_BYTES;
};

/* per-thread staging of one BK slice in its global encoding; every chunk is 8 k of one
 * row: activations 16 B fp16 or 32 B fp32, weights 8 B int8 (Q8), 4 B nibbles + the
 * block's [min, step] (Q4), 16 B fp16 */
template <class C, int WT, bool AF16>
struct Stage {
    static constexpr int CH = C::BM * (BK / 8), XI = (CH + C::NT - 1) / C::NT, XW = AF16 ? 4 : 8;
    static constexpr int WCH = C::BN * (BK / 8), WI = (WCH + C::NT - 1) / C::NT;
    static constexpr int WW = (WT == ARIA_WQ8) ? 2 : (WT == ARIA_WQ4) ? 3 : 4;
    static_assert(C::BM % 32 == 0 && C::BN % 32 == 0, "tiles are whole MFMA blocks");
    uint32_t x[XI][XW];
    uint32_t w[WI][WW];
};

template <class C, int WT, bool AF16>
struct Tile {
    using S = Stage<C, WT, AF16>;
    const QArgs &q;
    int tid, m0, n0;
    uint16_t *Xs, *Ws;   /* [2][rows * LDS_STRIDE] */

    /* rows past the edge re-read the last row: their products land only in output rows
     * or columns the epilogue never stores, and the branch-free loads keep the vmcnt
     * accounting exact so the prefetch stays in flight */
    __device__ __forceinline__ void load(S &s, int kt) const {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < S::XI; i++) {
            const int c = tid + i * C::NT;
            if (S::CH % C::NT != 0 && c >= S::CH) break;
            const int m = min(m0 + slot_row(c), q.M - 1), k = k0 + 8 * slot_chunk(c);
            if (AF16) {
                const uint4 u = *reinterpret_cast<const uint4 *>((const uint16_t *)q.x + (size_t)m * q.K + k);
                s.x[i][0] = u.x; s.x[i][1] = u.y; s.x[i][2] = u.z; s.x[i][3] = u.w;
            } else {
                const uint4 *p = reinterpret_cast<const uint4 *>((const float *)q.x + (size_t)m * q.K + k);
                const uint4 u0 = p[0], u1 = p[1];
                s.x[i][0] = u0.x; s.x[i][1] = u0.y; s.x[i][2] = u0.z; s.x[i][3] = u0.w;
                s.x[i][4] = u1.x; s.x[i][5] = u1.y; s.x[i][6] = u1.z; s.x[i][7] = u1.w;
            }
        }
#pragma unroll
        for (int i = 0; i < S::WI; i++) {
            const int c = tid + i * C::NT;
            if (S::WCH % C::NT != 0 && c >= S::WCH) break;
            const int n = min(n0 + slot_row(c), q.N - 1), k = k0 + 8 * slot_chunk(c);
            if (WT == ARIA_WQ8) {
                const uint2 u = *reinterpret_cast<const uint2 *>((const int8_t *)q.q + (size_t)n * q.K + k);
                s.w[i][0] = u.x; s.w[i][1] = u.y;
            } else if (WT == ARIA_WQ4) {
                s.w[i][0] = *reinterpret_cast<const uint32_t *>((const uint8_t *)q.q + (size_t)n * (q.K >> 1) + (k >> 1));
                const uint2 pr = *reinterpret_cast<const uint2 *>(q.scale + ((size_t)n * q.nblk + (k >> 5)) * 2);
                s.w[i][1] = pr.x; s.w[i][2] = pr.y;
            } else {
                const uint4 u = *reinterpret_cast<const uint4 *>((const uint16_t *)q.q + (size_t)n * q.K + k);
                s.w[i][0] = u.x; s.w[i][1] = u.y; s.w[i][2] = u.z; s.w[i][3] = u.w;
            }
        }
    }

    /* unpack to fp16 and write the slice into LDS buffer buf */
    __device__ __forceinline__ void store(const S &s, int buf) const {
        uint16_t *X = Xs + buf * (C::BM * LDS_STRIDE), *W = Ws + buf * (C::BN * LDS_STRIDE);
#pragma unroll
        for (int i = 0; i < S::XI; i++) {
            const int c = tid + i * C::NT;
            if (S::CH % C::NT != 0 && c >= S::CH) break;
            uint4 o;
            if (AF16) {
                o = make_uint4(s.x[i][0], s.x[i][1], s.x[i][2], s.x[i][3]);
            } else {
                const float *f = reinterpret_cast<const float *>(s.x[i]);
                o = make_uint4(pack2h(f[0], f[1]), pack2h(f[2], f[3]), pack2h(f[4], f[5]), pack2h(f[6], f[7]));
            }
            *reinterpret_cast<uint4 *>(&X[lds_off(slot_row(c), slot_chunk(c))]) = o;
        }
#pragma unroll
        for (int i = 0; i < S::WI; i++) {
            const int c = tid + i * C::NT;
            if (S::WCH % C::NT != 0 && c >= S::WCH) break;
            uint4 o;
            if (WT == ARIA_WQ8) {
                q8x4_to_h(s.w[i][0], o.x, o.y);
                q8x4_to_h(s.w[i][1], o.z, o.w);
            } else if (WT == ARIA_WQ4) {
                /* w = min + nib * step in fp32 (the reference's dequant value), rounded to
                 * fp16; even k in the low nibble */
                const float mn = __builtin_bit_cast(float, s.w[i][1]), st = __builtin_bit_cast(float, s.w[i][2]);
                const uint32_t lo = s.w[i][0] & 0x0F0F0F0Fu, hi = (s.w[i][0] >> 4) & 0x0F0F0F0Fu;
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    h[e] = pack2h(__builtin_fmaf((float)((lo >> (8 * e)) & 0xFF), st, mn),
                                  __builtin_fmaf((float)((hi >> (8 * e)) & 0xFF), st, mn));
                o = make_uint4(h[0], h[1], h[2], h[3]);
            } else {
                o = make_uint4(s.w[i][0], s.w[i][1], s.w[i][2], s.w[i][3]);
            }
            *reinterpret_cast<uint4 *>(&W[lds_off(slot_row(c), slot_chunk(c))]) = o;
        }
    }
};

template <class C, int WT, bool AF16>
__global__ __launch_bounds__(C::NT, C::MINB) void k_qgemm_mfma(QArgs a, int NTN, int T) {
    using TL = Tile<C, WT, AF16>;
    using S = typename TL::S;
    constexpr int FM = C::FM, FN = C::FN, BM = C::BM, BN = C::BN;
    __shared__ __attribute__((aligned(16))) uint16_t lds[C::LDS_BYTES / 2];
    uint16_t *Xs = lds, *Ws = lds + 2 * BM * LDS_STRIDE;

    const int t = xcd_tile(blockIdx.x, T);
    if (t >= T) return;                     /* uniform per workgroup */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WGN, wn = wave % C::WGN;
    const TL tl{a, tid, (t / NTN) * BM, (t % NTN) * BN, Xs, Ws};
    const int KT = a.K / BK;

    /* acc[i][j]: the 32x32 block (weight rows j, activation rows i), computed as
     * W x^T so a lane holds 4 consecutive n of one m */
    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int lrow = lane & 31, lh = lane >> 5;
    auto compute = [&](int buf) {
        const uint16_t *X = Xs + buf * (BM * LDS_STRIDE), *W = Ws + buf * (BN * LDS_STRIDE);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            half8_t xf[FM], wf[FN];
#pragma unroll
            for (int j = 0; j < FN; j++)
                wf[j] = *reinterpret_cast<const half8_t *>(&W[lds_off(wn * 32 * FN + j * 32 + lrow, 2 * ks + lh)]);
#pragma unroll
            for (int i = 0; i < FM; i++)
                xf[i] = *reinterpret_cast<const half8_t *>(&X[lds_off(wm * 32 * FM + i * 32 + lrow, 2 * ks + lh)]);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[j], xf[i], acc[i][j], 0, 0, 0);
        }
    };

    /* ring of three register stages: at slice kt, stage (kt+1)%3 holds slice kt+1 and
     * stage kt%3 receives slice kt+3. Steady-state steps store and load unconditionally
     * (no path without the loads, so the compiler's vmcnt waits stay exact); the last
     * few steps run the guarded form. */
    S s0, s1, s2;
    tl.load(s0, 0);
    if (KT > 1) tl.load(s1, 1);
    if (KT > 2) tl.load(s2, 2);
    tl.store(s0, 0);
    __syncthreads();
    auto full = [&](int kt, S &nxt, S &fill) {
        compute(kt & 1);
        tl.store(nxt, (kt + 1) & 1);
        tl.load(fill, kt + 3);
        __syncthreads();
    };
    auto step = [&](int kt, S &nxt, S &fill) {
        compute(kt & 1);
        if (kt + 1 < KT) tl.store(nxt, (kt + 1) & 1);
        if (kt + 3 < KT) tl.load(fill, kt + 3);
        __syncthreads();
    };
    int kt = 0;
    for (; kt + 6 <= KT; kt += 3) {
        full(kt, s1, s0);
        full(kt + 1, s2, s1);
        full(kt + 2, s0, s2);
    }
    for (; kt + 3 <= KT; kt += 3) {
        step(kt, s1, s0);
        step(kt + 1, s2, s1);
        step(kt + 2, s0, s2);
    }
    if (kt < KT) step(kt, s1, s0);
    if (kt + 1 < KT) step(kt + 1, s2, s1);

    /* the last slice's barrier has released the tile buffers */
    float *E = reinterpret_cast<float *>(lds) + wave * (32 * C::EPI_STRIDE / 4);
    epilogue<FM, FN, WT, EPI_ANY>(a, acc, E, lane, tl.m0 + wm * 32 * FM, tl.n0 + wn * 32 * FN);
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

template <class C, int WT, bool AF16>
static void launch_cfg(const QArgs &a, hipStream_t s) {
    const int MT = (a.M + C::BM - 1) / C::BM, NTN = (a.N + C::BN - 1) / C::BN, T = MT * NTN;
    const int grid = ((T + 7) / 8) * 8;
    hipLaunchKernelGGL((k_qgemm_mfma<C, WT, AF16>), dim3(grid), dim3(C::NT), 0, s, a, NTN, T);
}

/* workgroup tiles (activation rows x weight rows), index = the `tiles` argument - 1 */
using C1 = Cfg<3, 2, 2, 2>;   /* 192 x 128 */
using C2 = Cfg<2, 2, 2, 2>;   /* 128 x 128 */
using C3 = Cfg<3, 2, 1, 4>;   /*  96 x 256 */
using C4 = Cfg<3, 1, 1, 4>;   /*  96 x 128 */
using C5 = Cfg<2, 4, 2, 2>;   /* 128 x 256 */
using C6 = Cfg<1, 2, 2, 2>;   /*  64 x 128 */
using C7 = Cfg<2, 1, 2, 2>;   /* 128 x  64 */
using C8 = Cfg<1, 1, 2, 2>;   /*  64 x  64 */
#define NCFG 8
static const int cfg_bm[NCFG] = {192, 128, 96, 96, 128, 64, 128, 64};
static const int cfg_bn[NCFG] = {128, 128, 256, 128, 256, 128, 64, 64};
static const int cfg_fn[NCFG] = {2, 2, 2, 1, 4, 2, 1, 1};   /* 32x32 blocks per wave along n */

/* Tile shape from the shape (measured on MI355X at the DiT's shapes): the largest tile
 * that still gives every CU about two workgroups wins (per-tile efficiency grows with
 * the tile, but a tile count near the CU count leaves CUs idle at the tail); when none
 * does, the one with the most tiles. Order of preference: 192x128, 128x128, 64x128 /
 * 128x64, 64x64. HEADS epilogues need a 64-column head inside one wave (FN >= 2). */
static int pick_tiles(int M, int N, bool heads) {
    static const int order[5] = {0, 1, 5, 6, 7};
    int most = -1;
    long most_t = -1;
    for (int k = 0; k < 5; k++) {
        const int i = order[k];
        if (heads && cfg_fn[i] < 2) continue;   /* a head's 64 columns must sit in one wave */
        const long T = (long)((M + cfg_bm[i] - 1) / cfg_bm[i]) * ((N + cfg_bn[i] - 1) / cfg_bn[i]);
        if (T >= 384) return i;
        if (T > most_t) { most_t = T; most = i; }
    }
    return most;
}

/* Weights-in-registers kernel pick (Q8/Q4, fp16 activations, K % 64 == 0): BM = 32 * FM
 * rows by 256 weight rows per workgroup, FM = 1..4. Cost model fitted to MI355X sweeps of
 * the DiT's GEMMs (M = 2592; N/K = 3072/1024, 1024/1024, 4096/1024, 1024/4096,
 * 8192/1024): rounds of workgroups over 256 CUs (two resident per CU for FM <= 2) times
 * the per-workgroup time, which grows with FM and with the workgroups sharing a CU,
 * scaled by a per-FM efficiency (LDS and L1 traffic per MFMA fall with FM; FM = 4 runs one
 * wave per SIMD and hides less latency). */
static int pick_wr(int M, int N, int K) {
    (void)K;
    static const float eff[5] = {0.0f, 1.6f, 1.25f, 1.1f, 1.35f};
    int best = 2;
    float best_c = 1e30f;
    for (int fm = 1; fm <= 4; fm++) {
        const long T = (long)((M + 32 * fm - 1) / (32 * fm)) * ((N + 255) / 256);
        const int occ = fm <= 2 ? 2 : 1;
        const long rounds = (T + 256L * occ - 1) / (256L * occ);
        const long share = T >= 256 * occ ? occ : (T + 255) / 256;   /* workgroups per CU at once */
        const float c = (float)(rounds * fm * (share < 1 ? 1 : share)) * eff[fm];
        if (c < best_c) { best_c = c; best = fm; }
    }
    return best;
}

template <int WT, bool AF16>
static hipError_t launch_q(const QArgs &a, int tiles, hipStream_t s) {
    const bool aligned = a.K % BK == 0 && a.N % 4 == 0 && ((uintptr_t)a.x & 15u) == 0 &&
                         ((uintptr_t)a.q & 15u) == 0 && ((uintptr_t)a.y & 15u) == 0 &&
                         (a.bias == nullptr || ((uintptr_t)a.bias & 15u) == 0) &&
                         (WT != ARIA_WQ8 || ((uintptr_t)a.scale & 15u) == 0) &&
                         (WT != ARIA_WQ4 || ((uintptr_t)a.scale & 7u) == 0);
    if (!aligned) {
        if (a.epi.mode != ARIA_EPI_STORE) return hipErrorInvalidValue;   /* fused epilogues need the MFMA path */
        dim3 grid((a.N + 63) / 64, (a.M + 63) / 64);
        hipLaunchKernelGGL((k_qgemm_simt<WT, AF16>), grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    if constexpr (!AF16) {   /* fp32 activations: the fallback when no fp16 staging buffer was available */
        if (a.epi.mode == ARIA_EPI_HEADS) return hipErrorInvalidValue;
        launch_cfg<C2, WT, AF16>(a, s);
        return hipGetLastError();
    } else {
    if constexpr (WT == ARIA_WF16) {
        /* fp16 weights on the LDS-DMA kernel: explicit tiles 13.., or the configuration that
         * qgemm_big_f16_pick chooses for the shape (HEADS, which needs 64 columns per wave,
         * stays on the LDS-operand kernel) */
        if (tiles >= 13) return qgemm_big_launch(a, WT, tiles - 13, s);
        if (tiles == 0 && a.K % 64 == 0 && (!a.gelu || a.epi.mode == ARIA_EPI_STORE) &&
            a.epi.mode != ARIA_EPI_HEADS)
            return qgemm_big_launch(a, WT, qgemm_big_f16_pick(a.M, a.N), s);
    }
    if constexpr (WT != ARIA_WF16) {
        /* the LDS-DMA kernel (k_qgemm_big.hip): explicit tiles 13.. (configuration tiles - 13),
         * or picked for the shapes where it measured fastest: N <= 1024 without HEADS (96 x 128
         * tiles, two workgroups per CU), HEADS with N <= 3072 (the qkv projection: 64 x 512 in
         * 8-wave workgroups, one per CU), other N <= 3072 without HEADS (128 x 128, two per CU), N = 4096
         * (192 x 256 in 8-wave workgroups, one per CU) and wider (224 x 128); N <= 1024 with an
         * even number of K-tiles in 96 x 128
         * tiles of 8 waves, the two halves of K on their own pipelines (216 tiles at M = 2592
         * leave 40 CUs idle; the split doubles the waves on the busy ones), and HEADS with N <=
         * 1024 (ca_q) likewise in 64 x 256 tiles (164 tiles: one workgroup per busy CU, so the
         * split's second half is what gives those CUs two waves per SIMD; 15.6 -> 15.2 us);
         * HEADS wider than 3072 stays on the weights-in-registers kernel */
        if (tiles >= 13) return qgemm_big_launch(a, WT, tiles - 13, s);
        if (tiles == 0 && a.K % 64 == 0 && (WT != ARIA_WQ4 || ((uintptr_t)a.scale & 15u) == 0) &&
            (!a.gelu || a.epi.mode == ARIA_EPI_STORE)) {
            const bool heads = a.epi.mode == ARIA_EPI_HEADS;
            const int cfg = heads ? (a.N <= 1024 && (a.K / 64) % 2 == 0 ? 6 : a.N <= 3072 ? 8 : -1)
                          : a.N <= 1024 ? ((a.K / 64) % 2 == 0 ? 5 : 0) : a.N <= 3072 ? 1 : a.N <= 4096 ? 7 : 4;
            if (cfg >= 0) return qgemm_big_launch(a, WT, cfg, s);
        }
        /* weights-in-registers kernel: explicit tiles 9..12 (BM = 32 * (tiles - 8)), or the pick */
        int fm = (tiles > NCFG) ? tiles - NCFG : (tiles == 0 ? pick_wr(a.M, a.N, a.K) : 0);
        /* Q8 with N and K <= 1024 (the DiT's sa_out / ca_out): 64 x 64 LDS-operand tiles, 2.5
         * workgroups per CU, measured 8 % faster than the weights-in-registers pick */
        if (tiles == 0 && WT == ARIA_WQ8 && a.N <= 1024 && a.K <= 1024 && a.epi.mode != ARIA_EPI_HEADS) fm = 0;
        const bool wr_ok = a.K % 64 == 0 && (!a.gelu || a.epi.mode == ARIA_EPI_STORE);
        if (fm > 0 && wr_ok) return qgemm_wr_launch(a, WT, fm, s);
        if (tiles == 0 && fm == 0 && WT == ARIA_WQ8 && a.N <= 1024 && a.K <= 1024 && a.epi.mode != ARIA_EPI_HEADS) {
            launch_cfg<C8, WT, AF16>(a, s);
            return hipGetLastError();
        }
    }
    int c = (tiles >= 1 && tiles <= NCFG) ? tiles - 1 : pick_tiles(a.M, a.N, a.epi.mode == ARIA_EPI_HEADS);
    if (a.epi.mode == ARIA_EPI_HEADS && cfg_fn[c] < 2) c = pick_tiles(a.M, a.N, true);
    switch (c) {
        case 0: launch_cfg<C1, WT, AF16>(a, s); break;
        case 1: launch_cfg<C2, WT, AF16>(a, s); break;
        case 2: launch_cfg<C3, WT, AF16>(a, s); break;
        case 3: launch_cfg<C4, WT, AF16>(a, s); break;
        case 4: launch_cfg<C5, WT, AF16>(a, s); break;
        case 5: launch_cfg<C6, WT, AF16>(a, s); break;
        case 6: launch_cfg<C7, WT, AF16>(a, s); break;
        default: launch_cfg<C8, WT, AF16>(a, s); break;
    }
    return hipGetLastError();
    }
}

extern "C" hipError_t aria_k_qgemm_e(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                                     const float *scale, const float *bias, int M, int K, int N, int tiles,
                                     int gelu, const aria_qgemm_epi *epi, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    QArgs a;
    a.y = y; a.x = x; a.q = q; a.scale = scale; a.bias = bias;
    a.M = M; a.K = K; a.N = N; a.y_f16 = y_f16; a.nblk = (K + 31) / 32; a.gelu = gelu;
    a.xscale = nullptr;
    if (epi) a.epi = *epi;
    else { memset(&a.epi, 0, sizeof a.epi); a.epi.mode = ARIA_EPI_STORE; }
    if (a.epi.mode == ARIA_EPI_HEADS) {
        if (N % 64 || a.epi.nsec < 1 || a.epi.nsec > 3 || a.epi.heads * 64 * a.epi.nsec != N ||
            a.epi.rows_per_batch <= 0 || (a.epi.rot && (a.epi.rot > 64 || (a.epi.rot & 7)))) return hipErrorInvalidValue;
        a.y = (void *)a.epi.dst[0];   /* alignment check only; y is not written */
    } else if (a.epi.mode == ARIA_EPI_GLU) {
        if (N % 4 || a.gelu) return hipErrorInvalidValue;
    } else if (a.epi.mode == ARIA_EPI_ADD_DYT) {   /* the decoder's fp16-weight GEMMs only */
        if (wtype != ARIA_WF16 || !x_f16 || y_f16 || a.gelu || a.epi.rows_per_batch <= 0 || !a.epi.dst[0] ||
            !a.epi.w[0] || !a.epi.w[1] || ((uintptr_t)a.epi.dst[0] & 7u) || ((uintptr_t)a.epi.w[0] & 15u) ||
            ((uintptr_t)a.epi.w[1] & 15u))
            return hipErrorInvalidValue;
    } else if (a.epi.mode == ARIA_EPI_DYT_ROPE) {   /* the decoder's to_qkv only */
        const aria_qgemm_epi &e = a.epi;
        const int rot = e.rot;
        bool ok = wtype == ARIA_WF16 && x_f16 && !y_f16 && !a.gelu && e.heads > 0 && N == 5 * 64 * e.heads &&
                  e.rows_per_batch > 0 && (rot == 0 || rot == 8 || rot == 16 || rot == 32);
        for (int i = 0; ok && i < 4; i++) ok = e.w[i] && ((uintptr_t)e.w[i] & 15u) == 0;
        if (ok && rot) ok = e.cos_t && e.sin_t && ((uintptr_t)e.cos_t & 15u) == 0 && ((uintptr_t)e.sin_t & 15u) == 0;
        if (!ok) return hipErrorInvalidValue;
    } else if (a.epi.mode > ARIA_EPI_DYT_ROPE || a.epi.mode < 0) {
        return hipErrorInvalidValue;
    } else if (a.epi.mode != ARIA_EPI_STORE) {
        if (y_f16 || a.epi.rows_per_batch <= 0) return hipErrorInvalidValue;
    }
    if (wtype == ARIA_WQ8) return x_f16 ? launch_q<ARIA_WQ8, true>(a, tiles, s) : launch_q<ARIA_WQ8, false>(a, tiles, s);
    if (wtype == ARIA_WQ4) return x_f16 ? launch_q<ARIA_WQ4, true>(a, tiles, s) : launch_q<ARIA_WQ4, false>(a, tiles, s);
    if (wtype == ARIA_WF16)
        return x_f16 ? launch_q<ARIA_WF16, true>(a, tiles, s) : launch_q<ARIA_WF16, false>(a, tiles, s);
    return hipErrorInvalidValue;
}

extern "C" hipError_t aria_k_qgemm_t(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                                     const float *scale, const float *bias, int M, int K, int N, int tiles,
                                     int gelu, hipStream_t s) {
    return aria_k_qgemm_e(y, y_f16, x, x_f16, wtype, q, scale, bias, M, K, N, tiles, gelu, nullptr, s);
}

extern "C" hipError_t aria_k_qgemm(void *y, int y_f16, const void *x, int x_f16, int wtype, const void *q,
                                   const float *scale, const float *bias, int M, int K, int N, hipStream_t s) {
    return aria_k_qgemm_t(y, y_f16, x, x_f16, wtype, q, scale, bias, M, K, N, 0, 0, s);
}
