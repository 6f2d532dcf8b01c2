/*
 * k_qgemm_big.hip - the large-tile dequant-on-use GEMM (gfx950 MFMA):
 * y[M,N] = x[M,K] W[N,K]^T (+ b) for Q8 / Q4 / fp16 weights and fp16 activations (and the
 * W8A8 int8 form), K % 64 == 0.
 * Replaces the same reference functions as k_qgemm.hip (aria_linear_q8 / aria_linear_q4,
 * src/aria_quant.c:98-145, 469-538; the reference's device form dequantizes into an fp16
 * scratch and calls cublasGemmEx, src/aria_cuda.cu:1009-1035). Shares the argument block,
 * the unpack and the fused epilogue with the other GEMM kernels (qgemm_dev.h).
 *
 * Workgroup: 4 waves share one activation tile of BM = 32 FM rows; wave w owns FN blocks
 * of 32 weight rows (BN = 128 FN per workgroup). Both operands travel HBM -> LDS by LDS DMA
 * (global_load_lds_dwordx4: no staging registers, no VALU): the activation tile is spread over
 * all four waves' transfers and read by all of them; wave w moves its own weight rows and reads
 * them back in the MFMA operand layout (Q8 / Q4 unpacked in registers, fp16 and int8 used as
 * they are). The cost that grows with the tile is the unpack: each weight is unpacked once per
 * workgroup and feeds BM rows, so unpack VALU per MFMA falls as 1 / FM.
 *
 * Pipeline, K-tile 64 (128 for int8), NST = 3 stages: K-tile t lands in stage t % 3 two
 * K-tiles before it is multiplied. Step t: issue the transfers of t + 2, multiply t, wait for
 * this wave's transfers of t + 1 (vmcnt, the ones of t + 2 stay in flight), barrier. The
 * barrier carries no memory fence (a fence would drain every transfer in flight) but waits
 * for the step's LDS reads (lgkmcnt(0)): stage t % 3 is refilled by the transfers issued in
 * step t + 1, so no fragment read of step t may still be in flight when any wave passes the
 * barrier. Stage offsets are compile-time constants (the loop is unrolled by NST), and the
 * transfers are inline assembly with a memory clobber, so the compiler neither waits for them
 * nor moves fragment reads across them.
 *
 * Contraction order inside a K-tile (as in k_qgemm_wr.hip): lane half h = l / 32 covers
 * k in [32h, 32h + 32) and MFMA step ks its 8 k at 32h + 8ks, for both operands; a Q4
 * lane's range is exactly one quantization block (one [min, step] pair per K-tile). So the
 * accumulation order over k, and with it every output bit, equals k_qgemm_wr's.
 */
#include "qgemm_dev.h"

namespace {

constexpr int KB = 64;   /* K-tile (fp16 activations) */
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

/* activation tile [BM][64] halves: 8 chunks of 16 B per row, logical chunk c of row r at
 * c ^ ((r >> 1) & 7) (conflict-free fragment reads: 32 rows x one chunk per lane half) */
__device__ __forceinline__ int xo(int r, int c) { return r * KB + ((c ^ ((r >> 1) & 7)) << 3); }

template <int WT, int FN>
struct WSt {              /* one lane's raw weights of one K-tile, FN 32-row blocks */
    static constexpr int NW = (WT == ARIA_WQ8) ? 8 : 6;   /* Q8: 32 B; Q4: 16 B nibbles + [min, step] */
    uint32_t w[FN][NW];
};

__device__ __forceinline__ uint32_t and_or_v(uint32_t w, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(mask), "v"(magic));
    return r;
}

/* the per-block offsets of the Q4 unpack: (1024 + n) * step + (min - 1024 step) = min + n step
 * for a low nibble, (1024 + 16 n) * step / 16 + (min - 64 step) for a high one */
struct QOff { float a, b, st, s16; };
template <int WT, int FN>
__device__ __forceinline__ QOff qoff(const WSt<WT, FN> &s, int j) {
    QOff o;
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

/* the 8 fp16 weights of block j for MFMA step ks (see k_qgemm_wr.hip for the arithmetic:
 * the value the reference dequantizes, rounded to fp16) */
template <int WT, int FN>
__device__ __forceinline__ half8_t wfrag(const WSt<WT, FN> &s, int j, int ks, uint32_t magic, const QOff &f) {
    uint32_t o[4];
    if constexpr (WT == ARIA_WQ4) {
        const uint32_t w = s.w[j][ks], u = w >> 8;
        const half2_t t0 = __builtin_bit_cast(half2_t, and_or_v(w, 0x000F000Fu, magic));
        const half2_t t1 = __builtin_bit_cast(half2_t, and_or_v(w, 0x00F000F0u, magic));
        const half2_t t2 = __builtin_bit_cast(half2_t, and_or_v(u, 0x000F000Fu, magic));
        const half2_t t3 = __builtin_bit_cast(half2_t, and_or_v(u, 0x00F000F0u, magic));
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

/* s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding) */
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

/* One LDS DMA instruction: every lane moves 16 B from global address g to LDS byte address
 * m0 + 16 * lane (m0 wave-uniform). Issued as inline assembly, so the compiler neither waits
 * for it nor reorders memory accesses across it: the kernel waits on vmcnt itself. */
__device__ __forceinline__ void dma16(const void *g, uint32_t m0) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(m0);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m), "v"(g) : "memory");
}

/* Layout of one pipeline stage in LDS (bytes):
 *   [0, 128 BM)            activations [BM][64] fp16 (W8A8: [BM][128] int8), chunk-swizzled (xo)
 *   Q8: [.., + 64 BN)      weights [BN][64] int8; 16 B chunk c of row r at c ^ ((r >> 2) & 3)
 *   W8A8: [.., + 128 BN)   weights [BN][128] int8, chunk-swizzled as the activations
 *   fp16: [.., + 128 BN)   weights [BN][64] fp16, chunk-swizzled as the activations
 *   Q4: [.., + 32 BN)      nibbles [BN][32 B]
 *       [.., + 4096 NSP)   [min, step] pairs of the K-tile, 16 B per row: wave w's 64 slots
 *                          at 1024 w (FN = 1: rows 32w.. in slots 0-31, 32-63 repeat them)
 * NSP = 2: 8 waves share the activation tile, each moving half as many of its slots, and
 * own 32 FN weight rows each (BN = 256 FN). */
template <int WT, int FM, int FN, int NSP = 1>
struct Stage {
    static constexpr int BM = 32 * FM, BN = 128 * FN * NSP;
    static constexpr int A = BM * 128;
    static constexpr int WQ = (WT == ARIA_WI8 || WT == ARIA_WF16) ? BN * 128 : WT == ARIA_WQ8 ? BN * 64 : BN * 32;
    static constexpr int WS = WT == ARIA_WQ4 ? 4096 * NSP : 0;
    static constexpr int BYTES = A + WQ + WS;
    /* activation transfers per wave and K-tile: the tile's 256 FM slots of 16 B over 4 NSP waves */
    static constexpr int AD = FM / NSP;
    /* VMEM instructions one wave issues per K-tile */
    static constexpr int DMA = AD + ((WT == ARIA_WI8 || WT == ARIA_WF16) ? 4 * FN : WT == ARIA_WQ8 ? 2 * FN : FN + 1);
    /* k per K-tile: 64 fp16 activations, or 128 int8 ones (W8A8), in the 128-byte rows */
    static constexpr int KK = WT == ARIA_WI8 ? 128 : 64;
};

}  // namespace

/* One tile per workgroup; MINB workgroups per CU (MINB = 2 when the tile's registers and
 * LDS allow two: the second workgroup's waves cover one workgroup's barrier waits and its
 * epilogue). The tiles of an XCD are a contiguous run in M-major order (xcd_tile). Wave w
 * owns weight rows [32 FN w, 32 FN (w + 1)) and every activation row of the tile. */
template <int WT, int FM, int FN, int MODE, bool GELU, int MINB, int NS, int NST, int KSPL, int NSP>
__global__ __launch_bounds__(256 * KSPL * NSP, MINB) void k_qgemm_big(QArgs a, int NTN, int T) {
    using St = Stage<WT, FM, FN, NSP>;   /* one 64-deep sub-tile; a pipeline stage holds NS of them */
    static_assert(NSP == 1 || (NSP == 2 && KSPL == 1 && FM % 2 == 0), "an N split of even row blocks, K unsplit");
    constexpr int SB = NS * St::BYTES;                                 /* stage bytes */
    constexpr int PD = NST - 1;                                        /* prefetch distance */
    static_assert(NST >= 2 && NST <= 4, "two to four stages");
    constexpr int BM = St::BM, BN = St::BN;
    constexpr int EPI_STRIDE = 32 * FN * 4 + 16;
    constexpr int EPI_WAVE = 32 * EPI_STRIDE;                          /* bytes per wave */
    static_assert(NST * SB >= 4 * NSP * EPI_WAVE, "the epilogue staging fits the stages");
    static_assert(KSPL == 1 || KSPL == 2, "one or two K halves");
    static_assert(KSPL * NST * SB <= 160 * 1024 / MINB, "the stages fit the LDS share of MINB workgroups");
    static_assert(KSPL == 1 || KSPL * NST * SB >= FM * FN * 16 * 256 * 4, "the second half's partial sums fit the stages");
    __shared__ __attribute__((aligned(16))) uint8_t smem_all[KSPL * NST * SB];

    const int t = xcd_tile(blockIdx.x, T);
    if (t >= T) return;                     /* uniform per workgroup, before any barrier */
    /* KSPL = 2: waves 4-7 run the second half of the K range on their own pipeline stages, and
     * their partial sums join the first half's before the epilogue (fixed order) */
    const int khalf = KSPL == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
    uint8_t *const smem = smem_all + khalf * (NST * SB);
    const int tid = threadIdx.x & (256 * NSP - 1), lane = tid & 63, wave = tid >> 6;
    const int lrow = lane & 31, lh = lane >> 5;
    const int KT = a.K / (St::KK * NS * KSPL);   /* pipeline steps of this half (host: divisible) */
    const int kofs = khalf * KT;                 /* this half's first step */
    uint32_t magic = 0x64006400u;           /* fp16 1024 in both halves, kept in a VGPR */
    asm volatile("" : "+v"(magic));
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;
    constexpr int NWQ = (WT == ARIA_WI8 || WT == ARIA_WF16) ? 4 * FN : WT == ARIA_WQ8 ? 2 * FN : FN;   /* weight DMA per wave */
    const int rbase = wave * 32 * FN;                    /* this wave's first weight row */

    /* per-lane global sources of this wave's DMA slots for K-tile 0 of tile (m0, n0);
     * K-tile kt adds kt * its step */
    const uint16_t *xsrc[St::AD];
    const uint8_t *wsrc[NWQ];
    const float *ssrc = nullptr;
    auto sources = [&](int m0, int n0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < St::AD; i++) {
            const int p = 256 * NSP * i + 64 * wave + lane, r = p >> 3, cp = p & 7;
            const int c = cp ^ ((r >> 1) & 7);
            if constexpr (WT == ARIA_WI8)   /* int8 rows: K bytes, 16 k per chunk */
                xsrc[i] = reinterpret_cast<const uint16_t *>((const int8_t *)a.x + (size_t)min(m0 + r, a.M - 1) * a.K + 16 * c);
            else
                xsrc[i] = (const uint16_t *)a.x + (size_t)min(m0 + r, a.M - 1) * a.K + 8 * c;
        }
#pragma unroll
        for (int i = 0; i < NWQ; i++) {
            const int p = 64 * i + lane;
            if constexpr (WT == ARIA_WI8 || WT == ARIA_WF16) {   /* 128-byte rows per K-tile */
                const int r = rbase + (p >> 3), c = (p & 7) ^ ((r >> 1) & 7);
                wsrc[i] = (const uint8_t *)a.q + (size_t)min(n0 + r, a.N - 1) * a.K * (WT == ARIA_WF16 ? 2 : 1) + 16 * c;
            } else if constexpr (WT == ARIA_WQ8) {
                const int r = rbase + (p >> 2), c = (p & 3) ^ ((r >> 2) & 3);
                wsrc[i] = (const uint8_t *)a.q + (size_t)min(n0 + r, a.N - 1) * a.K + 16 * c;
            } else {
                const int r = rbase + (p >> 1);
                wsrc[i] = (const uint8_t *)a.q + (size_t)min(n0 + r, a.N - 1) * (a.K >> 1) + 16 * (p & 1);
            }
        }
        if constexpr (WT == ARIA_WQ4) {
            const int r = rbase + (lane & (32 * FN - 1));
            ssrc = a.scale + (size_t)min(n0 + r, a.N - 1) * a.nblk * 2;
        }
    };
    /* all VMEM of step kt (sub-tiles NS kt .. NS kt + NS - 1) into stage B */
    auto issue = [&](int B, int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NS; u++) {
            const int k64 = NS * (kt + kofs) + u;
            const uint32_t st = sbase + B * SB + u * St::BYTES;
            if constexpr (WT == ARIA_WI8) {   /* 128 int8 k per K-tile: 128 bytes of every row */
#pragma unroll
                for (int i = 0; i < St::AD; i++)
                    dma16(reinterpret_cast<const uint8_t *>(xsrc[i]) + k64 * 128, st + (256 * NSP * i + 64 * wave) * 16);
#pragma unroll
                for (int i = 0; i < NWQ; i++) dma16(wsrc[i] + k64 * 128, st + St::A + rbase * 128 + 1024 * i);
                continue;
            }
#pragma unroll
            for (int i = 0; i < St::AD; i++) dma16(xsrc[i] + k64 * KB, st + (256 * NSP * i + 64 * wave) * 16);
            if constexpr (WT == ARIA_WF16) {
#pragma unroll
                for (int i = 0; i < NWQ; i++) dma16(wsrc[i] + k64 * 128, st + St::A + rbase * 128 + 1024 * i);
            } else if constexpr (WT == ARIA_WQ8) {
#pragma unroll
                for (int i = 0; i < NWQ; i++) dma16(wsrc[i] + k64 * KB, st + St::A + rbase * 64 + 1024 * i);
            } else {
#pragma unroll
                for (int i = 0; i < NWQ; i++) dma16(wsrc[i] + k64 * 32, st + St::A + rbase * 32 + 1024 * i);
                dma16(ssrc + 4 * k64, st + St::A + St::WQ + 1024 * wave);
            }
        }
    };
    constexpr int DMA = NS * St::DMA;        /* VMEM instructions of one step */

    using AccT = typename std::conditional<WT == ARIA_WI8, i32x16_t, f32x16_t>::type;
    AccT acc[FM][FN];

    /* one K-tile from stage B in 4 MFMA steps of FM x FN MFMAs. The operands of step ks + 1
     * (activation fragments from LDS; weight fragments from LDS, or unpacked in registers from
     * this lane's raw Q8 / Q4 words read at the start of the K-tile) are requested while step
     * ks's MFMAs run, and the order is pinned: each step is a scheduling region of its own in
     * which every MFMA is followed by one LDS read and a share of the unpack VALU. Left to
     * itself the scheduler sinks each fragment read next to its MFMA, and every MFMA then
     * waits out an LDS latency. */
    using FragT = typename std::conditional<WT == ARIA_WI8, i32x4_t, half8_t>::type;
    constexpr int NMF = FM * FN;                                             /* MFMAs per step */
    constexpr int NDS = FM + ((WT == ARIA_WF16 || WT == ARIA_WI8) ? FN : 0); /* LDS reads per step */
    constexpr int NVU = (WT == ARIA_WQ4) ? 14 * FN : (WT == ARIA_WQ8) ? 10 * FN : 0;   /* unpack VALU */
    auto pin = []() __attribute__((always_inline)) {
        static_for<NMF>([&](auto I) __attribute__((always_inline)) {
            constexpr int i = decltype(I)::value;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       /* one MFMA */
            constexpr int d = (NDS * (i + 1)) / NMF - (NDS * i) / NMF;
            if constexpr (d > 0) __builtin_amdgcn_sched_group_barrier(0x100, d, 0);  /* LDS reads */
            constexpr int v = (NVU * (i + 1)) / NMF - (NVU * i) / NMF;
            if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x002, v, 0);  /* VALU */
        });
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute = [&](auto BB) __attribute__((always_inline)) {
        constexpr int B = decltype(BB)::value;
        static_for<NS>([&](auto UU) __attribute__((always_inline)) {
        const uint8_t *S = smem + B * SB + decltype(UU)::value * St::BYTES;
        const uint16_t *X = reinterpret_cast<const uint16_t *>(S);
        /* W8A8: lane half h covers k in [64 h, 64 h + 64) of the 128-k tile and step ks its 16
         * k at 64 h + 16 ks on both sides (the int32 sums are exact, so any common order gives
         * the same bits); fp16: 8 k at 32 h + 8 ks, the order of the packed paths */
        auto afrag = [&](int i, int ks) __attribute__((always_inline)) {
            return *reinterpret_cast<const FragT *>(&X[xo(i * 32 + lrow, 4 * lh + ks)]);
        };
        WSt<WT == ARIA_WQ4 ? ARIA_WQ4 : ARIA_WQ8, FN> ws;
        QOff f[FN];
        if constexpr (WT == ARIA_WQ8 || WT == ARIA_WQ4) {
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int r = rbase + 32 * j + lrow;     /* weight row of the tile */
                if constexpr (WT == ARIA_WQ8) {
                    const uint8_t *row = S + St::A + r * 64;
                    const uint4 u0 = *reinterpret_cast<const uint4 *>(row + 16 * ((2 * lh) ^ ((r >> 2) & 3)));
                    const uint4 u1 = *reinterpret_cast<const uint4 *>(row + 16 * ((2 * lh + 1) ^ ((r >> 2) & 3)));
                    ws.w[j][0] = u0.x; ws.w[j][1] = u0.y; ws.w[j][2] = u0.z; ws.w[j][3] = u0.w;
                    ws.w[j][4] = u1.x; ws.w[j][5] = u1.y; ws.w[j][6] = u1.z; ws.w[j][7] = u1.w;
                } else {
                    const uint4 u = *reinterpret_cast<const uint4 *>(S + St::A + r * 32 + 16 * lh);
                    /* row r's [min, step] pairs sit in the 1 KB area of the wave that moved them,
                     * r / (32 FN), at slot r % (32 FN) */
                    const int dw = r / (32 * FN), slot = r % (32 * FN);
                    const uint2 pr = *reinterpret_cast<const uint2 *>(S + St::A + St::WQ + 1024 * dw + 16 * slot + 8 * lh);
                    ws.w[j][0] = u.x; ws.w[j][1] = u.y; ws.w[j][2] = u.z; ws.w[j][3] = u.w;
                    ws.w[j][4] = pr.x; ws.w[j][5] = pr.y;
                }
            }
#pragma unroll
            for (int j = 0; j < FN; j++) f[j] = qoff<WT == ARIA_WQ4 ? ARIA_WQ4 : ARIA_WQ8, FN>(ws, j);
        }
        auto bfrag = [&](int j, int ks) __attribute__((always_inline)) {
            if constexpr (WT == ARIA_WF16 || WT == ARIA_WI8) {
                const uint16_t *Wr = reinterpret_cast<const uint16_t *>(S + St::A);
                return *reinterpret_cast<const FragT *>(&Wr[xo(rbase + 32 * j + lrow, 4 * lh + ks)]);
            } else {
                return wfrag<WT, FN>(ws, j, ks, magic, f[j]);
            }
        };
        FragT xa[FM], xn[FM], wa[FN], wn[FN];
#pragma unroll
        for (int i = 0; i < FM; i++) xa[i] = afrag(i, 0);
#pragma unroll
        for (int j = 0; j < FN; j++) wa[j] = bfrag(j, 0);
        __builtin_amdgcn_sched_barrier(0);
        static_for<4>([&](auto KS) __attribute__((always_inline)) {
            constexpr int ks = decltype(KS)::value;
            if constexpr (ks < 3) {
#pragma unroll
                for (int i = 0; i < FM; i++) xn[i] = afrag(i, ks + 1);
#pragma unroll
                for (int j = 0; j < FN; j++) wn[j] = bfrag(j, ks + 1);
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    if constexpr (WT == ARIA_WI8)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa[j], xa[i], acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wa[j], xa[i], acc[i][j], 0, 0, 0);
                }
            if constexpr (ks < 3) {
                pin();
#pragma unroll
                for (int i = 0; i < FM; i++) xa[i] = xn[i];
#pragma unroll
                for (int j = 0; j < FN; j++) wa[j] = wn[j];
            }
        });
        });
    };

    /* workgroup barrier without a memory fence: the loop's only LDS writes are the DMA
     * transfers, whose completion each wave has waited for on vmcnt just before. Every LDS
     * read of the step must have returned before the barrier (lgkmcnt(0)): the compiler
     * places the last fragment reads' waits next to their MFMAs, which it may schedule
     * past the barrier, and a read still in flight there races with the next step's DMA
     * into the same stage (seen as one 32 x 32 block with a wrong k-slice). */
    auto barrier = []() __attribute__((always_inline)) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);   /* lgkmcnt(0); vmcnt and expcnt left at their maxima */
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    /* step kt (kt % NST == P): step kt + PD requested into stage (P + PD) % NST, step kt
     * multiplied from stage P, then this wave's transfers of step kt + 1 waited for (those of
     * later steps stay in flight) and the barrier publishes stage (P + 1) % NST */
    auto step = [&](auto PP, int kt) __attribute__((always_inline)) {
        constexpr int P = decltype(PP)::value;
        const bool more = kt + PD < KT;
        if (more) issue((P + PD) % NST, kt + PD);
        compute(IC<P>{});
        if constexpr (PD >= 2) {
            if (more) wait_vm<(PD - 1) * DMA>();
            else wait_vm<0>();
        } else {
            wait_vm<0>();
        }
        barrier();
    };

    const int m0 = (t / NTN) * BM, n0 = (t % NTN) * BN;
    sources(m0, n0);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    /* prologue: steps 0 .. PD - 1 in flight, then wait for step 0 */
    static_for<PD>([&](auto PP) __attribute__((always_inline)) {
        if (decltype(PP)::value < KT) issue(decltype(PP)::value, decltype(PP)::value);
    });
    if (KT >= PD) wait_vm<(PD - 1) * DMA>();
    else wait_vm<0>();
    barrier();
    int kt = 0;
    for (; kt + NST <= KT; kt += NST)
        static_for<NST>([&](auto PP) __attribute__((always_inline)) { step(PP, kt + decltype(PP)::value); });
    static_for<NST - 1>([&](auto PP) __attribute__((always_inline)) {
        if (kt + decltype(PP)::value < KT) step(PP, kt + decltype(PP)::value);
    });
    if constexpr (KSPL == 2) {
        /* every wave is past its last fragment read (the last step's barrier). The halves share
         * the epilogue: the first finalises row blocks 0 .. F0 - 1, the second the rest, each
         * taking the other half's partial sums of its blocks through the stage memory
         * (lane-major, conflict-free). Every element is acc_first + acc_second (an fp32 sum is
         * the same in either order; int32 exact). The second barrier keeps the partial sums
         * until both halves have read them, before the epilogue stages rows in that memory. */
        constexpr int F0 = (FM + 1) / 2;
        using ElT = typename std::conditional<WT == ARIA_WI8, int, float>::type;
        ElT *X = reinterpret_cast<ElT *>(smem_all) + tid;
#pragma unroll
        for (int i = 0; i < FM; i++)
            if ((khalf == 1) == (i < F0)) {
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) X[((i * FN + j) * 16 + r) * 256] = acc[i][j][r];
            }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < FM; i++)
            if ((khalf == 0) == (i < F0)) {
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = acc[i][j][r] + X[((i * FN + j) * 16 + r) * 256];
            }
        __syncthreads();
        float *E = reinterpret_cast<float *>(smem + wave * EPI_WAVE);
        if (khalf == 0) {
            epilogue<F0, FN, WT, MODE, GELU, AccT>(a, *reinterpret_cast<AccT(*)[F0][FN]>(&acc[0]), E, lane, m0,
                                                   n0 + wave * 32 * FN);
        } else if constexpr (FM > F0) {
            epilogue<FM - F0, FN, WT, MODE, GELU, AccT>(a, *reinterpret_cast<AccT(*)[FM - F0][FN]>(&acc[F0]), E, lane,
                                                        m0 + 32 * F0, n0 + wave * 32 * FN);
        }
        return;
    }
    /* every wave is past its last fragment read (the last step's barrier): the stages hold the
     * epilogue staging */
    float *E = reinterpret_cast<float *>(smem + wave * EPI_WAVE);
    epilogue<FM, FN, WT, MODE, GELU, AccT>(a, acc, E, lane, m0, n0 + rbase);
}

/* NST = 0: three stages where they fit the LDS share of MINB workgroups, else two */
template <int WT, int FM, int FN, int MODE, bool GELU = false, int MINB = 1, int KSPL = 1, int NSP = 1, int NS = 1,
          int NST = 0>
static void launch_big_m(const QArgs &a, hipStream_t s) {
    constexpr int BM = 32 * FM, BN = 128 * FN * NSP;
    constexpr int NSTA = NST ? NST : (3 * KSPL * NS * Stage<WT, FM, FN, NSP>::BYTES <= 160 * 1024 / MINB ? 3 : 2);
    const int MT = (a.M + BM - 1) / BM, NTN = (a.N + BN - 1) / BN, T = MT * NTN;
    const int grid = ((T + 7) / 8) * 8;
    hipLaunchKernelGGL((k_qgemm_big<WT, FM, FN, MODE, GELU, MINB, NS, NSTA, KSPL, NSP>), dim3(grid),
                       dim3(256 * KSPL * NSP), 0, s, a, NTN, T);
}

/* one kernel per fused epilogue mode (a run-time mode switch inside the store loop makes
 * every store wait for the loads of the modes that read); HEADS needs FN = 2 (a head's 64
 * columns in one wave) */
template <int WT, int FM, int FN, int MINB, int KSPL = 1, int NSP = 1>
static void launch_big(const QArgs &a, hipStream_t s) {
    switch (a.epi.mode) {
        case ARIA_EPI_GATE_RES: launch_big_m<WT, FM, FN, ARIA_EPI_GATE_RES, false, MINB, KSPL, NSP>(a, s); break;
        case ARIA_EPI_ADD: launch_big_m<WT, FM, FN, ARIA_EPI_ADD, false, MINB, KSPL, NSP>(a, s); break;
        case ARIA_EPI_ADD_DYT:
            if constexpr (WT == ARIA_WF16) launch_big_m<WT, FM, FN, ARIA_EPI_ADD_DYT, false, MINB, KSPL, NSP>(a, s);
            break;
        case ARIA_EPI_HEADS:
            if constexpr (FN >= 2) launch_big_m<WT, FM, FN, ARIA_EPI_HEADS, false, MINB, KSPL, NSP>(a, s);
            break;
        case ARIA_EPI_GLU: launch_big_m<WT, FM, FN, ARIA_EPI_GLU, false, MINB, KSPL, NSP>(a, s); break;
        case ARIA_EPI_DYT_ROPE:
            if constexpr (WT == ARIA_WF16) launch_big_m<WT, FM, FN, ARIA_EPI_DYT_ROPE, false, MINB, KSPL, NSP>(a, s);
            break;
        default:
            if (a.gelu) launch_big_m<WT, FM, FN, ARIA_EPI_STORE, true, MINB, KSPL, NSP>(a, s);
            else launch_big_m<WT, FM, FN, ARIA_EPI_STORE, false, MINB, KSPL, NSP>(a, s);
            break;
    }
}

/* the configurations compiled (FM, FN, workgroups per CU, K halves, N halves), index = the cfg
 * argument; measured at M = 2592 (DiT shapes), fp16 activations (the ones no longer picked stay
 * reachable as explicit tiles):
 *   0: 96 x 128, two per CU: N <= 1024 with an odd number of K-tiles
 *   1: 128 x 128, two per CU: N = 3072 without HEADS
 *   2: 64 x 256, two per CU: a head's 64 columns in one wave, the second workgroup per CU
 *      covering the other's HEADS epilogue (block 214 -> 204 us against 128 x 256 for qkv and the
 *      weights-in-registers ca_q); the HEADS projections now take 6 (ca_q) and 8 (qkv)
 *   3: 192 x 128, two per CU in two stages: N = 4096 before configuration 7 (448 tiles fill the
 *      512 slots once; Q8 36.5 -> 33.3 us, Q4 38.2 -> 36.0 us against the weights-in-registers
 *      kernel)
 *   4: 224 x 128, two per CU in two stages: N > 4096 (the GLU ff_in, N = 8192: Q8 74.4 ->
 *      58.3 us, Q4 73.4 -> 63.5 us)
 *   5: 96 x 128 in 8-wave workgroups, one per CU, waves 4-7 on the second half of the K range:
 *      N <= 1024 (sa_out, ca_out, ff_out: 216 tiles leave 40 CUs idle, and the split gives the
 *      busy ones two waves per SIMD; ff_out Q4 42.8 -> 38.6 us, Q8 36.4 -> 33.3 us)
 *   6: 64 x 256 in 8-wave workgroups with the K range split the same way: HEADS with N <= 1024
 *      (ca_q, 164 tiles; 15.6 -> 15.2 us against configuration 2)
 *   7: 192 x 256 in 8-wave workgroups, one per CU in three stages: each wave owns 32 weight
 *      rows as in configuration 3, but the 8 waves share one activation tile, so a CU moves
 *      24 KB of activations per K-tile instead of 48 and has the LDS for a third stage:
 *      3072 < N <= 4096 (ff_in: 224 tiles; Q8 32.7 -> 30.5 us, Q4 34.9 -> 33.0 us at K = 1024,
 *      -7 % at K = 2048, the same bits; at N = 8192 3-5 % slower than configuration 4)
 *   8: 64 x 512 in 8-wave workgroups, one per CU in three stages, each wave a head's 64 columns
 *      (configuration 2's waves, sharing one activation tile): HEADS with 1024 < N <= 3072
 *      (qkv: 246 tiles; 29.8 -> 28.8 us in the block, the same bits)
 * Larger FM amortises each unpacked weight over more rows; 96 x 256, 64 x 128 and 192 x 256
 * (one per CU) measured slower at every DiT shape. */
#define BIG_CFGS(X) X(0, 3, 1, 2, 1, 1) X(1, 4, 1, 2, 1, 1) X(2, 2, 2, 2, 1, 1) X(3, 6, 1, 2, 1, 1) X(4, 7, 1, 2, 1, 1) \
    X(5, 3, 1, 1, 2, 1) X(6, 2, 2, 1, 2, 1) X(7, 6, 1, 1, 1, 2) X(8, 2, 2, 1, 1, 2)
static const int big_fm[] = {3, 4, 2, 6, 7, 3, 2, 6, 2};
static const int big_fn[] = {1, 1, 2, 1, 1, 1, 2, 1, 2};
static const int big_ks[] = {1, 1, 1, 1, 1, 2, 2, 1, 1};    /* 2: the K range split inside the workgroup */
static const int big_nsp[] = {1, 1, 1, 1, 1, 1, 1, 2, 2};   /* 2: 8 waves, 256 FN weight rows */

int qgemm_big_ncfg() { return (int)(sizeof big_fm / sizeof big_fm[0]); }

/* fp16 weights (the decoder's GEMMs): 128-byte weight rows per K-tile, twice the Q8 bytes.
 * index = cfg: BM = 64, 96, 128, 160, 192 rows by 128 weight rows, two workgroups per CU (the
 * first in three stages, the others in two). qgemm_big_f16_pick chooses by a cost model fitted
 * to the decoder's GEMMs (M = 1870 and 11016; N / K = 3840 / 768, 4608 / 768, 768 / 768,
 * 768 / 2304): the CU with the most tiles, ceil(T / 256) of them, times the tile's rows times
 * a per-row time that falls with BM (each LDS weight fragment feeds more MFMAs). It picks the
 * fastest configuration at all eight shapes; against the LDS-operand kernel's 192 x 128
 * tiles: 105.6 -> 97.0 us (N = 3840), 136.7 -> 119.8 us (N = 4608) at M = 11016. */
#define BIG_F16_CFGS(X) X(0, 2, 1, 2, 1) X(1, 3, 1, 2, 1) X(2, 4, 1, 2, 1) X(3, 5, 1, 2, 1) X(4, 6, 1, 2, 1)
static const int big_f16_fn[] = {1, 1, 1, 1, 1};

int qgemm_big_f16_pick(int M, int N) {
    static const float row_us[5] = {0.088f, 0.092f, 0.082f, 0.075f, 0.070f};   /* FM = 2 .. 6 */
    int best = 0;
    float best_c = 1e30f;
    for (int c = 0; c < 5; c++) {
        const int bm = 32 * (c + 2);
        const long T = (long)((M + bm - 1) / bm) * ((N + 127) / 128);
        const float cost = (float)((T + 255) / 256) * (float)bm * row_us[c];
        if (cost < best_c) { best_c = cost; best = c; }
    }
    return best;
}

static hipError_t qgemm_big_f16_launch(const QArgs &a, int cfg, hipStream_t s) {
    if (cfg < 0 || cfg >= (int)(sizeof big_f16_fn / sizeof big_f16_fn[0]) ||
        (a.epi.mode == ARIA_EPI_HEADS && big_f16_fn[cfg] < 2))
        return hipErrorInvalidValue;
#define F16_CASE(i, fm, fn, mb, ks)                                \
    case i:                                                        \
        if ((a.K / KB) % ks) return hipErrorInvalidValue;          \
        launch_big<ARIA_WF16, fm, fn, mb, ks>(a, s);               \
        break;
    switch (cfg) {
        BIG_F16_CFGS(F16_CASE)
        default: return hipErrorInvalidValue;
    }
#undef F16_CASE
    return hipGetLastError();
}
int qgemm_big_bm(int cfg) { return 32 * big_fm[cfg]; }
int qgemm_big_bn(int cfg) { return 128 * big_fn[cfg] * big_nsp[cfg]; }

hipError_t qgemm_big_launch(const QArgs &a, int wt, int cfg, hipStream_t s) {
    if (wt == ARIA_WF16 && a.K % KB == 0 && (!a.gelu || a.epi.mode == ARIA_EPI_STORE)) return qgemm_big_f16_launch(a, cfg, s);
    if (a.K % KB || cfg < 0 || cfg >= qgemm_big_ncfg() || (a.gelu && a.epi.mode != ARIA_EPI_STORE) ||
        (a.epi.mode == ARIA_EPI_HEADS && big_fn[cfg] < 2) || (a.K / KB) % big_ks[cfg])
        return hipErrorInvalidValue;
#define BIG_CASE(i, fm, fn, mb, ks, nsp)                                        \
    case i:                                                                   \
        if (wt == ARIA_WQ8) launch_big<ARIA_WQ8, fm, fn, mb, ks, nsp>(a, s);  \
        else launch_big<ARIA_WQ4, fm, fn, mb, ks, nsp>(a, s);                 \
        break;
    if (wt != ARIA_WQ8 && wt != ARIA_WQ4) return hipErrorInvalidValue;
    /* the Q4 [min, step] pairs of a K-tile move 16 bytes at a time */
    if (wt == ARIA_WQ4 && ((uintptr_t)a.scale & 15u)) return hipErrorInvalidValue;
    switch (cfg) {
        BIG_CFGS(BIG_CASE)
        default: return hipErrorInvalidValue;
    }
#undef BIG_CASE
    return hipGetLastError();
}

/* W8A8 (int8 activations, Q8 weights, K % 128 == 0): the configurations compiled, index = cfg,
 * measured at M = 2592 against the weights-in-registers int8 kernel (k_gemm_i8.hip):
 *   0: 64 x 128, two workgroups per CU: N <= 1024 (K = 1024: 14.6 -> 9.9 us; K = 4096: 39.4 -> 23.4 us)
 *   1: 64 x 256, two per CU in two stages: HEADS (qkv and ca_q; W8A8 block 192.7 -> 188.0 us
 *      against 128 x 256 one per CU for qkv and 64 x 256 one per CU for ca_q)
 *   2: 128 x 128, two per CU in two stages: 1024 < N <= 3072 (N = 3072: 19.5 -> 17.6 us
 *      against 128 x 256 one per CU)
 *   3: 192 x 128, two per CU in two stages: N > 3072 (ff_in N = 4096: 29.3 -> 22.7 us;
 *      the GLU ff_in N = 8192: 61.4 -> 49.6 us)
 *   4: 96 x 128 in 8-wave workgroups (the K range split, two stages each): N <= 1024 with
 *      K >= 2048 (ff_out: 23.6 -> 21.7 us)
 *   5: 64 x 256 in 8-wave workgroups, the K range split: HEADS with N <= 1024 (ca_q) */
/* int8 (W8A8): the same forms with 128-deep K-tiles; 6 is configuration 7's 192 x 256 (N = 4096:
 * 22.2 -> 21.6 us, GELU 24.3 -> 23.6 us at K = 1024, the same bits; no faster at N = 8192).
 * The int8 form of configuration 8 (64 x 512 HEADS, two stages of 72 KB) made the W8A8 qkv
 * 21.1 -> 21.6 us: not compiled. */
#define BIG_I8_CFGS(X) X(0, 2, 1, 2, 1, 1) X(1, 2, 2, 2, 1, 1) X(2, 4, 1, 2, 1, 1) X(3, 6, 1, 2, 1, 1) X(4, 3, 1, 1, 2, 1) \
    X(5, 2, 2, 1, 2, 1) X(6, 6, 1, 1, 1, 2)
int qgemm_big_i8_ncfg() { return 7; }

hipError_t qgemm_big_i8_launch(const QArgs &a, int cfg, hipStream_t s) {
    if (a.K % 128 || (a.gelu && a.epi.mode != ARIA_EPI_STORE)) return hipErrorInvalidValue;
#define BIG_I8_CASE(i, fm, fn, mb, ks, nsp)                                                  \
    case i:                                                                                \
        if ((a.epi.mode == ARIA_EPI_HEADS && fn < 2) || (a.K / 128) % ks) return hipErrorInvalidValue; \
        launch_big<ARIA_WI8, fm, fn, mb, ks, nsp>(a, s);                                   \
        break;
    switch (cfg) {
        BIG_I8_CFGS(BIG_I8_CASE)
        default: return hipErrorInvalidValue;
    }
#undef BIG_I8_CASE
    return hipGetLastError();
}
