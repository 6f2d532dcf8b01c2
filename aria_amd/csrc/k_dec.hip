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
 *   k_dec_attn_mfma  one chunk-head of the differential self-attention, fused: both
 *                 softmax(q k^T / 8) v products over the chunk's 34 tokens on the fp32 MFMA,
 *                 their difference, merged fp16 (the q/k DynamicTanh norms and RoPE, 32
 *                 rotated dims, are the to_qkv GEMM's DYT_ROPE epilogue)
 *   k_dec_im2col  the k = 3 mapping convolution's input rows (the last 16 of each group)
 *   k_dec_map     the mapping convolution as an fp32 GEMM on the fp32 MFMA (the reference
 *                 keeps it fp32), trimmed to T * 16 rows and unpatched to stereo in its stores
 * Arithmetic follows the reference's order (built with -ffp-contract=off). tanh: block 0's pre
 * norm (k_dec_dyt) uses the device library's tanhf; the other 11 block norms (the ADD_DYT
 * epilogue of to_out / ff_out) and the q/k norms (the DYT_ROPE epilogue of to_qkv) use
 * tanh_fast (exp + rcp, a few 1e-7 absolute, before the fp16 rounding of the GEMM operand);
 * the softmax exponential is v_exp_f32 (~1 ulp).
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
    const float *qkv;           /* [nch * 34, 3840]: q | k | v | qd | kd, q / k normed and rotated */
};

/* ---- the chunk attention on the fp32 MFMA (v_mfma_f32_16x16x4_f32) ----
 * One (chunk, head) per workgroup of six waves; wave w computes pair p = w / 3 (0: q, k;
 * 1: qd, kd) for the 16 queries of block i = w % 3 of the chunk's 34 tokens padded to 48
 * (3 blocks of 16). The q / k sections of qkv arrive DynamicTanh-normed and rotated (the
 * to_qkv GEMM's DYT_ROPE epilogue, once per element). Against one wave per pair (288 MFMAs in
 * one wave's chain, 129 VGPRs, three waves per SIMD) each wave runs 96 MFMAs at 58 VGPRs:
 * decode 0.698 -> 0.686 ms at T = 108, 2.71 -> 2.63 ms at T = 646, same bits.
 *   v (34 rows x 64 dims, shared by all six waves) travels to LDS by LDS DMA first thing, so
 *     its fetch overlaps the q / k loads and takes no registers
 *   each wave loads its block's 16 q rows and 16 k rows once; the k rows go through LDS to the
 *     pair's other two waves (loading all 48 per wave doubled the L2 reads: slower at T = 2584)
 *   S = q k^T for the wave's query block: 1 x 3 blocks, 16 k-steps; lane l supplies row l % 16
 *     of q (A) and of k (B) at dim 16 (l / 16) + s in step s (16 consecutive dims of one row)
 *   softmax over the 34 valid keys in the accumulators (a row's 16 columns of a block sit in
 *     16 lanes: xor-shuffle reductions), probabilities through the wave's own 16 LDS rows
 *     (over the k space, once every wave's k reads are done) into the A layout
 *   O = P v: 1 x 4 blocks, 12 k-steps over keys 12 (l / 16) + s; output block j column n
 *     holds dim 4 n + j, so a lane's B operands of a step are one 16-byte LDS read of v and
 *     its four output dims of a row are adjacent (one 8-byte store)
 * The pair-1 waves leave O in LDS (lane-major, over the v space once every product is done),
 * the pair-0 wave of the same block writes half(O0 - O1) to the merged rows. Accumulator v of
 * lane l in a 16 x 16 block: row 4 (l / 16) + v, column l % 16. Padded q / k rows are zero and
 * padded keys are masked before the max and multiply zero v, so nothing past the chunk's rows
 * is used. Every output element is the same sequence of operations as with one wave per pair.
 * fp32 operands, as the reference keeps this attention fp32. */
#define DA_P 48            /* padded chunk */
#define DA_PS 52           /* LDS row stride of P (floats; 16-byte aligned rows) */
#define DA_KS 68           /* LDS row stride of k (floats; rows spread over the banks) */
#define DA_VCH 576         /* v staging: 16-byte chunks (34 rows x 16, rounded up to 9 x 64) */
#define DA_WAVES 6

typedef float f32x4_dec __attribute__((ext_vector_type(4)));

/* this lane's 16 dims (16 lq ..) of row r of the section at column off; rows past the chunk
 * are zero */
__device__ __forceinline__ void dec_ld_row(float (&f)[16], const float *base, int off, int r, int lq) {
    const bool ok = r < DEC_S;
    const float *row = base + (size_t)(ok ? r : 0) * DEC_QKV + off + lq * 16;
#pragma unroll
    for (int j4 = 0; j4 < 4; j4++) {
        const float4 x = *reinterpret_cast<const float4 *>(row + 4 * j4);
        f[4 * j4 + 0] = ok ? x.x : 0.0f; f[4 * j4 + 1] = ok ? x.y : 0.0f;
        f[4 * j4 + 2] = ok ? x.z : 0.0f; f[4 * j4 + 3] = ok ? x.w : 0.0f;
    }
}

__global__ __launch_bounds__(64 * DA_WAVES) void k_dec_attn_mfma(DecAttnArgs a, int H) {
    /* [0, 9216): v rows (256 B each); then k of both pairs (2 x 48 rows x 68 floats), later
     * reused for P (6 waves x 16 rows x 52); after every product: O of the pair-1 waves (3 x
     * 16 x 64 floats, lane-major) from offset 0 */
    __shared__ __attribute__((aligned(16))) float sm[DA_VCH * 4 + 2 * 48 * DA_KS];
    static_assert(2 * 48 * DA_KS >= DA_WAVES * 16 * DA_PS, "P fits the k space");
    float4 *Vs = reinterpret_cast<float4 *>(sm);
    const int ch = blockIdx.x / H, h = blockIdx.x % H;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int pair = wave / 3, qi = wave % 3;
    const int lr = lane & 15, lq = lane >> 4;
    const float *base = a.qkv + (size_t)ch * DEC_S * DEC_QKV + h * DEC_HD;

    /* v by LDS DMA: instruction i moves chunks 64 i .. 64 i + 63 (row p / 16, dims 4 (p % 16)
     * ..), wave w the instructions i = w, w + 6; chunks past the 34 rows re-read row 33 */
    {
        typedef __attribute__((address_space(3))) void lds_void_t;
        for (int i = wave; i < DA_VCH / 64; i += DA_WAVES) {
            const int p = 64 * i + lane, r = min(p >> 4, DEC_S - 1);
            __builtin_amdgcn_global_load_lds(base + (size_t)r * DEC_QKV + 1536 + 4 * (p & 15),
                                             (lds_void_t *)(sm + 256 * i), 16, 0, 0);
        }
    }
    /* q (or qd) rows 16 qi + lr in registers; k (or kd) rows 16 qi + lr through LDS to the
     * pair's three waves */
    float qf[16], kf[3][16];
    float *Ks = sm + DA_VCH * 4 + pair * (48 * DA_KS);
    {
        float kr[16];
        dec_ld_row(qf, base, pair ? 2304 : 0, qi * 16 + lr, lq);
        dec_ld_row(kr, base, pair ? 3072 : 768, qi * 16 + lr, lq);
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++)
            *reinterpret_cast<float4 *>(Ks + (qi * 16 + lr) * DA_KS + lq * 16 + 4 * j4) =
                make_float4(kr[4 * j4], kr[4 * j4 + 1], kr[4 * j4 + 2], kr[4 * j4 + 3]);
    }
    __syncthreads();   /* the pair's 48 k rows in LDS */
#pragma unroll
    for (int bk = 0; bk < 3; bk++)
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) {
            const float4 k4 = *reinterpret_cast<const float4 *>(Ks + (bk * 16 + lr) * DA_KS + lq * 16 + 4 * j4);
            kf[bk][4 * j4] = k4.x; kf[bk][4 * j4 + 1] = k4.y; kf[bk][4 * j4 + 2] = k4.z; kf[bk][4 * j4 + 3] = k4.w;
        }
    /* S = q k^T for the wave's query block */
    f32x4_dec sc[3];
#pragma unroll
    for (int j = 0; j < 3; j++) sc[j] = f32x4_dec{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 16; st++)
#pragma unroll
        for (int j = 0; j < 3; j++) sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[st], kf[j][st], sc[j], 0, 0, 0);
    __syncthreads();   /* every wave's k reads done before P overwrites them */

    /* softmax of each row over keys < 34 (block 2 holds keys 32 + lr) */
    float *P = sm + DA_VCH * 4 + wave * (16 * DA_PS);
#pragma unroll
    for (int v = 0; v < 4; v++) {
        float x0 = sc[0][v] * 0.125f, x1 = sc[1][v] * 0.125f;
        float x2 = lr < DEC_S - 32 ? sc[2][v] * 0.125f : -INFINITY;
        float mx = fmaxf(fmaxf(x0, x1), x2);
        mx = grp_max<16>(mx);   /* DPP within the row of 16 lanes, no LDS round trip */
        x0 = exp_fast(x0 - mx); x1 = exp_fast(x1 - mx); x2 = exp_fast(x2 - mx);
        float sum = (x0 + x1) + x2;
        sum = grp_sum<16>(sum);
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        const int row = 4 * lq + v;
        P[row * DA_PS + lr] = x0 * inv;
        P[row * DA_PS + 16 + lr] = x1 * inv;
        P[row * DA_PS + 32 + lr] = x2 * inv;
    }
    /* v in LDS: this wave's transfers done (vmcnt), then the barrier publishes every wave's
     * (and orders each wave's P stores before its reads below) */
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();

    /* O = P v over keys 12 lq + s (keys >= 34 have P = 0 and multiply zero v) */
    f32x4_dec oc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) oc[j] = f32x4_dec{0.0f, 0.0f, 0.0f, 0.0f};
    {
        float pf[12];
#pragma unroll
        for (int c4 = 0; c4 < 3; c4++) {
            const float4 p4 = *reinterpret_cast<const float4 *>(&P[lr * DA_PS + lq * 12 + 4 * c4]);
            pf[4 * c4 + 0] = p4.x; pf[4 * c4 + 1] = p4.y; pf[4 * c4 + 2] = p4.z; pf[4 * c4 + 3] = p4.w;
        }
#pragma unroll
        for (int s2 = 0; s2 < 12; s2++) {
            const int key = lq * 12 + s2;
            const float4 v4 = Vs[min(key, DEC_S - 1) * 16 + lr];
            const bool kv = key < DEC_S;
            const float vf[4] = {kv ? v4.x : 0.0f, kv ? v4.y : 0.0f, kv ? v4.z : 0.0f, kv ? v4.w : 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) oc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pf[s2], vf[j], oc[j], 0, 0, 0);
        }
    }
    /* every product done before the pair-1 waves' O overwrites v and P */
    __syncthreads();
    float *Os = sm + qi * (16 * 64);
    if (pair == 1) {
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) Os[(j * 4 + v) * 64 + lane] = oc[j][v];
    }
    __syncthreads();
    if (pair == 0) {
        uint2 *dst = reinterpret_cast<uint2 *>(a.merged + (size_t)ch * DEC_S * DEC_D + h * DEC_HD + 4 * lr);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int row = qi * 16 + 4 * lq + v;
            if (row < DEC_S) {
                uint32_t hv[4];
#pragma unroll
                for (int j = 0; j < 4; j++) hv[j] = f2h_bits(oc[j][v] - Os[(j * 4 + v) * 64 + lane]);
                dst[(size_t)row * (DEC_D / 4)] = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
            }
        }
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

/* ---- the mapping convolution as an fp32 GEMM on the fp32 MFMA, unpatch fused ----
 * audio[n / 256][m * 256 + n % 256] = sum_k xc[m][k] W[n][k] + b[n], m < M = T * 16, n < 512,
 * k < 2304 (src/aria_sa3_dec.c:100-116: the mapping GEMM, the trim and aria_unpatch_stereo).
 * v_mfma_f32_32x32x2_f32 keeps fp32 operands, as the reference keeps this GEMM in fp32.
 * 256 threads = 2 x 2 waves, each owning FM x FN blocks of 32 x 32 (tile 64 FM rows of xc by
 * 64 FN rows of W); k moves through LDS 32 at a time, double-buffered (one barrier per
 * slice), the next slice's global loads in flight during the current slice's MFMAs. KS = 2
 * doubles the workgroup: the second 256 threads take the second half of k on their own
 * buffers and hand their partial sums to the first (acc_first + acc_second). The
 * MFMA computes W xc^T, so a lane's accumulators hold 4 consecutive n of one m: 4
 * consecutive audio samples, one 16-byte store. Lane l of an MFMA supplies row l % 32 at
 * k = 16 (l / 32) + j of the slice, j = 0..15 (any fixed k order gives the dot product),
 * so each lane reads 16 consecutive floats of its row: four 16-byte LDS reads. Rows past
 * M re-read row M - 1 and are not stored. */
#define MAP_K 2304
#define MAP_N 512
#define MAP_KT 32
#define MAP_SA 36          /* LDS row stride (floats): 16-byte reads of 16 rows hit 64 distinct banks */

typedef float f32x16_dec __attribute__((ext_vector_type(16)));

template <int FM, int FN, int KS>
__global__ __launch_bounds__(256 * KS) void k_dec_map(float *audio, const float *xc, const float *W, const float *bias, int M) {
    constexpr int BM = 64 * FM, BN = 64 * FN;
    constexpr int LA = BM * MAP_KT / 4 / 256, LW = BN * MAP_KT / 4 / 256;   /* float4 loads per thread */
    /* KS = 2: threads 256.. (waves 4-7) run the second half of k on their own buffers, and
     * their partial sums join the first half's through LDS before the stores */
    __shared__ __attribute__((aligned(16))) float As_all[KS][2][BM * MAP_SA];
    __shared__ __attribute__((aligned(16))) float Ws_all[KS][2][BN * MAP_SA];
    static_assert(MAP_K % (MAP_KT * KS) == 0, "the k halves are whole slices");
    const int khalf = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));

    const int ntile = MAP_N / BN;
    const int m0 = (blockIdx.x / ntile) * BM, n0 = (blockIdx.x % ntile) * BN;
    const int tid = threadIdx.x & 255, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;

    f32x16_dec acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    auto compute = [&](int buf) {
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            float4 xa[FM], wa[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                xa[i] = *reinterpret_cast<const float4 *>(&As_all[khalf][buf][(wm * 32 * FM + i * 32 + lr) * MAP_SA + lh * 16 + q4 * 4]);
#pragma unroll
            for (int j = 0; j < FN; j++)
                wa[j] = *reinterpret_cast<const float4 *>(&Ws_all[khalf][buf][(wn * 32 * FN + j * 32 + lr) * MAP_SA + lh * 16 + q4 * 4]);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(wa[j][e], xa[i][e], acc[i][j], 0, 0, 0);
        }
    };

    /* per thread: float4 q = tid + 256 i of the slice, row q / 8, column 4 (q % 8) */
    const float *ga[LA], *gw[LW];
    constexpr int NK = MAP_K / MAP_KT / KS;   /* slices of this half */
    const int k0 = khalf * NK * MAP_KT;
#pragma unroll
    for (int i = 0; i < LA; i++) {
        const int q = tid + i * 256;
        ga[i] = xc + (size_t)min(m0 + (q >> 3), M - 1) * MAP_K + k0 + (q & 7) * 4;
    }
#pragma unroll
    for (int i = 0; i < LW; i++) {
        const int q = tid + i * 256;
        gw[i] = W + (size_t)(n0 + (q >> 3)) * MAP_K + k0 + (q & 7) * 4;
    }
    const int so = (tid >> 3) * MAP_SA + (tid & 7) * 4;   /* + 32 rows per i */
    float4 ra[LA], rw[LW];
#pragma unroll
    for (int i = 0; i < LA; i++) ra[i] = *reinterpret_cast<const float4 *>(ga[i]);
#pragma unroll
    for (int i = 0; i < LW; i++) rw[i] = *reinterpret_cast<const float4 *>(gw[i]);
#pragma unroll
    for (int i = 0; i < LA; i++) *reinterpret_cast<float4 *>(&As_all[khalf][0][so + i * 32 * MAP_SA]) = ra[i];
#pragma unroll
    for (int i = 0; i < LW; i++) *reinterpret_cast<float4 *>(&Ws_all[khalf][0][so + i * 32 * MAP_SA]) = rw[i];
    __syncthreads();
    for (int kt = 0; kt < NK; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < NK) {
#pragma unroll
            for (int i = 0; i < LA; i++) ra[i] = *reinterpret_cast<const float4 *>(ga[i] + (kt + 1) * MAP_KT);
#pragma unroll
            for (int i = 0; i < LW; i++) rw[i] = *reinterpret_cast<const float4 *>(gw[i] + (kt + 1) * MAP_KT);
        }
        compute(cur);
        if (kt + 1 < NK) {
#pragma unroll
            for (int i = 0; i < LA; i++) *reinterpret_cast<float4 *>(&As_all[khalf][cur ^ 1][so + i * 32 * MAP_SA]) = ra[i];
#pragma unroll
            for (int i = 0; i < LW; i++) *reinterpret_cast<float4 *>(&Ws_all[khalf][cur ^ 1][so + i * 32 * MAP_SA]) = rw[i];
        }
        __syncthreads();
    }

    if constexpr (KS == 2) {
        /* every wave is past its last LDS read (the loop's closing barrier): the second half's
         * partial sums go through its own buffers, lane-major, and the first half adds them
         * (acc_first + acc_second, a fixed order) and stores */
        float *X = &As_all[1][0][0] + tid;
        static_assert(FM * FN * 16 * 256 <= 2 * BM * MAP_SA, "the partial sums fit the second half's buffers");
        if (khalf == 1) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) X[((i * FN + j) * 16 + r) * 256] = acc[i][j][r];
        }
        __syncthreads();
        if (khalf == 0) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = acc[i][j][r] + X[((i * FN + j) * 16 + r) * 256];
        }
    }
    if (KS == 2 && khalf == 1) return;

    /* accumulator r of lane l: n = 8 (r / 4) + 4 (l / 32) + r % 4, m = l % 32 (per block) */
#pragma unroll
    for (int i = 0; i < FM; i++) {
        const int m = m0 + wm * 32 * FM + i * 32 + lr;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int n = n0 + wn * 32 * FN + j * 32 + 8 * g + 4 * lh;
                const float4 b = *reinterpret_cast<const float4 *>(bias + n);
                float4 o;
                o.x = acc[i][j][4 * g + 0] + b.x;
                o.y = acc[i][j][4 * g + 1] + b.y;
                o.z = acc[i][j][4 * g + 2] + b.z;
                o.w = acc[i][j][4 * g + 3] + b.w;
                *reinterpret_cast<float4 *>(audio + (size_t)(n >> 8) * M * 256 + (size_t)m * 256 + (n & 255)) = o;
            }
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
extern "C" hipError_t aria_k_dec_attn(uint16_t *merged, const float *qkv, int nch, hipStream_t s) {
    if (nch <= 0) return hipSuccess;
    DecAttnArgs a;
    a.merged = merged; a.qkv = qkv;
    hipLaunchKernelGGL(k_dec_attn_mfma, dim3(nch * 12), dim3(64 * DA_WAVES), 0, s, a, 12);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_dec_im2col(float *xc, const float *seq, int Lt, int Lout, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_im2col, grid_for((size_t)Lt * 3 * DEC_D), dim3(256), 0, s, xc, seq, Lt, Lout);
    return hipGetLastError();
}
/* audio [2, M * 256] = unpatch(xc [M, 2304] . W [512, 2304]^T + b) in 64 x 64 tiles: faster
 * than 128 x 64, 64 x 128 and 128 x 128 at every decoder length measured (T = 108, 646, 2584;
 * every tiling gives the same bits) */
extern "C" hipError_t aria_k_dec_map(float *audio, const float *xc, const float *W, const float *b, int M,
                                     hipStream_t s) {
    if (M <= 0) return hipSuccess;
    /* at most one tile per CU (T <= 128: 216 tiles at T = 108): the k range split over two
     * 4-wave halves gives each SIMD two waves (decode 0.688 -> 0.658 ms at T = 108); more tiles
     * keep one 4-wave workgroup per tile (the split measured 0.5 % slower at T = 646) */
    const int tiles = (M + 63) / 64 * (MAP_N / 64);
    if (tiles <= 256)
        hipLaunchKernelGGL((k_dec_map<1, 1, 2>), dim3(tiles), dim3(512), 0, s, audio, xc, W, b, M);
    else
        hipLaunchKernelGGL((k_dec_map<1, 1, 1>), dim3(tiles), dim3(256), 0, s, audio, xc, W, b, M);
    return hipGetLastError();
}
