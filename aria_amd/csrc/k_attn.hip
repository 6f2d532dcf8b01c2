/*
 * k_attn.hip - the DiT's attention on gfx950: head preparation and fused MFMA attention.
 *
 * k_qkv_prep replaces the reference block's extract_heads + q/k RMSNorm + RoPE
 * (src/aria_sa3_dit.c:183-194, 222-226; device twin k_extract_normrope,
 * src/aria_cuda.cu:447-470): from a projection row [S, nsec*dim] it writes
 * head-major fp16 [B, H, S, hd] tensors, RMS-normalising and rotating (rotate-half,
 * rot dims) the q and k sections. The 64-value head statistic is summed in fp32 over
 * 16 lanes and inverted with v_rsq_f32: against aria_rmsnorm's double sum it differs
 * by ~1e-7 relative, and it saves a 16-lane fp64 reduction plus an fp64 sqrt and
 * divide per row (about 5 us per DiT block when fused into the GEMM epilogue).
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
 * Precision: Q, K, V and P are fp16, accumulation fp32, exp via v_exp_f32. The row sum
 * l is accumulated (v_dot2_f32_f16, exact products) from the same fp16 P that multiplies
 * V. The running max is a lazy reference (moved only when a tile exceeds it by 2^8), so
 * the accumulators are rarely rescaled; O / l does not depend on the reference chosen.
 * Workgroup: QW = 3 to 6 waves x 32 queries of one (batch, head), twice the waves when the
 * keys are split in two halves inside the workgroup (long key sets); K and V tiles
 * of 64 keys are staged key-major in LDS (swizzled, conflict-free) by LDS DMA
 * (global_load_lds_dwordx4, no staging registers), the next tile's transfer running under
 * the current tile's math; the V^T operand is read with the gfx950 transpose load
 * (ds_read_b64_tr_b16).
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
        float ss = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        ss = grp_sum<16>(ss);
        const float inv = __builtin_amdgcn_rsqf(ss * (1.0f / 64) + a.eps);
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
            for (int e = 0; e < 4; e++) p[e] = rope_partner(o[e], lane, lp);
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
#define RESCALE_SLACK 8.0f    /* log2 units the running max may lag the true max */

struct AttnArgs {
    const uint16_t *q, *k, *v;   /* [B*H, N, 64] fp16 */
    void *o;                     /* [B, Nq, H*64] merged heads */
    int H, Nq, Nk;
    int nqb, T;                  /* query blocks (32 QW queries) per (batch, head); nqb * B*H */
    float scale_log2;            /* (1/sqrt(64)) * log2(e) */
    int o_f16;
    /* prefetch workgroups: blocks Tpad .. gridDim.x - 1 read pf[0 .. npf) and exit */
    int Tpad, npf;
    const uint4 *pf[ARIA_PF_SPANS];
    unsigned pf_n16[ARIA_PF_SPANS];
};

#ifndef ARIA_ATTN_PF_NT
#define ARIA_ATTN_PF_NT 0
#endif
/* prefetch workgroup w of nw: its share of every span, 4 16-byte loads per lane in flight; the
 * values only feed an empty asm statement, which keeps the loads */
__device__ __forceinline__ void attn_prefetch(const AttnArgs &a, int w, int nw) {
    for (int sp = 0; sp < a.npf; sp++) {
        const unsigned n = a.pf_n16[sp], per = (n + nw - 1) / nw, lo = min(n, w * per), hi = min(n, lo + per);
        const uint4 *p = a.pf[sp];
        for (unsigned i = lo + threadIdx.x; i < hi; i += 4 * blockDim.x) {
            uint4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const unsigned k = min(i + j * blockDim.x, hi - 1);
                if constexpr (ARIA_ATTN_PF_NT) {
                    typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
                    const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p + k));
                    v[j] = make_uint4(t.x, t.y, t.z, t.w);
                } else {
                    v[j] = p[k];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) asm volatile("" ::"v"(v[j].x));
        }
    }
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

__device__ __forceinline__ half8_t ld_h8(const uint16_t *p) { return *reinterpret_cast<const half8_t *>(p); }

/* K and V tiles are key-major [64 keys][64 d] fp16, 128 B rows, unpadded; the 16 B chunk
 * c (8 d) of key row r sits at position c ^ swizzle(r):
 *   K: (r >> 1) & 7 -- the fragment reads (32 keys x one chunk, 16 B per lane) and the
 *      producer writes (8 lanes per row) are bank-conflict free;
 *   V: ((r >> 1) & 1) << 2 -- the transpose reads below (4 keys x 32 d per 32 lanes,
 *      8 B per lane) and the producer writes are bank-conflict free. */
__device__ __forceinline__ int k_off(int key, int chunk) { return key * 64 + ((chunk ^ ((key >> 1) & 7)) << 3); }
__device__ __forceinline__ int v_off(int key, int d) {
    return key * 64 + ((((d >> 3) ^ (((key >> 1) & 1) << 2))) << 3) + (d & 7);
}

/* V^T operand of O^T = V^T P^T for one 16-key MFMA step: lane l (d row l%32 of block
 * dt, key group g = l/32) needs V[key][d] for keys kb + 4g + {0..3} and kb + 8 + 4g +
 * {0..3}. ds_read_b64_tr_b16 returns, to lane 4w+c of each 16-lane group, element c of
 * the 8 B rows addressed by lanes 4v+w (v = 0..3): addressing key kb' + v at d0 + 4w
 * delivers V[kb'+0..3][d0 + (lane & 15)] to each lane (voff below). */

/* max(a, b, c) in one v_max3_f32 */
__device__ __forceinline__ float max3f(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

/* fp32 pair -> packed fp16, round to nearest even */
__device__ __forceinline__ uint32_t pack2h_rn(float x, float y) {
    typedef float float2_v __attribute__((ext_vector_type(2)));
    typedef _Float16 half2_v __attribute__((ext_vector_type(2)));
    const float2_v f = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_v));
}

/* QW (3 to 6) waves of 32 queries per key half. KS = 1: all keys. KS = 2: 2 QW waves; waves QW..2 QW - 1
 * take the second half of the key tiles with their own LDS buffers, and the halves merge
 * (max, row sum, O) through LDS at the end: twice the waves per query block without any
 * exchange between workgroups. Both halves run the same number of loop trips, so every
 * barrier is reached by all waves. */
template <int KS, int QW>
__global__ __launch_bounds__(64 * QW * KS) __attribute__((amdgpu_waves_per_eu(4))) void k_flash_attn(AttnArgs a) {
    /* tile buffers, each [half][KT x 64] fp16, as four separate LDS objects: K and V tiles
     * arrive by LDS DMA (global_load_lds), whose writes count on vmcnt, and the compiler only
     * omits a vmcnt wait before a fragment read when the read provably targets another object
     * than the pending DMA. After the key loop Kb0s + Kb1s hold the merge exchange (4 waves x
     * 34 x 64 floats = 34.8 KB; the two objects are placed back to back, checked below). */
    __shared__ __attribute__((aligned(16))) uint16_t Kb0s[KS * KT * 64];
    __shared__ __attribute__((aligned(16))) uint16_t Kb1s[KS * KT * 64];
    __shared__ __attribute__((aligned(16))) uint16_t Vb0s[KS * KT * 64];
    __shared__ __attribute__((aligned(16))) uint16_t Vb1s[KS * KT * 64];

    static_assert(QW >= 3 && QW <= 6, "three to six query waves per key half");
    /* the wave index in a scalar register: everything derived from it stays scalar */
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int half = KS == 1 ? 0 : wid / QW;
    uint16_t *const Kb0 = Kb0s + half * (KT * 64), *const Kb1 = Kb1s + half * (KT * 64);
    uint16_t *const Vb0 = Vb0s + half * (KT * 64), *const Vb1 = Vb1s + half * (KT * 64);
    const int lane = threadIdx.x & 63, wave = wid % QW, g = lane >> 5, l32 = lane & 31;
    if ((int)blockIdx.x >= a.Tpad) {        /* a prefetch workgroup (uniform, before any barrier) */
        attn_prefetch(a, (int)blockIdx.x - a.Tpad, (int)gridDim.x - a.Tpad);
        return;
    }
    /* the query blocks of one (batch, head) run on one XCD, so its K and V are fetched
     * into that XCD's L2 once rather than into every XCD's */
    const int tix = xcd_tile(blockIdx.x, a.T);
    if (tix >= a.T) return;                 /* uniform per workgroup, before any barrier */
    const int bh = tix / a.nqb;
    const int q0 = (tix % a.nqb) * (32 * QW) + wave * 32;
    const uint16_t *Qh = a.q + (size_t)bh * a.Nq * 64;
    const uint16_t *Kh = a.k + (size_t)bh * a.Nk * 64;
    const uint16_t *Vh = a.v + (size_t)bh * a.Nk * 64;

    /* Q^T fragments (B operand of S^T = K Q^T): query q0 + l32, d = 16*ds + 8g + [0,8);
     * queries past Nq re-read the last one (their outputs are not stored) */
    half8_t qf[4];
    {
        const int qi = min(q0 + l32, a.Nq - 1);
#pragma unroll
        for (int ds = 0; ds < 4; ds++) qf[ds] = ld_h8(Qh + (size_t)qi * 64 + 16 * ds + 8 * g);
    }

    /* tile staging by LDS DMA: a tile is 512 slots of 16 B (key row p / 8, stored chunk p % 8)
     * in 8 blocks of 64; instruction i of wave w (of this half) fills block cb = QW i + w
     * (slots p = 64 cb + lane), so each lane fetches the global chunk that the swizzle places
     * there: K stores logical chunk c of row r at c ^ ((r >> 1) & 7), V at
     * c ^ (((r >> 1) & 1) << 2). Keys past Nk re-read the last key (their probabilities are
     * exactly zero). */
    typedef __attribute__((address_space(3))) void lds_void_t;
    auto dma = [&](int kt0, uint16_t *Kd, uint16_t *Vd) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < (8 + QW - 1) / QW; i++) {
            const int cb = QW * i + wave;
            if (8 % QW != 0 && cb >= 8) break;   /* uniform per wave */
            const int p = 64 * cb + lane, r = p >> 3, cp = p & 7;
            const size_t row = (size_t)min(kt0 + r, a.Nk - 1) * 64;
            const int ck = cp ^ ((r >> 1) & 7), cv = cp ^ (((r >> 1) & 1) << 2);
            __builtin_amdgcn_global_load_lds(Kh + row + 8 * ck, (lds_void_t *)(Kd + 64 * cb * 8), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(Vh + row + 8 * cv, (lds_void_t *)(Vd + 64 * cb * 8), 16, 0, 0);
        }
    };
    /* the DMA writes into LDS complete on vmcnt; each wave waits for its own before the
     * barrier that publishes the tile */
    auto dma_wait = []() __attribute__((always_inline)) { __builtin_amdgcn_s_waitcnt(0x0F70); };

    f32x16_t oacc[2];
#pragma unroll
    for (int r = 0; r < 16; r++) { oacc[0][r] = 0.0f; oacc[1][r] = 0.0f; }
    /* this lane's share of the row sum l (its 32 keys of each tile; the partner lane l^32
     * holds the other 32), accumulated from the same fp16 P that multiplies V */
    float lsum = 0.0f;
    typedef _Float16 half2_v __attribute__((ext_vector_type(2)));
    const half2_v one2 = {(_Float16)1.0f, (_Float16)1.0f};
    float m_use = -INFINITY;   /* running reference max, scaled (log2) units */

    /* per-lane LDS offsets (halves) of the fragment reads, hoisted out of the key loop. The
     * swizzles depend only on lane bits: K block kb (keys 32kb..) sits 32*64*kb further, V key
     * step s16 (keys 16 s16..) 16*64*s16 further and its second 8 keys 8*64 further, all
     * immediates, so six base offsets cover every read */
    int koff[4], voff[2];
#pragma unroll
    for (int ds = 0; ds < 4; ds++) koff[ds] = k_off(l32, 2 * ds + g);
    {
        const int v = (lane & 15) >> 2, w = lane & 3, G = lane >> 4;
#pragma unroll
        for (int dt = 0; dt < 2; dt++) voff[dt] = v_off(4 * (G >> 1) + v, 32 * dt + 16 * (G & 1) + 4 * w);
    }

    /* one 64-key tile from LDS buffer BUF (a compile-time constant, so every LDS offset
     * is an immediate) */
    auto tile = [&](const int kt0, const uint16_t *K, const uint16_t *V) {
        /* S^T [64 keys x 32 queries] as two 32-key blocks */
        f32x16_t sc[2];
#pragma unroll
        for (int r = 0; r < 16; r++) { sc[0][r] = 0.0f; sc[1][r] = 0.0f; }
        /* the two 32-key blocks alternate: each chain's MFMA waits on its predecessor, and
         * both fragments of a step arrive with one LDS wait */
#pragma unroll
        for (int ds = 0; ds < 4; ds++) {
            const half8_t k0 = ld_h8(K + koff[ds]), k1 = ld_h8(K + koff[ds] + 32 * 64);
            sc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, qf[ds], sc[0], 0, 0, 0);
            sc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(k1, qf[ds], sc[1], 0, 0, 0);
        }
        if (kt0 + KT > a.Nk) {   /* ragged last tile: keys past the end get -inf */
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (kt0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3) >= a.Nk) sc[kb][r] = -INFINITY;
        }
        /* tile max over this lane's 32 keys and the partner lane's 32: a tree of 3-input
         * maxima (15 v_max3_f32, depth 3; two-input fmaxf trees compile to twice as many ops) */
        float t1[11];
#pragma unroll
        for (int i = 0; i < 10; i++) t1[i] = max3f(sc[(3 * i) >> 4][(3 * i) & 15], sc[(3 * i + 1) >> 4][(3 * i + 1) & 15],
                                                   sc[(3 * i + 2) >> 4][(3 * i + 2) & 15]);
        t1[10] = fmaxf(sc[1][14], sc[1][15]);
        float mt = max3f(max3f(t1[0], t1[1], t1[2]), max3f(t1[3], t1[4], t1[5]), max3f(t1[6], t1[7], t1[8]));
        mt = max3f(mt, t1[9], t1[10]);
        mt = fmaxf(mt, xor32_f32(mt, lane)) * a.scale_log2;
        /* lazy rescale: the reference max only moves when the tile max exceeds it by more
         * than RESCALE_SLACK (probabilities stay <= 2^8, exact in fp16's range); the final
         * O / l is unchanged by the choice of reference */
        if (__ballot(mt > m_use + RESCALE_SLACK)) {
            /* a real branch: without the marker the compiler predicates the 33 multiplies
             * and runs them on every tile */
            asm volatile("" ::: "memory");
            const float m_new = fmaxf(m_use, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_use - m_new);
#pragma unroll
            for (int r = 0; r < 16; r++) { oacc[0][r] *= alpha; oacc[1][r] *= alpha; }
            lsum *= alpha;
            m_use = m_new;
        }
        /* P^T = exp2(s * scale - m) in fp16; MFMA step ks of block kb takes accumulator
         * registers 8ks..8ks+7 (keys 16ks + 4g + {0..3}, 16ks + 8 + 4g + {0..3}) */
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                /* the step's V^T fragments are requested before its exponentials, which then
                 * cover the LDS latency */
                const int s16 = 2 * kb + ks;
                half8_t vf[2];
#pragma unroll
                for (int dt = 0; dt < 2; dt++) {
                    const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(V + voff[dt] + 16 * 64 * s16));
                    const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(V + voff[dt] + 16 * 64 * s16 + 8 * 64));
                    const half4_t hl = __builtin_bit_cast(half4_t, lo), hh = __builtin_bit_cast(half4_t, hi);
                    vf[dt] = half8_t{hl[0], hl[1], hl[2], hl[3], hh[0], hh[1], hh[2], hh[3]};
                }
                __builtin_amdgcn_sched_barrier(0);
                float pv[8];
#pragma unroll
                for (int i = 0; i < 8; i++)
                    pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][8 * ks + i], a.scale_log2, -m_use));
                const half8_t pf = __builtin_bit_cast(half8_t, make_uint4(pack2h_rn(pv[0], pv[1]), pack2h_rn(pv[2], pv[3]),
                                                                          pack2h_rn(pv[4], pv[5]), pack2h_rn(pv[6], pv[7])));
#pragma unroll
                for (int dt = 0; dt < 2; dt++)
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[dt], pf, oacc[dt], 0, 0, 0);
                /* row sum of the rounded P: exact fp16 products, fp32 accumulation */
#pragma unroll
                for (int e = 0; e < 4; e++)
                    lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_v, __builtin_bit_cast(uint4, pf)[e]), one2, lsum, false);
            }
        }
    };

    /* this half's key tiles [tb, tb + nt); niter = trips every half runs */
    const int ntiles_all = (a.Nk + KT - 1) / KT;
    const int niter = (ntiles_all + KS - 1) / KS;
    const int tb = half * niter;
    const int nt = max(0, min(niter, ntiles_all - tb));
    const int kbase = tb * KT;
    const uint16_t *K0 = Kb0, *V0 = Vb0, *K1 = Kb1, *V1 = Vb1;
    if (nt > 0) dma(kbase, Kb0, Vb0);
    dma_wait();
    __syncthreads();
    /* two tiles per trip so each LDS buffer is a fixed address; buffer b^1 was last read
     * one tile earlier, before that tile's closing barrier. A wave whose 32 queries all lie
     * past Nq (in the last query block: 1296 = 6 x 192 + 144, so that block's sixth wave)
     * only stages tiles and meets the barriers; its products would never be stored. */
    const bool live = q0 < a.Nq;
    for (int t = 0; t < niter; t += 2) {
        if (t + 1 < nt) dma(kbase + (t + 1) * KT, Kb1, Vb1);
        if (live && t < nt) tile(kbase + t * KT, K0, V0);
        dma_wait();
        __syncthreads();
        if (t + 1 < niter) {
            if (t + 2 < nt) dma(kbase + (t + 2) * KT, Kb0, Vb0);
            if (live && t + 1 < nt) tile(kbase + (t + 1) * KT, K1, V1);
            dma_wait();
            __syncthreads();
        }
    }

    float lrow = lsum + xor32_f32(lsum, lane);   /* the query's full row sum */

    if constexpr (KS == 2) {
        /* merge: the second half hands (O, l, m) to the first through LDS (the tile buffers
         * are free after the last trip's barrier): per wave 64 lanes x 16 floats of each O
         * block, waves 0-3 in Kb0s / Kb1s (each object holds 4 x 16 x 64 floats), waves 4-5 in
         * Vb0s / Vb1s, and l and m in Vb0s after them */
        static_assert(KS * KT * 64 * 2 >= 4 * 16 * 64 * 4 && QW <= 6, "merge exchange fits the tile buffers");
        float *const xk0 = reinterpret_cast<float *>(Kb0s), *const xk1 = reinterpret_cast<float *>(Kb1s);
        float *const xv0 = reinterpret_cast<float *>(Vb0s), *const xv1 = reinterpret_cast<float *>(Vb1s);
        float *X0 = (wave < 4 ? xk0 + wave * 16 * 64 : xv0 + (wave - 4) * 16 * 64) + lane;
        float *X1 = (wave < 4 ? xk1 + wave * 16 * 64 : xv1 + (wave - 4) * 16 * 64) + lane;
        float *X2 = xv0 + (QW > 4 ? 2 * 16 * 64 : 0) + wave * 2 * 64 + lane;
        if (half == 1) {
#pragma unroll
            for (int r = 0; r < 16; r++) { X0[r * 64] = oacc[0][r]; X1[r * 64] = oacc[1][r]; }
            X2[0] = lrow;
            X2[64] = m_use;
        }
        __syncthreads();
        if (half == 1) return;
        const float m1 = X2[64], l1 = X2[0];
        const float m = fmaxf(m_use, m1);   /* finite for a live wave (half 0 always has keys); a
                                             * wave past Nq returns below without storing */
        const float a0 = __builtin_amdgcn_exp2f(m_use - m), a1 = __builtin_amdgcn_exp2f(m1 - m);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            oacc[0][r] = oacc[0][r] * a0 + X0[r * 64] * a1;
            oacc[1][r] = oacc[1][r] * a0 + X1[r * 64] * a1;
        }
        lrow = lrow * a0 + l1 * a1;
    }

    /* O[q, d] = O^T[d, q] / l ; lane holds query q0 + l32, d = 32dt + 8(r/4) + 4g + r%4 */
    const int qi = q0 + l32;
    if (qi >= a.Nq) return;
    const float inv = 1.0f / lrow;
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

extern "C" hipError_t aria_k_flash_attn_pf(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *o,
                                           int o_f16, int BH, int H, int Nq, int Nk, const aria_prefetch_set *pf,
                                           hipStream_t s) {
    if (BH <= 0 || Nq <= 0) return hipSuccess;
    AttnArgs a;
    a.npf = 0;
    if (pf && (pf->n < 0 || pf->n > ARIA_PF_SPANS)) return hipErrorInvalidValue;
    for (int i = 0; pf && i < pf->n; i++) {
        if (!pf->p[i] || !pf->bytes[i]) continue;
        if ((pf->bytes[i] & 15u) || ((uintptr_t)pf->p[i] & 15u) || pf->bytes[i] / 16 > 0xFFFFFFFFu)
            return hipErrorInvalidValue;
        a.pf[a.npf] = (const uint4 *)pf->p[i];
        a.pf_n16[a.npf++] = (unsigned)(pf->bytes[i] / 16);
    }
    a.q = q; a.k = k; a.v = v; a.o = o; a.H = H; a.Nq = Nq; a.Nk = Nk; a.o_f16 = o_f16;
    a.scale_log2 = 0.125f * ARIA_LOG2E;
    /* split the keys inside the workgroup when there are enough tiles for both halves
     * (S = 1296 self-attention: 21 tiles); short key sets (the 256 cross keys) run one half.
     * A CU running two workgroups takes nearly twice as long as one running a single one, so
     * the split form takes the fewest query waves per half (4, 5 or 6) whose blocks give every
     * CU at most one workgroup, else 4 (two per CU): S = 1296, 32 heads: 6, 224 blocks of 192
     * queries (31.9 -> 27.8 us against 352 blocks of 128; the same bits). The one-half form
     * takes the fewest query slots on the busiest CU (ceil(T / 256) blocks of 32 QW queries),
     * ties to 4: the cross attention at S = 1296, 32 heads takes 3 (10.8 -> 10.4 us) */
    const bool split = (Nk + KT - 1) / KT >= 8;
    int qw = 4;
    if (split) {
        for (int w = 4; w <= 6; w++)
            if ((long)((Nq + 32 * w - 1) / (32 * w)) * BH <= 256) { qw = w; break; }
    } else {
        const long t4 = (long)((Nq + 127) / 128) * BH, t3 = (long)((Nq + 95) / 96) * BH;
        if ((t3 + 255) / 256 * 3 < (t4 + 255) / 256 * 4) qw = 3;
    }
    a.nqb = (Nq + 32 * qw - 1) / (32 * qw);
    a.T = a.nqb * BH;
    a.Tpad = (a.T + 7) / 8 * 8;
    /* prefetch workgroups on the CUs the split form's one-per-CU workgroups leave idle */
    static int ncu = 0;
    if (!ncu) {
        int dev = 0, n = 0;
        ncu = (hipGetDevice(&dev) == hipSuccess &&
               hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? n : -1;
    }
    const int npw = (split && a.npf && ncu > a.Tpad) ? (ncu - a.Tpad) / 8 * 8 : 0;
    if (!npw) a.npf = 0;
    const dim3 grid(a.Tpad + npw);
    if (split) {
        if (qw == 6) hipLaunchKernelGGL((k_flash_attn<2, 6>), grid, dim3(768), 0, s, a);
        else if (qw == 5) hipLaunchKernelGGL((k_flash_attn<2, 5>), grid, dim3(640), 0, s, a);
        else hipLaunchKernelGGL((k_flash_attn<2, 4>), grid, dim3(512), 0, s, a);
    } else if (qw == 3) {
        hipLaunchKernelGGL((k_flash_attn<1, 3>), grid, dim3(192), 0, s, a);
    } else {
        hipLaunchKernelGGL((k_flash_attn<1, 4>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

extern "C" hipError_t aria_k_flash_attn(const uint16_t *q, const uint16_t *k, const uint16_t *v, void *o, int o_f16,
                                        int BH, int H, int Nq, int Nk, hipStream_t s) {
    return aria_k_flash_attn_pf(q, k, v, o, o_f16, BH, H, Nq, Nk, nullptr, s);
}
