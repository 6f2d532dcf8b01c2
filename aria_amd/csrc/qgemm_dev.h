/*
 * qgemm_dev.h - device code shared by the two dequant-on-use GEMM kernels
 * (k_qgemm.hip: both operands staged through LDS; k_qgemm_wr.hip: weights loaded
 * straight into registers): the kernel argument block, fp16 packing, the Q8 unpack,
 * the XCD-aware tile order and the fused epilogue. Included by those two files only.
 */
#ifndef ARIA_QGEMM_DEV_H
#define ARIA_QGEMM_DEV_H

#include "aria_dev.h"
#include "aria_hip_kernels.h"

#include <cstring>
#include <type_traits>

template <int I>
using IC = std::integral_constant<int, I>;
/* f(IC<0>{}), ..., f(IC<N-1>{}) */
template <int N, int I = 0, class Fn>
__device__ __forceinline__ void static_for(Fn &&f) {
    if constexpr (I < N) {
        f(IC<I>{});
        static_for<N, I + 1>(f);
    }
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
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
    const float *xscale;   /* ARIA_WI8: per-row activation scale sx[M] (unused otherwise) */
    aria_qgemm_epi epi;
};

/* two fp32 -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32) */
__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    const float2_t f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));
}

/* Q8: four int8 in one word -> two words of fp16 pairs, exactly. Each byte is biased to
 * unsigned (b ^ 0x80 = b + 128) and placed under the fp16 exponent of 1024
 * (0x64XX = 1024 + XX), then 1152 is subtracted: an exact integer in [-127, 127]. */
__device__ __forceinline__ void q8x4_to_h(uint32_t w, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = w ^ 0x80808080u;
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

/* xcd_tile (aria_dev.h) gives each XCD a contiguous run of tiles in M-major order, so an
 * XCD's L2 holds a few activation row panels and the weight panels instead of every
 * activation row. */

/* Epilogue of one wave: its FM x FN blocks of 32x32 accumulators are staged through
 * LDS 32 rows at a time (fp32, rows padded by 16 B) and written as whole row segments:
 * 16 B per lane, coalesced. acc register r of lane l holds n = 8*(r/4) + 4*(l/32) + r%4,
 * m = l%32 of its block. E is this wave's staging area (32 rows of 32*FN*4 + 16 bytes);
 * mw / nw are the first activation row and the first weight row of the wave's tile.
 * v = acc * scale (Q8) + bias, GELU'd when GELU, then the fused mode MODE (both compile
 * time; EPI_ANY dispatches on a.epi.mode and a.gelu once per call). A run-time GELU flag
 * inside the element loop is if-converted by the compiler: every output then pays the
 * GELU and a select whether or not it is wanted. Without a bias the lane adds -0.0,
 * which leaves every value (signed zeros and NaN included) unchanged, so the bias needs
 * neither a branch nor a select. Every global load of a 32-row
 * group (residual, gate, local cond, RoPE tables) is issued before its first store:
 * loads and stores retire in order, so a load issued after a store would make the next
 * wait cover that store's whole write latency.
 * HEADS: the 16 lanes of a 64-column head share a row m (the wave's column range is
 * head-aligned); the arithmetic is k_qkv_prep's (k_attn.hip): RMS statistic in fp32
 * over the head, (x * inv) * w, then rotate-half RoPE over the first rot dims. */
#define EPI_ANY (-1)
template <int FM, int FN, int WT, int MODE, bool GELU = false, typename AccT = f32x16_t>
__device__ __forceinline__ void epilogue(const QArgs &a, AccT (&acc)[FM][FN], float *E, int lane, int mw, int nw) {
    constexpr int EPI_STRIDE = 32 * FN * 4 + 16;
    constexpr int CW = 32 * FN;                 /* columns per wave */
    constexpr int LPR = CW / 4;                 /* lanes per row (16 B each) */
    constexpr int RPI = 64 / LPR;               /* rows per store instruction */
    constexpr int NIT = 32 / RPI;               /* store instructions per 32-row group */
    if constexpr (MODE == EPI_ANY) {
        const bool g = a.gelu != 0;
        switch (a.epi.mode) {
            case ARIA_EPI_GATE_RES:
                if (g) epilogue<FM, FN, WT, ARIA_EPI_GATE_RES, true>(a, acc, E, lane, mw, nw);
                else epilogue<FM, FN, WT, ARIA_EPI_GATE_RES>(a, acc, E, lane, mw, nw);
                return;
            case ARIA_EPI_ADD:
                if (g) epilogue<FM, FN, WT, ARIA_EPI_ADD, true>(a, acc, E, lane, mw, nw);
                else epilogue<FM, FN, WT, ARIA_EPI_ADD>(a, acc, E, lane, mw, nw);
                return;
            case ARIA_EPI_ADD_DYT: epilogue<FM, FN, WT, ARIA_EPI_ADD_DYT>(a, acc, E, lane, mw, nw); return;   /* no GELU */
            case ARIA_EPI_HEADS:
                if constexpr (LPR % 16 == 0) {
                    if (g) epilogue<FM, FN, WT, ARIA_EPI_HEADS, true>(a, acc, E, lane, mw, nw);
                    else epilogue<FM, FN, WT, ARIA_EPI_HEADS>(a, acc, E, lane, mw, nw);
                }
                return;
            case ARIA_EPI_GLU: epilogue<FM, FN, WT, ARIA_EPI_GLU>(a, acc, E, lane, mw, nw); return;   /* no GELU */
            case ARIA_EPI_DYT_ROPE: epilogue<FM, FN, WT, ARIA_EPI_DYT_ROPE>(a, acc, E, lane, mw, nw); return;   /* no GELU */
            default:
                if (g) epilogue<FM, FN, WT, ARIA_EPI_STORE, true>(a, acc, E, lane, mw, nw);
                else epilogue<FM, FN, WT, ARIA_EPI_STORE>(a, acc, E, lane, mw, nw);
                return;
        }
    } else {
    static_assert(MODE != ARIA_EPI_HEADS || LPR % 16 == 0, "a head's 64 columns must sit in one wave");
    const int lrow = lane & 31, lh = lane >> 5;
    const int ecol = (lane % LPR) * 4, erow = lane / LPR;
    const int nb = nw + ecol;                   /* this lane's 4 output columns */
    const bool col_ok = nb < a.N;
    float4 sc = make_float4(1.0f, 1.0f, 1.0f, 1.0f), bb = make_float4(-0.0f, -0.0f, -0.0f, -0.0f);
    if (col_ok) {
        if (WT == ARIA_WQ8 || WT == ARIA_WI8) sc = *reinterpret_cast<const float4 *>(a.scale + nb);
        if (a.bias) bb = *reinterpret_cast<const float4 *>(a.bias + nb);
        else if (WT == ARIA_WI8) bb = make_float4(0.0f, 0.0f, 0.0f, 0.0f);   /* the reference adds 0.0f */
    }
    /* GATE_RES: the gate depends on (batch, column) only, so sigmoid(1 - gate) is formed
     * once per lane for the (at most two) batches this wave's rows span; a tile spanning
     * more batches (sequences shorter than the tile) reads it per row */
    auto gate_at = [&](int bt, int col) -> float4 {
        float4 g = *reinterpret_cast<const float4 *>(a.epi.gate + (size_t)bt * a.epi.gate_bs + col);
        if (a.epi.gate2) {   /* the gate formed in place: chunk of to_scale_shift_gate + gcond */
            const float4 ga = *reinterpret_cast<const float4 *>(a.epi.gate2 + (size_t)bt * a.epi.gate2_bs + col);
            g = make_float4(g.x + ga.x, g.y + ga.y, g.z + ga.z, g.w + ga.w);
        }
        return g;
    };
    bool gpre = false;
    int blo = 0, bnd = 0;                       /* bnd: first row of batch blo + 1 */
    float4 gs0 = make_float4(0.f, 0.f, 0.f, 0.f), gs1 = gs0;
    if constexpr (MODE == ARIA_EPI_GATE_RES) {
        const int rpb = a.epi.rows_per_batch;
        const int mlast = min(mw + 32 * FM - 1, a.M - 1);
        blo = min(mw, a.M - 1) / rpb;
        bnd = (blo + 1) * rpb;
        gpre = mlast / rpb <= blo + 1;
        if (gpre) {
            const int nbc = col_ok ? nb : 0, bhi = min(blo + 1, (a.M - 1) / rpb);
            const float4 g0 = gate_at(blo, nbc), g1 = gate_at(bhi, nbc);
            gs0 = make_float4(gate_sig_f(g0.x), gate_sig_f(g0.y), gate_sig_f(g0.z), gate_sig_f(g0.w));
            gs1 = make_float4(gate_sig_f(g1.x), gate_sig_f(g1.y), gate_sig_f(g1.z), gate_sig_f(g1.w));
        }
    }
    /* HEADS: per-lane constants of the epilogue (section, head, norm gains, RoPE lanes) */
    const aria_qgemm_epi &e = a.epi;
    int hh = 0, l16 = 0, kind = 2, rh = 0, i0 = 0;
    bool rope = false, first = false;
    float4 gw = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    uint16_t *dsec = nullptr;                   /* this lane's head section (kernel-argument
                                                 * arrays indexed once, not per row) */
    if constexpr (MODE == ARIA_EPI_HEADS) {
        const int secw = e.heads * 64;
        const int sec = min(nb / secw, e.nsec - 1);
        hh = (nb % secw) >> 6;
        l16 = lane & 15;
        kind = e.kind[sec];
        dsec = e.dst[sec];
        const float *wsec = e.w[sec];
        if (kind != 2 && wsec) gw = *reinterpret_cast<const float4 *>(wsec + 4 * l16);
        rh = e.rot >> 1;
        const int d0 = 4 * l16;
        rope = kind != 2 && e.rot > 0 && e.cos_t && d0 < e.rot;
        first = d0 < rh;
        i0 = first ? d0 : d0 - rh;
    }
    /* DYT_ROPE: the lane's section kind (0 q-like, 1 k-like, 2 v), DynamicTanh gain (gw),
     * bias (dbv) and alpha, and its RoPE lanes. A wave's 32 FN columns start on a multiple of
     * 32, so the rotation partner d +- rot / 2 (rot <= 32) of the lane's four dims sits rot / 8
     * lanes away in the same row: lane ^ (rot / 8). */
    float4 dbv = make_float4(0.f, 0.f, 0.f, 0.f);
    float dal = 0.0f;
    if constexpr (MODE == ARIA_EPI_DYT_ROPE) {
        const int sec = nb / (e.heads * 64), d0 = nb & 63;
        kind = (!col_ok || sec == 2) ? 2 : (sec == 0 || sec == 3) ? 0 : 1;
        if (kind != 2) {
            gw = *reinterpret_cast<const float4 *>((kind == 0 ? e.w[0] : e.w[2]) + d0);
            dbv = *reinterpret_cast<const float4 *>((kind == 0 ? e.w[1] : e.w[3]) + d0);
            dal = kind == 0 ? e.eps : e.eps2;
        }
        rh = e.rot >> 1;
        rope = kind != 2 && e.rot > 0 && d0 < e.rot;
        first = d0 < rh;
        i0 = first ? d0 : d0 - rh;
    }
    /* HEADS, DYT_ROPE: (batch, position) of this lane's current row, m = hb * S + hs. The rows
     * a lane visits rise by RPI per store (and per 32-row group, NIT * RPI = 32), so the pair
     * is advanced by (RPI / S, RPI % S) with one carry instead of a division per row. */
    int hb = 0, hs = 0, hq = 0, hr = 0;
    if constexpr (MODE == ARIA_EPI_HEADS || MODE == ARIA_EPI_DYT_ROPE) {
        const int S = e.rows_per_batch, m0 = mw + erow;
        hb = m0 / S;
        hs = m0 - hb * S;
        hq = RPI / S;
        hr = RPI - hq * S;
    }
    /* GATE_RES, ADD, ADD_DYT: the fp32 residual rows (and the per-row gates or second addend)
     * of 32-row group i + 1 are requested as group i starts, so a group's load latency runs
     * under the previous group's staging and stores instead of after them (two groups of
     * registers, buffer i & 1) */
    constexpr bool RMW = MODE == ARIA_EPI_GATE_RES || MODE == ARIA_EPI_ADD || MODE == ARIA_EPI_ADD_DYT;
    float4 rr_b[2][NIT], g2_b[2][NIT];
    auto rmw_load = [&](int i, float4 (&rr)[NIT], float4 (&g2)[NIT]) __attribute__((always_inline)) {
        const int nbc = col_ok ? nb : 0;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int mc = min(mw + i * 32 + it * RPI + erow, a.M - 1);
            rr[it] = *reinterpret_cast<const float4 *>((const float *)a.y + (size_t)mc * a.N + nbc);
            if (MODE == ARIA_EPI_GATE_RES && !gpre) g2[it] = gate_at(mc / e.rows_per_batch, nbc);
            else if (MODE == ARIA_EPI_ADD && e.add2)
                g2[it] = *reinterpret_cast<const float4 *>(e.add2 + (size_t)mc * a.N + nbc);
        }
    };
    if constexpr (RMW) rmw_load(0, rr_b[0], g2_b[0]);
#pragma unroll
    for (int i = 0; i < FM; i++) {
        if constexpr (RMW) {
            if (i + 1 < FM) rmw_load(i + 1, rr_b[(i + 1) & 1], g2_b[(i + 1) & 1]);
        }
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<float4 *>(reinterpret_cast<char *>(E) + lrow * EPI_STRIDE +
                                            (j * 32 + 8 * g + 4 * lh) * 4) =
                    make_float4((float)acc[i][j][4 * g], (float)acc[i][j][4 * g + 1], (float)acc[i][j][4 * g + 2],
                                (float)acc[i][j][4 * g + 3]);   /* int32 (W8A8): v_cvt_f32_i32, nearest even */
        __builtin_amdgcn_wave_barrier();
        float v[NIT][4];
        int mrow[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int r = it * RPI + erow;
            mrow[it] = mw + i * 32 + r;
            const float4 v4 = *reinterpret_cast<const float4 *>(reinterpret_cast<const char *>(E) +
                                                                r * EPI_STRIDE + ecol * 4);
            v[it][0] = v4.x; v[it][1] = v4.y; v[it][2] = v4.z; v[it][3] = v4.w;
            const float scv[4] = {sc.x, sc.y, sc.z, sc.w}, bv[4] = {bb.x, bb.y, bb.z, bb.w};
            float xsv = 1.0f;   /* W8A8: (float)acc * sx[m] * scale[n], in that order */
            if constexpr (WT == ARIA_WI8) xsv = a.xscale[min(mrow[it], a.M - 1)];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (WT == ARIA_WI8) v[it][q] = v[it][q] * xsv;
                if (WT == ARIA_WQ8 || WT == ARIA_WI8) v[it][q] = v[it][q] * scv[q];
                v[it][q] = v[it][q] + bv[q];
                if constexpr (GELU) v[it][q] = gelu_tanh_f(v[it][q]);
            }
        }
        __builtin_amdgcn_wave_barrier();   /* staging reads done before the next group's writes */
        if constexpr (MODE == ARIA_EPI_STORE) {
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const int m = mrow[it];
                if (m >= a.M || !col_ok) continue;
                if (a.y_f16)
                    *reinterpret_cast<uint2 *>((uint16_t *)a.y + (size_t)m * a.N + nb) =
                        make_uint2(pack2h(v[it][0], v[it][1]), pack2h(v[it][2], v[it][3]));
                else
                    *reinterpret_cast<float4 *>((float *)a.y + (size_t)m * a.N + nb) =
                        make_float4(v[it][0], v[it][1], v[it][2], v[it][3]);
            }
        } else if constexpr (MODE == ARIA_EPI_GLU) {   /* (value, gate) pairs -> silu(gate) * value */
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const int m = mrow[it];
                if (m >= a.M || !col_ok) continue;
                const float g0 = silu_f(v[it][1]) * v[it][0], g1 = silu_f(v[it][3]) * v[it][2];
                if (a.y_f16)
                    *reinterpret_cast<uint32_t *>((uint16_t *)a.y + (size_t)m * (a.N >> 1) + (nb >> 1)) = pack2h(g0, g1);
                else   /* fp32 (the W8A8 block quantises the fp32 product) */
                    *reinterpret_cast<float2 *>((float *)a.y + (size_t)m * (a.N >> 1) + (nb >> 1)) = make_float2(g0, g1);
            }
        } else if constexpr (MODE == ARIA_EPI_GATE_RES || MODE == ARIA_EPI_ADD || MODE == ARIA_EPI_ADD_DYT) {
            /* read-modify-write of the fp32 residual (loaded one group ahead) */
            float4 dg = make_float4(0.f, 0.f, 0.f, 0.f), db = dg;   /* ADD_DYT: the norm's gain and bias */
            if constexpr (MODE == ARIA_EPI_ADD_DYT) {
                if (col_ok) {
                    dg = *reinterpret_cast<const float4 *>(e.w[0] + nb);
                    db = *reinterpret_cast<const float4 *>(e.w[1] + nb);
                }
            }
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const int m = mrow[it];
                if (m >= a.M || !col_ok) continue;
                float4 o;
                if (MODE == ARIA_EPI_GATE_RES) {
                    /* y += v * sigmoid(1 - gate): the rounding order of k_gate_residual */
                    float4 sg;
                    if (gpre) sg = (m < bnd) ? gs0 : gs1;
                    else sg = make_float4(gate_sig_f(g2_b[i & 1][it].x), gate_sig_f(g2_b[i & 1][it].y), gate_sig_f(g2_b[i & 1][it].z), gate_sig_f(g2_b[i & 1][it].w));
                    o = make_float4(rr_b[i & 1][it].x + v[it][0] * sg.x, rr_b[i & 1][it].y + v[it][1] * sg.y,
                                    rr_b[i & 1][it].z + v[it][2] * sg.z, rr_b[i & 1][it].w + v[it][3] * sg.w);
                } else {
                    o = make_float4(rr_b[i & 1][it].x + v[it][0], rr_b[i & 1][it].y + v[it][1], rr_b[i & 1][it].z + v[it][2], rr_b[i & 1][it].w + v[it][3]);
                    if (MODE == ARIA_EPI_ADD && e.add2)
                        o = make_float4(o.x + g2_b[i & 1][it].x, o.y + g2_b[i & 1][it].y, o.z + g2_b[i & 1][it].z, o.w + g2_b[i & 1][it].w);
                }
                *reinterpret_cast<float4 *>((float *)a.y + (size_t)m * a.N + nb) = o;
                if constexpr (MODE == ARIA_EPI_ADD_DYT) {
                    const float al = e.eps;
                    const float h0 = tanh_fast(al * o.x) * dg.x + db.x, h1 = tanh_fast(al * o.y) * dg.y + db.y;
                    const float h2 = tanh_fast(al * o.z) * dg.z + db.z, h3 = tanh_fast(al * o.w) * dg.w + db.w;
                    *reinterpret_cast<uint2 *>(e.dst[0] + (size_t)m * a.N + nb) = make_uint2(pack2h(h0, h1), pack2h(h2, h3));
                }
            }
        } else if constexpr (MODE == ARIA_EPI_DYT_ROPE) {
            /* tanh(alpha x) * g + b, then the rotation with the partner's normed value, in the
             * order of the reference's per-head norms and rotation (src/aria_taae.c:120-127) */
            const int S = e.rows_per_batch;
            float4 cs[NIT], sn[NIT];
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                if (rope) {   /* hs < S: the table row is in range past M too */
                    cs[it] = *reinterpret_cast<const float4 *>(e.cos_t + (size_t)hs * rh + i0);
                    sn[it] = *reinterpret_cast<const float4 *>(e.sin_t + (size_t)hs * rh + i0);
                }
                hs += hr;
                hb += hq;
                if (hs >= S) { hs -= S; hb++; }
            }
            const float gv[4] = {gw.x, gw.y, gw.z, gw.w}, dv[4] = {dbv.x, dbv.y, dbv.z, dbv.w};
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                float *w4 = v[it];
                if (kind != 2) {
#pragma unroll
                    for (int q = 0; q < 4; q++) w4[q] = tanh_fast(dal * w4[q]) * gv[q] + dv[q];
                }
                if (e.rot > 0) {   /* uniform: every lane takes part in the exchange */
                    float p[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) p[q] = __shfl_xor(w4[q], rh >> 2);
                    if (rope) {
                        const float cv[4] = {cs[it].x, cs[it].y, cs[it].z, cs[it].w};
                        const float sv[4] = {sn[it].x, sn[it].y, sn[it].z, sn[it].w};
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const float c0 = w4[q] * cv[q], s1 = p[q] * sv[q];
                            w4[q] = first ? c0 - s1 : c0 + s1;
                        }
                    }
                }
                const int m = mrow[it];
                if (m < a.M && col_ok)
                    *reinterpret_cast<float4 *>((float *)a.y + (size_t)m * a.N + nb) = make_float4(w4[0], w4[1], w4[2], w4[3]);
            }
        } else {   /* HEADS */
            const int S = e.rows_per_batch;
            float4 cs[NIT], sn[NIT];
            int sb[NIT], sp[NIT];
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                sb[it] = hb;
                sp[it] = hs;   /* hs < S: the table row is in range past M too */
                if (rope) {
                    cs[it] = *reinterpret_cast<const float4 *>(e.cos_t + (size_t)hs * rh + i0);
                    sn[it] = *reinterpret_cast<const float4 *>(e.sin_t + (size_t)hs * rh + i0);
                }
                hs += hr;
                hb += hq;
                if (hs >= S) { hs -= S; hb++; }
            }
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const int m = mrow[it];
                float *w4 = v[it];
                if (kind != 2) {
                    float ss = (w4[0] * w4[0] + w4[1] * w4[1]) + (w4[2] * w4[2] + w4[3] * w4[3]);
                    ss = grp_sum<16>(ss);
                    const float inv = __builtin_amdgcn_rsqf(ss * (1.0f / 64) + e.eps);
                    const float gv[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
                    for (int q = 0; q < 4; q++) w4[q] = (w4[q] * inv) * gv[q];   /* gv = 1 without gains */
                    if (e.rot > 0 && e.cos_t) {
                        const int lp = rh >> 2;   /* partner lane offset */
                        float p[4];
#pragma unroll
                        for (int q = 0; q < 4; q++) p[q] = rope_partner(w4[q], lane, lp);
                        if (rope) {
                            const float cv[4] = {cs[it].x, cs[it].y, cs[it].z, cs[it].w};
                            const float sv[4] = {sn[it].x, sn[it].y, sn[it].z, sn[it].w};
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                if (first) { float ac = w4[q] * cv[q], bs = p[q] * sv[q]; w4[q] = ac - bs; }
                                else { float bc = w4[q] * cv[q], as = p[q] * sv[q]; w4[q] = bc + as; }
                            }
                        }
                    }
                }
                if (m < a.M && col_ok) {
                    uint16_t *d = dsec + (((size_t)sb[it] * e.heads + hh) * S + sp[it]) * 64 + 4 * l16;
                    *reinterpret_cast<uint2 *>(d) = make_uint2(pack2h(w4[0], w4[1]), pack2h(w4[2], w4[3]));
                }
            }
        }
    }
    }
}

/* the weights-in-registers kernel's launcher (k_qgemm_wr.hip): BM = 32 * fm rows by
 * 256 weight rows per workgroup; wt is ARIA_WQ8 or ARIA_WQ4, activations fp16, K % 64 == 0 */
hipError_t qgemm_wr_launch(const QArgs &a, int wt, int fm, hipStream_t s);
/* the large-tile kernel's launcher (k_qgemm_big.hip): configuration cfg of
 * qgemm_big_ncfg(), BM = qgemm_big_bm(cfg) rows by qgemm_big_bn(cfg) weight rows per
 * workgroup; Q8 / Q4 weights, fp16 activations, K % 64 == 0 */
hipError_t qgemm_big_launch(const QArgs &a, int wt, int cfg, hipStream_t s);
int qgemm_big_ncfg();
int qgemm_big_bm(int cfg);
int qgemm_big_bn(int cfg);
/* the fp16-weight configuration for an M x N product (any K) */
int qgemm_big_f16_pick(int M, int N);
/* its W8A8 form (int8 activations with per-row scales in a.xscale, Q8 weights, K % 128 == 0) */
hipError_t qgemm_big_i8_launch(const QArgs &a, int cfg, hipStream_t s);
int qgemm_big_i8_ncfg();

#endif /* ARIA_QGEMM_DEV_H */
