/*
 * aria_dev.h - device helpers shared by the gfx950 kernels: wave64 reductions,
 * the reference's elementwise formulas in their exact evaluation order, and
 * half/float packing. Included by .hip translation units only.
 *
 * All kernels are compiled with -ffp-contract=off, so a*b+c below is two
 * roundings, as in the reference's -std=c11 CPU build; fused multiply-adds
 * are written out as __builtin_fmaf where one is intended.
 */
#ifndef ARIA_DEV_H
#define ARIA_DEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#define ARIA_WAVE 64

/* ---- wave64 reductions over groups of G lanes (G = 4, 8, 16, 32 or 64) ----
 * Within a 16-lane DPP row the butterfly runs on DPP lane swizzles (quad xor 1,
 * quad xor 2, half-row mirror, row mirror), which read the neighbour's VGPR in the
 * same instruction with no LDS round trip. Across rows: one xor-16 shuffle for
 * G = 32, and four readlanes of the row results for G = 64. Every lane of a
 * group ends with the same value (each step combines a symmetric pair with a
 * commutative operation). */
enum { DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_ROW_HALF_MIRROR = 0x141, DPP_ROW_MIRROR = 0x140 };

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

/* the value of lane l ^ 32 (lane = this lane's index in the wave): gfx950's
 * v_permlane32_swap exchanges the wave's two 32-lane halves in registers, without the LDS
 * round trip of ds_bpermute */
__device__ __forceinline__ float xor32_f32(float v, int lane) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, lane < 32 ? r[1] : r[0]);
}

struct OpSum {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpMin {
    __device__ __forceinline__ float operator()(float a, float b) const { return fminf(a, b); }
};

template <int G, typename Op>
__device__ __forceinline__ float grp_reduce(float v, Op op) {
    static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
    v = op(v, dpp_f32<DPP_QUAD_XOR1>(v));
    v = op(v, dpp_f32<DPP_QUAD_XOR2>(v));
    if (G >= 8) v = op(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
    if (G >= 16) v = op(v, dpp_f32<DPP_ROW_MIRROR>(v));
    if (G == 32) v = op(v, __shfl_xor(v, 16, ARIA_WAVE));
    if (G == 64) v = op(op(readlane_f32(v, 0), readlane_f32(v, 16)), op(readlane_f32(v, 32), readlane_f32(v, 48)));
    return v;
}
template <int G>
__device__ __forceinline__ double grp_reduce_sum_f64(double v) {
    static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
    v += dpp_f64<DPP_QUAD_XOR1>(v);
    v += dpp_f64<DPP_QUAD_XOR2>(v);
    if (G >= 8) v += dpp_f64<DPP_ROW_HALF_MIRROR>(v);
    if (G >= 16) v += dpp_f64<DPP_ROW_MIRROR>(v);
    if (G == 32) v += __shfl_xor(v, 16, ARIA_WAVE);
    if (G == 64) v = (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
    return v;
}

template <int G> __device__ __forceinline__ float grp_sum(float v) { return grp_reduce<G>(v, OpSum()); }
template <int G> __device__ __forceinline__ double grp_sum(double v) { return grp_reduce_sum_f64<G>(v); }
template <int G> __device__ __forceinline__ float grp_max(float v) { return grp_reduce<G>(v, OpMax()); }
template <int G> __device__ __forceinline__ float grp_min(float v) { return grp_reduce<G>(v, OpMin()); }

/* Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2):
 * workgroup g runs on XCD g % 8. Tile t = (g % 8) * ceil(T/8) + g / 8 gives each XCD a
 * contiguous run of tiles; launch a multiple of 8 workgroups and skip t >= T. */
__device__ __forceinline__ int xcd_tile(int g, int T) {
    const int per = (T + 7) >> 3;
    return (g & 7) * per + (g >> 3);
}

/* ---- exp2-based transcendentals (v_exp_f32 / v_rcp_f32, ~1 ulp each) ----
 * exp(x) = 2^(x*log2 e); the rounding of x*log2 e gives a relative error of about
 * |x| * 4e-8, far inside the 1e-5 gates for the ranges these ops see. */
#define ARIA_LOG2E 1.44269504088896341f
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * ARIA_LOG2E); }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

/* ---- rotate-half RoPE partner within a 16-lane group holding one 64-wide head ----
 * Lane l holds dims 4l..4l+3; dim d < rh pairs with d + rh (rh = rot/2), so lane l < lp
 * (lp = rh/4) pairs with lane l + lp and lane l in [lp, 2lp) with lane l - lp (lanes past
 * 2lp hold unrotated dims; their partner value is unused). One ds_bpermute per value:
 * DPP row shifts need a compile-time shift and were slower here. */
__device__ __forceinline__ float rope_partner(float v, int lane, int lp) {
    const int l16 = lane & 15;
    return __shfl(v, (lane & 48) | (l16 < lp ? l16 + lp : l16 - lp), ARIA_WAVE);
}

/* ---- reference formulas, evaluation order as written in the reference C ---- */

/* tanh GELU, src/aria_cpu.c:742-749: (0.5*v)*(1 + tanh(u)), u = c*(v + 0.044715*v^3).
 * Evaluated through 1 + tanh(u) = 2/(1 + e^{-2u}), i.e. gelu(v) = v / (1 + e^{-2u}),
 * with -2u*log2(e) = v*(k1 + k2*v^2) and the constants folded: v*v, one fma, a mul,
 * v_exp_f32, an add, v_rcp_f32 and a mul, 7 VALU where the tanh form takes 14 (no
 * contraction). Error ~3 ulp near 0 and relative ~|u|*4e-7 in the tail, inside the
 * 1e-5 gates. Limits match the reference: 1 + e^{-2u} -> 1 gives v exactly (tanh = 1),
 * e^{-2u} -> inf gives v*0 = -0 for v < 0 (0.5*v*(1 - 1)), v = -inf gives NaN as
 * 0.5*(-inf)*0 does. */
__device__ __forceinline__ float gelu_tanh_f(float v) {
    constexpr float k1 = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634);
    constexpr float k2 = (float)(-2.0 * 0.7978845608028654 * 0.044715 * 1.4426950408889634);
    const float t = __builtin_fmaf(k2, v * v, k1);
    const float e = __builtin_amdgcn_exp2f(v * t);
    return v * rcp_fast(1.0f + e);
}

/* tanh through tanh(x) = 1 - 2/(e^{2x} + 1): v_exp_f32, an add, v_rcp_f32 and an fma, where
 * the device library's tanhf takes ~30 instructions with branches. Absolute error a few
 * 1e-7 (near 0 the subtraction cancels, so the relative error grows as 1e-7/|x| while the
 * absolute error stays); the limits are exact: e^{2x} -> inf gives 1, -> 0 gives -1. Used by
 * the decoder's DynamicTanh norms inside GEMM epilogues (the q/k norms of DYT_ROPE and the
 * block norms of ADD_DYT, whose outputs are rounded to fp16 right after), where the error
 * is far inside the decoder's gate (1e-3 + 5e-3 * max). */
__device__ __forceinline__ float tanh_fast(float x) {
    return __builtin_fmaf(-2.0f, rcp_fast(__builtin_amdgcn_exp2f(x * (2.0f * ARIA_LOG2E)) + 1.0f), 1.0f);
}

/* silu, src/aria_cpu.c:735-740: v / (1 + exp(-v)), as v * rcp(1 + exp(-v)). */
__device__ __forceinline__ float silu_f(float v) { return v * rcp_fast(1.0f + exp_fast(-v)); }

/* sigmoid(1 - g) as the DiT gate uses it (src/aria_sa3_dit.c:85-90). */
__device__ __forceinline__ float gate_sig_f(float g) { return rcp_fast(1.0f + exp_fast(-(1.0f - g))); }

/* IEEE half, round to nearest even (== aria_float_to_half for finite values). */
__device__ __forceinline__ uint16_t f2h_bits(float v) {
    _Float16 h = (_Float16)v;
    return __builtin_bit_cast(uint16_t, h);
}

/* W8A8 activation quantisation of four values (src/aria_quant.c:264-266): rint (ties to
 * even, as lrintf in the default rounding mode) of v * inv, clamped to [-127, 127], packed
 * as four int8 in one word (element 0 in the low byte) */
__device__ __forceinline__ uint32_t q8_pack4(float4 v, float inv) {
    const float f[4] = {v.x * inv, v.y * inv, v.z * inv, v.w * inv};
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = min(max((int)__builtin_rintf(f[i]), -127), 127);
        w |= (uint32_t)(q & 0xFF) << (8 * i);
    }
    return w;
}

/* non-temporal 128-bit load/store of a float4 (streamed-once data) */
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float4 *p) {
    f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float4 *p, float4 o) {
    f32x4_t v = {o.x, o.y, o.z, o.w};
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t *>(p));
}

/* float4 element access by compile-time or run-time index */
__device__ __forceinline__ float f4get(const float4 &v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ void f4set(float4 &v, int i, float x) {
    if (i == 0) v.x = x; else if (i == 1) v.y = x; else if (i == 2) v.z = x; else v.w = x;
}

#endif /* ARIA_DEV_H */
