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

/* ---- wave64 butterfly reductions over groups of G lanes (G a power of two) ---- */
template <int G>
__device__ __forceinline__ float grp_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, ARIA_WAVE);
    return v;
}
template <int G>
__device__ __forceinline__ double grp_sum(double v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, ARIA_WAVE);
    return v;
}
template <int G>
__device__ __forceinline__ float grp_max(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, ARIA_WAVE));
    return v;
}
template <int G>
__device__ __forceinline__ float grp_min(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, ARIA_WAVE));
    return v;
}

/* ---- reference formulas, evaluation order as written in the reference C ---- */

/* tanh GELU, src/aria_cpu.c:742-749: inner = c*(v + ((0.044715*v)*v)*v);
 * out = (0.5*v)*(1 + tanh(inner)). */
__device__ __forceinline__ float gelu_tanh_f(float v) {
    const float c = 0.7978845608028654f;
    float cube = 0.044715f * v;
    cube = cube * v;
    cube = cube * v;
    float inner = c * (v + cube);
    float h = 0.5f * v;
    return h * (1.0f + tanhf(inner));
}

/* silu, src/aria_cpu.c:735-740: v / (1 + exp(-v)). */
__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

/* sigmoid(1 - g) as the DiT gate uses it (src/aria_sa3_dit.c:85-90). */
__device__ __forceinline__ float gate_sig_f(float g) { return 1.0f / (1.0f + expf(-(1.0f - g))); }

/* IEEE half, round to nearest even (== aria_float_to_half for finite values). */
__device__ __forceinline__ uint16_t f2h_bits(float v) {
    _Float16 h = (_Float16)v;
    return __builtin_bit_cast(uint16_t, h);
}

/* float4 element access by compile-time or run-time index */
__device__ __forceinline__ float f4get(const float4 &v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ void f4set(float4 &v, int i, float x) {
    if (i == 0) v.x = x; else if (i == 1) v.y = x; else if (i == 2) v.z = x; else v.w = x;
}

#endif /* ARIA_DEV_H */
