/*
 * probe_micro.hip - issue-rate and bandwidth probes of the MI355X (gfx950) that the kernel designs
 * lean on: the fp16 MFMA rate, the issue cost of a wave64 fp32 FMA, exp2 and reciprocal, and the
 * LDS and L1 read bandwidth per CU. Measurement only: built into its own library,
 * aria_amd/libaria_probe.so, which bench.py --micro loads; the product library does not contain
 * these kernels.
 *
 * Every probe runs a fixed number of iterations of independent dependency chains per wave, so
 * the unit under test, not latency, sets the pace, and folds its chains into one store per lane
 * so nothing is optimised away. The host side times a launch with HIP events and converts:
 *   MICRO_MFMA  4 chains of v_mfma_f32_32x32x16_f16 per wave     -> FLOP / s
 *   MICRO_FMA   8 chains of v_fma_f32                            -> wave instructions / s
 *   MICRO_EXP   8 chains of v_exp_f32 (x = exp2(-x), stays in (0, 1])
 *   MICRO_RCP   8 chains of v_rcp_f32 (x = 1 / x)
 *   MICRO_LDS   8 ds_read_b128 per lane and iteration from a 16 KB LDS table -> bytes / s
 *   MICRO_L1    8 global_load_dwordx4 per lane and iteration from a 16 KB table per workgroup
 *               (resident in the CU's L1 after the first pass)                -> bytes / s
 *   MICRO_MIX_FMA  4 MFMA chains + 32 v_fma_f32 per trip (128 + 128 SIMD cycles if issued alone)
 *   MICRO_MIX_EXP  4 MFMA chains + 16 v_exp_f32 per trip (128 + 128)            -> trips / s
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x16_m __attribute__((ext_vector_type(16)));
typedef _Float16 half8_m __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void k_micro_mfma(float *out, int iters) {
    const int t = threadIdx.x;
    half8_m a, b;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        a[j] = (_Float16)(0.125f * (float)((t + j) & 7));
        b[j] = (_Float16)(0.0625f * (float)((t * 3 + j) & 7));
    }
    f32x16_m c0, c1, c2, c3;
#pragma unroll
    for (int r = 0; r < 16; r++) { c0[r] = 0.0f; c1[r] = 0.0f; c2[r] = 0.0f; c3[r] = 0.0f; }
    for (int i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) s += (c0[r] + c1[r]) + (c2[r] + c3[r]);
    out[(size_t)blockIdx.x * 256 + t] = s;
}

template <int OP>
__global__ __launch_bounds__(256) void k_micro_valu(float *out, int iters, float m, float k) {
    const int t = threadIdx.x;
    float x[8];
#pragma unroll
    for (int c = 0; c < 8; c++) x[c] = 0.5f + 0.001f * (float)(t + c);
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
            if constexpr (OP == 0) x[c] = __builtin_fmaf(x[c], m, k);
            else if constexpr (OP == 1) x[c] = __builtin_amdgcn_exp2f(-x[c]);
            else x[c] = __builtin_amdgcn_rcpf(x[c]);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; c++) s += x[c];
    out[(size_t)blockIdx.x * 256 + t] = s;
}

/* MFMA chains and VALU chains in one wave: per trip 4 MFMAs (4 x 32 cycles of the matrix pipe)
 * and 8 NV independent v_fma_f32 (OP 0) or v_exp_f32 (OP 1); whether the SIMD overlaps the two
 * shows as a trip time near the larger of the two instead of their sum */
template <int OP, int NV>
__global__ __launch_bounds__(256) void k_micro_mix(float *out, int iters, float m, float k) {
    const int t = threadIdx.x;
    half8_m a, b;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        a[j] = (_Float16)(0.125f * (float)((t + j) & 7));
        b[j] = (_Float16)(0.0625f * (float)((t * 3 + j) & 7));
    }
    f32x16_m c0, c1, c2, c3;
#pragma unroll
    for (int r = 0; r < 16; r++) { c0[r] = 0.0f; c1[r] = 0.0f; c2[r] = 0.0f; c3[r] = 0.0f; }
    float x[8];
#pragma unroll
    for (int c = 0; c < 8; c++) x[c] = 0.5f + 0.001f * (float)(t + c);
    for (int i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < NV; v++)
#pragma unroll
            for (int c = 0; c < 8; c++) {
                if (v == NV / 2 && c == 0) {
                    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
                    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
                }
                if constexpr (OP == 0) x[c] = __builtin_fmaf(x[c], m, k);
                else x[c] = __builtin_amdgcn_exp2f(-x[c]);
            }
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) s += (c0[r] + c1[r]) + (c2[r] + c3[r]);
#pragma unroll
    for (int c = 0; c < 8; c++) s += x[c];
    out[(size_t)blockIdx.x * 256 + t] = s;
}

__global__ __launch_bounds__(256) void k_micro_lds(float *out, int iters) {
    __shared__ uint4 tab[1024];
    const int t = threadIdx.x;
    for (int i = t; i < 1024; i += 256) tab[i] = make_uint4(i, i * 3u, i * 5u, i * 7u);
    __syncthreads();
    uint4 acc[8];
#pragma unroll
    for (int u = 0; u < 8; u++) acc[u] = make_uint4(0u, 0u, 0u, 0u);
    int idx = t & 63;
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint4 v = tab[(idx + 64 * u) & 1023];
            acc[u].x ^= v.x; acc[u].y ^= v.y; acc[u].z ^= v.z; acc[u].w ^= v.w;
        }
        idx += 512 + 1;
    }
    uint32_t s = 0;
#pragma unroll
    for (int u = 0; u < 8; u++) s ^= acc[u].x ^ acc[u].y ^ acc[u].z ^ acc[u].w;
    out[(size_t)blockIdx.x * 256 + t] = (float)s;
}

__global__ __launch_bounds__(256) void k_micro_l1(float *out, const uint4 *tab, int iters) {
    const int t = threadIdx.x;
    const uint4 *base = tab + (size_t)blockIdx.x * 1024;   /* this workgroup's 16 KB */
    uint4 acc[8];
#pragma unroll
    for (int u = 0; u < 8; u++) acc[u] = make_uint4(0u, 0u, 0u, 0u);
    int idx = t & 63;
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint4 v = base[(idx + 64 * u) & 1023];
            acc[u].x ^= v.x; acc[u].y ^= v.y; acc[u].z ^= v.z; acc[u].w ^= v.w;
        }
        idx += 512 + 1;
    }
    uint32_t s = 0;
#pragma unroll
    for (int u = 0; u < 8; u++) s ^= acc[u].x ^ acc[u].y ^ acc[u].z ^ acc[u].w;
    out[(size_t)blockIdx.x * 256 + t] = (float)s;
}

/* One launch of probe `which` (MICRO_* above, 0..7) with `grid` workgroups of 256 lanes and
 * `iters` loop trips on `stream`; out: grid * 256 floats; tab (MICRO_L1 only): grid * 16 KB of
 * device memory. Returns the hipError_t code of the launch (0 on success). */
extern "C" int aria_probe_micro(int which, int grid, int iters, float *out, const void *tab, void *stream) {
    if (grid <= 0 || iters <= 0 || !out) return hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    switch (which) {
        case 0: hipLaunchKernelGGL(k_micro_mfma, dim3(grid), dim3(256), 0, s, out, iters); break;
        case 1: hipLaunchKernelGGL(k_micro_valu<0>, dim3(grid), dim3(256), 0, s, out, iters, 0.999f, 0.001f); break;
        case 2: hipLaunchKernelGGL(k_micro_valu<1>, dim3(grid), dim3(256), 0, s, out, iters, 0.999f, 0.001f); break;
        case 3: hipLaunchKernelGGL(k_micro_valu<2>, dim3(grid), dim3(256), 0, s, out, iters, 0.999f, 0.001f); break;
        case 4: hipLaunchKernelGGL(k_micro_lds, dim3(grid), dim3(256), 0, s, out, iters); break;
        case 5:
            if (!tab) return hipErrorInvalidValue;
            hipLaunchKernelGGL(k_micro_l1, dim3(grid), dim3(256), 0, s, out, (const uint4 *)tab, iters);
            break;
        case 6: hipLaunchKernelGGL((k_micro_mix<0, 4>), dim3(grid), dim3(256), 0, s, out, iters, 0.999f, 0.001f); break;
        case 7: hipLaunchKernelGGL((k_micro_mix<1, 2>), dim3(grid), dim3(256), 0, s, out, iters, 0.999f, 0.001f); break;
        default: return hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}
