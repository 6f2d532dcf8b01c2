/*
 * k_quant.hip - device-side Q8 / Q4 weight packing and unpacking, bit-exact
 * with the reference host quantizer.
 *
 * Layouts (src/aria_quant.h:9-13, 56-71):
 *   Q8: q int8 [N, K] row-major, scale fp32 [N]; scale = max|W[n,:]|/127,
 *       q = clamp(lrintf(W * (1/scale)), -127, 127), zero row -> q = 0.
 *   Q4: q u8 [N, ceil(K/2)], even k -> low nibble, odd k -> high nibble;
 *       scale fp32 [N, 2*ceil(K/32)] as [min, step] per 32-block, step =
 *       (max-min)/15, nib = clamp(lrintf((W-min) * (1/step)), 0, 15), step 0 -> 0.
 * Bit-exactness rests on IEEE division (HIP's default fp32 divide is correctly
 * rounded; __fdiv_rn makes it explicit), round-half-even conversion
 * (__float2int_rn == lrintf in the default rounding mode) and no contraction.
 *
 * Q8: one wave64 per row (max-reduce then quantize, the row stays in L1).
 * Q4: one thread per 32-element block; a block owns whole bytes (k0 is even),
 * so threads never share an output byte.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

static __device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* ---- Q8 ---- */
__global__ __launch_bounds__(256) void k_q8_quant(int8_t *q, float *scale, const float *W, int N, int K,
                                                  int vec) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const float *wr = W + (size_t)n * K;
    int8_t *qr = q + (size_t)n * K;
    float amax = 0.0f;
    if (vec) {
        const float4 *w4 = reinterpret_cast<const float4 *>(wr);
        for (int k = lane; k < K / 4; k += 64) {
            float4 v = w4[k];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(wr[k]));
    }
    amax = grp_max<64>(amax);
    const float s = __fdiv_rn(amax, 127.0f);
    if (lane == 0) scale[n] = s;
    const float inv = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    if (vec) {
        const float4 *w4 = reinterpret_cast<const float4 *>(wr);
        for (int k = lane; k < K / 4; k += 64) {
            float4 v = w4[k];
            char4 o;
            o.x = (signed char)(s > 0.0f ? clampi(__float2int_rn(__fmul_rn(v.x, inv)), -127, 127) : 0);
            o.y = (signed char)(s > 0.0f ? clampi(__float2int_rn(__fmul_rn(v.y, inv)), -127, 127) : 0);
            o.z = (signed char)(s > 0.0f ? clampi(__float2int_rn(__fmul_rn(v.z, inv)), -127, 127) : 0);
            o.w = (signed char)(s > 0.0f ? clampi(__float2int_rn(__fmul_rn(v.w, inv)), -127, 127) : 0);
            reinterpret_cast<char4 *>(qr)[k] = o;
        }
    } else {
        for (int k = lane; k < K; k += 64)
            qr[k] = (int8_t)(s > 0.0f ? clampi(__float2int_rn(__fmul_rn(wr[k], inv)), -127, 127) : 0);
    }
}

extern "C" hipError_t aria_k_q8_quant(int8_t *q, float *scale, const float *W, int N, int K, hipStream_t s) {
    if (N <= 0 || K <= 0) return hipSuccess;
    /* float4 rows need K % 4 == 0 and aligned bases; anything else takes the scalar loop */
    const int vec = K % 4 == 0 && ((uintptr_t)W & 15u) == 0 && ((uintptr_t)q & 3u) == 0;
    hipLaunchKernelGGL(k_q8_quant, dim3((N + 3) / 4), dim3(256), 0, s, q, scale, W, N, K, vec);
    return hipGetLastError();
}

/* ---- Q4 ---- */
__global__ __launch_bounds__(256) void k_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K,
                                                  int nblk, int rb) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (size_t)N * nblk) return;
    const int n = (int)(t / nblk), bi = (int)(t % nblk);
    const int k0 = bi * 32, k1 = k0 + 32 < K ? k0 + 32 : K, len = k1 - k0;
    const float *wr = W + (size_t)n * K + k0;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = i < len ? wr[i] : 0.0f;
    float mn = v[0], mx = v[0];
#pragma unroll
    for (int i = 1; i < 32; i++)
        if (i < len) { if (v[i] < mn) mn = v[i]; if (v[i] > mx) mx = v[i]; }
    const float st = __fdiv_rn(__fsub_rn(mx, mn), 15.0f);
    float2 pr; pr.x = mn; pr.y = st;
    reinterpret_cast<float2 *>(scale)[(size_t)n * nblk + bi] = pr;
    const float inv = st > 0.0f ? __fdiv_rn(1.0f, st) : 0.0f;
    uint8_t *qr = q + (size_t)n * rb + (k0 >> 1);
    uint32_t wv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        uint32_t nib = 0;
        if (i < len && st > 0.0f) nib = (uint32_t)clampi(__float2int_rn(__fmul_rn(__fsub_rn(v[i], mn), inv)), 0, 15);
        wv[i >> 3] |= nib << (4 * (i & 7));
    }
    const int nbytes = (len + 1) >> 1;
    if (nbytes == 16 && (((uintptr_t)qr) & 15u) == 0) {
        uint4 o; o.x = wv[0]; o.y = wv[1]; o.z = wv[2]; o.w = wv[3];
        *reinterpret_cast<uint4 *>(qr) = o;
    } else {
        for (int i = 0; i < nbytes; i++) qr[i] = (uint8_t)(wv[i >> 2] >> (8 * (i & 3)));
    }
}

extern "C" hipError_t aria_k_q4_quant(uint8_t *q, float *scale, const float *W, int N, int K, hipStream_t s) {
    if (N <= 0 || K <= 0) return hipSuccess;
    if (((uintptr_t)scale & 7u) != 0) return hipErrorInvalidValue;
    const int nblk = (K + 31) / 32, rb = (K + 1) / 2;
    const size_t nt = (size_t)N * nblk;
    hipLaunchKernelGGL(k_q4_quant, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, s, q, scale, W, N, K,
                       nblk, rb);
    return hipGetLastError();
}

/* ---- dequant (unpack) to fp32: the value each dequant-on-use GEMM consumes ---- */
__global__ __launch_bounds__(256) void k_q8_dequant(float *W, const int8_t *q, const float *scale, int N,
                                                    int K) {
    const size_t n_el = (size_t)N * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n_el; i += (size_t)gridDim.x * 256)
        W[i] = (float)q[i] * scale[i / K];
}
__global__ __launch_bounds__(256) void k_q4_dequant(float *W, const uint8_t *q, const float *scale, int N,
                                                    int K, int nblk, int rb) {
    const size_t n_el = (size_t)N * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n_el; i += (size_t)gridDim.x * 256) {
        const int n = (int)(i / K), k = (int)(i % K);
        const uint8_t byte = q[(size_t)n * rb + (k >> 1)];
        const int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
        const size_t si = ((size_t)n * nblk + k / 32) * 2;
        W[i] = scale[si] + (float)nib * scale[si + 1];
    }
}
static inline dim3 grid_cap(size_t n) {
    size_t b = (n + 255) / 256;
    if (b > 256 * 32) b = 256 * 32;
    return dim3((unsigned)(b ? b : 1));
}
extern "C" hipError_t aria_k_q8_dequant(float *W, const int8_t *q, const float *scale, int N, int K,
                                        hipStream_t s) {
    if (N <= 0 || K <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_q8_dequant, grid_cap((size_t)N * K), dim3(256), 0, s, W, q, scale, N, K);
    return hipGetLastError();
}
extern "C" hipError_t aria_k_q4_dequant(float *W, const uint8_t *q, const float *scale, int N, int K,
                                        hipStream_t s) {
    if (N <= 0 || K <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_q4_dequant, grid_cap((size_t)N * K), dim3(256), 0, s, W, q, scale, N, K,
                       (K + 31) / 32, (K + 1) / 2);
    return hipGetLastError();
}
