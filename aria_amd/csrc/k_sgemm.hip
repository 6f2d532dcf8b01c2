/*
 * k_sgemm.hip - fp32 SIMT GEMM and conv1d for the op-level ABI entries that the
 * reference serves with fp32 math: aria_cuda_linear / _linear_dev / _matmul /
 * _attention's two contractions / _conv1d (src/aria_gpu.h:40-60).
 *
 * These are not the dequant hot path (that is k_qgemm.hip on MFMA); they keep
 * fp32 operands so the op-level parity of the reference's test_cuda.c holds
 * (linear 1e-3 + 2e-4*max). Tiling: 64x64 output tile per 256-thread
 * workgroup, 4x4 outputs per thread, K staged through LDS 16 at a time,
 * fp32 FMA accumulation, alpha applied after the sum, bias added last.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

#define TM 64
#define TN 64
#define TK 16

__global__ __launch_bounds__(256) void k_sgemm(float *C, const float *A, const float *B, const float *bias,
                                               int M, int N, int K, int transB, float alpha,
                                               long long sA, long long sB, long long sC) {
    __shared__ float As[TK][TM + 4];
    __shared__ float Bs[TK][TN + 4];
    const int bz = blockIdx.z;
    A += (size_t)bz * sA;
    B += (size_t)bz * sB;
    C += (size_t)bz * sC;
    const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    const int tid = threadIdx.x;
    const int tr = tid / 16, tc = tid % 16;   /* 16x16 threads, 4x4 each */
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;

    for (int k0 = 0; k0 < K; k0 += TK) {
        /* A tile: 64 rows x 16 k, 1024 elements, 4 per thread */
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int idx = tid + e * 256;
            int r = idx / TK, kk = idx % TK;
            int gm = m0 + r, gk = k0 + kk;
            As[kk][r] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int idx = tid + e * 256;
            if (transB) {   /* B [N, K] */
                int c = idx / TK, kk = idx % TK;
                int gn = n0 + c, gk = k0 + kk;
                Bs[kk][c] = (gn < N && gk < K) ? B[(size_t)gn * K + gk] : 0.0f;
            } else {        /* B [K, N] */
                int kk = idx / TN, c = idx % TN;
                int gn = n0 + c, gk = k0 + kk;
                Bs[kk][c] = (gn < N && gk < K) ? B[(size_t)gk * N + gn] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TK; kk++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = As[kk][tr * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = Bs[kk][tc * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int gm = m0 + tr * 4 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int gn = n0 + tc * 4 + j;
            if (gn >= N) continue;
            float v = acc[i][j];
            if (alpha != 1.0f) v = v * alpha;
            if (bias) v = v + bias[gn];
            C[(size_t)gm * N + gn] = v;
        }
    }
}

extern "C" hipError_t aria_k_sgemm(float *C, const float *A, const float *B, const float *bias, int M,
                                   int N, int K, int transB, float alpha, int batch, long long sA,
                                   long long sB, long long sC, hipStream_t s) {
    if (M <= 0 || N <= 0 || batch <= 0) return hipSuccess;
    dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM, batch);
    hipLaunchKernelGGL(k_sgemm, grid, dim3(256), 0, s, C, A, B, bias, M, N, K, transB, alpha, sA, sB, sC);
    return hipGetLastError();
}

/* conv1d, stride 1 (src/aria_cpu.c:941-968): out[o,t] = b[o] + sum_i sum_k w[o,i,k]*in[i,t+k-pad],
 * accumulated in the reference's order (i outer, k inner). */
__global__ __launch_bounds__(256) void k_conv1d(float *out, const float *in, const float *w, const float *bias,
                                                int Cin, int Cout, int K, int pad, int L) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)Cout * L) return;
    const int o = (int)(idx / L), t = (int)(idx % L);
    float acc = bias ? bias[o] : 0.0f;
    const float *wo = w + (size_t)o * Cin * K;
    for (int i = 0; i < Cin; i++)
        for (int k = 0; k < K; k++) {
            int ti = t + k - pad;
            if (ti >= 0 && ti < L) { float p = wo[(size_t)i * K + k] * in[(size_t)i * L + ti]; acc = acc + p; }
        }
    out[idx] = acc;
}

extern "C" hipError_t aria_k_conv1d(float *out, const float *in, const float *w, const float *bias, int Cin,
                                    int Cout, int K, int pad, int L, hipStream_t s) {
    size_t n = (size_t)Cout * L;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_conv1d, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, in, w, bias, Cin,
                       Cout, K, pad, L);
    return hipGetLastError();
}
