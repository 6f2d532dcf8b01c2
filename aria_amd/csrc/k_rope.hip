/*
 * k_rope.hip - rotate-half rotary embedding in place on x [H, N, D].
 *
 * Replaces aria_rope_apply (src/aria_cpu.c:790-809) and the reference's k_rope
 * (src/aria_cuda.cu:433-445). For each row (h, p) and i < rot/2 with
 * a = x[i], b = x[i + rot/2], c = cos[p, i], s = sin[p, i]:
 *   x[i] = a*c - b*s,  x[i + rot/2] = b*c + a*s   (separate roundings);
 * dims >= rot are neither read nor written, so HBM traffic is 2*rot*4 bytes
 * per row plus the small position tables, which stay in cache across heads.
 *
 * Vector path (rot/2 % 4 == 0, D % 4 == 0): a thread rotates 4 pairs with two
 * float4 loads of x and two of the tables.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

__device__ __forceinline__ void rot1(float &a, float &b, float c, float s) {
    float ac = a * c, bs = b * s, bc = b * c, as = a * s;
    a = ac - bs;
    b = bc + as;
}

/* x0 and (when non-NULL) x1 are rotated in one launch: threads [0, nt1) take x0,
 * [nt1, 2*nt1) take x1 (q and k share the tables and the shape). */
__global__ __launch_bounds__(256) void k_rope4(float *x0, float *x1, const float *cos_t, const float *sin_t,
                                               int N, int D, int rh, size_t nt1, size_t nthreads) {
    const int tpr = rh >> 2;
    for (size_t tt = (size_t)blockIdx.x * 256 + threadIdx.x; tt < nthreads; tt += (size_t)gridDim.x * 256) {
        const bool second = tt >= nt1;
        const size_t t = second ? tt - nt1 : tt;
        float *x = second ? x1 : x0;
        size_t row = t / tpr;
        int j = (int)(t % tpr) * 4;
        int p = (int)(row % (size_t)N);
        float *r = x + row * D;
        float4 a = *reinterpret_cast<float4 *>(r + j);
        float4 b = *reinterpret_cast<float4 *>(r + rh + j);
        float4 c = *reinterpret_cast<const float4 *>(cos_t + (size_t)p * rh + j);
        float4 s = *reinterpret_cast<const float4 *>(sin_t + (size_t)p * rh + j);
        rot1(a.x, b.x, c.x, s.x); rot1(a.y, b.y, c.y, s.y);
        rot1(a.z, b.z, c.z, s.z); rot1(a.w, b.w, c.w, s.w);
        *reinterpret_cast<float4 *>(r + j) = a;
        *reinterpret_cast<float4 *>(r + rh + j) = b;
    }
}

__global__ __launch_bounds__(256) void k_rope1(float *x0, float *x1, const float *cos_t, const float *sin_t,
                                               int N, int D, int rh, size_t nt1, size_t nthreads) {
    for (size_t tt = (size_t)blockIdx.x * 256 + threadIdx.x; tt < nthreads; tt += (size_t)gridDim.x * 256) {
        const bool second = tt >= nt1;
        const size_t t = second ? tt - nt1 : tt;
        float *x = second ? x1 : x0;
        size_t row = t / rh;
        int i = (int)(t % rh);
        int p = (int)(row % (size_t)N);
        float *r = x + row * D;
        float a = r[i], b = r[i + rh];
        rot1(a, b, cos_t[(size_t)p * rh + i], sin_t[(size_t)p * rh + i]);
        r[i] = a;
        r[i + rh] = b;
    }
}

extern "C" hipError_t aria_k_rope2(float *x0, float *x1, const float *cos_t, const float *sin_t, int H, int N,
                                   int D, int rot_dim, hipStream_t s) {
    const int rh = rot_dim / 2;
    if (H <= 0 || N <= 0 || rh <= 0) return hipSuccess;
    const size_t rows = (size_t)H * N;
    const bool vec = rh % 4 == 0 && D % 4 == 0 && ((uintptr_t)x0 & 15u) == 0 && ((uintptr_t)x1 & 15u) == 0 &&
                     ((uintptr_t)cos_t & 15u) == 0 && ((uintptr_t)sin_t & 15u) == 0;
    const size_t nt1 = vec ? rows * (rh / 4) : rows * rh;
    const size_t nt = x1 ? 2 * nt1 : nt1;
    size_t blocks = (nt + 255) / 256;
    if (blocks > 256 * 64) blocks = 256 * 64;
    if (vec)
        hipLaunchKernelGGL(k_rope4, dim3((unsigned)blocks), dim3(256), 0, s, x0, x1, cos_t, sin_t, N, D, rh, nt1, nt);
    else
        hipLaunchKernelGGL(k_rope1, dim3((unsigned)blocks), dim3(256), 0, s, x0, x1, cos_t, sin_t, N, D, rh, nt1, nt);
    return hipGetLastError();
}

extern "C" hipError_t aria_k_rope(float *x, const float *cos_t, const float *sin_t, int H, int N, int D,
                                  int rot_dim, hipStream_t s) {
    return aria_k_rope2(x, nullptr, cos_t, sin_t, H, N, D, rot_dim, s);
}
