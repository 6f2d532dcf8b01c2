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
 * Vector path (rot/2 % 4 == 0, D % 4 == 0): a thread rotates 4 pairs in each of up to 4
 * head rows of one position, one float4 of each table shared by the rows.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

__device__ __forceinline__ void rot1(float &a, float &b, float c, float s) {
    float ac = a * c, bs = b * s, bc = b * c, as = a * s;
    a = ac - bs;
    b = bc + as;
}

/* x0 and (when non-NULL) x1 are rotated in one launch (q and k share the tables and the
 * shape). x is streamed once, with non-temporal loads and stores (the standalone op is the
 * only user: the DiT rotates q and k in its projection's epilogue); the tables, shared by
 * every head, load normally. A thread rotates 4 pairs (dims j..j+3 and rh+j..rh+j+3) of position p in HG
 * consecutive head rows: the HG rows' 2 HG float4 loads are all in flight before the first
 * rotation (a launch over 21-42 MB is one round of workgroups waiting on the same HBM latency,
 * so bytes in flight per lane set its pace), and the position's cos / sin float4s are read
 * once for the HG rows. Thread t: tensor, head group, position, 4-dim chunk, in that order
 * from the slowest, so the 8 lanes of one position cover its rotated half-rows contiguously. */
template <int HG>
__global__ __launch_bounds__(256) void k_rope4(float *x0, float *x1, const float *cos_t, const float *sin_t,
                                               int N, int D, int rh, size_t nt1, size_t nthreads) {
    const int tpr = rh >> 2;
    const size_t tt = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (tt >= nthreads) return;
    const bool second = tt >= nt1;
    const size_t t = second ? tt - nt1 : tt;
    float *x = second ? x1 : x0;
    const size_t pg = t / tpr;                 /* (head group, position) */
    const int j = (int)(t % tpr) * 4;
    const int p = (int)(pg % (size_t)N);
    const size_t g = pg / (size_t)N;
    float *r0 = x + ((g * HG) * (size_t)N + p) * D;
    const size_t hs = (size_t)N * D;           /* one head further */
    float4 a[HG], b[HG];
#pragma unroll
    for (int i = 0; i < HG; i++) {
        a[i] = ld_nt(reinterpret_cast<const float4 *>(r0 + i * hs + j));
        b[i] = ld_nt(reinterpret_cast<const float4 *>(r0 + i * hs + rh + j));
    }
    const float4 c = *reinterpret_cast<const float4 *>(cos_t + (size_t)p * rh + j);
    const float4 sn = *reinterpret_cast<const float4 *>(sin_t + (size_t)p * rh + j);
#pragma unroll
    for (int i = 0; i < HG; i++) {
        rot1(a[i].x, b[i].x, c.x, sn.x); rot1(a[i].y, b[i].y, c.y, sn.y);
        rot1(a[i].z, b[i].z, c.z, sn.z); rot1(a[i].w, b[i].w, c.w, sn.w);
        st_nt(reinterpret_cast<float4 *>(r0 + i * hs + j), a[i]);
        st_nt(reinterpret_cast<float4 *>(r0 + i * hs + rh + j), b[i]);
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
    const bool vec = rh % 4 == 0 && D % 4 == 0 && ((uintptr_t)x0 & 15u) == 0 && (!x1 || ((uintptr_t)x1 & 15u) == 0) &&
                     ((uintptr_t)cos_t & 15u) == 0 && ((uintptr_t)sin_t & 15u) == 0;
    if (vec) {
        /* four head rows per thread when H allows, else two, else one */
        const int hg = H % 4 == 0 ? 4 : H % 2 == 0 ? 2 : 1;
        const size_t nt1 = rows / hg * (rh / 4);
        const size_t nt = x1 ? 2 * nt1 : nt1;
        const dim3 grid((unsigned)((nt + 255) / 256));
        if (hg == 4) hipLaunchKernelGGL((k_rope4<4>), grid, dim3(256), 0, s, x0, x1, cos_t, sin_t, N, D, rh, nt1, nt);
        else if (hg == 2) hipLaunchKernelGGL((k_rope4<2>), grid, dim3(256), 0, s, x0, x1, cos_t, sin_t, N, D, rh, nt1, nt);
        else hipLaunchKernelGGL((k_rope4<1>), grid, dim3(256), 0, s, x0, x1, cos_t, sin_t, N, D, rh, nt1, nt);
    } else {
        const size_t nt1 = rows * rh;
        const size_t nt = x1 ? 2 * nt1 : nt1;
        size_t blocks = (nt + 255) / 256;
        if (blocks > 256 * 64) blocks = 256 * 64;
        hipLaunchKernelGGL(k_rope1, dim3((unsigned)blocks), dim3(256), 0, s, x0, x1, cos_t, sin_t, N, D, rh, nt1, nt);
    }
    return hipGetLastError();
}

extern "C" hipError_t aria_k_rope(float *x, const float *cos_t, const float *sin_t, int H, int N, int D,
                                  int rot_dim, hipStream_t s) {
    return aria_k_rope2(x, nullptr, cos_t, sin_t, H, N, D, rot_dim, s);
}
