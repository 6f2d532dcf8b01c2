/*
 * k_softmax.hip - in-place row softmax with optional additive mask.
 *
 * Replaces aria_softmax_inplace (src/aria_cpu.c:758-776) and the reference's
 * k_softmax / k_softmax_w (src/aria_cuda.cu:315-426). Semantics per row:
 *   v = x + mask; m = max v; e = expf(v - m); s = sum e;
 *   inv = s > 0 ? 1/s : 0; x = e * inv.
 * The reference sums e sequentially; here each lane sums its share and a
 * wave64 butterfly finishes, which stays inside the 1e-5 gate. exp(v - m) is
 * computed as 2^((v - m)*log2e) with v_exp_f32 (relative error ~|v-m| * 4e-8),
 * so the kernel stays bandwidth-bound; v - m is formed first, as in the
 * reference, so rows masked with -3.4e38 stay finite. The score tensor is
 * streamed once, so loads and stores are non-temporal.
 *
 * Mapping: one wave64 per row, the row held in registers (NV float4 per lane,
 * lane l owns vectors l, l+64, ...), so the row is read once and written once:
 * 8 bytes of HBM traffic per element. Rows up to 64*4*16 = 4096 columns stay
 * in registers; longer rows use a three-pass kernel that re-reads from cache.
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

template <int NV>
__global__ __launch_bounds__(256) void k_softmax_v(float *x, int rows, int cols, const float *mask) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int n4 = cols >> 2;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * cols);
    const float4 *mr = mask ? reinterpret_cast<const float4 *>(mask + (size_t)row * cols) : nullptr;
    /* every load of the row is issued before any is used: folding the max into the
     * guarded load loop made each load wait for the previous one (~12% slower) */
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int idx = j * 64 + lane;
        v[j] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (idx < n4) v[j] = ld_nt(xr + idx);
    }
    if (mr) {
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int idx = j * 64 + lane;
            if (idx < n4) {
                const float4 k = mr[idx];
                v[j].x += k.x; v[j].y += k.y; v[j].z += k.z; v[j].w += k.w;
            }
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; j++) m = fmaxf(fmaxf(m, v[j].x), fmaxf(v[j].y, fmaxf(v[j].z, v[j].w)));
    m = grp_max<64>(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int idx = j * 64 + lane;
        if (idx < n4) {
            v[j].x = __builtin_amdgcn_exp2f((v[j].x - m) * ARIA_LOG2E);
            v[j].y = __builtin_amdgcn_exp2f((v[j].y - m) * ARIA_LOG2E);
            v[j].z = __builtin_amdgcn_exp2f((v[j].z - m) * ARIA_LOG2E);
            v[j].w = __builtin_amdgcn_exp2f((v[j].w - m) * ARIA_LOG2E);
            s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
        }
    }
    s = grp_sum<64>(s);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int idx = j * 64 + lane;
        if (idx < n4) {
            float4 o = v[j];
            o.x *= inv; o.y *= inv; o.z *= inv; o.w *= inv;
            st_nt(xr + idx, o);
        }
    }
}

/* scalar register path for cols not a multiple of 4 (NS values per lane) */
template <int NS>
__global__ __launch_bounds__(256) void k_softmax_s(float *x, int rows, int cols, const float *mask) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float *xr = x + (size_t)row * cols;
    const float *mr = mask ? mask + (size_t)row * cols : nullptr;
    float v[NS];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NS; j++) {
        const int c = j * 64 + lane;
        if (c < cols) {
            v[j] = xr[c] + (mr ? mr[c] : 0.0f);
            m = fmaxf(m, v[j]);
        }
    }
    m = grp_max<64>(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; j++) {
        const int c = j * 64 + lane;
        if (c < cols) { v[j] = expf(v[j] - m); s += v[j]; }
    }
    s = grp_sum<64>(s);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
#pragma unroll
    for (int j = 0; j < NS; j++) {
        const int c = j * 64 + lane;
        if (c < cols) xr[c] = v[j] * inv;
    }
}

/* long rows: max pass, exp+sum pass (stores e), scale pass */
__global__ __launch_bounds__(256) void k_softmax_long(float *x, int rows, int cols, const float *mask) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float *xr = x + (size_t)row * cols;
    const float *mr = mask ? mask + (size_t)row * cols : nullptr;
    float m = -INFINITY;
    for (int c = lane; c < cols; c += 64) {
        float v = xr[c] + (mr ? mr[c] : 0.0f);
        m = fmaxf(m, v);
    }
    m = grp_max<64>(m);
    float s = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        float e = expf(xr[c] + (mr ? mr[c] : 0.0f) - m);
        xr[c] = e;
        s += e;
    }
    s = grp_sum<64>(s);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    for (int c = lane; c < cols; c += 64) xr[c] *= inv;
}

extern "C" hipError_t aria_k_softmax(float *x, int rows, int cols, const float *mask, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    dim3 grid((rows + 3) / 4), blk(256);
    const bool vec = cols % 4 == 0 && ((uintptr_t)x & 15u) == 0 && (!mask || ((uintptr_t)mask & 15u) == 0);
    if (vec) {
        const int nv = (cols / 4 + 63) / 64;
        if (nv <= 1) hipLaunchKernelGGL(k_softmax_v<1>, grid, blk, 0, s, x, rows, cols, mask);
        else if (nv <= 2) hipLaunchKernelGGL(k_softmax_v<2>, grid, blk, 0, s, x, rows, cols, mask);
        else if (nv <= 4) hipLaunchKernelGGL(k_softmax_v<4>, grid, blk, 0, s, x, rows, cols, mask);
        else if (nv <= 6) hipLaunchKernelGGL(k_softmax_v<6>, grid, blk, 0, s, x, rows, cols, mask);
        else if (nv <= 8) hipLaunchKernelGGL(k_softmax_v<8>, grid, blk, 0, s, x, rows, cols, mask);
        else if (nv <= 16) hipLaunchKernelGGL(k_softmax_v<16>, grid, blk, 0, s, x, rows, cols, mask);
        else hipLaunchKernelGGL(k_softmax_long, grid, blk, 0, s, x, rows, cols, mask);
    } else {
        const int ns = (cols + 63) / 64;
        if (ns <= 1) hipLaunchKernelGGL(k_softmax_s<1>, grid, blk, 0, s, x, rows, cols, mask);
        else if (ns <= 2) hipLaunchKernelGGL(k_softmax_s<2>, grid, blk, 0, s, x, rows, cols, mask);
        else if (ns <= 4) hipLaunchKernelGGL(k_softmax_s<4>, grid, blk, 0, s, x, rows, cols, mask);
        else if (ns <= 8) hipLaunchKernelGGL(k_softmax_s<8>, grid, blk, 0, s, x, rows, cols, mask);
        else if (ns <= 16) hipLaunchKernelGGL(k_softmax_s<16>, grid, blk, 0, s, x, rows, cols, mask);
        else if (ns <= 32) hipLaunchKernelGGL(k_softmax_s<32>, grid, blk, 0, s, x, rows, cols, mask);
        else hipLaunchKernelGGL(k_softmax_long, grid, blk, 0, s, x, rows, cols, mask);
    }
    return hipGetLastError();
}
