/*
 * k_elementwise.hip - bandwidth-bound elementwise and broadcast kernels.
 *
 * Replaces aria_add/addto/scale/axpy (src/aria_cpu.c:989-1000), aria_silu,
 * aria_gelu_tanh, aria_silu_gate, aria_softcap, aria_dynamic_tanh
 * (src/aria_cpu.c:684-756), the DiT glue adaln_modulate / gate_sigmoid + residual
 * (src/aria_sa3_dit.c:71-97, 211-215, 280-284), the GLU combine
 * (src/aria_sa3_dit.c:108-121) and the pingpong update (src/aria_sampler.c:216-220).
 *
 * Every kernel streams 128-bit float4 vectors with a grid-stride loop when the
 * element count and the pointers allow it (one read of each input, one write),
 * and falls back to a scalar loop otherwise. Arithmetic follows the reference's
 * evaluation order with separate roundings (built with -ffp-contract=off).
 */
#include "aria_dev.h"
#include "aria_hip_kernels.h"

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* Grid for a streaming kernel over n4 float4: enough workgroups to fill 256 CUs
 * several times, each thread then strides. */
static inline dim3 stream_grid(size_t n4) {
    size_t blocks = (n4 + 255) / 256;
    const size_t cap = 256 * 32;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    return dim3((unsigned)blocks);
}

#define GRID_STRIDE(i, n) \
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (size_t)gridDim.x * blockDim.x)

/* ---- unary maps y = f(x) ---- */
enum { U_GELU = 0, U_SILU = 1, U_SCALE = 2, U_SOFTCAP = 3 };

template <int OP>
__device__ __forceinline__ float unary_f(float v, float a) {
    if (OP == U_GELU) return gelu_tanh_f(v);
    if (OP == U_SILU) return silu_f(v);
    if (OP == U_SCALE) return v * a;
    /* softcap, src/aria_cpu.c:730-733: cap * tanh(s / cap) */
    return a * tanhf(v / a);
}

template <int OP>
__global__ __launch_bounds__(256) void k_unary4(float4 *y, const float4 *x, float a, size_t n4) {
    GRID_STRIDE(i, n4) {
        float4 v = x[i];
        v.x = unary_f<OP>(v.x, a); v.y = unary_f<OP>(v.y, a);
        v.z = unary_f<OP>(v.z, a); v.w = unary_f<OP>(v.w, a);
        y[i] = v;
    }
}
template <int OP>
__global__ __launch_bounds__(256) void k_unary1(float *y, const float *x, float a, size_t n) {
    GRID_STRIDE(i, n) y[i] = unary_f<OP>(x[i], a);
}

template <int OP>
static hipError_t launch_unary(float *y, const float *x, float a, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && al16(x) && al16(y))
        hipLaunchKernelGGL(k_unary4<OP>, stream_grid(n / 4), dim3(256), 0, s, (float4 *)y,
                           (const float4 *)x, a, n / 4);
    else
        hipLaunchKernelGGL(k_unary1<OP>, stream_grid((n + 3) / 4), dim3(256), 0, s, y, x, a, n);
    return hipGetLastError();
}

extern "C" hipError_t aria_k_gelu_tanh(float *y, const float *x, size_t n, hipStream_t s) {
    return launch_unary<U_GELU>(y, x, 0.0f, n, s);
}
extern "C" hipError_t aria_k_silu(float *y, const float *x, size_t n, hipStream_t s) {
    return launch_unary<U_SILU>(y, x, 0.0f, n, s);
}
extern "C" hipError_t aria_k_scale(float *y, const float *x, float a, size_t n, hipStream_t s) {
    return launch_unary<U_SCALE>(y, x, a, n, s);
}
extern "C" hipError_t aria_k_softcap(float *y, const float *x, float cap, size_t n, hipStream_t s) {
    return launch_unary<U_SOFTCAP>(y, x, cap, n, s);
}

/* ---- binary maps ---- */
enum { B_ADD = 0, B_AXPY = 1, B_SILU_GATE = 2 };

template <int OP>
__device__ __forceinline__ float binary_f(float a, float b, float s) {
    if (OP == B_ADD) return a + b;           /* y = a + b */
    if (OP == B_AXPY) return a + s * b;      /* y += s*x: a = y, b = x */
    return silu_f(a) * b;                    /* silu(gate) * up */
}

template <int OP>
__global__ __launch_bounds__(256) void k_binary4(float4 *y, const float4 *a, const float4 *b, float s,
                                                 size_t n4) {
    GRID_STRIDE(i, n4) {
        float4 p = a[i], q = b[i], r;
        r.x = binary_f<OP>(p.x, q.x, s); r.y = binary_f<OP>(p.y, q.y, s);
        r.z = binary_f<OP>(p.z, q.z, s); r.w = binary_f<OP>(p.w, q.w, s);
        y[i] = r;
    }
}
template <int OP>
__global__ __launch_bounds__(256) void k_binary1(float *y, const float *a, const float *b, float s,
                                                 size_t n) {
    GRID_STRIDE(i, n) y[i] = binary_f<OP>(a[i], b[i], s);
}

template <int OP>
static hipError_t launch_binary(float *y, const float *a, const float *b, float s, size_t n,
                                hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && al16(y) && al16(a) && al16(b))
        hipLaunchKernelGGL(k_binary4<OP>, stream_grid(n / 4), dim3(256), 0, st, (float4 *)y,
                           (const float4 *)a, (const float4 *)b, s, n / 4);
    else
        hipLaunchKernelGGL(k_binary1<OP>, stream_grid((n + 3) / 4), dim3(256), 0, st, y, a, b, s, n);
    return hipGetLastError();
}

extern "C" hipError_t aria_k_add(float *y, const float *a, const float *b, size_t n, hipStream_t s) {
    return launch_binary<B_ADD>(y, a, b, 0.0f, n, s);
}
extern "C" hipError_t aria_k_axpy(float *y, const float *x, float a, size_t n, hipStream_t s) {
    return launch_binary<B_AXPY>(y, y, x, a, n, s);
}
extern "C" hipError_t aria_k_silu_gate(float *out, const float *gate, const float *up, size_t n,
                                       hipStream_t s) {
    return launch_binary<B_SILU_GATE>(out, gate, up, 0.0f, n, s);
}

/* ---- row-broadcast kernels over [rows, dim], per-batch vectors [nbatch, dim] ---- */

/* y = x*(1+scale)+shift (src/aria_sa3_dit.c:71-82) */
__global__ __launch_bounds__(256) void k_modulate4(float4 *y, const float4 *x, const float4 *scale,
                                                   const float4 *shift, int dim4, size_t per_batch4,
                                                   size_t n4) {
    GRID_STRIDE(i, n4) {
        size_t bt = i / per_batch4;
        int c = (int)(i % (size_t)dim4);
        float4 v = x[i], sc = scale[bt * dim4 + c], sh = shift[bt * dim4 + c], o;
        o.x = v.x * (1.0f + sc.x) + sh.x; o.y = v.y * (1.0f + sc.y) + sh.y;
        o.z = v.z * (1.0f + sc.z) + sh.z; o.w = v.w * (1.0f + sc.w) + sh.w;
        y[i] = o;
    }
}
__global__ __launch_bounds__(256) void k_modulate1(float *y, const float *x, const float *scale,
                                                   const float *shift, int dim, size_t per_batch,
                                                   size_t n) {
    GRID_STRIDE(i, n) {
        size_t bt = i / per_batch;
        int c = (int)(i % (size_t)dim);
        y[i] = x[i] * (1.0f + scale[bt * dim + c]) + shift[bt * dim + c];
    }
}
extern "C" hipError_t aria_k_modulate(float *y, const float *x, const float *scale,
                                      const float *shift, int rows, int dim, int rows_per_batch,
                                      hipStream_t s) {
    size_t n = (size_t)rows * dim;
    if (n == 0) return hipSuccess;
    if (rows_per_batch <= 0) rows_per_batch = rows;
    size_t per = (size_t)rows_per_batch * dim;
    if (dim % 4 == 0 && al16(y) && al16(x) && al16(scale) && al16(shift))
        hipLaunchKernelGGL(k_modulate4, stream_grid(n / 4), dim3(256), 0, s, (float4 *)y,
                           (const float4 *)x, (const float4 *)scale, (const float4 *)shift, dim / 4,
                           per / 4, n / 4);
    else
        hipLaunchKernelGGL(k_modulate1, stream_grid((n + 3) / 4), dim3(256), 0, s, y, x, scale, shift,
                           dim, per, n);
    return hipGetLastError();
}

/* out = res + (o [+ b]) * sigmoid(1-gate); the bias binds to o first and a NULL
 * bias adds nothing (src/aria_cuda.cu:620-628 keeps -0.0 the same way). */
__device__ __forceinline__ float gate_res_f(float r, float o, float g, const float *b, int c) {
    float ov = b ? o + b[c] : o;
    float t = ov * gate_sig_f(g);
    return r + t;
}
__global__ __launch_bounds__(256) void k_gate_res4(float4 *out, const float4 *res, const float4 *o,
                                                   const float *gate, const float *b, int dim4,
                                                   size_t per_batch4, size_t n4) {
    GRID_STRIDE(i, n4) {
        size_t bt = i / per_batch4;
        int c4 = (int)(i % (size_t)dim4);
        const float *g = gate + bt * (size_t)dim4 * 4;
        float4 r = res[i], v = o[i], y;
        int c = 4 * c4;
        y.x = gate_res_f(r.x, v.x, g[c + 0], b, c + 0);
        y.y = gate_res_f(r.y, v.y, g[c + 1], b, c + 1);
        y.z = gate_res_f(r.z, v.z, g[c + 2], b, c + 2);
        y.w = gate_res_f(r.w, v.w, g[c + 3], b, c + 3);
        out[i] = y;
    }
}
__global__ __launch_bounds__(256) void k_gate_res1(float *out, const float *res, const float *o,
                                                   const float *gate, const float *b, int dim,
                                                   size_t per_batch, size_t n) {
    GRID_STRIDE(i, n) {
        size_t bt = i / per_batch;
        int c = (int)(i % (size_t)dim);
        out[i] = gate_res_f(res[i], o[i], gate[bt * dim + c], b, c);
    }
}
extern "C" hipError_t aria_k_gate_residual(float *out, const float *res, const float *o,
                                           const float *gate, const float *bias, int rows, int dim,
                                           int rows_per_batch, hipStream_t s) {
    size_t n = (size_t)rows * dim;
    if (n == 0) return hipSuccess;
    if (rows_per_batch <= 0) rows_per_batch = rows;
    size_t per = (size_t)rows_per_batch * dim;
    if (dim % 4 == 0 && al16(out) && al16(res) && al16(o))
        hipLaunchKernelGGL(k_gate_res4, stream_grid(n / 4), dim3(256), 0, s, (float4 *)out,
                           (const float4 *)res, (const float4 *)o, gate, bias, dim / 4, per / 4, n / 4);
    else
        hipLaunchKernelGGL(k_gate_res1, stream_grid((n + 3) / 4), dim3(256), 0, s, out, res, o, gate,
                           bias, dim, per, n);
    return hipGetLastError();
}

/* GLU combine: out[r,i] = silu(g) * u with u = proj[r,i] (+b[i]),
 * g = proj[r,inner+i] (+b[inner+i]) (src/aria_sa3_dit.c:108-121, src/aria_cuda.cu:712-731) */
__global__ __launch_bounds__(256) void k_glu(void *out, int f16, const float *proj, const float *b,
                                             int inner, size_t n) {
    GRID_STRIDE(i, n) {
        size_t r = i / (size_t)inner;
        int c = (int)(i % (size_t)inner);
        const float *pr = proj + r * 2 * (size_t)inner;
        float u = pr[c], g = pr[inner + c];
        if (b) { u = u + b[c]; g = g + b[inner + c]; }
        float v = silu_f(g) * u;
        if (f16) ((uint16_t *)out)[i] = f2h_bits(v);
        else ((float *)out)[i] = v;
    }
}
extern "C" hipError_t aria_k_glu_combine(void *out, int out_f16, const float *proj, const float *bias,
                                         int rows, int inner, hipStream_t s) {
    size_t n = (size_t)rows * inner;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_glu, stream_grid((n + 3) / 4), dim3(256), 0, s, out, out_f16, proj, bias,
                       inner, n);
    return hipGetLastError();
}

/* DynamicTanh, src/aria_cpu.c:684-701: y = tanh(alpha*x)*w + b (w, b optional) */
__global__ __launch_bounds__(256) void k_dyt(float *y, const float *x, float alpha, const float *w,
                                             const float *b, int dim, size_t n) {
    GRID_STRIDE(i, n) {
        int c = (int)(i % (size_t)dim);
        float t = tanhf(alpha * x[i]);
        float p = t * (w ? w[c] : 1.0f);
        y[i] = p + (b ? b[c] : 0.0f);
    }
}
extern "C" hipError_t aria_k_dynamic_tanh(float *y, const float *x, float alpha, const float *w,
                                          const float *b, int rows, int dim, hipStream_t s) {
    size_t n = (size_t)rows * dim;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dyt, stream_grid((n + 3) / 4), dim3(256), 0, s, y, x, alpha, w, b, dim, n);
    return hipGetLastError();
}

/* pingpong, src/aria_sampler.c:216-220 and the reference device twin: each
 * operation rounded on its own (no FMA) so the device loop matches the host loop. */
__device__ __forceinline__ float pingpong_f(float x, float v, float z, float tc, float tn) {
    float d = __fsub_rn(x, __fmul_rn(tc, v));
    return __fadd_rn(__fmul_rn(__fsub_rn(1.0f, tn), d), __fmul_rn(tn, z));
}
__global__ __launch_bounds__(256) void k_pingpong4(float4 *x, const float4 *v, const float4 *z, float tc,
                                                   float tn, size_t n4) {
    GRID_STRIDE(i, n4) {
        float4 a = x[i], b = v[i], c = z[i];
        a.x = pingpong_f(a.x, b.x, c.x, tc, tn); a.y = pingpong_f(a.y, b.y, c.y, tc, tn);
        a.z = pingpong_f(a.z, b.z, c.z, tc, tn); a.w = pingpong_f(a.w, b.w, c.w, tc, tn);
        x[i] = a;
    }
}
__global__ __launch_bounds__(256) void k_pingpong1(float *x, const float *v, const float *z, float tc,
                                                   float tn, size_t n) {
    GRID_STRIDE(i, n) x[i] = pingpong_f(x[i], v[i], z[i], tc, tn);
}
extern "C" hipError_t aria_k_pingpong(float *x, const float *v, const float *noise, float tc,
                                      float tn, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && al16(x) && al16(v) && al16(noise))
        hipLaunchKernelGGL(k_pingpong4, stream_grid(n / 4), dim3(256), 0, s, (float4 *)x,
                           (const float4 *)v, (const float4 *)noise, tc, tn, n / 4);
    else
        hipLaunchKernelGGL(k_pingpong1, stream_grid((n + 3) / 4), dim3(256), 0, s, x, v, noise, tc, tn,
                           n);
    return hipGetLastError();
}

/* batched 2-D transpose through a 32x33 LDS tile: dst[b][c][r] = src[b][r][c]
 * (the DiT step's [C,T] <-> [T,C] latent reshapes, src/aria_sa3_dit.c:585-597) */
__global__ __launch_bounds__(256) void k_transpose(float *dst, const float *src, int rows, int cols) {
    __shared__ float t[32][33];
    const size_t base = (size_t)blockIdx.z * rows * cols;
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   /* 32 x 8 threads */
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) t[i][tx] = src[base + (size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) dst[base + (size_t)c * rows + r] = t[tx][i];
    }
}
extern "C" hipError_t aria_k_transpose(float *dst, const float *src, int rows, int cols, int batch, hipStream_t s) {
    if (rows <= 0 || cols <= 0 || batch <= 0) return hipSuccess;
    dim3 grid((cols + 31) / 32, (rows + 31) / 32, batch);
    hipLaunchKernelGGL(k_transpose, grid, dim3(256), 0, s, dst, src, rows, cols);
    return hipGetLastError();
}

/* DiT modulation (src/aria_sa3_dit.c:152-156): mod = to_scale_shift_gate + gcond[b],
 * written chunk-major mod[c][b][i] (c < 6) so each of the six [B, dim] slices
 * (scale_self, shift_self, gate_self, scale_ff, shift_ff, gate_ff) is contiguous. */
__global__ __launch_bounds__(256) void k_mod_chunks(float *mod, const float *tssg, const float *gcond, int B,
                                                    int dim, size_t n) {
    GRID_STRIDE(idx, n) {
        const int i = (int)(idx % (size_t)dim);
        const int b = (int)((idx / dim) % (size_t)B);
        const int c = (int)(idx / ((size_t)dim * B));
        const float t = tssg[(size_t)c * dim + i];
        mod[idx] = gcond ? t + gcond[(size_t)b * 6 * dim + (size_t)c * dim + i] : t;
    }
}
extern "C" hipError_t aria_k_mod_chunks(float *mod, const float *tssg, const float *gcond, int B, int dim,
                                        hipStream_t s) {
    const size_t n = (size_t)6 * B * dim;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_mod_chunks, stream_grid((n + 3) / 4), dim3(256), 0, s, mod, tssg, gcond, B, dim, n);
    return hipGetLastError();
}

/* fp32 -> fp16 RTNE (the reference's k_f32_to_f16 / aria_f32_to_f16_n): the GEMMs' staging of
 * fp32 activations, and weight and K/V conversions at set-up. Streamed: wave g converts float4
 * [256 g, 256 g + 256), lane l the four at 256 g + l + 64 j, all four loads issued before any
 * store (the index is clamped instead of guarded: a guarded load compiles to a branch that
 * waits for each load before the next). The fp32 source is read once (non-temporal loads); the
 * fp16 copy is stored normally, so it stays in the caches for the GEMM that reads it next
 * (non-temporal stores made the K = 4096 staging + GEMM 3 us slower). */
__global__ __launch_bounds__(256) void k_f2h4(uint2 *y, const float4 *x, size_t n4) {
    const size_t base = ((size_t)blockIdx.x * 256 + (threadIdx.x & ~63u)) * 4 + (threadIdx.x & 63);
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = ld_nt(x + min(base + 64 * j, n4 - 1));
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const size_t i = base + 64 * j;
        if (i < n4)
            y[i] = make_uint2((uint32_t)f2h_bits(v[j].x) | ((uint32_t)f2h_bits(v[j].y) << 16),
                              (uint32_t)f2h_bits(v[j].z) | ((uint32_t)f2h_bits(v[j].w) << 16));
    }
}
__global__ __launch_bounds__(256) void k_f2h(uint16_t *y, const float *x, size_t n) {
    GRID_STRIDE(i, n) y[i] = f2h_bits(x[i]);
}
extern "C" hipError_t aria_k_f32_to_f16(uint16_t *y, const float *x, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && al16(x) && ((uintptr_t)y & 7u) == 0)
        hipLaunchKernelGGL(k_f2h4, dim3((unsigned)((n / 4 + 1023) / 1024)), dim3(256), 0, s, (uint2 *)y,
                           (const float4 *)x, n / 4);
    else
        hipLaunchKernelGGL(k_f2h, stream_grid((n + 3) / 4), dim3(256), 0, s, y, x, n);
    return hipGetLastError();
}
