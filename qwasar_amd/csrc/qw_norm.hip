// qw_norm.hip -- RMS normalisation: the reference's qw_op_rms_norm, and the
// residual step that joins the layers of a MoE stack,
//
//     h <- bf16(h + y);   x = rms_norm(h)
//
// (activations carried in bf16 between layers, normalised in fp32).
//
// One workgroup per row.  The sum of squares: each thread an fmaf chain over
// its columns (column c goes to thread (c / 4) % 256, four at a time), the
// threads of a wave by the xor tree, then the four waves' partials in wave
// order.  inv = 1 / sqrt(ss / dim + eps) * out_scale, the form of
// qwasar_cpu.c:68-82 (metal/norm.metal:47-72 takes rsqrt of the same).
#include "qw_device.h"
#include "qw_kernels.h"

#define QN_THREADS 256

__device__ __forceinline__ float qn_block_sum(float v, float *part)
{
    v = qw_xor_sum<64>(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wave] = v;
    __syncthreads();
    float s = part[0];
#pragma unroll
    for (int i = 1; i < QN_THREADS / 64; i++) s = s + part[i];
    return s;
}

__device__ __forceinline__ uint16_t qn_bf16(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// y = x * inv (* w) (* sigmoid(gate), the delta net's output gate):
// dim % 4 == 0, rows are float4-aligned
__global__ void __launch_bounds__(QN_THREADS) k_rms_norm(float *__restrict__ y, const float *__restrict__ x,
                                                         const uint16_t *__restrict__ w, int dim, float eps,
                                                         float out_scale, const float *__restrict__ gate)
{
    __shared__ float part[QN_THREADS / 64];
    const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)blockIdx.x * dim);
    float4 *yr = reinterpret_cast<float4 *>(y + (size_t)blockIdx.x * dim);
    const int n4 = dim / 4;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n4; i += QN_THREADS) {
        const float4 v = xr[i];
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
    }
    ss = qn_block_sum(ss, part);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps) * out_scale;
    for (int i = threadIdx.x; i < n4; i += QN_THREADS) {
        float4 v = xr[i];
        v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
        if (w) {
            const uint2 wb = reinterpret_cast<const uint2 *>(w)[i];
            v.x *= __uint_as_float(wb.x << 16);
            v.y *= __uint_as_float(wb.x & 0xFFFF0000u);
            v.z *= __uint_as_float(wb.y << 16);
            v.w *= __uint_as_float(wb.y & 0xFFFF0000u);
        }
        if (gate) {
            const float4 g = reinterpret_cast<const float4 *>(gate + (size_t)blockIdx.x * dim)[i];
            v.x *= 1.0f / (1.0f + expf(-g.x));
            v.y *= 1.0f / (1.0f + expf(-g.y));
            v.z *= 1.0f / (1.0f + expf(-g.z));
            v.w *= 1.0f / (1.0f + expf(-g.w));
        }
        yr[i] = v;
    }
}

// h_out (bf16 [rows, dim]) = bf16(h + y) when y is given, else h (h_out may
// be h); x = rms_norm(h_out)
__global__ void __launch_bounds__(QN_THREADS) k_resid_rms_bf16(const uint16_t *h, uint16_t *h_out,
                                                               float *__restrict__ x,
                                                               const float *__restrict__ y, int dim, float eps)
{
    __shared__ float part[QN_THREADS / 64];
    const uint2 *hr = reinterpret_cast<const uint2 *>(h + (size_t)blockIdx.x * dim);
    uint2 *ho = reinterpret_cast<uint2 *>(h_out + (size_t)blockIdx.x * dim);
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)blockIdx.x * dim);
    const float4 *yr = y ? reinterpret_cast<const float4 *>(y + (size_t)blockIdx.x * dim) : nullptr;
    const int n4 = dim / 4;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n4; i += QN_THREADS) {
        uint2 hb = hr[i];
        float v[4] = {__uint_as_float(hb.x << 16), __uint_as_float(hb.x & 0xFFFF0000u),
                      __uint_as_float(hb.y << 16), __uint_as_float(hb.y & 0xFFFF0000u)};
        if (yr) {
            const float4 a = yr[i];
            const float s[4] = {v[0] + a.x, v[1] + a.y, v[2] + a.z, v[3] + a.w};
            uint16_t b[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                b[q] = qn_bf16(s[q]);
                v[q] = __uint_as_float((uint32_t)b[q] << 16);
            }
            hb = make_uint2((uint32_t)b[0] | ((uint32_t)b[1] << 16), (uint32_t)b[2] | ((uint32_t)b[3] << 16));
        }
        if (yr || ho != hr) ho[i] = hb;
#pragma unroll
        for (int q = 0; q < 4; q++) ss = __builtin_fmaf(v[q], v[q], ss);
    }
    ss = qn_block_sum(ss, part);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = threadIdx.x; i < n4; i += QN_THREADS) {
        const uint2 hb = ho[i];   // this thread's own values, written above
        xr[i] = make_float4(__uint_as_float(hb.x << 16) * inv, __uint_as_float(hb.x & 0xFFFF0000u) * inv,
                            __uint_as_float(hb.y << 16) * inv, __uint_as_float(hb.y & 0xFFFF0000u) * inv);
    }
}

extern "C" int qwk_rms_norm(hipStream_t s, float *y, const float *x, const uint16_t *w, int dim, int rows,
                            float eps, float out_scale)
{
    if (rows <= 0) return 0;
    if (dim <= 0 || dim % 4 || ((uintptr_t)x & 15u) || ((uintptr_t)y & 15u) || ((uintptr_t)w & 7u))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(QN_THREADS), 0, s, y, x, w, dim, eps, out_scale, nullptr);
    return (int)hipGetLastError();
}

extern "C" int qwk_rms_norm_gated_sigmoid(hipStream_t s, float *y, const float *x, const uint16_t *w,
                                          const float *gate, int dim, int rows, float eps, float out_scale)
{
    if (rows <= 0) return 0;
    if (!gate || dim <= 0 || dim % 4 || ((uintptr_t)x & 15u) || ((uintptr_t)y & 15u) || ((uintptr_t)w & 7u) ||
        ((uintptr_t)gate & 15u))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(QN_THREADS), 0, s, y, x, w, dim, eps, out_scale, gate);
    return (int)hipGetLastError();
}

extern "C" int qwk_resid_rms_bf16(hipStream_t s, const uint16_t *h, uint16_t *h_out, float *x, const float *y,
                                  int dim, int rows, float eps)
{
    if (rows <= 0) return 0;
    if (dim <= 0 || dim % 4 || ((uintptr_t)h & 7u) || ((uintptr_t)h_out & 7u) || ((uintptr_t)x & 15u) ||
        ((uintptr_t)y & 15u))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_resid_rms_bf16, dim3(rows), dim3(QN_THREADS), 0, s, h, h_out, x, y, dim, eps);
    return (int)hipGetLastError();
}
