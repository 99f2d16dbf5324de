// qw_elem.hip -- the MoE block's elementwise steps: SwiGLU (split halves and
// interleaved per pair), the weighted combine with and without the gated
// shared expert, the shared expert's row scale, and an in-place add.
#include "qw_device.h"
#include "qw_kernels.h"

#define QW_EW_THREADS 256

static dim3 ew_grid(int64_t n) { return dim3((unsigned)((n + QW_EW_THREADS - 1) / QW_EW_THREADS)); }

__global__ void k_swiglu(float *__restrict__ y, const float *__restrict__ g,
                         const float *__restrict__ u, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * QW_EW_THREADS + threadIdx.x;
    if (i < n) y[i] = qw_silu(g[i]) * u[i];
}

// act[p, i] = silu(gu[p, i]) * gu[p, I + i]
__global__ void k_swiglu_split(float *__restrict__ act, const float *__restrict__ gu, int pairs, int I)
{
    const int64_t t = (int64_t)blockIdx.x * QW_EW_THREADS + threadIdx.x;
    if (t >= (int64_t)pairs * I) return;
    const int64_t p = t / I, i = t % I;
    act[t] = qw_silu(gu[p * 2 * I + i]) * gu[p * 2 * I + I + i];
}

// out[r, i] = [sh[r, i] * sigmoid(g[r])] + sum_k w[r, k] * y[r*K + k, i], an fma
// chain in slot order starting from the shared term (or from 0 without one).
// out[r, i] = sigmoid(g[r]) * sh[r, i] (if sh) + sum_k w[r, k] * y[r K + k, i],
// the shared term first, then one fma a slot in slot order.  Row r is
// blockIdx.y; a thread takes 4 consecutive columns (H % 4 == 0: float4), or
// one column in the scalar form.
template <bool V4>
__global__ void k_moe_combine(float *__restrict__ out, const float *__restrict__ y,
                              const float *__restrict__ w, const float *__restrict__ sh,
                              const float *__restrict__ g, int rows, int K, int H)
{
    const int r = blockIdx.y;
    const int i = (blockIdx.x * QW_EW_THREADS + threadIdx.x) * (V4 ? 4 : 1);
    if (i >= H) return;
    const size_t row = (size_t)r * H;
    if (V4) {
        // every load in flight together: the shared row's, then every
        // slot's, unconditional (a slot past the last reads the last
        // again), since a guarded load becomes a branch that waits for the
        // loads before it; the shared term is used only after
        const float4 shv = sh ? *reinterpret_cast<const float4 *>(sh + row + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        // the gate logit and the slots' weights (uniform: scalar loads) with
        // the rows, not one wait each inside the sum
        const float gl = sh ? g[r] : 0.0f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 yv[16];
        float wv[16];
        for (int k0 = 0; k0 < K; k0 += 16) {
            const int kn = min(16, K - k0);
#pragma unroll
            for (int k = 0; k < 16; k++) wv[k] = w[(size_t)r * K + k0 + min(k, kn - 1)];
#pragma unroll
            for (int k = 0; k < 16; k++)
                yv[k] = *reinterpret_cast<const float4 *>(y + ((size_t)r * K + k0 + min(k, kn - 1)) * H + i);
#pragma unroll
            for (int k = 0; k < 16; k++) asm volatile("" ::"s"(wv[k]));   // (requested with the rows, not in the sum)
            if (k0 == 0 && sh) {
                const float gs = qw_sigmoid(gl);
                acc = make_float4(shv.x * gs, shv.y * gs, shv.z * gs, shv.w * gs);
            }
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (k < kn) {
                    const float wk = wv[k];
                    acc.x = __builtin_fmaf(wk, yv[k].x, acc.x);
                    acc.y = __builtin_fmaf(wk, yv[k].y, acc.y);
                    acc.z = __builtin_fmaf(wk, yv[k].z, acc.z);
                    acc.w = __builtin_fmaf(wk, yv[k].w, acc.w);
                }
        }
        *reinterpret_cast<float4 *>(out + row + i) = acc;
    } else {
        float acc = sh ? sh[row + i] * qw_sigmoid(g[r]) : 0.0f;
        for (int k = 0; k < K; k++) acc = __builtin_fmaf(w[(size_t)r * K + k], y[((size_t)r * K + k) * H + i], acc);
        out[row + i] = acc;
    }
}

__global__ void k_scale_rows_sigmoid(float *__restrict__ y, const float *__restrict__ g, int rows, int dim)
{
    const int64_t t = (int64_t)blockIdx.x * QW_EW_THREADS + threadIdx.x;
    if (t < (int64_t)rows * dim) y[t] *= qw_sigmoid(g[t / dim]);
}

__global__ void k_add_inplace(float *__restrict__ y, const float *__restrict__ x, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * QW_EW_THREADS + threadIdx.x;
    if (i < n) y[i] += x[i];
}

extern "C" int qwk_swiglu(hipStream_t s, float *y, const float *gate, const float *up, int64_t n)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_swiglu, ew_grid(n), dim3(QW_EW_THREADS), 0, s, y, gate, up, n);
    return (int)hipGetLastError();
}

extern "C" int qwk_swiglu_split(hipStream_t s, float *act, const float *gu, int pairs, int I)
{
    if ((int64_t)pairs * I <= 0) return 0;
    hipLaunchKernelGGL(k_swiglu_split, ew_grid((int64_t)pairs * I), dim3(QW_EW_THREADS), 0, s, act, gu, pairs, I);
    return (int)hipGetLastError();
}

extern "C" int qwk_moe_combine(hipStream_t s, float *out, const float *y, const float *w,
                               const float *sh, const float *g, int rows, int K, int H)
{
    if ((int64_t)rows * H <= 0) return 0;
    const bool v4 = H % 4 == 0 && ((uintptr_t)out & 15u) == 0 && ((uintptr_t)y & 15u) == 0 &&
                    (!sh || ((uintptr_t)sh & 15u) == 0);
    const int per = v4 ? 4 * QW_EW_THREADS : QW_EW_THREADS;
    const dim3 grid((unsigned)((H + per - 1) / per), (unsigned)rows);
    if (v4) hipLaunchKernelGGL(k_moe_combine<true>, grid, dim3(QW_EW_THREADS), 0, s, out, y, w, sh, g, rows, K, H);
    else hipLaunchKernelGGL(k_moe_combine<false>, grid, dim3(QW_EW_THREADS), 0, s, out, y, w, sh, g, rows, K, H);
    return (int)hipGetLastError();
}

extern "C" int qwk_scale_rows_sigmoid(hipStream_t s, float *y, const float *g, int rows, int dim)
{
    if ((int64_t)rows * dim <= 0) return 0;
    hipLaunchKernelGGL(k_scale_rows_sigmoid, ew_grid((int64_t)rows * dim), dim3(QW_EW_THREADS), 0, s,
                       y, g, rows, dim);
    return (int)hipGetLastError();
}

extern "C" int qwk_add_inplace(hipStream_t s, float *y, const float *x, int64_t n)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_add_inplace, ew_grid(n), dim3(QW_EW_THREADS), 0, s, y, x, n);
    return (int)hipGetLastError();
}
