// qw_hc.hip -- the hyper-connection mixer that wraps every Flash-Next block
// (the step on either side of the MoE layer; reference semantics
// metal/sparse.metal:14-189, qwasar_flash_cpu.c:57-70 and 263-293):
//
//   n4  = grouped_rms_norm(h4) * w            (S streams of H, each its own norm)
//   x   = mean_s sigmoid(up(silu(down(n4) / S)))_s * n4_s
//   inj = block_inject(n4)                    (raw logits, [S])
//   h4 += out (x) 2 sigmoid(inj / S)          (a block's output into the streams)
//
// Memory-bound elementwise and row kernels, and two fused kernels for a
// decode step: k_hc_pre (inject, grouped norm, down-projection and injection
// logits in one launch) and k_hc_mix_up (up-projection, its silu and the
// stream mix at few rows).  The row sums run in the order of qw_norm.hip:
// each of 256 threads an fmaf chain over its float4 chunks, the xor tree, the
// four wave partials in order.
#include "qw_device.h"
#include "qw_kernels.h"

#define QH_THREADS 256
#define QH_PRE_MAXS 4             // streams a fused decode kernel takes


__device__ __forceinline__ float qh_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

__device__ __forceinline__ float qh_block_sum(float v, float *part)
{
    v = qw_xor_sum<64>(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wave] = v;
    __syncthreads();
    float s = part[0];
#pragma unroll
    for (int i = 1; i < QH_THREADS / 64; i++) s = s + part[i];
    return s;
}

// h4[r, s*H + i] = x[r, i]
__global__ void k_repeat_cols(float4 *__restrict__ h4, const float4 *__restrict__ x, int rows, int H4, int S)
{
    const int64_t n = (int64_t)rows * S * H4;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = j / ((int64_t)S * H4);
        h4[j] = x[r * H4 + j % H4];
    }
}

// One workgroup per (row, group): y = x * inv * w[g], dim % 4 == 0.  With
// `out` and `inj` set, x first takes the block's output (x += out * 2
// sigmoid(inj / S)) and is written back: qw_hc_inject and the norm in one pass.
// NI > 0: each thread's NI float4s held in registers between the passes
// (dim <= NI * 1024), so the second pass reads nothing again; NI == 0 loops.
template <int NI>
__global__ void __launch_bounds__(QH_THREADS) k_norm_grouped(float *__restrict__ y, float *x,
                                                             const uint16_t *__restrict__ w, int dim, int groups,
                                                             float eps, const float *__restrict__ out,
                                                             const float *__restrict__ inj)
{
    __shared__ float part[QH_THREADS / 64];
    const int q = blockIdx.x, g = q % groups, r = q / groups;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)q * dim);
    float4 *yr = reinterpret_cast<float4 *>(y + (size_t)q * dim);
    const uint2 *wr = reinterpret_cast<const uint2 *>(w + (size_t)g * dim);
    const int n4 = dim / 4, t = threadIdx.x;
    float wgt = 0.0f;
    const float4 *orow = nullptr;
    if (out) {
        wgt = 2.0f * qh_sigmoid(inj[(size_t)r * groups + g] / (float)groups);
        orow = reinterpret_cast<const float4 *>(out + (size_t)r * dim);
    }
    auto take = [&](int i, float4 v, float &ss) -> float4 {
        if (out) {
            const float4 o = orow[i];
            v.x += o.x * wgt; v.y += o.y * wgt; v.z += o.z * wgt; v.w += o.w * wgt;
            xr[i] = v;
        }
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
        return v;
    };
    auto put = [&](int i, float4 v, float inv) {
        const uint2 wb = wr[i];
        v.x = v.x * inv * __uint_as_float(wb.x << 16);
        v.y = v.y * inv * __uint_as_float(wb.x & 0xFFFF0000u);
        v.z = v.z * inv * __uint_as_float(wb.y << 16);
        v.w = v.w * inv * __uint_as_float(wb.y & 0xFFFF0000u);
        yr[i] = v;
    };
    float ss = 0.0f;
    if (NI > 0) {
        constexpr int NR = NI > 0 ? NI : 1;
        float4 hv[NR];
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
            hv[j] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
            if (i < n4) hv[j] = take(i, hv[j], ss);
        }
        ss = qh_block_sum(ss, part);
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
            if (i < n4) put(i, hv[j], inv);
        }
    } else {
        for (int i = t; i < n4; i += QH_THREADS) take(i, xr[i], ss);
        ss = qh_block_sum(ss, part);
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
        for (int i = t; i < n4; i += QH_THREADS) put(i, xr[i], inv);   // this thread's own values
    }
}

static void qh_norm_launch(hipStream_t s, int blocks, float *y, float *x, const uint16_t *w, int dim, int groups,
                           float eps, const float *out, const float *inj)
{
    const int ni = (dim / 4 + QH_THREADS - 1) / QH_THREADS;
    const dim3 g((unsigned)blocks), b(QH_THREADS);
    switch (ni) {
    case 1: hipLaunchKernelGGL(k_norm_grouped<1>, g, b, 0, s, y, x, w, dim, groups, eps, out, inj); break;
    case 2: hipLaunchKernelGGL(k_norm_grouped<2>, g, b, 0, s, y, x, w, dim, groups, eps, out, inj); break;
    case 3: hipLaunchKernelGGL(k_norm_grouped<3>, g, b, 0, s, y, x, w, dim, groups, eps, out, inj); break;
    case 4: hipLaunchKernelGGL(k_norm_grouped<4>, g, b, 0, s, y, x, w, dim, groups, eps, out, inj); break;
    default: hipLaunchKernelGGL(k_norm_grouped<0>, g, b, 0, s, y, x, w, dim, groups, eps, out, inj); break;
    }
}

// y = silu(y * scale)
__global__ void k_silu_scale(float *__restrict__ y, int64_t n, float scale)
{
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
        const float v = y[j] * scale;
        y[j] = v * qh_sigmoid(v);
    }
}

// x[r, i] = (sum_s sigmoid(m) n, in stream order) / S
__global__ void k_hc_mix(float *__restrict__ x, const float *__restrict__ n, const float *__restrict__ m, int rows,
                         int H, int S)
{
    const int64_t total = (int64_t)rows * H;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < total; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = j / H, i = j % H;
        float acc = 0.0f;
        for (int s = 0; s < S; s++) {
            const int64_t q = r * S * H + (int64_t)s * H + i;
            acc = acc + qh_sigmoid(m[q]) * n[q];
        }
        x[j] = acc / (float)S;
    }
}

// h4[r, s*H+i] += out[r, i] * 2 sigmoid(inj[r, s] / S)
__global__ void k_hc_inject(float *__restrict__ h4, const float *__restrict__ out, const float *__restrict__ inj,
                            int rows, int H, int S)
{
    const int64_t total = (int64_t)rows * S * H;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < total; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = j / ((int64_t)S * H), s = (j / H) % S, i = j % H;
        h4[j] += out[r * H + i] * (2.0f * qh_sigmoid(inj[r * S + s] / (float)S));
    }
}

// The mixer's up-projection, its input silu and the stream mix, for few rows:
// a wave per output i holds the S up-projection rows s*H + i that feed it
// (lane: 8-input words wi = lane, lane + 64, ...), each row's dot an fmaf
// chain over the lane's words then the xor tree; lane 0 mixes the streams in
// order.  S <= 4.
__global__ void __launch_bounds__(QH_THREADS) k_hc_mix_up(float *__restrict__ x, const float *__restrict__ d,
                                                          const float *__restrict__ n4,
                                                          const uint32_t *__restrict__ w,
                                                          const uint16_t *__restrict__ sc,
                                                          const uint16_t *__restrict__ bi, int k, int H, int S,
                                                          int rows, float scale, int lgG)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * (QH_THREADS / 64) + (threadIdx.x >> 6);
    if (i >= H) return;   // whole waves
    const int words = k / 8, groups = k >> lgG;
    for (int r = 0; r < rows; r++) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, nv[4];
        // the streams' values this output mixes, requested with the weights
#pragma unroll
        for (int s = 0; s < 4; s++) nv[s] = s < S ? n4[(size_t)r * S * H + (size_t)s * H + i] : 0.0f;
        for (int wi = lane; wi < words; wi += 64) {
            float xs[8];
            const float4 *dv = reinterpret_cast<const float4 *>(d + (size_t)r * k + 8 * wi);
            const float4 d0 = dv[0], d1 = dv[1];
            const float dd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float v = dd[j] * scale;
                xs[j] = v * qh_sigmoid(v);
            }
            const int gi = (8 * wi) >> lgG;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                if (s >= S) break;
                const size_t row = (size_t)s * H + i;
                const uint32_t q = w[row * words + wi];
                const float sv = __uint_as_float((uint32_t)sc[row * groups + gi] << 16);
                const float bv = __uint_as_float((uint32_t)bi[row * groups + gi] << 16);
#pragma unroll
                for (int j = 0; j < 8; j++)
                    acc[s] = __builtin_fmaf(__builtin_fmaf(sv, (float)((q >> (4 * j)) & 0xFu), bv), xs[j], acc[s]);
            }
        }
        float mix = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const float m = qw_xor_sum<64>(acc[s]);
            if (s < S) mix = mix + qh_sigmoid(m) * nv[s];
        }
        if (lane == 0) x[(size_t)r * H + i] = mix / (float)S;
    }
}

static dim3 qh_grid(int64_t n)
{
    const int64_t b = (n + QH_THREADS - 1) / QH_THREADS;
    return dim3((unsigned)(b < 16384 ? (b > 0 ? b : 1) : 16384));
}

// The LDS slot of float4 p of the normed streams when the injection logits
// read them (SW16): within each run of 16 (a 64-input chunk) rotated by the
// run's index, so the lanes reading the same float4 of consecutive chunks hit
// different banks.
__device__ __forceinline__ int qh_swz16(int p) { return (p & ~15) | ((p + (p >> 4)) & 15); }

// Inject and grouped norm of one row into LDS (nl: S*H floats): the streams
// with the block's output injected, then each normed with its gains -- per
// stream the order of k_norm_grouped (a chain over this thread's float4s
// ascending, the xor tree, the wave partials in order).  Stream `ws` (< 0:
// none) is also written to h4_out and n4.  inv gets the streams' 1/rms.
// after_loads() runs once this function's loads are issued, so loads it
// issues come after them in the memory counter's order (the norm does not
// wait for them).  Every thread of the workgroup calls it (it holds
// barriers).
template <int NI, bool SW16 = false, typename F>
__device__ __forceinline__ void qh_inject_norm(float4 *nl, float (*part)[QH_THREADS / 64], int ws,
                                               float *__restrict__ h4_out, float *__restrict__ n4,
                                               const float *__restrict__ h4, const float *__restrict__ out,
                                               const float *__restrict__ inj, const uint16_t *__restrict__ wn,
                                               int H, int S, float eps, float (&inv)[QH_PRE_MAXS], F &&after_loads)
{
    const int t = threadIdx.x, n4q = H / 4;
    const int wave = t >> 6, lane = t & 63;
    const float4 *orow = reinterpret_cast<const float4 *>(out);
    float injv[QH_PRE_MAXS], wgt[QH_PRE_MAXS], ss[QH_PRE_MAXS];
#pragma unroll
    for (int s = 0; s < QH_PRE_MAXS; s++) {
        injv[s] = s < S ? inj[s] : 0.0f;
        ss[s] = 0.0f;
    }
    constexpr int NR = NI > 0 ? NI : 1;
    float4 hv[QH_PRE_MAXS][NR], ov[NR];
    uint2 gw[QH_PRE_MAXS][NR];
    if (NI > 0) {
        // every value this thread needs, requested at once
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
            const bool ok = i < n4q;
            ov[j] = ok ? orow[i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int s = 0; s < QH_PRE_MAXS; s++) {
                const bool in = ok && s < S;
                hv[s][j] = in ? reinterpret_cast<const float4 *>(h4 + (size_t)s * H)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                gw[s][j] = in ? reinterpret_cast<const uint2 *>(wn + (size_t)s * H)[i] : make_uint2(0, 0);
            }
        }
    }
    after_loads();
#pragma unroll
    for (int s = 0; s < QH_PRE_MAXS; s++) wgt[s] = s < S ? 2.0f * qh_sigmoid(injv[s] / (float)S) : 0.0f;
    // inject and the sums of squares of all streams together
    auto inject = [&](int s, int i, float4 &v, float4 o) {
        v.x += o.x * wgt[s]; v.y += o.y * wgt[s]; v.z += o.z * wgt[s]; v.w += o.w * wgt[s];
        if (ws == s) reinterpret_cast<float4 *>(h4_out + (size_t)s * H)[i] = v;
        ss[s] = __builtin_fmaf(v.x, v.x, ss[s]);
        ss[s] = __builtin_fmaf(v.y, v.y, ss[s]);
        ss[s] = __builtin_fmaf(v.z, v.z, ss[s]);
        ss[s] = __builtin_fmaf(v.w, v.w, ss[s]);
    };
    auto scale = [&](int s, int i, float4 v, uint2 wb) {
        v.x = v.x * inv[s] * __uint_as_float(wb.x << 16);
        v.y = v.y * inv[s] * __uint_as_float(wb.x & 0xFFFF0000u);
        v.z = v.z * inv[s] * __uint_as_float(wb.y << 16);
        v.w = v.w * inv[s] * __uint_as_float(wb.y & 0xFFFF0000u);
        nl[SW16 ? qh_swz16(s * n4q + i) : s * n4q + i] = v;
        if (ws == s) reinterpret_cast<float4 *>(n4 + (size_t)s * H)[i] = v;
    };
    if (NI > 0) {
        // the injected values stay in registers until they are scaled
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
#pragma unroll
            for (int s = 0; s < QH_PRE_MAXS; s++)
                if (s < S && i < n4q) inject(s, i, hv[s][j], ov[j]);
        }
    } else {
        for (int i = t; i < n4q; i += QH_THREADS) {
            const float4 o = orow[i];
#pragma unroll
            for (int s = 0; s < QH_PRE_MAXS; s++)
                if (s < S) {
                    float4 v = reinterpret_cast<const float4 *>(h4 + (size_t)s * H)[i];
                    inject(s, i, v, o);
                    nl[SW16 ? qh_swz16(s * n4q + i) : s * n4q + i] = v;
                }
        }
    }
#pragma unroll
    for (int s = 0; s < QH_PRE_MAXS; s++) {
        const float v = qw_xor_sum<64>(ss[s]);
        if (lane == 0) part[s][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < QH_PRE_MAXS; s++) {
        float tot = part[s][0];
#pragma unroll
        for (int w = 1; w < QH_THREADS / 64; w++) tot = tot + part[s][w];
        inv[s] = 1.0f / sqrtf(tot / (float)H + eps);
    }
    if (NI > 0) {
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
#pragma unroll
            for (int s = 0; s < QH_PRE_MAXS; s++)
                if (s < S && i < n4q) scale(s, i, hv[s][j], gw[s][j]);
        }
    } else {
        for (int i = t; i < n4q; i += QH_THREADS) {
#pragma unroll
            for (int s = 0; s < QH_PRE_MAXS; s++)
                if (s < S) scale(s, i, nl[SW16 ? qh_swz16(s * n4q + i) : s * n4q + i], reinterpret_cast<const uint2 *>(wn + (size_t)s * H)[i]);
        }
    }
    __syncthreads();
}

// The LDS slot of float4 i of a stream normed by qh_norm1: within each run of 8
// (a 32-input segment) rotated by the run's index, so 8 lanes reading the same
// float4 of 8 consecutive segments hit different banks.
__device__ __forceinline__ int qh_swz(int i) { return (i & ~7) | ((i + (i >> 3)) & 7); }

// Stream s alone of qh_inject_norm: the same arithmetic for that stream (its
// injected values, sum of squares, 1/rms and normed values bit for bit),
// normed into nl (float4 i at qh_swz(i), i < H / 4), nothing written to
// memory; returns the 1/rms.
// after_loads() runs once the stream's loads are issued.  Every thread of
// the workgroup calls it (it holds barriers).
template <int NI, typename F>
__device__ __forceinline__ float qh_norm1(float4 *nl, float (*part)[QH_THREADS / 64], int s,
                                          const float *__restrict__ h4, const float *__restrict__ out,
                                          const float *__restrict__ inj, const uint16_t *__restrict__ wn, int H,
                                          int S, float eps, F &&after_loads)
{
    const int t = threadIdx.x, n4q = H / 4;
    const int wave = t >> 6, lane = t & 63;
    const float4 *hrow = reinterpret_cast<const float4 *>(h4 + (size_t)s * H);
    const float4 *orow = reinterpret_cast<const float4 *>(out);
    const uint2 *wrow = reinterpret_cast<const uint2 *>(wn + (size_t)s * H);
    const float injv = inj[s];
    constexpr int NR = NI > 0 ? NI : 1;
    float4 hv[NR], ov[NR];
    uint2 gw[NR];
    if (NI > 0) {
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
            const bool ok = i < n4q;
            ov[j] = ok ? orow[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            hv[j] = ok ? hrow[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            gw[j] = ok ? wrow[i] : make_uint2(0, 0);
        }
    }
    after_loads();
    const float wgt = 2.0f * qh_sigmoid(injv / (float)S);
    float ss = 0.0f;
    auto inject = [&](float4 &v, float4 o) {
        v.x += o.x * wgt; v.y += o.y * wgt; v.z += o.z * wgt; v.w += o.w * wgt;
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
    };
    if (NI > 0) {
#pragma unroll
        for (int j = 0; j < NR; j++)
            if (t + QH_THREADS * j < n4q) inject(hv[j], ov[j]);
    } else {
        for (int i = t; i < n4q; i += QH_THREADS) {
            float4 v = hrow[i];
            inject(v, orow[i]);
            nl[qh_swz(i)] = v;
        }
    }
    {
        const float v = qw_xor_sum<64>(ss);
        if (lane == 0) part[0][wave] = v;
    }
    __syncthreads();
    float tot = part[0][0];
#pragma unroll
    for (int w = 1; w < QH_THREADS / 64; w++) tot = tot + part[0][w];
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
    auto scale = [&](int i, float4 v, uint2 wb) {
        v.x = v.x * inv * __uint_as_float(wb.x << 16);
        v.y = v.y * inv * __uint_as_float(wb.x & 0xFFFF0000u);
        v.z = v.z * inv * __uint_as_float(wb.y << 16);
        v.w = v.w * inv * __uint_as_float(wb.y & 0xFFFF0000u);
        nl[qh_swz(i)] = v;
    };
    if (NI > 0) {
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int i = t + QH_THREADS * j;
            if (i < n4q) scale(i, hv[j], gw[j]);
        }
    } else {
        for (int i = t; i < n4q; i += QH_THREADS) scale(i, nl[qh_swz(i)], wrow[i]);
    }
    __syncthreads();
    return inv;
}

// Injection logit s (order R: a thread per 64-input chunk, each chunk an
// fmaf chain from 0, the chunk sums left to right) of the normed row in LDS.
// Every thread of the workgroup calls it (it holds a barrier).
// qh_inj_load requests thread t's chunk of weights (row s) into ww; then
// qh_inj_logit(nl, pc, ww, ...) takes them.
__device__ __forceinline__ void qh_inj_load(const uint16_t *__restrict__ bj, int s, int HH, uint4 (&ww)[8])
{
    const int t = threadIdx.x;
    if (t < HH / 64) {
        const uint4 *wr = reinterpret_cast<const uint4 *>(bj + (size_t)s * HH + 64 * t);
#pragma unroll
        for (int q = 0; q < 8; q++) ww[q] = wr[q];
    }
}
template <bool SW16 = false>
__device__ __forceinline__ void qh_inj_logit(const float4 *nl, float *pc, const uint4 (&ww)[8], int s, int HH,
                                             float *__restrict__ inj_out)
{
    const int t = threadIdx.x, nch = HH / 64;
    if (t < nch) {
        float4 xa[16];
#pragma unroll
        for (int q = 0; q < 16; q++) xa[q] = nl[SW16 ? qh_swz16(16 * t + q) : 16 * t + q];
        float p = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const uint32_t wd[4] = {ww[q].x, ww[q].y, ww[q].z, ww[q].w};
            const float4 a = xa[2 * q], c = xa[2 * q + 1];
            const float xx[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                p = __builtin_fmaf(__uint_as_float(wd[j] << 16), xx[2 * j], p);
                p = __builtin_fmaf(__uint_as_float(wd[j] & 0xFFFF0000u), xx[2 * j + 1], p);
            }
        }
        pc[t] = p;
    }
    __syncthreads();
    if (t == 0) {
        float tot = pc[0];
        for (int e = 1; e < nch; e++) tot = tot + pc[e];
        inj_out[s] = tot;
    }
}
__device__ __forceinline__ void qh_inj_logit(const float4 *nl, float *pc, const uint16_t *__restrict__ bj, int s,
                                             int HH, float *__restrict__ inj_out)
{
    // the chunk's 64 weights and inputs all requested before the chain
    uint4 ww[8];
    qh_inj_load(bj, s, HH, ww);
    qh_inj_logit(nl, pc, ww, s, HH, inj_out);
}

// The mixer's first half at decode (one row) in one launch: inject + grouped
// norm, the down-projection and the injection logits.  Every workgroup redoes
// the inject and the norm of all S streams (S*H floats, from L2) into LDS --
// the same arithmetic, in the same order, as k_norm_grouped -- so nothing
// waits on another workgroup.  Workgroup b < lowrank then computes d[b] (a
// 4-bit row over S*H inputs; thread t takes segments t, t + 256, ..., the
// block sum in wave order), and workgroup lowrank + s the injection logit s
// in order R (a thread per 64-input chunk, chunk sums left to right).
// Workgroup s < S writes stream s of h4_out and n4.  h4_out must not alias h4.
// NI > 0: each thread holds exactly NI float4s a stream (n4q <= NI * 256), all
// loaded up front; NI == 0: a loop over them
template <int NI>
__global__ void __launch_bounds__(QH_THREADS) k_hc_pre(float *__restrict__ h4_out, float *__restrict__ n4,
                                                       float *__restrict__ d, float *__restrict__ inj_out,
                                                       const float *__restrict__ h4, const float *__restrict__ out,
                                                       const float *__restrict__ inj, const uint16_t *__restrict__ wn,
                                                       qwk_q4 dn, const uint16_t *__restrict__ bj, int H, int S,
                                                       int lowrank, int G, float eps)
{
    extern __shared__ float4 nl[];          // [S * H / 4]
    __shared__ float part[QH_PRE_MAXS][QH_THREADS / 64];
    __shared__ float pc[QH_THREADS];
    const int b = blockIdx.x, t = threadIdx.x, n4q = H / 4, HH = S * H;
    const int wave = t >> 6, lane = t & 63;
    const int words = HH / 8, groups = HH / G, nseg = HH / 32;

    // the down row's weights, requested after the streams: their latency runs
    // under the norm
    uint4 wv[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    float sc[2] = {0.0f, 0.0f}, bi[2] = {0.0f, 0.0f};
    auto weights = [&]() {
        if (b < lowrank) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int seg = t + QH_THREADS * j;
                if (seg < nseg) {
                    const int g = seg * 32 / G;
                    wv[j] = *reinterpret_cast<const uint4 *>(dn.w + (size_t)b * words + seg * 4);
                    sc[j] = qw_bf16(dn.s[(size_t)b * groups + g]);
                    bi[j] = qw_bf16(dn.b[(size_t)b * groups + g]);
                }
            }
        }
    };

    float inv[QH_PRE_MAXS];
    qh_inject_norm<NI>(nl, part, b < S ? b : -1, h4_out, n4, h4, out, inj, wn, H, S, eps, inv, weights);
    if (b < lowrank) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int seg = t + QH_THREADS * j;
            if (seg < nseg) {
                float xs[32];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float4 v = nl[seg * 8 + q];
                    xs[4 * q] = v.x; xs[4 * q + 1] = v.y; xs[4 * q + 2] = v.z; xs[4 * q + 3] = v.w;
                }
                float xsum = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; e++) xsum += xs[e];
                float dd = qw_dot8_q(wv[j].x, xs, 0.0f);
                dd = qw_dot8_q(wv[j].y, xs + 8, dd);
                dd = qw_dot8_q(wv[j].z, xs + 16, dd);
                dd = qw_dot8_q(wv[j].w, xs + 24, dd);
                acc = __builtin_fmaf(sc[j], dd, acc);
                acc = __builtin_fmaf(bi[j], xsum, acc);
            }
        }
        acc = qh_block_sum(acc, &part[0][0]);
        if (t == 0) d[b] = acc;
    } else {
        qh_inj_logit(nl, pc, bj, b - lowrank, HH, inj_out);
    }
}

extern "C" int qwk_hc_pre_decode(hipStream_t s, float *h4_out, float *n4, float *d, float *inj_out, const float *h4,
                                 const float *out, const float *inj, const uint16_t *wn, qwk_q4 dn,
                                 const uint16_t *bj, int H, int S, int lowrank, int group, float eps)
{
    const int HH = S * H;
    if (H <= 0 || H % 4 || S < 1 || S > QH_PRE_MAXS || HH % 64 || HH / 64 > QH_THREADS || HH > 15360 ||   /* LDS: S*H floats plus ~1 KB static */
        lowrank < 1 || (group != 32 && group != 64 && group != 128) || HH % group || h4_out == h4 ||
        inj_out == inj || ((uintptr_t)h4 & 15u) || ((uintptr_t)h4_out & 15u) || ((uintptr_t)n4 & 15u) ||
        ((uintptr_t)out & 15u) || ((uintptr_t)wn & 7u) || ((uintptr_t)dn.w & 15u) || ((uintptr_t)bj & 15u))
        return (int)hipErrorInvalidValue;
    const int ni = (H / 4 + QH_THREADS - 1) / QH_THREADS;
#define QH_PRE_LAUNCH(N)                                                                                             \
    hipLaunchKernelGGL(k_hc_pre<N>, dim3((unsigned)(lowrank + S)), dim3(QH_THREADS), (size_t)HH * 4, s, h4_out, n4, \
                       d, inj_out, h4, out, inj, wn, dn, bj, H, S, lowrank, group, eps)
    switch (ni) {
    case 1: QH_PRE_LAUNCH(1); break;
    case 2: QH_PRE_LAUNCH(2); break;
    case 3: QH_PRE_LAUNCH(3); break;
    case 4: QH_PRE_LAUNCH(4); break;
    default: QH_PRE_LAUNCH(0); break;
    }
#undef QH_PRE_LAUNCH
    return (int)hipGetLastError();
}

extern "C" int qwk_repeat_cols(hipStream_t s, float *h4, const float *x, int rows, int H, int S)
{
    if (rows <= 0) return 0;
    if (H % 4 || S < 1 || ((uintptr_t)h4 & 15u) || ((uintptr_t)x & 15u)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_repeat_cols, qh_grid((int64_t)rows * S * H / 4), dim3(QH_THREADS), 0, s,
                       reinterpret_cast<float4 *>(h4), reinterpret_cast<const float4 *>(x), rows, H / 4, S);
    return (int)hipGetLastError();
}

extern "C" int qwk_rms_norm_grouped(hipStream_t s, float *y, const float *x, const uint16_t *w, int dim, int groups,
                                    int rows, float eps)
{
    if (rows <= 0) return 0;
    if (dim <= 0 || dim % 4 || groups < 1 || !w || ((uintptr_t)x & 15u) || ((uintptr_t)y & 15u) || ((uintptr_t)w & 7u))
        return (int)hipErrorInvalidValue;
    qh_norm_launch(s, rows * groups, y, const_cast<float *>(x), w, dim, groups, eps, nullptr, nullptr);
    return (int)hipGetLastError();
}

extern "C" int qwk_hc_inject_norm(hipStream_t s, float *h4, const float *out, const float *inj, const uint16_t *w,
                                  float *n4, int rows, int H, int S, float eps)
{
    if (rows <= 0) return 0;
    if (H <= 0 || H % 4 || S < 1 || !w || !out || !inj || ((uintptr_t)h4 & 15u) || ((uintptr_t)n4 & 15u) ||
        ((uintptr_t)out & 15u) || ((uintptr_t)w & 7u))
        return (int)hipErrorInvalidValue;
    qh_norm_launch(s, rows * S, n4, h4, w, H, S, eps, out, inj);
    return (int)hipGetLastError();
}

extern "C" int qwk_silu_scale(hipStream_t s, float *y, int64_t n, float scale)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_silu_scale, qh_grid(n), dim3(QH_THREADS), 0, s, y, n, scale);
    return (int)hipGetLastError();
}

extern "C" int qwk_hc_mix(hipStream_t s, float *x, const float *n, const float *m, int rows, int H, int S)
{
    if (rows <= 0) return 0;
    if (H <= 0 || S < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hc_mix, qh_grid((int64_t)rows * H), dim3(QH_THREADS), 0, s, x, n, m, rows, H, S);
    return (int)hipGetLastError();
}

extern "C" int qwk_hc_inject(hipStream_t s, float *h4, const float *out, const float *inj, int rows, int H, int S)
{
    if (rows <= 0) return 0;
    if (H <= 0 || S < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hc_inject, qh_grid((int64_t)rows * S * H), dim3(QH_THREADS), 0, s, h4, out, inj, rows, H, S);
    return (int)hipGetLastError();
}

extern "C" int qwk_hc_mix_up(hipStream_t s, float *x, const float *d, const float *n4, const uint32_t *w,
                             const uint16_t *sc, const uint16_t *bi, int k, int H, int S, int rows, float scale,
                             int group)
{
    if (rows <= 0) return 0;
    if (S < 1 || S > 4 || k <= 0 || k % 8 || H <= 0 || (group != 32 && group != 64 && group != 128) ||
        k % group || ((uintptr_t)d & 15u))
        return (int)hipErrorInvalidValue;
    const int lgG = group == 32 ? 5 : group == 64 ? 6 : 7;
    hipLaunchKernelGGL(k_hc_mix_up, dim3((unsigned)((H + 3) / 4)), dim3(QH_THREADS), 0, s, x, d, n4, w, sc, bi, k, H,
                       S, rows, scale, lgG);
    return (int)hipGetLastError();
}

// ---- a whole decode step of the mixer in one launch ------------------------------
//
// k_hc_pre and k_hc_mix_up fused: the up-projection's weights are requested
// at the start, so their memory latency runs under the norm and the
// down-projection instead of after them.  Roles by workgroup:
//
//   b < nd           down: stream s = b % S of QH_DR rows of d: the stream
//                    injected and normed alone (a grouped norm keeps the
//                    streams apart: the same bits as k_hc_pre's), then each
//                    row's dot over the stream's H inputs, 32 lanes a row;
//                    the partials leave as tagged words {epoch, bits}; the
//                    workgroups of rows 0.. also publish their stream's
//                    1/rms.  Then a done word in each of QH_DREP copies.
//   nd <= b < nd+S   stream s = b - nd: inject + norm, writes stream s of
//                    h4_out and n4 and the injection logit s (as k_hc_pre).
//   the rest         up: OW = 32 / S outputs, 8 lanes on each of their S up
//                    rows (lane: words lr, lr + 8, ...).  Weights in
//                    registers first; then one wave polls the down
//                    workgroups' done words (the copy of its XCD), the
//                    workgroup reads the partials and 1/rms (tags checked),
//                    adds each row's S partials in stream order into d,
//                    takes silu(scale d) into LDS, and each row's dot meets in an
//                    xor tree; n4's values for its outputs are recomputed
//                    from h4, out and the 1/rms, and the streams mixed in
//                    order.
//
// Nothing waits on a workgroup dispatched after it (the down workgroups come
// first), and every wait is bounded: on giving up it raises the error word
// (the launch's epoch, unless set) and the workgroup finishes.
#define QH_DR 8                   // down rows a workgroup (of one stream; 32 lanes a row)
#define QH_DLPR (QH_THREADS / QH_DR)   // lanes a down row
#define QH_NSJ 8                  // 32-input segments a down lane holds (H <= 32 * QH_DLPR * QH_NSJ)
#define QH_MAX_LR 512             // lowrank
#define QH_UP_NJ 8                // words an up lane holds (k <= 512)
#define QH_DREP 8                 // copies of the done words
#define QH_DSTRIDE (QH_PRE_MAXS * QH_MAX_LR / QH_DR + 8)   // words between copies (>= the down workgroups)
#define QH_TD 8                   // tag words: [0, S) 1/rms, [QH_TD, + S lowrank) d's partials
#define QH_TDONE (QH_TD + QH_PRE_MAXS * QH_MAX_LR)   // (stream-major), then the done copies
#define QH_TAG_WORDS (QH_TDONE + QH_DREP * QH_DSTRIDE)
#define QH_SPIN_LIMIT (1 << 16)
#define QH_SLEEP 1                // s_sleep between polls (units of 64 clocks)


__device__ __forceinline__ unsigned long long qh_ld(const uint2 *p)
{
    return __hip_atomic_load(reinterpret_cast<const unsigned long long *>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void qh_st(uint2 *p, uint32_t epoch, uint32_t v)
{
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), (unsigned long long)epoch | ((unsigned long long)v << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void qh_raise(uint32_t *err, uint32_t epoch)
{
    uint32_t expect = 0u;
    __hip_atomic_compare_exchange_strong(err, &expect, epoch, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}

// One wave: until words p[0, n) all hold the epoch; false (the error word
// raised) if the wait gave up or another wait already had.
__device__ bool qh_wait_words(const uint2 *p, int n, uint32_t *err, uint32_t epoch)
{
    const int lane = threadIdx.x & 63;
    for (int spins = 0;; spins++) {
        bool stale = false;
        for (int i = lane; i < n; i += 64) stale |= (uint32_t)qh_ld(p + i) != epoch;
        const uint32_t e = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__ballot(stale) == 0ull) return true;
        if (spins >= QH_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
            if (lane == 0) qh_raise(err, epoch);
            return false;
        }
        __builtin_amdgcn_s_sleep(QH_SLEEP);
    }
}

#define QH_UP_RATE 200.0     // bytes a 100 MHz tick through one CU's L1 (~20 GB/s), for up_delay

struct QhArgs {
    float *x, *h4_out, *n4, *d, *inj_out;
    const float *h4, *out, *inj;
    const uint16_t *wn, *bj;
    qwk_q4 dn, up;
    int H, S, lowrank, lgG, nd, ow;
    float eps, scale;
    uint32_t *err;
    uint2 *tw;
    uint32_t epoch;
    uint32_t up_delay;        // wall-clock ticks (100 MHz) before the up role requests its weights
};

template <int NI>
__global__ void __launch_bounds__(QH_THREADS) k_hc_decode(QhArgs a)
{
    extern __shared__ float4 nl[];          // [S * H / 4]; the up role's staging
    __shared__ float part[QH_PRE_MAXS][QH_THREADS / 64];
    __shared__ float pc[QH_THREADS];
    const int b = blockIdx.x, t = threadIdx.x, H = a.H, S = a.S, HH = S * H, k = a.lowrank;
    const int wave = t >> 6, lane = t & 63;
    if (b < a.nd) {
        const int sd = b % S, r0 = (b / S) * QH_DR, words = HH / 8, nsg = H / 32;
        const int q = t / QH_DLPR, l = t % QH_DLPR, r = r0 + q;
        const bool rok = r < k;
        // the rows' words of this stream, requested after the stream: their
        // latency runs under the norm
        uint4 wv[QH_NSJ];
        float sc[QH_NSJ], bi[QH_NSJ];
        auto weights = [&]() {
#pragma unroll
            for (int j = 0; j < QH_NSJ; j++) {
                const int seg = l + QH_DLPR * j;
                const bool ok = rok && seg < nsg;
                const int in0 = sd * H + 32 * seg, g = in0 >> a.lgG;
                const size_t gi = (size_t)r * (HH >> a.lgG) + g;
                wv[j] = ok ? *reinterpret_cast<const uint4 *>(a.dn.w + (size_t)r * words + in0 / 8)
                           : make_uint4(0, 0, 0, 0);
                sc[j] = ok ? qw_bf16(a.dn.s[gi]) : 0.0f;
                bi[j] = ok ? qw_bf16(a.dn.b[gi]) : 0.0f;
            }
        };
        const float inv = qh_norm1<NI>(nl, part, sd, a.h4, a.out, a.inj, a.wn, H, S, a.eps, weights);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < QH_NSJ; j++) {
            const int seg = l + QH_DLPR * j;
            if (seg < nsg) {
                float xs[32];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float4 v = nl[qh_swz(seg * 8 + e)];
                    xs[4 * e] = v.x; xs[4 * e + 1] = v.y; xs[4 * e + 2] = v.z; xs[4 * e + 3] = v.w;
                }
                float xsum = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; e++) xsum += xs[e];
                float dd = qw_dot8_q(wv[j].x, xs, 0.0f);
                dd = qw_dot8_q(wv[j].y, xs + 8, dd);
                dd = qw_dot8_q(wv[j].z, xs + 16, dd);
                dd = qw_dot8_q(wv[j].w, xs + 24, dd);
                acc = __builtin_fmaf(sc[j], dd, acc);
                acc = __builtin_fmaf(bi[j], xsum, acc);
            }
        }
        acc = qw_xor_sum<QH_DLPR>(acc);
        if (l == 0 && rok) qh_st(a.tw + QH_TD + sd * k + r, a.epoch, __float_as_uint(acc));
        if (r0 == 0 && t == 0) qh_st(a.tw + sd, a.epoch, __float_as_uint(inv));
        // the done words follow without waiting for those stores'
        // acknowledgement: a reader checks every partial's tag and re-reads
        // stale ones, so the done words only say when to start reading
        __syncthreads();
        if (t < QH_DREP) qh_st(a.tw + QH_TDONE + t * QH_DSTRIDE + b, a.epoch, 0u);
        return;
    }
    if (b < a.nd + S) {
        const int s = b - a.nd;
        float inv[QH_PRE_MAXS];
        // the injection row requested behind the streams: its latency runs
        // under the norm
        uint4 ww[8];
        qh_inject_norm<NI, true>(nl, part, s, a.h4_out, a.n4, a.h4, a.out, a.inj, a.wn, H, S, a.eps, inv,
                                 [&] { qh_inj_load(a.bj, s, HH, ww); });
        qh_inj_logit<true>(nl, pc, ww, s, HH, a.inj_out);
        return;
    }
    // up
    const int u = b - a.nd - S, ow = a.ow, i0 = u * ow;
    const int rl = t >> 3, lr = t & 7, o = rl / S, s = rl % S;
    const bool on = o < ow && i0 + o < H;
    const int i = min(i0 + o, H - 1);
    const size_t grow = (size_t)s * H + i;
    const int words = k / 8, groups = k >> a.lgG;
    // The up rows wait until the down workgroups have read their streams
    // and rows (about the time those bytes take through a CU's L1): the two
    // roles share CUs, and the down phase is the critical path.
    {
        const unsigned long long t0 = wall_clock64();
        while (wall_clock64() - t0 < a.up_delay) __builtin_amdgcn_s_sleep(2);
    }
    uint32_t wq[QH_UP_NJ], sb[QH_UP_NJ];
#pragma unroll
    for (int j = 0; j < QH_UP_NJ; j++) {
        const int wi = lr + 8 * j;
        const bool ok = on && wi < words;
        const size_t gi = grow * groups + ((8 * wi) >> a.lgG);
        wq[j] = ok ? a.up.w[grow * words + wi] : 0u;
        sb[j] = ok ? (uint32_t)a.up.s[gi] | ((uint32_t)a.up.b[gi] << 16) : 0u;
    }
    // this row's stream value with the block's output injected (as the
    // inject of k_hc_pre), normed once the 1/rms is in
    float v = 0.0f, wnv = 0.0f;
    if (on && lr == 0) {
        const float wgt = 2.0f * qh_sigmoid(a.inj[s] / (float)S);
        v = a.h4[grow];
        v += a.out[i] * wgt;
        wnv = __uint_as_float((uint32_t)a.wn[grow] << 16);
    }
    float *xsl = reinterpret_cast<float *>(nl);            // [k]
    float *dl = xsl + QH_MAX_LR;                            // [k]
    float *invl = dl + QH_MAX_LR;                           // [S]
    float *mixv = invl + QH_PRE_MAXS;                       // [ow][S]
    // one wave polls the down workgroups' done words (its XCD's copy: the
    // polling stays off the words the down workgroups write), then the
    // workgroup reads d's partials and the 1/rms, every tag checked (the
    // done words were stored after them, so a stale word is rare: the
    // workgroup then reads them all again)
    __shared__ int fail;
    if (t == 0) fail = 0;
    __syncthreads();
    if (wave == 0 && !qh_wait_words(a.tw + QH_TDONE + (b & (QH_DREP - 1)) * QH_DSTRIDE, a.nd, a.err, a.epoch))
        fail = 1;
    __syncthreads();
    if (!fail) {
        for (int spins = 0;; spins++) {
            bool stale = false;
            // every word this thread reads requested at once: rows t + 256 j
            // (j < QH_UPJ), their S partials each, and the 1/rms words
            constexpr int QH_UPJ = (QH_MAX_LR + QH_THREADS - 1) / QH_THREADS;
            unsigned long long q[QH_UPJ][QH_PRE_MAXS], qi = 0;
#pragma unroll
            for (int j = 0; j < QH_UPJ; j++) {
                const int r = t + QH_THREADS * j;
#pragma unroll
                for (int sp = 0; sp < QH_PRE_MAXS; sp++)
                    q[j][sp] = r < k && sp < S ? qh_ld(a.tw + QH_TD + sp * k + r) : (unsigned long long)a.epoch;
            }
            if (t < S) qi = qh_ld(a.tw + t);
#pragma unroll
            for (int j = 0; j < QH_UPJ; j++) {
                const int r = t + QH_THREADS * j;
                if (r < k) {
                    // the row's partials, added in stream order
                    float dv = __uint_as_float((uint32_t)(q[j][0] >> 32));
                    stale |= (uint32_t)q[j][0] != a.epoch;
#pragma unroll
                    for (int sp = 1; sp < QH_PRE_MAXS; sp++)
                        if (sp < S) {
                            stale |= (uint32_t)q[j][sp] != a.epoch;
                            dv = dv + __uint_as_float((uint32_t)(q[j][sp] >> 32));
                        }
                    dl[r] = dv;
                    dv = dv * a.scale;
                    xsl[r] = dv * qh_sigmoid(dv);
                }
            }
            if (t < S) {
                stale |= (uint32_t)qi != a.epoch;
                invl[t] = __uint_as_float((uint32_t)(qi >> 32));
            }
            if (!__syncthreads_or(stale)) break;
            if (spins >= QH_SPIN_LIMIT) {
                if (t == 0) qh_raise(a.err, a.epoch);
                break;
            }
            __builtin_amdgcn_s_sleep(QH_SLEEP);
        }
    }
    __syncthreads();
    if (u == 0)
        for (int r = t; r < k; r += QH_THREADS) a.d[r] = dl[r];
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < QH_UP_NJ; j++) {
        const int wi = lr + 8 * j;
        if (wi < words) {
            const float sv = __uint_as_float(sb[j] << 16), bv = __uint_as_float(sb[j] & 0xFFFF0000u);
#pragma unroll
            for (int e = 0; e < 8; e++)
                acc = __builtin_fmaf(__builtin_fmaf(sv, (float)((wq[j] >> (4 * e)) & 0xFu), bv), xsl[8 * wi + e], acc);
        }
    }
    acc = qw_xor_sum<8>(acc);
    if (on && lr == 0) mixv[o * S + s] = qh_sigmoid(acc) * (v * invl[s] * wnv);
    __syncthreads();
    if (t < ow && i0 + t < H) {
        float mix = 0.0f;
        for (int q = 0; q < S; q++) mix = mix + mixv[t * S + q];
        a.x[i0 + t] = mix / (float)S;
    }
}

extern "C" size_t qwk_hc_decode_tag_words(void) { return QH_TAG_WORDS; }

extern "C" int qwk_hc_decode(hipStream_t s, float *x, float *h4_out, float *n4, float *d, float *inj_out,
                             const float *h4, const float *out, const float *inj, const uint16_t *wn, qwk_q4 dn,
                             const uint16_t *bj, qwk_q4 up, int H, int S, int lowrank, int group, float eps,
                             float scale, uint32_t *err, void *tags, uint32_t epoch)
{
    const int HH = S * H;
    if (H <= 0 || H % 4 || S < 1 || S > QH_PRE_MAXS || HH % 64 || HH / 64 > QH_THREADS || HH > 15360 ||
        H % 32 || H > 32 * QH_DLPR * QH_NSJ || lowrank < 8 || lowrank > QH_MAX_LR || lowrank % 8 || (group != 32 && group != 64 && group != 128) ||
        HH % group || lowrank % group || h4_out == h4 || inj_out == inj || !err || !tags || epoch == 0u ||
        ((uintptr_t)h4 & 15u) || ((uintptr_t)h4_out & 15u) || ((uintptr_t)n4 & 15u) || ((uintptr_t)out & 15u) ||
        ((uintptr_t)wn & 7u) || ((uintptr_t)dn.w & 15u) || ((uintptr_t)bj & 15u) || ((uintptr_t)up.w & 3u))
        return (int)hipErrorInvalidValue;
    QhArgs a;
    a.x = x; a.h4_out = h4_out; a.n4 = n4; a.d = d; a.inj_out = inj_out;
    a.h4 = h4; a.out = out; a.inj = inj; a.wn = wn; a.bj = bj; a.dn = dn; a.up = up;
    a.H = H; a.S = S; a.lowrank = lowrank; a.lgG = group == 32 ? 5 : group == 64 ? 6 : 7;
    a.nd = S * ((lowrank + QH_DR - 1) / QH_DR);
    a.ow = 32 / S;
    a.eps = eps; a.scale = scale;
    a.err = err; a.tw = (uint2 *)tags; a.epoch = epoch;
    {
        // a down workgroup's bytes (its stream, the out row, the stream's
        // norm gains, its rows' words, scales and biases of the stream) at
        // ~20 GB/s, a CU's L1 under load: 2.2 us at H 3072, S 4 (A/B, us a
        // step: twice the wait 12.0, half 11.3-11.4, none 11.4-11.5, this
        // 11.2-11.3)
        const double bytes = (double)H * 4 + (double)H * 4 + (double)H * 2 +
                             (double)QH_DR * ((double)H / 2 + 4.0 * (H / group));
        a.up_delay = (uint32_t)(bytes / QH_UP_RATE);
    }
    const int nu = (H + a.ow - 1) / a.ow;
    const int grid = a.nd + S + nu;
    // LDS: the normed streams, or the up role's inputs, 1/rms and mix terms
    const size_t lds = (size_t)HH * 4 > (size_t)(2 * QH_MAX_LR + QH_PRE_MAXS + 32) * 4
                           ? (size_t)HH * 4 : (size_t)(2 * QH_MAX_LR + QH_PRE_MAXS + 32) * 4;
    const int ni = (H / 4 + QH_THREADS - 1) / QH_THREADS;
    switch (ni) {
    case 1: hipLaunchKernelGGL(k_hc_decode<1>, dim3(grid), dim3(QH_THREADS), lds, s, a); break;
    case 2: hipLaunchKernelGGL(k_hc_decode<2>, dim3(grid), dim3(QH_THREADS), lds, s, a); break;
    case 3: hipLaunchKernelGGL(k_hc_decode<3>, dim3(grid), dim3(QH_THREADS), lds, s, a); break;
    case 4: hipLaunchKernelGGL(k_hc_decode<4>, dim3(grid), dim3(QH_THREADS), lds, s, a); break;
    default: hipLaunchKernelGGL(k_hc_decode<0>, dim3(grid), dim3(QH_THREADS), lds, s, a); break;
    }
    return (int)hipGetLastError();
}
