// qw_gdn.hip -- the gated DeltaNet's three kernels (reference contract
// qwasar_gpu.h:318-358, CPU semantics qwasar_cpu.c:217-283):
//
//   k_conv1d_causal_silu  the causal depthwise conv over the mixed q/k/v
//                         channels with silu, its window carried in `state`
//   k_gdn_gates           g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)
//   k_gated_delta<PREP>   the delta-rule recurrence per value head,
//                             S *= g;  kv = S k;  S += k (v - kv) beta;  y = S q
//                         and, with PREP, q and k l2-normed and the gates
//                         computed inside the kernel; with CONV (one decode
//                         step) the conv too, for the channels it reads
//
// The recurrence is serial in time but independent across the rows of each
// head's [dv, dk] state.  A wave owns two value rows: each half-wave one
// row, each lane four consecutive key columns held in registers for the
// whole call, so the state crosses HBM once per call, not once per step.  A
// workgroup (four waves) owns eight rows of one head; the timesteps' q, k,
// v and gates are staged 16 at a time into LDS, which the eight rows share,
// so the serial loop reads only LDS.  Both dot products of a step reduce over
// the half-wave with the fixed xor tree (four DPP steps and one swizzle).
#include "qw_device.h"
#include "qw_kernels.h"

#define QG_DK 128
#define QG_DV 128
#define QG_ROWS_PER_WG 8
#define QG_CHUNK 16
#define QG_THREADS 256

__device__ __forceinline__ float qg_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// ---- causal conv ------------------------------------------------------------

// Output t of a channel depends only on the inputs t - KS + 1 .. t (the
// carried window standing in for t < 0), never on an earlier output, so the
// launch runs over (channel, run of QG_CONV_T steps) in parallel: a thread
// a channel of one run, its window loaded once, each step one fma chain over
// the taps oldest first (from 0) and silu.  Snapshot t (t < n_snap) is the
// window after step t: inputs t - KS + 2 .. t.  The thread of a channel's
// first run is the only one that reads the carried window, and it also writes
// the window after the last step (the last KS - 1 inputs, older ones from the
// window it read), so the window is updated in place without a race between
// workgroups.
#define QG_CONV_T 16
template <int KS>
__global__ void __launch_bounds__(256) k_conv1d_causal_silu(float *__restrict__ y, const float *__restrict__ x,
                                                            float *__restrict__ state, const uint16_t *__restrict__ w,
                                                            int channels, int rows, float *__restrict__ snap,
                                                            int n_snap, int snap_stride)
{
    const int ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= channels) return;
    const int t0 = blockIdx.y * QG_CONV_T, t1 = min(t0 + QG_CONV_T, rows);
    float taps[KS], win[KS + QG_CONV_T], old[KS - 1];
#pragma unroll
    for (int j = 0; j < KS; j++) taps[j] = qw_bf16(w[(size_t)ch * KS + j]);
    // win[i] = input t0 - (KS - 1) + i
    if (t0 == 0) {
#pragma unroll
        for (int j = 0; j < KS - 1; j++) win[j] = old[j] = state[(size_t)j * channels + ch];
    } else {
#pragma unroll
        for (int j = 0; j < KS - 1; j++) win[j] = x[(size_t)(t0 - (KS - 1) + j) * channels + ch];
    }
#pragma unroll
    for (int u = 0; u < QG_CONV_T; u++) win[KS - 1 + u] = t0 + u < t1 ? x[(size_t)(t0 + u) * channels + ch] : 0.0f;
#pragma unroll
    for (int u = 0; u < QG_CONV_T; u++) {
        const int t = t0 + u;
        if (t < t1) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < KS; j++) acc = __builtin_fmaf(win[u + j], taps[j], acc);
            y[(size_t)t * channels + ch] = acc / (1.0f + expf(-acc));
            if (t < n_snap) {
#pragma unroll
                for (int j = 0; j < KS - 1; j++) snap[(size_t)t * snap_stride + (size_t)j * channels + ch] = win[u + 1 + j];
            }
        }
    }
    if (t0 == 0) {
        // the window after the last step: inputs rows - KS + 1 .. rows - 1
#pragma unroll
        for (int j = 0; j < KS - 1; j++) {
            const int t = rows - (KS - 1) + j;
            float v = 0.0f;
#pragma unroll
            for (int m = 0; m < KS - 1; m++)
                if (m == KS - 1 + t) v = old[m];                       // rows < KS - 1: from the window read
            state[(size_t)j * channels + ch] = t >= 0 ? x[(size_t)t * channels + ch] : v;
        }
    }
}

// ---- gates ------------------------------------------------------------------

__device__ __forceinline__ void qg_gates(float a, float b, float A, float dt, float &g, float &beta)
{
    g = expf(-expf(A) * qg_softplus(a + dt));
    beta = 1.0f / (1.0f + expf(-b));
}

__global__ void __launch_bounds__(256) k_gdn_gates(float *__restrict__ g, float *__restrict__ beta,
                                                   const float *__restrict__ a, const float *__restrict__ b,
                                                   const uint16_t *__restrict__ A_log,
                                                   const uint16_t *__restrict__ dt_bias, int hv, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int h = i % hv;
    qg_gates(a[i], b[i], qw_bf16(A_log[h]), qw_bf16(dt_bias[h]), g[i], beta[i]);
}

// ---- the recurrence -----------------------------------------------------------

struct qg_prep {
    const float *a, *b;
    const uint16_t *A_log, *dt_bias;
    float l2eps, q_scale, k_scale;
};

// The fused decode step's conv: the mixed channels before the conv, the
// window in and out (distinct buffers), the taps.
struct qg_conv {
    const float *x, *win;
    float *wout;
    const uint16_t *w;
    int channels;
};

// One channel of the causal conv with silu at one step, the arithmetic of
// k_conv1d_causal_silu (taps against the window oldest first, then the
// new sample, in one fma chain from 0); the window after the step goes to
// wout when `own`.
__device__ __forceinline__ float qg_conv1(const qg_conv &cv, int ch, bool own)
{
    const int C = cv.channels;
    float win[4], acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 3; j++) win[j] = cv.win[(size_t)j * C + ch];
    win[3] = cv.x[ch];
#pragma unroll
    for (int j = 0; j < 4; j++) acc = __builtin_fmaf(win[j], qw_bf16(cv.w[(size_t)ch * 4 + j]), acc);
    if (own) {
#pragma unroll
        for (int j = 0; j < 3; j++) cv.wout[(size_t)j * C + ch] = win[j + 1];
    }
    return acc / (1.0f + expf(-acc));
}

// CONV (one step, PREP): q, k and v are the conv's outputs over the mixed
// channels [0, hk dk), [hk dk, 2 hk dk) and [2 hk dk, ...), computed here
// for the channels this workgroup reads; the first workgroup of each key
// head's group writes the window of its q and k channels, every workgroup
// that of its own v channels.
template <bool PREP, bool CONV = false>
__global__ void __launch_bounds__(QG_THREADS) k_gated_delta(float *__restrict__ y, const float *__restrict__ q,
                                                            const float *__restrict__ k, const float *__restrict__ v,
                                                            const float *__restrict__ g,
                                                            const float *__restrict__ beta, float *state, int hk,
                                                            int hv, int rows, float *__restrict__ snap, int n_snap,
                                                            int snap_stride, qg_prep pp, qg_conv cv = {})
{
    __shared__ float4 sq[QG_CHUNK][QG_DK / 4], sk[QG_CHUNK][QG_DK / 4];
    __shared__ float sv[QG_CHUNK][QG_ROWS_PER_WG];
    __shared__ float sg[QG_CHUNK][2];   // g, beta
    __shared__ float sn[QG_CHUNK][2];   // PREP: q and k norm factors

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int groups = QG_DV / QG_ROWS_PER_WG;
    const int h = blockIdx.x / groups, r0 = (blockIdx.x % groups) * QG_ROWS_PER_WG;
    const int hx = h / (hv / hk);
    const int rl = 2 * wave + (lane >> 5);        // row within the workgroup
    const int row = r0 + rl;
    const int c4 = lane & 31;                      // float4 column index

    float4 *sp = reinterpret_cast<float4 *>(state + ((size_t)h * QG_DV + row) * QG_DK) + c4;
    float4 st = *sp;
    const float A = PREP ? qw_bf16(pp.A_log[h]) : 0.0f;
    const float dt = PREP ? qw_bf16(pp.dt_bias[h]) : 0.0f;
    const size_t qstride = (size_t)hk * QG_DK, vstride = (size_t)hv * QG_DV;

    for (int c0 = 0; c0 < rows; c0 += QG_CHUNK) {
        const int n = min(QG_CHUNK, rows - c0);
        __syncthreads();                           // the previous chunk is consumed
        if (CONV) {
            const int kd = hk * QG_DK;
            const bool own_qk = h % (hv / hk) == 0 && r0 == 0;
            float *fq = reinterpret_cast<float *>(&sq[0][0]), *fk = reinterpret_cast<float *>(&sk[0][0]);
            if (tid < QG_DK) fq[tid] = qg_conv1(cv, hx * QG_DK + tid, own_qk);
            else if (tid < 2 * QG_DK) fk[tid - QG_DK] = qg_conv1(cv, kd + hx * QG_DK + tid - QG_DK, own_qk);
            if (tid < QG_ROWS_PER_WG) sv[0][tid] = qg_conv1(cv, 2 * kd + h * QG_DV + r0 + tid, true);
        } else {
            for (int i = tid; i < n * (QG_DK / 4); i += QG_THREADS) {
                const int t = i / (QG_DK / 4), c = i % (QG_DK / 4);
                const size_t off = (size_t)(c0 + t) * qstride + (size_t)hx * QG_DK;
                sq[t][c] = reinterpret_cast<const float4 *>(q + off)[c];
                sk[t][c] = reinterpret_cast<const float4 *>(k + off)[c];
            }
            if (tid < n * QG_ROWS_PER_WG) {
                const int t = tid / QG_ROWS_PER_WG, j = tid % QG_ROWS_PER_WG;
                sv[t][j] = v[(size_t)(c0 + t) * vstride + (size_t)h * QG_DV + r0 + j];
            }
        }
        if (tid >= 128 && tid < 128 + n) {
            const int t = tid - 128;
            const size_t gi = (size_t)(c0 + t) * hv + h;
            if (PREP) {
                qg_gates(pp.a[gi], pp.b[gi], A, dt, sg[t][0], sg[t][1]);
            } else {
                sg[t][0] = g[gi];
                sg[t][1] = beta[gi];
            }
        }
        if (PREP) {
            __syncthreads();
            // the l2 norms of the chunk's q and k vectors: a wave per (step,
            // vector), each lane two of the 128 values, then the wave's xor tree
            for (int p = wave; p < 2 * n; p += QG_THREADS / 64) {
                const int t = p >> 1, isk = p & 1;
                const float *src = reinterpret_cast<const float *>(isk ? &sk[t][0] : &sq[t][0]);
                const float a0 = src[lane], a1 = src[lane + 64];
                float ss = __builtin_fmaf(a0, a0, 0.0f);
                ss = __builtin_fmaf(a1, a1, ss);
                ss = qw_xor_sum<64>(ss);
                if (lane == 0)
                    sn[t][isk] = 1.0f / sqrtf(ss / (float)QG_DK + pp.l2eps) * (isk ? pp.k_scale : pp.q_scale);
            }
        }
        __syncthreads();
        for (int t = 0; t < n; t++) {
            float4 qv = sq[t][c4], kv4 = sk[t][c4];
            if (PREP) {
                const float iq = sn[t][0], ik = sn[t][1];
                qv.x *= iq; qv.y *= iq; qv.z *= iq; qv.w *= iq;
                kv4.x *= ik; kv4.y *= ik; kv4.z *= ik; kv4.w *= ik;
            }
            const float gt = sg[t][0], bt = sg[t][1];
            st.x *= gt; st.y *= gt; st.z *= gt; st.w *= gt;
            float kv = st.x * kv4.x;
            kv = __builtin_fmaf(st.y, kv4.y, kv);
            kv = __builtin_fmaf(st.z, kv4.z, kv);
            kv = __builtin_fmaf(st.w, kv4.w, kv);
            kv = qw_xor_sum<32>(kv);
            const float delta = (sv[t][rl] - kv) * bt;
            st.x = __builtin_fmaf(kv4.x, delta, st.x);
            st.y = __builtin_fmaf(kv4.y, delta, st.y);
            st.z = __builtin_fmaf(kv4.z, delta, st.z);
            st.w = __builtin_fmaf(kv4.w, delta, st.w);
            float o = st.x * qv.x;
            o = __builtin_fmaf(st.y, qv.y, o);
            o = __builtin_fmaf(st.z, qv.z, o);
            o = __builtin_fmaf(st.w, qv.w, o);
            o = qw_xor_sum<32>(o);
            const int tt = c0 + t;
            if (c4 == 0) y[(size_t)tt * vstride + (size_t)h * QG_DV + row] = o;
            if (tt < n_snap)
                reinterpret_cast<float4 *>(snap + (size_t)tt * snap_stride + ((size_t)h * QG_DV + row) * QG_DK)[c4] = st;
        }
    }
    *sp = st;
}

// ---- launchers ----------------------------------------------------------------

extern "C" int qwk_conv1d_causal_silu(hipStream_t s, float *y, const float *x, float *state, const uint16_t *w,
                                      int channels, int rows, int ksize, float *snap, int n_snap, int snap_stride)
{
    if (ksize != 4 || channels < 1 || rows < 0 || n_snap < 0 || (n_snap > 0 && (!snap || snap_stride < 3 * channels)))
        return hipErrorInvalidValue;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(k_conv1d_causal_silu<4>, dim3((channels + 255) / 256, (rows + QG_CONV_T - 1) / QG_CONV_T),
                       dim3(256), 0, s, y, x, state, w,
                       channels, rows, snap, n_snap, snap_stride);
    return (int)hipGetLastError();
}

extern "C" int qwk_gdn_decode(hipStream_t s, float *y, const float *x, const float *win, float *wout,
                              const uint16_t *w, const qwk_gdn_prep *prep, float *state, int hk, int hv, int dk,
                              int dv)
{
    if (dk != QG_DK || dv != QG_DV || hk < 1 || hv < 1 || hv % hk || !prep || !x || !win || !wout || !w)
        return hipErrorInvalidValue;
    const int channels = 2 * hk * dk + hv * dv;
    const qg_prep pp = { prep->a, prep->b, prep->A_log, prep->dt_bias, prep->l2eps, prep->q_scale, prep->k_scale };
    const qg_conv cv = { x, win, wout, w, channels };
    hipLaunchKernelGGL((k_gated_delta<true, true>), dim3(hv * (QG_DV / QG_ROWS_PER_WG)), dim3(QG_THREADS), 0, s, y,
                       nullptr, nullptr, nullptr, nullptr, nullptr, state, hk, hv, 1, nullptr, 0, 0, pp, cv);
    return (int)hipGetLastError();
}

extern "C" int qwk_gdn_gates(hipStream_t s, float *g, float *beta, const float *a, const float *b,
                             const uint16_t *A_log, const uint16_t *dt_bias, int hv, int rows)
{
    if (hv < 1 || rows < 0) return hipErrorInvalidValue;
    const int n = hv * rows;
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_gdn_gates, dim3((n + 255) / 256), dim3(256), 0, s, g, beta, a, b, A_log, dt_bias, hv, n);
    return (int)hipGetLastError();
}

extern "C" int qwk_gated_delta(hipStream_t s, float *y, const float *q, const float *k, const float *v,
                               const float *g, const float *beta, float *state, int hk, int hv, int dk, int dv,
                               int rows, float *snap, int n_snap, int snap_stride, const qwk_gdn_prep *prep)
{
    if (dk != QG_DK || dv != QG_DV || hk < 1 || hv < 1 || hv % hk || rows < 0 || n_snap < 0 ||
        (n_snap > 0 && (!snap || snap_stride < hv * dv * dk || snap_stride % 4)))
        return hipErrorInvalidValue;
    if (rows == 0) return 0;
    const dim3 grid(hv * (QG_DV / QG_ROWS_PER_WG));
    if (prep) {
        const qg_prep pp = { prep->a, prep->b, prep->A_log, prep->dt_bias, prep->l2eps, prep->q_scale, prep->k_scale };
        hipLaunchKernelGGL(k_gated_delta<true>, grid, dim3(QG_THREADS), 0, s, y, q, k, v, nullptr, nullptr, state,
                           hk, hv, rows, snap, n_snap, snap_stride, pp);
    } else {
        const qg_prep pp = {};
        hipLaunchKernelGGL(k_gated_delta<false>, grid, dim3(QG_THREADS), 0, s, y, q, k, v, g, beta, state, hk, hv,
                           rows, snap, n_snap, snap_stride, pp);
    }
    return (int)hipGetLastError();
}
