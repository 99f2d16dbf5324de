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
// head's [dv, dk] state.  A wave owns four value rows: each 16-lane row of
// the wave one state row, each lane eight consecutive key columns held in
// registers for the whole call, so the state crosses HBM once per call, not
// once per step.  A workgroup (four waves) owns sixteen rows of one head; the
// timesteps' q, k, v and gates are staged 16 at a time into LDS, which the
// sixteen rows share (with PREP, q and k already scaled by their norms), so
// the serial loop reads only LDS.  Each dot product of a step is two fma
// chains of four columns in a lane, their sum, then the fixed xor tree over
// the 16 lanes (four DPP steps inside the row, no cross-row traffic).
#include "qw_device.h"
#include "qw_kernels.h"

#define QG_DK 128
#define QG_DV 128
#define QG_ROWS_PER_WG 16
#define QG_CHUNK 16
#define QG_PRE_MIN_ROWS 64      // prepared calls from this many steps on take k_gdn_pre
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
    // from k_gdn_pre (or null): each step's q and k norm factors
    // [rows][hk][2] and gates (g, beta) [rows][hv][2]
    const float *nrm, *gb;
};

// The l2 norm factor of one 128-value q or k vector, by a whole wave: lane
// l squares values l and l + 64 (an fma chain from 0), then the wave's xor
// tree.  Every lane gets the factor.
__device__ __forceinline__ float qg_norm(float a0, float a1, float l2eps, float scale)
{
    float ss = __builtin_fmaf(a0, a0, 0.0f);
    ss = __builtin_fmaf(a1, a1, ss);
    ss = qw_xor_sum<64>(ss);
    return 1.0f / sqrtf(ss / (float)QG_DK + l2eps) * scale;
}

// A long prepared call's norms and gates ahead of the recurrence, in
// parallel over every step: the first nvw / 4 workgroups a wave a vector
// (vector w: step w / (2 hk), key head (w / 2) % hk, k if w is odd), the
// rest a thread a (step, value head) gate; the recurrence's own functions,
// so the same bits as computed inside it.
__global__ void __launch_bounds__(256) k_gdn_pre(qg_prep pp, const float *__restrict__ q, const float *__restrict__ k,
                                                 int hk, int hv, int rows)
{
    const int nvw = rows * hk * 2, nbv = (nvw + 3) / 4;
    float *nrm = const_cast<float *>(pp.nrm), *gb = const_cast<float *>(pp.gb);
    if ((int)blockIdx.x < nbv) {
        const int w = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
        if (w >= nvw) return;
        const float *src = ((w & 1) ? k : q) + (size_t)(w >> 1) * QG_DK;
        const float f = qg_norm(src[lane], src[lane + 64], pp.l2eps, (w & 1) ? pp.k_scale : pp.q_scale);
        if (lane == 0) nrm[w] = f;
    } else {
        const int i = (blockIdx.x - nbv) * 256 + threadIdx.x;
        if (i >= rows * hv) return;
        const int h = i % hv;
        qg_gates(pp.a[i], pp.b[i], qw_bf16(pp.A_log[h]), qw_bf16(pp.dt_bias[h]), gb[2 * i], gb[2 * i + 1]);
    }
}

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
    const int rl = 4 * wave + (lane >> 4);        // row within the workgroup
    const int row = r0 + rl;
    const int c8 = lane & 15;                      // columns 8 c8 .. 8 c8 + 7

    float4 *sp = reinterpret_cast<float4 *>(state + ((size_t)h * QG_DV + row) * QG_DK) + 2 * c8;
    float4 st = sp[0], su = sp[1];
    const float A = PREP ? qw_bf16(pp.A_log[h]) : 0.0f;
    const float dt = PREP ? qw_bf16(pp.dt_bias[h]) : 0.0f;
    const size_t qstride = (size_t)hk * QG_DK, vstride = (size_t)hv * QG_DV;

    // Without CONV a chunk's q, k, v and gate inputs are fetched into
    // registers one chunk ahead, so their loads run under the previous
    // chunk's steps: thread tid holds float4s tid and tid + 256 of the
    // chunk's [16][32] q and k, value (tid / 16, tid % 16) and, for tid in
    // [128, 144), step tid - 128's gate inputs.
    static_assert(QG_CHUNK * (QG_DK / 4) == 2 * QG_THREADS && QG_CHUNK * QG_ROWS_PER_WG == QG_THREADS,
                  "one chunk's staging is two float4s of q and of k and one value a thread");
    float4 fq0 = {}, fq1 = {}, fk0 = {}, fk1 = {};
    float fv = 0.0f, fa = 0.0f, fb = 0.0f, fn = 0.0f;
    const bool pre = PREP && !CONV && pp.nrm;
    auto fetch = [&](int c) __attribute__((always_inline)) {
        const int nn = min(QG_CHUNK, rows - c);
        const int t0 = tid / (QG_DK / 4), t1 = t0 + QG_THREADS / (QG_DK / 4), cc = tid % (QG_DK / 4);
        const size_t o0 = (size_t)(c + t0) * qstride + (size_t)hx * QG_DK, o1 = o0 + (size_t)(t1 - t0) * qstride;
        if (t0 < nn) {
            fq0 = reinterpret_cast<const float4 *>(q + o0)[cc];
            fk0 = reinterpret_cast<const float4 *>(k + o0)[cc];
        }
        if (t1 < nn) {
            fq1 = reinterpret_cast<const float4 *>(q + o1)[cc];
            fk1 = reinterpret_cast<const float4 *>(k + o1)[cc];
        }
        if (tid / QG_ROWS_PER_WG < nn)
            fv = v[(size_t)(c + tid / QG_ROWS_PER_WG) * vstride + (size_t)h * QG_DV + r0 + tid % QG_ROWS_PER_WG];
        if (tid >= 128 && tid < 128 + nn) {
            const size_t gi = (size_t)(c + tid - 128) * hv + h;
            fa = pre ? pp.gb[2 * gi] : PREP ? pp.a[gi] : g[gi];
            fb = pre ? pp.gb[2 * gi + 1] : PREP ? pp.b[gi] : beta[gi];
        }
        if (pre && tid >= 160 && tid < 160 + 2 * nn)
            fn = pp.nrm[((size_t)(c + (tid - 160) / 2) * hk + hx) * 2 + (tid & 1)];
    };
    if (!CONV) fetch(0);

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
            if (tid >= 128 && tid < 128 + n) {
                const size_t gi = (size_t)(c0 + tid - 128) * hv + h;
                qg_gates(pp.a[gi], pp.b[gi], A, dt, sg[tid - 128][0], sg[tid - 128][1]);
            }
        } else {
            const int t0 = tid / (QG_DK / 4), t1 = t0 + QG_THREADS / (QG_DK / 4), cc = tid % (QG_DK / 4);
            sq[t0][cc] = fq0;
            sk[t0][cc] = fk0;
            sq[t1][cc] = fq1;
            sk[t1][cc] = fk1;
            sv[tid / QG_ROWS_PER_WG][tid % QG_ROWS_PER_WG] = fv;
            if (tid >= 128 && tid < 128 + n) {
                if (PREP && !pre) qg_gates(fa, fb, A, dt, sg[tid - 128][0], sg[tid - 128][1]);
                else {
                    sg[tid - 128][0] = fa;
                    sg[tid - 128][1] = fb;
                }
            }
            if (pre && tid >= 160 && tid < 160 + 2 * n) sn[(tid - 160) / 2][tid & 1] = fn;
            if (c0 + QG_CHUNK < rows) fetch(c0 + QG_CHUNK);
        }
        if (PREP) {
            __syncthreads();
            // the l2 norms of the chunk's q and k vectors: a wave per (step,
            // vector), each lane two of the 128 values, then the wave's xor
            // tree; in a whole chunk a wave's eight vectors are loaded first
            // and their trees run side by side
            auto norm = [&](int p, float a0, float a1) __attribute__((always_inline)) {
                const float f = qg_norm(a0, a1, pp.l2eps, (p & 1) ? pp.k_scale : pp.q_scale);
                if (lane == 0) sn[p >> 1][p & 1] = f;
            };
            auto vec = [&](int p) __attribute__((always_inline)) {
                return reinterpret_cast<const float *>((p & 1) ? &sk[p >> 1][0] : &sq[p >> 1][0]);
            };
            if (pre) {
                // the factors came with the chunk
            } else if (n == QG_CHUNK) {
                static_assert(2 * QG_CHUNK == 8 * (QG_THREADS / 64), "eight vectors a wave");
                float a0[8], a1[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    a0[j] = vec(wave + 4 * j)[lane];
                    a1[j] = vec(wave + 4 * j)[lane + 64];
                }
#pragma unroll
                for (int j = 0; j < 8; j++) norm(wave + 4 * j, a0[j], a1[j]);
            } else {
                for (int p = wave; p < 2 * n; p += QG_THREADS / 64) norm(p, vec(p)[lane], vec(p)[lane + 64]);
            }
            __syncthreads();
            for (int i = tid; i < n * (QG_DK / 4); i += QG_THREADS) {
                const int t = i / (QG_DK / 4), c = i % (QG_DK / 4);
                const float iq = sn[t][0], ik = sn[t][1];
                float4 a = sq[t][c], b = sk[t][c];
                a.x *= iq; a.y *= iq; a.z *= iq; a.w *= iq;
                b.x *= ik; b.y *= ik; b.z *= ik; b.w *= ik;
                sq[t][c] = a;
                sk[t][c] = b;
            }
        }
        __syncthreads();
        // a step; whole chunks unrolled, so that a step's output dot and
        // the next step's LDS reads overlap the state's serial chain
        auto step = [&](int t) __attribute__((always_inline)) {
            const float4 q0 = sq[t][2 * c8], q1 = sq[t][2 * c8 + 1], k0 = sk[t][2 * c8], k1 = sk[t][2 * c8 + 1];
            const float gt = sg[t][0], bt = sg[t][1];
            st.x *= gt; st.y *= gt; st.z *= gt; st.w *= gt;
            su.x *= gt; su.y *= gt; su.z *= gt; su.w *= gt;
            float ka = st.x * k0.x, kb = su.x * k1.x;
            ka = __builtin_fmaf(st.y, k0.y, ka);
            kb = __builtin_fmaf(su.y, k1.y, kb);
            ka = __builtin_fmaf(st.z, k0.z, ka);
            kb = __builtin_fmaf(su.z, k1.z, kb);
            ka = __builtin_fmaf(st.w, k0.w, ka);
            kb = __builtin_fmaf(su.w, k1.w, kb);
            const float kv = qw_xor_sum<16>(ka + kb);
            const float delta = (sv[t][rl] - kv) * bt;
            st.x = __builtin_fmaf(k0.x, delta, st.x);
            st.y = __builtin_fmaf(k0.y, delta, st.y);
            st.z = __builtin_fmaf(k0.z, delta, st.z);
            st.w = __builtin_fmaf(k0.w, delta, st.w);
            su.x = __builtin_fmaf(k1.x, delta, su.x);
            su.y = __builtin_fmaf(k1.y, delta, su.y);
            su.z = __builtin_fmaf(k1.z, delta, su.z);
            su.w = __builtin_fmaf(k1.w, delta, su.w);
            float oa = st.x * q0.x, ob = su.x * q1.x;
            oa = __builtin_fmaf(st.y, q0.y, oa);
            ob = __builtin_fmaf(su.y, q1.y, ob);
            oa = __builtin_fmaf(st.z, q0.z, oa);
            ob = __builtin_fmaf(su.z, q1.z, ob);
            oa = __builtin_fmaf(st.w, q0.w, oa);
            ob = __builtin_fmaf(su.w, q1.w, ob);
            const float o = qw_xor_sum<16>(oa + ob);
            const int tt = c0 + t;
            if (c8 == 0) y[(size_t)tt * vstride + (size_t)h * QG_DV + row] = o;
            if (tt < n_snap) {
                float4 *sn4 = reinterpret_cast<float4 *>(snap + (size_t)tt * snap_stride + ((size_t)h * QG_DV + row) * QG_DK) + 2 * c8;
                sn4[0] = st;
                sn4[1] = su;
            }
        };
        if (n == QG_CHUNK) {
#pragma unroll
            for (int t = 0; t < QG_CHUNK; t++) step(t);
        } else {
            for (int t = 0; t < n; t++) step(t);
        }
    }
    sp[0] = st;
    sp[1] = su;
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
    const qg_prep pp = { prep->a, prep->b, prep->A_log, prep->dt_bias, prep->l2eps, prep->q_scale, prep->k_scale,
                         nullptr, nullptr };
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

extern "C" size_t qwk_gated_delta_work(int hk, int hv, int rows, int prep)
{
    if (!prep || rows < QG_PRE_MIN_ROWS || hk < 1 || hv < 1) return 0;
    return ((size_t)rows * hk * 2 + (size_t)rows * hv * 2) * sizeof(float);
}

extern "C" int qwk_gated_delta(hipStream_t s, float *y, const float *q, const float *k, const float *v,
                               const float *g, const float *beta, float *state, int hk, int hv, int dk, int dv,
                               int rows, float *snap, int n_snap, int snap_stride, const qwk_gdn_prep *prep,
                               void *work)
{
    if (dk != QG_DK || dv != QG_DV || hk < 1 || hv < 1 || hv % hk || rows < 0 || n_snap < 0 ||
        (n_snap > 0 && (!snap || snap_stride < hv * dv * dk || snap_stride % 4)))
        return hipErrorInvalidValue;
    if (rows == 0) return 0;
    const dim3 grid(hv * (QG_DV / QG_ROWS_PER_WG));
    if (prep) {
        qg_prep pp = { prep->a, prep->b, prep->A_log, prep->dt_bias, prep->l2eps, prep->q_scale, prep->k_scale,
                       nullptr, nullptr };
        if (work && qwk_gated_delta_work(hk, hv, rows, 1) > 0) {
            pp.nrm = static_cast<float *>(work);
            pp.gb = pp.nrm + (size_t)rows * hk * 2;
            const int nbv = (rows * hk * 2 + 3) / 4, nbg = (rows * hv + 255) / 256;
            hipLaunchKernelGGL(k_gdn_pre, dim3(nbv + nbg), dim3(256), 0, s, pp, q, k, hk, hv, rows);
        }
        hipLaunchKernelGGL(k_gated_delta<true>, grid, dim3(QG_THREADS), 0, s, y, q, k, v, nullptr, nullptr, state,
                           hk, hv, rows, snap, n_snap, snap_stride, pp);
    } else {
        const qg_prep pp = {};
        hipLaunchKernelGGL(k_gated_delta<false>, grid, dim3(QG_THREADS), 0, s, y, q, k, v, g, beta, state, hk, hv,
                           rows, snap, n_snap, snap_stride, pp);
    }
    return (int)hipGetLastError();
}
