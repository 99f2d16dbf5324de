// qw_decode.hip -- the MoE block at decode (1..8 tokens) in three launches.
//
//   front   router logits (order R) for every expert, the shared expert's
//           gate and up rows, and its gate logit; the last workgroup to
//           finish routes every token (softmax, top-K, renormalise), writes
//           idx/w, and lists the union of the selected experts with the
//           (token, slot) pairs that use each one
//   experts gate and up rows of each selected expert -- each weight byte read
//           once and applied to every token routed to that expert -- and
//           the shared expert's down projection, SwiGLU on load
//   down    each selected expert's down projection, SwiGLU on load, into
//           per-pair rows; the last workgroup to finish a block of output
//           rows combines it: shared * sigmoid(gate) + sum_k w_k * y_k,
//           an fma chain in slot order (deterministic whatever the arrival
//           order)
//
// "Last to finish" is an agent-scope acq_rel atomic on a counter that the
// finishing workgroup resets, so the counters are zero between calls.
#include "qw_device.h"
#include "qw_kernels.h"

#define QD_WAVES 4
#define QD_THREADS (QD_WAVES * 64)
#define QD_RIT 4
#define QD_MAXT QWK_DECODE_MAX_ROWS
#define QD_MAXCH (QWK_DMAT_MAX_K / 64)
#define QD_MAXU (QWK_DECODE_MAX_ROWS * QWK_ROUTE_MAX_K)

struct QdLayout {
    size_t logits, g1, shgu, shout, uinfo, gu, ey, total;
    int nrb;        // down row blocks
};

static __host__ __device__ size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

static __host__ __device__ int qd_lpr(int k)
{
    const int S = k / 32;
    int l = 1;
    while (l < 64 && S % (2 * l) == 0) l *= 2;
    return l;
}

static __host__ __device__ int qd_rows_per_wg(int k) { return QD_WAVES * (64 / qd_lpr(k)) * QD_RIT; }

static QdLayout qd_layout(const qwk_moe *M, int rows)
{
    QdLayout L;
    const int umax = rows * M->K < M->E ? rows * M->K : M->E;
    L.nrb = (M->H + qd_rows_per_wg(M->I) - 1) / qd_rows_per_wg(M->I);
    size_t o = 0;
    L.logits = o; o += al((size_t)rows * M->E * 4);
    L.g1 = o;     o += al((size_t)rows * 4);
    L.shgu = o;   o += al((size_t)rows * 2 * M->SI * 4);
    L.shout = o;  o += al((size_t)rows * M->H * 4);
    L.uinfo = o;  o += al((size_t)(1 + 2 * umax + umax * rows) * 4);
    L.gu = o;     o += al((size_t)rows * M->K * 2 * M->I * 4);
    L.ey = o;     o += al((size_t)rows * M->K * M->H * 4);
    L.total = o;
    return L;
}

struct QdArgs {
    qwk_moe m;
    const float *x;
    float *out;
    int32_t *idx;
    float *w;
    int rows, umax, nrb;
    int n_router_wg, n_shared_wg;       // front
    int n_gu_wg_per_u, n_shdown_wg;     // experts
    int *ctr;
    float *logits, *g1, *shgu, *shout, *gu, *ey;
    int *uinfo;                          // [0] = U, [1..umax] experts, then counts, then pair lists
};

__device__ __forceinline__ int *qd_uexp(const QdArgs &a) { return a.uinfo + 1; }
__device__ __forceinline__ int *qd_ucnt(const QdArgs &a) { return a.uinfo + 1 + a.umax; }
__device__ __forceinline__ int *qd_upair(const QdArgs &a) { return a.uinfo + 1 + 2 * a.umax; }

// Rows [row0, row0 + slots*RIT) of a quantised matrix (one wave) against up to
// QD_MAXT input vectors: y_t[row] = W[row] . in_t, in_t = x_t or
// silu(x_t) * u_t.  Weights are loaded once per segment and reused for every
// token.
template <int G, int LPR, bool SWIGLU>
__device__ __forceinline__ void qd_rows(const uint32_t *__restrict__ wm, const uint16_t *__restrict__ sm,
                                        const uint16_t *__restrict__ bm, int n, int k, int row0, int nt,
                                        const float *const *xp, const float *const *up, float *const *yp)
{
    constexpr int SLOTS = 64 / LPR;
    const int lane = threadIdx.x & 63, slot = lane / LPR, lr = lane % LPR;
    const int words = k / 8, groups = k / G;
    float acc[QD_MAXT][QD_RIT];
#pragma unroll
    for (int t = 0; t < QD_MAXT; t++)
#pragma unroll
        for (int i = 0; i < QD_RIT; i++) acc[t][i] = 0.0f;

    const int spl = (k / 32) / LPR;
    for (int j = 0; j < spl; j++) {
        const int seg = j * LPR + lr, g = seg * 32 / G;
        uint4 wv[QD_RIT];
        float sc[QD_RIT], bi[QD_RIT];
#pragma unroll
        for (int i = 0; i < QD_RIT; i++) {
            const int row = row0 + slot + SLOTS * i;
            if (row < n) {
                wv[i] = *reinterpret_cast<const uint4 *>(wm + (size_t)row * words + seg * 4);
                sc[i] = qw_bf16(sm[(size_t)row * groups + g]);
                bi[i] = qw_bf16(bm[(size_t)row * groups + g]);
            } else {
                wv[i] = make_uint4(0, 0, 0, 0);
                sc[i] = 0.0f;
                bi[i] = 0.0f;
            }
        }
#pragma unroll
        for (int t = 0; t < QD_MAXT; t++) {
            if (t < nt) {
                float xs[32];
                const float4 *xv = reinterpret_cast<const float4 *>(xp[t] + seg * 32);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float4 v = xv[q];
                    xs[4 * q] = v.x; xs[4 * q + 1] = v.y; xs[4 * q + 2] = v.z; xs[4 * q + 3] = v.w;
                }
                if (SWIGLU) {
                    const float4 *uv = reinterpret_cast<const float4 *>(up[t] + seg * 32);
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        const float4 v = uv[q];
                        xs[4 * q] = qw_silu(xs[4 * q]) * v.x;
                        xs[4 * q + 1] = qw_silu(xs[4 * q + 1]) * v.y;
                        xs[4 * q + 2] = qw_silu(xs[4 * q + 2]) * v.z;
                        xs[4 * q + 3] = qw_silu(xs[4 * q + 3]) * v.w;
                    }
                }
                float xsum = 0.0f;
#pragma unroll
                for (int q = 0; q < 32; q++) xsum += xs[q];
#pragma unroll
                for (int i = 0; i < QD_RIT; i++) {
                    float d = qw_dot8_q(wv[i].x, xs, 0.0f);
                    d = qw_dot8_q(wv[i].y, xs + 8, d);
                    d = qw_dot8_q(wv[i].z, xs + 16, d);
                    d = qw_dot8_q(wv[i].w, xs + 24, d);
                    acc[t][i] = __builtin_fmaf(sc[i], d, acc[t][i]);
                    acc[t][i] = __builtin_fmaf(bi[i], xsum, acc[t][i]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < QD_MAXT; t++) {
#pragma unroll
        for (int i = 0; i < QD_RIT; i++) {
            const float v = qw_xor_sum<LPR>(acc[t][i]);
            const int row = row0 + slot + SLOTS * i;
            if (t < nt && lr == 0 && row < n) yp[t][row] = v;
        }
    }
}

template <int G, bool SWIGLU>
__device__ __forceinline__ void qd_rows_k(int k, const uint32_t *wm, const uint16_t *sm, const uint16_t *bm,
                                          int n, int row0, int nt, const float *const *xp,
                                          const float *const *up, float *const *yp)
{
    switch (qd_lpr(k)) {
    case 64: qd_rows<G, 64, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    case 32: qd_rows<G, 32, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    case 16: qd_rows<G, 16, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    case 8:  qd_rows<G, 8, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    case 4:  qd_rows<G, 4, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    case 2:  qd_rows<G, 2, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    default: qd_rows<G, 1, SWIGLU>(wm, sm, bm, n, k, row0, nt, xp, up, yp); break;
    }
}

// Order-R dot of one bf16 row with up to `nt` token rows; one wave.  Chunk
// partials meet in `part` (this wave's slice) and lane t adds token t's.
__device__ __forceinline__ void qd_router_row(const uint16_t *__restrict__ wr, const float *__restrict__ x,
                                              int k, int nt, float (*part)[QD_MAXT], float *y, int ystride)
{
    const int lane = threadIdx.x & 63, nch = k / 64;
    for (int c = lane; c < nch; c += 64) {
        float p[QD_MAXT];
#pragma unroll
        for (int t = 0; t < QD_MAXT; t++) p[t] = 0.0f;
        const uint4 *wv = reinterpret_cast<const uint4 *>(wr + c * 64);
        for (int q = 0; q < 8; q++) {
            const uint4 ww = wv[q];
            const uint32_t wd[4] = {ww.x, ww.y, ww.z, ww.w};
            float wf[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                wf[2 * j] = __uint_as_float(wd[j] << 16);
                wf[2 * j + 1] = __uint_as_float(wd[j] & 0xFFFF0000u);
            }
#pragma unroll
            for (int t = 0; t < QD_MAXT; t++) {
                if (t < nt) {
                    const float4 *xv = reinterpret_cast<const float4 *>(x + (size_t)t * k + c * 64 + q * 8);
                    const float4 a = xv[0], b = xv[1];
                    float s = p[t];
                    s = __builtin_fmaf(wf[0], a.x, s);
                    s = __builtin_fmaf(wf[1], a.y, s);
                    s = __builtin_fmaf(wf[2], a.z, s);
                    s = __builtin_fmaf(wf[3], a.w, s);
                    s = __builtin_fmaf(wf[4], b.x, s);
                    s = __builtin_fmaf(wf[5], b.y, s);
                    s = __builtin_fmaf(wf[6], b.z, s);
                    s = __builtin_fmaf(wf[7], b.w, s);
                    p[t] = s;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < QD_MAXT; t++) part[c][t] = p[t];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    if (lane < nt) {
        float total = part[0][lane];
        for (int c = 1; c < nch; c++) total = total + part[c][lane];
        y[(size_t)lane * ystride] = total;
    }
    __builtin_amdgcn_wave_barrier();
}

// Returns true in every thread of the workgroup that arrived last at *ctr
// (of `expect`); that workgroup also resets the counter.
__device__ __forceinline__ bool qd_last_arrival(int *ctr, int expect)
{
    __shared__ int last;
    // Every wave publishes its own stores at agent scope before the count.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = old == expect - 1;
        if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return last;
}

// Route every token (one wave per token), then list the union of selected
// experts, ascending, and for each the pairs t*K + k that use it, in pair
// order.
__device__ void qd_route_all(const QdArgs &a)
{
    __shared__ int picks[QD_MAXU];
    __shared__ int mark[QWK_ROUTE_MAX_E];
    __shared__ int upos[QWK_ROUTE_MAX_E];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int E = a.m.E, K = a.m.K;
    for (int e = t; e < E; e += QD_THREADS) mark[e] = 0;
    for (int r = wave; r < a.rows; r += QD_WAVES) {
        // The same wave routine as the standalone route kernel.
        float v[QWK_ROUTE_MAX_E / 64];
        const float *l = a.logits + (size_t)r * E;
        float m = -__builtin_huge_valf();
#pragma unroll
        for (int j = 0; j < QWK_ROUTE_MAX_E / 64; j++) {
            const int e = lane + 64 * j;
            v[j] = e < E ? l[e] : -__builtin_huge_valf();
            m = fmaxf(m, v[j]);
        }
        m = qw_wave_max(m);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < QWK_ROUTE_MAX_E / 64; j++) {
            const int e = lane + 64 * j;
            if (e < E) { v[j] = qw_exp_spec(v[j] - m); s = s + v[j]; }
        }
        s = qw_xor_sum<64>(s);
#pragma unroll
        for (int j = 0; j < QWK_ROUTE_MAX_E / 64; j++) {
            const int e = lane + 64 * j;
            v[j] = e < E ? v[j] / s : -2.0f;
        }
        float mine_w = 0.0f;
        int mine_i = 0;
        for (int n = 0; n < K; n++) {
            float bv = -2.0f;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < QWK_ROUTE_MAX_E / 64; j++)
                if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
            qw_wave_argmax(bv, bi);
#pragma unroll
            for (int j = 0; j < QWK_ROUTE_MAX_E / 64; j++)
                if (lane + 64 * j == bi) v[j] = -1.0f;
            if (lane == n) { mine_w = bv; mine_i = bi; }
        }
        float wsum = 0.0f;
        for (int n = 0; n < K; n++) wsum = wsum + __shfl(mine_w, n, 64);
        if (lane < K) {
            a.idx[(size_t)r * K + lane] = mine_i;
            a.w[(size_t)r * K + lane] = a.m.norm ? mine_w / wsum : mine_w;
            picks[r * K + lane] = mine_i;
        }
    }
    __syncthreads();
    const int npk = a.rows * K;
    for (int p = t; p < npk; p += QD_THREADS) mark[picks[p]] = 1;
    __syncthreads();
    if (t == 0) {
        int u = 0;
        for (int e = 0; e < E; e++) {
            if (mark[e]) { upos[e] = u; qd_uexp(a)[u] = e; qd_ucnt(a)[u] = 0; u++; }
        }
        for (int p = 0; p < npk; p++) {
            const int uu = upos[picks[p]];
            qd_upair(a)[uu * a.rows + qd_ucnt(a)[uu]++] = p;
        }
        a.uinfo[0] = u;
    }
    __syncthreads();
}

template <int G>
__global__ __launch_bounds__(QD_THREADS) void k_decode_front(QdArgs a)
{
    __shared__ float part[QD_WAVES][QD_MAXCH][QD_MAXT];
    __shared__ const float *xp[QD_MAXT];
    __shared__ float *yp[QD_MAXT];
    const int wave = threadIdx.x >> 6, b = blockIdx.x;
    const int H = a.m.H, E = a.m.E, SI = a.m.SI;
    if (b < a.n_router_wg) {
        // Router rows, plus the shared gate logit as row E.
        const int o = b * QD_WAVES + wave;
        if (o < E)
            qd_router_row(a.m.router + (size_t)o * H, a.x, H, a.rows, part[wave], a.logits + o, E);
        else if (o == E)
            qd_router_row(a.m.sh_gate_w, a.x, H, a.rows, part[wave], a.g1, 1);
    } else {
        // Shared gate (z = 0) and up (z = 1) rows.
        const int sb = b - a.n_router_wg;
        const int half = a.n_shared_wg / 2;
        const int z = sb >= half ? 1 : 0;
        const int row0 = ((sb - z * half) * QD_WAVES + wave) * (qd_rows_per_wg(H) / QD_WAVES);
        if (threadIdx.x < QD_MAXT) {
            const int t = threadIdx.x;
            xp[t] = a.x + (size_t)min(t, a.rows - 1) * H;
            yp[t] = a.shgu + ((size_t)min(t, a.rows - 1) * 2 + z) * SI;
        }
        __syncthreads();
        const qwk_q4 q = z ? a.m.sh_up : a.m.sh_gate;
        if (row0 < SI) qd_rows_k<G, false>(H, q.w, q.s, q.b, SI, row0, a.rows, xp, nullptr, yp);
    }
    if (qd_last_arrival(a.ctr, gridDim.x)) qd_route_all(a);
}

template <int G>
__global__ __launch_bounds__(QD_THREADS) void k_decode_experts(QdArgs a)
{
    __shared__ const float *xp[QD_MAXT];
    __shared__ const float *upp[QD_MAXT];
    __shared__ float *yp[QD_MAXT];
    const int wave = threadIdx.x >> 6, b = blockIdx.x;
    const int H = a.m.H, I = a.m.I, SI = a.m.SI, K = a.m.K;
    const int ngu = a.umax * a.n_gu_wg_per_u;
    if (b < ngu) {
        const int u = b / a.n_gu_wg_per_u, rb = b % a.n_gu_wg_per_u;
        if (u >= min(a.uinfo[0], a.umax)) return;
        const int e = qd_uexp(a)[u], nt = min(qd_ucnt(a)[u], a.rows);
        if (e < 0 || e >= a.m.E || nt < 1) return;
        // Split banks: z = gate / up, each I rows; fused: one bank of 2I rows.
        const int nz = a.m.split ? 2 : 1, nrow = a.m.split ? I : 2 * I;
        const int per_z = a.n_gu_wg_per_u / nz;
        const int z = rb / per_z;
        const int row0 = ((rb % per_z) * QD_WAVES + wave) * (qd_rows_per_wg(H) / QD_WAVES);
        if (threadIdx.x < QD_MAXT) {
            const int t = threadIdx.x;
            const int p = min(max(qd_upair(a)[u * a.rows + min(t, nt - 1)], 0), a.rows * K - 1);
            xp[t] = a.x + (size_t)(p / K) * H;
            yp[t] = a.gu + (size_t)p * 2 * I + z * I;
        }
        __syncthreads();
        const qwk_q4 q = a.m.split ? (z ? a.m.up : a.m.gate) : a.m.gate_up;
        const size_t words = H / 8, groups = H / G;
        if (row0 < nrow)
            qd_rows_k<G, false>(H, q.w + (size_t)e * nrow * words, q.s + (size_t)e * nrow * groups,
                                q.b + (size_t)e * nrow * groups, nrow, row0, nt, xp, nullptr, yp);
    } else {
        // The shared expert's down projection, SwiGLU on load.
        const int rb = b - ngu;
        const int row0 = (rb * QD_WAVES + wave) * (qd_rows_per_wg(SI) / QD_WAVES);
        if (threadIdx.x < QD_MAXT) {
            const int t = min((int)threadIdx.x, a.rows - 1);
            xp[threadIdx.x] = a.shgu + (size_t)t * 2 * SI;
            upp[threadIdx.x] = a.shgu + (size_t)t * 2 * SI + SI;
            yp[threadIdx.x] = a.shout + (size_t)t * H;
        }
        __syncthreads();
        if (row0 < H)
            qd_rows_k<G, true>(SI, a.m.sh_down.w, a.m.sh_down.s, a.m.sh_down.b, H, row0, a.rows, xp, upp, yp);
    }
}

template <int G>
__global__ __launch_bounds__(QD_THREADS) void k_decode_down(QdArgs a)
{
    __shared__ const float *xp[QD_MAXT];
    __shared__ const float *upp[QD_MAXT];
    __shared__ float *yp[QD_MAXT];
    const int wave = threadIdx.x >> 6, b = blockIdx.x;
    const int H = a.m.H, I = a.m.I, K = a.m.K;
    const int u = b / a.nrb, rb = b % a.nrb;
    const int U = min(a.uinfo[0], a.umax);
    if (u >= U) return;
    const int e = qd_uexp(a)[u], nt = min(qd_ucnt(a)[u], a.rows);
    const bool ok = e >= 0 && e < a.m.E && nt >= 1;
    const int rpw = qd_rows_per_wg(I);
    const int row0 = rb * rpw + wave * (rpw / QD_WAVES);
    if (threadIdx.x < QD_MAXT) {
        const int t = threadIdx.x;
        const int p = ok ? min(max(qd_upair(a)[u * a.rows + min(t, nt - 1)], 0), a.rows * K - 1) : 0;
        xp[t] = a.gu + (size_t)p * 2 * I;
        upp[t] = a.gu + (size_t)p * 2 * I + I;
        yp[t] = a.ey + (size_t)p * H;
    }
    __syncthreads();
    const size_t words = I / 8, groups = I / G;
    if (ok && row0 < H)
        qd_rows_k<G, true>(I, a.m.down.w + (size_t)e * H * words, a.m.down.s + (size_t)e * H * groups,
                           a.m.down.b + (size_t)e * H * groups, H, row0, nt, xp, upp, yp);
    if (qd_last_arrival(a.ctr + 4 + rb, U)) {
        // Combine this block of output rows for every token.
        const int h0 = rb * rpw, h1 = min(H, h0 + rpw);
        const int span = h1 - h0;
        for (int i = threadIdx.x; i < a.rows * span; i += QD_THREADS) {
            const int t = i / span, h = h0 + i % span;
            float acc = a.shout[(size_t)t * H + h] * qw_sigmoid(a.g1[t]);
            for (int k = 0; k < K; k++)
                acc = __builtin_fmaf(a.w[(size_t)t * K + k], a.ey[((size_t)t * K + k) * H + h], acc);
            a.out[(size_t)t * H + h] = acc;
        }
    }
}

extern "C" size_t qwk_moe_decode_scratch(const qwk_moe *M, int rows)
{
    return qd_layout(M, rows).total;
}

extern "C" int qwk_moe_decode_counters(const qwk_moe *M)
{
    return 4 + qd_layout(M, 1).nrb;
}

template <int G>
static int qd_launch(hipStream_t s, QdArgs &a, hipEvent_t *ev)
{
    const dim3 blk(QD_THREADS);
    if (ev) (void)hipEventRecord(ev[0], s);
    hipLaunchKernelGGL(k_decode_front<G>, dim3(a.n_router_wg + a.n_shared_wg), blk, 0, s, a);
    if (ev) (void)hipEventRecord(ev[1], s);
    hipLaunchKernelGGL(k_decode_experts<G>, dim3(a.umax * a.n_gu_wg_per_u + a.n_shdown_wg), blk, 0, s, a);
    if (ev) (void)hipEventRecord(ev[2], s);
    hipLaunchKernelGGL(k_decode_down<G>, dim3(a.umax * a.nrb), blk, 0, s, a);
    if (ev) (void)hipEventRecord(ev[3], s);
    return (int)hipGetLastError();
}

extern "C" int qwk_moe_decode(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                              const qwk_moe *M, int rows, void *scratch, size_t scratch_bytes,
                              int *counters, int ncounters, hipEvent_t *ev)
{
    if (rows < 1 || rows > QWK_DECODE_MAX_ROWS || M->K < 1 || M->K > QWK_ROUTE_MAX_K ||
        M->E < M->K || M->E > QWK_ROUTE_MAX_E || M->H % 64 || M->I % 32 || M->SI % 32 ||
        M->H > QWK_DMAT_MAX_K || (M->group != 32 && M->group != 64 && M->group != 128) ||
        M->H % M->group || M->I % M->group || M->SI % M->group)
        return (int)hipErrorInvalidValue;
    const QdLayout L = qd_layout(M, rows);
    if (scratch_bytes < L.total || ((uintptr_t)x & 15u) || ncounters < 4 + L.nrb)
        return (int)hipErrorInvalidValue;
    char *S = (char *)scratch;
    QdArgs a;
    a.m = *M;
    a.x = x; a.out = out; a.idx = idx; a.w = w; a.rows = rows;
    a.umax = rows * M->K < M->E ? rows * M->K : M->E;
    a.nrb = L.nrb;
    a.n_router_wg = (M->E + 1 + QD_WAVES - 1) / QD_WAVES;
    const int rpw_h = qd_rows_per_wg(M->H);
    a.n_shared_wg = 2 * ((M->SI + rpw_h - 1) / rpw_h);
    const int nz = M->split ? 2 : 1, nrow = M->split ? M->I : 2 * M->I;
    a.n_gu_wg_per_u = nz * ((nrow + rpw_h - 1) / rpw_h);
    const int rpw_si = qd_rows_per_wg(M->SI);
    a.n_shdown_wg = (M->H + rpw_si - 1) / rpw_si;
    a.ctr = counters;
    a.logits = (float *)(S + L.logits);
    a.g1 = (float *)(S + L.g1);
    a.shgu = (float *)(S + L.shgu);
    a.shout = (float *)(S + L.shout);
    a.uinfo = (int *)(S + L.uinfo);
    a.gu = (float *)(S + L.gu);
    a.ey = (float *)(S + L.ey);
    switch (M->group) {
    case 32: return qd_launch<32>(s, a, ev);
    case 64: return qd_launch<64>(s, a, ev);
    default: return qd_launch<128>(s, a, ev);
    }
}
