// qw_decode.hip -- the MoE block at decode (1..8 tokens) in three launches,
// with no communication between workgroups inside a launch.
//
//   front    router logits (order R) for every expert and the shared
//            expert's gate logit; the shared expert's gate and up rows, a
//            wave taking the same rows of both, and its SwiGLU activation
//   experts  every workgroup first routes every token itself from the
//            logits (softmax, top-K, renormalise: cheap, and it saves a
//            launch and any cross-workgroup handoff) and lists the union of
//            the selected experts; then the gate and up rows of one selected
//            expert for every token routed to it -- each weight byte read
//            once -- and their SwiGLU activation; workgroup 0 writes idx / w
//   down     per (block of output rows, token): the down rows of the shared
//            expert and of each of the token's K experts, and the combine in
//            registers: sigmoid(g) * shared + sum_k w_k * y_k, an fma chain
//            in slot order
//
// A lane issues all its weight loads for a matrix (or a batch of matrices)
// before its first multiply, so each wave keeps those reads in flight at once.
#include "qw_device.h"
#include "qw_kernels.h"

#define QD_MAXT QWK_DECODE_MAX_ROWS
#define QD_MAXU (QWK_DECODE_MAX_ROWS * QWK_ROUTE_MAX_K)
#define QD_MAXCH (QWK_DMAT_MAX_K / 64)
#define QD_WAVES 4

static __host__ __device__ int qd_lpr(int k)
{
    const int S = k / 32;
    int l = 1;
    while (l < 64 && S % (2 * l) == 0) l *= 2;
    return l;
}

static int qd_splmax(int spl) { return spl <= 4 ? spl : 8; }
// Row slots a lane carries per matrix: fewer as segments per lane grow.
static __host__ __device__ constexpr int qd_rit(int splmax) { return splmax <= 2 ? 2 : 1; }

struct QdLayout {
    size_t logits, g1, shact, act, total;
};

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

static QdLayout qd_layout(const qwk_moe *M, int rows)
{
    QdLayout L;
    size_t o = 0;
    L.logits = o; o += al((size_t)rows * M->E * 4);
    L.g1 = o;     o += al((size_t)rows * 4);
    L.shact = o;  o += al((size_t)rows * M->SI * 4);
    L.act = o;    o += al((size_t)rows * M->K * M->I * 4);
    L.total = o;
    return L;
}

struct QdArgs {
    qwk_moe m;
    const float *x;
    float *out;
    int32_t *idx;
    float *w;
    int rows, umax, lgG;
    int n_router_wg, n_shared_wg;   // front
    int gu_wg_per_u;                // experts
    int down_rows_per_wg, n_down_rb;
    float *logits, *g1, *shact, *act;
};

// ---- gate and up rows with SwiGLU -----------------------------------------------
//
// Rows row0 + slot + SLOTS*i (i < RIT) of a gate matrix and the same rows of
// an up matrix (k inputs, LPR lanes to a row) against up to QD_MAXT inputs
// xp[t]: yp[t][row] = silu(gate . x_t) * (up . x_t).  A row's k/32 segments of
// 16 bytes go to its lanes round-robin; segment s lies in group (32 s) >> lgG.
template <int LPR, int SPLMAX, int RIT>
__device__ __forceinline__ void qd_glu_rows(const qwk_q4 gm, const qwk_q4 um, int n, int k, int lgG, int row0,
                                            int nt, const float *const *xp, float *const *yp)
{
    constexpr int SLOTS = 64 / LPR;
    const int lane = threadIdx.x & 63, slot = lane / LPR, lr = lane % LPR;
    const int words = k / 8, groups = k >> lgG;
    const int spl = (k / 32) / LPR;
    uint4 wv[2][SPLMAX][RIT];
    float sc[2][SPLMAX][RIT], bi[2][SPLMAX][RIT];
#pragma unroll
    for (int z = 0; z < 2; z++) {
        const qwk_q4 q = z ? um : gm;
#pragma unroll
        for (int j = 0; j < SPLMAX; j++) {
            const int seg = j * LPR + lr, g = (seg * 32) >> lgG;
#pragma unroll
            for (int i = 0; i < RIT; i++) {
                const int row = row0 + slot + SLOTS * i;
                if (j < spl && row < n) {
                    wv[z][j][i] = *reinterpret_cast<const uint4 *>(q.w + (size_t)row * words + seg * 4);
                    sc[z][j][i] = qw_bf16(q.s[(size_t)row * groups + g]);
                    bi[z][j][i] = qw_bf16(q.b[(size_t)row * groups + g]);
                } else {
                    wv[z][j][i] = make_uint4(0, 0, 0, 0);
                    sc[z][j][i] = 0.0f;
                    bi[z][j][i] = 0.0f;
                }
            }
        }
    }
#pragma unroll 1
    for (int t = 0; t < nt; t++) {
        float acc[2][RIT];
#pragma unroll
        for (int i = 0; i < RIT; i++) acc[0][i] = acc[1][i] = 0.0f;
#pragma unroll
        for (int j = 0; j < SPLMAX; j++) {
            if (j < spl) {
                const int seg = j * LPR + lr;
                float xs[32];
                const float4 *xv = reinterpret_cast<const float4 *>(xp[t] + seg * 32);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float4 v = xv[q];
                    xs[4 * q] = v.x; xs[4 * q + 1] = v.y; xs[4 * q + 2] = v.z; xs[4 * q + 3] = v.w;
                }
                float xsum = 0.0f;
#pragma unroll
                for (int q = 0; q < 32; q++) xsum += xs[q];
#pragma unroll
                for (int z = 0; z < 2; z++) {
#pragma unroll
                    for (int i = 0; i < RIT; i++) {
                        float d = qw_dot8_q(wv[z][j][i].x, xs, 0.0f);
                        d = qw_dot8_q(wv[z][j][i].y, xs + 8, d);
                        d = qw_dot8_q(wv[z][j][i].z, xs + 16, d);
                        d = qw_dot8_q(wv[z][j][i].w, xs + 24, d);
                        acc[z][i] = __builtin_fmaf(sc[z][j][i], d, acc[z][i]);
                        acc[z][i] = __builtin_fmaf(bi[z][j][i], xsum, acc[z][i]);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const float g = qw_xor_sum<LPR>(acc[0][i]);
            const float u = qw_xor_sum<LPR>(acc[1][i]);
            const int row = row0 + slot + SLOTS * i;
            if (lr == 0 && row < n) yp[t][row] = qw_silu(g) * u;
        }
    }
}

// ---- front: router logits and the shared expert's gate / up ----------------------

// Order-R dot of one bf16 row with nt token rows (one wave): lane l computes
// the fmaf chains of chunks l, l+64, ...; the chunk partials are then added
// left to right, read lane by lane with readlane, so every lane holds the
// total.
__device__ __forceinline__ void qd_router_row(const uint16_t *__restrict__ wr, const float *__restrict__ x,
                                              int k, int nt, float *y, int ystride)
{
    constexpr int CPL = QD_MAXCH / 64;      // chunks per lane at most
    const int lane = threadIdx.x & 63, nch = k / 64;
#pragma unroll 1
    for (int t = 0; t < nt; t++) {
        float p[CPL];
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int c = lane + 64 * j;
            float s = 0.0f;
            if (c < nch) {
                const uint4 *wp = reinterpret_cast<const uint4 *>(wr + c * 64);
                const float4 *xv = reinterpret_cast<const float4 *>(x + (size_t)t * k + c * 64);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const uint4 w = wp[q];
                    const float4 a = xv[2 * q], b = xv[2 * q + 1];
                    s = __builtin_fmaf(__uint_as_float(w.x << 16), a.x, s);
                    s = __builtin_fmaf(__uint_as_float(w.x & 0xFFFF0000u), a.y, s);
                    s = __builtin_fmaf(__uint_as_float(w.y << 16), a.z, s);
                    s = __builtin_fmaf(__uint_as_float(w.y & 0xFFFF0000u), a.w, s);
                    s = __builtin_fmaf(__uint_as_float(w.z << 16), b.x, s);
                    s = __builtin_fmaf(__uint_as_float(w.z & 0xFFFF0000u), b.y, s);
                    s = __builtin_fmaf(__uint_as_float(w.w << 16), b.z, s);
                    s = __builtin_fmaf(__uint_as_float(w.w & 0xFFFF0000u), b.w, s);
                }
            }
            p[j] = s;
        }
        float total = qw_lane(p[0], 0);
#pragma unroll
        for (int j = 0; j < CPL; j++)
            for (int l = j == 0 ? 1 : 0; l < 64 && 64 * j + l < nch; l++) total = total + qw_lane(p[j], l);
        if (lane == 0) y[(size_t)t * ystride] = total;
    }
}

template <int LPR, int SPLMAX>
__global__ __launch_bounds__(QD_WAVES * 64) void k_decode_front(QdArgs a)
{
    __shared__ const float *xp[QD_MAXT];
    __shared__ float *yp[QD_MAXT];
    const int wave = threadIdx.x >> 6, b = blockIdx.x;
    const int H = a.m.H, E = a.m.E, SI = a.m.SI;
    if (b < a.n_router_wg) {
        const int o = b * QD_WAVES + wave;
        if (o < E)
            qd_router_row(a.m.router + (size_t)o * H, a.x, H, a.rows, a.logits + o, E);
        else if (o == E)
            qd_router_row(a.m.sh_gate_w, a.x, H, a.rows, a.g1, 1);
        return;
    }
    constexpr int RIT = qd_rit(SPLMAX);
    constexpr int RPW = (64 / LPR) * RIT;
    const int row0 = ((b - a.n_router_wg) * QD_WAVES + wave) * RPW;
    if (threadIdx.x < QD_MAXT) {
        const int t = min((int)threadIdx.x, a.rows - 1);
        xp[threadIdx.x] = a.x + (size_t)t * H;
        yp[threadIdx.x] = a.shact + (size_t)t * SI;
    }
    __syncthreads();
    if (row0 < SI)
        qd_glu_rows<LPR, SPLMAX, RIT>(a.m.sh_gate, a.m.sh_up, SI, H, a.lgG, row0, a.rows, xp, yp);
}

// ---- experts: routing in the prologue, then gate / up of one selected expert ----

struct QdRoute {
    int U;
    int picks[QD_MAXU];
    float pw[QD_MAXU];
    int uexp[QD_MAXU];
    int ucnt[QD_MAXU];
    int ustart[QD_MAXU];
    int upair[QD_MAXU];       // pairs grouped by unique expert, ascending pair index
    int mark[QWK_ROUTE_MAX_E];
    int scratch[QD_WAVES][4 * QWK_ROUTE_MAX_K];
};

// Routes every token (a wave per token) with the arithmetic of the
// standalone route kernel, then builds the union of selected experts with,
// for each, its pairs in ascending order.  One token's picks are distinct, so
// for one token the union is the picks themselves, in pick order.
template <int PL>
__device__ void qd_route_all(const QdArgs &a, QdRoute &R)
{
    const int t = threadIdx.x, nthr = blockDim.x, wave = t >> 6, lane = t & 63, nw = nthr >> 6;
    const int E = a.m.E, K = a.m.K;
    for (int r = wave; r < a.rows; r += nw) {
        int pi;
        float pw;
        qw_route_wave<PL>(a.logits + (size_t)r * E, E, K, a.m.norm, lane, &pi, &pw, R.scratch[wave]);
        if (lane < K) {
            R.picks[r * K + lane] = pi;
            R.pw[r * K + lane] = pw;
        }
    }
    __syncthreads();
    if (a.rows == 1) {
        if (t < K) {
            R.uexp[t] = R.picks[t];
            R.ucnt[t] = 1;
            R.ustart[t] = t;
            R.upair[t] = t;
        }
        if (t == 0) R.U = K;
        __syncthreads();
        return;
    }
    for (int e = t; e < E; e += nthr) R.mark[e] = 0;
    __syncthreads();
    const int npk = a.rows * K;
    for (int p = t; p < npk; p += nthr) R.mark[R.picks[p]] = 1;
    __syncthreads();
    // Compact the marked experts in ascending order, 64 at a time with ballots.
    if (wave == 0) {
        int base = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const bool on = e < E && R.mark[e];
            const unsigned long long bal = __ballot(on);
            if (on) R.uexp[base + __popcll(bal & ((1ull << lane) - 1ull))] = e;
            base += __popcll(bal);
        }
        if (lane == 0) R.U = base;
    }
    __syncthreads();
    for (int u = t; u < R.U; u += nthr) {
        const int e = R.uexp[u];
        int c = 0;
        for (int p = 0; p < npk; p++) c += R.picks[p] == e;
        R.ucnt[u] = c;
    }
    __syncthreads();
    if (t == 0) {
        int s = 0;
        for (int u = 0; u < R.U; u++) { R.ustart[u] = s; s += R.ucnt[u]; }
    }
    __syncthreads();
    for (int u = t; u < R.U; u += nthr) {
        const int e = R.uexp[u];
        int c = R.ustart[u];
        for (int p = 0; p < npk; p++)
            if (R.picks[p] == e) R.upair[c++] = p;
    }
    __syncthreads();
}

template <int LPR, int SPLMAX, int PL>
__global__ __launch_bounds__(QD_WAVES * 64) void k_decode_experts(QdArgs a)
{
    __shared__ QdRoute R;
    __shared__ const float *xp[QD_MAXT];
    __shared__ float *yp[QD_MAXT];
    const int wave = threadIdx.x >> 6, b = blockIdx.x;
    const int H = a.m.H, I = a.m.I, K = a.m.K;
    const int u = b / a.gu_wg_per_u, rb = b % a.gu_wg_per_u;
    qd_route_all<PL>(a, R);
    if (b == 0)
        for (int p = threadIdx.x; p < a.rows * K; p += blockDim.x) {
            a.idx[p] = R.picks[p];
            a.w[p] = R.pw[p];
        }
    if (u >= R.U) return;
    const int e = R.uexp[u], nt = R.ucnt[u], p0 = R.ustart[u];
    constexpr int RIT = qd_rit(SPLMAX);
    constexpr int RPW = (64 / LPR) * RIT;
    const int row0 = (rb * QD_WAVES + wave) * RPW;
    if (threadIdx.x < QD_MAXT) {
        const int t = threadIdx.x;
        const int p = R.upair[p0 + min(t, nt - 1)];
        xp[t] = a.x + (size_t)(p / K) * H;
        yp[t] = a.act + (size_t)p * I;
    }
    __syncthreads();
    // Split banks: gate and up [E, I, H]; fused: gate_up [E, 2I, H], gate rows
    // first, so up row r of expert e is row I + r of its slice.
    const size_t words = H / 8, groups = H >> a.lgG;
    qwk_q4 gm, um;
    if (a.m.split) {
        const size_t off = (size_t)e * I;
        gm = {a.m.gate.w + off * words, a.m.gate.s + off * groups, a.m.gate.b + off * groups};
        um = {a.m.up.w + off * words, a.m.up.s + off * groups, a.m.up.b + off * groups};
    } else {
        const size_t off = (size_t)e * 2 * I;
        gm = {a.m.gate_up.w + off * words, a.m.gate_up.s + off * groups, a.m.gate_up.b + off * groups};
        um = {gm.w + (size_t)I * words, gm.s + (size_t)I * groups, gm.b + (size_t)I * groups};
    }
    if (row0 < I) qd_glu_rows<LPR, SPLMAX, RIT>(gm, um, I, H, a.lgG, row0, nt, xp, yp);
}

// ---- down: the shared expert and every expert of a token, and the combine -------
//
// A workgroup owns RIT * 64/LPR output rows of one token; wave w computes those
// rows of matrix w, w + nw, ... (matrix 0 = the shared expert, matrix 1 + k =
// the token's k-th expert), so each wave has one round of loads in flight.
// The per-matrix rows meet in LDS and the combine runs in slot order.
#define QD_DOWN_MAXW 16
static __host__ __device__ constexpr int qd_down_rit(int splmax) { return splmax <= 2 ? 4 : splmax <= 4 ? 2 : 1; }

template <int LPR, int SPLMAX>
__global__ __launch_bounds__(QD_DOWN_MAXW * 64) void k_decode_down(QdArgs a)
{
    constexpr int RIT = qd_down_rit(SPLMAX);
    constexpr int SLOTS = 64 / LPR, RPG = SLOTS * RIT;
    __shared__ float ys[QWK_ROUTE_MAX_K + 1][RPG];
    const int H = a.m.H, I = a.m.I, SI = a.m.SI, K = a.m.K;
    const int rb = blockIdx.x % a.n_down_rb, t = blockIdx.x / a.n_down_rb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int slot = lane / LPR, lr = lane % LPR;
    const int row0 = rb * RPG;
    const int lgG = a.lgG;
    for (int m = wave; m <= K; m += nw) {
        const int kin = m == 0 ? SI : I;
        const int words = kin / 8, groups = kin >> lgG, spl = (kin / 32) / LPR;
        const uint32_t *wm = a.m.sh_down.w;
        const uint16_t *sm = a.m.sh_down.s, *bm = a.m.sh_down.b;
        const float *av = a.shact + (size_t)t * SI;
        if (m > 0) {
            const size_t e = (size_t)a.idx[t * K + m - 1];
            wm = a.m.down.w + e * H * words;
            sm = a.m.down.s + e * H * groups;
            bm = a.m.down.b + e * H * groups;
            av = a.act + ((size_t)t * K + m - 1) * I;
        }
        uint4 wv[SPLMAX][RIT];
        float sc[SPLMAX][RIT], bi[SPLMAX][RIT];
#pragma unroll
        for (int j = 0; j < SPLMAX; j++) {
            const int seg = j * LPR + lr, g = (seg * 32) >> lgG;
#pragma unroll
            for (int i = 0; i < RIT; i++) {
                const int row = row0 + slot + SLOTS * i;
                if (j < spl && row < H) {
                    wv[j][i] = *reinterpret_cast<const uint4 *>(wm + (size_t)row * words + seg * 4);
                    sc[j][i] = qw_bf16(sm[(size_t)row * groups + g]);
                    bi[j][i] = qw_bf16(bm[(size_t)row * groups + g]);
                } else {
                    wv[j][i] = make_uint4(0, 0, 0, 0);
                    sc[j][i] = 0.0f;
                    bi[j][i] = 0.0f;
                }
            }
        }
        float y[RIT];
#pragma unroll
        for (int i = 0; i < RIT; i++) y[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < SPLMAX; j++) {
            if (j < spl) {
                const int seg = j * LPR + lr;
                float xs[32];
                const float4 *xv = reinterpret_cast<const float4 *>(av + seg * 32);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float4 v = xv[q];
                    xs[4 * q] = v.x; xs[4 * q + 1] = v.y; xs[4 * q + 2] = v.z; xs[4 * q + 3] = v.w;
                }
                float xsum = 0.0f;
#pragma unroll
                for (int q = 0; q < 32; q++) xsum += xs[q];
#pragma unroll
                for (int i = 0; i < RIT; i++) {
                    float d = qw_dot8_q(wv[j][i].x, xs, 0.0f);
                    d = qw_dot8_q(wv[j][i].y, xs + 8, d);
                    d = qw_dot8_q(wv[j][i].z, xs + 16, d);
                    d = qw_dot8_q(wv[j][i].w, xs + 24, d);
                    y[i] = __builtin_fmaf(sc[j][i], d, y[i]);
                    y[i] = __builtin_fmaf(bi[j][i], xsum, y[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const float v = qw_xor_sum<LPR>(y[i]);
            if (lr == 0) ys[m][slot + SLOTS * i] = v;
        }
    }
    __syncthreads();
    // The combine: the shared term first, then an fma per slot, in order.
    for (int r = threadIdx.x; r < RPG; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= H) continue;
        float acc = ys[0][r] * qw_sigmoid(a.g1[t]);
        for (int k = 0; k < K; k++) acc = __builtin_fmaf(a.w[t * K + k], ys[1 + k][r], acc);
        a.out[(size_t)t * H + row] = acc;
    }
}

// ---- host side -------------------------------------------------------------------

extern "C" size_t qwk_moe_decode_scratch(const qwk_moe *M, int rows)
{
    return qd_layout(M, rows).total;
}

extern "C" int qwk_moe_decode_counters(const qwk_moe *M)
{
    (void)M;
    return 0;
}

template <int LPR, int SPLMAX>
static void launch_fe(hipStream_t s, QdArgs &a, hipEvent_t *ev)
{
    if (ev) (void)hipEventRecord(ev[0], s);
    hipLaunchKernelGGL((k_decode_front<LPR, SPLMAX>), dim3(a.n_router_wg + a.n_shared_wg),
                       dim3(QD_WAVES * 64), 0, s, a);
    if (ev) (void)hipEventRecord(ev[1], s);
    const dim3 grid(a.umax * a.gu_wg_per_u), blk(QD_WAVES * 64);
    if (a.m.E <= 256) hipLaunchKernelGGL((k_decode_experts<LPR, SPLMAX, 4>), grid, blk, 0, s, a);
    else if (a.m.E <= 512) hipLaunchKernelGGL((k_decode_experts<LPR, SPLMAX, 8>), grid, blk, 0, s, a);
    else hipLaunchKernelGGL((k_decode_experts<LPR, SPLMAX, 16>), grid, blk, 0, s, a);
    if (ev) (void)hipEventRecord(ev[2], s);
}

template <int LPR>
static bool launch_fe_spl(int splmax, hipStream_t s, QdArgs &a, hipEvent_t *ev)
{
    switch (splmax) {
    case 1: launch_fe<LPR, 1>(s, a, ev); return true;
    case 2: launch_fe<LPR, 2>(s, a, ev); return true;
    case 3: launch_fe<LPR, 3>(s, a, ev); return true;
    case 4: launch_fe<LPR, 4>(s, a, ev); return true;
    case 8: launch_fe<LPR, 8>(s, a, ev); return true;
    default: return false;
    }
}

template <int LPR, int SPLMAX>
static void launch_down(hipStream_t s, QdArgs &a)
{
    const int nw = a.m.K + 1 < QD_DOWN_MAXW ? a.m.K + 1 : QD_DOWN_MAXW;
    hipLaunchKernelGGL((k_decode_down<LPR, SPLMAX>), dim3(a.rows * a.n_down_rb), dim3(nw * 64), 0, s, a);
}

template <int LPR>
static bool launch_down_spl(int splmax, hipStream_t s, QdArgs &a)
{
    switch (splmax) {
    case 1: launch_down<LPR, 1>(s, a); return true;
    case 2: launch_down<LPR, 2>(s, a); return true;
    case 3: launch_down<LPR, 3>(s, a); return true;
    case 4: launch_down<LPR, 4>(s, a); return true;
    case 8: launch_down<LPR, 8>(s, a); return true;
    default: return false;
    }
}

extern "C" int qwk_moe_decode(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                              const qwk_moe *M, int rows, void *scratch, size_t scratch_bytes,
                              int *counters, int ncounters, hipEvent_t *ev)
{
    (void)counters; (void)ncounters;
    const int G = M->group;
    if (rows < 1 || rows > QWK_DECODE_MAX_ROWS || M->K < 1 || M->K > QWK_ROUTE_MAX_K ||
        M->E < M->K || M->E > QWK_ROUTE_MAX_E || M->H % 64 || M->I % 32 || M->SI % 32 ||
        M->H > QWK_DMAT_MAX_K || (G != 32 && G != 64 && G != 128) ||
        M->H % G || M->I % G || M->SI % G || ((uintptr_t)x & 15u))
        return (int)hipErrorInvalidValue;
    const QdLayout L = qd_layout(M, rows);
    if (scratch_bytes < L.total) return (int)hipErrorInvalidValue;
    // Lanes per row: k = H for the front and expert launches; for down one
    // width that divides the segment counts of both I and SI.
    const int lpr_h = qd_lpr(M->H);
    int lpr_d = qd_lpr(M->I);
    const int lpr_si = qd_lpr(M->SI);
    if (lpr_si < lpr_d) lpr_d = lpr_si;
    const int kmax_d = M->I > M->SI ? M->I : M->SI;
    if ((M->H / 32) / lpr_h > 8 || (kmax_d / 32) / lpr_d > 8 || lpr_h < 2 || lpr_d < 2)
        return (int)hipErrorInvalidValue;
    const int spl_h = qd_splmax((M->H / 32) / lpr_h);
    const int spl_d = qd_splmax((kmax_d / 32) / lpr_d);

    char *S = (char *)scratch;
    QdArgs a;
    a.m = *M;
    a.x = x; a.out = out; a.idx = idx; a.w = w; a.rows = rows;
    a.umax = rows * M->K < M->E ? rows * M->K : M->E;
    a.lgG = G == 32 ? 5 : G == 64 ? 6 : 7;
    a.n_router_wg = (M->E + 1 + QD_WAVES - 1) / QD_WAVES;
    const int rpg_h = QD_WAVES * (64 / lpr_h) * qd_rit(spl_h);
    a.n_shared_wg = (M->SI + rpg_h - 1) / rpg_h;
    a.gu_wg_per_u = (M->I + rpg_h - 1) / rpg_h;
    a.down_rows_per_wg = qd_down_rit(spl_d) * (64 / lpr_d);
    a.n_down_rb = (M->H + a.down_rows_per_wg - 1) / a.down_rows_per_wg;
    a.logits = (float *)(S + L.logits);
    a.g1 = (float *)(S + L.g1);
    a.shact = (float *)(S + L.shact);
    a.act = (float *)(S + L.act);

    bool ok;
    switch (lpr_h) {
    case 2: ok = launch_fe_spl<2>(spl_h, s, a, ev); break;
    case 4: ok = launch_fe_spl<4>(spl_h, s, a, ev); break;
    case 8: ok = launch_fe_spl<8>(spl_h, s, a, ev); break;
    case 16: ok = launch_fe_spl<16>(spl_h, s, a, ev); break;
    case 32: ok = launch_fe_spl<32>(spl_h, s, a, ev); break;
    default: ok = launch_fe_spl<64>(spl_h, s, a, ev); break;
    }
    if (!ok) return (int)hipErrorInvalidValue;
    switch (lpr_d) {
    case 2: ok = launch_down_spl<2>(spl_d, s, a); break;
    case 4: ok = launch_down_spl<4>(spl_d, s, a); break;
    case 8: ok = launch_down_spl<8>(spl_d, s, a); break;
    case 16: ok = launch_down_spl<16>(spl_d, s, a); break;
    case 32: ok = launch_down_spl<32>(spl_d, s, a); break;
    default: ok = launch_down_spl<64>(spl_d, s, a); break;
    }
    if (ev) (void)hipEventRecord(ev[3], s);
    if (!ok) return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}
