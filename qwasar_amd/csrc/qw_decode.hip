// qw_decode.hip -- the MoE block at decode (1..8 tokens) in three launches,
// with no communication between workgroups inside a launch.
//
//   front    router logits (order R, fp32) for every expert and the shared
//            expert's gate logit; the input rows staged as q16 units
//   experts  the shared expert's gate / up rows (no routing needed), and, in
//            the other workgroups, routing of every token (softmax, top-K,
//            renormalise: cheap, and it saves a launch and any
//            cross-workgroup handoff) followed by the gate / up rows of one
//            selected expert for every token routed to it -- each weight
//            byte read once; the SwiGLU activations leave staged as q16
//            units; workgroup 0 writes idx / w
//   down     per (block of output rows, token): the down rows of the shared
//            expert and of each of the token's K experts, and the combine in
//            registers: sigmoid(g) * shared + sum_k w_k * y_k, an fma chain
//            in slot order
//
// The 4-bit products use the q16 dot (qw_unit_dot): staged activations are
// loaded straight into registers next to the weights, and a lane issues all
// its loads before its first multiply.
#include <hip/hip_ext.h>

#include "qw_device.h"
#include "qw_kernels.h"

#define QD_MAXT QWK_DECODE_MAX_ROWS
#define QD_MAXU (QWK_DECODE_MAX_ROWS * QWK_ROUTE_MAX_K)
#define QD_MAXCH (QWK_DMAT_MAX_K / 64)
#define QD_FRONT_WAVES 4
#define QD_GU_WAVES 16       // experts workgroup: 16 waves
#define QD_GU_MAXRPB (QD_GU_WAVES * 4)
#define QD_GU_LDS (48 * 1024)  // LDS for staged input vectors
#define QD_DOWN_MAXW 16
#define QD_DOWN_RIT 2        // down rows per lane slot

// Lanes per row for a row of `units` q16 units, and units per lane.
static __host__ __device__ constexpr int qd_lpr(int units) { return units >= 128 ? 64 : units >= 64 ? 32 : 16; }
static int qd_nul(int units, int lpr)
{
    const int n = (units + lpr - 1) / lpr;
    return n <= 4 ? n : n <= 8 ? 8 : -1;
}

struct QdLayout {
    size_t logits, g1, qx, qsh, qact, total;
};

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

static QdLayout qd_layout(const qwk_moe *M, int rows)
{
    QdLayout L;
    size_t o = 0;
    L.logits = o; o += al((size_t)rows * M->E * 4);
    L.g1 = o;     o += al((size_t)rows * 4);
    L.qx = o;     o += al((size_t)rows * (M->H / 16) * QW_Q16_BYTES);
    L.qsh = o;    o += al((size_t)rows * (M->SI / 16) * QW_Q16_BYTES);
    L.qact = o;   o += al((size_t)rows * M->K * (M->I / 16) * QW_Q16_BYTES);
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
    int n_router_wg;                // front
    int n_shared_wg, gu_wg_per_u;   // experts
    int tch;                        // input vectors per LDS pass
    int n_down_rb;                  // down
    float *logits, *g1;
    uint4 *qx, *qsh, *qact;         // q16 units: [vector][units][3]
};

// ---- front: router logits and the staged input ----------------------------------

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

__global__ __launch_bounds__(QD_FRONT_WAVES * 64) void k_decode_front(QdArgs a)
{
    const int wave = threadIdx.x >> 6, b = blockIdx.x;
    const int H = a.m.H, E = a.m.E;
    if (b < a.n_router_wg) {
        const int o = b * QD_FRONT_WAVES + wave;
        if (o < E)
            qd_router_row(a.m.router + (size_t)o * H, a.x, H, a.rows, a.logits + o, E);
        else if (o == E)
            qd_router_row(a.m.sh_gate_w, a.x, H, a.rows, a.g1, 1);
        return;
    }
    // one workgroup per token: a unit per thread
    const int t = b - a.n_router_wg, units = H / 16;
    for (int u = threadIdx.x; u < units; u += blockDim.x) {
        const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)t * H + 16 * u);
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = src[q];
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
        qw_q16_stage(v, a.qx + ((size_t)t * units + u) * 3);
    }
}

// ---- experts: gate / up rows with SwiGLU --------------------------------------------
//
// A workgroup owns RPB = QD_GU_WAVES * 64/LPR consecutive rows of one gate / up
// pair (the shared expert's, or one routed expert's) for nt input vectors.
// Lane (slot, lr) of wave w takes row row0 + w * 64/LPR + slot and its units
// lr, lr + LPR, ... (NUL of them), in both matrices; its weights stay in
// registers while the input vectors pass through LDS, up to `tch` at a time.
// The per-row results meet in LDS and leave as q16 units of the activation
// vectors.

// Copies staged vectors vin[t] (t < n; vector t when vin is NULL) of src,
// `units` units each, into LDS, with threads tid0.. of the workgroup.
__device__ __forceinline__ void qd_copy_vecs(uint4 *xs, const uint4 *src, const int *vin, int n, int units,
                                             int tid0, int nthr)
{
    const int per = units * 3;
    for (int i = threadIdx.x - tid0; i < n * per; i += nthr) {
        const int t = i / per, o = i % per;
        xs[i] = src[(size_t)(vin ? vin[t] : t) * per + o];
    }
}

template <int LPR, int NUL>
__device__ __forceinline__ void qd_glu_block(const qwk_q4 gm, const qwk_q4 um, int n, int k, int lgG, int row0,
                                             int nt, int tch, bool staged, uint4 *xs, const uint4 *src,
                                             const int *vin, const int *vout, uint4 *dst,
                                             float (*ys)[QD_GU_MAXRPB])
{
    constexpr int SL = 64 / LPR, RPB = QD_GU_WAVES * SL;
    static_assert(RPB % 16 == 0 && RPB <= QD_GU_MAXRPB, "rows per block");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, slot = lane / LPR, lr = lane % LPR;
    const int units = k / 16, words = k / 8, groups = k >> lgG;
    const int rl = wave * SL + slot, row = row0 + rl;
    uint2 wv[2][NUL];
    float sc[2][NUL], bi[2][NUL];
#pragma unroll
    for (int z = 0; z < 2; z++) {
        const qwk_q4 q = z ? um : gm;
#pragma unroll
        for (int j = 0; j < NUL; j++) {
            const int c = j * LPR + lr;
            if (row < n && c < units) {
                wv[z][j] = *reinterpret_cast<const uint2 *>(q.w + (size_t)row * words + 2 * c);
                sc[z][j] = qw_bf16(q.s[(size_t)row * groups + ((16 * c) >> lgG)]);
                bi[z][j] = qw_bf16(q.b[(size_t)row * groups + ((16 * c) >> lgG)]);
            } else {
                wv[z][j] = make_uint2(0, 0);
                sc[z][j] = bi[z][j] = 0.0f;
            }
        }
    }
    for (int t0 = 0; t0 < nt; t0 += tch) {
        const int tn = min(tch, nt - t0);
        if (!staged) {
            __syncthreads();
            qd_copy_vecs(xs, src, vin + t0, tn, units, 0, blockDim.x);
        }
        __syncthreads();
#pragma unroll 1
        for (int t = 0; t < tn; t++) {
            const uint4 *xt = xs + (size_t)t * units * 3;
            float acc[2] = {0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NUL; j++) {
                const int c = j * LPR + lr;
                if (c < units) {
                    const uint4 p0 = xt[3 * c], p1 = xt[3 * c + 1];
                    const uint4 rr = xt[3 * c + 2];
                    const float4 r = *reinterpret_cast<const float4 *>(&rr);
#pragma unroll
                    for (int z = 0; z < 2; z++)
                        acc[z] = qw_unit_dot(wv[z][j], p0, p1, r, sc[z][j], bi[z][j], acc[z]);
                }
            }
            const float g = qw_xor_sum<LPR>(acc[0]);
            const float u = qw_xor_sum<LPR>(acc[1]);
            if (lr == 0) ys[t0 + t][rl] = qw_silu(g) * u;
        }
    }
    __syncthreads();
    // one thread per (vector, unit) of this block's rows
    constexpr int upb = RPB / 16;
    const int outunits = n / 16;
    for (int i = threadIdx.x; i < nt * upb; i += blockDim.x) {
        const int t = i / upb, uu = i % upb;
        if (row0 + 16 * uu >= n) continue;
        float v[16];
#pragma unroll
        for (int q = 0; q < 16; q++) v[q] = ys[t][16 * uu + q];
        qw_q16_stage(v, dst + ((size_t)vout[t] * outunits + row0 / 16 + uu) * 3);
    }
}

struct QdRoute {
    int U;
    int picks[QD_MAXU];
    float pw[QD_MAXU];
    int uexp[QD_MAXU];
    int ucnt[QD_MAXU];
    int ustart[QD_MAXU];
    int upair[QD_MAXU];       // pairs grouped by unique expert, ascending pair index
    int mark[QWK_ROUTE_MAX_E];
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
        qw_route_wave<PL>(a.logits + (size_t)r * E, E, K, a.m.norm, lane, &pi, &pw);
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

// 8 waves per SIMD: two 16-wave workgroups per CU, which takes at most 64
// VGPRs and 78 SGPRs a wave (at 80 SGPRs a CU holds one).
template <int LPR, int NUL, int PL>
__global__ __launch_bounds__(QD_GU_WAVES * 64, 8) void k_decode_experts(QdArgs a)
{
    extern __shared__ uint4 xs[];     // [tch][units][3]
    __shared__ QdRoute R;
    __shared__ int vin[QD_MAXT], vout[QD_MAXT];
    __shared__ float ys[QD_MAXT][QD_GU_MAXRPB];
    constexpr int RPB = QD_GU_WAVES * (64 / LPR);
    const int b = blockIdx.x;
    const int H = a.m.H, I = a.m.I, K = a.m.K, SI = a.m.SI;
    const int xunits = H / 16;
    if (b < a.n_shared_wg) {
        if (threadIdx.x < QD_MAXT) vin[threadIdx.x] = vout[threadIdx.x] = threadIdx.x;
        __syncthreads();
        qd_glu_block<LPR, NUL>(a.m.sh_gate, a.m.sh_up, SI, H, a.lgG, b * RPB, a.rows, a.tch, false,
                               xs, a.qx, vin, vout, a.qsh, ys);
        return;
    }
    const int bb = b - a.n_shared_wg;
    const int u = bb / a.gu_wg_per_u, rb = bb % a.gu_wg_per_u;
    // One token: its input goes to LDS (waves 1..) while wave 0 routes.
    const bool one = a.rows == 1;
    if (one && threadIdx.x >= 64) qd_copy_vecs(xs, a.qx, nullptr, 1, xunits, 64, blockDim.x - 64);
    qd_route_all<PL>(a, R);
    if (bb == 0)
        for (int p = threadIdx.x; p < a.rows * K; p += blockDim.x) {
            a.idx[p] = R.picks[p];
            a.w[p] = R.pw[p];
        }
    if (u >= R.U) return;
    const int e = R.uexp[u], nt = R.ucnt[u], p0 = R.ustart[u];
    if (threadIdx.x < nt) {
        const int p = R.upair[p0 + threadIdx.x];
        vin[threadIdx.x] = p / K;
        vout[threadIdx.x] = p;
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
    qd_glu_block<LPR, NUL>(gm, um, I, H, a.lgG, rb * RPB, nt, a.tch, one, xs, a.qx, vin, vout, a.qact, ys);
}

// ---- down: the shared expert and every expert of a token, and the combine -------
//
// A workgroup owns RPG = QD_DOWN_RIT * 64/LPR output rows of one token; wave m
// computes those rows of matrix m (0 = the shared expert, 1 + k = the token's
// k-th expert) against that matrix's staged input, so each wave has one round
// of loads in flight.  The per-matrix rows meet in LDS and the combine runs in
// slot order.
template <int LPR, int NUL>
__global__ __launch_bounds__(QD_DOWN_MAXW * 64) void k_decode_down(QdArgs a)
{
    constexpr int RPP = 64 / LPR, RPG = RPP * QD_DOWN_RIT;
    __shared__ float ys[QWK_ROUTE_MAX_K + 1][RPG];
    const int H = a.m.H, I = a.m.I, SI = a.m.SI, K = a.m.K;
    const int rb = blockIdx.x % a.n_down_rb, t = blockIdx.x / a.n_down_rb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int slot = lane / LPR, lr = lane % LPR;
    const int row0 = rb * RPG;
    const int lgG = a.lgG;
    for (int m = wave; m <= K; m += nw) {
        const int kin = m == 0 ? SI : I;
        const int units = kin / 16, words = kin / 8, groups = kin >> lgG;
        const uint32_t *wm = a.m.sh_down.w;
        const uint16_t *sm = a.m.sh_down.s, *bm = a.m.sh_down.b;
        const uint4 *xv = a.qsh + (size_t)t * (SI / 16) * 3;
        if (m > 0) {
            const size_t e = (size_t)a.idx[t * K + m - 1];
            wm = a.m.down.w + e * H * words;
            sm = a.m.down.s + e * H * groups;
            bm = a.m.down.b + e * H * groups;
            xv = a.qact + ((size_t)t * K + m - 1) * (I / 16) * 3;
        }
        uint2 wv[NUL][QD_DOWN_RIT];
        float sc[NUL][QD_DOWN_RIT], bi[NUL][QD_DOWN_RIT];
        uint4 xp[NUL][3];
#pragma unroll
        for (int j = 0; j < NUL; j++) {
            const int c = j * LPR + lr;
            const int g = (16 * c) >> lgG;
#pragma unroll
            for (int i = 0; i < QD_DOWN_RIT; i++) {
                const int row = row0 + slot + RPP * i;
                if (c < units && row < H) {
                    wv[j][i] = *reinterpret_cast<const uint2 *>(wm + (size_t)row * words + 2 * c);
                    sc[j][i] = qw_bf16(sm[(size_t)row * groups + g]);
                    bi[j][i] = qw_bf16(bm[(size_t)row * groups + g]);
                } else {
                    wv[j][i] = make_uint2(0, 0);
                    sc[j][i] = bi[j][i] = 0.0f;
                }
            }
            if (c < units) {
                const uint4 *src = xv + (size_t)c * 3;
                xp[j][0] = src[0]; xp[j][1] = src[1]; xp[j][2] = src[2];
            } else {
                xp[j][0] = xp[j][1] = xp[j][2] = make_uint4(0, 0, 0, 0);
            }
        }
        float y[QD_DOWN_RIT];
#pragma unroll
        for (int i = 0; i < QD_DOWN_RIT; i++) y[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < NUL; j++) {
            const float4 r = *reinterpret_cast<const float4 *>(&xp[j][2]);
#pragma unroll
            for (int i = 0; i < QD_DOWN_RIT; i++)
                y[i] = qw_unit_dot(wv[j][i], xp[j][0], xp[j][1], r, sc[j][i], bi[j][i], y[i]);
        }
#pragma unroll
        for (int i = 0; i < QD_DOWN_RIT; i++) {
            const float v = qw_xor_sum<LPR>(y[i]);
            if (lr == 0) ys[m][slot + RPP * i] = v;
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

// A launch, with its own start / end stamps when e0 / e1 are given.
template <typename F>
static void qd_launch(F kern, dim3 grid, dim3 blk, size_t lds, hipStream_t s, hipEvent_t e0, hipEvent_t e1,
                      const QdArgs &a)
{
    if (e0) hipExtLaunchKernelGGL(kern, grid, blk, (uint32_t)lds, s, e0, e1, 0, a);
    else hipLaunchKernelGGL(kern, grid, blk, lds, s, a);
}

template <int LPR, int NUL>
static void launch_experts(hipStream_t s, QdArgs &a, hipEvent_t e0, hipEvent_t e1)
{
    const dim3 grid(a.n_shared_wg + a.umax * a.gu_wg_per_u), blk(QD_GU_WAVES * 64);
    const size_t lds = (size_t)a.tch * (a.m.H / 16) * QW_Q16_BYTES;
    if (a.m.E <= 256) qd_launch(k_decode_experts<LPR, NUL, 4>, grid, blk, lds, s, e0, e1, a);
    else if (a.m.E <= 512) qd_launch(k_decode_experts<LPR, NUL, 8>, grid, blk, lds, s, e0, e1, a);
    else qd_launch(k_decode_experts<LPR, NUL, 16>, grid, blk, lds, s, e0, e1, a);
}

template <int LPR, int NUL>
static void launch_down(hipStream_t s, QdArgs &a, hipEvent_t e0, hipEvent_t e1)
{
    const int nw = a.m.K + 1 < QD_DOWN_MAXW ? a.m.K + 1 : QD_DOWN_MAXW;
    qd_launch(k_decode_down<LPR, NUL>, dim3(a.rows * a.n_down_rb), dim3(nw * 64), 0, s, e0, e1, a);
}

// Instantiates F<LPR, NUL> for the supported (LPR, NUL) pairs.
#define QD_DISPATCH_GU(F, lpr, nul, ...)                                               \
    do {                                                                               \
        ok = true;                                                                     \
        switch ((lpr) * 16 + (nul)) {                                                  \
        case 16 * 16 + 1: F<16, 1>(__VA_ARGS__); break;                                \
        case 16 * 16 + 2: F<16, 2>(__VA_ARGS__); break;                                \
        case 16 * 16 + 3: F<16, 3>(__VA_ARGS__); break;                                \
        case 16 * 16 + 4: F<16, 4>(__VA_ARGS__); break;                                \
        case 32 * 16 + 2: F<32, 2>(__VA_ARGS__); break;                                \
        case 32 * 16 + 3: F<32, 3>(__VA_ARGS__); break;                                \
        case 32 * 16 + 4: F<32, 4>(__VA_ARGS__); break;                                \
        case 64 * 16 + 2: F<64, 2>(__VA_ARGS__); break;                                \
        case 64 * 16 + 3: F<64, 3>(__VA_ARGS__); break;                                \
        case 64 * 16 + 4: F<64, 4>(__VA_ARGS__); break;                                \
        default: ok = false;                                                           \
        }                                                                              \
    } while (0)
#define QD_DISPATCH_DOWN(F, nul, ...)                                                  \
    do {                                                                               \
        ok = true;                                                                     \
        switch (nul) {                                                                 \
        case 1: F<16, 1>(__VA_ARGS__); break;                                          \
        case 2: F<16, 2>(__VA_ARGS__); break;                                          \
        case 3: F<16, 3>(__VA_ARGS__); break;                                          \
        case 4: F<16, 4>(__VA_ARGS__); break;                                          \
        default: ok = false;                                                           \
        }                                                                              \
    } while (0)

// Lane layouts: gate / up rows have k = H; down rows k = I (routed) or SI
// (shared), one layout covering the larger.  Units per lane at most 4.
static bool qd_shapes(const qwk_moe *M, int *lpr_h, int *nul_h, int *nul_d)
{
    const int uh = M->H / 16, ud = (M->I > M->SI ? M->I : M->SI) / 16;
    *lpr_h = qd_lpr(uh);
    *nul_h = qd_nul(uh, *lpr_h);
    *nul_d = qd_nul(ud, 16);
    return *nul_h > 0 && *nul_h <= 4 && *nul_d > 0 && *nul_d <= 4;
}

extern "C" int qwk_moe_decode_supported(const qwk_moe *M, int rows)
{
    int a, b, c;
    const int G = M->group;
    return rows >= 1 && rows <= QWK_DECODE_MAX_ROWS && M->K >= 1 && M->K <= QWK_ROUTE_MAX_K &&
           M->E >= M->K && M->E <= QWK_ROUTE_MAX_E && M->H % 64 == 0 && M->I % 16 == 0 &&
           M->SI % 16 == 0 && M->H <= QWK_DMAT_MAX_K && (G == 32 || G == 64 || G == 128) &&
           M->H % G == 0 && M->I % G == 0 && M->SI % G == 0 && qd_shapes(M, &a, &b, &c);
}

extern "C" int qwk_moe_decode(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                              const qwk_moe *M, int rows, void *scratch, size_t scratch_bytes,
                              hipEvent_t *ev)
{
    const int G = M->group;
    if (!qwk_moe_decode_supported(M, rows) || ((uintptr_t)x & 15u)) return (int)hipErrorInvalidValue;
    const QdLayout L = qd_layout(M, rows);
    if (scratch_bytes < L.total) return (int)hipErrorInvalidValue;
    int lpr_h, nul_h, nul_d;
    qd_shapes(M, &lpr_h, &nul_h, &nul_d);
    const int lpr_d = 16;

    char *S = (char *)scratch;
    QdArgs a;
    a.m = *M;
    a.x = x; a.out = out; a.idx = idx; a.w = w; a.rows = rows;
    a.umax = rows * M->K < M->E ? rows * M->K : M->E;
    a.lgG = G == 32 ? 5 : G == 64 ? 6 : 7;
    a.n_router_wg = (M->E + 1 + QD_FRONT_WAVES - 1) / QD_FRONT_WAVES;
    const int rpb = QD_GU_WAVES * (64 / lpr_h);
    const int vbytes = (M->H / 16) * QW_Q16_BYTES;
    a.tch = QD_GU_LDS / vbytes < rows ? QD_GU_LDS / vbytes : rows;
    a.n_shared_wg = (M->SI + rpb - 1) / rpb;
    a.gu_wg_per_u = (M->I + rpb - 1) / rpb;
    a.n_down_rb = (M->H + QD_DOWN_RIT * (64 / lpr_d) - 1) / (QD_DOWN_RIT * (64 / lpr_d));
    a.logits = (float *)(S + L.logits);
    a.g1 = (float *)(S + L.g1);
    a.qx = (uint4 *)(S + L.qx);
    a.qsh = (uint4 *)(S + L.qsh);
    a.qact = (uint4 *)(S + L.qact);

    bool ok;
    hipEvent_t no[6] = {0, 0, 0, 0, 0, 0};
    hipEvent_t *e = ev ? ev : no;
    qd_launch(k_decode_front, dim3(a.n_router_wg + rows), dim3(QD_FRONT_WAVES * 64), 0, s, e[0], e[1], a);
    QD_DISPATCH_GU(launch_experts, lpr_h, nul_h, s, a, e[2], e[3]);
    if (!ok) return (int)hipErrorInvalidValue;
    QD_DISPATCH_DOWN(launch_down, nul_d, s, a, e[4], e[5]);
    if (!ok) return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}
