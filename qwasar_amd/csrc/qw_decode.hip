// qw_decode.hip -- the MoE block at decode over a batch of 1..8 tokens, in
// launches with no waits between workgroups (the one-token path's single
// launch is qw_decode1.hip; this path serves 2..8 tokens, and one token of a
// layer shape the single launch does not take):
//
//   router     order-R logits of every token and the shared expert's gate
//              logits (k_dmat_few in qw_route.hip, one launch)
//   route      one workgroup: every token routed (a wave each, the standalone
//              route's arithmetic), the table of the batch's unique experts
//   gate / up  per unique expert, every token routed there: the weight rows
//              read once for all of them; SwiGLU fused
//   down       per (token, block of output rows): the down rows of the shared
//              expert and the token's K experts, each applied to its
//              activation vector, then the combine
//              sigmoid(g) * shared + sum_k w_k * y_k, an fma chain in slot order
//
// The 4-bit products use the q16 dot (qw_unit_dot): staged activations are
// loaded straight into registers next to the weights.
#include "qw_device.h"
#include "qw_kernels.h"
#include "qw_few.h"

#include <algorithm>

#define QD_MAXT QWK_DECODE_MAX_ROWS
#define QD_MAXU (QWK_DECODE_MAX_ROWS * QWK_DECODE_MAX_K)
#define QD_WAVES 16
#define QD_THREADS (QD_WAVES * 64)
#define QD_GU_MAXRPB (QD_WAVES * 4)
#define QD_LDS (64 * 1024)          // dynamic LDS: staged inputs
#define QD_DOWN_LPR 16
#define QD_DOWN_RIT 4               // down rows per lane slot
#define QD_DOWN_RPG ((64 / QD_DOWN_LPR) * QD_DOWN_RIT)

// Lanes per row for a row of `units` q16 units, and units per lane.
static __host__ __device__ constexpr int qd_lpr(int units) { return units >= 128 ? 64 : units >= 64 ? 32 : 16; }
static int qd_nul(int units, int lpr)
{
    const int n = (units + lpr - 1) / lpr;
    return n <= 4 ? n : -1;
}

// One q16 uint4 written device-coherently, as two 64-bit halves.
__device__ __forceinline__ void qd_st4(uint4 *p, uint4 v)
{
    unsigned long long *q = reinterpret_cast<unsigned long long *>(p);
    __hip_atomic_store(q, (unsigned long long)v.x | ((unsigned long long)v.y << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (unsigned long long)v.z | ((unsigned long long)v.w << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

struct QdArgs {
    qwk_moe m;
    const float *x;
    float *out;
    int32_t *idx;
    float *w;
    int rows, umax, lgG;
    int n_sh, gu_wg_per_u, n_ex, n_down_rb;
    int tch;                        // input vectors per LDS pass
    char *scr;                      // the scratch base
    uint4 *qx, *qsh, *qact;         // q16 units: [vector][units][3]
};

// ---- gate / up rows with SwiGLU ----------------------------------------------------
//
// A workgroup owns RPB = QD_WAVES * 64/LPR consecutive rows of one gate / up
// pair (the shared expert's, or one routed expert's) for nt input vectors.
// Lane (slot, lr) of wave w takes row row0 + w * 64/LPR + slot and its units
// lr, lr + LPR, ... (NUL of them), in both matrices; its weights stay in
// registers while the input vectors pass through LDS, up to `tch` at a time.
// The per-row results meet in LDS and leave as q16 units of the activation
// vectors at dst.  Unless `staged` (the inputs already in LDS), the inputs
// are copied from the staged token rows (a.qx).
template <int LPR, int NUL, bool PLAINX = false>
__device__ __forceinline__ void qd_glu_block(const qwk_q4 gm, const qwk_q4 um, int n, const QdArgs &a,
                                             int row0, int nt, bool staged, uint4 *xs, const int *vin,
                                             const int *vout, uint4 *dst, float (*ys)[QD_GU_MAXRPB])
{
    constexpr int SL = 64 / LPR, RPB = QD_WAVES * SL;
    static_assert(RPB % 16 == 0 && RPB <= QD_GU_MAXRPB, "rows per block");
    const int k = a.m.H, lgG = a.lgG;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, slot = lane / LPR, lr = lane % LPR;
    const int units = k / 16, words = k / 8, groups = k >> lgG;
    const int rl = wave * SL + slot, row = row0 + rl;
    // Every load is issued (at a clamped, valid address) before any is used;
    // out-of-range lanes are zeroed afterwards.
    //
    // With a whole wave on a row (LPR 64), lane lr takes the unit pairs
    // (2 lr, 2 lr + 1) and (128 + 2 lr, 128 + 2 lr + 1): two 16-byte loads a
    // matrix, each instruction of the wave reading whole lines, and a scale
    // and a bias a pair (a pair is 32 inputs, inside one group); else lane lr
    // takes units lr, lr + LPR, ... (NUL of them).
    constexpr bool CG = LPR == 64;
    constexpr int NW = CG ? 4 : NUL;               // units a lane
    uint2 wv[2][NW];
    uint32_t sb[2][CG ? 2 : NUL];                  // bf16 scale (low half) and bias (high half)
    const int rowc = min(row, n - 1);
    if constexpr (CG) {
        // lane lr: unit pairs (2 lr, 2 lr + 1) and (128 + 2 lr, 128 + 2 lr + 1),
        // so each 16-byte load instruction of the wave reads whole lines
        uint4 w4[2][2];
        uint32_t sv[2][2], bv[2][2];
        bool okp[2];
#pragma unroll
        for (int h = 0; h < 2; h++) okp[h] = row < n && 128 * h + 2 * lr + 1 < units;
#pragma unroll
        for (int z = 0; z < 2; z++) {
            const qwk_q4 q = z ? um : gm;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int c0 = min(128 * h + 2 * lr, units - 2);
                w4[z][h] = *reinterpret_cast<const uint4 *>(q.w + (size_t)rowc * words + 2 * c0);
                const size_t gi = (size_t)rowc * groups + ((16 * c0) >> lgG);
                sv[z][h] = q.s[gi];
                bv[z][h] = q.b[gi];
            }
        }
#pragma unroll
        for (int z = 0; z < 2; z++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                wv[z][2 * h] = okp[h] ? make_uint2(w4[z][h].x, w4[z][h].y) : make_uint2(0, 0);
                wv[z][2 * h + 1] = okp[h] ? make_uint2(w4[z][h].z, w4[z][h].w) : make_uint2(0, 0);
                sb[z][h] = okp[h] ? sv[z][h] | (bv[z][h] << 16) : 0u;
            }
    } else {
        uint32_t sv[2][NUL], bv[2][NUL];
#pragma unroll
        for (int z = 0; z < 2; z++) {
            const qwk_q4 q = z ? um : gm;
#pragma unroll
            for (int j = 0; j < NUL; j++) {
                const int c = min(j * LPR + lr, units - 1);
                wv[z][j] = *reinterpret_cast<const uint2 *>(q.w + (size_t)rowc * words + 2 * c);
                const size_t gi = (size_t)rowc * groups + ((16 * c) >> lgG);
                sv[z][j] = q.s[gi];
                bv[z][j] = q.b[gi];
            }
        }
#pragma unroll
        for (int z = 0; z < 2; z++)
#pragma unroll
            for (int j = 0; j < NUL; j++) {
                const bool ok = row < n && j * LPR + lr < units;
                wv[z][j] = ok ? wv[z][j] : make_uint2(0, 0);
                sb[z][j] = ok ? sv[z][j] | (bv[z][j] << 16) : 0u;
            }
    }
    for (int t0 = 0; t0 < nt; t0 += a.tch) {
        const int tn = min(a.tch, nt - t0);
        if (!staged) {
            __syncthreads();
            const int per = units * 3;
            for (int i0 = 0; i0 < tn * per; i0 += 4 * QD_THREADS) {
                uint4 v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = min(i0 + (int)threadIdx.x + r * QD_THREADS, tn * per - 1);
                    const uint32_t off = (uint32_t)((vin[t0 + i / per] * per + i % per) * 16);
                    // PLAINX: the rows were staged by an earlier launch, so cached loads see them
                    v[r] = PLAINX ? a.qx[off / 16] : qw_ld4_coh(a.qx, off);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) asm volatile("" : "+v"(v[r].x), "+v"(v[r].y), "+v"(v[r].z), "+v"(v[r].w));
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (i0 + (int)threadIdx.x + r * QD_THREADS < tn * per) xs[i0 + threadIdx.x + r * QD_THREADS] = v[r];
            }
        }
        __syncthreads();
#pragma unroll 1
        for (int t = 0; t < tn; t++) {
            const uint4 *xt = xs + (size_t)t * units * 3;
            float acc[2] = {0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NW; j++) {
                const int c = CG ? min(128 * (j / 2) + 2 * lr + (j % 2), units - 1) : j * LPR + lr;
                if (CG || c < units) {
                    const uint4 p0 = xt[3 * c], p1 = xt[3 * c + 1];
                    const uint4 rr = xt[3 * c + 2];
                    const float4 r = *reinterpret_cast<const float4 *>(&rr);
                    const int si = CG ? j / 2 : j;
#pragma unroll
                    for (int z = 0; z < 2; z++)
                        acc[z] = qw_unit_dot(wv[z][j], p0, p1, r, __uint_as_float(sb[z][si] << 16),
                                             __uint_as_float(sb[z][si] & 0xFFFF0000u), acc[z]);
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
        uint4 s[3];
        qw_q16_make(v, s);
        {
            uint4 *d = dst + ((size_t)vout[t] * outunits + row0 / 16 + uu) * 3;
            qd_st4(d, s[0]);
            qd_st4(d + 1, s[1]);
            qd_st4(d + 2, s[2]);
        }
    }
}

// ---- the batch's routing table -----------------------------------------------------

struct QdRoute {
    int picks[QD_MAXU];
    int ustart[QD_MAXU];      // unique expert u's first slot in the pair order
    int mark[QWK_ROUTE_MAX_E];// the unique-expert slot of each selected expert
    struct alignas(16) {
        uint32_t sx[QD_MAXT][QW_ROUTE_SX];  // selection scratch of routing wave w (w < rows <= QD_MAXT)
    } rs;
};

// The instantiated shapes: (LPR, NUL) of the gate / up rows (k = H), NULD of
// the down rows (k = max(I, SI), 16 lanes a row), PL logits per lane (E).
#define QD_SHAPES(X)                                                                   \
    X(16, 1, 1, 4) X(16, 1, 2, 4) X(16, 2, 1, 4) X(16, 2, 2, 4)                         \
    X(32, 2, 2, 8) X(64, 2, 2, 8) X(64, 3, 2, 8) X(64, 4, 2, 8)

static bool qd_shapes(const qwk_moe *M, int *lpr_h, int *nul_h, int *nul_d, int *pl)
{
    const int uh = M->H / 16, ud = (M->I > M->SI ? M->I : M->SI) / 16;
    *lpr_h = qd_lpr(uh);
    *nul_h = qd_nul(uh, *lpr_h);
    *nul_d = qd_nul(ud, QD_DOWN_LPR);
    *pl = M->E <= 256 ? 4 : M->E <= 512 ? 8 : 16;
#define QD_HAS(L, N, D, P) if (*lpr_h == L && *nul_h == N && *nul_d == D && *pl == P) return true;
    QD_SHAPES(QD_HAS)
#undef QD_HAS
    return false;
}

extern "C" int qwk_moe_decode_batch_supported(const qwk_moe *M, int rows)
{
    int a, b, c, d;
    const int G = M->group;
    return rows >= 1 && rows <= QWK_DECODE_MAX_ROWS && M->K >= 1 && M->K <= QWK_DECODE_MAX_K &&
           M->E >= M->K && M->E <= QWK_ROUTE_MAX_E && M->H % 64 == 0 && M->I % 16 == 0 &&
           M->SI % 16 == 0 && M->H <= 4096 && (G == 32 || G == 64 || G == 128) &&
           M->H % G == 0 && M->I % G == 0 && M->SI % G == 0 && qd_shapes(M, &a, &b, &c, &d);
}

// ---- the launches ----------------------------------------------------------------
//
// A one-launch form would route every token in every experts and down
// workgroup and need more workgroups than fit at once (measured at 8 tokens,
// config 2: ~16 us routing in each of ~4000 workgroups).  Here each step is
// its own launch, so nothing waits on another workgroup and the grid size is
// free:
//
//   router     order-R logits of every token
//   (k_dmat_few in qw_route.hip, with the shared expert's gate logits in
//              the same launch)
//   k_batch_route   one workgroup: every token routed (a wave each, the
//              standalone route's arithmetic), the table of unique experts
//              (ascending, each with its pairs in ascending order), and the
//              token rows staged as q16 units
//   k_batch_gu      per (unique expert, 16-row block), and the shared
//              expert's blocks: the weight rows read once for every token
//              routed there (requested before the staged rows are copied into
//              LDS); SwiGLU fused; the activations leave as q16 units
//   k_batch_down    per (token, 16 output rows): the down rows of the shared
//              expert and the token's K experts, each applied to its
//              activation vector, then the combine in slot order.  A row
//              block's workgroups for all tokens sit on one XCD (block index
//              = rb mod 8 there), so an expert several tokens share is read
//              from that XCD's L2 after the first.

#define QB_TAB_U 0
#define QB_TAB_UEXP 1
#define QB_TAB_UCNT (1 + QD_MAXU)
#define QB_TAB_USTART (1 + 2 * QD_MAXU)
#define QB_TAB_UPAIR (1 + 3 * QD_MAXU)
#define QB_TAB_GATE (1 + 4 * QD_MAXU)
#define QB_TAB_INTS (1 + 4 * QD_MAXU + QD_MAXT)

struct QbLayout {
    size_t logits, tab, qx, qact, qsh, xh, xF, perm, tiles, act, ey, total;
};

// The batch's gate / up runs on the matrix cores (qwk_gmm16, the shared
// expert as one more expert of the grouped product) when the shared expert's
// width is the routed experts' and the product takes the shapes and banks;
// else as q16 dots (k_batch_gu).
static qwk_q4 qb_up_bank(const qwk_moe *M)
{
    if (M->split) return M->up;
    const qwk_q4 g = M->gate_up;
    return qwk_q4{g.w + (size_t)M->I * (M->H / 8), g.s + (size_t)M->I * (M->H / M->group),
                  g.b + (size_t)M->I * (M->H / M->group)};
}
static bool qb_gmm(const qwk_moe *M)
{
    return M->SI == M->I && qwk_gmm16_supported(M->H, M->group, (M->split ? M->gate : M->gate_up).w, qb_up_bank(M).w) &&
           qwk_gmm16_supported(M->H, M->group, M->sh_gate.w, M->sh_up.w);
}

// ... and both grouped products run as one weight stream a wave
// (qwk_gmm16_stream: gate / up with fp32 activations, then the down into
// per-pair rows and the combine) when they take the shapes and banks.
static bool qb_stream(const qwk_moe *M)
{
    if (!qb_gmm(M)) return false;
    const int G = M->group;
    const qwk_q4 g0 = M->split ? M->gate : M->gate_up, u0 = qb_up_bank(M);
    const qwk_gmm_extra xgu = {M->sh_gate, M->sh_up, M->E, 0}, xd = {M->sh_down, M->sh_down, M->E, 0};
    return qwk_gmm16_stream_supported(M->H, M->I, G, 1, g0, u0, &xgu, (long)(M->split ? 1 : 2) * M->I * (M->H / G)) &&
           qwk_gmm16_stream_supported(M->I, M->H, G, 0, M->down, M->down, &xd, (long)M->H * (M->I / G));
}

static QbLayout qb_layout(const qwk_moe *M, int rows)
{
    QbLayout L;
    size_t o = 0;
    const bool gmm = qb_gmm(M);
    L.logits = o; o += al((size_t)rows * M->E * 4);
    L.qx = o;     o += gmm ? 0 : al((size_t)rows * (M->H / 16) * QW_Q16_BYTES);
    L.tab = o;    o += al((size_t)QB_TAB_INTS * 4);
    L.qact = o;   o += al((size_t)rows * M->K * (M->I / 16) * QW_Q16_BYTES);
    L.qsh = o;    o += al((size_t)rows * (M->SI / 16) * QW_Q16_BYTES);
    // the matrix-core gate / up: the token rows staged as f16, the pairs by
    // expert (then the shared expert's rows), a tile per unique expert and
    // one for the shared expert, the activations in fp32
    const size_t npk = (size_t)rows * M->K;
    L.xh = o;     o += gmm ? al((size_t)rows * M->H * 2) : 0;
    L.xF = o;     o += gmm ? al((size_t)rows * 4) : 0;
    L.perm = o;   o += gmm ? al((npk + rows) * 4) : 0;
    L.tiles = o;  o += gmm ? al((1 + 3 * ((size_t)QD_MAXU + 1)) * 4) : 0;
    L.act = o;    o += gmm ? al((npk + rows) * M->I * 4) : 0;
    // the streamed down's rows: every pair's, then the shared expert's
    L.ey = o;     o += qb_stream(M) ? al((npk + rows) * M->H * 4) : 0;
    L.total = o;
    return L;
}

struct QbArgs {
    QdArgs d;                 // shapes, x, out, idx, w, rows, lgG, tch, qact, qsh
    const float *logits;
    int32_t *tab;
    int xstaged;              // the router launch staged the token rows into qx
    int gmm;                  // gate / up on the matrix cores: emit perm and tiles
    int32_t *perm, *tiles;
    const float *act;         // their fp32 activations [pairs + rows][I]
    uint16_t *xh;             // the token rows staged as f16 (matrix-core gate / up)
    float *xF;                //   and their scales
};

#define QB_SPIN_LIMIT (1 << 16)

// Every token routed and the batch's tables, by one workgroup of QD_MAXT
// waves (the logits of token r at logits + r E: global memory, or LDS in
// the router-and-route launch).
template <int PL>
__device__ __forceinline__ void qb_route_body(const QbArgs &b, const float *logits)
{
    __shared__ QdRoute R;
    // per token a bitmask of its picks; per 64-expert chunk its unique
    // experts and pairs
    __shared__ uint32_t tmask[QD_MAXT][QWK_ROUTE_MAX_E / 32];
    __shared__ int ctu[QWK_ROUTE_MAX_E / 64], ctp[QWK_ROUTE_MAX_E / 64];
    const QdArgs &a = b.d;
    const int t = threadIdx.x, nthr = blockDim.x, wave = t >> 6, lane = t & 63;
    const int E = a.m.E, K = a.m.K, H = a.m.H;
    for (int i = t; i < QD_MAXT * (QWK_ROUTE_MAX_E / 32); i += nthr) (&tmask[0][0])[i] = 0u;
    __syncthreads();
    if (wave < a.rows) {
        int pi;
        float pw;
        qw_route_wave<PL>(logits + (size_t)wave * E, E, K, a.m.norm, lane, &pi, &pw, R.rs.sx[wave]);
        if (lane < K) {
            R.picks[wave * K + lane] = pi;
            a.idx[wave * K + lane] = pi;
            a.w[wave * K + lane] = pw;
            atomicOr(&tmask[wave][pi >> 5], 1u << (pi & 31));
        }
    }
    // the token rows as q16 units for the gate / up launch (unless the
    // router's launch did)
    const int units = H / 16;
    for (int i = t; i < (b.xstaged ? 0 : a.rows * units); i += nthr) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = reinterpret_cast<const float4 *>(a.x + (size_t)i * 16)[q];
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
        uint4 u[3];
        qw_q16_make(v, u);
        a.qx[(size_t)i * 3] = u[0];
        a.qx[(size_t)i * 3 + 1] = u[1];
        a.qx[(size_t)i * 3 + 2] = u[2];
    }
    __syncthreads();
    // The union of the picks, ascending, with each expert's pairs in
    // ascending order: a wave a 64-expert chunk (its count of pairs from the
    // token masks, its unique experts by ballot, the pairs' running count by
    // an in-wave scan); the chunks' totals meet in LDS; a pair's place in its
    // expert's run is the number of earlier tokens that picked the same
    // expert (a token's picks are distinct, so pairs of one expert are
    // ordered by token).
    const int npk = a.rows * K, nchk = (E + 63) / 64;
    constexpr int CW = QWK_ROUTE_MAX_E / 64 / QD_MAXT;       // chunks a wave
    int cnt[CW], incl[CW];
    unsigned long long bal[CW];
#pragma unroll
    for (int c = 0; c < CW; c++) {
        const int ch = wave + QD_MAXT * c, e = 64 * ch + lane;
        int n = 0;
        if (ch < nchk && e < E)
            for (int r = 0; r < a.rows; r++) n += (tmask[r][e >> 5] >> (e & 31)) & 1;
        bal[c] = __ballot(n > 0);
        int in = n;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(in, o, 64);
            if (lane >= o) in += y;
        }
        cnt[c] = n;
        incl[c] = in;
        if (ch < nchk && lane == 63) {
            ctu[ch] = __popcll(bal[c]);
            ctp[ch] = in;
        }
    }
    __syncthreads();
    int U = 0;
    for (int ch = 0; ch < nchk; ch++) U += ctu[ch];
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int c = 0; c < CW; c++) {
        const int ch = wave + QD_MAXT * c, e = 64 * ch + lane;
        if (ch >= nchk || cnt[c] == 0) continue;
        int ub = 0, pb = 0;
        for (int q = 0; q < ch; q++) { ub += ctu[q]; pb += ctp[q]; }
        const int u = ub + (int)__popcll(bal[c] & below), st = pb + incl[c] - cnt[c];
        R.mark[e] = u;
        R.ustart[u] = st;
        b.tab[QB_TAB_UEXP + u] = e;
        b.tab[QB_TAB_UCNT + u] = cnt[c];
        b.tab[QB_TAB_USTART + u] = st;
        if (b.gmm) {
            // the grouped product's tile list: unique expert u's pairs
            b.tiles[1 + 3 * u] = e;
            b.tiles[2 + 3 * u] = st;
            b.tiles[3 + 3 * u] = cnt[c];
        }
    }
    if (t == 0) {
        b.tab[QB_TAB_U] = U;
        if (b.gmm) {
            // then the shared expert (expert E) on the token rows, pairs npk + r
            b.tiles[0] = U + 1;
            b.tiles[1 + 3 * U] = E;
            b.tiles[2 + 3 * U] = npk;
            b.tiles[3 + 3 * U] = a.rows;
        }
    }
    if (b.gmm)
        for (int r = t; r < a.rows; r += nthr) b.perm[npk + r] = npk + r;
    __syncthreads();
    for (int p = t; p < npk; p += nthr) {
        const int e = R.picks[p], tk = p / K;
        int rank = 0;
        for (int q = 0; q < tk; q++) rank += (tmask[q][e >> 5] >> (e & 31)) & 1u;
        const int dst = R.ustart[R.mark[e]] + rank;
        b.tab[QB_TAB_UPAIR + dst] = p;
        if (b.gmm) b.perm[dst] = p;
    }
}

template <int PL>
__global__ __launch_bounds__(QD_MAXT * 64) void k_batch_route(QbArgs b)
{
    qb_route_body<PL>(b, b.logits);
}

// The router's logits and the routing in one launch: blocks (x < nxb, y)
// are k_dmat_few's (the logits leave as tagged words, device scope); the
// last block, (gridDim.x - 1, gridDim.y - 1), dispatched after every other,
// polls them into LDS (wave r: token r's E logits, every tag checked,
// bounded as the one-token launch's waits) and routes.  The grid's other
// blocks past column nxb return at once.
template <int PL>
__global__ __launch_bounds__(QD_MAXT * 64) void k_batch_router(QbArgs b, uint2 *ty, uint32_t *err, uint32_t epoch)
{
    static_assert(QD_MAXT == QW_DF_WAVES, "the logits' body takes the launch's waves, one an output");
    extern __shared__ float xl[];
    const QdArgs &a = b.d;
    const int E = a.m.E, H = a.m.H;
    // columns past the logits' (the grid is a multiple of 8 wide, so that
    // column bx sits on XCD bx mod 8 for every group of token rows and its
    // router rows are read from memory once, then from that XCD's L2)
    const int nxb = (E + 1 + QW_DF_WAVES - 1) / QW_DF_WAVES;
    if ((int)blockIdx.x < nxb) {
        qw_few_body<true>(nullptr, reinterpret_cast<float *>(b.tab + QB_TAB_GATE), a.x, a.m.router, a.m.sh_gate_w,
                          H, E, a.rows, nullptr, b.xh, b.xF, ty, epoch, blockIdx.x, blockIdx.y, xl);
        return;
    }
    if (blockIdx.y != gridDim.y - 1 || blockIdx.x != gridDim.x - 1) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *lg = xl;                                  // [rows][E]
    if (wave < a.rows) {
        const uint2 *tw = ty + (size_t)wave * E;
        for (int spins = 0;; spins++) {
            unsigned long long q[PL];
#pragma unroll
            for (int i = 0; i < PL; i++) {
                const uint2 *pi = tw + min(lane + 64 * i, E - 1);
                asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q[i]) : "v"(pi) : "memory");
            }
            uint32_t e;
            asm volatile("global_load_dword %0, %1, off sc1" : "=v"(e) : "v"(err) : "memory");
            asm volatile("s_waitcnt vmcnt(0)" : "+v"(e) : : "memory");
            bool stale = false;
#pragma unroll
            for (int i = 0; i < PL; i++) {
                asm volatile("" : "+v"(q[i]));
                stale |= lane + 64 * i < E && (uint32_t)q[i] != epoch;
            }
            if (__ballot(stale) == 0ull || spins >= QB_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
                if (__ballot(stale) != 0ull && lane == 0)
                    __hip_atomic_store(err, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int i = 0; i < PL; i++)
                    if (lane + 64 * i < E) lg[(size_t)wave * E + lane + 64 * i] = __uint_as_float((uint32_t)(q[i] >> 32));
                break;
            }
            // (no sleep between polls: the launch has nothing else on the
            // memory side by then; 57.42 -> 56.78 us a step against a sleep
            // of 2, five alternating runs)
            __builtin_amdgcn_s_sleep(0);
        }
    }
    __syncthreads();
    qb_route_body<PL>(b, lg);
}

// The matrix-core gate / up's fp32 activations as the q16 vectors the down
// launch reads, where the product does not write them itself: pair p's into qact, the shared expert's (rows npk + t) into
// qsh.  A thread per (vector, 16-unit).
__global__ __launch_bounds__(256) void k_batch_act_q16(QbArgs b)
{
    const QdArgs &a = b.d;
    const int I = a.m.I, units = I / 16, npk = a.rows * a.m.K;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (npk + a.rows) * units) return;
    const int v = i / units, u = i % units;
    float f[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 x = reinterpret_cast<const float4 *>(b.act + (size_t)v * I + 16 * u)[q];
        f[4 * q] = x.x; f[4 * q + 1] = x.y; f[4 * q + 2] = x.z; f[4 * q + 3] = x.w;
    }
    uint4 q3[3];
    qw_q16_make(f, q3);
    uint4 *d = v < npk ? a.qact + ((size_t)v * units + u) * 3 : a.qsh + ((size_t)(v - npk) * units + u) * 3;
    d[0] = q3[0];
    d[1] = q3[1];
    d[2] = q3[2];
}

template <int LPR, int NUL>
__global__ __launch_bounds__(QD_THREADS, 8) void k_batch_gu(QbArgs b)
{
    extern __shared__ uint4 xs[];                    // [tch][units][3]
    __shared__ int vin[QD_MAXT], vout[QD_MAXT];
    __shared__ float ys[QD_MAXT][QD_GU_MAXRPB];
    const QdArgs &a = b.d;
    constexpr int RPB = QD_WAVES * (64 / LPR);
    const int H = a.m.H, I = a.m.I, K = a.m.K;
    const int bb = blockIdx.x;
    if (bb < a.n_ex) {
        const int u = bb / a.gu_wg_per_u, rb = bb % a.gu_wg_per_u;
        if (u >= b.tab[QB_TAB_U]) return;                              // uniform
        const int e = b.tab[QB_TAB_UEXP + u], nt = b.tab[QB_TAB_UCNT + u], p0 = b.tab[QB_TAB_USTART + u];
        if (threadIdx.x < nt) {
            const int p = b.tab[QB_TAB_UPAIR + p0 + threadIdx.x];
            vin[threadIdx.x] = p / K;
            vout[threadIdx.x] = p;
        }
        __syncthreads();
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
        // the weights are requested first; the token rows follow from the
        // staged copy, pass by pass
        qd_glu_block<LPR, NUL, true>(gm, um, I, a, rb * RPB, nt, false, xs, vin, vout, a.qact, ys);
    } else {
        const int sb = bb - a.n_ex;
        if (threadIdx.x < QD_MAXT) vin[threadIdx.x] = vout[threadIdx.x] = threadIdx.x;
        __syncthreads();
        qd_glu_block<LPR, NUL, true>(a.m.sh_gate, a.m.sh_up, a.m.SI, a, sb * RPB, a.rows, false, xs, vin, vout,
                                     a.qsh, ys);
    }
}

template <int NUL>
__global__ __launch_bounds__(QD_THREADS, 8) void k_batch_down(QbArgs b)
{
    extern __shared__ uint4 xa[];                    // the K + 1 activation vectors
    __shared__ float ys[QWK_DECODE_MAX_K + 1][QD_DOWN_RPG];
    const QdArgs &a = b.d;
    constexpr int LPR = QD_DOWN_LPR, RPP = 64 / LPR, RIT = QD_DOWN_RIT, RPG = QD_DOWN_RPG;
    const int H = a.m.H, I = a.m.I, SI = a.m.SI, K = a.m.K;
    // block -> (token, row block): all tokens of row block rb on XCD rb mod 8
    const int q = blockIdx.x >> 3, xcd = blockIdx.x & 7;
    const int t = q % a.rows, rb = (q / a.rows) * 8 + xcd;
    if (rb >= a.n_down_rb) return;                   // uniform
    const int lane = threadIdx.x & 63, m = threadIdx.x >> 6;
    const int slot = lane / LPR, lr = lane % LPR;
    const int row0 = rb * RPG, lgG = a.lgG;
    const bool busy = m <= K;
    const int kin = m == 0 ? SI : I;
    const int units = kin / 16, words = kin / 8, groups = kin >> lgG;
    const uint32_t *wm = a.m.sh_down.w;
    const uint16_t *sm = a.m.sh_down.s, *bm = a.m.sh_down.b;
    if (busy && m > 0) {
        const size_t e = (size_t)a.idx[t * K + m - 1];
        wm = a.m.down.w + e * H * words;
        sm = a.m.down.s + e * H * groups;
        bm = a.m.down.b + e * H * groups;
    }
    uint2 wv[NUL][RIT];
    uint32_t sv[NUL][RIT], bv[NUL][RIT];
#pragma unroll
    for (int j = 0; j < NUL; j++) {
        const int c = min(j * LPR + lr, units - 1);
        const int g = (16 * c) >> lgG;
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const int row = min(row0 + slot + RPP * i, H - 1);
            wv[j][i] = qw_ld2(wm, (uint32_t)(row * words + 2 * c) * 4u);
            sv[j][i] = qw_ldu16(sm, (uint32_t)(row * groups + g) * 2u);
            bv[j][i] = qw_ldu16(bm, (uint32_t)(row * groups + g) * 2u);
        }
    }
    // this matrix's activation vector into the wave's own LDS region
    const int nv = units * 3;
    constexpr int XW = (3 * NUL * LPR + 63) / 64;
    uint4 *xw = xa + (m == 0 ? 0 : (SI / 16) * 3 + (m - 1) * ((I / 16) * 3));
    if (busy) {
        const uint4 *xm = m == 0 ? a.qsh + (size_t)t * ((SI / 16) * 3)
                                 : a.qact + ((size_t)t * K + (m - 1)) * ((I / 16) * 3);
        uint4 v[XW];
#pragma unroll
        for (int r = 0; r < XW; r++) v[r] = xm[min(lane + 64 * r, nv - 1)];
#pragma unroll
        for (int r = 0; r < XW; r++)
            if (lane + 64 * r < nv) xw[lane + 64 * r] = v[r];
    }
    const float gate = qw_sigmoid(__int_as_float(b.tab[QB_TAB_GATE + t]));
    if (busy) {
        uint32_t sb[NUL][RIT];
#pragma unroll
        for (int j = 0; j < NUL; j++)
#pragma unroll
            for (int i = 0; i < RIT; i++) {
                const bool ok = j * LPR + lr < units && row0 + slot + RPP * i < H;
                wv[j][i] = ok ? wv[j][i] : make_uint2(0, 0);
                sb[j][i] = ok ? sv[j][i] | (bv[j][i] << 16) : 0u;
            }
        float y[RIT];
#pragma unroll
        for (int i = 0; i < RIT; i++) y[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < NUL; j++) {
            const int c = j * LPR + lr;
            if (c < units) {
                const uint4 p0 = xw[3 * c], p1 = xw[3 * c + 1], rr = xw[3 * c + 2];
                const float4 r = *reinterpret_cast<const float4 *>(&rr);
#pragma unroll
                for (int i = 0; i < RIT; i++)
                    y[i] = qw_unit_dot(wv[j][i], p0, p1, r, __uint_as_float(sb[j][i] << 16),
                                       __uint_as_float(sb[j][i] & 0xFFFF0000u), y[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const float v = qw_xor_sum<LPR>(y[i]);
            if (lr == 0) ys[m][slot + RPP * i] = v;
        }
    }
    __syncthreads();
    // the combine: the shared term first, then an fma per slot, in order
    for (int r = threadIdx.x; r < RPG; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= H) continue;
        float acc = ys[0][r] * gate;
        for (int k = 0; k < K; k++) acc = __builtin_fmaf(a.w[t * K + k], ys[1 + k][r], acc);
        a.out[(size_t)t * H + row] = acc;
    }
}

extern "C" size_t qwk_moe_decode_batch_scratch(const qwk_moe *M, int rows)
{
    return qb_layout(M, rows).total;
}

extern "C" int qwk_moe_decode_batch(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                                    const qwk_moe *M, int rows, void *scratch, size_t scratch_bytes, void *tags,
                                    size_t tag_words, uint32_t *err, uint32_t epoch, int *handoff)
{
    if (handoff) *handoff = 0;
    const int G = M->group;
    if (rows < 1 || !qwk_moe_decode_batch_supported(M, rows) || !x || ((uintptr_t)x & 15u)) return (int)hipErrorInvalidValue;
    const QbLayout L = qb_layout(M, rows);
    if (scratch_bytes < L.total) return (int)hipErrorInvalidValue;
    int lpr_h, nul_h, nul_d, pl;
    qd_shapes(M, &lpr_h, &nul_h, &nul_d, &pl);
    char *S = (char *)scratch;
    QbArgs b;
    QdArgs &a = b.d;
    a = QdArgs{};
    a.m = *M;
    a.x = x; a.out = out; a.idx = idx; a.w = w; a.rows = rows;
    a.umax = rows * M->K < M->E ? rows * M->K : M->E;
    a.lgG = G == 32 ? 5 : G == 64 ? 6 : 7;
    const int rpb = QD_WAVES * (64 / lpr_h);
    const int vbytes = (M->H / 16) * QW_Q16_BYTES;
    a.tch = QD_LDS / vbytes < rows ? QD_LDS / vbytes : rows;
    a.n_sh = (M->SI + rpb - 1) / rpb;
    a.gu_wg_per_u = (M->I + rpb - 1) / rpb;
    a.n_ex = a.umax * a.gu_wg_per_u;
    a.n_down_rb = (M->H + QD_DOWN_RPG - 1) / QD_DOWN_RPG;
    a.scr = S;
    a.qx = (uint4 *)(S + L.qx);
    a.qact = (uint4 *)(S + L.qact);
    a.qsh = (uint4 *)(S + L.qsh);
    b.logits = (const float *)(S + L.logits);
    b.tab = (int32_t *)(S + L.tab);
    const qwk_q4 g0 = M->split ? M->gate : M->gate_up, u0 = qb_up_bank(M);
    const int npk = rows * M->K;
    b.gmm = qb_gmm(M);
    b.perm = (int32_t *)(S + L.perm);
    b.tiles = (int32_t *)(S + L.tiles);
    b.act = (const float *)(S + L.act);
    b.xh = (uint16_t *)(S + L.xh);
    b.xF = (float *)(S + L.xF);
    const size_t xs_bytes = (size_t)a.tch * vbytes;
    const size_t xa_bytes = ((size_t)(M->SI / 16) + (size_t)M->K * (M->I / 16)) * QW_Q16_BYTES;
    if (a.tch < 1 || xa_bytes > QD_LDS || a.umax > QD_MAXU) return (int)hipErrorInvalidValue;
    // the router logits and the shared expert's gate logits, one launch
    float *lg = (float *)(S + L.logits), *gl = (float *)(b.tab + QB_TAB_GATE);
    // The matrix-core gate / up with the hand-off words at hand: the logits,
    // the f16 staging and the routing in one launch (k_batch_router).
    const int ygroups = (rows + QW_DF_TPG - 1) / QW_DF_TPG, xblocks = (M->E + 1 + QW_DF_WAVES - 1) / QW_DF_WAVES;
    const bool fused = b.gmm && tags && err && epoch && (size_t)rows * M->E <= tag_words && M->H % 64 == 0 &&
                       M->H <= 64 * 64 && rows <= QW_DF_MAXR && ((uintptr_t)M->router & 15u) == 0 &&
                       ((uintptr_t)M->sh_gate_w & 15u) == 0;
    int rc = 0;
    bool staged16 = true;
    b.xstaged = 1;
    if (fused && handoff) *handoff = 1;
    if (!fused) {
        // (which also stages the token rows as q16 for the gate / up launch,
        // or, for the matrix-core gate / up, as f16 rows with a scale each)
        rc = qwk_dmat_bf16_gate(s, lg, gl, x, M->router, M->sh_gate_w, M->H, M->E, rows, b.gmm ? nullptr : a.qx,
                                b.gmm ? b.xh : nullptr, b.gmm ? b.xF : nullptr);
        staged16 = rc == 0;
        if (rc == (int)hipErrorInvalidValue) {   // a layout the one launch does not take: two order-R launches
            b.xstaged = b.gmm;
            rc = qwk_dmat_bf16(s, lg, x, M->router, M->H, M->E, rows);
            if (!rc) rc = qwk_dmat_bf16(s, gl, x, M->sh_gate_w, M->H, 1, rows);
        }
        if (!rc && b.gmm && !staged16) rc = qwk_stage16(s, b.xh, b.xF, x, rows, M->H);
    }
    const size_t few_lds = (size_t)min(rows, QW_DF_TPG) * (M->H / 64) * QW_DF_PAD * sizeof(float);
    const size_t rt_lds = std::max(few_lds, (size_t)rows * M->E * sizeof(float));
    if (rc) return rc;
    const int nrb8 = (a.n_down_rb + 7) / 8 * 8;
    const qwk_gmm_extra xgu = {M->sh_gate, M->sh_up, M->E, npk}, xd = {M->sh_down, M->sh_down, M->E, npk};
    const bool stream = qb_stream(M);
    float *ey = (float *)(S + L.ey);
    // the activations leave the grouped product directly as the down
    // launch's q16 vectors where it takes that form (16-row tiles), else as
    // fp32 for k_batch_act_q16
    const qwk_gmm_q16out q16o = {a.qact, a.qsh, npk};
    const bool q16d = b.gmm && qwk_gmm16_q16_supported(M->H, G, rows);
    const int nvu = (npk + rows) * (M->I / 16);
#define QB_GO(L_, N_, D_, P_)                                                                                   \
    if (lpr_h == L_ && nul_h == N_ && nul_d == D_ && pl == P_) {                                              \
        if (fused)                                                                                            \
            hipLaunchKernelGGL(k_batch_router<P_>, dim3((xblocks + 8) / 8 * 8, ygroups), dim3(QD_MAXT * 64), rt_lds, s, b,\
                               (uint2 *)tags, err, epoch);                                                    \
        else                                                                                                  \
            hipLaunchKernelGGL(k_batch_route<P_>, dim3(1), dim3(QD_MAXT * 64), 0, s, b);                      \
        if (stream) {                                                                                         \
            int rg = qwk_gmm16_stream(s, (float *)b.act, M->I, (const uint16_t *)(S + L.xh),                 \
                                      (const float *)(S + L.xF), nullptr, b.perm, b.tiles, a.umax + 1, g0, u0, \
                                      (long)(M->split ? 1 : 2) * M->I * (M->H / 8),                            \
                                      (long)(M->split ? 1 : 2) * M->I * (M->H / G), M->H, M->I, M->K, 0, G, 1,\
                                      &xgu, nullptr);                                                         \
            if (!rg) rg = qwk_gmm16_stream(s, ey, M->H, nullptr, nullptr, b.act, b.perm, b.tiles, a.umax + 1,   \
                                           M->down, M->down, (long)M->H * (M->I / 8), (long)M->H * (M->I / G), \
                                           M->I, M->H, M->K, 1, G, 0, &xd, nullptr);                          \
            if (!rg) rg = qwk_moe_combine(s, out, ey, w, ey + (size_t)npk * M->H, gl, rows, M->K, M->H);      \
            return rg ? rg : (int)hipGetLastError();                                                          \
        }                                                                                                     \
        if (b.gmm) {                                                                                          \
            const int rg = qwk_gmm16(s, (float *)b.act, M->I, (const uint16_t *)(S + L.xh),                   \
                                     (const float *)(S + L.xF), b.perm, b.tiles, a.umax + 1, g0, u0,           \
                                     (long)(M->split ? 1 : 2) * M->I * (M->H / 8),                             \
                                     (long)(M->split ? 1 : 2) * M->I * (M->H / G), M->H, M->I, M->K, 0, G, 1, \
                                     0, &xgu, rows, q16d ? &q16o : nullptr);                                  \
            if (rg) return rg;                                                                                \
            if (!q16d) hipLaunchKernelGGL(k_batch_act_q16, dim3((nvu + 255) / 256), dim3(256), 0, s, b);      \
        } else {                                                                                              \
            hipLaunchKernelGGL((k_batch_gu<L_, N_>), dim3(a.n_ex + a.n_sh), dim3(QD_THREADS), xs_bytes, s, b);\
        }                                                                                                     \
        hipLaunchKernelGGL(k_batch_down<D_>, dim3(rows * nrb8), dim3(QD_THREADS), xa_bytes, s, b);            \
        return (int)hipGetLastError();                                                                        \
    } else
    QD_SHAPES(QB_GO)
#undef QB_GO
    return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}
