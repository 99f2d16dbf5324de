// qw_qmv.hip -- 4-bit MLX-affine matvecs for decode: one matrix, an expert
// bank addressed per (token, slot) pair, two banks in one launch (gate and
// up), SwiGLU computed on load (down), and up to four matrices sharing one
// input.  HBM-bound: every weight byte is read once, with 16-byte loads.
//
// Plan.  A row of k inputs is S = k/32 segments of 16 bytes (4 words,
// 32 nibbles).  LPR lanes share a row (LPR = the largest power of two <= 64
// dividing S), so one wave instruction reads 64/LPR rows side by side, each
// as one contiguous run of LPR * 16 bytes; a lane walks segments lr, lr+LPR,
// ... of its row.  A wave owns RIT such row slots in turn, and a segment's
// activations, loaded once, serve all of them.
//
// Arithmetic per segment (one quantisation group or half of one):
//   acc += scale * sum_i(q_i * x_i) + bias * sum_i(x_i)
// i.e. the affine map applied after the nibble dot -- the same sum as
// sum_i (scale*q_i + bias) * x_i, in fewer operations.
#include "qw_device.h"
#include "qw_kernels.h"

#define QW_MV_WAVES 4
#define QW_MV_RIT 4
#define QW_MV_MAXMAT 4

struct QwMvArgs {
    float *y[QW_MV_MAXMAT];
    qwk_q4 m[QW_MV_MAXMAT];
    int n[QW_MV_MAXMAT];
    const float *x;
    const float *up;
    const int32_t *idx;
    int xstride, k, pairs, K, x_by_pair;
};

template <int G, int LPR, bool SWIGLU>
__global__ __launch_bounds__(QW_MV_WAVES * 64) void k_q4mv(QwMvArgs a)
{
    constexpr int SLOTS = 64 / LPR;
    constexpr int RPW = SLOTS * QW_MV_RIT;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = lane / LPR, lr = lane % LPR;
    const int z = blockIdx.z, p = blockIdx.y;
    const int n = a.n[z];
    const int row0 = (blockIdx.x * QW_MV_WAVES + wave) * RPW;
    if (row0 >= n) return;

    const int k = a.k, words = k / 8, groups = k / G;
    const size_t e = a.idx ? (size_t)a.idx[p] : 0;
    const uint32_t *wm = a.m[z].w + e * (size_t)n * words;
    const uint16_t *sm = a.m[z].s + e * (size_t)n * groups;
    const uint16_t *bm = a.m[z].b + e * (size_t)n * groups;
    const int xrow = SWIGLU ? p : (a.x_by_pair ? p : p / a.K);
    const float *xr = a.x + (size_t)xrow * a.xstride;
    const float *ur = SWIGLU ? a.up + (size_t)p * a.xstride : nullptr;

    float acc[QW_MV_RIT];
#pragma unroll
    for (int i = 0; i < QW_MV_RIT; i++) acc[i] = 0.0f;

    const int spl = (k / 32) / LPR;
    for (int j = 0; j < spl; j++) {
        const int seg = j * LPR + lr;
        const int g = seg * 32 / G;
        uint4 wv[QW_MV_RIT];
        float sc[QW_MV_RIT], bi[QW_MV_RIT];
#pragma unroll
        for (int i = 0; i < QW_MV_RIT; i++) {
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
        float xs[32];
        const float4 *xv = reinterpret_cast<const float4 *>(xr + seg * 32);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float4 t = xv[q];
            xs[4 * q] = t.x; xs[4 * q + 1] = t.y; xs[4 * q + 2] = t.z; xs[4 * q + 3] = t.w;
        }
        if (SWIGLU) {
            const float4 *uv = reinterpret_cast<const float4 *>(ur + seg * 32);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 t = uv[q];
                xs[4 * q] = qw_silu(xs[4 * q]) * t.x;
                xs[4 * q + 1] = qw_silu(xs[4 * q + 1]) * t.y;
                xs[4 * q + 2] = qw_silu(xs[4 * q + 2]) * t.z;
                xs[4 * q + 3] = qw_silu(xs[4 * q + 3]) * t.w;
            }
        }
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) xsum += xs[i];
#pragma unroll
        for (int i = 0; i < QW_MV_RIT; i++) {
            float d = qw_dot8_q(wv[i].x, xs, 0.0f);
            d = qw_dot8_q(wv[i].y, xs + 8, d);
            d = qw_dot8_q(wv[i].z, xs + 16, d);
            d = qw_dot8_q(wv[i].w, xs + 24, d);
            acc[i] = __builtin_fmaf(sc[i], d, acc[i]);
            acc[i] = __builtin_fmaf(bi[i], xsum, acc[i]);
        }
    }
    float *y = a.y[z] + (size_t)p * n;
#pragma unroll
    for (int i = 0; i < QW_MV_RIT; i++) {
        const float v = qw_xor_sum<LPR>(acc[i]);
        const int row = row0 + slot + SLOTS * i;
        if (lr == 0 && row < n) y[row] = v;
    }
}

// Few rows over a long input (the mixer's down-projection at decode: n = 320,
// k = 4 H), where a wave per RIT rows would leave most CUs idle: a
// workgroup per row slot set, its QW_MV_WAVES waves splitting the segments
// (wave w takes segments w, w + QW_MV_WAVES, ... of each lane's walk), the
// wave partials added in wave order through LDS.  One matrix, one token row,
// no expert index.
template <int G, int LPR>
__global__ __launch_bounds__(QW_MV_WAVES * 64) void k_q4mv_ks(QwMvArgs a)
{
    constexpr int SLOTS = 64 / LPR;
    __shared__ float part[QW_MV_WAVES][SLOTS];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = lane / LPR, lr = lane % LPR;
    const int n = a.n[0], k = a.k, words = k / 8, groups = k / G;
    const int row = blockIdx.x * SLOTS + slot;
    const bool live = row < n;
    const uint32_t *wr = a.m[0].w + (size_t)(live ? row : 0) * words;
    const uint16_t *sr = a.m[0].s + (size_t)(live ? row : 0) * groups;
    const uint16_t *br = a.m[0].b + (size_t)(live ? row : 0) * groups;
    const int spl = (k / 32) / LPR;
    float acc = 0.0f;
    for (int j = wave; j < spl; j += QW_MV_WAVES) {
        const int seg = j * LPR + lr;
        const int g = seg * 32 / G;
        const uint4 wv = *reinterpret_cast<const uint4 *>(wr + seg * 4);
        const float sc = qw_bf16(sr[g]), bi = qw_bf16(br[g]);
        float xs[32];
        const float4 *xv = reinterpret_cast<const float4 *>(a.x + seg * 32);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float4 t = xv[q];
            xs[4 * q] = t.x; xs[4 * q + 1] = t.y; xs[4 * q + 2] = t.z; xs[4 * q + 3] = t.w;
        }
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) xsum += xs[i];
        float d = qw_dot8_q(wv.x, xs, 0.0f);
        d = qw_dot8_q(wv.y, xs + 8, d);
        d = qw_dot8_q(wv.z, xs + 16, d);
        d = qw_dot8_q(wv.w, xs + 24, d);
        acc = __builtin_fmaf(sc, d, acc);
        acc = __builtin_fmaf(bi, xsum, acc);
    }
    acc = qw_xor_sum<LPR>(acc);
    if (lr == 0) part[wave][slot] = acc;
    __syncthreads();
    if (wave == 0 && lr == 0 && live) {
        float v = part[0][slot];
#pragma unroll
        for (int w = 1; w < QW_MV_WAVES; w++) v = v + part[w][slot];
        a.y[0][row] = v;
    }
}

template <int G>
static void launch_ks(int lpr, int n, hipStream_t s, const QwMvArgs &a)
{
    const dim3 blk(QW_MV_WAVES * 64);
    const int slots = 64 / lpr;
    const dim3 grid((unsigned)((n + slots - 1) / slots));
    switch (lpr) {
    case 64: hipLaunchKernelGGL((k_q4mv_ks<G, 64>), grid, blk, 0, s, a); break;
    case 32: hipLaunchKernelGGL((k_q4mv_ks<G, 32>), grid, blk, 0, s, a); break;
    default: hipLaunchKernelGGL((k_q4mv_ks<G, 16>), grid, blk, 0, s, a); break;
    }
}

static int qw_lpr(int k)
{
    const int S = k / 32;
    int l = 1;
    while (l < 64 && S % (2 * l) == 0) l *= 2;
    return l;
}

template <int G, bool SW>
static void launch_lpr(int lpr, dim3 grid, hipStream_t s, const QwMvArgs &a)
{
    const dim3 blk(QW_MV_WAVES * 64);
    switch (lpr) {
    case 64: hipLaunchKernelGGL((k_q4mv<G, 64, SW>), grid, blk, 0, s, a); break;
    case 32: hipLaunchKernelGGL((k_q4mv<G, 32, SW>), grid, blk, 0, s, a); break;
    case 16: hipLaunchKernelGGL((k_q4mv<G, 16, SW>), grid, blk, 0, s, a); break;
    case 8:  hipLaunchKernelGGL((k_q4mv<G, 8, SW>), grid, blk, 0, s, a); break;
    case 4:  hipLaunchKernelGGL((k_q4mv<G, 4, SW>), grid, blk, 0, s, a); break;
    case 2:  hipLaunchKernelGGL((k_q4mv<G, 2, SW>), grid, blk, 0, s, a); break;
    default: hipLaunchKernelGGL((k_q4mv<G, 1, SW>), grid, blk, 0, s, a); break;
    }
}

static int qw_mv_launch(hipStream_t s, const QwMvArgs &a, int nmat, int group, bool swiglu)
{
    const int lpr = qw_lpr(a.k);
    const int rpb = QW_MV_WAVES * (64 / lpr) * QW_MV_RIT;
    int nmax = 0;
    for (int i = 0; i < nmat; i++) nmax = a.n[i] > nmax ? a.n[i] : nmax;
    const dim3 grid((nmax + rpb - 1) / rpb, a.pairs, nmat);
    // Split the segments across a workgroup's waves when the row plan would
    // give under 4 waves a CU and each lane has at least 4 segments to walk.
    if (nmat == 1 && a.pairs == 1 && !a.idx && !swiglu && lpr >= 16 &&
        (long)grid.x * QW_MV_WAVES < 4L * 256 && (a.k / 32) / lpr >= QW_MV_WAVES) {
        if (group == 64) launch_ks<64>(lpr, a.n[0], s, a);
        else if (group == 32) launch_ks<32>(lpr, a.n[0], s, a);
        else if (group == 128) launch_ks<128>(lpr, a.n[0], s, a);
        else return (int)hipErrorInvalidValue;
        return (int)hipGetLastError();
    }
    if (group == 64) {
        if (swiglu) launch_lpr<64, true>(lpr, grid, s, a); else launch_lpr<64, false>(lpr, grid, s, a);
    } else if (group == 32) {
        if (swiglu) launch_lpr<32, true>(lpr, grid, s, a); else launch_lpr<32, false>(lpr, grid, s, a);
    } else if (group == 128) {
        if (swiglu) launch_lpr<128, true>(lpr, grid, s, a); else launch_lpr<128, false>(lpr, grid, s, a);
    } else {
        return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int qwk_q4mv(hipStream_t s, float *y, const float *x, const float *up, int xstride,
                        const int32_t *idx, const qwk_q4 *mats, int nmat,
                        int k, int n, int pairs, int K, int x_by_pair, int group)
{
    if (nmat < 1 || nmat > 2 || k < 32 || k % 32 || group < 32 || k % group || n < 1 ||
        pairs < 1 || K < 1 || xstride % 4 || !aligned16(x) || (up && !aligned16(up)))
        return (int)hipErrorInvalidValue;
    QwMvArgs a = {};
    for (int i = 0; i < nmat; i++) {
        if (!aligned16(mats[i].w)) return (int)hipErrorInvalidValue;
        a.y[i] = y + (size_t)i * pairs * n;
        a.m[i] = mats[i];
        a.n[i] = n;
    }
    a.x = x; a.up = up; a.idx = idx; a.xstride = xstride; a.k = k; a.pairs = pairs;
    a.K = K; a.x_by_pair = x_by_pair;
    return qw_mv_launch(s, a, nmat, group, up != nullptr);
}

extern "C" int qwk_q4mv_multi(hipStream_t s, const float *x, int k, int group, int count,
                              const qwk_q4 *mats, float *const *ys, const int *ns)
{
    if (count < 1 || count > QW_MV_MAXMAT || k < 32 || k % 32 || group < 32 || k % group ||
        !aligned16(x))
        return (int)hipErrorInvalidValue;
    QwMvArgs a = {};
    for (int i = 0; i < count; i++) {
        if (ns[i] < 1 || !aligned16(mats[i].w)) return (int)hipErrorInvalidValue;
        a.y[i] = ys[i]; a.m[i] = mats[i]; a.n[i] = ns[i];
    }
    a.x = x; a.up = nullptr; a.idx = nullptr; a.xstride = k; a.k = k; a.pairs = 1;
    a.K = 1; a.x_by_pair = 1;
    return qw_mv_launch(s, a, count, group, false);
}
