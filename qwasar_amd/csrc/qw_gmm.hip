// qw_gmm.hip -- the grouped (per-expert) 4-bit GEMM for prefill, on gfx950
// MFMA (v_mfma_f32_16x16x32_f16), and its dense twin for the shared expert.
//
// Per workgroup: one tile of up to BM pairs routed to one expert (gathered
// through perm) against a 64-row block of that expert's weights.  Four waves
// each own 16 weight rows and all BM token rows.
//
// Exactness of the weight operand.  A nibble q is fed to the MFMA as the f16
// value 1024 + q, which is exact, built from the packed word with one shift
// and one and-or per pair ((w >> 4j) & 0x000F000F | 0x64006400).  The MFMA
// sums (1024 + q) * x over one quantisation group in fp32; the group's affine
// map is applied afterwards on the fp32 partial:
//
//   sum_i (s q_i + b) x_i = s * C_g + (b - 1024 s) * X_g,
//   C_g = sum_i (1024 + q_i) x_i,   X_g = sum_i x_i
//
// so the weights enter with no rounding at all.  Activations are rounded to
// f16 (relative error <= 2^-11 per element) -- the only approximation.
//
// k order within an MFMA.  The shift-and-or above leaves a word's nibbles in
// register order 0,4,1,5,2,6,3,7; the activation tile is written to LDS in
// the same order within every 8-element block, so A and B agree.
#include "qw_device.h"
#include "qw_kernels.h"

typedef _Float16 qw_h8 __attribute__((ext_vector_type(8)));
typedef float qw_f4 __attribute__((ext_vector_type(4)));

#define QW_GMM_BN 64
#define QW_GMM_BK 128
#define QW_GMM_THREADS 256
#define QW_GMM_APAD 8            // halves of padding per A row
#define QW_GMM_BSTRIDE 18        // words per B row in LDS (16 + 2: conflict-free b32 reads)

struct QwGmmArgs {
    float *y;
    const float *x;
    const int32_t *perm;
    const int32_t *tiles;
    qwk_q4 m;
    int k, n, K, x_by_pair, rows, nblk;
    int kslice;      // k range of a blockIdx.y slice (k: no split)
    float *part;     // dense split-K: slice s writes part[s][rows][n]
};

union qw_h8u { qw_h8 h; uint32_t u[4]; uint4 v; };

template <int G, int BM, bool DENSE>
__global__ __launch_bounds__(QW_GMM_THREADS) void k_gather_gemm(QwGmmArgs a)
{
    constexpr int MT = BM / 16;
    constexpr int GPS = (QW_GMM_BK / G) > 0 ? QW_GMM_BK / G : 1;   // groups per stage
    __shared__ __align__(16) _Float16 As[BM][QW_GMM_BK + QW_GMM_APAD];
    __shared__ __align__(16) uint32_t Bw[QW_GMM_BN][QW_GMM_BSTRIDE];
    __shared__ float Xb[BM][QW_GMM_BK / 8];
    __shared__ float Xs[BM][GPS];

    // XCD-aware order: consecutive virtual blocks (the n-blocks of one tile,
    // which share its activation rows) land on the same XCD and its L2.
    const unsigned total = gridDim.x, b = blockIdx.x;
    const unsigned v = (total % 8u == 0u) ? (b % 8u) * (total / 8u) + b / 8u : b;
    const int tile = (int)(v / (unsigned)a.nblk), nb = (int)(v % (unsigned)a.nblk);

    int expert, first, len;
    if (DENSE) {
        first = tile * BM;
        if (first >= a.rows) return;
        expert = 0;
        len = min(BM, a.rows - first);
    } else {
        if (tile >= a.tiles[0]) return;
        expert = a.tiles[1 + 3 * tile];
        first = a.tiles[2 + 3 * tile];
        len = a.tiles[3 + 3 * tile];
    }
    const int k = a.k, n = a.n, words = k / 8, groups = k / G;
    const int n0 = nb * QW_GMM_BN;
    const int kb = (int)blockIdx.y * a.kslice, ke = min(k, kb + a.kslice);
    const uint32_t *wb = a.m.w + (size_t)expert * n * words;
    const uint16_t *sb = a.m.s + (size_t)expert * n * groups;
    const uint16_t *bb = a.m.b + (size_t)expert * n * groups;

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int ln = lane & 15, lg = lane >> 4;
    const int col = n0 + wave * 16 + ln;                 // this lane's weight row

    qw_f4 acc[MT], C[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        acc[mt] = qw_f4{0.f, 0.f, 0.f, 0.f};
        C[mt] = acc[mt];
    }

    for (int k0 = kb; k0 < ke; k0 += QW_GMM_BK) {
        const int klen = min(QW_GMM_BK, ke - k0);
        // Activations: 8-element blocks, f16, written in nibble register order.
        for (int blk = t; blk < BM * (QW_GMM_BK / 8); blk += QW_GMM_THREADS) {
            const int m = blk / (QW_GMM_BK / 8), bk = blk % (QW_GMM_BK / 8);
            qw_h8u h;
            float bsum = 0.0f;
            if (m < len && bk * 8 < klen) {
                const int p = DENSE ? first + m : a.perm[first + m];
                const int xr = DENSE ? p : (a.x_by_pair ? p : p / a.K);
                const float4 *xv = reinterpret_cast<const float4 *>(a.x + (size_t)xr * k + k0 + bk * 8);
                const float4 lo = xv[0], hi = xv[1];
                const float f[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                _Float16 q[8];
#pragma unroll
                for (int i = 0; i < 8; i++) { q[i] = (_Float16)f[i]; bsum += (float)q[i]; }
                h.h = qw_h8{q[0], q[4], q[1], q[5], q[2], q[6], q[3], q[7]};
            } else {
                h.v = make_uint4(0, 0, 0, 0);
            }
            *reinterpret_cast<uint4 *>(&As[m][bk * 8]) = h.v;
            Xb[m][bk] = bsum;
        }
        // Weights: 64 rows x 16 words, one 16-byte load per thread.
        {
            const int nn = t >> 2, q4 = t & 3;
            const int gn = n0 + nn, wk = k0 / 8 + q4 * 4;
            uint4 wv = make_uint4(0, 0, 0, 0);
            if (gn < n && q4 * 32 < klen)
                wv = *reinterpret_cast<const uint4 *>(wb + (size_t)gn * words + wk);
            uint2 *dst = reinterpret_cast<uint2 *>(&Bw[nn][q4 * 4]);
            dst[0] = make_uint2(wv.x, wv.y);
            dst[1] = make_uint2(wv.z, wv.w);
        }
        __syncthreads();
        for (int i = t; i < BM * GPS; i += QW_GMM_THREADS) {
            const int m = i / GPS, gi = i % GPS;
            float s = 0.0f;
            for (int j = 0; j < G / 8 && gi * (G / 8) + j < QW_GMM_BK / 8; j++) s += Xb[m][gi * (G / 8) + j];
            Xs[m][gi] = s;
        }
        __syncthreads();

        const int nsteps = klen / 32;
        for (int s = 0; s < nsteps; s++) {
            const int kk = k0 + 32 * s;
            if (kk % G == 0) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) C[mt] = qw_f4{0.f, 0.f, 0.f, 0.f};
            }
            const uint32_t wd = Bw[wave * 16 + ln][4 * s + lg];
            qw_h8u bf;
            bf.u[0] = (wd & 0x000F000Fu) | 0x64006400u;
            bf.u[1] = ((wd >> 4) & 0x000F000Fu) | 0x64006400u;
            bf.u[2] = ((wd >> 8) & 0x000F000Fu) | 0x64006400u;
            bf.u[3] = ((wd >> 12) & 0x000F000Fu) | 0x64006400u;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const qw_h8 af = *reinterpret_cast<const qw_h8 *>(&As[mt * 16 + ln][32 * s + 8 * lg]);
                C[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf.h, C[mt], 0, 0, 0);
            }
            if ((kk + 32) % G == 0 || kk + 32 >= ke) {
                const int gabs = kk / G, gi = (kk - k0) / G;
                float sc = 0.0f, bp = 0.0f;
                if (col < n) {
                    sc = qw_bf16(sb[(size_t)col * groups + gabs]);
                    bp = qw_bf16(bb[(size_t)col * groups + gabs]) - 1024.0f * sc;
                }
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float xg = Xs[mt * 16 + 4 * lg + i][gi];
                        acc[mt][i] = __builtin_fmaf(sc, C[mt][i], __builtin_fmaf(bp, xg, acc[mt][i]));
                    }
                }
            }
        }
        __syncthreads();
    }

    float *yo = DENSE && a.part ? a.part + (size_t)blockIdx.y * a.rows * n : a.y;
    if (col < n) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = mt * 16 + 4 * lg + i;
                if (m < len) {
                    const int row = DENSE ? first + m : a.perm[first + m];
                    yo[(size_t)row * n + col] = acc[mt][i];
                }
            }
        }
    }
}

// y[i] = part[0][i] + part[1][i] + ... in slice order
__global__ void k_qmm_reduce(float *__restrict__ y, const float *__restrict__ part, long total, int splits)
{
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
        float v = part[i];
        for (int sp = 1; sp < splits; sp++) v = v + part[(size_t)sp * total + i];
        y[i] = v;
    }
}

template <int G, bool DENSE>
static int gmm_bm(int bm, dim3 grid, hipStream_t s, const QwGmmArgs &a)
{
    const dim3 blk(QW_GMM_THREADS);
    switch (bm) {
    case 16: hipLaunchKernelGGL((k_gather_gemm<G, 16, DENSE>), grid, blk, 0, s, a); break;
    case 32: hipLaunchKernelGGL((k_gather_gemm<G, 32, DENSE>), grid, blk, 0, s, a); break;
    case 64: hipLaunchKernelGGL((k_gather_gemm<G, 64, DENSE>), grid, blk, 0, s, a); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

template <bool DENSE>
static int gmm_launch(hipStream_t s, const QwGmmArgs &a, int group, int bm, int ntiles, int splits = 1)
{
    if (ntiles <= 0) return 0;
    const dim3 grid((unsigned)(a.nblk * ntiles), (unsigned)splits);
    switch (group) {
    case 32: return gmm_bm<32, DENSE>(bm, grid, s, a);
    case 64: return gmm_bm<64, DENSE>(bm, grid, s, a);
    case 128: return gmm_bm<128, DENSE>(bm, grid, s, a);
    default: return (int)hipErrorInvalidValue;
    }
}

static bool gmm_shape_ok(const float *x, qwk_q4 m, int k, int n, int group)
{
    return k >= 32 && k % 32 == 0 && n >= 1 && (group == 32 || group == 64 || group == 128) &&
           k % group == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)m.w & 15u) == 0;
}

extern "C" int qwk_gather_gemm(hipStream_t s, float *y, const float *x, const int32_t *perm,
                               const int32_t *tiles, qwk_q4 m, int k, int n, int K, int x_by_pair,
                               int group, int bm, int max_tiles)
{
    if (!gmm_shape_ok(x, m, k, n, group) || K < 1) return (int)hipErrorInvalidValue;
    QwGmmArgs a = {y, x, perm, tiles, m, k, n, K, x_by_pair, 0, (n + QW_GMM_BN - 1) / QW_GMM_BN, k, nullptr};
    return gmm_launch<false>(s, a, group, bm, max_tiles);
}

// Split-K for the dense product when the tiles alone would leave the chip
// under two workgroups a CU: enough k slices for ~QW_QMM_SPLIT_WG workgroups,
// each a whole number of QW_GMM_BK steps (so of quantisation groups) and no
// shorter than QW_QMM_SPLIT_MIN_K.  The plan is a function of the shape only.
#define QW_QMM_SPLIT_BELOW 512
#define QW_QMM_SPLIT_WG 1024
#define QW_QMM_SPLIT_MIN_K 512

static int qmm_bm(int rows) { return rows >= 64 ? 64 : (rows >= 32 ? 32 : 16); }

static int qmm_splits(int k, int n, int rows, int *kslice)
{
    const int bm = qmm_bm(rows);
    const long tiles = (long)((n + QW_GMM_BN - 1) / QW_GMM_BN) * ((rows + bm - 1) / bm);
    *kslice = k;
    if (tiles >= QW_QMM_SPLIT_BELOW) return 1;
    long sp = (QW_QMM_SPLIT_WG + tiles - 1) / tiles;
    if (sp > k / QW_QMM_SPLIT_MIN_K) sp = k / QW_QMM_SPLIT_MIN_K;
    if (sp < 2) return 1;
    const int ks = (int)(((k + sp - 1) / sp + QW_GMM_BK - 1) / QW_GMM_BK * QW_GMM_BK);
    *kslice = ks;
    return (k + ks - 1) / ks;
}

extern "C" size_t qwk_qmm_work_bytes(int k, int n, int rows)
{
    int ks;
    const int sp = k > 0 && n > 0 && rows > 0 ? qmm_splits(k, n, rows, &ks) : 1;
    return sp > 1 ? (size_t)sp * rows * n * sizeof(float) : 0;
}

extern "C" int qwk_qmm(hipStream_t s, float *y, const float *x, qwk_q4 m, int k, int n, int rows, int group,
                       void *work, size_t work_bytes)
{
    if (!gmm_shape_ok(x, m, k, n, group) || rows < 1) return (int)hipErrorInvalidValue;
    const int bm = qmm_bm(rows);
    int ks;
    int sp = qmm_splits(k, n, rows, &ks);
    if (sp > 1 && (!work || work_bytes < qwk_qmm_work_bytes(k, n, rows) || ((uintptr_t)work & 15u))) {
        sp = 1;
        ks = k;
    }
    QwGmmArgs a = {y, x, nullptr, nullptr, m, k, n, 1, 1, rows, (n + QW_GMM_BN - 1) / QW_GMM_BN, ks,
                   sp > 1 ? static_cast<float *>(work) : nullptr};
    int rc = gmm_launch<true>(s, a, group, bm, (rows + bm - 1) / bm, sp);
    if (rc || sp == 1) return rc;
    const long total = (long)rows * n;
    const long want = (total + 255) / 256;
    hipLaunchKernelGGL(k_qmm_reduce, dim3((unsigned)(want < 4096 ? want : 4096)), dim3(256), 0, s, y,
                       static_cast<const float *>(work), total, sp);
    return (int)hipGetLastError();
}
