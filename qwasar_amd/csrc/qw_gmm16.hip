// qw_gmm16.hip -- the prefill products on gfx950 MFMA (v_mfma_f32_16x16x32_f16)
// over activations staged once as f16.
//
// Staging (k_stage16).  A row of k activations is scaled by one power of two
// 2^sh chosen so that its largest magnitude lands in [2^14, 2^15), and
// rounded to f16: h = f16(x 2^sh).  The stage keeps F = 2^-sh per row and
// Xh = sum(h) per (row, quantisation group of G).  No input overflows f16;
// f16's normal range then covers every value within 2^-28 of the row's
// largest.  Within every 8-element block the f16 values are stored in the
// order 0,4,1,5,2,6,3,7: the order in which one packed weight word yields its
// nibbles (below), so A and B fragments agree element for element.
//
// Exactness of the weight operand.  A nibble q enters the MFMA as the f16
// value 1024 + q, built from its packed word with one and-or per pair
// ((w >> 4j) & 0x000F000F | 0x64006400).  Per group the MFMA accumulates
// C = sum_i (1024 + q_i) h_i in fp32, and the group's affine map is applied
// to that partial:
//
//   sum_i (s q_i + b) x_i = F (s C + (b - 1024 s) Xh)
//
// so weights carry no rounding; activations carry f16 rounding only.
//
// Tiles.  A workgroup (4 waves) owns up to 32 rows (a tile of one expert's
// pairs, or of dense rows) against 128 weight rows: with SWIGLU, 64 gate and
// the same 64 up features, so gate and up meet in one lane and leave as
// silu(g) * u.  Wave w holds 2 weight tiles of 16 rows against 2 row tiles of
// 16.  K streams in chunks of KC (256 where k allows): the activation chunk
// through double-buffered LDS, the next one's loads in flight while the
// current one runs; each lane's own weight words straight from memory into
// registers, one chunk ahead.  Within a quantisation group of G, lane group
// kg (lanes 16 kg .. 16 kg + 15) holds words [kg G/32, (kg + 1) G/32) of each
// row and MFMA step s of the group takes word kg G/32 + s from every lane
// group, so a step never spans two groups and a chunk's loads cover whole
// 128-byte lines of every weight row at once.
//
// Order of tiles.  Workgroup b runs on XCD b % 8; an expert's column blocks
// stay on one XCD (they share its activation rows in that XCD's L2) and
// consecutive tiles go to consecutive XCDs.
#include "qw_device.h"
#include "qw_kernels.h"

typedef _Float16 g16_h8 __attribute__((ext_vector_type(8)));
typedef float g16_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t g16_u4 __attribute__((ext_vector_type(4)));   // native vectors: selects stay in registers
typedef uint32_t g16_u2 __attribute__((ext_vector_type(2)));

#define G16_BM 32
#define G16_BN 128
#define G16_THREADS 256

// ---- staging ------------------------------------------------------------------------

// One wave per row.  Pass 1: the row's largest magnitude.  Pass 2: lane l
// converts 8-blocks l, l + 64, ...; a group is G / 8 consecutive blocks, so
// G / 8 consecutive lanes, whose sum meets by xor steps.
template <int G>
__global__ __launch_bounds__(G16_THREADS) void k_stage16(_Float16 *__restrict__ h, float *__restrict__ F,
                                                         float *__restrict__ X, const float *__restrict__ x,
                                                         int rows, int k)
{
    constexpr int TPG = G / 8;
    const int row = blockIdx.x * (G16_THREADS / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nb = k / 8;
    const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * k);
    float m = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const float4 lo = xr[2 * b], hi = xr[2 * b + 1];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(lo.x), fabsf(lo.y)), fmaxf(fabsf(lo.z), fabsf(lo.w))));
        m = fmaxf(m, fmaxf(fmaxf(fabsf(hi.x), fabsf(hi.y)), fmaxf(fabsf(hi.z), fabsf(hi.w))));
    }
    m = qw_wave_max(m);
    int sh = 0;
    if (m > 0.0f && m <= 3.40282346638528859812e+38f) {
        sh = 15 - __builtin_amdgcn_frexp_expf(m);
        sh = sh < -126 ? -126 : sh > 126 ? 126 : sh;
    }
    if (lane == 0) F[row] = __builtin_ldexpf(1.0f, -sh);
    g16_h8 *hr = reinterpret_cast<g16_h8 *>(h + (size_t)row * k);
    float *Xr = X + (size_t)row * (k / G);
    for (int b0 = 0; b0 < nb; b0 += 64) {
        const int b = b0 + lane;
        float v[8];
        if (b < nb) {
            const float4 lo = xr[2 * b], hi = xr[2 * b + 1];
            v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
            v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        }
        _Float16 q[8];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            q[j] = (_Float16)__builtin_ldexpf(v[j], sh);
            s += (float)q[j];
        }
        s = qw_xor_sum<TPG>(s);
        if (b < nb) {
            hr[b] = g16_h8{q[0], q[4], q[1], q[5], q[2], q[6], q[3], q[7]};
            if (b % TPG == 0) Xr[b / TPG] = s;
        }
    }
}

// ---- the product ------------------------------------------------------------------

// (w >> 4j) nibble pairs into f16 1024 + q.  Plain C++ (not inline asm, so
// the compiler sees the instruction and keeps its wait states against MFMAs
// still reading registers); with the mask in an SGPR and the f16 1024
// pattern in a VGPR it selects one v_and_or_b32.
__device__ __forceinline__ uint32_t g16_nib(uint32_t w, uint32_t mask, uint32_t magic)
{
    return (w & mask) | magic;
}

struct Gmm16Args {
    float *y;
    long ldy;
    const _Float16 *ah;             // staged A [source rows, k]
    const float *aF, *aX;           // [source rows, k / G]
    const int32_t *perm, *tiles;    // grouped: pair permutation and tile list
    const uint32_t *w0, *w1;        // weight banks (w1: the up rows with SWIGLU)
    const uint16_t *s0, *b0, *s1, *b1;
    long ew, eg;                    // per-expert stride of the banks: words, groups
    int k, n;                       // inner size; output columns (features with SWIGLU)
    int K, x_by_pair;               // grouped A row of pair p: x_by_pair ? p : p / K
    int rows;                       // dense: rows
    int nblk;                       // column blocks per tile
    int nbw;                        // column blocks a workgroup runs back to back
};

#ifndef G16_OCC
#define G16_OCC 2
#endif
template <int G, bool SWIGLU, bool DENSE, int KC>
__global__ __launch_bounds__(G16_THREADS, G16_OCC) void k_gmm16(Gmm16Args a)
{
    constexpr int GPC = KC / G;              // groups per chunk
    constexpr int SPG = G / 32;              // MFMA steps per group (= words a lane holds per group)
    constexpr int WPC = KC / 32;             // words a lane holds per chunk, per weight tile
    constexpr int AST = KC + 8;              // halfs per A row in LDS (pad: conflict-free fragment reads)
    constexpr int AU4 = G16_BM * KC / 8 / G16_THREADS;   // uint4 of A a thread moves per chunk
    static_assert(G <= KC && KC % G == 0 && AU4 >= 1, "chunk shape");
    __shared__ __align__(16) _Float16 As[2][G16_BM][AST];
    __shared__ float Xs[2][G16_BM][GPC];
    __shared__ float Fr[G16_BM];
    __shared__ int srow[G16_BM], drow[G16_BM];

    // Workgroup b: XCD b % 8; tile (r / ng) * 8 + b % 8 and column blocks
    // [nb0, nb0 + nitems) with r = b / 8, run as one stream of chunks.
    const int bid = blockIdx.x, xcd = bid & 7, r = bid >> 3, ngr = (a.nblk + a.nbw - 1) / a.nbw;
    const int tile = (r / ngr) * 8 + xcd, nb0 = (r % ngr) * a.nbw, nitems = min(a.nbw, a.nblk - nb0);
    int expert, first, len;
    if (DENSE) {
        first = tile * G16_BM;
        if (first >= a.rows) return;
        expert = 0;
        len = min(G16_BM, a.rows - first);
    } else {
        if (tile >= a.tiles[0]) return;
        expert = a.tiles[1 + 3 * tile];
        first = a.tiles[2 + 3 * tile];
        len = a.tiles[3 + 3 * tile];
    }
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, ln = lane & 15, kg = lane >> 4;
    const int k = a.k, words = k / 8, groups = k / G, nch = k / KC, T = nitems * nch;
    if (t < G16_BM) {
        int sr = -1, dr = -1;
        if (t < len) {
            const int p = DENSE ? first + t : a.perm[first + t];
            sr = DENSE ? p : (a.x_by_pair ? p : p / a.K);
            dr = p;
        }
        srow[t] = sr;
        drow[t] = dr;
        Fr[t] = sr >= 0 ? a.aF[sr] : 0.0f;
    }
    __syncthreads();

    // Loads are buffer loads: a wave-uniform base (a descriptor in SGPRs) and a
    // 32-bit per-lane offset in place of a 64-bit address.
    //
    // Activations: thread t moves AU4 consecutive uint4 of A row t / TPR and
    // (t < 32 GPC) the group sum of row t / GPC.  Loads go to valid (clamped)
    // addresses; rows outside the tile are zeroed by selects.
    constexpr int TPR = KC / 8 / AU4;        // threads per A row
    const int am = t / TPR, aseg = (t % TPR) * AU4 * 8;   // row, first half
    const bool aok = srow[am] >= 0;
    const __amdgpu_buffer_rsrc_t rA = qw_rsrc(a.ah), rX = qw_rsrc(a.aX);
    const uint32_t offA = (uint32_t)(((aok ? srow[am] : 0) * k + aseg) * 2);
    const int xm = t / GPC, xgi = t % GPC;
    const bool xw = t < G16_BM * GPC;
    const int xsrc = xw ? srow[xm] : -1;
    const uint32_t offX = (uint32_t)(((xsrc >= 0 ? xsrc : 0) * groups + xgi) * 4);
    g16_u4 ra[AU4];
    float rx;
    // every fetch is issued, at a chunk clamped to the last: the same loads in
    // every pass, so the waits before each use count exactly
    auto fetch_a = [&](int step) {
        const int c = min(step, T - 1) % nch;
#pragma unroll
        for (int i = 0; i < AU4; i++)
            ra[i] = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rA, offA + c * KC * 2 + 16 * i, 0, 0));
        rx = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rX, offX + c * GPC * 4, 0, 0));
    };
    auto stash_a = [&](int q) {
        const g16_u4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < AU4; i++) *reinterpret_cast<g16_u4 *>(&As[q][am][aseg + 8 * i]) = aok ? ra[i] : z;
        if (xw) Xs[q][xm][xgi] = xsrc >= 0 ? rx : 0.0f;
    };

    // Weights: lane (ln, kg) of wave w owns weight row col(item, nt) of tile
    // nt; per chunk, SPG words of each of the GPC groups, and the groups'
    // scales and biases (GPC consecutive bf16 each).
    __amdgpu_buffer_rsrc_t rW[2], rS[2], rB[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const bool up = SWIGLU && nt == 1;
        rW[nt] = qw_rsrc((up ? a.w1 : a.w0) + (size_t)expert * a.ew);
        rS[nt] = qw_rsrc((up ? a.s1 : a.s0) + (size_t)expert * a.eg);
        rB[nt] = qw_rsrc((up ? a.b1 : a.b0) + (size_t)expert * a.eg);
    }
    auto colof = [&](int item, int nt) {
        const int nb = nb0 + item;
        return SWIGLU ? nb * 64 + wave * 16 + ln : nb * G16_BN + wave * 32 + nt * 16 + ln;
    };
    // wq holds, group by group, the words of the chunk being computed; as
    // soon as group gg is consumed its registers take the next step's group
    // gg (an in-place ring: the loads get the rest of the chunk to land).
    uint32_t wq[2][WPC];
    uint32_t sq[2][(GPC + 1) / 2], bq[2][(GPC + 1) / 2];   // bf16 pairs
    auto fetch_group = [&](int step, int gg) {
        step = min(step, T - 1);
        const int item = step / nch, c = step % nch;
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int col = colof(item, nt), cc = col < a.n ? col : 0;
            const uint32_t o = (uint32_t)((cc * words + kg * SPG + c * (KC / 8) + gg * (G / 8)) * 4);
            if (SPG == 1) wq[nt][gg] = __builtin_amdgcn_raw_buffer_load_b32(rW[nt], o, 0, 0);
            if (SPG == 2) {
                const g16_u2 v = __builtin_bit_cast(g16_u2, __builtin_amdgcn_raw_buffer_load_b64(rW[nt], o, 0, 0));
                wq[nt][2 * gg] = v.x; wq[nt][2 * gg + 1] = v.y;
            }
            if (SPG == 4) {
                const g16_u4 v = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rW[nt], o, 0, 0));
                wq[nt][4 * gg] = v.x; wq[nt][4 * gg + 1] = v.y; wq[nt][4 * gg + 2] = v.z; wq[nt][4 * gg + 3] = v.w;
            }
        }
    };
    // the chunk's GPC scales and biases of each weight tile, as bf16 pairs
    auto fetch_sb = [&](int step) {
        step = min(step, T - 1);
        const int item = step / nch, c = step % nch;
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int col = colof(item, nt), cc = col < a.n ? col : 0;
            const uint32_t o = (uint32_t)((cc * groups + c * GPC) * 2);
            if (GPC == 1) {
                sq[nt][0] = __builtin_amdgcn_raw_buffer_load_b16(rS[nt], o, 0, 0);
                bq[nt][0] = __builtin_amdgcn_raw_buffer_load_b16(rB[nt], o, 0, 0);
            }
            if (GPC == 2) {
                sq[nt][0] = __builtin_amdgcn_raw_buffer_load_b32(rS[nt], o, 0, 0);
                bq[nt][0] = __builtin_amdgcn_raw_buffer_load_b32(rB[nt], o, 0, 0);
            }
            if (GPC == 4) {
                const g16_u2 vs = __builtin_bit_cast(g16_u2, __builtin_amdgcn_raw_buffer_load_b64(rS[nt], o, 0, 0));
                const g16_u2 vb = __builtin_bit_cast(g16_u2, __builtin_amdgcn_raw_buffer_load_b64(rB[nt], o, 0, 0));
                sq[nt][0] = vs.x; sq[nt][1] = vs.y; bq[nt][0] = vb.x; bq[nt][1] = vb.y;
            }
            if (GPC == 8) {
                const g16_u4 vs = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rS[nt], o, 0, 0));
                const g16_u4 vb = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rB[nt], o, 0, 0));
                sq[nt][0] = vs.x; sq[nt][1] = vs.y; sq[nt][2] = vs.z; sq[nt][3] = vs.w;
                bq[nt][0] = vb.x; bq[nt][1] = vb.y; bq[nt][2] = vb.z; bq[nt][3] = vb.w;
            }
        }
    };

    g16_f4 acc[2][2], C[2][2];
    uint32_t magic = 0x64006400u, mask = 0x000F000Fu;
    asm volatile("" : "+v"(magic), "+s"(mask));   // one in a VGPR, one in an SGPR
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) acc[mt][nt] = g16_f4{0.f, 0.f, 0.f, 0.f};

    fetch_a(0);
    stash_a(0);
    fetch_a(1);
#pragma unroll
    for (int gg = 0; gg < GPC; gg++) fetch_group(0, gg);
    fetch_sb(0);
    __syncthreads();

    for (int i = 0; i < T; i++) {
        const int q = i & 1, item = i / nch, c = i % nch;
        // this chunk's scales and biases (kept raw), then the next chunk's in flight
        uint32_t sqc[2][(GPC + 1) / 2], bqc[2][(GPC + 1) / 2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < (GPC + 1) / 2; i++) {
                sqc[nt][i] = sq[nt][i];
                bqc[nt][i] = bq[nt][i];
            }
        fetch_sb(i + 1);
        // Group gg's MFMAs, then group gg - 1's affine epilogue: the epilogue
        // reads partials whose MFMAs had the current group's to finish behind.
        g16_f4 Cp[2][2];
#pragma unroll
        for (int gg = 0; gg <= GPC; gg++) {
            // keeps each group's LDS reads from being hoisted into earlier ones
            __builtin_amdgcn_sched_barrier(0);
            if (gg < GPC) {
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) C[mt][nt] = g16_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < SPG; s++) {
                    g16_h8 bf[2];
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) {
                        uint32_t wd = wq[nt][gg * SPG + s];
                        asm volatile("" : "+v"(wd));      // dequantised here, not ahead of time
                        const g16_u4 u = {g16_nib(wd, mask, magic), g16_nib(wd >> 4, mask, magic),
                                          g16_nib(wd >> 8, mask, magic), g16_nib(wd >> 12, mask, magic)};
                        bf[nt] = __builtin_bit_cast(g16_h8, u);
                    }
                    const int ah = gg * G + 8 * (kg * SPG + s);
#pragma unroll
                    for (int mt = 0; mt < 2; mt++) {
                        const g16_h8 af = *reinterpret_cast<const g16_h8 *>(&As[q][mt * 16 + ln][ah]);
#pragma unroll
                        for (int nt = 0; nt < 2; nt++)
                            C[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[nt], C[mt][nt], 0, 0, 0);
                    }
                }
                fetch_group(i + 1, gg);
            }
            if (gg > 0) {
                const int pg = gg - 1;
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const float sc = __uint_as_float((sqc[nt][pg / 2] >> (16 * (pg % 2))) << 16);
                    const float bc =
                        __builtin_fmaf(-1024.0f, sc, __uint_as_float((bqc[nt][pg / 2] >> (16 * (pg % 2))) << 16));
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float xg = Xs[q][mt * 16 + 4 * kg + e][pg];
                            acc[mt][nt][e] = __builtin_fmaf(sc, Cp[mt][nt][e], __builtin_fmaf(bc, xg, acc[mt][nt][e]));
                        }
                }
            }
            if (gg < GPC) {
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) Cp[mt][nt] = C[mt][nt];
            }
        }
        if (c == nch - 1) {
            // the item is done: out, y = F (acc), with SWIGLU silu(F g) * (F u)
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = mt * 16 + 4 * kg + e;
                    const int dr = drow[m];
                    if (dr >= 0) {
                        const float f = Fr[m];
                        float *yr = a.y + (size_t)dr * a.ldy;
                        if (SWIGLU) {
                            const int col = colof(item, 0);
                            if (col < a.n) yr[col] = qw_silu(f * acc[mt][0][e]) * (f * acc[mt][1][e]);
                        } else {
#pragma unroll
                            for (int nt = 0; nt < 2; nt++) {
                                const int col = colof(item, nt);
                                if (col < a.n) yr[col] = f * acc[mt][nt][e];
                            }
                        }
                    }
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) acc[mt][nt][e] = 0.0f;
                }
        }
        stash_a(q ^ 1);
        fetch_a(i + 2);
        __syncthreads();
    }
}

// ---- host side ---------------------------------------------------------------------

extern "C" int qwk_stage16(hipStream_t s, uint16_t *hb, float *F, float *X, const float *x, int rows, int k,
                           int group)
{
    _Float16 *h = reinterpret_cast<_Float16 *>(hb);
    if (rows < 1 || k < group || k % group || ((uintptr_t)x & 15u) || ((uintptr_t)h & 15u))
        return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + G16_THREADS / 64 - 1) / (G16_THREADS / 64))), blk(G16_THREADS);
    switch (group) {
    case 32: hipLaunchKernelGGL(k_stage16<32>, grid, blk, 0, s, h, F, X, x, rows, k); break;
    case 64: hipLaunchKernelGGL(k_stage16<64>, grid, blk, 0, s, h, F, X, x, rows, k); break;
    case 128: hipLaunchKernelGGL(k_stage16<128>, grid, blk, 0, s, h, F, X, x, rows, k); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

template <int G, int KC>
static void g16_launch(hipStream_t s, const Gmm16Args &a, int swiglu, int dense, unsigned grid)
{
    const dim3 g(grid), b(G16_THREADS);
    if (swiglu && dense) hipLaunchKernelGGL((k_gmm16<G, true, true, KC>), g, b, 0, s, a);
    else if (swiglu) hipLaunchKernelGGL((k_gmm16<G, true, false, KC>), g, b, 0, s, a);
    else if (dense) hipLaunchKernelGGL((k_gmm16<G, false, true, KC>), g, b, 0, s, a);
    else hipLaunchKernelGGL((k_gmm16<G, false, false, KC>), g, b, 0, s, a);
}

extern "C" int qwk_gmm16(hipStream_t s, float *y, long ldy, const uint16_t *ahb, const float *aF,
                         const float *aX, const int32_t *perm, const int32_t *tiles, int max_tiles,
                         qwk_q4 m0, qwk_q4 m1, long ew, long eg, int k, int n, int K, int x_by_pair,
                         int group, int swiglu, int dense_rows)
{
    // chunks of G16_KC where k allows, else 64 (groups up to 64)
#ifndef G16_KC
#define G16_KC 256
#endif
    const int kc = k % G16_KC == 0 ? G16_KC : 64;
    if (k < 64 || k % kc || n < 1 || (group != 32 && group != 64 && group != 128) || group > kc ||
        ((uintptr_t)ahb & 15u) || ((uintptr_t)m0.w & 15u) || (swiglu && ((uintptr_t)m1.w & 15u)))
        return (int)hipErrorInvalidValue;
    const _Float16 *ah = reinterpret_cast<const _Float16 *>(ahb);
    const bool dense = dense_rows > 0;
    if (!dense && (!perm || !tiles || K < 1)) return (int)hipErrorInvalidValue;
    Gmm16Args a;
    a.y = y; a.ldy = ldy; a.ah = ah; a.aF = aF; a.aX = aX; a.perm = perm; a.tiles = tiles;
    a.w0 = m0.w; a.s0 = m0.s; a.b0 = m0.b;
    a.w1 = swiglu ? m1.w : m0.w; a.s1 = swiglu ? m1.s : m0.s; a.b1 = swiglu ? m1.b : m0.b;
    a.ew = ew; a.eg = eg; a.k = k; a.n = n; a.K = K; a.x_by_pair = x_by_pair; a.rows = dense_rows;
    a.nblk = swiglu ? (n + 63) / 64 : (n + G16_BN - 1) / G16_BN;
    const int ntiles = dense ? (dense_rows + G16_BM - 1) / G16_BM : max_tiles;
    if (ntiles <= 0) return 0;
    // column blocks per workgroup: long streams, but enough workgroups to
    // fill the chip (max_tiles bounds the grouped tile count from above)
    {
        const long per = (long)ntiles * a.nblk / 1024;
        a.nbw = per < 1 ? 1 : per > 8 ? 8 : (int)per;
        if (a.nbw > a.nblk) a.nbw = a.nblk;
    }
    // tile = (r / ngr) * 8 + b % 8 with r = b / 8: a multiple of 8 tiles
    const int ngr = (a.nblk + a.nbw - 1) / a.nbw;
    const unsigned grid = (unsigned)(ngr * ((ntiles + 7) / 8) * 8);
    if (kc == G16_KC) {
        switch (group) {
        case 32: g16_launch<32, G16_KC>(s, a, swiglu, dense, grid); break;
        case 64: g16_launch<64, G16_KC>(s, a, swiglu, dense, grid); break;
        default: g16_launch<128, G16_KC>(s, a, swiglu, dense, grid); break;
        }
    } else {
        switch (group) {
        case 32: g16_launch<32, 64>(s, a, swiglu, dense, grid); break;
        default: g16_launch<64, 64>(s, a, swiglu, dense, grid); break;
        }
    }
    return (int)hipGetLastError();
}
