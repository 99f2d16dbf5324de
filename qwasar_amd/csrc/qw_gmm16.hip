// qw_gmm16.hip -- the prefill products on gfx950 MFMA (v_mfma_f32_16x16x32_f16)
// over activations staged once as f16.
//
// Staging (k_stage16).  A row of k activations is scaled by one power of two
// 2^sh chosen so that its largest magnitude lands in [2^14, 2^15), and
// rounded to f16: h = f16(x 2^sh); the stage keeps F = 2^-sh per row.  No
// input overflows f16; f16's normal range then covers every value within
// 2^-28 of the row's largest.  Within every 8-element block the f16 values
// are stored in the order 0,4,1,5,2,6,3,7: the order in which one packed
// weight word yields its nibble pairs (below), so A and B fragments agree
// element for element.
//
// Weight operand.  Each packed word is dequantised in registers to four f16
// pairs w = s q + b (one rounding each, g16_dq) and fed to the MFMA as the
// B fragment; accumulation is fp32 across all of k, and the output row is
// scaled by F at the end.  Activations and weights both carry one f16
// rounding.
//
// Tiles.  A workgroup (8 waves, one a CU) owns up to 64 rows (a tile of one
// expert's pairs, or of dense rows) against 512 weight rows: with SWIGLU,
// 256 gate and the same 256 up features, so gate and up meet in one lane and
// leave as silu(g) * u.  Wave w holds 4 weight tiles of 16 rows against 4
// row tiles of 16.  K streams in chunks of KC (256 where k allows):
//   activations  through double-buffered LDS, loaded two chunks ahead;
//   weights      each lane's own words straight into registers, a ring
//                refilled with the next chunk's words as soon as a load
//                group is dequantised;
//   scales and   blocks of up to 16 groups a row, loaded straight into LDS
//   biases       (buffer loads with the lds bit), one block ahead.
// Per chunk lane group kg (lanes 16 kg .. 16 kg + 15) holds KC / 4
// consecutive k of each of its weight rows (one quantisation group when
// G = KC / 4), so the 4 lane groups' loads cover whole 128-byte lines.  MFMA
// step s runs while step s + 1's A fragments are read and its words
// dequantised.
//
// Order of tiles.  Workgroup b runs on XCD b % 8.  Each XCD takes a
// contiguous range of tiles, walked with the column block fastest: the
// workgroups resident together on one XCD share activation chunks and (for
// an expert's adjacent tiles) weight lines in that XCD's L2.
#include "qw_device.h"
#include "qw_kernels.h"

typedef _Float16 g16_h8 __attribute__((ext_vector_type(8)));
typedef float g16_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t g16_u4 __attribute__((ext_vector_type(4)));   // native vectors: selects stay in registers
typedef uint32_t g16_u2 __attribute__((ext_vector_type(2)));
typedef _Float16 g16_h2 __attribute__((ext_vector_type(2)));

#define G16_BM 64
#define G16_BN 512
#define G16_THREADS 512

// ---- staging ------------------------------------------------------------------------

// One wave per row.  Pass 1: the row's largest magnitude.  Pass 2: lane l
// converts 8-blocks l, l + 64, ...
__global__ __launch_bounds__(G16_THREADS) void k_stage16(_Float16 *__restrict__ h, float *__restrict__ F,
                                                         const float *__restrict__ x, int rows, int k)
{
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
    for (int b = lane; b < nb; b += 64) {
        const float4 lo = xr[2 * b], hi = xr[2 * b + 1];
        const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        _Float16 q[8];
#pragma unroll
        for (int j = 0; j < 8; j++) q[j] = (_Float16)__builtin_ldexpf(v[j], sh);
        hr[b] = g16_h8{q[0], q[4], q[1], q[5], q[2], q[6], q[3], q[7]};
    }
}

// ---- the product ------------------------------------------------------------------

// One packed word (8 nibbles, k order 0..7) into 4 f16 pairs in the staged
// order (0,4),(1,5),(2,6),(3,7), each w = s q + b rounded once to f16.  The
// and-or puts a nibble pair into the mantissa of an f16 pair whose exponent
// makes the nibble an exact integer offset: 1024 + q for bits 0-3 (ulp 1),
// 64 + q for bits 4-7 (ulp 1/16).  Subtracting the offset is exact; the fma
// rounds once.  lo, hi: the two and-or patterns, kept in VGPRs by the caller
// (with the masks as SGPR literals each and-or reads one scalar).
__device__ __forceinline__ void g16_dq(uint32_t w, g16_h2 s2, g16_h2 b2, uint32_t lo, uint32_t hi,
                                       uint32_t (&o)[4])
{
    const uint32_t w8 = w >> 8;
    const g16_h2 o1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f}, o64 = {(_Float16)-64.0f, (_Float16)-64.0f};
    const g16_h2 q0 = __builtin_bit_cast(g16_h2, (w & 0x000F000Fu) | lo) + o1024;
    const g16_h2 q1 = __builtin_bit_cast(g16_h2, (w & 0x00F000F0u) | hi) + o64;
    const g16_h2 q2 = __builtin_bit_cast(g16_h2, (w8 & 0x000F000Fu) | lo) + o1024;
    const g16_h2 q3 = __builtin_bit_cast(g16_h2, (w8 & 0x00F000F0u) | hi) + o64;
    o[0] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q0, s2, b2));
    o[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q1, s2, b2));
    o[2] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q2, s2, b2));
    o[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q3, s2, b2));
}

// bf16 (low or high half of a word) to an f16 pair holding it twice
__device__ __forceinline__ g16_h2 g16_bf2h2(uint32_t v, int hi)
{
    const _Float16 h = (_Float16)__uint_as_float(hi ? (v & 0xFFFF0000u) : (v << 16));
    return g16_h2{h, h};
}

struct Gmm16Args {
    float *y;
    long ldy;
    const _Float16 *ah;             // staged A [source rows, k]
    const float *aF;                // [source rows]: the stage's per-row scale
    const int32_t *perm, *tiles;    // grouped: pair permutation and tile list
    const uint32_t *w0, *w1;        // weight banks (w1: the up rows with SWIGLU)
    const uint16_t *s0, *b0, *s1, *b1;
    long ew, eg;                    // per-expert stride of the banks: words, groups
    int k, n;                       // inner size; output columns (features with SWIGLU)
    int K, x_by_pair;               // grouped A row of pair p: x_by_pair ? p : p / K
    int rows;                       // dense: rows
    int nblk;                       // column blocks per tile
    int nbw;                        // column blocks a workgroup runs back to back
    int cpx;                        // CUs an XCD (workgroups one round of items runs at once)
    int gpb;                        // quantisation groups per scale / bias block (1 .. 16)
    // the extra bank: tiles of expert xe use it; pairs p >= xpairs read A row
    // p - xpairs (when not x_by_pair)
    const uint32_t *xw0, *xw1;
    const uint16_t *xs0, *xb0, *xs1, *xb1;
    int xe, xpairs;
    // with SWIGLU, the activations as q16 units instead of fp32: pair p < qnpk
    // into qa[p], pair qnpk + r into qs[r] (vectors of n / 16 units)
    uint4 *qa, *qs;
    int qnpk;
};


template <int G, bool SWIGLU, bool DENSE, int KC, int BM, bool Q16 = false>
__global__ __launch_bounds__(G16_THREADS, BM == 64 ? 1 : 2) void k_gmm16(Gmm16Args a)
{
    static_assert(!Q16 || (SWIGLU && !DENSE && BM == 16), "q16 output: grouped SwiGLU, 16-row tiles");
    constexpr int WPL = KC / 32;                         // words (MFMA k steps) per lane per chunk
    constexpr int KPL = WPL * 8;                         // k a lane covers per chunk
    constexpr int NGL = KPL > G ? KPL / G : 1;           // quantisation groups in that span
    constexpr int AST = KC + 8;                          // halfs per A row in LDS (pad: conflict-free reads)
    constexpr int AU4 = BM * KC / 8 / G16_THREADS;   // uint4 of A a thread moves per chunk
    static_assert(NGL <= 2 && AU4 >= 1 && (WPL == 2 || WPL == 4 || WPL == 8), "chunk shape");
    static_assert(BM * (KC + 8) < 65536, "LDS offsets of A fit 16 bits");
    static_assert(G16_THREADS == G16_BN, "a thread per weight row loads the scale / bias blocks");
    __shared__ __align__(16) _Float16 As[2][BM][AST];
    // scale / bias blocks (below): 4 regions of 16 bytes a row, 2 for 16-row
    // tiles (whose blocks the host keeps to at most 8 groups of 16-byte runs)
    __shared__ __align__(16) uint8_t Sb[2][(BM == 64 ? 4 : 2) * G16_BN * 16];
    __shared__ float Fr[BM];
    __shared__ int srow[BM], drow[BM];
    // with q16 output (16-row tiles, one item a workgroup): the item's
    // activations, fp32, until the last step is done
    __shared__ float Lq[Q16 ? BM : 1][Q16 ? G16_BN / 2 : 1];

    // Workgroup b runs on XCD b % 8 (round-robin dispatch).  Each XCD takes a
    // contiguous range of tiles, and with r = b / 8 its workgroups walk
    // (tile, column group) with the column group fastest.  Workgroups that
    // run together on one XCD then share each activation chunk, and the
    // tiles of one expert (adjacent in the list) share its weights, in that
    // XCD's L2.  A workgroup runs column blocks [nb0, nb0 + nitems) as one
    // stream of chunks.
    //
    // The items of an XCD (its tiles times their column groups) run on its
    // cpx CUs in rounds.  The items past the last whole round are cut into
    // shorter ones, so a part-filled last round holds short items spread
    // over more CUs rather than whole ones on a few: into single column
    // blocks; single blocks, when twice their number fits the CUs, into
    // halves (half the weight rows: each wave owns 2 weight tiles of 16, not
    // 4), and those, when twice their number fits again, into the tile's row
    // halves.
    const int bid = blockIdx.x, xcd = bid & 7, r = bid >> 3, ngr = (a.nblk + a.nbw - 1) / a.nbw;
    const int ntl = DENSE ? (a.rows + BM - 1) / BM : a.tiles[0];
    const int tpx = (ntl + 7) / 8;
    const int items = min(max(ntl - xcd * tpx, 0), tpx) * ngr, full = items - items % a.cpx;
    int tl, nb0, nitems, hc = 0, rh = -1;
    bool half = false;
    if (r < full) {
        tl = r / ngr;
        nb0 = (r % ngr) * a.nbw;
        nitems = min(a.nbw, a.nblk - nb0);
    } else if (a.nbw == 1) {
        const int rem = items - full, cs = 4 * rem <= 2 * a.cpx ? 2 : 1, rs = BM == 64 && cs == 2 && 4 * rem <= a.cpx ? 2 : 1;
        const int per = cs * rs, it = full + (r - full) / per, pc = (r - full) % per;
        if (it >= items) return;
        tl = it / ngr;
        nb0 = it % ngr;
        nitems = 1;
        half = cs == 2;
        hc = half ? pc & 1 : 0;
        rh = rs == 2 ? pc >> 1 : -1;
    } else {
        const int it = full + (r - full) / a.nbw;
        if (it >= items) return;
        tl = it / ngr;
        nb0 = (it % ngr) * a.nbw + (r - full) % a.nbw;
        if (nb0 >= a.nblk) return;
        nitems = 1;
    }
    const int tile = xcd * tpx + tl;
    // NT weight tiles of 16 a wave: the item's BNT weight rows
    auto body = [&](auto ntc) {
    constexpr int NT = decltype(ntc)::value, NH = NT / 2, BNT = NT * 16 * (G16_THREADS / 64);
    int expert, first, len;
    if (DENSE) {
        first = tile * BM;
        expert = 0;
        len = min(BM, a.rows - first);
    } else {
        expert = a.tiles[1 + 3 * tile];
        first = a.tiles[2 + 3 * tile];
        len = a.tiles[3 + 3 * tile];
    }
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, ln = lane & 15, kg = lane >> 4;
    const int k = a.k, words = k / 8, groups = k / G, nch = k / KC, T = nitems * nch;
    const int gpb = a.gpb, sbc = gpb * G / KC, nbk = groups / gpb;   // chunks a block, blocks an item
    if (t < BM) {
        int sr = -1, dr = -1;
        if (t < len && (rh < 0 || (t >> 5) == rh)) {
            const int p = DENSE ? first + t : a.perm[first + t];
            sr = DENSE ? p : (a.x_by_pair ? p : (p < a.xpairs ? p / a.K : p - a.xpairs));
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
    // Activations: a chunk is BM rows of KC halfs, LPR 128-byte lines a
    // row.  Load i of thread t takes 16 bytes (t % 8) of line
    // i * (threads / 8) + t / 8, so each load instruction of a wave covers 8
    // whole lines (a cache tag per 128 bytes).  Loads go to valid (clamped)
    // addresses; rows outside the tile are zeroed by selects.
    constexpr int LPR = KC * 2 / 128;
    const __amdgpu_buffer_rsrc_t rA = qw_rsrc(a.ah);
    uint32_t offA[AU4];
    uint16_t ldsA[AU4];
    uint32_t aokm = 0;
#pragma unroll
    for (int i = 0; i < AU4; i++) {
        const int L = i * (G16_THREADS / 8) + (t >> 3), row = L / LPR, seg = L % LPR;
        const int sr = srow[row];
        if (sr >= 0) aokm |= 1u << i;
        // a row outside the tile gets an offset past the descriptor's range:
        // its lanes read zeros without touching memory (the instruction is
        // still issued, so the counted waits below stay exact)
        offA[i] = sr >= 0 ? (uint32_t)((sr * k + seg * 64 + (t & 7) * 8) * 2) : 0x80000000u;
        ldsA[i] = (uint16_t)(row * AST + seg * 64 + (t & 7) * 8);
    }
    g16_u4 ra[AU4];
    // every fetch is issued, at a chunk clamped to the last: the same loads in
    // every pass, so the waits before each use count exactly
    auto fetch_a = [&](int step) {
        const int c = min(step, T - 1) % nch;
#pragma unroll
        for (int i = 0; i < AU4; i++)
            ra[i] = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rA, offA[i] + c * KC * 2, 0, 0));
    };
    auto stash_a = [&](int q) {
        const g16_u4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < AU4; i++)
            *reinterpret_cast<g16_u4 *>(&As[q][0][0] + ldsA[i]) = (aokm >> i) & 1 ? ra[i] : z;
    };

    // Weight rows.  Row j of the workgroup's G16_BN (the LDS row of the scale
    // / bias blocks) is column col(item, j); with SWIGLU rows [0, BN/2) are
    // gate features and [BN/2, BN) the same features of up.  Lane (ln, kg) of
    // wave w owns rows rowof(w, nt) of 4 tiles of 16: with SWIGLU tiles 0, 1
    // are gate and 2, 3 up, so gate and up of a feature meet in one lane.
    __amdgpu_buffer_rsrc_t rW[2], rS[2], rB[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const bool up = SWIGLU && h == 1;
        if (!DENSE && expert == a.xe) {
            rW[h] = qw_rsrc(up ? a.xw1 : a.xw0);
            rS[h] = qw_rsrc(up ? a.xs1 : a.xs0);
            rB[h] = qw_rsrc(up ? a.xb1 : a.xb0);
        } else {
            rW[h] = qw_rsrc((up ? a.w1 : a.w0) + (size_t)expert * a.ew);
            rS[h] = qw_rsrc((up ? a.s1 : a.s0) + (size_t)expert * a.eg);
            rB[h] = qw_rsrc((up ? a.b1 : a.b0) + (size_t)expert * a.eg);
        }
    }
    auto rowof = [&](int nt) {
        return SWIGLU ? (nt / NH) * (BNT / 2) + wave * (NH * 16) + (nt % NH) * 16 + ln : wave * (NT * 16) + nt * 16 + ln;
    };
    auto colof = [&](int item, int j) {
        const int nb = nb0 + item;
        return SWIGLU ? nb * (G16_BN / 2) + hc * (BNT / 2) + (j % (BNT / 2)) : nb * G16_BN + hc * BNT + j;
    };
    // Per chunk, lane kg holds the KPL consecutive k from kg KPL of each of
    // its rows: WPL consecutive words.  MFMA step s takes word s of every
    // lane, so the A fragment of lane group kg is k = c KC + kg KPL + 8 s ...
    // Weight words come in load groups of WGP (one 16- or 8-byte load a
    // row): group lg of chunk `step` into wq[nt][lg WGP ..].
    constexpr int WGP = WPL == 2 ? 2 : 4, NLG = WPL / WGP;
    auto fetch_bg = [&](int step, int lg, uint32_t (&wq)[NT][WPL]) {
        step = min(step, T - 1);
        const int item = step / nch, c = step % nch;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int h = SWIGLU ? nt / NH : 0;
            const int col = colof(item, rowof(nt)), cc = col < a.n ? col : 0;
            const uint32_t o = (uint32_t)((cc * words + c * (KC / 8) + kg * WPL + lg * WGP) * 4);
            if (WGP == 2) {
                const g16_u2 v = __builtin_bit_cast(g16_u2, __builtin_amdgcn_raw_buffer_load_b64(rW[h], o, 0, 0));
                wq[nt][lg * WGP] = v.x; wq[nt][lg * WGP + 1] = v.y;
            } else {
                const g16_u4 v = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rW[h], o, 0, 0));
                wq[nt][lg * WGP] = v.x; wq[nt][lg * WGP + 1] = v.y;
                wq[nt][lg * WGP + 2] = v.z; wq[nt][lg * WGP + 3] = v.w;
            }
        }
    };
    // Scales and biases, a block of gpb groups (sbc chunks) at a time, loaded
    // straight into LDS (buffer loads with the lds bit: no registers, so
    // nothing for the compiler to wait on or copy): thread t moves row t's
    // run of the block, DS bytes a load, for one cache tag per row per block
    // where a per-chunk load takes one per row per chunk.  A load of wave w
    // writes its lanes LS bytes apart, so region j of a block holds
    // [row][LS bytes]: scales in regions [0, nrg), biases in [nrg, 2 nrg).
    // A sub-dword load still puts each lane a dword apart in LDS, so the
    // 2-byte load (one group a block) has LS = 4, its value in the low half.
    // Blocks follow the stream: block beta = item * nbk + c / sbc.
    const int nblocks = nitems * nbk;
    const int DS = gpb >= 8 ? 16 : gpb >= 2 ? 4 : 2, gpr = DS / 2, nrg = gpb / gpr;   // bytes a load, groups a region
    const int LS = DS == 2 ? 4 : DS;                                                   // LDS bytes a row a region
    auto fetch_sb = [&](int beta, int q) {
        beta = min(beta, nblocks - 1);
        const int item = beta / nbk, blk = beta % nbk;
        if (NT < 4 && t >= BNT) return;    // (wave-uniform) no row of this item
        const int h = SWIGLU ? __builtin_amdgcn_readfirstlane(t / (BNT / 2)) : 0;
        const int col = colof(item, t), cc = col < a.n ? col : 0;
        const uint32_t o = (uint32_t)((cc * groups + blk * gpb) * 2);
        // this wave's 64 rows of region j start at j * BN * LS + wave * 64 * LS
        __attribute__((address_space(3))) uint8_t *base =
            (__attribute__((address_space(3))) uint8_t *)(&Sb[q][0]) + wave * 64 * LS;
        for (int j = 0; j < nrg; j++) {
            if (DS == 16) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rS[h], base + j * G16_BN * 16, 16, o + 16 * j, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rB[h], base + (nrg + j) * G16_BN * 16, 16, o + 16 * j, 0, 0, 0);
            } else if (DS == 4) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rS[h], base + j * G16_BN * 4, 4, o + 4 * j, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rB[h], base + (nrg + j) * G16_BN * 4, 4, o + 4 * j, 0, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rS[h], base + j * G16_BN * 4, 2, o + 2 * j, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rB[h], base + (nrg + j) * G16_BN * 4, 2, o + 2 * j, 0, 0, 0);
            }
        }
    };
    // scale / bias of group gl of LDS row j in block buffer q, as bf16 bits
    auto sb_at = [&](int q, int j, int gl, int bias) -> uint32_t {
        const uint8_t *p = &Sb[q][((bias ? nrg : 0) + gl / gpr) * G16_BN * LS + j * LS + (gl % gpr) * 2];
        return *reinterpret_cast<const uint16_t *>(p);
    };
    // loads a step issues after the block's: the weights (the wait before the
    // barrier that publishes a block leaves them in flight)
    constexpr int NBL = NT * (WPL == 2 ? 1 : WPL / 4);

    g16_f4 acc[BM / 16][NT];
#pragma unroll
    for (int mt = 0; mt < BM / 16; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = g16_f4{0.f, 0.f, 0.f, 0.f};
    uint32_t lo = 0x64006400u, hi = 0x54005400u;
    asm volatile("" : "+v"(lo), "+v"(hi));

    // One chunk: MFMAs from As[i & 1], the weights in wq and the scale /
    // bias block in Sb.  MFMA step s runs while step s + 1's A fragments are
    // read and its weight words dequantised; a load group of wq is refilled
    // with the next chunk's words as soon as its last word is dequantised (a
    // ring: every word has a chunk's time to land).  At a block's first chunk
    // the next block's scales and biases are issued; the chunk after next's
    // activations go to registers once this one's are in LDS.
    uint32_t wq[NT][WPL];
    auto step = [&](int i) {
        const int q = i & 1, item = i / nch, c = i % nch;
        const int beta = item * nbk + c / sbc;
        const bool bstart = c % sbc == 0;
        g16_h2 s2[NT][NGL], b2[NT][NGL];
        {
            const int gl = ((c % sbc) * KC + kg * KPL) / G;
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int g = 0; g < NGL; g++) {
                    s2[nt][g] = g16_bf2h2(sb_at(beta & 1, rowof(nt), gl + g, 0), 0);
                    b2[nt][g] = g16_bf2h2(sb_at(beta & 1, rowof(nt), gl + g, 1), 0);
                }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (bstart) fetch_sb(beta + 1, (beta + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        auto lda = [&](int st, g16_h8 (&o)[BM / 16]) {
            const int ah = kg * KPL + 8 * st;
#pragma unroll
            for (int mt = 0; mt < BM / 16; mt++) o[mt] = *reinterpret_cast<const g16_h8 *>(&As[q][mt * 16 + ln][ah]);
        };
        auto dqs = [&](int st, g16_h8 (&o)[NT]) {
            const int g = NGL == 1 ? 0 : st * 8 / G;
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                uint32_t d[4];
                g16_dq(wq[nt][st], s2[nt][g], b2[nt][g], lo, hi, d);
                o[nt] = __builtin_bit_cast(g16_h8, g16_u4{d[0], d[1], d[2], d[3]});
            }
        };
        g16_h8 af[2][BM / 16], bf[2][NT];
        lda(0, af[0]);
        dqs(0, bf[0]);
#pragma unroll
        for (int st = 0; st < WPL; st++) {
            const int cu = st & 1;
            if (st + 1 < WPL) {
                lda(st + 1, af[cu ^ 1]);
                dqs(st + 1, bf[cu ^ 1]);
            }
#pragma unroll
            for (int mt = 0; mt < BM / 16; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[cu][mt], bf[cu][nt], acc[mt][nt], 0, 0, 0);
            // word st + 1 was a load group's last: refill the group
            if (st + 1 < WPL && (st + 2) % WGP == 0) {
                __builtin_amdgcn_sched_barrier(0);
                fetch_bg(i + 1, (st + 1) / WGP, wq);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (c == nch - 1) {
            // the item is done: out, y = F acc, with SWIGLU silu(F g) * (F u)
#pragma unroll
            for (int mt = 0; mt < BM / 16; mt++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = mt * 16 + 4 * kg + e;
                    const int dr = drow[m];
                    if (dr >= 0) {
                        const float f = Fr[m];
                        float *yr = a.y + (size_t)dr * a.ldy;
                        if constexpr (Q16) {
                            // (into LDS: the q16 units are made after the last step)
#pragma unroll
                            for (int nt = 0; nt < NH; nt++) {
                                const int col = colof(item, rowof(nt));
                                if (col < a.n) Lq[m][col & (G16_BN / 2 - 1)] = qw_silu(f * acc[mt][nt][e]) * (f * acc[mt][nt + NH][e]);
                            }
                        } else if (SWIGLU) {
#pragma unroll
                            for (int nt = 0; nt < NH; nt++) {
                                const int col = colof(item, rowof(nt));
                                if (col < a.n) yr[col] = qw_silu(f * acc[mt][nt][e]) * (f * acc[mt][nt + NH][e]);
                            }
                        } else {
#pragma unroll
                            for (int nt = 0; nt < NT; nt++) {
                                const int col = colof(item, rowof(nt));
                                if (col < a.n) yr[col] = f * acc[mt][nt][e];
                            }
                        }
                    }
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) acc[mt][nt][e] = 0.0f;
                }
        }
        // with at most 2 chunks an item, the two buffers hold every chunk
        // once step 0 has stashed chunk 1, and the tile's rows are the same
        // for every item: the activations are not read again
        if (nch > 2 || i == 0) stash_a(q ^ 1);
        // the next block's scales and biases landed in LDS (the weights
        // issued after them stay in flight) before the barrier publishes them
        if (bstart) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NBL) : "memory");
        if (nch > 2) fetch_a(i + 2);
        __syncthreads();
    };

    // the same issue order as a step's (scales and biases, weights, then
    // activations two ahead), so the loop head waits for the same loads from
    // either side
    fetch_a(0);
    fetch_sb(0, 0);
#pragma unroll
    for (int lg = 0; lg < NLG; lg++) fetch_bg(0, lg, wq);
    stash_a(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NBL) : "memory");
    fetch_a(1);
    __syncthreads();
    for (int i = 0; i < T; i++) step(i);
    if constexpr (Q16) {
        {
            // the item's q16 units: row m, 16 features from the item's first
            __syncthreads();
            const int units = a.n >> 4, c0 = colof(0, 0), upr = (BNT / 2) / 16;
            for (int q = t; q < BM * upr; q += G16_THREADS) {
                const int m = q / upr, uu = q % upr, dr = drow[m];
                const int col = c0 + 16 * uu;
                if (dr < 0 || col >= a.n) continue;
                float v[16];
#pragma unroll
                for (int z = 0; z < 16; z++) v[z] = Lq[m][(col & (G16_BN / 2 - 1)) + z];
                uint4 *qv = (dr < a.qnpk ? a.qa + (size_t)dr * units * 3 : a.qs + (size_t)(dr - a.qnpk) * units * 3) +
                            (size_t)(col >> 4) * 3;
                qw_q16_stage(v, qv);
            }
        }
    }
    };
    if (half) body(std::integral_constant<int, 2>{});
    else body(std::integral_constant<int, 4>{});
}

// ---- the batch decode's gate / up: one stream a wave ------------------------------
//
// Grouped SwiGLU with tiles of at most 16 rows and q16 output (a decode
// batch: a tile is one unique expert's pairs, or the shared expert's token
// rows), where the bytes are the experts' weights, each read once.  The
// product above moves them in chunk steps its 8 waves take together (the
// activation chunk through LDS, the scale / bias blocks by DMA, a barrier a
// chunk), so each of its loads waits behind the others and a workgroup holds
// about one chunk in flight.  Here:
//   - a workgroup (8 waves) owns one tile and 128 features; it stages the
//     tile's rows (all of k) and its 256 weight rows' scales and biases (four
//     contiguous runs) in LDS once, and from then on its waves never wait
//     for one another;
//   - wave w owns features f0 = 16 (8 fb + w) .. f0 + 15: its 16 gate and 16
//     up rows, a weight tile of 16 each, with the product's lane layout
//     (lane group kg holds k from kg 64 of each 256-chunk, 8 words);
//   - a chunk's words load into one slot of a D-slot register ring and are
//     consumed D chunks later: every wait in the loop is a counted one on the
//     words of one chunk;
//   - the 16 features of a row are one q16 unit of the down launch: the wave
//     makes its rows' units itself.
// Scales and biases are not loaded a chunk at a time: a 2-byte load a lane
// touches 16 rows' lines for 32 bytes of use and doubled the requests the
// weights make (11 of 35 us at config 2's batch).
// Workgroup b is item b: tile b / nfb, feature block b % nfb (the items of
// a tile on consecutive XCDs).
// ring slots: two chunks (one and three measured within a microsecond)
constexpr int GS_DEPTH = 2;
// LDS of k_gmm16_stream, for k <= GS_MAXK and k / G <= GS_MAXG: the tile's
// rows (16 of k + 8 halfs), four scale / bias runs (gate s, gate b, up s,
// up b: 128 rows of k / G bf16, a run's stride rounded up to whole 1 KB DMA
// slabs) and the waves' output squares; 153 KB of the CU's 160
#define GS_MAXK 3072
#define GS_MAXG 48
static __host__ __device__ inline int gs_run_stride(int groups) { return (128 * groups * 2 + 1023) / 1024 * 1024; }

template <int G, int D>
__global__ __launch_bounds__(G16_THREADS, 1) void k_gmm16_stream(Gmm16Args a)
{
    constexpr int KC = 256, WPL = 8, KPL = 64, NGL = KPL > G ? KPL / G : 1;
    static_assert(NGL <= 2, "at most two groups a lane a chunk");
    __shared__ __align__(16) _Float16 As[16 * (GS_MAXK + 8)];
    __shared__ __align__(16) uint8_t Sb[4 * 128 * GS_MAXG * 2];
    __shared__ float Lw[(G16_THREADS / 64) * 16 * 17];
    __shared__ float Fr[16];
    __shared__ int srow[16], drow[16];
    const int k = a.k, AST = k + 8, words = k / 8, groups = k / G, nch = k / KC;
    const int RS = gs_run_stride(groups);
    const int nfb = (a.n + 127) / 128, tile = blockIdx.x / nfb, fb = blockIdx.x % nfb;
    if (tile >= a.tiles[0]) return;
    const int expert = a.tiles[1 + 3 * tile], first = a.tiles[2 + 3 * tile], len = a.tiles[3 + 3 * tile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, ln = lane & 15, kg = lane >> 4;
    // the wave's rows: gate and up of features f0 + ln (row j of the block)
    const int f0 = fb * 128 + wave * 16, f = min(f0 + ln, a.n - 1), j = wave * 16 + ln;
    const bool xe = expert == a.xe;
    const __amdgpu_buffer_rsrc_t rW0 = qw_rsrc(xe ? a.xw0 : a.w0 + (size_t)expert * a.ew),
                                 rW1 = qw_rsrc(xe ? a.xw1 : a.w1 + (size_t)expert * a.ew);
    const uint32_t wrow = (uint32_t)(f * words + kg * WPL) * 4;
    uint32_t wq[D][2][WPL];
    // chunk c's words (clamped to the last: the same loads every chunk) into
    // slot z: 4 loads
    auto fetch = [&](int c, auto zc) {
        constexpr int z = decltype(zc)::value;
        c = min(c, nch - 1);
        const uint32_t wo = wrow + (uint32_t)c * (KC / 8) * 4;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const __amdgpu_buffer_rsrc_t rw = h ? rW1 : rW0;
            const g16_u4 v0 = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, 0));
            const g16_u4 v1 = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo + 16, 0, 0));
            wq[z][h][0] = v0.x; wq[z][h][1] = v0.y; wq[z][h][2] = v0.z; wq[z][h][3] = v0.w;
            wq[z][h][4] = v1.x; wq[z][h][5] = v1.y; wq[z][h][6] = v1.z; wq[z][h][7] = v1.w;
        }
    };
    // Start-up.  Loads complete in issue order, and every workgroup starts
    // at once.  The tile's pair order is read first, alone (one barrier);
    // then each wave issues the tile's rows, the scale / bias runs (DMA into
    // LDS) and only then the ring's first D slots.
    if (t < 16) {
        int sr = -1, dr = -1;
        if (t < len) {
            dr = a.perm[first + t];
            sr = a.x_by_pair ? dr : (dr < a.xpairs ? dr / a.K : dr - a.xpairs);
        }
        srow[t] = sr;
        drow[t] = dr;
    }
    __syncthreads();
    constexpr int AREG = 16 * GS_MAXK / 8 / G16_THREADS;   // uint4 a thread at most
    const int au = 16 * words;                          // uint4 of the tile
    g16_u4 ra[AREG];
    const __amdgpu_buffer_rsrc_t rA = qw_rsrc(a.ah);
#pragma unroll
    for (int i = 0; i < AREG; i++) {
        const int u = t + i * G16_THREADS, row = u / words, cw = u % words;
        const int sr = u < au ? srow[row] : -1;
        ra[i] = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(
                    rA, sr >= 0 ? (uint32_t)((sr * k + cw * 8) * 2) : 0x80000000u, 0, 0));
    }
    const int mysr = t < 16 ? srow[t] : -1;
    const float myF = mysr >= 0 ? a.aF[mysr] : 0.0f;
    {
        // run r: rows fb 128 .. of (gate s, gate b, up s, up b), contiguous
        // in its bank; 1 KB slabs a wave instruction (lane l: bytes 16 l ..)
        const int rows = min(128, a.n - fb * 128), rbytes = rows * groups * 2, slabs = RS / 1024;
        const uint32_t off0 = (uint32_t)(fb * 128 * groups * 2);
        for (int q = wave; q < 4 * slabs; q += G16_THREADS / 64) {
            const int r = q / slabs, sl = q % slabs, h = r >> 1;
            const uint16_t *bank = (r & 1) ? (xe ? (h ? a.xb1 : a.xb0) : (h ? a.b1 : a.b0))
                                           : (xe ? (h ? a.xs1 : a.xs0) : (h ? a.s1 : a.s0));
            if (!xe) bank += (size_t)expert * a.eg;
            const int bo = sl * 1024 + lane * 16;
            __attribute__((address_space(3))) uint8_t *dst =
                (__attribute__((address_space(3))) uint8_t *)(&Sb[r * RS + sl * 1024]);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(qw_rsrc(bank), dst, 16,
                                                     bo < rbytes ? off0 + (uint32_t)bo : 0x80000000u, 0, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    fetch(0, std::integral_constant<int, 0>{});
    if constexpr (D > 1) fetch(1, std::integral_constant<int, 1>{});
    if constexpr (D > 2) fetch(2, std::integral_constant<int, 2>{});
    if constexpr (D > 3) fetch(3, std::integral_constant<int, 3>{});
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < AREG; i++) {
        const int u = t + i * G16_THREADS, row = u / words, cw = u % words;
        if (u < au) *reinterpret_cast<g16_u4 *>(&As[row * AST + cw * 8]) = ra[i];
    }
    if (t < 16) Fr[t] = myF;
    // the runs landed (the ring's 4 D loads after them stay in flight)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * D) : "memory");
    __syncthreads();
    if (f0 >= a.n) return;      // (wave-uniform) no features of this wave

    g16_f4 acc[2][2];
#pragma unroll
    for (int jj = 0; jj < 2; jj++)
#pragma unroll
        for (int h = 0; h < 2; h++) acc[jj][h] = g16_f4{0.f, 0.f, 0.f, 0.f};
    uint32_t lo = 0x64006400u, hi = 0x54005400u;
    asm volatile("" : "+v"(lo), "+v"(hi));
    // scale / bias of the lane's row j, group gl, run r (as bf16 bits; two
    // groups in one dword where NGL = 2)
    const uint8_t *sbl = &Sb[j * groups * 2];
    auto sbat = [&](int r, int gl) -> uint32_t {
        const uint8_t *p = sbl + r * RS + gl * 2;
        return NGL == 2 ? *reinterpret_cast<const uint32_t *>(p) : *reinterpret_cast<const uint16_t *>(p);
    };
    auto step = [&](int c, auto zc) {
        constexpr int z = decltype(zc)::value;
        const int gl = (c * KC + kg * KPL) / G;
        g16_h2 s2[2][NGL], b2[2][NGL];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t sv = sbat(2 * h, gl), bv = sbat(2 * h + 1, gl);
#pragma unroll
            for (int g = 0; g < NGL; g++) {
                s2[h][g] = g16_bf2h2(sv, g);
                b2[h][g] = g16_bf2h2(bv, g);
            }
        }
        const _Float16 *ar = &As[ln * AST + c * KC + kg * KPL];
#pragma unroll
        for (int st = 0; st < WPL; st++) {
            const g16_h8 af = *reinterpret_cast<const g16_h8 *>(ar + 8 * st);
            const int g = NGL == 1 ? 0 : st * 8 / G;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint32_t d[4];
                g16_dq(wq[z][h][st], s2[h][g], b2[h][g], lo, hi, d);
                const g16_h8 bf = __builtin_bit_cast(g16_h8, g16_u4{d[0], d[1], d[2], d[3]});
                acc[st & 1][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[st & 1][h], 0, 0, 0);
            }
        }
        fetch(c + D, zc);
    };
    int c = 0;
    for (; c + D <= nch; c += D) {
        step(c, std::integral_constant<int, 0>{});
        if constexpr (D > 1) step(c + 1, std::integral_constant<int, 1>{});
        if constexpr (D > 2) step(c + 2, std::integral_constant<int, 2>{});
        if constexpr (D > 3) step(c + 3, std::integral_constant<int, 3>{});
    }
    if (c < nch) { step(c, std::integral_constant<int, 0>{}); c++; }
    if constexpr (D > 2) if (c < nch) { step(c, std::integral_constant<int, 1>{}); c++; }
    if constexpr (D > 3) if (c < nch) { step(c, std::integral_constant<int, 2>{}); c++; }
    // silu(F g) * (F u) of row 4 kg + e, feature f0 + ln: fp32 into y, or
    // through the wave's LDS square, lane m < 16 then making row m's unit
    float *sq = Lw + wave * 16 * 17;
    if (!a.qa) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = 4 * kg + e;
            const float fr = Fr[m];
            if (m < len && f0 + ln < a.n)
                a.y[(size_t)(first + m) * a.ldy + f0 + ln] =
                    qw_silu(fr * (acc[0][0][e] + acc[1][0][e])) * (fr * (acc[0][1][e] + acc[1][1][e]));
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int m = 4 * kg + e;
        const float fr = Fr[m];
        sq[m * 17 + ln] = qw_silu(fr * (acc[0][0][e] + acc[1][0][e])) * (fr * (acc[0][1][e] + acc[1][1][e]));
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 16) {
        const int dr = drow[lane];
        if (dr >= 0) {
            float v[16];
#pragma unroll
            for (int q = 0; q < 16; q++) v[q] = sq[lane * 17 + q];
            const int units = a.n >> 4;
            uint4 *qv = (dr < a.qnpk ? a.qa + (size_t)dr * units * 3 : a.qs + (size_t)(dr - a.qnpk) * units * 3) +
                        (size_t)(f0 >> 4) * 3;
            qw_q16_stage(v, qv);
        }
    }
}

// The same for the batch's down product: y[p] = A_p . W^T for every pair p
// of a tile (its expert's n output rows over k = I inputs), fp32 out by
// pair, the combine left to the caller.  A workgroup owns one tile and
// GSD_RB output rows; wave w walks its GSD_NB blocks of 16 rows, block bi
// being rows rb0 + 16 (8 bi + w) .. + 15 (the 8 waves read 128 consecutive
// rows at a time), a chunk of k a step, with a GSD_D-step register ring, so
// that a wave dequantises and multiplies one block while the next ones'
// words are in flight.  (With every word requested at once the dequant ran
// as a tail after the last words landed: 18 us against 12.7 us of reads.)
// The tile's rows come in as fp32 activations in slot order (row s of ax:
// the pair at perm[s]) and are staged in LDS as k_stage16 stages rows: one
// power of two a row, f16, the 8-blocks in the weight words' order.
#define GSD_MAXK 1024
#define GSD_MAXG 16
#define GSD_NB 6
#define GSD_D 4
#define GSD_RB (GSD_NB * 16 * (G16_THREADS / 64))
#define GSD_DMA ((2 * GSD_RB * GSD_MAXG * 2 / 1024 + G16_THREADS / 64 - 1) / (G16_THREADS / 64))
static __host__ __device__ inline int gsd_run_stride(int groups) { return (GSD_RB * groups * 2 + 1023) / 1024 * 1024; }

template <int G>
__global__ __launch_bounds__(G16_THREADS, 1) void k_gmm16_stream_down(Gmm16Args a, const float *ax)
{
    constexpr int KC = 256, WPL = 8, KPL = 64, NGL = KPL > G ? KPL / G : 1, D = GSD_D;
    static_assert(NGL <= 2, "at most two groups a lane a chunk");
    __shared__ __align__(16) _Float16 As[16 * (GSD_MAXK + 8)];
    __shared__ __align__(16) uint8_t Sb[2 * GSD_RB * GSD_MAXG * 2];
    __shared__ __align__(16) uint8_t Sd[1024];
    __shared__ float Fr[16];
    __shared__ int drow[16];
    const int k = a.k, AST = k + 8, words = k / 8, groups = k / G, nch = k / KC, RS = gsd_run_stride(groups);
    const int nrb = (a.n + GSD_RB - 1) / GSD_RB, tile = blockIdx.x / nrb, rb0 = (blockIdx.x % nrb) * GSD_RB;
    if (tile >= a.tiles[0]) return;
    const int expert = a.tiles[1 + 3 * tile], first = a.tiles[2 + 3 * tile], len = a.tiles[3 + 3 * tile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, ln = lane & 15, kg = lane >> 4;
    const bool xe = expert == a.xe;
    const __amdgpu_buffer_rsrc_t rW = qw_rsrc(xe ? a.xw0 : a.w0 + (size_t)expert * a.ew);
    const int T = GSD_NB * nch;                       // steps: block bi = s / nch, chunk s % nch
    // Start-up.  The tile's rows are its slots first .. first + len - 1 of
    // ax, so they need no pair order: they are requested first, then the
    // slots' pair ids (wanted only at the end), the scale and bias runs
    // (GSD_DMA 1 KB slabs a wave, a fixed count: the lanes of a slab past
    // the runs read nothing and land in a spare KB) and last the ring's
    // first D steps.  Staging waits for the rows alone.
    constexpr int XB = GSD_MAXK / 8 / 64;
    float4 xv[2][XB][2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int m = wave + 8 * h;
#pragma unroll
        for (int q = 0; q < XB; q++) {
            const int b8 = lane + 64 * q;
            const bool ok = m < len && b8 < words;
            const float4 *src = reinterpret_cast<const float4 *>(ax + (size_t)(ok ? first + m : 0) * k + (ok ? b8 : 0) * 8);
            xv[h][q][0] = ok ? src[0] : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[h][q][1] = ok ? src[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    const int mydr = t < 16 && t < len ? a.perm[first + t] : -1;
    {
        // the runs of the block's rows (contiguous in their banks): slab q
        // of 2 slabs is run q / slabs, its KB q % slabs
        const int rows = min(GSD_RB, a.n - rb0), rbytes = rows * groups * 2, slabs = RS / 1024;
        const uint32_t off0 = (uint32_t)(rb0 * groups * 2);
#pragma unroll
        for (int i = 0; i < GSD_DMA; i++) {
            const int q = wave + 8 * i, r = q / slabs, sl = q % slabs, bo = sl * 1024 + lane * 16;
            const bool in = q < 2 * slabs;
            const uint16_t *bank = r ? (xe ? a.xb0 : a.b0 + (size_t)expert * a.eg) : (xe ? a.xs0 : a.s0 + (size_t)expert * a.eg);
            __attribute__((address_space(3))) uint8_t *dst =
                (__attribute__((address_space(3))) uint8_t *)(in ? &Sb[r * RS + sl * 1024] : &Sd[0]);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(qw_rsrc(in ? bank : a.s0), dst, 16,
                                                     in && bo < rbytes ? off0 + (uint32_t)bo : 0x80000000u, 0, 0, 0);
        }
    }
    // the ring: step s's words (block s / nch, chunk s % nch) into slot z, 2 loads
    uint32_t wq[D][WPL];
    auto rowof = [&](int bi) { return min(rb0 + 16 * (8 * bi + wave) + ln, a.n - 1); };
    auto fetch = [&](int st, auto zc) {
        constexpr int z = decltype(zc)::value;
        st = min(st, T - 1);
        const int bi = st / nch, c = st % nch;
        const uint32_t wo = (uint32_t)(rowof(bi) * words + c * (KC / 8) + kg * WPL) * 4;
        const g16_u4 v0 = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rW, wo, 0, 0));
        const g16_u4 v1 = __builtin_bit_cast(g16_u4, __builtin_amdgcn_raw_buffer_load_b128(rW, wo + 16, 0, 0));
        wq[z][0] = v0.x; wq[z][1] = v0.y; wq[z][2] = v0.z; wq[z][3] = v0.w;
        wq[z][4] = v1.x; wq[z][5] = v1.y; wq[z][6] = v1.z; wq[z][7] = v1.w;
    };
    __builtin_amdgcn_sched_barrier(0);
    fetch(0, std::integral_constant<int, 0>{});
    fetch(1, std::integral_constant<int, 1>{});
    fetch(2, std::integral_constant<int, 2>{});
    fetch(3, std::integral_constant<int, 3>{});
    __builtin_amdgcn_sched_barrier(0);
    // stage: one power of two a row (its largest magnitude into [2^14,
    // 2^15)), f16, each 8-block in the order 0,4,1,5,2,6,3,7
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int row = wave + 8 * h;
        float mx = 0.0f;
#pragma unroll
        for (int q = 0; q < XB; q++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float4 f = xv[h][q][u];
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
            }
        mx = qw_wave_max(mx);
        int sh = 0;
        if (mx > 0.0f && mx <= 3.40282346638528859812e+38f) {
            sh = 15 - __builtin_amdgcn_frexp_expf(mx);
            sh = sh < -126 ? -126 : sh > 126 ? 126 : sh;
        }
        if (lane == 0) Fr[row] = row < len ? __builtin_ldexpf(1.0f, -sh) : 0.0f;
#pragma unroll
        for (int q = 0; q < XB; q++) {
            const int b8 = lane + 64 * q;
            if (b8 < words) {
                const float4 lo4 = xv[h][q][0], hi4 = xv[h][q][1];
                const float v[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
                _Float16 hq[8];
#pragma unroll
                for (int jj = 0; jj < 8; jj++) hq[jj] = (_Float16)__builtin_ldexpf(v[jj], sh);
                *reinterpret_cast<g16_h8 *>(&As[row * AST + b8 * 8]) =
                    g16_h8{hq[0], hq[4], hq[1], hq[5], hq[2], hq[6], hq[3], hq[7]};
            }
        }
    }
    if (t < 16) drow[t] = mydr;
    // the runs landed (the ring's 2 D loads after them stay in flight)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * D) : "memory");
    __syncthreads();

    g16_f4 acc[2];
    acc[0] = g16_f4{0.f, 0.f, 0.f, 0.f};
    acc[1] = g16_f4{0.f, 0.f, 0.f, 0.f};
    uint32_t lo = 0x64006400u, hi = 0x54005400u;
    asm volatile("" : "+v"(lo), "+v"(hi));
    int dr4[4];
    float fr4[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        dr4[e] = drow[4 * kg + e];
        fr4[e] = Fr[4 * kg + e];
    }
    auto step = [&](int st, auto zc) {
        constexpr int z = decltype(zc)::value;
        const int bi = st / nch, c = st % nch, j = 16 * (8 * bi + wave) + ln;
        const int gl = (c * KC + kg * KPL) / G;
        const uint8_t *sp = &Sb[(j * groups + gl) * 2];
        const uint32_t sv = NGL == 2 ? *reinterpret_cast<const uint32_t *>(sp) : *reinterpret_cast<const uint16_t *>(sp);
        const uint32_t bv = NGL == 2 ? *reinterpret_cast<const uint32_t *>(sp + RS) : *reinterpret_cast<const uint16_t *>(sp + RS);
        g16_h2 s2[NGL], b2[NGL];
#pragma unroll
        for (int g = 0; g < NGL; g++) {
            s2[g] = g16_bf2h2(sv, g);
            b2[g] = g16_bf2h2(bv, g);
        }
        const _Float16 *ar = &As[ln * AST + c * KC + kg * KPL];
#pragma unroll
        for (int s8 = 0; s8 < WPL; s8++) {
            const g16_h8 af = *reinterpret_cast<const g16_h8 *>(ar + 8 * s8);
            const int g = NGL == 1 ? 0 : s8 * 8 / G;
            uint32_t d[4];
            g16_dq(wq[z][s8], s2[g], b2[g], lo, hi, d);
            const g16_h8 bf = __builtin_bit_cast(g16_h8, g16_u4{d[0], d[1], d[2], d[3]});
            acc[s8 & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[s8 & 1], 0, 0, 0);
        }
        fetch(st + D, zc);
        if (c == nch - 1) {
            // block bi done: y[pair of row 4 kg + e][its output row] = F acc
            const int row = rb0 + 16 * (8 * bi + wave) + ln;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (dr4[e] >= 0 && row < a.n) a.y[(size_t)dr4[e] * a.ldy + row] = fr4[e] * (acc[0][e] + acc[1][e]);
            }
            acc[0] = g16_f4{0.f, 0.f, 0.f, 0.f};
            acc[1] = g16_f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    int st = 0;
    for (; st + D <= T; st += D) {
        step(st, std::integral_constant<int, 0>{});
        step(st + 1, std::integral_constant<int, 1>{});
        step(st + 2, std::integral_constant<int, 2>{});
        step(st + 3, std::integral_constant<int, 3>{});
    }
    if (st < T) { step(st, std::integral_constant<int, 0>{}); st++; }
    if (st < T) { step(st, std::integral_constant<int, 1>{}); st++; }
    if (st < T) { step(st, std::integral_constant<int, 2>{}); st++; }
}

// ---- host side ---------------------------------------------------------------------

extern "C" int qwk_stage16(hipStream_t s, uint16_t *hb, float *F, const float *x, int rows, int k)
{
    _Float16 *h = reinterpret_cast<_Float16 *>(hb);
    if (rows < 1 || k < 8 || k % 8 || ((uintptr_t)x & 15u) || ((uintptr_t)h & 15u))
        return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + G16_THREADS / 64 - 1) / (G16_THREADS / 64))), blk(G16_THREADS);
    hipLaunchKernelGGL(k_stage16, grid, blk, 0, s, h, F, x, rows, k);
    return (int)hipGetLastError();
}

template <int G, int KC, int BM>
static void g16_launch_bm(hipStream_t s, const Gmm16Args &a, int swiglu, int dense, unsigned grid)
{
    const dim3 g(grid), b(G16_THREADS);
    if (swiglu && dense) hipLaunchKernelGGL((k_gmm16<G, true, true, KC, BM>), g, b, 0, s, a);
    else if (swiglu) hipLaunchKernelGGL((k_gmm16<G, true, false, KC, BM>), g, b, 0, s, a);
    else if (dense) hipLaunchKernelGGL((k_gmm16<G, false, true, KC, BM>), g, b, 0, s, a);
    else hipLaunchKernelGGL((k_gmm16<G, false, false, KC, BM>), g, b, 0, s, a);
}
// (16-row tiles: grouped products only, the chunks of 256)
template <int G, int KC>
static void g16_launch(hipStream_t s, const Gmm16Args &a, int swiglu, int dense, unsigned grid, int bm)
{
    if constexpr (KC == 256) {
        if (bm == 16 && !dense) {
            const dim3 g(grid), b(G16_THREADS);
            if (swiglu && a.qa) hipLaunchKernelGGL((k_gmm16<G, true, false, KC, 16, true>), g, b, 0, s, a);
            else if (swiglu) hipLaunchKernelGGL((k_gmm16<G, true, false, KC, 16>), g, b, 0, s, a);
            else hipLaunchKernelGGL((k_gmm16<G, false, false, KC, 16>), g, b, 0, s, a);
            return;
        }
    }
    g16_launch_bm<G, KC, 64>(s, a, swiglu, dense, grid);
}

// CUs an XCD: the device's CUs over its 8 XCDs (of the current device, read
// once; every device this library drives is an MI355X)
static int g16_cus_per_xcd()
{
    static int cpx = 0;
    if (!cpx) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        cpx = n >= 8 ? n / 8 : 1;
    }
    return cpx;
}

// Whether qwk_gmm16 takes this inner size, group and these weight banks
// (as its own checks; the scale / bias block must exist).
extern "C" int qwk_gmm16_supported(int k, int group, const void *w0, const void *w1)
{
    const int kc = k % 256 == 0 ? 256 : 64;
    if (k < 64 || k % kc || (group != 32 && group != 64 && group != 128) || k % group ||
        ((uintptr_t)w0 & 15u) || ((uintptr_t)w1 & 15u))
        return 0;
    const int groups = k / group;
    for (int g = 16; g >= 1; g /= 2)
        if (groups % g == 0 && (g * group) % kc == 0) return 1;
    return 0;
}

// Whether qwk_gmm16 writes q16 activations for a grouped SwiGLU product of
// inner size k and this group with tiles of at most tile_rows rows (16-row
// tiles: chunks of 256, a scale / bias block of at most 8 groups).
extern "C" int qwk_gmm16_q16_supported(int k, int group, int tile_rows)
{
    if (tile_rows > 16 || k % 256 || (group != 32 && group != 64 && group != 128) || k % group) return 0;
    const int groups = k / group;
    for (int g = 8; g >= 1; g /= 2)
        if (groups % g == 0 && (g * group) % 256 == 0) return 1;
    return 0;
}

extern "C" int qwk_gmm16(hipStream_t s, float *y, long ldy, const uint16_t *ahb, const float *aF,
                         const int32_t *perm, const int32_t *tiles, int max_tiles,
                         qwk_q4 m0, qwk_q4 m1, long ew, long eg, int k, int n, int K, int x_by_pair,
                         int group, int swiglu, int dense_rows, const qwk_gmm_extra *xb, int tile_rows,
                         const qwk_gmm_q16out *q16)
{
    // chunks of 256 where k allows, else 64
    const int kc = k % 256 == 0 ? 256 : 64;
    // 16-row tiles (two workgroups a CU) where the caller's tiles hold at most
    // 16 rows and the shapes allow; else 64
    int bm = tile_rows <= 16 && dense_rows <= 0 && kc == 256 ? 16 : 64;
    if (k < 64 || k % kc || n < 1 || (group != 32 && group != 64 && group != 128) || k % group ||
        ((uintptr_t)ahb & 15u) || ((uintptr_t)m0.w & 15u) || (swiglu && ((uintptr_t)m1.w & 15u)))
        return (int)hipErrorInvalidValue;
    const _Float16 *ah = reinterpret_cast<const _Float16 *>(ahb);
    const bool dense = dense_rows > 0;
    if (q16 && (!swiglu || dense || n % 16 || !q16->qa || !q16->qs || tile_rows > 16)) return (int)hipErrorInvalidValue;
    if (!dense && (!perm || !tiles || K < 1)) return (int)hipErrorInvalidValue;
    Gmm16Args a;
    a.y = y; a.ldy = ldy; a.ah = ah; a.aF = aF; a.perm = perm; a.tiles = tiles;
    a.w0 = m0.w; a.s0 = m0.s; a.b0 = m0.b;
    a.w1 = swiglu ? m1.w : m0.w; a.s1 = swiglu ? m1.s : m0.s; a.b1 = swiglu ? m1.b : m0.b;
    a.ew = ew; a.eg = eg; a.k = k; a.n = n; a.K = K; a.x_by_pair = x_by_pair; a.rows = dense_rows;
    if (xb && !dense) {
        if (((uintptr_t)xb->m0.w & 15u) || (swiglu && ((uintptr_t)xb->m1.w & 15u))) return (int)hipErrorInvalidValue;
        a.xw0 = xb->m0.w; a.xs0 = xb->m0.s; a.xb0 = xb->m0.b;
        a.xw1 = swiglu ? xb->m1.w : xb->m0.w; a.xs1 = swiglu ? xb->m1.s : xb->m0.s; a.xb1 = swiglu ? xb->m1.b : xb->m0.b;
        a.xe = xb->expert; a.xpairs = xb->pairs;
    } else {
        a.xw0 = a.xw1 = m0.w; a.xs0 = a.xs1 = m0.s; a.xb0 = a.xb1 = m0.b;
        a.xe = -1; a.xpairs = 0x7FFFFFFF;
    }
    a.qa = q16 ? static_cast<uint4 *>(q16->qa) : nullptr;
    a.qs = q16 ? static_cast<uint4 *>(q16->qs) : nullptr;
    a.qnpk = q16 ? q16->npk : 0;
    a.nblk = swiglu ? (n + G16_BN / 2 - 1) / (G16_BN / 2) : (n + G16_BN - 1) / G16_BN;
    {
        // the largest scale / bias block (groups) that divides a row's groups
        // and ends on a chunk boundary
        const int groups = k / group;
        for (int pass = 0; pass < 2; pass++) {
            a.gpb = 0;
            for (int g = bm == 16 ? 8 : 16; g >= 1 && !a.gpb; g /= 2)
                if (groups % g == 0 && (g * group) % kc == 0) a.gpb = g;
            if (a.gpb || bm == 64) break;
            bm = 64;             // (no block of at most 8 groups ends on a chunk boundary)
        }
        if (!a.gpb || (q16 && bm != 16)) return (int)hipErrorInvalidValue;
    }
    const int ntiles = dense ? (dense_rows + bm - 1) / bm : max_tiles;
    if (ntiles <= 0) return 0;
    // column blocks per workgroup: long streams, but enough workgroups to
    // fill the chip (max_tiles bounds the grouped tile count from above)
    {
        // the largest divisor of nblk up to the target, so every workgroup
        // of a tile runs the same number of blocks
        const long per = (long)ntiles * a.nblk / 1024;
        int nbw = per < 1 ? 1 : per > 8 ? 8 : (int)per;
        if (nbw > a.nblk) nbw = a.nblk;
        while (a.nblk % nbw) nbw--;
        a.nbw = q16 ? 1 : nbw;        // (q16 output: one item a workgroup, its activations held in LDS)
    }
    a.cpx = g16_cus_per_xcd() * (bm == 16 ? 2 : 1);   // workgroups an XCD holds at once
    // r = b / 8 < ngr * ceil(ntiles / 8) covers every XCD's whole items, and
    // cpx * max(nbw, 4) more the pieces of its last round's (fewer than cpx)
    const int ngr = (a.nblk + a.nbw - 1) / a.nbw;
    const unsigned grid = (unsigned)((ngr * ((ntiles + 7) / 8) + a.cpx * (a.nbw > 4 ? a.nbw : 4)) * 8);
    if (kc == 256) {
        switch (group) {
        case 32: g16_launch<32, 256>(s, a, swiglu, dense, grid, bm); break;
        case 64: g16_launch<64, 256>(s, a, swiglu, dense, grid, bm); break;
        default: g16_launch<128, 256>(s, a, swiglu, dense, grid, bm); break;
        }
    } else {
        switch (group) {
        case 32: g16_launch<32, 64>(s, a, swiglu, dense, grid, bm); break;
        case 64: g16_launch<64, 64>(s, a, swiglu, dense, grid, bm); break;
        default: g16_launch<128, 64>(s, a, swiglu, dense, grid, bm); break;
        }
    }
    return (int)hipGetLastError();
}

// The decode batch's grouped products as one weight stream a wave: whether
// the shapes and banks suit them, and the launch.
extern "C" int qwk_gmm16_stream_supported(int k, int n, int group, int swiglu, qwk_q4 m0, qwk_q4 m1,
                                          const qwk_gmm_extra *xb, long eg)
{
    if (group != 32 && group != 64 && group != 128) return 0;
    if (k < 256 || k % 256 || n < 16 || n % 16 || (eg * 2) % 16) return 0;
    if (swiglu ? (k > GS_MAXK || k / group > GS_MAXG) : (k > GSD_MAXK || k / group > GSD_MAXG)) return 0;
    auto al = [](const void *p) { return p && ((uintptr_t)p & 15u) == 0; };
    if (!al(m0.w) || !al(m0.s) || !al(m0.b)) return 0;
    if (swiglu && (!al(m1.w) || !al(m1.s) || !al(m1.b))) return 0;
    if (xb && (!al(xb->m0.w) || !al(xb->m0.s) || !al(xb->m0.b) ||
               (swiglu && (!al(xb->m1.w) || !al(xb->m1.s) || !al(xb->m1.b)))))
        return 0;
    return 1;
}

extern "C" int qwk_gmm16_stream(hipStream_t s, float *y, long ldy, const uint16_t *ah, const float *aF,
                                const float *ax, const int32_t *perm, const int32_t *tiles, int max_tiles,
                                qwk_q4 m0, qwk_q4 m1, long ew, long eg, int k, int n, int K, int x_by_pair,
                                int group, int swiglu, const qwk_gmm_extra *xb, const qwk_gmm_q16out *q16)
{
    if (!qwk_gmm16_stream_supported(k, n, group, swiglu, m0, m1, xb, eg) || !perm || !tiles || K < 1 ||
        (swiglu ? (!ah || !aF || ((uintptr_t)ah & 15u) || (!q16 && !y)) : (!ax || ((uintptr_t)ax & 15u) || !y || q16)) ||
        (q16 && (!q16->qa || !q16->qs)))
        return (int)hipErrorInvalidValue;
    if (max_tiles <= 0) return 0;
    Gmm16Args a{};
    a.y = y; a.ldy = ldy; a.ah = reinterpret_cast<const _Float16 *>(ah); a.aF = aF; a.perm = perm; a.tiles = tiles;
    a.w0 = m0.w; a.s0 = m0.s; a.b0 = m0.b;
    a.w1 = swiglu ? m1.w : m0.w; a.s1 = swiglu ? m1.s : m0.s; a.b1 = swiglu ? m1.b : m0.b;
    a.ew = ew; a.eg = eg; a.k = k; a.n = n; a.K = K; a.x_by_pair = x_by_pair;
    if (xb) {
        a.xw0 = xb->m0.w; a.xs0 = xb->m0.s; a.xb0 = xb->m0.b;
        a.xw1 = swiglu ? xb->m1.w : xb->m0.w; a.xs1 = swiglu ? xb->m1.s : xb->m0.s; a.xb1 = swiglu ? xb->m1.b : xb->m0.b;
        a.xe = xb->expert; a.xpairs = xb->pairs;
    } else {
        a.xw0 = a.xw1 = m0.w; a.xs0 = a.xs1 = m0.s; a.xb0 = a.xb1 = m0.b;
        a.xe = -1; a.xpairs = 0x7FFFFFFF;
    }
    a.qa = q16 ? static_cast<uint4 *>(q16->qa) : nullptr;
    a.qs = q16 ? static_cast<uint4 *>(q16->qs) : nullptr;
    a.qnpk = q16 ? q16->npk : 0;
    const dim3 b(G16_THREADS);
    if (swiglu) {
        const dim3 grid((unsigned)max_tiles * (unsigned)((n + 127) / 128));
        switch (group) {
        case 32: hipLaunchKernelGGL((k_gmm16_stream<32, GS_DEPTH>), grid, b, 0, s, a); break;
        case 64: hipLaunchKernelGGL((k_gmm16_stream<64, GS_DEPTH>), grid, b, 0, s, a); break;
        default: hipLaunchKernelGGL((k_gmm16_stream<128, GS_DEPTH>), grid, b, 0, s, a); break;
        }
    } else {
        const dim3 grid((unsigned)max_tiles * (unsigned)((n + GSD_RB - 1) / GSD_RB));
        switch (group) {
        case 32: hipLaunchKernelGGL(k_gmm16_stream_down<32>, grid, b, 0, s, a, ax); break;
        case 64: hipLaunchKernelGGL(k_gmm16_stream_down<64>, grid, b, 0, s, a, ax); break;
        default: hipLaunchKernelGGL(k_gmm16_stream_down<128>, grid, b, 0, s, a, ax); break;
        }
    }
    return (int)hipGetLastError();
}
