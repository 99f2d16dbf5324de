// qw_route.hip -- router logits, softmax/top-k routing and the dispatch
// permutation, for gfx950.
//
// Routing must agree bit for bit with the host's restatement, so the router
// dot product and the softmax follow specified orders:
//
//   order R   dot(w, x) = p_0 + p_1 + ... (left to right), where p_c is the
//             fmaf chain, from 0, over the 64 consecutive elements of chunk c
//   softmax   m = max; e_i = qw_exp_spec(l_i - m); lane l of a wave sums
//             e_l, e_{l+64}, ... serially; the 64 lane sums meet in an xor
//             butterfly with ascending offsets 1..32; p_i = e_i / sum
//             (correctly rounded)
//   top-k     the K largest probabilities, ties to the lower expert index,
//             in descending order (what K rounds of a serial scan with '>'
//             pick), found exactly by a K-round wave tournament
//   renorm    wsum = w_0 + w_1 + ... in pick order; w_k / wsum
#include "qw_device.h"
#include "qw_kernels.h"

#define QW_DMAT_WAVES 4
#define QW_DMAT_RB 8                       // token rows per block
#define QW_DMAT_MAXCH (QWK_DMAT_MAX_K / 64)

// y[r, o] = order-R dot of bf16 row w[o] with fp32 row x[r].  A wave owns one
// output and up to QW_DMAT_RB token rows; lane l computes the partials of
// chunks l, l+64, ...; partials meet in LDS and lane r adds row r's chunk
// partials left to right.
template <bool VEC>
__global__ __launch_bounds__(QW_DMAT_WAVES * 64) void k_dmat_bf16(
    float *__restrict__ y, const float *__restrict__ x, const uint16_t *__restrict__ w,
    int k, int n, int rows)
{
    __shared__ float part[QW_DMAT_WAVES][QW_DMAT_MAXCH][QW_DMAT_RB];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int o = blockIdx.x * QW_DMAT_WAVES + wave;
    const int r0 = blockIdx.y * QW_DMAT_RB;
    const int nr = min(QW_DMAT_RB, rows - r0);
    const int nch = (k + 63) / 64;
    if (o < n) {
        const uint16_t *wr = w + (size_t)o * k;
        for (int c = lane; c < nch; c += 64) {
            float p[QW_DMAT_RB];
#pragma unroll
            for (int r = 0; r < QW_DMAT_RB; r++) p[r] = 0.0f;
            const int i0 = c * 64, len = min(64, k - i0);
            if (VEC && len == 64) {
                const uint4 *wv = reinterpret_cast<const uint4 *>(wr + i0);
#pragma unroll 2
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
                    for (int r = 0; r < QW_DMAT_RB; r++) {
                        if (r < nr) {
                            const float4 *xv = reinterpret_cast<const float4 *>(
                                x + (size_t)(r0 + r) * k + i0 + q * 8);
                            const float4 a = xv[0], b = xv[1];
                            float t = p[r];
                            t = __builtin_fmaf(wf[0], a.x, t);
                            t = __builtin_fmaf(wf[1], a.y, t);
                            t = __builtin_fmaf(wf[2], a.z, t);
                            t = __builtin_fmaf(wf[3], a.w, t);
                            t = __builtin_fmaf(wf[4], b.x, t);
                            t = __builtin_fmaf(wf[5], b.y, t);
                            t = __builtin_fmaf(wf[6], b.z, t);
                            t = __builtin_fmaf(wf[7], b.w, t);
                            p[r] = t;
                        }
                    }
                }
            } else {
                for (int i = 0; i < len; i++) {
                    const float wf = qw_bf16(wr[i0 + i]);
#pragma unroll
                    for (int r = 0; r < QW_DMAT_RB; r++)
                        if (r < nr) p[r] = __builtin_fmaf(wf, x[(size_t)(r0 + r) * k + i0 + i], p[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < QW_DMAT_RB; r++) part[wave][c][r] = p[r];
        }
    }
    __syncthreads();
    if (o < n && lane < nr) {
        float total = part[wave][0][lane];
        for (int c = 1; c < nch; c++) total = total + part[wave][c][lane];
        y[(size_t)(r0 + lane) * n + o] = total;
    }
}

// The same order-R logits for many token rows, register-tiled: one wave owns
// a 32 x 32 block of (token row, output); lane (ty, tx) keeps 4 x 4 of them.
// Chunk c of 64 inputs is staged in LDS transposed (x as [k][row], w as
// [k][out] in fp32), and every output runs its own fmaf chain over the chunk
// in index order from 0, then joins the running total (total = p_0, then
// total + p_c) -- the order above, element for element.  The next chunk is
// loaded into registers while the current one is consumed.  k % 64 == 0.
#define QW_DT 32
__global__ __launch_bounds__(64) void k_dmat_tiled(float *__restrict__ y, const float *__restrict__ x,
                                                   const uint16_t *__restrict__ w, int k, int n, int rows)
{
    __shared__ float4 xs[64][QW_DT / 4];      // [k][row / 4]
    __shared__ float4 ws[64][QW_DT / 4];      // [k][out / 4]
    const int lane = threadIdx.x, ty = lane / 8, tx = lane % 8;
    const int r0 = blockIdx.y * QW_DT, o0 = blockIdx.x * QW_DT;
    // staging: x rows r0 + lane / 2 (32 rows, two lanes a row, 32 inputs each);
    // w rows o0 + lane / 2 likewise (bf16, 32 inputs = 4 uint4)
    const int sr = lane / 2, sh = (lane % 2) * 32;
    const bool xok = r0 + sr < rows, wok = o0 + sr < n;
    const float4 *xg = reinterpret_cast<const float4 *>(x + (size_t)(xok ? r0 + sr : 0) * k + sh);
    const uint4 *wg = reinterpret_cast<const uint4 *>(w + (size_t)(wok ? o0 + sr : 0) * k + sh);
    float4 xr[8];
    uint4 wr[4];
    auto fetch = [&](int c) {
#pragma unroll
        for (int i = 0; i < 8; i++) xr[i] = xok ? xg[c * 16 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 4; i++) wr[i] = wok ? wg[c * 8 + i] : make_uint4(0, 0, 0, 0);
    };
    float tot[4][4], p[4][4];
    const int nch = k / 64;
    fetch(0);
    for (int c = 0; c < nch; c++) {
        __syncthreads();
        // transpose into LDS: element (row sr, input sh + 4i + j)
        float *xsf = reinterpret_cast<float *>(xs), *wsf = reinterpret_cast<float *>(ws);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float v[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) xsf[(sh + 4 * i + j) * QW_DT + sr] = v[j];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v[4] = {wr[i].x, wr[i].y, wr[i].z, wr[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                wsf[(sh + 8 * i + 2 * j) * QW_DT + sr] = __uint_as_float(v[j] << 16);
                wsf[(sh + 8 * i + 2 * j + 1) * QW_DT + sr] = __uint_as_float(v[j] & 0xFFFF0000u);
            }
        }
        __syncthreads();
        if (c + 1 < nch) fetch(c + 1);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) p[i][j] = 0.0f;
#pragma unroll 8
        for (int kk = 0; kk < 64; kk++) {
            const float4 a = xs[kk][ty], b = ws[kk][tx];
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) p[i][j] = __builtin_fmaf(bv[j], av[i], p[i][j]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) tot[i][j] = c == 0 ? p[i][j] : tot[i][j] + p[i][j];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = r0 + 4 * ty + i;
        if (r >= rows) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int o = o0 + 4 * tx + j;
            if (o < n) y[(size_t)r * n + o] = tot[i][j];
        }
    }
}

// The same order R on the fp32 matrix cores.  A K=1 MFMA,
// v_mfma_f32_16x16x1f32, is four independent 16x16 outer products
// D_b = C_b + a_b b_b^T, each element one fused multiply-add -- fmaf(a, b, c)
// -- so a chunk's chain (from 0, k in index order) is 64 MFMAs on one
// accumulator.  A workgroup owns 64 rows x 64 outputs; wave w owns rows
// 16 w .. 16 w + 15 against all 64 outputs as the instruction's four blocks
// (block b: outputs 16 b ..): lane l feeds block l / 16 with x[row l % 16][k]
// and w[output l % 16][k].  The operands pass through LDS QW_DM_NC chunks at a
// time (coalesced loads, the next stage requested while this one runs); a
// wave runs the stage's chunk chains interleaved -- independent, so the
// matrix pipe always has one ready -- and adds their partials to its running
// total in chunk order (total = p_0, then total + p_c: the order above).
// k % 64 == 0.
typedef float qr_f16v __attribute__((ext_vector_type(16)));
#define QW_DM_T 64
#define QW_DM_NC 2                                 // chunks a stage (4 measured slower)
#define QW_DM_KS (64 * QW_DM_NC + 4)               // floats a row of a stage (+ pad)
__global__ __launch_bounds__(256) void k_dmat_mfma(float *__restrict__ y, const float *__restrict__ x,
                                                   const uint16_t *__restrict__ w, int k, int n, int rows)
{
    extern __shared__ float4 dm_lds[];
    float *xs = reinterpret_cast<float *>(dm_lds), *ws = xs + QW_DM_T * QW_DM_KS;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, blk = lane >> 4, i = lane & 15;
    // Workgroup b runs on XCD b % 8: each XCD takes a contiguous range of
    // tiles in (row tile, column tile) order, so the column tiles of one row
    // tile share its token rows in that XCD's L2
    const int nct = (n + QW_DM_T - 1) / QW_DM_T, ntt = nct * ((rows + QW_DM_T - 1) / QW_DM_T);
    const int lt = (blockIdx.x & 7) * ((ntt + 7) / 8) + (blockIdx.x >> 3);
    if (lt >= ntt) return;
    const int r0 = lt / nct * QW_DM_T, o0 = lt % nct * QW_DM_T;
    const int nch = k / 64, rounds = (nch + QW_DM_NC - 1) / QW_DM_NC;
    constexpr int SK = 64 * QW_DM_NC;                    // k a stage
    constexpr int XF4 = QW_DM_T * SK / 4 / 256, WU4 = QW_DM_T * SK / 8 / 256;
    // staging: x [64 rows][SK] as float4s, w [64 outputs][SK] bf16 as uint4s,
    // consecutive threads along a row
    float4 xr[XF4];
    uint4 wr[WU4];
    auto fetch = [&](int rd) {
        const int k0 = SK * rd, kl = min(SK, k - k0);
#pragma unroll
        for (int j = 0; j < XF4; j++) {
            const int q = t + 256 * j, row = q / (SK / 4), c4 = q % (SK / 4);
            const int gr = min(r0 + row, rows - 1);
            xr[j] = 4 * c4 < kl ? reinterpret_cast<const float4 *>(x + (size_t)gr * k + k0)[c4]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < WU4; j++) {
            const int q = t + 256 * j, o = q / (SK / 8), c8 = q % (SK / 8);
            const int go = min(o0 + o, n - 1);
            wr[j] = 8 * c8 < kl ? reinterpret_cast<const uint4 *>(w + (size_t)go * k + k0)[c8] : make_uint4(0, 0, 0, 0);
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int j = 0; j < XF4; j++) {
            const int q = t + 256 * j, row = q / (SK / 4), c4 = q % (SK / 4);
            *reinterpret_cast<float4 *>(xs + row * QW_DM_KS + 4 * c4) = xr[j];
        }
#pragma unroll
        for (int j = 0; j < WU4; j++) {
            const int q = t + 256 * j, o = q / (SK / 8), c8 = q % (SK / 8);
            const uint32_t v[4] = {wr[j].x, wr[j].y, wr[j].z, wr[j].w};
            float f[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                f[2 * e] = __uint_as_float(v[e] << 16);
                f[2 * e + 1] = __uint_as_float(v[e] & 0xFFFF0000u);
            }
            float4 *d = reinterpret_cast<float4 *>(ws + o * QW_DM_KS + 8 * c8);
            d[0] = make_float4(f[0], f[1], f[2], f[3]);
            d[1] = make_float4(f[4], f[5], f[6], f[7]);
        }
    };
    const qr_f16v zero = {};
    qr_f16v tot = zero;
    fetch(0);
    const float *xa = xs + (16 * wave + i) * QW_DM_KS, *wa = ws + (16 * blk + i) * QW_DM_KS;
    for (int rd = 0; rd < rounds; rd++) {
        __syncthreads();                            // the previous stage is consumed
        stash();
        __syncthreads();
        if (rd + 1 < rounds) fetch(rd + 1);
        const int nc = min(QW_DM_NC, nch - QW_DM_NC * rd);
        qr_f16v acc[QW_DM_NC];
#pragma unroll
        for (int c = 0; c < QW_DM_NC; c++) acc[c] = zero;
#pragma unroll 2
        for (int kk = 0; kk < 64; kk += 4) {
            float4 av[QW_DM_NC], bv[QW_DM_NC];
#pragma unroll
            for (int c = 0; c < QW_DM_NC; c++) {
                av[c] = *reinterpret_cast<const float4 *>(xa + 64 * c + kk);
                bv[c] = *reinterpret_cast<const float4 *>(wa + 64 * c + kk);
            }
#pragma unroll
            for (int c = 0; c < QW_DM_NC; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x1f32(av[c].x, bv[c].x, acc[c], 0, 0, 0);
#pragma unroll
            for (int c = 0; c < QW_DM_NC; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x1f32(av[c].y, bv[c].y, acc[c], 0, 0, 0);
#pragma unroll
            for (int c = 0; c < QW_DM_NC; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x1f32(av[c].z, bv[c].z, acc[c], 0, 0, 0);
#pragma unroll
            for (int c = 0; c < QW_DM_NC; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x1f32(av[c].w, bv[c].w, acc[c], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < QW_DM_NC; c++)
            if (c < nc) {
#pragma unroll
                for (int e = 0; e < 16; e++) tot[e] = rd == 0 && c == 0 ? acc[c][e] : tot[e] + acc[c][e];
            }
    }
    // block b's values of this lane: rows 4 (lane / 16) + e of the wave's 16,
    // output 16 b + lane % 16
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int b = e >> 2;
        const int row = r0 + 16 * wave + 4 * (lane >> 4) + (e & 3), o = o0 + 16 * b + (lane & 15);
        if (row < rows && o < n) y[(size_t)row * n + o] = tot[e];
    }
}

// A few outputs (the shared expert's gate, n = 1; the mixer's injection
// logits, n = 4) over many token rows: one wave per row; lane c loads chunk c
// of the row once and runs its fmaf chain for every output (c < 64 * 4), the
// partials meet in LDS and lane o adds output o's left to right.  k % 64 == 0.
#define QW_DROWS_WAVES 4
#define QW_DROWS_MAXN 8                    // outputs a row (n < 8 takes this path)
// STAGE (k <= 64 * 64): the row also leaves staged as f16, as k_stage16
// stages it (the same bits): from the chunk each lane holds, the row's
// largest magnitude by a wave maximum, then h = f16(x 2^sh) in 8-blocks
// ordered 0,4,1,5,2,6,3,7, and F = 2^-sh.
template <bool STAGE>
__global__ __launch_bounds__(QW_DROWS_WAVES * 64) void k_dmat_rows(float *__restrict__ y, const float *__restrict__ x,
                                                                  const uint16_t *__restrict__ w, int k, int n,
                                                                  int rows, uint16_t *__restrict__ hx,
                                                                  float *__restrict__ hF)
{
    __shared__ float part[QW_DROWS_WAVES][QW_DROWS_MAXN][QW_DMAT_MAXCH];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * QW_DROWS_WAVES + wave;
    if (r >= rows) return;
    const int nch = k / 64;
    const float *xr = x + (size_t)r * k;
    float4 xa[16];        // with STAGE (nch <= 64): lane c's chunk, after the loop
    for (int c = lane; c < nch; c += 64) {
        // the row's chunk once, for every output
        const float4 *xv = reinterpret_cast<const float4 *>(xr + c * 64);
#pragma unroll
        for (int q = 0; q < 16; q++) xa[q] = xv[q];
        for (int o = 0; o < n; o++) {
            const uint4 *wv = reinterpret_cast<const uint4 *>(w + (size_t)o * k + c * 64);
            float p = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint4 ww = wv[q];
                const float4 a = xa[2 * q], b = xa[2 * q + 1];
                p = __builtin_fmaf(__uint_as_float(ww.x << 16), a.x, p);
                p = __builtin_fmaf(__uint_as_float(ww.x & 0xFFFF0000u), a.y, p);
                p = __builtin_fmaf(__uint_as_float(ww.y << 16), a.z, p);
                p = __builtin_fmaf(__uint_as_float(ww.y & 0xFFFF0000u), a.w, p);
                p = __builtin_fmaf(__uint_as_float(ww.z << 16), b.x, p);
                p = __builtin_fmaf(__uint_as_float(ww.z & 0xFFFF0000u), b.y, p);
                p = __builtin_fmaf(__uint_as_float(ww.w << 16), b.z, p);
                p = __builtin_fmaf(__uint_as_float(ww.w & 0xFFFF0000u), b.w, p);
            }
            part[wave][o][c] = p;
        }
    }
    if (STAGE) {
        const int c = lane;
        float m = 0.0f;
        if (c < nch) {
#pragma unroll
            for (int q = 0; q < 16; q++)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(xa[q].x), fabsf(xa[q].y)), fmaxf(fabsf(xa[q].z), fabsf(xa[q].w))));
        }
        m = qw_wave_max(m);
        int sh = 0;
        if (m > 0.0f && m <= 3.40282346638528859812e+38f) {
            sh = 15 - __builtin_amdgcn_frexp_expf(m);
            sh = sh < -126 ? -126 : sh > 126 ? 126 : sh;
        }
        if (c == 0) hF[r] = __builtin_ldexpf(1.0f, -sh);
        if (c < nch) {
            typedef _Float16 dr_h8 __attribute__((ext_vector_type(8)));
            dr_h8 *hr = reinterpret_cast<dr_h8 *>(hx + (size_t)r * k + c * 64);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 a = xa[2 * q], b = xa[2 * q + 1];
                const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                _Float16 h[8];
#pragma unroll
                for (int j = 0; j < 8; j++) h[j] = (_Float16)__builtin_ldexpf(v[j], sh);
                hr[q] = dr_h8{h[0], h[4], h[1], h[5], h[2], h[6], h[3], h[7]};
            }
        }
    }
    // the wave's LDS accesses run in order: lane o reads what the wave wrote
    if (lane < n) {
        float total = part[wave][lane][0];
        for (int c = 1; c < nch; c++) total = total + part[wave][lane][c];
        y[(size_t)r * n + lane] = total;
    }
}

// Few outputs over a long input (the mixer's injection logits: n = 4, k =
// 4 H) for a few token rows: a workgroup per output, a thread per 64-input
// chunk (every load issued before the chain), the chunk partials to LDS and
// added left to right by one thread a row -- order R, in one memory round trip
// where a wave per output walks its chunks one after another.
#define QW_DW_THREADS 256
#define QW_DW_MAXCH 256
#define QW_DW_MAXR 8
__global__ __launch_bounds__(QW_DW_THREADS) void k_dmat_wide(float *__restrict__ y, const float *__restrict__ x,
                                                             const uint16_t *__restrict__ w, int k, int n, int rows)
{
    __shared__ float part[QW_DW_MAXCH][QW_DW_MAXR];
    const int o = blockIdx.x, c = threadIdx.x, nch = k / 64;
    if (c < nch) {
        const uint4 *wv = reinterpret_cast<const uint4 *>(w + (size_t)o * k + 64 * c);
        uint4 ww[8];
#pragma unroll
        for (int q = 0; q < 8; q++) ww[q] = wv[q];
        for (int r = 0; r < rows; r++) {
            const float4 *xv = reinterpret_cast<const float4 *>(x + (size_t)r * k + 64 * c);
            float4 xa[16];
#pragma unroll
            for (int q = 0; q < 16; q++) xa[q] = xv[q];
            float t = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t wd[4] = {ww[q].x, ww[q].y, ww[q].z, ww[q].w};
                const float4 a = xa[2 * q], b = xa[2 * q + 1];
                const float xx[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    t = __builtin_fmaf(__uint_as_float(wd[j] << 16), xx[2 * j], t);
                    t = __builtin_fmaf(__uint_as_float(wd[j] & 0xFFFF0000u), xx[2 * j + 1], t);
                }
            }
            part[c][r] = t;
        }
    }
    __syncthreads();
    if (threadIdx.x < rows) {
        const int r = threadIdx.x;
        float tot = part[0][r];
        for (int i = 1; i < nch; i++) tot = tot + part[i][r];
        y[(size_t)r * n + o] = tot;
    }
}

#include "qw_few.h"

__global__ __launch_bounds__(QW_DF_WAVES * 64) void k_dmat_few(float *__restrict__ y, float *__restrict__ g,
                                                               const float *__restrict__ x,
                                                               const uint16_t *__restrict__ w,
                                                               const uint16_t *__restrict__ w2, int k, int n,
                                                               int rows, uint4 *__restrict__ qx,
                                                               uint16_t *__restrict__ hx, float *__restrict__ hF)
{
    extern __shared__ float xl[];                    // [rows of this group][nch][QW_DF_PAD]
    qw_few_body<false>(y, g, x, w, w2, k, n, rows, qx, hx, hF, nullptr, 0u, blockIdx.x, blockIdx.y, xl);
}

static bool qw_few_ok(const float *x, const uint16_t *w, int k, int rows)
{
    return rows >= 1 && rows <= QW_DF_MAXR && k % 64 == 0 && k <= 64 * 64 && ((uintptr_t)w % 16) == 0 &&
           ((uintptr_t)x % 16) == 0;
}

static int qw_launch_few(hipStream_t s, float *y, float *g, const float *x, const uint16_t *w, const uint16_t *w2,
                         int k, int n, int rows, uint4 *qx = nullptr, uint16_t *hx = nullptr, float *hF = nullptr)
{
    const size_t lds = (size_t)min(rows, QW_DF_TPG) * (k / 64) * QW_DF_PAD * sizeof(float);
    static bool attr = false;
    if (!attr) {
        attr = true;
        // 8 rows of k = 4096: 139,264 bytes of token rows (with 16 KB of partials)
        (void)hipFuncSetAttribute((const void *)k_dmat_few, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  QW_DF_MAXR * 64 * QW_DF_PAD * (int)sizeof(float));
        (void)hipGetLastError();
    }
    const int outs = n + (w2 ? 1 : 0);
    hipLaunchKernelGGL(k_dmat_few, dim3((outs + QW_DF_WAVES - 1) / QW_DF_WAVES, (rows + QW_DF_TPG - 1) / QW_DF_TPG),
                       dim3(QW_DF_WAVES * 64), lds, s, y, g, x, w, w2, k, n, rows, qx, hx, hF);
    return (int)hipGetLastError();
}

extern "C" int qwk_dmat_bf16_gate(hipStream_t s, float *y, float *g, const float *x, const uint16_t *w,
                                  const uint16_t *w2, int k, int n, int rows, void *qx, uint16_t *hx, float *hF)
{
    if (n < 1 || !qw_few_ok(x, w, k, rows) || (w2 && ((uintptr_t)w2 % 16) != 0) || ((uintptr_t)qx % 16) != 0 ||
        ((uintptr_t)hx % 16) != 0 || (hx && (!hF || k % 8)))
        return (int)hipErrorInvalidValue;
    return qw_launch_few(s, y, g, x, w, w2, k, n, rows, static_cast<uint4 *>(qx), hx, hF);
}

extern "C" int qwk_dmat_rows_stage16(hipStream_t s, float *y, uint16_t *hx, float *hF, const float *x,
                                     const uint16_t *w, int k, int n, int rows)
{
    if (k < 64 || k % 64 || k > 64 * 64 || n < 1 || n > QW_DROWS_MAXN || rows < 1 || !hx || !hF ||
        ((uintptr_t)w % 16) || ((uintptr_t)x % 16) || ((uintptr_t)hx % 16))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dmat_rows<true>, dim3((unsigned)((rows + QW_DROWS_WAVES - 1) / QW_DROWS_WAVES)),
                       dim3(QW_DROWS_WAVES * 64), 0, s, y, x, w, k, n, rows, hx, hF);
    return (int)hipGetLastError();
}

extern "C" int qwk_dmat_bf16(hipStream_t s, float *y, const float *x, const uint16_t *w,
                             int k, int n, int rows)
{
    if (k < 1 || k > QWK_DMAT_MAX_K || n < 1 || rows < 1) return (int)hipErrorInvalidValue;
    const bool vec = k % 8 == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)x % 16) == 0;
    if (vec && k % 64 == 0 && n < 8 && rows <= QW_DW_MAXR && k / 64 <= QW_DW_MAXCH && k >= 64 * 64) {
        hipLaunchKernelGGL(k_dmat_wide, dim3((unsigned)n), dim3(QW_DW_THREADS), 0, s, y, x, w, k, n, rows);
        return (int)hipGetLastError();
    }
    if (vec && k % 64 == 0 && n < 8 && rows >= 8) {
        hipLaunchKernelGGL(k_dmat_rows<false>, dim3((unsigned)((rows + QW_DROWS_WAVES - 1) / QW_DROWS_WAVES)),
                           dim3(QW_DROWS_WAVES * 64), 0, s, y, x, w, k, n, rows, nullptr, nullptr);
        return (int)hipGetLastError();
    }
    if (vec && n >= 8 && qw_few_ok(x, w, k, rows)) return qw_launch_few(s, y, nullptr, x, w, nullptr, k, n, rows);
    if (vec && k % 64 == 0 && rows >= QW_DT && n >= QW_DM_T) {
        const int lds = 2 * QW_DM_T * QW_DM_KS * (int)sizeof(float);
        static bool attr = false;
        if (!attr) {
            attr = true;
            (void)hipFuncSetAttribute((const void *)k_dmat_mfma, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
            (void)hipGetLastError();
        }
        const int ntt = ((n + QW_DM_T - 1) / QW_DM_T) * ((rows + QW_DM_T - 1) / QW_DM_T);
        hipLaunchKernelGGL(k_dmat_mfma, dim3((ntt + 7) / 8 * 8), dim3(256), lds,
                           s, y, x, w, k, n, rows);
        return (int)hipGetLastError();
    }
    if (vec && k % 64 == 0 && rows >= QW_DT) {
        hipLaunchKernelGGL(k_dmat_tiled, dim3((n + QW_DT - 1) / QW_DT, (rows + QW_DT - 1) / QW_DT), dim3(64), 0, s,
                           y, x, w, k, n, rows);
        return (int)hipGetLastError();
    }
    dim3 grid((n + QW_DMAT_WAVES - 1) / QW_DMAT_WAVES, (rows + QW_DMAT_RB - 1) / QW_DMAT_RB);
    if (vec) hipLaunchKernelGGL(k_dmat_bf16<true>, grid, dim3(QW_DMAT_WAVES * 64), 0, s, y, x, w, k, n, rows);
    else hipLaunchKernelGGL(k_dmat_bf16<false>, grid, dim3(QW_DMAT_WAVES * 64), 0, s, y, x, w, k, n, rows);
    return (int)hipGetLastError();
}

// ---- route -------------------------------------------------------------------

__global__ __launch_bounds__(64) void k_route(int *__restrict__ idx, float *__restrict__ w,
                                              const float *__restrict__ logits, int rows,
                                              int E, int K, int norm)
{
    __shared__ __align__(16) uint32_t sx[QW_ROUTE_SX];
    const int r = blockIdx.x, lane = threadIdx.x;
    int pi;
    float pw;
    const float *l = logits + (size_t)r * E;
    if (E <= 256) qw_route_wave<4>(l, E, K, norm, lane, &pi, &pw, sx);
    else if (E <= 512) qw_route_wave<8>(l, E, K, norm, lane, &pi, &pw, sx);
    else qw_route_wave<16>(l, E, K, norm, lane, &pi, &pw, sx);
    if (lane < K) { idx[(size_t)r * K + lane] = pi; w[(size_t)r * K + lane] = pw; }
}

extern "C" int qwk_route(hipStream_t s, int32_t *idx, float *w, const float *logits,
                         int rows, int E, int K, int norm)
{
    if (rows < 1 || E < 1 || E > QWK_ROUTE_MAX_E || K < 1 || K > QWK_ROUTE_MAX_K || K > E)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route, dim3(rows), dim3(64), 0, s, idx, w, logits, rows, E, K, norm);
    return (int)hipGetLastError();
}

// ---- the dispatch permutation ------------------------------------------------
//
// Pairs sorted by expert, stably: within an expert, ascending pair index.
// The pairs are cut into chunks of QW_GROUP_CHUNK, one workgroup each, and
// within a chunk into eight contiguous runs, one a wave.  Three launches:
//
//   count  per (chunk, expert) counts (order-free LDS atomics)
//   scan   one workgroup: an exclusive scan over experts and then, within an
//          expert, over the chunks gives every (chunk, expert) its first
//          slot; the tile list follows from the per-expert totals
//   place  each workgroup counts its chunk's runs again, per (wave, expert),
//          and adds them in wave order to its (chunk, expert) slots; each
//          wave then walks its run 64 pairs at a time, ranking a lane among
//          the lower lanes that share its expert with ballots over the
//          expert id's bits
// (The scan reads chunk counts, not (chunk, wave) ones: a single workgroup
// moving 8x the counts through one CU's L1 took 12.6 of the 26 us at 2048
// tokens.)
//
// The counts live in a work buffer of qwk_moe_group_work_bytes(pairs, E).
// `extra` rows may follow the pairs as one more expert, E (the prefill's
// shared expert, run in the same grouped launches): slots pairs .. pairs +
// extra - 1 in order, and their tiles after all the others.

#define QW_GROUP_WAVES 8
#define QW_GROUP_THREADS (QW_GROUP_WAVES * 64)
#define QW_GROUP_RUN 256                                    // pairs a wave walks
#define QW_GROUP_CHUNK (QW_GROUP_WAVES * QW_GROUP_RUN)
#define QW_SCAN_THREADS 1024

// Exclusive scan of v over the block (nthr values); returns the prefix and
// writes the total to *total.
__device__ int qw_block_excl_scan(int v, int *tmp, int *total, int nthr)
{
    const int t = threadIdx.x;
    tmp[t] = v;
    __syncthreads();
    for (int off = 1; off < nthr; off <<= 1) {
        const int add = t >= off ? tmp[t - off] : 0;
        __syncthreads();
        tmp[t] += add;
        __syncthreads();
    }
    const int incl = tmp[t];
    *total = tmp[nthr - 1];
    __syncthreads();
    return incl - v;
}

// work[(chunk * WAVES + wave) * E + e] = pairs of expert e in that run
__global__ __launch_bounds__(QW_GROUP_THREADS) void k_group_count(int *__restrict__ work,
                                                                  const int *__restrict__ idx, int pairs, int E)
{
    __shared__ int cnt[QWK_GROUP_MAX_E];
    const int t = threadIdx.x;
    for (int i = t; i < E; i += QW_GROUP_THREADS) cnt[i] = 0;
    __syncthreads();
    const int p0 = min(pairs, blockIdx.x * QW_GROUP_CHUNK), p1 = min(pairs, p0 + QW_GROUP_CHUNK);
    for (int p = p0 + t; p < p1; p += QW_GROUP_THREADS) atomicAdd(&cnt[idx[p]], 1);
    __syncthreads();
    int *w = work + (size_t)blockIdx.x * E;
    for (int i = t; i < E; i += QW_GROUP_THREADS) w[i] = cnt[i];
}

__global__ __launch_bounds__(QW_SCAN_THREADS) void k_group_scan(int *__restrict__ work, int *__restrict__ tiles,
                                                                 int *__restrict__ perm, int pairs, int extra,
                                                                 int nruns, int E, int bm, int max_tiles)
{
    __shared__ int tmp[QW_SCAN_THREADS];
    const int t = threadIdx.x;
    const int per_t = (E + QW_SCAN_THREADS - 1) / QW_SCAN_THREADS;
    const int e0 = min(E, t * per_t), e1 = min(E, e0 + per_t);
    // the run counts are read 16 at a time (independent loads in flight
    // together, not one memory round trip each)
    constexpr int RB = 16;
    int mytot = 0, mytiles = 0;
    for (int e = e0; e < e1; e++) {
        int c = 0;
        for (int r0 = 0; r0 < nruns; r0 += RB) {
            int v[RB];
#pragma unroll
            for (int j = 0; j < RB; j++) v[j] = r0 + j < nruns ? work[(size_t)(r0 + j) * E + e] : 0;
#pragma unroll
            for (int j = 0; j < RB; j++) c += v[j];
        }
        mytot += c;
        mytiles += (c + bm - 1) / bm;
    }
    int total_pairs, total_tiles;
    int base = qw_block_excl_scan(mytot, tmp, &total_pairs, QW_SCAN_THREADS);
    int tbase = qw_block_excl_scan(mytiles, tmp, &total_tiles, QW_SCAN_THREADS);
    for (int e = e0; e < e1; e++) {
        int run = base;
        for (int r0 = 0; r0 < nruns; r0 += RB) {
            int v[RB];
#pragma unroll
            for (int j = 0; j < RB; j++) v[j] = r0 + j < nruns ? work[(size_t)(r0 + j) * E + e] : 0;
#pragma unroll
            for (int j = 0; j < RB; j++) {
                if (r0 + j < nruns) work[(size_t)(r0 + j) * E + e] = run;
                run += v[j];
            }
        }
        const int c = run - base;
        for (int s = 0; s < c; s += bm, tbase++) {
            if (tbase < max_tiles) {
                tiles[1 + 3 * tbase + 0] = e;
                tiles[1 + 3 * tbase + 1] = base + s;
                tiles[1 + 3 * tbase + 2] = min(bm, c - s);
            }
        }
        base = run;
    }
    // `extra` rows after the pairs: expert E, identity slots, tiles of bm
    const int xt = (extra + bm - 1) / bm;
    for (int j = t; j < xt; j += QW_SCAN_THREADS) {
        const int tb = total_tiles + j;
        if (tb < max_tiles) {
            tiles[1 + 3 * tb + 0] = E;
            tiles[1 + 3 * tb + 1] = pairs + j * bm;
            tiles[1 + 3 * tb + 2] = min(bm, extra - j * bm);
        }
    }
    for (int j = t; j < extra; j += QW_SCAN_THREADS) perm[pairs + j] = pairs + j;
    if (t == 0) tiles[0] = min(total_tiles + xt, max_tiles);
}

__global__ __launch_bounds__(QW_GROUP_THREADS) void k_group_place(int *__restrict__ perm,
                                                                  const int *__restrict__ work,
                                                                  const int *__restrict__ idx, int pairs, int E)
{
    __shared__ int cnt[QW_GROUP_WAVES][QWK_GROUP_MAX_E];
    const int t = threadIdx.x, wave = t / 64, lane = t % 64;
    for (int i = t; i < QW_GROUP_WAVES * E; i += QW_GROUP_THREADS) cnt[i / E][i % E] = 0;
    __syncthreads();
    const int p0 = min(pairs, blockIdx.x * QW_GROUP_CHUNK + wave * QW_GROUP_RUN), p1 = min(pairs, p0 + QW_GROUP_RUN);
    for (int p = p0 + lane; p < p1; p += 64) atomicAdd(&cnt[wave][idx[p]], 1);
    __syncthreads();
    // (wave, expert) slots: the chunk's slot for the expert plus the counts
    // of the expert's pairs in the runs of the lower waves
    const int *w = work + (size_t)blockIdx.x * E;
    for (int e = t; e < E; e += QW_GROUP_THREADS) {
        int run = w[e];
#pragma unroll
        for (int v = 0; v < QW_GROUP_WAVES; v++) {
            const int c = cnt[v][e];
            cnt[v][e] = run;
            run += c;
        }
    }
    __syncthreads();
    int nbits = 1;
    while ((1 << nbits) < E) nbits++;
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int pb = p0; pb < p1; pb += 64) {
        const int p = pb + lane;
        const bool valid = p < p1;
        const int e = valid ? idx[p] : 0;
        unsigned long long same = __ballot(valid);
        for (int b = 0; b < nbits; b++) {
            const bool bit = (e >> b) & 1;
            const unsigned long long bb = __ballot(valid && bit);
            same &= bit ? bb : ~bb;
        }
        if (valid) {
            const int rank = __popcll(same & below);
            perm[cnt[wave][e] + rank] = p;
        }
        __builtin_amdgcn_wave_barrier();
        // The highest lane of each run of equal experts advances the cursor.
        if (valid && (same >> lane) == 1ull) cnt[wave][e] += __popcll(same);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
    }
}

extern "C" size_t qwk_moe_group_work_bytes(int pairs, int E)
{
    const size_t chunks = pairs > 0 ? (size_t)(pairs + QW_GROUP_CHUNK - 1) / QW_GROUP_CHUNK : 1;
    return chunks * (size_t)(E > 0 ? E : 1) * sizeof(int);
}

extern "C" int qwk_moe_group(hipStream_t s, int32_t *perm, int32_t *tiles, const int32_t *idx,
                             int pairs, int E, int bm, int max_tiles, void *work, size_t work_bytes,
                             int extra)
{
    if (pairs < 0 || E < 1 || E > QWK_GROUP_MAX_E || bm < 1 || max_tiles < 0 || !work || extra < 0 ||
        work_bytes < qwk_moe_group_work_bytes(pairs, E))
        return (int)hipErrorInvalidValue;
    const int chunks = pairs > 0 ? (pairs + QW_GROUP_CHUNK - 1) / QW_GROUP_CHUNK : 1;
    int *wk = static_cast<int *>(work);
    hipLaunchKernelGGL(k_group_count, dim3(chunks), dim3(QW_GROUP_THREADS), 0, s, wk, idx, pairs, E);
    hipLaunchKernelGGL(k_group_scan, dim3(1), dim3(QW_SCAN_THREADS), 0, s, wk, tiles, perm, pairs, extra,
                       chunks, E, bm, max_tiles);
    hipLaunchKernelGGL(k_group_place, dim3(chunks), dim3(QW_GROUP_THREADS), 0, s, perm, wk, idx, pairs, E);
    return (int)hipGetLastError();
}
