// qw_qsa.hip -- Qwen Sparse Attention on gfx950: the indexer's block scores,
// the stored block keys, top-k block selection and attention over the
// selected positions (reference contract qwasar_gpu.h:617-646, CPU semantics
// qwasar_flash_cpu.c:347-478).
//
// Block key (k_qsa_scores phase 1, k_qsa_pool): a wave per block, lane l
// owning dims l, l+64, ...: the serial mean of the block's `ratio` raw keys,
// the rms norm with the k_layernorm gain, then the rotary pair (j, j+32) of
// the first 64 dims at the block's first position -- lanes j and j+32, one
// swizzle apart.
//
// Score (phase 2): the keys are transposed through LDS so that a thread owns
// one block's key in registers; the row's query heads sit in LDS and are read
// as broadcast float4s.  Thread (wave w, lane l) scores block l against heads
// w, w+4, ...: per head a serial fma chain over the dims, the positive dots
// summed in head order; the four waves' partials meet as (p0 + p1) + (p2 +
// p3), then / sqrt(d).  The arithmetic does not depend on how many rows or
// blocks a call has, and the pooled path runs the same phase 2 on stored keys,
// so scores and pooled scores agree bit for bit.
//
// Selection (k_qsa_select): a workgroup of 1024 threads per query.  Scores
// map to 32-bit keys that order as the floats do (-0 as +0; -FLT_MAX, -inf
// and NaN, which the reference's scan never picks, to 0).  A radix search in
// three passes of 11, 11 and 10 bits finds the exact key T of the last block
// taken; keys above T are taken and the rest of the budget comes from keys
// equal to T in block order.  Each thread owns a contiguous run of blocks, so
// block order is thread order and the position list is one prefix sum.
//
// Masked attention (k_attn_masked<G>): a workgroup per (query row, kv head)
// with its G query heads.  Positions from the list go 256 at a time: a thread
// per position scores its fp16 key row against the G heads, the chunk's
// maxima and exponentials update an online softmax, and the waves accumulate
// the chunk's value rows with lanes over dims (each value row one coalesced
// 512-byte read).
#include "qw_device.h"
#include "qw_kernels.h"

#include <float.h>

#define QS_BLK 64
#define QS_THREADS 256
#define QS_ROWS 8          // query rows a scoring workgroup walks
#define QS_ROTARY 64

// ---- block keys ---------------------------------------------------------------

template <int M>   // dims per lane: d <= 64 * M
__device__ __forceinline__ void qs_block_key(float (&kn)[M], const float *__restrict__ ikeys,
                                             const uint16_t *__restrict__ kw, const float *__restrict__ inv_freq,
                                             int b, int d, int ratio, float eps, int lane)
{
    float ss = 0.0f;
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int dim = lane + 64 * m;
        kn[m] = 0.0f;
        if (dim < d) {
            const float *p = ikeys + (size_t)b * ratio * d + dim;
            float acc = p[0];
            for (int t = 1; t < ratio; t++) acc += p[(size_t)t * d];
            kn[m] = acc / (float)ratio;
            ss = __builtin_fmaf(kn[m], kn[m], ss);
        }
    }
    ss = qw_xor_sum<64>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)d + eps);
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int dim = lane + 64 * m;
        if (dim < d) kn[m] = kn[m] * inv * qw_bf16(kw[dim]);
    }
    const float partner = __shfl_xor(kn[0], 32, 64);
    const float ang = (float)(b * ratio) * inv_freq[lane & 31];
    const float c = cosf(ang), s = sinf(ang);
    // written as explicit fmas so every kernel inlining this rounds alike
    kn[0] = lane < 32 ? __builtin_fmaf(kn[0], c, -(partner * s)) : __builtin_fmaf(kn[0], c, partner * s);
}

// ---- scores ---------------------------------------------------------------------

// phase 2 over one WG's QS_BLK keys (LDS, row stride D + 4) for rows r0.. of
// the tile; `kl` holds the keys, `ql` one row's heads, `part` the partials.
template <int D>
__device__ __forceinline__ void qs_score_rows(float *__restrict__ scores, const float *__restrict__ qn,
                                              const float *kl, float *ql, float *part, int b0, int r0, int rows,
                                              int nq, int d, int ratio, int base_pos, int max_blocks)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float kr[D];
#pragma unroll
    for (int i = 0; i < D; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(kl + lane * (D + 4) + i);
        kr[i] = v.x; kr[i + 1] = v.y; kr[i + 2] = v.z; kr[i + 3] = v.w;
    }
    const float rs = sqrtf((float)d);
    for (int r = r0; r < min(r0 + QS_ROWS, rows); r++) {
        const int nb = (base_pos + r + 1) / ratio;
        if (nb <= b0) continue;                      // uniform: nothing of this row here
        __syncthreads();                             // ql free
        const float *qr = qn + (size_t)r * nq * d;
        for (int i = tid; i < nq * D; i += QS_THREADS) {
            const int h = i / D, j = i % D;
            ql[i] = j < d ? qr[(size_t)h * d + j] : 0.0f;
        }
        __syncthreads();
        float p = 0.0f;
        for (int h = wave; h < nq; h += QS_THREADS / 64) {
            const float4 *q4 = reinterpret_cast<const float4 *>(ql + h * D);
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < D / 4; i++) {
                const float4 qv = q4[i];
                dot = __builtin_fmaf(qv.x, kr[4 * i], dot);
                dot = __builtin_fmaf(qv.y, kr[4 * i + 1], dot);
                dot = __builtin_fmaf(qv.z, kr[4 * i + 2], dot);
                dot = __builtin_fmaf(qv.w, kr[4 * i + 3], dot);
            }
            if (dot > 0.0f) p += dot;
        }
        part[wave * QS_BLK + lane] = p;
        __syncthreads();
        const int b = b0 + lane;
        if (wave == 0 && b < nb) {
            const float s = (part[lane] + part[QS_BLK + lane]) + (part[2 * QS_BLK + lane] + part[3 * QS_BLK + lane]);
            scores[(size_t)r * max_blocks + b] = s / rs;
        }
    }
}

template <int D, bool POOLED>
__global__ void __launch_bounds__(QS_THREADS) k_qsa_scores(float *__restrict__ scores, const float *__restrict__ qn,
                                                           const float *__restrict__ src,
                                                           const uint16_t *__restrict__ kw,
                                                           const float *__restrict__ inv_freq, int rows, int nq,
                                                           int d, int ratio, int base_pos, int max_blocks, float eps)
{
    extern __shared__ float4 qs_lds[];
    float *kl = reinterpret_cast<float *>(qs_lds);            // [QS_BLK][D + 4]
    float *part = kl + QS_BLK * (D + 4);                       // [4][QS_BLK]
    float *ql = part + 4 * QS_BLK;                             // [nq][D]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b0 = blockIdx.x * QS_BLK, r0 = blockIdx.y * QS_ROWS;
    const int nb_hi = (base_pos + min(r0 + QS_ROWS, rows)) / ratio;   // blocks any row of the tile sees
    if (nb_hi <= b0) return;                                   // uniform
    if (POOLED) {
        for (int i = tid; i < QS_BLK * (D / 4); i += QS_THREADS) {
            const int bl = i / (D / 4), j = 4 * (i % (D / 4));
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const int b = b0 + bl;
            if (b < nb_hi) {
                const float *p = src + (size_t)b * d + j;
                if (j + 3 < d) v = make_float4(p[0], p[1], p[2], p[3]);
                else {
                    if (j < d) v.x = p[0];
                    if (j + 1 < d) v.y = p[1];
                    if (j + 2 < d) v.z = p[2];
                }
            }
            *reinterpret_cast<float4 *>(kl + bl * (D + 4) + j) = v;
        }
    } else {
        for (int bl = wave; bl < QS_BLK; bl += QS_THREADS / 64) {
            const int b = b0 + bl;
            float kn[D / 64];
            if (b < nb_hi) qs_block_key<D / 64>(kn, src, kw, inv_freq, b, d, ratio, eps, lane);
            else {
#pragma unroll
                for (int m = 0; m < D / 64; m++) kn[m] = 0.0f;
            }
#pragma unroll
            for (int m = 0; m < D / 64; m++) kl[bl * (D + 4) + lane + 64 * m] = kn[m];
        }
    }
    __syncthreads();
    qs_score_rows<D>(scores, qn, kl, ql, part, b0, r0, rows, nq, d, ratio, base_pos, max_blocks);
}

template <int M>
__global__ void __launch_bounds__(QS_THREADS) k_qsa_pool(float *__restrict__ pool, const float *__restrict__ ikeys,
                                                         const uint16_t *__restrict__ kw,
                                                         const float *__restrict__ inv_freq, int d, int ratio,
                                                         int b0, int n, float eps)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * (QS_THREADS / 64) + (threadIdx.x >> 6);
    if (i >= n) return;
    const int b = b0 + i;
    float kn[M];
    qs_block_key<M>(kn, ikeys, kw, inv_freq, b, d, ratio, eps, lane);
#pragma unroll
    for (int m = 0; m < M; m++)
        if (lane + 64 * m < d) pool[(size_t)b * d + lane + 64 * m] = kn[m];
}

// ---- selection ------------------------------------------------------------------

#define QS_SEL_THREADS 1024
#define QS_SEL_WAVES (QS_SEL_THREADS / 64)
#define QS_SEL_MAX_BLOCKS 65536

__device__ __forceinline__ uint32_t qs_key(float v)
{
    if (!(v > -FLT_MAX)) return 0u;                 // never picked (also NaN)
    const uint32_t u = __float_as_uint(v + 0.0f);   // -0 -> +0
    return (u >> 31) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum of one value per thread over the workgroup, thread
// order; *total gets the sum.  Every thread calls it.
__device__ __forceinline__ uint32_t qs_scan(uint32_t v, uint32_t *wt, uint32_t *total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wt[wave] = x;
    __syncthreads();
    if (wave == 0) {
        uint32_t t = lane < QS_SEL_WAVES ? wt[lane] : 0u, s = t;
#pragma unroll
        for (int o = 1; o < QS_SEL_WAVES; o <<= 1) {
            const uint32_t y = __shfl_up(s, o, 64);
            if (lane >= o) s += y;
        }
        if (lane < QS_SEL_WAVES) wt[lane] = s - t;
        if (lane == QS_SEL_WAVES - 1) *total = s;
    }
    __syncthreads();
    const uint32_t r = x - v + wt[wave];
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(QS_SEL_THREADS) k_qsa_select(uint8_t *__restrict__ mask, uint32_t *__restrict__ list,
                                                               const float *__restrict__ scores, int ratio,
                                                               int base_pos, int block_topk, int max_ctx,
                                                               int max_blocks, int cap)
{
    extern __shared__ uint8_t sel[];
    __shared__ uint32_t hist[2048];
    __shared__ uint32_t wt[QS_SEL_WAVES];
    __shared__ uint32_t sh_total, sh_bin, sh_need;
    const int tid = threadIdx.x, r = blockIdx.x;
    const int n_keys = base_pos + r + 1, nb = n_keys / ratio;
    const float *sc = scores + (size_t)r * max_blocks;
    const int per = (nb + QS_SEL_THREADS - 1) / QS_SEL_THREADS;
    const int lo = min(tid * per, nb), hi = min(lo + per, nb);

    uint32_t cnt = 0;
    for (int b = lo; b < hi; b++) {
        sel[b] = 0;
        cnt += qs_key(sc[b]) != 0u;
    }
    qs_scan(cnt, wt, &sh_total);
    const uint32_t S = sh_total;
    const uint32_t take = min((uint32_t)max(block_topk, 0), S);
    if (take == S) {
        for (int b = lo; b < hi; b++) sel[b] = qs_key(sc[b]) != 0u;
    } else if (take > 0) {
        uint32_t prefix = 0, known = 0, need = take;
        const int shifts[3] = { 21, 10, 0 }, widths[3] = { 11, 11, 10 };
        for (int p = 0; p < 3; p++) {
            const int shift = shifts[p], nbins = 1 << widths[p];
            const uint32_t bmask = (uint32_t)nbins - 1u;
            for (int i = tid; i < nbins; i += QS_SEL_THREADS) hist[i] = 0;
            __syncthreads();
            for (int b = tid; b < nb; b += QS_SEL_THREADS) {
                const uint32_t k = qs_key(sc[b]);
                if ((k & known) == prefix) atomicAdd(&hist[(k >> shift) & bmask], 1u);
            }
            __syncthreads();
            // bins from the top: thread t holds bins nbins-1-2t and nbins-2-2t
            // (one bin, nbins-1-t, in the 10-bit pass)
            const int per_t = nbins / QS_SEL_THREADS;
            const int top = nbins - 1 - per_t * tid;
            const uint32_t c0 = hist[top], c1 = per_t == 2 ? hist[top - 1] : 0u;
            const uint32_t above = qs_scan(c0 + c1, wt, &sh_total);
            if (above < need && above + c0 + c1 >= need) {
                if (above + c0 >= need) { sh_bin = (uint32_t)top; sh_need = need - above; }
                else { sh_bin = (uint32_t)(top - 1); sh_need = need - above - c0; }
            }
            __syncthreads();
            prefix |= sh_bin << shift;
            known |= bmask << shift;
            need = sh_need;
            __syncthreads();
        }
        const uint32_t T = prefix;
        uint32_t eq = 0;
        for (int b = lo; b < hi; b++) {
            const uint32_t k = qs_key(sc[b]);
            if (k > T) sel[b] = 1;
            else eq += k == T;
        }
        uint32_t rank = qs_scan(eq, wt, &sh_total);
        for (int b = lo; b < hi && rank < need; b++)
            if (qs_key(sc[b]) == T) { sel[b] = 1; rank++; }
    }
    __syncthreads();
    uint32_t mine = 0;
    for (int b = lo; b < hi; b++) mine += sel[b];
    const uint32_t first = qs_scan(mine, wt, &sh_total);
    const uint32_t n_sel = sh_total;
    uint32_t *lr = list + (size_t)r * (1 + cap);
    uint32_t at = first * ratio;
    for (int b = lo; b < hi; b++)
        if (sel[b])
            for (int t = 0; t < ratio; t++) lr[1 + at++] = (uint32_t)(b * ratio + t);
    if (tid == 0) {
        uint32_t n = n_sel * ratio;
        for (int t = nb * ratio; t < n_keys; t++) lr[1 + n++] = (uint32_t)t;
        lr[0] = n;
    }
    uint8_t *mr = mask + (size_t)r * max_ctx;
    for (int t = tid; t < n_keys; t += QS_SEL_THREADS) mr[t] = t >= nb * ratio ? 1 : sel[t / ratio];
}

// ---- masked attention -------------------------------------------------------------

#define QA_D 256
#define QA_CHUNK 256

__device__ __forceinline__ float qa_f16(uint32_t bits)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
}

__device__ __forceinline__ void qa_h8(uint4 u, float *f)
{
    const uint32_t w[4] = { u.x, u.y, u.z, u.w };
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = qa_f16(w[i] & 0xFFFFu);
        f[2 * i + 1] = qa_f16(w[i] >> 16);
    }
}

template <int G>
__global__ void __launch_bounds__(256) k_attn_masked(float *__restrict__ out, const float *__restrict__ gate,
                                                     const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                     const uint16_t *__restrict__ vc, const uint32_t *__restrict__ list,
                                                     int q_heads, int kv_heads, int max_ctx, float scale, int cap)
{
    __shared__ float4 qs4[G][QA_D / 4];          // the G heads, pre-scaled
    __shared__ float ps[G][QA_CHUNK];            // the chunk's scores, then weights
    __shared__ float red[G][4];
    __shared__ float accw[4][G][QA_D];           // the waves' partial outputs
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = blockIdx.x / kv_heads, kvh = blockIdx.x % kv_heads;
    const uint32_t *lr = list + (size_t)row * (1 + cap);
    const int n_sel = (int)lr[0];
    const float *qp = q + ((size_t)row * q_heads + (size_t)kvh * G) * QA_D;
    for (int i = tid; i < G * QA_D; i += 256) reinterpret_cast<float *>(qs4)[i] = qp[i] * scale;
    const uint16_t *kbase = kc + (size_t)kvh * max_ctx * QA_D;
    const uint16_t *vbase = vc + (size_t)kvh * max_ctx * QA_D;

    float m[G], l[G], acc[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -FLT_MAX; l[g] = 0.0f;
        acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.0f;
    }
    __syncthreads();
    for (int j0 = 0; j0 < n_sel; j0 += QA_CHUNK) {
        const int n = min(QA_CHUNK, n_sel - j0);
        // scores: a thread per position
        if (tid < n) {
            const uint4 *kr = reinterpret_cast<const uint4 *>(kbase + (size_t)lr[1 + j0 + tid] * QA_D);
            float s[G];
#pragma unroll
            for (int g = 0; g < G; g++) s[g] = 0.0f;
            for (int c = 0; c < QA_D / 8; c++) {
                float kf[8];
                qa_h8(kr[c], kf);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float4 a = qs4[g][2 * c], b = qs4[g][2 * c + 1];
                    s[g] = __builtin_fmaf(a.x, kf[0], s[g]);
                    s[g] = __builtin_fmaf(a.y, kf[1], s[g]);
                    s[g] = __builtin_fmaf(a.z, kf[2], s[g]);
                    s[g] = __builtin_fmaf(a.w, kf[3], s[g]);
                    s[g] = __builtin_fmaf(b.x, kf[4], s[g]);
                    s[g] = __builtin_fmaf(b.y, kf[5], s[g]);
                    s[g] = __builtin_fmaf(b.z, kf[6], s[g]);
                    s[g] = __builtin_fmaf(b.w, kf[7], s[g]);
                }
            }
#pragma unroll
            for (int g = 0; g < G; g++) ps[g][tid] = s[g];
        }
        __syncthreads();
        // the chunk's max per head
#pragma unroll
        for (int g = 0; g < G; g++) {
            float v = tid < n ? ps[g][tid] : -FLT_MAX;
            v = qw_wave_max(v);
            if (lane == 0) red[g][wave] = v;
        }
        __syncthreads();
        float scale_old[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float cm = fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3]));
            const float mn = fmaxf(m[g], cm);
            scale_old[g] = expf(m[g] - mn);
            m[g] = mn;
        }
        __syncthreads();                             // red free, every thread has the maxima
        // weights, and the chunk's sum per head (lane-serial, then the wave
        // trees, then the waves in order)
#pragma unroll
        for (int g = 0; g < G; g++) {
            float e = 0.0f;
            if (tid < n) {
                e = expf(ps[g][tid] - m[g]);
                ps[g][tid] = e;
            }
            e = qw_xor_sum<64>(e);
            if (lane == 0) red[g][wave] = e;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++) {
            l[g] = l[g] * scale_old[g] + ((red[g][0] + red[g][1]) + (red[g][2] + red[g][3]));
#pragma unroll
            for (int i = 0; i < 4; i++) acc[g][i] *= scale_old[g];
        }
        // values: wave w takes positions w, w+4, ...; lane owns dims 4l..4l+3
        for (int jj = wave; jj < n; jj += 4) {
            const uint2 u = *reinterpret_cast<const uint2 *>(vbase + (size_t)lr[1 + j0 + jj] * QA_D + 4 * lane);
            const float v0 = qa_f16(u.x & 0xFFFFu);
            const float v1 = qa_f16(u.x >> 16);
            const float v2 = qa_f16(u.y & 0xFFFFu);
            const float v3 = qa_f16(u.y >> 16);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = ps[g][jj];
                acc[g][0] = __builtin_fmaf(p, v0, acc[g][0]);
                acc[g][1] = __builtin_fmaf(p, v1, acc[g][1]);
                acc[g][2] = __builtin_fmaf(p, v2, acc[g][2]);
                acc[g][3] = __builtin_fmaf(p, v3, acc[g][3]);
            }
        }
        __syncthreads();                             // ps and red free for the next chunk
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < 4; i++) accw[wave][g][4 * lane + i] = acc[g][i];
    __syncthreads();
    for (int i = tid; i < G * QA_D; i += 256) {
        const int g = i / QA_D, dim = i % QA_D;
        const float s = (accw[0][g][dim] + accw[1][g][dim]) + (accw[2][g][dim] + accw[3][g][dim]);
        float o = l[g] > 0.0f ? s / l[g] : 0.0f;
        const size_t oi = ((size_t)row * q_heads + (size_t)kvh * G + g) * QA_D + dim;
        if (gate) o *= 1.0f / (1.0f + expf(-gate[oi]));
        out[oi] = o;
    }
}

// ---- launchers ----------------------------------------------------------------------

static bool qs_shape_ok(int d, int rotary_dim) { return rotary_dim == QS_ROTARY && d >= 64 && d % 32 == 0 && d <= 256; }

template <bool POOLED>
static int qs_launch_scores(hipStream_t s, float *scores, const float *qn, const float *src, const uint16_t *kw,
                            const float *inv_freq, int rows, int nq, int d, int ratio, int base_pos,
                            int max_blocks, float eps)
{
    const int blocks = (base_pos + rows) / ratio;
    if (blocks == 0) return 0;
    const dim3 grid((blocks + QS_BLK - 1) / QS_BLK, (rows + QS_ROWS - 1) / QS_ROWS);
    const int D = d <= 64 ? 64 : d <= 128 ? 128 : d <= 192 ? 192 : 256;
    const size_t lds = ((size_t)QS_BLK * (D + 4) + 4 * QS_BLK + (size_t)nq * D) * sizeof(float);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
#define QS_GO(DD) hipLaunchKernelGGL((k_qsa_scores<DD, POOLED>), grid, dim3(QS_THREADS), lds, s, scores, qn, src, kw, \
                                     inv_freq, rows, nq, d, ratio, base_pos, max_blocks, eps)
    switch (D) {
    case 64: QS_GO(64); break;
    case 128: QS_GO(128); break;
    case 192: QS_GO(192); break;
    default: QS_GO(256); break;
    }
#undef QS_GO
    return (int)hipGetLastError();
}

extern "C" int qwk_qsa_scores(hipStream_t s, float *scores, const float *qn, const float *ikeys, const uint16_t *kw,
                              const float *inv_freq, int rows, int nq, int d, int ratio, int base_pos,
                              int rotary_dim, int max_blocks, float eps)
{
    if (!qs_shape_ok(d, rotary_dim) || rows < 0 || nq < 1 || ratio < 1 || base_pos < 0 ||
        (base_pos + rows) / ratio > max_blocks)
        return hipErrorInvalidValue;
    static bool attr = false;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute((const void *)k_qsa_scores<256, false>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)k_qsa_scores<192, false>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)k_qsa_scores<256, true>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)k_qsa_scores<192, true>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)k_qsa_scores<128, false>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)k_qsa_scores<128, true>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    }
    return qs_launch_scores<false>(s, scores, qn, ikeys, kw, inv_freq, rows, nq, d, ratio, base_pos, max_blocks, eps);
}

extern "C" int qwk_qsa_scores_pooled(hipStream_t s, float *scores, const float *qn, const float *pool, int rows,
                                     int nq, int d, int ratio, int base_pos, int max_blocks)
{
    if (!qs_shape_ok(d, QS_ROTARY) || rows < 0 || nq < 1 || ratio < 1 || base_pos < 0 ||
        (base_pos + rows) / ratio > max_blocks)
        return hipErrorInvalidValue;
    return qs_launch_scores<true>(s, scores, qn, pool, nullptr, nullptr, rows, nq, d, ratio, base_pos, max_blocks, 0.0f);
}

extern "C" int qwk_qsa_pool(hipStream_t s, float *pool, const float *ikeys, const uint16_t *kw, const float *inv_freq,
                            int d, int ratio, int b0, int b1, int rotary_dim, float eps)
{
    if (!qs_shape_ok(d, rotary_dim) || ratio < 1 || b0 < 0) return hipErrorInvalidValue;
    if (b1 <= b0) return 0;
    const int n = b1 - b0;
    const dim3 grid((n + 3) / 4);
    if (d <= 64) hipLaunchKernelGGL(k_qsa_pool<1>, grid, dim3(QS_THREADS), 0, s, pool, ikeys, kw, inv_freq, d, ratio, b0, n, eps);
    else if (d <= 128) hipLaunchKernelGGL(k_qsa_pool<2>, grid, dim3(QS_THREADS), 0, s, pool, ikeys, kw, inv_freq, d, ratio, b0, n, eps);
    else if (d <= 192) hipLaunchKernelGGL(k_qsa_pool<3>, grid, dim3(QS_THREADS), 0, s, pool, ikeys, kw, inv_freq, d, ratio, b0, n, eps);
    else hipLaunchKernelGGL(k_qsa_pool<4>, grid, dim3(QS_THREADS), 0, s, pool, ikeys, kw, inv_freq, d, ratio, b0, n, eps);
    return (int)hipGetLastError();
}

extern "C" int qwk_qsa_select(hipStream_t s, uint8_t *mask, uint32_t *list, const float *scores, int rows, int ratio,
                              int base_pos, int block_topk, int max_ctx, int max_blocks)
{
    if (rows < 0 || ratio < 1 || base_pos < 0 || block_topk < 0 || base_pos + rows > max_ctx ||
        (base_pos + rows) / ratio > max_blocks || max_blocks > QS_SEL_MAX_BLOCKS)
        return hipErrorInvalidValue;
    if (rows == 0) return 0;
    const int cap = block_topk * ratio + ratio;
    const size_t lds = ((size_t)((base_pos + rows) / ratio) + 16) & ~(size_t)15;
    static bool attr = false;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute((const void *)k_qsa_select, hipFuncAttributeMaxDynamicSharedMemorySize, QS_SEL_MAX_BLOCKS + 16);
    }
    hipLaunchKernelGGL(k_qsa_select, dim3(rows), dim3(QS_SEL_THREADS), lds, s, mask, list, scores, ratio, base_pos,
                       block_topk, max_ctx, max_blocks, cap);
    return (int)hipGetLastError();
}

extern "C" int qwk_attn_masked(hipStream_t s, float *out, const float *gate, const float *q, const uint16_t *kc,
                               const uint16_t *vc, const uint32_t *list, int rows, int q_heads, int kv_heads,
                               int head_dim, int max_ctx, float scale, int cap)
{
    if (head_dim != QA_D || kv_heads < 1 || q_heads % kv_heads || rows < 0 || cap < 0) return hipErrorInvalidValue;
    if (rows == 0) return 0;
    const dim3 grid(rows * kv_heads);
    switch (q_heads / kv_heads) {
    case 1: hipLaunchKernelGGL(k_attn_masked<1>, grid, dim3(256), 0, s, out, gate, q, kc, vc, list, q_heads, kv_heads, max_ctx, scale, cap); break;
    case 2: hipLaunchKernelGGL(k_attn_masked<2>, grid, dim3(256), 0, s, out, gate, q, kc, vc, list, q_heads, kv_heads, max_ctx, scale, cap); break;
    case 4: hipLaunchKernelGGL(k_attn_masked<4>, grid, dim3(256), 0, s, out, gate, q, kc, vc, list, q_heads, kv_heads, max_ctx, scale, cap); break;
    case 8: hipLaunchKernelGGL(k_attn_masked<8>, grid, dim3(256), 0, s, out, gate, q, kc, vc, list, q_heads, kv_heads, max_ctx, scale, cap); break;
    default: return hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}
