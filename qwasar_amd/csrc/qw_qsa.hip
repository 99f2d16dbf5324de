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
// and NaN, which the reference's scan never picks, to 0).  A radix search
// over key - kmin (the selectable keys' range), 8 bits a pass from the
// range's top bit and counted into per-wave histograms, finds the exact key
// T of the last block taken (scores of similar size share their leading
// bits: counted from bit 31 they would pile into a few bins and serialise
// the atomics); keys above T are taken and the rest of the budget comes from keys
// equal to T in block order.  One wave sums the bins and finds the cut with a
// suffix scan over its lanes; a pass whose cut bin holds exactly the blocks
// still needed ends the search.  Each thread owns a contiguous run of blocks,
// its keys loaded at once into registers, so block order is thread order and
// the position list is one prefix sum.
//
// Masked attention (k_attn_masked<G>): a workgroup per (query row, kv head,
// split of the position list) with its G query heads.  Positions go 32 at a
// time, 8 a wave: eight lanes per position score its fp16 key row against
// the G heads, each wave's maxima and weights (2^(s - max), scores in log2
// units) update its own online softmax, and the wave accumulates its
// positions' value rows with lanes over dims (each value row one coalesced
// 512-byte read); the four waves' states meet at the end.  When rows x kv heads alone would leave
// the chip idle (decode), the list is split over enough workgroups to fill
// it and k_attn_merge combines the splits' softmax states in split order.
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
    // keeps the key in registers: without this the compiler re-reads it from
    // LDS inside every head's dot
#pragma unroll
    for (int i = 0; i < D; i++) asm volatile("" : "+v"(kr[i]));
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

// Phase 1: the workgroup's QS_BLK block keys into LDS, row stride D + 4, dims
// past d and blocks from nb_hi on zero.
template <int D, bool POOLED>
__device__ __forceinline__ void qs_keys_to_lds(float *kl, const float *__restrict__ src, const uint16_t *__restrict__ kw,
                                               const float *__restrict__ inv_freq, int b0, int nb_hi, int d,
                                               int ratio, float eps)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (POOLED) {
        for (int i = tid; i < QS_BLK * (D / 4); i += QS_THREADS) {
            const int bl = i / (D / 4), j = 4 * (i % (D / 4));
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const int b = b0 + bl;
            if (b < nb_hi && j < d)   // d % 32 == 0: a float4 is wholly in or out
                v = *reinterpret_cast<const float4 *>(src + (size_t)b * d + j);
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
}

template <int D, bool POOLED>
__global__ void __launch_bounds__(QS_THREADS) __attribute__((amdgpu_waves_per_eu(1, 2))) k_qsa_scores(float *__restrict__ scores, const float *__restrict__ qn,
                                                           const float *__restrict__ src,
                                                           const uint16_t *__restrict__ kw,
                                                           const float *__restrict__ inv_freq, int rows, int nq,
                                                           int d, int ratio, int base_pos, int max_blocks, float eps)
{
    extern __shared__ float4 qs_lds[];
    float *kl = reinterpret_cast<float *>(qs_lds);            // [QS_BLK][D + 4]
    float *part = kl + QS_BLK * (D + 4);                       // [4][QS_BLK]
    float *ql = part + 4 * QS_BLK;                             // [nq][D]
    const int b0 = blockIdx.x * QS_BLK, r0 = blockIdx.y * QS_ROWS;
    const int nb_hi = (base_pos + min(r0 + QS_ROWS, rows)) / ratio;   // blocks any row of the tile sees
    if (nb_hi <= b0) return;                                   // uniform
    qs_keys_to_lds<D, POOLED>(kl, src, kw, inv_freq, b0, nb_hi, d, ratio, eps);
    __syncthreads();
    qs_score_rows<D>(scores, qn, kl, ql, part, b0, r0, rows, nq, d, ratio, base_pos, max_blocks);
}

// The same scores on the fp32 matrix cores (nq <= 16, D <= 128, many rows).
// v_mfma_f32_16x16x1_4b_f32 adds a 16x16 outer product to its accumulator in
// each of four blocks, one rounding per element: element (i, j) of a block
// takes fmaf(a_i, b_j, c), so D of them in dim order are phase 2's chain
// (from 0, dims ascending), bit for bit.  Lane l feeds B column l % 16 of
// block l / 16 with its own block's key -- block b0 + l, held in registers
// for the whole tile -- and A row l % 16 of every block with one query row's
// head hd(l % 16), hd(i) = 4 (i % 4) + i / 4 (heads past nq zero: a zero dot,
// never summed).  Accumulator e of lane l is then block column 16 (e / 4) +
// l % 16 against A row 4 (l / 16) + e % 4, head l / 16 + 4 (e % 4): the lanes
// of group g = l / 16 hold heads g, g + 4, g + 8, g + 12 in e order, the
// heads phase 2's wave g sums, in its order.  Two xor shuffles (16, then 32)
// form (p0 + p1) + (p2 + p3) (each pair's sum the same bits whichever lane
// adds it), and lane l writes block b0 + l.  A workgroup scores its 64 blocks
// against QM_ROWS rows, eight at a time: the eight rows' heads are staged in
// LDS (over the block keys, once those are in registers), each wave runs two
// rows' chains interleaved.
#define QM_ROWS 32
#define QM_GROUP 8                                 // rows staged at once: 2 a wave
template <int D, bool POOLED>
__global__ void __launch_bounds__(QS_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) k_qsa_scores_mx(
    float *__restrict__ scores, const float *__restrict__ qn, const float *__restrict__ src,
    const uint16_t *__restrict__ kw, const float *__restrict__ inv_freq, int rows, int nq, int d, int ratio,
    int base_pos, int max_blocks, float eps)
{
    typedef float f16v __attribute__((ext_vector_type(4 * 4)));
    constexpr int QST = 16 * (D + 4);                          // floats a staged row
    __shared__ float4 lds4[(QM_GROUP * QST > QS_BLK * (D + 4) ? QM_GROUP * QST : QS_BLK * (D + 4)) / 4];
    float *lds = reinterpret_cast<float *>(lds4);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b0 = blockIdx.x * QS_BLK, r0 = blockIdx.y * QM_ROWS;
    const int rend = min(r0 + QM_ROWS, rows);
    const int nb_hi = (base_pos + rend) / ratio;
    if (nb_hi <= b0) return;                                   // uniform
    qs_keys_to_lds<D, POOLED>(lds, src, kw, inv_freq, b0, nb_hi, d, ratio, eps);
    __syncthreads();
    float kr[D];
#pragma unroll
    for (int i = 0; i < D; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(lds + lane * (D + 4) + i);
        kr[i] = v.x; kr[i + 1] = v.y; kr[i + 2] = v.z; kr[i + 3] = v.w;
    }
    const float rs = sqrtf((float)d);
    const int g = lane >> 4;
    const float *qa = lds + (2 * wave) * QST + (lane & 15) * (D + 4), *qb = qa + QST;
    for (int g0 = r0; g0 < rend; g0 += QM_GROUP) {
        const int gl = min(g0 + QM_GROUP, rend);
        if ((base_pos + gl) / ratio <= b0) continue;           // uniform: no row of the group sees these blocks
        __syncthreads();                                       // the keys are in registers / the last group is done
        // stage: A row i of staged row t holds head hd(i) (4 x 4 transpose: its own inverse)
        for (int q = tid; q < QM_GROUP * 16 * (D / 4); q += QS_THREADS) {
            const int t = q / (16 * (D / 4)), i = (q / (D / 4)) % 16, j = 4 * (q % (D / 4));
            const int h = 4 * (i % 4) + i / 4, r = g0 + t;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r < gl && h < nq && j < d) v = *reinterpret_cast<const float4 *>(qn + ((size_t)r * nq + h) * d + j);
            *reinterpret_cast<float4 *>(lds + t * QST + i * (D + 4) + j) = v;
        }
        __syncthreads();
        f16v acc0 = {}, acc1 = {};
#pragma unroll
        for (int k = 0; k < D; k += 4) {
            const float4 a0 = *reinterpret_cast<const float4 *>(qa + k), a1 = *reinterpret_cast<const float4 *>(qb + k);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x1f32(a0.x, kr[k], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x1f32(a1.x, kr[k], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x1f32(a0.y, kr[k + 1], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x1f32(a1.y, kr[k + 1], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x1f32(a0.z, kr[k + 2], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x1f32(a1.z, kr[k + 2], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x1f32(a0.w, kr[k + 3], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x1f32(a1.w, kr[k + 3], acc1, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int r = g0 + 2 * wave + u;
            const f16v &acc = u ? acc1 : acc0;
            float mine = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float p = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; t++)
                    if (acc[4 * c + t] > 0.0f) p += acc[4 * c + t];
                const float x = p + __shfl_xor(p, 16, 64);
                const float sc = x + __shfl_xor(x, 32, 64);
                if (c == g) mine = sc;
            }
            const int b = b0 + lane;
            if (r < gl && b < (base_pos + r + 1) / ratio) scores[(size_t)r * max_blocks + b] = mine / rs;
        }
    }
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


#define QS_SEL_KREG 8      // keys a thread keeps in registers (up to 8192 blocks)

// A thread's contiguous run of blocks [lo, hi): its keys, from registers
// when the run fits, else from the scores.
#define QS_RUN(body)                                                              \
    if (in_regs) {                                                                \
        _Pragma("unroll") for (int i = 0; i < QS_SEL_KREG; i++)                   \
            if (lo + i < hi) { const int b = lo + i; const uint32_t k = kr[i]; body } \
    } else {                                                                      \
        for (int b = lo; b < hi; b++) { const uint32_t k = qs_key(sc[b]); body }  \
    }

// The count, minimum and maximum of the selectable keys over the workgroup
// (one barrier); every thread gets all three.
__device__ __forceinline__ void qs_reduce3(uint32_t &cnt, uint32_t &mn, uint32_t &mx, uint4 *wt3)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        cnt += (uint32_t)__shfl_xor((int)cnt, o, 64);
        mn = min(mn, (uint32_t)__shfl_xor((int)mn, o, 64));
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, o, 64));
    }
    if (lane == 0) wt3[wave] = make_uint4(cnt, mn, mx, 0u);
    __syncthreads();
    cnt = 0; mn = 0xFFFFFFFFu; mx = 0u;
#pragma unroll
    for (int w = 0; w < QS_SEL_WAVES; w++) {
        const uint4 v = wt3[w];
        cnt += v.x; mn = min(mn, v.y); mx = max(mx, v.z);
    }
}

__global__ void __launch_bounds__(QS_SEL_THREADS) k_qsa_select(uint8_t *__restrict__ mask, uint32_t *__restrict__ list,
                                                               const float *__restrict__ scores, int ratio,
                                                               int base_pos, int block_topk, int max_ctx,
                                                               int max_blocks, int cap)
{
    extern __shared__ uint8_t sel[];
    // a histogram per wave (no cross-wave atomics), two sets: a pass counts
    // into one while it clears the other for the next pass
    __shared__ uint32_t hist[2][QS_SEL_WAVES][256];
    __shared__ uint32_t wt[QS_SEL_WAVES];
    __shared__ uint4 wt3[QS_SEL_WAVES];
    __shared__ uint32_t sh_total, sh_bin, sh_need, sh_exact;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = blockIdx.x;
    const int n_keys = base_pos + r + 1, nb = n_keys / ratio;
    const float *sc = scores + (size_t)r * max_blocks;
    const int per = (nb + QS_SEL_THREADS - 1) / QS_SEL_THREADS;
    const int lo = min(tid * per, nb), hi = min(lo + per, nb);
    const bool in_regs = per <= QS_SEL_KREG;
    // every load of the run issued before the first use (in-range addresses
    // for the lanes past the run, whose keys are then dropped)
    uint32_t kr[QS_SEL_KREG];
    if (in_regs && nb > 0) {
        float v[QS_SEL_KREG];
        if (per == QS_SEL_KREG && (reinterpret_cast<uintptr_t>(sc) & 15) == 0 && lo + QS_SEL_KREG <= max_blocks) {
            // two 16-byte loads (the run starts at a multiple of 8 blocks)
            const float4 a = reinterpret_cast<const float4 *>(sc + lo)[0];
            const float4 b = reinterpret_cast<const float4 *>(sc + lo)[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < QS_SEL_KREG; i++) v[i] = sc[min(lo + i, nb - 1)];
        }
#pragma unroll
        for (int i = 0; i < QS_SEL_KREG; i++) kr[i] = lo + i < hi ? qs_key(v[i]) : 0u;
    } else {
#pragma unroll
        for (int i = 0; i < QS_SEL_KREG; i++) kr[i] = 0u;
    }
    uint4 *h0 = reinterpret_cast<uint4 *>(&hist[0][0][0]);
    h0[tid] = make_uint4(0u, 0u, 0u, 0u);   // 16 x 256 words: one uint4 a thread

    uint32_t S = 0, mn = 0xFFFFFFFFu, mx = 0u;
    QS_RUN(if (k) { S++; mn = min(mn, k); mx = max(mx, k); })
    qs_reduce3(S, mn, mx, wt3);
    const uint32_t take = min((uint32_t)max(block_topk, 0), S);
    // blocks taken: key > T, then the first `need` blocks whose key equals T
    uint32_t T = 0u, need = 0u;
    if (take == 0) {
        T = 0xFFFFFFFFu;
    } else if (take < S) {
        // the key of the take-th largest.  The passes count u = key - kmin
        // (kmin, kmax: the selectable keys' range), 8 bits at a time from
        // the range's top bit, so even scores that share their leading bits
        // spread over the bins.  A pass whose bin holds exactly the blocks
        // still needed ends the search: the bin's lowest key bounds the take.
        const uint32_t range = mx - mn;
        const int nbits = range ? 32 - __builtin_clz(range) : 0;
        uint32_t prefix = 0;
        bool exact = false;
        int prev = 32, shift = nbits > 8 ? nbits - 8 : 0, cur = 0;
        need = take;
        while (true) {
            const uint32_t bmask = prev - shift >= 32 ? 0xFFFFFFFFu : ((1u << (prev - shift)) - 1u);
            const uint32_t hp = prev >= 32 ? 0u : prefix >> prev;
            reinterpret_cast<uint4 *>(&hist[cur ^ 1][0][0])[tid] = make_uint4(0u, 0u, 0u, 0u);
            QS_RUN(if (k) {
                const uint32_t u = k - mn;
                if ((prev >= 32 ? 0u : u >> prev) == hp) atomicAdd(&hist[cur][wave][(u >> shift) & bmask], 1u);
            })
            __syncthreads();
            if (wave == 0) {
                // lane l: bins 4l .. 4l+3 summed over the waves; counts above
                // a lane's bins are a suffix sum over the lanes
                uint4 c = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
                for (int w = 0; w < QS_SEL_WAVES; w++) {
                    const uint4 v = reinterpret_cast<const uint4 *>(&hist[cur][w][0])[lane];
                    c.x += v.x; c.y += v.y; c.z += v.z; c.w += v.w;
                }
                const uint32_t tl = c.x + c.y + c.z + c.w;
                uint32_t sfx = tl;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const uint32_t y = (uint32_t)__shfl_down((int)sfx, o, 64);
                    if (lane + o < 64) sfx += y;
                }
                uint32_t a = sfx - tl;
                const uint32_t cj[4] = {c.w, c.z, c.y, c.x};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (a < need && a + cj[j] >= need) {
                        sh_bin = (uint32_t)(4 * lane + 3 - j);
                        sh_need = need - a;
                        sh_exact = a + cj[j] == need;
                    }
                    a += cj[j];
                }
            }
            __syncthreads();
            prefix |= sh_bin << shift;
            need = sh_need;
            exact = sh_exact != 0u;
            if (exact || shift == 0) break;
            prev = shift;
            shift = shift > 8 ? shift - 8 : 0;
            cur ^= 1;
        }
        T = prefix + mn;   // back from the range's offset to the key
        if (exact) { T -= 1u; need = 0u; }   // T >= kmin >= 1
    }
    uint32_t selm = 0, eq = 0;
    if (in_regs) {
#pragma unroll
        for (int i = 0; i < QS_SEL_KREG; i++) {
            if (lo + i < hi) {
                if (kr[i] > T) selm |= 1u << i;
                else eq += kr[i] == T;
            }
        }
    } else {
        for (int b = lo; b < hi; b++) {
            const uint32_t k = qs_key(sc[b]);
            sel[b] = k > T;
            eq += k == T;
        }
    }
    if (need > 0u) {   // uniform
        uint32_t rank = qs_scan(eq, wt, &sh_total);
        QS_RUN(if (k == T && rank < need) {
            if (in_regs) selm |= 1u << (b - lo); else sel[b] = 1;
            rank++;
        })
    }
    uint32_t mine = 0;
    if (in_regs) {
#pragma unroll
        for (int i = 0; i < QS_SEL_KREG; i++)
            if (lo + i < hi) sel[lo + i] = (uint8_t)((selm >> i) & 1u);
        mine = __builtin_popcount(selm);
    } else {
        for (int b = lo; b < hi; b++) mine += sel[b];
    }
    const uint32_t first = qs_scan(mine, wt, &sh_total);   // its barriers publish sel
    const uint32_t n_sel = sh_total;
    uint32_t *lr = list + (size_t)r * (1 + cap);
    uint32_t at = 1 + first * ratio;
    if (in_regs) {
#pragma unroll
        for (int i = 0; i < QS_SEL_KREG; i++)
            if ((selm >> i) & 1u)
                for (int t = 0; t < ratio; t++) lr[at++] = (uint32_t)((lo + i) * ratio + t);
    } else {
        for (int b = lo; b < hi; b++)
            if (sel[b])
                for (int t = 0; t < ratio; t++) lr[at++] = (uint32_t)(b * ratio + t);
    }
    if (tid == 0) {
        uint32_t n = n_sel * ratio;
        for (int t = nb * ratio; t < n_keys; t++) lr[1 + n++] = (uint32_t)t;
        lr[0] = n;
    }
    uint8_t *mr = mask + (size_t)r * max_ctx;
    int t0 = 0;
    if (ratio == 4 && (reinterpret_cast<uintptr_t>(mr) & 15) == 0) {
        // four blocks (16 positions) a 16-byte store
        const int n4 = nb >> 2;
        for (int w = tid; w < n4; w += QS_SEL_THREADS) {
            const uint32_t x = reinterpret_cast<const uint32_t *>(sel)[w];
            reinterpret_cast<uint4 *>(mr)[w] = make_uint4((x & 1u) * 0x01010101u, ((x >> 8) & 1u) * 0x01010101u,
                                                          ((x >> 16) & 1u) * 0x01010101u, (x >> 24) * 0x01010101u);
        }
        t0 = n4 * 16;
    }
    for (int t = t0 + tid; t < n_keys; t += QS_SEL_THREADS) mr[t] = t >= nb * ratio ? 1 : sel[t / ratio];
}
#undef QS_RUN

// ---- masked attention -------------------------------------------------------------

#define QA_D 256
#define QA_P 32            // positions a workgroup takes per pass
#define QA_QPOS(i) ((i) + (i) / 8)   // float4 i of a head in its padded LDS row
#define QA_QROW (QA_D / 4 + QA_D / 32)

#define QA_LOG2E 1.44269504088896340736f

// 2^x by the hardware's exp2 (v_exp_f32); results below the normal range
// flush to zero, which a softmax weight relative to the maximum can afford
__device__ __forceinline__ float qa_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float qa_f16(uint32_t bits)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
}

// A workgroup per (query row, kv head, split): the split's share of the
// row's listed positions, QA_P at a time.  With one split it writes the
// output; otherwise its softmax state (max, sum, unnormalised output per
// head) goes to `part` and k_attn_merge combines the splits in order.
template <int G>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) k_attn_masked(float *__restrict__ out, const float *__restrict__ gate,
                                                     const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                     const uint16_t *__restrict__ vc, const uint32_t *__restrict__ list,
                                                     int q_heads, int kv_heads, int max_ctx, float scale, int cap,
                                                     int nsplit, float *__restrict__ part)
{
    // the G heads, pre-scaled; each 32-dim piece padded by 16 bytes so the
    // eight pieces a score reads at once start in different banks
    __shared__ float4 qs4[G][QA_QROW];
    __shared__ float ps[G][QA_P];                // a pass's weights (wave w: [8w, 8w + 8))
    __shared__ float wm[4][G], wl[4][G];         // the waves' softmax states
    __shared__ float wbuf[G][QA_D];              // the waves' partial outputs meet here
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x % nsplit, rk = blockIdx.x / nsplit;
    const int row = rk / kv_heads, kvh = rk % kv_heads;
    const uint32_t *lr = list + (size_t)row * (1 + cap);
    // the splits divide the list's capacity, so a split knows its range
    // before the list's length arrives: its first pass's entries are
    // requested with the length (entries past the length are not positions
    // and are clamped to a valid row, then dropped)
    const int per = ((cap + QA_P - 1) / QA_P + nsplit - 1) / nsplit;
    const int j_lo = min(split * per * QA_P, cap), j_cap = min(j_lo + per * QA_P, cap);
    const int jb = (QA_P / 4) * wave, jj = tid >> 3, kp = tid & 7;
    uint32_t vi[QA_P / 4], ki = 0;
    auto load_list = [&](int j0) {
#pragma unroll
        for (int i = 0; i < QA_P / 4; i++) vi[i] = lr[1 + min(j0 + jb + i, cap - 1)];
        ki = lr[1 + min(j0 + jj, cap - 1)];
    };
    const int n_sel = (int)lr[0];
    if (j_lo < j_cap) load_list(j_lo);
    const int j_hi = min(j_cap, n_sel);
    const float4 *qp = reinterpret_cast<const float4 *>(q + ((size_t)row * q_heads + (size_t)kvh * G) * QA_D);
    const float sl2 = scale * QA_LOG2E;   // scores in log2 units: weights are 2^(s - max)
    {
        constexpr int NQ = (G * QA_D / 4 + 255) / 256;
        float4 qv[NQ];
#pragma unroll
        for (int u = 0; u < NQ; u++)
            if (tid + 256 * u < G * QA_D / 4) qv[u] = qp[tid + 256 * u];
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int f = tid + 256 * u;
            if (f < G * QA_D / 4)
                qs4[f / (QA_D / 4)][QA_QPOS(f % (QA_D / 4))] =
                    make_float4(qv[u].x * sl2, qv[u].y * sl2, qv[u].z * sl2, qv[u].w * sl2);
        }
    }
    const uint16_t *kbase = kc + (size_t)kvh * max_ctx * QA_D;
    const uint16_t *vbase = vc + (size_t)kvh * max_ctx * QA_D;

    float m[G], l[G], acc[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -FLT_MAX; l[g] = 0.0f;
        acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.0f;
    }
    __syncthreads();
    for (int j0 = j_lo; j0 < j_hi; j0 += QA_P) {
        const int n = min(QA_P, j_hi - j0), nj = max(0, min(QA_P / 4, n - jb));
        if (j0 != j_lo) load_list(j0);
        // every key and value row of the pass at once, the keys first
#pragma unroll
        for (int i = 0; i < QA_P / 4; i++) vi[i] = min(vi[i], (uint32_t)(max_ctx - 1));
        ki = min(ki, (uint32_t)(max_ctx - 1));
        uint4 kv[4];
        {
            const uint4 *kr = reinterpret_cast<const uint4 *>(kbase + (size_t)ki * QA_D + 32 * kp);
#pragma unroll
            for (int c = 0; c < 4; c++) kv[c] = kr[c];
        }
        uint2 vv[QA_P / 4];
#pragma unroll
        for (int i = 0; i < QA_P / 4; i++)
            vv[i] = *reinterpret_cast<const uint2 *>(vbase + (size_t)vi[i] * QA_D + 4 * lane);
        // the key rows, issued before the value rows, are waited for here
        // (the value rows stay in flight through the scores)
#pragma unroll
        for (int c = 0; c < 4; c++) asm volatile("" : "+v"(kv[c].x), "+v"(kv[c].y), "+v"(kv[c].z), "+v"(kv[c].w));
        // scores: eight threads per position, 32 dims each (one 64-byte
        // piece of the fp16 key row); the eight partial dots meet in the xor
        // tree of their 8-lane run.  Wave w scores positions 8w .. 8w+7 of
        // the pass, the ones its values take below, so the pass needs no
        // barrier: each wave runs its own softmax state
        const bool valid = jj < n;
        float sg[G];
#pragma unroll
        for (int g = 0; g < G; g++) sg[g] = 0.0f;
        if (valid) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t w[4] = { kv[c].x, kv[c].y, kv[c].z, kv[c].w };
                const int d0 = 32 * kp + 8 * c;
                float kf[8];
#pragma unroll
                for (int e = 0; e < 4; e++) { kf[2 * e] = qa_f16(w[e] & 0xFFFFu); kf[2 * e + 1] = qa_f16(w[e] >> 16); }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float4 a = qs4[g][QA_QPOS(d0 / 4)], b = qs4[g][QA_QPOS(d0 / 4) + 1];
                    sg[g] = __builtin_fmaf(a.x, kf[0], sg[g]);
                    sg[g] = __builtin_fmaf(a.y, kf[1], sg[g]);
                    sg[g] = __builtin_fmaf(a.z, kf[2], sg[g]);
                    sg[g] = __builtin_fmaf(a.w, kf[3], sg[g]);
                    sg[g] = __builtin_fmaf(b.x, kf[4], sg[g]);
                    sg[g] = __builtin_fmaf(b.y, kf[5], sg[g]);
                    sg[g] = __builtin_fmaf(b.z, kf[6], sg[g]);
                    sg[g] = __builtin_fmaf(b.w, kf[7], sg[g]);
                }
            }
        }
        // per head: the wave's maximum over its positions (lane bits 3-5),
        // the online rescale, the weights (into this wave's slice of ps) and
        // their sum in a fixed tree.  The 8 lanes of a position hold one
        // value, so the xor steps 8, 16, 32 are a row mirror (it pairs
        // position 2r with 2r + 1, as xor 8 does) and the row sums read from
        // lanes 0, 16, 32, 48, added (0 + 16) + (32 + 48) as xor 16 then 32
        // add them: the same bits, in the VALU (a shuffle goes through LDS)
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float sc = qw_xor_sum<8>(sg[g]);
            float cm = valid ? sc : -FLT_MAX;
            cm = fmaxf(cm, qw_dpp<QW_DPP_MIRROR>(cm));
            cm = fmaxf(fmaxf(qw_lane(cm, 0), qw_lane(cm, 16)), fmaxf(qw_lane(cm, 32), qw_lane(cm, 48)));
            const float mn = fmaxf(m[g], cm);
            const float rs = qa_exp2(m[g] - mn);
            m[g] = mn;
            float e = valid ? qa_exp2(sc - mn) : 0.0f;
            if (kp == 0) ps[g][jj] = e;
            e = e + qw_dpp<QW_DPP_MIRROR>(e);
            e = (qw_lane(e, 0) + qw_lane(e, 16)) + (qw_lane(e, 32) + qw_lane(e, 48));
            l[g] = l[g] * rs + e;
#pragma unroll
            for (int i = 0; i < 4; i++) acc[g][i] *= rs;
        }
        // values: lane dims 4l..4l+3 of the wave's positions (their rows
        // were requested with the keys); the weights come back from the
        // wave's own slice of ps (its writes above, in program order)
#pragma unroll
        for (int i = 0; i < QA_P / 4; i++) {
            if (i < nj) {
                const float v0 = qa_f16(vv[i].x & 0xFFFFu), v1 = qa_f16(vv[i].x >> 16);
                const float v2 = qa_f16(vv[i].y & 0xFFFFu), v3 = qa_f16(vv[i].y >> 16);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = ps[g][jb + i];
                    acc[g][0] = __builtin_fmaf(p, v0, acc[g][0]);
                    acc[g][1] = __builtin_fmaf(p, v1, acc[g][1]);
                    acc[g][2] = __builtin_fmaf(p, v2, acc[g][2]);
                    acc[g][3] = __builtin_fmaf(p, v3, acc[g][3]);
                }
            }
        }
    }
    // the four waves' states meet: the common maximum, each wave's factor,
    // the sums (w0 + w1) + (w2 + w3), and the outputs in the same tree
    // through wbuf and the query array (no longer read)
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) { wm[wave][g] = m[g]; wl[wave][g] = l[g]; }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float M = fmaxf(fmaxf(wm[0][g], wm[1][g]), fmaxf(wm[2][g], wm[3][g]));
        const float f = qa_exp2(m[g] - M);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[g][i] *= f;
        if (wave == 0) {
            l[g] = (wl[0][g] * qa_exp2(wm[0][g] - M) + wl[1][g] * qa_exp2(wm[1][g] - M)) +
                   (wl[2][g] * qa_exp2(wm[2][g] - M) + wl[3][g] * qa_exp2(wm[3][g] - M));
            m[g] = M;
        }
    }
    float *bufA = &wbuf[0][0], *bufB = reinterpret_cast<float *>(&qs4[0][0]);
    __syncthreads();                                 // every wave's scores are done with qs4
    if (wave == 1 || wave == 3) {
        float *dst = wave == 1 ? bufA : bufB;
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) dst[g * QA_D + 4 * lane + i] = acc[g][i];
    }
    __syncthreads();
    if (wave == 0 || wave == 2) {
        const float *src = wave == 0 ? bufA : bufB;
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[g][i] = acc[g][i] + src[g * QA_D + 4 * lane + i];
    }
    __syncthreads();
    if (wave == 2) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) bufA[g * QA_D + 4 * lane + i] = acc[g][i];
    }
    __syncthreads();
    if (wave != 0) return;
    if (nsplit == 1) {
        // the gate rows requested together, before the first is used
        float4 gv[G];
        if (gate) {
#pragma unroll
            for (int g = 0; g < G; g++)
                gv[g] = *reinterpret_cast<const float4 *>(gate + ((size_t)row * q_heads + (size_t)kvh * G + g) * QA_D + 4 * lane);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const size_t ob = ((size_t)row * q_heads + (size_t)kvh * G + g) * QA_D + 4 * lane;
            const float gg[4] = {gv[g].x, gv[g].y, gv[g].z, gv[g].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float s = acc[g][i] + bufA[g * QA_D + 4 * lane + i];
                float o = l[g] > 0.0f ? s / l[g] : 0.0f;
                if (gate) o *= 1.0f / (1.0f + expf(-gg[i]));
                out[ob + i] = o;
            }
        }
    } else {
        float *pr = part + (size_t)blockIdx.x * G * (QA_D + 2);
#pragma unroll
        for (int g = 0; g < G; g++) {
            if (lane == 0) { pr[g] = m[g]; pr[G + g] = l[g]; }
#pragma unroll
            for (int i = 0; i < 4; i++) pr[2 * G + g * QA_D + 4 * lane + i] = acc[g][i] + bufA[g * QA_D + 4 * lane + i];
        }
    }
}

// The splits of one (row, kv head, head), combined in split order: their
// maxima and sums go to LDS first, then thread t adds dim t of every split's
// output with all its loads in flight at once.
#define QA_MAX_SPLITS 128

template <int G>
__global__ void __launch_bounds__(256) k_attn_merge(float *__restrict__ out, const float *__restrict__ gate,
                                                    const float *__restrict__ part, int q_heads, int kv_heads,
                                                    int nsplit)
{
    __shared__ float sm[QA_MAX_SPLITS], sl[QA_MAX_SPLITS], sf[QA_MAX_SPLITS];
    __shared__ float sL;
    const int g = blockIdx.x % G, rk = blockIdx.x / G, row = rk / kv_heads, kvh = rk % kv_heads, t = threadIdx.x;
    const size_t stride = (size_t)G * (QA_D + 2);
    const float *pr = part + (size_t)rk * nsplit * stride;
    // dim t of every split's output, requested with the maxima and sums (one
    // round trip for the kernel's loads)
    float a[QA_MAX_SPLITS];
#pragma unroll
    for (int s = 0; s < QA_MAX_SPLITS; s++)
        if (s < nsplit) a[s] = pr[s * stride + 2 * G + (size_t)g * QA_D + t];
    if (t < nsplit) {
        sm[t] = pr[t * stride + g];
        sl[t] = pr[t * stride + G + g];
    }
    __syncthreads();
    // the maximum, each split's factor and the weighted sum of the splits'
    // sums, a lane a split (up to 128: two waves), the sum in a fixed tree
    // (each wave's xor tree, then wave 0's plus wave 1's)
    __shared__ float wmax[2], wsum[2];
    if (t < 128) {
        float v = t < nsplit ? sm[t] : -FLT_MAX;
        v = qw_wave_max(v);
        if ((t & 63) == 0) wmax[t >> 6] = v;
    }
    __syncthreads();
    if (t < 128) {
        const float M = fmaxf(wmax[0], wmax[1]);
        float f = 0.0f, c = 0.0f;
        if (t < nsplit) {
            f = qa_exp2(sm[t] - M);
            sf[t] = f;
            c = sl[t] * f;
        }
        c = qw_xor_sum<64>(c);
        if ((t & 63) == 0) wsum[t >> 6] = c;
    }
    __syncthreads();
    if (t == 0) sL = wsum[0] + wsum[1];
    __syncthreads();
    float A = 0.0f;
#pragma unroll
    for (int s = 0; s < QA_MAX_SPLITS; s++)
        if (s < nsplit) A = __builtin_fmaf(a[s], sf[s], A);
    const float L = sL;
    const size_t oi = ((size_t)row * q_heads + (size_t)kvh * G + g) * QA_D + t;
    float o = L > 0.0f ? A / L : 0.0f;
    if (gate) o *= 1.0f / (1.0f + expf(-gate[oi]));
    out[oi] = o;
}

// ---- launchers ----------------------------------------------------------------------

#define QS_MX_MIN_ROWS 16                  // rows from which the scores take the matrix cores

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
    if (rows >= QS_MX_MIN_ROWS && nq <= 16 && D <= 128) {
        const dim3 gm((blocks + QS_BLK - 1) / QS_BLK, (rows + QM_ROWS - 1) / QM_ROWS);
        if (D == 64)
            hipLaunchKernelGGL((k_qsa_scores_mx<64, POOLED>), gm, dim3(QS_THREADS), 0, s, scores, qn, src, kw, inv_freq,
                               rows, nq, d, ratio, base_pos, max_blocks, eps);
        else
            hipLaunchKernelGGL((k_qsa_scores_mx<128, POOLED>), gm, dim3(QS_THREADS), 0, s, scores, qn, src, kw, inv_freq,
                               rows, nq, d, ratio, base_pos, max_blocks, eps);
        return (int)hipGetLastError();
    }
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

// Splits of the position list per (row, kv head): enough workgroups to
// cover the chip when rows * kv_heads alone would not, each split at least
// one pass of QA_P positions.
static int qa_splits(int rows, int kv_heads, int cap)
{
    const int rk = rows * kv_heads, passes = (cap + QA_P - 1) / QA_P;
    if (rk >= 256 || passes <= 1) return 1;
    return max(1, min(min(passes, QA_MAX_SPLITS), (512 + rk - 1) / rk));
}

extern "C" size_t qwk_attn_masked_work_bytes(int rows, int q_heads, int kv_heads, int cap)
{
    if (kv_heads < 1 || rows < 1) return 0;
    const int ns = qa_splits(rows, kv_heads, cap);
    if (ns == 1) return 0;
    return (size_t)rows * kv_heads * ns * (q_heads / kv_heads) * (QA_D + 2) * sizeof(float);
}

template <int G>
static void qa_launch(hipStream_t s, float *out, const float *gate, const float *q, const uint16_t *kc,
                      const uint16_t *vc, const uint32_t *list, int rows, int q_heads, int kv_heads, int max_ctx,
                      float scale, int cap, int ns, float *part)
{
    hipLaunchKernelGGL(k_attn_masked<G>, dim3(rows * kv_heads * ns), dim3(256), 0, s, out, gate, q, kc, vc, list,
                       q_heads, kv_heads, max_ctx, scale, cap, ns, part);
    if (ns > 1)
        hipLaunchKernelGGL(k_attn_merge<G>, dim3(rows * kv_heads * G), dim3(256), 0, s, out, gate, part, q_heads,
                           kv_heads, ns);
}

extern "C" int qwk_attn_masked(hipStream_t s, float *out, const float *gate, const float *q, const uint16_t *kc,
                               const uint16_t *vc, const uint32_t *list, int rows, int q_heads, int kv_heads,
                               int head_dim, int max_ctx, float scale, int cap, void *work, size_t work_bytes)
{
    if (head_dim != QA_D || kv_heads < 1 || q_heads % kv_heads || rows < 0 || cap < 0) return hipErrorInvalidValue;
    if (rows == 0) return 0;
    int ns = qa_splits(rows, kv_heads, cap);
    if (ns > 1 && (!work || work_bytes < qwk_attn_masked_work_bytes(rows, q_heads, kv_heads, cap))) ns = 1;
    float *part = (float *)work;
    switch (q_heads / kv_heads) {
    case 1: qa_launch<1>(s, out, gate, q, kc, vc, list, rows, q_heads, kv_heads, max_ctx, scale, cap, ns, part); break;
    case 2: qa_launch<2>(s, out, gate, q, kc, vc, list, rows, q_heads, kv_heads, max_ctx, scale, cap, ns, part); break;
    case 4: qa_launch<4>(s, out, gate, q, kc, vc, list, rows, q_heads, kv_heads, max_ctx, scale, cap, ns, part); break;
    case 8: qa_launch<8>(s, out, gate, q, kc, vc, list, rows, q_heads, kv_heads, max_ctx, scale, cap, ns, part); break;
    case 12: qa_launch<12>(s, out, gate, q, kc, vc, list, rows, q_heads, kv_heads, max_ctx, scale, cap, ns, part); break;
    case 16: qa_launch<16>(s, out, gate, q, kc, vc, list, rows, q_heads, kv_heads, max_ctx, scale, cap, ns, part); break;
    default: return hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}
