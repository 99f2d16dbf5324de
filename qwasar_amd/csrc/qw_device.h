// qw_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Wave64 throughout: every reduction below is over 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw_kernels.h"

#define QW_WAVE 64

// Timeline stamps inside shared helpers; a kernel file that records a trace
// defines QW_STAMP before including this header.
#ifndef QW_STAMP
#define QW_STAMP(slot) do { } while (0)
#endif

__device__ __forceinline__ float qw_bf16(uint16_t v) {
    return __uint_as_float((uint32_t)v << 16);
}

// e^x, the specified exponential that decides routing: Cody-Waite range
// reduction (k = rint(x log2 e), r = x - k ln2 in two fmaf steps, ln2 split
// as 0.693145751953125 + 1.428606765330187045e-06) and a degree-7 Taylor
// polynomial in Horner form, then one ldexp.  Operations and order are fixed
// so that the host restatement of the same method gives identical bits.
__device__ __forceinline__ float qw_exp_spec(float x) {
    // Branch-free: the polynomial runs on every input and the special cases
    // are selected afterwards (their operands may overflow; they are dropped).
    const float kf = __builtin_rintf(__fmul_rn(x, 1.44269502162933349609375f));
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.428606765330187045e-06f, r);
    float p = 1.98412698412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ki = (int)__builtin_fmaxf(__builtin_fminf(kf, 200.0f), -200.0f);
    float y = __builtin_ldexpf(p, ki);
    y = x < -103.972084045410f ? 0.0f : y;
    y = x > 88.72283935546875f ? __builtin_huge_valf() : y;
    return x != x ? x : y;
}

// Activation numerics: sigmoid(x) = 1 / (1 + e^-x), silu(x) = x * sigmoid(x),
// as the reference's scalar path computes them (qwasar_flash_cpu.c:28-29).
__device__ __forceinline__ float qw_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float qw_silu(float x) { return x * qw_sigmoid(x); }

// ---- cross-lane steps ----------------------------------------------------------
//
// DPP moves run in the VALU at register latency; a shuffle (ds_bpermute)
// round-trips through the LDS unit.  Reductions below use DPP within a row of
// 16 lanes and readlane across the four rows.
//
// A butterfly step with offset 2^s pairs each lane with one in the partner
// half of its 2^(s+1)-lane block.  After the steps below 2^s every lane of a
// 2^s block holds the same value, so any such pairing gives the same bits as
// the xor pairing: quad_perm for offsets 1 and 2, row_half_mirror (i <-> 7-i)
// for 4, row_mirror (i <-> 15-i) for 8.

template <int CTRL>
__device__ __forceinline__ float qw_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int qw_dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
#define QW_DPP_XOR1 0xB1     // quad_perm [1,0,3,2]
#define QW_DPP_XOR2 0x4E     // quad_perm [2,3,0,1]
#define QW_DPP_HMIRROR 0x141 // row_half_mirror
#define QW_DPP_MIRROR 0x140  // row_mirror

__device__ __forceinline__ float qw_lane(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Sum over each aligned run of `width` lanes (a power of two); every lane of
// a run ends with its run's sum.  For width 64 the tree is the xor butterfly
// with ascending offsets 1, 2, 4, 8, 16, 32 -- the order routing is specified
// in -- and every lane gets the same bits.
template <int width>
__device__ __forceinline__ float qw_xor_sum(float v)
{
    if (width >= 2) v = v + qw_dpp<QW_DPP_XOR1>(v);
    if (width >= 4) v = v + qw_dpp<QW_DPP_XOR2>(v);
    if (width >= 8) v = v + qw_dpp<QW_DPP_HMIRROR>(v);
    if (width >= 16) v = v + qw_dpp<QW_DPP_MIRROR>(v);
    if (width == 32) v = v + __shfl_xor(v, 16, 64);
    if (width == 64) {
        const float a = qw_lane(v, 0) + qw_lane(v, 16);
        const float b = qw_lane(v, 32) + qw_lane(v, 48);
        v = a + b;
    }
    return v;
}

__device__ __forceinline__ float qw_wave_max(float v)
{
    v = fmaxf(v, qw_dpp<QW_DPP_XOR1>(v));
    v = fmaxf(v, qw_dpp<QW_DPP_XOR2>(v));
    v = fmaxf(v, qw_dpp<QW_DPP_HMIRROR>(v));
    v = fmaxf(v, qw_dpp<QW_DPP_MIRROR>(v));
    return fmaxf(fmaxf(qw_lane(v, 0), qw_lane(v, 16)), fmaxf(qw_lane(v, 32), qw_lane(v, 48)));
}

// Eight nibbles of one packed word against eight activations.  Returns
// sum_j q_j * x_j; the group's scale and bias are applied by the caller.
__device__ __forceinline__ float qw_dot8_q(uint32_t w, const float *x, float acc) {
    // Keeps the compiler from converting every preloaded word up front (which
    // holds 8 floats per word in registers): the conversions start here.
    asm volatile("" : "+v"(w));
    const uint32_t lo = w & 0x0F0F0F0Fu;          // nibbles 0, 2, 4, 6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // nibbles 1, 3, 5, 7
    // (float)(byte j of v) compiles to one v_cvt_f32_ubyte<j>.
    acc = __builtin_fmaf((float)(lo & 0xFFu), x[0], acc);
    acc = __builtin_fmaf((float)(hi & 0xFFu), x[1], acc);
    acc = __builtin_fmaf((float)((lo >> 8) & 0xFFu), x[2], acc);
    acc = __builtin_fmaf((float)((hi >> 8) & 0xFFu), x[3], acc);
    acc = __builtin_fmaf((float)((lo >> 16) & 0xFFu), x[4], acc);
    acc = __builtin_fmaf((float)((hi >> 16) & 0xFFu), x[5], acc);
    acc = __builtin_fmaf((float)(lo >> 24), x[6], acc);
    acc = __builtin_fmaf((float)(hi >> 24), x[7], acc);
    return acc;
}

// ---- q16: activations staged for the 4-bit dot ----------------------------------
//
// An activation vector is staged in units of 16 elements, 48 bytes each:
//
//   pairs[2]  uint4 per 8-element word: f16 pairs (h0,h4) (h2,h6) (h1,h5) (h3,h7)
//   rec       float4 { X = sum of the unit's values as staged, unscaled,
//                      Y = 1024 * (sum of even positions) + 64 * (sum of odd),
//                      f = 2^-sh, 0 }
//
// where h = f16(x * 2^sh) with sh chosen per unit so that the unit's largest
// magnitude lands in [2^14, 2^15): no f16 overflow, full f16 precision.
//
// A packed word w holds nibbles q0..q7 (q_i at bit 4i).  Inserting the
// nibbles into the f16 pattern 0x6400 (1024.0) gives exact f16 values:
//   bfi(0x000F000F, w)      -> (1024 + q0, 1024 + q4)
//   bfi(0x00F000F0, w)      -> (1024 + 16 q1, 1024 + 16 q5)
//   bfi(0x000F000F, w >> 8) -> (1024 + q2, 1024 + q6)
//   bfi(0x00F000F0, w >> 8) -> (1024 + 16 q3, 1024 + 16 q7)
// so two fp32 dot2 chains give d = sum_even (1024 + q) h and
// d2 = sum_odd (1024 + 16 q) h, and sum_i q_i h_i = d + d2/16 - Y exactly up
// to fp32 rounding.  A unit against one row of a group with scale s, bias b:
//   s * sum q x + b * sum x = (s f) (d + d2/16 - Y) + b X.
#define QW_Q16_BYTES 48

typedef _Float16 qw_h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t qw_bfi(uint32_t mask, uint32_t w, uint32_t base)
{
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(w), "v"(base));
    return r;
}

__device__ __forceinline__ float qw_dot2(uint32_t a, uint32_t b, float c)
{
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(qw_h2, a), __builtin_bit_cast(qw_h2, b), c, false);
}

// One packed word against its four staged pairs: d += even terms, d2 += odd.
__device__ __forceinline__ void qw_word_dot(uint32_t w, uint4 xp, uint32_t magic, float &d, float &d2)
{
    const uint32_t w8 = w >> 8;
    d = qw_dot2(qw_bfi(0x000F000Fu, w, magic), xp.x, d);
    d2 = qw_dot2(qw_bfi(0x00F000F0u, w, magic), xp.z, d2);
    d = qw_dot2(qw_bfi(0x000F000Fu, w8, magic), xp.y, d);
    d2 = qw_dot2(qw_bfi(0x00F000F0u, w8, magic), xp.w, d2);
}

// One staged unit x (p0, p1, r) against 16 nibbles (w0, w1) of a row with
// group scale s and bias b: acc += s * sum q x + b * sum x.
__device__ __forceinline__ float qw_unit_dot(uint2 w, uint4 p0, uint4 p1, float4 r, float s, float b, float acc)
{
    const uint32_t magic = 0x64006400u;
    // Keeps the dequantised halves (8 registers a word) from being built
    // ahead of their use -- across units or out of a token loop: each unit's
    // are rebuilt right before its dot products.
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(w.x), "+v"(w.y));
    float d = 0.0f, d2 = 0.0f;
    qw_word_dot(w.x, p0, magic, d, d2);
    qw_word_dot(w.y, p1, magic, d, d2);
    const float t = __builtin_fmaf(d2, 0.0625f, d) - r.y;
    acc = __builtin_fmaf(b, r.x, acc);
    return __builtin_fmaf(s * r.z, t, acc);
}

__device__ __forceinline__ uint32_t qw_pack_h2(float a, float b)
{
    qw_h2 h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

// Stages 16 values into one unit: the three uint4 of the unit in u[].
__device__ __forceinline__ void qw_q16_make(const float v[16], uint4 u[3])
{
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
    int sh = 0;
    if (m > 0.0f && m <= 3.40282346638528859812e+38f) {
        sh = 15 - __builtin_amdgcn_frexp_expf(m);
        sh = sh < -126 ? -126 : sh > 126 ? 126 : sh;
    }
    float h[16];
#pragma unroll
    for (int i = 0; i < 16; i++) h[i] = (float)(_Float16)__builtin_ldexpf(v[i], sh);
    float xa = 0.0f, xb = 0.0f;
#pragma unroll
    for (int wd = 0; wd < 2; wd++) {
        const float *q = h + 8 * wd;
        u[wd] = make_uint4(qw_pack_h2(q[0], q[4]), qw_pack_h2(q[2], q[6]),
                           qw_pack_h2(q[1], q[5]), qw_pack_h2(q[3], q[7]));
        xa += (q[0] + q[4]) + (q[2] + q[6]);
        xb += (q[1] + q[5]) + (q[3] + q[7]);
    }
    const float f = __builtin_ldexpf(1.0f, -sh);
    const float4 r = make_float4((xa + xb) * f, __builtin_fmaf(1024.0f, xa, 64.0f * xb), f, 0.0f);
    u[2] = *reinterpret_cast<const uint4 *>(&r);
}

// Stages 16 values into one unit at dst (three uint4 stores).
__device__ __forceinline__ void qw_q16_stage(const float v[16], uint4 *dst)
{
    uint4 u[3];
    qw_q16_make(v, u);
    dst[0] = u[0];
    dst[1] = u[1];
    dst[2] = u[2];
}

// ---- routing of one token ----------------------------------------------------------
//
// Softmax over E logits and the K picks of a serial scan with strict '>'
// from e = 0 -- the K largest probabilities, ties to the lower expert, in
// descending (p, then ascending index) order -- by one wave, exactly, as a
// K-round tournament:
//
//   each lane keeps the best of its own experts (lane, lane + 64, ...: the
//   first of equal values, so the lowest index); a round takes the wave's
//   largest value V, and of the lanes holding V the lowest candidate index
//   (one ballot bit in the common case, a min-reduction otherwise); the
//   owning lane retires that expert (p = -1, below every probability) and
//   rescans its slots.
//
// The renormalising sum adds the picks in pick order, as the serial scan
// does.  Every lane ends holding pick `lane` (lane < K) in *pick_i / *pick_w.
__device__ __forceinline__ int qw_wave_min_i(int v)
{
    v = min(v, qw_dpp_i<QW_DPP_XOR1>(v));
    v = min(v, qw_dpp_i<QW_DPP_XOR2>(v));
    v = min(v, qw_dpp_i<QW_DPP_HMIRROR>(v));
    v = min(v, qw_dpp_i<QW_DPP_MIRROR>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Wave maximum of ints (probability bits, which order as the values for
// p >= 0, or negative sentinels below every probability).
// The row maxima (every lane of a row) meet across rows by row_bcast:15
// (rows 1 and 3 take lane 15 of the row before) and row_bcast:31 (rows 2
// and 3 take lane 31): lane 63 ends with the wave's maximum, read once.
__device__ __forceinline__ int qw_wave_max_i(int v)
{
    v = max(v, qw_dpp_i<QW_DPP_XOR1>(v));
    v = max(v, qw_dpp_i<QW_DPP_XOR2>(v));
    v = max(v, qw_dpp_i<QW_DPP_HMIRROR>(v));
    v = max(v, qw_dpp_i<QW_DPP_MIRROR>(v));
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false));   // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xC, 0xF, false));   // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// Device-coherent loads (cache policy sc1: served past this XCD's L2, so
// they see other XCDs' sc1 stores), as buffer loads the compiler batches
// like ordinary ones.  `base` must be wave-uniform; `off` is in bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t qw_rsrc(const void *base)
{
    // the compiler cannot see that `base` is wave-uniform; say so
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    // (readfirstlane returns int: widen through uint32_t, not by sign extension)
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint64_t u = (uint64_t)lo | ((uint64_t)hi << 32);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(u), (short)0, 0x7FFFFFFF, 0x00020000);
}
#define QW_CPOL_SC1 16
__device__ __forceinline__ float qw_ldf_coh(const float *base, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(qw_rsrc(base), off, 0, QW_CPOL_SC1));
}
__device__ __forceinline__ uint4 qw_ld4_coh(const void *base, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qw_rsrc(base), off, 0, QW_CPOL_SC1));
}

// Plain (cached) buffer loads from a wave-uniform base: 32-bit offsets in
// place of 64-bit per-lane addresses.
__device__ __forceinline__ uint2 qw_ld2(const void *base, uint32_t off)
{
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(qw_rsrc(base), off, 0, 0));
}
__device__ __forceinline__ uint4 qw_ld4(const void *base, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qw_rsrc(base), off, 0, 0));
}
__device__ __forceinline__ uint32_t qw_ldu16(const void *base, uint32_t off)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(qw_rsrc(base), off, 0, 0);
}

// Phase hooks inside routing for timing probes; empty unless the includer
// defines them.
#ifndef QW_RSTAMP
#define QW_RSTAMP(slot) do { } while (0)
#endif

// Words of LDS scratch the routing selection takes (8-byte aligned): 66
// survivor keys, then QWK_ROUTE_MAX_K pick keys, 64 bits each.
#define QW_ROUTE_SX 196

// The second half of routing one token in one wave: v[j] = e^(l - max) of
// expert lane + 64 j (0 past E), the softmax p = v / sum, and the top K by
// p, descending, ties to the lower expert.  The sum adds a lane's v[j] in j
// order from 0, then the lane partials by the 64-lane xor tree.
#define QW_ROUTE_PRIO 3
// on_ids(id) is called by the whole wave once the picks' experts are final
// (lane n < K: pick n) and before their weights are computed, so a caller
// can hand the ids on while the renormalisation runs.
struct QwNoIds {
    __device__ __forceinline__ void operator()(int) const {}
};
template <int PL, class OnIds = QwNoIds>
__device__ __forceinline__ void qw_route_finish(float (&v)[PL], int E, int K, int norm, int lane,
                                               int *pick_i, float *pick_w, uint32_t *sx, OnIds on_ids = OnIds{})
{
    // One wave's chain of dependent steps, on a SIMD it shares with the
    // other waves of its CU's workgroups: issued ahead of them while it runs
    if (QW_ROUTE_PRIO > 0) __builtin_amdgcn_s_setprio(QW_ROUTE_PRIO);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < PL; j++) s = s + v[j];
    QW_RSTAMP(2);
    s = qw_xor_sum<64>(s);
    QW_RSTAMP(3);
    // p = v / s, correctly rounded: with y = 1/s correctly rounded and
    // q = v*y, q + (v - s q) y rounds to v/s (Markstein) for results in the
    // normal range; s >= 1 (the largest term is e^0), so only v below 2^-100
    // can leave it and those take the division itself.
    const float y = 1.0f / s;
    int pb[PL];
    bool tiny = false;
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const float q = __fmul_rn(v[j], y);
        const float p = __builtin_fmaf(__builtin_fmaf(-s, q, v[j]), y, q);
        pb[j] = __float_as_int(p);
        tiny |= v[j] != 0.0f && v[j] < 7.888609052210118e-31f;
    }
    if (__ballot(tiny)) {
#pragma unroll
        for (int j = 0; j < PL; j++)
            if (lane + 64 * j < E) pb[j] = __float_as_int(v[j] / s);
    }
    QW_STAMP(7);
    QW_RSTAMP(4);
    // Selection.  The order: bits(p) descending (p >= 0, so the bits order as
    // the values), then e ascending.  tau, at most the K-th largest of the 64
    // lane maxima, bounds the K-th largest p from below (K lanes hold a value
    // >= tau), so every pick has p >= tau.  The survivors (p >= tau; about K
    // for softmax outputs) go to LDS as keys bits(p) << 32 | (0xFFFF - e),
    // larger = earlier; each lane ranks its survivor against all of them, and
    // ranks below K are the picks in order.  With more than 64 survivors
    // (heavy ties) a K-round tournament picks instead; both give the order
    // above exactly.
    {
        int mx = -1;
#pragma unroll
        for (int j = 0; j < PL; j++)
            if (lane + 64 * j < E) mx = max(mx, pb[j]);
        // Two bits a step.  p <= 1 leaves bit 30 clear; the bits below 16 are
        // left at zero, which lowers tau by under 2^-7 relative and only adds
        // survivors.
        uint32_t pref = 0;
#pragma unroll
        for (int b = 28; b >= 16; b -= 2) {
            const uint32_t c1 = pref | (1u << b), c2 = pref | (2u << b), c3 = pref | (3u << b);
            const int n1 = __popcll(__ballot(mx >= (int)c1));
            const int n2 = __popcll(__ballot(mx >= (int)c2));
            const int n3 = __popcll(__ballot(mx >= (int)c3));
            pref = n3 >= K ? c3 : n2 >= K ? c2 : n1 >= K ? c1 : pref;
        }
        const int tau = (int)pref;
        QW_RSTAMP(5);
        // survivors to keys[0 .. C) in slot order, stored by the surviving
        // lanes only (a position past 63 goes to the sink keys[64]; C > 64
        // takes the tournament below).  Every lane storing, the others into
        // the sink, made each slot's store one address for most of the wave.
        uint64_t *keys = reinterpret_cast<uint64_t *>(sx);  // [66]: 64 is a sink
        uint64_t *picks = keys + 66;                         // [QWK_ROUTE_MAX_K]
        const unsigned long long below = (1ull << lane) - 1ull;
        int C = 0;
#pragma unroll
        for (int j = 0; j < PL; j++) {
            const bool on = lane + 64 * j < E && pb[j] >= tau;
            const unsigned long long sm = __ballot(on);
            if (on)
                keys[min(C + (int)__popcll(sm & below), 64)] =
                    ((uint64_t)(uint32_t)pb[j] << 32) | (uint32_t)(0xFFFF - (lane + 64 * j));
            C += __popcll(sm);
        }
        if (C <= 64) {
            __builtin_amdgcn_wave_barrier();
            const uint64_t mk = lane < C ? keys[lane] : 0;
            QW_RSTAMP(6);
            // each lane's rank among the C keys (C is wave-uniform; keys are
            // distinct), the keys read four at a time as LDS broadcasts, all
            // four requested before the first is compared (slots past C
            // hold stale words inside sx and are masked)
            int rank = 0;
            for (int q = 0; q < C; q += 4) {
                uint64_t kq[4];
#pragma unroll
                for (int i = 0; i < 4; i++) kq[i] = keys[q + i];
#pragma unroll
                for (int i = 0; i < 4; i++) rank += (q + i < C) & (kq[i] > mk);
            }
            QW_RSTAMP(7);
            if (lane < C && rank < K) picks[rank] = mk;
            __builtin_amdgcn_wave_barrier();
            const uint64_t pk = lane < K ? picks[lane] : 0;
            *pick_i = lane < K ? 0xFFFF - (int)(uint32_t)pk : 0;
            on_ids(*pick_i);
            // the renormalising sum adds the picks in pick order, read back
            // as LDS broadcasts
            const float mw = __uint_as_float((uint32_t)(pk >> 32));
            float wsum = 0.0f;
            for (int n = 0; n < K; n += 4) {
                float pw[4];
#pragma unroll
                for (int i = 0; i < 4; i++) pw[i] = __uint_as_float((uint32_t)(picks[min(n + i, K - 1)] >> 32));
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (n + i < K) wsum = wsum + pw[i];
            }
            *pick_w = norm ? mw / wsum : mw;
            QW_RSTAMP(8);
            if (QW_ROUTE_PRIO > 0) __builtin_amdgcn_s_setprio(0);
            return;
        }
    }
    // A lane's slots in groups of four, each group sorted once by the key
    // (bits(p) + 2) << 2 | (3 - slot % 4): p < 2 has bits below 2^30, so the
    // key orders by p and then by the lower slot.  A slot past E has key < 4,
    // an emptied one 0, both below every probability (keys >= 8).
    constexpr int NG = PL / 4;
    uint32_t g[NG][4];
#pragma unroll
    for (int k = 0; k < NG; k++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = 4 * k + i;
            const int bits = lane + 64 * j < E ? pb[j] : -2;
            g[k][i] = ((uint32_t)(bits + 2) << 2) | (uint32_t)(3 - i);
        }
        // sort descending: (0,1) (2,3) (0,2) (1,3) (1,2)
#define QW_CE(x, y) { const uint32_t hi = max(g[k][x], g[k][y]), lo = min(g[k][x], g[k][y]); g[k][x] = hi; g[k][y] = lo; }
        QW_CE(0, 1) QW_CE(2, 3) QW_CE(0, 2) QW_CE(1, 3) QW_CE(1, 2)
#undef QW_CE
    }
    float wsum = 0.0f, mine_w = 0.0f;
    int mine_i = 0;
    for (int n = 0; n < K; n++) {
        // the lane's best: the best group head, ties to the lower group
        uint32_t hk = g[0][0];
        int hg = 0;
#pragma unroll
        for (int k = 1; k < NG; k++) {
            const bool gt = (g[k][0] >> 2) > (hk >> 2);
            hk = gt ? g[k][0] : hk;
            hg = gt ? k : hg;
        }
        const int bv = (int)(hk >> 2) - 2;
        const int bj = 4 * hg + 3 - (int)(hk & 3u);
        const int V = qw_wave_max_i(bv);
        const unsigned long long at = __ballot(bv == V);
        int I;
        if ((at & (at - 1)) == 0) {
            const int owner = __builtin_ctzll(at);
            I = owner + 64 * __builtin_amdgcn_readlane(bj, owner);
        } else {
            I = qw_wave_min_i(bv == V ? lane + 64 * bj : 0x7FFFFFFF);
        }
        I = __builtin_amdgcn_readfirstlane(I);
        const float Vf = __int_as_float(V);
        wsum = wsum + Vf;
        mine_i = lane == n ? I : mine_i;
        mine_w = lane == n ? Vf : mine_w;
        // the owner pops its best group's head
        const bool own = lane == (I & 63);
#pragma unroll
        for (int k = 0; k < NG; k++) {
            const bool pop = own && hg == k;
            g[k][0] = pop ? g[k][1] : g[k][0];
            g[k][1] = pop ? g[k][2] : g[k][1];
            g[k][2] = pop ? g[k][3] : g[k][2];
            g[k][3] = pop ? 0u : g[k][3];
        }
    }
    *pick_i = mine_i;
    on_ids(mine_i);
    *pick_w = norm ? mine_w / wsum : mine_w;
    if (QW_ROUTE_PRIO > 0) __builtin_amdgcn_s_setprio(0);
}

// COH: the logits were written by other workgroups of the same launch and are
// read with device-coherent loads (past this XCD's L2).

// Routes one token in one wave: lane l holds experts l + 64 j, j < PL.
// Expert e's logit is l[e * STRIDE].
template <int PL, bool COH = false, int STRIDE = 1>
__device__ __forceinline__ void qw_route_wave(const float *__restrict__ l, int E, int K, int norm,
                                              int lane, int *pick_i, float *pick_w, uint32_t *sx)
{
    float v[PL];
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int ec = min(lane + 64 * j, E - 1) * STRIDE;
        v[j] = COH ? qw_ldf_coh(l, (uint32_t)ec * 4u) : l[ec];
    }
    // every load issued before the first is used (one memory round trip)
#pragma unroll
    for (int j = 0; j < PL; j++) asm volatile("" : "+v"(v[j]));
#pragma unroll
    for (int j = 0; j < PL; j++) {
        v[j] = lane + 64 * j < E ? v[j] : -__builtin_huge_valf();
        m = fmaxf(m, v[j]);
    }
    QW_RSTAMP(0);
    m = qw_wave_max(m);
    QW_STAMP(6);
    QW_RSTAMP(1);
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const float ex = qw_exp_spec(v[j] - m);
        v[j] = lane + 64 * j < E ? ex : 0.0f;
    }
    qw_route_finish<PL>(v, E, K, norm, lane, pick_i, pick_w, sx);
}

// Words of LDS qw_route_block takes besides the selection scratch.
#define QW_ROUTE_BLOCK_LDS (QWK_ROUTE_MAX_E + 16)

// Routes one token with a whole workgroup of at least PL waves (every
// thread calls it; it holds __syncthreads): wave j < PL brings the logit of
// expert 64 j + lane in x (-inf past E; other waves' x is not read), takes the
// exponentials of its slice, and wave 0 sums and selects exactly as
// qw_route_wave does, so the picks and weights are the same bits.  The results
// land in wave 0's lanes (lane n < K: pick n).
template <int PL, class OnIds = QwNoIds>
__device__ __forceinline__ void qw_route_block(float x, int E, int K, int norm, int wave, int lane, int *pick_i,
                                               float *pick_w, uint32_t *sx, float *vb, OnIds on_ids = OnIds{})
{
    float *wm = vb + QWK_ROUTE_MAX_E;
    const int e = lane + 64 * wave;
    const bool on = wave < PL && e < E;
    if (wave < PL) {
        x = on ? x : -__builtin_huge_valf();
        const float mw = qw_wave_max(x);
        if (lane == 0) wm[wave] = mw;
    }
    __syncthreads();
    if (wave < PL) {
        float m = wm[0];
#pragma unroll
        for (int j = 1; j < PL; j++) m = fmaxf(m, wm[j]);
        QW_STAMP(6);
        const float ex = qw_exp_spec(x - m);
        vb[e] = on ? ex : 0.0f;
    }
    __syncthreads();
    if (wave == 0) {
        float v[PL];
#pragma unroll
        for (int j = 0; j < PL; j++) v[j] = vb[lane + 64 * j];
        qw_route_finish<PL>(v, E, K, norm, lane, pick_i, pick_w, sx, on_ids);
    }
}
