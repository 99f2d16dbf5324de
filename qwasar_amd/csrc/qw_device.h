// qw_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Wave64 throughout: every reduction below is over 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw_kernels.h"

#define QW_WAVE 64

__device__ __forceinline__ float qw_bf16(uint16_t v) {
    return __uint_as_float((uint32_t)v << 16);
}

// e^x, the specified exponential that decides routing: Cody-Waite range
// reduction (k = rint(x log2 e), r = x - k ln2 in two fmaf steps, ln2 split
// as 0.693145751953125 + 1.428606765330187045e-06) and a degree-7 Taylor
// polynomial in Horner form, then one ldexp.  Operations and order are fixed
// so that the host restatement of the same method gives identical bits.
__device__ __forceinline__ float qw_exp_spec(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_huge_valf();
    if (x < -103.972084045410f) return 0.0f;
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
    return __builtin_ldexpf(p, (int)kf);
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

// Arg-max over the wave: highest value, ties to the lowest index.  The same
// (value, index) lands in every lane.
__device__ __forceinline__ void qw_argmax_step(float &v, int &i, float ov, int oi)
{
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__device__ __forceinline__ void qw_wave_argmax(float &v, int &i)
{
    qw_argmax_step(v, i, qw_dpp<QW_DPP_XOR1>(v), qw_dpp_i<QW_DPP_XOR1>(i));
    qw_argmax_step(v, i, qw_dpp<QW_DPP_XOR2>(v), qw_dpp_i<QW_DPP_XOR2>(i));
    qw_argmax_step(v, i, qw_dpp<QW_DPP_HMIRROR>(v), qw_dpp_i<QW_DPP_HMIRROR>(i));
    qw_argmax_step(v, i, qw_dpp<QW_DPP_MIRROR>(v), qw_dpp_i<QW_DPP_MIRROR>(i));
    float bv = qw_lane(v, 0);
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 1; r < 4; r++) qw_argmax_step(bv, bi, qw_lane(v, 16 * r), __builtin_amdgcn_readlane(i, 16 * r));
    v = bv;
    i = bi;
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

// ---- routing of one token ----------------------------------------------------------
//
// Softmax over E logits and the K picks of a serial scan with strict '>'
// from e = 0 -- the K largest probabilities, ties to the lower expert, in
// descending (p, then ascending index) order -- by one wave, exactly:
//
//   1. key_e = bits(p_e) + 1 for every expert (p >= 0, so the bits order as
//      the values; 0 marks a lane slot past E).
//   2. Radix select: the K-th largest key T, one bit at a time from the top,
//      counting keys >= candidate with ballots (no cross-lane data moves).
//   3. Select every key > T and, of the keys == T, the lowest-indexed
//      K - #(> T).
//   4. The K selected entries are compacted into LDS, and each of K lanes
//      counts the entries ahead of its own: its output position.
//
// Lane l holds experts l, l + 64, ..., so expert order is slot-major.
// `lds` is this wave's scratch of 4 * QWK_ROUTE_MAX_K ints.  Every lane ends
// holding pick `lane` (lane < K) in *pick_i / *pick_w.
template <int PL>
__device__ __forceinline__ void qw_route_wave(const float *__restrict__ l, int E, int K, int norm,
                                              int lane, int *pick_i, float *pick_w, int *lds)
{
    float v[PL];
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? l[e] : -__builtin_huge_valf();
        m = fmaxf(m, v[j]);
    }
    m = qw_wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        if (e < E) { v[j] = qw_exp_spec(v[j] - m); s = s + v[j]; }
    }
    s = qw_xor_sum<64>(s);
    uint32_t key[PL];
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        key[j] = e < E ? __float_as_uint(v[j] / s) + 1u : 0u;
    }
    // 2. the K-th largest key
    uint32_t T = 0;
    for (int b = 30; b >= 0; b--) {
        const uint32_t cand = T | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < PL; j++) cnt += __popcll(__ballot(key[j] >= cand));
        if (cnt >= K) T = cand;
    }
    // 3. the selection
    int gt = 0;
#pragma unroll
    for (int j = 0; j < PL; j++) gt += __popcll(__ballot(key[j] > T));
    const int need = K - gt;
    const unsigned long long below = (1ull << lane) - 1ull;
    int eq_before = 0, sel_before = 0;
    int *ek = lds, *ei = lds + QWK_ROUTE_MAX_K;
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const unsigned long long eq = __ballot(key[j] == T);
        const bool is_eq = key[j] == T;
        const int r = eq_before + __popcll(eq & below);
        const bool sel = key[j] > T || (is_eq && r < need);
        const unsigned long long sm = __ballot(sel);
        if (sel) {
            const int pos = sel_before + __popcll(sm & below);
            ek[pos] = (int)key[j];
            ei[pos] = lane + 64 * j;
        }
        eq_before += __popcll(eq);
        sel_before += __popcll(sm);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    // 4. positions: entries ahead = larger key, or equal key and lower index
    const uint32_t mk = lane < K ? (uint32_t)ek[lane] : 0u;
    const int mi = lane < K ? ei[lane] : 0;
    int rank = 0;
    for (int n = 0; n < K; n++) {
        const uint32_t kn = (uint32_t)__builtin_amdgcn_readlane((int)mk, n);
        const int in = __builtin_amdgcn_readlane(mi, n);
        rank += (kn > mk || (kn == mk && in < mi)) ? 1 : 0;
    }
    int *ok = lds + 2 * QWK_ROUTE_MAX_K, *oi = lds + 3 * QWK_ROUTE_MAX_K;
    __builtin_amdgcn_wave_barrier();
    if (lane < K) { ok[rank] = (int)mk; oi[rank] = mi; }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    const float mine_w = lane < K ? __uint_as_float((uint32_t)ok[lane] - 1u) : 0.0f;
    const int mine_i = lane < K ? oi[lane] : 0;
    float wsum = 0.0f;
    for (int n = 0; n < K; n++) wsum = wsum + qw_lane(mine_w, n);
    *pick_i = mine_i;
    *pick_w = norm ? mine_w / wsum : mine_w;
}
