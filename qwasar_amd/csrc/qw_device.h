// qw_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Wave64 throughout: every reduction below is over 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Sum over a power-of-two run of `width` lanes with an xor butterfly; every
// lane of the run ends with the same bits (fp32 add commutes).
template <int width>
__device__ __forceinline__ float qw_xor_sum(float v) {
#pragma unroll
    for (int off = width / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, QW_WAVE);
    return v;
}

__device__ __forceinline__ float qw_wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, QW_WAVE));
    return v;
}

// Arg-max over the wave: highest value, ties to the lowest index.  The same
// (value, index) lands in every lane.
__device__ __forceinline__ void qw_wave_argmax(float &v, int &i) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, QW_WAVE);
        const int oi = __shfl_xor(i, off, QW_WAVE);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
}

// Eight nibbles of one packed word against eight activations.  Returns
// sum_j q_j * x_j; the group's scale and bias are applied by the caller.
__device__ __forceinline__ float qw_dot8_q(uint32_t w, const float *x, float acc) {
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
