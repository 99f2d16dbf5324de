// qw_synth.hip -- seeded synthetic tensors generated on the device, for the
// benchmark's and the tests' layer stacks (config 4 holds ~65 GB of weights,
// which a host generator would take minutes to produce and a pinned mirror
// would double).
//
// Every value comes from a counter-based SplitMix64 stream: value i of the
// stream keyed k is mix(k + (i + 1) * 0x9E3779B97F4A7C15), which is exactly
// the i-th output of the sequential SplitMix64 generator seeded with k
// (Steele, Lea and Flood, "Fast splittable pseudorandom number generators",
// OOPSLA 2014; the constants are those of Vigna's public-domain splitmix64.c).
// So any element can be made by any thread, and the host restates the same
// arithmetic to check it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw_kernels.h"

__device__ __forceinline__ uint64_t qs_mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t qs_at(uint64_t key, uint64_t i)
{
    return qs_mix(key + (i + 1ull) * 0x9E3779B97F4A7C15ull);
}

// 53-bit uniform in [0, 1)
__device__ __forceinline__ double qs_u53(uint64_t r) { return (double)(r >> 11) * (1.0 / 9007199254740992.0); }

// fp32 -> bf16 bits, round to nearest even (finite inputs)
__device__ __forceinline__ uint16_t qs_bf16(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float qs_bf16_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Box-Muller on outputs 2i and 2i+1: std * sqrt(-2 ln u1) cos(2 pi u2), with
// u1 in (0, 1] so the logarithm is finite.
__device__ __forceinline__ float qs_normal(uint64_t key, uint64_t i, float std)
{
    const uint64_t r1 = qs_at(key, 2 * i), r2 = qs_at(key, 2 * i + 1);
    const double u1 = ((double)(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = qs_u53(r2);
    return (float)((double)std * sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

__global__ void k_synth(void *dst, int kind, int64_t n, uint64_t key, float a, float b)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        switch (kind) {
        case QWK_SYNTH_U32:
            static_cast<uint32_t *>(dst)[i] = (uint32_t)(qs_at(key, (uint64_t)i) >> 32);
            break;
        case QWK_SYNTH_BF16_UNIFORM:
        case QWK_SYNTH_BF16_NEG8: {
            const uint16_t s = qs_bf16((float)((double)a + ((double)b - (double)a) * qs_u53(qs_at(key, (uint64_t)i))));
            static_cast<uint16_t *>(dst)[i] = kind == QWK_SYNTH_BF16_UNIFORM ? s : qs_bf16(-8.0f * qs_bf16_f32(s));
            break;
        }
        case QWK_SYNTH_BF16_NORMAL:
            static_cast<uint16_t *>(dst)[i] = qs_bf16(qs_normal(key, (uint64_t)i, a));
            break;
        case QWK_SYNTH_F32_BF16_NORMAL:
            static_cast<float *>(dst)[i] = qs_bf16_f32(qs_bf16(qs_normal(key, (uint64_t)i, a)));
            break;
        default:
            break;
        }
    }
}

extern "C" int qwk_synth(hipStream_t s, void *dst, int kind, int64_t n, uint64_t key, float a, float b)
{
    if (!dst || n < 0 || kind < QWK_SYNTH_U32 || kind > QWK_SYNTH_F32_BF16_NORMAL) return (int)hipErrorInvalidValue;
    if (n == 0) return 0;
    const int threads = 256;
    const int64_t want = (n + threads - 1) / threads;
    const int blocks = (int)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(k_synth, dim3(blocks), dim3(threads), 0, s, dst, kind, n, key, a, b);
    return (int)hipGetLastError();
}
