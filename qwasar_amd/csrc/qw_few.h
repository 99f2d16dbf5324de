// qw_few.h -- the router's logits of a few token rows (decode batches):
// the body of k_dmat_few (qw_route.hip), shared with the batch decode's
// router-and-route launch (qw_decode.hip).
#ifndef QW_FEW_H
#define QW_FEW_H
#include "qw_device.h"

// A few token rows (<= 8) against many outputs (decode batches): a wave per
// output, lane c the order-R chain of chunk c for every row.  The token rows
// sit in LDS (chunk c of row r at (r nch + c) * QW_DF_PAD floats: the pad puts
// neighbouring lanes' float4 reads 4 banks apart); the lane's 64 weights are
// requested at once, before any is used.  Lane r then adds row r's chunk
// partials left to right.  Output o == n, when w2 is given, is the dot with
// the single row w2 into g[r] (the shared expert's gate, in the same launch).
#define QW_DF_WAVES 8
#define QW_DF_MAXR 8
#define QW_DF_PAD 68
#define QW_DF_TPG 2      // token rows a workgroup (1 or 3: the same; 4: +2 us a config-2 step)
// The body of one workgroup (bx, by) of k_dmat_few's grid, xl its dynamic
// LDS.  TAGGED: the logits leave as tagged words {epoch, value} in ty (device
// scope, past this XCD's L2) for a reader in the same launch, in place of y.
template <bool TAGGED>
__device__ __forceinline__ void qw_few_body(float *__restrict__ y, float *__restrict__ g, const float *__restrict__ x,
                                            const uint16_t *__restrict__ w, const uint16_t *__restrict__ w2, int k,
                                            int n, int rows, uint4 *__restrict__ qx, uint16_t *__restrict__ hx,
                                            float *__restrict__ hF, uint2 *__restrict__ ty, uint32_t epoch, int bx,
                                            int by, float *xl)
{
    __shared__ float part[QW_DF_WAVES][QW_DF_MAXR][64];
    __shared__ float smax[QW_DF_MAXR][QW_DF_WAVES];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nch = k / 64, o = bx * QW_DF_WAVES + wave;
    // by: a group of QW_DF_TPG token rows (a workgroup stages only its
    // group's rows: a CU's L1 passes a few tens of KB per round trip)
    const int r0 = by * QW_DF_TPG;
    x += (size_t)r0 * k;
    rows = min(QW_DF_TPG, rows - r0);
    const bool has = o < n || (o == n && w2);
    const uint16_t *wr = o < n ? w + (size_t)o * k : w2;
    uint4 wv[8];
    if (has && lane < nch) {
        const uint4 *src = reinterpret_cast<const uint4 *>(wr + 64 * lane);
#pragma unroll
        for (int q = 0; q < 8; q++) wv[q] = src[q];
    }
    // the token rows into LDS, eight float4 a thread in flight at a time
    const int n4 = rows * (k / 4);
    for (int i0 = 0; i0 < n4; i0 += 8 * QW_DF_WAVES * 64) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = min(i0 + j * QW_DF_WAVES * 64 + (int)threadIdx.x, n4 - 1);
            v[j] = reinterpret_cast<const float4 *>(x)[(size_t)(i / (k / 4)) * (k / 4) + i % (k / 4)];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = i0 + j * QW_DF_WAVES * 64 + (int)threadIdx.x;
            if (i < n4) {
                const int r = i / (k / 4), c4 = i % (k / 4);
                *reinterpret_cast<float4 *>(xl + ((size_t)r * nch + c4 / 16) * QW_DF_PAD + (c4 % 16) * 4) = v[j];
            }
        }
    }
    __syncthreads();
    // the logits first: a reader in the same launch waits for them, and the
    // staged rows below are read by the next launch only
    if (has && lane < nch) {
#pragma unroll
        for (int r = 0; r < QW_DF_MAXR; r++) {
            if (r < rows) {
                const float4 *xv = reinterpret_cast<const float4 *>(xl + ((size_t)r * nch + lane) * QW_DF_PAD);
                float p = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const uint4 ww = wv[q];
                    const float4 a = xv[2 * q], b = xv[2 * q + 1];
                    p = __builtin_fmaf(__uint_as_float(ww.x << 16), a.x, p);
                    p = __builtin_fmaf(__uint_as_float(ww.x & 0xFFFF0000u), a.y, p);
                    p = __builtin_fmaf(__uint_as_float(ww.y << 16), a.z, p);
                    p = __builtin_fmaf(__uint_as_float(ww.y & 0xFFFF0000u), a.w, p);
                    p = __builtin_fmaf(__uint_as_float(ww.z << 16), b.x, p);
                    p = __builtin_fmaf(__uint_as_float(ww.z & 0xFFFF0000u), b.y, p);
                    p = __builtin_fmaf(__uint_as_float(ww.w << 16), b.z, p);
                    p = __builtin_fmaf(__uint_as_float(ww.w & 0xFFFF0000u), b.w, p);
                }
                part[wave][r][lane] = p;
            }
        }
    }
    // a wave's LDS accesses run in order: lane r reads what the wave wrote
    if (has && lane < rows) {
        float tot = part[wave][lane][0];
        for (int c = 1; c < nch; c++) tot = tot + part[wave][lane][c];
        if (o < n) {
            if constexpr (TAGGED)
                __hip_atomic_store(reinterpret_cast<unsigned long long *>(ty + (size_t)(r0 + lane) * n + o),
                                   (unsigned long long)epoch | ((unsigned long long)__float_as_uint(tot) << 32),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                y[(size_t)(r0 + lane) * n + o] = tot;
        } else {
            g[r0 + lane] = tot;
        }
    }
    if (qx && bx == 0) {
        // the group's rows also leave as q16 units (16 values, 3 uint4 each),
        // for a launch that reads them after this one
        const int units = k / 16;
        for (int i = threadIdx.x; i < rows * units; i += QW_DF_WAVES * 64) {
            const int r = i / units, u = i % units;
            const float *src = xl + ((size_t)r * nch + (16 * u) / 64) * QW_DF_PAD + (16 * u) % 64;
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = src[j];
            uint4 q[3];
            qw_q16_make(v, q);
            uint4 *d = qx + ((size_t)(r0 + r) * units + u) * 3;
            d[0] = q[0];
            d[1] = q[1];
            d[2] = q[2];
        }
    }
    if (hx && bx == 0) {
        // the group's rows also leave staged as f16 with one power of two a
        // row, as k_stage16 stages them (the same bits): each row's largest
        // magnitude, then h = f16(x 2^sh) in 8-blocks ordered 0,4,1,5,2,6,3,7
        for (int r = 0; r < rows; r++) {
            float m = 0.0f;
            for (int c = threadIdx.x; c < k; c += QW_DF_WAVES * 64)
                m = fmaxf(m, fabsf(xl[((size_t)r * nch + c / 64) * QW_DF_PAD + c % 64]));
            m = qw_wave_max(m);
            if (lane == 0) smax[r][wave] = m;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < rows * (k / 8); i += QW_DF_WAVES * 64) {
            const int r = i / (k / 8), b8 = i % (k / 8);
            float m = smax[r][0];
#pragma unroll
            for (int v = 1; v < QW_DF_WAVES; v++) m = fmaxf(m, smax[r][v]);
            int sh = 0;
            if (m > 0.0f && m <= 3.40282346638528859812e+38f) {
                sh = 15 - __builtin_amdgcn_frexp_expf(m);
                sh = sh < -126 ? -126 : sh > 126 ? 126 : sh;
            }
            if (b8 == 0) hF[r0 + r] = __builtin_ldexpf(1.0f, -sh);
            const float *src = xl + ((size_t)r * nch + (8 * b8) / 64) * QW_DF_PAD + (8 * b8) % 64;
            _Float16 q[8];
#pragma unroll
            for (int j = 0; j < 8; j++) q[j] = (_Float16)__builtin_ldexpf(src[j], sh);
            typedef _Float16 df_h8 __attribute__((ext_vector_type(8)));
            reinterpret_cast<df_h8 *>(hx + (size_t)(r0 + r) * k)[b8] =
                df_h8{q[0], q[4], q[1], q[5], q[2], q[6], q[3], q[7]};
        }
    }
}


#endif
