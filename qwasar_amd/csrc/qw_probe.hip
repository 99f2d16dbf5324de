// Read-bandwidth probe: the HBM read ceiling the decode and prefill kernels
// are measured against.  One launch reads a set of byte ranges (16-byte
// words; each range 16-byte aligned) once, every load independent, and
// writes one word a workgroup (the xor of what it read) so that nothing is
// optimised away.  Used by the measurement driver, not by any layer op.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw_kernels.h"

#define QP_THREADS 256
#define QP_UNROLL 4

typedef unsigned int qp_u4 __attribute__((ext_vector_type(4)));

// One workgroup a piece: piece b is n 16-byte words at p, read by the
// workgroup's threads QP_UNROLL words at a time (all requests of a pass issued
// before any is used).
struct QpPiece {
    const qp_u4 *p;
    uint64_t n;
};

__global__ __launch_bounds__(QP_THREADS) void k_read_probe(const QpPiece *__restrict__ piece,
                                                           uint32_t *__restrict__ sink)
{
    const QpPiece pc = piece[blockIdx.x];
    qp_u4 acc = {0u, 0u, 0u, 0u};
    for (uint64_t w = threadIdx.x; w < pc.n; w += (uint64_t)QP_THREADS * QP_UNROLL) {
        qp_u4 v[QP_UNROLL];
#pragma unroll
        for (int u = 0; u < QP_UNROLL; u++) {
            const uint64_t q = w + (uint64_t)u * QP_THREADS;
            v[u] = q < pc.n ? __builtin_nontemporal_load(pc.p + q) : qp_u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < QP_UNROLL; u++) acc ^= v[u];
    }
    uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    __shared__ uint32_t part[QP_THREADS / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// Reads set (r % nsets) of `nsets` sets of nseg ranges on launch r, for
// `reps` launches, each bracketed by its own events on a stream of its own;
// ms[r] = launch r's duration.  Ranges: ptr[s nseg + i], bytes[s nseg + i]
// (multiples of 16 at 16-byte aligned addresses), cut into pieces of at most
// piece_bytes, one workgroup each.  Returns 0 on success.
extern "C" int qwk_read_probe(const void *const *ptr, const uint64_t *bytes, int nsets, int nseg, int reps,
                              uint64_t piece_bytes, float *ms)
{
    if (nsets < 1 || nseg < 1 || reps < 1 || piece_bytes < 16 || (piece_bytes & 15) || !ptr || !bytes || !ms)
        return -1;
    for (int i = 0; i < nsets * nseg; i++)
        if (((uintptr_t)ptr[i] & 15) || (bytes[i] & 15) || !ptr[i]) return -1;
    // pieces of every set, set after set
    size_t np = 0;
    for (int i = 0; i < nsets * nseg; i++) np += (bytes[i] + piece_bytes - 1) / piece_bytes;
    size_t *first = (size_t *)calloc((size_t)nsets + 1, sizeof(size_t));
    QpPiece *hp = (QpPiece *)calloc(np ? np : 1, sizeof(QpPiece));
    hipEvent_t *ev = (hipEvent_t *)calloc(2 * (size_t)reps, sizeof(hipEvent_t));
    QpPiece *dp_ = NULL;
    uint32_t *sink = NULL;
    size_t maxp = 0;
    int rc = -2;
    hipStream_t st;
    if (hipStreamCreate(&st) != hipSuccess) {
        free(first);
        free(hp);
        free(ev);
        return -2;
    }
    if (!first || !hp || !ev) goto out;
    {
        size_t k = 0;
        for (int s = 0; s < nsets; s++) {
            first[s] = k;
            for (int i = 0; i < nseg; i++) {
                const char *p = (const char *)ptr[s * nseg + i];
                for (uint64_t o = 0; o < bytes[s * nseg + i]; o += piece_bytes) {
                    const uint64_t n = bytes[s * nseg + i] - o < piece_bytes ? bytes[s * nseg + i] - o : piece_bytes;
                    hp[k].p = (const qp_u4 *)(p + o);
                    hp[k].n = n / 16;
                    k++;
                }
            }
            if (k - first[s] > maxp) maxp = k - first[s];
        }
        first[nsets] = k;
    }
    if (maxp == 0 || maxp > 0x7fffffff) goto out;
    if (hipMalloc((void **)&dp_, sizeof(QpPiece) * np) != hipSuccess ||
        hipMalloc((void **)&sink, sizeof(uint32_t) * maxp) != hipSuccess)
        goto out;
    if (hipMemcpy(dp_, hp, sizeof(QpPiece) * np, hipMemcpyHostToDevice) != hipSuccess) goto out;
    for (int r = 0; r < 2 * reps; r++)
        if (hipEventCreate(&ev[r]) != hipSuccess) goto out;
    for (int r = 0; r < reps; r++) {
        const int s = r % nsets;
        (void)hipEventRecord(ev[2 * r], st);
        hipLaunchKernelGGL(k_read_probe, dim3((unsigned)(first[s + 1] - first[s])), dim3(QP_THREADS), 0, st,
                           dp_ + first[s], sink);
        (void)hipEventRecord(ev[2 * r + 1], st);
    }
    if (hipStreamSynchronize(st) != hipSuccess) goto out;
    for (int r = 0; r < reps; r++) (void)hipEventElapsedTime(&ms[r], ev[2 * r], ev[2 * r + 1]);
    rc = 0;
out:
    if (ev)
        for (int r = 0; r < 2 * reps; r++)
            if (ev[r]) (void)hipEventDestroy(ev[r]);
    (void)hipStreamSynchronize(st);
    (void)hipFree(dp_);
    (void)hipFree(sink);
    (void)hipStreamDestroy(st);
    free(ev);
    free(hp);
    free(first);
    return rc;
}
