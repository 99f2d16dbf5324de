// qw_decode.hip -- the MoE block at decode (1..8 tokens) in ONE launch.
//
// The launch's workgroups take four roles, in block-index order:
//
//   router   one wave per router row (E rows, plus the shared expert's gate
//            vector): the order-R logits of every token
//   experts  per (selected expert, 16-row block): route every token, then
//            the gate / up rows of that expert for every token routed to it
//            -- each weight byte read once; SwiGLU fused; the activations
//            leave staged as q16 units
//   shared   the shared expert's gate / up rows and SwiGLU (needs only x)
//   down     per (token, block of output rows): route, load the down rows of
//            the shared expert and of each of the token's K experts into
//            registers; each matrix's wave waits for that matrix's
//            activations and computes; then the combine:
//            sigmoid(g) * shared + sum_k w_k * y_k, an fma chain in slot order
//
// For one token the router's logits need no flag: each is stored together
// with the launch's epoch in one 64-bit word, and the routing workgroups poll
// the words themselves.  Other hand-offs go through device memory past the
// per-XCD L2: the
// producer writes with device-coherent (sc1) stores, waits for them, and
// bumps a counter; the last arriver of a counter resets it to zero and
// publishes the launch's epoch in the counter's flag.  A consumer polls the
// flag with device-coherent loads and reads the data the same way.  So the
// down rows' weight fetch overlaps the gate / up fetch, and no launch
// boundary sits between router, routing, experts and down.
//
// Progress: a workgroup only waits on workgroups with smaller block indices,
// which the dispatcher has already placed (workgroups are dispatched in index
// order), so every wait ends.
//
// Placement: two workgroups share a CU, and of two that fetch weights at
// once the later-dispatched one waits a memory round trip longer (measured:
// the last 64 experts workgroups reached their first dot ~1.7 us after the
// rest).  The shared expert (done long before the down rows need it) sits
// after the experts, so the latest-dispatched fetchers are the ones with
// slack.  Each wait is also bounded: past a spin limit
// it raises the error word, every later wait gives up at once, and the host
// reports the error; no wave is left spinning.
//
// The 4-bit products use the q16 dot (qw_unit_dot): staged activations are
// loaded straight into registers next to the weights.
#include <hip/hip_ext.h>

#ifdef QD_TRACE
extern __device__ unsigned long long qd_trace[8192 * 16];
#define QW_STAMP(slot) do { if (threadIdx.x == 0) qd_trace[blockIdx.x * 16 + (slot)] = wall_clock64(); } while (0)
#define QW_RSTAMP(slot) do { if (threadIdx.x == 0) qd_trace[blockIdx.x * 16 + 7 + (slot)] = wall_clock64(); } while (0)
#endif
#include "qw_device.h"
#include "qw_kernels.h"

// Built with -DQD_TRACE, every workgroup stamps the device wall clock
// (100 MHz) at its phases into qd_trace[block][slot], for timelines.
#ifdef QD_TRACE
__device__ unsigned long long qd_trace[8192 * 16];
#define QD_TS(slot) do { if (threadIdx.x == 0) qd_trace[blockIdx.x * 16 + (slot)] = wall_clock64(); } while (0)
extern "C" int qd_trace_read(unsigned long long *dst)
{
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(qd_trace), sizeof(qd_trace));
}
// and where it ran: HW_ID (CU, SH, SE in bits 8..15) and XCC_ID << 24
__device__ unsigned int qd_hwid[8192];
#define QD_HWID() do { if (threadIdx.x == 0) qd_hwid[blockIdx.x] = \
    (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4) | ((unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 24); } while (0)
extern "C" int qd_hwid_read(unsigned int *dst)
{
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(qd_hwid), sizeof(qd_hwid));
}
#else
#define QD_TS(slot) do { } while (0)
#define QD_HWID() do { } while (0)
#endif

#define QD_MAXT QWK_DECODE_MAX_ROWS
#define QD_MAXU (QWK_DECODE_MAX_ROWS * QWK_DECODE_MAX_K)
#define QD_WAVES 16                 // every role: 16 waves
#define QD_THREADS (QD_WAVES * 64)
#define QD_GU_MAXRPB (QD_WAVES * 4)
#define QD_LDS (64 * 1024)          // dynamic LDS: staged inputs, or the router's rows and partials
#ifndef QD_DOWN_RATE
#define QD_DOWN_RATE 35000.0        // bytes a 100 MHz tick the experts' stream moves (see down_delay)
#endif
#define QD_DOWN_LPR 16
#define QD_DOWN_RIT 4               // down rows per lane slot
#define QD_DOWN_RPG ((64 / QD_DOWN_LPR) * QD_DOWN_RIT)
#define QD_SPIN_LIMIT (1 << 16)
// The sleep between polls (s_sleep units of 64 clocks): a longer one lets
// the polled memory settle (A/B on config 1: 0 -> 23.70, 1 -> 23.45,
// 4 -> 23.35, 8 -> 23.09–23.18, 16 -> 23.14–23.20 µs a token).
#ifndef QD_SLEEP
#define QD_SLEEP 8
#endif
#define QD_POLL_SLEEP() do { if (QD_SLEEP > 0) __builtin_amdgcn_s_sleep(QD_SLEEP); } while (0)     // polls (each a memory round trip plus a sleep)

static_assert(QWK_DECODE_MAX_K + 1 <= QD_WAVES, "down: one wave per matrix");
// down: the K + 1 activation vectors (at most 64 units each), one LDS region a wave
static_assert((QWK_DECODE_MAX_K + 1) * 64 * QW_Q16_BYTES <= QD_LDS, "down activations fit the dynamic LDS");


// Lanes per row for a row of `units` q16 units, and units per lane.
static __host__ __device__ constexpr int qd_lpr(int units) { return units >= 128 ? 64 : units >= 64 ? 32 : 16; }
static int qd_nul(int units, int lpr)
{
    const int n = (units + lpr - 1) / lpr;
    return n <= 4 ? n : -1;
}

// ---- hand-off state (zeroed once by the host) -------------------------------------
//
// Every hand-off between workgroups is a tagged word: a 64-bit store of
// {the launch's epoch, a 32-bit payload}, so a reader that sees this
// launch's epoch sees the payload with it, and the producer needs no store
// acknowledgement, counter or flag.  Words hold past epochs between launches;
// an epoch is never reused before the state is zeroed.
//
//   lgt    the router's logits (and the shared expert's gate logit at E)
//   rdone  router workgroup b's logits are all stored (its word b, payload
//          unused), in QD_RDREP copies: a reader polls the copy of its XCD
//          (blockIdx % 8), one wave, and then reads the logits once, rather
//          than every wave of every workgroup polling the same 4 KB
//   tact   the activation vectors the down rows read, as q16 units of 12
//          dwords: vector 0 the shared expert's, 1 + k the k-th pick's

#define QD_TU 32                  // q16 units a tagged activation vector holds (I, SI <= 512)
#define QD_RDREP 8                // copies of the router's done words
#define QD_RDSTRIDE 320           // words between copies (>= the router workgroups, (E + 4) / 4)

struct QdSync {
    uint32_t err;
    uint32_t pad[3];
    uint2 lgt[QWK_ROUTE_MAX_E + 1];
    uint2 rdone[QD_RDREP * QD_RDSTRIDE];
    uint2 tact[(QWK_DECODE_MAX_K + 1) * QD_TU * 12];
};

__device__ __forceinline__ void qd_stf(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// One q16 uint4 written device-coherently, as two 64-bit halves.
__device__ __forceinline__ void qd_st4(uint4 *p, uint4 v)
{
    unsigned long long *q = reinterpret_cast<unsigned long long *>(p);
    __hip_atomic_store(q, (unsigned long long)v.x | ((unsigned long long)v.y << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (unsigned long long)v.z | ((unsigned long long)v.w << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// A flag read for polling: volatile, so it is issued on every pass; the
// caller waits for a batch of them at once.
__device__ __forceinline__ uint32_t qd_poll_ld(const uint32_t *p)
{
    uint32_t v;
    asm volatile("global_load_dword %0, %1, off sc1" : "=v"(v) : "v"(p));
    return v;
}

// A wait gave up: the error word takes the launch's epoch unless an earlier
// failure already set it, so the host learns the first failing launch (and
// every later launch, whose waits see the word and give up at once, failed
// with it).  The word is never 0 once raised: epochs start at 1.
__device__ __forceinline__ void qd_raise(QdSync *S, uint32_t epoch)
{
    uint32_t expect = 0u;
    __hip_atomic_compare_exchange_strong(&S->err, &expect, epoch, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}

struct QdLayout {
    size_t qx, qsh, qact, total;
};

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

static QdLayout qd_layout(const qwk_moe *M, int rows)
{
    QdLayout L;
    size_t o = 0;
    L.qx = o;     o += al((size_t)rows * (M->H / 16) * QW_Q16_BYTES);
    L.qsh = o;    o += al((size_t)rows * (M->SI / 16) * QW_Q16_BYTES);
    L.qact = o;   o += al((size_t)rows * M->K * (M->I / 16) * QW_Q16_BYTES);
    L.total = o;
    return L;
}

struct QdArgs {
    qwk_moe m;
    const float *x;
    // with hin set, the input is x = rms_norm(bf16(hin + yprev)) instead
    const uint16_t *hin;
    const float *yprev;             // may be null: x = rms_norm(hin)
    uint16_t *hout;                 // bf16(hin + yprev), written by workgroup 0
    float *xout;                    // that x, written by workgroup 0
    float eps;
    const uint16_t *pf_router, *pf_gate_w;   // the next layer's router rows, to read ahead (may be null)
    float *out;
    int32_t *idx;
    float *w;
    int rows, umax, lgG;
    int n_rt, n_sh, gu_wg_per_u, ngu, n_ex, n_down_rb;
    int tch;                        // input vectors per LDS pass
    char *scr;                      // the scratch base (device-coherent loads are offsets from it)
    uint4 *qx, *qsh, *qact;         // q16 units: [vector][units][3]
    QdSync *sync;
    uint32_t epoch;
    uint32_t down_delay;            // wall-clock ticks (100 MHz) the down loads wait after routing
};

// One wave: each lane with `has` waits until its tagged word {epoch, value}
// at p holds this launch's epoch, bounded like qd_wait_flags (on giving up
// the error word is raised and the value is whatever was read).  Each pass
// reads the words and the error word in one batch.
__device__ __forceinline__ uint2 qd_poll_tag(const QdArgs &a, const uint2 *p, bool has)
{
    for (int spins = 0;; spins++) {
        unsigned long long v;
        asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
        uint32_t e = qd_poll_ld(&a.sync->err);
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(v), "+v"(e)::"memory");
        const uint2 r = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
        if (__ballot(has && r.x != a.epoch) == 0ull) return r;
        if (spins >= QD_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
            if ((threadIdx.x & 63) == 0) qd_raise(a.sync, a.epoch);
            return r;
        }
        QD_POLL_SLEEP();
    }
}

// Wave 0: waits until every router workgroup's done word (the copy of this
// workgroup's XCD) holds this launch's epoch, bounded like qd_poll_tag.
__device__ __forceinline__ void qd_wait_rdone(const QdArgs &a)
{
    const int lane = threadIdx.x & 63, n = a.n_rt;
    const uint2 *d = a.sync->rdone + (blockIdx.x & (QD_RDREP - 1)) * QD_RDSTRIDE;
    static_assert(QD_RDSTRIDE <= 5 * 64, "five words a lane");
    for (int spins = 0;; spins++) {
        unsigned long long q0, q1, q2, q3, q4;
        asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q0) : "v"(d + min(lane, n - 1)) : "memory");
        asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q1) : "v"(d + min(lane + 64, n - 1)) : "memory");
        asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q2) : "v"(d + min(lane + 128, n - 1)) : "memory");
        asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q3) : "v"(d + min(lane + 192, n - 1)) : "memory");
        asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q4) : "v"(d + min(lane + 256, n - 1)) : "memory");
        uint32_t e = qd_poll_ld(&a.sync->err);
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(q0), "+v"(q1), "+v"(q2), "+v"(q3), "+v"(q4), "+v"(e)::"memory");
        const uint32_t ep = a.epoch;
        const bool stale = (uint32_t)q0 != ep || (uint32_t)q1 != ep || (uint32_t)q2 != ep || (uint32_t)q3 != ep ||
                           (uint32_t)q4 != ep;
        if (__ballot(stale) == 0ull) return;
        if (spins >= QD_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
            if (lane == 0) qd_raise(a.sync, a.epoch);
            return;
        }
        QD_POLL_SLEEP();
    }
}

// ---- the residual step as the launch's prologue ----------------------------------
//
// With RES (a.hin set), the launch's input rows are x = rms_norm(bf16(hin + yprev))
// (the step between stacked layers).  Every workgroup that reads x builds the
// rows it stages from hin and yprev, with the arithmetic and the summation
// order of k_resid_rms_bf16 (qw_norm.hip: each of 256 threads an fmaf chain
// over its float4 chunks, the xor tree, the four wave partials in order), so
// x has the bits that kernel gives; workgroup 0 also writes hout and xout.

__device__ __forceinline__ float qd_bf16r(float f)
{
    const uint32_t u = __float_as_uint(f);
    return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

// bf16(hin + yprev) of row t, columns 4 i4 .. 4 i4 + 3
__device__ __forceinline__ float4 qd_v4(const QdArgs &a, int t, int i4)
{
    const uint2 hb = reinterpret_cast<const uint2 *>(a.hin + (size_t)t * a.m.H)[i4];
    float4 v = make_float4(__uint_as_float(hb.x << 16), __uint_as_float(hb.x & 0xFFFF0000u),
                           __uint_as_float(hb.y << 16), __uint_as_float(hb.y & 0xFFFF0000u));
    if (a.yprev) {
        const float4 y = reinterpret_cast<const float4 *>(a.yprev + (size_t)t * a.m.H)[i4];
        v = make_float4(qd_bf16r(v.x + y.x), qd_bf16r(v.y + y.y), qd_bf16r(v.z + y.z), qd_bf16r(v.w + y.w));
    }
    return v;
}

// x of row t, columns 4 i4 .. 4 i4 + 3, with the prologue (RES) or from a.x
template <bool RES>
__device__ __forceinline__ float4 qd_x4(const QdArgs &a, const float *qinv, int t, int i4)
{
    if constexpr (!RES) return reinterpret_cast<const float4 *>(a.x + (size_t)t * a.m.H)[i4];
    const float4 v = qd_v4(a, t, i4);
    const float r = qinv[t];
    return make_float4(v.x * r, v.y * r, v.z * r, v.w * r);
}

// qinv[t] = 1 / sqrt(mean(v^2) + eps) for every row; the whole workgroup
// (1024 threads: four rows at a time, 256 threads a row), ends in a barrier.
__device__ __forceinline__ void qd_norm_rows(const QdArgs &a, float *qinv, float *qpart)
{
    const int g = threadIdx.x >> 8, tid = threadIdx.x & 255, wave = threadIdx.x >> 6;
    const int n4 = a.m.H / 4;
    for (int t0 = 0; t0 < a.rows; t0 += 4) {
        const int t = t0 + g;
        float ss = 0.0f;
        if (t < a.rows)
            for (int i = tid; i < n4; i += 256) {
                const float4 v = qd_v4(a, t, i);
                ss = __builtin_fmaf(v.x, v.x, ss);
                ss = __builtin_fmaf(v.y, v.y, ss);
                ss = __builtin_fmaf(v.z, v.z, ss);
                ss = __builtin_fmaf(v.w, v.w, ss);
            }
        ss = qw_xor_sum<64>(ss);
        if ((threadIdx.x & 63) == 0) qpart[wave] = ss;
        __syncthreads();
        if (threadIdx.x < 4 && t0 + (int)threadIdx.x < a.rows) {
            const float *p = qpart + 4 * threadIdx.x;
            float sum = p[0];
            sum = sum + p[1];
            sum = sum + p[2];
            sum = sum + p[3];
            qinv[t0 + threadIdx.x] = 1.0f / sqrtf(sum / (float)a.m.H + a.eps);
        }
        __syncthreads();
    }
}

// workgroup 0: hout = bf16(hin + yprev), xout = x
__device__ __forceinline__ void qd_write_resid(const QdArgs &a, const float *qinv)
{
    const int n4 = a.m.H / 4;
    for (int j = threadIdx.x; j < a.rows * n4; j += blockDim.x) {
        const int t = j / n4, i = j % n4;
        const float4 v = qd_v4(a, t, i);
        const float r = qinv[t];
        reinterpret_cast<uint2 *>(a.hout)[j] =
            make_uint2((__float_as_uint(v.x) >> 16) | (__float_as_uint(v.y) & 0xFFFF0000u),
                       (__float_as_uint(v.z) >> 16) | (__float_as_uint(v.w) & 0xFFFF0000u));
        reinterpret_cast<float4 *>(a.xout)[j] = make_float4(v.x * r, v.y * r, v.z * r, v.w * r);
    }
}

// ---- router ---------------------------------------------------------------------
//
// QD_RT_ROWS router rows per workgroup, one wave each; the token rows pass
// through LDS one at a time, chunk c of 64 inputs at c * QD_XPAD floats (the
// pad makes the per-lane chunk reads conflict-free).

#ifndef QD_RT_ROWS
#define QD_RT_ROWS 4
#endif
#define QD_XPAD 68
#define QD_WPAD 36                  // dwords a router-row chunk takes in LDS (32 + pad)
// a padded token row (k <= 4096), every wave's partials, and the rows
static_assert((64 * QD_XPAD + QD_WAVES * 64 + QD_RT_ROWS * 64 * QD_WPAD) * 4 <= QD_LDS,
              "router: a padded token row, partials and the rows fit the dynamic LDS");

// Order-R dot of one bf16 row with one token row xl (LDS, padded chunks):
// lane l computes the fmaf chain of chunk l (k <= 64 * 64); the chunk
// partials go to LDS and lane 0 adds them left to right, from -0 (so the
// first addition is exact).
__device__ __forceinline__ void qd_router_row(const uint4 (&w)[8], const float *xl, int nch, uint2 *y,
                                              uint32_t epoch, float *part)
{
    const int lane = threadIdx.x & 63;
    if (lane < nch) {
        const float4 *xv = reinterpret_cast<const float4 *>(xl + lane * QD_XPAD);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            uint4 wq = w[q];
            // converted here, not all 64 values up front
            asm volatile("" : "+v"(wq.x), "+v"(wq.y), "+v"(wq.z), "+v"(wq.w));
            const float4 a = xv[2 * q], b = xv[2 * q + 1];
            s = __builtin_fmaf(__uint_as_float(wq.x << 16), a.x, s);
            s = __builtin_fmaf(__uint_as_float(wq.x & 0xFFFF0000u), a.y, s);
            s = __builtin_fmaf(__uint_as_float(wq.y << 16), a.z, s);
            s = __builtin_fmaf(__uint_as_float(wq.y & 0xFFFF0000u), a.w, s);
            s = __builtin_fmaf(__uint_as_float(wq.z << 16), b.x, s);
            s = __builtin_fmaf(__uint_as_float(wq.z & 0xFFFF0000u), b.y, s);
            s = __builtin_fmaf(__uint_as_float(wq.w << 16), b.z, s);
            s = __builtin_fmaf(__uint_as_float(wq.w & 0xFFFF0000u), b.w, s);
        }
        part[lane] = s;
    }
    // A wave's LDS accesses run in order: lane 0 reads what the wave wrote.
    if (lane == 0) {
        float total = -0.0f;
        int c = 0;
        for (; c + 4 <= nch; c += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(part + c);
            total = total + v.x;
            total = total + v.y;
            total = total + v.z;
            total = total + v.w;
        }
        for (; c < nch; c++) total = total + part[c];
        // the logit and the launch's epoch in one 64-bit store: a reader that
        // sees this epoch sees this logit
        __hip_atomic_store(reinterpret_cast<unsigned long long *>(y),
                           (unsigned long long)epoch | ((unsigned long long)__float_as_uint(total) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <bool RES>
__device__ __forceinline__ void qd_role_router(const QdArgs &a, int b, float *lds, float *qinv, float *qpart)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = a.m.H, E = a.m.E, nch = H / 64;
    const int o = b * QD_RT_ROWS + wave;
    float *xl = lds, *pbase = lds + nch * QD_XPAD, *part = pbase + wave * 64;
    if constexpr (RES) qd_norm_rows(a, qinv, qpart);
    QD_TS(1);
    // this wave's row in registers, lane c holding chunk c (64 inputs, 8
    // uint4).  Loaded contiguously (each load instruction covers 8 whole
    // cache lines, where lane-per-chunk loads would touch 64 lines for 16
    // bytes each), then passed through the wave's own LDS region, chunk c at
    // c * QD_WPAD dwords (conflict-free reads); a wave's LDS accesses run in
    // order, so no barrier.
    const bool row = wave < QD_RT_ROWS && o <= E;
    const uint16_t *wr = o < E ? a.m.router + (size_t)o * H : a.m.sh_gate_w;
    uint4 w[8];
    if (wave < QD_RT_ROWS) {
        uint32_t *wl = reinterpret_cast<uint32_t *>(pbase + QD_WAVES * 64) + wave * 64 * QD_WPAD;
        const int npc = H / 8;                      // uint4 pieces of the row
        uint4 v[8];
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int i = min(lane + 64 * r, npc - 1);
            v[r] = row ? reinterpret_cast<const uint4 *>(wr)[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int i = lane + 64 * r;
            if (i < npc) *reinterpret_cast<uint4 *>(wl + (i / 8) * QD_WPAD + (i % 8) * 4) = v[r];
        }
        const int c = min(lane, nch - 1);
#pragma unroll
        for (int q = 0; q < 8; q++) w[q] = *reinterpret_cast<const uint4 *>(wl + c * QD_WPAD + 4 * q);
#ifdef QD_TRACE
        if (threadIdx.x == 0)
            qd_trace[blockIdx.x * 16 + 3] = (w[7].w ^ w[0].x) == 0x12345678u ? 0 : wall_clock64();
#endif
    }
    for (int t = 0; t < a.rows; t++) {
        if (t) __syncthreads();
        for (int i = threadIdx.x; i < H / 4; i += blockDim.x) {
            const float4 v = qd_x4<RES>(a, qinv, t, i);
            *reinterpret_cast<float4 *>(xl + (i / 16) * QD_XPAD + (i % 16) * 4) = v;
        }
        __syncthreads();
        if (t == 0) QD_TS(4);
        if (row) qd_router_row(w, xl, nch, a.sync->lgt + (size_t)t * (E + 1) + o, a.epoch, part);
    }
    // the logit stores are acknowledged (past this XCD's L2) before the
    // done words say so
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x < QD_RDREP)
        __hip_atomic_store(reinterpret_cast<unsigned long long *>(a.sync->rdone + threadIdx.x * QD_RDSTRIDE + b),
                           (unsigned long long)a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    QD_TS(2);
    if constexpr (RES) {
        if (b == 0) qd_write_resid(a, qinv);
        // In a stack, the next layer's router workgroup b (same block, same
        // XCD) reads these same rows: read them now, while this layer's
        // experts stream, so that the next launch's router finds them in the
        // caches instead of HBM.
        if (a.pf_router && row) {
            const uint16_t *pr = o < E ? a.pf_router + (size_t)o * H : a.pf_gate_w;
            uint4 t[8];
#pragma unroll
            for (int r = 0; r < 8; r++) t[r] = reinterpret_cast<const uint4 *>(pr)[min(lane + 64 * r, H / 8 - 1)];
#pragma unroll
            for (int r = 0; r < 8; r++) asm volatile("" ::"v"(t[r].x));
        }
    }
}

// ---- gate / up rows with SwiGLU ----------------------------------------------------
//
// A workgroup owns RPB = QD_WAVES * 64/LPR consecutive rows of one gate / up
// pair (the shared expert's, or one routed expert's) for nt input vectors.
// Lane (slot, lr) of wave w takes row row0 + w * 64/LPR + slot and its units
// lr, lr + LPR, ... (NUL of them), in both matrices; its weights stay in
// registers while the input vectors pass through LDS, up to `tch` at a time.
// The per-row results meet in LDS and leave as q16 units of the activation
// vectors, written device-coherently.  Unless `staged` (the inputs already
// in LDS), the inputs are copied from the router role's staged rows.

// Stages token rows x[vin[t]] (t < n; token t when vin is NULL) into LDS as
// q16 units, with threads tid0.. of the workgroup.
template <bool RES>
__device__ __forceinline__ void qd_stage_x(uint4 *xs, const QdArgs &a, const float *qinv, const int *vin, int n,
                                           int tid0, int nthr)
{
    const int units = a.m.H / 16;
    for (int i = threadIdx.x - tid0; i < n * units; i += nthr) {
        const int t = i / units, u = i % units;
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = qd_x4<RES>(a, qinv, vin ? vin[t] : t, 4 * u + q);
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
        qw_q16_stage(v, xs + (size_t)i * 3);
    }
}

// TAGGED (the one-launch path): each output unit leaves as 12 tagged words
// {epoch, dword} in a.sync->tact, vector vout[t] (written without any wait);
// else as q16 units at dst (the batch path, read after the launch ends).
template <int LPR, int NUL, bool PLAINX = false, bool TAGGED = false>
__device__ __forceinline__ void qd_glu_block(const qwk_q4 gm, const qwk_q4 um, int n, const QdArgs &a,
                                             int row0, int nt, bool staged, uint4 *xs, const int *vin,
                                             const int *vout, uint4 *dst, float (*ys)[QD_GU_MAXRPB])
{
    constexpr int SL = 64 / LPR, RPB = QD_WAVES * SL;
    static_assert(RPB % 16 == 0 && RPB <= QD_GU_MAXRPB, "rows per block");
    const int k = a.m.H, lgG = a.lgG;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, slot = lane / LPR, lr = lane % LPR;
    const int units = k / 16, words = k / 8, groups = k >> lgG;
    const int rl = wave * SL + slot, row = row0 + rl;
    // Every load is issued (at a clamped, valid address) before any is used;
    // out-of-range lanes are zeroed afterwards.
    //
    // With a whole wave on a row (LPR 64), lane lr takes the unit pairs
    // (2 lr, 2 lr + 1) and (128 + 2 lr, 128 + 2 lr + 1): two 16-byte loads a
    // matrix, each instruction of the wave reading whole lines, and a scale
    // and a bias a pair (a pair is 32 inputs, inside one group); else lane lr
    // takes units lr, lr + LPR, ... (NUL of them).
    constexpr bool CG = LPR == 64;
    constexpr int NW = CG ? 4 : NUL;               // units a lane
    uint2 wv[2][NW];
    uint32_t sb[2][CG ? 2 : NUL];                  // bf16 scale (low half) and bias (high half)
    const int rowc = min(row, n - 1);
    if constexpr (CG) {
        // lane lr: unit pairs (2 lr, 2 lr + 1) and (128 + 2 lr, 128 + 2 lr + 1),
        // so each 16-byte load instruction of the wave reads whole lines
        uint4 w4[2][2];
        uint32_t sv[2][2], bv[2][2];
        bool okp[2];
#pragma unroll
        for (int h = 0; h < 2; h++) okp[h] = row < n && 128 * h + 2 * lr + 1 < units;
#pragma unroll
        for (int z = 0; z < 2; z++) {
            const qwk_q4 q = z ? um : gm;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int c0 = min(128 * h + 2 * lr, units - 2);
                w4[z][h] = *reinterpret_cast<const uint4 *>(q.w + (size_t)rowc * words + 2 * c0);
                const size_t gi = (size_t)rowc * groups + ((16 * c0) >> lgG);
                sv[z][h] = q.s[gi];
                bv[z][h] = q.b[gi];
            }
        }
#pragma unroll
        for (int z = 0; z < 2; z++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                wv[z][2 * h] = okp[h] ? make_uint2(w4[z][h].x, w4[z][h].y) : make_uint2(0, 0);
                wv[z][2 * h + 1] = okp[h] ? make_uint2(w4[z][h].z, w4[z][h].w) : make_uint2(0, 0);
                sb[z][h] = okp[h] ? sv[z][h] | (bv[z][h] << 16) : 0u;
            }
    } else {
        uint32_t sv[2][NUL], bv[2][NUL];
#pragma unroll
        for (int z = 0; z < 2; z++) {
            const qwk_q4 q = z ? um : gm;
#pragma unroll
            for (int j = 0; j < NUL; j++) {
                const int c = min(j * LPR + lr, units - 1);
                wv[z][j] = *reinterpret_cast<const uint2 *>(q.w + (size_t)rowc * words + 2 * c);
                const size_t gi = (size_t)rowc * groups + ((16 * c) >> lgG);
                sv[z][j] = q.s[gi];
                bv[z][j] = q.b[gi];
            }
        }
#pragma unroll
        for (int z = 0; z < 2; z++)
#pragma unroll
            for (int j = 0; j < NUL; j++) {
                const bool ok = row < n && j * LPR + lr < units;
                wv[z][j] = ok ? wv[z][j] : make_uint2(0, 0);
                sb[z][j] = ok ? sv[z][j] | (bv[z][j] << 16) : 0u;
            }
    }
    for (int t0 = 0; t0 < nt; t0 += a.tch) {
        const int tn = min(a.tch, nt - t0);
        if (!staged) {
            __syncthreads();
            const int per = units * 3;
            for (int i0 = 0; i0 < tn * per; i0 += 4 * QD_THREADS) {
                uint4 v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = min(i0 + (int)threadIdx.x + r * QD_THREADS, tn * per - 1);
                    const uint32_t off = (uint32_t)((vin[t0 + i / per] * per + i % per) * 16);
                    // PLAINX: the rows were staged by an earlier launch, so cached loads see them
                    v[r] = PLAINX ? a.qx[off / 16] : qw_ld4_coh(a.qx, off);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) asm volatile("" : "+v"(v[r].x), "+v"(v[r].y), "+v"(v[r].z), "+v"(v[r].w));
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (i0 + (int)threadIdx.x + r * QD_THREADS < tn * per) xs[i0 + threadIdx.x + r * QD_THREADS] = v[r];
            }
        }
        __syncthreads();
#pragma unroll 1
        for (int t = 0; t < tn; t++) {
            const uint4 *xt = xs + (size_t)t * units * 3;
            float acc[2] = {0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NW; j++) {
                const int c = CG ? min(128 * (j / 2) + 2 * lr + (j % 2), units - 1) : j * LPR + lr;
                if (CG || c < units) {
                    const uint4 p0 = xt[3 * c], p1 = xt[3 * c + 1];
                    const uint4 rr = xt[3 * c + 2];
                    const float4 r = *reinterpret_cast<const float4 *>(&rr);
                    const int si = CG ? j / 2 : j;
#pragma unroll
                    for (int z = 0; z < 2; z++)
                        acc[z] = qw_unit_dot(wv[z][j], p0, p1, r, __uint_as_float(sb[z][si] << 16),
                                             __uint_as_float(sb[z][si] & 0xFFFF0000u), acc[z]);
                }
            }
#ifdef QD_TRACE
            if (t0 + t == 0 && threadIdx.x == 0)
                qd_trace[blockIdx.x * 16 + 3] = __builtin_amdgcn_readfirstlane(__float_as_int(acc[0] + acc[1])) == 12345 ? 0 : wall_clock64();
#endif
            const float g = qw_xor_sum<LPR>(acc[0]);
            const float u = qw_xor_sum<LPR>(acc[1]);
            if (lr == 0) ys[t0 + t][rl] = qw_silu(g) * u;
        }
    }
    __syncthreads();
    // one thread per (vector, unit) of this block's rows
    constexpr int upb = RPB / 16;
    const int outunits = n / 16;
    for (int i = threadIdx.x; i < nt * upb; i += blockDim.x) {
        const int t = i / upb, uu = i % upb;
        if (row0 + 16 * uu >= n) continue;
        float v[16];
#pragma unroll
        for (int q = 0; q < 16; q++) v[q] = ys[t][16 * uu + q];
        uint4 s[3];
        qw_q16_make(v, s);
        if (TAGGED) {
            unsigned long long *d = reinterpret_cast<unsigned long long *>(
                a.sync->tact + ((size_t)vout[t] * QD_TU + row0 / 16 + uu) * 12);
            const uint32_t w[12] = {s[0].x, s[0].y, s[0].z, s[0].w, s[1].x, s[1].y, s[1].z, s[1].w,
                                    s[2].x, s[2].y, s[2].z, s[2].w};
#pragma unroll
            for (int j = 0; j < 12; j++)
                __hip_atomic_store(d + j, (unsigned long long)a.epoch | ((unsigned long long)w[j] << 32),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            uint4 *d = dst + ((size_t)vout[t] * outunits + row0 / 16 + uu) * 3;
            qd_st4(d, s[0]);
            qd_st4(d + 1, s[1]);
            qd_st4(d + 2, s[2]);
        }
    }
}

// ---- routing inside a workgroup -----------------------------------------------------

struct QdRoute {
    int U;
    int picks[QD_MAXU];
    float pw[QD_MAXU];
    int uexp[QD_MAXU];
    int ucnt[QD_MAXU];
    int ustart[QD_MAXU];
    int upair[QD_MAXU];       // pairs grouped by unique expert, ascending pair index
    int mark[QWK_ROUTE_MAX_E];// after routing: the unique-expert slot of each selected expert
    union alignas(16) {
        uint32_t sx[QD_MAXT][QW_ROUTE_SX];  // selection scratch of routing wave w (w < rows <= QD_MAXT)
        struct {                            // one token, routed by the whole workgroup
            uint32_t sx[QW_ROUTE_SX];
            float vb[QW_ROUTE_BLOCK_LDS];
        } one;
    } rs;
};

// Routes every token (a wave per token) with the arithmetic of the
// standalone route kernel, then builds the union of selected experts
// (ascending) with, for each, its pairs in ascending order, and mark[e] = the
// union slot of expert e.  One token's picks are distinct, so for one token
// the union is the picks themselves, in pick order.
template <int PL>
__device__ void qd_route_all(const QdArgs &a, QdRoute &R)
{
    const int t = threadIdx.x, nthr = blockDim.x, wave = t >> 6, lane = t & 63, nw = nthr >> 6;
    const int E = a.m.E, K = a.m.K;
    if (a.rows == 1 && nw >= PL) {
        // wave 0 waits for every router workgroup's done word, then each
        // wave reads its slice of the logits (their tags checked too)
        if (wave == 0) qd_wait_rdone(a);
        __syncthreads();
        float x = 0.0f;
        if (wave < PL) {
            const int e = lane + 64 * wave;
            x = __uint_as_float(qd_poll_tag(a, a.sync->lgt + min(e, E - 1), e < E).y);
        }
        int pi;
        float pw;
        qw_route_block<PL>(x, E, K, a.m.norm, wave, lane, &pi, &pw, R.rs.one.sx, R.rs.one.vb);
#ifdef QD_TRACE
        if (blockIdx.x >= a.n_rt && blockIdx.x < a.n_rt + a.n_ex) QD_TS(5);
#endif
        // clamped: after a given-up wait the logits are whatever was read,
        // and no pick may then address outside the banks
        if (wave == 0 && lane < K) {
            R.picks[lane] = min(max(pi, 0), E - 1);
            R.pw[lane] = pw;
        }
    } else {
        for (int r = wave; r < a.rows; r += nw) {
            int pi;
            float pw;
            // after the router's flag: the fp32 halves of row r's tagged words
            qw_route_wave<PL, true, 2>(reinterpret_cast<const float *>(a.sync->lgt + (size_t)r * (E + 1)) + 1, E, K,
                                       a.m.norm, lane, &pi, &pw, R.rs.sx[wave]);
            if (lane < K) {
                R.picks[r * K + lane] = min(max(pi, 0), E - 1);
                R.pw[r * K + lane] = pw;
            }
        }
    }
    __syncthreads();
    if (a.rows == 1) {
        if (t < K) {
            R.uexp[t] = R.picks[t];
            R.ucnt[t] = 1;
            R.ustart[t] = t;
            R.upair[t] = t;
            R.mark[R.picks[t]] = t;
        }
        if (t == 0) R.U = K;
        __syncthreads();
        return;
    }
    for (int e = t; e < E; e += nthr) R.mark[e] = 0;
    __syncthreads();
    const int npk = a.rows * K;
    for (int p = t; p < npk; p += nthr) R.mark[R.picks[p]] = 1;
    __syncthreads();
    // Compact the marked experts in ascending order, 64 at a time with ballots.
    if (wave == 0) {
        int base = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const bool on = e < E && R.mark[e];
            const unsigned long long bal = __ballot(on);
            if (on) R.uexp[base + __popcll(bal & ((1ull << lane) - 1ull))] = e;
            base += __popcll(bal);
        }
        if (lane == 0) R.U = base;
    }
    __syncthreads();
    for (int u = t; u < R.U; u += nthr) {
        const int e = R.uexp[u];
        int c = 0;
        for (int p = 0; p < npk; p++) c += R.picks[p] == e;
        R.ucnt[u] = c;
        R.mark[e] = u;
    }
    __syncthreads();
    if (t == 0) {
        int s = 0;
        for (int u = 0; u < R.U; u++) { R.ustart[u] = s; s += R.ucnt[u]; }
    }
    __syncthreads();
    for (int u = t; u < R.U; u += nthr) {
        const int e = R.uexp[u];
        int c = R.ustart[u];
        for (int p = 0; p < npk; p++)
            if (R.picks[p] == e) R.upair[c++] = p;
    }
    __syncthreads();
}

template <int LPR, int NUL, int PL, bool RES>
__device__ __forceinline__ void qd_role_experts(const QdArgs &a, int bb, uint4 *xs, QdRoute &R, int *vin,
                                                int *vout, float (*ys)[QD_GU_MAXRPB], float *qinv, float *qpart)
{
    constexpr int RPB = QD_WAVES * (64 / LPR);
    const int H = a.m.H, I = a.m.I, K = a.m.K;
    const int u = bb / a.gu_wg_per_u, rb = bb % a.gu_wg_per_u;
    // the token is staged into LDS while the router runs
    if constexpr (RES) qd_norm_rows(a, qinv, qpart);
    qd_stage_x<RES>(xs, a, qinv, nullptr, 1, 0, blockDim.x);
    QD_TS(1);
    qd_route_all<PL>(a, R);
    QD_TS(2);
    if (bb == 0 && threadIdx.x < K) {
        a.idx[threadIdx.x] = R.picks[threadIdx.x];
        a.w[threadIdx.x] = R.pw[threadIdx.x];
    }
    // one token: slot u is pick u; its activation vector is tagged vector 1 + u
    const int e = R.picks[u];
    if (threadIdx.x == 0) {
        vin[0] = 0;
        vout[0] = 1 + u;
    }
    __syncthreads();
    // Split banks: gate and up [E, I, H]; fused: gate_up [E, 2I, H], gate rows
    // first, so up row r of expert e is row I + r of its slice.
    const size_t words = H / 8, groups = H >> a.lgG;
    qwk_q4 gm, um;
    if (a.m.split) {
        const size_t off = (size_t)e * I;
        gm = {a.m.gate.w + off * words, a.m.gate.s + off * groups, a.m.gate.b + off * groups};
        um = {a.m.up.w + off * words, a.m.up.s + off * groups, a.m.up.b + off * groups};
    } else {
        const size_t off = (size_t)e * 2 * I;
        gm = {a.m.gate_up.w + off * words, a.m.gate_up.s + off * groups, a.m.gate_up.b + off * groups};
        um = {gm.w + (size_t)I * words, gm.s + (size_t)I * groups, gm.b + (size_t)I * groups};
    }
    qd_glu_block<LPR, NUL, false, true>(gm, um, I, a, rb * RPB, 1, true, xs, vin, vout, nullptr, ys);
    QD_TS(4);
}

// One wave: waits until tagged activation vector v (units q16 units) holds
// this launch's epoch in every word, then writes its dwords into the wave's
// LDS region xw in q16 layout (a wave's LDS accesses run in order: no
// barrier).  Every pass reads the whole vector (six words a lane): polling
// one word a unit first and reading the vector after costs a second round
// trip behind the last unit (measured: 0.56 µs a token more).  Bounded like
// qd_poll_tag; returns false (the error word raised) if a wait gave up.
__device__ __forceinline__ bool qd_wait_tact(const QdArgs &a, int v, int units, uint4 *xw)
{
    const int lane = threadIdx.x & 63;
    const uint2 *tv = a.sync->tact + (size_t)v * QD_TU * 12;
    const int nw = units * 12;
    uint32_t *x32 = reinterpret_cast<uint32_t *>(xw);
    static_assert(QD_TU * 12 <= 6 * 64, "six words a lane");
    for (int spins = 0;; spins++) {
        unsigned long long q[6];
#pragma unroll
        for (int j = 0; j < 6; j++)
            asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(q[j]) : "v"(tv + min(lane + 64 * j, nw - 1)) : "memory");
        uint32_t e = qd_poll_ld(&a.sync->err);
        // every loaded register is tied to the wait, so no use moves above it
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]), "+v"(e)::"memory");
        bool stale = false;
#pragma unroll
        for (int j = 0; j < 6; j++) stale |= lane + 64 * j < nw && (uint32_t)q[j] != a.epoch;
        if (__ballot(stale) == 0ull) {
#pragma unroll
            for (int j = 0; j < 6; j++)
                if (lane + 64 * j < nw) x32[lane + 64 * j] = (uint32_t)(q[j] >> 32);
            return true;
        }
        if (spins >= QD_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
            if (lane == 0) qd_raise(a.sync, a.epoch);
            return false;
        }
        QD_POLL_SLEEP();
    }
}

// ---- down: the shared expert and every expert of a token, and the combine -------
//
// A workgroup owns QD_DOWN_RPG output rows of one token; wave m holds those
// rows of matrix m (0 = the shared expert, 1 + k = the token's k-th expert)
// in registers from the moment routing is known, then waits for its own
// matrix's activation vector, loads it into registers and computes.  The
// per-matrix rows meet in LDS and the combine runs in slot order.
template <int NUL, int PL>
__device__ __forceinline__ void qd_role_down(const QdArgs &a, int bd, QdRoute &R, uint4 *xa,
                                             float (*ys)[QD_DOWN_RPG])
{
    constexpr int LPR = QD_DOWN_LPR, RPP = 64 / LPR, RIT = QD_DOWN_RIT, RPG = QD_DOWN_RPG;
    const int H = a.m.H, I = a.m.I, SI = a.m.SI, K = a.m.K;
    const int rb = bd;
    const int lane = threadIdx.x & 63, m = threadIdx.x >> 6;
    const int slot = lane / LPR, lr = lane % LPR;
    const int row0 = rb * RPG;
    const int lgG = a.lgG;
    QD_TS(1);
    qd_route_all<PL>(a, R);
    QD_TS(2);
    const bool busy = m <= K;
    const int kin = m == 0 ? SI : I;
    const int units = kin / 16, words = kin / 8, groups = kin >> lgG;
    const uint32_t *wm = a.m.sh_down.w;
    const uint16_t *sm = a.m.sh_down.s, *bm = a.m.sh_down.b;
    if (busy && m > 0) {
        const size_t e = (size_t)R.picks[m - 1];
        wm = a.m.down.w + e * H * words;
        sm = a.m.down.s + e * H * groups;
        bm = a.m.down.b + e * H * groups;
    }
    // The down rows are not needed before the experts' activations, and
    // each CU's L1 passes misses at a bounded rate: requested at once they
    // would slow the routed experts' gate/up stream on the CUs both share.
    // So they wait, after routing, about the time that stream takes.
    {
        const unsigned long long t0 = wall_clock64();
        while (wall_clock64() - t0 < a.down_delay) __builtin_amdgcn_s_sleep(2);
    }
    // Every load is issued (at a clamped, valid address) before any is used.
    // The scales and biases of the workgroup's RPG rows are contiguous
    // (RPG * groups bf16 each, at most 256: kin <= 512, groups of >= 32):
    // lanes 0-31 load the scales, 32-63 the biases, 16 bytes a lane, and
    // pass them through LDS, so they take one register quad, not a register
    // per (unit, row).
    uint2 wv[NUL][RIT];
#pragma unroll
    for (int j = 0; j < NUL; j++) {
        const int c = min(j * LPR + lr, units - 1);
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const int row = min(row0 + slot + RPP * i, H - 1);
            wv[j][i] = qw_ld2(wm, (uint32_t)(row * words + 2 * c) * 4u);
        }
    }
    const int nsb = RPG * groups, li = lane & 31;
    const uint32_t sboff = (uint32_t)(row0 * groups + 8 * li) * 2u;
    uint4 sbr = make_uint4(0, 0, 0, 0);
    if (busy && 8 * li < nsb) sbr = lane < 32 ? qw_ld4(sm, sboff) : qw_ld4(bm, sboff);
    // the shared expert's gate logit (its round trip overlaps the loads)
    const float gate = qw_sigmoid(__uint_as_float(
        qd_poll_tag(a, a.sync->lgt + a.m.E, (threadIdx.x & 63) == 0).y));
    // Wave m waits for its own matrix's activation vector (0: the shared
    // expert's, 1 + k: the k-th pick's), so the matrices start as their
    // experts finish and only the last one's wait and dot trail the last
    // expert.
    if (busy) {
        uint4 *xw = xa + (m == 0 ? 0 : (SI / 16) * 3 + (m - 1) * ((I / 16) * 3));
        uint16_t *sl = reinterpret_cast<uint16_t *>(xa + (SI / 16) * 3 + K * ((I / 16) * 3) + m * 64);
        if (8 * li < nsb) *reinterpret_cast<uint4 *>(sl + (lane < 32 ? 0 : 256) + 8 * li) = sbr;
        if (qd_wait_tact(a, m, units, xw)) {
            QD_TS(4);
            float y[RIT];
#pragma unroll
            for (int i = 0; i < RIT; i++) y[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < NUL; j++) {
                const int c = j * LPR + lr;
                if (c < units) {
                    const int g = (16 * c) >> lgG;
                    const uint4 p0 = xw[3 * c], p1 = xw[3 * c + 1], rr = xw[3 * c + 2];
                    const float4 r = *reinterpret_cast<const float4 *>(&rr);
#pragma unroll
                    for (int i = 0; i < RIT; i++) {
                        const int q = (slot + RPP * i) * groups + g;
                        y[i] = qw_unit_dot(wv[j][i], p0, p1, r, __uint_as_float((uint32_t)sl[q] << 16),
                                           __uint_as_float((uint32_t)sl[256 + q] << 16), y[i]);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < RIT; i++) {
                const float v = qw_xor_sum<LPR>(y[i]);
                if (lr == 0) ys[m][slot + RPP * i] = v;
            }
        }
    }
    QD_TS(6);
    __syncthreads();
    QD_TS(7);
    // The combine: the shared term first, then an fma per slot, in order.
    for (int r = threadIdx.x; r < RPG; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= H) continue;
        float acc = ys[0][r] * gate;
        for (int k = 0; k < K; k++) acc = __builtin_fmaf(R.pw[k], ys[1 + k][r], acc);
        a.out[row] = acc;
    }
    QD_TS(5);
}

// ---- the kernel --------------------------------------------------------------------

// 8 waves per SIMD: two 16-wave workgroups per CU, which takes at most 64
// VGPRs and 78 SGPRs a wave (at 80 SGPRs a CU holds one).
template <int LPR, int NUL, int NULD, int PL, bool RES>
__global__ __launch_bounds__(QD_THREADS, 8) void k_decode_fused(QdArgs a)
{
    extern __shared__ uint4 xs[];     // [tch][units][3], or the router's partials
    __shared__ QdRoute R;
    __shared__ int vin[QD_MAXT], vout[QD_MAXT];
    __shared__ float ys[QD_MAXT][QD_GU_MAXRPB];
    __shared__ float qinv[QD_MAXT], qpart[QD_WAVES];   // the residual prologue's row scales
    static_assert(QD_MAXT * QD_GU_MAXRPB >= (QWK_DECODE_MAX_K + 1) * QD_DOWN_RPG, "down shares ys");
    constexpr int RPB = QD_WAVES * (64 / LPR);
    QD_TS(0);
    QD_HWID();
    int b = blockIdx.x;
    if (b < a.n_rt) {
        qd_role_router<RES>(a, b, reinterpret_cast<float *>(xs), qinv, qpart);
        return;
    }
    b -= a.n_rt;
    if (b < a.n_ex) {
        qd_role_experts<LPR, NUL, PL, RES>(a, b, xs, R, vin, vout, ys, qinv, qpart);
        return;
    }
    b -= a.n_ex;
    if (b < a.n_sh) {
        // the shared expert's activation is tagged vector 0
        if (threadIdx.x == 0) vin[0] = vout[0] = 0;
        if constexpr (RES) qd_norm_rows(a, qinv, qpart);
        qd_stage_x<RES>(xs, a, qinv, nullptr, 1, 0, blockDim.x);
        __syncthreads();
        qd_glu_block<LPR, NUL, false, true>(a.m.sh_gate, a.m.sh_up, a.m.SI, a, b * RPB, 1, true, xs, vin, vout,
                                            nullptr, ys);
        QD_TS(4);
        return;
    }
    b -= a.n_sh;
    qd_role_down<NULD, PL>(a, b, R, xs, reinterpret_cast<float (*)[QD_DOWN_RPG]>(&ys[0][0]));
}

// ---- host side -------------------------------------------------------------------

extern "C" size_t qwk_moe_decode_scratch(const qwk_moe *M, int rows)
{
    return qd_layout(M, rows).total;
}

extern "C" size_t qwk_moe_decode_sync_bytes(void) { return sizeof(QdSync); }

extern "C" int qwk_decode_sync_words(void *sync, uint32_t **err, void **words, size_t *nwords)
{
    QdSync *S = static_cast<QdSync *>(sync);
    *err = &S->err;
    *words = S->tact;
    *nwords = sizeof(S->tact) / sizeof(S->tact[0]);
    return 0;
}

extern "C" int qwk_moe_decode_sync_error(const void *sync, uint32_t *err)
{
    return (int)hipMemcpy(err, &static_cast<const QdSync *>(sync)->err, sizeof *err, hipMemcpyDeviceToHost);
}

extern "C" int qwk_moe_decode_sync_raise(void *sync, uint32_t epoch)
{
    return (int)hipMemcpy(&static_cast<QdSync *>(sync)->err, &epoch, sizeof epoch, hipMemcpyHostToDevice);
}

template <int LPR, int NUL, int NULD, int PL, bool RES>
static void qd_launch(hipStream_t s, const QdArgs &a, int grid, hipEvent_t e0, hipEvent_t e1)
{
    auto kern = k_decode_fused<LPR, NUL, NULD, PL, RES>;
    if (e0) hipExtLaunchKernelGGL(kern, dim3(grid), dim3(QD_THREADS), QD_LDS, s, e0, e1, 0, a);
    else hipLaunchKernelGGL(kern, dim3(grid), dim3(QD_THREADS), QD_LDS, s, a);
}

// The instantiated shapes: (LPR, NUL) of the gate / up rows (k = H), NULD of
// the down rows (k = max(I, SI), 16 lanes a row), PL logits per lane (E).
#define QD_SHAPES(X)                                                                   \
    X(16, 1, 1, 4) X(16, 1, 2, 4) X(16, 2, 1, 4) X(16, 2, 2, 4)                         \
    X(32, 2, 2, 8) X(64, 2, 2, 8) X(64, 3, 2, 8) X(64, 4, 2, 8)

static bool qd_shapes(const qwk_moe *M, int *lpr_h, int *nul_h, int *nul_d, int *pl)
{
    const int uh = M->H / 16, ud = (M->I > M->SI ? M->I : M->SI) / 16;
    *lpr_h = qd_lpr(uh);
    *nul_h = qd_nul(uh, *lpr_h);
    *nul_d = qd_nul(ud, QD_DOWN_LPR);
    *pl = M->E <= 256 ? 4 : M->E <= 512 ? 8 : 16;
#define QD_HAS(L, N, D, P) if (*lpr_h == L && *nul_h == N && *nul_d == D && *pl == P) return true;
    QD_SHAPES(QD_HAS)
#undef QD_HAS
    return false;
}

extern "C" int qwk_moe_decode_supported(const qwk_moe *M, int rows)
{
    int a, b, c, d;
    const int G = M->group;
    return rows >= 1 && rows <= QWK_DECODE_MAX_ROWS && M->K >= 1 && M->K <= QWK_DECODE_MAX_K &&
           M->E >= M->K && M->E <= QWK_ROUTE_MAX_E && M->H % 64 == 0 && M->I % 16 == 0 &&
           M->SI % 16 == 0 && M->H <= 4096 && (G == 32 || G == 64 || G == 128) &&
           M->H % G == 0 && M->I % G == 0 && M->SI % G == 0 && qd_shapes(M, &a, &b, &c, &d);
}

extern "C" int qwk_moe_decode(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                              const qwk_resid *res, const qwk_moe *M, int rows, void *scratch,
                              size_t scratch_bytes, void *sync, uint32_t epoch, hipEvent_t *ev)
{
    const int G = M->group;
    // the fused launch serves one token; 2..8 take qwk_moe_decode_batch
    if (rows != 1 || !qwk_moe_decode_supported(M, rows) || !sync || epoch == 0u) return (int)hipErrorInvalidValue;
    if (res ? (!res->h || !res->h_out || !res->x_out || ((uintptr_t)res->h & 7u) || ((uintptr_t)res->h_out & 7u) ||
               ((uintptr_t)res->y & 15u) || ((uintptr_t)res->x_out & 15u) ||
               (const void *)res->h_out == (const void *)res->h || (const void *)res->h_out == (const void *)res->y)
            : (!x || ((uintptr_t)x & 15u)))
        return (int)hipErrorInvalidValue;
    const QdLayout L = qd_layout(M, rows);
    if (scratch_bytes < L.total) return (int)hipErrorInvalidValue;
    int lpr_h, nul_h, nul_d, pl;
    qd_shapes(M, &lpr_h, &nul_h, &nul_d, &pl);

    char *S = (char *)scratch;
    QdArgs a;
    a.m = *M;
    a.x = x; a.out = out; a.idx = idx; a.w = w; a.rows = rows;
    a.hin = res ? res->h : nullptr;
    a.yprev = res ? res->y : nullptr;
    a.hout = res ? res->h_out : nullptr;
    a.xout = res ? res->x_out : nullptr;
    a.pf_router = res ? res->next_router : nullptr;
    a.pf_gate_w = res ? res->next_gate_w : nullptr;
    a.eps = res ? res->eps : 0.0f;
    a.umax = rows * M->K < M->E ? rows * M->K : M->E;
    a.lgG = G == 32 ? 5 : G == 64 ? 6 : 7;
    const int rpb = QD_WAVES * (64 / lpr_h);
    const int vbytes = (M->H / 16) * QW_Q16_BYTES;
    a.tch = QD_LDS / vbytes < rows ? QD_LDS / vbytes : rows;
    a.n_rt = (M->E + 1 + QD_RT_ROWS - 1) / QD_RT_ROWS;
    a.n_sh = (M->SI + rpb - 1) / rpb;
    a.gu_wg_per_u = (M->I + rpb - 1) / rpb;
    a.n_ex = a.umax * a.gu_wg_per_u;
    a.n_down_rb = (M->H + QD_DOWN_RPG - 1) / QD_DOWN_RPG;
    a.scr = S;
    a.qx = (uint4 *)(S + L.qx);
    a.qsh = (uint4 *)(S + L.qsh);
    a.qact = (uint4 *)(S + L.qact);
    a.sync = (QdSync *)sync;
    a.epoch = epoch;
    {
        // the routed experts' gate/up bytes at the rate the chip's L1s pass
        // them (~3.5 TB/s, 35,000 bytes a tick): at config 1 (17.7 MB) ~5 us,
        // measured best at 4.5-6 (3: 22.3 us a token, 10: 26.1, none: 23.6)
        const double gu = (double)M->K * 2.0 * M->I * ((double)M->H / 2.0 + 4.0 * (M->H >> a.lgG));
        a.down_delay = (uint32_t)(gu / QD_DOWN_RATE);
    }
    // one token: K + 1 activation vectors of at most QD_TU q16 units each
    if (a.tch < 1 || a.umax > QD_MAXU || M->I / 16 > QD_TU || M->SI / 16 > QD_TU || a.n_rt > QD_RDSTRIDE)
        return (int)hipErrorInvalidValue;
    const int grid = a.n_rt + a.n_sh + a.n_ex + rows * a.n_down_rb;

    hipEvent_t e0 = ev ? ev[0] : 0, e1 = ev ? ev[1] : 0;
#define QD_GO(L_, N_, D_, P_) \
    if (lpr_h == L_ && nul_h == N_ && nul_d == D_ && pl == P_) {                                      \
        if (res) qd_launch<L_, N_, D_, P_, true>(s, a, grid, e0, e1);                                   \
        else qd_launch<L_, N_, D_, P_, false>(s, a, grid, e0, e1);                                      \
    } else
    QD_SHAPES(QD_GO)
#undef QD_GO
    return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

// ---- decode of 2..8 tokens: four launches over the batch's unique experts --------
//
// With several tokens the one-launch path above routes every token in every
// experts and down workgroup and needs more workgroups than fit at once;
// measured at 8 tokens (config 2) it spent ~16 us routing in each of ~4000
// workgroups.  Here each step is its own launch, so nothing waits on another
// workgroup and the grid size is free:
//
//   router     order-R logits of every token
//   (k_dmat_few in qw_route.hip, with the shared expert's gate logits in
//              the same launch)
//   k_batch_route   one workgroup: every token routed (a wave each, the
//              standalone route's arithmetic), the table of unique experts
//              (ascending, each with its pairs in ascending order), and the
//              token rows staged as q16 units
//   k_batch_gu      per (unique expert, 16-row block), and the shared
//              expert's blocks: the weight rows read once for every token
//              routed there (requested before the staged rows are copied into
//              LDS); SwiGLU fused; the activations leave as q16 units
//   k_batch_down    per (token, 16 output rows): the down rows of the shared
//              expert and the token's K experts, each applied to its
//              activation vector, then the combine in slot order (the
//              fused path's).  A row block's workgroups for all tokens sit on
//              one XCD (block index = rb mod 8 there), so an expert several
//              tokens share is read from that XCD's L2 after the first.

#define QB_TAB_U 0
#define QB_TAB_UEXP 1
#define QB_TAB_UCNT (1 + QD_MAXU)
#define QB_TAB_USTART (1 + 2 * QD_MAXU)
#define QB_TAB_UPAIR (1 + 3 * QD_MAXU)
#define QB_TAB_GATE (1 + 4 * QD_MAXU)
#define QB_TAB_INTS (1 + 4 * QD_MAXU + QD_MAXT)

struct QbLayout {
    size_t logits, tab, qx, qact, qsh, xh, xF, perm, tiles, act, total;
};

// The batch's gate / up runs on the matrix cores (qwk_gmm16, the shared
// expert as one more expert of the grouped product) when the shared expert's
// width is the routed experts' and the product takes the shapes and banks;
// else as q16 dots (k_batch_gu).
static qwk_q4 qb_up_bank(const qwk_moe *M)
{
    if (M->split) return M->up;
    const qwk_q4 g = M->gate_up;
    return qwk_q4{g.w + (size_t)M->I * (M->H / 8), g.s + (size_t)M->I * (M->H / M->group),
                  g.b + (size_t)M->I * (M->H / M->group)};
}
static bool qb_gmm(const qwk_moe *M)
{
#ifdef QB_NO_GMM
    return false;
#else
    return M->SI == M->I && qwk_gmm16_supported(M->H, M->group, (M->split ? M->gate : M->gate_up).w, qb_up_bank(M).w) &&
           qwk_gmm16_supported(M->H, M->group, M->sh_gate.w, M->sh_up.w);
#endif
}

static QbLayout qb_layout(const qwk_moe *M, int rows)
{
    QbLayout L;
    size_t o = 0;
    const bool gmm = qb_gmm(M);
    L.logits = o; o += al((size_t)rows * M->E * 4);
    L.qx = o;     o += gmm ? 0 : al((size_t)rows * (M->H / 16) * QW_Q16_BYTES);
    L.tab = o;    o += al((size_t)QB_TAB_INTS * 4);
    L.qact = o;   o += al((size_t)rows * M->K * (M->I / 16) * QW_Q16_BYTES);
    L.qsh = o;    o += al((size_t)rows * (M->SI / 16) * QW_Q16_BYTES);
    // the matrix-core gate / up: the token rows staged as f16, the pairs by
    // expert (then the shared expert's rows), a tile per unique expert and
    // one for the shared expert, the activations in fp32
    const size_t npk = (size_t)rows * M->K;
    L.xh = o;     o += gmm ? al((size_t)rows * M->H * 2) : 0;
    L.xF = o;     o += gmm ? al((size_t)rows * 4) : 0;
    L.perm = o;   o += gmm ? al((npk + rows) * 4) : 0;
    L.tiles = o;  o += gmm ? al((1 + 3 * ((size_t)QD_MAXU + 1)) * 4) : 0;
    L.act = o;    o += gmm ? al((npk + rows) * M->I * 4) : 0;
    L.total = o;
    return L;
}

struct QbArgs {
    QdArgs d;                 // shapes, x, out, idx, w, rows, lgG, tch, qact, qsh
    const float *logits;
    int32_t *tab;
    int xstaged;              // the router launch staged the token rows into qx
    int gmm;                  // gate / up on the matrix cores: emit perm and tiles
    int32_t *perm, *tiles;
    const float *act;         // their fp32 activations [pairs + rows][I]
};

template <int PL>
__global__ __launch_bounds__(QD_MAXT * 64) void k_batch_route(QbArgs b)
{
    __shared__ QdRoute R;
    const QdArgs &a = b.d;
    const int t = threadIdx.x, nthr = blockDim.x, wave = t >> 6, lane = t & 63;
    const int E = a.m.E, K = a.m.K, H = a.m.H;
    if (wave < a.rows) {
        int pi;
        float pw;
        qw_route_wave<PL>(b.logits + (size_t)wave * E, E, K, a.m.norm, lane, &pi, &pw, R.rs.sx[wave]);
        if (lane < K) {
            R.picks[wave * K + lane] = pi;
            R.pw[wave * K + lane] = pw;
            a.idx[wave * K + lane] = pi;
            a.w[wave * K + lane] = pw;
        }
    }
    // the token rows as q16 units for the gate / up launch (unless the
    // router's launch did)
    const int units = H / 16;
    for (int i = t; i < (b.xstaged ? 0 : a.rows * units); i += nthr) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = reinterpret_cast<const float4 *>(a.x + (size_t)i * 16)[q];
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
        uint4 u[3];
        qw_q16_make(v, u);
        a.qx[(size_t)i * 3] = u[0];
        a.qx[(size_t)i * 3 + 1] = u[1];
        a.qx[(size_t)i * 3 + 2] = u[2];
    }
    __syncthreads();
    // The union of the picks, ascending, with each expert's pairs in
    // ascending order, in parallel steps: per token a bitmask of its picks;
    // the marked experts compacted by ballots; counts by LDS atomics; the
    // starts by one wave's scan; a pair's place in its expert's run is the
    // number of earlier tokens that picked the same expert (a token's picks
    // are distinct, so pairs of one expert are ordered by token).
    __shared__ uint32_t tmask[QD_MAXT][QWK_ROUTE_MAX_E / 32];
    __shared__ int cnt[QWK_ROUTE_MAX_E];
    const int npk = a.rows * K, nwd = (E + 31) / 32;
    for (int i = t; i < QD_MAXT * (QWK_ROUTE_MAX_E / 32); i += nthr) (&tmask[0][0])[i] = 0u;
    for (int e = t; e < E; e += nthr) { R.mark[e] = 0; cnt[e] = 0; }
    __syncthreads();
    for (int p = t; p < npk; p += nthr) {
        const int e = R.picks[p];
        R.mark[e] = 1;
        atomicOr(&tmask[p / K][e >> 5], 1u << (e & 31));
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (wave == 0) {
        int base = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const bool on = e < E && R.mark[e];
            const unsigned long long bal = __ballot(on);
            if (on) {
                const int u = base + __popcll(bal & ((1ull << lane) - 1ull));
                R.uexp[u] = e;
                R.mark[e] = u;              // from here on: the expert's slot
            }
            base += __popcll(bal);
        }
        // starts: lane l scans slots 2l and 2l + 1 (U <= QD_MAXU <= 128)
        const int u0 = 2 * lane, u1 = 2 * lane + 1;
        const int c0 = u0 < base ? cnt[R.uexp[u0]] : 0, c1 = u1 < base ? cnt[R.uexp[u1]] : 0;
        int incl = c0 + c1;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        const int excl = incl - c0 - c1;
        if (u0 < base) { R.ucnt[u0] = c0; R.ustart[u0] = excl; }
        if (u1 < base) { R.ucnt[u1] = c1; R.ustart[u1] = excl + c0; }
        if (lane == 0) R.U = base;
    }
    __syncthreads();
    for (int p = t; p < npk; p += nthr) {
        const int e = R.picks[p], tk = p / K;
        int rank = 0;
        for (int q = 0; q < tk; q++) rank += (tmask[q][e >> 5] >> (e & 31)) & 1u;
        R.upair[R.ustart[R.mark[e]] + rank] = p;
    }
    __syncthreads();
    if (t == 0) b.tab[QB_TAB_U] = R.U;
    for (int u = t; u < R.U; u += nthr) {
        b.tab[QB_TAB_UEXP + u] = R.uexp[u];
        b.tab[QB_TAB_UCNT + u] = R.ucnt[u];
        b.tab[QB_TAB_USTART + u] = R.ustart[u];
    }
    for (int p = t; p < npk; p += nthr) b.tab[QB_TAB_UPAIR + p] = R.upair[p];
    if (b.gmm) {
        // the grouped product's tile list: unique expert u's pairs, then the
        // shared expert (expert E) on the token rows, pairs npk + r
        if (t == 0) {
            b.tiles[0] = R.U + 1;
            b.tiles[1 + 3 * R.U] = E;
            b.tiles[2 + 3 * R.U] = npk;
            b.tiles[3 + 3 * R.U] = a.rows;
        }
        for (int u = t; u < R.U; u += nthr) {
            b.tiles[1 + 3 * u] = R.uexp[u];
            b.tiles[2 + 3 * u] = R.ustart[u];
            b.tiles[3 + 3 * u] = R.ucnt[u];
        }
        for (int p = t; p < npk; p += nthr) b.perm[p] = R.upair[p];
        for (int r = t; r < a.rows; r += nthr) b.perm[npk + r] = npk + r;
    }
    (void)nwd;
}

// The matrix-core gate / up's fp32 activations as the q16 vectors the down
// launch reads: pair p's into qact, the shared expert's (rows npk + t) into
// qsh.  A thread per (vector, 16-unit).
__global__ __launch_bounds__(256) void k_batch_act_q16(QbArgs b)
{
    const QdArgs &a = b.d;
    const int I = a.m.I, units = I / 16, npk = a.rows * a.m.K;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (npk + a.rows) * units) return;
    const int v = i / units, u = i % units;
    float f[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 x = reinterpret_cast<const float4 *>(b.act + (size_t)v * I + 16 * u)[q];
        f[4 * q] = x.x; f[4 * q + 1] = x.y; f[4 * q + 2] = x.z; f[4 * q + 3] = x.w;
    }
    uint4 q3[3];
    qw_q16_make(f, q3);
    uint4 *d = v < npk ? a.qact + ((size_t)v * units + u) * 3 : a.qsh + ((size_t)(v - npk) * units + u) * 3;
    d[0] = q3[0];
    d[1] = q3[1];
    d[2] = q3[2];
}

template <int LPR, int NUL>
__global__ __launch_bounds__(QD_THREADS, 8) void k_batch_gu(QbArgs b)
{
    extern __shared__ uint4 xs[];                    // [tch][units][3]
    __shared__ int vin[QD_MAXT], vout[QD_MAXT];
    __shared__ float ys[QD_MAXT][QD_GU_MAXRPB];
    const QdArgs &a = b.d;
    constexpr int RPB = QD_WAVES * (64 / LPR);
    const int H = a.m.H, I = a.m.I, K = a.m.K;
    const int bb = blockIdx.x;
    QD_TS(0);
    if (bb < a.n_ex) {
        const int u = bb / a.gu_wg_per_u, rb = bb % a.gu_wg_per_u;
        if (u >= b.tab[QB_TAB_U]) return;                              // uniform
        const int e = b.tab[QB_TAB_UEXP + u], nt = b.tab[QB_TAB_UCNT + u], p0 = b.tab[QB_TAB_USTART + u];
        if (threadIdx.x < nt) {
            const int p = b.tab[QB_TAB_UPAIR + p0 + threadIdx.x];
            vin[threadIdx.x] = p / K;
            vout[threadIdx.x] = p;
        }
        __syncthreads();
        const size_t words = H / 8, groups = H >> a.lgG;
        qwk_q4 gm, um;
        if (a.m.split) {
            const size_t off = (size_t)e * I;
            gm = {a.m.gate.w + off * words, a.m.gate.s + off * groups, a.m.gate.b + off * groups};
            um = {a.m.up.w + off * words, a.m.up.s + off * groups, a.m.up.b + off * groups};
        } else {
            const size_t off = (size_t)e * 2 * I;
            gm = {a.m.gate_up.w + off * words, a.m.gate_up.s + off * groups, a.m.gate_up.b + off * groups};
            um = {gm.w + (size_t)I * words, gm.s + (size_t)I * groups, gm.b + (size_t)I * groups};
        }
        // the weights are requested first; the token rows follow from the
        // staged copy, pass by pass
        qd_glu_block<LPR, NUL, true>(gm, um, I, a, rb * RPB, nt, false, xs, vin, vout, a.qact, ys);
        QD_TS(5);
    } else {
        const int sb = bb - a.n_ex;
        if (threadIdx.x < QD_MAXT) vin[threadIdx.x] = vout[threadIdx.x] = threadIdx.x;
        __syncthreads();
        qd_glu_block<LPR, NUL, true>(a.m.sh_gate, a.m.sh_up, a.m.SI, a, sb * RPB, a.rows, false, xs, vin, vout,
                                     a.qsh, ys);
    }
}

template <int NUL>
__global__ __launch_bounds__(QD_THREADS, 8) void k_batch_down(QbArgs b)
{
    extern __shared__ uint4 xa[];                    // the K + 1 activation vectors
    __shared__ float ys[QWK_DECODE_MAX_K + 1][QD_DOWN_RPG];
    const QdArgs &a = b.d;
    constexpr int LPR = QD_DOWN_LPR, RPP = 64 / LPR, RIT = QD_DOWN_RIT, RPG = QD_DOWN_RPG;
    const int H = a.m.H, I = a.m.I, SI = a.m.SI, K = a.m.K;
    // block -> (token, row block): all tokens of row block rb on XCD rb mod 8
    const int q = blockIdx.x >> 3, xcd = blockIdx.x & 7;
    const int t = q % a.rows, rb = (q / a.rows) * 8 + xcd;
    if (rb >= a.n_down_rb) return;                   // uniform
    const int lane = threadIdx.x & 63, m = threadIdx.x >> 6;
    const int slot = lane / LPR, lr = lane % LPR;
    const int row0 = rb * RPG, lgG = a.lgG;
    const bool busy = m <= K;
    const int kin = m == 0 ? SI : I;
    const int units = kin / 16, words = kin / 8, groups = kin >> lgG;
    const uint32_t *wm = a.m.sh_down.w;
    const uint16_t *sm = a.m.sh_down.s, *bm = a.m.sh_down.b;
    if (busy && m > 0) {
        const size_t e = (size_t)a.idx[t * K + m - 1];
        wm = a.m.down.w + e * H * words;
        sm = a.m.down.s + e * H * groups;
        bm = a.m.down.b + e * H * groups;
    }
    uint2 wv[NUL][RIT];
    uint32_t sv[NUL][RIT], bv[NUL][RIT];
#pragma unroll
    for (int j = 0; j < NUL; j++) {
        const int c = min(j * LPR + lr, units - 1);
        const int g = (16 * c) >> lgG;
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const int row = min(row0 + slot + RPP * i, H - 1);
            wv[j][i] = qw_ld2(wm, (uint32_t)(row * words + 2 * c) * 4u);
            sv[j][i] = qw_ldu16(sm, (uint32_t)(row * groups + g) * 2u);
            bv[j][i] = qw_ldu16(bm, (uint32_t)(row * groups + g) * 2u);
        }
    }
    // this matrix's activation vector into the wave's own LDS region
    const int nv = units * 3;
    constexpr int XW = (3 * NUL * LPR + 63) / 64;
    uint4 *xw = xa + (m == 0 ? 0 : (SI / 16) * 3 + (m - 1) * ((I / 16) * 3));
    if (busy) {
        const uint4 *xm = m == 0 ? a.qsh + (size_t)t * ((SI / 16) * 3)
                                 : a.qact + ((size_t)t * K + (m - 1)) * ((I / 16) * 3);
        uint4 v[XW];
#pragma unroll
        for (int r = 0; r < XW; r++) v[r] = xm[min(lane + 64 * r, nv - 1)];
#pragma unroll
        for (int r = 0; r < XW; r++)
            if (lane + 64 * r < nv) xw[lane + 64 * r] = v[r];
    }
    const float gate = qw_sigmoid(__int_as_float(b.tab[QB_TAB_GATE + t]));
    if (busy) {
        uint32_t sb[NUL][RIT];
#pragma unroll
        for (int j = 0; j < NUL; j++)
#pragma unroll
            for (int i = 0; i < RIT; i++) {
                const bool ok = j * LPR + lr < units && row0 + slot + RPP * i < H;
                wv[j][i] = ok ? wv[j][i] : make_uint2(0, 0);
                sb[j][i] = ok ? sv[j][i] | (bv[j][i] << 16) : 0u;
            }
        float y[RIT];
#pragma unroll
        for (int i = 0; i < RIT; i++) y[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < NUL; j++) {
            const int c = j * LPR + lr;
            if (c < units) {
                const uint4 p0 = xw[3 * c], p1 = xw[3 * c + 1], rr = xw[3 * c + 2];
                const float4 r = *reinterpret_cast<const float4 *>(&rr);
#pragma unroll
                for (int i = 0; i < RIT; i++)
                    y[i] = qw_unit_dot(wv[j][i], p0, p1, r, __uint_as_float(sb[j][i] << 16),
                                       __uint_as_float(sb[j][i] & 0xFFFF0000u), y[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < RIT; i++) {
            const float v = qw_xor_sum<LPR>(y[i]);
            if (lr == 0) ys[m][slot + RPP * i] = v;
        }
    }
    __syncthreads();
    // the combine: the shared term first, then an fma per slot, in order
    for (int r = threadIdx.x; r < RPG; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= H) continue;
        float acc = ys[0][r] * gate;
        for (int k = 0; k < K; k++) acc = __builtin_fmaf(a.w[t * K + k], ys[1 + k][r], acc);
        a.out[(size_t)t * H + row] = acc;
    }
}

extern "C" size_t qwk_moe_decode_batch_scratch(const qwk_moe *M, int rows)
{
    return qb_layout(M, rows).total;
}

extern "C" int qwk_moe_decode_batch(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                                    const qwk_moe *M, int rows, void *scratch, size_t scratch_bytes)
{
    const int G = M->group;
    if (rows < 2 || !qwk_moe_decode_supported(M, rows) || !x || ((uintptr_t)x & 15u)) return (int)hipErrorInvalidValue;
    const QbLayout L = qb_layout(M, rows);
    if (scratch_bytes < L.total) return (int)hipErrorInvalidValue;
    int lpr_h, nul_h, nul_d, pl;
    qd_shapes(M, &lpr_h, &nul_h, &nul_d, &pl);
    char *S = (char *)scratch;
    QbArgs b;
    QdArgs &a = b.d;
    a = QdArgs{};
    a.m = *M;
    a.x = x; a.out = out; a.idx = idx; a.w = w; a.rows = rows;
    a.umax = rows * M->K < M->E ? rows * M->K : M->E;
    a.lgG = G == 32 ? 5 : G == 64 ? 6 : 7;
    const int rpb = QD_WAVES * (64 / lpr_h);
    const int vbytes = (M->H / 16) * QW_Q16_BYTES;
    a.tch = QD_LDS / vbytes < rows ? QD_LDS / vbytes : rows;
    a.n_sh = (M->SI + rpb - 1) / rpb;
    a.gu_wg_per_u = (M->I + rpb - 1) / rpb;
    a.n_ex = a.umax * a.gu_wg_per_u;
    a.n_down_rb = (M->H + QD_DOWN_RPG - 1) / QD_DOWN_RPG;
    a.scr = S;
    a.qx = (uint4 *)(S + L.qx);
    a.qact = (uint4 *)(S + L.qact);
    a.qsh = (uint4 *)(S + L.qsh);
    b.logits = (const float *)(S + L.logits);
    b.tab = (int32_t *)(S + L.tab);
    const qwk_q4 g0 = M->split ? M->gate : M->gate_up, u0 = qb_up_bank(M);
    const int npk = rows * M->K;
    b.gmm = qb_gmm(M);
    b.perm = (int32_t *)(S + L.perm);
    b.tiles = (int32_t *)(S + L.tiles);
    b.act = (const float *)(S + L.act);
    const size_t xs_bytes = (size_t)a.tch * vbytes;
    const size_t xa_bytes = ((size_t)(M->SI / 16) + (size_t)M->K * (M->I / 16)) * QW_Q16_BYTES;
    if (a.tch < 1 || xa_bytes > QD_LDS || a.umax > QD_MAXU) return (int)hipErrorInvalidValue;
    // the router logits and the shared expert's gate logits, one launch
    float *lg = (float *)(S + L.logits), *gl = (float *)(b.tab + QB_TAB_GATE);
    // (which also stages the token rows as q16 for the gate / up launch)
    b.xstaged = 1;
    // (or, for the matrix-core gate / up, as f16 rows with a scale each)
    int rc = qwk_dmat_bf16_gate(s, lg, gl, x, M->router, M->sh_gate_w, M->H, M->E, rows, b.gmm ? nullptr : a.qx,
                                b.gmm ? (uint16_t *)(S + L.xh) : nullptr, b.gmm ? (float *)(S + L.xF) : nullptr);
    bool staged16 = rc == 0;
    if (rc == (int)hipErrorInvalidValue) {   // a layout the one launch does not take: two order-R launches
        b.xstaged = b.gmm;
        rc = qwk_dmat_bf16(s, lg, x, M->router, M->H, M->E, rows);
        if (!rc) rc = qwk_dmat_bf16(s, gl, x, M->sh_gate_w, M->H, 1, rows);
    }
    if (!rc && b.gmm && !staged16) rc = qwk_stage16(s, (uint16_t *)(S + L.xh), (float *)(S + L.xF), x, rows, M->H);
    if (rc) return rc;
    const int nrb8 = (a.n_down_rb + 7) / 8 * 8;
    const qwk_gmm_extra xgu = {M->sh_gate, M->sh_up, M->E, npk};
    const int nvu = (npk + rows) * (M->I / 16);
#define QB_GO(L_, N_, D_, P_)                                                                                   \
    if (lpr_h == L_ && nul_h == N_ && nul_d == D_ && pl == P_) {                                              \
        hipLaunchKernelGGL(k_batch_route<P_>, dim3(1), dim3(QD_MAXT * 64), 0, s, b);                          \
        if (b.gmm) {                                                                                          \
            const int rg = qwk_gmm16(s, (float *)b.act, M->I, (const uint16_t *)(S + L.xh),                   \
                                     (const float *)(S + L.xF), b.perm, b.tiles, a.umax + 1, g0, u0,           \
                                     (long)(M->split ? 1 : 2) * M->I * (M->H / 8),                             \
                                     (long)(M->split ? 1 : 2) * M->I * (M->H / G), M->H, M->I, M->K, 0, G, 1, \
                                     0, &xgu);                                                                 \
            if (rg) return rg;                                                                                \
            hipLaunchKernelGGL(k_batch_act_q16, dim3((nvu + 255) / 256), dim3(256), 0, s, b);                 \
        } else {                                                                                              \
            hipLaunchKernelGGL((k_batch_gu<L_, N_>), dim3(a.n_ex + a.n_sh), dim3(QD_THREADS), xs_bytes, s, b);\
        }                                                                                                     \
        hipLaunchKernelGGL(k_batch_down<D_>, dim3(rows * nrb8), dim3(QD_THREADS), xa_bytes, s, b);            \
        return (int)hipGetLastError();                                                                        \
    } else
    QD_SHAPES(QB_GO)
#undef QB_GO
    return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}
