// qw_decode1.hip -- the MoE block decoding ONE token in ONE launch, laid out
// by XCD.
//
// MI355X has 8 XCDs of 32 CUs, each with its own L2; a launch's workgroups
// are dealt to them round-robin in block order (from an XCD that varies by
// launch), and each workgroup reads which one it runs on.  A store that
// another XCD must see goes past the L2 (device scope, sc1), and the load that
// polls for it is served by the memory side: a round trip through the fabric,
// slow while the expert weights stream.  Between CUs of one XCD the L2 is
// shared: a workgroup-scope store lands in it and a device-scope load (which
// skips the CU's L1) finds it there, without leaving the XCD.  So
// the launch crosses XCDs twice, both at quiet times, and every other
// hand-off stays inside an XCD:
//
//   router     (block 0 .. n_rt)  QX_RT_ROWS router rows a workgroup, one
//              wave a row, order R (the token staged in LDS while the rows
//              load); each logit leaves as a tagged word, device scope
//   gatherer   (8 consecutive blocks, one an XCD)  polls the E + 1 tagged logits once
//              for its XCD, routes (qw_route_block: the picks, their
//              weights, bit-exact to the oracle), and publishes the picks,
//              the weights and the shared expert's gate to its XCD's L2
//   worker     (W an XCD, on XCD x)  owns part of XCD x's share of
//              the work.  The work is cut into units, (matrix, slice): the
//              matrices are the shared expert (0) and the K picks (1 + k),
//              a slice is SW consecutive intermediate features (SW columns
//              of the down matrix).  Unit u goes to XCD u % 8.  Each worker
//                - computes its rows of XCD x's gate/up rows (the units'
//                  gate and up rows, 2 SW each) against the token, and
//                  hands the SwiGLU activations to its XCD as tagged words;
//                - holds its H / W output rows of every unit's down slice,
//                  requested as soon as the picks are known;
//                - waits for its XCD's activations, and computes its rows'
//                  partial output P_x = sum over XCD x's units (in unit
//                  order) of coef(unit) * down_slice . act_slice, with
//                  coef = sigmoid(shared gate) for the shared expert's
//                  units and the pick's weight for a pick's;
//                - on XCDs 0..6 stores P_x as tagged words, device scope;
//                  on XCD 7 waits for the other seven and writes
//                  out = ((P_0 + P_1) + ... + P_6) + P_7 for its rows.
//
// Each weight byte is read once, by one workgroup, and the work a CU does is
// the same on every CU to within a unit's share.  The output's summation
// order is fixed by the shapes alone, so every launch gives the same bits.
//
// Tagged words: a 64-bit store {launch epoch, 32-bit payload}; a reader that
// sees this launch's epoch sees the payload with it, so a producer needs no
// acknowledgement, counter or flag.  Words keep past epochs between launches;
// an epoch is never reused before the state is zeroed.
//
// Progress: routers wait on nothing; a gatherer waits on routers (lower block
// indices); a worker waits on its XCD's gatherer (lower) and on the other
// workers of its XCD, which fit on the XCD together with everything launched
// before them (QX_W_MAX workers and 64 / 8 routers and gatherers an XCD, at
// two workgroups a CU), so every wait ends.  Each wait is also bounded: past
// QX_SPIN_LIMIT polls it raises the error word, every later wait gives up at
// once, and the host reports the error.  A workgroup whose wait gave up still
// publishes what it computed, so no other wait is left without an end.
#include <hip/hip_ext.h>
#include <type_traits>

#ifdef QW_TRACE
// QW_TRACE_MASK: the slots that stamp (each stamp costs its wave time)
#ifndef QW_TRACE_MASK
#define QW_TRACE_MASK 0xffff
#endif
#define QX_TON(slot) ((((QW_TRACE_MASK) >> (slot)) & 1) != 0)
// (the routing helpers' phase hooks, in the same trace: slots 3..9 and 10, 11)
extern __device__ unsigned long long qx_trace[2048 * 16];
#define QW_RSTAMP(slot) do { if (QX_TON(1 + (slot)) && threadIdx.x == 0) qx_trace[blockIdx.x * 16 + 1 + (slot)] = wall_clock64(); } while (0)
#define QW_STAMP(slot) do { if (QX_TON(4 + (slot)) && threadIdx.x == 0) qx_trace[blockIdx.x * 16 + 4 + (slot)] = wall_clock64(); } while (0)
#endif
#include "qw_device.h"
#include "qw_kernels.h"

// One documented timing hook: built with -DQW_TRACE, thread 0 of every
// workgroup stamps the device wall clock (100 MHz) at its phases into
// qx_trace[block][slot], read back with qwk_decode_trace_read.  Empty otherwise.
#ifdef QW_TRACE
__device__ unsigned long long qx_trace[2048 * 16];
// slots 0..14 the phases (thread 0, or the first lane of wave w for
// QX_TSW); slot 15 where the workgroup ran (HW_REG_XCC_ID)
#define QX_TS(slot) do { if (QX_TON(slot) && threadIdx.x == 0) { qx_trace[blockIdx.x * 16 + (slot)] = wall_clock64(); \
    if ((slot) == 0) qx_trace[blockIdx.x * 16 + 15] = (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 20) | \
        ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4) << 32); } } while (0)
#define QX_TSW(w, slot) do { if (QX_TON(slot) && threadIdx.x == 64 * (w)) qx_trace[blockIdx.x * 16 + (slot)] = wall_clock64(); } while (0)
extern "C" int qwk_decode_trace_read(unsigned long long *dst, size_t n)
{
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(qx_trace), n * sizeof(unsigned long long));
}
#else
#define QX_TS(slot) do { } while (0)
#define QX_TSW(w, slot) do { } while (0)
#endif

#define QX_WAVES 16
#define QX_THREADS (QX_WAVES * 64)
#define QX_NX 8                    // XCDs
#define QX_LDS (72 * 1024)         // dynamic LDS of every role (two workgroups a CU)
#define QX_RT_ROWS 4               // router rows a router workgroup
#define QX_XPAD 68                 // floats a 64-input token chunk takes in the router's LDS
#define QX_WPAD 36                 // dwords a router-row chunk takes in LDS (32 + pad)
#define QX_PL 8                    // logits a routing lane holds: E <= 512
#define QX_MAX_H 4096
#define QX_W_MAX 32                // workers an XCD
#define QX_PICK_WORDS 64           // an XCD's picks record: ids [0, K), weights [K, 2K), shared gate 2K
#define QX_ACT_WORDS 1280          // an XCD's activations (its units' SW features each)
// gate/up row instructions a wave, at most, for NUPL units a lane a row:
// at most 32 registers of weight words a lane
#define QX_NRI_OF(X) X(1, 4) X(2, 4) X(3, 4) X(4, 3)
#define QX_MAX_UX 16               // units an XCD (at most)
// A wave waits for its loads in issue order, and the compiler makes any LDS
// read wait for every copy into LDS its wave has in flight: so the gate/up
// rows and the copies of the down slices are issued by different waves.
#define QX_GUW 12                  // waves 0..11: gate/up rows
#define QX_CPW (QX_WAVES - QX_GUW) // waves 12..15: the down slices' copies into LDS
#define QX_SPIN_LIMIT (1 << 16)
// sleep between polls, in s_sleep units of 64 clocks: the far polls (device
// scope) share the memory side with the weight stream, the near ones (L2) not
// (near polls with no sleep, and the partial sums' far polls too, measured
// 0.25 us a token faster than 1 and 2: 20.27 -> 20.02 over six alternating
// runs; a sleep of 6 for the partials' polls measured slower)
#define QX_SLEEP_FAR 8
#define QX_SLEEP_NEAR 0
// (the picks come a routing's time after the workers start: they poll slower)
#define QX_SLEEP_PICKS 2
// (the XCD that sums the partials polls last, with the weight stream over)
#define QX_SLEEP_PART 0

static_assert(QX_PICK_WORDS >= 2 * QWK_DECODE_MAX_K + 1, "picks record");
static_assert(QX_PL * 64 >= 512, "routing lanes");

// ---- hand-off state (zeroed by the host before first use) --------------------------

struct QxLocal {                   // written and read on one XCD only
    uint2 pick[QX_PICK_WORDS];
    uint2 act[QX_ACT_WORDS];
};

struct QxSync {
    uint32_t err;                  // epoch of the first launch whose wait gave up (0: none)
    uint32_t pad[63];
    uint2 lgt[QWK_ROUTE_MAX_E + 64];        // the router's logits, [E] the shared gate logit
    QxLocal loc[QX_NX];
    uint2 part[QX_NX - 1][QX_MAX_H];        // XCD x's partial output rows, read on XCD 7
};

struct QxArgs {
    qwk_moe m;
    const float *x;
    // with hin set the input is x = rms_norm(bf16(hin + yprev)) (yprev may be null)
    const uint16_t *hin;
    const float *yprev;
    uint16_t *hout;                // bf16(hin + yprev), written by worker 0 of XCD 0
    float *xout;                   // that x, written by the same worker
    float eps;
    float *out;
    int32_t *idx;
    float *w;
    QxSync *sync;
    uint32_t epoch;
    int lgG;                       // log2(group)
    int n_rt;                      // router workgroups
    int W;                         // workers an XCD
    int SW, NSU;                   // slice width (features) and its q16 units (SW / 16)
    int nus, nui, NU;              // slices of the shared expert, of a routed expert; units in all
    int lrg;                       // gate/up lanes a row: min(64, H / 16)
    int nri;                       // gate/up row instructions a wave
    int rpw;                       // down rows a worker: ceil(H / W)
    int pb;                        // bytes a copy of down words into LDS: 16, or 4 (rows not 16-byte aligned)
    int sb4;                       // scales and biases copied 2 groups (4 bytes) at a time, else one a dword slot
    int ngw;                       // dword slots of scales (and of biases) a down item
    int gsb4;                      // a gate/up row's scales copied 2 groups a dword, else one a dword slot
    int lgSW, lgppi, lgngw;        // log2 of SW, of the copies a down row (SW / 2 / pb), of ngw
    int sb16;                      // gate/up scales by one 16-byte load a lane (see the worker)
    int pre;                       // the shared expert's slices requested before the picks
};

// A plain load from global memory through a pointer the compiler cannot see
// is global (read back from LDS): without the cast it becomes a flat load,
// which also waits on the LDS counter.
__device__ __forceinline__ uint2 qx_ldg2(const uint32_t *p)
{
    const unsigned long long v = *(const __attribute__((address_space(1))) unsigned long long *)p;
    return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

typedef unsigned int qx_u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 qx_ldg4(const void *p)
{
    const qx_u4v v = *(const __attribute__((address_space(1))) qx_u4v *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- tagged words ---------------------------------------------------------------

__device__ __forceinline__ void qx_put_far(uint2 *p, uint32_t epoch, uint32_t v)
{
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p),
                       (unsigned long long)epoch | ((unsigned long long)v << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void qx_put_near(uint2 *p, uint32_t epoch, uint32_t v)
{
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p),
                       (unsigned long long)epoch | ((unsigned long long)v << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Loads for polling, volatile so that every pass issues them; the caller
// waits for a pass's loads at once (qx_wait ties their registers to the wait).
// Both are device-scope loads (sc1): they miss the CU's L1 and read the
// XCD's L2 where the line is held there, else the memory side.  A near word
// (a workgroup-scope store by a CU of the same XCD) is in that L2: measured
// on an idle MI355X, a poller on the writer's XCD sees a store after
// ~0.24 us, one on another XCD after ~1 us.  (Plain and workgroup-scope
// loads, with or without an L1 invalidate, kept returning the line an
// earlier poll cached and never saw the store.)  A far word is stored with
// device scope (sc1): another XCD sees it after ~0.5 us.
__device__ __forceinline__ unsigned long long qx_ld_far(const uint2 *p)
{
    unsigned long long v;
    asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ unsigned long long qx_ld_near(const uint2 *p) { return qx_ld_far(p); }
__device__ __forceinline__ uint32_t qx_ld_err(const QxSync *S)
{
    uint32_t v;
    asm volatile("global_load_dword %0, %1, off sc1" : "=v"(v) : "v"(&S->err) : "memory");
    return v;
}
template <int NW>
__device__ __forceinline__ void qx_wait(unsigned long long (&q)[NW], uint32_t &e)
{
    if constexpr (NW == 1) asm volatile("s_waitcnt vmcnt(0)" : "+v"(q[0]), "+v"(e)::"memory");
    else {
        static_assert(NW == 2, "one or two words a lane");
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(q[0]), "+v"(q[1]), "+v"(e)::"memory");
    }
}

__device__ __forceinline__ void qx_raise(QxSync *S, uint32_t epoch)
{
    uint32_t expect = 0u;
    __hip_atomic_compare_exchange_strong(&S->err, &expect, epoch, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}

// One wave: lane l waits for words p[l + 64 i] (i < NW, l + 64 i < n) to hold
// this launch's epoch and returns their payloads in v[i].  FAR (the words
// come from other XCDs): the error word is read with every pass; near (from
// this XCD): every 8th pass.  On giving up the
// error word is raised and v holds whatever was read.
template <int NW, bool FAR, int SLP = (FAR ? QX_SLEEP_FAR : QX_SLEEP_NEAR)>
__device__ __forceinline__ void qx_poll(const QxArgs &a, const uint2 *p, int n, uint32_t (&v)[NW])
{
    const int lane = threadIdx.x & 63;
    for (int spins = 0;; spins++) {
        unsigned long long q[NW];
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const uint2 *pi = p + min(lane + 64 * i, n - 1);
            q[i] = FAR ? qx_ld_far(pi) : qx_ld_near(pi);
        }
        uint32_t e = 0u;
        if (FAR || (spins & 7) == 7) e = qx_ld_err(a.sync);
        qx_wait<NW>(q, e);
        bool stale = false;
#pragma unroll
        for (int i = 0; i < NW; i++) {
            v[i] = (uint32_t)(q[i] >> 32);
            stale |= lane + 64 * i < n && (uint32_t)q[i] != a.epoch;
        }
        if (__ballot(stale) == 0ull) return;
        if (spins >= QX_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
            if (lane == 0) qx_raise(a.sync, a.epoch);
            return;
        }
        __builtin_amdgcn_s_sleep(SLP);
    }
}

// Sum over aligned runs of `width` lanes (a power of two, wave-uniform); for
// width 64 the xor tree of qw_xor_sum<64>.
__device__ __forceinline__ float qx_run_sum(float v, int width)
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

// A workgroup barrier without a memory fence: this wave's LDS accesses are
// complete (lgkmcnt 0), its global loads may still be in flight.
__device__ __forceinline__ void qx_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---- the residual step as the launch's prologue ----------------------------------
//
// With a.hin set, x = rms_norm(bf16(hin + yprev)), with the arithmetic and the
// summation order of k_resid_rms_bf16 (qw_norm.hip: each of 256 threads an
// fmaf chain over its float4 chunks, the xor tree, the four wave partials in
// order), so x has the bits that kernel gives.

__device__ __forceinline__ float qx_bf16r(float f)
{
    const uint32_t u = __float_as_uint(f);
    return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

// bf16(hin + yprev), columns 4 i4 .. 4 i4 + 3
__device__ __forceinline__ float4 qx_v4(const QxArgs &a, int i4)
{
    const uint2 hb = reinterpret_cast<const uint2 *>(a.hin)[i4];
    float4 v = make_float4(__uint_as_float(hb.x << 16), __uint_as_float(hb.x & 0xFFFF0000u),
                           __uint_as_float(hb.y << 16), __uint_as_float(hb.y & 0xFFFF0000u));
    if (a.yprev) {
        const float4 y = reinterpret_cast<const float4 *>(a.yprev)[i4];
        v = make_float4(qx_bf16r(v.x + y.x), qx_bf16r(v.y + y.y), qx_bf16r(v.z + y.z), qx_bf16r(v.w + y.w));
    }
    return v;
}

template <bool RES>
__device__ __forceinline__ float4 qx_x4(const QxArgs &a, float qinv, int i4)
{
    if constexpr (!RES) return reinterpret_cast<const float4 *>(a.x)[i4];
    const float4 v = qx_v4(a, i4);
    return make_float4(v.x * qinv, v.y * qinv, v.z * qinv, v.w * qinv);
}

// 1 / sqrt(mean(v^2) + eps) of the row, by the 256 threads t0 .. t0 + 255 as
// k_resid_rms_bf16's threads 0..255 (the whole workgroup calls it; it holds
// a barrier)
template <bool FENCE = true>
__device__ __forceinline__ float qx_norm(const QxArgs &a, float *qpart, int t0)
{
    const int tid = (int)threadIdx.x - t0, g = tid >> 6;
    const int n4 = a.m.H / 4;
    float ss = 0.0f;
    if (tid >= 0 && tid < 256)
        for (int i = tid; i < n4; i += 256) {
            const float4 v = qx_v4(a, i);
            ss = __builtin_fmaf(v.x, v.x, ss);
            ss = __builtin_fmaf(v.y, v.y, ss);
            ss = __builtin_fmaf(v.z, v.z, ss);
            ss = __builtin_fmaf(v.w, v.w, ss);
        }
    ss = qw_xor_sum<64>(ss);
    if ((tid & 63) == 0 && tid >= 0 && g < 4) qpart[g] = ss;
    if constexpr (FENCE) __syncthreads();
    else qx_barrier();           // (loads in flight stay in flight)
    float sum = qpart[0];
    sum = sum + qpart[1];
    sum = sum + qpart[2];
    sum = sum + qpart[3];
    return 1.0f / sqrtf(sum / (float)a.m.H + a.eps);
}

// ---- router -----------------------------------------------------------------------
//
// Wave r < QX_RT_ROWS takes router row o = b + n_rt r (row E: the shared
// expert's gate vector).  Order R: lane c computes the fmaf chain of 64-input
// chunk c; the chunk partials are added left to right from -0.  The row is
// loaded contiguously (each load instruction covers whole lines) and passed
// through the wave's LDS region to the lane-per-chunk layout; the token is
// loaded into LDS while the rows are in flight.
template <bool RES>
__device__ void qx_router(const QxArgs &a, int b, float *lds, float *qpart)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = a.m.H, E = a.m.E, nch = H / 64, npc = H / 8;
    // rows b, b + n_rt, ...: the router workgroups' requests spread over the
    // matrix rather than each walking a contiguous run in step
    const int o = b + a.n_rt * wave;
    const bool row = wave < QX_RT_ROWS && o <= E;
    float *xl = lds, *part = lds + 64 * QX_XPAD + wave * 64;
    uint32_t *wl = reinterpret_cast<uint32_t *>(lds + 64 * QX_XPAD + QX_WAVES * 64) + wave * 64 * QX_WPAD;
    // waves < QX_RT_ROWS load their rows (a wave past E loads the gate row and
    // drops it) and pass them through LDS; the others stage the token.  With
    // RES the token's row scale comes from waves QX_RT_ROWS .. QX_RT_ROWS + 3
    // while the rows are in flight, and the router waves meet its barrier with
    // their rows already in LDS (no registers held across it)
    float qinv = 1.0f;
    if (wave < QX_RT_ROWS) {
        const uint16_t *wr = o < E ? a.m.router + (size_t)o * H : a.m.sh_gate_w;
        uint4 v[8];
#pragma unroll
        for (int r = 0; r < 8; r++) v[r] = reinterpret_cast<const uint4 *>(wr)[min(lane + 64 * r, npc - 1)];
        // (unconditional: pieces past the row land in chunks >= nch of the
        // wave's 64-chunk region, which nothing reads)
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int i = lane + 64 * r;
            *reinterpret_cast<uint4 *>(wl + (i / 8) * QX_WPAD + (i % 8) * 4) = v[r];
        }
    }
    if constexpr (RES) qinv = qx_norm(a, qpart, 64 * QX_RT_ROWS);
    if (wave >= QX_RT_ROWS) {
        for (int i = threadIdx.x - 64 * QX_RT_ROWS; i < H / 4; i += QX_THREADS - 64 * QX_RT_ROWS)
            *reinterpret_cast<float4 *>(xl + (i / 16) * QX_XPAD + (i % 16) * 4) = qx_x4<RES>(a, qinv, i);
    }
    QX_TS(1);
    qx_barrier();          // the token is in LDS
    QX_TS(3);
    if (!row) return;
    const int c = min(lane, nch - 1);
    float s = 0.0f;
    if (lane < nch) {
        const float4 *xv = reinterpret_cast<const float4 *>(xl + lane * QX_XPAD);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const uint4 wq = *reinterpret_cast<const uint4 *>(wl + c * QX_WPAD + 4 * q);
            const float4 x0 = xv[2 * q], x1 = xv[2 * q + 1];
            s = __builtin_fmaf(__uint_as_float(wq.x << 16), x0.x, s);
            s = __builtin_fmaf(__uint_as_float(wq.x & 0xFFFF0000u), x0.y, s);
            s = __builtin_fmaf(__uint_as_float(wq.y << 16), x0.z, s);
            s = __builtin_fmaf(__uint_as_float(wq.y & 0xFFFF0000u), x0.w, s);
            s = __builtin_fmaf(__uint_as_float(wq.z << 16), x1.x, s);
            s = __builtin_fmaf(__uint_as_float(wq.z & 0xFFFF0000u), x1.y, s);
            s = __builtin_fmaf(__uint_as_float(wq.w << 16), x1.z, s);
            s = __builtin_fmaf(__uint_as_float(wq.w & 0xFFFF0000u), x1.w, s);
        }
        part[lane] = s;
    }
    // a wave's LDS accesses run in order: lane 0 reads what the wave wrote
    if (lane == 0) {
        float total = -0.0f;
        int k = 0;
        for (; k + 4 <= nch; k += 4) {
            const float4 p4 = *reinterpret_cast<const float4 *>(part + k);
            total = total + p4.x;
            total = total + p4.y;
            total = total + p4.z;
            total = total + p4.w;
        }
        for (; k < nch; k++) total = total + part[k];
        qx_put_far(a.sync->lgt + o, a.epoch, __float_as_uint(total));
    }
    QX_TS(2);
}

// ---- gatherer: the logits once an XCD, routing, the picks published ---------------

struct QxGatherLds {
    uint32_t sx[QW_ROUTE_SX];
    float vb[QW_ROUTE_BLOCK_LDS];
    float coef;
};

__device__ void qx_gather(const QxArgs &a, int x, QxGatherLds &G)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int E = a.m.E, K = a.m.K;
    int pi = 0;
    float pw = 0.0f;
    // Two passes over the same code: the first on made-up logits while the
    // router works, which brings the routing code into this CU's instruction
    // cache (a launch runs it once: cold, every miss a trip to memory); the
    // second on the real ones.
#pragma nounroll
    for (int pass = 0; pass < 2; pass++) {
        float lv = -0.01f * (float)(lane + 64 * wave);
        if (pass == 1) {
            if (wave < QX_PL && 64 * wave < E) {
                uint32_t v[1];
                qx_poll<1, true>(a, a.sync->lgt + 64 * wave, E - 64 * wave, v);
                lv = __uint_as_float(v[0]);
            } else if (wave == QX_PL) {
                uint32_t v[1];
                qx_poll<1, true>(a, a.sync->lgt + E, 1, v);
                if (lane == 0) G.coef = qw_sigmoid(__uint_as_float(v[0]));
            }
            QX_TS(1);
        }
        // The ids leave as soon as they are final (the workers' weight
        // streams wait on them); the weights and the shared gate, which only
        // the down dots use, follow once renormalised.  Ids are clamped:
        // after a wait that gave up the logits are whatever was read, and no
        // pick may then address outside the banks.
        QxLocal &L = a.sync->loc[x];
        auto put_ids = [&](int id) {
            if (pass == 1 && lane < K) qx_put_near(L.pick + lane, a.epoch, (uint32_t)min(max(id, 0), E - 1));
        };
        // (waves whose slice starts past E hold -inf there: qw_route_block masks e >= E)
        qw_route_block<QX_PL>(lv, E, K, a.m.norm, wave, lane, &pi, &pw, G.sx, G.vb, put_ids);
        __syncthreads();
    }
    if (wave == 0) {
        pi = min(max(pi, 0), E - 1);
        QxLocal &L = a.sync->loc[x];
        if (lane < K) {
            qx_put_near(L.pick + K + lane, a.epoch, __float_as_uint(pw));
        } else if (lane == K) {
            qx_put_near(L.pick + 2 * K, a.epoch, __float_as_uint(G.coef));
        }
        if (x == 0 && lane < K) {
            a.idx[lane] = pi;
            a.w[lane] = pw;
        }
    }
    QX_TS(2);
}

// ---- worker ------------------------------------------------------------------------

// A unit of this XCD's work (matrix, slice): where its rows start, and its
// coefficient in the combine.
struct QxUnit {
    const uint32_t *gw, *uw;     // gate / up words of the slice's first row
    const uint16_t *gs, *gb, *us, *ub;
    const uint32_t *dw;          // down words of row 0 at the slice's first column
    const uint16_t *ds, *db;     // down scales / biases of row 0 at the slice's first group
    int dwr, dgr;                // down words, groups a row (kin / 8, kin / group)
    float coef;                  // sigmoid(shared gate) or the pick's weight
};

struct QxWorkLds {
    int pick[QWK_DECODE_MAX_K];
    float coef[QWK_DECODE_MAX_K + 1];          // [0] shared, [1 + k] pick k
    float qpart[4];
    QxUnit unit[QX_MAX_UX];
};

// The table entry of unit u (global index) once the picks are known.
__device__ __forceinline__ QxUnit qx_unit(const QxArgs &a, const QxWorkLds &S, int u)
{
    const int H = a.m.H, words = H / 8, groups = H >> a.lgG;
    QxUnit U;
    if (u < a.nus) {
        const size_t r0 = (size_t)u * a.SW;
        U.gw = a.m.sh_gate.w + r0 * words; U.gs = a.m.sh_gate.s + r0 * groups; U.gb = a.m.sh_gate.b + r0 * groups;
        U.uw = a.m.sh_up.w + r0 * words; U.us = a.m.sh_up.s + r0 * groups; U.ub = a.m.sh_up.b + r0 * groups;
        const int c0 = u * a.SW, kin = a.m.SI;
        U.dwr = kin / 8; U.dgr = kin >> a.lgG;
        U.dw = a.m.sh_down.w + c0 / 8;
        U.ds = a.m.sh_down.s + (c0 >> a.lgG);
        U.db = a.m.sh_down.b + (c0 >> a.lgG);
        U.coef = S.coef[0];
        return U;
    }
    const int k = min((u - a.nus) / a.nui, a.m.K - 1), sl = (u - a.nus) % a.nui;
    const size_t e = (size_t)S.pick[k], I = a.m.I;
    const size_t rr = (size_t)sl * a.SW;
    if (a.m.split) {
        const size_t r0 = e * I + rr;
        U.gw = a.m.gate.w + r0 * words; U.gs = a.m.gate.s + r0 * groups; U.gb = a.m.gate.b + r0 * groups;
        U.uw = a.m.up.w + r0 * words; U.us = a.m.up.s + r0 * groups; U.ub = a.m.up.b + r0 * groups;
    } else {
        const size_t g0 = e * 2 * I + rr, u0 = g0 + I;
        U.gw = a.m.gate_up.w + g0 * words; U.gs = a.m.gate_up.s + g0 * groups; U.gb = a.m.gate_up.b + g0 * groups;
        U.uw = a.m.gate_up.w + u0 * words; U.us = a.m.gate_up.s + u0 * groups; U.ub = a.m.gate_up.b + u0 * groups;
    }
    const int c0 = sl * a.SW, kin = a.m.I;
    U.dwr = kin / 8; U.dgr = kin >> a.lgG;
    U.dw = a.m.down.w + e * a.m.H * U.dwr + c0 / 8;
    U.ds = a.m.down.s + e * a.m.H * U.dgr + (c0 >> a.lgG);
    U.db = a.m.down.b + e * a.m.H * U.dgr + (c0 >> a.lgG);
    U.coef = S.coef[1 + k];
    return U;
}

// The worker's LDS regions, byte offsets (the same on the host, which checks
// the total against the dynamic LDS): per unit, nr rows of the down slice's
// words (ustr pieces of PB bytes, a multiple of 64 pieces so that no copy
// runs into the next unit) and of its scales and biases (sstr dword slots);
// the 2 P gate/up rows' scales and biases (gst dword slots a row); the
// token's UH q16 units; the 2 P gate/up results; the XCD's rows_x
// activations and their q16 units; 8 partials of nr rows.
struct QxWL {
    int dW, dS, dB, gS, gB, xs, ys, af, xq, fp, total;
};
__host__ __device__ inline QxWL qx_wlayout(int UH, int rows_x, int P, int nux, int nr, int ustr, int pb, int sstr,
                                           int gst)
{
    QxWL L;
    int o = 0;
    auto take = [&](int bytes) { const int r = o; o += (bytes + 255) & ~255; return r; };
    L.dW = take(nux * ustr * pb);
    L.dS = take(nux * sstr * 4);
    L.dB = take(nux * sstr * 4);
    L.gS = take(2 * P * gst * 4);
    L.gB = take(2 * P * gst * 4);
    L.xs = take(UH * 48);
    L.ys = take(2 * P * 4);
    L.af = take(rows_x * 4);
    L.xq = take((rows_x / 16) * 48);
    L.fp = take(8 * nr * 4);
    L.total = o;
    return L;
}

__host__ __device__ constexpr int qx_up64(int n) { return (n + 63) / 64 * 64; }

// The order in which worker j requests its gate/up rows: the rows past the
// first n0 (those requested before the picks) go from slot n0 + s to row
// n0 + (s A + j 5) mod (nq - n0), A coprime with nq - n0.  Workers that walk
// their rows in step request the same memory channels at the same time
// (measured: 256 workgroups each streaming its own contiguous run move a
// third less than when their requests are scattered); spread over different
// strides and starts, the rows a chip requests at once fall on all of them.
__device__ __forceinline__ int qx_perm_a(int n)
{
    const int c[5] = {7, 11, 13, 5, 3};
    for (int i = 0; i < 5; i++) {
        int x = c[i], y = n;
        while (y) { const int t = x % y; x = y; y = t; }
        if (x == 1) return c[i];
    }
    return 1;
}
__device__ __forceinline__ int qx_slot_row(int s, int j, int n0, int nq, int A)
{
    return s < n0 || s >= nq ? s : n0 + ((s - n0) * A + j * 5) % (nq - n0);
}

// units of XCD x: x, x + 8, ...
__device__ __forceinline__ int qx_units_of(const QxArgs &a, int x) { return x < a.NU ? (a.NU - x + 7) / 8 : 0; }

template <int NUPL, int NRI, bool RES>
__device__ void qx_worker(const QxArgs &a, int x, int j, uint4 *lds, QxWorkLds &S)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = a.m.H, K = a.m.K, UH = H / 16;
    const int nux = qx_units_of(a, x);
    const int rows_x = nux * a.SW;                         // gate/up pairs of XCD x
    const int P = (rows_x + a.W - 1) / a.W;                // pairs a worker
    // worker j takes the XCD's pairs j, j + W, ... and output rows j, j + W, ...:
    // each a short run, so the requests an XCD has in flight spread over
    // whole matrices instead of each worker walking a contiguous block
    const int np_ = j < rows_x ? (rows_x - 1 - j) / a.W + 1 : 0;   // pairs of this worker
    const int nr = j < H ? (H - 1 - j) / a.W + 1 : 0;             // output rows of this worker
    const int PB = a.pb, lgppi = a.lgppi, ppi = 1 << lgppi;    // copies a down row
    const int ngw = a.ngw, lgngw = a.lgngw;
    const int ustr = qx_up64(a.rpw * ppi), sstr = qx_up64(a.rpw * ngw);
    const int groups = H >> a.lgG, gst = a.gsb4 ? groups / 2 : groups;
    const QxWL L = qx_wlayout(UH, rows_x, P, nux, a.rpw, ustr, PB, sstr, gst);
    char *lb = reinterpret_cast<char *>(lds);
    uint8_t *dW = reinterpret_cast<uint8_t *>(lb + L.dW);
    uint32_t *dS = reinterpret_cast<uint32_t *>(lb + L.dS);
    uint32_t *dB = reinterpret_cast<uint32_t *>(lb + L.dB);
    uint32_t *gS = reinterpret_cast<uint32_t *>(lb + L.gS);
    uint32_t *gB = reinterpret_cast<uint32_t *>(lb + L.gB);
    uint4 *xs = reinterpret_cast<uint4 *>(lb + L.xs);
    float *ys = reinterpret_cast<float *>(lb + L.ys);
    float *af = reinterpret_cast<float *>(lb + L.af);
    uint4 *xq = reinterpret_cast<uint4 *>(lb + L.xq);
    float *fp = reinterpret_cast<float *>(lb + L.fp);          // [8][nr]

    // the token, staged as q16 units (every thread calls it: it holds a
    // barrier).  With RES it waits on the token's row scale (a read of the
    // row, a barrier, a second read), so it runs while the picks are awaited,
    // after the first requests (its barrier fence-free: they stay in flight);
    // else first.
    auto stage_token = [&]() {
        float qinv = 1.0f;
        if constexpr (RES) qinv = qx_norm<false>(a, S.qpart, 0);
        for (int u = threadIdx.x; u < UH; u += QX_THREADS) {
            float v[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 f = qx_x4<RES>(a, qinv, 4 * u + q);
                v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
            }
            qw_q16_stage(v, xs + 3 * u);
        }
        if constexpr (RES) {
            if (x == 0 && j == 0)
                for (int i = threadIdx.x; i < H / 4; i += QX_THREADS) {
                    const float4 v = qx_v4(a, i);
                    reinterpret_cast<uint2 *>(a.hout)[i] =
                        make_uint2((__float_as_uint(v.x) >> 16) | (__float_as_uint(v.y) & 0xFFFF0000u),
                                   (__float_as_uint(v.z) >> 16) | (__float_as_uint(v.w) & 0xFFFF0000u));
                    reinterpret_cast<float4 *>(a.xout)[i] = make_float4(v.x * qinv, v.y * qinv, v.z * qinv, v.w * qinv);
                }
        }
    };
    if constexpr (!RES) stage_token();
    // ---- requests.  Gate/up: row q of the worker (q < 2 np_) is pair
    // j + W (q / 2), gate (q even) or up; wave w's instruction i covers rows
    // (w + QX_GUW i) rpi + slot.  The shared expert needs no routing, so when
    // this XCD's first unit is one of its slices (x < nus) its rows (the
    // first nq_sh of this worker's) and their down slices are requested
    // before the picks are known (pass A), the rest after (pass B) ----
    const int lrg = a.lrg, rpi = 64 / lrg, slot = lane / lrg, lr = lane % lrg;
    const int nq = 2 * np_, words = H / 8, lgSW = a.lgSW;
    const int nq_sh = a.pre && x < a.nus ? 2 * (j < a.SW ? (a.SW - 1 - j) / a.W + 1 : 0) : 0;
    const int pa = qx_perm_a(max(nq - nq_sh, 1));
    uint2 gw[NRI][NUPL];
    int gq[NRI];
    const int sbp = groups / 8;                        // 16-byte pieces of a row's scales
    // The gate/up waves (< QX_GUW) request rows' words into registers and
    // the rows' scales and biases into LDS (row q at slot q gst), every load
    // at a clamped, valid address and none used yet.  With one row an
    // instruction and 16-byte runs of scales (a.sb16), one 16-byte load a
    // lane (lane i: the wave's instruction i / 16, biases when (i / 8) % 2,
    // piece i % 8), issued before the words, so that its store into LDS waits
    // for it alone; else copies into LDS a dword (or a bf16) a lane, a row an
    // instruction.  Only instruction 0 of a wave is ever a shared row
    // (nq_sh <= QX_GUW - 1, one row an instruction).
    auto sb_load = [&](bool want, uint4 &v, int &vq) {
        const int ri = lane >> 4, isb = (lane >> 3) & 1, pc = lane & 7;
        const int qs = wave + QX_GUW * ri, q = qx_slot_row(qs, j, nq_sh, nq, pa);
        vq = -1;
        if (want && ri < a.nri && qs < nq && pc < sbp) {
            const int p = j + a.W * (q >> 1);
            const QxUnit &U = S.unit[p >> lgSW];
            const uint16_t *rb = isb ? ((q & 1) ? U.ub : U.gb) : ((q & 1) ? U.us : U.gs);
            v = qx_ldg4(rb + (size_t)(p & (a.SW - 1)) * groups + 8 * pc);
            vq = q;
        }
    };
    auto sb_store = [&](const uint4 &v, int vq) {
        if (vq >= 0) *reinterpret_cast<uint4 *>(((lane >> 3) & 1 ? gB : gS) + vq * gst + 4 * (lane & 7)) = v;
    };
    auto row_load = [&](int i) {
        const int qs = (wave + QX_GUW * i) * rpi + slot, q = qx_slot_row(qs, j, nq_sh, nq, pa);
        gq[i] = i < a.nri && qs < nq ? q : -1;
        const int qc = min(q, max(nq - 1, 0));
        const int p = min(j + a.W * (qc >> 1), max(rows_x - 1, 0));
        const QxUnit &U = S.unit[p >> lgSW];
        const uint32_t *rw = ((qc & 1) ? U.uw : U.gw) + (size_t)(p & (a.SW - 1)) * words;
#pragma unroll
        for (int n = 0; n < NUPL; n++)
            gw[i][n] = qx_ldg2(rw + 2 * min(lr + lrg * n, UH - 1));
    };
    auto sc_copy = [&](int i0, int i1) {
        for (int i = i0; i < i1; i++)
            for (int sl = 0; sl < rpi; sl++) {
                const int qs = (wave + QX_GUW * i) * rpi + sl, q = qx_slot_row(qs, j, nq_sh, nq, pa);
                if (qs >= nq || lane >= gst) continue;
                const int p = j + a.W * (q >> 1);
                const QxUnit &U = S.unit[p >> lgSW];
                const size_t ro = (size_t)(p & (a.SW - 1)) * groups + (a.gsb4 ? 2 : 1) * lane;
                const uint16_t *ps = ((q & 1) ? U.us : U.gs) + ro, *pb = ((q & 1) ? U.ub : U.gb) + ro;
                __attribute__((address_space(3))) void *ds_ =
                    (__attribute__((address_space(3))) void *)(gS + q * gst);
                __attribute__((address_space(3))) void *db_ =
                    (__attribute__((address_space(3))) void *)(gB + q * gst);
                if (a.gsb4) {
                    __builtin_amdgcn_global_load_lds(ps, ds_, 4, 0, 0);
                    __builtin_amdgcn_global_load_lds(pb, db_, 4, 0, 0);
                } else {
                    __builtin_amdgcn_global_load_lds(ps, ds_, 2, 0, 0);
                    __builtin_amdgcn_global_load_lds(pb, db_, 2, 0, 0);
                }
            }
    };
    // The rest of a gate/up wave's requests, then its dots; instantiated with
    // and without instruction 0 already requested, so that no register holds
    // either of two loads (a merge of registers with loads in flight waits
    // for them).
    auto gu_rest = [&](auto pre0, auto sb16c) {
        constexpr bool P0 = decltype(pre0)::value, SB = decltype(sb16c)::value;
        uint4 sbv;                                 // (no initial value: a write would wait for the load)
        int sbq = -1;
        if (SB) sb_load(!P0 || (lane >> 4) > 0, sbv, sbq);
#pragma unroll
        for (int i = P0 ? 1 : 0; i < NRI; i++) row_load(i);
        if (SB) sb_store(sbv, sbq);
        else sc_copy(P0 ? 1 : 0, a.nri);
        QX_TSW(0, 7);
        // ---- gate/up dots (the first LDS read waits for this wave's loads) ----
#pragma unroll
        for (int i = 0; i < NRI; i++) {
            if (i >= a.nri) break;
            float acc = 0.0f;
#pragma unroll
            for (int n = 0; n < NUPL; n++) {
                const int c = lr + lrg * n;
                if (c < UH && gq[i] >= 0) {
                    const uint4 x0 = xs[3 * c], x1 = xs[3 * c + 1], rr = xs[3 * c + 2];
                    // bf16 g of the row's slots (two a dword), or the low half of slot g
                    const int g = (16 * c) >> a.lgG, hw = a.gsb4 ? g : 2 * g;
                    const uint32_t sv = reinterpret_cast<const uint16_t *>(gS + gq[i] * gst)[hw];
                    const uint32_t bv = reinterpret_cast<const uint16_t *>(gB + gq[i] * gst)[hw];
                    acc = qw_unit_dot(gw[i][n], x0, x1, *reinterpret_cast<const float4 *>(&rr),
                                      __uint_as_float(sv << 16), __uint_as_float(bv << 16), acc);
                }
            }
            acc = qx_run_sum(acc, lrg);
            if (lr == 0 && gq[i] >= 0) ys[gq[i]] = acc;
            if (i == 0) QX_TSW(0, 8);
        }
    };
    // The copy waves copy the units' down slices straight into LDS
    // (global_load_lds: no registers held): unit ui's rows j, j + W, ... of
    // its slice in PB-byte pieces (lane order = LDS order: piece q of the
    // unit is row q / ppi), then their scales and biases (ngw dword slots a
    // row: two groups a dword, or one bf16 in a dword's low half).  Pass 0
    // the shared unit (unit 0, when nq_sh > 0), pass 1 the others.
    auto issue_cp = [&](int pass) {
        {
            const int cw = wave - QX_GUW;
            // pass 0: unit 0 when it is a shared slice; pass 1: the rest
            const int u_lo = pass == 0 ? 0 : (nq_sh > 0 ? 1 : 0), u_hi = pass == 0 ? (nq_sh > 0 ? 1 : 0) : nux;
            for (int uk = u_lo; uk < u_hi; uk++) {
                // (workers start on different units: spread over channels)
                const int ui = u_lo + (uk - u_lo + j) % (u_hi - u_lo);
                const QxUnit &U = S.unit[ui];
                for (int q0 = 64 * cw; q0 < nr * ppi; q0 += 64 * QX_CPW) {
                    const int q = min(q0 + lane, nr * ppi - 1);
                    const uint8_t *src =
                        reinterpret_cast<const uint8_t *>(U.dw + (size_t)(j + a.W * (q >> lgppi)) * U.dwr) +
                        (q & (ppi - 1)) * PB;
                    __attribute__((address_space(3))) void *dst =
                        (__attribute__((address_space(3))) void *)(dW + ((size_t)ui * ustr + q0) * PB);
                    if (PB == 16) __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
                    else __builtin_amdgcn_global_load_lds(src, dst, 4, 0, 0);
                }
                for (int q0 = 64 * cw; q0 < nr * ngw; q0 += 64 * QX_CPW) {
                    const int q = min(q0 + lane, nr * ngw - 1);
                    const size_t ro = (size_t)(j + a.W * (q >> lgngw)) * U.dgr + (a.sb4 ? 2 : 1) * (q & (ngw - 1));
                    __attribute__((address_space(3))) void *ds_ =
                        (__attribute__((address_space(3))) void *)(dS + ui * sstr + q0);
                    __attribute__((address_space(3))) void *db_ =
                        (__attribute__((address_space(3))) void *)(dB + ui * sstr + q0);
                    if (a.sb4) {
                        __builtin_amdgcn_global_load_lds(U.ds + ro, ds_, 4, 0, 0);
                        __builtin_amdgcn_global_load_lds(U.db + ro, db_, 4, 0, 0);
                    } else {
                        __builtin_amdgcn_global_load_lds(U.ds + ro, ds_, 2, 0, 0);
                        __builtin_amdgcn_global_load_lds(U.db + ro, db_, 2, 0, 0);
                    }
                }
            }
        }
    };
#pragma unroll
    for (int i = 0; i < NRI; i++) gq[i] = -1;

    // The two roles run as separate branches with matching barriers (without
    // a fence: a fence would make every wave wait for all its loads in
    // flight), so that the gate/up waves' first LDS read waits only for their
    // own loads, not for copies into LDS on some other path.
    // The gate/up branch, instantiated for each way of bringing the scales
    // (the copies into LDS of the other way would make the compiler wait for
    // every load before the dots' first LDS read).
    auto gu_branch = [&](auto sb16c) {
        constexpr bool SB = decltype(sb16c)::value;
        const bool pre0 = wave < nq_sh;            // (instruction 0 is a shared row: rpi = 1)
        // pass A: the shared unit's table entry (its pointers need no routing), its rows
        if (nq_sh > 0) {
            if (threadIdx.x == 0) S.unit[0] = qx_unit(a, S, x);
            qx_barrier();
        }
        if (pre0) {
            if (SB) {
                uint4 v;
                int vq;
                sb_load((lane >> 4) == 0, v, vq);
                row_load(0);
                sb_store(v, vq);
            } else {
                row_load(0);
                sc_copy(0, 1);
            }
        }
        if constexpr (RES) stage_token();
        // the picks of this XCD's gatherer, polled by a wave with nothing in
        // flight (a poll waits for its wave's earlier loads): the last gate/up
        // wave, whose rows are not the shared unit's (nq_sh <= QX_GUW - 1)
        if (wave == QX_GUW - 1) {
            uint32_t v[1];
            qx_poll<1, false, QX_SLEEP_PICKS>(a, a.sync->loc[x].pick, K, v);
            // (clamped: after a wait that gave up the words are whatever was read)
            if (lane < K) S.pick[lane] = (int)min(v[0], (uint32_t)(a.m.E - 1));
        }
        qx_barrier();
        // the rest of the table (an XCD without units still fills entry 0, with
        // a valid unit: its gate/up waves issue their clamped loads through it
        // and drop them); the units' combine coefficients are set after
        // the gate/up, once the weights have come
        if ((int)threadIdx.x < max(nux, 1) && !(threadIdx.x == 0 && nq_sh > 0))
            S.unit[threadIdx.x] = qx_unit(a, S, min(x + 8 * (int)threadIdx.x, a.NU - 1));
        qx_barrier();      // the table is in LDS before pass B reads it
        QX_TS(1);
        // pass B
        if (pre0) gu_rest(std::true_type{}, sb16c);
        else gu_rest(std::false_type{}, sb16c);
    };
    if (wave < QX_GUW) {
        if (a.sb16) gu_branch(std::true_type{});
        else gu_branch(std::false_type{});
    } else {
        if (nq_sh > 0) {
            qx_barrier();
            issue_cp(0);
        }
        if constexpr (RES) stage_token();
        qx_barrier();
        qx_barrier();
        issue_cp(1);
        QX_TSW(QX_GUW, 10);
    }
    qx_barrier();          // (B2) every gate/up row result is in LDS (the down copies may be in flight)
    QX_TS(3);
    for (int t = threadIdx.x; t < np_; t += QX_THREADS)
        qx_put_near(a.sync->loc[x].act + j + a.W * t, a.epoch, __float_as_uint(qw_silu(ys[2 * t]) * ys[2 * t + 1]));

    // ---- the picks' weights and the shared gate (published after the ids),
    // then the XCD's activations, as q16 units ----
    if (wave == QX_WAVES - 1) {
        uint32_t v[1];
        qx_poll<1, false>(a, a.sync->loc[x].pick + K, K + 1, v);
        if (lane < K) S.coef[1 + lane] = __uint_as_float(v[0]);
        else if (lane == K) S.coef[0] = __uint_as_float(v[0]);
    }
    {
        const uint2 *src = a.sync->loc[x].act;
        for (int c0 = 64 * wave; c0 < rows_x; c0 += 64 * QX_WAVES) {
            uint32_t v[1];
            qx_poll<1, false>(a, src + c0, rows_x - c0, v);
            if (c0 + lane < rows_x) af[c0 + lane] = __uint_as_float(v[0]);
        }
    }
    qx_barrier();
    if ((int)threadIdx.x < nux) {
        const int u = x + 8 * threadIdx.x;
        S.unit[threadIdx.x].coef = u < a.nus ? S.coef[0] : S.coef[1 + min((u - a.nus) / a.nui, K - 1)];
    }
    QX_TS(4);
    for (int u = threadIdx.x; u < rows_x / 16; u += QX_THREADS) qw_q16_stage(af + 16 * u, xq + 3 * u);
    QX_TS(11);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's copies into LDS have landed
    QX_TSW(15, 12);
    __syncthreads();
    QX_TS(13);

    // ---- down dots, fused with this XCD's combine: lane (slot, dl) of wave w
    // holds local row (w + 16 m) spr + slot (output row j + W r) of every
    // unit, columns 16 dl ..
    // 16 dl + 15 of the unit's slice, and sums coef(unit) * its dot over the
    // units in order; NSU lanes then add their sums: P_x of the row ----
    {
        const int nsu = a.NSU, spr = 64 / nsu, slot = lane / nsu, dl = lane % nsu;
        const int gi = (16 * dl) >> a.lgG;                   // the lane's group within the slice
        const int hw = a.sb4 ? gi : 2 * gi;                  // as a bf16 index into the row's slots
        for (int r0 = wave * spr; r0 < nr; r0 += QX_WAVES * spr) {
            const int r = r0 + slot, rc = min(r, nr - 1);
            float acc = 0.0f;
            for (int ui = 0; ui < nux; ui++) {
                const uint4 *xu = xq + 3 * (ui * nsu + dl);
                const uint4 x0 = xu[0], x1 = xu[1], rr = xu[2];
                const uint32_t wo = (uint32_t)((ui * ustr + rc * ppi) * PB + 8 * dl);
                const uint2 wv = *reinterpret_cast<const uint2 *>(dW + wo);
                const uint32_t so = (uint32_t)(ui * sstr + rc * ngw);
                const uint32_t sv = reinterpret_cast<const uint16_t *>(dS + so)[hw];
                const uint32_t bv = reinterpret_cast<const uint16_t *>(dB + so)[hw];
                const float d = qw_unit_dot(wv, x0, x1, *reinterpret_cast<const float4 *>(&rr),
                                            __uint_as_float(sv << 16), __uint_as_float(bv << 16), 0.0f);
                acc = __builtin_fmaf(S.unit[ui].coef, d, acc);
            }
            acc = qx_run_sum(acc, nsu);
            if (dl == 0 && r < nr) {
                if (x < QX_NX - 1) qx_put_far(a.sync->part[x] + j + a.W * r, a.epoch, __float_as_uint(acc));
                else fp[(QX_NX - 1) * nr + r] = acc;
            }
        }
    }
    QX_TS(5);
    if (x < QX_NX - 1 || nr <= 0) return;
    // XCD 7: the other XCDs' partials of these rows (an XCD without units
    // contributes 0 and stores nothing)
    const int nxw = min(a.NU, QX_NX - 1);
    for (int c0 = 64 * wave; c0 < nxw * nr; c0 += 64 * QX_WAVES) {
        const int c = min(c0 + lane, nxw * nr - 1);
        const int xx = c / nr, r = c % nr;
        uint32_t v = 0u;
        const uint2 *pw = a.sync->part[xx] + j + a.W * r;
        for (int spins = 0;; spins++) {
            unsigned long long q[1] = {qx_ld_far(pw)};
            uint32_t e = qx_ld_err(a.sync);
            qx_wait<1>(q, e);
            v = (uint32_t)(q[0] >> 32);
            if (__ballot((uint32_t)q[0] != a.epoch) == 0ull) break;
            if (spins >= QX_SPIN_LIMIT || __ballot(e != 0u) != 0ull) {
                if (lane == 0) qx_raise(a.sync, a.epoch);
                break;
            }
            __builtin_amdgcn_s_sleep(QX_SLEEP_PART);
        }
        if (c0 + lane < nxw * nr) fp[c0 + lane] = __uint_as_float(v);
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nr; r += QX_THREADS) {
        float acc = nxw > 0 ? fp[r] : 0.0f;
        for (int xx = 1; xx < nxw; xx++) acc = acc + fp[xx * nr + r];
        a.out[j + a.W * r] = acc + fp[(QX_NX - 1) * nr + r];
    }
    QX_TS(6);
}

// ---- the kernel ---------------------------------------------------------------------

// Two 16-wave workgroups a CU: at most 64 VGPRs a wave.
template <int NUPL, int NRI, bool RES>
__global__ __launch_bounds__(QX_THREADS, 8) void k_decode1(QxArgs a)
{
    extern __shared__ uint4 lds[];
    __shared__ QxGatherLds G;
    __shared__ QxWorkLds S;
    QX_TS(0);
    const int b = blockIdx.x;
    if (b < a.n_rt) {
        qx_router<RES>(a, b, reinterpret_cast<float *>(lds), S.qpart);
        return;
    }
    // The XCD this workgroup runs on, as the hardware reports it: the
    // dispatcher deals a launch's workgroups to the 8 XCDs round-robin in
    // block order, but the XCD that takes block 0 differs from launch to
    // launch.  So 8 consecutive blocks sit on the 8 XCDs, and (block - first
    // worker) / 8 numbers the workers of each XCD 0..W-1.
    const int xcd = (int)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & (QX_NX - 1));   // HW_REG_XCC_ID
    if (b < a.n_rt + QX_NX) {
        qx_gather(a, xcd, G);
        return;
    }
    qx_worker<NUPL, NRI, RES>(a, xcd, (b - a.n_rt - QX_NX) / QX_NX, lds, S);
}

// ---- host side ------------------------------------------------------------------

struct QxPlan {
    int nupl, lrg, nri, W, SW, NSU, nus, nui, NU, rpw, pb, sb4, ngw, gsb4, lgSW, lgppi, lgngw, sb16, pre;
};

// The launch's shape for a layer, or false when the one-token launch does
// not take it.
static bool qx_plan(const qwk_moe *M, QxPlan *p)
{
    const int H = M->H, I = M->I, SI = M->SI, G = M->group, UH = H / 16;
    if (M->K < 1 || M->K > QWK_DECODE_MAX_K || M->E < M->K || M->E > QX_PL * 64) return false;
    if (H % 64 || H > QX_MAX_H || I % 16 || SI % 16 || I < 16 || SI < 16) return false;
    if (!(G == 32 || G == 64 || G == 128) || H % G || I % G || SI % G) return false;
    // gate/up lanes a row: whole 64-lane runs of units, or a power of two below
    if (UH >= 64 ? UH % 64 : (64 % UH)) return false;
    p->lrg = UH >= 64 ? 64 : UH;
    p->nupl = UH >= 64 ? UH / 64 : 1;
    if (p->nupl > 4) return false;
    // slice: the widest of 256, 128, 64, 32, 16 features dividing I and SI
    int sw = 256;
    while (sw > 16 && (I % sw || SI % sw)) sw /= 2;
    p->SW = sw;
    p->NSU = sw / 16;
    p->nus = SI / sw;
    p->nui = I / sw;
    p->NU = p->nus + M->K * p->nui;
    const int nux = (p->NU + 7) / 8;
    if (nux > QX_MAX_UX || nux * sw > QX_ACT_WORDS) return false;
    p->W = QX_W_MAX;
    const int P = (nux * sw + p->W - 1) / p->W;
    if (2 * P > 2 * QX_ACT_WORDS / QX_W_MAX + 64) return false;
    const int rpi = 64 / p->lrg;
    p->nri = (2 * P + QX_GUW * rpi - 1) / (QX_GUW * rpi);
    // registers: the gate/up weights a lane holds (the instantiated NRI)
    int nri_max = 0;
#define QX_MAXOF(N_, R_) if (p->nupl == N_) nri_max = R_;
    QX_NRI_OF(QX_MAXOF)
#undef QX_MAXOF
    if (p->nri > nri_max) return false;
    p->rpw = (H + p->W - 1) / p->W;
    // copies into LDS need aligned sources: 16 bytes where every down row
    // and slice starts on 16, else 4 (kin % 16 == 0 makes rows 8-byte
    // multiples); scales two groups a dword where rows hold even group counts
    p->pb = (sw / 2) % 16 == 0 && I % 32 == 0 && SI % 32 == 0 ? 16 : 4;
    p->sb4 = sw >= 2 * G && (I / G) % 2 == 0 && (SI / G) % 2 == 0;
    p->ngw = p->sb4 ? sw / (2 * G) : (sw >= G ? sw / G : 1);
    p->gsb4 = (H / G) % 2 == 0;
    if ((p->gsb4 ? H / G / 2 : H / G) > 64) return false;   // a gate/up row's scales: one copy instruction
    auto lg2 = [](int v) { int l = 0; while ((1 << l) < v) l++; return l; };
    p->lgSW = lg2(sw);
    p->lgppi = lg2(sw / 2 / p->pb);
    p->lgngw = lg2(p->ngw);
    // one row an instruction, a row's scales whole 16-byte runs (8 groups),
    // at most 8 runs, and the rows a wave holds in 16 lanes each
    p->sb16 = p->lrg == 64 && (H / G) % 8 == 0 && H / G <= 64 && p->nri <= 4 && p->gsb4;
    // the shared slices' rows ahead of the picks: at most one a XCD, and no
    // more rows a worker than leave the last gate/up wave free to poll
    p->pre = p->nus <= QX_NX && 2 * ((sw + p->W - 1) / p->W) <= QX_GUW - 1 && p->lrg == 64;
    if (qx_wlayout(UH, nux * sw, P, nux, p->rpw, qx_up64(p->rpw * (sw / 2 / p->pb)), p->pb, qx_up64(p->rpw * p->ngw),
                   p->gsb4 ? H / G / 2 : H / G).total > QX_LDS)
        return false;
    return true;
}

extern "C" int qwk_decode1_supported(const qwk_moe *M)
{
    QxPlan p;
    return qx_plan(M, &p);
}

extern "C" int qwk_moe_decode_supported(const qwk_moe *M, int rows)
{
    return (rows == 1 && qwk_decode1_supported(M)) || qwk_moe_decode_batch_supported(M, rows);
}

extern "C" size_t qwk_moe_decode_sync_bytes(void) { return sizeof(QxSync); }

extern "C" int qwk_decode_sync_words(void *sync, uint32_t **err, void **words, size_t *nwords)
{
    QxSync *S = static_cast<QxSync *>(sync);
    *err = &S->err;
    *words = S->part;
    *nwords = sizeof(S->part) / sizeof(S->part[0][0]);
    return 0;
}

extern "C" int qwk_moe_decode_sync_error(const void *sync, uint32_t *err)
{
    return (int)hipMemcpy(err, &static_cast<const QxSync *>(sync)->err, sizeof *err, hipMemcpyDeviceToHost);
}

extern "C" int qwk_moe_decode_sync_raise(void *sync, uint32_t epoch)
{
    return (int)hipMemcpy(&static_cast<QxSync *>(sync)->err, &epoch, sizeof epoch, hipMemcpyHostToDevice);
}

template <int NUPL, int NRI, bool RES>
static void qx_launch(hipStream_t s, const QxArgs &a, int grid, hipEvent_t e0, hipEvent_t e1)
{
    auto kern = k_decode1<NUPL, NRI, RES>;
    if (e0) hipExtLaunchKernelGGL(kern, dim3(grid), dim3(QX_THREADS), QX_LDS, s, e0, e1, 0, a);
    else hipLaunchKernelGGL(kern, dim3(grid), dim3(QX_THREADS), QX_LDS, s, a);
}

extern "C" int qwk_moe_decode(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                              const qwk_resid *res, const qwk_moe *M, void *sync, uint32_t epoch, hipEvent_t *ev)
{
    QxPlan p;
    if (!qx_plan(M, &p) || !sync || epoch == 0u) return (int)hipErrorInvalidValue;
    if (res ? (!res->h || !res->h_out || !res->x_out || ((uintptr_t)res->h & 7u) || ((uintptr_t)res->h_out & 7u) ||
               ((uintptr_t)res->y & 15u) || ((uintptr_t)res->x_out & 15u) ||
               (const void *)res->h_out == (const void *)res->h || (const void *)res->h_out == (const void *)res->y)
            : (!x || ((uintptr_t)x & 15u)))
        return (int)hipErrorInvalidValue;
    QxArgs a;
    a.m = *M;
    a.x = x;
    a.hin = res ? res->h : nullptr;
    a.yprev = res ? res->y : nullptr;
    a.hout = res ? res->h_out : nullptr;
    a.xout = res ? res->x_out : nullptr;
    a.eps = res ? res->eps : 0.0f;
    a.out = out;
    a.idx = idx;
    a.w = w;
    a.sync = static_cast<QxSync *>(sync);
    a.epoch = epoch;
    a.lgG = M->group == 32 ? 5 : M->group == 64 ? 6 : 7;
    a.n_rt = (M->E + 1 + QX_RT_ROWS - 1) / QX_RT_ROWS;
    a.W = p.W;
    a.SW = p.SW;
    a.NSU = p.NSU;
    a.nus = p.nus;
    a.nui = p.nui;
    a.NU = p.NU;
    a.lrg = p.lrg;
    a.nri = p.nri;
    a.rpw = p.rpw;
    a.pb = p.pb;
    a.sb4 = p.sb4;
    a.ngw = p.ngw;
    a.gsb4 = p.gsb4;
    a.lgSW = p.lgSW;
    a.lgppi = p.lgppi;
    a.lgngw = p.lgngw;
    a.sb16 = p.sb16;
    a.pre = p.pre;
    const int grid = a.n_rt + QX_NX + QX_NX * p.W;
    hipEvent_t e0 = ev ? ev[0] : 0, e1 = ev ? ev[1] : 0;
#define QX_GO(N_, R_)                                                      \
    if (p.nupl == N_) {                                                    \
        if (res) qx_launch<N_, R_, true>(s, a, grid, e0, e1);              \
        else qx_launch<N_, R_, false>(s, a, grid, e0, e1);                 \
        return (int)hipGetLastError();                                     \
    }
    QX_NRI_OF(QX_GO)
#undef QX_GO
    return (int)hipErrorInvalidValue;
}
