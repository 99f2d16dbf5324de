/* qwasar_hip.c -- the HIP backend behind qwasar_gpu.h for one MI355X.
 *
 * The reference's backend is qwasar_metal.m: Metal buffers in unified
 * memory, command buffers that run at commit, and a pipeline per kernel.  On
 * an MI355X the weights must sit in HBM and the host cannot cheaply read
 * device memory, so this backend differs in mechanism while keeping the
 * reference's contract:
 *
 *   qw_buf   a device allocation plus a host mirror (pinned, or the caller's
 *            memory for qw_buf_wrap).  Two flags say which side is stale.
 *            qw_buf_contents hands out the mirror and marks the device copy
 *            stale; an op that touches a stale buffer uploads it first.  An
 *            op that writes a buffer marks the mirror stale; qw_cmd_wait
 *            copies written buffers back if their mirror was ever handed out.
 *   qw_cmd   the backend's single in-order HIP stream plus this command's
 *            first error, its written buffers and its profiling events.  Ops
 *            launch as they are encoded (reference qwasar_metal.m:1606-1611
 *            encodes and runs at commit; both give encode-order execution).
 *   ops      each qw_op_* validates its shape, launches through the C ABI in
 *            qw_kernels.h, and records a launch failure as the command's
 *            error, reported by qw_cmd_error after qw_cmd_wait.
 *
 * Host code only: built with gcc against the HIP runtime's C API. */

#include "qwasar_gpu.h"
#include "qw_kernels.h"

#include <hip/hip_runtime_api.h>

#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

/* The MoE layer runs its experts grouped above QWK_DECODE_MAX_ROWS rows and
 * through the fused decode path at or below it (the reference switches at
 * 8 rows, qwasar_flash_graph.c:28; here a verify batch of 8 stays on the
 * decode path, which dedups expert reads across its tokens). */
/* Rows at or above which qw_op_qmat_q4 takes the MFMA product. */
#define QW_QMM_MIN_ROWS 8

struct qw_buf_s {
    void *host;
    void *dev;
    size_t len;
    int owns_host;   /* host mirror allocated here (pinned, at the first qw_buf_contents) */
    int host_stale;  /* device holds newer data */
    int dev_stale;   /* host mirror may hold newer data */
    int exposed;     /* qw_buf_contents was called (or the memory is the caller's) */
};

typedef struct { const char *label; hipEvent_t a, b; } qw_mark;

struct qw_cmd_s {
    hipError_t err;
    char msg[256];
    qw_buf *written;
    int nwritten, capwritten;
    qw_mark *marks;
    int nmarks, capmarks;
    hipEvent_t *evs;         /* every event this command created */
    int nevs, capevs;
    hipEvent_t last;         /* where the next mark starts */
    uint32_t ep_hi[2];       /* per hand-off state: the last decode epoch this command launched (0: none unchecked) */
    struct qw_cmd_s *next;   /* live commands, for qw_buf_free */
};

static struct {
    int ready;
    int device;
    hipStream_t stream;
    char name[320];
    uint64_t free0, total;
    int prof;
    qw_cmd live;
    void *scratch;
    size_t scratch_len;
    /* The decode launch's hand-off states: [QW_DS_HEAP] allocated at first
     * use, [QW_DS_STATIC] at the head of the static device array that the
     * allocation-free entry uses (its staging follows it there). */
    struct { void *sync; uint32_t epoch; } ds[2];
    char *static_stage;   /* the static array past its hand-off state */
    size_t static_stage_len;
} G;

#define QW_DS_HEAP 0
#define QW_DS_STATIC 1

/* places in a command's written list from qw_cmd_begin (the list grows past
 * them for every op but the allocation-free one) */
#define QW_CMD_FIXED_WRITTEN 16

/* ---- profiling table ---------------------------------------------------- */

#define QW_PROF_MAX 64
static struct { const char *label; double ms; int64_t count; } P[QW_PROF_MAX];
static int NP;

/* every mark's own duration, in completion order, since the last reset (the
 * first QW_PROF_KEEP): what a median over steps is taken from */
#define QW_PROF_KEEP 8192
static struct { const char *label; float ms; } PK[QW_PROF_KEEP];
static int NPK;

static void prof_add(const char *label, double ms) {
    if (NPK < QW_PROF_KEEP) { PK[NPK].label = label; PK[NPK].ms = (float)ms; NPK++; }
    for (int i = 0; i < NP; i++)
        if (P[i].label == label || !strcmp(P[i].label, label)) { P[i].ms += ms; P[i].count++; return; }
    if (NP < QW_PROF_MAX) { P[NP].label = label; P[NP].ms = ms; P[NP].count = 1; NP++; }
}

bool qw_prof_enabled(void) { return G.prof != 0; }
void qw_prof_set_enabled(bool on) { G.prof = on ? 1 : 0; }
void qw_prof_reset(void) { NP = 0; NPK = 0; }

/* Not in the reference interface: the individual durations of `label`'s
 * marks since the last reset, oldest first, up to cap; returns how many. */
int32_t qw_prof_mark_times(const char *label, float *ms, int32_t cap) {
    int32_t n = 0;
    for (int i = 0; i < NPK && n < cap; i++)
        if (PK[i].label == label || !strcmp(PK[i].label, label)) ms[n++] = PK[i].ms;
    return n;
}

double qw_prof_ms(const char *label, int64_t *count) {
    for (int i = 0; i < NP; i++)
        if (!strcmp(P[i].label, label)) { if (count) *count = P[i].count; return P[i].ms; }
    if (count) *count = 0;
    return 0.0;
}

void qw_prof_report(FILE *out, long tokens) {
    double total = 0.0;
    for (int i = 0; i < NP; i++) total += P[i].ms;
    if (!out || total <= 0.0) return;
    fprintf(out, "qwasar profile (%s, %ld tokens):\n", G.name, tokens);
    for (int i = 0; i < NP; i++)
        fprintf(out, "  %-28s %9.4f ms/token %5.1f%%  (%lld marks)\n", P[i].label,
                tokens > 0 ? P[i].ms / (double)tokens : P[i].ms, 100.0 * P[i].ms / total,
                (long long)P[i].count);
}

/* The hand-off state's size, rounded up to the fill kernel's 16 bytes (and
 * allocated at that size). */
static size_t dsync_bytes(void) { return (qwk_moe_decode_sync_bytes() + 15) & ~(size_t)15; }

/* ---- device --------------------------------------------------------------- */

bool qw_gpu_init(char *err, size_t errcap) {
    if (G.ready) return true;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        if (err && errcap) snprintf(err, errcap, "no HIP device");
        return false;
    }
    hipDeviceProp_t prop;
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        if (err && errcap) snprintf(err, errcap, "cannot open HIP device 0");
        return false;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (err && errcap) snprintf(err, errcap, "device is %s; kernels are built for gfx950", prop.gcnArchName);
        return false;
    }
    if (hipStreamCreateWithFlags(&G.stream, hipStreamNonBlocking) != hipSuccess) {
        if (err && errcap) snprintf(err, errcap, "cannot create a HIP stream");
        return false;
    }
    /* The static device array of the allocation-free decode entry: its
     * address on this device, once, and zeroed.  Without it that entry
     * refuses; everything else works. */
    {
        size_t sb = 0;
        char *sp = qwk_static_init(G.stream) == 0 ? qwk_static_scratch(&sb) : NULL;
        const size_t hs = (qwk_moe_decode_sync_bytes() + 255) & ~(size_t)255;
        /* the hand-off state is zeroed on every init: epochs restart at 1,
         * so words and an error left by an earlier session must not survive */
        if (sp && sb > hs && qwk_zero_fill(G.stream, sp, dsync_bytes()) == 0 &&
            hipStreamSynchronize(G.stream) == hipSuccess) {
            G.ds[QW_DS_STATIC].sync = sp;
            G.ds[QW_DS_STATIC].epoch = 0;
            G.static_stage = sp + hs;
            G.static_stage_len = sb - hs;
        }
    }
    size_t fr = 0, tot = 0;
    (void)hipMemGetInfo(&fr, &tot);
    G.free0 = fr;
    G.total = tot;
    snprintf(G.name, sizeof G.name, "%.200s (%.64s)", prop.name, prop.gcnArchName);
    const char *pe = getenv("QWASAR_PROFILE");
    G.prof = pe && *pe && strcmp(pe, "0") != 0;
    G.device = 0;
    G.ready = 1;
    return true;
}

static int ensure_init(void) {
    if (G.ready) return 1;
    char e[128];
    if (!qw_gpu_init(e, sizeof e)) { fprintf(stderr, "qwasar: %s\n", e); return 0; }
    return 1;
}

void qw_gpu_shutdown(void) {
    if (!G.ready) return;
    hipStreamSynchronize(G.stream);
    if (G.scratch) hipFree(G.scratch);
    G.scratch = NULL;
    G.scratch_len = 0;
    if (G.ds[QW_DS_HEAP].sync) hipFree(G.ds[QW_DS_HEAP].sync);
    G.ds[QW_DS_HEAP].sync = NULL;
    G.ds[QW_DS_STATIC].sync = NULL;   /* the static array stays with the process */
    hipStreamDestroy(G.stream);
    G.ready = 0;
}

const char *qw_gpu_name(void) { return G.ready ? G.name : "none"; }
uint64_t qw_gpu_working_set_limit(void) { return G.free0; }
uint64_t qw_gpu_max_buffer_length(void) { return G.total; }

/* ---- buffers --------------------------------------------------------------- */

qw_buf qw_buf_alloc(size_t len) {
    if (!ensure_init()) return NULL;
    qw_buf b = calloc(1, sizeof *b);
    if (!b) return NULL;
    const size_t n = len ? len : 1;
    if (hipMalloc(&b->dev, n) != hipSuccess) { free(b); return NULL; }
    /* The pinned mirror waits for the first qw_buf_contents, so buffers the
     * host never reads (weights filled on the device) cost no host memory. */
    hipMemsetAsync(b->dev, 0, n, G.stream);
    hipStreamSynchronize(G.stream);
    b->len = len;
    b->owns_host = 1;
    return b;
}

/* For the checkpoint loader (qw_load.c), not exported: a device buffer
 * holding `len` bytes copied from host memory the caller keeps. */
__attribute__((visibility("hidden"))) qw_buf qw_buf_from_bytes_(const void *src, size_t len) {
    qw_buf b = qw_buf_alloc(len);
    if (b && len && hipMemcpy(b->dev, src, len, hipMemcpyHostToDevice) != hipSuccess) {
        qw_buf_free(b);
        return NULL;
    }
    if (b) b->host_stale = 1;   /* the device copy is the data */
    return b;
}

qw_buf qw_buf_wrap(void *ptr, size_t len) {
    if (!ensure_init() || !ptr) return NULL;
    qw_buf b = calloc(1, sizeof *b);
    if (!b) return NULL;
    if (hipMalloc(&b->dev, len ? len : 1) != hipSuccess) { free(b); return NULL; }
    if (len && hipMemcpy(b->dev, ptr, len, hipMemcpyHostToDevice) != hipSuccess) {
        hipFree(b->dev);
        free(b);
        return NULL;
    }
    b->host = ptr;
    b->len = len;
    b->exposed = 1;
    return b;
}

void qw_buf_free(qw_buf b) {
    if (!b) return;
    for (qw_cmd c = G.live; c; c = c->next)
        for (int i = 0; i < c->nwritten; i++)
            if (c->written[i] == b) c->written[i] = c->written[--c->nwritten];
    hipStreamSynchronize(G.stream);
    hipFree(b->dev);
    if (b->owns_host && b->host) hipHostFree(b->host);
    free(b);
}

void *qw_buf_contents(qw_buf b) {
    if (!b) return NULL;
    if (!b->host) {
        const size_t n = b->len ? b->len : 1;
        if (hipHostMalloc(&b->host, n, hipHostMallocDefault) != hipSuccess) { b->host = NULL; return NULL; }
        if (!b->host_stale) memset(b->host, 0, n);   /* nothing has written the device copy */
    }
    if (b->host_stale) {
        hipStreamSynchronize(G.stream);
        hipMemcpy(b->host, b->dev, b->len, hipMemcpyDeviceToHost);
        b->host_stale = 0;
    }
    b->dev_stale = 1;
    b->exposed = 1;
    return b->host;
}

size_t qw_buf_length(qw_buf b) { return b ? b->len : 0; }

/* ---- commands ---------------------------------------------------------------- */

/* A new event owned by the command, optionally recorded on the stream now. */
static hipEvent_t cmd_event(qw_cmd c, int record) {
    hipEvent_t e = NULL;
    if (hipEventCreate(&e) != hipSuccess) return NULL;
    if (c->nevs == c->capevs) {
        c->capevs = c->capevs ? 2 * c->capevs : 16;
        c->evs = realloc(c->evs, (size_t)c->capevs * sizeof *c->evs);
    }
    c->evs[c->nevs++] = e;
    if (record) hipEventRecord(e, G.stream);
    return e;
}

static void cmd_add_mark(qw_cmd c, const char *label, hipEvent_t a, hipEvent_t b) {
    if (!a || !b) return;
    if (c->nmarks == c->capmarks) {
        c->capmarks = c->capmarks ? 2 * c->capmarks : 16;
        c->marks = realloc(c->marks, (size_t)c->capmarks * sizeof *c->marks);
    }
    c->marks[c->nmarks].label = label;
    c->marks[c->nmarks].a = a;
    c->marks[c->nmarks].b = b;
    c->nmarks++;
}

qw_cmd qw_cmd_begin(void) {
    if (!ensure_init()) return NULL;
    qw_cmd c = calloc(1, sizeof *c);
    if (!c) return NULL;
    /* the written list starts with room for QW_CMD_FIXED_WRITTEN buffers, so
     * the allocation-free entry can record its outputs without growing it */
    c->written = malloc(QW_CMD_FIXED_WRITTEN * sizeof *c->written);
    if (!c->written) { free(c); return NULL; }
    c->capwritten = QW_CMD_FIXED_WRITTEN;
    c->next = G.live;
    G.live = c;
    if (G.prof) c->last = cmd_event(c, 1);
    return c;
}

static void cmd_fail(qw_cmd c, hipError_t e, const char *fmt, ...) {
    if (!c || c->err != hipSuccess) return;
    c->err = e == hipSuccess ? hipErrorUnknown : e;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(c->msg, sizeof c->msg, fmt, ap);
    va_end(ap);
}

/* Makes the device copy of r's buffer current; notes it as written. */
static void touch(qw_cmd c, qw_ref r, int writes) {
    qw_buf b = r.buf;
    if (!b) return;
    if (b->dev_stale) {
        hipMemcpyAsync(b->dev, b->host, b->len, hipMemcpyHostToDevice, G.stream);
        hipStreamSynchronize(G.stream);
        b->dev_stale = 0;
    }
    if (!writes) return;
    b->host_stale = 1;
    for (int i = 0; i < c->nwritten; i++) if (c->written[i] == b) return;
    if (c->nwritten == c->capwritten) {
        c->capwritten = c->capwritten ? 2 * c->capwritten : 16;
        c->written = realloc(c->written, (size_t)c->capwritten * sizeof *c->written);
    }
    c->written[c->nwritten++] = b;
}

static void *dp(qw_ref r) { return r.buf ? (char *)r.buf->dev + r.off : NULL; }

/* touch() that never grows the command's written list: a written buffer is
 * recorded only while the list has room (qw_cmd_begin gives it
 * QW_CMD_FIXED_WRITTEN places), so qw_cmd_wait copies it back as it does for
 * every other op.  Returns 0 when the list is full.  For the
 * allocation-free entry. */
static int touch_fixed(qw_cmd c, qw_ref r, int writes) {
    qw_buf b = r.buf;
    if (!b) return 1;
    if (b->dev_stale) {
        hipMemcpyAsync(b->dev, b->host, b->len, hipMemcpyHostToDevice, G.stream);
        hipStreamSynchronize(G.stream);
        b->dev_stale = 0;
    }
    if (!writes) return 1;
    b->host_stale = 1;
    for (int i = 0; i < c->nwritten; i++) if (c->written[i] == b) return 1;
    if (c->nwritten >= c->capwritten) return 0;
    c->written[c->nwritten++] = b;
    return 1;
}


/* A decode hand-off state: the heap one is allocated on first use; both are
 * zeroed (epochs restarting at 1) at first use, after a launch reported an
 * error and before an epoch would repeat.  Zeroed by a fill kernel. */

static int dsync_reset(int k) {
    hipStreamSynchronize(G.stream);
    if (!G.ds[k].sync) {
        if (k == QW_DS_STATIC) return 0;   /* set up at init or not at all */
        if (hipMalloc(&G.ds[k].sync, dsync_bytes()) != hipSuccess) {
            G.ds[k].sync = NULL;
            return 0;
        }
    }
    if (qwk_zero_fill(G.stream, G.ds[k].sync, dsync_bytes()) != 0 ||
        hipStreamSynchronize(G.stream) != hipSuccess)
        return 0;
    G.ds[k].epoch = 0;
    return 1;
}

/* With the stream drained: reads state k's error word, which holds the
 * epoch of the first decode launch whose wait gave up.  That launch and
 * every later one on the state failed, so every live command that launched
 * an epoch at or after it is failed, whichever command is waiting.  Then the
 * state is zeroed and, every launch so far being checked, the commands'
 * epoch marks for it are cleared.  Returns 0 when the state could not be
 * read or zeroed. */
static int dsync_check(int k, int force_reset) {
    if (!G.ds[k].sync) return 1;
    int pending = force_reset;
    for (qw_cmd q = G.live; q; q = q->next) pending |= q->ep_hi[k] != 0;
    if (!pending) return 1;
    uint32_t first = 0;
    if (qwk_moe_decode_sync_error(G.ds[k].sync, &first) != 0) first = 1;   /* unreadable: fail them all */
    if (first != 0)
        for (qw_cmd q = G.live; q; q = q->next)
            if (q->ep_hi[k] >= first)
                cmd_fail(q, hipErrorLaunchFailure,
                         "decode: a hand-off wait gave up (launch %u of this state)", first);
    for (qw_cmd q = G.live; q; q = q->next) q->ep_hi[k] = 0;
    return first != 0 || force_reset ? dsync_reset(k) : 1;
}

/* For tests of the failure path: the hand-off error word is set as if the
 * next decode launch's first wait had given up, so every wait of that launch
 * and of later ones gives up at once (each kernel still runs to its end) and
 * the waiting command reports the failure. */
bool qw_debug_decode_handoff_fail(void) {
    if (!ensure_init()) return false;
    if (!G.ds[QW_DS_HEAP].sync && !dsync_reset(QW_DS_HEAP)) return false;
    hipStreamSynchronize(G.stream);
    return qwk_moe_decode_sync_raise(G.ds[QW_DS_HEAP].sync, G.ds[QW_DS_HEAP].epoch + 1u) == 0;
}

/* Launch result of one op: a refusal (invalid shape) is printed, as the
 * reference prints unsupported shapes; either kind becomes the error. */
static void launched(qw_cmd c, const char *op, int rc) {
    if (rc == 0) return;
    if (rc == (int)hipErrorInvalidValue) fprintf(stderr, "qwasar: %s: shape or alignment unsupported\n", op);
    cmd_fail(c, (hipError_t)rc, "%s: %s", op, hipGetErrorString((hipError_t)rc));
}

void qw_cmd_commit(qw_cmd c) { (void)c; }
void qw_cmd_flush(qw_cmd c) { (void)c; }
void qw_cmd_parallel(qw_cmd c, bool on) { (void)c; (void)on; }

void qw_cmd_mark(qw_cmd c, const char *label) {
    if (!c || !G.prof) return;
    hipEvent_t e = cmd_event(c, 1);
    if (c->last) cmd_add_mark(c, label, c->last, e);
    c->last = e;
}

void qw_cmd_wait(qw_cmd c) {
    if (!c) return;
    hipError_t e = hipStreamSynchronize(G.stream);
    if (e != hipSuccess) cmd_fail(c, e, "device: %s", hipGetErrorString(e));
    dsync_check(QW_DS_HEAP, 0);
    dsync_check(QW_DS_STATIC, 0);
    for (int i = 0; i < c->nwritten; i++) {
        qw_buf b = c->written[i];
        if (b->exposed && b->host_stale) {
            hipMemcpy(b->host, b->dev, b->len, hipMemcpyDeviceToHost);
            b->host_stale = 0;
        }
    }
    c->nwritten = 0;
    for (int i = 0; i < c->nmarks; i++) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, c->marks[i].a, c->marks[i].b) == hipSuccess)
            prof_add(c->marks[i].label, ms);
    }
    c->nmarks = 0;
    /* Keep only the event the next mark starts from. */
    int kept = 0;
    for (int i = 0; i < c->nevs; i++) {
        if (c->evs[i] == c->last) c->evs[kept++] = c->evs[i];
        else hipEventDestroy(c->evs[i]);
    }
    c->nevs = kept;
}

const char *qw_cmd_error(qw_cmd c) { return c && c->err != hipSuccess ? c->msg : NULL; }

void qw_cmd_free(qw_cmd c) {
    if (!c) return;
    for (qw_cmd *pp = &G.live; *pp; pp = &(*pp)->next)
        if (*pp == c) { *pp = c->next; break; }
    for (int i = 0; i < c->nevs; i++) hipEventDestroy(c->evs[i]);
    free(c->evs);
    free(c->marks);
    free(c->written);
    free(c);
}

qw_residency qw_residency_new(qw_buf *bufs, int32_t n) { (void)bufs; (void)n; return NULL; }
void qw_residency_free(qw_residency r) { (void)r; }

/* ---- ops ------------------------------------------------------------------- */

#define QW_OP(c) if (!(c)) return

static qwk_q4 q4(qw_ref w, qw_ref s, qw_ref b) {
    qwk_q4 m = { (const uint32_t *)dp(w), (const uint16_t *)dp(s), (const uint16_t *)dp(b) };
    return m;
}

void qw_op_qmv_q4(qw_cmd c, qw_ref y, qw_ref x, qw_ref w, qw_ref scales, qw_ref biases,
                  int32_t k, int32_t n, int32_t rows, int32_t group) {
    QW_OP(c);
    touch(c, x, 0); touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0); touch(c, y, 1);
    const qwk_q4 m = q4(w, scales, biases);
    launched(c, "qmv_q4", qwk_q4mv(G.stream, dp(y), dp(x), NULL, k, NULL, &m, 1, k, n, rows, 1, 1, group));
}

void qw_op_qmvb_q4(qw_cmd c, qw_ref y, qw_ref x, qw_ref w, qw_ref scales, qw_ref biases,
                   int32_t k, int32_t n, int32_t rows, int32_t group) {
    qw_op_qmv_q4(c, y, x, w, scales, biases, k, n, rows, group);
}

/* The backend's device scratch, grown on demand (defined below). */
static void *scratch(size_t bytes);

void qw_op_qmm_q4(qw_cmd c, qw_ref y, qw_ref x, qw_ref w, qw_ref scales, qw_ref biases,
                  int32_t k, int32_t n, int32_t rows, int32_t group) {
    QW_OP(c);
    touch(c, x, 0); touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0); touch(c, y, 1);
    const size_t wb = qwk_qmm_work_bytes(k, n, rows);
    void *work = wb ? scratch(wb) : NULL;
    launched(c, "qmm_q4", qwk_qmm(G.stream, dp(y), dp(x), q4(w, scales, biases), k, n, rows, group, work,
                                  work ? wb : 0));
}

void qw_op_qmat_q4(qw_cmd c, qw_ref y, qw_ref x, qw_ref w, qw_ref scales, qw_ref biases,
                   int32_t k, int32_t n, int32_t rows, int32_t group) {
    if (rows >= QW_QMM_MIN_ROWS && k % 32 == 0)
        qw_op_qmm_q4(c, y, x, w, scales, biases, k, n, rows, group);
    else
        qw_op_qmv_q4(c, y, x, w, scales, biases, k, n, rows, group);
}

bool qw_op_qmv_q4_multi(qw_cmd c, qw_ref x, int32_t k, int32_t group, int32_t count,
                        const qw_qmv_part *parts) {
    /* The reference's contract (qwasar_gpu.h:105-107): one to four parts
     * over an input of at least 2048, else false and nothing encoded; its
     * caller then falls back to one qmv per part. */
    if (count < 1 || count > 4 || k < 2048) return false;
    if (!c) return true;
    if (!parts) return false;
    qwk_q4 m[4];
    float *ys[4];
    int ns[4];
    touch(c, x, 0);
    for (int32_t i = 0; i < count; i++) {
        touch(c, parts[i].w, 0); touch(c, parts[i].scales, 0); touch(c, parts[i].biases, 0);
        touch(c, parts[i].y, 1);
        m[i] = q4(parts[i].w, parts[i].scales, parts[i].biases);
        ys[i] = dp(parts[i].y);
        ns[i] = parts[i].n;
    }
    const int rc = qwk_q4mv_multi(G.stream, dp(x), k, group, count, m, ys, ns);
    launched(c, "qmv_q4_multi", rc);
    return rc == 0;
}

void qw_op_dmat_bf16(qw_cmd c, qw_ref y, qw_ref x, qw_ref w, int32_t k, int32_t n, int32_t rows) {
    QW_OP(c);
    touch(c, x, 0); touch(c, w, 0); touch(c, y, 1);
    launched(c, "dmat_bf16", qwk_dmat_bf16(G.stream, dp(y), dp(x), dp(w), k, n, rows));
}

void qw_op_swiglu(qw_cmd c, qw_ref y, qw_ref gate, qw_ref up, int32_t n) {
    QW_OP(c);
    touch(c, gate, 0); touch(c, up, 0); touch(c, y, 1);
    launched(c, "swiglu", qwk_swiglu(G.stream, dp(y), dp(gate), dp(up), n));
}

void qw_op_add_inplace(qw_cmd c, qw_ref y, qw_ref x, int32_t n) {
    QW_OP(c);
    touch(c, x, 0); touch(c, y, 1);
    launched(c, "add_inplace", qwk_add_inplace(G.stream, dp(y), dp(x), n));
}

void qw_op_rms_norm(qw_cmd c, qw_ref y, qw_ref x, qw_ref weight,
                    int32_t dim, int32_t rows, float eps, float out_scale) {
    QW_OP(c);
    touch(c, x, 0); touch(c, weight, 0); touch(c, y, 1);
    launched(c, "rms_norm", qwk_rms_norm(G.stream, dp(y), dp(x), dp(weight), dim, rows, eps, out_scale));
}

void qw_op_residual_rms_norm_bf16(qw_cmd c, qw_ref h, qw_ref x, qw_ref y, int32_t dim, int32_t rows, float eps) {
    QW_OP(c);
    touch(c, y, 0); touch(c, h, 1); touch(c, x, 1);
    launched(c, "residual_rms_norm_bf16", qwk_resid_rms_bf16(G.stream, dp(h), dp(h), dp(x), dp(y), dim, rows, eps));
}

/* ---- the hyper-connection mixer (reference qwasar_gpu.h:549-578) ------------ */

void qw_op_repeat_cols(qw_cmd c, qw_ref h4, qw_ref x, int32_t rows, int32_t H, int32_t S) {
    QW_OP(c);
    touch(c, x, 0); touch(c, h4, 1);
    launched(c, "repeat_cols", qwk_repeat_cols(G.stream, dp(h4), dp(x), rows, H, S));
}

void qw_op_rms_norm_grouped(qw_cmd c, qw_ref y, qw_ref x, qw_ref weight,
                            int32_t dim, int32_t groups, int32_t rows, float eps) {
    QW_OP(c);
    touch(c, x, 0); touch(c, weight, 0); touch(c, y, 1);
    launched(c, "rms_norm_grouped", qwk_rms_norm_grouped(G.stream, dp(y), dp(x), dp(weight), dim, groups, rows, eps));
}

void qw_op_hc_inject_norm(qw_cmd c, qw_ref h4, qw_ref out, qw_ref inj, qw_ref w, qw_ref n4,
                          int32_t rows, int32_t H, int32_t S, float eps) {
    QW_OP(c);
    touch(c, out, 0); touch(c, inj, 0); touch(c, w, 0); touch(c, h4, 1); touch(c, n4, 1);
    launched(c, "hc_inject_norm", qwk_hc_inject_norm(G.stream, dp(h4), dp(out), dp(inj), dp(w), dp(n4), rows, H, S, eps));
}

bool qw_op_hc_mix_up(qw_cmd c, qw_ref x, qw_ref d, qw_ref n4, qw_ref w, qw_ref scales, qw_ref biases,
                     int32_t k, int32_t H, int32_t S, int32_t rows, float scale, int32_t group) {
    if (S < 1 || S > 4) return false;
    if (!c) return true;
    touch(c, d, 0); touch(c, n4, 0); touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0); touch(c, x, 1);
    const int rc = qwk_hc_mix_up(G.stream, dp(x), dp(d), dp(n4), dp(w), dp(scales), dp(biases), k, H, S, rows,
                                 scale, group);
    launched(c, "hc_mix_up", rc);
    return rc == 0;
}

/* Whether [a, a + la) and [b, b + lb) share a byte of one buffer. */
static bool refs_overlap(qw_ref a, size_t la, qw_ref b, size_t lb) {
    return a.buf && a.buf == b.buf && a.off < b.off + lb && b.off < a.off + la;
}

bool qw_op_hc_pre_decode(qw_cmd c, qw_ref h4_out, qw_ref n4, qw_ref d, qw_ref inj_out, qw_ref h4, qw_ref out,
                         qw_ref inj, qw_ref norm_w, qw_ref down_w, qw_ref down_s, qw_ref down_b, qw_ref inj_w,
                         int32_t H, int32_t S, int32_t lowrank, int32_t group, float eps) {
    const int32_t HH = S * H;
    if (H < 4 || H % 4 || S < 1 || S > 4 || HH % 64 || HH > 15360 || lowrank < 1 || HH % group ||
        (group != 32 && group != 64 && group != 128))
        return false;
    /* Every workgroup reads all of h4, out and inj while others write the
     * outputs, so no output may share a byte with an input or another output. */
    const qw_ref outs[4] = { h4_out, n4, d, inj_out }, ins[3] = { h4, out, inj };
    const size_t lo[4] = { 4u * (size_t)HH, 4u * (size_t)HH, 4u * (size_t)lowrank, 4u * (size_t)S };
    const size_t li[3] = { 4u * (size_t)HH, 4u * (size_t)H, 4u * (size_t)S };
    for (int i = 0; i < 4; i++) {
        for (int j = 0; j < 3; j++) if (refs_overlap(outs[i], lo[i], ins[j], li[j])) return false;
        for (int j = i + 1; j < 4; j++) if (refs_overlap(outs[i], lo[i], outs[j], lo[j])) return false;
    }
    if (!c) return true;
    touch(c, h4, 0); touch(c, out, 0); touch(c, inj, 0); touch(c, norm_w, 0);
    touch(c, down_w, 0); touch(c, down_s, 0); touch(c, down_b, 0); touch(c, inj_w, 0);
    touch(c, h4_out, 1); touch(c, n4, 1); touch(c, d, 1); touch(c, inj_out, 1);
    const int rc = qwk_hc_pre_decode(G.stream, dp(h4_out), dp(n4), dp(d), dp(inj_out), dp(h4), dp(out), dp(inj),
                                     dp(norm_w), q4(down_w, down_s, down_b), dp(inj_w), H, S, lowrank, group, eps);
    launched(c, "hc_pre_decode", rc);
    return rc == 0;
}

bool qw_op_hc_decode(qw_cmd c, qw_ref x, qw_ref h4_out, qw_ref n4, qw_ref d, qw_ref inj_out, qw_ref h4,
                     qw_ref out, qw_ref inj, qw_ref norm_w, qw_ref down_w, qw_ref down_s, qw_ref down_b,
                     qw_ref inj_w, qw_ref up_w, qw_ref up_s, qw_ref up_b, int32_t H, int32_t S, int32_t lowrank,
                     int32_t group, float eps, float scale) {
    const int32_t HH = S * H;
    if (H < 4 || H % 4 || S < 1 || S > 4 || HH % 64 || HH > 15360 || lowrank < 8 || lowrank > 512 ||
        lowrank % 8 || (group != 32 && group != 64 && group != 128) || HH % group || lowrank % group)
        return false;
    /* as qw_op_hc_pre_decode: no output shares a byte with an input or
     * another output (x included) */
    const qw_ref outs[5] = { h4_out, n4, d, inj_out, x }, ins[3] = { h4, out, inj };
    const size_t lo[5] = { 4u * (size_t)HH, 4u * (size_t)HH, 4u * (size_t)lowrank, 4u * (size_t)S, 4u * (size_t)H };
    const size_t li[3] = { 4u * (size_t)HH, 4u * (size_t)H, 4u * (size_t)S };
    for (int i = 0; i < 5; i++) {
        for (int j = 0; j < 3; j++) if (refs_overlap(outs[i], lo[i], ins[j], li[j])) return false;
        for (int j = i + 1; j < 5; j++) if (refs_overlap(outs[i], lo[i], outs[j], lo[j])) return false;
    }
    if (!c) return true;
    touch(c, h4, 0); touch(c, out, 0); touch(c, inj, 0); touch(c, norm_w, 0);
    touch(c, down_w, 0); touch(c, down_s, 0); touch(c, down_b, 0); touch(c, inj_w, 0);
    touch(c, up_w, 0); touch(c, up_s, 0); touch(c, up_b, 0);
    touch(c, h4_out, 1); touch(c, n4, 1); touch(c, d, 1); touch(c, inj_out, 1); touch(c, x, 1);
    /* the decode hand-off state and its epochs, shared with the MoE decode
     * launch (stream order keeps them apart) */
    const int k = QW_DS_HEAP;
    if (!G.ds[k].sync && !dsync_reset(k)) {
        cmd_fail(c, hipErrorOutOfMemory, "hc_decode: decode hand-off state");
        return false;
    }
    if (G.ds[k].epoch == UINT32_MAX && !dsync_check(k, 1)) {
        cmd_fail(c, hipErrorUnknown, "hc_decode: decode hand-off state");
        return false;
    }
    uint32_t *err = NULL;
    void *words = NULL;
    size_t nwords = 0;
    qwk_decode_sync_words(G.ds[k].sync, &err, &words, &nwords);
    if (nwords < qwk_hc_decode_tag_words()) {
        cmd_fail(c, hipErrorInvalidValue, "hc_decode: hand-off state too small");
        return false;
    }
    const uint32_t epoch = ++G.ds[k].epoch;
    const int rc = qwk_hc_decode(G.stream, dp(x), dp(h4_out), dp(n4), dp(d), dp(inj_out), dp(h4), dp(out), dp(inj),
                                 dp(norm_w), q4(down_w, down_s, down_b), dp(inj_w), q4(up_w, up_s, up_b), H, S,
                                 lowrank, group, eps, scale, err, words, epoch);
    c->ep_hi[k] = epoch;
    launched(c, "hc_decode", rc);
    return rc == 0;
}

void qw_op_silu_scale(qw_cmd c, qw_ref y, int32_t n, float scale) {
    QW_OP(c);
    touch(c, y, 1);
    launched(c, "silu_scale", qwk_silu_scale(G.stream, dp(y), n, scale));
}

void qw_op_hc_mix(qw_cmd c, qw_ref x, qw_ref n, qw_ref m, int32_t rows, int32_t H, int32_t S) {
    QW_OP(c);
    touch(c, n, 0); touch(c, m, 0); touch(c, x, 1);
    launched(c, "hc_mix", qwk_hc_mix(G.stream, dp(x), dp(n), dp(m), rows, H, S));
}

void qw_op_hc_inject(qw_cmd c, qw_ref h4, qw_ref out, qw_ref inj, int32_t rows, int32_t H, int32_t S) {
    QW_OP(c);
    touch(c, out, 0); touch(c, inj, 0); touch(c, h4, 1);
    launched(c, "hc_inject", qwk_hc_inject(G.stream, dp(h4), dp(out), dp(inj), rows, H, S));
}

void qw_op_synth(qw_cmd c, qw_ref dst, int32_t kind, int64_t n, uint64_t key, float a, float b) {
    QW_OP(c);
    touch(c, dst, 1);
    launched(c, "synth", qwk_synth(G.stream, dp(dst), kind, n, key, a, b));
}

void qw_op_moe_combine_shared(qw_cmd c, qw_ref out, qw_ref y, qw_ref w, qw_ref sh, qw_ref g,
                              int32_t rows, int32_t K, int32_t H) {
    QW_OP(c);
    touch(c, y, 0); touch(c, w, 0); touch(c, sh, 0); touch(c, g, 0); touch(c, out, 1);
    launched(c, "moe_combine_shared", qwk_moe_combine(G.stream, dp(out), dp(y), dp(w), dp(sh), dp(g), rows, K, H));
}

void qw_op_moe_combine(qw_cmd c, qw_ref out, qw_ref y, qw_ref w, int32_t rows, int32_t K, int32_t H) {
    QW_OP(c);
    touch(c, y, 0); touch(c, w, 0); touch(c, out, 1);
    launched(c, "moe_combine", qwk_moe_combine(G.stream, dp(out), dp(y), dp(w), NULL, NULL, rows, K, H));
}

void qw_op_scale_rows_sigmoid(qw_cmd c, qw_ref y, qw_ref g, int32_t rows, int32_t dim) {
    QW_OP(c);
    touch(c, g, 0); touch(c, y, 1);
    launched(c, "scale_rows_sigmoid", qwk_scale_rows_sigmoid(G.stream, dp(y), dp(g), rows, dim));
}

void qw_op_swiglu_split(qw_cmd c, qw_ref act, qw_ref gu, int32_t pairs, int32_t I) {
    QW_OP(c);
    touch(c, gu, 0); touch(c, act, 1);
    launched(c, "swiglu_split", qwk_swiglu_split(G.stream, dp(act), dp(gu), pairs, I));
}

void qw_op_moe_route(qw_cmd c, qw_ref idx, qw_ref w, qw_ref logits, int32_t rows, int32_t E,
                     int32_t K, bool norm) {
    if (K > QWK_ROUTE_MAX_K || E > QWK_ROUTE_MAX_E) {
        fprintf(stderr, "qwasar: moe top-%d of %d unsupported (max top-%d of %d)\n", K, E,
                QWK_ROUTE_MAX_K, QWK_ROUTE_MAX_E);
        return;
    }
    QW_OP(c);
    touch(c, logits, 0); touch(c, idx, 1); touch(c, w, 1);
    launched(c, "moe_route", qwk_route(G.stream, dp(idx), dp(w), dp(logits), rows, E, K, norm ? 1 : 0));
}

void qw_op_qmv_q4_bank(qw_cmd c, qw_ref y, qw_ref x, qw_ref idx, qw_ref w, qw_ref scales,
                       qw_ref biases, int32_t k, int32_t n, int32_t pairs, int32_t K,
                       bool x_by_pair, int32_t group) {
    QW_OP(c);
    touch(c, x, 0); touch(c, idx, 0); touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0);
    touch(c, y, 1);
    const qwk_q4 m = q4(w, scales, biases);
    launched(c, "qmv_q4_bank", qwk_q4mv(G.stream, dp(y), dp(x), NULL, k, dp(idx), &m, 1, k, n, pairs, K,
                                        x_by_pair ? 1 : 0, group));
}

bool qw_op_qmv_q4_bank2(qw_cmd c, qw_ref y, qw_ref x, qw_ref idx, qw_ref w, qw_ref scales,
                        qw_ref biases, qw_ref w2, qw_ref scales2, qw_ref biases2, int32_t k,
                        int32_t n, int32_t pairs, int32_t K, int32_t group) {
    /* The reference declines inputs too short to split (k < 2048,
     * qwasar_metal.m:516,1700) and its caller falls back to two banks. */
    if (k < 2048) return false;
    if (!c) return true;
    touch(c, x, 0); touch(c, idx, 0);
    touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0);
    touch(c, w2, 0); touch(c, scales2, 0); touch(c, biases2, 0);
    touch(c, y, 1);
    const qwk_q4 m[2] = { q4(w, scales, biases), q4(w2, scales2, biases2) };
    launched(c, "qmv_q4_bank2", qwk_q4mv(G.stream, dp(y), dp(x), NULL, k, dp(idx), m, 2, k, n, pairs, K, 0, group));
    return true;
}

void qw_op_qmv_q4_swiglu(qw_cmd c, qw_ref y, qw_ref gate, qw_ref up, int32_t stride, qw_ref idx,
                         qw_ref w, qw_ref scales, qw_ref biases, int32_t k, int32_t n, int32_t rows,
                         int32_t group) {
    QW_OP(c);
    touch(c, gate, 0); touch(c, up, 0); touch(c, idx, 0);
    touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0); touch(c, y, 1);
    const qwk_q4 m = q4(w, scales, biases);
    launched(c, "qmv_q4_swiglu", qwk_q4mv(G.stream, dp(y), dp(gate), dp(up), stride, dp(idx), &m, 1, k, n,
                                          rows, 1, 1, group));
}

static int32_t tiles_for(int32_t pairs, int32_t E, int32_t bm) {
    return (pairs < E ? pairs : E) + (pairs + bm - 1) / bm;
}

int32_t qw_moe_max_tiles(int32_t pairs, int32_t E) { return tiles_for(pairs, E, 16); }

int32_t qw_moe_tile_rows(int32_t pairs, int32_t E) {
    /* Expected pairs per expert decide the tile height: a tile pads its
     * pairs up to the height with idle MFMA rows, and a taller tile reads
     * each expert's weights fewer times. */
    const int64_t avg4 = E > 0 ? (int64_t)4 * pairs / E : 0;   /* 4 x average */
    if (avg4 >= 4 * 24) return 64;
    if (avg4 >= 4 * 12) return 32;
    return 16;
}

void qw_op_moe_group(qw_cmd c, qw_ref perm, qw_ref tiles, qw_ref cursor, qw_ref idx,
                     int32_t pairs, int32_t E) {
    (void)cursor;
    QW_OP(c);
    if (E > QWK_GROUP_MAX_E) {
        fprintf(stderr, "qwasar: moe grouping of %d experts unsupported (max %d)\n", E, QWK_GROUP_MAX_E);
        return;
    }
    touch(c, idx, 0); touch(c, perm, 1); touch(c, tiles, 1);
    const int32_t bm = qw_moe_tile_rows(pairs, E);
    const size_t wb = qwk_moe_group_work_bytes(pairs, E);
    void *work = scratch(wb);
    if (!work) { cmd_fail(c, hipErrorOutOfMemory, "moe_group: scratch of %zu bytes", wb); return; }
    launched(c, "moe_group", qwk_moe_group(G.stream, dp(perm), dp(tiles), dp(idx), pairs, E, bm,
                                           tiles_for(pairs, E, bm), work, wb, 0));
}

void qw_op_qmm_q4_gather(qw_cmd c, qw_ref y, qw_ref x, qw_ref perm, qw_ref tiles, qw_ref w,
                         qw_ref scales, qw_ref biases, int32_t k, int32_t n, int32_t pairs,
                         int32_t E, int32_t K, bool x_by_pair, int32_t group) {
    QW_OP(c);
    if (k % 32 != 0) {
        fprintf(stderr, "qwasar: grouped qmm needs k divisible by 32, got %d\n", k);
        return;
    }
    touch(c, x, 0); touch(c, perm, 0); touch(c, tiles, 0);
    touch(c, w, 0); touch(c, scales, 0); touch(c, biases, 0); touch(c, y, 1);
    const int32_t bm = qw_moe_tile_rows(pairs, E);
    launched(c, "qmm_q4_gather", qwk_gather_gemm(G.stream, dp(y), dp(x), dp(perm), dp(tiles),
                                                 q4(w, scales, biases), k, n, K, x_by_pair ? 1 : 0,
                                                 group, bm, tiles_for(pairs, E, bm)));
}

/* ---- the whole MoE layer ------------------------------------------------------ */

static void *scratch(size_t bytes) {
    if (bytes <= G.scratch_len) return G.scratch;
    hipStreamSynchronize(G.stream);
    if (G.scratch) hipFree(G.scratch);
    G.scratch = NULL;
    G.scratch_len = 0;
    if (hipMalloc(&G.scratch, bytes) != hipSuccess) return NULL;
    G.scratch_len = bytes;
    return G.scratch;
}

static qwk_q4 q4r(const qw_q4_ref *r) { return q4(r->w, r->scales, r->biases); }

static void touch_q4(qw_cmd c, const qw_q4_ref *r) {
    touch(c, r->w, 0); touch(c, r->scales, 0); touch(c, r->biases, 0);
}

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

/* Prefill: the grouped path on the one stream.  Activations are staged as
 * f16 once (x, then the SwiGLU output); the routed products run on MFMA with
 * SwiGLU fused into gate / up.  When the shared expert has the routed
 * experts' shape (SI == I, one group size) its rows join the same grouped
 * launches as one more expert, E: its pairs are the token rows, appended
 * after the routed pairs, and its down outputs are the combine's shared
 * term.  Otherwise it runs as dense products of its own. */
#define QW_PF_BM 64    /* tile height of the prefill product (qw_gmm16.hip) */
static bool moe_prefill(qw_cmd c, float *out, int32_t *idx, float *w, const float *x,
                        const qw_moe_layer *M, int32_t rows) {
    const int32_t H = M->H, E = M->E, K = M->K, I = M->I, SI = M->SI, pairs = rows * K;
    const int32_t grp = M->split ? M->gate.group : M->gate_up.group;
    const bool fuse = SI == I && M->sh_gate.group == grp && M->sh_up.group == grp && M->sh_down.group == grp;
    const int32_t xr = fuse ? rows : 0, ntot = pairs + xr;
    /* 16-row tiles (two workgroups a CU) where the experts average under 8
     * pairs, so that 64-row tiles would be mostly idle rows; else 64 (at 8 to
     * 12 a Zipf-skewed config 3 measured slower with 16: its hottest expert's
     * ~500 pairs then read its weights 32 times) */
    const int32_t bm = (int64_t)pairs < (int64_t)8 * E ? 16 : QW_PF_BM;
    const int32_t mt = tiles_for(pairs, E, bm) + (xr + bm - 1) / bm;
    const int32_t srows = fuse ? 0 : rows;      /* the unfused shared expert's buffers */
    size_t off = 0;
    const size_t o_xh = off;     off += al256((size_t)rows * H * 2);
    const size_t o_xF = off;     off += al256((size_t)rows * 4);
    const size_t o_logits = off; off += al256((size_t)rows * E * 4);
    const size_t o_perm = off;   off += al256((size_t)ntot * 4);
    const size_t o_tiles = off;  off += al256((size_t)(1 + 3 * mt) * 4);
    const size_t o_act = off;    off += al256((size_t)ntot * I * 4);
    const size_t o_ah = off;     off += al256((size_t)ntot * I * 2);
    const size_t o_aF = off;     off += al256((size_t)ntot * 4);
    const size_t o_ey = off;     off += al256((size_t)ntot * H * 4);
    const size_t o_sa = off;     off += al256((size_t)srows * SI * 4);
    const size_t o_sh16 = off;   off += al256((size_t)srows * SI * 2);
    const size_t o_sF = off;     off += al256((size_t)srows * 4);
    const size_t o_sh = off;     off += al256((size_t)srows * H * 4);
    const size_t o_g1 = off;     off += al256((size_t)rows * 4);
    const size_t o_gw = off;     off += al256(qwk_moe_group_work_bytes(pairs, E));
    char *S = scratch(off);
    if (!S) { cmd_fail(c, hipErrorOutOfMemory, "moe_layer: scratch of %zu bytes", off); return false; }
    uint16_t *xh = (uint16_t *)(S + o_xh), *ah = (uint16_t *)(S + o_ah), *sh16 = (uint16_t *)(S + o_sh16);
    float *xF = (float *)(S + o_xF), *aF = (float *)(S + o_aF), *sF = (float *)(S + o_sF);
    float *logits = (float *)(S + o_logits), *act = (float *)(S + o_act), *ey = (float *)(S + o_ey);
    float *sa = (float *)(S + o_sa), *sh = (float *)(S + o_sh), *g1 = (float *)(S + o_g1);
    int32_t *perm = (int32_t *)(S + o_perm), *tiles = (int32_t *)(S + o_tiles);
    hipStream_t s = G.stream;
    const long words = H / 8, groups = H / grp;
    const qwk_gmm_extra xgu = { q4r(&M->sh_gate), q4r(&M->sh_up), E, pairs };
    const qwk_gmm_extra xdn = { q4r(&M->sh_down), q4r(&M->sh_down), E, pairs };
    /* the token rows staged as f16 by the shared gate's launch (one read of
     * them for both), or by their own launch where it does not take them */
    int rc = qwk_dmat_rows_stage16(s, g1, xh, xF, x, dp(M->sh_gate_w), H, 1, rows);
    const bool gated = rc == 0;
    if (!gated) rc = qwk_stage16(s, xh, xF, x, rows, H);
    if (!rc) rc = qwk_dmat_bf16(s, logits, x, dp(M->router), H, E, rows);
    if (!rc) rc = qwk_route(s, idx, w, logits, rows, E, K, M->norm ? 1 : 0);
    if (!rc) rc = qwk_moe_group(s, perm, tiles, idx, pairs, E, bm, mt, S + o_gw,
                                qwk_moe_group_work_bytes(pairs, E), xr);
    /* 16-row tiles: the grouped products as one weight stream a wave where
     * they take the shapes (the down stages the activations itself) */
    const qwk_q4 gb = M->split ? q4r(&M->gate) : q4r(&M->gate_up);
    const qwk_q4 ub = M->split ? q4r(&M->up) : (qwk_q4){ gb.w + (size_t)I * words, gb.s + (size_t)I * groups,
                                                        gb.b + (size_t)I * groups };
    const long gew = (M->split ? 1L : 2L) * I * words, geg = (M->split ? 1L : 2L) * I * groups;
    const bool stream = bm == 16 &&
        qwk_gmm16_stream_supported(H, I, grp, 1, gb, ub, fuse ? &xgu : NULL, geg) &&
        qwk_gmm16_stream_supported(I, H, grp, 0, q4r(&M->down), q4r(&M->down), fuse ? &xdn : NULL,
                                   (long)H * (I / grp));
    if (stream) {
        if (!rc) rc = qwk_gmm16_stream(s, act, I, xh, xF, NULL, perm, tiles, mt, gb, ub, gew, geg, H, I, K, 0, grp, 1,
                                       fuse ? &xgu : NULL, NULL);
        if (!rc) rc = qwk_gmm16_stream(s, ey, H, NULL, NULL, act, perm, tiles, mt, q4r(&M->down), q4r(&M->down),
                                       (long)H * (I / 8), (long)H * (I / grp), I, H, K, 1, grp, 0,
                                       fuse ? &xdn : NULL, NULL);
    } else if (M->split) {
        if (!rc) rc = qwk_gmm16(s, act, I, xh, xF, perm, tiles, mt, q4r(&M->gate), q4r(&M->up),
                                (long)I * words, (long)I * groups, H, I, K, 0, grp, 1, 0, fuse ? &xgu : NULL, bm, NULL);
    } else {
        const qwk_q4 g0 = q4r(&M->gate_up);
        const qwk_q4 u0 = { g0.w + (size_t)I * words, g0.s + (size_t)I * groups, g0.b + (size_t)I * groups };
        if (!rc) rc = qwk_gmm16(s, act, I, xh, xF, perm, tiles, mt, g0, u0,
                                2L * I * words, 2L * I * groups, H, I, K, 0, grp, 1, 0, fuse ? &xgu : NULL, bm, NULL);
    }
    if (!stream) {
        if (!rc) rc = qwk_stage16(s, ah, aF, act, ntot, I);
        if (!rc) rc = qwk_gmm16(s, ey, H, ah, aF, perm, tiles, mt, q4r(&M->down), q4r(&M->down),
                                (long)H * (I / 8), (long)H * (I / grp), I, H, K, 1, grp, 0, 0, fuse ? &xdn : NULL, bm,
                                NULL);
    }
    if (!fuse) {
        if (!rc) rc = qwk_gmm16(s, sa, SI, xh, xF, NULL, NULL, 0, q4r(&M->sh_gate), q4r(&M->sh_up),
                                0, 0, H, SI, 1, 0, grp, 1, rows, NULL, 64, NULL);
        if (!rc) rc = qwk_stage16(s, sh16, sF, sa, rows, SI);
        if (!rc) rc = qwk_gmm16(s, sh, H, sh16, sF, NULL, NULL, 0, q4r(&M->sh_down), q4r(&M->sh_down),
                                0, 0, SI, H, 1, 0, grp, 0, rows, NULL, 64, NULL);
    }
    if (!rc && !gated) rc = qwk_dmat_bf16(s, g1, x, dp(M->sh_gate_w), H, 1, rows);
    if (!rc) rc = qwk_moe_combine(s, out, ey, w, fuse ? ey + (size_t)pairs * H : sh, g1, rows, K, H);
    launched(c, "moe_layer (prefill)", rc);
    return rc == 0;
}

static void moe_desc(qwk_moe *mp, const qw_moe_layer *M) {
    qwk_moe m;
    m.H = M->H; m.E = M->E; m.K = M->K; m.I = M->I; m.SI = M->SI;
    m.group = M->split ? M->gate.group : M->gate_up.group;
    m.norm = M->norm ? 1 : 0;
    m.split = M->split ? 1 : 0;
    m.router = dp(M->router);
    m.gate = q4r(&M->gate); m.up = q4r(&M->up); m.gate_up = q4r(&M->gate_up);
    m.down = q4r(&M->down);
    m.sh_gate = q4r(&M->sh_gate); m.sh_up = q4r(&M->sh_up); m.sh_down = q4r(&M->sh_down);
    m.sh_gate_w = dp(M->sh_gate_w);
    *mp = m;
}

/* Decode over only the selected experts: one launch for one token, the
 * batch path's launches otherwise.  The hand-off state and the batch path's
 * staging are the backend's heap scratch (k = QW_DS_HEAP) or the static
 * device array (k = QW_DS_STATIC: nothing allocated; the caller has checked
 * that the staging fits). */
/* Decode scratch: none for the one-launch path (one token; everything it
 * hands over sits in the hand-off state), else the batch path's. */
static int decode_one_launch(const qwk_moe *m, int32_t rows) { return rows == 1 && qwk_decode1_supported(m); }
static size_t decode_need(const qwk_moe *m, int32_t rows) {
    return decode_one_launch(m, rows) ? 0 : qwk_moe_decode_batch_scratch(m, rows);
}

static bool moe_decode(qw_cmd c, float *out, int32_t *idx, float *w, const float *x,
                       const qwk_resid *res, const qwk_moe *mp, int32_t rows, int k) {
    const qwk_moe m = *mp;
    const size_t need = decode_need(&m, rows);
    if (!decode_one_launch(&m, rows)) {
        /* several tokens (or a shape the one launch does not take): the
         * batch path over their unique experts, after the residual step as
         * its own pass when there is one */
        void *S = k == QW_DS_STATIC ? (void *)G.static_stage : scratch(need);
        const size_t have = k == QW_DS_STATIC ? G.static_stage_len : need;
        if (!S) { cmd_fail(c, hipErrorOutOfMemory, "moe_layer: scratch of %zu bytes", need); return false; }
        /* the hand-off words, for the router-and-route launch */
        uint32_t *err = NULL, epoch = 0;
        void *words = NULL;
        size_t nwords = 0;
        if ((G.ds[k].sync || dsync_reset(k)) && (G.ds[k].epoch != UINT32_MAX || dsync_check(k, 1))) {
            qwk_decode_sync_words(G.ds[k].sync, &err, &words, &nwords);
            epoch = G.ds[k].epoch + 1;
        }
        int handoff = 0;
        int rc = 0;
        if (res) {
            rc = qwk_resid_rms_bf16(G.stream, res->h, res->h_out, res->x_out, res->y, m.H, rows, res->eps);
            x = res->x_out;
        }
        if (!rc) rc = qwk_moe_decode_batch(G.stream, out, idx, w, x, &m, rows, S, have, words, nwords, err, epoch,
                                           &handoff);
        if (handoff) {            /* the epoch is taken only by a launch that hands off */
            G.ds[k].epoch = epoch;
            c->ep_hi[k] = epoch;
        }
        launched(c, k == QW_DS_STATIC ? "moe_layer_noalloc" : "moe_layer (decode batch)", rc);
        return rc == 0;
    }
    if (!G.ds[k].sync && !dsync_reset(k)) {
        cmd_fail(c, hipErrorOutOfMemory, "moe_layer: decode hand-off state");
        return false;
    }
    /* Tagged words hold past epochs, so an epoch is not reused
     * until the state is zeroed again (0 is "never"). */
    if (G.ds[k].epoch == UINT32_MAX && !dsync_check(k, 1)) {
        cmd_fail(c, hipErrorUnknown, "moe_layer: decode hand-off state");
        return false;
    }
    const uint32_t epoch = ++G.ds[k].epoch;
    hipEvent_t ev[2] = { NULL, NULL };
    const int per_kernel = k == QW_DS_HEAP && G.prof && (ev[0] = cmd_event(c, 0)) && (ev[1] = cmd_event(c, 0));
    const int rc = qwk_moe_decode(G.stream, out, idx, w, x, res, &m, G.ds[k].sync, epoch,
                                  per_kernel ? ev : NULL);
    if (per_kernel) cmd_add_mark(c, "moe decode", ev[0], ev[1]);
    c->ep_hi[k] = epoch;
    launched(c, k == QW_DS_STATIC ? "moe_layer_noalloc" : "moe_layer (decode)", rc);
    return rc == 0;
}

/* The layer's shape checks (false: refused, nothing encoded). */
static bool moe_layer_ok(const qw_moe_layer *M, int32_t rows) {
    if (!M || rows < 1 || M->K > QWK_ROUTE_MAX_K || M->E > QWK_ROUTE_MAX_E || M->K > M->E ||
        M->H % 64 || M->I % 64 || M->SI % 64 || M->H > QWK_DMAT_MAX_K)
        return false;
    const int32_t grp = M->split ? M->gate.group : M->gate_up.group;
    return !(M->down.group != grp || M->sh_gate.group != grp || M->sh_up.group != grp ||
             M->sh_down.group != grp || (M->split && M->up.group != grp));
}

static void touch_layer(qw_cmd c, const qw_moe_layer *M) {
    touch(c, M->router, 0); touch(c, M->sh_gate_w, 0);
    if (M->split) { touch_q4(c, &M->gate); touch_q4(c, &M->up); } else touch_q4(c, &M->gate_up);
    touch_q4(c, &M->down); touch_q4(c, &M->sh_gate); touch_q4(c, &M->sh_up); touch_q4(c, &M->sh_down);
}

bool qw_op_moe_layer(qw_cmd c, qw_ref out, qw_ref idx, qw_ref w, qw_ref x,
                     const qw_moe_layer *M, int32_t rows) {
    if (!moe_layer_ok(M, rows)) return false;
    if (!c) return true;
    touch(c, x, 0);
    touch_layer(c, M);
    touch(c, out, 1); touch(c, idx, 1); touch(c, w, 1);
    qwk_moe m;
    moe_desc(&m, M);
    if (rows > QWK_DECODE_MAX_ROWS || !qwk_moe_decode_supported(&m, rows))
        return moe_prefill(c, dp(out), dp(idx), dp(w), dp(x), M, rows);
    return moe_decode(c, dp(out), dp(idx), dp(w), dp(x), NULL, &m, rows, QW_DS_HEAP);
}

bool qw_op_moe_layer_noalloc(qw_cmd c, qw_ref out, qw_ref idx, qw_ref w, qw_ref x,
                             const qw_moe_layer *M, int32_t rows) {
    if (!moe_layer_ok(M, rows)) return false;
    qwk_moe m;
    moe_desc(&m, M);
    if (rows > QWK_DECODE_MAX_ROWS || !qwk_moe_decode_supported(&m, rows)) return false;
    if (!G.static_stage) {
        fprintf(stderr, "qwasar: moe_layer_noalloc: the static device scratch is not set up (qw_gpu_init)\n");
        return false;
    }
    const size_t need = decode_need(&m, rows);
    if (need > G.static_stage_len) {
        fprintf(stderr, "qwasar: moe_layer_noalloc: %d rows of this layer stage %zu bytes, over the %zu the "
                "static scratch holds\n", rows, need, G.static_stage_len);
        return false;
    }
    if (!c) return true;
    const qw_ref in[] = { x, M->router, M->sh_gate_w, M->gate_up.w, M->gate_up.scales, M->gate_up.biases,
                          M->gate.w, M->gate.scales, M->gate.biases, M->up.w, M->up.scales, M->up.biases,
                          M->down.w, M->down.scales, M->down.biases, M->sh_gate.w, M->sh_gate.scales,
                          M->sh_gate.biases, M->sh_up.w, M->sh_up.scales, M->sh_up.biases, M->sh_down.w,
                          M->sh_down.scales, M->sh_down.biases };
    /* the outputs go on the command's written list (room for them is checked
     * before anything is touched), so qw_cmd_wait refreshes their mirrors */
    {
        int room = c->capwritten - c->nwritten;
        const qw_buf o3[3] = { out.buf, idx.buf, w.buf };
        for (int j = 0; j < 3; j++) {
            int have = !o3[j];
            for (int i = 0; i < c->nwritten && !have; i++) have = c->written[i] == o3[j];
            for (int i = 0; i < j && !have; i++) have = o3[i] == o3[j];
            room -= !have;
        }
        if (room < 0) {
            cmd_fail(c, hipErrorInvalidValue, "moe_layer_noalloc: the command's written list is full (%d buffers); "
                     "wait on the command before encoding more", QW_CMD_FIXED_WRITTEN);
            fprintf(stderr, "qwasar: %s\n", c->msg);
            return false;
        }
    }
    for (size_t i = 0; i < sizeof in / sizeof in[0]; i++) touch_fixed(c, in[i], 0);
    touch_fixed(c, out, 1); touch_fixed(c, idx, 1); touch_fixed(c, w, 1);
    return moe_decode(c, dp(out), dp(idx), dp(w), dp(x), NULL, &m, rows, QW_DS_STATIC);
}

bool qw_op_moe_layer_residual(qw_cmd c, qw_ref out, qw_ref idx, qw_ref w, qw_ref h, qw_ref y_prev,
                              qw_ref h_out, qw_ref x_out, const qw_moe_layer *M, int32_t rows, float eps) {
    if (!moe_layer_ok(M, rows) || !h.buf || !h_out.buf || !x_out.buf) return false;
    if (h_out.buf == h.buf || (y_prev.buf && h_out.buf == y_prev.buf)) return false;
    if (!c) return true;
    touch(c, h, 0); touch(c, y_prev, 0);
    touch_layer(c, M);
    touch(c, h_out, 1); touch(c, x_out, 1);
    touch(c, out, 1); touch(c, idx, 1); touch(c, w, 1);
    qwk_moe m;
    moe_desc(&m, M);
    if (rows > QWK_DECODE_MAX_ROWS || !qwk_moe_decode_supported(&m, rows)) {
        const int rc = qwk_resid_rms_bf16(G.stream, dp(h), dp(h_out), dp(x_out), dp(y_prev), M->H, rows, eps);
        launched(c, "moe_layer_residual (norm)", rc);
        if (rc != 0) return false;
        return moe_prefill(c, dp(out), dp(idx), dp(w), dp(x_out), M, rows);
    }
    const qwk_resid res = { dp(h), dp(y_prev), dp(h_out), dp(x_out), eps };
    return moe_decode(c, dp(out), dp(idx), dp(w), NULL, &res, &m, rows, QW_DS_HEAP);
}

/* ---- gated DeltaNet (reference qwasar_gpu.h:318-358, qwasar_metal.m:1101-1215) ---- */

void qw_op_conv1d_causal_silu(qw_cmd c, qw_ref y, qw_ref x, qw_ref state, qw_ref weight, int32_t channels,
                              int32_t rows, int32_t ksize, qw_ref snap, int32_t n_snap, int32_t snap_stride) {
    QW_OP(c);
    if (ksize != 4) {
        fprintf(stderr, "qwasar: conv kernel size %d unsupported (expected 4)\n", ksize);
        return;
    }
    touch(c, x, 0); touch(c, weight, 0); touch(c, state, 1); touch(c, y, 1);
    if (n_snap > 0) touch(c, snap, 1);
    launched(c, "conv1d_causal_silu", qwk_conv1d_causal_silu(G.stream, dp(y), dp(x), dp(state), dp(weight), channels,
                                                             rows, ksize, n_snap > 0 ? dp(snap) : NULL, n_snap,
                                                             snap_stride));
}

void qw_op_gdn_gates(qw_cmd c, qw_ref g, qw_ref beta, qw_ref a, qw_ref b, qw_ref A_log, qw_ref dt_bias,
                     int32_t n_v_heads, int32_t rows) {
    QW_OP(c);
    touch(c, a, 0); touch(c, b, 0); touch(c, A_log, 0); touch(c, dt_bias, 0); touch(c, g, 1); touch(c, beta, 1);
    launched(c, "gdn_gates", qwk_gdn_gates(G.stream, dp(g), dp(beta), dp(a), dp(b), dp(A_log), dp(dt_bias),
                                           n_v_heads, rows));
}

static void gated_delta(qw_cmd c, qw_ref y, qw_ref q, qw_ref k, qw_ref v, qw_ref g, qw_ref beta,
                        const qw_gdn_prep *prep, qw_ref state, int32_t hk, int32_t hv, int32_t dk, int32_t dv,
                        int32_t rows, qw_ref snap, int32_t n_snap, int32_t snap_stride) {
    QW_OP(c);
    if (dk != 128 || dv != 128) {
        fprintf(stderr, "qwasar: gated-delta head dims %dx%d unsupported (kernel is built for 128x128)\n", dk, dv);
        return;
    }
    touch(c, q, 0); touch(c, k, 0); touch(c, v, 0); touch(c, state, 1); touch(c, y, 1);
    if (n_snap > 0) touch(c, snap, 1);
    qwk_gdn_prep pp;
    if (prep) {
        touch(c, prep->a, 0); touch(c, prep->b, 0); touch(c, prep->A_log, 0); touch(c, prep->dt_bias, 0);
        pp.a = dp(prep->a); pp.b = dp(prep->b); pp.A_log = dp(prep->A_log); pp.dt_bias = dp(prep->dt_bias);
        pp.l2eps = prep->l2eps; pp.q_scale = prep->q_scale; pp.k_scale = prep->k_scale;
    } else {
        touch(c, g, 0); touch(c, beta, 0);
    }
    const size_t wb = qwk_gated_delta_work(hk, hv, rows, prep != NULL);
    void *work = wb ? scratch(wb) : NULL;
    if (wb && !work) { cmd_fail(c, hipErrorOutOfMemory, "gated_delta: scratch of %zu bytes", wb); return; }
    launched(c, prep ? "gated_delta_prep" : "gated_delta",
             qwk_gated_delta(G.stream, dp(y), dp(q), dp(k), dp(v), dp(g), dp(beta), dp(state), hk, hv, dk, dv, rows,
                             n_snap > 0 ? dp(snap) : NULL, n_snap, snap_stride, prep ? &pp : NULL, work));
}

void qw_op_gated_delta(qw_cmd c, qw_ref y, qw_ref q, qw_ref k, qw_ref v, qw_ref g, qw_ref beta, qw_ref state,
                       int32_t hk, int32_t hv, int32_t dk, int32_t dv, int32_t rows, qw_ref snap, int32_t n_snap,
                       int32_t snap_stride) {
    gated_delta(c, y, q, k, v, g, beta, NULL, state, hk, hv, dk, dv, rows, snap, n_snap, snap_stride);
}

void qw_op_gated_delta_prep(qw_cmd c, qw_ref y, qw_ref q, qw_ref k, qw_ref v, const qw_gdn_prep *prep,
                            qw_ref state, int32_t hk, int32_t hv, int32_t dk, int32_t dv, int32_t rows, qw_ref snap,
                            int32_t n_snap, int32_t snap_stride) {
    if (!prep) return;
    const qw_ref none = { 0 };
    gated_delta(c, y, q, k, v, none, none, prep, state, hk, hv, dk, dv, rows, snap, n_snap, snap_stride);
}

bool qw_op_gdn_decode(qw_cmd c, qw_ref y, qw_ref x, qw_ref conv_state, qw_ref conv_state_out, qw_ref conv_weight,
                      const qw_gdn_prep *prep, qw_ref state, int32_t hk, int32_t hv, int32_t dk, int32_t dv) {
    if (!prep || dk != 128 || dv != 128 || hk < 1 || hv < 1 || hv % hk) return false;
    /* every workgroup reads the old window of the q and k channels while one
     * writes the new: the window out may not share a byte with the window in
     * or with x */
    const size_t ch = (size_t)2 * hk * dk + (size_t)hv * dv;
    if (refs_overlap(conv_state_out, 12 * ch, conv_state, 12 * ch) || refs_overlap(conv_state_out, 12 * ch, x, 4 * ch))
        return false;
    if (!c) return true;
    touch(c, x, 0); touch(c, conv_state, 0); touch(c, conv_weight, 0);
    touch(c, prep->a, 0); touch(c, prep->b, 0); touch(c, prep->A_log, 0); touch(c, prep->dt_bias, 0);
    touch(c, conv_state_out, 1); touch(c, state, 1); touch(c, y, 1);
    qwk_gdn_prep pp;
    pp.a = dp(prep->a); pp.b = dp(prep->b); pp.A_log = dp(prep->A_log); pp.dt_bias = dp(prep->dt_bias);
    pp.l2eps = prep->l2eps; pp.q_scale = prep->q_scale; pp.k_scale = prep->k_scale;
    const int rc = qwk_gdn_decode(G.stream, dp(y), dp(x), dp(conv_state), dp(conv_state_out), dp(conv_weight), &pp,
                                  dp(state), hk, hv, dk, dv);
    launched(c, "gdn_decode", rc);
    return rc == 0;
}

void qw_op_rms_norm_gated_sigmoid(qw_cmd c, qw_ref y, qw_ref x, qw_ref weight, qw_ref gate, int32_t dim,
                                  int32_t rows, float eps, float out_scale) {
    QW_OP(c);
    touch(c, x, 0); touch(c, weight, 0); touch(c, gate, 0); touch(c, y, 1);
    launched(c, "rms_norm_gated_sigmoid", qwk_rms_norm_gated_sigmoid(G.stream, dp(y), dp(x), dp(weight), dp(gate),
                                                                     dim, rows, eps, out_scale));
}

/* ---- QSA (reference qwasar_gpu.h:621-646, qwasar_metal.m:1898-1966,2042-2068) ---- */

static bool qsa_shape_ok(int32_t rotary_dim, int32_t d) {
    if (rotary_dim == 64 && d % 32 == 0 && d >= 64 && d <= 256) return true;
    fprintf(stderr, "qwasar: QSA indexer shape (rotary %d, head %d) unsupported\n", rotary_dim, d);
    return false;
}

void qw_op_qsa_scores(qw_cmd c, qw_ref scores, qw_ref qn, qw_ref ikeys, qw_ref k_norm, qw_ref inv_freq,
                      int32_t rows, int32_t nq, int32_t d, int32_t ratio, int32_t base_pos, int32_t rotary_dim,
                      int32_t max_blocks, float eps) {
    if (!qsa_shape_ok(rotary_dim, d)) return;
    QW_OP(c);
    touch(c, qn, 0); touch(c, ikeys, 0); touch(c, k_norm, 0); touch(c, inv_freq, 0); touch(c, scores, 1);
    launched(c, "qsa_scores", qwk_qsa_scores(G.stream, dp(scores), dp(qn), dp(ikeys), dp(k_norm), dp(inv_freq), rows,
                                             nq, d, ratio, base_pos, rotary_dim, max_blocks, eps));
}

void qw_op_qsa_pool(qw_cmd c, qw_ref pool, qw_ref ikeys, qw_ref k_norm, qw_ref inv_freq, int32_t d, int32_t ratio,
                    int32_t b0, int32_t b1, int32_t rotary_dim, float eps) {
    if (b1 <= b0) return;
    if (!qsa_shape_ok(rotary_dim, d)) return;
    QW_OP(c);
    touch(c, ikeys, 0); touch(c, k_norm, 0); touch(c, inv_freq, 0); touch(c, pool, 1);
    launched(c, "qsa_pool", qwk_qsa_pool(G.stream, dp(pool), dp(ikeys), dp(k_norm), dp(inv_freq), d, ratio, b0, b1,
                                         rotary_dim, eps));
}

void qw_op_qsa_scores_pooled(qw_cmd c, qw_ref scores, qw_ref qn, qw_ref pool, int32_t rows, int32_t nq, int32_t d,
                             int32_t ratio, int32_t base_pos, int32_t max_blocks) {
    if (!qsa_shape_ok(64, d)) return;
    QW_OP(c);
    touch(c, qn, 0); touch(c, pool, 0); touch(c, scores, 1);
    launched(c, "qsa_scores_pooled", qwk_qsa_scores_pooled(G.stream, dp(scores), dp(qn), dp(pool), rows, nq, d, ratio,
                                                           base_pos, max_blocks));
}

void qw_op_qsa_select(qw_cmd c, qw_ref mask, qw_ref list, qw_ref scores, int32_t rows, int32_t ratio,
                      int32_t base_pos, int32_t block_topk, int32_t max_ctx, int32_t max_blocks) {
    QW_OP(c);
    touch(c, scores, 0); touch(c, mask, 1); touch(c, list, 1);
    launched(c, "qsa_select", qwk_qsa_select(G.stream, dp(mask), dp(list), dp(scores), rows, ratio, base_pos,
                                             block_topk, max_ctx, max_blocks));
}

void qw_op_attn_masked_gated(qw_cmd c, qw_ref out, qw_ref gate, qw_ref q, qw_ref kcache, qw_ref vcache, qw_ref list,
                             int32_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t max_ctx,
                             int32_t base_pos, float scale, int32_t block_topk, int32_t ratio) {
    (void)base_pos;   /* the list names the positions */
    if (head_dim != 256) {
        fprintf(stderr, "qwasar: attention head_dim %d unsupported (kernel is built for 256)\n", head_dim);
        return;
    }
    QW_OP(c);
    touch(c, q, 0); touch(c, kcache, 0); touch(c, vcache, 0); touch(c, list, 0); touch(c, gate, 0);
    touch(c, out, 1);
    const int32_t cap = qw_qsa_list_cap(block_topk, ratio);
    const size_t wb = kv_heads > 0 && rows > 0 ? qwk_attn_masked_work_bytes(rows, q_heads, kv_heads, cap) : 0;
    void *work = wb ? scratch(wb) : NULL;
    launched(c, "attn_masked", qwk_attn_masked(G.stream, dp(out), dp(gate), dp(q), dp(kcache), dp(vcache), dp(list),
                                               rows, q_heads, kv_heads, head_dim, max_ctx, scale, cap, work,
                                               work ? wb : 0));
}

void qw_op_attn_masked(qw_cmd c, qw_ref out, qw_ref q, qw_ref kcache, qw_ref vcache, qw_ref list, int32_t rows,
                       int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t max_ctx, int32_t base_pos,
                       float scale, int32_t block_topk, int32_t ratio) {
    const qw_ref none = { 0 };
    qw_op_attn_masked_gated(c, out, none, q, kcache, vcache, list, rows, q_heads, kv_heads, head_dim, max_ctx,
                            base_pos, scale, block_topk, ratio);
}

/* ---- measurement probe ---------------------------------------------------------
 * Not part of the reference interface: the HBM read ceiling the kernels are
 * measured against.  Launch r reads set (r % nsets) of nseg ranges
 * (segs[s * nseg + i], bytes[...]: 16-byte multiples at 16-byte-aligned
 * offsets) once, one workgroup a piece of at most piece_bytes, and ms[r] is
 * its duration.  The bytes' values are not used, so
 * host mirrors are not consulted.  Returns false on bad arguments or a HIP
 * error. */
bool qw_probe_read(const qw_ref *segs, const uint64_t *bytes, int32_t nsets, int32_t nseg, int32_t reps,
                   uint64_t piece_bytes, float *ms) {
    if (!G.ready || !segs || !bytes || !ms || nsets < 1 || nseg < 1 || reps < 1) return false;
    const size_t n = (size_t)nsets * (size_t)nseg;
    const void **p = (const void **)calloc(n, sizeof(void *));
    if (!p) return false;
    bool ok = true;
    for (size_t i = 0; i < n && ok; i++) {
        p[i] = dp(segs[i]);
        ok = p[i] && segs[i].off + bytes[i] <= segs[i].buf->len;
    }
    /* (the library's queued work first, so that none of it runs under the probe) */
    if (ok) ok = hipStreamSynchronize(G.stream) == hipSuccess;
    if (ok) ok = qwk_read_probe(p, bytes, nsets, nseg, reps, piece_bytes, ms) == 0;
    free(p);
    return ok;
}
