/* qw_load.c -- binds a checkpoint's MoE blocks to device buffers, for both
 * on-disk formats the reference reads:
 *
 *   - fused experts: `experts.gate_up_proj` [E, 2I, H/8] and
 *     `experts.down_proj`, group 64, bf16 router (transformers export);
 *   - MLX split experts: `switch_mlp.{gate,up,down}_proj`, group 32, with the
 *     router and the shared-expert gate quantised 8-bit.
 *
 * The reference does this in qwasar.c: config parse (:700-775), the
 * safetensors table, qw_bind_moe (:1532-1563) with qw_bind_qbank
 * (:1469-1495), qw_bind_qlinear (:906-940), qw_qgroup_from_shapes (:892-903)
 * and qw_bind_small (:1426-1461).  What a checkpoint must satisfy is the
 * same -- the tensor names and shapes the formats dictate, and a small
 * quantised matrix expanded to bf16 as w = scale * q + bias per group,
 * rounded to nearest even -- but the checks here run from a per-format plan
 * through one shape check of their own (see "binding" below).
 *
 * Files are mapped read-only; each bound tensor is copied once into its own
 * device buffer, and the mapping is released when the checkpoint is closed.
 * Host code only: this file touches the device through qw_buf_from_bytes_. */
#define _GNU_SOURCE
#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "qwasar_gpu.h"

/* Defined in qwasar_hip.c, not exported: a device buffer holding `len`
 * bytes copied from host memory. */
qw_buf qw_buf_from_bytes_(const void *src, size_t len);

static void errf(char *err, size_t cap, const char *fmt, ...)
{
    if (!err || !cap) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, cap, fmt, ap);
    va_end(ap);
}

/* ---- a JSON reader over a NUL-terminated text ------------------------------
 * Enough for config.json and safetensors headers: members are found by key,
 * values are read as integers, booleans, strings and integer arrays.  Keys
 * are compared as written (these files carry no escapes in their keys). */

static const char *js_ws(const char *p)
{
    while (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t') p++;
    return p;
}

/* p at '"': past the closing quote, or NULL */
static const char *js_str_end(const char *p)
{
    for (p++; *p; p++) {
        if (*p == '\\') { if (!*++p) return NULL; }
        else if (*p == '"') return p + 1;
    }
    return NULL;
}

/* past the value at p, or NULL if it is malformed */
static const char *js_skip(const char *p)
{
    p = js_ws(p);
    if (*p == '"') return js_str_end(p);
    if (*p == '{' || *p == '[') {
        int depth = 0;
        while (*p) {
            if (*p == '"') { if (!(p = js_str_end(p))) return NULL; continue; }
            if (*p == '{' || *p == '[') depth++;
            else if (*p == '}' || *p == ']') { if (--depth == 0) return p + 1; }
            p++;
        }
        return NULL;
    }
    const char *q = p;
    while (*p && !strchr(",}] \n\r\t", *p)) p++;
    return p > q ? p : NULL;
}

/* Iterates an object's members: *it starts at '{' (first call) and then at
 * the position returned.  Returns 1 with the key span and value start, 0 at
 * the end, -1 on malformed input. */
static int js_member(const char **it, const char **key, size_t *klen, const char **val)
{
    const char *p = js_ws(*it);
    if (*p == '{') p = js_ws(p + 1);
    else if (*p == ',') p = js_ws(p + 1);
    if (*p == '}') return 0;
    if (*p != '"') return -1;
    const char *ke = js_str_end(p);
    if (!ke) return -1;
    *key = p + 1;
    *klen = (size_t)(ke - p - 2);
    p = js_ws(ke);
    if (*p != ':') return -1;
    *val = js_ws(p + 1);
    const char *ve = js_skip(*val);
    if (!ve) return -1;
    *it = js_ws(ve);
    if (**it != ',' && **it != '}') return -1;
    return 1;
}

static const char *js_get(const char *obj, const char *name)
{
    if (!obj || *js_ws(obj) != '{') return NULL;
    const char *it = js_ws(obj), *k, *v;
    size_t kl;
    const size_t nl = strlen(name);
    while (js_member(&it, &k, &kl, &v) == 1)
        if (kl == nl && !memcmp(k, name, nl)) return v;
    return NULL;
}

static int64_t js_int_or(const char *obj, const char *name, int64_t dflt)
{
    const char *v = js_get(obj, name);
    if (!v || !(*v == '-' || (*v >= '0' && *v <= '9'))) return dflt;
    return strtoll(v, NULL, 10);
}

static bool js_bool_or(const char *obj, const char *name, bool dflt)
{
    const char *v = js_get(obj, name);
    if (v && !strncmp(v, "true", 4)) return true;
    if (v && !strncmp(v, "false", 5)) return false;
    return dflt;
}

/* copies a string value (no unescaping); false if v is not a string */
static bool js_str(const char *v, char *out, size_t cap)
{
    if (!v || *v != '"') return false;
    const char *e = js_str_end(v);
    if (!e) return false;
    size_t n = (size_t)(e - v - 2);
    if (n >= cap) n = cap - 1;
    memcpy(out, v + 1, n);
    out[n] = 0;
    return true;
}

/* an array of up to `cap` integers; the count, or -1 */
static int js_ints(const char *v, int64_t *out, int cap)
{
    if (!v || *v != '[') return -1;
    const char *p = js_ws(v + 1);
    int n = 0;
    if (*p == ']') return 0;
    for (;;) {
        char *e;
        errno = 0;
        const long long x = strtoll(p, &e, 10);
        if (e == p || errno || n == cap) return -1;
        out[n++] = x;
        p = js_ws(e);
        if (*p == ']') return n;
        if (*p != ',') return -1;
        p = js_ws(p + 1);
    }
}

static char *read_text(const char *path, char *err, size_t cap)
{
    FILE *f = fopen(path, "rb");
    if (!f) { errf(err, cap, "cannot open %s: %s", path, strerror(errno)); return NULL; }
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *s = n >= 0 ? malloc((size_t)n + 1) : NULL;
    if (!s || fread(s, 1, (size_t)n, f) != (size_t)n) {
        errf(err, cap, "cannot read %s", path);
        free(s);
        fclose(f);
        return NULL;
    }
    s[n] = 0;
    fclose(f);
    return s;
}

/* ---- the tensor table ---------------------------------------------------- */

enum { DT_BF16, DT_F16, DT_F32, DT_U32, DT_I32, DT_U8, DT_I8, DT_I64, DT_U64, DT_F64, DT_I16, DT_U16,
       DT_BOOL, DT_F8E4M3, DT_F8E5M2, DT_COUNT };
static const char *const dt_names[DT_COUNT] = {"BF16", "F16", "F32", "U32", "I32", "U8", "I8", "I64", "U64",
                                               "F64", "I16", "U16", "BOOL", "F8_E4M3", "F8_E5M2"};
static const int dt_size[DT_COUNT] = {2, 2, 4, 4, 4, 1, 1, 8, 8, 8, 2, 2, 1, 1, 1};

typedef struct {
    char *name;
    int dtype, ndim;
    int64_t shape[8];
    const uint8_t *data;
    size_t nbytes;
} st_tensor;

typedef struct {
    void *map;
    size_t len;
} st_file;

struct qw_checkpoint_s {
    st_file *files;
    int nfiles;
    st_tensor *t;
    size_t nt, cap;
    int32_t H, E, K, I, SI, layers;
    bool norm;
};

static int cmp_name(const void *a, const void *b)
{
    return strcmp(((const st_tensor *)a)->name, ((const st_tensor *)b)->name);
}

static const st_tensor *find(const qw_checkpoint ck, const char *name)
{
    st_tensor key = {.name = (char *)name};
    return bsearch(&key, ck->t, ck->nt, sizeof *ck->t, cmp_name);
}

static bool add_file(qw_checkpoint ck, const char *path, char *err, size_t cap)
{
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { errf(err, cap, "cannot open %s: %s", path, strerror(errno)); return false; }
    struct stat sb;
    if (fstat(fd, &sb) || sb.st_size < 8) {
        errf(err, cap, "%s is not a safetensors file", path);
        close(fd);
        return false;
    }
    const size_t len = (size_t)sb.st_size;
    void *map = mmap(NULL, len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { errf(err, cap, "cannot map %s: %s", path, strerror(errno)); return false; }
    st_file *nf = realloc(ck->files, (size_t)(ck->nfiles + 1) * sizeof *nf);
    if (!nf) { munmap(map, len); errf(err, cap, "out of memory"); return false; }
    ck->files = nf;
    ck->files[ck->nfiles++] = (st_file){map, len};

    uint64_t hlen;
    memcpy(&hlen, map, 8);                 /* little-endian, as the format fixes */
    if (hlen > len - 8) { errf(err, cap, "%s: header of %llu bytes overruns the file", path, (unsigned long long)hlen); return false; }
    char *hdr = malloc(hlen + 1);
    if (!hdr) { errf(err, cap, "out of memory"); return false; }
    memcpy(hdr, (const char *)map + 8, hlen);
    hdr[hlen] = 0;
    const uint8_t *base = (const uint8_t *)map + 8 + hlen;
    const size_t body = len - 8 - hlen;

    const char *it = js_ws(hdr), *k, *v;
    size_t kl;
    int r = 0;
    bool ok = *it == '{';
    while (ok && (r = js_member(&it, &k, &kl, &v)) == 1) {
        if (kl == 12 && !memcmp(k, "__metadata__", 12)) continue;
        st_tensor t = {0};
        char dt[16];
        int64_t off[2];
        if (!js_str(js_get(v, "dtype"), dt, sizeof dt) || js_ints(js_get(v, "data_offsets"), off, 2) != 2 ||
            (t.ndim = js_ints(js_get(v, "shape"), t.shape, 8)) < 0) {
            errf(err, cap, "%s: malformed entry %.*s", path, (int)kl, k);
            ok = false;
            break;
        }
        t.dtype = -1;
        for (int i = 0; i < DT_COUNT; i++)
            if (!strcmp(dt, dt_names[i])) t.dtype = i;
        if (t.dtype < 0) { errf(err, cap, "%s: %.*s has unknown dtype %s", path, (int)kl, k, dt); ok = false; break; }
        /* the element count and byte size, each product checked: a header
         * with negative or huge dims must not wrap to the data's length */
        uint64_t bytes = (uint64_t)dt_size[t.dtype];
        bool dims_ok = true;
        for (int i = 0; i < t.ndim && dims_ok; i++)
            dims_ok = t.shape[i] >= 0 && !__builtin_mul_overflow(bytes, (uint64_t)t.shape[i], &bytes);
        if (!dims_ok) {
            errf(err, cap, "%s: %.*s has a negative or oversized shape", path, (int)kl, k);
            ok = false;
            break;
        }
        if (off[0] < 0 || off[1] < off[0] || (uint64_t)off[1] > body || (uint64_t)(off[1] - off[0]) != bytes) {
            errf(err, cap, "%s: %.*s's data offsets [%lld, %lld) do not hold its shape", path, (int)kl, k,
                 (long long)off[0], (long long)off[1]);
            ok = false;
            break;
        }
        t.data = base + off[0];
        t.nbytes = (size_t)(off[1] - off[0]);
        t.name = strndup(k, kl);
        if (ck->nt == ck->cap) {
            const size_t nc = ck->cap ? 2 * ck->cap : 256;
            st_tensor *nt = realloc(ck->t, nc * sizeof *nt);
            if (!nt || !t.name) { free(t.name); errf(err, cap, "out of memory"); ok = false; break; }
            ck->t = nt;
            ck->cap = nc;
        }
        if (!t.name) { errf(err, cap, "out of memory"); ok = false; break; }
        ck->t[ck->nt++] = t;
    }
    if (ok && r < 0) { errf(err, cap, "%s: malformed header", path); ok = false; }
    if (!ok && !(err && err[0])) errf(err, cap, "%s: malformed header", path);
    free(hdr);
    return ok;
}

static int cmp_str(const void *a, const void *b) { return strcmp(*(char *const *)a, *(char *const *)b); }

static bool read_config(qw_checkpoint ck, const char *dir, char *err, size_t cap)
{
    char path[4096];
    snprintf(path, sizeof path, "%s/config.json", dir);
    char *s = read_text(path, err, cap);
    if (!s) return false;
    const char *root = js_ws(s);
    char model_type[64] = "";
    js_str(js_get(root, "model_type"), model_type, sizeof model_type);
    const char *tc = js_get(root, "text_config");
    if (!tc && !strcmp(model_type, "qwen4_exp_text")) tc = root;  /* text-only export: fields at the root */
    if (!tc || *tc != '{') {
        errf(err, cap, "config.json has no text_config -- is this a Qwen3.8 VLM checkpoint?");
        free(s);
        return false;
    }
    ck->H = (int32_t)js_int_or(tc, "hidden_size", 0);
    ck->I = (int32_t)js_int_or(tc, "moe_intermediate_size", 0);
    ck->E = (int32_t)js_int_or(tc, "num_experts", 0);
    ck->K = (int32_t)js_int_or(tc, "num_experts_per_tok", 0);
    ck->SI = (int32_t)js_int_or(tc, "shared_expert_intermediate_size", 0);
    ck->layers = (int32_t)js_int_or(tc, "num_hidden_layers", 0);
    ck->norm = js_bool_or(tc, "norm_topk_prob", true);
    free(s);
    if (ck->H <= 0 || ck->I <= 0 || ck->E <= 0 || ck->K <= 0 || ck->K > ck->E || ck->SI <= 0 || ck->layers <= 0) {
        errf(err, cap, "config.json: not a MoE text config (hidden_size %d, moe_intermediate_size %d, "
             "num_experts %d, num_experts_per_tok %d, shared_expert_intermediate_size %d, num_hidden_layers %d)",
             ck->H, ck->I, ck->E, ck->K, ck->SI, ck->layers);
        return false;
    }
    return true;
}

qw_checkpoint qw_checkpoint_open(const char *dir, char *err, size_t errcap)
{
    if (err && errcap) err[0] = 0;
    if (!dir) { errf(err, errcap, "no checkpoint directory"); return NULL; }
    qw_checkpoint ck = calloc(1, sizeof *ck);
    if (!ck) { errf(err, errcap, "out of memory"); return NULL; }
    if (!read_config(ck, dir, err, errcap)) { free(ck); return NULL; }

    DIR *d = opendir(dir);
    if (!d) { errf(err, errcap, "cannot open %s: %s", dir, strerror(errno)); free(ck); return NULL; }
    char **names = NULL;
    size_t nn = 0;
    struct dirent *de;
    while ((de = readdir(d))) {
        const size_t l = strlen(de->d_name);
        if (l > 12 && !strcmp(de->d_name + l - 12, ".safetensors")) {
            char **nx = realloc(names, (nn + 1) * sizeof *nx);
            if (!nx) break;
            names = nx;
            names[nn++] = strdup(de->d_name);
        }
    }
    closedir(d);
    qsort(names, nn, sizeof *names, cmp_str);
    bool ok = nn > 0;
    if (!ok) errf(err, errcap, "%s holds no .safetensors files", dir);
    for (size_t i = 0; i < nn; i++) {
        char path[4096];
        snprintf(path, sizeof path, "%s/%s", dir, names[i]);
        if (ok && names[i]) ok = add_file(ck, path, err, errcap);
        free(names[i]);
    }
    free(names);
    if (ok) {
        qsort(ck->t, ck->nt, sizeof *ck->t, cmp_name);
        for (size_t i = 1; i < ck->nt && ok; i++)
            if (!strcmp(ck->t[i - 1].name, ck->t[i].name)) {
                errf(err, errcap, "tensor %s appears twice", ck->t[i].name);
                ok = false;
            }
    }
    if (!ok) { qw_checkpoint_close(ck); return NULL; }
    return ck;
}

void qw_checkpoint_close(qw_checkpoint ck)
{
    if (!ck) return;
    for (size_t i = 0; i < ck->nt; i++) free(ck->t[i].name);
    free(ck->t);
    for (int i = 0; i < ck->nfiles; i++) munmap(ck->files[i].map, ck->files[i].len);
    free(ck->files);
    free(ck);
}

int32_t qw_checkpoint_layers(qw_checkpoint ck) { return ck ? ck->layers : 0; }

bool qw_checkpoint_tensor(qw_checkpoint ck, const char *name, const void **data, size_t *nbytes,
                          int32_t *ndim, int64_t shape[8], char dtype[16])
{
    const st_tensor *t = ck && name ? find(ck, name) : NULL;
    if (!t) return false;
    if (data) *data = t->data;
    if (nbytes) *nbytes = t->nbytes;
    if (ndim) *ndim = t->ndim;
    if (shape) for (int i = 0; i < t->ndim; i++) shape[i] = t->shape[i];
    if (dtype) snprintf(dtype, 16, "%s", dt_names[t->dtype]);
    return true;
}

/* ---- binding ------------------------------------------------------------------
 *
 * A layer is bound from a plan: the list of tensors its format holds (fused
 * or MLX split banks, the shared expert, the router and the shared gate),
 * each with the dims the config implies.  Every tensor goes through one
 * check, expect(), which names the tensor and prints what was found beside
 * what the layer needs.  Quantised matrices take their group from the scale
 * columns; the two small matrices are taken as bf16, or expanded to bf16 from
 * 4 or 8 bits a group at a time. */

static uint16_t f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static float bf16_to_f32(uint16_t b)
{
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static bool upload(qw_ref *r, const void *src, size_t len, const char *what, char *err, size_t cap)
{
    qw_buf b = qw_buf_from_bytes_(src, len);
    if (!b) { errf(err, cap, "%s: no device memory for %zu bytes", what, len); return false; }
    *r = (qw_ref){b, 0};
    return true;
}

/* Element types a slot accepts: packed words (U32 or I32, as exporters
 * differ) or bf16. */
enum { ANY_WORDS, ANY_BF16 };

static bool type_ok(const st_tensor *t, int want)
{
    return want == ANY_BF16 ? t->dtype == DT_BF16 : (t->dtype == DT_U32 || t->dtype == DT_I32);
}

static void dims_text(char *buf, size_t cap, int nd, const int64_t *d)
{
    size_t n = (size_t)snprintf(buf, cap, "[");
    for (int i = 0; i < nd && n < cap; i++)
        n += (size_t)snprintf(buf + n, cap - n, i ? ",%lld" : "%lld", (long long)d[i]);
    if (n < cap) snprintf(buf + n, cap - n, "]");
}

/* The tensor `name`, required present with element type `want` and dims
 * d[0..nd) (d[i] < 0: any); NULL with a message otherwise. */
static const st_tensor *expect(qw_checkpoint ck, const char *name, int want, int nd, const int64_t *d, char *err,
                               size_t cap)
{
    const st_tensor *t = find(ck, name);
    if (!t) { errf(err, cap, "checkpoint has no tensor %s", name); return NULL; }
    bool fits = type_ok(t, want) && t->ndim == nd;
    for (int i = 0; fits && i < nd; i++) fits = d[i] < 0 || t->shape[i] == d[i];
    if (fits) return t;
    char got[96], need[96];
    dims_text(got, sizeof got, t->ndim, t->shape);
    dims_text(need, sizeof need, nd, d);   /* -1 marks a free dim */
    errf(err, cap, "%s: stored as %s %s; this layer needs %s %s", name, dt_names[t->dtype], got,
         want == ANY_BF16 ? "BF16" : "U32 (or I32)", need);
    return NULL;
}

/* One quantised slot of the plan: `nbank` matrices (0: a single matrix) of
 * [out, in], 4-bit, at "<base>.{weight,scales,biases}". */
typedef struct {
    qw_q4_ref *dst;
    char base[200];
    int32_t nbank, out, in;
} q4_slot;

static bool bind_slot(qw_checkpoint ck, const q4_slot *sl, char *err, size_t cap)
{
    char nw[224], ns[224], nb[224];
    snprintf(nw, sizeof nw, "%s.weight", sl->base);
    snprintf(ns, sizeof ns, "%s.scales", sl->base);
    snprintf(nb, sizeof nb, "%s.biases", sl->base);
    if (sl->in % 8) { errf(err, cap, "%s: %d inputs do not pack into 4-bit words", sl->base, sl->in); return false; }
    /* dims: [nbank,] out, cols; rc points at [out, cols] */
    const int lead = sl->nbank ? 1 : 0, nd = 2 + lead;
    int64_t d[3] = {sl->nbank, 0, 0};
    int64_t *rc = d + lead;
    rc[0] = sl->out;
    rc[1] = sl->in / 8;
    const st_tensor *w = expect(ck, nw, ANY_WORDS, nd, d, err, cap);
    if (!w) return false;
    /* the scale columns fix the group: one scale per `group` inputs */
    rc[1] = -1;
    const st_tensor *sc = expect(ck, ns, ANY_BF16, nd, d, err, cap);
    if (!sc) return false;
    const int64_t ncol = sc->shape[nd - 1];
    const int64_t group = ncol > 0 && sl->in % ncol == 0 ? sl->in / ncol : 0;
    if (group != 32 && group != 64) {
        errf(err, cap, "%s: %lld scale columns over %d inputs; the kernels take groups of 32 or 64", ns,
             (long long)ncol, sl->in);
        return false;
    }
    rc[1] = ncol;
    const st_tensor *bi = expect(ck, nb, ANY_BF16, nd, d, err, cap);
    if (!bi) return false;
    sl->dst->group = (int32_t)group;
    return upload(&sl->dst->w, w->data, w->nbytes, nw, err, cap) &&
           upload(&sl->dst->scales, sc->data, sc->nbytes, ns, err, cap) &&
           upload(&sl->dst->biases, bi->data, bi->nbytes, nb, err, cap);
}

/* A small [rows, cols] matrix bound as bf16: "<base>.weight" as stored when
 * bf16, else expanded on the host from packed 4- or 8-bit values with
 * per-group bf16 scales and biases, w = s * q + b rounded to nearest even
 * (the reference's arithmetic for these, qwasar.c:1426-1461). */
static bool bind_bf16(qw_checkpoint ck, qw_ref *dst, const char *base, int64_t rows, int64_t cols, char *err,
                      size_t cap)
{
    char nw[224], ns[224], nb[224];
    snprintf(nw, sizeof nw, "%s.weight", base);
    const st_tensor *w = find(ck, nw);
    if (!w) { errf(err, cap, "checkpoint has no tensor %s", nw); return false; }
    const int64_t d[2] = {rows, cols};
    if (w->dtype == DT_BF16) {
        if (!expect(ck, nw, ANY_BF16, 2, d, err, cap)) return false;
        return upload(dst, w->data, w->nbytes, nw, err, cap);
    }
    /* packed: the word count per row says how wide a value is */
    const int64_t dw[2] = {rows, -1};
    if (!expect(ck, nw, ANY_WORDS, 2, dw, err, cap)) return false;
    const int64_t wpr = w->shape[1];
    const int bits = wpr * 8 == cols ? 4 : wpr * 4 == cols ? 8 : 0;
    if (!bits) {
        errf(err, cap, "%s: %lld words a row hold neither 4- nor 8-bit values for %lld columns", nw,
             (long long)wpr, (long long)cols);
        return false;
    }
    snprintf(ns, sizeof ns, "%s.scales", base);
    snprintf(nb, sizeof nb, "%s.biases", base);
    const st_tensor *sc = expect(ck, ns, ANY_BF16, 2, dw, err, cap);
    if (!sc) return false;
    const int64_t ng = sc->shape[1], gw = ng > 0 && cols % ng == 0 ? cols / ng : 0;
    if (gw == 0 || gw % (32 / bits)) {
        errf(err, cap, "%s: %lld scale columns do not cut %lld %d-bit columns into whole words", ns,
             (long long)ng, (long long)cols, bits);
        return false;
    }
    const int64_t db[2] = {rows, ng};
    const st_tensor *bi = expect(ck, nb, ANY_BF16, 2, db, err, cap);
    if (!bi) return false;
    uint16_t *o = malloc((size_t)(rows * cols) * sizeof *o);
    if (!o) { errf(err, cap, "%s: host memory for the bf16 copy", nw); return false; }
    const uint32_t *W = (const uint32_t *)w->data;   /* safetensors data is 8-byte aligned in the file */
    const uint16_t *S = (const uint16_t *)sc->data, *B = (const uint16_t *)bi->data;
    const int vals = 32 / bits;
    const uint32_t m = (1u << bits) - 1u;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t g = 0; g < ng; g++) {
            const float s = bf16_to_f32(S[r * ng + g]), b = bf16_to_f32(B[r * ng + g]);
            const uint32_t *src = W + r * wpr + g * (gw / vals);
            uint16_t *dst_row = o + r * cols + g * gw;
            for (int64_t k = 0; k < gw; k++) {
                const uint32_t q = (src[k / vals] >> (bits * (int)(k % vals))) & m;
                dst_row[k] = f32_to_bf16(s * (float)q + b);
            }
        }
    const bool ok = upload(dst, o, (size_t)(rows * cols) * sizeof *o, nw, err, cap);
    free(o);
    return ok;
}

bool qw_moe_layer_load(qw_checkpoint ck, int32_t layer, qw_moe_layer *m, char *err, size_t errcap)
{
    if (err && errcap) err[0] = 0;
    if (!ck || !m) { errf(err, errcap, "no checkpoint or layer"); return false; }
    memset(m, 0, sizeof *m);
    if (layer < 0 || layer >= ck->layers) {
        errf(err, errcap, "layer %d is outside 0..%d", layer, ck->layers - 1);
        return false;
    }
    const int32_t H = ck->H, I = ck->I, SI = ck->SI, E = ck->E;
    m->H = H; m->E = E; m->K = ck->K; m->I = I; m->SI = SI; m->norm = ck->norm;
    char mlp[160], base[200];
    snprintf(mlp, sizeof mlp, "language_model.model.layers.%d.mlp", layer);
    snprintf(base, sizeof base, "%s.switch_mlp.gate_proj.weight", mlp);
    m->split = find(ck, base) != NULL;

    /* the plan: banks first, then the shared expert's three matrices */
    typedef struct { qw_q4_ref *dst; const char *leaf; int32_t nbank, out, in; } plan_row;
    plan_row plan[6];
    int n = 0;
    if (m->split) {
        plan[n++] = (plan_row){&m->gate, "switch_mlp.gate_proj", E, I, H};
        plan[n++] = (plan_row){&m->up, "switch_mlp.up_proj", E, I, H};
        plan[n++] = (plan_row){&m->down, "switch_mlp.down_proj", E, H, I};
    } else {
        plan[n++] = (plan_row){&m->gate_up, "experts.gate_up_proj", E, 2 * I, H};
        plan[n++] = (plan_row){&m->down, "experts.down_proj", E, H, I};
    }
    plan[n++] = (plan_row){&m->sh_gate, "shared_expert.gate_proj", 0, SI, H};
    plan[n++] = (plan_row){&m->sh_up, "shared_expert.up_proj", 0, SI, H};
    plan[n++] = (plan_row){&m->sh_down, "shared_expert.down_proj", 0, H, SI};

    snprintf(base, sizeof base, "%s.gate", mlp);
    bool ok = bind_bf16(ck, &m->router, base, E, H, err, errcap);
    for (int i = 0; ok && i < n; i++) {
        q4_slot sl = {plan[i].dst, "", plan[i].nbank, plan[i].out, plan[i].in};
        snprintf(sl.base, sizeof sl.base, "%s.%s", mlp, plan[i].leaf);
        ok = bind_slot(ck, &sl, err, errcap);
    }
    snprintf(base, sizeof base, "%s.shared_expert_gate", mlp);
    if (ok) ok = bind_bf16(ck, &m->sh_gate_w, base, 1, H, err, errcap);
    if (!ok) qw_moe_layer_free(m);
    return ok;
}

static void free_ref(qw_ref *r)
{
    if (r->buf) qw_buf_free(r->buf);
    r->buf = NULL;
}

static void free_q4(qw_q4_ref *q)
{
    free_ref(&q->w);
    free_ref(&q->scales);
    free_ref(&q->biases);
}

void qw_moe_layer_free(qw_moe_layer *m)
{
    if (!m) return;
    free_ref(&m->router);
    free_q4(&m->gate_up);
    free_q4(&m->gate);
    free_q4(&m->up);
    free_q4(&m->down);
    free_q4(&m->sh_gate);
    free_q4(&m->sh_up);
    free_q4(&m->sh_down);
    free_ref(&m->sh_gate_w);
}
