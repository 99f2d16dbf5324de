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
 * and qw_bind_small (:1426-1461).  Same tensor names, same shape checks and
 * the same dequantisation of a small quantised matrix to bf16 (w = scale * q
 * + bias per group, rounded to nearest even), done on the host at load.
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

static const st_tensor *findf(const qw_checkpoint ck, const char *fmt, const char *prefix)
{
    char name[400];
    snprintf(name, sizeof name, fmt, prefix);
    return find(ck, name);
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
        int64_t count = 1;
        for (int i = 0; i < t.ndim; i++) count *= t.shape[i];
        if (off[0] < 0 || off[1] < off[0] || (uint64_t)off[1] > body ||
            (uint64_t)(off[1] - off[0]) != (uint64_t)count * (uint64_t)dt_size[t.dtype]) {
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

/* ---- binding --------------------------------------------------------------- */

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
    if (!b) { errf(err, cap, "cannot place %s (%zu bytes) on the device", what, len); return false; }
    *r = (qw_ref){b, 0};
    return true;
}

static bool is_word(const st_tensor *t) { return t->dtype == DT_U32 || t->dtype == DT_I32; }

/* group from the scale count, as qwasar.c:892-903: 32 or 64 */
static bool group_from_shapes(const st_tensor *sc, int32_t in, const char *prefix, int32_t *g, char *err,
                              size_t cap)
{
    const int64_t groups = sc->ndim ? sc->shape[sc->ndim - 1] : 0;
    const int32_t gs = groups > 0 ? (int32_t)(in / groups) : 0;
    if ((gs != 32 && gs != 64) || (int64_t)gs * groups != in) {
        errf(err, cap, "%s: %lld scale groups over %d inputs is not group 32 or 64", prefix, (long long)groups, in);
        return false;
    }
    *g = gs;
    return true;
}

/* a 4-bit matrix [out, in] (count == 0) or bank [count, out, in] */
static bool bind_q4(qw_checkpoint ck, qw_q4_ref *q, const char *prefix, int32_t count, int32_t in, int32_t out,
                    char *err, size_t cap)
{
    const st_tensor *w = findf(ck, "%s.weight", prefix), *s = findf(ck, "%s.scales", prefix),
                    *b = findf(ck, "%s.biases", prefix);
    if (!w || !s || !b) {
        errf(err, cap, count ? "missing quantised bank %s" : "missing quantised tensors for %s", prefix);
        return false;
    }
    int32_t g;
    if (!group_from_shapes(s, in, prefix, &g, err, cap)) return false;
    const int nd = count ? 3 : 2;
    const int64_t lead = count ? count : out, mid = count ? out : in / 8, words = in / 8, groups = in / g;
    if (!is_word(w) || w->ndim != nd || w->shape[0] != lead || (count && w->shape[1] != out) ||
        w->shape[nd - 1] != words || in % 8) {
        if (count)
            errf(err, cap, "%s.weight is [%lld,%lld,%lld], expected [%d,%d,%lld]", prefix, (long long)w->shape[0],
                 (long long)(w->ndim > 1 ? w->shape[1] : 0), (long long)(w->ndim > 2 ? w->shape[2] : 0), count, out,
                 (long long)words);
        else
            errf(err, cap, "%s.weight is [%lld,%lld], expected [%d,%lld]", prefix, (long long)w->shape[0],
                 (long long)(w->ndim > 1 ? w->shape[1] : 0), out, (long long)mid);
        return false;
    }
    if (s->dtype != DT_BF16 || s->ndim != nd || s->shape[0] != lead || (count && s->shape[1] != out) ||
        s->shape[nd - 1] != groups) {
        errf(err, cap, "%s.scales has %lld groups, expected %lld", prefix, (long long)s->shape[s->ndim - 1],
             (long long)groups);
        return false;
    }
    if (b->dtype != DT_BF16 || b->nbytes != s->nbytes) {
        errf(err, cap, "%s.biases does not match its scales", prefix);
        return false;
    }
    q->group = g;
    return upload(&q->w, w->data, w->nbytes, prefix, err, cap) &&
           upload(&q->scales, s->data, s->nbytes, prefix, err, cap) &&
           upload(&q->biases, b->data, b->nbytes, prefix, err, cap);
}

/* A small bf16 [rows, cols] matrix: as stored when bf16, else dequantised
 * from a 4- or 8-bit affine matrix (qwasar.c:1426-1461). */
static bool bind_small(qw_checkpoint ck, qw_ref *r, const char *prefix, int64_t rows, int64_t cols, char *err,
                       size_t cap)
{
    char p[320];
    snprintf(p, sizeof p, "%s.weight", prefix);
    const st_tensor *w = find(ck, p);
    if (w && w->dtype == DT_BF16) {
        if (w->ndim != 2 || w->shape[0] != rows || w->shape[1] != cols) {
            errf(err, cap, "%s is BF16 [%lld,%lld], expected bf16 [%lld,%lld]", p, (long long)w->shape[0],
                 (long long)(w->ndim > 1 ? w->shape[1] : 0), (long long)rows, (long long)cols);
            return false;
        }
        return upload(r, w->data, w->nbytes, p, err, cap);
    }
    const st_tensor *sc = findf(ck, "%s.scales", prefix), *bi = findf(ck, "%s.biases", prefix);
    if (!w || !sc || !bi || !is_word(w) || w->ndim != 2 || w->shape[0] != rows || sc->ndim != 2 ||
        sc->shape[0] != rows || sc->dtype != DT_BF16 || bi->dtype != DT_BF16 || bi->nbytes != sc->nbytes) {
        errf(err, cap, "%s: neither bf16 [%lld,%lld] nor a quantised matrix of that shape", prefix, (long long)rows,
             (long long)cols);
        return false;
    }
    const int64_t bits = w->shape[1] * 32 / cols, groups = sc->shape[1];
    const int64_t group = groups ? cols / groups : 0;
    if ((bits != 4 && bits != 8) || w->shape[1] * 32 != bits * cols || group * groups != cols ||
        group % (32 / bits) != 0) {
        errf(err, cap, "%s: %lld words and %lld groups per row do not describe %lld inputs", prefix,
             (long long)w->shape[1], (long long)groups, (long long)cols);
        return false;
    }
    uint16_t *out = malloc((size_t)(rows * cols) * 2);
    if (!out) { errf(err, cap, "out of memory for %s", p); return false; }
    const int64_t per = 32 / bits, words = w->shape[1];
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t i = 0; i < rows; i++) {
        for (int64_t j = 0; j < cols; j++) {
            uint32_t word;
            uint16_t s, b;
            memcpy(&word, w->data + 4 * (i * words + j / per), 4);
            memcpy(&s, sc->data + 2 * (i * groups + j / group), 2);
            memcpy(&b, bi->data + 2 * (i * groups + j / group), 2);
            const uint32_t q = (word >> (bits * (j % per))) & mask;
            out[i * cols + j] = f32_to_bf16(bf16_to_f32(s) * (float)q + bf16_to_f32(b));
        }
    }
    const bool ok = upload(r, out, (size_t)(rows * cols) * 2, p, err, cap);
    free(out);
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
    char prefix[256], p[320];
    snprintf(prefix, sizeof prefix, "language_model.model.layers.%d.mlp", layer);
    bool ok;
    snprintf(p, sizeof p, "%s.gate", prefix);
    ok = bind_small(ck, &m->router, p, E, H, err, errcap);
    m->split = findf(ck, "%s.switch_mlp.gate_proj.weight", prefix) != NULL;
    if (ok && m->split) {
        snprintf(p, sizeof p, "%s.switch_mlp.gate_proj", prefix);
        ok = bind_q4(ck, &m->gate, p, E, H, I, err, errcap);
        snprintf(p, sizeof p, "%s.switch_mlp.up_proj", prefix);
        if (ok) ok = bind_q4(ck, &m->up, p, E, H, I, err, errcap);
        snprintf(p, sizeof p, "%s.switch_mlp.down_proj", prefix);
    } else if (ok) {
        snprintf(p, sizeof p, "%s.experts.gate_up_proj", prefix);
        ok = bind_q4(ck, &m->gate_up, p, E, H, 2 * I, err, errcap);
        snprintf(p, sizeof p, "%s.experts.down_proj", prefix);
    }
    if (ok) ok = bind_q4(ck, &m->down, p, E, I, H, err, errcap);
    snprintf(p, sizeof p, "%s.shared_expert.gate_proj", prefix);
    if (ok) ok = bind_q4(ck, &m->sh_gate, p, 0, H, SI, err, errcap);
    snprintf(p, sizeof p, "%s.shared_expert.up_proj", prefix);
    if (ok) ok = bind_q4(ck, &m->sh_up, p, 0, H, SI, err, errcap);
    snprintf(p, sizeof p, "%s.shared_expert.down_proj", prefix);
    if (ok) ok = bind_q4(ck, &m->sh_down, p, 0, SI, H, err, errcap);
    snprintf(p, sizeof p, "%s.shared_expert_gate", prefix);
    if (ok) ok = bind_small(ck, &m->sh_gate_w, p, 1, H, err, errcap);
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
