/* encode_moe.c -- a C99 caller of include/qwasar_gpu.h, linked against
 * libqwasar_hip.so, that drives the MoE block op by op in the sequence the
 * reference's graph builder uses (qwasar_flash_graph.c:517-632, encode_moe
 * and encode_shared_down; qwasar_graph.c:492-520, the qlinear helpers):
 *
 *   decode (rows < 8): dmat_bf16 (router) | shared gate+up (qmv_q4_multi,
 *     else one qmat per part) | dmat_bf16 (shared gate) ; moe_route ;
 *     the shared down (qmv_q4_swiglu at one row, else swiglu + qmat) ;
 *     gate/up (qmv_q4_bank2, else two qmv_q4_bank; one bank when fused) ;
 *     qmv_q4_swiglu (down) ; moe_combine_shared
 *   prefill (rows >= 8): the same router and shared gate/up ; moe_route ;
 *     moe_group ; qmm_q4_gather x2 + swiglu (split) or x1 + swiglu_split
 *     (fused) ; qmm_q4_gather (down, by pair) ; the shared down ;
 *     moe_combine_shared
 *
 * It reads a layer and its input from a directory of raw little-endian
 * files written by tests/test_gpu_c_boundary.py (meta.txt holds
 * "H E K I SI split norm group rows"), runs the chain in one command, and
 * writes out.bin (f32 [rows, H]), idx.bin (i32 [rows, K]) and w.bin
 * (f32 [rows, K]) there.  Exit status 0 on success. */
#define _POSIX_C_SOURCE 200112L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qwasar_gpu.h"

#define GROUP_ROWS 8   /* the reference's QW_MOE_GROUP_ROWS */

static char dir[512];

static qw_buf load(const char *name, size_t want) {
    char path[600];
    sprintf(path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "encode_moe: cannot open %s\n", path); exit(2); }
    void *p = NULL;
    if (posix_memalign(&p, 4096, want ? want : 1) != 0) exit(3);
    if (fread(p, 1, want, f) != want) { fprintf(stderr, "encode_moe: %s is short\n", path); exit(2); }
    fclose(f);
    /* qw_buf_wrap: a page-aligned host pointer that outlives the buffer */
    qw_buf b = qw_buf_wrap(p, want);
    if (!b) { fprintf(stderr, "encode_moe: qw_buf_wrap(%s) failed\n", name); exit(3); }
    return b;
}

static qw_buf scratch(size_t n) {
    qw_buf b = qw_buf_alloc(n);
    if (!b) { fprintf(stderr, "encode_moe: qw_buf_alloc(%lu) failed\n", (unsigned long)n); exit(3); }
    return b;
}

static void save(const char *name, qw_buf b, size_t n) {
    char path[600];
    sprintf(path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(qw_buf_contents(b), 1, n, f) != n) { fprintf(stderr, "encode_moe: cannot write %s\n", path); exit(2); }
    fclose(f);
}

/* A quantised linear of the layer: [out, in], 4-bit, `group`. */
typedef struct { qw_buf w, s, b; int32_t in, out, group; } qlin;

static qlin load_q4(const char *stem, int32_t count, int32_t out, int32_t in, int32_t group) {
    char n[64];
    const size_t m = (size_t)(count ? count : 1) * (size_t)out;
    qlin q;
    sprintf(n, "%s.w", stem); q.w = load(n, m * (size_t)in / 2);
    sprintf(n, "%s.s", stem); q.s = load(n, m * (size_t)(in / group) * 2);
    sprintf(n, "%s.b", stem); q.b = load(n, m * (size_t)(in / group) * 2);
    q.in = in; q.out = out; q.group = group;
    return q;
}

static qw_ref at(qw_buf b, size_t off) { qw_ref r; r.buf = b; r.off = off; return r; }

/* qw_encode_qlinear: one projection over `rows` rows. */
static void qlinear(qw_cmd c, const qlin *q, qw_ref out, qw_ref in, int32_t rows) {
    qw_op_qmat_q4(c, out, in, at(q->w, 0), at(q->s, 0), at(q->b, 0), q->in, q->out, rows, q->group);
}

/* qw_encode_qlinear_many: one fused launch at one row when the backend takes
 * it (qw_op_qmv_q4_multi), else one projection each. */
static void qlinear_many(qw_cmd c, qw_ref in, int32_t rows, int32_t count, const qlin *const *q, const qw_ref *out) {
    int fuse = rows == 1 && count <= 4;
    int32_t i;
    for (i = 1; fuse && i < count; i++) fuse = q[i]->in == q[0]->in && q[i]->group == q[0]->group;
    if (fuse) {
        qw_qmv_part parts[4];
        for (i = 0; i < count; i++) {
            parts[i].y = out[i]; parts[i].w = at(q[i]->w, 0); parts[i].scales = at(q[i]->s, 0);
            parts[i].biases = at(q[i]->b, 0); parts[i].n = q[i]->out;
        }
        if (qw_op_qmv_q4_multi(c, in, q[0]->in, q[0]->group, count, parts)) return;
    }
    for (i = 0; i < count; i++) qlinear(c, q[i], out[i], in, rows);
}

/* The layer, its input and the graph builder's scratch (the reference's
 * qw_flash_state fields of the same names). */
typedef struct {
    int32_t H, E, K, I, SI, split, norm, G, rows;
    qw_buf router, sh_gate_w, x;
    qlin gate, up, gate_up, down, sh_gate, sh_up, sh_down;
    qw_buf logits, sh_g, sh_u, sh_gs, ridx, rw, perm, cursor, tiles, exp_gu, exp_act, exp_y, sh_out, out;
} layer;

/* encode_shared_down: the shared expert's SwiGLU and down projection. */
static void shared_down(qw_cmd c, const layer *L) {
    if (L->rows == 1) {
        qw_ref none;
        none.buf = NULL; none.off = 0;
        qw_op_qmv_q4_swiglu(c, at(L->sh_out, 0), at(L->sh_g, 0), at(L->sh_u, 0), L->SI, none, at(L->sh_down.w, 0),
                            at(L->sh_down.s, 0), at(L->sh_down.b, 0), L->SI, L->H, 1, L->G);
        return;
    }
    qw_op_swiglu(c, at(L->sh_g, 0), at(L->sh_g, 0), at(L->sh_u, 0), L->rows * L->SI);
    qlinear(c, &L->sh_down, at(L->sh_out, 0), at(L->sh_g, 0), L->rows);
}

/* The routed experts of many rows: group by expert, gather products. */
static void routed_grouped(qw_cmd c, const layer *L) {
    const int32_t H = L->H, E = L->E, K = L->K, I = L->I, G = L->G, pairs = L->rows * K;
    const qw_ref x = at(L->x, 0), perm = at(L->perm, 0), tiles = at(L->tiles, 0);
    qw_op_moe_group(c, perm, tiles, at(L->cursor, 0), at(L->ridx, 0), pairs, E);
    if (L->split) {
        const qw_ref g = at(L->exp_gu, 0), u = at(L->exp_gu, (size_t)pairs * I * 4);
        qw_op_qmm_q4_gather(c, g, x, perm, tiles, at(L->gate.w, 0), at(L->gate.s, 0), at(L->gate.b, 0),
                            H, I, pairs, E, K, false, G);
        qw_op_qmm_q4_gather(c, u, x, perm, tiles, at(L->up.w, 0), at(L->up.s, 0), at(L->up.b, 0),
                            H, I, pairs, E, K, false, G);
        qw_op_swiglu(c, at(L->exp_act, 0), g, u, pairs * I);
    } else {
        qw_op_qmm_q4_gather(c, at(L->exp_gu, 0), x, perm, tiles, at(L->gate_up.w, 0), at(L->gate_up.s, 0),
                            at(L->gate_up.b, 0), H, 2 * I, pairs, E, K, false, G);
        qw_op_swiglu_split(c, at(L->exp_act, 0), at(L->exp_gu, 0), pairs, I);
    }
    qw_op_qmm_q4_gather(c, at(L->exp_y, 0), at(L->exp_act, 0), perm, tiles, at(L->down.w, 0), at(L->down.s, 0),
                        at(L->down.b, 0), I, H, pairs, E, K, true, G);
}

/* The routed experts of few rows: a matvec per pair; the shared expert's
 * down shares the parallel region with gate/up. */
static void routed_decode(qw_cmd c, const layer *L) {
    const int32_t H = L->H, K = L->K, I = L->I, G = L->G, pairs = L->rows * K;
    const qw_ref x = at(L->x, 0), idx = at(L->ridx, 0), g = at(L->exp_gu, 0);
    qw_ref u;
    int32_t stride;
    qw_cmd_parallel(c, true);
    shared_down(c, L);
    if (L->split) {
        u = at(L->exp_gu, (size_t)pairs * I * 4);
        stride = I;
        if (!qw_op_qmv_q4_bank2(c, g, x, idx, at(L->gate.w, 0), at(L->gate.s, 0), at(L->gate.b, 0),
                                at(L->up.w, 0), at(L->up.s, 0), at(L->up.b, 0), H, I, pairs, K, G)) {
            qw_op_qmv_q4_bank(c, g, x, idx, at(L->gate.w, 0), at(L->gate.s, 0), at(L->gate.b, 0),
                              H, I, pairs, K, false, G);
            qw_op_qmv_q4_bank(c, u, x, idx, at(L->up.w, 0), at(L->up.s, 0), at(L->up.b, 0),
                              H, I, pairs, K, false, G);
        }
    } else {
        u = at(L->exp_gu, (size_t)I * 4);
        stride = 2 * I;
        qw_op_qmv_q4_bank(c, g, x, idx, at(L->gate_up.w, 0), at(L->gate_up.s, 0), at(L->gate_up.b, 0),
                          H, 2 * I, pairs, K, false, G);
    }
    qw_cmd_parallel(c, false);
    qw_op_qmv_q4_swiglu(c, at(L->exp_y, 0), g, u, stride, idx, at(L->down.w, 0), at(L->down.s, 0),
                        at(L->down.b, 0), I, H, pairs, G);
}

static void encode_moe(qw_cmd c, const layer *L) {
    const qw_ref x = at(L->x, 0);
    const qlin *ql[2];
    qw_ref o[2];
    qw_cmd_parallel(c, true);
    qw_op_dmat_bf16(c, at(L->logits, 0), x, at(L->router, 0), L->H, L->E, L->rows);
    ql[0] = &L->sh_gate; ql[1] = &L->sh_up; o[0] = at(L->sh_g, 0); o[1] = at(L->sh_u, 0);
    qlinear_many(c, x, L->rows, 2, ql, o);
    qw_op_dmat_bf16(c, at(L->sh_gs, 0), x, at(L->sh_gate_w, 0), L->H, 1, L->rows);
    qw_cmd_parallel(c, false);
    qw_op_moe_route(c, at(L->ridx, 0), at(L->rw, 0), at(L->logits, 0), L->rows, L->E, L->K, L->norm != 0);
    qw_cmd_mark(c, "moe router");
    if (L->rows >= GROUP_ROWS) {
        routed_grouped(c, L);
        shared_down(c, L);
    } else {
        routed_decode(c, L);
    }
    qw_cmd_mark(c, "moe routed experts");
    qw_op_moe_combine_shared(c, at(L->out, 0), at(L->exp_y, 0), at(L->rw, 0), at(L->sh_out, 0), at(L->sh_gs, 0),
                             L->rows, L->K, L->H);
}

int main(int argc, char **argv) {
    layer L;
    char err[256], p[600];
    FILE *mf;
    qw_cmd c;
    const char *e;
    int32_t pairs;
    const size_t f4 = sizeof(float);
    if (argc != 2) { fprintf(stderr, "usage: encode_moe DIR\n"); return 2; }
    strncpy(dir, argv[1], sizeof dir - 1);
    memset(&L, 0, sizeof L);
    sprintf(p, "%s/meta.txt", dir);
    mf = fopen(p, "r");
    if (!mf || fscanf(mf, "%d %d %d %d %d %d %d %d %d", &L.H, &L.E, &L.K, &L.I, &L.SI, &L.split, &L.norm, &L.G,
                      &L.rows) != 9) {
        fprintf(stderr, "encode_moe: bad meta.txt\n");
        return 2;
    }
    fclose(mf);
    if (!qw_gpu_init(err, sizeof err)) { fprintf(stderr, "encode_moe: %s\n", err); return 4; }
    printf("encode_moe on %s: H %d E %d K %d I %d SI %d %s rows %d\n", qw_gpu_name(), L.H, L.E, L.K, L.I, L.SI,
           L.split ? "split" : "fused", L.rows);
    fflush(stdout);
    pairs = L.rows * L.K;
    L.router = load("router.bin", (size_t)L.E * L.H * 2);
    L.sh_gate_w = load("sh_gate_w.bin", (size_t)L.H * 2);
    L.x = load("x.bin", (size_t)L.rows * L.H * f4);
    if (L.split) {
        L.gate = load_q4("gate", L.E, L.I, L.H, L.G);
        L.up = load_q4("up", L.E, L.I, L.H, L.G);
    } else {
        L.gate_up = load_q4("gate_up", L.E, 2 * L.I, L.H, L.G);
    }
    L.down = load_q4("down", L.E, L.H, L.I, L.G);
    L.sh_gate = load_q4("sh_gate", 0, L.SI, L.H, L.G);
    L.sh_up = load_q4("sh_up", 0, L.SI, L.H, L.G);
    L.sh_down = load_q4("sh_down", 0, L.H, L.SI, L.G);
    L.logits = scratch((size_t)L.rows * L.E * f4);
    L.sh_g = scratch((size_t)L.rows * L.SI * f4);
    L.sh_u = scratch((size_t)L.rows * L.SI * f4);
    L.sh_gs = scratch((size_t)L.rows * f4);
    L.ridx = scratch((size_t)pairs * 4);
    L.rw = scratch((size_t)pairs * f4);
    L.perm = scratch((size_t)pairs * 4);
    L.cursor = scratch((size_t)L.E * 4);
    L.tiles = scratch((size_t)(1 + 3 * qw_moe_max_tiles(pairs, L.E)) * 4);
    L.exp_gu = scratch((size_t)pairs * 2 * L.I * f4);
    L.exp_act = scratch((size_t)pairs * L.I * f4);
    L.exp_y = scratch((size_t)pairs * L.H * f4);
    L.sh_out = scratch((size_t)L.rows * L.H * f4);
    L.out = scratch((size_t)L.rows * L.H * f4);

    c = qw_cmd_begin();
    encode_moe(c, &L);
    qw_cmd_commit(c);
    qw_cmd_wait(c);
    e = qw_cmd_error(c);
    if (e) { fprintf(stderr, "encode_moe: %s\n", e); return 5; }
    qw_cmd_free(c);
    save("out.bin", L.out, (size_t)L.rows * L.H * f4);
    save("idx.bin", L.ridx, (size_t)pairs * 4);
    save("w.bin", L.rw, (size_t)pairs * f4);
    qw_gpu_shutdown();
    printf("encode_moe: done\n");
    return 0;
}
