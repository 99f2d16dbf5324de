/* moe_ref.c -- CPU oracle for the Flash-Next MoE layer.  TEST INFRASTRUCTURE
 * ONLY: see moe_ref.h for what it restates, the two specified orders, and
 * the checks that pin each function.  Build with -ffp-contract=off so every
 * product and sum below rounds where it is written. */

#include "moe_ref.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

float qr_bf16_to_f32(uint16_t v) {
    /* bf16 is the top half of an fp32 (qwasar_cpu.c:15-19). */
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)v << 16;
    return c.f;
}

uint16_t qr_f32_to_bf16(float f) {
    /* Round to nearest even, as tests/test_sparse.c:45 does. */
    union { float f; uint32_t u; } c;
    c.f = f;
    return (uint16_t)((c.u + 0x7FFFu + ((c.u >> 16) & 1u)) >> 16);
}

/* e^x by Cody-Waite range reduction and a Taylor polynomial.
 *
 *   k = rint(x * log2(e))           x = k ln2 + r,  |r| <= ln2/2 (+ rounding)
 *   r = (x - k ln2_hi) - k ln2_lo   two fmaf steps; ln2_hi has 8 significant
 *                                   bits, so k * ln2_hi is exact for |k| < 2^16
 *   e^r = 1 + r + r^2/2! + ... + r^7/7!   Horner, fmaf per step
 *   e^x = ldexp(e^r, k)             one correctly rounded scaling
 *
 * The truncation error of the degree-7 polynomial at |r| = ln2/2 is
 * (ln2/2)^8 / 8! ~ 5e-9, well under half an ulp; the result is within a
 * couple of ulp of e^x.  The device twin performs the same operations in
 * the same order, so the two agree bit for bit. */
float qr_exp(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410f) return 0.0f;
    const float kf = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(kf, -0.693145751953125f, x);
    r = fmaf(kf, -1.428606765330187045e-06f, r);
    float p = 1.98412698412698412698e-4f;            /* 1/7! */
    p = fmaf(p, r, 1.38888888888888888889e-3f);      /* 1/6! */
    p = fmaf(p, r, 8.33333333333333333333e-3f);      /* 1/5! */
    p = fmaf(p, r, 4.16666666666666666667e-2f);      /* 1/4! */
    p = fmaf(p, r, 1.66666666666666666667e-1f);      /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)kf);
}

void qr_exp_vec(float *out, const float *in, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = qr_exp(in[i]);
}

void qr_dequant_row(float *out, const uint32_t *w, const uint16_t *scales,
                    const uint16_t *biases, int32_t k, int32_t row, int32_t group) {
    /* MLX affine: element i at bit 4*(i%8) of word i/8; w = scale*nib + bias
     * per group of `group` (qwasar_cpu.c:21-38, metal/common.metal:37-46). */
    const uint32_t *wr = w + (size_t)row * (size_t)(k / 8);
    const uint16_t *sr = scales + (size_t)row * (size_t)(k / group);
    const uint16_t *br = biases + (size_t)row * (size_t)(k / group);
    for (int32_t i = 0; i < k; i++) {
        const uint32_t q = (wr[i >> 3] >> (4 * (i & 7))) & 0xFu;
        const float s = qr_bf16_to_f32(sr[i / group]);
        const float b = qr_bf16_to_f32(br[i / group]);
        out[i] = s * (float)q + b;
    }
}

void qr_qmv_q4(float *y, const float *x, const uint32_t *w, const uint16_t *scales,
               const uint16_t *biases, int32_t k, int32_t n, int32_t rows, int32_t group) {
    /* Serial fp32 accumulation of (scale*nib + bias) * x, one output at a
     * time (qwasar_cpu.c:40-63). */
    const size_t words = (size_t)(k / 8), groups = (size_t)(k / group);
    for (int32_t r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * (size_t)k;
        for (int32_t o = 0; o < n; o++) {
            const uint32_t *wr = w + (size_t)o * words;
            const uint16_t *sr = scales + (size_t)o * groups;
            const uint16_t *br = biases + (size_t)o * groups;
            float acc = 0.0f;
            for (int32_t i = 0; i < k; i++) {
                const uint32_t q = (wr[i >> 3] >> (4 * (i & 7))) & 0xFu;
                const float wv = qr_bf16_to_f32(sr[i / group]) * (float)q + qr_bf16_to_f32(br[i / group]);
                acc += wv * xr[i];
            }
            y[(size_t)r * (size_t)n + (size_t)o] = acc;
        }
    }
}

/* Order R: partial_c = fmaf chain over the 64 elements of chunk c starting
 * from 0; the dot is partial_0 + partial_1 + ... added left to right. */
float qr_dot_bf16(const uint16_t *w, const float *x, int32_t k) {
    float total = 0.0f;
    for (int32_t c0 = 0; c0 < k; c0 += QR_ROUTER_CHUNK) {
        const int32_t c1 = c0 + QR_ROUTER_CHUNK < k ? c0 + QR_ROUTER_CHUNK : k;
        float part = 0.0f;
        for (int32_t i = c0; i < c1; i++) part = fmaf(qr_bf16_to_f32(w[i]), x[i], part);
        total = c0 == 0 ? part : total + part;
    }
    return total;
}

void qr_dmat_bf16(float *y, const float *x, const uint16_t *w, int32_t k, int32_t n, int32_t rows) {
    for (int32_t r = 0; r < rows; r++)
        for (int32_t o = 0; o < n; o++)
            y[(size_t)r * (size_t)n + (size_t)o] =
                qr_dot_bf16(w + (size_t)o * (size_t)k, x + (size_t)r * (size_t)k, k);
}

/* The tree sum of the softmax: 64 lane sums, serial within a lane over
 * e = l, l+64, ..., then an xor butterfly over the lanes with ascending
 * offsets 1, 2, 4, 8, 16, 32 (adjacent pairs first). */
static float tree_sum(const float *v, int32_t n) {
    float lane[QR_SUM_LANES];
    for (int32_t l = 0; l < QR_SUM_LANES; l++) {
        float s = 0.0f;
        for (int32_t e = l; e < n; e += QR_SUM_LANES) s = s + v[e];
        lane[l] = s;
    }
    for (int32_t off = 1; off < QR_SUM_LANES; off <<= 1) {
        float nxt[QR_SUM_LANES];
        for (int32_t l = 0; l < QR_SUM_LANES; l++) nxt[l] = lane[l] + lane[l ^ off];
        memcpy(lane, nxt, sizeof lane);
    }
    return lane[0];
}

/* K picks by strict '>' scanning up from e = 0, a pick struck to -1
 * (qwasar_flash_cpu.c:505-514), then the optional renormalisation (:521). */
static void pick_topk(int32_t *idx, float *w, float *p, int32_t E, int32_t K, int32_t norm) {
    float wsum = 0.0f;
    for (int32_t n = 0; n < K; n++) {
        int32_t best = -1;
        for (int32_t e = 0; e < E; e++)
            if (p[e] >= 0.0f && (best < 0 || p[e] > p[best])) best = e;
        idx[n] = best;
        w[n] = p[best];
        wsum += w[n];
        p[best] = -1.0f;
    }
    if (norm)
        for (int32_t n = 0; n < K; n++) w[n] /= wsum;
}

void qr_route(int32_t *idx, float *w, const float *logits, int32_t rows, int32_t E,
              int32_t K, int32_t norm) {
    float *p = malloc((size_t)E * sizeof(float));
    for (int32_t r = 0; r < rows; r++) {
        const float *l = logits + (size_t)r * (size_t)E;
        float m = -FLT_MAX;
        for (int32_t e = 0; e < E; e++) if (l[e] > m) m = l[e];
        for (int32_t e = 0; e < E; e++) p[e] = qr_exp(l[e] - m);
        const float sum = tree_sum(p, E);
        for (int32_t e = 0; e < E; e++) p[e] = p[e] / sum;
        pick_topk(idx + (size_t)r * (size_t)K, w + (size_t)r * (size_t)K, p, E, K, norm);
    }
    free(p);
}

void qr_route_literal(int32_t *idx, float *w, const float *logits, int32_t rows, int32_t E,
                      int32_t K, int32_t norm) {
    float *p = malloc((size_t)E * sizeof(float));
    for (int32_t r = 0; r < rows; r++) {
        const float *l = logits + (size_t)r * (size_t)E;
        float m = -FLT_MAX;
        for (int32_t e = 0; e < E; e++) if (l[e] > m) m = l[e];
        float sum = 0.0f;
        for (int32_t e = 0; e < E; e++) { p[e] = expf(l[e] - m); sum += p[e]; }
        for (int32_t e = 0; e < E; e++) p[e] /= sum;
        pick_topk(idx + (size_t)r * (size_t)K, w + (size_t)r * (size_t)K, p, E, K, norm);
    }
    free(p);
}

int32_t qr_max_tiles(int32_t pairs, int32_t E, int32_t bm) {
    /* Every expert with pairs opens at most one partial tile, and full tiles
     * number at most pairs / bm (reference qw_moe_max_tiles,
     * qwasar_metal.m:1757-1764). */
    return (pairs < E ? pairs : E) + (pairs + bm - 1) / bm;
}

int32_t qr_moe_group(int32_t *perm, int32_t *tiles, const int32_t *idx, int32_t pairs,
                     int32_t E, int32_t bm, int32_t max_tiles) {
    /* Counting sort by expert, stable in pair index; the reference's tile
     * list format (metal/sparse.metal:340-392) with its atomic scatter
     * replaced by this defined order. */
    int32_t *cnt = calloc((size_t)E + 1, sizeof(int32_t));
    for (int32_t p = 0; p < pairs; p++) cnt[idx[p]]++;
    int32_t running = 0, nt = 0;
    for (int32_t e = 0; e < E; e++) {
        const int32_t c = cnt[e];
        for (int32_t s = 0; s < c && nt < max_tiles; s += bm) {
            tiles[1 + 3 * nt + 0] = e;
            tiles[1 + 3 * nt + 1] = running + s;
            tiles[1 + 3 * nt + 2] = c - s < bm ? c - s : bm;
            nt++;
        }
        cnt[e] = running;
        running += c;
    }
    tiles[0] = nt;
    for (int32_t p = 0; p < pairs; p++) perm[cnt[idx[p]]++] = p;
    free(cnt);
    return nt;
}

float qr_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float qr_silu(float x) { return x * qr_sigmoid(x); }

/* y[0:n] = rows [row0, row0+n) of a quantised matrix times x. */
static void qmv_rows(float *y, const float *x, const qr_q4 *q, int64_t row0, int32_t n, int32_t k) {
    const size_t words = (size_t)(k / 8), groups = (size_t)(k / q->group);
    qr_qmv_q4(y, x, q->w + (size_t)row0 * words, q->s + (size_t)row0 * groups,
              q->b + (size_t)row0 * groups, k, n, 1, q->group);
}

void qr_moe_forward(float *out, int32_t *idx, float *w, const float *x, int32_t rows,
                    const qr_moe *M) {
    const int32_t H = M->H, E = M->E, K = M->K, I = M->I, SI = M->SI;
    float *logits = malloc((size_t)E * sizeof(float));
    float *gu = malloc((size_t)2 * (size_t)I * sizeof(float));
    float *act = malloc((size_t)I * sizeof(float));
    float *y = malloc((size_t)H * sizeof(float));
    float *sg = malloc((size_t)SI * sizeof(float));
    float *su = malloc((size_t)SI * sizeof(float));

    for (int32_t r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * (size_t)H;
        float *o = out + (size_t)r * (size_t)H;
        int32_t *ir = idx + (size_t)r * (size_t)K;
        float *wr = w + (size_t)r * (size_t)K;

        qr_dmat_bf16(logits, xr, M->router, H, E, 1);
        qr_route(ir, wr, logits, 1, E, K, M->norm);

        for (int32_t i = 0; i < H; i++) o[i] = 0.0f;
        for (int32_t n = 0; n < K; n++) {
            const int64_t e = ir[n];
            if (M->split) {
                qmv_rows(gu, xr, &M->gate, e * I, I, H);
                qmv_rows(gu + I, xr, &M->up, e * I, I, H);
            } else {
                qmv_rows(gu, xr, &M->gate_up, e * 2 * I, 2 * I, H);
            }
            for (int32_t i = 0; i < I; i++) act[i] = qr_silu(gu[i]) * gu[I + i];
            qmv_rows(y, act, &M->down, e * H, H, I);
            for (int32_t i = 0; i < H; i++) o[i] += wr[n] * y[i];
        }

        qmv_rows(sg, xr, &M->sh_gate, 0, SI, H);
        qmv_rows(su, xr, &M->sh_up, 0, SI, H);
        for (int32_t i = 0; i < SI; i++) sg[i] = qr_silu(sg[i]) * su[i];
        qmv_rows(y, sg, &M->sh_down, 0, H, SI);
        const float gs = qr_sigmoid(qr_dot_bf16(M->sh_gate_w, xr, H));
        for (int32_t i = 0; i < H; i++) o[i] += gs * y[i];
    }
    free(logits); free(gu); free(act); free(y); free(sg); free(su);
}

void qr_rms_norm(float *y, const float *x, int32_t dim, int32_t rows, float eps) {
    /* Unit-weight RMS norm in the form of qwasar_cpu.c:68-82. */
    for (int32_t r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * (size_t)dim;
        float *yr = y + (size_t)r * (size_t)dim;
        float ss = 0.0f;
        for (int32_t i = 0; i < dim; i++) ss += xr[i] * xr[i];
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
        for (int32_t i = 0; i < dim; i++) yr[i] = xr[i] * inv;
    }
}

/* ---- the hyper-connection mixer ------------------------------------------- */

void qr_rms_norm_grouped(float *y, const float *x, const uint16_t *w, int32_t dim, int32_t groups,
                         int32_t rows, float eps) {
    /* qwasar_flash_cpu.c:57-70 per row: each group normalised on its own
     * (qwasar_cpu.c:68-82's form), times its slice of the full-width weight */
    for (int32_t r = 0; r < rows; r++)
        for (int32_t g = 0; g < groups; g++) {
            const size_t o = ((size_t)r * groups + g) * (size_t)dim;
            float ss = 0.0f;
            for (int32_t i = 0; i < dim; i++) ss += x[o + i] * x[o + i];
            const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
            for (int32_t i = 0; i < dim; i++) {
                float v = x[o + i] * inv;
                v *= qr_bf16_to_f32(w[(size_t)g * dim + i]);
                y[o + i] = v;
            }
        }
}

void qr_silu_scale(float *y, int64_t n, float scale) {
    for (int64_t i = 0; i < n; i++) y[i] = qr_silu(y[i] * scale);
}

void qr_hc_mix(float *x, const float *n, const float *m, int32_t rows, int32_t H, int32_t S) {
    /* qwasar_flash_cpu.c:275-282 */
    for (int32_t r = 0; r < rows; r++)
        for (int32_t i = 0; i < H; i++) {
            float acc = 0.0f;
            for (int32_t s = 0; s < S; s++) {
                const size_t j = (size_t)r * S * H + (size_t)s * H + i;
                acc += qr_sigmoid(m[j]) * n[j];
            }
            x[(size_t)r * H + i] = acc / (float)S;
        }
}

void qr_hc_inject(float *h4, const float *out, const float *inj, int32_t rows, int32_t H, int32_t S) {
    /* qwasar_flash_cpu.c:283-285 and :289-293, with the GPU op's raw logits */
    for (int32_t r = 0; r < rows; r++)
        for (int32_t s = 0; s < S; s++) {
            const float wgt = 2.0f * qr_sigmoid(inj[(size_t)r * S + s] / (float)S);
            for (int32_t i = 0; i < H; i++)
                h4[((size_t)r * S + s) * H + i] += out[(size_t)r * H + i] * wgt;
        }
}

void qr_repeat_cols(float *h4, const float *x, int32_t rows, int32_t H, int32_t S) {
    for (int32_t r = 0; r < rows; r++)
        for (int32_t s = 0; s < S; s++)
            for (int32_t i = 0; i < H; i++) h4[((size_t)r * S + s) * H + i] = x[(size_t)r * H + i];
}
