/* sparse_ref.c -- CPU oracle for the rest of a Flash-Next layer: QSA's block
 * indexer, block selection and masked attention, and the gated DeltaNet
 * (causal conv, gates, delta-rule recurrence, output norm gate).
 *
 * TEST INFRASTRUCTURE ONLY, like moe_ref.c: only tests/ call it, as the
 * checker.  Built with -ffp-contract=off; every sum is serial fp32 in the
 * order written, as the reference's scalar twins are.
 *
 * What each function restates:
 *   qr_rope_tables, qr_rope_at     qwasar_cpu.c:290-319 (every axis at one position)
 *   qr_qsa_block_key               qwasar_flash_cpu.c:378-388 (mean of `ratio` raw keys,
 *                                  qw_cpu_rms_norm with k_norm, rope at the block's first position)
 *   qr_qsa_scores[_pooled], _pool  qwasar_flash_cpu.c:389-392; contract qwasar_gpu.h:620-633
 *   qr_qsa_select                  qwasar_flash_cpu.c:370-402 (k rounds of a serial argmax,
 *                                  strict >, ties to the lower block); list: qwasar_gpu.h:634-641
 *   qr_attn_masked                 qwasar_flash_cpu.c:455-478 over the listed positions, with the
 *                                  fp16 cache arithmetic of qw_cpu_attn_decode (qwasar_cpu.c:357-390)
 *   qr_conv1d_causal_silu          qwasar_cpu.c:217-237; snapshots as qwasar_gpu.h:325-333
 *   qr_gdn_gates                   qwasar_cpu.c:239-249
 *   qr_gated_delta                 qwasar_cpu.c:251-283; snapshots as qwasar_gpu.h:339-348
 *   qr_gated_delta_prep            qwasar_gpu.h:349-358: q, k l2-normed as qw_cpu_rms_norm
 *                                  (no weight, out_scale), gates as qr_gdn_gates, then the recurrence
 *   qr_rms_norm_gated_sigmoid      qwasar_flash_cpu.c:331-338 (qw_cpu_rms_norm, then * sigmoid(gate))
 */
#include "sparse_ref.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static float bf(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float qr_f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        float f = (float)m * 5.9604644775390625e-8f;
        memcpy(&u, &f, 4);
        u |= s;
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }
static float silu_c(float x) { return x / (1.0f + expf(-x)); }     /* qwasar_cpu.c:66 */
static float softplus_c(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* qw_cpu_rms_norm's arithmetic on one row (qwasar_cpu.c:68-82). */
static void rms_row(float *y, const float *x, const uint16_t *w, int32_t dim, float eps, float out_scale) {
    float ss = 0.0f;
    for (int32_t i = 0; i < dim; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps) * out_scale;
    for (int32_t i = 0; i < dim; i++) {
        float v = x[i] * inv;
        if (w) v *= bf(w[i]);
        y[i] = v;
    }
}

void qr_rope_tables(uint8_t *axis, float *inv_freq, int32_t rotary_dim, float theta,
                    const int32_t mrope_section[3]) {
    const int32_t half = rotary_dim / 2;
    for (int32_t j = 0; j < half; j++) {
        axis[j] = 0;
        inv_freq[j] = 1.0f / powf(theta, (float)(2 * j) / (float)rotary_dim);
    }
    for (int32_t a = 1; a <= 2; a++) {
        int32_t lim = mrope_section[a] * 3;
        if (lim > half) lim = half;
        for (int32_t j = a; j < lim; j += 3) axis[j] = (uint8_t)a;
    }
}

void qr_rope_at(float *x, int32_t pos, const float *inv_freq, int32_t heads, int32_t head_dim,
                int32_t rotary_dim) {
    const int32_t half = rotary_dim / 2;
    for (int32_t h = 0; h < heads; h++) {
        float *v = x + (size_t)h * head_dim;
        for (int32_t j = 0; j < half; j++) {
            const float ang = (float)pos * inv_freq[j];
            const float c = cosf(ang), s = sinf(ang);
            const float x0 = v[j], x1 = v[j + half];
            v[j] = x0 * c - x1 * s;
            v[j + half] = x1 * c + x0 * s;
        }
    }
}

void qr_qsa_block_key(float *kn, const float *ikeys, const uint16_t *k_norm, const float *inv_freq,
                      int32_t b, int32_t d, int32_t ratio, int32_t rotary_dim, float eps) {
    float *pooled = malloc((size_t)d * sizeof(float));
    for (int32_t i = 0; i < d; i++) pooled[i] = 0.0f;
    for (int32_t t = 0; t < ratio; t++)
        for (int32_t i = 0; i < d; i++) pooled[i] += ikeys[(size_t)(b * ratio + t) * d + i];
    for (int32_t i = 0; i < d; i++) pooled[i] /= (float)ratio;
    rms_row(kn, pooled, k_norm, d, eps, 1.0f);
    qr_rope_at(kn, b * ratio, inv_freq, 1, d, rotary_dim);
    free(pooled);
}

static float block_score(const float *qn_row, const float *kn, int32_t nq, int32_t d) {
    float sc = 0.0f;
    for (int32_t h = 0; h < nq; h++) {
        float dot = 0.0f;
        for (int32_t i = 0; i < d; i++) dot += qn_row[(size_t)h * d + i] * kn[i];
        if (dot > 0.0f) sc += dot;
    }
    return sc / sqrtf((float)d);
}

void qr_qsa_scores(float *scores, const float *qn, const float *ikeys, const uint16_t *k_norm,
                   const float *inv_freq, int32_t rows, int32_t nq, int32_t d, int32_t ratio,
                   int32_t base_pos, int32_t rotary_dim, int32_t max_blocks, float eps) {
    float *kn = malloc((size_t)d * sizeof(float));
    const int32_t nb_max = (base_pos + rows) / ratio;
    for (int32_t b = 0; b < nb_max; b++) {
        qr_qsa_block_key(kn, ikeys, k_norm, inv_freq, b, d, ratio, rotary_dim, eps);
        for (int32_t r = 0; r < rows; r++)
            if (b < (base_pos + r + 1) / ratio)
                scores[(size_t)r * max_blocks + b] = block_score(qn + (size_t)r * nq * d, kn, nq, d);
    }
    free(kn);
}

void qr_qsa_pool(float *pool, const float *ikeys, const uint16_t *k_norm, const float *inv_freq,
                 int32_t d, int32_t ratio, int32_t b0, int32_t b1, int32_t rotary_dim, float eps) {
    for (int32_t b = b0; b < b1; b++)
        qr_qsa_block_key(pool + (size_t)b * d, ikeys, k_norm, inv_freq, b, d, ratio, rotary_dim, eps);
}

void qr_qsa_scores_pooled(float *scores, const float *qn, const float *pool, int32_t rows, int32_t nq,
                          int32_t d, int32_t ratio, int32_t base_pos, int32_t max_blocks) {
    for (int32_t r = 0; r < rows; r++) {
        const int32_t nb = (base_pos + r + 1) / ratio;
        for (int32_t b = 0; b < nb; b++)
            scores[(size_t)r * max_blocks + b] = block_score(qn + (size_t)r * nq * d, pool + (size_t)b * d, nq, d);
    }
}

void qr_qsa_select(uint8_t *mask, uint32_t *list, const float *scores, int32_t rows, int32_t ratio,
                   int32_t base_pos, int32_t block_topk, int32_t max_ctx, int32_t max_blocks) {
    const int32_t cap = block_topk * ratio + ratio;
    for (int32_t r = 0; r < rows; r++) {
        const int32_t n_keys = base_pos + r + 1, n_blocks = n_keys / ratio;
        uint8_t *m = mask + (size_t)r * max_ctx;
        uint32_t *l = list + (size_t)r * (1 + cap);
        memset(m, 0, (size_t)n_keys);
        for (int32_t t = n_blocks * ratio; t < n_keys; t++) m[t] = 1;
        if (n_blocks > 0) {
            float *s = malloc((size_t)n_blocks * sizeof(float));
            memcpy(s, scores + (size_t)r * max_blocks, (size_t)n_blocks * sizeof(float));
            const int32_t take = block_topk < n_blocks ? block_topk : n_blocks;
            for (int32_t n = 0; n < take; n++) {
                int32_t best = -1;
                for (int32_t b = 0; b < n_blocks; b++)
                    if (s[b] > -FLT_MAX && (best < 0 || s[b] > s[best])) best = b;
                if (best < 0) break;
                for (int32_t t = 0; t < ratio; t++) m[best * ratio + t] = 1;
                s[best] = -FLT_MAX;
            }
            free(s);
        }
        uint32_t n = 0;
        for (int32_t t = 0; t < n_keys; t++)
            if (m[t]) l[1 + n++] = (uint32_t)t;
        l[0] = n;
    }
}

void qr_attn_masked(float *out, const float *gate, const float *q, const uint16_t *kc, const uint16_t *vc,
                    const uint32_t *list, int32_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t max_ctx, float scale, int32_t list_cap) {
    const int32_t gqa = q_heads / kv_heads;
    for (int32_t r = 0; r < rows; r++) {
        const uint32_t *l = list + (size_t)r * (1 + list_cap);
        const int32_t n = (int32_t)l[0];
        float *probs = malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
        for (int32_t h = 0; h < q_heads; h++) {
            const int32_t kvh = h / gqa;
            const float *qv = q + ((size_t)r * q_heads + h) * head_dim;
            float *ov = out + ((size_t)r * q_heads + h) * head_dim;
            float m = -FLT_MAX;
            for (int32_t j = 0; j < n; j++) {
                const uint16_t *kv = kc + ((size_t)kvh * max_ctx + l[1 + j]) * head_dim;
                float s = 0.0f;
                for (int32_t i = 0; i < head_dim; i++) s += qv[i] * scale * qr_f16_to_f32(kv[i]);
                probs[j] = s;
                if (s > m) m = s;
            }
            float sum = 0.0f;
            for (int32_t j = 0; j < n; j++) { probs[j] = expf(probs[j] - m); sum += probs[j]; }
            for (int32_t i = 0; i < head_dim; i++) ov[i] = 0.0f;
            for (int32_t j = 0; j < n; j++) {
                const uint16_t *vv = vc + ((size_t)kvh * max_ctx + l[1 + j]) * head_dim;
                const float p = probs[j] / sum;
                for (int32_t i = 0; i < head_dim; i++) ov[i] += p * qr_f16_to_f32(vv[i]);
            }
            if (gate)
                for (int32_t i = 0; i < head_dim; i++) ov[i] *= sigm(gate[((size_t)r * q_heads + h) * head_dim + i]);
        }
        free(probs);
    }
}

void qr_conv1d_causal_silu(float *y, const float *x, float *state, const uint16_t *w, int32_t channels,
                           int32_t rows, int32_t ksize, float *snap, int32_t n_snap, int32_t snap_stride) {
    for (int32_t ch = 0; ch < channels; ch++) {
        float win[8];
        for (int32_t j = 0; j < ksize - 1; j++) win[j] = state[(size_t)j * channels + ch];
        for (int32_t t = 0; t < rows; t++) {
            win[ksize - 1] = x[(size_t)t * channels + ch];
            float acc = 0.0f;
            for (int32_t j = 0; j < ksize; j++) acc += win[j] * bf(w[(size_t)ch * ksize + j]);
            y[(size_t)t * channels + ch] = silu_c(acc);
            for (int32_t j = 0; j < ksize - 1; j++) win[j] = win[j + 1];
            if (t < n_snap)
                for (int32_t j = 0; j < ksize - 1; j++)
                    snap[(size_t)t * snap_stride + (size_t)j * channels + ch] = win[j];
        }
        for (int32_t j = 0; j < ksize - 1; j++) state[(size_t)j * channels + ch] = win[j];
    }
}

void qr_gdn_gates(float *g, float *beta, const float *a, const float *b, const uint16_t *A_log,
                  const uint16_t *dt_bias, int32_t hv, int32_t rows) {
    for (int32_t i = 0; i < rows * hv; i++) {
        const int32_t h = i % hv;
        const float A = bf(A_log[h]), dt = bf(dt_bias[h]);
        g[i] = expf(-expf(A) * softplus_c(a[i] + dt));
        beta[i] = sigm(b[i]);
    }
}

void qr_gated_delta(float *y, const float *q, const float *k, const float *v, const float *g,
                    const float *beta, float *state, int32_t hk, int32_t hv, int32_t dk, int32_t dv,
                    int32_t rows, float *snap, int32_t n_snap, int32_t snap_stride) {
    const int32_t gqa = hv / hk;
    for (int32_t t = 0; t < rows; t++) {
        for (int32_t h = 0; h < hv; h++) {
            const int32_t hx = h / gqa;
            const float *qt = q + ((size_t)t * hk + hx) * dk;
            const float *kt = k + ((size_t)t * hk + hx) * dk;
            const float *vt = v + ((size_t)t * hv + h) * dv;
            float *yt = y + ((size_t)t * hv + h) * dv;
            float *S = state + (size_t)h * dv * dk;
            const float gt = g[(size_t)t * hv + h], bt = beta[(size_t)t * hv + h];
            for (int32_t r = 0; r < dv; r++) {
                float *Sr = S + (size_t)r * dk;
                float kv = 0.0f;
                for (int32_t c = 0; c < dk; c++) { Sr[c] *= gt; kv += Sr[c] * kt[c]; }
                const float delta = (vt[r] - kv) * bt;
                float o = 0.0f;
                for (int32_t c = 0; c < dk; c++) { Sr[c] += kt[c] * delta; o += Sr[c] * qt[c]; }
                yt[r] = o;
            }
        }
        if (t < n_snap) memcpy(snap + (size_t)t * snap_stride, state, (size_t)hv * dv * dk * sizeof(float));
    }
}

void qr_gated_delta_prep(float *y, const float *q, const float *k, const float *v, const float *a,
                         const float *b, const uint16_t *A_log, const uint16_t *dt_bias, float l2eps,
                         float q_scale, float k_scale, float *state, int32_t hk, int32_t hv, int32_t dk,
                         int32_t dv, int32_t rows, float *snap, int32_t n_snap, int32_t snap_stride) {
    const size_t qn = (size_t)rows * hk * dk, gn = (size_t)rows * hv;
    float *qq = malloc(qn * sizeof(float)), *kk = malloc(qn * sizeof(float));
    float *g = malloc(gn * sizeof(float)), *be = malloc(gn * sizeof(float));
    for (size_t i = 0; i < (size_t)rows * hk; i++) {
        rms_row(qq + i * dk, q + i * dk, NULL, dk, l2eps, q_scale);
        rms_row(kk + i * dk, k + i * dk, NULL, dk, l2eps, k_scale);
    }
    qr_gdn_gates(g, be, a, b, A_log, dt_bias, hv, rows);
    qr_gated_delta(y, qq, kk, v, g, be, state, hk, hv, dk, dv, rows, snap, n_snap, snap_stride);
    free(qq); free(kk); free(g); free(be);
}

void qr_rms_norm_gated_sigmoid(float *y, const float *x, const uint16_t *w, const float *gate,
                               int32_t dim, int32_t rows, float eps, float out_scale) {
    for (int32_t r = 0; r < rows; r++) {
        rms_row(y + (size_t)r * dim, x + (size_t)r * dim, w, dim, eps, out_scale);
        for (int32_t i = 0; i < dim; i++) y[(size_t)r * dim + i] *= sigm(gate[(size_t)r * dim + i]);
    }
}
