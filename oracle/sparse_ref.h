/* sparse_ref.h -- CPU oracle for QSA (block indexer, selection, masked
 * attention) and the gated DeltaNet.  TEST INFRASTRUCTURE ONLY: nothing in
 * the product links it.  Each function's reference lines are listed at the
 * top of sparse_ref.c. */
#ifndef QW_SPARSE_REF_H
#define QW_SPARSE_REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float qr_f16_to_f32(uint16_t h);

void qr_rope_tables(uint8_t *axis, float *inv_freq, int32_t rotary_dim, float theta,
                    const int32_t mrope_section[3]);
/* Rotary embedding of the first rotary_dim dims of `heads` vectors, every
 * axis at position `pos`. */
void qr_rope_at(float *x, int32_t pos, const float *inv_freq, int32_t heads, int32_t head_dim,
                int32_t rotary_dim);

void qr_qsa_block_key(float *kn, const float *ikeys, const uint16_t *k_norm, const float *inv_freq,
                      int32_t b, int32_t d, int32_t ratio, int32_t rotary_dim, float eps);
void qr_qsa_scores(float *scores, const float *qn, const float *ikeys, const uint16_t *k_norm,
                   const float *inv_freq, int32_t rows, int32_t nq, int32_t d, int32_t ratio,
                   int32_t base_pos, int32_t rotary_dim, int32_t max_blocks, float eps);
void qr_qsa_pool(float *pool, const float *ikeys, const uint16_t *k_norm, const float *inv_freq,
                 int32_t d, int32_t ratio, int32_t b0, int32_t b1, int32_t rotary_dim, float eps);
void qr_qsa_scores_pooled(float *scores, const float *qn, const float *pool, int32_t rows, int32_t nq,
                          int32_t d, int32_t ratio, int32_t base_pos, int32_t max_blocks);
void qr_qsa_select(uint8_t *mask, uint32_t *list, const float *scores, int32_t rows, int32_t ratio,
                   int32_t base_pos, int32_t block_topk, int32_t max_ctx, int32_t max_blocks);
void qr_attn_masked(float *out, const float *gate, const float *q, const uint16_t *kc, const uint16_t *vc,
                    const uint32_t *list, int32_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t max_ctx, float scale, int32_t list_cap);

void qr_conv1d_causal_silu(float *y, const float *x, float *state, const uint16_t *w, int32_t channels,
                           int32_t rows, int32_t ksize, float *snap, int32_t n_snap, int32_t snap_stride);
void qr_gdn_gates(float *g, float *beta, const float *a, const float *b, const uint16_t *A_log,
                  const uint16_t *dt_bias, int32_t hv, int32_t rows);
void qr_gated_delta(float *y, const float *q, const float *k, const float *v, const float *g,
                    const float *beta, float *state, int32_t hk, int32_t hv, int32_t dk, int32_t dv,
                    int32_t rows, float *snap, int32_t n_snap, int32_t snap_stride);
void qr_gated_delta_prep(float *y, const float *q, const float *k, const float *v, const float *a,
                         const float *b, const uint16_t *A_log, const uint16_t *dt_bias, float l2eps,
                         float q_scale, float k_scale, float *state, int32_t hk, int32_t hv, int32_t dk,
                         int32_t dv, int32_t rows, float *snap, int32_t n_snap, int32_t snap_stride);
void qr_rms_norm_gated_sigmoid(float *y, const float *x, const uint16_t *w, const float *gate,
                               int32_t dim, int32_t rows, float eps, float out_scale);

#ifdef __cplusplus
}
#endif

#endif
