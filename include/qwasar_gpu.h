#ifndef QWASAR_GPU_H
#define QWASAR_GPU_H

/* qwasar_gpu.h -- the GPU op boundary for qwasar's Flash-Next MoE layer, as
 * implemented for one AMD Instinct MI355X (gfx950) by qwasar_hip.c.
 *
 * This is the subset of the reference's own qwasar_gpu.h that the MoE path
 * crosses (reference qwasar_gpu.h:13-82 runtime, :102-118 and :180-192
 * quantised/dense products, :316-317 swiglu, :384 add, :559-616 MoE ops).
 * Every declaration keeps the reference's name, argument order, argument
 * meaning and error convention, so the reference's callers
 * (qwasar_flash_graph.c:531-632 encode_moe, tests/test_sparse.c,
 * tools/bench/gmmbench.c) link against this backend unchanged.  The last
 * section lists additions that have no counterpart in the reference.
 *
 * Conventions (as in the reference):
 *   - void ops return without encoding anything when `c` is NULL;
 *   - an unsupported shape prints one line to stderr and encodes nothing;
 *   - bool ops return false, encoding nothing, when the shape does not apply;
 *   - device errors are reported by qw_cmd_error after qw_cmd_wait.
 *
 * Buffers are host-visible: qw_buf_contents returns host memory that mirrors
 * the device copy.  Write a buffer through the pointer returned by a fresh
 * qw_buf_contents call; the next op that touches the buffer uploads it.  After
 * qw_cmd_wait, every buffer an op wrote and whose contents were ever taken is
 * copied back, so pointers held across the wait see the results. */

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device (reference qwasar_gpu.h:16-28) ---------------------------------- */

typedef struct qw_buf_s *qw_buf;

/* Brings up the first HIP device and the backend's stream.  Returns false and
 * fills `err` when there is no usable gfx950 device. */
bool qw_gpu_init(char *err, size_t errcap);
void qw_gpu_shutdown(void);
const char *qw_gpu_name(void);
uint64_t qw_gpu_working_set_limit(void);   /* free device memory at init */
uint64_t qw_gpu_max_buffer_length(void);   /* total device memory */

/* ---- buffers (reference qwasar_gpu.h:30-37) --------------------------------- */

/* Copies `len` bytes at `ptr` to a new device buffer once; `ptr` must stay
 * valid for the buffer's lifetime and is what qw_buf_contents returns. */
qw_buf qw_buf_wrap(void *ptr, size_t len);
/* A device buffer with a pinned host mirror, zero-filled. */
qw_buf qw_buf_alloc(size_t len);
void   qw_buf_free(qw_buf b);
void  *qw_buf_contents(qw_buf b);
size_t qw_buf_length(qw_buf b);

/* ---- dispatch (reference qwasar_gpu.h:39-69) -------------------------------- */

typedef struct { qw_buf buf; size_t off; } qw_ref;

static inline qw_ref qw_ref_at(qw_buf b, size_t off) { qw_ref r = { b, off }; return r; }
static inline qw_ref qw_ref_offset(qw_ref r, size_t off) { r.off += off; return r; }

typedef struct qw_cmd_s *qw_cmd;

/* Ops are launched on the backend's one in-order HIP stream as they are
 * encoded; commit and flush therefore only mark submission points. */
qw_cmd qw_cmd_begin(void);
void   qw_cmd_commit(qw_cmd c);
void   qw_cmd_wait(qw_cmd c);
void   qw_cmd_flush(qw_cmd c);
/* Regions whose ops the caller vouches are independent.  Accepted and
 * ignored: the in-order stream is always a correct schedule. */
void   qw_cmd_parallel(qw_cmd c, bool on);
void   qw_cmd_free(qw_cmd c);
const char *qw_cmd_error(qw_cmd c);

/* ---- residency (reference qwasar_gpu.h:71-75) ------------------------------- */

/* Device buffers never page out on this backend; always NULL. */
typedef void *qw_residency;
qw_residency qw_residency_new(qw_buf *bufs, int32_t n);
void         qw_residency_free(qw_residency r);

/* ---- profiling (reference qwasar_gpu.h:77-82) ------------------------------- */

/* QWASAR_PROFILE=1: qw_cmd_mark records a HIP event on the stream and charges
 * the device time since the previous mark (or since qw_cmd_begin) to `label`;
 * totals are gathered at qw_cmd_wait. */
bool qw_prof_enabled(void);
void qw_cmd_mark(qw_cmd c, const char *label);
void qw_prof_report(FILE *out, long tokens);
void qw_prof_reset(void);

/* ---- quantised and dense products (reference qwasar_gpu.h:84-192) ---------- */

/* y[r][n] = sum_k dequant(w)[n][k] * x[r][k]; w U32 [n, k/8] MLX affine 4-bit,
 * scales/biases BF16 [n, k/group], x F32 [rows, k], y F32 [rows, n]. */
void qw_op_qmat_q4(qw_cmd c, qw_ref y, qw_ref x,
                   qw_ref w, qw_ref scales, qw_ref biases,
                   int32_t k, int32_t n, int32_t rows, int32_t group);

/* Up to four one-token matvecs sharing x [1, k] and group, in one launch.
 * False, nothing encoded, for count outside 1..4 or k < 2048 (reference
 * qwasar_gpu.h:105-110); the caller then encodes one qmv per part. */
typedef struct { qw_ref y, w, scales, biases; int32_t n; } qw_qmv_part;
bool qw_op_qmv_q4_multi(qw_cmd c, qw_ref x, int32_t k, int32_t group,
                        int32_t count, const qw_qmv_part *parts);

void qw_op_qmv_q4(qw_cmd c, qw_ref y, qw_ref x,
                  qw_ref w, qw_ref scales, qw_ref biases,
                  int32_t k, int32_t n, int32_t rows, int32_t group);
void qw_op_qmm_q4(qw_cmd c, qw_ref y, qw_ref x,
                  qw_ref w, qw_ref scales, qw_ref biases,
                  int32_t k, int32_t n, int32_t rows, int32_t group);
void qw_op_qmvb_q4(qw_cmd c, qw_ref y, qw_ref x,
                   qw_ref w, qw_ref scales, qw_ref biases,
                   int32_t k, int32_t n, int32_t rows, int32_t group);

/* y = x * w^T, w BF16 [n, k], x F32 [rows, k], y F32 [rows, n].  Summed in
 * order R (64-element fmaf chains added left to right), the order routing's
 * bit-exactness is defined in. */
void qw_op_dmat_bf16(qw_cmd c, qw_ref y, qw_ref x, qw_ref w,
                     int32_t k, int32_t n, int32_t rows);

/* ---- normalisation (reference qwasar_gpu.h:269-276) ------------------------- */

/* RMS norm over the last axis of an [rows, dim] fp32 buffer; `weight` (bf16
 * [dim]) may be a null ref; `out_scale` applies after normalising, before the
 * weight.  dim % 4 == 0 here. */
void qw_op_rms_norm(qw_cmd c, qw_ref y, qw_ref x, qw_ref weight,
                    int32_t dim, int32_t rows, float eps, float out_scale);

/* ---- elementwise (reference qwasar_gpu.h:316-317, :384) --------------------- */

void qw_op_swiglu(qw_cmd c, qw_ref y, qw_ref gate, qw_ref up, int32_t n);
void qw_op_add_inplace(qw_cmd c, qw_ref y, qw_ref x, int32_t n);

/* ---- the hyper-connection mixer around a block (reference qwasar_gpu.h:549-578) -
 *
 * S streams of H per row (h4 [rows, S*H]).  H % 4 == 0 here. */

/* h4 += out (x) 2*sigmoid(inj / S) per stream, then n4 = the streams normed
 * with gains w (qw_op_hc_inject, qw_op_rms_norm_grouped): one pass. */
void qw_op_hc_inject_norm(qw_cmd c, qw_ref h4, qw_ref out, qw_ref inj, qw_ref w, qw_ref n4,
                          int32_t rows, int32_t H, int32_t S, float eps);
/* x = mean_s sigmoid(W_s . silu(scale * d)) * n4_s, W_s the up-projection's
 * rows s*H.. (4-bit, `group`), for few rows.  False, nothing encoded, if S > 4. */
bool qw_op_hc_mix_up(qw_cmd c, qw_ref x, qw_ref d, qw_ref n4, qw_ref w, qw_ref scales, qw_ref biases,
                     int32_t k, int32_t H, int32_t S, int32_t rows, float scale, int32_t group);
/* The first half of a decode step (one row) in one launch: h4_out = h4 with
 * the block's output injected, n4 its grouped norm (qw_op_hc_inject_norm),
 * d = down . n4 (4-bit [lowrank, S*H], `group`), inj_out = inj_w . n4 (bf16
 * [S, S*H], order R).  No output (h4_out, n4, d, inj_out) may overlap an
 * input (h4, out, inj) or another output.  False, nothing encoded, for such
 * an overlap, for S above 4, or S*H above 15360 or not a multiple of 64. */
bool qw_op_hc_pre_decode(qw_cmd c, qw_ref h4_out, qw_ref n4, qw_ref d, qw_ref inj_out, qw_ref h4, qw_ref out,
                         qw_ref inj, qw_ref norm_w, qw_ref down_w, qw_ref down_s, qw_ref down_b, qw_ref inj_w,
                         int32_t H, int32_t S, int32_t lowrank, int32_t group, float eps);
/* A whole mixer decode step (one row) in one launch: qw_op_hc_pre_decode's
 * outputs (h4_out, n4, d, inj_out) and qw_op_hc_mix_up's x at rows 1 with
 * the given scale, the up-projection 4-bit [S*H, lowrank].  The launch
 * hands d over between its workgroups (a hand-off failure is reported as
 * the MoE decode's is, by qw_cmd_error after qw_cmd_wait).  No counterpart
 * op in the reference, which runs these steps as separate passes
 * (metal/sparse.metal:14-189).  False, nothing encoded, for the overlaps and
 * shapes qw_op_hc_pre_decode refuses (x counting as an output), and for
 * lowrank above 512 or not a multiple of 8 and of group. */
bool qw_op_hc_decode(qw_cmd c, qw_ref x, qw_ref h4_out, qw_ref n4, qw_ref d, qw_ref inj_out, qw_ref h4,
                     qw_ref out, qw_ref inj, qw_ref norm_w, qw_ref down_w, qw_ref down_s, qw_ref down_b,
                     qw_ref inj_w, qw_ref up_w, qw_ref up_s, qw_ref up_b, int32_t H, int32_t S, int32_t lowrank,
                     int32_t group, float eps, float scale);
/* h4[r, s*H+i] = x[r, i]. */
void qw_op_repeat_cols(qw_cmd c, qw_ref h4, qw_ref x, int32_t rows, int32_t H, int32_t S);
/* Grouped RMS norm: `groups` streams of `dim` per row, weight [groups*dim]. */
void qw_op_rms_norm_grouped(qw_cmd c, qw_ref y, qw_ref x, qw_ref weight,
                            int32_t dim, int32_t groups, int32_t rows, float eps);
/* y = silu(y * scale) in place. */
void qw_op_silu_scale(qw_cmd c, qw_ref y, int32_t n, float scale);
/* x[r] = mean over streams of sigmoid(m) * n. */
void qw_op_hc_mix(qw_cmd c, qw_ref x, qw_ref n, qw_ref m, int32_t rows, int32_t H, int32_t S);
/* h4 += out (x) 2*sigmoid(inj / S), per stream. */
void qw_op_hc_inject(qw_cmd c, qw_ref h4, qw_ref out, qw_ref inj, int32_t rows, int32_t H, int32_t S);

/* ---- gated DeltaNet (reference qwasar_gpu.h:318-358) ------------------------
 *
 * The recurrent sublayer's ops.  They carry state across calls: `state` is
 * read and written in place.  `snap` receives the state as it stood after
 * each of the first n_snap rows, snap_stride floats apart (n_snap 0: none). */

/* Causal depthwise conv over [rows, channels] with silu fused; state
 * [ksize-1, channels] fp32 in and out, oldest sample first; weight bf16
 * [channels, ksize].  ksize 4 only (refused otherwise, as the reference's). */
void qw_op_conv1d_causal_silu(qw_cmd c, qw_ref y, qw_ref x, qw_ref state,
                              qw_ref weight, int32_t channels, int32_t rows,
                              int32_t ksize, qw_ref snap, int32_t n_snap,
                              int32_t snap_stride);
/* g = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b);
 * a, b, g, beta F32 [rows, n_v_heads]; A_log, dt_bias BF16 [n_v_heads]. */
void qw_op_gdn_gates(qw_cmd c, qw_ref g, qw_ref beta, qw_ref a, qw_ref b,
                     qw_ref A_log, qw_ref dt_bias, int32_t n_v_heads, int32_t rows);
/* The delta rule per value head over `rows` timesteps: S *= g; kv = S k;
 * S += k (v - kv) beta; y = S q.  state F32 [hv, dv, dk]; q, k [rows, hk, dk]
 * already l2-normed; v, y [rows, hv, dv]; value head h reads key head
 * h / (hv / hk).  dk = dv = 128 only (refused otherwise, as the reference's). */
void qw_op_gated_delta(qw_cmd c, qw_ref y, qw_ref q, qw_ref k, qw_ref v,
                       qw_ref g, qw_ref beta, qw_ref state,
                       int32_t hk, int32_t hv, int32_t dk, int32_t dv, int32_t rows,
                       qw_ref snap, int32_t n_snap, int32_t snap_stride);
/* The same with its inputs' preparation inside: q and k raw, normed as
 * x / sqrt(mean x^2 + l2eps) * q_scale (k_scale); g and beta from a, b,
 * A_log and dt_bias as qw_op_gdn_gates. */
typedef struct {
    qw_ref a, b, A_log, dt_bias;
    float l2eps, q_scale, k_scale;
} qw_gdn_prep;
void qw_op_gated_delta_prep(qw_cmd c, qw_ref y, qw_ref q, qw_ref k, qw_ref v,
                            const qw_gdn_prep *prep, qw_ref state,
                            int32_t hk, int32_t hv, int32_t dk, int32_t dv, int32_t rows,
                            qw_ref snap, int32_t n_snap, int32_t snap_stride);
/* One decode step of the recurrent sublayer in one launch: the conv with
 * silu over the mixed channels x [2 hk dk + hv dv], then the prepared delta
 * rule on its q [0, hk dk), k [hk dk, 2 hk dk) and v [2 hk dk, ...) channels
 * (the split of the reference's gdn_step, qwasar_flash_cpu.c:318-320).  No
 * counterpart in the reference, which runs qw_op_conv1d_causal_silu and then
 * qw_op_gated_delta_prep on the conv's output; the same bits as those two.
 * The conv window is read from conv_state and written to conv_state_out
 * ([3, channels] each, oldest first), which may not overlap conv_state or x
 * (callers alternate two windows); state as qw_op_gated_delta.  dk = dv =
 * 128; false and nothing encoded for other shapes or overlapping windows. */
bool qw_op_gdn_decode(qw_cmd c, qw_ref y, qw_ref x, qw_ref conv_state, qw_ref conv_state_out,
                      qw_ref conv_weight, const qw_gdn_prep *prep, qw_ref state,
                      int32_t hk, int32_t hv, int32_t dk, int32_t dv);
/* rms_norm(x, weight) * sigmoid(gate) per row of `dim` (reference
 * qwasar_gpu.h:618-620): the delta net's output gate.  weight may be a null
 * ref (unit gain). */
void qw_op_rms_norm_gated_sigmoid(qw_cmd c, qw_ref y, qw_ref x, qw_ref weight, qw_ref gate,
                                  int32_t dim, int32_t rows, float eps, float out_scale);

/* ---- QSA: block indexer, selection, masked attention (reference
 * qwasar_gpu.h:621-646) ------------------------------------------------------
 *
 * A query row r sits at position base_pos + r and sees keys 0..base_pos + r;
 * its complete blocks of `ratio` keys are n = (base_pos + r + 1) / ratio.
 * Block scores: scores F32 [rows, max_blocks], entry (r, b) for b < n:
 *   key_b = rope(rms_norm(mean of the block's raw keys) * k_norm) at position
 *           b * ratio (the first 64 dims, pairs (j, j + 32));
 *   score = sum over query heads of max(0, qn[r, h] . key_b) / sqrt(d).
 * qn F32 [rows, nq, d] normed and rotated by the caller; ikeys F32
 * [max_ctx, d]; k_norm BF16 [d]; inv_freq F32 [32].  rotary_dim 64 and d a
 * multiple of 32 up to 256 (refused otherwise, as the reference's). */
void qw_op_qsa_scores(qw_cmd c, qw_ref scores, qw_ref qn, qw_ref ikeys, qw_ref k_norm,
                      qw_ref inv_freq, int32_t rows, int32_t nq, int32_t d, int32_t ratio,
                      int32_t base_pos, int32_t rotary_dim, int32_t max_blocks, float eps);
/* Blocks [b0, b1)'s keys, computed exactly as qw_op_qsa_scores does, into
 * pool F32 [max_blocks, d]; qw_op_qsa_scores_pooled scores from them and
 * gives qw_op_qsa_scores' bits. */
void qw_op_qsa_pool(qw_cmd c, qw_ref pool, qw_ref ikeys, qw_ref k_norm, qw_ref inv_freq,
                    int32_t d, int32_t ratio, int32_t b0, int32_t b1, int32_t rotary_dim, float eps);
void qw_op_qsa_scores_pooled(qw_cmd c, qw_ref scores, qw_ref qn, qw_ref pool, int32_t rows,
                             int32_t nq, int32_t d, int32_t ratio, int32_t base_pos, int32_t max_blocks);
/* Selection: the block_topk best complete blocks (score descending, ties to
 * the lower block; a score of -FLT_MAX or below, or NaN, is never taken, as in
 * the reference's CPU selection, qwasar_flash_cpu.c:395-402; its Metal kernel,
 * metal/sparse.metal:965-1030, instead orders every float, NaN above +inf and
 * -inf lowest, and always takes min(block_topk, blocks)) and the incomplete
 * tail are visible.  mask U8 [rows, max_ctx] gets 1/0 for
 * positions 0..base_pos + r; list U32 [rows, 1 + qw_qsa_list_cap] the count,
 * then the visible positions ascending.  Up to 65536 blocks a row. */
static inline int32_t qw_qsa_list_cap(int32_t block_topk, int32_t ratio) {
    return block_topk * ratio + ratio;
}
void qw_op_qsa_select(qw_cmd c, qw_ref mask, qw_ref list, qw_ref scores, int32_t rows, int32_t ratio,
                      int32_t base_pos, int32_t block_topk, int32_t max_ctx, int32_t max_blocks);
/* Attention over the listed positions only: out F32 [rows, q_heads, 256] =
 * softmax(scale q . K) V, q F32 [rows, q_heads, 256], the caches FP16
 * [kv_heads, max_ctx, 256]; query head h reads kv head h / (q_heads /
 * kv_heads), a ratio of 1, 2, 4, 8, 12 or 16.  The gated form then multiplies by
 * sigmoid(gate) [rows, q_heads, 256].  head_dim 256 only. */
void qw_op_attn_masked(qw_cmd c, qw_ref out, qw_ref q, qw_ref kcache, qw_ref vcache, qw_ref list,
                       int32_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                       int32_t max_ctx, int32_t base_pos, float scale, int32_t block_topk, int32_t ratio);
void qw_op_attn_masked_gated(qw_cmd c, qw_ref out, qw_ref gate, qw_ref q, qw_ref kcache, qw_ref vcache,
                             qw_ref list, int32_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                             int32_t max_ctx, int32_t base_pos, float scale, int32_t block_topk, int32_t ratio);

/* ---- the MoE block (reference qwasar_gpu.h:559-616) ------------------------- */

/* out[r] = sum_k w[r,k] y[r*K+k] + sigmoid(g[r]) sh[r]. */
void qw_op_moe_combine_shared(qw_cmd c, qw_ref out, qw_ref y, qw_ref w, qw_ref sh, qw_ref g,
                              int32_t rows, int32_t K, int32_t H);
/* Softmax over E in fp32, top-K (ties to the lower index), renormalised when
 * `norm`.  idx I32 [rows, K], w F32 [rows, K].  Refuses K > 32 or E > 1024. */
void qw_op_moe_route(qw_cmd c, qw_ref idx, qw_ref w, qw_ref logits,
                     int32_t rows, int32_t E, int32_t K, bool norm);
/* y[p] = bank[idx[p]] . x[x_by_pair ? p : p / K] for `pairs` pairs. */
void qw_op_qmv_q4_bank(qw_cmd c, qw_ref y, qw_ref x, qw_ref idx,
                       qw_ref w, qw_ref scales, qw_ref biases,
                       int32_t k, int32_t n, int32_t pairs, int32_t K, bool x_by_pair,
                       int32_t group);
/* Two banks of one shape against x (p / K), y [2, pairs, n].  False, nothing
 * encoded, for k < 2048, as in the reference. */
bool qw_op_qmv_q4_bank2(qw_cmd c, qw_ref y, qw_ref x, qw_ref idx,
                        qw_ref w, qw_ref scales, qw_ref biases,
                        qw_ref w2, qw_ref scales2, qw_ref biases2,
                        int32_t k, int32_t n, int32_t pairs, int32_t K, int32_t group);
/* y[p] = W . (silu(gate[p]) * up[p]), rows p at p * stride; W is expert
 * idx[p] of a bank, or the one matrix when idx.buf is NULL. */
void qw_op_qmv_q4_swiglu(qw_cmd c, qw_ref y, qw_ref gate, qw_ref up, int32_t stride, qw_ref idx,
                         qw_ref w, qw_ref scales, qw_ref biases,
                         int32_t k, int32_t n, int32_t rows, int32_t group);
/* Prefill's grouped experts.  qw_op_moe_group sorts the pairs by expert --
 * stably: ascending pair index within an expert, so perm is deterministic --
 * into tiles [1 + 3 * qw_moe_max_tiles] = (count, (expert, start, len)...);
 * qw_op_qmm_q4_gather runs one tiled product per tile.  cursor [E] is
 * accepted for the reference's signature and not used. */
int32_t qw_moe_max_tiles(int32_t pairs, int32_t E);
void qw_op_moe_group(qw_cmd c, qw_ref perm, qw_ref tiles, qw_ref cursor, qw_ref idx,
                     int32_t pairs, int32_t E);
void qw_op_qmm_q4_gather(qw_cmd c, qw_ref y, qw_ref x, qw_ref perm, qw_ref tiles,
                         qw_ref w, qw_ref scales, qw_ref biases,
                         int32_t k, int32_t n, int32_t pairs, int32_t E, int32_t K,
                         bool x_by_pair, int32_t group);
/* act[p, i] = silu(gu[p, i]) * gu[p, I+i]. */
void qw_op_swiglu_split(qw_cmd c, qw_ref act, qw_ref gu, int32_t pairs, int32_t I);
/* out[r] = sum_k w[r, k] * y[r*K + k]. */
void qw_op_moe_combine(qw_cmd c, qw_ref out, qw_ref y, qw_ref w, int32_t rows, int32_t K, int32_t H);
/* y[r, :] *= sigmoid(g[r]). */
void qw_op_scale_rows_sigmoid(qw_cmd c, qw_ref y, qw_ref g, int32_t rows, int32_t dim);

/* ---- additions without a reference counterpart ------------------------------ */

/* The residual step between the layers of a MoE stack:
 * h BF16 [rows, dim] <- bf16(h + y) (h kept when y is a null ref), then
 * x F32 [rows, dim] = rms_norm(h), unit weight -- the reference's
 * qw_op_add_inplace and qw_op_rms_norm with the bf16 carry between them,
 * in one pass. */
void qw_op_residual_rms_norm_bf16(qw_cmd c, qw_ref h, qw_ref x, qw_ref y,
                                  int32_t dim, int32_t rows, float eps);

/* Seeded synthetic data written on the device, for benchmarks and tests:
 * n elements of `kind` from the counter-based SplitMix64 stream `key`.
 *   0  u32 words (4-bit nibbles: the high 32 bits of each output)
 *   1  bf16 uniform in [a, b)
 *   2  bf16 of -8 * (kind 1's value for the same key, a, b): MLX biases
 *   3  bf16 N(0, a) by Box-Muller
 *   4  kind 3's value stored as fp32 */
void qw_op_synth(qw_cmd c, qw_ref dst, int32_t kind, int64_t n, uint64_t key, float a, float b);

/* The tile height the grouping and the grouped product agree on for a
 * given (pairs, E): 16, 32 or 64 rows. */
int32_t qw_moe_tile_rows(int32_t pairs, int32_t E);

/* One quantised matrix or bank. */
typedef struct { qw_ref w, scales, biases; int32_t group; } qw_q4_ref;

/* The MoE block's tensors, as the reference's qw_moe (qwasar_model.h:137-153). */
typedef struct {
    int32_t H, E, K, I, SI;
    bool norm;                   /* norm_topk_prob */
    bool split;                  /* gate/up banks [E, I, H]; else gate_up [E, 2I, H] */
    qw_ref router;               /* BF16 [E, H] */
    qw_q4_ref gate_up, gate, up; /* banks */
    qw_q4_ref down;              /* bank [E, H, I] */
    qw_q4_ref sh_gate, sh_up;    /* [SI, H] */
    qw_q4_ref sh_down;           /* [H, SI] */
    qw_ref sh_gate_w;            /* BF16 [1, H] */
} qw_moe_layer;

/* The whole MoE block -- router, routing, routed experts, gated shared
 * expert, combine -- for `rows` tokens, in the fewest launches this backend
 * has: out F32 [rows, H]; idx I32 [rows, K] and w F32 [rows, K] receive the
 * routing.  Decode (rows <= 8) is a fused path over only the selected
 * experts; prefill is the grouped path.  Scratch is owned by the backend.
 * False, nothing encoded, for shapes outside what the kernels take. */
bool qw_op_moe_layer(qw_cmd c, qw_ref out, qw_ref idx, qw_ref w, qw_ref x,
                     const qw_moe_layer *M, int32_t rows);

/* One layer of a stack whose layers are joined by the residual bf16 RMS norm
 * (qw_op_residual_rms_norm_bf16), with that step folded in:
 * h_out = bf16(h + y_prev) (h when y_prev is a null ref), x_out =
 * rms_norm(h_out) (unit weight), then out = MoE(x_out) as qw_op_moe_layer.  At decode sizes
 * the step runs inside the layer's one launch.  h_out must be a buffer other
 * than h and y_prev.  False (nothing encoded) where qw_op_moe_layer refuses. */
bool qw_op_moe_layer_residual(qw_cmd c, qw_ref out, qw_ref idx, qw_ref w, qw_ref h, qw_ref y_prev,
                              qw_ref h_out, qw_ref x_out, const qw_moe_layer *M, int32_t rows, float eps);

/* qw_op_moe_layer's decode path (rows <= 8) with no allocation.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The launch's staging and hand-off state live in a
 * static device array of 2 MiB per GPU (held until the process ends), whose
 * address the library resolves at qw_gpu_init; this call makes no
 * allocation of any kind and gives qw_op_moe_layer's bits (the one-launch
 * path for one token, the batch path for 2..8).  False, nothing encoded,
 * where qw_op_moe_layer would not take a decode path (past 8 rows, or shapes
 * the decode kernels do not take), or where the layer's staging at `rows`
 * exceeds what the array holds past its 317 KiB hand-off state (1,772,800
 * bytes: config 1's shape at 8 rows stages 1,466,624; H 3072 with K 15 at 8
 * rows, 2,101,504, is refused, at 6 rows, 1,577,216, taken).
 * Every call on one GPU shares the array and finds it as the last call
 * left it (the hand-off state stays valid between calls, and qw_gpu_init
 * zeroes it; the staging needs no clearing).  The outputs go on the
 * command's written list like any op's (qw_cmd_begin leaves room for 16
 * buffers; a command already holding 16 others is refused, nothing
 * encoded).  Calls whose launches overlap on one GPU -- the library's
 * single stream serialises its own -- would race on it.  Hand-off failures are reported as qw_op_moe_layer's
 * are, by qw_cmd_error after qw_cmd_wait. */
bool qw_op_moe_layer_noalloc(qw_cmd c, qw_ref out, qw_ref idx, qw_ref w, qw_ref x,
                             const qw_moe_layer *M, int32_t rows);

/* ---- checkpoint loading (reference qwasar.c:700-775 config, :1426-1461
 * qw_bind_small, :1469-1495 qw_bind_qbank, :1532-1563 qw_bind_moe) ---------
 *
 * A checkpoint directory: config.json (text fields under text_config, or at
 * the root of a qwen4_exp_text export) and every *.safetensors file in it,
 * mapped read-only.  NULL / false with a message in err on failure. */
typedef struct qw_checkpoint_s *qw_checkpoint;
qw_checkpoint qw_checkpoint_open(const char *dir, char *err, size_t errcap);
void qw_checkpoint_close(qw_checkpoint ck);
/* num_hidden_layers */
int32_t qw_checkpoint_layers(qw_checkpoint ck);
/* One tensor of the table, by name: its bytes in the mapping (valid until
 * close), shape and safetensors dtype name.  False if absent. */
bool qw_checkpoint_tensor(qw_checkpoint ck, const char *name, const void **data, size_t *nbytes,
                          int32_t *ndim, int64_t shape[8], char dtype[16]);
/* Layer `layer`'s MoE block (language_model.model.layers.<layer>.mlp) in new
 * device buffers: the fused `experts.gate_up_proj` bank or the MLX split
 * `switch_mlp.*` banks (whichever the checkpoint holds), the shared expert,
 * and the router and shared-expert gate as bf16 -- dequantised from 4 or 8
 * bits when stored quantised.  Group 32 or 64, read from the scale shapes.
 * The checkpoint may be closed afterwards. */
bool qw_moe_layer_load(qw_checkpoint ck, int32_t layer, qw_moe_layer *m, char *err, size_t errcap);
/* Frees the buffers qw_moe_layer_load made and clears their refs. */
void qw_moe_layer_free(qw_moe_layer *m);

/* Profiling for harnesses: force profiling on or off (overrides
 * QWASAR_PROFILE), and read one label's accumulated device milliseconds and
 * mark count. */
void   qw_prof_set_enabled(bool on);
double qw_prof_ms(const char *label, int64_t *count);

/* For tests of the decode path's failure handling; no reference counterpart
 * (the Metal backend has no cross-workgroup waits).  Sets the hand-off error
 * word as if the next decode launch's first bounded wait had given up: every
 * wait of that launch and of later ones gives up at once (each kernel still
 * runs to its end), qw_cmd_error of every command that launched one of them
 * reports it after qw_cmd_wait, and the state is then zeroed so that the
 * next launch runs normally. */
bool qw_debug_decode_handoff_fail(void);

#ifdef __cplusplus
}
#endif

#endif /* QWASAR_GPU_H */
