/* qw_kernels.h -- the thin C ABI between the C backend (qwasar_hip.c) and the
 * gfx950 kernels.  Plain device pointers, sizes and a HIP stream; every
 * function launches asynchronously on `s` and returns a hipError_t as int
 * (0 = launched).  Shapes are validated here, before any launch, so a shape
 * a kernel does not support is refused rather than run. */
#ifndef QW_KERNELS_H
#define QW_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWK_DMAT_MAX_K   16384
#define QWK_ROUTE_MAX_E  1024
#define QWK_ROUTE_MAX_K  32
#define QWK_GROUP_MAX_E  1024

/* One MLX affine 4-bit matrix, or the base of a bank of them. */
typedef struct { const uint32_t *w; const uint16_t *s; const uint16_t *b; } qwk_q4;

/* Router logits / dense bf16 matvec in order R: y[rows, n] = x[rows, k] . w[n, k]^T. */
int qwk_dmat_bf16(hipStream_t s, float *y, const float *x, const uint16_t *w,
                  int k, int n, int rows);

/* The same for up to 8 token rows (k % 64 == 0, k <= 4096, 16-byte aligned),
 * with, when w2 is given, one more output: g[r] = order-R dot of w2 [k] with
 * x row r, in the same launch; when qx is given, x staged there as q16
 * units ([rows][k / 16][3] uint4, 16-byte aligned); when hx is given, x
 * staged there as qwk_stage16 stages it (hx [rows, k] f16, 16-byte aligned,
 * hF [rows]). */
/* y[rows, n] as qwk_dmat_bf16 (order R, n <= 8, k % 64 == 0, k <= 4096,
 * 16-byte aligned) and, in the same launch, x staged into hx / hF exactly as
 * qwk_stage16 stages it. */
int qwk_dmat_rows_stage16(hipStream_t s, float *y, uint16_t *hx, float *hF, const float *x,
                          const uint16_t *w, int k, int n, int rows);
int qwk_dmat_bf16_gate(hipStream_t s, float *y, float *g, const float *x, const uint16_t *w,
                       const uint16_t *w2, int k, int n, int rows, void *qx, uint16_t *hx, float *hF);

/* Softmax, top-K, renormalise: idx/w [rows, K]. */
int qwk_route(hipStream_t s, int32_t *idx, float *w, const float *logits,
              int rows, int E, int K, int norm);

/* Stable sort of pairs by expert; tiles = [count, (expert, start, len)...]. */
int qwk_moe_group(hipStream_t s, int32_t *perm, int32_t *tiles, const int32_t *idx,
                  int pairs, int E, int bm, int max_tiles, void *work, size_t work_bytes, int extra);
/* Bytes of the work buffer qwk_moe_group needs for `pairs` pairs of E experts. */
size_t qwk_moe_group_work_bytes(int pairs, int E);

/* Quantised matvec over (token, slot) pairs.
 *   y[z][p, 0:n] = W_z(e_p) . in(p)
 * with e_p = idx[p] (idx NULL: the single matrix), W_z the z-th of `nmat`
 * matrices (bank2: gate and up), and in(p) either x row (x_by_pair ? p : p/K)
 * at stride `xstride`, or, with `up` non-NULL, silu(x[p*xstride + i]) *
 * up[p*xstride + i].  y[z] = y + z * pairs * n. */
int qwk_q4mv(hipStream_t s, float *y, const float *x, const float *up, int xstride,
             const int32_t *idx, const qwk_q4 *mats, int nmat,
             int k, int n, int pairs, int K, int x_by_pair, int group);

/* Up to 4 one-token matvecs sharing x [1, k]: y_i = W_i . x. */
int qwk_q4mv_multi(hipStream_t s, const float *x, int k, int group, int count,
                   const qwk_q4 *mats, float *const *ys, const int *ns);

/* The grouped (prefill) product: per tile of pairs routed to one expert,
 * y[perm[j], :] = W_e . in(perm[j]), in(p) = x row (x_by_pair ? p : p/K).
 * Tiles were cut at `bm` rows by qwk_moe_group; `max_tiles` bounds the grid. */
int qwk_gather_gemm(hipStream_t s, float *y, const float *x, const int32_t *perm,
                    const int32_t *tiles, qwk_q4 m, int k, int n, int K, int x_by_pair,
                    int group, int bm, int max_tiles);

/* Dense prefill product y[rows, n] = x[rows, k] . W^T (the shared expert). */
/* work: qwk_qmm_work_bytes(k, n, rows) bytes for the split-K partials (none
 * needed when it returns 0; with less, the product runs unsplit). */
int qwk_qmm(hipStream_t s, float *y, const float *x, qwk_q4 m, int k, int n, int rows, int group,
            void *work, size_t work_bytes);
size_t qwk_qmm_work_bytes(int k, int n, int rows);

/* A second weight bank for grouped tiles of expert `expert` (qwk_moe_group's
 * extra rows): its pairs p >= `pairs` read A row p - pairs when not
 * x_by_pair. */
typedef struct { qwk_q4 m0, m1; int expert, pairs; } qwk_gmm_extra;

/* Prefill products on MFMA over f16-staged activations (qw_gmm16.hip).
 * Staging: per row, h = f16(x 2^sh) with the row's largest magnitude in
 * [2^14, 2^15) and F = 2^-sh; h in 8-blocks ordered 0,4,1,5,2,6,3,7.
 * h [rows, k] f16 (bits), F [rows].  k % 8 == 0. */
int qwk_stage16(hipStream_t s, uint16_t *h, float *F, const float *x, int rows, int k);
/* y[row, :] = W_e . A(row) in fp32, weights dequantised to f16 (one rounding).
 * Grouped (dense_rows == 0): tiles from qwk_moe_group cut at 64 rows; tile
 * row j is pair p = perm[start + j], its A row is (x_by_pair ? p : p / K),
 * its output row p.  Dense (dense_rows > 0): rows 0..dense_rows-1, expert 0.
 * m0 (and with swiglu m1, the up rows) point at expert 0 of the bank; ew/eg
 * are the per-expert strides in words / groups.  With swiglu, n = features
 * and y = silu(W0 A) * (W1 A).  k % 64 == 0 and k % group == 0. */
/* With swiglu (grouped): the activations leave as q16 units (the decode
 * staging format, [vectors][n / 16][48 bytes]) in place of fp32 y: pair
 * p < npk into qa's vector p, pair npk + r into qs's vector r. */
typedef struct {
    void *qa, *qs;
    int npk;
} qwk_gmm_q16out;
int qwk_gmm16_q16_supported(int k, int group, int tile_rows);
/* The decode batch's grouped products (tiles of at most 16 rows, each tile
 * one expert's pairs, the extra bank's tile the shared expert's rows), one
 * weight stream a wave.  swiglu: the staged f16 rows ah / aF against gate
 * (m0) and up (m1), out as q16 units (q16, by pair) or fp32 rows in slot
 * order (y row s: the pair at perm[s]); else the down: the fp32 rows ax in
 * that slot order against m0, out fp32 by pair, y[p][n].  Needs
 * k % 256 == 0 (k <= 3072 and k / group <= 48 with swiglu, else k <= 1024
 * and k / group <= 16), n % 16 == 0 and 16-byte aligned banks. */
int qwk_gmm16_stream_supported(int k, int n, int group, int swiglu, qwk_q4 m0, qwk_q4 m1,
                               const qwk_gmm_extra *xb, long eg);
int qwk_gmm16_stream(hipStream_t s, float *y, long ldy, const uint16_t *ah, const float *aF,
                     const float *ax, const int32_t *perm, const int32_t *tiles, int max_tiles,
                     qwk_q4 m0, qwk_q4 m1, long ew, long eg, int k, int n, int K, int x_by_pair,
                     int group, int swiglu, const qwk_gmm_extra *xb, const qwk_gmm_q16out *q16);
int qwk_gmm16_supported(int k, int group, const void *w0, const void *w1);
int qwk_gmm16(hipStream_t s, float *y, long ldy, const uint16_t *ah, const float *aF,
              const int32_t *perm, const int32_t *tiles, int max_tiles, qwk_q4 m0, qwk_q4 m1, long ew,
              long eg, int k, int n, int K, int x_by_pair, int group, int swiglu, int dense_rows,
              const qwk_gmm_extra *xb, int tile_rows, const qwk_gmm_q16out *q16);

/* Elementwise. */
int qwk_swiglu(hipStream_t s, float *y, const float *gate, const float *up, int64_t n);
int qwk_swiglu_split(hipStream_t s, float *act, const float *gu, int pairs, int I);
int qwk_moe_combine(hipStream_t s, float *out, const float *y, const float *w,
                    const float *sh, const float *g, int rows, int K, int H);
int qwk_scale_rows_sigmoid(hipStream_t s, float *y, const float *g, int rows, int dim);
int qwk_add_inplace(hipStream_t s, float *y, const float *x, int64_t n);

/* ---- the fused MoE layer -------------------------------------------------- */

typedef struct {
    int H, E, K, I, SI, group, norm, split;
    const uint16_t *router;          /* bf16 [E, H] */
    qwk_q4 gate, up;                 /* banks [E, I, H] (split) */
    qwk_q4 gate_up;                  /* bank [E, 2I, H] (fused: gate rows first) */
    qwk_q4 down;                     /* bank [E, H, I] */
    qwk_q4 sh_gate, sh_up, sh_down;  /* [SI, H], [SI, H], [H, SI] */
    const uint16_t *sh_gate_w;       /* bf16 [H] */
} qwk_moe;

/* Bytes of the decode path's hand-off state.  It must be zeroed once before
 * first use (and again after an error); each launch then needs an epoch one
 * greater than the last (never 0; zero the state again before an epoch
 * repeats), and launches on one state run in order. */
size_t qwk_moe_decode_sync_bytes(void);
/* Reads the state's error word.  Non-zero: the epoch of the first launch
 * whose bounded wait gave up; that launch's outputs and those of every later
 * launch on the state are garbage, and the state must be zeroed.
 * Synchronous. */
int qwk_moe_decode_sync_error(const void *sync, uint32_t *err);
/* Sets the error word as a failed wait of launch `epoch` would (synchronous);
 * every wait of a later launch then gives up at once. */
int qwk_moe_decode_sync_raise(void *sync, uint32_t epoch);
/* Another one-launch decode kernel (qwk_hc_decode) may share a hand-off
 * state and its epochs: its error word and the 64-bit tagged words it may
 * use (the two kernels run in stream order, so each finds only past epochs). */
int qwk_decode_sync_words(void *sync, uint32_t **err, void **words, size_t *nwords);
/* The allocation-free decode entry's device scratch (qw_static.hip): a
 * file-scope device array of this many bytes per GPU, holding the hand-off
 * state and then the staging area. */
#define QWK_STATIC_SCRATCH_BYTES (2048u * 1024u)
/* Resolves the array's address on the current device (hipGetSymbolAddress)
 * and zeroes it; once per device, at init.  Synchronous. */
int qwk_static_init(hipStream_t s);
/* The array's address on the current device (NULL before qwk_static_init),
 * and its size in *bytes. */
void *qwk_static_scratch(size_t *bytes);
/* Zeroes `bytes` (a multiple of 16, 16-byte aligned) at p with a fill kernel
 * on s (no memset node, so it may sit in a captured graph). */
int qwk_zero_fill(hipStream_t s, void *p, size_t bytes);
/* Non-zero when the decode path takes this layer shape and token count: the
 * one-token launch (qwk_decode1_supported) or the batch path
 * (qwk_moe_decode_batch_supported, 1..QWK_DECODE_MAX_ROWS tokens). */
int qwk_moe_decode_supported(const qwk_moe *M, int rows);
int qwk_decode1_supported(const qwk_moe *M);
int qwk_moe_decode_batch_supported(const qwk_moe *M, int rows);
/* The residual step before a layer of a stack: the layer's input is
 * x = rms_norm(bf16(h + y)) (rms_norm(h) when y is NULL), unit weight;
 * h_out receives bf16(h + y) (or h), x_out that x.  h_out must not alias h
 * or y on the decode path, whose workgroups read h while one writes h_out. */
typedef struct {
    const uint16_t *h;
    const float *y;
    uint16_t *h_out;
    float *x_out;
    float eps;
} qwk_resid;

/* Decode of one token in one launch (qwk_decode1_supported layers), K <=
 * QWK_DECODE_MAX_K: out [H], idx/w [K]; the input is x, or, when `res` is
 * not NULL, the residual step's x computed inside the launch.  It needs no
 * scratch beyond the hand-off state `sync` (qwk_moe_decode_sync_bytes) and
 * LDS.  `ev`, when not NULL, holds 2 events, the launch's start and end,
 * stamped by the dispatch itself. */
#define QWK_DECODE_MAX_ROWS 8
#define QWK_DECODE_MAX_K 15
int qwk_moe_decode(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                   const qwk_resid *res, const qwk_moe *M, void *sync, uint32_t epoch, hipEvent_t *ev);
/* Decode of 1..QWK_DECODE_MAX_ROWS tokens over the batch's unique experts:
 * router logits, routing and the unique-expert table, gate/up per unique
 * expert, down and combine per token.  With the decode hand-off words (tags,
 * tag_words of them, the error word and a fresh epoch: from
 * qwk_decode_sync_words) and the matrix-core gate/up, the logits and the
 * routing share one launch (its routing workgroup waits for the logits'
 * tagged words; *handoff = 1); else they are launches of their own
 * (*handoff = 0).  Same shapes as
 * qwk_moe_decode; scratch of qwk_moe_decode_batch_scratch bytes, nothing in it
 * initialised. */
size_t qwk_moe_decode_batch_scratch(const qwk_moe *M, int rows);
int qwk_moe_decode_batch(hipStream_t s, float *out, int32_t *idx, float *w, const float *x,
                         const qwk_moe *M, int rows, void *scratch, size_t scratch_bytes, void *tags,
                         size_t tag_words, uint32_t *err, uint32_t epoch, int *handoff);

/* RMS norm of [rows, dim] fp32 rows (dim % 4 == 0), optional bf16 weight:
 * y = x / sqrt(mean(x^2) + eps) * out_scale (* w). */
int qwk_rms_norm(hipStream_t s, float *y, const float *x, const uint16_t *w, int dim, int rows,
                 float eps, float out_scale);
/* The residual step between stacked layers: h_out bf16 [rows, dim] =
 * bf16(h + y) (h when y is NULL; h_out may be h), then x = rms_norm(h_out)
 * in fp32, unit weight. */
int qwk_resid_rms_bf16(hipStream_t s, const uint16_t *h, uint16_t *h_out, float *x, const float *y, int dim,
                       int rows, float eps);

/* Seeded synthetic tensors (counter-based SplitMix64; value i of key k is
 * the i-th output of SplitMix64 seeded with k). */
#define QWK_SYNTH_U32 0             /* u32 words: the high half of each output */
#define QWK_SYNTH_BF16_UNIFORM 1    /* bf16 of a + (b - a) u, u a 53-bit uniform */
#define QWK_SYNTH_BF16_NEG8 2       /* bf16 of -8 times kind 1's value for the same key */
#define QWK_SYNTH_BF16_NORMAL 3     /* bf16 of N(0, a), Box-Muller on outputs 2i, 2i+1 */
#define QWK_SYNTH_F32_BF16_NORMAL 4 /* kind 3's value, stored as fp32 */
int qwk_synth(hipStream_t s, void *dst, int kind, int64_t n, uint64_t key, float a, float b);

/* The hyper-connection mixer around a block (qw_hc.hip); H % 4 == 0. */
int qwk_repeat_cols(hipStream_t s, float *h4, const float *x, int rows, int H, int S);
int qwk_rms_norm_grouped(hipStream_t s, float *y, const float *x, const uint16_t *w, int dim, int groups,
                         int rows, float eps);
int qwk_hc_inject_norm(hipStream_t s, float *h4, const float *out, const float *inj, const uint16_t *w,
                       float *n4, int rows, int H, int S, float eps);
int qwk_silu_scale(hipStream_t s, float *y, int64_t n, float scale);
int qwk_hc_pre_decode(hipStream_t s, float *h4_out, float *n4, float *d, float *inj_out, const float *h4,
                      const float *out, const float *inj, const uint16_t *wn, qwk_q4 dn, const uint16_t *bj,
                      int H, int S, int lowrank, int group, float eps);
int qwk_hc_mix(hipStream_t s, float *x, const float *n, const float *m, int rows, int H, int S);
int qwk_hc_inject(hipStream_t s, float *h4, const float *out, const float *inj, int rows, int H, int S);
/* A mixer decode step (one row) in one launch: qwk_hc_pre_decode and
 * qwk_hc_mix_up(rows 1) fused, handing d over by tagged words in `tags`
 * (qwk_hc_decode_tag_words() of them) under `epoch`; a wait that gives up
 * raises *err.  lowrank <= 512, a multiple of 8 and of group. */
size_t qwk_hc_decode_tag_words(void);
int qwk_hc_decode(hipStream_t s, float *x, float *h4_out, float *n4, float *d, float *inj_out, const float *h4,
                  const float *out, const float *inj, const uint16_t *wn, qwk_q4 dn, const uint16_t *bj, qwk_q4 up,
                  int H, int S, int lowrank, int group, float eps, float scale, uint32_t *err, void *tags,
                  uint32_t epoch);
int qwk_hc_mix_up(hipStream_t s, float *x, const float *d, const float *n4, const uint32_t *w,
                  const uint16_t *sc, const uint16_t *bi, int k, int H, int S, int rows, float scale, int group);

/* The gated DeltaNet (qw_gdn.hip).  dk = dv = 128; ksize 4. */
typedef struct {
    const float *a, *b;
    const uint16_t *A_log, *dt_bias;
    float l2eps, q_scale, k_scale;
} qwk_gdn_prep;
int qwk_conv1d_causal_silu(hipStream_t s, float *y, const float *x, float *state, const uint16_t *w,
                           int channels, int rows, int ksize, float *snap, int n_snap, int snap_stride);
int qwk_gdn_gates(hipStream_t s, float *g, float *beta, const float *a, const float *b,
                  const uint16_t *A_log, const uint16_t *dt_bias, int hv, int rows);
/* prep NULL: q, k normed and g, beta given; else g and beta are unused.
 * work: qwk_gated_delta_work() bytes of device memory (NULL when that is 0):
 * a long prepared call computes its norms and gates there first, in
 * parallel, instead of a chunk at a time inside the recurrence. */
size_t qwk_gated_delta_work(int hk, int hv, int rows, int prep);
int qwk_gated_delta(hipStream_t s, float *y, const float *q, const float *k, const float *v,
                    const float *g, const float *beta, float *state, int hk, int hv, int dk, int dv,
                    int rows, float *snap, int n_snap, int snap_stride, const qwk_gdn_prep *prep, void *work);
/* One decode step: the conv over x [2 hk dk + hv dv] (window win in, wout
 * out: distinct buffers, [3, channels] oldest first), then the prepared delta
 * rule on its q, k and v channels; the bits of qwk_conv1d_causal_silu then
 * qwk_gated_delta with prep. */
int qwk_gdn_decode(hipStream_t s, float *y, const float *x, const float *win, float *wout, const uint16_t *w,
                   const qwk_gdn_prep *prep, float *state, int hk, int hv, int dk, int dv);
/* rms_norm(x) (* w) * sigmoid(gate) per row (qw_norm.hip); dim % 4 == 0. */
int qwk_rms_norm_gated_sigmoid(hipStream_t s, float *y, const float *x, const uint16_t *w, const float *gate,
                               int dim, int rows, float eps, float out_scale);

/* QSA (qw_qsa.hip): rotary_dim 64, d % 32 == 0, 64 <= d <= 256. */
int qwk_qsa_scores(hipStream_t s, float *scores, const float *qn, const float *ikeys, const uint16_t *kw,
                   const float *inv_freq, int rows, int nq, int d, int ratio, int base_pos,
                   int rotary_dim, int max_blocks, float eps);
int qwk_qsa_pool(hipStream_t s, float *pool, const float *ikeys, const uint16_t *kw, const float *inv_freq,
                 int d, int ratio, int b0, int b1, int rotary_dim, float eps);
int qwk_qsa_scores_pooled(hipStream_t s, float *scores, const float *qn, const float *pool, int rows,
                          int nq, int d, int ratio, int base_pos, int max_blocks);
int qwk_qsa_select(hipStream_t s, uint8_t *mask, uint32_t *list, const float *scores, int rows, int ratio,
                   int base_pos, int block_topk, int max_ctx, int max_blocks);
/* head_dim 256; q_heads / kv_heads in {1, 2, 4, 8, 12, 16}; gate may be NULL.
 * work: qwk_attn_masked_work_bytes bytes for the split partials (none needed
 * when it returns 0; with less, the list is not split). */
int qwk_attn_masked(hipStream_t s, float *out, const float *gate, const float *q, const uint16_t *kc,
                    const uint16_t *vc, const uint32_t *list, int rows, int q_heads, int kv_heads,
                    int head_dim, int max_ctx, float scale, int cap, void *work, size_t work_bytes);
size_t qwk_attn_masked_work_bytes(int rows, int q_heads, int kv_heads, int cap);

/* Read-bandwidth probe (measurement only): launch r reads set r % nsets of
 * nseg 16-byte-aligned ranges once, one workgroup a piece of at most
 * piece_bytes; ms[r] its event-timed duration. */
int qwk_read_probe(const void *const *ptr, const uint64_t *bytes, int nsets, int nseg, int reps,
                   uint64_t piece_bytes, float *ms);

#ifdef __cplusplus
}
#endif
#endif
