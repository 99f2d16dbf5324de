/* moe_ref.h -- CPU oracle for the Flash-Next MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (qwasar_amd/, include/)
 * links, loads or calls this code; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg do, and only as the checker or the timed CPU
 * baseline.
 *
 * It restates the reference's scalar MoE step, `moe_step` in
 * qwasar_flash_cpu.c:490-555, and its helpers in qwasar_cpu.c:15-63,98-110,
 * with two deliberate, documented refinements so that routing can be held
 * bit-exact against the GPU:
 *
 *   1. Router logits use a specified summation order ("order R", below)
 *      instead of the reference's serial sum, whose order under -ffast-math
 *      is up to the compiler (reference Makefile:14).
 *   2. The softmax uses qr_exp, a self-written exponential (Cody-Waite range
 *      reduction plus a degree-7 Taylor polynomial in Horner form) instead of
 *      libm expf, and sums the exponentials in a specified tree order.
 *
 * Everything else -- dequantisation, the expert matvecs, SwiGLU, the shared
 * expert and its sigmoid gate, the combine -- follows the reference's scalar
 * arithmetic literally (serial fp32 sums, no contraction: build with
 * -ffp-contract=off).
 *
 * Parity pins (each tested in tests/test_oracle.py):
 *   qr_bf16_to_f32, qr_qmv_q4, qr_dequant_row  bit-exact against the
 *       reference's own qw_cpu_* compiled from /root/reference (oracle/_ref)
 *       and against hand vectors and the tiny-q4 fixture banks.
 *   qr_dot_bf16 (order R)  within fp32 error of qw_cpu_dmv_bf16 and of an
 *       fp64 brute force; its order by a hand-built cancellation vector.
 *   qr_exp  within 2 ulp of libm expf over a dense sweep; exact at 0.
 *   qr_route  against a full sort by (-p, e), against the reference's literal
 *       serial route on decisive inputs, and on constructed ties.
 *   qr_moe_group  permutation/stability/tile invariants and a brute force.
 *   qr_moe_forward  against an fp64 numpy restatement on config 0.
 */
#ifndef QW_MOE_REF_H
#define QW_MOE_REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Chunk length of order R: a dot product is the left-to-right sum of the
 * fmaf-chain partials of consecutive 64-element chunks. */
#define QR_ROUTER_CHUNK 64
/* Lanes of the softmax sum's tree: lane l sums e = l, l+64, ... serially,
 * then the 64 lane sums meet in an xor butterfly with ascending offsets
 * 1, 2, 4, 8, 16, 32. */
#define QR_SUM_LANES 64

float qr_bf16_to_f32(uint16_t v);
uint16_t qr_f32_to_bf16(float f);
float qr_exp(float x);
void qr_exp_vec(float *out, const float *in, int64_t n);

/* Dequantised row `row` of an MLX affine 4-bit matrix (qwasar_cpu.c:21-38). */
void qr_dequant_row(float *out, const uint32_t *w, const uint16_t *scales,
                    const uint16_t *biases, int32_t k, int32_t row, int32_t group);
/* y[r][o] = sum_i dequant(w)[o][i] * x[r][i], serial (qwasar_cpu.c:40-63). */
void qr_qmv_q4(float *y, const float *x, const uint32_t *w, const uint16_t *scales,
               const uint16_t *biases, int32_t k, int32_t n, int32_t rows, int32_t group);

/* Order-R dot of a bf16 row with an fp32 vector. */
float qr_dot_bf16(const uint16_t *w, const float *x, int32_t k);
/* y[r][o] = qr_dot_bf16(w[o], x[r]) -- the router's logits and the shared
 * expert's gate logit (reference qw_cpu_dmv_bf16, qwasar_cpu.c:98-110). */
void qr_dmat_bf16(float *y, const float *x, const uint16_t *w, int32_t k, int32_t n, int32_t rows);

/* Softmax over E in fp32 (qr_exp, tree sum), K picks by strict '>' from
 * e = 0 (ties to the lower index), renormalised when `norm`
 * (qwasar_flash_cpu.c:499-521).  idx, w are [rows, K]. */
void qr_route(int32_t *idx, float *w, const float *logits, int32_t rows, int32_t E,
              int32_t K, int32_t norm);
/* The reference's literal route: libm expf, serial sum (qwasar_flash_cpu.c:499-521).
 * For cross-checking qr_route on inputs with decisive cuts. */
void qr_route_literal(int32_t *idx, float *w, const float *logits, int32_t rows, int32_t E,
                      int32_t K, int32_t norm);

/* The stable dispatch permutation: pairs sorted by expert, ascending pair
 * index within an expert; tiles = [count, (expert, start, len) ...] with
 * len <= bm.  Returns the tile count. */
int32_t qr_max_tiles(int32_t pairs, int32_t E, int32_t bm);
int32_t qr_moe_group(int32_t *perm, int32_t *tiles, const int32_t *idx, int32_t pairs,
                     int32_t E, int32_t bm, int32_t max_tiles);

/* silu(x) = x * sigmoid(x), sigmoid = 1 / (1 + expf(-x)) (qwasar_flash_cpu.c:28-29). */
float qr_silu(float x);
float qr_sigmoid(float x);

/* One quantised matrix: a bank of `banks` experts of [out, in] each, or a
 * single matrix (banks = 1). */
typedef struct {
    const uint32_t *w;
    const uint16_t *s;
    const uint16_t *b;
    int32_t group;
} qr_q4;

/* The MoE block's tensors (reference qw_moe, qwasar_model.h:137-153). */
typedef struct {
    int32_t H, E, K, I, SI;
    int32_t norm;        /* norm_topk_prob */
    int32_t split;       /* 1: gate and up banks [E, I, H]; 0: gate_up [E, 2I, H], gate rows first */
    const uint16_t *router;      /* bf16 [E, H] */
    qr_q4 gate_up, gate, up;     /* banks */
    qr_q4 down;                  /* bank [E, H, I] */
    qr_q4 sh_gate, sh_up;        /* [SI, H] */
    qr_q4 sh_down;               /* [H, SI] */
    const uint16_t *sh_gate_w;   /* bf16 [H] */
} qr_moe;

/* The whole block for `rows` tokens, each independently
 * (qwasar_flash_cpu.c:490-555): out [rows, H]; idx, w [rows, K]. */
void qr_moe_forward(float *out, int32_t *idx, float *w, const float *x, int32_t rows,
                    const qr_moe *M);

/* One RMS norm with unit weight, eps (qwasar_cpu.c:68-82). */
void qr_rms_norm(float *y, const float *x, int32_t dim, int32_t rows, float eps);

/* ---- the hyper-connection mixer around a block (qwasar_flash_cpu.c:57-70,
 * 263-293; the GPU ops' semantics, metal/sparse.metal:14-189) ---------------- */

/* y[r, g*dim + i] = x * inv_g * w[g*dim + i], inv_g over group g of row r,
 * each group in the form of qwasar_cpu.c:68-82. */
void qr_rms_norm_grouped(float *y, const float *x, const uint16_t *w, int32_t dim, int32_t groups,
                         int32_t rows, float eps);
/* y = silu(y * scale), n elements. */
void qr_silu_scale(float *y, int64_t n, float scale);
/* x[r, i] = (sum over s, in order, of sigmoid(m[r, s*H+i]) * n[r, s*H+i]) / S. */
void qr_hc_mix(float *x, const float *n, const float *m, int32_t rows, int32_t H, int32_t S);
/* h4[r, s*H+i] += out[r, i] * (2 * sigmoid(inj[r, s] / S)). */
void qr_hc_inject(float *h4, const float *out, const float *inj, int32_t rows, int32_t H, int32_t S);
/* h4[r, s*H+i] = x[r, i]. */
void qr_repeat_cols(float *h4, const float *x, int32_t rows, int32_t H, int32_t S);

#ifdef __cplusplus
}
#endif
#endif
