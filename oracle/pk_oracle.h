/* pk_oracle.h — CPU restatement of picchio's quantized-MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * path and the host-CPU baseline timed beside it. Only tests/, the smoke
 * check and bench.py's cpu_baseline leg load it; the product library never
 * links or calls it.
 *
 * Every function follows one reference function, cited file:line into
 * picchio (quant.h, picchio.c, convert.py). Arithmetic order follows the
 * reference as built by its Makefile (gcc -O3 with AVX2/FMA enabled, default
 * -ffp-contract=fast): matmuls keep quant.h's 8-lane accumulators and hsum256
 * tree, and every `a += b * c` the compiler contracts is an explicit fmaf here.
 *
 * Parity status per function (what pins it; all checks in tests/test_oracle.py,
 * golden vectors recorded from picchio's own C build by tests/golden/make_golden.py):
 *   po_quantize_int4_gs    convert.py's algorithm restated in numpy (bit-equal on
 *                          ragged, odd, zero and sub-1e-8 groups) + known answers
 *                          for ties / zero groups; nibble decode exhaustive
 *   po_quantize_int8_rows  convert.py's algorithm restated in numpy + known answers
 *   po_quantize_rows_i4    golden vectors (quant.h) + the self-test KAT
 *   po_matmul_*            golden vectors (quant.h), bit-identical; float64 brute force
 *   po_rmsnorm/po_softmax  golden vectors + the self-test KATs
 *   po_swiglu_clamped      float64 closed form incl. both clamps; inside moe golden
 *   po_moe_forward/po_expert_apply   golden vectors (picchio.c) + float64
 *                          restatement of router, top-k tie rule, softmax, combine
 *   po_gqa_attention/rope/yarn  golden vectors + float64 restatement (window, sinks,
 *                          sink = -inf reducing to plain softmax, YaRN closed form)
 *   po_forward_token/po_prefill_tokens  golden token streams (picchio.c)
 *   po_model_build / po_fill_normal     the synthetic-input generator (not a
 *                          reference function); the GPU generator is checked
 *                          against it bit-for-bit in the GPU tests.
 *   po_act_limbs           (the library's own int8 prefill arithmetic) the
 *                          exponent's frexp definition, limb ranges incl. the
 *                          +-64 boundaries, nearest-grid bound, exactness on
 *                          grid points, ties to even
 *   po_mfma_matvec         float64 brute force with exact int64 group sums,
 *                          inside the fp32 fold's error bound (a planted wrong
 *                          limb weight fails it)
 * Nothing here is "parity unpinned". Transcendentals (expf, cosf, sinf, powf,
 * logf) are glibc's, as in the reference build, so the oracle matches the
 * reference bit-for-bit on this image; the GPU path's own transcendentals are
 * compared within relative L2 1e-4 instead.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stdint.h>
#include "../include/picchio_hip.h"   /* pk_cfg: the shared configuration type */

#ifdef __cplusplus
extern "C" {
#endif

/* ── quantizers ── */
void po_quantize_int4_gs(const float *w, int O, int I, int gs,
                         uint8_t *packed, float *scales);
void po_quantize_int8_rows(const float *w, int O, int I, int8_t *q, float *scales);
void po_quantize_rows_i4(const float *w, int O, int I, uint8_t *q4, float *scales);

/* ── matmuls: y[S,O] = x[S,I] · Wᵀ ── */
void po_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O);
void po_matmul_q8(float *y, const float *x, const int8_t *q, const float *scale,
                  int S, int I, int O);
void po_matmul_i4(float *y, const float *x, const uint8_t *q4, const float *scale,
                  int S, int I, int O);
void po_matmul_i4_gs(float *y, const float *x, const uint8_t *q4, const float *scale,
                     int S, int I, int O, int gs);

/* ── elementwise ── */
void po_rmsnorm(float *out, const float *x, const float *w, int D, float eps);
void po_softmax(float *x, int n);
void po_swiglu_clamped(float *gu, int inter, float limit, float alpha);

/* ── synthetic model (weights drawn with pk_synth.h) ── */
typedef struct po_model po_model;

/* Builds every tensor of `cfg` from `seed`. Experts are drawn fp32 and
 * quantized with po_quantize_int4_gs(group_size); norms are 1.0. */
po_model *po_model_build(const pk_cfg *cfg, uint64_t seed, int n_threads);
void po_model_free(po_model *m);
void po_model_reset_kv(po_model *m);
/* Positions 0..n_pos-1 of layer's K and V caches drawn N(0,1) from the raw
 * stream seeds sk and sv (a synthetic prefilled context; test support). */
void po_model_fill_kv(po_model *m, int layer, int n_pos, uint64_t sk, uint64_t sv);

/* Raw views of one expert (reference layout) for tests. */
int po_model_expert(po_model *m, int layer, int eid,
                    const uint8_t **gu_q4, const float **gu_s,
                    const uint8_t **d_q4, const float **d_s,
                    const float **gu_b, const float **d_b);
const float *po_model_router(po_model *m, int layer, const float **bias);
/* Dense fp32 tensor of the model by pk_synth kind (PK_T_ROUTER.. PK_T_LM_HEAD;
 * kind 0 = final norm, kind -1/-2 = in_ln/post_ln of `layer`); for INT8
 * lm_head, PK_T_LM_HEAD returns the int8 rows and *scales the row scales. */
const void *po_model_tensor(po_model *m, int kind, int layer, const float **scales);
/* Counter-based N(0,1)*std samples of pk_synth.h stream (seed, kind, layer, idx). */
void po_fill_normal(uint64_t seed, int kind, int layer, int idx, int64_t first,
                    int64_t n, float std, float *out);

/* expert_apply (picchio.c:1768-1791): dst += w · expert(x). */
void po_expert_apply(po_model *m, int layer, int eid, const float *x, float *dst, float w);
/* moe_forward (picchio.c:1309-1466): out = Σ_k w_k·expert_k(x). */
void po_moe_forward(po_model *m, int layer, const float *x, float *out,
                    int *sel, float *wsel, float *logits);
/* gqa_attention (picchio.c:504-623): writes K/V at pos, returns out[D]. */
void po_gqa_attention(po_model *m, int layer, const float *x, int pos, float *out);
/* rope_apply (picchio.c:455-473) on q[n_heads*hd], k[n_kv_heads*hd]. */
void po_rope_apply(const pk_cfg *c, float *q, float *k, int pos);
float po_yarn_inv_freq(const pk_cfg *c, int j);
/* embed_token (picchio.c:1472-1503), fp32 table. */
void po_embed(po_model *m, int tok, float *x);
/* forward_token (picchio.c:1655-1756) with greedy sampling; logits optional. */
int po_forward_token(po_model *m, int tok, int pos, float *logits);
/* Test diagnostics: every po_moe_forward appends its router logits to buf
 * (until cap_floats), NULL: off. */
void po_set_router_trace(float *buf, int64_t cap_floats);
int64_t po_router_trace_used(void);
/* forward_prefill (picchio.c:1795-1932) for n tokens at pos_base. */
int po_forward_prefill(po_model *m, const int *ids, int n, int pos_base);
/* prefill_tokens (picchio.c:1936-1975): chunks of `batch` through forward_prefill. */
int po_prefill_tokens(po_model *m, const int *ids, int n, int pos_base, int batch);
/* greedy branch of sample_logits (picchio.c:1555-1560). */
int po_argmax(const float *logits, int n);

/* sample_logits (picchio.c:1509-1649) with its globals as explicit state:
 * repetition penalty over the sampled history, greedy below temperature
 * 1e-6, temperature, top-k by the K-th largest value (ties kept), softmax,
 * top-p over the probabilities > 1e-10 sorted descending, then the
 * xorshift64 draw and the cumulative pick in vocabulary order. Modifies
 * logits in place as the reference does. */
typedef struct po_sampler {
    float temperature, top_p;
    int top_k;
    float rep_penalty;
    uint64_t rng;
    int history_len;
    int history[4096];
} po_sampler;
void po_sampler_init(po_sampler *s, float temperature, float top_p, int top_k, float rep_penalty,
                     uint64_t seed);
float po_rng_float(uint64_t *state);
int po_sample_logits(po_sampler *s, float *logits, int vocab);
/* Not a reference function: the library's sampler arithmetic, which beyond
 * 4096 kept entries makes every sum exact (64-bit integers of the values
 * times a power of two, rounded once) where the reference adds floats one at
 * a time; up to 4096 kept entries it is po_sample_logits. */
int po_sample_logits_fx(po_sampler *s, float *logits, int vocab);

/* ── the opt-in integer-dot expert arithmetic, restated ──
 * Not a reference function: the arithmetic of the library's v_dot8 GEMV.
 * po_act_records: per 32 values (n % 32 == 0) a record of 24 ints: k = frexp
 * exponent of the largest magnitude (0 if none), A = rint(x 2^(18-k)) as five
 * balanced base-16 digits d_i in [-8, 7] (A = sum d_i 16^i), int 4i + w =
 * digit i of columns 8w..8w+7 (nibble n = column 8w+n), int 20 = k.
 * po_i4_dot_matvec: y[o] = sum over groups (in order) of
 * t_g = S_g0 C_g0 then fma(S_g1, C_g1, t_g), acc = acc + t_g, + bias, with
 * C = sum (q-8) A exact and S = (16 s) 2^(k-22). */
void po_act_records(const float *x, int n, int32_t *rec);
void po_i4_dot_matvec(const uint8_t *q4, const float *s, const float *bias, int O, int I,
                      const int32_t *rec, float *y);

/* ── the GPU's expert-grouped (int8 matrix core) path, restated ──
 * Not a reference function: the exact arithmetic the library's grouped
 * prefill uses, so its integer parts and fold order can be checked bit for
 * bit. Per row: k = binary exponent of max|x| (0 if all zero),
 * A = rint(x 2^(20-k)) = a0 2^14 + a1 2^7 + a2, limbs[3][rows][cols]. */
void po_act_limbs(const float *x, int rows, int cols, int8_t *limbs, int32_t *exps);
/* y[o] = (sum_g fma-fold of (16 s[o][g]) * (float) C_g) 2^(k-24) + bias[o],
 * C_g = sum over the group of A q (exact int32), for one activation row
 * given as its three limb rows (l0, l1, l2) and exponent k. */
void po_mfma_matvec(const uint8_t *q4, const float *s, const float *bias, int O, int I,
                    const int8_t *l0, const int8_t *l1, const int8_t *l2, int k, float *y);

#ifdef __cplusplus
}
#endif
#endif
