/* picchio_hip.h — C ABI of the MI355X (gfx950) quantized-MoE expert path.
 *
 * Drop-in boundary for picchio's expert path. Each entry point replaces one
 * reference function (cited file:line into picchio) at its existing call
 * site; all arguments are plain pointers, sizes and opaque handles.
 *
 * Conventions
 *  - Every function returns PK_OK (0) or a negative PK_ERR_* code and never
 *    exits the process; pk_last_error() gives a message for the calling thread.
 *    (The reference exits on OOM / unknown format, quant.h:60-72, :334-336, and
 *    silently skips a missing expert, picchio.c:730-733 / :1394; here both are
 *    error codes, and a missing expert is fatal for the call.)
 *  - Pointers named *_dev are device (HBM) pointers; *_host are host pointers.
 *    Device work is queued on the engine's stream; functions that return host
 *    results synchronise that stream before returning.
 *  - Weight tensors are handed over in picchio's host layout (pk_qt_host ==
 *    QT, quant.h:32-40) and re-laid out in HBM by the library.
 */
#ifndef PICCHIO_HIP_H
#define PICCHIO_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_OK               0
#define PK_ERR_ARG         -1   /* bad argument: null pointer, shape, id      */
#define PK_ERR_HIP         -2   /* HIP runtime error                           */
#define PK_ERR_OOM         -3   /* device allocation / store budget exceeded   */
#define PK_ERR_UNSUPPORTED -4   /* format or shape the path does not implement */
#define PK_ERR_MISSING     -5   /* expert / layer / tensor never uploaded      */
#define PK_ERR_CONTEXT_FULL -6  /* pos >= context capacity                     */

/* Tensor formats: QT.fmt values (quant.h:33). */
#define PK_FMT_F32  0
#define PK_FMT_INT8 1
#define PK_FMT_INT4 2

/* Model configuration. Field-for-field the parameter set of picchio's Cfg
 * (picchio.c:53-83, defaults picchio.c:363-392), plus the two settings that
 * picchio reads from the checkpoint instead of config.json (group_size,
 * inferred at picchio.c:781-784; lm_head_fmt, picchio.c:2534-2650). */
typedef struct pk_cfg {
    int32_t hidden;            /* D (2880)                                  */
    int32_t n_layers;          /* 24 (20B) / 36 (120B)                      */
    int32_t n_heads;           /* 64                                        */
    int32_t n_kv_heads;        /* 8                                         */
    int32_t head_dim;          /* 64                                        */
    int32_t n_experts;         /* 32 (20B) / 128 (120B)                     */
    int32_t topk;              /* 4                                         */
    int32_t moe_inter;         /* gate_up rows = 2 * intermediate (5760)    */
    int32_t vocab;             /* 201088                                    */
    int32_t ctx_len;           /* KV capacity in positions (kv_init max_pos)*/
    int32_t sliding_window;    /* 128                                       */
    float   eps;               /* RMSNorm epsilon (1e-5)                    */
    float   theta;             /* RoPE base (150000)                        */
    float   rope_factor;       /* YaRN factor (32)                          */
    float   rope_beta_fast;    /* 32                                        */
    float   rope_beta_slow;    /* 1                                         */
    int32_t rope_original_ctx; /* 4096                                      */
    int32_t rope_truncate;     /* 0/1                                       */
    float   rope_attn_factor;  /* 0.1*ln(factor)+1 when factor > 1          */
    float   swiglu_limit;      /* 7.0                                       */
    float   swiglu_alpha;      /* 1.702                                     */
    float   routed_scale;      /* 1.0                                       */
    int32_t group_size;        /* expert INT4 scale group (64)              */
    int32_t lm_head_fmt;       /* PK_FMT_F32 or PK_FMT_INT8                 */
    int8_t  layer_type[128];   /* 0 = sliding window, 1 = full causal       */
} pk_cfg;

/* Host tensor in picchio's QT layout (quant.h:32-40):
 *  F32 : data = float[O][I]
 *  INT8: data = int8[O][I],  s = float[O]                 (per row)
 *  INT4: data = uint8[O][ceil(I/2)], low nibble = even column, value = nib-8;
 *        block_size == 0 -> s = float[O] (per row, quant.h:191-253)
 *        block_size  > 0 -> s = float[O][ceil(I/block_size)] (quant.h:259-319) */
typedef struct pk_qt_host {
    int32_t fmt;
    const void *data;
    const float *s;
    int32_t O, I;
    int32_t block_size;
} pk_qt_host;

typedef struct pk_engine pk_engine;   /* one GPU, one stream, one HBM store  */
typedef struct pk_qt pk_qt;           /* a weight tensor resident in HBM     */

const char *pk_last_error(void);
const char *pk_version(void);

/* ── engine ────────────────────────────────────────────────────────────── */

/* Creates an engine on `device` for `cfg`: allocates the HBM expert store
 * (n_layers x n_experts slots, replacing the LRU pool of picchio.c:117-136 and
 * its sizing at picchio.c:2938-3000), the dense-weight slots and the KV cache
 * (kv_init, picchio.c:479-490). */
int pk_engine_create(const pk_cfg *cfg, int device, pk_engine **out);
int pk_engine_destroy(pk_engine *e);
/* hipStream_t the engine queues its work on. */
void *pk_engine_stream(pk_engine *e);
int pk_engine_sync(pk_engine *e);
/* Bytes of HBM held by the engine (store + dense + KV + scratch). */
int64_t pk_engine_device_bytes(pk_engine *e);

/* ── loading (replaces expert_load / load_dense_weights; picchio.c:698-888,
 *    :2534-2650). Host tensors are copied; the caller keeps ownership. ── */

/* One expert of one layer: gate_up [moe_inter][hidden], down [hidden][moe_inter/2],
 * both INT4 group-scaled (block_size == cfg.group_size); biases fp32. */
int pk_store_expert(pk_engine *e, int layer, int eid,
                    const pk_qt_host *gate_up, const pk_qt_host *down,
                    const float *gu_bias_host, const float *d_bias_host);

/* Dense tensors of one layer (Layer, picchio.c:89-116). wq/wk/wv/wo must be F32. */
typedef struct pk_layer_host {
    const float *in_ln, *post_ln;              /* [hidden]                     */
    pk_qt_host wq, wk, wv, wo;                 /* F32                          */
    const float *bq, *bk, *bv, *bo;            /* biases                       */
    const float *sinks;                        /* [n_heads]                    */
    const float *router;                       /* [n_experts][hidden]          */
    const float *router_bias;                  /* [n_experts]                  */
} pk_layer_host;
int pk_store_layer(pk_engine *e, int layer, const pk_layer_host *l);

/* Embedding (F32), lm_head (F32 or INT8 per row) and the final norm. */
int pk_store_globals(pk_engine *e, const pk_qt_host *embed,
                     const pk_qt_host *lm_head, const float *final_norm_host);

/* ── converted checkpoints (convert.py output: config.json + safetensors
 *    shards). Replaces cfg_load (picchio.c:349-420), the shard discovery of
 *    main (picchio.c:2848-2915), load_dense_weights (picchio.c:2534-2650) and
 *    expert_load / load_expert_bias (picchio.c:634-888) for every expert:
 *    the whole model is made resident. ── */

/* <dir>/config.json into cfg with cfg_load's keys and defaults, plus what
 * picchio reads from the shards: the experts' group size (picchio.c:781-784)
 * and the lm_head format (INT8 rows or F32). ctx_len > 0 replaces
 * max_position_embeddings as the KV capacity. Reads host files only. */
int pk_cfg_from_container(const char *dir, int ctx_len, pk_cfg *cfg);

/* Every tensor of the container into the engine (created with that cfg):
 * embedding (F32/BF16/F16, or INT8/INT4 rows dequantized as embed_token
 * does), lm_head (F32 or INT8 rows), norms (1.0 when absent), F32 attention
 * and biases (0 when absent), sinks, router (either name) and its bias, and
 * the INT4 experts (the three name spellings, ".qs" group scales) with their
 * biases (per expert, aggregated [E][n], or the legacy INT4 bias). Formats
 * the GPU path does not hold (F32/BF16 experts, BF16 attention, INT4
 * lm_head) return PK_ERR_UNSUPPORTED; a missing expert PK_ERR_MISSING.
 * n_threads shard readers (<= 0: 8). */
int pk_load_container(pk_engine *e, const char *dir, int n_threads);

/* Builds every tensor of the engine's cfg from `seed` with the generator of
 * pk_synth.h (N(0,0.02) weights, norms 1.0), quantizing the experts on the GPU
 * with pk_quantize_int4_gs. `what`: bit 0 experts+routers, bit 1 attention,
 * bit 2 embedding/lm_head/final norm. */
int pk_engine_build_synthetic(pk_engine *e, uint64_t seed, int what, int n_threads);

/* ── quantization (convert.py:45-93, the gs64 converter) ── */

/* Device fp32 w[O][I] -> packed uint8[O][ceil(I/2)] + float[O][ceil(I/gs)],
 * byte-identical to convert.quantize_int4(w, group_size=gs). */
int pk_quantize_int4_gs(pk_engine *e, const float *w_dev, int O, int I, int gs,
                        uint8_t *packed_dev, float *scales_dev);

/* ── tensors and matmul_qt (quant.h:323-337) ── */

int pk_qt_upload(pk_engine *e, const pk_qt_host *h, pk_qt **out);
int pk_qt_free(pk_engine *e, pk_qt *t);
/* y_dev[S][O] = x_dev[S][I] · Wᵀ (matmul_qt, quant.h:323). INT4 group-scaled
 * results are bit-identical to quant.h's AVX2 matmul_i4_gs. */
int pk_matmul_qt(pk_engine *e, float *y_dev, const float *x_dev, const pk_qt *w, int S);

/* ── expert path ── */

/* expert_apply (picchio.c:1768-1791): dst_dev[hidden] += w · expert(x_dev). */
int pk_expert_apply(pk_engine *e, int layer, int eid, const float *x_dev,
                    float *dst_dev, float w);

/* The two expert matmul_qt call sites of moe_forward, each batched over n
 * experts of one layer in a single launch (eids_dev: n device int32 ids):
 *  gate_up (picchio.c:1399, bias :1400-1402, clamped SwiGLU :1415-1424):
 *    act_dev[n][moe_inter/2] = SwiGLU(gate_up_k · x_dev + b)
 *  down (picchio.c:1431, bias :1432-1434):
 *    eo_dev[n][hidden] = down_k · act_dev[k] + b
 * Same bits as the matching steps of pk_moe_forward. */
int pk_expert_gate_up(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                      const float *x_dev, float *act_dev);
int pk_expert_down(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                   const float *act_dev, float *eo_dev);

/* ── integer-dot expert arithmetic (no reference counterpart; opt-in for one
 *    sequence, the default of pk_decode_batch) ──
 * The expert GEMVs on v_dot8 instead of picchio's fp32 FMA chains: each
 * 32-value half-group of an input row becomes A = rint(x 2^(18-k)) (k the
 * frexp exponent of its largest magnitude) in five balanced base-16 digits,
 * a record of 24 ints; a group's sum over the stored nibbles is then exact
 * in int32 and folded in fp32 as (16 s) 2^(k-22) C. Results are within
 * ~5e-6 relative of picchio's (the north star's bar is 1e-4) instead of
 * bit-identical; measured ~3.5 % faster per MoE token. */
/* With on != 0 the three-launch MoE layer (pk_moe_forward, forward_token,
 * generate) runs on it: the router writes the input's records, the gate_up
 * launch its SwiGLU outputs' records for the down launch. Default off
 * (also PK_I4_DOT=1 in the environment at engine creation). */
int pk_set_i4_dot(pk_engine *e, int on);
/* How batch-1 MoE layers (pk_moe_forward, pk_forward_token, pk_generate)
 * run their routed experts (the router is a launch of its own):
 *   1 (default) one launch of one workgroup per gate_up row block and
 *     expert, the first of them also taking the down row blocks (k_moe_ffn);
 *   2 one launch with every CU streaming the same bytes (k_moe_bal: one
 *     workgroup per CU, each holding an equal share of the experts' 64x64
 *     tiles, values handed between workgroups as tagged words; measured
 *     slower than mode 1: three hand-overs follow the stream); where the
 *     shape or the CU count does not allow it, mode 1;
 *   0 a gate_up launch and a down launch.
 * Same results in every mode. PK_MOE_FUSED=<mode> in the environment sets
 * it at engine creation. */
int pk_set_moe_fused(pk_engine *e, int mode);
/* Diagnostic (no reference counterpart; no device work): how the one-launch
 * experts place their down tasks for gu_RB x K gate_up workgroups on a
 * device of n_cu compute units. down_task[t] (optional, n_out >= gu_RB*K
 * entries) receives the down task of workgroup t, a permutation of the
 * workgroups for every n_cu. Returns 1 if the one-launch form runs on such a
 * device (its waiting down tasks leave a free workgroup slot), 0 if the
 * layer falls back to two launches, or a negative PK_ERR_* code. */
int pk_moe_ffn_plan(int gu_RB, int dn_RB, int K, int n_cu, int dot, int *down_task, int n_out);
/* Diagnostic (no reference counterpart; no device work): the unit ranges of
 * mode 2's W workgroups for K experts of gu_RB x gu_NG gate_up and dn_RB x
 * dn_NG down tiles. ranges (optional, n_out >= 4 W) receives per workgroup
 * [gate_up first, gate_up end, down first, down end) in the unit numbering
 * (item, row block, group), group fastest. Returns 1 if mode 2 runs this
 * shape on W workgroups, 0 if it falls back, or a negative PK_ERR_* code. */
int pk_moe_bal_plan(int K, int gu_RB, int gu_NG, int dn_RB, int dn_NG, int W, int *ranges, int n_out);
/* Diagnostic (no reference counterpart; no device work): where the device KV
 * caches keep each value. For one (sequence, layer) region of ctx positions
 * x KVH heads x hd values, k_off[f] receives the float offset of K value f
 * (f = (pos * KVH + kvh) * hd + i, picchio's kv_store order, picchio.c:492-498):
 * positions in chunks of 128, inside a chunk by KV head, then by the head's
 * float4 column, then by position. V stays in picchio's order (offset f).
 * n_out >= ctx * KVH * hd. Returns 0 or a negative PK_ERR_* code. */
int pk_kv_layout(int ctx, int KVH, int hd, int64_t *k_off, int64_t n_out);
/* Batch-1 decode attention (pk_forward_token, pk_generate; gqa_attention,
 * picchio.c:504-623) and its output projection with the residual
 * (picchio.c:615-616, :1690) as one launch per layer (k_attn_oproj: the
 * projection's weight rows stream in while the attention runs) or as two
 * launches. Same results either way. Default on (PK_ATT_FUSED=0 in the
 * environment at engine creation: off). */
int pk_set_attn_fused(pk_engine *e, int on);
/* Records of x_dev[0..n) (n a multiple of 32) into rec_dev[n/32][24]. */
int pk_act_records(pk_engine *e, const float *x_dev, int n, int32_t *rec_dev);
/* pk_expert_gate_up / pk_expert_down on records: rec_dev = the input row's
 * records (shared by the n experts); act_rec_dev (optional) receives the
 * records of each expert's SwiGLU outputs, [n][moe_inter/64][24], which are
 * pk_expert_down_dot's input. */
int pk_expert_gate_up_dot(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                          const int32_t *rec_dev, float *act_dev, int32_t *act_rec_dev);
int pk_expert_down_dot(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                       const int32_t *act_rec_dev, float *eo_dev);

/* moe_forward's router (picchio.c:1316-1324): logits_dev[E] = R·x + b, the
 * launch pk_moe_forward makes first (no top-k: its expert launch selects
 * the experts). Asynchronous on the engine stream. */
int pk_router_logits(pk_engine *e, int layer, const float *x_dev, float *logits_dev);

/* moe_forward (picchio.c:1309-1466): out_dev = Σ_k (w_k·routed_scale)·expert_k(x).
 * Optional host outputs: sel_host[topk], w_host[topk] (softmaxed weights) —
 * passing either forces a stream sync. */
int pk_moe_forward(pk_engine *e, int layer, const float *x_dev, float *out_dev,
                   int32_t *sel_host, float *w_host);

/* ── several independent sequences ──
 * picchio decodes one sequence; these run its forward_token arithmetic for
 * n_seq sequences in lockstep (BASELINE config 4's batch-32 decode), each
 * sequence with its own KV cache, every weight read once per step for all
 * of them. Per sequence the result is forward_token's within the fp32 bar
 * (fp32 dot products in a different order; the MoE on the integer-dot
 * arithmetic above, the (token, expert) pairs grouped by expert so that each
 * expert block is read once per 4 pairs: within ~5e-6 of picchio's
 * arithmetic. PK_I4_DOT_BATCH=0 at engine creation: picchio's fp32 chains,
 * one launch item per pair, bit-identical GEMVs). */

/* KV caches for n_seq sequences (sequence 0 is the one pk_forward_token,
 * pk_prefill_tokens and pk_generate use). Growing the count clears every
 * cache. */
int pk_batch_reserve(pk_engine *e, int n_seq);
/* Positions 0..n_pos-1 of sequence seq's cache, every layer, filled with
 * deterministic N(0,1) rows (a synthetic prefilled context for decode
 * benchmarks; no reference counterpart). */
int pk_kv_fill_synthetic(pk_engine *e, int seq, int n_pos, uint64_t seed);
/* prefill_tokens (picchio.c:1936-1975) into sequence seq's cache. */
int pk_prefill_seq(pk_engine *e, int seq, const int32_t *ids, int n, int pos_base,
                   int32_t *next_host);
/* n_steps greedy steps of sequences 0..n_seq-1 at positions pos..pos+n_steps-1,
 * starting from toks_host[n_seq]; out_host[n_steps][n_seq] = the tokens
 * produced (each step feeds the next on the device). */
int pk_decode_batch(pk_engine *e, int n_seq, const int32_t *toks_host, int pos, int n_steps,
                    int32_t *out_host);

/* Expert-grouped prefill MoE on the matrix cores (forward_prefill's MoE,
 * picchio.c:1829-1916, as one grouped GEMM per projection): the T*topk
 * (token, expert) pairs are grouped by expert; per 64-column scale group the
 * dot products run on the f16 MFMA with the activations split in two halves
 * (default), or exactly on int8 limbs of pk_quantize_act_i8x3
 * (pk_set_grouped_f16(e, 0)), then fold in fp32 (within ~1e-6 of the
 * reference's fp32 path either way).
 * sel_dev [T][topk] / w_dev [T][topk] (combine weights, softmax x
 * routed_scale): the routing to use, both or neither (null: the layer's
 * router). out_dev [T][hidden] = each token's weighted sum in the batch's
 * first-request expert order. act_dev [T*topk][moe_inter/2] and eo_dev
 * [T*topk][hidden] (pair p = t*topk + k) optionally receive the SwiGLU
 * activations and expert outputs. */
int pk_moe_forward_grouped(pk_engine *e, int layer, const float *x_dev, int T,
                           const int32_t *sel_dev, const float *w_dev, float *out_dev,
                           float *act_dev, float *eo_dev);

/* Arithmetic of pk_moe_forward_grouped (and of the prompt's MoE on the matrix
 * cores). on = 1 (the default): activations as two halves, hi = f16(x') and
 * lo = f16(x' - hi) with x' = x 2^(15-k), weights exactly q in f16, sums in
 * fp32 on v_mfma_f32_32x32x16_f16 (~1e-7 from the reference's fp32 path, the
 * MFMA's own summation order). on = 0: the exact int8 limbs of
 * pk_quantize_act_i8x3 (bit-reproducible by a CPU restatement). No reference
 * counterpart: the reference has one fp32 path. Not while capturing. */
int pk_set_grouped_f16(pk_engine *e, int on);

/* Integer activation quantization of the grouped path: per row, k = binary
 * exponent of max|x| (x = m 2^k, m in [0.5,1)), A = rint(x 2^(20-k)), split
 * as A = a0 2^14 + a1 2^7 + a2 into limbs_dev[3][rows][cols] (int8, column
 * order as x); exps_dev[rows] = k. No reference counterpart: the reference
 * keeps fp32 activations; this is the exact integer form the MFMA path uses. */
int pk_quantize_act_i8x3(pk_engine *e, const float *x_dev, int rows, int cols,
                         int8_t *limbs_dev, int32_t *exps_dev);

/* Batched form for T tokens at once (the expert-grouped prefill of
 * forward_prefill, picchio.c:1829-1916): x_dev[T][hidden] -> out_dev[T][hidden];
 * sel_dev[T][topk] / w_dev[T][topk] optional device outputs. */
int pk_moe_forward_batch(pk_engine *e, int layer, const float *x_dev, int T,
                         float *out_dev, int32_t *sel_dev, float *w_dev);

/* No counterpart in the reference: pk_moe_forward_batch for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid it). Same arguments and results (the same kernels), but its
 * scratch (router logits, routing, the pairs' activations and outputs) is a
 * fixed 16 MiB device array, one per GPU, held until the process ends; the
 * call allocates and frees nothing. Up to about 120 tokens of the
 * GPT-OSS-20B shape fit (hidden 2880, top-4); a T that needs more scratch is
 * refused with PK_ERR_UNSUPPORTED. Calls on one GPU share that array: calls
 * that overlap on one GPU (other engines or streams) race, and each call
 * leaves its contents behind. */
int pk_moe_forward_batch_noalloc(pk_engine *e, int layer, const float *x_dev, int T,
                                 float *out_dev, int32_t *sel_dev, float *w_dev);

/* gqa_attention (picchio.c:504-623) for one token at `pos`; writes K/V. */
int pk_gqa_attention(pk_engine *e, int layer, const float *x_dev, int pos,
                     float *out_dev);

/* forward_token (picchio.c:1655-1756): returns the next token id in
 * *next_host, drawn by the engine's sampler (greedy until pk_set_sampling
 * asks otherwise); logits_dev optional [vocab]: the logits, or with sampling
 * on the array sample_logits leaves (probabilities, 0 where dropped). */
int pk_forward_token(pk_engine *e, int tok, int pos, int32_t *next_host,
                     float *logits_dev);

/* prefill_tokens (picchio.c:1936-1975): runs ids[0..n) at pos_base.. and
 * returns the token sampled after the last one. */
int pk_prefill_tokens(pk_engine *e, const int32_t *ids_host, int n, int pos_base,
                      int32_t *next_host);

/* A turn's generation (picchio.c:2771-2790 without the protocol): the
 * prompt through prefill_tokens (PREFILL_BATCH positions per chunk, default
 * 64; 1 = position by position), then n_steps - 1 replays of one captured
 * decode step with token and position carried on the device;
 * out_host[n_steps] token ids, out_host[0] the prompt's next token. Tokens
 * are drawn by the engine's sampler. */
int pk_generate(pk_engine *e, const int32_t *prompt_host, int n_prompt,
                int n_steps, int32_t *out_host);

/* n_steps greedy decode steps from (tok, pos) over the existing KV cache,
 * replaying the captured step (for timing); out_host[n_steps] token ids.
 * The captured step's attention covers positions below a power of two of at
 * least 1024; a call that goes past it captures the step again (once per
 * doubling). */
int pk_decode_replay(pk_engine *e, int tok, int pos, int n_steps, int32_t *out_host);

/* ── sampling (sample_logits, picchio.c:1509-1649) on the device ──
 * One sampler state per engine, in device memory: temperature, top-p,
 * top-k, repetition penalty, the xorshift64 state and the penalty history
 * (4096 ids). Every token the decode path produces (forward_token, each
 * prefill chunk, each generate step) is drawn from it as the reference
 * draws: penalty over the history, greedy below temperature 1e-6, top-k
 * threshold with ties kept, softmax, top-p over probabilities > 1e-10,
 * cumulative pick, and the pick appended to the history. Results equal the
 * reference's up to the device expf's last ulp (a draw within an ulp of a
 * boundary may differ). Until configured the engine is greedy. Batched
 * decode (pk_decode_batch) stays greedy and refuses to run with sampling on. */

/* The start-up settings TEMPERATURE, TOPP, TOPK, REP and SEED
 * (picchio.c:3033-3037, defaults 1.0 / 0.95 / 50 / 1.1 at :1510-1513):
 * replaces every parameter, seeds the rng and empties the history.
 * Temperature < 1e-6 with rep_penalty <= 1 is the plain argmax. */
int pk_set_sampling(pk_engine *e, float temperature, float top_p, int top_k,
                    float rep_penalty, uint64_t seed);
/* A TURN's per-request temperature, top-p and top-k (picchio.c:2737-2743,
 * with its clamp: temperature to [0, 5], top-p outside (0, 1] -> 1, negative
 * top-k -> 0); penalty, rng and history carry on. */
int pk_set_turn_sampling(pk_engine *e, float temperature, float top_p, int top_k);
/* RESET's history clear (picchio.c:2711-2716). */
int pk_reset_history(pk_engine *e);
/* sample_logits(logits, vocab) (picchio.c:1540) on a device vector, which is
 * modified in place as the reference modifies its array; the id into
 * *tok_host. Advances the rng and the history like any draw. */
int pk_sample_logits(pk_engine *e, float *logits_dev, int vocab, int32_t *tok_host);
/* No reference counterpart (a speed option): with on != 0, draws that keep
 * more than 4096 entries (no top-k over a large vocabulary) add their floats
 * exactly, as 64-bit integers of the values times a power of two, rounded to
 * float once, instead of one at a time in the reference's order; the top-p
 * cut is the shortest descending prefix whose exact sum reaches top_p and the
 * pick the first index whose exact running sum reaches the draw. About ten
 * times faster there; the probabilities differ from the reference's by its
 * own float rounding (about 1e-5 relative at 200k entries), which over a
 * flat distribution moves a top-p cut or a pick now and then. Draws keeping
 * up to 4096 entries are unaffected. Default off. */
int pk_set_sampling_fast_sums(pk_engine *e, int on);
/* The sampler's rng state and history (up to cap ids into history_host,
 * which may be NULL); *history_len the full length. */
int pk_sampler_state(pk_engine *e, uint64_t *rng, int32_t *history_host, int cap,
                     int *history_len);

/* ── measurement (no reference counterpart: benchmark plumbing) ──
 * With profiling on, the engine brackets each launch of the listed kernels
 * with a pair of HIP events on its stream; pk_engine_profile_read syncs and
 * returns the summed kernel time and launch count since the last reset. */
#define PK_PROF_EXPERT_GATE_UP 0   /* INT4 gate_up GEMV + SwiGLU (all top-k experts) */
#define PK_PROF_EXPERT_DOWN    1   /* INT4 down GEMV                                 */
#define PK_PROF_ROUTER         2   /* router GEMV + top-k                            */
#define PK_PROF_COMBINE        3   /* weighted combine                               */
#define PK_PROF_MOE_FFN        4   /* batch-1 experts in one launch: gate_up .. combine */
#define PK_PROF_LM_HEAD        5   /* lm_head GEMV + greedy argmax                   */
#define PK_PROF_ATTENTION      6   /* QKV .. O-projection of one layer (5 launches)  */
#define PK_PROF_N              8
int pk_engine_profile(pk_engine *e, int enable);
int pk_engine_profile_read(pk_engine *e, int kernel, double *total_ms, int64_t *launches);
/* ── diagnostics (no device work of their own beyond copies; not while
 *    capturing a graph) ──
 * Router trace: while buf_dev is set, every MoE router launch appends its
 * logits (+ bias) to buf_dev in launch order — batch-1 layers one row of
 * n_experts floats each (pk_moe_forward, pk_forward_token), batched rows
 * [rows][n_experts] per layer (pk_decode_batch, pk_prefill_*) — until
 * cap_floats would be exceeded; pk_router_trace_used gives the floats
 * written. The logits are what the top-k (picchio.c:1327-1339) ranks, so a
 * caller sees how close each routing decision was. NULL turns it off. */
int pk_set_router_trace(pk_engine *e, float *buf_dev, int64_t cap_floats);
int64_t pk_router_trace_used(pk_engine *e);
/* picchio's TRACE_NUMERIC (picchio.c:251-288, :1356-1360, :1666-1745): with
 * on != 0 (or TRACE_NUMERIC=1 in the environment at engine creation) each
 * eager pk_forward_token prints to stderr, per stage, the residual's min,
 * max, rms and count of non-finite entries, per layer the routing (experts,
 * softmax weights, and the 4th / 5th logit margin), and the top-10 logits.
 * Synchronises the stream at every stage; replayed graphs print nothing. */
int pk_set_numeric_trace(pk_engine *e, int on);
/* Queues a bounded idle kernel (about `usec` microseconds, at most 1 s) so
 * that the host can queue work ahead of the GPU before a profiled pass. */
int pk_engine_stall(pk_engine *e, int usec);
/* No reference counterpart (picchio runs on the host). The one-launch forms
 * (pk_set_moe_fused modes 1 and 2, pk_set_attn_fused) hand values between
 * workgroups of one launch and so need all of them resident at once. On a
 * device shared with other work a device-side wait can reach its bound; all
 * waves still end. The engine then turns both options off, so that the
 * separate launches (no waits) run from then on, and the call that saw it
 * runs again:
 *   - pk_forward_token (with next_host), pk_generate, pk_decode_replay,
 *     pk_prefill_tokens, pk_prefill_seq and pk_moe_forward (with host outputs,
 *     not in place) redo the call themselves;
 *   - pk_engine_sync returns PK_ERR_HIP, since the queued work is unknown.
 * pk_wait_fallbacks counts these switches. pk_set_poll_bound sets the polls
 * a wait makes before it gives up (0: the default, 2^18, several ms); a test
 * sets a tiny one to take the path. */
int pk_set_poll_bound(pk_engine *e, uint32_t polls);
int64_t pk_wait_fallbacks(pk_engine *e);

/* ── HIP graphs (no reference counterpart: launch amortisation) ──
 * Everything the engine queues between pk_capture_begin and pk_capture_end
 * (calls that return host results are refused while capturing) becomes one
 * executable graph; pk_graph_launch replays it on the engine stream. */
typedef struct pk_graph pk_graph;
int pk_capture_begin(pk_engine *e);
int pk_capture_end(pk_engine *e, pk_graph **out);
int pk_graph_launch(pk_engine *e, pk_graph *g);
int pk_graph_destroy(pk_graph *g);

#ifdef __cplusplus
}
#endif
#endif /* PICCHIO_HIP_H */
