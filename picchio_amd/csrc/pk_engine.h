// pk_engine.h — engine state shared by the host-side translation units.
#pragma once

#include "pk_internal.h"

struct pk_layer_dev {
    float *in_ln = nullptr, *post_ln = nullptr;
    float *wqkv = nullptr, *bqkv = nullptr;   // [(H + 2 KVH) hd][D], bias
    float *wo = nullptr, *bo = nullptr;       // [D][H hd], bias
    float *sinks = nullptr;                   // [H]
    float *router = nullptr, *router_b = nullptr;  // [E][D], [E]
    float *wqkv_t = nullptr, *wo_t = nullptr;  // the batched GEMM's tile-order copies (pk_dense_tiles)
    bool have_attn = false, have_router = false;
};

// Decode state in device memory: the step reads tok/pos and its argmax
// writes next, appends to the output list (n_out) and advances pos.
struct pk_dstate {
    int32_t tok, pos, n_out, next;
};

// Sampler state in device memory (picchio.c:1509-1520): parameters, the
// xorshift64 state and the repetition-penalty history. The sampling kernel
// reads and advances it, so a captured decode step samples on replay.
constexpr int PK_HISTORY_CAP = 4096;
struct pk_sampler_dev {
    float temperature, top_p, rep_penalty;
    int top_k;
    uint64_t rng;
    int32_t history_len, last;
    int32_t fast_sums;                        // exact integer sums beyond 4096 kept entries (opt-in)
    int32_t pad;
    int32_t history[PK_HISTORY_CAP];
};

// counters[] layout (uint32, zero-initialised, re-armed by their users)
constexpr int PK_CTR_ROUTER = 0;          // router+top-k arrivals
constexpr int PK_CTR_MOE_EPOCH = 8;      // router launches so far: k_moe_ffn's hand-over tag
constexpr int PK_CTR_ATT_EPOCH = 16;     // fused-QKV launches so far: k_attn_oproj's hand-over tag
constexpr int PK_CTR_MOE_STATUS = 40;    // k_moe_ffn / k_attn_oproj: 1 once a wait gave up (checked by the host)
constexpr int PK_CTR_POLL_BOUND = 41;    // their bound on polls per wait (0: the default)
constexpr int PK_CTR_COMBINE = 64;        // [row blocks] down+combine arrivals
constexpr int PK_CTR_ATTN = 4096;         // [rows x heads] attention chunk arrivals
constexpr int PK_CTR_ATTN_N = 4096;
constexpr int PK_CTR_N = PK_CTR_ATTN + PK_CTR_ATTN_N;

struct pk_engine {
    pk_cfg c{};
    int device = 0;
    hipStream_t stream = nullptr;
    int64_t device_bytes = 0;

    // expert store: n_layers * n_experts slots of `ex.stride` bytes
    pk_expert_layout ex{};
    uint8_t *store = nullptr;
    uint8_t *expert_ready = nullptr;          // host flags [L*E]

    pk_layer_dev *L = nullptr;                // host array of device pointers
    float *embed = nullptr;                   // [vocab][D] fp32
    float *lm_f32 = nullptr;                  // [vocab][D]
    float *lm_t = nullptr;                    // its tile-order copy (pk_dense_tiles)
    // the tile-order copies are current when tiles_ver == dense_ver; every
    // upload or build of the fp32 projections and lm_head advances dense_ver
    int64_t dense_ver = 1, tiles_ver = 0;
    int8_t *lm_q8 = nullptr;                  // [vocab][D]
    float *lm_s = nullptr;                    // [vocab]
    float *final_norm = nullptr;
    bool have_globals = false;

    float *rope = nullptr;                    // [ctx][hd/2][2] (cos, sin) * attn_factor
    float *K = nullptr, *V = nullptr;         // [n_seq][L] regions of ctx x kv_dim (K chunked: pk_k_off)
    int n_seq = 1;                            // sequences with a KV cache (pk_batch_reserve)
    int64_t seq_stride = 0;                   // floats per sequence in K / V

    // staging for uploads / synthetic builds
    uint8_t *stage = nullptr;
    int64_t stage_bytes = 0;

    // decode scratch
    float *x_in = nullptr, *h = nullptr, *hn = nullptr, *attn_out = nullptr;
    float *qkv = nullptr, *att = nullptr, *logits = nullptr;
    float *r_logits = nullptr, *w_scaled = nullptr, *w_soft = nullptr;
    int32_t *sel = nullptr;
    float *act = nullptr, *eo = nullptr;
    float *attn_part = nullptr;               // split-K attention partials
    int32_t *argmax_out = nullptr;
    uint32_t *counters = nullptr;
    // integer-dot expert arithmetic of the three-launch MoE layer (opt-in:
    // PK_I4_DOT=1 or pk_set_i4_dot; default picchio's fp32 chains, bit-identical)
    bool i4_dot = false;
    // batch-1 MoE experts: 1 one launch of one workgroup per gate_up row
    // block and expert (k_moe_ffn), 2 one launch with every CU streaming the
    // same bytes (k_moe_bal; k_moe_ffn where that does not fit), 0 two
    // launches (PK_MOE_FUSED=n)
    int moe_fused = 1;
    bool i4_dot_batch = true;                 // pk_decode_batch's MoE on it (PK_I4_DOT_BATCH=0: not)
    int32_t *hn_q = nullptr;                  // the layer input's half-group records
    int32_t *act_q = nullptr;                 // [topk] SwiGLU outputs' records
    uint64_t *moe_act_t = nullptr;            // k_moe_ffn hand-over words: [topk][max(gu RB x 24, moe_inter/2)]
    uint64_t *moe_eo_t = nullptr;             // k_moe_ffn hand-over words: [topk][hidden]
    uint64_t *moe_cont_t = nullptr;           // k_moe_bal hand-over words: [topk x (gu RB + dn RB)][64]
    // batch-1 decode attention and its output projection as one k_attn_oproj
    // launch (PK_ATT_FUSED=0: two launches)
    bool attn_fused = true;
    int64_t wait_fallbacks = 0;          // calls redone with the separate launches
    uint64_t *att_t = nullptr;                // k_attn_oproj hand-over words: [heads x head_dim]

    bool capturing = false;                  // inside pk_capture_begin/end

    // diagnostics (outside graph capture only): every MoE router launch
    // appends its logits [rows][E] to rtrace (pk_set_router_trace); with
    // trace_numeric forward_token prints picchio's TRACE_NUMERIC lines
    float *rtrace = nullptr;
    int64_t rtrace_cap = 0, rtrace_used = 0;
    bool trace_numeric = false;

    // decode step (pk_decode.hip)
    bool dec_ready = false;
    pk_dstate *dstate = nullptr;              // device
    pk_dstate *pin_state = nullptr;           // pinned host staging [ctx_len]
    float *lm_bval = nullptr;                 // lm_head block maxima
    int32_t *lm_bidx = nullptr;
    hipGraphExec_t step_exec = nullptr;       // captured decode step (pk_decode_replay)
    int step_cap = -1;                        // att_pos_cap the step graph was captured with
    // Decode attention from the device state: the grid covers positions
    // 0..att_pos_cap (-1: the whole context), set by the callers that know
    // the highest position a launch or a replayed graph will reach
    int att_pos_cap = -1;
    int32_t *step_out = nullptr;

    // opt-in per-kernel timing (pk_engine_profile)
    bool prof = false;
    static constexpr int PROF_CAP = 16384;
    hipEvent_t *prof_ev = nullptr;           // [PROF_CAP][2]
    int *prof_kind = nullptr;                // [PROF_CAP]
    int prof_n = 0;
    double prof_ms[PK_PROF_N] = {0};
    int64_t prof_cnt[PK_PROF_N] = {0};

    int n_cu = 256;                          // compute units of the device
    uint8_t *noalloc_scratch = nullptr;      // this device's fixed scratch array (pk_noalloc_scratch_init)

    // batched MoE scratch for up to batch_cap tokens (pk_prefill.hip)
    int64_t batch_cap = 0;
    float *b_logits = nullptr, *b_w = nullptr, *b_act = nullptr, *b_eo = nullptr;
    // split-K workspace of the skinny fp32 GEMM over several rows (PK_SKINNY_WS floats)
    float *skinny_ws = nullptr;
    int32_t *b_sel = nullptr, *b_perm = nullptr;
    int32_t *b_xq = nullptr, *b_actq = nullptr;   // integer-dot records (rows, pairs' SwiGLU outputs)
    int32_t *b_pairs = nullptr, *b_tiles = nullptr;  // pairs grouped by expert (tiles of 4)
    bool dot_tiles_off = false;                   // PK_DOT_TILES=0: one launch item per pair
    // prompt-chunk scratch for up to p_cap positions (pk_prefill.hip)
    int p_cap = 0;
    float *p_H = nullptr, *p_XN = nullptr, *p_qkv = nullptr, *p_att = nullptr, *p_part = nullptr;
    int32_t *p_ids = nullptr;
    // batched decode (pk_decode_batch): logits [n_seq][vocab], token ring
    int bd_cap = 0, bd_steps = 0;
    float *bd_logits = nullptr;
    int32_t *bd_toks = nullptr;
    // grouped MFMA scratch for up to g_cap pairs (pk_prefill.hip)
    int64_t g_cap = 0;
    int8_t *g_limbs = nullptr;                 // int8 limbs (3 planes) or f16 hi/lo (2 planes of halves)
    // grouped arithmetic: true = f16 hi/lo on v_mfma_f32_32x32x16_f16 (the
    // default), false = exact int8 limbs (PK_GROUPED_F16 / pk_set_grouped_f16)
    bool grouped_f16 = true;
    int32_t *g_exps = nullptr, *g_pairs = nullptr, *g_tiles = nullptr;
    // sampler (pk_sample.hip): device state, host mirror of its parameters,
    // kept entries (value, index) for vocabularies up to samp_cap entries
    pk_sampler_dev *samp = nullptr;
    pk_sampler_dev samp_params{};             // temperature .. rng as last set from the host
    bool samp_on = false;                     // the decode step samples instead of argmax
    int samp_cap = 0;
    float *samp_av = nullptr;
    int32_t *samp_ai = nullptr;
};

// Fixed device array of pk_moe_forward_batch_noalloc (pk_prefill.hip): its
// size, and its address on the engine's device into e->noalloc_scratch.
constexpr int64_t PK_NOALLOC_SCRATCH_BYTES = 16ll << 20;
constexpr int PK_NOALLOC_MAX_DEVICES = 64;
int pk_noalloc_scratch_init(pk_engine *e);

int pk_dev_alloc(pk_engine *e, void **p, int64_t bytes);
void pk_dev_free(pk_engine *e, void *p);
int pk_stage_reserve(pk_engine *e, int64_t bytes);

// kernels defined in pk_dense.hip / pk_attn.hip without a launcher above
int pk_launch_topk_records(const float *logits, int T, int E, int K, float routed_scale, int32_t *sel,
                           float *w_scaled, const float *x, int n, int32_t *rec, hipStream_t st);
int pk_launch_topk_batch(const float *logits, int T, int E, int K, float routed_scale,
                         int32_t *sel, float *w_scaled, float *w_soft, hipStream_t st);
int pk_launch_combine(float *out, const float *eo, const float *w, int K, int D,
                      const float *residual, float *res_out, hipStream_t st);
int pk_launch_axpy(float *dst, const float *eo, float w, int D, hipStream_t st);
int pk_launch_fill_normal(float *out, int64_t n, uint64_t stream_seed, float std, hipStream_t st);
// The same values for n_pos positions of a K cache region, in its chunk layout (pk_k_off).
int pk_launch_fill_normal_k(float *out, int n_pos, int ctx, int KVH, int hd, uint64_t stream_seed, float std,
                            hipStream_t st);
int pk_launch_fill_const(float *out, int64_t n, float v, hipStream_t st);

// profiling brackets around a launch (no-ops unless profiling is on)
int pk_prof_begin(pk_engine *e, int kind);
int pk_prof_end(pk_engine *e, int slot);

// internal MoE pieces reused by the decode and prompt drivers
int pk_moe_layer(pk_engine *e, int layer, const float *x_dev, float *out_dev,
                 const float *residual, float *res_out, const float *norm_w = nullptr);
int pk_check_layer_experts(pk_engine *e, int layer);
pk_i4_items pk_expert_items(pk_engine *e, int layer, bool down);

// ── expert-grouped MFMA GEMM (pk_mfma.hip) ──
struct pk_mfma_args {
    const uint8_t *base;                       // expert store
    int64_t slot_stride, off_tiles, off_scales, off_bias;
    int32_t slot_base;                         // layer * n_experts
    int O, NG;                                 // output rows, 64-column groups
    const int8_t *limbs;                       // 3 planes of activation limbs (permuted columns)
    int64_t plane;                             // bytes between limb planes
    int lrow;                                  // bytes per activation row (= its columns)
    const int32_t *exps;                       // per activation row: scale exponent
    const uint16_t *xf;                        // half-precision path: hi plane, lo plane at + fplane (halves)
    int64_t fplane;
    int frow;                                  // halves per activation row (= its columns)
    const int32_t *pairs;                      // pair ids grouped by expert
    int x_div;                                 // activation row of pair p = p / x_div
    const int32_t *tile_exp, *tile_beg, *tile_cnt, *n_tiles;
    const int32_t *tile_grp;                   // per tile: the expert's first tile, tile count (or null)
    float *y;                                  // output rows by pair id
    int64_t y_stride;
    float lim, alpha;                          // SwiGLU clamp / slope
};
int pk_launch_act_limbs(const float *x, int64_t x_stride, int rows, int cols, int8_t *limbs, int64_t plane,
                        int32_t *exps, int permuted, hipStream_t st);
// tile_pairs: pairs per tile (0: the MFMA GEMM's 32)
int pk_launch_group_pairs(const int32_t *sel, int P, int E, int32_t *pairs, int32_t *tile_exp,
                          int32_t *tile_beg, int32_t *tile_cnt, int32_t *n_tiles, hipStream_t st,
                          int tile_pairs = 0, int32_t *tile_grp = nullptr);
int pk_launch_moe_mfma(const pk_mfma_args &a, int max_tiles, int epilogue, hipStream_t st);
constexpr int64_t PK_SKINNY_WS = (int64_t)2 << 20;   // floats: 12 K splits x 32 rows x 5120 outputs
// half-precision pair arithmetic (pk_mfma.hip): activation planes, grouped GEMM
// over tiles of PK_F16_TILE pairs
constexpr int PK_F16_TILE = 64;
int pk_launch_act_f16(const float *x, int64_t x_stride, int rows, int cols, uint16_t *xf, int64_t fplane,
                      int32_t *exps, hipStream_t st);
int pk_launch_moe_f16(const pk_mfma_args &a, int max_tiles, int epilogue, hipStream_t st);

// Builds (outside a capture) the tile-order copies of the fp32 QKV and
// O-projection weights and of the fp32 lm_head for the batched GEMM, when
// they are not current; pk_tiles_current says whether they may be read.
int pk_dense_tiles(pk_engine *e);
inline bool pk_tiles_current(const pk_engine *e) { return e->tiles_ver == e->dense_ver; }

// decode driver pieces (pk_decode.hip) reused by the prompt driver
int pk_decode_reserve(pk_engine *e);
int pk_check_model(pk_engine *e);
int pk_set_state(pk_engine *e, int tok, int pos);
// Rows r = 0..n-1 at position (st ? st->pos : pos_base + r * pos_step) of
// sequence seq0 + r * seq_step.
// norm_w (n == 1 only): xn is the raw residual row, normalised inside the QKV GEMV.
// exact: the prompt rows in the reference's operation order (pk_exact.hip).
int pk_attention_rows(pk_engine *e, int l, const pk_dstate *st, int pos_base, int pos_step, int seq0,
                      int seq_step, int n, const float *xn, float *qkv, float *part, float *att, float *h,
                      const float *norm_w = nullptr, bool exact = false);
// the prompt path's dense steps in the reference's order (pk_exact.hip)
int pk_launch_gemm_chain8(const float *X, int64_t ldx, const float *W, const float *bias, float *out, int64_t ldo,
                          int S, int I, int O, bool add_res, hipStream_t st);
int pk_launch_gemm_chain8_q8(const float *X, const int8_t *W, const float *scale, float *out, int S, int I, int O,
                             hipStream_t st);
int pk_launch_attn_rows_exact(int pos_base, int n, const float *qkv, int64_t qkv_stride, const float *Kl,
                              const float *Vl, int H, int KVH, int hd, int ctx, int sliding, int window,
                              const float *sinks, float *att, hipStream_t st);
int pk_launch_router_seq(const float *X, const float *R, const float *bias, int S, int D, int E, float *logits,
                         hipStream_t st);
int pk_lm_head_step(pk_engine *e, const float *hn, float *logits_dev, int32_t *out_toks, int out_cap);
// sampler (pk_sample.hip): draw from logits[0..vocab) with the engine's
// sampler state; st != nullptr also updates the decode state like the argmax
int pk_sample_reserve(pk_engine *e, int vocab);
// block_max[0..n_blocks): optional maxima of blocks of the logits before the
// penalty; write_back = false when nobody reads the logits afterwards
int pk_launch_sample(pk_engine *e, float *logits, int vocab, pk_dstate *st, int32_t *out_toks, int out_cap,
                     const float *block_max, int n_blocks, bool write_back);
// prompt tokens into the repetition-penalty history (prefill_tokens, picchio.c:1960-1967)
int pk_sample_seed_history(pk_engine *e, const int32_t *ids_dev, int n);
// one forward_token step for (tok, pos), greedy id appended to out_toks
int pk_decode_token(pk_engine *e, int tok, int pos, int32_t *out_toks, int out_cap);
// prefill_tokens (pk_prefill.hip): the prompt, next id into the decode state / out_toks
int pk_prefill_run(pk_engine *e, int seq, const int32_t *ids, int n, int pos_base, int32_t *out_toks,
                   int out_cap);

// Diagnostics: the router trace append (no-op unless set and not capturing),
// and the numeric trace lines of forward_token (host syncs; trace_numeric only).
int pk_trace_router(pk_engine *e, const float *logits_dev, int rows);
int pk_trace_vec(pk_engine *e, const char *stage, int layer, const float *dev, int n);
int pk_trace_route(pk_engine *e, int layer, const float *logits_dev);
int pk_trace_top_logits(pk_engine *e, const float *logits_dev);
// After a stream sync: if a device-side wait gave up, the one-launch forms
// are switched off (the separate launches do not wait) and *redo is set, so
// that the caller runs its call again; an error if it happened with them off.
int pk_wait_fallback(pk_engine *e, bool *redo);
