// pk_engine.hip — host side of the C ABI: engine, HBM expert store, uploads,
// matmul_qt and the MoE call chain.
#include "pk_engine.h"
#include "pk_synth.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

// ───────────────────────── errors ─────────────────────────
static thread_local char g_err[512] = "";

void pk_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" const char *pk_last_error(void) { return g_err; }
extern "C" const char *pk_version(void) { return "picchio-amd 0.1 (gfx950)"; }

// ───────────────────────── memory ─────────────────────────
int pk_dev_alloc(pk_engine *e, void **p, int64_t bytes) {
    *p = nullptr;
    if (bytes <= 0) return PK_OK;
    hipError_t rc = hipMalloc(p, (size_t)bytes);
    if (rc != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        pk_set_error("hipMalloc(%lld bytes) failed: %s", (long long)bytes, hipGetErrorString(rc));
        return PK_ERR_OOM;
    }
    e->device_bytes += bytes;
    return PK_OK;
}

void pk_dev_free(pk_engine *e, void *p) {
    (void)e;
    if (p) (void)hipFree(p);
}

int pk_stage_reserve(pk_engine *e, int64_t bytes) {
    if (bytes <= e->stage_bytes) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "uploads are not available while capturing a graph");
    PK_HIP(hipStreamSynchronize(e->stream));
    if (e->stage) {
        pk_dev_free(e, e->stage);
        e->device_bytes -= e->stage_bytes;
        e->stage = nullptr;
        e->stage_bytes = 0;
    }
    PK_TRY(pk_dev_alloc(e, (void **)&e->stage, bytes));
    e->stage_bytes = bytes;
    return PK_OK;
}

#define ALLOC(ptr, bytes) PK_TRY(pk_dev_alloc(e, (void **)&(ptr), (int64_t)(bytes)))

// ───────────────────────── configuration ─────────────────────────
static int cfg_check(const pk_cfg *c) {
    PK_CHECK(c, PK_ERR_ARG, "cfg is null");
    PK_CHECK(c->hidden > 0 && c->n_layers > 0 && c->n_experts > 0 && c->topk > 0, PK_ERR_ARG,
             "cfg: non-positive dimension");
    PK_CHECK(c->topk <= c->n_experts && c->topk <= 16 && c->n_experts <= 128, PK_ERR_UNSUPPORTED,
             "cfg: topk=%d n_experts=%d (supported: topk <= 16, experts <= 128)", c->topk,
             c->n_experts);
    PK_CHECK(c->moe_inter > 0 && c->moe_inter % 2 == 0, PK_ERR_ARG, "cfg: moe_inter must be even");
    PK_CHECK(c->group_size == PK_GS, PK_ERR_UNSUPPORTED,
             "cfg: expert group_size %d (the HBM store holds gs64 experts)", c->group_size);
    PK_CHECK(c->hidden % PK_GS == 0 && (c->moe_inter / 2) % PK_GS == 0, PK_ERR_UNSUPPORTED,
             "cfg: hidden and moe_inter/2 must be multiples of 64");
    PK_CHECK(c->n_layers <= 128, PK_ERR_UNSUPPORTED, "cfg: more than 128 layers");
    PK_CHECK(c->n_heads > 0 && c->n_kv_heads > 0 && c->n_heads % c->n_kv_heads == 0, PK_ERR_ARG,
             "cfg: n_heads must be a multiple of n_kv_heads");
    PK_CHECK(c->head_dim >= 16 && c->head_dim <= 128 && (c->head_dim & (c->head_dim - 1)) == 0,
             PK_ERR_UNSUPPORTED, "cfg: head_dim %d (supported: 16, 32, 64, 128)", c->head_dim);
    PK_CHECK(c->ctx_len > 0 && c->vocab > 0, PK_ERR_ARG, "cfg: ctx_len / vocab must be positive");
    PK_CHECK(c->lm_head_fmt == PK_FMT_F32 || c->lm_head_fmt == PK_FMT_INT8, PK_ERR_UNSUPPORTED,
             "cfg: lm_head_fmt %d", c->lm_head_fmt);
    return PK_OK;
}

static pk_expert_layout make_layout(const pk_cfg *c) {
    pk_expert_layout L{};
    L.gu = pk_i4_make_shape(c->moe_inter, c->hidden);
    L.dn = pk_i4_make_shape(c->hidden, c->moe_inter / 2);
    int64_t off = 0;
    L.off_gu_tiles = off;   off = pk_align256(off + L.gu.tile_bytes);
    L.off_dn_tiles = off;   off = pk_align256(off + L.dn.tile_bytes);
    L.off_gu_scales = off;  off = pk_align256(off + L.gu.scale_bytes);
    L.off_dn_scales = off;  off = pk_align256(off + L.dn.scale_bytes);
    L.off_gu_bias = off;    off = pk_align256(off + (int64_t)c->moe_inter * 4);
    L.off_dn_bias = off;    off = pk_align256(off + (int64_t)c->hidden * 4);
    L.stride = off;
    return L;
}

// RoPE table: cos/sin(pos * yarn_inv_freq(j)) * attn_factor in host libm,
// exactly as rope_apply computes them (picchio.c:431-466).
static float yarn_inv_freq(const pk_cfg *c, int j) {
    const int dim = c->head_dim;
    const float pos_freq = powf(c->theta, 2.0f * (float)j / (float)dim);
    const float extrap = 1.0f / pos_freq;
    if (c->rope_factor <= 1.0f) return extrap;
    const float pi = (float)M_PI;
    float low = (float)dim * logf((float)c->rope_original_ctx / (c->rope_beta_fast * 2.0f * pi)) /
                (2.0f * logf(c->theta));
    float high = (float)dim * logf((float)c->rope_original_ctx / (c->rope_beta_slow * 2.0f * pi)) /
                 (2.0f * logf(c->theta));
    if (c->rope_truncate) { low = floorf(low); high = ceilf(high); }
    if (low < 0) low = 0;
    if (high > dim - 1) high = (float)(dim - 1);
    if (low == high) high += 0.001f;
    float ramp = ((float)j - low) / (high - low);
    if (ramp < 0) ramp = 0;
    if (ramp > 1) ramp = 1;
    const float ef = 1.0f - ramp;
    const float interp = extrap / c->rope_factor;
    return fmaf(interp, 1.0f - ef, extrap * ef);   // contracted as in the reference build
}

static int build_rope_table(pk_engine *e) {
    const pk_cfg *c = &e->c;
    const int half = c->head_dim / 2;
    std::vector<float> inv(half), tab((size_t)c->ctx_len * half * 2);
    for (int j = 0; j < half; ++j) inv[j] = yarn_inv_freq(c, j);
    for (int p = 0; p < c->ctx_len; ++p)
        for (int j = 0; j < half; ++j) {
            const float ang = (float)p * inv[j];
            tab[((size_t)p * half + j) * 2 + 0] = cosf(ang) * c->rope_attn_factor;
            tab[((size_t)p * half + j) * 2 + 1] = sinf(ang) * c->rope_attn_factor;
        }
    PK_HIP(hipMemcpy(e->rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice));
    return PK_OK;
}

static void engine_free(pk_engine *e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    void *ptrs[] = {e->store, e->embed, e->lm_f32, e->lm_q8, e->lm_s, e->final_norm, e->rope,
                    e->K, e->V, e->stage, e->x_in, e->h, e->hn, e->attn_out, e->qkv, e->att,
                    e->logits, e->r_logits, e->w_scaled, e->w_soft, e->sel, e->act, e->eo,
                    e->attn_part, e->argmax_out, e->counters, e->b_logits, e->b_w, e->b_act,
                    e->b_eo, e->b_sel, e->b_perm, e->p_H, e->p_XN, e->p_qkv, e->p_att,
                    e->p_part, e->p_ids, e->bd_logits, e->bd_toks, e->g_limbs, e->g_exps, e->g_pairs, e->g_tiles,
                    e->lm_bval, e->lm_bidx, e->dstate, e->step_out, e->samp, e->samp_av, e->samp_ai, e->hn_q, e->act_q, e->b_xq, e->b_actq, e->b_pairs, e->b_tiles,
                    e->moe_act_t, e->moe_eo_t, e->moe_cont_t, e->att_t, e->skinny_ws, e->lm_t};
    for (void *p : ptrs) pk_dev_free(e, p);
    if (e->L) {
        for (int l = 0; l < e->c.n_layers; ++l) {
            pk_layer_dev &d = e->L[l];
            void *lp[] = {d.in_ln, d.post_ln, d.wqkv, d.bqkv, d.wo, d.bo, d.sinks, d.router, d.router_b,
                          d.wqkv_t, d.wo_t};
            for (void *p : lp) pk_dev_free(e, p);
        }
        delete[] e->L;
    }
    free(e->expert_ready);
    if (e->step_exec) (void)hipGraphExecDestroy(e->step_exec);
    if (e->pin_state) (void)hipHostFree(e->pin_state);
    if (e->prof_ev) {
        for (int i = 0; i < 2 * pk_engine::PROF_CAP; ++i) (void)hipEventDestroy(e->prof_ev[i]);
        delete[] e->prof_ev;
        delete[] e->prof_kind;
    }
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

static int engine_init(pk_engine *e) {
    const pk_cfg *c = &e->c;
    const int D = c->hidden, E = c->n_experts, L = c->n_layers;
    const int H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim, K = c->topk;
    const int half = c->moe_inter / 2;
    e->ex = make_layout(c);
    PK_HIP(hipDeviceGetAttribute(&e->n_cu, hipDeviceAttributeMultiprocessorCount, e->device));
    PK_TRY(pk_noalloc_scratch_init(e));
    ALLOC(e->store, e->ex.stride * (int64_t)L * E);
    e->expert_ready = (uint8_t *)calloc((size_t)L * E, 1);
    PK_CHECK(e->expert_ready, PK_ERR_OOM, "host allocation failed");
    e->L = new pk_layer_dev[L];
    e->seq_stride = (int64_t)L * c->ctx_len * KVH * hd;
    e->n_seq = 1;
    const int64_t kv = e->seq_stride * 4;
    ALLOC(e->K, kv);
    ALLOC(e->V, kv);
    PK_HIP(hipMemsetAsync(e->K, 0, kv, e->stream));
    PK_HIP(hipMemsetAsync(e->V, 0, kv, e->stream));
    ALLOC(e->rope, (int64_t)c->ctx_len * hd * 4);
    PK_TRY(build_rope_table(e));
    const int qkv_rows = (H + 2 * KVH) * hd;
    ALLOC(e->x_in, D * 4);
    ALLOC(e->h, D * 4);
    ALLOC(e->hn, D * 4);
    ALLOC(e->attn_out, D * 4);
    ALLOC(e->qkv, qkv_rows * 4);
    ALLOC(e->att, H * hd * 4);
    ALLOC(e->logits, (int64_t)c->vocab * 4);
    ALLOC(e->r_logits, E * 4);
    ALLOC(e->w_scaled, K * 4);
    ALLOC(e->w_soft, K * 4);
    ALLOC(e->sel, K * 4);
    ALLOC(e->act, (int64_t)K * half * 4);
    ALLOC(e->eo, (int64_t)K * D * 4);
    ALLOC(e->argmax_out, 64);
    ALLOC(e->counters, PK_CTR_N * 4);
    ALLOC(e->hn_q, (int64_t)((D + 31) / 32) * PK_XQ_INTS * 4);
    ALLOC(e->act_q, (int64_t)K * e->ex.gu.RB * PK_XQ_INTS * 4);
    const int64_t act_words = std::max<int64_t>((int64_t)e->ex.gu.RB * PK_XQ_INTS, half);
    ALLOC(e->moe_act_t, (int64_t)K * act_words * 8);
    ALLOC(e->moe_eo_t, (int64_t)K * D * 8);
    PK_HIP(hipMemsetAsync(e->moe_act_t, 0, (int64_t)K * act_words * 8, e->stream));
    PK_HIP(hipMemsetAsync(e->moe_eo_t, 0, (int64_t)K * D * 8, e->stream));
    const int64_t cont_bytes = (int64_t)K * (e->ex.gu.RB + e->ex.dn.RB) * 64 * 8;
    ALLOC(e->moe_cont_t, cont_bytes);
    PK_HIP(hipMemsetAsync(e->moe_cont_t, 0, cont_bytes, e->stream));
    ALLOC(e->att_t, (int64_t)c->n_heads * c->head_dim * 8);
    PK_HIP(hipMemsetAsync(e->att_t, 0, (int64_t)c->n_heads * c->head_dim * 8, e->stream));
    if (const char *v = getenv("PK_I4_DOT")) e->i4_dot = atoi(v) != 0;
    if (const char *v = getenv("PK_GROUPED_F16")) e->grouped_f16 = atoi(v) != 0;
    if (const char *v = getenv("PK_DOT_TILES")) e->dot_tiles_off = atoi(v) == 0;
    if (const char *v = getenv("PK_I4_DOT_BATCH")) e->i4_dot_batch = atoi(v) != 0;
    if (const char *v = getenv("PK_MOE_FUSED")) e->moe_fused = atoi(v);
    if (const char *v = getenv("PK_ATT_FUSED")) e->attn_fused = atoi(v) != 0;
    if (const char *v = getenv("TRACE_NUMERIC")) e->trace_numeric = atoi(v) != 0;   // picchio.c:2826-2827
    PK_HIP(hipMemsetAsync(e->counters, 0, PK_CTR_N * 4, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

extern "C" int pk_engine_create(const pk_cfg *cfg, int device, pk_engine **out) {
    PK_CHECK(out, PK_ERR_ARG, "out is null");
    *out = nullptr;
    PK_TRY(cfg_check(cfg));
    int n = 0;
    PK_HIP(hipGetDeviceCount(&n));
    PK_CHECK(device >= 0 && device < n, PK_ERR_ARG, "device %d not present (%d devices)", device, n);
    PK_HIP(hipSetDevice(device));
    pk_engine *e = new pk_engine();
    e->c = *cfg;
    e->device = device;
    hipError_t rc = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
    if (rc != hipSuccess) {
        pk_set_error("hipStreamCreate: %s", hipGetErrorString(rc));
        delete e;
        return PK_ERR_HIP;
    }
    int st = engine_init(e);
    if (st != PK_OK) {
        char msg[512];
        snprintf(msg, sizeof(msg), "%s", pk_last_error());
        engine_free(e);
        pk_set_error("%s", msg);
        return st;
    }
    *out = e;
    return PK_OK;
}

extern "C" int pk_engine_destroy(pk_engine *e) {
    engine_free(e);
    return PK_OK;
}

extern "C" void *pk_engine_stream(pk_engine *e) { return e ? (void *)e->stream : nullptr; }

// After a stream sync: whether a device-side wait of k_moe_ffn, k_moe_bal or
// k_attn_oproj gave up since the last look (the flag is cleared).
static int take_wait_failure(pk_engine *e, bool *failed) {
    uint32_t st = 0;
    PK_HIP(hipMemcpy(&st, e->counters + PK_CTR_MOE_STATUS, 4, hipMemcpyDeviceToHost));
    *failed = st != 0;
    if (st) {
        PK_HIP(hipMemsetAsync(e->counters + PK_CTR_MOE_STATUS, 0, 4, e->stream));
        PK_HIP(hipStreamSynchronize(e->stream));
    }
    return PK_OK;
}

// The one-launch forms hand values between workgroups of one launch, so all
// their workgroups must be resident at once; on a device shared with other
// work a wait can give up (all waves still end). The engine then takes the
// separate launches, which wait for nothing, from here on: the captured step
// graph is dropped and the caller redoes its call.
int pk_wait_fallback(pk_engine *e, bool *redo) {
    *redo = false;
    bool failed = false;
    PK_TRY(take_wait_failure(e, &failed));
    if (!failed) return PK_OK;
    if (e->moe_fused == 0 && !e->attn_fused) {
        pk_set_error("a device-side wait gave up with the one-launch forms off: results are invalid");
        return PK_ERR_HIP;
    }
    if (e->step_exec) {
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    e->moe_fused = 0;
    e->attn_fused = false;
    e->wait_fallbacks += 1;
    *redo = true;
    return PK_OK;
}

extern "C" int pk_set_poll_bound(pk_engine *e, uint32_t polls) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_poll_bound: not available while capturing");
    PK_HIP(hipMemcpyAsync(e->counters + PK_CTR_POLL_BOUND, &polls, 4, hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

extern "C" int64_t pk_wait_fallbacks(pk_engine *e) { return e ? e->wait_fallbacks : 0; }

// ───────────────────────── diagnostics ─────────────────────────
// The router logits of every MoE router launch, appended in launch order
// (batch-1: one row per layer; batched rows: [rows][E] per layer), so that a
// caller can see how close each routing decision was (the 4th / 5th logit
// margin of moe_forward's top-k, picchio.c:1327-1339). Not while capturing.
extern "C" int pk_set_router_trace(pk_engine *e, float *buf_dev, int64_t cap_floats) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_router_trace: not available while capturing");
    PK_CHECK(buf_dev == nullptr || cap_floats > 0, PK_ERR_ARG, "router trace: capacity %lld", (long long)cap_floats);
    e->rtrace = buf_dev;
    e->rtrace_cap = buf_dev ? cap_floats : 0;
    e->rtrace_used = 0;
    return PK_OK;
}

extern "C" int64_t pk_router_trace_used(pk_engine *e) { return e ? e->rtrace_used : -1; }

int pk_trace_router(pk_engine *e, const float *logits_dev, int rows) {
    if (!e->rtrace || e->capturing) return PK_OK;
    const int64_t n = (int64_t)rows * e->c.n_experts;
    if (e->rtrace_used + n > e->rtrace_cap) return PK_OK;        // full: later launches are not kept
    PK_HIP(hipMemcpyAsync(e->rtrace + e->rtrace_used, logits_dev, (size_t)n * 4, hipMemcpyDeviceToDevice,
                          e->stream));
    e->rtrace_used += n;
    return PK_OK;
}

// picchio's TRACE_NUMERIC (picchio.c:251-288, :1356-1360, :1666-1745): per
// stage of forward_token the vector's min, max, rms over its finite entries
// and the count of non-finite ones; per layer the routing (and here also
// the 4th / 5th logit margin); the top-10 logits. Lines go to stderr.
extern "C" int pk_set_numeric_trace(pk_engine *e, int on) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    e->trace_numeric = on != 0;
    return PK_OK;
}

static int trace_fetch(pk_engine *e, const float *dev, int n, std::vector<float> &host) {
    host.resize((size_t)n);
    PK_HIP(hipMemcpyAsync(host.data(), dev, (size_t)n * 4, hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

int pk_trace_vec(pk_engine *e, const char *stage, int layer, const float *dev, int n) {
    if (!e->trace_numeric || e->capturing) return PK_OK;
    std::vector<float> v;
    PK_TRY(trace_fetch(e, dev, n, v));
    int bad = 0;
    float lo = INFINITY, hi = -INFINITY;
    double ss = 0.0;
    for (float x : v) {
        if (!std::isfinite(x)) { ++bad; continue; }
        lo = std::min(lo, x);
        hi = std::max(hi, x);
        ss += (double)x * x;
    }
    fprintf(stderr, "  numeric L=%d %-18s min=% .6g max=% .6g rms=%.6g bad=%d\n", layer, stage, lo, hi,
            n > bad ? std::sqrt(ss / (n - bad)) : NAN, bad);
    return PK_OK;
}

int pk_trace_route(pk_engine *e, int layer, const float *logits_dev) {
    if (!e->trace_numeric || e->capturing) return PK_OK;
    const int E = e->c.n_experts, K = e->c.topk;
    std::vector<float> v;
    PK_TRY(trace_fetch(e, logits_dev, E, v));
    // repeated argmax with strict '>' (the lowest index wins a tie), as moe_forward
    std::vector<int> sel;
    std::vector<bool> taken((size_t)E, false);
    for (int k = 0; k <= K && k < E; ++k) {
        int bi = -1;
        for (int i = 0; i < E; ++i)
            if (!taken[i] && (bi < 0 || v[i] > v[bi])) bi = i;
        taken[bi] = true;
        sel.push_back(bi);
    }
    float m = -INFINITY, sum = 0.0f, w[16];
    const int kk = std::min(K, 16);
    for (int k = 0; k < kk; ++k) m = std::max(m, v[sel[k]]);
    for (int k = 0; k < kk; ++k) { w[k] = std::exp(v[sel[k]] - m); sum += w[k]; }
    fprintf(stderr, "  numeric route L=%d:", layer);
    for (int k = 0; k < kk; ++k) fprintf(stderr, " e%d=%.7g", sel[k], w[k] / sum);
    if ((int)sel.size() > K) fprintf(stderr, " margin%d/%d=%.3g", K, K + 1, v[sel[K - 1]] - v[sel[K]]);
    fprintf(stderr, "\n");
    return PK_OK;
}

int pk_trace_top_logits(pk_engine *e, const float *logits_dev) {
    if (!e->trace_numeric || e->capturing) return PK_OK;
    const int V = e->c.vocab;
    std::vector<float> v;
    PK_TRY(trace_fetch(e, logits_dev, V, v));
    int ids[10], bad = 0;
    float vals[10];
    for (int k = 0; k < 10; ++k) { ids[k] = -1; vals[k] = -INFINITY; }
    for (int i = 0; i < V; ++i) {
        if (!std::isfinite(v[i])) { ++bad; continue; }
        if (v[i] <= vals[9]) continue;
        int k = 9;
        while (k > 0 && vals[k - 1] < v[i]) { vals[k] = vals[k - 1]; ids[k] = ids[k - 1]; --k; }
        vals[k] = v[i];
        ids[k] = i;
    }
    fprintf(stderr, "  numeric logits bad=%d top10:", bad);
    for (int k = 0; k < 10; ++k) fprintf(stderr, " %d=%.6g", ids[k], vals[k]);
    fprintf(stderr, "\n");
    return PK_OK;
}

extern "C" int pk_engine_sync(pk_engine *e) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_HIP(hipStreamSynchronize(e->stream));
    bool redo = false;
    PK_TRY(pk_wait_fallback(e, &redo));
    if (redo) {
        pk_set_error("a device-side wait gave up: the work queued since the last sync is invalid and is to be "
                     "queued again (the engine now runs the separate launches)");
        return PK_ERR_HIP;
    }
    return PK_OK;
}

extern "C" int64_t pk_engine_device_bytes(pk_engine *e) { return e ? e->device_bytes : -1; }

// ───────────────────────── profiling ─────────────────────────
static int prof_flush(pk_engine *e) {
    if (!e->prof_n) return PK_OK;
    PK_HIP(hipStreamSynchronize(e->stream));
    for (int i = 0; i < e->prof_n; ++i) {
        float ms = 0.f;
        PK_HIP(hipEventElapsedTime(&ms, e->prof_ev[2 * i], e->prof_ev[2 * i + 1]));
        e->prof_ms[e->prof_kind[i]] += ms;
        e->prof_cnt[e->prof_kind[i]] += 1;
    }
    e->prof_n = 0;
    return PK_OK;
}

int pk_prof_begin(pk_engine *e, int kind) {
    if (!e->prof || e->capturing) return -1;
    if (e->prof_n == pk_engine::PROF_CAP && prof_flush(e) != PK_OK) return -1;
    const int slot = e->prof_n++;
    e->prof_kind[slot] = kind;
    if (hipEventRecord(e->prof_ev[2 * slot], e->stream) != hipSuccess) return -1;
    return slot;
}

int pk_prof_end(pk_engine *e, int slot) {
    if (slot < 0) return PK_OK;
    PK_HIP(hipEventRecord(e->prof_ev[2 * slot + 1], e->stream));
    return PK_OK;
}

extern "C" int pk_engine_profile(pk_engine *e, int enable) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    if (enable && !e->prof_ev) {
        e->prof_ev = new hipEvent_t[2 * pk_engine::PROF_CAP];
        e->prof_kind = new int[pk_engine::PROF_CAP];
        for (int i = 0; i < 2 * pk_engine::PROF_CAP; ++i) PK_HIP(hipEventCreate(&e->prof_ev[i]));
    }
    PK_TRY(prof_flush(e));
    for (int k = 0; k < PK_PROF_N; ++k) { e->prof_ms[k] = 0.0; e->prof_cnt[k] = 0; }
    e->prof = enable != 0;
    return PK_OK;
}

extern "C" int pk_engine_profile_read(pk_engine *e, int kernel, double *total_ms, int64_t *launches) {
    PK_CHECK(e && kernel >= 0 && kernel < PK_PROF_N, PK_ERR_ARG, "bad argument");
    PK_TRY(prof_flush(e));
    if (total_ms) *total_ms = e->prof_ms[kernel];
    if (launches) *launches = e->prof_cnt[kernel];
    return PK_OK;
}

// One wave sleeping in bounded steps: s_sleep 127 is ~8k cycles (~3.4 us).
__global__ void k_stall(int iters) {
    for (int i = 0; i < iters; ++i) __builtin_amdgcn_s_sleep(127);
}

extern "C" int pk_engine_stall(pk_engine *e, int usec) {
    PK_CHECK(e && usec >= 0, PK_ERR_ARG, "bad argument");
    if (usec > 1000000) usec = 1000000;
    hipLaunchKernelGGL(k_stall, dim3(1), dim3(64), 0, e->stream, usec / 3 + 1);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── graphs ─────────────────────────
struct pk_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" int pk_capture_begin(pk_engine *e) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "already capturing");
    PK_HIP(hipStreamSynchronize(e->stream));
    PK_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    e->capturing = true;
    return PK_OK;
}

extern "C" int pk_capture_end(pk_engine *e, pk_graph **out) {
    PK_CHECK(e && out, PK_ERR_ARG, "null argument");
    PK_CHECK(e->capturing, PK_ERR_ARG, "not capturing");
    *out = nullptr;
    e->capturing = false;
    pk_graph *g = new pk_graph();
    hipError_t rc = hipStreamEndCapture(e->stream, &g->graph);
    if (rc == hipSuccess) rc = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (rc != hipSuccess) {
        pk_set_error("graph capture failed: %s", hipGetErrorString(rc));
        if (g->graph) (void)hipGraphDestroy(g->graph);
        delete g;
        return PK_ERR_HIP;
    }
    *out = g;
    return PK_OK;
}

extern "C" int pk_graph_launch(pk_engine *e, pk_graph *g) {
    PK_CHECK(e && g && g->exec, PK_ERR_ARG, "null argument");
    PK_HIP(hipGraphLaunch(g->exec, e->stream));
    return PK_OK;
}

extern "C" int pk_graph_destroy(pk_graph *g) {
    if (!g) return PK_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return PK_OK;
}

// ───────────────────────── expert store ─────────────────────────
static int check_i4_host(const pk_qt_host *t, int O, int I, int gs, const char *what) {
    PK_CHECK(t && t->data && t->s, PK_ERR_ARG, "%s: null tensor", what);
    PK_CHECK(t->fmt == PK_FMT_INT4, PK_ERR_UNSUPPORTED, "%s: fmt %d (store holds INT4)", what, t->fmt);
    PK_CHECK(t->O == O && t->I == I, PK_ERR_ARG, "%s: shape [%d,%d], expected [%d,%d]", what, t->O,
             t->I, O, I);
    PK_CHECK(t->block_size == gs, PK_ERR_UNSUPPORTED, "%s: block_size %d, expected %d", what,
             t->block_size, gs);
    return PK_OK;
}

// host ref layout -> staging -> tiles in the slot
static int upload_i4(pk_engine *e, const pk_qt_host *t, uint8_t *tiles, float *sc16) {
    const int64_t qbytes = (int64_t)t->O * ((t->I + 1) / 2);
    const int64_t sbytes = (int64_t)t->O * (t->I / PK_GS) * 4;
    PK_TRY(pk_stage_reserve(e, pk_align256(qbytes) + sbytes));
    uint8_t *dq = e->stage;
    float *ds = (float *)(e->stage + pk_align256(qbytes));
    PK_HIP(hipMemcpyAsync(dq, t->data, qbytes, hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipMemcpyAsync(ds, t->s, sbytes, hipMemcpyHostToDevice, e->stream));
    PK_TRY(pk_launch_i4_repack(dq, ds, t->O, t->I, tiles, sc16, e->stream));
    return PK_OK;
}

static uint8_t *slot_ptr(pk_engine *e, int layer, int eid) {
    return e->store + ((int64_t)layer * e->c.n_experts + eid) * e->ex.stride;
}

extern "C" int pk_store_expert(pk_engine *e, int layer, int eid, const pk_qt_host *gu,
                               const pk_qt_host *dn, const float *gu_bias, const float *d_bias) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    const pk_cfg *c = &e->c;
    PK_CHECK(layer >= 0 && layer < c->n_layers && eid >= 0 && eid < c->n_experts, PK_ERR_ARG,
             "expert (%d,%d) out of range", layer, eid);
    PK_CHECK(gu_bias && d_bias, PK_ERR_ARG, "expert biases are null");
    PK_TRY(check_i4_host(gu, c->moe_inter, c->hidden, c->group_size, "gate_up"));
    PK_TRY(check_i4_host(dn, c->hidden, c->moe_inter / 2, c->group_size, "down"));
    uint8_t *s = slot_ptr(e, layer, eid);
    PK_TRY(upload_i4(e, gu, s + e->ex.off_gu_tiles, (float *)(s + e->ex.off_gu_scales)));
    PK_TRY(upload_i4(e, dn, s + e->ex.off_dn_tiles, (float *)(s + e->ex.off_dn_scales)));
    PK_HIP(hipMemcpyAsync(s + e->ex.off_gu_bias, gu_bias, (size_t)c->moe_inter * 4,
                          hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipMemcpyAsync(s + e->ex.off_dn_bias, d_bias, (size_t)c->hidden * 4,
                          hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    e->expert_ready[(int64_t)layer * c->n_experts + eid] = 1;
    return PK_OK;
}

int pk_dense_tiles(pk_engine *e) {
    if (pk_tiles_current(e)) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "tile copies: not built while capturing");
    const pk_cfg *c = &e->c;
    const int D = c->hidden, A = c->n_heads * c->head_dim, Q = (c->n_heads + 2 * c->n_kv_heads) * c->head_dim;
    const int64_t ver = e->dense_ver;
    for (int l = 0; l < c->n_layers; ++l) {
        pk_layer_dev &d = e->L[l];
        if (!d.have_attn) continue;
        if (!d.wqkv_t) ALLOC(d.wqkv_t, pk_skinny_tile_floats(Q, D) * 4);
        if (!d.wo_t) ALLOC(d.wo_t, pk_skinny_tile_floats(D, A) * 4);
        PK_TRY(pk_launch_tile_skinny(d.wqkv, Q, D, d.wqkv_t, e->stream));
        PK_TRY(pk_launch_tile_skinny(d.wo, D, A, d.wo_t, e->stream));
    }
    if (e->lm_f32) {
        if (!e->lm_t) ALLOC(e->lm_t, pk_skinny_tile_floats(c->vocab, D) * 4);
        PK_TRY(pk_launch_tile_skinny(e->lm_f32, c->vocab, D, e->lm_t, e->stream));
    }
    e->tiles_ver = ver;
    return PK_OK;
}

static int upload_f32(pk_engine *e, float **dst, const float *src, int64_t n) {
    if (!*dst) ALLOC(*dst, n * 4);
    PK_HIP(hipMemcpyAsync(*dst, src, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
    return PK_OK;
}

extern "C" int pk_store_layer(pk_engine *e, int layer, const pk_layer_host *l) {
    PK_CHECK(e && l, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    PK_CHECK(layer >= 0 && layer < c->n_layers, PK_ERR_ARG, "layer %d out of range", layer);
    const int D = c->hidden, H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim, E = c->n_experts;
    pk_layer_dev &d = e->L[layer];
    if (l->in_ln) PK_TRY(upload_f32(e, &d.in_ln, l->in_ln, D));
    if (l->post_ln) PK_TRY(upload_f32(e, &d.post_ln, l->post_ln, D));
    if (l->router) {
        PK_CHECK(l->router_bias, PK_ERR_ARG, "router bias is null");
        PK_TRY(upload_f32(e, &d.router, l->router, (int64_t)E * D));
        PK_TRY(upload_f32(e, &d.router_b, l->router_bias, E));
        d.have_router = true;
    }
    if (l->wq.data) {
        const pk_qt_host *ws[3] = {&l->wq, &l->wk, &l->wv};
        const int rows[3] = {H * hd, KVH * hd, KVH * hd};
        const float *bs[3] = {l->bq, l->bk, l->bv};
        for (int i = 0; i < 3; ++i) {
            PK_CHECK(ws[i]->fmt == PK_FMT_F32 && ws[i]->O == rows[i] && ws[i]->I == D && ws[i]->data,
                     PK_ERR_UNSUPPORTED, "attention projection %d: need F32 [%d,%d]", i, rows[i], D);
            PK_CHECK(bs[i], PK_ERR_ARG, "attention bias %d is null", i);
        }
        PK_CHECK(l->wo.fmt == PK_FMT_F32 && l->wo.O == D && l->wo.I == H * hd && l->wo.data && l->bo,
                 PK_ERR_UNSUPPORTED, "wo: need F32 [%d,%d] and bias", D, H * hd);
        PK_CHECK(l->sinks && l->in_ln && l->post_ln, PK_ERR_ARG, "sinks / norms are null");
        const int64_t nq = (int64_t)H * hd * D, nk = (int64_t)KVH * hd * D;
        if (!d.wqkv) ALLOC(d.wqkv, (nq + 2 * nk) * 4);
        if (!d.bqkv) ALLOC(d.bqkv, (int64_t)(H + 2 * KVH) * hd * 4);
        PK_HIP(hipMemcpyAsync(d.wqkv, l->wq.data, nq * 4, hipMemcpyHostToDevice, e->stream));
        PK_HIP(hipMemcpyAsync(d.wqkv + nq, l->wk.data, nk * 4, hipMemcpyHostToDevice, e->stream));
        PK_HIP(hipMemcpyAsync(d.wqkv + nq + nk, l->wv.data, nk * 4, hipMemcpyHostToDevice, e->stream));
        PK_HIP(hipMemcpyAsync(d.bqkv, l->bq, (size_t)H * hd * 4, hipMemcpyHostToDevice, e->stream));
        PK_HIP(hipMemcpyAsync(d.bqkv + H * hd, l->bk, (size_t)KVH * hd * 4, hipMemcpyHostToDevice, e->stream));
        PK_HIP(hipMemcpyAsync(d.bqkv + (H + KVH) * hd, l->bv, (size_t)KVH * hd * 4, hipMemcpyHostToDevice,
                              e->stream));
        PK_TRY(upload_f32(e, &d.wo, (const float *)l->wo.data, (int64_t)D * H * hd));
        PK_TRY(upload_f32(e, &d.bo, l->bo, D));
        PK_TRY(upload_f32(e, &d.sinks, l->sinks, H));
        d.have_attn = true;
        ++e->dense_ver;
    }
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

extern "C" int pk_store_globals(pk_engine *e, const pk_qt_host *embed, const pk_qt_host *lm_head,
                                const float *final_norm) {
    PK_CHECK(e && embed && lm_head && final_norm, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    const int D = c->hidden;
    PK_CHECK(embed->fmt == PK_FMT_F32 && embed->O == c->vocab && embed->I == D && embed->data,
             PK_ERR_UNSUPPORTED, "embedding: need F32 [%d,%d]", c->vocab, D);
    PK_CHECK(lm_head->fmt == c->lm_head_fmt && lm_head->O == c->vocab && lm_head->I == D &&
                 lm_head->data, PK_ERR_UNSUPPORTED, "lm_head: need fmt %d [%d,%d]", c->lm_head_fmt,
             c->vocab, D);
    PK_TRY(upload_f32(e, &e->embed, (const float *)embed->data, (int64_t)c->vocab * D));
    if (c->lm_head_fmt == PK_FMT_F32) {
        PK_TRY(upload_f32(e, &e->lm_f32, (const float *)lm_head->data, (int64_t)c->vocab * D));
        ++e->dense_ver;
    } else {
        PK_CHECK(lm_head->s, PK_ERR_ARG, "lm_head scales are null");
        if (!e->lm_q8) ALLOC(e->lm_q8, (int64_t)c->vocab * D);
        PK_HIP(hipMemcpyAsync(e->lm_q8, lm_head->data, (size_t)c->vocab * D, hipMemcpyHostToDevice, e->stream));
        PK_TRY(upload_f32(e, &e->lm_s, lm_head->s, c->vocab));
    }
    PK_TRY(upload_f32(e, &e->final_norm, final_norm, D));
    PK_HIP(hipStreamSynchronize(e->stream));
    e->have_globals = true;
    return PK_OK;
}

// ───────────────────────── synthetic build ─────────────────────────
static int synth_fill(pk_engine *e, float *dst, int64_t n, uint64_t seed, uint32_t kind,
                      uint32_t layer, uint32_t idx, float std) {
    return pk_launch_fill_normal(dst, n, pk_stream(seed, kind, layer, idx), std, e->stream);
}

static int synth_expert_matrix(pk_engine *e, int O, int I, uint64_t seed, uint32_t kind, int layer,
                               int eid, uint8_t *tiles, float *sc16) {
    const int64_t n = (int64_t)O * I;
    const int64_t qbytes = (int64_t)O * (I / 2), sbytes = (int64_t)O * (I / PK_GS) * 4;
    const int64_t need = pk_align256(n * 4) + pk_align256(qbytes) + sbytes;
    PK_TRY(pk_stage_reserve(e, need));
    float *w = (float *)e->stage;
    uint8_t *q = e->stage + pk_align256(n * 4);
    float *s = (float *)(q + pk_align256(qbytes));
    PK_TRY(synth_fill(e, w, n, seed, kind, layer, eid, 0.02f));
    PK_TRY(pk_launch_quantize_i4(w, O, I, PK_GS, q, s, e->stream));
    PK_TRY(pk_launch_i4_repack(q, s, O, I, tiles, sc16, e->stream));
    return PK_OK;
}

extern "C" int pk_engine_build_synthetic(pk_engine *e, uint64_t seed, int what, int n_threads) {
    (void)n_threads;
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    const pk_cfg *c = &e->c;
    const int D = c->hidden, E = c->n_experts, H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim;
    const int inter = c->moe_inter, half = inter / 2;
    for (int l = 0; l < c->n_layers; ++l) {
        pk_layer_dev &d = e->L[l];
        if (!d.in_ln) { ALLOC(d.in_ln, D * 4); PK_TRY(pk_launch_fill_const(d.in_ln, D, 1.0f, e->stream)); }
        if (!d.post_ln) { ALLOC(d.post_ln, D * 4); PK_TRY(pk_launch_fill_const(d.post_ln, D, 1.0f, e->stream)); }
        if (what & 1) {
            if (!d.router) ALLOC(d.router, (int64_t)E * D * 4);
            if (!d.router_b) ALLOC(d.router_b, E * 4);
            PK_TRY(synth_fill(e, d.router, (int64_t)E * D, seed, PK_T_ROUTER, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.router_b, E, seed, PK_T_ROUTER_B, l, 0, 0.02f));
            d.have_router = true;
                for (int x = 0; x < E; ++x) {
                uint8_t *s = slot_ptr(e, l, x);
                PK_TRY(synth_expert_matrix(e, inter, D, seed, PK_T_GU, l, x, s + e->ex.off_gu_tiles,
                                           (float *)(s + e->ex.off_gu_scales)));
                PK_TRY(synth_expert_matrix(e, D, half, seed, PK_T_DOWN, l, x, s + e->ex.off_dn_tiles,
                                           (float *)(s + e->ex.off_dn_scales)));
                PK_TRY(synth_fill(e, (float *)(s + e->ex.off_gu_bias), inter, seed, PK_T_GU_B, l, x, 0.02f));
                PK_TRY(synth_fill(e, (float *)(s + e->ex.off_dn_bias), D, seed, PK_T_DOWN_B, l, x, 0.02f));
                e->expert_ready[(int64_t)l * E + x] = 1;
            }
        }
        if (what & 2) {
            const int64_t nq = (int64_t)H * hd * D, nk = (int64_t)KVH * hd * D;
            if (!d.wqkv) ALLOC(d.wqkv, (nq + 2 * nk) * 4);
            if (!d.bqkv) ALLOC(d.bqkv, (int64_t)(H + 2 * KVH) * hd * 4);
            if (!d.wo) ALLOC(d.wo, (int64_t)D * H * hd * 4);
            if (!d.bo) ALLOC(d.bo, D * 4);
            if (!d.sinks) ALLOC(d.sinks, H * 4);
            PK_TRY(synth_fill(e, d.wqkv, nq, seed, PK_T_WQ, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.wqkv + nq, nk, seed, PK_T_WK, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.wqkv + nq + nk, nk, seed, PK_T_WV, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.bqkv, H * hd, seed, PK_T_BQ, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.bqkv + H * hd, KVH * hd, seed, PK_T_BK, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.bqkv + (H + KVH) * hd, KVH * hd, seed, PK_T_BV, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.wo, (int64_t)D * H * hd, seed, PK_T_WO, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.bo, D, seed, PK_T_BO, l, 0, 0.02f));
            PK_TRY(synth_fill(e, d.sinks, H, seed, PK_T_SINKS, l, 0, 0.02f));
            d.have_attn = true;
            ++e->dense_ver;
        }
    }
    if (what & 4) {
        const int64_t n = (int64_t)c->vocab * D;
        if (!e->embed) ALLOC(e->embed, n * 4);
        PK_TRY(synth_fill(e, e->embed, n, seed, PK_T_EMBED, 0, 0, 0.02f));
        if (c->lm_head_fmt == PK_FMT_F32) {
            if (!e->lm_f32) ALLOC(e->lm_f32, n * 4);
            PK_TRY(synth_fill(e, e->lm_f32, n, seed, PK_T_LM_HEAD, 0, 0, 0.02f));
            ++e->dense_ver;
        } else {
            pk_set_error("synthetic INT8 lm_head is built by the host loader");
            return PK_ERR_UNSUPPORTED;
        }
        if (!e->final_norm) ALLOC(e->final_norm, D * 4);
        PK_TRY(pk_launch_fill_const(e->final_norm, D, 1.0f, e->stream));
        e->have_globals = true;
    }
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

// ───────────────────────── quantizer ─────────────────────────
extern "C" int pk_quantize_int4_gs(pk_engine *e, const float *w_dev, int O, int I, int gs,
                                   uint8_t *packed_dev, float *scales_dev) {
    PK_CHECK(e && w_dev && packed_dev && scales_dev, PK_ERR_ARG, "null argument");
    PK_TRY(pk_launch_quantize_i4(w_dev, O, I, gs, packed_dev, scales_dev, e->stream));
    return PK_OK;
}

// ───────────────────────── tensors / matmul_qt ─────────────────────────
extern "C" int pk_qt_upload(pk_engine *e, const pk_qt_host *h, pk_qt **out) {
    PK_CHECK(e && h && out && h->data, PK_ERR_ARG, "null argument");
    PK_CHECK(h->O > 0 && h->I > 0, PK_ERR_ARG, "tensor shape [%d,%d]", h->O, h->I);
    *out = nullptr;
    pk_qt *t = new pk_qt();
    t->fmt = h->fmt; t->O = h->O; t->I = h->I; t->gs = h->block_size; t->tiled = 0;
    int rc = PK_OK;
    const int64_t n = (int64_t)h->O * h->I;
    if (h->fmt == PK_FMT_F32) {
        rc = pk_dev_alloc(e, &t->data, n * 4);
        if (rc == PK_OK) rc = hipMemcpy(t->data, h->data, n * 4, hipMemcpyHostToDevice) == hipSuccess ? PK_OK : PK_ERR_HIP;
    } else if (h->fmt == PK_FMT_INT8) {
        rc = h->s ? pk_dev_alloc(e, &t->data, n) : PK_ERR_ARG;
        if (rc == PK_OK) rc = pk_dev_alloc(e, (void **)&t->s, (int64_t)h->O * 4);
        if (rc == PK_OK) rc = hipMemcpy(t->data, h->data, n, hipMemcpyHostToDevice) == hipSuccess ? PK_OK : PK_ERR_HIP;
        if (rc == PK_OK) rc = hipMemcpy(t->s, h->s, (size_t)h->O * 4, hipMemcpyHostToDevice) == hipSuccess ? PK_OK : PK_ERR_HIP;
    } else if (h->fmt == PK_FMT_INT4) {
        const int64_t qb = (int64_t)h->O * ((h->I + 1) / 2);
        const int gs = h->block_size;
        const int64_t nsc = gs > 0 ? (int64_t)h->O * ((h->I + gs - 1) / gs) : h->O;
        if (!h->s) rc = PK_ERR_ARG;
        else if (gs == PK_GS && h->I % PK_GS == 0) {
            t->tiled = 1;
            t->sh = pk_i4_make_shape(h->O, h->I);
            rc = pk_dev_alloc(e, &t->data, t->sh.tile_bytes);
            if (rc == PK_OK) rc = pk_dev_alloc(e, (void **)&t->s, t->sh.scale_bytes);
            if (rc == PK_OK) {
                pk_qt_host hh = *h;
                rc = upload_i4(e, &hh, (uint8_t *)t->data, t->s);
                if (rc == PK_OK) rc = hipStreamSynchronize(e->stream) == hipSuccess ? PK_OK : PK_ERR_HIP;
            }
        } else {
            rc = pk_dev_alloc(e, &t->data, qb);
            if (rc == PK_OK) rc = pk_dev_alloc(e, (void **)&t->s, nsc * 4);
            if (rc == PK_OK) rc = hipMemcpy(t->data, h->data, qb, hipMemcpyHostToDevice) == hipSuccess ? PK_OK : PK_ERR_HIP;
            if (rc == PK_OK) rc = hipMemcpy(t->s, h->s, nsc * 4, hipMemcpyHostToDevice) == hipSuccess ? PK_OK : PK_ERR_HIP;
        }
    } else {
        rc = PK_ERR_UNSUPPORTED;
    }
    if (rc != PK_OK) {
        if (rc == PK_ERR_UNSUPPORTED) pk_set_error("matmul_qt: format %d not supported", h->fmt);
        else if (rc == PK_ERR_ARG) pk_set_error("tensor: scales are null");
        else if (rc == PK_ERR_HIP) pk_set_error("tensor upload failed");
        pk_dev_free(e, t->data);
        pk_dev_free(e, t->s);
        delete t;
        return rc;
    }
    *out = t;
    return PK_OK;
}

extern "C" int pk_qt_free(pk_engine *e, pk_qt *t) {
    if (!t) return PK_OK;
    if (e) (void)hipStreamSynchronize(e->stream);
    pk_dev_free(e, t->data);
    pk_dev_free(e, t->s);
    delete t;
    return PK_OK;
}

extern "C" int pk_matmul_qt(pk_engine *e, float *y, const float *x, const pk_qt *w, int S) {
    PK_CHECK(e && y && x && w, PK_ERR_ARG, "null argument");
    PK_CHECK(S > 0, PK_ERR_ARG, "S=%d", S);
    switch (w->fmt) {
    case PK_FMT_F32:    // quant.h:117-148's chains and tree: the reference's bits
        return pk_launch_gemm_chain8(x, w->I, (const float *)w->data, nullptr, y, w->O, S, w->I, w->O, false,
                                     e->stream);
    case PK_FMT_INT8:   // quant.h:152-186, likewise
        return pk_launch_gemm_chain8_q8(x, (const int8_t *)w->data, w->s, y, S, w->I, w->O, e->stream);
    case PK_FMT_INT4:
        if (w->gs <= 0)
            return pk_launch_i4_rowscale_gemv(y, x, (const uint8_t *)w->data, w->s, S, w->I, w->O, e->stream);
        if (w->tiled) {
            pk_i4_items it{};
            it.base = (const uint8_t *)w->data;
            it.slot_stride = 0;
            it.off_tiles = 0;
            it.off_scales = (const uint8_t *)w->s - (const uint8_t *)w->data;
            it.off_bias = -1;
            it.slots = nullptr;
            it.x = x; it.x_stride = w->I;
            it.y = y; it.y_stride = w->O;
            it.n_items = S;
            return pk_launch_i4_gemv(it, w->sh, PK_EPI_PLAIN, 0.f, 0.f, nullptr, e->stream);
        }
        return pk_launch_i4_gemv_ref(y, x, (const uint8_t *)w->data, w->s, S, w->I, w->O, w->gs, e->stream);
    default:
        pk_set_error("matmul_qt: format %d not supported", w->fmt);
        return PK_ERR_UNSUPPORTED;
    }
}

// ───────────────────────── expert path ─────────────────────────
pk_i4_items pk_expert_items(pk_engine *e, int layer, bool down) {
    pk_i4_items it{};
    it.base = e->store;
    it.slot_stride = e->ex.stride;
    it.off_tiles = down ? e->ex.off_dn_tiles : e->ex.off_gu_tiles;
    it.off_scales = down ? e->ex.off_dn_scales : e->ex.off_gu_scales;
    it.off_bias = down ? e->ex.off_dn_bias : e->ex.off_gu_bias;
    it.slot_base = layer * e->c.n_experts;
    return it;
}

int pk_check_layer_experts(pk_engine *e, int layer) {
    const pk_cfg *c = &e->c;
    PK_CHECK(layer >= 0 && layer < c->n_layers, PK_ERR_ARG, "layer %d out of range", layer);
    PK_CHECK(e->L[layer].have_router, PK_ERR_MISSING, "layer %d: router not loaded", layer);
    for (int x = 0; x < c->n_experts; ++x)
        PK_CHECK(e->expert_ready[(int64_t)layer * c->n_experts + x], PK_ERR_MISSING,
                 "layer %d expert %d not loaded", layer, x);
    return PK_OK;
}

// FFN of the experts listed in sel (device, n entries): act <- SwiGLU(gate_up x + b),
// eo <- down act + b; with comb, the down launch also combines the n outputs
// (weights comb->w) into comb->out (+ residual).
// With route, the gate_up launch selects the experts from the router logits
// and writes sel_dev (and the routing weights) for the down launch.
// dot: the integer-dot arithmetic, inputs from e->hn_q (one row shared by
// the items), the SwiGLU outputs' records through e->act_q.
static int experts_ffn(pk_engine *e, int layer, const int32_t *sel_dev, int n, const float *x,
                       int64_t x_stride, float *act, float *eo, const pk_combine_args *comb,
                       const pk_route_args *route = nullptr, bool dot = false) {
    const pk_cfg *c = &e->c;
    pk_i4_items gu = pk_expert_items(e, layer, false);
    gu.slots = route ? nullptr : sel_dev;
    gu.x = x; gu.x_stride = x_stride;
    gu.y = act; gu.y_stride = c->moe_inter / 2;
    gu.n_items = n;
    if (dot) {
        gu.xq = e->hn_q;
        gu.xq_stride = 0;
        gu.yq = e->act_q;
        gu.yq_stride = (int64_t)e->ex.gu.RB * PK_XQ_INTS;
    }
    int ps = pk_prof_begin(e, PK_PROF_EXPERT_GATE_UP);
    PK_TRY(pk_launch_i4_gemv(gu, e->ex.gu, PK_EPI_SWIGLU, c->swiglu_limit, c->swiglu_alpha,
                             nullptr, e->stream, route));
    PK_TRY(pk_prof_end(e, ps));
    pk_i4_items dn = pk_expert_items(e, layer, true);
    dn.slots = sel_dev;
    dn.x = act; dn.x_stride = c->moe_inter / 2;
    dn.y = eo; dn.y_stride = c->hidden;
    dn.n_items = n;
    if (dot) {
        dn.xq = e->act_q;
        dn.xq_stride = (int64_t)e->ex.gu.RB * PK_XQ_INTS;
    }
    ps = pk_prof_begin(e, PK_PROF_EXPERT_DOWN);
    PK_TRY(pk_launch_i4_gemv(dn, e->ex.dn, comb ? PK_EPI_COMBINE : PK_EPI_PLAIN, 0.f, 0.f, comb,
                             e->stream));
    PK_TRY(pk_prof_end(e, ps));
    return PK_OK;
}

// Shapes and devices k_moe_ffn takes (pk_launch_moe_ffn checks the same):
// its waiting down tasks must leave a free workgroup slot on this device.
static bool moe_ffn_fits(const pk_engine *e, bool dot) {
    const pk_cfg *c = &e->c;
    return e->ex.gu.NG <= 45 && e->ex.dn.NG <= 45 && e->ex.gu.O == e->ex.gu.RB * 64 &&
           e->ex.dn.NG * 64 == e->ex.gu.O / 2 && c->topk <= 4 && e->ex.dn.RB <= e->ex.gu.RB &&
           e->ex.stride < ((int64_t)1 << 31) &&   // 32-bit offsets in a slot
           pk_moe_ffn_supported(e->ex.gu.RB, e->ex.dn.RB, c->topk, e->n_cu, dot);
}

// norm_w: x_dev is the raw residual row; the router normalises it (rmsnorm
// fused) and writes the normalised row to e->hn, which the experts read.
// The MoE layer's router launch (logits into `logits`; with norm_w the
// normalised row into e->hn; with the integer dot the input's records).
static int moe_router(pk_engine *e, int layer, const float *x_dev, const float *norm_w, bool dot,
                      float *logits) {
    const pk_cfg *c = &e->c;
    const pk_layer_dev &d = e->L[layer];
    return pk_launch_router_topk(x_dev, d.router, d.router_b, c->n_experts, c->hidden, c->topk,
                                 c->routed_scale, logits, e->sel, e->w_scaled, e->w_soft, nullptr, e->stream,
                                 norm_w, c->eps, norm_w ? e->hn : nullptr, dot ? e->hn_q : nullptr,
                                 e->counters + PK_CTR_MOE_EPOCH);
}

int pk_moe_layer(pk_engine *e, int layer, const float *x_dev, float *out_dev,
                 const float *residual, float *res_out, const float *norm_w) {
    const pk_cfg *c = &e->c;
    // the router launch writes the logits only; the expert launch selects
    // the experts from them and publishes the routing (sel, weights)
    int ps = pk_prof_begin(e, PK_PROF_ROUTER);
    // integer-dot arithmetic: the router also writes the input's records, the
    // gate_up epilogue those of its SwiGLU outputs for the down launch
    const bool dot = e->i4_dot && c->hidden % 64 == 0 && c->moe_inter % 128 == 0;
    PK_TRY(moe_router(e, layer, x_dev, norm_w, dot, e->r_logits));
    PK_TRY(pk_prof_end(e, ps));
    PK_TRY(pk_trace_router(e, e->r_logits, 1));
    PK_TRY(pk_trace_route(e, layer, e->r_logits));
    pk_route_args rt{};
    rt.logits = e->r_logits;
    rt.E = c->n_experts;
    rt.K = c->topk;
    rt.routed_scale = c->routed_scale;
    rt.sel = e->sel;
    rt.w_scaled = e->w_scaled;
    rt.w_soft = e->w_soft;
    // the down launch combines the top-k outputs (routing order) + residual
    pk_combine_args cb{};
    cb.w = e->w_scaled;
    cb.out = residual ? res_out : out_dev;
    cb.residual = residual;
    cb.counters = e->counters + PK_CTR_COMBINE;
    const float *xin = norm_w ? e->hn : x_dev;
    if (e->moe_fused && moe_ffn_fits(e, dot)) {
        pk_moe_ffn_args a{};
        a.store = e->store;
        a.slot_stride = e->ex.stride;
        a.slot_base = layer * c->n_experts;
        a.gu_tiles = (uint32_t)e->ex.off_gu_tiles;
        a.gu_scales = (uint32_t)e->ex.off_gu_scales;
        a.dn_tiles = (uint32_t)e->ex.off_dn_tiles;
        a.dn_scales = (uint32_t)e->ex.off_dn_scales;
        a.gu_bias = (int32_t)e->ex.off_gu_bias;
        a.dn_bias = (int32_t)e->ex.off_dn_bias;
        a.gu_NG = e->ex.gu.NG; a.gu_O = e->ex.gu.O; a.gu_RB = e->ex.gu.RB;
        a.dn_NG = e->ex.dn.NG; a.dn_O = e->ex.dn.O; a.dn_RB = e->ex.dn.RB;
        a.K = c->topk;
        a.n_cu = e->n_cu;
        a.dot = dot;
        a.lim = c->swiglu_limit;
        a.alpha = c->swiglu_alpha;
        a.x = xin;
        a.xq = dot ? e->hn_q : nullptr;
        a.out = cb.out;
        a.residual = cb.residual;
        a.rt = rt;
        a.act_t = e->moe_act_t;
        a.eo_t = e->moe_eo_t;
        a.cont_t = e->moe_cont_t;
        a.epoch = e->counters + PK_CTR_MOE_EPOCH;
        a.status = e->counters + PK_CTR_MOE_STATUS;
        ps = pk_prof_begin(e, PK_PROF_MOE_FFN);
        if (e->moe_fused == 2 && pk_moe_bal_fits_cu(dot) && pk_moe_bal_supported(a, e->n_cu))
            PK_TRY(pk_launch_moe_bal(a, e->stream));
        else
            PK_TRY(pk_launch_moe_ffn(a, e->stream));
        return pk_prof_end(e, ps);
    }
    PK_TRY(experts_ffn(e, layer, e->sel, c->topk, xin, 0, e->act, e->eo, &cb, &rt, dot));
    return PK_OK;
}

extern "C" int pk_set_i4_dot(pk_engine *e, int on) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_i4_dot: not available while capturing");
    if (e->i4_dot != (on != 0) && e->step_exec) {      // the captured step holds the other kernels
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    e->i4_dot = on != 0;
    return PK_OK;
}

extern "C" int pk_set_grouped_f16(pk_engine *e, int on) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_grouped_f16: not available while capturing");
    e->grouped_f16 = on != 0;
    return PK_OK;
}

extern "C" int pk_set_moe_fused(pk_engine *e, int mode) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(mode >= 0 && mode <= 2, PK_ERR_ARG, "set_moe_fused: mode %d (0, 1 or 2)", mode);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_moe_fused: not available while capturing");
    if (e->moe_fused != mode && e->step_exec) {   // the captured step holds the other kernels
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    e->moe_fused = mode;
    return PK_OK;
}

extern "C" int pk_set_attn_fused(pk_engine *e, int on) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_attn_fused: not available while capturing");
    if (e->attn_fused != (on != 0) && e->step_exec) {   // the captured step holds the other kernels
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    e->attn_fused = on != 0;
    return PK_OK;
}

extern "C" int pk_router_logits(pk_engine *e, int layer, const float *x_dev, float *logits_dev) {
    PK_CHECK(e && x_dev && logits_dev, PK_ERR_ARG, "null argument");
    PK_CHECK(layer >= 0 && layer < e->c.n_layers && e->L[layer].have_router, PK_ERR_MISSING,
             "layer %d: router not loaded", layer);
    const pk_cfg *c = &e->c;
    const bool dot = e->i4_dot && c->hidden % 64 == 0 && c->moe_inter % 128 == 0;
    return moe_router(e, layer, x_dev, nullptr, dot, logits_dev);
}

extern "C" int pk_moe_forward(pk_engine *e, int layer, const float *x_dev, float *out_dev,
                              int32_t *sel_host, float *w_host) {
    PK_CHECK(e && x_dev && out_dev, PK_ERR_ARG, "null argument");
    PK_TRY(pk_check_layer_experts(e, layer));
    PK_CHECK(!(e->capturing && (sel_host || w_host)), PK_ERR_ARG,
             "moe_forward: host routing outputs are not available while capturing a graph");
    PK_TRY(pk_moe_layer(e, layer, x_dev, out_dev, nullptr, nullptr));
    if (sel_host || w_host) {
        if (sel_host)
            PK_HIP(hipMemcpyAsync(sel_host, e->sel, e->c.topk * 4, hipMemcpyDeviceToHost, e->stream));
        if (w_host)
            PK_HIP(hipMemcpyAsync(w_host, e->w_soft, e->c.topk * 4, hipMemcpyDeviceToHost, e->stream));
        PK_HIP(hipStreamSynchronize(e->stream));
        bool redo = false;
        PK_TRY(pk_wait_fallback(e, &redo));
        if (redo) {
            // the input is intact unless the layer ran in place
            PK_CHECK(x_dev != out_dev, PK_ERR_HIP,
                     "a device-side wait gave up in an in-place moe_forward: the output is invalid (the engine now "
                     "runs the separate launches)");
            return pk_moe_forward(e, layer, x_dev, out_dev, sel_host, w_host);
        }
    }
    return PK_OK;
}

extern "C" int pk_expert_apply(pk_engine *e, int layer, int eid, const float *x_dev, float *dst_dev,
                               float w) {
    PK_CHECK(e && x_dev && dst_dev, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    PK_CHECK(layer >= 0 && layer < c->n_layers && eid >= 0 && eid < c->n_experts, PK_ERR_ARG,
             "expert (%d,%d) out of range", layer, eid);
    PK_CHECK(e->expert_ready[(int64_t)layer * c->n_experts + eid], PK_ERR_MISSING,
             "layer %d expert %d not loaded", layer, eid);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "expert_apply: not available while capturing a graph");
    // a one-entry slot list in device scratch (sel[0] is free outside moe_forward)
    PK_HIP(hipMemcpyAsync(e->sel, &eid, 4, hipMemcpyHostToDevice, e->stream));
    PK_TRY(experts_ffn(e, layer, e->sel, 1, x_dev, 0, e->act, e->eo, nullptr));
    PK_TRY(pk_launch_axpy(dst_dev, e->eo, w, c->hidden, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

static int check_expert_batch(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                              const void *in, const void *out) {
    const pk_cfg *c = &e->c;
    PK_CHECK(eids_dev && in && out, PK_ERR_ARG, "null argument");
    PK_CHECK(n > 0 && n <= c->n_experts, PK_ERR_ARG, "%d experts per launch (1..%d)", n, c->n_experts);
    PK_TRY(pk_check_layer_experts(e, layer));
    return PK_OK;
}

extern "C" int pk_expert_gate_up(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                                 const float *x_dev, float *act_dev) {
    PK_CHECK(e, PK_ERR_ARG, "null engine");
    PK_TRY(check_expert_batch(e, layer, eids_dev, n, x_dev, act_dev));
    const pk_cfg *c = &e->c;
    pk_i4_items gu = pk_expert_items(e, layer, false);
    gu.slots = eids_dev;
    gu.x = x_dev; gu.x_stride = 0;
    gu.y = act_dev; gu.y_stride = c->moe_inter / 2;
    gu.n_items = n;
    int ps = pk_prof_begin(e, PK_PROF_EXPERT_GATE_UP);
    PK_TRY(pk_launch_i4_gemv(gu, e->ex.gu, PK_EPI_SWIGLU, c->swiglu_limit, c->swiglu_alpha,
                             nullptr, e->stream));
    return pk_prof_end(e, ps);
}

extern "C" int pk_act_records(pk_engine *e, const float *x_dev, int n, int32_t *rec_dev) {
    PK_CHECK(e && x_dev && rec_dev, PK_ERR_ARG, "null argument");
    return pk_launch_act_records(x_dev, n, rec_dev, e->stream);
}

extern "C" int pk_expert_gate_up_dot(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                                     const int32_t *rec_dev, float *act_dev, int32_t *act_rec_dev) {
    PK_CHECK(e && rec_dev, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    PK_CHECK(c->hidden % 64 == 0 && c->moe_inter % 128 == 0, PK_ERR_UNSUPPORTED,
             "integer-dot experts need hidden %% 64 == 0 and moe_inter %% 128 == 0");
    PK_TRY(check_expert_batch(e, layer, eids_dev, n, rec_dev, act_dev));
    pk_i4_items gu = pk_expert_items(e, layer, false);
    gu.slots = eids_dev;
    gu.x = nullptr; gu.x_stride = 0;
    gu.xq = rec_dev; gu.xq_stride = 0;
    gu.y = act_dev; gu.y_stride = c->moe_inter / 2;
    gu.yq = act_rec_dev; gu.yq_stride = (int64_t)e->ex.gu.RB * PK_XQ_INTS;
    gu.n_items = n;
    return pk_launch_i4_gemv(gu, e->ex.gu, PK_EPI_SWIGLU, c->swiglu_limit, c->swiglu_alpha, nullptr, e->stream);
}

extern "C" int pk_expert_down_dot(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                                  const int32_t *act_rec_dev, float *eo_dev) {
    PK_CHECK(e && act_rec_dev, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    PK_CHECK(c->hidden % 64 == 0 && c->moe_inter % 128 == 0, PK_ERR_UNSUPPORTED,
             "integer-dot experts need hidden %% 64 == 0 and moe_inter %% 128 == 0");
    PK_TRY(check_expert_batch(e, layer, eids_dev, n, act_rec_dev, eo_dev));
    pk_i4_items dn = pk_expert_items(e, layer, true);
    dn.slots = eids_dev;
    dn.x = nullptr; dn.x_stride = 0;
    dn.xq = act_rec_dev; dn.xq_stride = (int64_t)e->ex.gu.RB * PK_XQ_INTS;
    dn.y = eo_dev; dn.y_stride = c->hidden;
    dn.n_items = n;
    return pk_launch_i4_gemv(dn, e->ex.dn, PK_EPI_PLAIN, 0.f, 0.f, nullptr, e->stream);
}

extern "C" int pk_expert_down(pk_engine *e, int layer, const int32_t *eids_dev, int n,
                              const float *act_dev, float *eo_dev) {
    PK_CHECK(e, PK_ERR_ARG, "null engine");
    PK_TRY(check_expert_batch(e, layer, eids_dev, n, act_dev, eo_dev));
    const pk_cfg *c = &e->c;
    pk_i4_items dn = pk_expert_items(e, layer, true);
    dn.slots = eids_dev;
    dn.x = act_dev; dn.x_stride = c->moe_inter / 2;
    dn.y = eo_dev; dn.y_stride = c->hidden;
    dn.n_items = n;
    int ps = pk_prof_begin(e, PK_PROF_EXPERT_DOWN);
    PK_TRY(pk_launch_i4_gemv(dn, e->ex.dn, PK_EPI_PLAIN, 0.f, 0.f, nullptr, e->stream));
    return pk_prof_end(e, ps);
}

