/* ref_harness.c — exposes picchio's own C functions for golden vectors.
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile into oracle/_ref/ from
 * the reference sources where they lie (/root/reference/picchio.c and the
 * headers it includes); nothing from the reference is copied into this tree.
 * picchio.c is compiled as part of this translation unit (its `main` renamed)
 * so its static functions — matmul_qt kernels, moe_forward, gqa_attention,
 * forward_token, prefill_tokens — can be called on a Model whose tensors point
 * at a po_model built by the oracle from the same seed. All experts are
 * preloaded into the LRU pool with ecap = n_experts, as self_test does
 * (picchio.c:2188-2214), so no disk path runs.
 */
#define main picchio_reference_main
#include "picchio.c"
#undef main

#include "pk_oracle.h"
#include "../picchio_amd/csrc/pk_synth.h"

static Model g_ref;
static int g_ref_ready = 0;

/* ── quant.h kernels, called directly ── */
void ref_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O) {
    matmul_f32(y, x, W, S, I, O);
}
void ref_matmul_q8(float *y, const float *x, const int8_t *q, const float *s,
                   int S, int I, int O) {
    matmul_q8(y, x, q, s, S, I, O);
}
void ref_matmul_i4(float *y, const float *x, const uint8_t *q4, const float *s,
                   int S, int I, int O) {
    matmul_i4(y, x, q4, s, S, I, O);
}
void ref_matmul_i4_gs(float *y, const float *x, const uint8_t *q4, const float *s,
                      int S, int I, int O, int gs) {
    matmul_i4_gs(y, x, q4, s, S, I, O, gs);
}
void ref_quantize_rows_i4(const float *w, uint8_t *q4, float *s, int O, int I) {
    quantize_rows_i4(w, q4, s, O, I);
}
void ref_rmsnorm(float *o, const float *x, const float *w, int D, float eps) {
    rmsnorm(o, x, w, D, eps);
}
void ref_softmax(float *x, int n) { softmax(x, n); }

/* sample_logits (picchio.c:1509-1649) with its globals set from the
 * arguments: the token, the logits as it leaves them, and in *rng the state
 * after the draw. */
int ref_sample_logits(float *logits, int vocab, float temperature, float top_p, int top_k,
                      float rep_penalty, uint64_t *rng, const int *history, int history_len) {
    g_temperature = temperature;
    g_top_p = top_p;
    g_top_k = top_k;
    g_rep_penalty = rep_penalty;
    g_rng = *rng;
    g_history_len = history_len < 4096 ? history_len : 4096;
    memcpy(g_history, history, (size_t)g_history_len * sizeof(int));
    const int t = sample_logits(logits, vocab);
    *rng = g_rng;
    return t;
}

/* ── model attached to an oracle po_model ── */

static void ref_cfg_from(Cfg *c, const pk_cfg *p) {
    memset(c, 0, sizeof(*c));
    c->hidden = p->hidden; c->n_layers = p->n_layers; c->n_heads = p->n_heads;
    c->n_kv_heads = p->n_kv_heads; c->head_dim = p->head_dim;
    c->n_experts = p->n_experts; c->topk = p->topk; c->moe_inter = p->moe_inter;
    c->dense_inter = p->moe_inter / 2; c->vocab = p->vocab; c->ctx_len = p->ctx_len;
    c->sliding_window = p->sliding_window; c->eps = p->eps; c->theta = p->theta;
    c->rope_factor = p->rope_factor; c->rope_beta_fast = p->rope_beta_fast;
    c->rope_beta_slow = p->rope_beta_slow; c->rope_original_ctx = p->rope_original_ctx;
    c->rope_truncate = p->rope_truncate; c->rope_attn_factor = p->rope_attn_factor;
    c->swiglu_limit = p->swiglu_limit; c->swiglu_alpha = p->swiglu_alpha;
    c->routed_scale = p->routed_scale; c->has_attn_bias = 1;
    c->stop_ids[0] = 200002; c->stop_ids[1] = 200012; c->n_stop = 2;
    for (int i = 0; i < 128; i++) c->layer_type[i] = p->layer_type[i];
}

static void qt_f32(QT *t, const float *p, int O, int I) {
    memset(t, 0, sizeof(*t));
    t->fmt = 0; t->qf = (float *)p; t->O = O; t->I = I;
}

int ref_attach(po_model *pm, const pk_cfg *pc) {
    Model *m = &g_ref;
    memset(m, 0, sizeof(*m));
    ref_cfg_from(&m->c, pc);
    Cfg *c = &m->c;
    int D = c->hidden, H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim;
    int E = c->n_experts, L = c->n_layers;

    qt_f32(&m->embed, po_model_tensor(pm, PK_T_EMBED, 0, NULL), c->vocab, D);
    const float *lm_s = NULL;
    const void *lm = po_model_tensor(pm, PK_T_LM_HEAD, 0, &lm_s);
    memset(&m->lm_head, 0, sizeof(QT));
    m->lm_head.O = c->vocab; m->lm_head.I = D;
    if (pc->lm_head_fmt == PK_FMT_INT8) {
        m->lm_head.fmt = 1; m->lm_head.q8 = (int8_t *)lm; m->lm_head.s = (float *)lm_s;
    } else {
        m->lm_head.fmt = 0; m->lm_head.qf = (float *)lm;
    }
    m->final_norm = (float *)po_model_tensor(pm, 0, 0, NULL);

    m->L = calloc((size_t)L, sizeof(Layer));
    m->ecap = E;
    m->ecache = calloc((size_t)L, sizeof(ESlot *));
    m->ecn = calloc((size_t)L, sizeof(int));
    m->pin = calloc((size_t)L, sizeof(ESlot *));
    m->npin = calloc((size_t)L, sizeof(int));
    m->eusage = calloc((size_t)L, sizeof(uint32_t *));
    m->eheat = calloc((size_t)L, sizeof(uint32_t *));
    for (int l = 0; l < L; l++) {
        Layer *ly = &m->L[l];
        ly->layer_type = c->layer_type[l];
        ly->in_ln = (float *)po_model_tensor(pm, -1, l, NULL);
        ly->post_ln = (float *)po_model_tensor(pm, -2, l, NULL);
        qt_f32(&ly->wq, po_model_tensor(pm, PK_T_WQ, l, NULL), H * hd, D);
        qt_f32(&ly->wk, po_model_tensor(pm, PK_T_WK, l, NULL), KVH * hd, D);
        qt_f32(&ly->wv, po_model_tensor(pm, PK_T_WV, l, NULL), KVH * hd, D);
        qt_f32(&ly->wo, po_model_tensor(pm, PK_T_WO, l, NULL), D, H * hd);
        ly->bq = (float *)po_model_tensor(pm, PK_T_BQ, l, NULL);
        ly->bk = (float *)po_model_tensor(pm, PK_T_BK, l, NULL);
        ly->bv = (float *)po_model_tensor(pm, PK_T_BV, l, NULL);
        ly->bo = (float *)po_model_tensor(pm, PK_T_BO, l, NULL);
        ly->sinks = (float *)po_model_tensor(pm, PK_T_SINKS, l, NULL);
        ly->router = (float *)po_model_tensor(pm, PK_T_ROUTER, l, NULL);
        ly->router_bias = (float *)po_model_tensor(pm, PK_T_ROUTER_B, l, NULL);
        m->ecache[l] = calloc((size_t)E, sizeof(ESlot));
        m->ecn[l] = E;
        for (int e = 0; e < E; e++) {
            ESlot *es = &m->ecache[l][e];
            const uint8_t *gq, *dq;
            const float *gs_, *ds_, *gb, *db;
            po_model_expert(pm, l, e, &gq, &gs_, &dq, &ds_, &gb, &db);
            es->eid = e; es->layer = l;
            es->gu.fmt = 2; es->gu.q4 = (uint8_t *)gq; es->gu.s = (float *)gs_;
            es->gu.O = c->moe_inter; es->gu.I = D; es->gu.block_size = pc->group_size;
            es->d.fmt = 2; es->d.q4 = (uint8_t *)dq; es->d.s = (float *)ds_;
            es->d.O = D; es->d.I = c->moe_inter / 2; es->d.block_size = pc->group_size;
            es->gu_bias = (float *)gb; es->d_bias = (float *)db;
        }
    }
    kv_init(&m->kv, L, KVH, hd, c->ctx_len);
    /* Greedy sampling, no repetition penalty (TEMPERATURE=0 REP=1). */
    g_temperature = 0.0f;
    g_rep_penalty = 1.0f;
    g_history_len = 0;
    g_ref_ready = 1;
    return 0;
}

void ref_reset_kv(void) {
    Model *m = &g_ref;
    int kv_dim = m->c.n_kv_heads * m->c.head_dim;
    for (int l = 0; l < m->c.n_layers; l++) {
        memset(m->kv.K[l], 0, (size_t)m->kv.max_pos * kv_dim * sizeof(float));
        memset(m->kv.V[l], 0, (size_t)m->kv.max_pos * kv_dim * sizeof(float));
    }
    g_history_len = 0;
}

int ref_moe_forward(int layer, const float *x, float *out) {
    if (!g_ref_ready) return -1;
    moe_forward(out, x, &g_ref, layer, &g_ref.c);
    return 0;
}

int ref_expert_apply(int layer, int eid, const float *x, float *dst, float w) {
    if (!g_ref_ready) return -1;
    expert_apply(&g_ref.ecache[layer][eid], x, dst, w, &g_ref.c);
    return 0;
}

int ref_gqa_attention(int layer, const float *x, int pos, float *out) {
    if (!g_ref_ready) return -1;
    gqa_attention(out, x, &g_ref.L[layer], &g_ref.kv, layer, pos, &g_ref.c);
    return 0;
}

void ref_rope_apply(const pk_cfg *pc, float *q, float *k, int pos) {
    Cfg c;
    ref_cfg_from(&c, pc);
    rope_apply(q, k, pos, c.head_dim, c.n_heads, c.n_kv_heads, &c);
}

float ref_yarn_inv_freq(const pk_cfg *pc, int j) {
    Cfg c;
    ref_cfg_from(&c, pc);
    return yarn_inv_freq(&c, j);
}

int ref_forward_token(int tok, int pos) {
    if (!g_ref_ready) return -1;
    return forward_token(&g_ref, tok, pos);
}

/* prefill_tokens with PREFILL_BATCH = batch (picchio.c:1936-1975). */
int ref_prefill_tokens(const int *ids, int n, int pos_base, int batch) {
    if (!g_ref_ready) return -1;
    char b[32];
    snprintf(b, sizeof(b), "%d", batch);
    setenv("PREFILL_BATCH", b, 1);
    return prefill_tokens(&g_ref, ids, n, pos_base);
}

/* Per-stage .npy dumps of picchio's ORACLE_DIR mode (picchio.c:204-249) into
 * `dir` (NULL: off). With dumps on, forward_token writes its logits to
 * <dir>/logits.npy (picchio.c:1746) and prefill_tokens runs position by
 * position (picchio.c:1947-1948), so switch them on after a batched prefill. */
void ref_set_dump_dir(const char *dir) { g_oracle_dir = dir; }
