/* pk_oracle.c — CPU restatement of picchio's quantized-MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + host-CPU baseline); never linked
 * into the product library. See pk_oracle.h for the per-function pinning.
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -fopenmp -ffp-contract=off).
 * Contraction is switched off and every product-sum the reference compiler
 * fuses (gcc -O3 -march=native defaults to -ffp-contract=fast) is written as
 * fmaf(), so the bits do not depend on this compiler's fusion choices.
 */
#include "pk_oracle.h"
#include "../picchio_amd/csrc/pk_synth.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#ifdef __AVX2__
#include <immintrin.h>
#endif

/* ═══════════════════ quantizers ═══════════════════ */

/* convert.py:45-93, quantize_int4(tensor, group_size) with group_size > 0 and
 * group_size < I: per (row, group) amax (fp32), scale = amax/7 in fp32 or 1e-8
 * when amax <= 1e-8, q = clip(round_half_even(w/scale), -8, 7), packed two per
 * byte, even column in the low nibble (convert.py:84-91). group_size <= 0 or
 * >= I takes the per-row branch (convert.py:57-61), same rules per row. */
void po_quantize_int4_gs(const float *w, int O, int I, int gs,
                         uint8_t *packed, float *scales) {
    int per_row = (gs <= 0 || gs >= I);
    int g_len = per_row ? I : gs;
    int ng = per_row ? 1 : (I + gs - 1) / gs;
    int rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        uint8_t *pr = packed + (int64_t)o * rb;
        memset(pr, 0, (size_t)rb);
        for (int g = 0; g < ng; g++) {
            int a0 = g * g_len, a1 = a0 + g_len < I ? a0 + g_len : I;
            float amax = 0.0f;
            for (int i = a0; i < a1; i++) {
                float v = fabsf(wr[i]);
                if (v > amax) amax = v;
            }
            float s = amax > 1e-8f ? amax / 7.0f : 1e-8f;
            scales[(int64_t)o * ng + g] = s;
            for (int i = a0; i < a1; i++) {
                float r = rintf(wr[i] / s);       /* np.round: half to even */
                if (r > 7.0f) r = 7.0f;
                if (r < -8.0f) r = -8.0f;
                uint8_t nib = (uint8_t)((int)r + 8) & 0xF;
                pr[i >> 1] |= (i & 1) ? (uint8_t)(nib << 4) : nib;
            }
        }
    }
}

/* convert.py:106-126, quantize_int8: per-row amax/127 (1.0 when amax == 0),
 * q = clip(rint(w/s), -127, 127). */
void po_quantize_int8_rows(const float *w, int O, int I, int8_t *q, float *scales) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        float amax = 0.0f;
        for (int i = 0; i < I; i++) {
            float v = fabsf(wr[i]);
            if (v > amax) amax = v;
        }
        float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        scales[o] = s;
        for (int i = 0; i < I; i++) {
            float r = rintf(wr[i] / s);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[(int64_t)o * I + i] = (int8_t)r;
        }
    }
}

/* quant.h:366-392, quantize_rows_i4: per-row amax/7 clamped to >= 1e-8 after
 * the division, lrintf, clip [-8, 7]. */
void po_quantize_rows_i4(const float *w, int O, int I, uint8_t *q4, float *scales) {
    int rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        float amax = 0.0f;
        for (int i = 0; i < I; i++) {
            float v = fabsf(wr[i]);
            if (v > amax) amax = v;
        }
        float s = amax / 7.0f;
        if (s < 1e-8f) s = 1e-8f;
        scales[o] = s;
        for (int i = 0; i < I; i += 2) {
            long v0 = lrintf(wr[i] / s), v1 = 0;
            if (v0 > 7) v0 = 7;
            if (v0 < -8) v0 = -8;
            if (i + 1 < I) {
                v1 = lrintf(wr[i + 1] / s);
                if (v1 > 7) v1 = 7;
                if (v1 < -8) v1 = -8;
            }
            q4[(int64_t)o * rb + (i >> 1)] = (uint8_t)((v0 + 8) | ((v1 + 8) << 4));
        }
    }
}

/* ═══════════════════ matmul kernels ═══════════════════
 * The reference's AVX2 kernels keep eight fp32 accumulators: lane j of a
 * 16-column step takes columns c+j (first FMA) and c+8+j (second FMA), and the
 * eight lanes are folded by hsum256 (quant.h:94-103) as
 *     ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7)).
 * lanes8_sum() is that fold. */

static inline float lanes8_sum(const float l[8]) {
    float b0 = l[0] + l[4], b1 = l[1] + l[5], b2 = l[2] + l[6], b3 = l[3] + l[7];
    return (b0 + b2) + (b1 + b3);
}

#ifdef __AVX2__
static inline float avx_lanes_sum(__m256 v) {
    float l[8];
    _mm256_storeu_ps(l, v);
    return lanes8_sum(l);
}
/* 8 packed bytes -> 16 floats (nib - 8), column order: byte b gives columns
 * 2b (low nibble) and 2b+1 (high nibble). */
static inline void avx_nibbles16(const uint8_t *p, __m256 *c0_7, __m256 *c8_15) {
    uint64_t b8;
    memcpy(&b8, p, 8);
    __m128i bytes = _mm_cvtsi64_si128((long long)b8);
    __m128i lo = _mm_and_si128(bytes, _mm_set1_epi8(0x0F));
    __m128i hi = _mm_and_si128(_mm_srli_epi16(bytes, 4), _mm_set1_epi8(0x0F));
    __m128i cols = _mm_unpacklo_epi8(lo, hi);             /* columns 0..15 */
    __m256i off = _mm256_set1_epi32(8);
    *c0_7 = _mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_cvtepu8_epi32(cols), off));
    *c8_15 = _mm256_cvtepi32_ps(
        _mm256_sub_epi32(_mm256_cvtepu8_epi32(_mm_unpackhi_epi64(cols, cols)), off));
}
#endif

static inline float nib_val(const uint8_t *w, int col) {
    uint8_t b = w[col >> 1];
    return (float)((int)((col & 1) ? (b >> 4) : (b & 0xF)) - 8);
}

/* quant.h:117-148 (AVX2 branch). */
void po_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *w = W + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            int i = 0;
            float a;
#ifdef __AVX2__
            __m256 acc = _mm256_setzero_ps();
            for (; i + 8 <= I; i += 8)
                acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + i), _mm256_loadu_ps(w + i), acc);
            a = avx_lanes_sum(acc);
#else
            float l[8] = {0};
            for (; i + 8 <= I; i += 8)
                for (int j = 0; j < 8; j++) l[j] = fmaf(xs[i + j], w[i + j], l[j]);
            a = lanes8_sum(l);
#endif
            /* Ragged tail (I % 8 columns), as gcc 11.4 -O3 vectorises the
             * scalar loop of quant.h:132: a block of 4 products is formed
             * first and added in order (not contracted), the last <= 3
             * columns are contracted fmas. */
            if (I - i >= 4) {
                float p0 = xs[i] * w[i], p1 = xs[i + 1] * w[i + 1];
                float p2 = xs[i + 2] * w[i + 2], p3 = xs[i + 3] * w[i + 3];
                a = a + p0; a = a + p1; a = a + p2; a = a + p3;
                i += 4;
            }
            for (; i < I; i++) a = fmaf(xs[i], w[i], a);
            y[(int64_t)s * O + o] = a;
        }
    }
}

/* quant.h:152-186 (AVX2 branch): fp32 accumulation of x·q, one multiply by
 * the row scale at the end. */
void po_matmul_q8(float *y, const float *x, const int8_t *q, const float *scale,
                  int S, int I, int O) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const int8_t *w = q + (int64_t)o * I;
        float sc = scale[o];
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            int i = 0;
            float a;
#ifdef __AVX2__
            __m256 acc = _mm256_setzero_ps();
            for (; i + 8 <= I; i += 8) {
                int64_t b8;
                memcpy(&b8, w + i, 8);
                __m256 wf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_cvtsi64_si128(b8)));
                acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + i), wf, acc);
            }
            a = avx_lanes_sum(acc);
#else
            float l[8] = {0};
            for (; i + 8 <= I; i += 8)
                for (int j = 0; j < 8; j++) l[j] = fmaf(xs[i + j], (float)w[i + j], l[j]);
            a = lanes8_sum(l);
#endif
            for (; i < I; i++) a = fmaf(xs[i], (float)w[i], a);
            y[(int64_t)s * O + o] = a * sc;
        }
    }
}

/* quant.h:191-253 (AVX2 branch), per-row INT4. The pair tail
 * `a += x0*lo + x1*hi` is contracted by gcc as a + fma(x0, lo, x1*hi). */
void po_matmul_i4(float *y, const float *x, const uint8_t *q4, const float *scale,
                  int S, int I, int O) {
    int rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        float sc = scale[o];
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            int i = 0;
            float a;
#ifdef __AVX2__
            __m256 acc = _mm256_setzero_ps();
            for (; i + 16 <= I; i += 16) {
                __m256 c0, c1;
                avx_nibbles16(w + (i >> 1), &c0, &c1);
                acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + i), c0, acc);
                acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + i + 8), c1, acc);
            }
            a = avx_lanes_sum(acc);
#else
            float l[8] = {0};
            for (; i + 16 <= I; i += 16) {
                for (int j = 0; j < 8; j++) l[j] = fmaf(xs[i + j], nib_val(w + (i >> 1), j), l[j]);
                for (int j = 0; j < 8; j++) l[j] = fmaf(xs[i + 8 + j], nib_val(w + (i >> 1), 8 + j), l[j]);
            }
            a = lanes8_sum(l);
#endif
            for (; i + 1 < I; i += 2) {
                uint8_t b = w[i >> 1];
                float lo = (float)((int)(b & 0xF) - 8), hi = (float)((int)(b >> 4) - 8);
                a = a + fmaf(xs[i], lo, xs[i + 1] * hi);
            }
            if (i < I) a = fmaf(xs[i], (float)((int)(w[i >> 1] & 0xF) - 8), a);
            y[(int64_t)s * O + o] = a * sc;
        }
    }
}

/* quant.h:259-319 (AVX2 branch), group-scaled INT4. Per group: eight lane
 * chains over the full 16-column steps, lanes8_sum, then the scalar tail
 * (contracted: ga = fma(x, q, ga)), then a = fma(ga, scale_g, a). */
void po_matmul_i4_gs(float *y, const float *x, const uint8_t *q4, const float *scale,
                     int S, int I, int O, int gs) {
    int rb = (I + 1) / 2;
    int ng = (I + gs - 1) / gs;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        const float *sc = scale + (int64_t)o * ng;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float a = 0.0f;
            for (int g = 0; g < ng; g++) {
                int g0 = g * gs, g1 = g0 + gs < I ? g0 + gs : I;
                int gi = g0;
                float ga;
#ifdef __AVX2__
                __m256 acc = _mm256_setzero_ps();
                for (; gi + 16 <= g1; gi += 16) {
                    __m256 c0, c1;
                    avx_nibbles16(w + (gi >> 1), &c0, &c1);
                    acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + gi), c0, acc);
                    acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + gi + 8), c1, acc);
                }
                ga = avx_lanes_sum(acc);
#else
                float l[8] = {0};
                for (; gi + 16 <= g1; gi += 16) {
                    const uint8_t *p = w + (gi >> 1);
                    for (int j = 0; j < 8; j++) l[j] = fmaf(xs[gi + j], nib_val(p, j), l[j]);
                    for (int j = 0; j < 8; j++) l[j] = fmaf(xs[gi + 8 + j], nib_val(p, 8 + j), l[j]);
                }
                ga = lanes8_sum(l);
#endif
                for (; gi < g1; gi += 2) {
                    uint8_t b = w[gi >> 1];
                    ga = fmaf(xs[gi], (float)((int)(b & 0xF) - 8), ga);
                    if (gi + 1 < g1) ga = fmaf(xs[gi + 1], (float)((int)(b >> 4) - 8), ga);
                }
                a = fmaf(ga, sc[g], a);
            }
            y[(int64_t)s * O + o] = a;
        }
    }
}

/* ═══════════════════ elementwise ═══════════════════ */

/* quant.h:396-402: double accumulation of x², one float rsqrt, (x*r)*w. */
void po_rmsnorm(float *out, const float *x, const float *w, int D, float eps) {
    double ms = 0.0;
    for (int i = 0; i < D; i++) ms += (double)x[i] * (double)x[i];
    float r = 1.0f / sqrtf((float)(ms / D) + eps);
    for (int i = 0; i < D; i++) out[i] = x[i] * r * w[i];
}

/* quant.h:406-412. */
void po_softmax(float *x, int n) {
    float m = -1e30f;
    for (int i = 0; i < n; i++) if (x[i] > m) m = x[i];
    float s = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); s += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= s;
}

static inline float po_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }  /* quant.h:417 */

/* picchio.c:1413-1424: interleaved gate/up, gate clamped above, up clamped
 * both sides, out[i] = ((up + 1) * gate) * sigmoid(alpha * gate), in place. */
void po_swiglu_clamped(float *gu, int inter, float limit, float alpha) {
    int half = inter / 2;
    for (int i = 0; i < half; i++) {
        float gate = gu[2 * i], up = gu[2 * i + 1];
        if (gate > limit) gate = limit;
        if (up > limit) up = limit;
        if (up < -limit) up = -limit;
        gu[i] = (up + 1.0f) * gate * po_sigmoid(alpha * gate);
    }
}

/* ═══════════════════ synthetic model ═══════════════════ */

typedef struct {
    uint8_t *gu_q4, *d_q4;
    float *gu_s, *d_s, *gu_b, *d_b;
} po_expert;

typedef struct {
    float *in_ln, *post_ln;
    float *wq, *wk, *wv, *wo, *bq, *bk, *bv, *bo, *sinks;
    float *router, *router_b;
    po_expert *ex;
    float *K, *V;                     /* [ctx_len][kv_dim] */
} po_layer;

struct po_model {
    pk_cfg c;
    int with_attn, with_head;
    float *embed, *lm_head, *lm_s, *final_norm;
    int8_t *lm_q8;
    po_layer *L;
};

static float *po_alloc(int64_t n) {
    float *p = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!p) { fprintf(stderr, "po_alloc: OOM (%lld floats)\n", (long long)n); abort(); }
    return p;
}

static float *po_normal(uint64_t seed, uint32_t kind, uint32_t layer, uint32_t idx,
                        int64_t n, float std) {
    float *p = po_alloc(n);
    uint64_t s = pk_stream(seed, kind, layer, idx);
    int64_t chunk = 1 << 16;
    #pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < (n + chunk - 1) / chunk; b++) {
        int64_t a0 = b * chunk, cnt = n - a0 < chunk ? n - a0 : chunk;
        pk_fill_normal(p + a0, cnt, s, std, a0);
    }
    return p;
}

static float *po_ones(int64_t n) {
    float *p = po_alloc(n);
    for (int64_t i = 0; i < n; i++) p[i] = 1.0f;
    return p;
}

po_model *po_model_build(const pk_cfg *cfg, uint64_t seed, int n_threads) {
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#endif
    (void)n_threads;
    po_model *m = (po_model *)calloc(1, sizeof(po_model));
    m->c = *cfg;
    const pk_cfg *c = &m->c;
    int D = c->hidden, E = c->n_experts, H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim;
    int inter = c->moe_inter, half = inter / 2, gs = c->group_size;
    m->L = (po_layer *)calloc((size_t)c->n_layers, sizeof(po_layer));
    for (int l = 0; l < c->n_layers; l++) {
        po_layer *ly = &m->L[l];
        ly->in_ln = po_ones(D);
        ly->post_ln = po_ones(D);
        ly->router = po_normal(seed, PK_T_ROUTER, l, 0, (int64_t)E * D, 0.02f);
        ly->router_b = po_normal(seed, PK_T_ROUTER_B, l, 0, E, 0.02f);
        ly->ex = (po_expert *)calloc((size_t)E, sizeof(po_expert));
        for (int e = 0; e < E; e++) {
            po_expert *x = &ly->ex[e];
            float *w = po_normal(seed, PK_T_GU, l, e, (int64_t)inter * D, 0.02f);
            x->gu_q4 = (uint8_t *)malloc((size_t)inter * ((D + 1) / 2));
            x->gu_s = po_alloc((int64_t)inter * ((D + gs - 1) / gs));
            po_quantize_int4_gs(w, inter, D, gs, x->gu_q4, x->gu_s);
            free(w);
            w = po_normal(seed, PK_T_DOWN, l, e, (int64_t)D * half, 0.02f);
            x->d_q4 = (uint8_t *)malloc((size_t)D * ((half + 1) / 2));
            x->d_s = po_alloc((int64_t)D * ((half + gs - 1) / gs));
            po_quantize_int4_gs(w, D, half, gs, x->d_q4, x->d_s);
            free(w);
            x->gu_b = po_normal(seed, PK_T_GU_B, l, e, inter, 0.02f);
            x->d_b = po_normal(seed, PK_T_DOWN_B, l, e, D, 0.02f);
        }
        ly->wq = po_normal(seed, PK_T_WQ, l, 0, (int64_t)H * hd * D, 0.02f);
        ly->wk = po_normal(seed, PK_T_WK, l, 0, (int64_t)KVH * hd * D, 0.02f);
        ly->wv = po_normal(seed, PK_T_WV, l, 0, (int64_t)KVH * hd * D, 0.02f);
        ly->wo = po_normal(seed, PK_T_WO, l, 0, (int64_t)D * H * hd, 0.02f);
        ly->bq = po_normal(seed, PK_T_BQ, l, 0, H * hd, 0.02f);
        ly->bk = po_normal(seed, PK_T_BK, l, 0, KVH * hd, 0.02f);
        ly->bv = po_normal(seed, PK_T_BV, l, 0, KVH * hd, 0.02f);
        ly->bo = po_normal(seed, PK_T_BO, l, 0, D, 0.02f);
        ly->sinks = po_normal(seed, PK_T_SINKS, l, 0, H, 0.02f);
        ly->K = (float *)calloc((size_t)c->ctx_len * KVH * hd, sizeof(float));
        ly->V = (float *)calloc((size_t)c->ctx_len * KVH * hd, sizeof(float));
    }
    m->embed = po_normal(seed, PK_T_EMBED, 0, 0, (int64_t)c->vocab * D, 0.02f);
    float *lm = po_normal(seed, PK_T_LM_HEAD, 0, 0, (int64_t)c->vocab * D, 0.02f);
    if (c->lm_head_fmt == PK_FMT_INT8) {
        m->lm_q8 = (int8_t *)malloc((size_t)c->vocab * D);
        m->lm_s = po_alloc(c->vocab);
        po_quantize_int8_rows(lm, c->vocab, D, m->lm_q8, m->lm_s);
        free(lm);
    } else {
        m->lm_head = lm;
    }
    m->final_norm = po_ones(D);
    return m;
}

void po_model_free(po_model *m) {
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; l++) {
        po_layer *ly = &m->L[l];
        for (int e = 0; e < m->c.n_experts; e++) {
            po_expert *x = &ly->ex[e];
            free(x->gu_q4); free(x->gu_s); free(x->d_q4); free(x->d_s);
            free(x->gu_b); free(x->d_b);
        }
        free(ly->ex);
        free(ly->in_ln); free(ly->post_ln); free(ly->router); free(ly->router_b);
        free(ly->wq); free(ly->wk); free(ly->wv); free(ly->wo);
        free(ly->bq); free(ly->bk); free(ly->bv); free(ly->bo); free(ly->sinks);
        free(ly->K); free(ly->V);
    }
    free(m->L);
    free(m->embed); free(m->lm_head); free(m->lm_s); free(m->lm_q8); free(m->final_norm);
    free(m);
}

void po_model_reset_kv(po_model *m) {
    size_t n = (size_t)m->c.ctx_len * m->c.n_kv_heads * m->c.head_dim;
    for (int l = 0; l < m->c.n_layers; l++) {
        memset(m->L[l].K, 0, n * sizeof(float));
        memset(m->L[l].V, 0, n * sizeof(float));
    }
}

void po_model_fill_kv(po_model *m, int layer, int n_pos, uint64_t sk, uint64_t sv) {
    if (layer < 0 || layer >= m->c.n_layers || n_pos < 0 || n_pos > m->c.ctx_len) return;
    int64_t n = (int64_t)n_pos * m->c.n_kv_heads * m->c.head_dim;
    pk_fill_normal(m->L[layer].K, n, sk, 1.0f, 0);
    pk_fill_normal(m->L[layer].V, n, sv, 1.0f, 0);
}

int po_model_expert(po_model *m, int layer, int eid,
                    const uint8_t **gu_q4, const float **gu_s,
                    const uint8_t **d_q4, const float **d_s,
                    const float **gu_b, const float **d_b) {
    if (layer < 0 || layer >= m->c.n_layers || eid < 0 || eid >= m->c.n_experts) return -1;
    po_expert *x = &m->L[layer].ex[eid];
    *gu_q4 = x->gu_q4; *gu_s = x->gu_s; *d_q4 = x->d_q4; *d_s = x->d_s;
    *gu_b = x->gu_b; *d_b = x->d_b;
    return 0;
}

const float *po_model_router(po_model *m, int layer, const float **bias) {
    if (bias) *bias = m->L[layer].router_b;
    return m->L[layer].router;
}

const void *po_model_tensor(po_model *m, int kind, int layer, const float **scales) {
    po_layer *ly = (layer >= 0 && layer < m->c.n_layers) ? &m->L[layer] : NULL;
    if (scales) *scales = NULL;
    switch (kind) {
    case 0: return m->final_norm;
    case -1: return ly ? ly->in_ln : NULL;
    case -2: return ly ? ly->post_ln : NULL;
    case PK_T_ROUTER: return ly ? ly->router : NULL;
    case PK_T_ROUTER_B: return ly ? ly->router_b : NULL;
    case PK_T_WQ: return ly ? ly->wq : NULL;
    case PK_T_WK: return ly ? ly->wk : NULL;
    case PK_T_WV: return ly ? ly->wv : NULL;
    case PK_T_WO: return ly ? ly->wo : NULL;
    case PK_T_BQ: return ly ? ly->bq : NULL;
    case PK_T_BK: return ly ? ly->bk : NULL;
    case PK_T_BV: return ly ? ly->bv : NULL;
    case PK_T_BO: return ly ? ly->bo : NULL;
    case PK_T_SINKS: return ly ? ly->sinks : NULL;
    case PK_T_EMBED: return m->embed;
    case PK_T_LM_HEAD:
        if (m->c.lm_head_fmt == PK_FMT_INT8) {
            if (scales) *scales = m->lm_s;
            return m->lm_q8;
        }
        return m->lm_head;
    default: return NULL;
    }
}

void po_fill_normal(uint64_t seed, int kind, int layer, int idx, int64_t first,
                    int64_t n, float std, float *out) {
    pk_fill_normal(out, n, pk_stream(seed, (uint32_t)kind, (uint32_t)layer, (uint32_t)idx),
                   std, first);
}

/* ═══════════════════ expert path ═══════════════════ */

/* A scalar `acc += a[i] * b[i]` loop of picchio.c as gcc -O3 builds it: the
 * loop is vectorised as an in-order reduction, so the products of the first
 * 4*floor(n/4) terms are rounded on their own and added one by one (not
 * contracted); only the last n % 4 terms are fused multiply-adds. */
static inline float dot_inorder(const float *a, const float *b, int n, float acc) {
    int n4 = n & ~3, i = 0;
    for (; i < n4; i++) { float p = a[i] * b[i]; acc = acc + p; }
    for (; i < n; i++) acc = fmaf(a[i], b[i], acc);
    return acc;
}

/* The FFN of one expert shared by moe_forward (picchio.c:1392-1436) and
 * expert_apply (picchio.c:1768-1791): gate_up + bias, clamped SwiGLU, down +
 * bias; eo[D] receives the expert output. */
static void po_expert_ffn(const pk_cfg *c, const po_expert *x, const float *in,
                          float *gu, float *eo) {
    int D = c->hidden, inter = c->moe_inter, half = inter / 2, gs = c->group_size;
    po_matmul_i4_gs(gu, in, x->gu_q4, x->gu_s, 1, D, inter, gs);
    for (int i = 0; i < inter; i++) gu[i] += x->gu_b[i];
    po_swiglu_clamped(gu, inter, c->swiglu_limit, c->swiglu_alpha);
    po_matmul_i4_gs(eo, gu, x->d_q4, x->d_s, 1, half, D, gs);
    for (int i = 0; i < D; i++) eo[i] += x->d_b[i];
}

void po_expert_apply(po_model *m, int layer, int eid, const float *x, float *dst, float w) {
    const pk_cfg *c = &m->c;
    float *gu = po_alloc(c->moe_inter), *eo = po_alloc(c->hidden);
    po_expert_ffn(c, &m->L[layer].ex[eid], x, gu, eo);
    for (int i = 0; i < c->hidden; i++) dst[i] = fmaf(w, eo[i], dst[i]);
    free(gu); free(eo);
}

/* picchio.c:1330-1341: top-k by repeated argmax, strict '>' (lowest index
 * wins a tie), already-chosen experts skipped; weights[k] = raw logit. */
static void po_topk(const float *scores, int E, int K, int *sel, float *wsel) {
    for (int k = 0; k < K; k++) {
        int best = -1;
        float best_s = -1e30f;
        for (int e = 0; e < E; e++) {
            int taken = 0;
            for (int j = 0; j < k; j++) if (sel[j] == e) { taken = 1; break; }
            if (!taken && scores[e] > best_s) { best_s = scores[e]; best = e; }
        }
        sel[k] = best;
        wsel[k] = best_s;
    }
}

/* Test diagnostics (no reference counterpart): while set, every
 * po_moe_forward appends its router logits here, so that a test can see how
 * close each routing decision along a token chain was. */
static float *g_rtrace = NULL;
static int64_t g_rtrace_cap = 0, g_rtrace_used = 0;
void po_set_router_trace(float *buf, int64_t cap_floats) {
    g_rtrace = buf;
    g_rtrace_cap = buf ? cap_floats : 0;
    g_rtrace_used = 0;
}
int64_t po_router_trace_used(void) { return g_rtrace_used; }

/* picchio.c:1309-1466. Router logit = in-order dot, router bias added after
 * the dot (picchio.c:1317-1324). */
void po_moe_forward(po_model *m, int layer, const float *x, float *out,
                    int *sel, float *wsel, float *logits) {
    const pk_cfg *c = &m->c;
    int D = c->hidden, E = c->n_experts, K = c->topk;
    po_layer *ly = &m->L[layer];
    float *scores = po_alloc(E);
    for (int e = 0; e < E; e++) {
        float dot = dot_inorder(x, ly->router + (int64_t)e * D, D, 0.0f);
        scores[e] = dot + ly->router_b[e];
    }
    if (logits) memcpy(logits, scores, (size_t)E * sizeof(float));
    if (g_rtrace && g_rtrace_used + E <= g_rtrace_cap) {
        memcpy(g_rtrace + g_rtrace_used, scores, (size_t)E * sizeof(float));
        g_rtrace_used += E;
    }
    int s_loc[64];
    float w_loc[64];
    po_topk(scores, E, K, s_loc, w_loc);
    po_softmax(w_loc, K);
    memset(out, 0, (size_t)D * sizeof(float));
    float *gu = po_alloc(c->moe_inter), *eo = po_alloc(D);
    for (int k = 0; k < K; k++) {
        po_expert_ffn(c, &ly->ex[s_loc[k]], x, gu, eo);
        float w = w_loc[k] * c->routed_scale;
        for (int i = 0; i < D; i++) out[i] = fmaf(w, eo[i], out[i]);
    }
    if (sel) memcpy(sel, s_loc, (size_t)K * sizeof(int));
    if (wsel) memcpy(wsel, w_loc, (size_t)K * sizeof(float));
    free(gu); free(eo); free(scores);
}

/* ═══════════════════ attention ═══════════════════ */

/* picchio.c:431-453. The final blend `interp*(1-ef) + extrap*ef` is
 * contracted as fma(interp, 1-ef, extrap*ef). */
float po_yarn_inv_freq(const pk_cfg *c, int j) {
    int dim = c->head_dim;
    float pos_freq = powf(c->theta, 2.0f * (float)j / (float)dim);
    float extrap = 1.0f / pos_freq;
    if (c->rope_factor <= 1.0f) return extrap;
    float low = (float)dim * logf((float)c->rope_original_ctx /
                (c->rope_beta_fast * 2.0f * (float)M_PI)) / (2.0f * logf(c->theta));
    float high = (float)dim * logf((float)c->rope_original_ctx /
                 (c->rope_beta_slow * 2.0f * (float)M_PI)) / (2.0f * logf(c->theta));
    if (c->rope_truncate) { low = floorf(low); high = ceilf(high); }
    if (low < 0) low = 0;
    if (high > dim - 1) high = (float)(dim - 1);
    if (low == high) high += 0.001f;
    float ramp = ((float)j - low) / (high - low);
    if (ramp < 0) ramp = 0;
    if (ramp > 1) ramp = 1;
    float ef = 1.0f - ramp;
    float interp = extrap / c->rope_factor;
    return fmaf(interp, 1.0f - ef, extrap * ef);
}

/* picchio.c:455-473: halves [j, j+hd/2], cos/sin scaled by attn_factor;
 * a*cs - b*sn -> fma(a, cs, -(b*sn)), a*sn + b*cs -> fma(a, sn, b*cs). */
void po_rope_apply(const pk_cfg *c, float *q, float *k, int pos) {
    int hd = c->head_dim, half = hd / 2;
    for (int kind = 0; kind < 2; kind++) {
        float *base = kind == 0 ? q : k;
        int heads = kind == 0 ? c->n_heads : c->n_kv_heads;
        for (int h = 0; h < heads; h++) {
            float *v = base + h * hd;
            for (int j = 0; j < half; j++) {
                float ang = (float)pos * po_yarn_inv_freq(c, j);
                float cs = cosf(ang) * c->rope_attn_factor;
                float sn = sinf(ang) * c->rope_attn_factor;
                float a = v[j], b = v[j + half];
                v[j] = fmaf(a, cs, -(b * sn));
                v[j + half] = fmaf(a, sn, b * cs);
            }
        }
    }
}

/* picchio.c:504-623. */
void po_gqa_attention(po_model *m, int layer, const float *x, int pos, float *out) {
    const pk_cfg *c = &m->c;
    po_layer *ly = &m->L[layer];
    int D = c->hidden, H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim;
    int kv_dim = KVH * hd, group = H / KVH;
    float *q = po_alloc(H * hd), *k = po_alloc(kv_dim), *v = po_alloc(kv_dim);
    po_matmul_f32(q, x, ly->wq, 1, D, H * hd);
    po_matmul_f32(k, x, ly->wk, 1, D, kv_dim);
    po_matmul_f32(v, x, ly->wv, 1, D, kv_dim);
    for (int i = 0; i < H * hd; i++) q[i] += ly->bq[i];
    for (int i = 0; i < kv_dim; i++) k[i] += ly->bk[i];
    for (int i = 0; i < kv_dim; i++) v[i] += ly->bv[i];
    po_rope_apply(c, q, k, pos);
    if (pos < c->ctx_len) {                              /* kv_store, :492-498 */
        memcpy(ly->K + (int64_t)pos * kv_dim, k, (size_t)kv_dim * sizeof(float));
        memcpy(ly->V + (int64_t)pos * kv_dim, v, (size_t)kv_dim * sizeof(float));
    }
    float *att = (float *)calloc((size_t)H * hd, sizeof(float));
    int start = 0, end = pos;
    if (end >= c->ctx_len) end = c->ctx_len - 1;
    if (c->layer_type[layer] == 0) {
        start = end - c->sliding_window + 1;
        if (start < 0) start = 0;
    }
    int n_pos = end - start + 1;
    if (n_pos <= 0) n_pos = 1;
    float *sc = po_alloc(n_pos);
    float scale = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < H; h++) {
        int kvh = h / group;
        const float *qh = q + h * hd;
        for (int t = start; t <= end; t++) {
            float dot = dot_inorder(qh, ly->K + (int64_t)t * kv_dim + kvh * hd, hd, 0.0f);
            sc[t - start] = dot * scale;
        }
        float mx = ly->sinks[h];
        for (int i = 0; i < n_pos; i++) if (sc[i] > mx) mx = sc[i];
        float sum = expf(ly->sinks[h] - mx);
        for (int i = 0; i < n_pos; i++) { sc[i] = expf(sc[i] - mx); sum += sc[i]; }
        for (int i = 0; i < n_pos; i++) sc[i] /= sum;
        float *oh = att + h * hd;
        for (int t = start; t <= end; t++) {
            const float *vt = ly->V + (int64_t)t * kv_dim + kvh * hd;
            float w = sc[t - start];
            for (int i = 0; i < hd; i++) oh[i] = fmaf(w, vt[i], oh[i]);
        }
    }
    po_matmul_f32(out, att, ly->wo, 1, H * hd, D);
    for (int i = 0; i < D; i++) out[i] += ly->bo[i];
    free(q); free(k); free(v); free(att); free(sc);
}

/* ═══════════════════ decode driver ═══════════════════ */

void po_embed(po_model *m, int tok, float *x) {            /* picchio.c:1472-1481 */
    int D = m->c.hidden;
    if (tok < 0 || tok >= m->c.vocab) { memset(x, 0, (size_t)D * sizeof(float)); return; }
    memcpy(x, m->embed + (int64_t)tok * D, (size_t)D * sizeof(float));
}

int po_argmax(const float *logits, int n) {                /* picchio.c:1555-1560 */
    int best = 0;
    for (int i = 1; i < n; i++) if (logits[i] > logits[best]) best = i;
    return best;
}

/* ───────────────────────── sampling (picchio.c:1509-1649) ───────────────────────── */
void po_sampler_init(po_sampler *s, float temperature, float top_p, int top_k, float rep_penalty,
                     uint64_t seed) {
    s->temperature = temperature;
    s->top_p = top_p;
    s->top_k = top_k;
    s->rep_penalty = rep_penalty;
    s->rng = seed;
    s->history_len = 0;
}

/* xorshift64 (picchio.c:1520-1526): shifts 13, 7, 17; the top 31 bits of the
 * state over 2^31 */
float po_rng_float(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (float)(x >> 33) / (float)(1ULL << 31);
}

typedef struct { float val; int idx; } po_iv;
/* descending; equal values compare equal (the reference's comparators) */
static int po_desc_iv(const void *a, const void *b) {
    const float fa = ((const po_iv *)a)->val, fb = ((const po_iv *)b)->val;
    return (fa < fb) - (fa > fb);
}
static int po_desc_f(const void *a, const void *b) {
    const float fa = *(const float *)a, fb = *(const float *)b;
    return (fa < fb) - (fa > fb);
}

static int po_sample_record(po_sampler *s, int tok) {
    if (s->history_len < 4096) s->history[s->history_len++] = tok;
    return tok;
}

int po_sample_logits(po_sampler *s, float *logits, int vocab) {
    /* 1. repetition penalty, once per history entry (picchio.c:1541-1551) */
    if (s->rep_penalty > 1.0f)
        for (int i = 0; i < s->history_len; i++) {
            const int t = s->history[i];
            if (t >= 0 && t < vocab) {
                if (logits[t] > 0) logits[t] /= s->rep_penalty;
                else logits[t] *= s->rep_penalty;
            }
        }
    /* 2. greedy below 1e-6 (first maximum), else temperature */
    if (s->temperature < 1e-6f) return po_sample_record(s, po_argmax(logits, vocab));
    const float inv_temp = 1.0f / s->temperature;
    for (int i = 0; i < vocab; i++) logits[i] *= inv_temp;
    /* 3. top-k: the K-th largest of a sorted copy; below it -> -1e30 */
    if (s->top_k > 0 && s->top_k < vocab) {
        float *cp = (float *)malloc((size_t)vocab * sizeof(float));
        memcpy(cp, logits, (size_t)vocab * sizeof(float));
        qsort(cp, (size_t)vocab, sizeof(float), po_desc_f);
        const float thr = cp[s->top_k - 1];
        free(cp);
        for (int i = 0; i < vocab; i++)
            if (logits[i] < thr) logits[i] = -1e30f;
    }
    /* 4. softmax in vocabulary order */
    float mx = -1e30f;
    for (int i = 0; i < vocab; i++) if (logits[i] > mx) mx = logits[i];
    float sum = 0.0f;
    for (int i = 0; i < vocab; i++) {
        logits[i] = expf(logits[i] - mx);
        sum += logits[i];
    }
    for (int i = 0; i < vocab; i++) logits[i] /= sum;
    /* 5. top-p over the probabilities > 1e-10, sorted descending */
    if (s->top_p < 1.0f && s->top_p > 0.0f) {
        int n = 0;
        for (int i = 0; i < vocab; i++) if (logits[i] > 1e-10f) n++;
        if (n > 1) {
            po_iv *v = (po_iv *)malloc((size_t)n * sizeof(po_iv));
            int k = 0;
            for (int i = 0; i < vocab; i++)
                if (logits[i] > 1e-10f) { v[k].val = logits[i]; v[k].idx = i; k++; }
            qsort(v, (size_t)n, sizeof(po_iv), po_desc_iv);
            float cum = 0.0f;
            int cut = n;
            for (int i = 0; i < n; i++) {
                cum += v[i].val;
                if (cum >= s->top_p) { cut = i + 1; break; }
            }
            for (int i = cut; i < n; i++) logits[v[i].idx] = 0.0f;
            sum = 0.0f;
            for (int i = 0; i < vocab; i++) sum += logits[i];
            if (sum > 0) for (int i = 0; i < vocab; i++) logits[i] /= sum;
            free(v);
        }
    }
    /* 6. the draw, cumulative in vocabulary order; else the last p > 0 */
    const float r = po_rng_float(&s->rng);
    float cum = 0.0f;
    for (int i = 0; i < vocab; i++) {
        cum += logits[i];
        if (cum >= r) return po_sample_record(s, i);
    }
    for (int i = vocab - 1; i >= 0; i--)
        if (logits[i] > 0) return po_sample_record(s, i);
    return 0;
}

/* ── the library's arithmetic beyond 4096 kept entries (not a reference
 * function) ── Sums exact: each value times 2^S truncated to a 64-bit
 * integer (exact above 2^(23-S)), added as integers, the total rounded to
 * float once. Top-p: the shortest prefix of the candidates (> 1e-10), sorted
 * by value descending then index, whose exact sum reaches top_p; the pick:
 * the first index whose exact cumulative sum reaches the draw. Everything
 * else as po_sample_logits, which it is outright up to 4096 kept entries. */
static uint64_t po_fx(float v, int S) {
    uint32_t b;
    memcpy(&b, &v, 4);
    const int e = (int)(b >> 23) & 255;
    if (e == 0 || (b >> 31)) return 0;
    const uint64_t m = (b & 0x7fffffu) | 0x800000u;
    const int sh = e - 150 + S;
    if (sh >= 0) return m << sh;
    return sh <= -24 ? 0 : m >> (-sh);
}
static float po_unfx(uint64_t q, int S) { return ldexpf((float)q, -S); }
static int po_desc_iv_idx(const void *a, const void *b) {
    const po_iv *x = (const po_iv *)a, *y = (const po_iv *)b;
    if (x->val != y->val) return x->val > y->val ? -1 : 1;
    return (x->idx > y->idx) - (x->idx < y->idx);
}

int po_sample_logits_fx(po_sampler *s, float *logits, int vocab) {
    if (s->temperature < 1e-6f) return po_sample_logits(s, logits, vocab);
    const float inv_temp = 1.0f / s->temperature;
    float *cp = (float *)malloc((size_t)vocab * sizeof(float));
    memcpy(cp, logits, (size_t)vocab * sizeof(float));
    if (s->rep_penalty > 1.0f)
        for (int i = 0; i < s->history_len; i++) {
            const int t = s->history[i];
            if (t >= 0 && t < vocab) cp[t] = cp[t] > 0 ? cp[t] / s->rep_penalty : cp[t] * s->rep_penalty;
        }
    for (int i = 0; i < vocab; i++) cp[i] *= inv_temp;
    int n = vocab;
    float thr = -INFINITY;
    if (s->top_k > 0 && s->top_k < vocab) {
        float *sc = (float *)malloc((size_t)vocab * sizeof(float));
        memcpy(sc, cp, (size_t)vocab * sizeof(float));
        qsort(sc, (size_t)vocab, sizeof(float), po_desc_f);
        thr = sc[s->top_k - 1];
        free(sc);
        n = 0;
        for (int i = 0; i < vocab; i++) n += !(cp[i] < thr);
    }
    if (n <= 4096) {
        free(cp);
        return po_sample_logits(s, logits, vocab);
    }
    /* cp holds the penalised, scaled logits; -1e30 below the threshold -> 0 */
    float mx = -1e30f;
    for (int i = 0; i < vocab; i++)
        if (!(cp[i] < thr) && cp[i] > mx) mx = cp[i];
    int bits = 0;
    while ((n >> bits) != 0) bits++;
    const int se = 63 - bits;
    uint64_t q = 0;
    for (int i = 0; i < vocab; i++) {
        logits[i] = (cp[i] < thr) ? 0.0f : expf(cp[i] - mx);
        q += po_fx(logits[i], se);
    }
    free(cp);
    const float sum = po_unfx(q, se);
    for (int i = 0; i < vocab; i++) logits[i] /= sum;
    if (s->top_p < 1.0f && s->top_p > 0.0f) {
        int na = 0;
        for (int i = 0; i < vocab; i++) if (logits[i] > 1e-10f) na++;
        if (na > 1) {
            po_iv *v = (po_iv *)malloc((size_t)na * sizeof(po_iv));
            int k = 0;
            for (int i = 0; i < vocab; i++)
                if (logits[i] > 1e-10f) { v[k].val = logits[i]; v[k].idx = i; k++; }
            qsort(v, (size_t)na, sizeof(po_iv), po_desc_iv_idx);
            uint64_t target = po_fx(s->top_p, 62);
            if (target == 0) target = 1;
            uint64_t acc = 0;
            int cut = na;
            for (int i = 0; i < na; i++) {
                acc += po_fx(v[i].val, 62);
                if (acc >= target) { cut = i + 1; break; }
            }
            for (int i = cut; i < na; i++) logits[v[i].idx] = 0.0f;
            uint64_t q2 = 0;
            for (int i = 0; i < vocab; i++) q2 += po_fx(logits[i], 62);
            const float s2 = po_unfx(q2, 62);
            if (s2 > 0) for (int i = 0; i < vocab; i++) logits[i] /= s2;
            free(v);
        }
    }
    const float r = po_rng_float(&s->rng);
    if (r <= 0.0f) return po_sample_record(s, 0);
    const uint64_t R = po_fx(r, 62);
    uint64_t acc = 0;
    for (int i = 0; i < vocab; i++) {
        acc += po_fx(logits[i], 62);
        if (acc >= R) return po_sample_record(s, i);
    }
    for (int i = vocab - 1; i >= 0; i--)
        if (logits[i] > 0) return po_sample_record(s, i);
    return 0;
}

static void po_lm_head(po_model *m, const float *hn, float *logits) {
    const pk_cfg *c = &m->c;
    if (c->lm_head_fmt == PK_FMT_INT8)
        po_matmul_q8(logits, hn, m->lm_q8, m->lm_s, 1, c->hidden, c->vocab);
    else
        po_matmul_f32(logits, hn, m->lm_head, 1, c->hidden, c->vocab);
}

/* picchio.c:1655-1756 with TEMPERATURE=0, REP=1 (greedy). */
int po_forward_token(po_model *m, int tok, int pos, float *logits_out) {
    const pk_cfg *c = &m->c;
    int D = c->hidden;
    float *h = po_alloc(D), *hn = po_alloc(D), *ao = po_alloc(D), *fo = po_alloc(D);
    po_embed(m, tok, h);
    for (int l = 0; l < c->n_layers; l++) {
        po_layer *ly = &m->L[l];
        po_rmsnorm(hn, h, ly->in_ln, D, c->eps);
        po_gqa_attention(m, l, hn, pos, ao);
        for (int i = 0; i < D; i++) h[i] += ao[i];
        po_rmsnorm(hn, h, ly->post_ln, D, c->eps);
        po_moe_forward(m, l, hn, fo, NULL, NULL, NULL);
        for (int i = 0; i < D; i++) h[i] += fo[i];
    }
    po_rmsnorm(hn, h, m->final_norm, D, c->eps);
    float *logits = po_alloc(c->vocab);
    po_lm_head(m, hn, logits);
    int next = po_argmax(logits, c->vocab);
    if (logits_out) memcpy(logits_out, logits, (size_t)c->vocab * sizeof(float));
    free(h); free(hn); free(ao); free(fo); free(logits);
    return next;
}

/* picchio.c:1795-1932. Router here starts the dot at the bias
 * (picchio.c:1840-1844); each token's expert outputs are accumulated in the
 * order the experts were first requested in the chunk (uniq[]). */
int po_forward_prefill(po_model *m, const int *ids, int n, int pos_base) {
    const pk_cfg *c = &m->c;
    int D = c->hidden, E = c->n_experts, K = c->topk;
    float *H = po_alloc((int64_t)n * D), *XN = po_alloc((int64_t)n * D);
    float *hn = po_alloc(D), *ao = po_alloc(D), *scores = po_alloc(E);
    int *sel_all = (int *)malloc((size_t)n * K * sizeof(int));
    float *w_all = po_alloc((int64_t)n * K);
    int *uniq = (int *)malloc((size_t)E * sizeof(int));
    unsigned char *seen = (unsigned char *)malloc((size_t)E);
    for (int p = 0; p < n; p++) po_embed(m, ids[p], H + (int64_t)p * D);
    for (int l = 0; l < c->n_layers; l++) {
        po_layer *ly = &m->L[l];
        for (int p = 0; p < n; p++) {
            float *h = H + (int64_t)p * D;
            po_rmsnorm(hn, h, ly->in_ln, D, c->eps);
            po_gqa_attention(m, l, hn, pos_base + p, ao);
            for (int i = 0; i < D; i++) h[i] += ao[i];
        }
        memset(seen, 0, (size_t)E);
        int n_uniq = 0;
        for (int p = 0; p < n; p++) {
            float *xn = XN + (int64_t)p * D;
            po_rmsnorm(xn, H + (int64_t)p * D, ly->post_ln, D, c->eps);
            for (int e = 0; e < E; e++) {
                scores[e] = dot_inorder(xn, ly->router + (int64_t)e * D, D, ly->router_b[e]);
            }
            int *sel = sel_all + (size_t)p * K;
            float *wg = w_all + (size_t)p * K;
            po_topk(scores, E, K, sel, wg);
            po_softmax(wg, K);
            for (int k = 0; k < K; k++)
                if (!seen[sel[k]]) { seen[sel[k]] = 1; uniq[n_uniq++] = sel[k]; }
        }
        float *moe = (float *)calloc((size_t)n * D, sizeof(float));
        for (int u = 0; u < n_uniq; u++) {
            int eid = uniq[u];
            for (int p = 0; p < n; p++)
                for (int k = 0; k < K; k++)
                    if (sel_all[(size_t)p * K + k] == eid)
                        po_expert_apply(m, l, eid, XN + (int64_t)p * D, moe + (int64_t)p * D,
                                        w_all[(size_t)p * K + k] * c->routed_scale);
        }
        for (int p = 0; p < n; p++)
            for (int i = 0; i < D; i++) H[(int64_t)p * D + i] += moe[(int64_t)p * D + i];
        free(moe);
    }
    po_rmsnorm(hn, H + (int64_t)(n - 1) * D, m->final_norm, D, c->eps);
    float *logits = po_alloc(c->vocab);
    po_lm_head(m, hn, logits);
    int next = po_argmax(logits, c->vocab);
    free(logits); free(H); free(XN); free(hn); free(ao); free(scores);
    free(sel_all); free(w_all); free(uniq); free(seen);
    return next;
}

/* picchio.c:1936-1975 (no oracle dumps / tracing, REP=1). */
int po_prefill_tokens(po_model *m, const int *ids, int n, int pos_base, int batch) {
    int last = ids[0];
    if (batch <= 1 || n <= 1) {
        for (int i = 0; i < n; i++) {
            last = po_forward_token(m, ids[i], pos_base + i, NULL);
            if (last < 0 || last >= m->c.vocab) last = 0;
        }
        return last;
    }
    for (int off = 0; off < n; off += batch) {
        int len = n - off < batch ? n - off : batch;
        last = po_forward_prefill(m, ids + off, len, pos_base + off);
        if (last < 0 || last >= m->c.vocab) last = 0;
    }
    return last;
}

/* ═══════════════ the grouped int8 path's arithmetic (not a reference function) ═══════════════ */

/* ── the library's opt-in integer-dot expert arithmetic, restated ──
 * Not a reference function (pk_i4_device.h pk_write_digits / pk_dot_group). */
void po_act_records(const float *x, int n, int32_t *rec) {
    for (int h = 0; h < n / 32; h++) {
        const float *v = x + 32 * h;
        float m = 0.0f;
        for (int c = 0; c < 32; c++) m = fmaxf(m, fabsf(v[c]));
        int k = 0;
        if (m > 0.0f) (void)frexpf(m, &k);
        int32_t *r = rec + (int64_t)h * 24;
        memset(r, 0, 24 * sizeof(int32_t));
        for (int c = 0; c < 32; c++) {
            int A = (int)rintf(ldexpf(v[c], 18 - k));
            for (int i = 0; i < 5; i++) {
                const int d = ((A + 8) & 15) - 8;
                r[4 * i + c / 8] |= (int32_t)((uint32_t)(d & 15) << (4 * (c % 8)));
                A = (A - d) >> 4;
            }
        }
        r[20] = k;
    }
}

void po_i4_dot_matvec(const uint8_t *q4, const float *s, const float *bias, int O, int I,
                      const int32_t *rec, float *y) {
    const int NG = I / 64;
    for (int o = 0; o < O; o++) {
        const uint8_t *qr = q4 + (int64_t)o * (I / 2);
        float acc = 0.0f;
        for (int g = 0; g < NG; g++) {
            const float s16 = 16.0f * s[(int64_t)o * NG + g];
            float t = 0.0f;
            for (int h = 0; h < 2; h++) {
                const int32_t *r = rec + (int64_t)(2 * g + h) * 24;
                int P[5] = {0, 0, 0, 0, 0};
                for (int c = 0; c < 32; c++) {
                    const int col = 64 * g + 32 * h + c;
                    const int q = (col & 1) ? (qr[col / 2] >> 4) : (qr[col / 2] & 15);
                    for (int i = 0; i < 5; i++) {
                        int d = (int)(((uint32_t)r[4 * i + c / 8] >> (4 * (c % 8))) & 15u);
                        if (d >= 8) d -= 16;
                        P[i] += (q - 8) * d;
                    }
                }
                const int C = P[0] + 16 * (P[1] + 16 * (P[2] + 16 * (P[3] + 16 * P[4])));
                const float S = ldexpf(s16, r[20] - 22);
                t = h ? fmaf(S, (float)C, t) : S * (float)C;
            }
            acc = acc + t;
        }
        y[o] = bias ? acc + bias[o] : acc;
    }
}

void po_act_limbs(const float *x, int rows, int cols, int8_t *limbs, int32_t *exps) {
    const int64_t plane = (int64_t)rows * cols;
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (int64_t)r * cols;
        float m = 0.0f;
        for (int i = 0; i < cols; i++) m = fmaxf(m, fabsf(xr[i]));
        int k = 0;
        if (m > 0.0f) (void)frexpf(m, &k);
        exps[r] = k;
        for (int i = 0; i < cols; i++) {
            int A = (int)rintf(ldexpf(xr[i], 20 - k));
            int a0 = (A + 8192) >> 14;
            int rem = A - a0 * 16384;
            int a1 = (rem + 64) >> 7;
            int a2 = rem - a1 * 128;
            int64_t o = (int64_t)r * cols + i;
            limbs[o] = (int8_t)a0;
            limbs[plane + o] = (int8_t)a1;
            limbs[2 * plane + o] = (int8_t)a2;
        }
    }
}

void po_mfma_matvec(const uint8_t *q4, const float *s, const float *bias, int O, int I,
                    const int8_t *l0, const int8_t *l1, const int8_t *l2, int k, float *y) {
    const int ng = I / 64, rb = (I + 1) / 2;
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        float acc = 0.0f;
        for (int g = 0; g < ng; g++) {
            int32_t C = 0;
            for (int i = g * 64; i < g * 64 + 64; i++) {
                const int nib = (i & 1) ? (w[i >> 1] >> 4) : (w[i >> 1] & 15);
                const int A = l0[i] * 16384 + l1[i] * 128 + l2[i];
                C += A * (nib - 8);
            }
            acc = fmaf(16.0f * s[(int64_t)o * ng + g], (float)C, acc);
        }
        y[o] = ldexpf(acc, k - 24);
        if (bias) y[o] = y[o] + bias[o];
    }
}
