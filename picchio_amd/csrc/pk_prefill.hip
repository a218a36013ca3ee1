// pk_prefill.hip — the prompt path: prefill_tokens / forward_prefill
// (picchio.c:1795-1975) and the batched MoE of a chunk of tokens.
//
// A prompt runs in chunks of PREFILL_BATCH positions (64 unless the
// environment says otherwise, read as picchio.c:1937-1938 reads it; 1 selects
// the position-by-position path). Per chunk and layer, on n positions at once:
//   RMSNorm -> QKV GEMV -> RoPE + KV store of every position -> causal /
//   sliding attention of every position (each sees its own window) -> O
//   projection + residual -> RMSNorm -> router logits -> top-k + softmax ->
//   gate_up + SwiGLU and down over all n*K (token, expert) pairs, one launch
//   each -> per-token sum in the chunk's expert order + residual.
// Then the last position's final norm, lm_head and greedy argmax.
#include "pk_engine.h"

#include <stdlib.h>

#include <algorithm>
#include <mutex>

namespace {

__global__ __launch_bounds__(256) void k_embed_rows(const int32_t *ids, const float *embed, int vocab,
                                                    float *H, int D) {
    const int p = blockIdx.x;
    const int tok = ids[p];
    const bool ok = tok >= 0 && tok < vocab;           // embed_token, picchio.c:1476-1480
    const float *row = embed + (int64_t)(ok ? tok : 0) * D;
    float *h = H + (int64_t)p * D;
    for (int i = threadIdx.x; i < D; i += 256) h[i] = ok ? row[i] : 0.0f;
}

// forward_prefill's expert order (picchio.c:1846-1852, :1885-1902): experts are
// ranked by first request, scanning positions, then k; each token adds its
// experts in rank order. perm[p][j] = k of the token's j-th expert. One
// workgroup: first request of each expert by atomic min, rank = number of
// experts requested earlier, then each token orders its k by rank.
constexpr int UP_LDS = 16384;           // routing entries staged in LDS (all loads in flight at once)
__global__ __launch_bounds__(1024) void k_uniq_perm(const int32_t *sel, int n, int K, int E, int32_t *perm) {
    __shared__ int first[128], rank[128];
    __shared__ int s_sel[UP_LDS];
    const int P = n * K;
    const bool staged = P <= UP_LDS && (int)blockDim.x * 16 >= UP_LDS;
    for (int e = threadIdx.x; e < E; e += blockDim.x) first[e] = 0x7fffffff;
    __syncthreads();
    if (staged) {
        int ev[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = threadIdx.x + u * blockDim.x;
            ev[u] = i < P ? sel[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = threadIdx.x + u * blockDim.x;
            if (i < P) {
                s_sel[i] = ev[u];
                if (ev[u] >= 0 && ev[u] < E) atomicMin(&first[ev[u]], i);
            }
        }
    } else {
        for (int i = threadIdx.x; i < P; i += blockDim.x) {
            const int e = sel[i];
            if (e >= 0 && e < E) atomicMin(&first[e], i);
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int r = 0;
        for (int f = 0; f < E; ++f) r += first[f] < first[e];
        rank[e] = first[e] == 0x7fffffff ? 0x7fffffff : r;
    }
    __syncthreads();
    // the token's K ranks into registers first (K <= 16, the engine's
    // bound): read once, not again after every store to perm
    for (int p = threadIdx.x; p < n; p += blockDim.x) {
        const int32_t *sp = staged ? s_sel + p * K : sel + (int64_t)p * K;
        int r[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int ek = k < K ? sp[k] : -1;
            r[k] = (ek >= 0 && ek < E) ? rank[ek] : 0x7fffffff;
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            if (k >= K) break;
            int pos = 0;
#pragma unroll
            for (int k2 = 0; k2 < 16; ++k2)
                if (k2 < K) pos += (r[k2] < r[k]) || (r[k2] == r[k] && k2 < k);
            perm[(int64_t)p * K + pos] = k;
        }
    }
}

// moe = 0; moe = fma(w_k, eo_k, moe) in rank order (expert_apply's
// dst += w * eo, picchio.c:1788); out = residual + moe (picchio.c:1910-1914)
// or moe alone.
// The same sums four columns per thread (D % 4 == 0, 16-byte aligned rows).
__global__ __launch_bounds__(256) void k_combine_rows4(float *out, const float *residual, const float *eo,
                                                       const float *w, const int32_t *perm, int K, int D) {
    const int p = blockIdx.y;
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= D) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < K; ++j) {
        const int k = perm ? perm[p * K + j] : j;
        const float wk = w[p * K + k];
        const float4 e = *reinterpret_cast<const float4 *>(eo + ((int64_t)p * K + k) * D + i);
        acc.x = __builtin_fmaf(wk, e.x, acc.x);
        acc.y = __builtin_fmaf(wk, e.y, acc.y);
        acc.z = __builtin_fmaf(wk, e.z, acc.z);
        acc.w = __builtin_fmaf(wk, e.w, acc.w);
    }
    const int64_t o = (int64_t)p * D + i;
    if (residual) {
        const float4 rr = *reinterpret_cast<const float4 *>(residual + o);
        acc = make_float4(rr.x + acc.x, rr.y + acc.y, rr.z + acc.z, rr.w + acc.w);
    }
    *reinterpret_cast<float4 *>(out + o) = acc;
}

__global__ __launch_bounds__(256) void k_combine_rows(float *out, const float *residual, const float *eo,
                                                      const float *w, const int32_t *perm, int K, int D) {
    const int p = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= D) return;
    float acc = 0.0f;
    for (int j = 0; j < K; ++j) {
        const int k = perm ? perm[p * K + j] : j;
        acc = __builtin_fmaf(w[p * K + k], eo[((int64_t)p * K + k) * D + i], acc);   // perm null: k order
    }
    const int64_t o = (int64_t)p * D + i;
    out[o] = residual ? residual[o] + acc : acc;
}

}  // namespace

// out[t] = (residual ? residual[t] : 0) + the weighted rows of token t's pairs
static int launch_combine(pk_engine *e, float *out, const float *residual, const float *eo, const float *w,
                          const int32_t *perm, int K, int D, int T) {
    const bool v4 = (D & 3) == 0 && (((uintptr_t)out | (uintptr_t)eo | (uintptr_t)residual) & 15) == 0;
    if (v4)
        hipLaunchKernelGGL(k_combine_rows4, dim3((D / 4 + 255) / 256, T), dim3(256), 0, e->stream, out, residual,
                           eo, w, perm, K, D);
    else
        hipLaunchKernelGGL(k_combine_rows, dim3((D + 255) / 256, T), dim3(256), 0, e->stream, out, residual, eo,
                           w, perm, K, D);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

static int batch_reserve(pk_engine *e, int T) {
    if (T <= e->batch_cap) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "batch buffers must be sized before capturing a graph");
    const pk_cfg *c = &e->c;
    PK_CHECK((int64_t)T * c->topk <= 65535, PK_ERR_UNSUPPORTED, "batched MoE: %d tokens x top-%d", T,
             c->topk);
    PK_HIP(hipStreamSynchronize(e->stream));
    void *ptrs[] = {e->b_logits, e->b_w, e->b_act, e->b_eo, e->b_sel, e->b_perm, e->b_xq, e->b_actq,
                    e->b_pairs, e->b_tiles};
    for (void *p : ptrs) pk_dev_free(e, p);
    e->b_logits = e->b_w = e->b_act = e->b_eo = nullptr;
    e->b_sel = e->b_perm = e->b_xq = e->b_actq = e->b_pairs = e->b_tiles = nullptr;
    e->batch_cap = 0;
    const int64_t TK = (int64_t)T * c->topk;
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_logits, (int64_t)T * c->n_experts * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_w, TK * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_sel, TK * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_perm, TK * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_act, TK * (c->moe_inter / 2) * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_eo, TK * c->hidden * 4));
    // integer-dot records: the token rows', each pair's SwiGLU outputs'
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_xq, (int64_t)T * ((c->hidden + 31) / 32) * PK_XQ_INTS * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_actq, TK * e->ex.gu.RB * PK_XQ_INTS * 4));
    // pairs grouped by expert for the tiled integer-dot launches (tiles of 4)
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_pairs, TK * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->b_tiles, (3 * (TK / 4 + 1 + c->n_experts) + 1) * 4));
    if (!e->skinny_ws) PK_TRY(pk_dev_alloc(e, (void **)&e->skinny_ws, PK_SKINNY_WS * 4));
    e->batch_cap = T;
    return PK_OK;
}

// Scratch of the batched MoE over T rows: router logits, routing, the
// chunk's expert order, the pairs' activations and outputs, and the
// integer-dot records and pair tiles.
struct rows_scratch {
    float *logits, *w, *act, *eo;
    int32_t *sel, *perm, *xq, *actq, *pairs, *tiles;
};

static rows_scratch engine_rows_scratch(pk_engine *e) {
    return {e->b_logits, e->b_w, e->b_act, e->b_eo, e->b_sel, e->b_perm, e->b_xq, e->b_actq, e->b_pairs, e->b_tiles};
}

// Router logits, top-k and softmax of T rows into sc.sel / sc.w. The prompt's
// router (picchio.c:1840-1844) starts each dot at the bias and adds the
// products in order; the lockstep decode of several sequences sums them in a
// fixed tree and adds the bias last (within the fp32 bar of moe_forward's
// order, picchio.c:1316-1324).
// With xq: the top-k launch also writes the records of the T rows of x into
// xq (the integer-dot arithmetic's input).
static int route_rows(pk_engine *e, const rows_scratch &sc, int layer, const float *x, int T, bool prompt_order,
                      int32_t *xq = nullptr) {
    const pk_cfg *c = &e->c;
    const pk_layer_dev &d = e->L[layer];
    if (prompt_order)
        PK_TRY(pk_launch_router_seq(x, d.router, d.router_b, T, c->hidden, c->n_experts, sc.logits, e->stream));
    else
        PK_TRY(pk_launch_gemv_f32(sc.logits, x, d.router, d.router_b, T, c->hidden, c->n_experts, e->stream));
    PK_TRY(pk_trace_router(e, sc.logits, T));
    if (xq)
        return pk_launch_topk_records(sc.logits, T, c->n_experts, c->topk, c->routed_scale, sc.sel, sc.w, x,
                                      T * c->hidden, xq, e->stream);
    return pk_launch_topk_batch(sc.logits, T, c->n_experts, c->topk, c->routed_scale, sc.sel, sc.w, nullptr,
                                e->stream);
}

// The MoE of forward_prefill (picchio.c:1829-1916) for T tokens x [T][D]:
// out[t] = (residual ? residual[t] : 0) + sum over the token's experts, in the
// batch's expert order, of (w_k * routed_scale) * expert_k(x[t]). With
// decode_order the sum runs in routing order instead, as moe_forward adds
// (picchio.c:1445-1454): T independent decode tokens.
static int moe_rows_on(pk_engine *e, const rows_scratch &sc, int layer, const float *x, int T, float *out,
                       const float *residual, bool decode_order) {
    const pk_cfg *c = &e->c;
    const int D = c->hidden, E = c->n_experts, K = c->topk, half = c->moe_inter / 2;
    // the integer-dot option: records of the token rows (written by the top-k
    // launch), then of each pair's SwiGLU outputs (the lockstep decode of
    // several sequences, decode_order, uses it by default)
    const bool dot = (e->i4_dot || (decode_order && e->i4_dot_batch)) && D % 64 == 0 && c->moe_inter % 128 == 0;
    const int64_t xq_row = (int64_t)(D / 32) * PK_XQ_INTS, aq_row = (int64_t)e->ex.gu.RB * PK_XQ_INTS;
    PK_TRY(route_rows(e, sc, layer, x, T, !decode_order, dot ? sc.xq : nullptr));
    if (!decode_order) {
        hipLaunchKernelGGL(k_uniq_perm, dim3(1), dim3(1024), 0, e->stream, sc.sel, T, K, E, sc.perm);
        PK_HIP(hipGetLastError());
    }
    pk_i4_items gu = pk_expert_items(e, layer, false);
    gu.slots = sc.sel;
    gu.x = x; gu.x_stride = D; gu.x_div = K;
    gu.y = sc.act; gu.y_stride = half;
    gu.n_items = T * K;
    if (dot) {
        gu.xq = sc.xq; gu.xq_stride = xq_row;
        gu.yq = sc.actq; gu.yq_stride = aq_row;
    }
    // with the integer dot, pairs of one expert share each weight load (tiles of 4)
    const int P = T * K;
    const int mt = P / 4 + 1 + E;
    pk_i4_tiles tl{sc.pairs, sc.tiles, sc.tiles + mt, sc.tiles + 2 * mt, sc.tiles + 3 * mt};
    // (the tile kernel keeps 4 pairs' group sums in LDS: rows of at most 64 groups)
    const bool tiled = dot && !e->dot_tiles_off && e->ex.gu.NG <= 64 && e->ex.dn.NG <= 64 && E <= 128;
    if (tiled)
        PK_TRY(pk_launch_group_pairs(sc.sel, P, E, sc.pairs, sc.tiles, sc.tiles + mt,
                                     sc.tiles + 2 * mt, sc.tiles + 3 * mt, e->stream, 4));
    int ps = pk_prof_begin(e, PK_PROF_EXPERT_GATE_UP);
    if (tiled)
        PK_TRY(pk_launch_i4_dot_tiles(gu, tl, e->ex.gu, PK_EPI_SWIGLU, c->swiglu_limit, c->swiglu_alpha, mt,
                                      e->stream));
    else
        PK_TRY(pk_launch_i4_gemv(gu, e->ex.gu, PK_EPI_SWIGLU, c->swiglu_limit, c->swiglu_alpha, nullptr,
                                 e->stream));
    PK_TRY(pk_prof_end(e, ps));
    pk_i4_items dn = pk_expert_items(e, layer, true);
    dn.slots = sc.sel;
    dn.x = sc.act; dn.x_stride = half;
    dn.y = sc.eo; dn.y_stride = D;
    dn.n_items = T * K;
    if (dot) {
        dn.xq = sc.actq; dn.xq_stride = aq_row;
    }
    ps = pk_prof_begin(e, PK_PROF_EXPERT_DOWN);
    if (tiled)
        PK_TRY(pk_launch_i4_dot_tiles(dn, tl, e->ex.dn, PK_EPI_PLAIN, 0.f, 0.f, mt, e->stream));
    else
        PK_TRY(pk_launch_i4_gemv(dn, e->ex.dn, PK_EPI_PLAIN, 0.f, 0.f, nullptr, e->stream));
    PK_TRY(pk_prof_end(e, ps));
    return launch_combine(e, out, residual, sc.eo, sc.w, decode_order ? nullptr : sc.perm, K, D, T);
}

static int moe_rows(pk_engine *e, int layer, const float *x, int T, float *out, const float *residual,
                    bool decode_order = false) {
    PK_TRY(batch_reserve(e, T));
    return moe_rows_on(e, engine_rows_scratch(e), layer, x, T, out, residual, decode_order);
}

static int grouped_reserve(pk_engine *e, int T) {
    const pk_cfg *c = &e->c;
    const int64_t P = (int64_t)T * c->topk;
    if (P <= e->g_cap) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "grouped buffers must be sized before capturing a graph");
    PK_HIP(hipStreamSynchronize(e->stream));
    void *ptrs[] = {e->g_limbs, e->g_exps, e->g_pairs, e->g_tiles};
    for (void *p : ptrs) pk_dev_free(e, p);
    e->g_limbs = nullptr;
    e->g_exps = e->g_pairs = e->g_tiles = nullptr;
    e->g_cap = 0;
    const int64_t plane = std::max((int64_t)T * c->hidden, P * (c->moe_inter / 2));
    const int64_t max_tiles = (P + 31) / 32 + c->n_experts;
    PK_TRY(pk_dev_alloc(e, (void **)&e->g_limbs, 4 * plane));     // 3 int8 planes or 2 half planes
    PK_TRY(pk_dev_alloc(e, (void **)&e->g_exps, std::max((int64_t)T, P) * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->g_pairs, P * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->g_tiles, (5 * max_tiles + 1) * 4));
    e->g_cap = P;
    return PK_OK;
}

// The same MoE as moe_rows on the matrix cores: pairs grouped by expert,
// activations as two halves (hi, lo) on the f16 MFMA over 64-pair tiles, or
// as three int8 limbs over 32-pair tiles (grouped_f16 off), gate_up
// (+SwiGLU) and down as grouped GEMMs (pk_mfma.hip), then the per-token sum
// in the batch's expert order. sel_in / w_in: routing supplied by the caller
// (device [T][K], combine weights already x routed_scale), else the router's.
static int moe_rows_mfma(pk_engine *e, int layer, const float *x, int T, float *out, const float *residual,
                         const int32_t *sel_in, const float *w_in, bool decode_order = false) {
    const pk_cfg *c = &e->c;
    const int D = c->hidden, E = c->n_experts, K = c->topk, half = c->moe_inter / 2;
    const int P = T * K;
    PK_TRY(batch_reserve(e, T));
    PK_TRY(grouped_reserve(e, T));
    if (sel_in) {
        PK_HIP(hipMemcpyAsync(e->b_sel, sel_in, (size_t)P * 4, hipMemcpyDeviceToDevice, e->stream));
        PK_HIP(hipMemcpyAsync(e->b_w, w_in, (size_t)P * 4, hipMemcpyDeviceToDevice, e->stream));
    } else {
        PK_TRY(route_rows(e, engine_rows_scratch(e), layer, x, T, !decode_order));
    }
    if (!decode_order) {
        hipLaunchKernelGGL(k_uniq_perm, dim3(1), dim3(1024), 0, e->stream, e->b_sel, T, K, E, e->b_perm);
        PK_HIP(hipGetLastError());
    }
    const bool f16 = e->grouped_f16;
    const int tile = f16 ? PK_F16_TILE : 32;
    const int max_tiles = (P + tile - 1) / tile + E;           // within the 32-pair tiles' buffer
    int32_t *tile_exp = e->g_tiles, *tile_beg = tile_exp + max_tiles, *tile_cnt = tile_beg + max_tiles;
    int32_t *n_tiles = tile_cnt + max_tiles;
    int32_t *tile_grp = f16 ? n_tiles + 1 : nullptr;            // [2 x max_tiles]
    PK_TRY(pk_launch_group_pairs(e->b_sel, P, E, e->g_pairs, tile_exp, tile_beg, tile_cnt, n_tiles, e->stream,
                                 tile, tile_grp));
    const int64_t plane = std::max((int64_t)T * D, (int64_t)P * half);
    pk_mfma_args a{};
    a.base = e->store;
    a.slot_stride = e->ex.stride;
    a.slot_base = layer * E;
    a.limbs = e->g_limbs;
    a.plane = plane;
    a.xf = reinterpret_cast<const uint16_t *>(e->g_limbs);
    a.fplane = plane;
    uint16_t *xf = reinterpret_cast<uint16_t *>(e->g_limbs);
    a.exps = e->g_exps;
    a.pairs = e->g_pairs;
    a.tile_exp = tile_exp; a.tile_beg = tile_beg; a.tile_cnt = tile_cnt; a.n_tiles = n_tiles;
    a.tile_grp = tile_grp;
    a.lim = c->swiglu_limit;
    a.alpha = c->swiglu_alpha;
    // gate_up + SwiGLU: activation rows are the T tokens
    if (f16) PK_TRY(pk_launch_act_f16(x, D, T, D, xf, plane, e->g_exps, e->stream));
    else PK_TRY(pk_launch_act_limbs(x, D, T, D, e->g_limbs, plane, e->g_exps, 1, e->stream));
    a.off_tiles = e->ex.off_gu_tiles; a.off_scales = e->ex.off_gu_scales; a.off_bias = e->ex.off_gu_bias;
    a.O = c->moe_inter; a.NG = D / 64; a.lrow = D; a.frow = D; a.x_div = K;
    a.y = e->b_act; a.y_stride = half;
    int ps = pk_prof_begin(e, PK_PROF_EXPERT_GATE_UP);
    if (f16) PK_TRY(pk_launch_moe_f16(a, max_tiles, PK_EPI_SWIGLU, e->stream));
    else PK_TRY(pk_launch_moe_mfma(a, max_tiles, PK_EPI_SWIGLU, e->stream));
    PK_TRY(pk_prof_end(e, ps));
    // down: activation rows are the P pairs' SwiGLU outputs
    if (f16) PK_TRY(pk_launch_act_f16(e->b_act, half, P, half, xf, plane, e->g_exps, e->stream));
    else PK_TRY(pk_launch_act_limbs(e->b_act, half, P, half, e->g_limbs, plane, e->g_exps, 1, e->stream));
    a.off_tiles = e->ex.off_dn_tiles; a.off_scales = e->ex.off_dn_scales; a.off_bias = e->ex.off_dn_bias;
    a.O = D; a.NG = half / 64; a.lrow = half; a.frow = half; a.x_div = 1;
    a.y = e->b_eo; a.y_stride = D;
    ps = pk_prof_begin(e, PK_PROF_EXPERT_DOWN);
    if (f16) PK_TRY(pk_launch_moe_f16(a, max_tiles, PK_EPI_PLAIN, e->stream));
    else PK_TRY(pk_launch_moe_mfma(a, max_tiles, PK_EPI_PLAIN, e->stream));
    PK_TRY(pk_prof_end(e, ps));
    return launch_combine(e, out, residual, e->b_eo, e->b_w, decode_order ? nullptr : e->b_perm, K, D, T);
}

extern "C" int pk_moe_forward_grouped(pk_engine *e, int layer, const float *x_dev, int T,
                                      const int32_t *sel_dev, const float *w_dev, float *out_dev,
                                      float *act_dev, float *eo_dev) {
    PK_CHECK(e && x_dev && out_dev && T > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(!sel_dev == !w_dev, PK_ERR_ARG, "sel_dev and w_dev go together");
    PK_TRY(pk_check_layer_experts(e, layer));
    PK_TRY(moe_rows_mfma(e, layer, x_dev, T, out_dev, nullptr, sel_dev, w_dev));
    const pk_cfg *c = &e->c;
    const size_t P = (size_t)T * c->topk;
    if (act_dev)
        PK_HIP(hipMemcpyAsync(act_dev, e->b_act, P * (c->moe_inter / 2) * 4, hipMemcpyDeviceToDevice, e->stream));
    if (eo_dev)
        PK_HIP(hipMemcpyAsync(eo_dev, e->b_eo, P * c->hidden * 4, hipMemcpyDeviceToDevice, e->stream));
    return PK_OK;
}

extern "C" int pk_quantize_act_i8x3(pk_engine *e, const float *x_dev, int rows, int cols, int8_t *limbs_dev,
                                    int32_t *exps_dev) {
    PK_CHECK(e && x_dev && limbs_dev && exps_dev && rows > 0 && cols > 0, PK_ERR_ARG, "bad argument");
    return pk_launch_act_limbs(x_dev, cols, rows, cols, limbs_dev, (int64_t)rows * cols, exps_dev, 0, e->stream);
}

extern "C" int pk_moe_forward_batch(pk_engine *e, int layer, const float *x_dev, int T,
                                    float *out_dev, int32_t *sel_dev, float *w_dev) {
    PK_CHECK(e && x_dev && out_dev && T > 0, PK_ERR_ARG, "bad argument");
    PK_TRY(pk_check_layer_experts(e, layer));
    PK_TRY(moe_rows(e, layer, x_dev, T, out_dev, nullptr));
    const int K = e->c.topk;
    if (sel_dev)
        PK_HIP(hipMemcpyAsync(sel_dev, e->b_sel, (size_t)T * K * 4, hipMemcpyDeviceToDevice, e->stream));
    if (w_dev)
        PK_HIP(hipMemcpyAsync(w_dev, e->b_w, (size_t)T * K * 4, hipMemcpyDeviceToDevice, e->stream));
    return PK_OK;
}

// ───────────── the batched MoE on a fixed device array ─────────────
// For callers that cannot allocate (graph capture, serving loops): the
// scratch of pk_moe_forward_batch_noalloc lives in this file-scope array,
// one copy per GPU for the life of the process. Host code uses the address
// hipGetSymbolAddress returns on each device (pk_noalloc_scratch_init, at
// engine creation), never the array's name.
static __device__ __align__(256) uint8_t scratch[PK_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static uint8_t *g_scratch_dev[PK_NOALLOC_MAX_DEVICES];

int pk_noalloc_scratch_init(pk_engine *e) {
    PK_CHECK(e->device >= 0 && e->device < PK_NOALLOC_MAX_DEVICES, PK_ERR_UNSUPPORTED,
             "device %d: no fixed scratch beyond %d devices", e->device, PK_NOALLOC_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[e->device]) {
        int cur = 0;
        PK_HIP(hipGetDevice(&cur));
        if (cur != e->device) PK_HIP(hipSetDevice(e->device));
        void *p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != e->device) PK_HIP(hipSetDevice(cur));
        PK_CHECK(rc == hipSuccess && p, PK_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", e->device,
                 hipGetErrorString(rc));
        g_scratch_dev[e->device] = (uint8_t *)p;
    }
    e->noalloc_scratch = g_scratch_dev[e->device];
    return PK_OK;
}

// The pieces of rows_scratch for T rows carved from base (256-byte aligned,
// the sizes batch_reserve allocates); returns the bytes used.
static int64_t rows_scratch_carve(pk_engine *e, int T, uint8_t *base, rows_scratch *sc) {
    const pk_cfg *c = &e->c;
    const int64_t TK = (int64_t)T * c->topk;
    int64_t off = 0;
    auto take = [&](int64_t bytes) { uint8_t *p = base ? base + off : nullptr; off = pk_align256(off + bytes); return p; };
    sc->logits = (float *)take((int64_t)T * c->n_experts * 4);
    sc->w = (float *)take(TK * 4);
    sc->sel = (int32_t *)take(TK * 4);
    sc->perm = (int32_t *)take(TK * 4);
    sc->act = (float *)take(TK * (c->moe_inter / 2) * 4);
    sc->eo = (float *)take(TK * c->hidden * 4);
    sc->xq = (int32_t *)take((int64_t)T * ((c->hidden + 31) / 32) * PK_XQ_INTS * 4);
    sc->actq = (int32_t *)take(TK * e->ex.gu.RB * PK_XQ_INTS * 4);
    sc->pairs = (int32_t *)take(TK * 4);
    sc->tiles = (int32_t *)take((3 * (TK / 4 + 1 + c->n_experts) + 1) * 4);
    return off;
}

extern "C" int pk_moe_forward_batch_noalloc(pk_engine *e, int layer, const float *x_dev, int T, float *out_dev,
                                            int32_t *sel_dev, float *w_dev) {
    PK_CHECK(e && x_dev && out_dev && T > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(e->noalloc_scratch, PK_ERR_HIP, "fixed scratch not set up on device %d", e->device);
    PK_CHECK((int64_t)T * e->c.topk <= 65535, PK_ERR_UNSUPPORTED, "batched MoE: %d tokens x top-%d", T, e->c.topk);
    PK_TRY(pk_check_layer_experts(e, layer));
    rows_scratch sc{};
    const int64_t need = rows_scratch_carve(e, T, nullptr, &sc);
    PK_CHECK(need <= PK_NOALLOC_SCRATCH_BYTES, PK_ERR_UNSUPPORTED,
             "moe_forward_batch_noalloc: %d tokens need %lld bytes of scratch, the fixed array holds %lld", T,
             (long long)need, (long long)PK_NOALLOC_SCRATCH_BYTES);
    rows_scratch_carve(e, T, e->noalloc_scratch, &sc);
    PK_TRY(moe_rows_on(e, sc, layer, x_dev, T, out_dev, nullptr, false));
    const int K = e->c.topk;
    if (sel_dev)
        PK_HIP(hipMemcpyAsync(sel_dev, sc.sel, (size_t)T * K * 4, hipMemcpyDeviceToDevice, e->stream));
    if (w_dev)
        PK_HIP(hipMemcpyAsync(w_dev, sc.w, (size_t)T * K * 4, hipMemcpyDeviceToDevice, e->stream));
    return PK_OK;
}

static int prefill_reserve(pk_engine *e, int B) {
    if (B <= e->p_cap) return PK_OK;
    PK_HIP(hipStreamSynchronize(e->stream));
    void *ptrs[] = {e->p_H, e->p_XN, e->p_qkv, e->p_att, e->p_part, e->p_ids};
    for (void *p : ptrs) pk_dev_free(e, p);
    e->p_H = e->p_XN = e->p_qkv = e->p_att = e->p_part = nullptr;
    e->p_ids = nullptr;
    e->p_cap = 0;
    const pk_cfg *c = &e->c;
    const int64_t qkv_dim = (int64_t)(c->n_heads + 2 * c->n_kv_heads) * c->head_dim;
    const int max_chunks = (c->ctx_len + 127) / 128;
    PK_TRY(pk_dev_alloc(e, (void **)&e->p_H, (int64_t)B * c->hidden * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->p_XN, (int64_t)B * c->hidden * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->p_qkv, B * qkv_dim * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->p_att, (int64_t)B * c->n_heads * c->head_dim * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->p_part,
                        (int64_t)B * c->n_heads * max_chunks * (c->head_dim + 2) * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->p_ids, (int64_t)c->ctx_len * 4));
    e->p_cap = B;
    return PK_OK;
}

// forward_prefill (picchio.c:1795-1932) of ids_dev[0..n) at positions
// pos_base..pos_base+n-1; the greedy next token goes to the decode state
// (and to out_toks when given).
static int prefill_chunk(pk_engine *e, int seq, const int32_t *ids_dev, int last_tok, int n, int pos_base,
                         int32_t *out_toks, int out_cap, bool mfma) {
    const pk_cfg *c = &e->c;
    const int D = c->hidden;
    hipLaunchKernelGGL(k_embed_rows, dim3(n), dim3(256), 0, e->stream, ids_dev, e->embed, c->vocab, e->p_H, D);
    PK_HIP(hipGetLastError());
    for (int l = 0; l < c->n_layers; ++l) {
        PK_TRY(pk_launch_rmsnorm(e->p_XN, e->p_H, e->L[l].in_ln, D, c->eps, n, e->stream));
        PK_TRY(pk_attention_rows(e, l, nullptr, pos_base, 1, seq, 0, n, e->p_XN, e->p_qkv, e->p_part, e->p_att,
                                 e->p_H, nullptr, true));
        PK_TRY(pk_launch_rmsnorm(e->p_XN, e->p_H, e->L[l].post_ln, D, c->eps, n, e->stream));
        if (mfma)
            PK_TRY(moe_rows_mfma(e, l, e->p_XN, n, e->p_H, e->p_H, nullptr, nullptr));
        else
            PK_TRY(moe_rows(e, l, e->p_XN, n, e->p_H, e->p_H));
    }
    PK_TRY(pk_launch_rmsnorm(e->hn, e->p_H + (int64_t)(n - 1) * D, e->final_norm, D, c->eps, 1, e->stream));
    PK_TRY(pk_set_state(e, last_tok, pos_base + n - 1));
    return pk_lm_head_step(e, e->hn, nullptr, out_toks, out_cap);
}

int pk_prefill_run(pk_engine *e, int seq, const int32_t *ids, int n, int pos_base, int32_t *out_toks,
                   int out_cap) {
    int batch = 64;
    if (const char *v = getenv("PREFILL_BATCH")) batch = atoi(v);
    if ((batch <= 1 || n <= 1) && seq == 0) {
        for (int i = 0; i < n; ++i) PK_TRY(pk_decode_token(e, ids[i], pos_base + i, out_toks, out_cap));
        return PK_OK;
    }
    if (batch < 1) batch = 1;
    const int B = batch < n ? batch : n;
    // PK_PREFILL_MFMA=1: the chunk's MoE on the grouped matrix-core GEMM
    // (f16 hi/lo activations by default, held to a tolerance; the exact int8
    // limbs with pk_set_grouped_f16 off)
    const char *mv = getenv("PK_PREFILL_MFMA");
    const bool mfma = mv && atoi(mv) != 0;
    PK_TRY(prefill_reserve(e, B));
    PK_TRY(batch_reserve(e, B));
    PK_HIP(hipMemcpyAsync(e->p_ids, ids, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
    // a repetition penalty counts the prompt itself (picchio.c:1960-1967)
    PK_TRY(pk_sample_seed_history(e, e->p_ids, n));
    for (int off = 0; off < n; off += B) {
        const int len = n - off < B ? n - off : B;
        PK_TRY(prefill_chunk(e, seq, e->p_ids + off, ids[off + len - 1], len, pos_base + off, out_toks, out_cap,
                             mfma));
    }
    PK_HIP(hipStreamSynchronize(e->stream));           // ids is the caller's pageable memory
    return PK_OK;
}

extern "C" int pk_prefill_tokens(pk_engine *e, const int32_t *ids, int n, int pos_base, int32_t *next_host) {
    PK_CHECK(e && ids && n > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(pos_base >= 0 && pos_base + n <= e->c.ctx_len, PK_ERR_CONTEXT_FULL,
             "positions %d..%d exceed context %d", pos_base, pos_base + n - 1, e->c.ctx_len);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "prefill_tokens: not available while capturing");
    PK_TRY(pk_check_model(e));
    PK_TRY(pk_decode_reserve(e));
    PK_TRY(pk_prefill_run(e, 0, ids, n, pos_base, nullptr, 0));
    pk_dstate s{};
    PK_HIP(hipMemcpyAsync(&s, e->dstate, sizeof(s), hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    // a one-token prompt runs the fused decode step, whose waits may give up
    bool redo = false;
    PK_TRY(pk_wait_fallback(e, &redo));
    if (redo) return pk_prefill_tokens(e, ids, n, pos_base, next_host);
    if (next_host) *next_host = s.next;
    return PK_OK;
}

// ───────────────────── several independent sequences ─────────────────────

namespace {

// Greedy id of each row of logits [rows][V] (first maximum, picchio.c:1555-1560).
__global__ __launch_bounds__(1024) void k_argmax_rows(const float *logits, int V, int32_t *out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const float *lg = logits + (int64_t)blockIdx.x * V;
    float v = -INFINITY;
    int i = 0x7fffffff;
    // a thread's indices increase: the first maximum within the thread
    auto take = [&](float x, int j) {
        if (x > v) { v = x; i = j; }
    };
    // 16-byte loads, eight in flight per thread (rows are 16-byte aligned when V % 4 == 0)
    const int V4 = (V & 3) == 0 ? V >> 2 : 0;
    const float4 *l4 = reinterpret_cast<const float4 *>(lg);
    constexpr int U = 8;
    for (int j0 = threadIdx.x; j0 < V4; j0 += 1024 * U) {
        float4 q[U];
#pragma unroll
        for (int u = 0; u < U; ++u) q[u] = l4[min(j0 + 1024 * u, V4 - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + 1024 * u;
            if (j < V4) {
                take(q[u].x, 4 * j);
                take(q[u].y, 4 * j + 1);
                take(q[u].z, 4 * j + 2);
                take(q[u].w, 4 * j + 3);
            }
        }
    }
    for (int j = 4 * V4 + (int)threadIdx.x; j < V; j += 1024) take(lg[j], j);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(i, o, 64);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = v; bi[threadIdx.x >> 6] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > v || (bv[w] == v && bi[w] < i)) { v = bv[w]; i = bi[w]; }
        // the reference's scan starts at index 0 and moves on a strictly
        // greater value only: a NaN (or the maximum) at index 0 keeps 0
        out[blockIdx.x] = (i == 0x7fffffff || !(v > lg[0])) ? 0 : i;
    }
}

}  // namespace

extern "C" int pk_batch_reserve(pk_engine *e, int n_seq) {
    PK_CHECK(e && n_seq > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "batch_reserve: not available while capturing");
    if (n_seq <= e->n_seq) return PK_OK;
    PK_HIP(hipStreamSynchronize(e->stream));
    const int64_t bytes = (int64_t)n_seq * e->seq_stride * 4;
    pk_dev_free(e, e->K);
    pk_dev_free(e, e->V);
    e->K = e->V = nullptr;
    e->device_bytes -= 2 * (int64_t)e->n_seq * e->seq_stride * 4;
    if (e->step_exec) {                       // the captured step addresses the old cache
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    e->n_seq = 0;
    PK_TRY(pk_dev_alloc(e, (void **)&e->K, bytes));
    PK_TRY(pk_dev_alloc(e, (void **)&e->V, bytes));
    PK_HIP(hipMemsetAsync(e->K, 0, bytes, e->stream));
    PK_HIP(hipMemsetAsync(e->V, 0, bytes, e->stream));
    e->n_seq = n_seq;
    return PK_OK;
}

extern "C" int pk_kv_fill_synthetic(pk_engine *e, int seq, int n_pos, uint64_t seed) {
    PK_CHECK(e && seq >= 0 && seq < e->n_seq && n_pos >= 0 && n_pos <= e->c.ctx_len, PK_ERR_ARG,
             "kv fill: seq %d / %d positions", seq, n_pos);
    const pk_cfg *c = &e->c;
    const int64_t kv_dim = (int64_t)c->n_kv_heads * c->head_dim;
    for (int l = 0; l < c->n_layers; ++l) {
        const int64_t off = seq * e->seq_stride + (int64_t)l * c->ctx_len * kv_dim;
        const uint64_t s = seed * 0x9E3779B97F4A7C15ull + (uint64_t)(seq * 1024 + l) * 2;
        PK_TRY(pk_launch_fill_normal_k(e->K + off, n_pos, c->ctx_len, c->n_kv_heads, c->head_dim, s, 1.0f,
                                       e->stream));
        PK_TRY(pk_launch_fill_normal(e->V + off, n_pos * kv_dim, s + 1, 1.0f, e->stream));
    }
    return PK_OK;
}

extern "C" int pk_prefill_seq(pk_engine *e, int seq, const int32_t *ids, int n, int pos_base,
                              int32_t *next_host) {
    PK_CHECK(e && ids && n > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(seq >= 0 && seq < e->n_seq, PK_ERR_ARG, "sequence %d of %d", seq, e->n_seq);
    PK_CHECK(pos_base >= 0 && pos_base + n <= e->c.ctx_len, PK_ERR_CONTEXT_FULL,
             "positions %d..%d exceed context %d", pos_base, pos_base + n - 1, e->c.ctx_len);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "prefill_seq: not available while capturing");
    PK_TRY(pk_check_model(e));
    PK_TRY(pk_decode_reserve(e));
    PK_TRY(pk_prefill_run(e, seq, ids, n, pos_base, nullptr, 0));
    pk_dstate s{};
    PK_HIP(hipMemcpyAsync(&s, e->dstate, sizeof(s), hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    // a one-token prompt runs the fused decode step, whose waits may give up
    bool redo = false;
    PK_TRY(pk_wait_fallback(e, &redo));
    if (redo) return pk_prefill_seq(e, seq, ids, n, pos_base, next_host);
    if (next_host) *next_host = s.next;
    return PK_OK;
}

// n_steps greedy forward_token steps of sequences 0..n_seq-1, all at
// positions pos .. pos+n_steps-1: each step embeds the n_seq tokens, runs
// every layer on the n_seq rows at once (weights read once per step), and
// writes the next tokens on the device for the following step.
extern "C" int pk_decode_batch(pk_engine *e, int n_seq, const int32_t *toks_host, int pos, int n_steps,
                               int32_t *out_host) {
    PK_CHECK(e && toks_host && out_host && n_seq > 0 && n_steps > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(n_seq <= e->n_seq, PK_ERR_ARG, "%d sequences, %d reserved (pk_batch_reserve)", n_seq, e->n_seq);
    PK_CHECK(pos >= 0 && pos + n_steps <= e->c.ctx_len, PK_ERR_CONTEXT_FULL, "positions exceed context");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "decode_batch: not available while capturing");
    PK_CHECK(!e->samp_on, PK_ERR_UNSUPPORTED,
             "decode_batch: greedy only (one sampler state is one sequence's history and rng)");
    PK_TRY(pk_check_model(e));
    PK_TRY(pk_decode_reserve(e));
    // the batched projections read the tile-order weight copies
    PK_TRY(pk_dense_tiles(e));
    const pk_cfg *c = &e->c;
    const int D = c->hidden, V = c->vocab;
    PK_TRY(prefill_reserve(e, n_seq));
    PK_TRY(batch_reserve(e, n_seq));
    if (n_seq > e->bd_cap || n_steps + 1 > e->bd_steps) {
        PK_HIP(hipStreamSynchronize(e->stream));
        pk_dev_free(e, e->bd_logits);
        pk_dev_free(e, e->bd_toks);
        e->bd_logits = nullptr;
        e->bd_toks = nullptr;
        e->bd_cap = e->bd_steps = 0;
        PK_TRY(pk_dev_alloc(e, (void **)&e->bd_logits, (int64_t)n_seq * V * 4));
        PK_TRY(pk_dev_alloc(e, (void **)&e->bd_toks, (int64_t)(n_steps + 1) * n_seq * 4));
        e->bd_cap = n_seq;
        e->bd_steps = n_steps + 1;
    }
    // With PK_BATCH_MFMA_MIN=n (n > 0) and at least n sequences the MoE runs
    // on the grouped matrix-core GEMM (pairs grouped by expert; the f16 hi/lo
    // activations by default, the exact int8 limbs with pk_set_grouped_f16
    // off). Off by default: at 32 sequences over 128 experts most experts get
    // one or two pairs, and a 32-pair tile per expert costs more (25.5
    // against 22.3 ms per 120B-shaped step). Without it each row's MoE runs
    // on the integer-dot arithmetic (within 2e-5 of picchio's; the experts of
    // a step grouped by expert), or with PK_I4_DOT_BATCH=0 in the
    // environment at engine creation on forward_token's exact bits.
    int mfma_min = 0;
    if (const char *v = getenv("PK_BATCH_MFMA_MIN")) mfma_min = atoi(v);
    const bool moe_mfma = mfma_min > 0 && n_seq >= mfma_min;
    if (moe_mfma) PK_TRY(grouped_reserve(e, n_seq));
    PK_HIP(hipMemcpyAsync(e->bd_toks, toks_host, (size_t)n_seq * 4, hipMemcpyHostToDevice, e->stream));
    for (int step = 0; step < n_steps; ++step) {
        const int32_t *tk = e->bd_toks + (int64_t)step * n_seq;
        hipLaunchKernelGGL(k_embed_rows, dim3(n_seq), dim3(256), 0, e->stream, tk, e->embed, V, e->p_H, D);
        PK_HIP(hipGetLastError());
        for (int l = 0; l < c->n_layers; ++l) {
            PK_TRY(pk_launch_rmsnorm(e->p_XN, e->p_H, e->L[l].in_ln, D, c->eps, n_seq, e->stream));
            PK_TRY(pk_attention_rows(e, l, nullptr, pos + step, 0, 0, 1, n_seq, e->p_XN, e->p_qkv, e->p_part,
                                     e->p_att, e->p_H));
            PK_TRY(pk_launch_rmsnorm(e->p_XN, e->p_H, e->L[l].post_ln, D, c->eps, n_seq, e->stream));
            if (moe_mfma)
                PK_TRY(moe_rows_mfma(e, l, e->p_XN, n_seq, e->p_H, e->p_H, nullptr, nullptr, true));
            else
                PK_TRY(moe_rows(e, l, e->p_XN, n_seq, e->p_H, e->p_H, true));
        }
        PK_TRY(pk_launch_rmsnorm(e->p_XN, e->p_H, e->final_norm, D, c->eps, n_seq, e->stream));
        const int ps = pk_prof_begin(e, PK_PROF_LM_HEAD);
        if (c->lm_head_fmt == PK_FMT_INT8)
            PK_TRY(pk_launch_gemv_q8(e->bd_logits, e->p_XN, e->lm_q8, e->lm_s, n_seq, D, V, e->stream));
        else
            PK_TRY(pk_launch_gemv_f32(e->bd_logits, e->p_XN, e->lm_f32, nullptr, n_seq, D, V, e->stream,
                                      e->skinny_ws, e->skinny_ws ? PK_SKINNY_WS : 0,
                                      pk_tiles_current(e) ? e->lm_t : nullptr));
        hipLaunchKernelGGL(k_argmax_rows, dim3(n_seq), dim3(1024), 0, e->stream, e->bd_logits, V,
                           e->bd_toks + (int64_t)(step + 1) * n_seq);
        PK_HIP(hipGetLastError());
        PK_TRY(pk_prof_end(e, ps));
    }
    PK_HIP(hipMemcpyAsync(out_host, e->bd_toks + n_seq, (size_t)n_steps * n_seq * 4, hipMemcpyDeviceToHost,
                          e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}
