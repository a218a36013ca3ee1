// pk_moe_seq.hip — one persistent kernel for a sequence of batch-1 MoE steps.
//
// Each MoE step (moe_forward, picchio.c:1309-1466) is split into tasks:
//   router tasks  : one router row each -> logit (picchio.c:1316-1324); the
//                   last one to finish also runs top-k + softmax (:1330-1355)
//   gate_up tasks : (expert k, 64-row block) -> SwiGLU activations (:1399-1424)
//   down tasks    : (expert k, 64-row block) -> expert output rows (:1430-1434)
// and the last down task of a row block combines the top-k outputs in routing
// order (:1445-1454). Workgroups claim tasks in sequence order from an atomic
// counter; a task only waits for tasks claimed before it, so the kernel can
// not deadlock, and every wait is bounded (on timeout an error flag is raised
// and all workgroups drain). Intermediates move between workgroups through
// per-step buffers with device-coherent (sc1) stores/loads, so no L2
// writeback is needed: one launch replaces five kernels per step.
//
// Workgroups are small (5 waves) so several share a CU and cover each
// other's memory latency; down tasks issue their first weight loads before
// waiting for the activations they consume.
//
// With `chain` set, step t+1 starts only after step t is fully combined —
// the dependency of consecutive layers in decode.
#include "pk_engine.h"
#include "pk_i4_device.h"
#include "pk_dev.h"

#include <algorithm>
#include <vector>

namespace {

typedef const __attribute__((address_space(4))) float *cfloat_p;

constexpr int NW = 15;                 // waves per workgroup (45 groups = 15 x 3)
constexpr int RING = 3;                // weight groups in flight per wave
#ifndef PK_SEQ_SLEEP
#define PK_SEQ_SLEEP 100
#endif
constexpr int SLEEP = PK_SEQ_SLEEP;        // s_sleep units (64 cycles) between polls
constexpr uint32_t SPIN_LIMIT = 1u << 20;

struct seq_args {
    const uint8_t *store;
    int64_t slot_stride;
    int64_t off_gu_t, off_gu_s, off_gu_b, off_dn_t, off_dn_s, off_dn_b;
    const float *const *router;        // [L]
    const float *const *router_b;      // [L]
    const int32_t *layer_of;           // [T]
    const float *x;                    // [T][D]
    float *out;                        // [T][D]
    float *logits;                     // [T][E]
    int32_t *sel;                      // [T][K]
    float *w;                          // [T][K] softmax weight * routed_scale
    float *act;                        // [T][K][act_stride]
    float *eo;                         // [T][K][eo_stride]
    uint32_t *ctr;                     // [2 + T * CT]
    int T, E, K, D, half, RB_gu, RB_dn, NG_gu, NG_dn, n_rt, chain;
    int64_t act_stride, eo_stride;
    float lim, alpha, rs;
    uint64_t *trace;                   // optional [tasks][4] timestamps (100 MHz)
};

// Task timeline (tracing): start, dependencies ready, math done, end.
__device__ __forceinline__ void trace_mark(const seq_args &a, int task, int i) {
    if (a.trace && threadIdx.x == 0) a.trace[(int64_t)task * 4 + i] = wall_clock64();
}

__device__ __forceinline__ uint32_t ld_dev(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf_dev(float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ldi_dev(int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stf_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sti_dev(int32_t *p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_dev(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// all memory operations of this wave complete (stores acknowledged)
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

// Thread 0 polls *p until >= target; false on error/timeout (flag raised).
__device__ bool wait_geq(uint32_t *p, uint32_t target, uint32_t *err) {
    for (uint32_t i = 0;; ++i) {
        if (ld_dev(p) >= target) return true;
        if (ld_dev(err) != 0) return false;
        if (i >= SPIN_LIMIT) {
            add_dev(err, 1);
            return false;
        }
        __builtin_amdgcn_s_sleep(SLEEP);
    }
}

// Counters of step t: [router][routed][gu x K][dn x RB_dn][done]
__device__ __forceinline__ uint32_t *c_router(const seq_args &a, int t) {
    return a.ctr + 2 + (int64_t)t * (a.K + a.RB_dn + 3);
}
__device__ __forceinline__ uint32_t *c_routed(const seq_args &a, int t) { return c_router(a, t) + 1; }
__device__ __forceinline__ uint32_t *c_gu(const seq_args &a, int t, int k) { return c_router(a, t) + 2 + k; }
__device__ __forceinline__ uint32_t *c_dn(const seq_args &a, int t, int rb) {
    return c_router(a, t) + 2 + a.K + rb;
}
__device__ __forceinline__ uint32_t *c_done(const seq_args &a, int t) {
    return c_router(a, t) + 2 + a.K + a.RB_dn;
}

// Top-k by repeated argmax (strict '>', lowest index on ties, chosen experts
// skipped; picchio.c:1330-1341) and softmax over the k logits
// (quant.h:406-412), by one wave; lane 0 publishes sel / w of step t.
__device__ void topk_publish(const seq_args &a, int t, float *sv_lds, int *si_lds) {
    const int lane = threadIdx.x & 63;
    float *lg = a.logits + (int64_t)t * a.E;
    const int E = a.E, K = a.K;
    float v0 = lane < E ? ldf_dev(lg + lane) : -INFINITY;
    float v1 = lane + 64 < E ? ldf_dev(lg + lane + 64) : -INFINITY;
    bool t0 = lane >= E, t1 = lane + 64 >= E;
    for (int k = 0; k < K; ++k) {
        float bv = -1e30f;
        int bi = 0x7fffffff;
        if (!t0 && v0 > bv) { bv = v0; bi = lane; }
        if (!t1 && v1 > bv) { bv = v1; bi = lane + 64; }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        // no logit above -1e30 (NaN inputs): the reference leaves -1;
        // here the index stays inside the store
        if (bi >= E) bi = 0;
        if (lane == 0) { si_lds[k] = bi; sv_lds[k] = bv; }
        if (bi == lane) t0 = true;
        if (bi == lane + 64) t1 = true;
    }
    if (lane == 0) {
        float m = -1e30f;
        for (int k = 0; k < K; ++k) if (sv_lds[k] > m) m = sv_lds[k];
        float s = 0.0f;
        for (int k = 0; k < K; ++k) { sv_lds[k] = expf(sv_lds[k] - m); s += sv_lds[k]; }
        for (int k = 0; k < K; ++k) {
            sti_dev(a.sel + (int64_t)t * K + k, si_lds[k]);
            stf_dev(a.w + (int64_t)t * K + k, (sv_lds[k] / s) * a.rs);
        }
    }
    wait_mem();
    if (lane == 0) add_dev(c_routed(a, t), 1);
}

// Router row e (one per workgroup): the row is split over all waves, every
// lane issues its loads before its FMAs, partial sums are reduced in a fixed
// order (fp32, not the reference's sequential order: within 1e-6 relative).
__device__ void router_task(const seq_args &a, int t, int e, float *red, float *sv_lds, int *si_lds,
                            int *flag_lds) {
    constexpr int PER_LANE = 4;                       // columns per lane per pass
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int layer = a.layer_of[t];
    const float *x = a.x + (int64_t)t * a.D;
    const float *row = a.router[layer] + (int64_t)e * a.D;
    float acc = 0.0f;
    for (int c0 = threadIdx.x; c0 < a.D; c0 += NW * 64 * PER_LANE) {
        float xv[PER_LANE], wv[PER_LANE];
#pragma unroll
        for (int u = 0; u < PER_LANE; ++u) {
            const int c = c0 + u * NW * 64;
            xv[u] = c < a.D ? x[c] : 0.0f;
            wv[u] = c < a.D ? row[c] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < PER_LANE; ++u) acc = __builtin_fmaf(xv[u], wv[u], acc);
    }
    acc = pk_wave_sum_f(acc);
    if (lane == 0) red[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = 0.0f;
        for (int w = 0; w < NW; ++w) v += red[w];
        stf_dev(a.logits + (int64_t)t * a.E + e, v + a.router_b[layer][e]);
        wait_mem();
        *flag_lds = (add_dev(c_router(a, t), 1) == (uint32_t)(a.n_rt - 1));
    }
    __syncthreads();
    if (*flag_lds && wave == 0) topk_publish(a, t, sv_lds, si_lds);   // last router task
}

// Tiles of one group for this wave: two 16-byte halves + the row's scale.
struct tile_regs {
    uint4 a, b;
    float s;
};

__device__ __forceinline__ void load_group(const uint4 *tiles, const float *sc, int g, tile_regs &r) {
    const int lane = threadIdx.x & 63;
    r.a = pk_load_nt(&tiles[g * 128 + lane]);
    r.b = pk_load_nt(&tiles[g * 128 + 64 + lane]);
    r.s = sc[g * 64 + lane];
}

// The first RING groups of this wave (wave, wave+NW, ...), issued early.
__device__ __forceinline__ void load_prologue(const uint4 *tiles, const float *sc, int NG,
                                              tile_regs (&r)[RING], int wave) {
#pragma unroll
    for (int u = 0; u < RING; ++u)
        if (wave + NW * u < NG) load_group(tiles, sc, wave + NW * u, r[u]);
}

// Partial sums of this workgroup's 64 rows into LDS, streaming this wave's
// groups (wave, wave+NW, ...) through a RING-deep register ring (RING loads
// always in flight), then wave 0 folds the groups of each row in order (the
// bit-exact order). NG is a compile-time constant so the ring is indexed
// statically. xs: the 64-column activations in LDS (broadcast reads).
template <int NG, typename XP>
__device__ __forceinline__ float i4_rows(const uint4 *tiles, const float *sc, XP xs,
                                         float *part, float *scl, tile_regs (&r)[RING], int wave) {
    const int lane = threadIdx.x & 63;
    constexpr int J = (NG + NW - 1) / NW;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int g = wave + NW * j;
        if (g < NG) {
            const tile_regs cur = r[j % RING];
            if (g + NW * RING < NG) load_group(tiles, sc, g + NW * RING, r[j % RING]);
            part[g * 64 + lane] = pk_group_dot(cur.a, cur.b, xs + g * 64);
            scl[g * 64 + lane] = cur.s;
        }
    }
    __syncthreads();
    float acc = 0.0f;
    if (wave == 0) {
#pragma unroll 9
        for (int g = 0; g < NG; ++g) acc = __builtin_fmaf(part[g * 64 + lane], scl[g * 64 + lane], acc);
    }
    return acc;
}

template <int NG>
__global__ __launch_bounds__(NW * 64) void k_moe_seq(seq_args a) {
    extern __shared__ float lds[];
    __shared__ int s_ok, s_flag, s_slot;
    __shared__ int si[16];
    __shared__ float sv[16];
    float *part = lds;
    float *scl = lds + NG * 64;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t *err = a.ctr + 1;
    const int per_step = a.n_rt + a.K * (a.RB_gu + a.RB_dn);
    // One workgroup per task, block ids in dependency order: a task waits only
    // for tasks with lower block ids, which the dispatcher issues first.
    const int task = blockIdx.x;
    trace_mark(a, task, 0);
    {
        const int t = task / per_step;
        int r = task - t * per_step;

        if (r < a.n_rt) {                                   // ── router
            if (threadIdx.x == 0)
                s_ok = (!a.chain || t == 0) ? 1 : wait_geq(c_done(a, t - 1), a.RB_dn, err);
            __syncthreads();
            trace_mark(a, task, 1);
            if (s_ok) router_task(a, t, r, part, sv, si, &s_flag);
            trace_mark(a, task, 3);
            return;
        }
        r -= a.n_rt;
        const bool is_gu = r < a.K * a.RB_gu;
        if (!is_gu) r -= a.K * a.RB_gu;
        const int RB = is_gu ? a.RB_gu : a.RB_dn;
        const int k = r / RB, rb = r - k * RB;

        if (threadIdx.x == 0) {
            s_ok = wait_geq(c_routed(a, t), 1, err);
            s_slot = a.layer_of[t] * a.E + ldi_dev(a.sel + (int64_t)t * a.K + k);
        }
        __syncthreads();
        trace_mark(a, task, 1);
        if (!s_ok) return;
        const int slot = __builtin_amdgcn_readfirstlane(s_slot);
        const uint8_t *base = a.store + (int64_t)slot * a.slot_stride;
        tile_regs ring[RING];

        if (is_gu) {                                        // ── gate_up + SwiGLU
            const uint4 *tiles = reinterpret_cast<const uint4 *>(base + a.off_gu_t) + (int64_t)rb * NG * 128;
            const float *sc = reinterpret_cast<const float *>(base + a.off_gu_s) + (int64_t)rb * NG * 64;
            load_prologue(tiles, sc, NG, ring, wave);
            // the step input was written before launch: immutable in this
            // kernel, read through the constant address space (scalar loads)
            const cfloat_p x = (cfloat_p)(a.x + (int64_t)t * a.D);
            float v = i4_rows<NG>(tiles, sc, x, part, scl, ring, wave);
            trace_mark(a, task, 2);
            if (wave == 0) {
                const int row = rb * 64 + lane;
                const int O = 2 * a.half;
                if (row < O) v = v + reinterpret_cast<const float *>(base + a.off_gu_b)[row];
                const float up = __shfl_down(v, 1, 64);
                if ((lane & 1) == 0 && row + 1 < O)
                    stf_dev(a.act + ((int64_t)t * a.K + k) * a.act_stride + (row >> 1),
                            pk_swiglu(v, up, a.lim, a.alpha));
                wait_mem();
                if (lane == 0) add_dev(c_gu(a, t, k), 1);
            }
            trace_mark(a, task, 3);
        } else {                                            // ── down + combine
            const uint4 *tiles = reinterpret_cast<const uint4 *>(base + a.off_dn_t) + (int64_t)rb * NG * 128;
            const float *sc = reinterpret_cast<const float *>(base + a.off_dn_s) + (int64_t)rb * NG * 64;
            load_prologue(tiles, sc, NG, ring, wave);       // in flight during the wait
            if (threadIdx.x == 0) s_ok = wait_geq(c_gu(a, t, k), a.RB_gu, err);
            __syncthreads();
            trace_mark(a, task, 1);
            if (!s_ok) return;
            // Activations of expert k, written by other workgroups with
            // device-coherent stores. This step's buffer was never read
            // before in this launch, so no cache holds a stale copy and
            // scalar loads see the stored values. The empty asm makes the
            // pointer opaque so the loads cannot be hoisted above the wait.
            const float *act = a.act + ((int64_t)t * a.K + k) * a.act_stride;
            asm volatile("" : "+s"(act));
            float v = i4_rows<NG>(tiles, sc, (cfloat_p)act, part, scl, ring, wave);
            trace_mark(a, task, 2);
            if (wave == 0) {
                const int row = rb * 64 + lane;
                if (row < a.D) {
                    v = v + reinterpret_cast<const float *>(base + a.off_dn_b)[row];
                    stf_dev(a.eo + ((int64_t)t * a.K + k) * a.eo_stride + row, v);
                }
                wait_mem();
                uint32_t arrived = 0;
                if (lane == 0) arrived = add_dev(c_dn(a, t, rb), 1);
                arrived = __shfl(arrived, 0, 64);
                if (arrived == (uint32_t)(a.K - 1)) {        // last expert of this row block
                    if (row < a.D) {
                        float o = 0.0f;
                        for (int kk = 0; kk < a.K; ++kk)
                            o = __builtin_fmaf(ldf_dev(a.w + (int64_t)t * a.K + kk),
                                               ldf_dev(a.eo + ((int64_t)t * a.K + kk) * a.eo_stride + row), o);
                        stf_dev(a.out + (int64_t)t * a.D + row, o);
                    }
                    wait_mem();
                    if (lane == 0) add_dev(c_done(a, t), 1);
                }
            }
            trace_mark(a, task, 3);
        }
    }
}

__global__ void k_zero_u32(uint32_t *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

// ───────────────────────── host side ─────────────────────────

// GPT-OSS shapes: hidden 2880 and moe_inter/2 2880 are both 45 groups of 64.
static constexpr int kSeqNG = 45;

static int seq_reserve(pk_engine *e, int T) {
    const pk_cfg *c = &e->c;
    if (T <= e->seq_cap && e->seq_ready) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "sequence buffers must be sized before capturing a graph");
    PK_HIP(hipStreamSynchronize(e->stream));
    void *ptrs[] = {e->s_logits, e->s_act, e->s_eo, e->s_ctr, e->s_sel, e->s_w};
    for (void *p : ptrs) pk_dev_free(e, p);
    e->s_logits = e->s_act = e->s_eo = e->s_w = nullptr;
    e->s_ctr = nullptr;
    e->s_sel = nullptr;
    e->seq_cap = 0;
    const int K = c->topk;
    const int RB_dn = e->ex.dn.RB;
    e->s_act_stride = pk_align256((int64_t)(c->moe_inter / 2) * 4) / 4;
    e->s_eo_stride = pk_align256((int64_t)c->hidden * 4) / 4;
    PK_TRY(pk_dev_alloc(e, (void **)&e->s_logits, pk_align256((int64_t)T * c->n_experts * 4)));
    PK_TRY(pk_dev_alloc(e, (void **)&e->s_sel, pk_align256((int64_t)T * K * 4)));
    PK_TRY(pk_dev_alloc(e, (void **)&e->s_w, pk_align256((int64_t)T * K * 4)));
    PK_TRY(pk_dev_alloc(e, (void **)&e->s_act, (int64_t)T * K * e->s_act_stride * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->s_eo, (int64_t)T * K * e->s_eo_stride * 4));
    e->s_ctr_n = 2 + (int64_t)T * (K + RB_dn + 3);
    PK_TRY(pk_dev_alloc(e, (void **)&e->s_ctr, e->s_ctr_n * 4));
    e->seq_cap = T;
    e->seq_ready = true;
    return PK_OK;
}

int pk_refresh_router_table(pk_engine *e) {
    const pk_cfg *c = &e->c;
    if (!e->router_tab) {
        PK_TRY(pk_dev_alloc(e, (void **)&e->router_tab, (int64_t)2 * c->n_layers * sizeof(void *)));
    }
    std::vector<const float *> tab(2 * c->n_layers);
    for (int l = 0; l < c->n_layers; ++l) {
        tab[l] = e->L[l].router;
        tab[c->n_layers + l] = e->L[l].router_b;
    }
    PK_HIP(hipMemcpy(e->router_tab, tab.data(), tab.size() * sizeof(void *), hipMemcpyHostToDevice));
    e->router_tab_dirty = false;
    return PK_OK;
}

extern "C" int pk_moe_forward_seq(pk_engine *e, const int32_t *layers_dev, const float *x_dev, int T,
                                  float *out_dev, int chain) {
    PK_CHECK(e && layers_dev && x_dev && out_dev && T > 0, PK_ERR_ARG, "bad argument");
    const pk_cfg *c = &e->c;
    for (int l = 0; l < c->n_layers; ++l) {
        PK_CHECK(e->L[l].have_router, PK_ERR_MISSING, "layer %d: router not loaded", l);
        for (int x = 0; x < c->n_experts; ++x)
            PK_CHECK(e->expert_ready[(int64_t)l * c->n_experts + x], PK_ERR_MISSING,
                     "layer %d expert %d not loaded", l, x);
    }
    if (e->router_tab_dirty || !e->router_tab) {
        PK_CHECK(!e->capturing, PK_ERR_ARG, "router table must be built before capturing a graph");
        PK_TRY(pk_refresh_router_table(e));
    }
    PK_CHECK(e->ex.gu.NG == kSeqNG && e->ex.dn.NG == kSeqNG, PK_ERR_UNSUPPORTED,
             "persistent MoE kernel is built for hidden = moe_inter/2 = %d (use pk_moe_forward)",
             kSeqNG * 64);
    PK_TRY(seq_reserve(e, T));
    seq_args a{};
    a.store = e->store;
    a.slot_stride = e->ex.stride;
    a.off_gu_t = e->ex.off_gu_tiles; a.off_gu_s = e->ex.off_gu_scales; a.off_gu_b = e->ex.off_gu_bias;
    a.off_dn_t = e->ex.off_dn_tiles; a.off_dn_s = e->ex.off_dn_scales; a.off_dn_b = e->ex.off_dn_bias;
    a.router = (const float *const *)e->router_tab;
    a.router_b = (const float *const *)e->router_tab + c->n_layers;
    a.layer_of = layers_dev;
    a.x = x_dev; a.out = out_dev;
    a.logits = e->s_logits; a.sel = e->s_sel; a.w = e->s_w;
    a.act = e->s_act; a.eo = e->s_eo; a.ctr = e->s_ctr;
    a.T = T; a.E = c->n_experts; a.K = c->topk; a.D = c->hidden; a.half = c->moe_inter / 2;
    a.RB_gu = e->ex.gu.RB; a.RB_dn = e->ex.dn.RB; a.NG_gu = e->ex.gu.NG; a.NG_dn = e->ex.dn.NG;
    a.n_rt = c->n_experts;                  // one router row per workgroup
    a.chain = chain ? 1 : 0;
    a.act_stride = e->s_act_stride; a.eo_stride = e->s_eo_stride;
    a.lim = c->swiglu_limit; a.alpha = c->swiglu_alpha; a.rs = c->routed_scale;
    a.trace = e->seq_trace;
    const int64_t total = (int64_t)T * (a.n_rt + a.K * (a.RB_gu + a.RB_dn));
    PK_CHECK(total < (int64_t)1 << 30, PK_ERR_ARG, "sequence too long (%lld tasks)", (long long)total);
    hipLaunchKernelGGL(k_zero_u32, dim3((unsigned)((e->s_ctr_n + 255) / 256)), dim3(256), 0, e->stream,
                       e->s_ctr, e->s_ctr_n);
    PK_HIP(hipGetLastError());
    const int grid = (int)total;
    const size_t lds = (size_t)kSeqNG * 64 * 2 * sizeof(float);
    int ps = pk_prof_begin(e, PK_PROF_MOE_SEQ);
    hipLaunchKernelGGL(k_moe_seq<kSeqNG>, dim3(grid), dim3(NW * 64), lds, e->stream, a);
    PK_HIP(hipGetLastError());
    PK_TRY(pk_prof_end(e, ps));
    return PK_OK;
}

extern "C" int pk_moe_seq_trace(pk_engine *e, uint64_t *trace_dev) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    e->seq_trace = trace_dev;
    return PK_OK;
}

extern "C" int pk_moe_seq_reserve(pk_engine *e, int T) {
    PK_CHECK(e && T > 0, PK_ERR_ARG, "bad argument");
    return seq_reserve(e, T);
}

extern "C" int pk_moe_seq_status(pk_engine *e) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "status read while capturing");
    if (!e->s_ctr) return PK_OK;
    uint32_t flag = 0;
    PK_HIP(hipMemcpyAsync(&flag, e->s_ctr + 1, 4, hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    PK_CHECK(flag == 0, PK_ERR_HIP, "moe sequence kernel: a dependency wait timed out (%u)", flag);
    return PK_OK;
}
