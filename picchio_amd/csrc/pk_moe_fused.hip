// pk_moe_fused.hip — one batch-1 MoE layer (moe_forward, picchio.c:1309-1466)
// in a single launch.
//
// Grid: K x RB_gu workgroups of 15 waves. Workgroup w owns gate_up row block
// w % RB_gu of the (w / RB_gu)-th routed expert and, when w % RB_gu < RB_dn,
// the down row block of the same index of that expert.
//
//  1. router: workgroups w, w + G, ... < E compute logit w with
//     k_router_topk's per-thread order and tree (same bits), store it
//     device-coherently and count themselves in. Meanwhile every workgroup
//     stages its input row in LDS (normalised there when rmsnorm is fused,
//     with the same double reduction as k_rmsnorm).
//  2. every workgroup waits for the E logits and runs top-k + softmax itself
//     (k_router_topk's arithmetic), so routing costs one round trip.
//  3. gate_up: its 64-row block's groups are loaded (3 per wave), summed
//     with quant.h's eight chains and folded in group order exactly as
//     k_i4_gemv; bias; clamped SwiGLU; activations go out device-coherently
//     and the expert's arrival counter is bumped.
//  4. down: the workgroup loads its down row block's weights, waits until
//     all RB_gu gate_up blocks of its expert have arrived, stages the
//     activations in LDS, folds, and stores its rows device-coherently.
//  5. combine: the last of the K down blocks of a row block adds them in
//     routing order, out = fma(w_k, eo_k, out), then the residual (as the
//     COMBINE epilogue of k_i4_gemv); the last combine re-arms the counters.
//
// Results are bit-identical to the three-launch path (router, gate_up,
// down+combine). Waits only target workgroups that are resident together:
// the launcher checks that the whole grid fits on the device at once, and
// every wait is bounded — on timeout an error flag is raised, every
// workgroup drains, and pk_engine_status reports and clears it.
#include "pk_engine.h"
#include "pk_dev.h"
#include "pk_i4_device.h"

namespace {

constexpr int NW = 15;                    // waves per workgroup
constexpr int GPW = 3;                    // groups per wave per pass (45 = 15 x 3)
constexpr int NTHR = NW * 64;
constexpr int KMAX = 16;
constexpr uint32_t SPIN_LIMIT = 1u << 20; // polls before a wait gives up

// counter block (uint32): [router arrivals][combines done][error][gate_up
// arrivals x K][combine arrivals x RB_dn]
constexpr int FC_ROUTER = 0, FC_DONE = 1, FC_ERR = 2, FC_GU = 3;

struct fused_args {
    const uint8_t *store;
    int64_t slot_stride;
    int32_t off_gu_t, off_gu_s, off_gu_b, off_dn_t, off_dn_s, off_dn_b;   // inside a slot
    int32_t slot_base;                    // layer * n_experts
    const float *R, *Rb;                  // router [E][D], bias [E]
    const float *x;                       // input row (raw residual row when nw)
    const float *nw;                      // optional rmsnorm weight
    float eps;
    const float *residual;                // optional: out = residual + moe
    float *out;
    float *logits;                        // [E] exchange
    int32_t *sel;                         // [K] routing results for callers
    float *w_scaled, *w_soft;             // [K]
    float *act;                           // [K][half] exchange
    float *eo;                            // [K][D] exchange
    uint32_t *ctr;
    uint64_t *trace;                      // optional [grid][6] timestamps (100 MHz)
    int E, K, D, half, RB_gu, RB_dn, NG_gu, NG_dn;
    float lim, alpha, rs;
};

__device__ __forceinline__ uint32_t ld_u(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_f(float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_u(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ void mark(const fused_args &a, int i) {
    if (a.trace && threadIdx.x == 0) a.trace[(int64_t)blockIdx.x * 6 + i] = wall_clock64();
}

// Thread 0 polls *p until it reaches target; false on timeout or when
// another workgroup raised the error flag.
__device__ bool wait_geq(uint32_t *p, uint32_t target, uint32_t *err) {
    for (uint32_t i = 0;; ++i) {
        if (ld_u(p) >= target) return true;
        if (ld_u(err) != 0) return false;
        if (i >= SPIN_LIMIT) {
            add_u(err, 1);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// One 64-row block's groups (NG <= NW * GPW): wave w takes groups w, w + NW,
// w + 2 NW. load_groups issues the loads, group_partials writes the per-group
// sums and scales to LDS once x is there.
struct blk {
    uint4 a[GPW], b[GPW];
    float s[GPW];
};

__device__ __forceinline__ void load_groups(blk &w, const uint4 *tiles, const float *sc, int NG, int wave,
                                            int lane) {
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        const int g = wave + u * NW;
        if (g < NG) {
            w.a[u] = pk_load_nt(&tiles[g * 128 + lane]);
            w.b[u] = pk_load_nt(&tiles[g * 128 + 64 + lane]);
            w.s[u] = sc[g * 64 + lane];
        }
    }
}

__device__ __forceinline__ void group_partials(const blk &w, const float *xs, float *part, float *scl, int NG,
                                               int wave, int lane) {
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        const int g = wave + u * NW;
        if (g < NG) {
            part[g * 64 + lane] = pk_group_dot(w.a[u], w.b[u], xs + g * 64);
            scl[g * 64 + lane] = w.s[u];
        }
    }
}

// 8 waves per SIMD: two workgroups per CU, so K x RB_gu = 360 fit on 256 CUs
__global__ __launch_bounds__(NTHR, 8) void k_moe_fused(fused_args a) {
    extern __shared__ float lds[];
    const int NGm = max(a.NG_gu, a.NG_dn);
    float *part = lds;                    // [NGm][64]
    float *scl = part + NGm * 64;         // [NGm][64]
    float *xs = scl + NGm * 64;           // [max(D, half)]
    __shared__ float red[4];
    __shared__ double npart[4];
    __shared__ int ok;
    __shared__ int si[KMAX];
    __shared__ float sw[KMAX];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = gridDim.x;
    const int wg = blockIdx.x;
    const int D = a.D;
    const int n4 = D >> 2;
    uint32_t *err = a.ctr + FC_ERR;
    mark(a, 0);

    // ── 1. router rows (their loads go out before the norm reduction) ──
    constexpr int U = 4;                  // float4 per thread per chunk (k_router_topk's GEMV_U)
    float4 wf[U];
    const bool router = wg < a.E;
    if (router && tid < 256) {
        const float4 *w4 = reinterpret_cast<const float4 *>(a.R + (int64_t)wg * D);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = tid + u * 256;
            wf[u] = i < n4 ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float rn = 1.0f;
    if (a.nw) {
        if (tid < 256) {
            double acc = 0.0;
            for (int i = tid; i < D; i += 256) acc += (double)a.x[i] * (double)a.x[i];
            acc = pk_dev_wave_sum_d(acc);
            if (lane == 0) npart[wave] = acc;
        }
        __syncthreads();
        const double ms = (npart[0] + npart[1]) + (npart[2] + npart[3]);
        rn = 1.0f / sqrtf((float)(ms / D) + a.eps);
        for (int i = tid; i < D; i += NTHR) xs[i] = a.x[i] * rn * a.nw[i];
    } else {
        for (int i = tid; i < D; i += NTHR) xs[i] = a.x[i];
    }
    __syncthreads();
    for (int r = wg; r < a.E; r += G) {
        const float4 *w4 = reinterpret_cast<const float4 *>(a.R + (int64_t)r * D);
        const float4 *x4 = reinterpret_cast<const float4 *>(xs);
        float acc = 0.0f;
        if (tid < 256) {
            for (int i0 = tid; i0 < n4; i0 += 256 * U) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int i = i0 + u * 256;
                    if (r != wg || i0 != tid) wf[u] = i < n4 ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int i = i0 + u * 256;
                    const float4 xv = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                    acc = __builtin_fmaf(xv.x, wf[u].x, acc);
                    acc = __builtin_fmaf(xv.y, wf[u].y, acc);
                    acc = __builtin_fmaf(xv.z, wf[u].z, acc);
                    acc = __builtin_fmaf(xv.w, wf[u].w, acc);
                }
            }
            for (int i = (n4 << 2) + tid; i < D; i += 256)
                acc = __builtin_fmaf(xs[i], a.R[(int64_t)r * D + i], acc);
            acc = wave_sum(acc);
            if (lane == 0) red[wave] = acc;
        }
        __syncthreads();
        if (tid == 0) {
            const float v = (red[0] + red[1]) + (red[2] + red[3]);
            st_f(a.logits + r, v + a.Rb[r]);
            __builtin_amdgcn_s_waitcnt(0);
            add_u(a.ctr + FC_ROUTER, 1u);
        }
        __syncthreads();
    }

    // ── 2. wait for the E logits; top-k + softmax in every workgroup ──
    if (tid == 0) ok = wait_geq(a.ctr + FC_ROUTER, (uint32_t)a.E, err);
    __syncthreads();
    if (!ok) return;
    mark(a, 1);
    if (wave == 0) {
        const int E = a.E, K = a.K;
        float v0 = lane < E ? ld_f(a.logits + lane) : -INFINITY;
        float v1 = lane + 64 < E ? ld_f(a.logits + lane + 64) : -INFINITY;
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
            if (lane == 0) { si[k] = bi; sw[k] = bv; }
            if (bi == lane) t0 = true;
            if (bi == lane + 64) t1 = true;
        }
        if (lane == 0) {
            float m = -1e30f;
            for (int k = 0; k < K; ++k) if (sw[k] > m) m = sw[k];
            float s = 0.0f;
            for (int k = 0; k < K; ++k) { sw[k] = expf(sw[k] - m); s += sw[k]; }
            for (int k = 0; k < K; ++k) {
                const float p = sw[k] / s;
                sw[k] = p * a.rs;
                if (wg == 0) {
                    a.sel[k] = si[k];
                    if (a.w_soft) a.w_soft[k] = p;
                    a.w_scaled[k] = p * a.rs;
                }
            }
        }
    }
    __syncthreads();

    // ── 3. gate_up row block of expert k ──
    const int k = wg / a.RB_gu;
    if (k >= a.K) return;
    const int rbg = wg - k * a.RB_gu;
    const int slot = __builtin_amdgcn_readfirstlane(a.slot_base + si[k]);
    const uint8_t *base = a.store + (int64_t)slot * a.slot_stride;
    {
        blk gw;
        load_groups(gw, reinterpret_cast<const uint4 *>(base + a.off_gu_t) + rbg * a.NG_gu * 128,
                    reinterpret_cast<const float *>(base + a.off_gu_s) + rbg * a.NG_gu * 64, a.NG_gu, wave, lane);
        group_partials(gw, xs, part, scl, a.NG_gu, wave, lane);
    }
    __syncthreads();
    const bool has_dn = rbg < a.RB_dn;
    const int O_gu = 2 * a.half;
    if (wave == 0) {
        float acc = 0.0f;
        for (int g = 0; g < a.NG_gu; ++g) acc = __builtin_fmaf(part[g * 64 + lane], scl[g * 64 + lane], acc);
        const int row = rbg * 64 + lane;
        if (row < O_gu) acc = acc + reinterpret_cast<const float *>(base + a.off_gu_b)[row];
        const float up = __shfl_down(acc, 1, 64);
        if ((lane & 1) == 0 && row + 1 < O_gu)
            st_f(a.act + (int64_t)k * a.half + (row >> 1), pk_swiglu(acc, up, a.lim, a.alpha));
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0) add_u(a.ctr + FC_GU + k, 1u);
    }
    mark(a, 2);
    if (!has_dn) return;

    // ── 4. down row block: weights in flight while the activations complete ──
    const int rbd = rbg;
    blk dw;
    load_groups(dw, reinterpret_cast<const uint4 *>(base + a.off_dn_t) + rbd * a.NG_dn * 128,
                reinterpret_cast<const float *>(base + a.off_dn_s) + rbd * a.NG_dn * 64, a.NG_dn, wave, lane);
    if (tid == 0) ok = wait_geq(a.ctr + FC_GU + k, (uint32_t)a.RB_gu, err);
    __syncthreads();
    if (!ok) return;
    mark(a, 3);
    {
        float *src = a.act + (int64_t)k * a.half;
        for (int i0 = tid; i0 < a.half; i0 += NTHR * 4) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * NTHR;
                v[u] = i < a.half ? ld_f(src + i) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * NTHR;
                if (i < a.half) xs[i] = v[u];
            }
        }
    }
    __syncthreads();
    group_partials(dw, xs, part, scl, a.NG_dn, wave, lane);
    __syncthreads();
    if (wave != 0) return;
    float acc = 0.0f;
    for (int g = 0; g < a.NG_dn; ++g) acc = __builtin_fmaf(part[g * 64 + lane], scl[g * 64 + lane], acc);
    const int row = rbd * 64 + lane;
    if (row < D) {
        acc = acc + reinterpret_cast<const float *>(base + a.off_dn_b)[row];
        st_f(a.eo + (int64_t)k * D + row, acc);
    }
    __builtin_amdgcn_s_waitcnt(0);
    mark(a, 4);

    // ── 5. combine: the last of the K down blocks of this row block ──
    uint32_t arrived = 0;
    if (lane == 0) arrived = add_u(a.ctr + FC_GU + a.K + rbd, 1u);
    arrived = __shfl(arrived, 0, 64);
    if (arrived != (uint32_t)(a.K - 1)) return;
    if (row < D) {
        float o = 0.0f;
        for (int j0 = 0; j0 < a.K; j0 += 4) {
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = j0 + j < a.K ? ld_f(a.eo + (int64_t)(j0 + j) * D + row) : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (j0 + j < a.K) o = __builtin_fmaf(sw[j0 + j], v[j], o);
        }
        a.out[row] = a.residual ? a.residual[row] + o : o;
    }
    if (lane == 0) {
        st_u(a.ctr + FC_GU + a.K + rbd, 0u);
        // every workgroup has passed its waits once all row blocks combined
        if (add_u(a.ctr + FC_DONE, 1u) == (uint32_t)(a.RB_dn - 1)) {
            st_u(a.ctr + FC_ROUTER, 0u);
            for (int j = 0; j < a.K; ++j) st_u(a.ctr + FC_GU + j, 0u);
            st_u(a.ctr + FC_DONE, 0u);
        }
    }
    mark(a, 5);
}

size_t fused_lds(const pk_engine *e) {
    const int NGm = std::max(e->ex.gu.NG, e->ex.dn.NG);
    const int XM = std::max(e->c.hidden, e->c.moe_inter / 2);
    return ((size_t)NGm * 64 * 2 + XM) * sizeof(float);
}

}  // namespace

// Whether the single-launch layer applies: shapes it covers and a grid that
// is resident all at once (the waits depend on it).
bool pk_moe_fused_fits(pk_engine *e) {
    if (e->fused_fit >= 0) return e->fused_fit != 0;
    const pk_cfg *c = &e->c;
    const pk_expert_layout &ex = e->ex;
    bool fit = c->topk <= KMAX && c->n_experts <= 128 && (c->hidden & 3) == 0 &&
               ex.dn.RB <= ex.gu.RB && ex.gu.NG <= NW * GPW && ex.dn.NG <= NW * GPW &&
               ex.stride < ((int64_t)1 << 31) &&
               ex.gu.NG * 64 == c->hidden && ex.dn.NG * 64 == c->moe_inter / 2 &&
               FC_GU + c->topk + ex.dn.RB <= PK_CTR_ATTN - PK_CTR_FUSED;
    const size_t lds = fused_lds(e);
    fit = fit && lds + 512 <= 65536;
    if (fit) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_fused, NTHR, lds) != hipSuccess)
            per_cu = 0;
        (void)hipGetLastError();
        const int64_t grid = (int64_t)c->topk * ex.gu.RB;
        fit = per_cu > 0 && grid <= (int64_t)per_cu * e->n_cu;
        e->fused_occ = per_cu;
    }
    e->fused_fit = fit ? 1 : 0;
    return fit;
}

int pk_moe_fused_launch(pk_engine *e, int layer, const float *x, float *out, const float *residual,
                        const float *norm_w) {
    const pk_cfg *c = &e->c;
    const pk_layer_dev &d = e->L[layer];
    PK_CHECK(pk_moe_fused_fits(e), PK_ERR_UNSUPPORTED, "single-launch MoE layer does not fit this shape");
    PK_CHECK(((uintptr_t)d.router & 15) == 0 && ((uintptr_t)x & 15) == 0, PK_ERR_UNSUPPORTED,
             "moe layer: needs 16-byte aligned rows");
    fused_args a{};
    a.store = e->store;
    a.slot_stride = e->ex.stride;
    a.off_gu_t = e->ex.off_gu_tiles;
    a.off_gu_s = e->ex.off_gu_scales;
    a.off_gu_b = e->ex.off_gu_bias;
    a.off_dn_t = e->ex.off_dn_tiles;
    a.off_dn_s = e->ex.off_dn_scales;
    a.off_dn_b = e->ex.off_dn_bias;
    a.slot_base = layer * c->n_experts;
    a.R = d.router;
    a.Rb = d.router_b;
    a.x = x;
    a.nw = norm_w;
    a.eps = c->eps;
    a.residual = residual;
    a.out = out;
    a.logits = e->r_logits;
    a.sel = e->sel;
    a.w_scaled = e->w_scaled;
    a.w_soft = e->w_soft;
    a.act = e->act;
    a.eo = e->eo;
    a.ctr = e->counters + PK_CTR_FUSED;
    a.trace = e->fused_trace;
    a.E = c->n_experts;
    a.K = c->topk;
    a.D = c->hidden;
    a.half = c->moe_inter / 2;
    a.RB_gu = e->ex.gu.RB;
    a.RB_dn = e->ex.dn.RB;
    a.NG_gu = e->ex.gu.NG;
    a.NG_dn = e->ex.dn.NG;
    a.lim = c->swiglu_limit;
    a.alpha = c->swiglu_alpha;
    a.rs = c->routed_scale;
    const int grid = c->topk * e->ex.gu.RB;
    hipLaunchKernelGGL(k_moe_fused, dim3(grid), dim3(NTHR), fused_lds(e), e->stream, a);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

extern "C" int pk_set_moe_fused(pk_engine *e, int on) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    if (on && !pk_moe_fused_fits(e)) {
        pk_set_error("single-launch MoE layer: shape or occupancy does not allow it "
                     "(%d workgroups per CU)", e->fused_occ);
        return PK_ERR_UNSUPPORTED;
    }
    e->moe_fused = on != 0;
    return PK_OK;
}

extern "C" int pk_moe_fused_trace(pk_engine *e, uint64_t *trace_dev) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    e->fused_trace = trace_dev;
    return PK_OK;
}

extern "C" int pk_engine_status(pk_engine *e) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "status read while capturing");
    if (!e->counters) return PK_OK;
    uint32_t flag = 0;
    PK_HIP(hipMemcpyAsync(&flag, e->counters + PK_CTR_FUSED + FC_ERR, 4, hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    if (flag == 0) return PK_OK;
    // re-arm: counters of the single-launch layer and the flag
    PK_HIP(hipMemsetAsync(e->counters + PK_CTR_FUSED, 0, (size_t)(PK_CTR_ATTN - PK_CTR_FUSED) * 4, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    pk_set_error("MoE layer kernel: a dependency wait timed out (%u); its outputs are invalid", flag);
    return PK_ERR_HIP;
}
