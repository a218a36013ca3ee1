// pk_moe_fused.hip — one batch-1 MoE layer (moe_forward, picchio.c:1309-1466)
// in a single launch, its work spread evenly over the compute units.
//
// One workgroup per CU, 16 waves. Waves 0..14 load and multiply weights (3 of
// the 45 column groups of a 64-row block each); wave 15 steers: routing,
// dependency waits, the in-order folds, epilogues and the combine. The
// steering wave issues no weight loads, so waiting for its own stores never
// waits for weights in flight.
//
// A token's work is K x RB_gu gate_up blocks followed by K x RB_dn down
// blocks (540 blocks of 64 rows at top-4 of the 20B / 120B shapes);
// workgroup w takes blocks w, w + G, w + 2G (two or three per CU on 256
// CUs), gate_up before down.
//
//  1. router: workgroups w, w + G, ... < E compute logit w with
//     k_router_topk's per-thread order and tree (same bits) and publish it as
//     a tagged 64-bit slot. With rmsnorm fused every workgroup meanwhile
//     writes its own normalised copy of the row (k_rmsnorm's double
//     reduction, same bits) for its gate_up blocks.
//  2. the steering wave waits for the E slots and runs top-k + softmax with
//     k_router_topk's arithmetic.
//  3. every math wave keeps one block of weights in flight: after the sums
//     of its group u of block j it issues the loads of group u of block j+1,
//     so data arrives progressively and the math overlaps it.
//  4. per block, the math waves write the per-group sums (quant.h's eight
//     chains) into one of two LDS buffers while the steering wave folds the
//     previous block in group order, adds the bias and either applies the
//     clamped SwiGLU (gate_up: activations stored device-coherently, the
//     expert's counter bumped) or stores the expert's rows (down: the last of
//     the K down blocks of a row block adds them in routing order,
//     out = fma(w_k, eo_k, out), then the residual). Before a down block the
//     steering wave publishes every earlier block of its own workgroup and
//     then waits for all gate_up blocks of that expert, so no wait closes a
//     cycle.
//  5. the last combine re-arms the slots and counters.
//
// Control memory is laid out against hot spots: the router slots are
// replicated 8 times (a workgroup polls replica w % 8) and every counter that
// is polled sits in its own 4 KiB page.
//
// The weight math reads its input row with scalar loads (the same code as
// k_i4_gemv): for gate_up the kernel's input row, or the workgroup's own
// normalised copy; for a down block the expert's activations, which the
// workgroup copies after the wait (one batch of device-coherent loads) into
// a private row that no scalar load has touched in this launch. Each copy is
// written by the workgroup's own stores before a barrier, and the pointer is
// made opaque after it, so no load is hoisted above and the scalar loads see
// the stored values.
//
// Results are bit-identical to the three-launch path (router, gate_up,
// down+combine). Waits only target workgroups that are resident together
// (the launcher checks that the whole grid fits at once) and every wait is
// bounded: on timeout an error flag is raised, every workgroup drains, and
// pk_engine_status reports and clears it.
#include "pk_engine.h"
#include "pk_dev.h"
#include "pk_i4_device.h"

#include <algorithm>

namespace {

constexpr int NW = 16;                    // waves per workgroup
constexpr int NMATH = 15;                 // weight waves; wave 15 steers
constexpr int GPW = 3;                    // groups per weight wave (45 = 15 x 3)
constexpr int NTHR = NW * 64;
constexpr int STEER = NMATH * 64;         // first thread of the steering wave
constexpr int KMAX = 16;
constexpr int MAXB = 3;                   // blocks per workgroup
constexpr uint32_t SPIN_LIMIT = 1u << 20; // polls before a wait gives up

// control block (bytes): router slot replica r at r * 4096 (uint64 [E],
// (tag << 32) | logit bits); gate_up arrivals of expert k at CTL_GU + 4096 k;
// combines done, error flag; combine arrivals of down row block rb at
// CTL_CB + 4 rb
constexpr int NREP = 8, CTL_REP = 4096;
constexpr int CTL_GU = NREP * CTL_REP, CTL_GU_STRIDE = 4096;
constexpr int CTL_DONE = CTL_GU + KMAX * CTL_GU_STRIDE, CTL_ERR = CTL_DONE + 256, CTL_CB = CTL_DONE + 512;
constexpr int CB_MAX = (PK_FUSED_CTL_BYTES - CTL_CB) / 4;   // down row blocks

typedef const __attribute__((address_space(4))) float *cfloat_p;

struct fused_args {
    const uint8_t *store;
    int64_t slot_stride;
    int32_t off_gu_t, off_gu_s, off_gu_b, off_dn_t, off_dn_s, off_dn_b;   // inside a slot
    int32_t slot_base;                    // layer * n_experts
    const float *R, *Rb;                  // router [E][D], bias [E]
    const float *x;                       // input row (raw residual row when nw)
    const float *nw;                      // optional rmsnorm weight
    float eps;
    float *xn;                            // [grid][2][xs] per workgroup: normalised row, activations
    const float *residual;                // optional: out = residual + moe
    float *out;
    int32_t *sel;                         // [K] routing results for callers
    float *w_scaled, *w_soft;             // [K]
    float *act;                           // [K][half] exchange
    float *eo;                            // [K][D] exchange
    uint8_t *ctl;                         // control block
    uint64_t *trace;                      // optional [grid][6]: 5 timestamps (100 MHz), placement
    int E, K, D, half, RB_gu, RB_dn, NG_gu, NG_dn, xs;
    float lim, alpha, rs;
};

__device__ __forceinline__ uint32_t ld_u(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_u64(uint64_t *p) {
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
__device__ __forceinline__ void st_u64(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_u(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t *ctl_u(const fused_args &a, int off) {
    return reinterpret_cast<uint32_t *>(a.ctl + off);
}
__device__ __forceinline__ uint64_t *slot_rep(const fused_args &a, int r) {
    return reinterpret_cast<uint64_t *>(a.ctl + r * CTL_REP);
}
__device__ __forceinline__ uint32_t *gu_ctr(const fused_args &a, int k) {
    return ctl_u(a, CTL_GU + k * CTL_GU_STRIDE);
}

__device__ __forceinline__ float wave_sum(float v) { return pk_wave_sum_f(v); }

__device__ __forceinline__ void mark(const fused_args &a, int i) {
    if (a.trace && threadIdx.x == STEER) a.trace[(int64_t)blockIdx.x * 6 + i] = wall_clock64();
}

// One lane polls *p until it reaches target; false on timeout or when
// another workgroup raised the error flag (checked every 64 polls).
__device__ bool wait_geq(uint32_t *p, uint32_t target, uint32_t *err) {
    for (uint32_t i = 0;; ++i) {
        if (ld_u(p) >= target) return true;
        if ((i & 63) == 63 && ld_u(err) != 0) return false;
        if (i >= SPIN_LIMIT) {
            add_u(err, 1);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Weights of one 64-row block for one math wave: groups wave, wave + 15,
// wave + 30 (NG <= 45).
struct blk {
    uint4 a[GPW], b[GPW];
    float s[GPW];
};

// Block id -> (down?, expert rank k, row block rb).
struct binfo {
    int down, k, rb;
};
__device__ __forceinline__ binfo block_info(const fused_args &a, int id) {
    binfo b;
    const int nb_gu = a.K * a.RB_gu;
    b.down = id >= nb_gu;
    const int d = b.down ? id - nb_gu : id;
    const int per = b.down ? a.RB_dn : a.RB_gu;
    b.k = d / per;
    b.rb = d - b.k * per;
    return b;
}

__device__ __forceinline__ const uint8_t *slot_base(const fused_args &a, const int *si, int k) {
    const int slot = __builtin_amdgcn_readfirstlane(a.slot_base + si[k]);
    return a.store + (int64_t)slot * a.slot_stride;
}

// Group u (g = wave + 15 u) of block `id` into slot u of w.
__device__ __forceinline__ void load_group(blk &w, int u, const fused_args &a, const int *si, int id, int wave,
                                           int lane) {
    const binfo b = block_info(a, id);
    const int NG = b.down ? a.NG_dn : a.NG_gu;
    const int g = wave + u * NMATH;
    if (g >= NG) return;
    const uint8_t *base = slot_base(a, si, b.k);
    const uint4 *tiles = reinterpret_cast<const uint4 *>(base + (b.down ? a.off_dn_t : a.off_gu_t)) +
                         (b.rb * NG + g) * 128;
    const float *sc = reinterpret_cast<const float *>(base + (b.down ? a.off_dn_s : a.off_gu_s)) +
                      (b.rb * NG + g) * 64;
    w.a[u] = pk_load_nt(&tiles[lane]);
    w.b[u] = pk_load_nt(&tiles[64 + lane]);
    w.s[u] = sc[lane];
}

// Per-group sums of block `id` into LDS (math waves), x read by scalar
// loads; after each group the same slot is refilled with block `next`
// (-1: none).
__device__ __forceinline__ void block_partials(blk &w, const fused_args &a, const int *si, int id, int next,
                                               cfloat_p x, float *part, float *scl, int wave, int lane) {
    const binfo b = block_info(a, id);
    const int NG = b.down ? a.NG_dn : a.NG_gu;
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        const int g = wave + u * NMATH;
        if (g < NG) {
            part[g * 64 + lane] = pk_group_dot(w.a[u], w.b[u], x + g * 64);
            scl[g * 64 + lane] = w.s[u];
        }
        if (next >= 0) load_group(w, u, a, si, next, wave, lane);
    }
}

// Bias of this lane's row of block `id` (0 beyond the rows).
__device__ __forceinline__ float block_bias(const fused_args &a, const int *si, int id, int lane) {
    const binfo b = block_info(a, id);
    const uint8_t *base = slot_base(a, si, b.k);
    const int row = b.rb * 64 + lane;
    const int O = b.down ? a.D : 2 * a.half;
    return row < O ? reinterpret_cast<const float *>(base + (b.down ? a.off_dn_b : a.off_gu_b))[row] : 0.0f;
}

// Steering wave: fold block `id` (partials in part/scl) and publish it.
__device__ __forceinline__ void fold_publish(const fused_args &a, const float *sw, int id, float bias,
                                             const float *part, const float *scl, int lane) {
    const binfo b = block_info(a, id);
    const int NG = b.down ? a.NG_dn : a.NG_gu;
    float acc = 0.0f;
    for (int g = 0; g < NG; ++g) acc = __builtin_fmaf(part[g * 64 + lane], scl[g * 64 + lane], acc);
    const int row = b.rb * 64 + lane;
    if (!b.down) {
        const int O = 2 * a.half;
        if (row < O) acc = acc + bias;
        const float up = __shfl_down(acc, 1, 64);
        if ((lane & 1) == 0 && row + 1 < O)
            st_f(a.act + (int64_t)b.k * a.half + (row >> 1), pk_swiglu(acc, up, a.lim, a.alpha));
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0) add_u(gu_ctr(a, b.k), 1u);
        return;
    }
    const int D = a.D;
    if (row < D) {
        acc = acc + bias;
        st_f(a.eo + (int64_t)b.k * D + row, acc);
    }
    __builtin_amdgcn_s_waitcnt(0);
    uint32_t arrived = 0;
    if (lane == 0) arrived = add_u(ctl_u(a, CTL_CB + 4 * b.rb), 1u);
    arrived = __shfl(arrived, 0, 64);
    if (arrived != (uint32_t)(a.K - 1)) return;
    // the last of the K down blocks of this row block combines them
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
    uint32_t done = 0;
    if (lane == 0) {
        st_u(ctl_u(a, CTL_CB + 4 * b.rb), 0u);
        done = add_u(ctl_u(a, CTL_DONE), 1u);
    }
    done = __shfl(done, 0, 64);
    if (done != (uint32_t)(a.RB_dn - 1)) return;
    // every workgroup has passed its waits once all row blocks combined
    for (int i = lane; i < NREP * a.E; i += 64) st_u64(slot_rep(a, i / a.E) + i % a.E, 0ull);
    if (lane < a.K) st_u(gu_ctr(a, lane), 0u);
    if (lane == 0) st_u(ctl_u(a, CTL_DONE), 0u);
}

__global__ __launch_bounds__(NTHR) void k_moe_fused(fused_args a) {
    extern __shared__ float lds[];
    const int NGm = max(a.NG_gu, a.NG_dn);
    float *bufs = lds;                    // [2][part, scl][NGm][64]
    float *xs = lds + 4 * NGm * 64;       // [D] router input (router workgroups)
    __shared__ float red[4];
    __shared__ double npart[4];
    __shared__ int ok;
    __shared__ int si[KMAX];
    __shared__ float sw[KMAX];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool steer = wave == NMATH;
    const int G = gridDim.x;
    const int wg = blockIdx.x;
    const int D = a.D;
    const int n4 = D >> 2;
    uint32_t *err = ctl_u(a, CTL_ERR);
    mark(a, 0);

    // ── 1. the gate_up input and the router rows (their first loads go out
    //       before the norm reduction) ──
    const bool router = wg < a.E;
    constexpr int U = 4;                  // float4 per thread per chunk (k_router_topk's GEMV_U)
    float4 wf[U];
    if (router && tid < 256) {
        const float4 *w4 = reinterpret_cast<const float4 *>(a.R + (int64_t)wg * D);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = tid + u * 256;
            wf[u] = i < n4 ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    if (a.nw) {
        // every workgroup normalises the row itself (k_rmsnorm's double
        // reduction) into its own copy; router workgroups also into LDS
        if (tid < 256) {
            double acc = 0.0;
            for (int i = tid; i < D; i += 256) acc += (double)a.x[i] * (double)a.x[i];
            acc = pk_dev_wave_sum_d(acc);
            if (lane == 0) npart[wave] = acc;
        }
        __syncthreads();
        const double ms = (npart[0] + npart[1]) + (npart[2] + npart[3]);
        const float rn = 1.0f / sqrtf((float)(ms / D) + a.eps);
        float *xp = a.xn + (int64_t)wg * 2 * a.xs;
        for (int i = tid; i < D; i += NTHR) {
            const float v = a.x[i] * rn * a.nw[i];
            xp[i] = v;
            if (router) xs[i] = v;
        }
        __builtin_amdgcn_s_waitcnt(0);
    } else if (router) {
        for (int i = tid; i < D; i += NTHR) xs[i] = a.x[i];
    }
    __syncthreads();
    if (router) {
        for (int r = wg; r < a.E; r += G) {
            const float4 *w4 = reinterpret_cast<const float4 *>(a.R + (int64_t)r * D);
            const float4 *x4 = reinterpret_cast<const float4 *>(xs);
            if (tid < 256) {
                float acc = 0.0f;
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
            if (tid < NREP) {
                const float v = (red[0] + red[1]) + (red[2] + red[3]);
                st_u64(slot_rep(a, tid) + r, (1ull << 32) | (uint64_t)__float_as_uint(v + a.Rb[r]));
            }
            __syncthreads();
        }
    }

    // ── 2. routing: the steering wave waits for the E slots, runs top-k ──
    if (steer) {
        const int E = a.E, K = a.K;
        uint64_t *slots = slot_rep(a, wg % NREP);
        float v0 = -INFINITY, v1 = -INFINITY;
        bool good = false;
        for (uint32_t it = 0;; ++it) {
            const uint64_t s0 = lane < E ? ld_u64(slots + lane) : (1ull << 32);
            const uint64_t s1 = lane + 64 < E ? ld_u64(slots + lane + 64) : (1ull << 32);
            if (__all((s0 >> 32) != 0 && (s1 >> 32) != 0)) {
                if (lane < E) v0 = __uint_as_float((uint32_t)s0);
                if (lane + 64 < E) v1 = __uint_as_float((uint32_t)s1);
                good = true;
                break;
            }
            if ((it & 63) == 63 && ld_u(err) != 0) break;
            if (it >= SPIN_LIMIT) {
                if (lane == 0) add_u(err, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (good) {
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
        if (lane == 0) ok = good;
    }
    __syncthreads();
    if (!ok) return;
    mark(a, 1);

    // ── 3. this workgroup's blocks: the first block's weights go out now ──
    const int nbt = a.K * (a.RB_gu + a.RB_dn);
    const int nb = wg < nbt ? min(MAXB, (nbt - 1 - wg) / G + 1) : 0;
    blk w;
    if (!steer && nb > 0) {
#pragma unroll
        for (int u = 0; u < GPW; ++u) load_group(w, u, a, si, wg, wave, lane);
    }
    // the gate_up input: the kernel's row, or this workgroup's normalised copy
    const float *xg = a.nw ? a.xn + (int64_t)wg * 2 * a.xs : a.x;
    asm volatile("" : "+s"(xg));
    // the steering wave's biases for its folds, loaded now
    float bias0 = 0.0f, bias1 = 0.0f, bias2 = 0.0f;
    if (steer) {
        if (nb > 0) bias0 = block_bias(a, si, wg, lane);
        if (nb > 1) bias1 = block_bias(a, si, wg + G, lane);
        if (nb > 2) bias2 = block_bias(a, si, wg + 2 * G, lane);
    }
#define PK_FUSED_BIAS(J) ((J) == 0 ? bias0 : (J) == 1 ? bias1 : bias2)
    // a down block's input: expert k's activations, copied by the whole
    // workgroup into its private row once they are complete
    float *xd = a.xn + ((int64_t)wg * 2 + 1) * a.xs;
#define PK_FUSED_STAGE(K)                                                                         \
    {                                                                                             \
        float *src_ = a.act + (int64_t)(K) * a.half;                                             \
        for (int i0 = tid; i0 < a.half; i0 += NTHR * 4) {                                         \
            float v_[4];                                                                          \
            _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                      \
                const int i = i0 + u * NTHR;                                                      \
                v_[u] = i < a.half ? ld_f(src_ + i) : 0.0f;                                       \
            }                                                                                     \
            _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                      \
                const int i = i0 + u * NTHR;                                                      \
                if (i < a.half) xd[i] = v_[u];                                                    \
            }                                                                                     \
        }                                                                                         \
        __builtin_amdgcn_s_waitcnt(0);                                                            \
        __syncthreads();                                                                          \
        asm volatile("" : "+s"(xd));                                                              \
    }

    // ── 4. blocks in order; the steering wave folds one block behind ──
    // A first block that is a down block (grids as wide as the gate_up work)
    // waits for its expert's activations like any later one.
    if (nb > 0 && block_info(a, wg).down) {
        if (steer) {
            bool got = true;
            if (lane == 0) got = wait_geq(gu_ctr(a, block_info(a, wg).k), (uint32_t)a.RB_gu, err);
            if (lane == 0) ok = got;
        }
        __syncthreads();
        if (!ok) return;
        PK_FUSED_STAGE(block_info(a, wg).k)
    }
    uint32_t folded = 0;                  // bit i: block i published (steering wave)
#define PK_FUSED_STEP(I)                                                                          \
    if ((I) < nb) {                                                                               \
        float *part = bufs + ((I) & 1) * 2 * NGm * 64;                                           \
        const binfo bi_ = block_info(a, wg + (I) * G);                                            \
        if (!steer) {                                                                             \
            const int nx_ = (I) + 1 < nb ? wg + ((I) + 1) * G : -1;                               \
            block_partials(w, a, si, wg + (I) * G, nx_, (cfloat_p)(bi_.down ? xd : xg), part,     \
                           part + NGm * 64, wave, lane);                                          \
        } else if ((I) > 0 && !(folded & (1u << ((I) - 1)))) {                                    \
            const float *pp = bufs + (((I) - 1) & 1) * 2 * NGm * 64;                             \
            fold_publish(a, sw, wg + ((I) - 1) * G, PK_FUSED_BIAS((I) - 1), pp, pp + NGm * 64,    \
                         lane);                                                                   \
            folded |= 1u << ((I) - 1);                                                            \
        }                                                                                         \
        __syncthreads();                                                                          \
        if ((I) + 1 < nb && block_info(a, wg + ((I) + 1) * G).down) {                             \
            if (steer) {                                                                          \
                if (!(folded & (1u << (I)))) {                                                    \
                    fold_publish(a, sw, wg + (I) * G, PK_FUSED_BIAS(I), part, part + NGm * 64,    \
                                 lane);                                                           \
                    folded |= 1u << (I);                                                          \
                }                                                                                 \
                bool got = true;                                                                  \
                if (lane == 0)                                                                    \
                    got = wait_geq(gu_ctr(a, block_info(a, wg + ((I) + 1) * G).k),                \
                                   (uint32_t)a.RB_gu, err);                                       \
                if (lane == 0) ok = got;                                                          \
                mark(a, 3);                                                                       \
            }                                                                                     \
            __syncthreads();                                                                      \
            if (!ok) return;                                                                      \
            PK_FUSED_STAGE(block_info(a, wg + ((I) + 1) * G).k)                                   \
        }                                                                                         \
    }
    PK_FUSED_STEP(0)
    mark(a, 2);
    PK_FUSED_STEP(1)
    PK_FUSED_STEP(2)
#undef PK_FUSED_STEP
#undef PK_FUSED_STAGE
    if (steer && nb > 0 && !(folded & (1u << (nb - 1)))) {
        const float *pp = bufs + ((nb - 1) & 1) * 2 * NGm * 64;
        fold_publish(a, sw, wg + (nb - 1) * G, nb == 1 ? bias0 : nb == 2 ? bias1 : bias2, pp, pp + NGm * 64,
                     lane);
    }
#undef PK_FUSED_BIAS
    mark(a, 4);
    // where the workgroup ran: XCC_ID << 32 | HW_ID (CU, SH, SE fields)
    if (a.trace && tid == STEER)
        a.trace[(int64_t)wg * 6 + 5] = ((uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |
                                       __builtin_amdgcn_s_getreg((31 << 11) | 4);
}

size_t fused_lds(const pk_engine *e) {
    const int NGm = std::max(e->ex.gu.NG, e->ex.dn.NG);
    return ((size_t)NGm * 64 * 4 + e->c.hidden) * sizeof(float);
}

int fused_grid(const pk_engine *e) {
    const int nbt = e->c.topk * (e->ex.gu.RB + e->ex.dn.RB);
    return std::max(1, std::min(e->n_cu, nbt));
}

}  // namespace

// Whether the single-launch layer applies: shapes it covers and a grid that
// is resident all at once (the waits depend on it).
bool pk_moe_fused_fits(pk_engine *e) {
    if (e->fused_fit >= 0) return e->fused_fit != 0;
    const pk_cfg *c = &e->c;
    const pk_expert_layout &ex = e->ex;
    const int nbt = c->topk * (ex.gu.RB + ex.dn.RB);
    bool fit = c->topk <= KMAX && c->n_experts <= 128 && (c->hidden & 3) == 0 &&
               ex.gu.NG <= NMATH * GPW && ex.dn.NG <= NMATH * GPW && ex.gu.NG * 64 == c->hidden &&
               ex.dn.NG * 64 == c->moe_inter / 2 && (c->moe_inter / 2) % 32 == 0 &&
               ex.stride < ((int64_t)1 << 31) && ex.dn.RB <= CB_MAX &&
               nbt <= MAXB * fused_grid(e) && fused_grid(e) <= e->n_cu && e->fused_ctl && e->fused_xn;
    const size_t lds = fused_lds(e);
    fit = fit && lds + 1024 <= 65536;
    if (fit) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_fused, NTHR, lds) != hipSuccess)
            per_cu = 0;
        (void)hipGetLastError();
        fit = per_cu > 0 && fused_grid(e) <= (int64_t)per_cu * e->n_cu;
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
    a.off_gu_t = (int32_t)e->ex.off_gu_tiles;
    a.off_gu_s = (int32_t)e->ex.off_gu_scales;
    a.off_gu_b = (int32_t)e->ex.off_gu_bias;
    a.off_dn_t = (int32_t)e->ex.off_dn_tiles;
    a.off_dn_s = (int32_t)e->ex.off_dn_scales;
    a.off_dn_b = (int32_t)e->ex.off_dn_bias;
    a.slot_base = layer * c->n_experts;
    a.R = d.router;
    a.Rb = d.router_b;
    a.x = x;
    a.nw = norm_w;
    a.eps = c->eps;
    a.xn = e->fused_xn;
    a.residual = residual;
    a.out = out;
    a.sel = e->sel;
    a.w_scaled = e->w_scaled;
    a.w_soft = e->w_soft;
    a.act = e->act;
    a.eo = e->eo;
    a.ctl = e->fused_ctl;
    a.trace = e->fused_trace;
    a.E = c->n_experts;
    a.K = c->topk;
    a.D = c->hidden;
    a.half = c->moe_inter / 2;
    a.RB_gu = e->ex.gu.RB;
    a.RB_dn = e->ex.dn.RB;
    a.NG_gu = e->ex.gu.NG;
    a.NG_dn = e->ex.dn.NG;
    a.xs = pk_fused_row(c);
    a.lim = c->swiglu_limit;
    a.alpha = c->swiglu_alpha;
    a.rs = c->routed_scale;
    hipLaunchKernelGGL(k_moe_fused, dim3(fused_grid(e)), dim3(NTHR), fused_lds(e), e->stream, a);
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
    if (!e->fused_ctl) return PK_OK;
    uint32_t flag = 0;
    PK_HIP(hipMemcpyAsync(&flag, e->fused_ctl + CTL_ERR, 4, hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    if (flag == 0) return PK_OK;
    // re-arm: slots, counters and the flag of the single-launch layer
    PK_HIP(hipMemsetAsync(e->fused_ctl, 0, PK_FUSED_CTL_BYTES, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    pk_set_error("MoE layer kernel: a dependency wait timed out (%u); its outputs are invalid", flag);
    return PK_ERR_HIP;
}
