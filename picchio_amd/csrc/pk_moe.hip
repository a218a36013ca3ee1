// pk_moe.hip — a token's routed experts in one launch with every CU
// streaming the same bytes (batch-1 decode MoE, moe_forward's experts,
// picchio.c:1392-1454). An option (pk_set_moe_fused mode 2), bit-identical
// to the default k_moe_ffn and measured slower than it: the stream ends
// balanced, but three hand-overs follow it (the activations, a split down
// row block's accumulator, the combine), and the fp32 down arithmetic can
// only start once the activations are gathered.
//
// Work unit: one 64-row x 64-column tile of one expert matrix (lane = row,
// the k_i4_gemv arithmetic per (row, group)). The K routed experts give
// Ug = K x gu_RB x NG gate_up units and Ud = K x dn_RB x NG down units,
// numbered (item, row block, group) with the group fastest. One workgroup
// per CU (16 waves, grid = the device's CUs): workgroup c owns a contiguous
// range of gate_up units and one of down units, sized so that every
// workgroup holds ~(Ug + Ud) / grid units: the down units go in thirds of a
// row block (2 or 3 thirds per workgroup) and the gate_up ranges make up
// the rest. Every weight load of a wave is issued at entry, gate_up first,
// so that the gate_up tiles (whose outputs every down tile waits for) arrive
// ahead of the down tiles everywhere at once.
//
// Bit-identity with quant.h's order: a row's groups are folded in group
// order, a = fma(p_g, s_g, a) (integer dot: a = a + p_g). A row block split
// between workgroups c and c + 1 (its first groups at the end of c's range)
// is folded by c over its groups first and continued by c + 1 from c's
// accumulator, handed over as tagged words (pk_tagged.h) — the same
// sequence of roundings as one fold. Each workgroup walks its ranges from
// the end, so that the groups it hands over load first and the groups that
// wait for a hand-over load last. No row block spans more than two
// workgroups (the launcher checks the ranges).
//
// Hand-overs (tagged words, tag = the epoch the router launch advances):
//  * gate_up row block -> its 32 SwiGLU activations (or their record on the
//    integer dot), the inputs of every down unit of that expert;
//  * a split row block's accumulator -> the workgroup that continues it;
//  * down row block of item k < K-1 -> its rows; item K-1's workgroup adds
//    the K rows in routing order, out = fma(w_k, eo_k, out) (picchio.c:1387,
//    :1445-1454), then the residual (forward_token, picchio.c:1716).
// Every wave of every workgroup waits for others: all workgroups must be
// resident at once (one per CU; the launcher sizes the grid to the CUs and
// reserves enough LDS that no CU holds two). Polls are bounded.
#include "pk_internal.h"

#include "pk_i4_device.h"
#include "pk_tagged.h"

namespace {

constexpr int BW = 16;       // waves per workgroup
constexpr int NDW = 13;      // waves holding down units (the other three fold gate_up row blocks)
constexpr int BSG = 5;       // gate_up units per wave, at most (a range of <= 80)
constexpr int BSD = 4;       // down units per down wave, at most (a range of <= 52)
constexpr int PD = 2;        // weight slots in flight per wave (2: measured faster than 3 or 5)
constexpr int NU = 15;       // down units whose inputs a gathering wave polls (3 waves: ranges of <= 45)
constexpr int BKM = 4;       // routed experts, at most
constexpr int BTHIRDS = 3;   // down row blocks are dealt in thirds
// LDS: gate_up partials + scales [80][64] each, down partials + scales +
// inputs [52][64] each, the combine weights; at least 84 KB so that no CU
// holds two workgroups
constexpr int BLDS_FLOATS = 2 * BW * BSG * 64 + 3 * NDW * BSD * 64 + 16;
constexpr size_t BLDS_BYTES = (size_t)BLDS_FLOATS * 4 > 84 * 1024 ? (size_t)BLDS_FLOATS * 4 : 84 * 1024;

// Workgroup c's unit ranges [g0, g1) of gate_up and [d0, d1) of down.
struct bal_range {
    int g0, g1, d0, d1;
};
__host__ __device__ inline bal_range bal_range_of(int c, int W, int Ug, int Ud, int NGd) {
    const int P = NGd / BTHIRDS;
    const int64_t pieces = Ud / P, tot = (int64_t)Ug + Ud;
    bal_range r;
    r.d0 = (int)((int64_t)c * pieces / W) * P;
    r.d1 = (int)((int64_t)(c + 1) * pieces / W) * P;
    r.g0 = (int)((int64_t)c * tot / W) - r.d0;
    r.g1 = (int)((int64_t)(c + 1) * tot / W) - r.d1;
    return r;
}

// The row-block piece i (0, 1, 2) of a range [u0, u1) over row blocks of
// NG units: global row block R, groups [glo, ghi); starts / ends: whether
// the range holds the row block's first / last group.
struct bal_piece {
    int R, glo, ghi;
    bool valid, starts, ends;
};
__host__ __device__ inline bal_piece bal_piece_of(int u0, int u1, int NG, int i) {
    bal_piece p{};
    if (u1 <= u0) return p;
    const int R = u0 / NG + i;
    if (R > (u1 - 1) / NG) return p;
    const int lo = u0 > R * NG ? u0 : R * NG, hi = u1 < (R + 1) * NG ? u1 : (R + 1) * NG;
    p.R = R;
    p.glo = lo - R * NG;
    p.ghi = hi - R * NG;
    p.valid = true;
    p.starts = p.glo == 0;
    p.ends = p.ghi == NG;
    return p;
}

// The fold of groups [glo, ghi) of one row from LDS, continuing acc.
// Group g's partial is at pp[-64 g + lane] (the ranges are walked from the
// end, so the LDS index falls as g rises); ss likewise (fp32 chains).
template <bool DOT>
__device__ __forceinline__ float bal_fold(const float *pp, const float *ss, int glo, int ghi, float acc) {
    const int lane = threadIdx.x & 63;
    constexpr int C = 8;
    for (int g0 = glo; g0 < ghi; g0 += C) {
        float p[C], q[C];
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int g = min(g0 + j, ghi - 1);
            p[j] = pp[-64 * g + lane];
            if constexpr (!DOT) q[j] = ss[-64 * g + lane];
        }
#pragma unroll
        for (int j = 0; j < C; ++j)
            if (g0 + j < ghi) {
                if constexpr (DOT) acc = acc + p[j];
                else acc = __builtin_fmaf(p[j], q[j], acc);
            }
    }
    return acc;
}

// wave-uniform select of item k's value (k < BKM)
__device__ __forceinline__ int bal_pick(const int *v, int k) {
    return k == 0 ? v[0] : k == 1 ? v[1] : k == 2 ? v[2] : v[3];
}

template <bool DOT>
__global__ __launch_bounds__(BW * 64, 1) void k_moe_bal(pk_moe_ffn_args a) {
    extern __shared__ float lds[];
    float *gpart = lds;                          // [BW*BSG][64] gate_up partials
    float *gscl = gpart + BW * BSG * 64;         // and scales (fp32 chains)
    float *dpart = gscl + BW * BSG * 64;         // [NDW*BSD][64] down partials
    float *dscl = dpart + NDW * BSD * 64;
    uint32_t *dact = reinterpret_cast<uint32_t *>(dscl + NDW * BSD * 64);   // [NDW*BSD][64] down inputs
    float *cwl = reinterpret_cast<float *>(dact + NDW * BSD * 64);         // [K] combine weights
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, NGg = a.gu_NG, NGd = a.dn_NG;
    const int per_g = a.gu_RB * NGg, per_d = a.dn_RB * NGd;
    const bal_range rg = bal_range_of(blockIdx.x, gridDim.x, K * per_g, K * per_d, NGd);
    const int ng = rg.g1 - rg.g0, nd = rg.d1 - rg.d0;

    // every wave takes the K experts (the top-k rounds of moe_forward)
    const pk_wave_logits lg = pk_load_wave_logits(a.rt.logits, a.rt.E);
    int ex[BKM];
    {
        float ev[BKM];
        pk_wave_topk_all<BKM>(lg, a.rt.E, K, ex, ev);
#pragma unroll
        for (int k = 0; k < BKM; ++k) ex[k] = __builtin_amdgcn_readfirstlane(k < K ? ex[k] : 0);
    }
    auto expert_base = [&](int item) {
        return a.store + (int64_t)(a.slot_base + bal_pick(ex, item)) * a.slot_stride;
    };
    const uint32_t tag = *pk_const(a.epoch);
    const int64_t act_stride = DOT ? (int64_t)a.gu_RB * PK_XQ_INTS : a.gu_O / 2;
    uint64_t *d_cont = a.cont_t + (int64_t)K * a.gu_RB * 64;     // the down row blocks' words

    // The pieces split with the neighbouring workgroups: the last row block
    // of each range ends past it (its first groups, at the range's end: the
    // first units walked) and is folded as soon as its units are in, then
    // handed over.
    const bal_piece gh = bal_piece_of(rg.g0, rg.g1, NGg, (rg.g1 - 1) / NGg - rg.g0 / NGg);
    const int g_head_slot = gh.valid && !gh.ends ? (gh.ghi - 1) / BW : -1;   // its units: indices 0 .. ghi-1
    const int g_head_wave = NDW + (rg.g1 - 1) / NGg - rg.g0 / NGg;
    const bal_piece dh = bal_piece_of(rg.d0, rg.d1, NGd, (rg.d1 - 1) / NGd - rg.d0 / NGd);
    const int d_head_slot = nd > 0 && dh.valid && !dh.ends ? (dh.ghi - 1) / NDW : -1;
    const int d_head_wave = (rg.d1 - 1) / NGd - rg.d0 / NGd;

    // gate_up unit of slot k: loads, then its partial into LDS
    uint4 ga[BSG], gb[BSG];
    float gs[BSG];
    auto issue_gu = [&](int k) {
        const int j = k * BW + wave;                          // index from the range's end
        const int u = rg.g1 - 1 - min(j, ng - 1);
        const int item = u / per_g, t = u - item * per_g;    // t = rb * NG + g
        const uint8_t *eb = expert_base(item);
        const uint4 *tp = reinterpret_cast<const uint4 *>(eb + a.gu_tiles) + (int64_t)t * (PK_TILE_BYTES / 16);
        ga[k] = pk_load_nt(tp + lane);
        gb[k] = pk_load_nt(tp + 64 + lane);
        gs[k] = reinterpret_cast<const float *>(eb + a.gu_scales)[(int64_t)t * 64 + lane];
    };
    auto compute_gu = [&](int k) {
        const int j = k * BW + wave;
        if (j >= ng) return;
        const int u = rg.g1 - 1 - j;
        const int g = (u - (u / per_g) * per_g) % NGg;
        if constexpr (DOT) {
            const pk_cptr<int32_t> xq = pk_const(a.xq);
            gpart[j * 64 + lane] =
                pk_dot_group(ga[k], gb[k], xq + 2 * g * PK_XQ_INTS, xq + (2 * g + 1) * PK_XQ_INTS, gs[k]);
        } else {
            gpart[j * 64 + lane] = pk_group_dot(ga[k], gb[k], pk_const(a.x) + g * 64);
            gscl[j * 64 + lane] = gs[k];
        }
    };
    // after slot k's partials: the gate_up piece handed over, once its units are in
    auto gate_up_head = [&](int k) {
        if (k != g_head_slot) return;
        __syncthreads();
        if (wave == g_head_wave) {
            const int jb = rg.g1 - 1 - gh.R * NGg;     // unit R*NG + g sits at index jb - g
            const float acc = bal_fold<DOT>(gpart + jb * 64, gscl + jb * 64, 0, gh.ghi, 0.0f);
            pk_put_tagged(a.cont_t + (int64_t)gh.R * 64 + lane, tag, __float_as_uint(acc));
        }
    };
    auto down_head = [&](int k) {
        if (k != d_head_slot) return;
        __syncthreads();
        if (wave == d_head_wave) {
            __builtin_amdgcn_s_setprio(3);
            const int jb = rg.d1 - 1 - dh.R * NGd;
            const float acc = bal_fold<DOT>(dpart + jb * 64, dscl + jb * 64, 0, dh.ghi, 0.0f);
            pk_put_tagged(d_cont + (int64_t)dh.R * 64 + lane, tag, __float_as_uint(acc));
            __builtin_amdgcn_s_setprio(0);
        }
    };

    // Roles. Waves 0..NDW-1 hold the down units (unit j at slot j / NDW of
    // wave j % NDW) besides their gate_up units; waves NDW.. hold gate_up
    // units only, then fold the range's gate_up row blocks (one each) and
    // gather the down units' inputs into LDS — with no weights outstanding
    // their polls are not held back (the load counter retires in order).
    // Waves 0..2 fold the down row blocks once every down unit is in. Both
    // roles pass the same workgroup barriers in the same order.
    if (wave < NDW) {
        uint4 da[BSD], db[BSD];
        float ds[BSD];
        auto issue_dn = [&](int s) {
            const int j = s * NDW + wave;
            const int u = max(rg.d1 - 1 - min(j, max(nd - 1, 0)), 0);   // (a valid tile when nd = 0)
            const int item = u / per_d, t = u - item * per_d;
            const uint8_t *eb = expert_base(item);
            const uint4 *tp = reinterpret_cast<const uint4 *>(eb + a.dn_tiles) + (int64_t)t * (PK_TILE_BYTES / 16);
            da[s] = pk_load_nt(tp + lane);
            db[s] = pk_load_nt(tp + 64 + lane);
            ds[s] = reinterpret_cast<const float *>(eb + a.dn_scales)[(int64_t)t * 64 + lane];
        };
        auto issue = [&](int k) {
            if (k < BSG) issue_gu(k);
            else issue_dn(k - BSG);
        };
        // PD weight slots in flight: gate_up units, then down units
#pragma unroll
        for (int k = 0; k < PD; ++k) issue(k);
#pragma unroll
        for (int k = 0; k < BSG; ++k) {
            if (k + PD < BSG + BSD) issue(k + PD);
            compute_gu(k);
            gate_up_head(k);
        }
#pragma unroll
        for (int k = BSG + PD; k < BSG + BSD; ++k) issue(k);
        // the down epilogue's operands, behind the down units
        const bal_piece dp = bal_piece_of(rg.d0, rg.d1, NGd, wave < 3 ? wave : 3);
        const bool d_fold = wave < 3 && dp.valid && dp.ends;
        const int d_item = d_fold ? dp.R / a.dn_RB : 0, d_row = (dp.R - d_item * a.dn_RB) * 64 + lane;
        const bool combiner = d_fold && d_item == K - 1;
        float dbias = 0.0f, dres = 0.0f;
        if (d_fold) {
            if (a.dn_bias >= 0)
                dbias = reinterpret_cast<const float *>(expert_base(d_item) + a.dn_bias)[min(d_row, a.dn_O - 1)];
            if (combiner && a.residual) dres = a.residual[min(d_row, a.dn_O - 1)];
        }
        __syncthreads();                     // gate_up partials
        __syncthreads();                     // the down units' inputs
        // down partials from the LDS inputs, each as its weights land
#pragma unroll
        for (int s = 0; s < BSD; ++s) {
            const int j = s * NDW + wave;
            if (j < nd) {
                const uint32_t *xin = dact + j * 64;
                if constexpr (DOT) {
                    const int32_t *xr = reinterpret_cast<const int32_t *>(xin);
                    dpart[j * 64 + lane] = pk_dot_group(da[s], db[s], xr, xr + PK_XQ_INTS, ds[s]);
                } else {
                    dpart[j * 64 + lane] = pk_group_dot(da[s], db[s], reinterpret_cast<const float *>(xin));
                    dscl[j * 64 + lane] = ds[s];
                }
            }
            down_head(s);
        }
        __syncthreads();                     // down partials

        // ── down epilogues: every row block that ends in this range takes
        // its bias, then publishes its rows or, for item K-1, combines
        if (!d_fold) return;
        __builtin_amdgcn_s_setprio(3);
        const int jb = rg.d1 - 1 - dp.R * NGd;
        float acc = 0.0f;
        if (!dp.starts)   // continued from the workgroup before
            acc = __uint_as_float(pk_wait_tagged(d_cont + (int64_t)dp.R * 64 + lane, true, tag, a.status));
        acc = bal_fold<DOT>(dpart + jb * 64, dscl + jb * 64, dp.glo, NGd, acc);
        if (a.dn_bias >= 0 && d_row < a.dn_O) acc = acc + dbias;
        if (!combiner) {
            if (d_row < a.dn_O) pk_put_tagged(a.eo_t + (int64_t)d_item * a.dn_O + d_row, tag, __float_as_uint(acc));
            return;
        }
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < BKM; ++k)
            if (k < K) {
                const float ek = k == d_item ? acc
                                             : __uint_as_float(pk_wait_tagged(
                                                   a.eo_t + (int64_t)k * a.dn_O + min(d_row, a.dn_O - 1),
                                                   d_row < a.dn_O, tag, a.status));
                o = __builtin_fmaf(cwl[k], ek, o);
            }
        if (d_row < a.dn_O) a.out[d_row] = a.residual ? dres + o : o;
        return;
    }

    // ── the gate_up-only waves
    const int gw = wave - NDW;
    const bal_piece gp = bal_piece_of(rg.g0, rg.g1, NGg, gw);
    const bool g_fold = gp.valid && gp.ends;
    const int g_item = g_fold ? gp.R / a.gu_RB : 0, g_rb = gp.R - g_item * a.gu_RB;
    const int g_row = g_rb * 64 + lane;
    float gbias = 0.0f;
    if (g_fold && a.gu_bias >= 0)
        gbias = reinterpret_cast<const float *>(expert_base(g_item) + a.gu_bias)[min(g_row, a.gu_O - 1)];
#pragma unroll
    for (int k = 0; k < PD && k < BSG; ++k) issue_gu(k);
#pragma unroll
    for (int k = 0; k < BSG; ++k) {
        if (k + PD < BSG) issue_gu(k + PD);
        compute_gu(k);
        gate_up_head(k);
    }
    __syncthreads();                         // gate_up partials
    // gate_up epilogue of the row block this wave folds (if it ends here)
    if (g_fold) {
        __builtin_amdgcn_s_setprio(3);
        const int jb = rg.g1 - 1 - gp.R * NGg;
        float acc = 0.0f;
        if (!gp.starts)   // continued from the workgroup before
            acc = __uint_as_float(pk_wait_tagged(a.cont_t + (int64_t)gp.R * 64 + lane, true, tag, a.status));
        acc = bal_fold<DOT>(gpart + jb * 64, gscl + jb * 64, gp.glo, NGg, acc);
        if (a.gu_bias >= 0 && g_row < a.gu_O) acc = acc + gbias;
        const float up = __shfl_down(acc, 1, 64);
        const bool has = (lane & 1) == 0 && g_row + 1 < a.gu_O;
        const float v = pk_swiglu(acc, up, a.lim, a.alpha);
        uint64_t *dst = a.act_t + g_item * act_stride;
        if constexpr (DOT) {
            // the row block's 32 outputs are one half-group of the down input
            const int32_t word = pk_record_word<2>(v, has);
            if (lane < PK_XQ_INTS) pk_put_tagged(dst + g_rb * PK_XQ_INTS + lane, tag, (uint32_t)word);
        } else {
            if (has) pk_put_tagged(dst + (g_row >> 1), tag, __float_as_uint(v));
        }
        __builtin_amdgcn_s_setprio(0);
    }
    // the down units' inputs into LDS: unit j (of this range, from its end)
    // gets its group's 64 activations (or two half-group records); wave gw
    // takes units gw, gw + 3, ..., every poll of a lane in flight at once.
    // (Polling one word per producing row block first, then reading the
    // rest in one round, measured slower: a second round trip.)
    {
        auto src = [&](int i) {      // unit gw + 3 i's input word of this lane
            const int u = max(rg.d1 - 1 - min(gw + 3 * i, max(nd - 1, 0)), 0);
            const int item = u / per_d, g = (u - item * per_d) % NGd;
            return a.act_t + item * act_stride +
                   (DOT ? 2 * g * PK_XQ_INTS + min(lane, 2 * PK_XQ_INTS - 1) : g * 64 + lane);
        };
        auto used = [&](int i) { return gw + 3 * i < nd && (!DOT || lane < 2 * PK_XQ_INTS); };
        uint64_t w[NU];
#pragma unroll
        for (int i = 0; i < NU; ++i)
            w[i] = used(i) ? __hip_atomic_load(src(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                           : (uint64_t)tag << 32;
        uint32_t n_poll = 0;
        const uint32_t bound = pk_poll_bound(a.status);
        for (;;) {
            bool wait = false;
#pragma unroll
            for (int i = 0; i < NU; ++i) wait |= (uint32_t)(w[i] >> 32) != tag;
            if (!__any(wait)) break;
            if (++n_poll >= bound) {
                if (lane == 0) __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int i = 0; i < NU; ++i)
                if ((uint32_t)(w[i] >> 32) != tag)
                    w[i] = __hip_atomic_load(src(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int i = 0; i < NU; ++i)
            if (gw + 3 * i < nd) dact[(gw + 3 * i) * 64 + lane] = (uint32_t)w[i];
    }
    // the combine weights (item K-1's rows combine in this workgroup), and
    // from one wave of the launch the routing (sel, weights) for the
    // launches and the host after it
    if (gw == 2) {
        int ci[BKM];
        float cw[BKM], wp[BKM];
        pk_wave_route<BKM>(a.rt, lg, ci, cw, wp);
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < BKM; ++k)
                if (k < K) {
                    cwl[k] = cw[k];
                    if (blockIdx.x == gridDim.x - 1) {
                        a.rt.sel[k] = ci[k];
                        if (a.rt.w_soft) a.rt.w_soft[k] = wp[k];
                        a.rt.w_scaled[k] = cw[k];
                    }
                }
        }
    }
    __syncthreads();                         // the down units' inputs
#pragma unroll
    for (int s = 0; s < BSD; ++s) down_head(s);
    __syncthreads();                         // down partials
}

}  // namespace

// Whether k_moe_bal's ranges hold for this shape on W workgroups: every
// gate_up and down range fits the wave slots, no row block spans more than
// two workgroups, and no range lies inside one row block without its ends.
bool pk_moe_bal_supported(const pk_moe_ffn_args &a, int W) {
    if (W <= 0 || a.K <= 0 || a.K > BKM || a.gu_NG <= 0 || a.dn_NG <= 0 || a.dn_NG % BTHIRDS) return false;
    if (a.gu_O != a.gu_RB * 64 || a.dn_NG * 64 != a.gu_O / 2 || a.dn_RB * 64 < a.dn_O) return false;
    const int Ug = a.K * a.gu_RB * a.gu_NG, Ud = a.K * a.dn_RB * a.dn_NG;
    for (int c = 0; c < W; ++c) {
        const bal_range r = bal_range_of(c, W, Ug, Ud, a.dn_NG);
        const int ng = r.g1 - r.g0, nd = r.d1 - r.d0;
        if (ng < 1 || ng > BW * BSG || nd < 0 || nd > NDW * BSD || nd > 3 * NU) return false;
        for (int i = 0; i < 3; ++i) {
            const bal_piece g = bal_piece_of(r.g0, r.g1, a.gu_NG, i);
            if (g.valid && !g.starts && !g.ends) return false;       // inside one row block
            const bal_piece d = bal_piece_of(r.d0, r.d1, a.dn_NG, i);
            if (d.valid && !d.starts && !d.ends) return false;
        }
        // at most three row blocks per range (fold waves 0..2)
        if (bal_piece_of(r.g0, r.g1, a.gu_NG, 3).valid || bal_piece_of(r.d0, r.d1, a.dn_NG, 3).valid) return false;
    }
    return true;
}

int pk_launch_moe_bal(const pk_moe_ffn_args &a, hipStream_t st) {
    PK_CHECK(a.rt.logits && a.rt.sel && a.rt.w_scaled && a.rt.E > 0 && a.rt.E <= 128 && a.K > 0 &&
                 a.K <= a.rt.E && a.rt.K == a.K,
             PK_ERR_ARG, "moe bal: routing of K=%d over E=%d", a.K, a.rt.E);
    PK_CHECK(a.store && a.out && a.act_t && a.eo_t && a.cont_t && a.epoch && a.status, PK_ERR_ARG,
             "moe bal: missing buffers");
    PK_CHECK(a.dot ? a.xq != nullptr : a.x != nullptr, PK_ERR_ARG, "moe bal: missing input");
    const int W = a.n_cu;
    PK_CHECK(pk_moe_bal_supported(a, W), PK_ERR_UNSUPPORTED, "moe bal: shape or %d CUs not supported", W);
    if (a.dot) hipLaunchKernelGGL(k_moe_bal<true>, dim3(W), dim3(BW * 64), BLDS_BYTES, st, a);
    else hipLaunchKernelGGL(k_moe_bal<false>, dim3(W), dim3(BW * 64), BLDS_BYTES, st, a);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// One workgroup per CU must fit (the kernel's registers and LDS): checked
// once per arithmetic with the occupancy query.
bool pk_moe_bal_fits_cu(bool dot) {
    static int occ[2] = {-1, -1};
    int &o = occ[dot ? 1 : 0];
    if (o < 0) {
        int n = 0;
        const hipError_t rc =
            dot ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(k_moe_bal<true>),
                                                               BW * 64, BLDS_BYTES)
                : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(k_moe_bal<false>),
                                                               BW * 64, BLDS_BYTES);
        if (rc != hipSuccess) return false;
        o = n;
    }
    return o >= 1;
}

// Diagnostic export: the ranges k_moe_bal gives workgroup c of W, for the
// host-side checks of the partition (no device work).
extern "C" int pk_moe_bal_plan(int K, int gu_RB, int gu_NG, int dn_RB, int dn_NG, int W, int *ranges, int n_out) {
    PK_CHECK(K > 0 && gu_RB > 0 && gu_NG > 0 && dn_RB > 0 && dn_NG > 0 && W > 0, PK_ERR_ARG, "moe bal plan: bad shape");
    PK_CHECK(ranges == nullptr || n_out >= 4 * W, PK_ERR_ARG, "moe bal plan: %d outputs for %d workgroups", n_out, W);
    pk_moe_ffn_args a{};
    a.K = K;
    a.gu_RB = gu_RB; a.gu_NG = gu_NG; a.gu_O = gu_RB * 64;
    a.dn_RB = dn_RB; a.dn_NG = dn_NG; a.dn_O = dn_RB * 64;
    if (dn_NG % BTHIRDS == 0 && ranges) {
        const int Ug = K * gu_RB * gu_NG, Ud = K * dn_RB * dn_NG;
        for (int c = 0; c < W; ++c) {
            const bal_range r = bal_range_of(c, W, Ug, Ud, dn_NG);
            ranges[4 * c + 0] = r.g0; ranges[4 * c + 1] = r.g1;
            ranges[4 * c + 2] = r.d0; ranges[4 * c + 3] = r.d1;
        }
    }
    return pk_moe_bal_supported(a, W) ? 1 : 0;
}
