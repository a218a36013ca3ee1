// pk_i4.hip — INT4 group-scaled kernels for gfx950.
//
// Replaces quant.h:259-319 (matmul_i4_gs) and the gs64 converter
// convert.py:45-93. Results are bit-identical to the reference:
//
//  * Each lane owns one (row, 64-column group) of a tile and runs the eight
//    fp32 FMA chains of quant.h's AVX2 loop in the same order: chain j takes
//    columns j, 8+j, ..., 56+j of the group. The chains are folded with
//    hsum256's tree ((c0+c4)+(c2+c6))+((c1+c5)+(c3+c7)) (quant.h:94-103).
//  * The per-group partial sums of a row are folded in group order,
//    a = fma(partial_g, scale_g, a), the contraction gcc applies to
//    quant.h:313 `a += ga * group_sc`.
//  * A nibble is decoded with one v_cvt_off_f32_i4 (SDWA byte select), which
//    yields q/16 exactly; the 1/16 is folded into the stored scales (x16),
//    and all scaling by 16 is exact, so every rounding matches the reference.
#include "pk_internal.h"

#include <algorithm>
#include <stdlib.h>

#include "pk_i4_device.h"
#include "pk_tagged.h"

// ───────────────────────── tiled GEMV ─────────────────────────
// grid = (RB, n_items); block = NW waves. Wave w handles groups w, w+NW, ...
// (GPW groups per pass, loads issued before the math); partial sums and
// scales meet in LDS; wave 0 folds the groups of its 64 rows in order.
// DOT: the integer-dot arithmetic (pk_dot_group) on the input records it.xq;
// each (row, group) value then goes to LDS and wave 0 adds them in group order.
template <int NW, int GPW, int EPI, bool DOT>
__global__ __launch_bounds__(NW * 64) void k_i4_gemv(pk_i4_items it, int O, int NG,
                                                     float lim, float alpha, pk_combine_args cb,
                                                     pk_route_args rt) {
    extern __shared__ float lds[];            // part[NG][64], scl[NG][64]
    float *part = lds;
    float *scl = lds + NG * 64;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = blockIdx.x;
    const int item = blockIdx.y;

    // the item's expert: given (slots), or selected here from the router
    // logits (round `item` of the top-k, computed by every wave)
    int slot;
    if (rt.logits) {
        float bv;
        slot = it.slot_base + pk_wave_topk_nth(rt.logits, rt.E, item, &bv);
    } else {
        slot = it.slot_base + (it.slots ? it.slots[item] : 0);
    }
    slot = __builtin_amdgcn_readfirstlane(slot);
    const uint8_t *base = it.base + (int64_t)slot * it.slot_stride;
    const uint4 *tiles = reinterpret_cast<const uint4 *>(base + it.off_tiles) +
                         (int64_t)rb * NG * (PK_TILE_BYTES / 16);
    const float *sc = reinterpret_cast<const float *>(base + it.off_scales) + (int64_t)rb * NG * 64;
    const float *__restrict__ x = it.x + (int64_t)(item / it.x_div) * it.x_stride;
    const int32_t *__restrict__ xq = DOT ? it.xq + (int64_t)(item / it.x_div) * it.xq_stride : nullptr;
    const int row = rb * 64 + lane;
    // the epilogue's operands go out with the weights, not after the fold
    // (a load issued there would put a memory round trip on the critical path)
    float bias = 0.0f, res = 0.0f, cw[16];
    if (wave == 0) {
        if (it.off_bias >= 0) bias = reinterpret_cast<const float *>(base + it.off_bias)[min(row, O - 1)];
        if constexpr (EPI == PK_EPI_COMBINE) {
            if (cb.residual) res = cb.residual[min(row, O - 1)];
#pragma unroll
            for (int k = 0; k < 16; ++k) cw[k] = k < it.n_items ? cb.w[k] : 0.0f;
        }
    }

    for (int g0 = wave; g0 < NG; g0 += NW * GPW) {
        uint4 wa[GPW], wb[GPW];
        float s[GPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int g = g0 + u * NW;
            if (g < NG) {
                wa[u] = pk_load_nt(&tiles[g * 128 + lane]);
                wb[u] = pk_load_nt(&tiles[g * 128 + 64 + lane]);
                s[u] = sc[g * 64 + lane];
            }
        }
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int g = g0 + u * NW;
            if (g < NG) {
                if constexpr (DOT) {
                    part[g * 64 + lane] = pk_dot_group(wa[u], wb[u], xq + 2 * g * PK_XQ_INTS,
                                                       xq + (2 * g + 1) * PK_XQ_INTS, s[u]);
                } else {
                    part[g * 64 + lane] = pk_group_dot(wa[u], wb[u], x + g * 64);
                    scl[g * 64 + lane] = s[u];
                }
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;

    float acc = pk_fold_groups<DOT>(part, scl, NG);
    if (it.off_bias >= 0 && row < O) acc = acc + bias;
    float *y = it.y + (int64_t)item * it.y_stride;
    if constexpr (EPI == PK_EPI_SWIGLU) {
        const float up = __shfl_down(acc, 1, 64);
        const bool has = (lane & 1) == 0 && row + 1 < O;
        const float a = pk_swiglu(acc, up, lim, alpha);
        if (has) y[row >> 1] = a;
        // the 32 outputs of this row block are one half-group of the next input
        if (it.yq) pk_write_digits<2>(a, has, it.yq + (int64_t)item * it.yq_stride + rb * PK_XQ_INTS);
    } else if constexpr (EPI == PK_EPI_COMBINE) {
        // moe_forward's accumulation (picchio.c:1387, :1445-1454) fused: each
        // item's rows go out device-coherently; the last item to finish this
        // row block adds them up in routing order, out = fma(w_k, eo_k, out),
        // then the residual (forward_token, picchio.c:1716), and re-arms the
        // block's arrival counter.
        // Ordering: every lane's row store is followed by a release fence at
        // device scope before lane 0 counts the item in (the wave issues the
        // fence of all lanes before the count); the last arriver's lanes
        // take an acquire fence before reading the other items' rows.
        if (row < O)
            __hip_atomic_store(y + row, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        uint32_t arrived = 0;
        if (lane == 0)
            arrived = __hip_atomic_fetch_add(cb.counters + rb, 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        arrived = __shfl(arrived, 0, 64);
        if (arrived != (uint32_t)(it.n_items - 1)) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (row < O) {
            float o = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (k < it.n_items)
                    o = __builtin_fmaf(cw[k],
                                       __hip_atomic_load(it.y + (int64_t)k * it.y_stride + row,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                       o);
            cb.out[row] = cb.residual ? res + o : o;
        }
        if (lane == 0)
            __hip_atomic_store(cb.counters + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        if (row < O) y[row] = acc;
    }
    // one wave of the launch publishes the routing for the launches after it
    if constexpr (EPI != PK_EPI_COMBINE)
        if (rt.logits && rb == 0 && item == 0) pk_wave_route_publish(rt);
}

// ───────────── persistent streaming GEMV (launches of many row blocks) ─────────────
// The k_i4_gemv body for launches whose tasks (n_items x RB row blocks) are
// well above the CUs: one 16-wave workgroup per CU walks tasks blockIdx.x,
// + gridDim.x, ... . Waves 0..14 keep the next task's weights in flight
// while they multiply the current one (a ring of two register slots; every
// refill is issued, past the workgroup's last task a same-address dummy, so
// that the load counter's waits stay exact) and write their partials to one
// of two LDS buffers by task parity; wave 15 folds each task in group order
// and writes its rows while the others move on. Two cumulative LDS counters
// per buffer order them (partials in; fold done). The same per-row
// arithmetic as k_i4_gemv, hence the same bits. Measured: 32 experts'
// gate_up in one launch 4.3 -> 4.5 TB/s, the 512-token prompt of config 2
// (its per-pair expert GEMVs) 0.43 -> 0.41 s; a ring of three slots was no
// faster.
constexpr int ST_NW = 15, ST_GPW = 3;     // load waves x groups per wave: NG <= 45

__device__ __forceinline__ void st_signal(int *c) {
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void st_wait(int *c, int target) {
    while (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(1);
}

template <int EPI, bool DOT>
__global__ __launch_bounds__((ST_NW + 1) * 64) void k_i4_gemv_stream(pk_i4_items it, int O, int NG, int RB,
                                                                     float lim, float alpha) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_task = it.n_items * RB, W = gridDim.x;
    const int my_n = (int)blockIdx.x < n_task ? (n_task - 1 - (int)blockIdx.x) / W + 1 : 0;
    float *part = lds;                                      // [2][NG][64]
    float *scl = lds + 2 * NG * 64;                         // [2][NG][64] (fp32 chains)
    int *cnt = reinterpret_cast<int *>(lds + (DOT ? 2 : 4) * NG * 64);   // partials in [2], folds done [2]
    if (threadIdx.x < 4) cnt[threadIdx.x] = 0;
    __syncthreads();
    const pk_cptr<int32_t> slots = pk_const(it.slots);
    // task k of this workgroup: item, row block, the item's expert slot
    auto task = [&](int k, int &item, int &rb) -> const uint8_t * {
        const int t = (int)blockIdx.x + k * W;
        item = t / RB;
        rb = t - item * RB;
        const int slot = it.slot_base + (it.slots ? slots[item] : 0);
        return it.base + (int64_t)slot * it.slot_stride;
    };

    if (wave < ST_NW) {
        uint4 wa0[ST_GPW], wb0[ST_GPW], wa1[ST_GPW], wb1[ST_GPW];
        float s0[ST_GPW], s1[ST_GPW];
        auto issue = [&](int k, uint4 (&wa)[ST_GPW], uint4 (&wb)[ST_GPW], float (&s)[ST_GPW]) {
            const bool real = k < my_n;
            int item, rb;
            const uint8_t *base = task(real ? k : 0, item, rb);
            const uint4 *tiles =
                reinterpret_cast<const uint4 *>(base + it.off_tiles) + (int64_t)rb * NG * (PK_TILE_BYTES / 16);
            const float *sc = reinterpret_cast<const float *>(base + it.off_scales) + (int64_t)rb * NG * 64;
            const int l = real ? lane : 0;
#pragma unroll
            for (int u = 0; u < ST_GPW; ++u) {
                const int g = min(wave + u * ST_NW, NG - 1);
                wa[u] = pk_load_nt(&tiles[g * 128 + l]);
                wb[u] = pk_load_nt(&tiles[g * 128 + 64 + l]);
                s[u] = sc[g * 64 + l];
            }
        };
        auto consume = [&](int k, const uint4 (&wa)[ST_GPW], const uint4 (&wb)[ST_GPW], const float (&s)[ST_GPW]) {
            const int b = k & 1;
            int item, rb;
            (void)task(k, item, rb);
            // buffer b is free once task k-2's fold is done
            if (k >= 2) st_wait(&cnt[2 + b], k >> 1);
            float *pb = part + b * NG * 64, *sb = scl + b * NG * 64;
            if constexpr (DOT) {
                const pk_cptr<int32_t> xq = pk_const(it.xq + (int64_t)(item / it.x_div) * it.xq_stride);
#pragma unroll
                for (int u = 0; u < ST_GPW; ++u) {
                    const int g = wave + u * ST_NW;
                    if (g < NG)
                        pb[g * 64 + lane] = pk_dot_group(wa[u], wb[u], xq + 2 * g * PK_XQ_INTS,
                                                         xq + (2 * g + 1) * PK_XQ_INTS, s[u]);
                }
            } else {
                const pk_cptr<float> x = pk_const(it.x + (int64_t)(item / it.x_div) * it.x_stride);
#pragma unroll
                for (int u = 0; u < ST_GPW; ++u) {
                    const int g = wave + u * ST_NW;
                    if (g < NG) {
                        pb[g * 64 + lane] = pk_group_dot(wa[u], wb[u], x + g * 64);
                        sb[g * 64 + lane] = s[u];
                    }
                }
            }
            st_signal(&cnt[b]);
        };
        issue(0, wa0, wb0, s0);
        issue(1, wa1, wb1, s1);
        for (int k = 0; k < my_n; k += 2) {
            consume(k, wa0, wb0, s0);
            issue(k + 2, wa0, wb0, s0);
            if (k + 1 < my_n) consume(k + 1, wa1, wb1, s1);
            issue(k + 3, wa1, wb1, s1);
        }
        return;
    }

    // wave ST_NW: fold and epilogue of each task
    for (int k = 0; k < my_n; ++k) {
        const int b = k & 1;
        int item, rb;
        const uint8_t *base = task(k, item, rb);
        const int row = rb * 64 + lane;
        const float bias = it.off_bias >= 0 ? reinterpret_cast<const float *>(base + it.off_bias)[min(row, O - 1)]
                                            : 0.0f;
        st_wait(&cnt[b], ST_NW * ((k >> 1) + 1));
        float acc = pk_fold_groups<DOT>(part + b * NG * 64, scl + b * NG * 64, NG);
        st_signal(&cnt[2 + b]);
        if (it.off_bias >= 0 && row < O) acc = acc + bias;
        float *y = it.y + (int64_t)item * it.y_stride;
        if constexpr (EPI == PK_EPI_SWIGLU) {
            const float up = __shfl_down(acc, 1, 64);
            const bool has = (lane & 1) == 0 && row + 1 < O;
            const float a = pk_swiglu(acc, up, lim, alpha);
            if (has) y[row >> 1] = a;
            if (it.yq) pk_write_digits<2>(a, has, it.yq + (int64_t)item * it.yq_stride + rb * PK_XQ_INTS);
        } else {
            if (row < O) y[row] = acc;
        }
    }
}

// ─────────────── integer-dot GEMV over expert-grouped pairs ───────────────
// grid = (RB, max_tiles); workgroup (rb, t) covers tile t's pairs (one expert,
// at most DT_M pairs): each wave loads its 3 groups of the expert's 64-row
// block once and runs the integer dot for every pair of the tile (inputs:
// the pair's records, it.xq + (pair / x_div) * xq_stride); wave j then adds
// pair j's groups in order and writes its rows (pair-indexed outputs, as the
// per-pair launch writes them: the same values).
constexpr int DT_M = 4;

template <int EPI>
__global__ __launch_bounds__(15 * 64) void k_i4_dot_tiles(pk_i4_items it, pk_i4_tiles tl, int O, int NG,
                                                          float lim, float alpha) {
    extern __shared__ float lds[];            // part[DT_M][NG][64]
    constexpr int NW = 15, GPW = 3;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = blockIdx.x, t = blockIdx.y;
    if (t >= *tl.n_tiles) return;
    const int beg = tl.tile_beg[t], cnt = tl.tile_cnt[t];
    const int slot = it.slot_base + tl.tile_exp[t];
    const uint8_t *base = it.base + (int64_t)slot * it.slot_stride;
    const uint4 *tiles = reinterpret_cast<const uint4 *>(base + it.off_tiles) +
                         (int64_t)rb * NG * (PK_TILE_BYTES / 16);
    const float *sc = reinterpret_cast<const float *>(base + it.off_scales) + (int64_t)rb * NG * 64;
    const int32_t *xr[DT_M];
#pragma unroll
    for (int j = 0; j < DT_M; ++j)
        xr[j] = it.xq + (int64_t)(tl.pairs[beg + min(j, cnt - 1)] / it.x_div) * it.xq_stride;

    for (int g0 = wave; g0 < NG; g0 += NW * GPW) {
        uint4 wa[GPW], wb[GPW];
        float s[GPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int g = g0 + u * NW;
            if (g < NG) {
                wa[u] = pk_load_nt(&tiles[g * 128 + lane]);
                wb[u] = pk_load_nt(&tiles[g * 128 + 64 + lane]);
                s[u] = sc[g * 64 + lane];
            }
        }
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int g = g0 + u * NW;
            if (g < NG) {
#pragma unroll
                for (int j = 0; j < DT_M; ++j)
                    if (j < cnt)
                        lds[((int64_t)j * NG + g) * 64 + lane] =
                            pk_dot_group(wa[u], wb[u], xr[j] + 2 * g * PK_XQ_INTS,
                                         xr[j] + (2 * g + 1) * PK_XQ_INTS, s[u]);
            }
        }
    }
    __syncthreads();
    if (wave >= cnt) return;
    const int pair = tl.pairs[beg + wave];
    float acc = pk_fold_groups<true>(lds + (int64_t)wave * NG * 64, nullptr, NG);
    const int row = rb * 64 + lane;
    if (it.off_bias >= 0 && row < O) acc = acc + reinterpret_cast<const float *>(base + it.off_bias)[row];
    float *y = it.y + (int64_t)pair * it.y_stride;
    if constexpr (EPI == PK_EPI_SWIGLU) {
        const float up = __shfl_down(acc, 1, 64);
        const bool has = (lane & 1) == 0 && row + 1 < O;
        const float a = pk_swiglu(acc, up, lim, alpha);
        if (has) y[row >> 1] = a;
        if (it.yq) pk_write_digits<2>(a, has, it.yq + (int64_t)pair * it.yq_stride + rb * PK_XQ_INTS);
    } else {
        if (row < O) y[row] = acc;
    }
}

int pk_launch_i4_dot_tiles(const pk_i4_items &it, const pk_i4_tiles &tl, const pk_i4_shape &sh, int epilogue,
                           float lim, float alpha, int max_tiles, hipStream_t st) {
    PK_CHECK(it.xq && tl.pairs && tl.tile_exp && tl.tile_beg && tl.tile_cnt && tl.n_tiles, PK_ERR_ARG,
             "dot tiles: missing buffers");
    PK_CHECK(epilogue != PK_EPI_COMBINE && max_tiles > 0 && sh.NG * DT_M * 64 * 4 <= 65536, PK_ERR_UNSUPPORTED,
             "dot tiles: epilogue %d, %d tiles, %d groups", epilogue, max_tiles, sh.NG);
    const dim3 grid(sh.RB, max_tiles);
    const size_t lds = (size_t)DT_M * sh.NG * 64 * sizeof(float);
    if (epilogue == PK_EPI_SWIGLU)
        hipLaunchKernelGGL(k_i4_dot_tiles<PK_EPI_SWIGLU>, grid, dim3(15 * 64), lds, st, it, tl, sh.O, sh.NG,
                           lim, alpha);
    else
        hipLaunchKernelGGL(k_i4_dot_tiles<PK_EPI_PLAIN>, grid, dim3(15 * 64), lds, st, it, tl, sh.O, sh.NG,
                           lim, alpha);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// Half-group records of x[0..n) (n a multiple of 32): one wave per record.
__global__ __launch_bounds__(64) void k_act_records(const float *x, int n, int32_t *rec) {
    const int lane = threadIdx.x;
    const int i = blockIdx.x * 32 + lane;
    const bool has = lane < 32 && i < n;
    pk_write_digits<1>(x[has ? i : 0], has, rec + (int64_t)blockIdx.x * PK_XQ_INTS);
}

int pk_launch_act_records(const float *x, int n, int32_t *rec, hipStream_t st) {
    PK_CHECK(n > 0 && n % 32 == 0, PK_ERR_ARG, "act records: n=%d is not a multiple of 32", n);
    hipLaunchKernelGGL(k_act_records, dim3(n / 32), dim3(64), 0, st, x, n, rec);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// compute units of the current device (cached per device)
static int pk_device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cus[dev] = n;
    }
    return cus[dev];
}

// PK_I4_STREAM=0 in the environment: the one-row-block-per-workgroup kernel only
static bool pk_i4_stream_on() {
    static const int on = getenv("PK_I4_STREAM") ? atoi(getenv("PK_I4_STREAM")) : 1;
    return on != 0;
}

int pk_launch_i4_gemv(const pk_i4_items &it, const pk_i4_shape &sh, int epilogue,
                      float lim, float alpha, const pk_combine_args *comb, hipStream_t st,
                      const pk_route_args *route) {
    pk_combine_args cb{};
    pk_route_args rt{};
    if (route) {
        PK_CHECK(route->logits && route->sel && route->w_scaled && route->E > 0 && route->E <= 128 &&
                     route->K > 0 && route->K <= 16 && it.n_items <= route->K && epilogue != PK_EPI_COMBINE,
                 PK_ERR_ARG, "i4 gemv: routing of %d items over E=%d K=%d", it.n_items, route->E, route->K);
        rt = *route;
    }
    if (epilogue == PK_EPI_COMBINE) {
        PK_CHECK(comb && comb->w && comb->out && comb->counters, PK_ERR_ARG, "combine: missing buffers");
        PK_CHECK(it.n_items <= 16, PK_ERR_UNSUPPORTED, "combine: %d items (at most 16)", it.n_items);
        PK_CHECK(sh.RB <= 1024, PK_ERR_UNSUPPORTED, "combine: %d row blocks", sh.RB);
        cb = *comb;
    }
    PK_CHECK(sh.NG > 0 && sh.RB > 0 && it.n_items > 0, PK_ERR_ARG, "i4 gemv: empty shape");
    PK_CHECK(sh.NG <= 128, PK_ERR_UNSUPPORTED, "i4 gemv: I=%d above 8192", sh.I);
    PK_CHECK(!it.yq || epilogue == PK_EPI_SWIGLU, PK_ERR_ARG, "i4 gemv: output records need the SwiGLU epilogue");
    // many row blocks without routing: the persistent streaming kernel (one
    // workgroup per CU, the next row block's weights in flight meanwhile)
    const int n_cu = pk_device_cus();
    if (!route && epilogue != PK_EPI_COMBINE && sh.NG <= ST_NW * ST_GPW && n_cu > 0 &&
        (int64_t)it.n_items * sh.RB >= 2 * (int64_t)n_cu && pk_i4_stream_on()) {
        const bool dot = it.xq != nullptr;
        // partials + scales in two buffers, the counters; at least half the
        // CU's LDS so that one workgroup runs per CU
        const size_t need = (size_t)(dot ? 2 : 4) * sh.NG * 64 * sizeof(float) + 4 * sizeof(int);
        const size_t lds = std::max(need, (size_t)82 * 1024);
        // as many workgroups as give every one the same count of row blocks
        // (2880 row blocks on 256 CUs: 240 x 12, not 64 x 12 + 192 x 11,
        // whose last round would stream from 64 CUs alone)
        const int64_t n_task = (int64_t)it.n_items * sh.RB;
        const int64_t per_wg = (n_task + n_cu - 1) / n_cu;
        const dim3 grid((unsigned)((n_task + per_wg - 1) / per_wg));
#define PK_I4_STREAM(E, D)                                                                              \
    hipLaunchKernelGGL((k_i4_gemv_stream<E, D>), grid, dim3((ST_NW + 1) * 64), lds, st, it, sh.O, sh.NG, \
                       sh.RB, lim, alpha)
        if (epilogue == PK_EPI_SWIGLU) {
            if (dot) PK_I4_STREAM(PK_EPI_SWIGLU, true); else PK_I4_STREAM(PK_EPI_SWIGLU, false);
        } else {
            if (dot) PK_I4_STREAM(PK_EPI_PLAIN, true); else PK_I4_STREAM(PK_EPI_PLAIN, false);
        }
#undef PK_I4_STREAM
        PK_HIP(hipGetLastError());
        return PK_OK;
    }
    const dim3 grid(sh.RB, it.n_items);
    const size_t lds = (size_t)sh.NG * 64 * 2 * sizeof(float);
    // 15 waves x 3 groups covers the 45 groups of a 2880-wide row in one pass.
    constexpr int NW = 15, GPW = 3;
#define PK_I4_LAUNCH(E, D)                                                                      \
    hipLaunchKernelGGL((k_i4_gemv<NW, GPW, E, D>), grid, dim3(NW * 64), lds, st, it, sh.O, sh.NG, \
                       lim, alpha, cb, rt)
    const bool dot = it.xq != nullptr;
    if (epilogue == PK_EPI_SWIGLU) {
        if (dot) PK_I4_LAUNCH(PK_EPI_SWIGLU, true); else PK_I4_LAUNCH(PK_EPI_SWIGLU, false);
    } else if (epilogue == PK_EPI_COMBINE) {
        if (dot) PK_I4_LAUNCH(PK_EPI_COMBINE, true); else PK_I4_LAUNCH(PK_EPI_COMBINE, false);
    } else {
        if (dot) PK_I4_LAUNCH(PK_EPI_PLAIN, true); else PK_I4_LAUNCH(PK_EPI_PLAIN, false);
    }
#undef PK_I4_LAUNCH
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────── a token's routed experts in one launch (batch-1 decode) ─────────────
// grid = the gate_up tasks (gu RB x K, item-minor); the first dn RB x K
// workgroups also take the down task of the same index (same item, so the
// same expert) once their gate_up math is done. Every workgroup selects its
// expert from the router logits (round `item` of the top-k).
// Values that cross workgroups travel as tagged words (pk_tagged.h); the
// tag is *epoch, a device word that the router launch before each expert
// launch advances.
//  * gate_up task: the k_i4_gemv SwiGLU body (fp32 chains, or the integer
//    dot on the input records); wave 0 publishes the row block's 32
//    activations (fp32) or their record (integer dot) as tagged words.
//  * down task: its weight loads go out as soon as the gate_up math has
//    freed the registers (before the gate_up epilogue); then, group by
//    group, each wave waits for that group's tagged inputs (two gate_up row
//    blocks) and runs the k_i4_gemv body; wave 0 publishes the row block's
//    rows as tagged words, except for item K-1, whose task waits for the
//    other items' rows and adds them in routing order,
//    out = fma(w_k, eo_k, out) (moe_forward, picchio.c:1387, :1445-1454),
//    then the residual (forward_token, picchio.c:1716).
// Deadlock freedom: only workgroups in their down task wait, and only for
// gate_up epilogues and other down tasks. The launcher keeps the down tasks
// below the workgroups the device holds at once, so a workgroup that has not
// started yet always finds a slot whatever the dispatch order.
// Wave 0 runs each epilogue at the highest wave priority (s_setprio): the
// epilogues are the launch's critical path.

// KM: an upper bound of the routed experts K. NW waves of GPW groups each
// cover a row block's groups in one pass; WPE: waves per SIMD the launch
// needs for two workgroups per CU.
template <bool DOT, int KM, int NW, int GPW, int WPE>
__global__ __launch_bounds__(NW * 64, WPE) void k_moe_ffn(pk_moe_ffn_args a) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int task = blockIdx.x;
    const int item = task % a.K;
    // the down task this workgroup also takes (a permutation of the grid for
    // any CU count; pk_moe_down_task)
    const int dtask = pk_moe_down_task(task, (int)gridDim.x, a.n_cu);
    const bool has_down = dtask < a.dn_RB * a.K;
    const int ditem = dtask % a.K;
    const pk_wave_logits lg = pk_load_wave_logits(a.rt.logits, a.rt.E);
    float bv;
    const int e = __builtin_amdgcn_readfirstlane(pk_wave_topk_nth(lg, a.rt.E, item, &bv));
    const uint8_t *eb = a.store + (int64_t)(a.slot_base + e) * a.slot_stride;   // the expert's slot
    const uint8_t *ebd = nullptr;                                               // the down task's
    const int64_t act_stride = DOT ? (int64_t)a.gu_RB * PK_XQ_INTS : a.gu_O / 2;
    float *part = lds;                                   // [NG][64] partials
    float *scl = lds + 64 * NW * GPW;                    // [NG][64] scales (fp32 chains)
    float *cwl = lds + 2 * 64 * NW * GPW;                // [K] combine weights
    uint4 wa[GPW], wb[GPW];
    float s[GPW];
    // one row block of one matrix of the expert: every group in one pass
    auto issue = [&](const uint8_t *xb, uint32_t off_tiles, uint32_t off_scales, int NG, int rb) {
        const uint4 *tiles = reinterpret_cast<const uint4 *>(xb + off_tiles) + (int64_t)rb * NG * (PK_TILE_BYTES / 16);
        const float *sc = reinterpret_cast<const float *>(xb + off_scales) + (int64_t)rb * NG * 64;
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int g = wave + u * NW;
            if (g < NG) {
                wa[u] = pk_load_nt(&tiles[g * 128 + lane]);
                wb[u] = pk_load_nt(&tiles[g * 128 + 64 + lane]);
                s[u] = sc[g * 64 + lane];
            }
        }
    };

    // ── gate_up task ──
    {
        const int NG = a.gu_NG, O = a.gu_O, rb = task / a.K;
        const int row = rb * 64 + lane;
        issue(eb, a.gu_tiles, a.gu_scales, NG, rb);
        // the down task's expert, while the gate_up weights stream in
        if (has_down) {
            const int ed = ditem == item ? e : __builtin_amdgcn_readfirstlane(pk_wave_topk_nth(lg, a.rt.E, ditem, &bv));
            ebd = a.store + (int64_t)(a.slot_base + ed) * a.slot_stride;
        }
        // while the weights stream in, wave 0 takes what else needs the
        // logits: the combine weights (the combining task: item K-1's) into
        // LDS, and the routing published for the launches (and the host)
        // after this one (the last workgroup)
        if (wave == 0) {
            if (has_down && ditem == a.K - 1) {
                int ci[KM];
                float cw[KM], wp[KM];
                pk_wave_route<KM>(a.rt, lg, ci, cw, wp);
#pragma unroll
                for (int k = 0; k < KM; ++k)
                    if (k < a.K && lane == 0) cwl[k] = cw[k];
            }
            if (task == (int)gridDim.x - 1) pk_wave_route_publish<KM>(a.rt, lg);
        }
        // (after the weight loads: a scalar load's wait would hold them back)
        const float bias = (wave == 0 && a.gu_bias >= 0)
                               ? reinterpret_cast<const float *>(eb + a.gu_bias)[min(row, O - 1)] : 0.0f;
        // the inputs come from an earlier launch: scalar loads
        const pk_cptr<float> x = pk_const(a.x);
        const pk_cptr<int32_t> xq = pk_const(a.xq);
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const int g = wave + u * NW;
            if (g < NG) {
                if constexpr (DOT) {
                    part[g * 64 + lane] = pk_dot_group(wa[u], wb[u], xq + 2 * g * PK_XQ_INTS,
                                                       xq + (2 * g + 1) * PK_XQ_INTS, s[u]);
                } else {
                    part[g * 64 + lane] = pk_group_dot(wa[u], wb[u], x + g * 64);
                    scl[g * 64 + lane] = s[u];
                }
            }
        }
        __syncthreads();
        // the down task's weights go out before the gate_up epilogue (wave 0
        // issues its share after it, so that the two do not meet in registers)
        if (wave != 0) {
            if (has_down) issue(ebd, a.dn_tiles, a.dn_scales, a.dn_NG, dtask / a.K);
        } else {
            __builtin_amdgcn_s_setprio(3);
            const uint32_t tag = *pk_const(a.epoch);
            float acc = pk_fold_groups<DOT>(part, scl, NG);
            if (a.gu_bias >= 0 && row < O) acc = acc + bias;
            const float up = __shfl_down(acc, 1, 64);
            const bool has = (lane & 1) == 0 && row + 1 < O;
            const float v = pk_swiglu(acc, up, a.lim, a.alpha);
            uint64_t *dst = a.act_t + item * act_stride;
            if constexpr (DOT) {
                // the row block's 32 outputs are one half-group of the down input
                const int32_t word = pk_record_word<2>(v, has);
                if (lane < PK_XQ_INTS) pk_put_tagged(dst + rb * PK_XQ_INTS + lane, tag, (uint32_t)word);
            } else {
                if (has) pk_put_tagged(dst + (row >> 1), tag, __float_as_uint(v));
            }
            __builtin_amdgcn_s_setprio(0);
            if (has_down) issue(ebd, a.dn_tiles, a.dn_scales, a.dn_NG, dtask / a.K);
        }
        if (!has_down) return;
        __syncthreads();                                  // part / scl are free again
    }

    // ── down task: row block dtask / K of item ditem's down matrix ──
    const int NG = a.dn_NG, O = a.dn_O, rb = dtask / a.K;
    const int row = rb * 64 + lane;
    const uint32_t tag = *pk_const(a.epoch);
    float bias = 0.0f, res = 0.0f;
    if (wave == 0) {
        if (a.dn_bias >= 0) bias = reinterpret_cast<const float *>(ebd + a.dn_bias)[min(row, O - 1)];
        if (ditem == a.K - 1 && a.residual) res = a.residual[min(row, O - 1)];
    }
    // group by group: wait for the tagged inputs (one per lane), read them
    // with v_readlane: group g's two records (48 ints) / 64 activations
    const uint64_t *src_item = a.act_t + ditem * act_stride;
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
        const int g = wave + u * NW;
        if (g < NG) {
            if constexpr (DOT) {
                const bool use = lane < 2 * PK_XQ_INTS;
                const int r = (int)pk_wait_tagged(src_item + 2 * g * PK_XQ_INTS + (use ? lane : 0), use, tag,
                                                  a.status);
                part[g * 64 + lane] = pk_dot_group(wa[u], wb[u], pk_lanes<int>{r, 0},
                                                   pk_lanes<int>{r, PK_XQ_INTS}, s[u]);
            } else {
                const int r = (int)pk_wait_tagged(src_item + g * 64 + lane, true, tag, a.status);
                part[g * 64 + lane] = pk_group_dot(wa[u], wb[u], pk_lanes<float>{r, 0});
                scl[g * 64 + lane] = s[u];
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;
    __builtin_amdgcn_s_setprio(3);
    float acc = pk_fold_groups<DOT>(part, scl, NG);
    if (a.dn_bias >= 0 && row < O) acc = acc + bias;
    // the combine: the row block's rows out as tagged words; item K-1's task
    // waits for the other items' rows and adds them in routing order
    if (ditem != a.K - 1) {
        if (row < O) pk_put_tagged(a.eo_t + (int64_t)ditem * O + row, tag, __float_as_uint(acc));
        return;
    }
    float o = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < a.K) {
            const float ek = k == ditem ? acc
                                       : __uint_as_float(pk_wait_tagged(a.eo_t + (int64_t)k * O + min(row, O - 1),
                                                                        row < O, tag, a.status));
            o = __builtin_fmaf(cwl[k], ek, o);
        }
    if (row < O) a.out[row] = a.residual ? res + o : o;
}

namespace {
constexpr int MF_NW = 15, MF_GPW = 3, MF_WPE = 8;
// partials + scales of NW x GPW groups, then the combine weights
constexpr size_t MF_LDS = (size_t)2 * MF_NW * MF_GPW * 64 * sizeof(float) + 16 * sizeof(float);

// workgroups of k_moe_ffn one CU holds at once (0 if the query fails)
int moe_ffn_wgs_per_cu(bool dot) {
    static int occ[2] = {-1, -1};
    int &o = occ[dot ? 1 : 0];
    if (o < 0) {
        int n = 0;
        const hipError_t rc =
            dot ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      &n, reinterpret_cast<const void *>(k_moe_ffn<true, 4, MF_NW, MF_GPW, MF_WPE>), MF_NW * 64, MF_LDS)
                : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      &n, reinterpret_cast<const void *>(k_moe_ffn<false, 4, MF_NW, MF_GPW, MF_WPE>), MF_NW * 64,
                      MF_LDS);
        if (rc != hipSuccess) return 0;           // (not cached: a later query may succeed)
        o = n;
    }
    return o;
}
}  // namespace

bool pk_moe_ffn_supported(int gu_RB, int dn_RB, int K, int n_cu, bool dot) {
    (void)gu_RB;
    if (n_cu <= 0 || K <= 0 || dn_RB <= 0) return false;
    const int64_t resident = (int64_t)n_cu * moe_ffn_wgs_per_cu(dot);
    return (int64_t)dn_RB * K < resident;
}

// Diagnostic: k_moe_ffn's placement for a device of n_cu CUs (grid =
// gu_RB x K workgroups): down_task[task] for every task, and whether the
// launcher would take the one-launch form (1) or refuse it (0). No device
// work; the occupancy query needs the HIP runtime only.
extern "C" int pk_moe_ffn_plan(int gu_RB, int dn_RB, int K, int n_cu, int dot, int *down_task, int n_out) {
    PK_CHECK(gu_RB > 0 && dn_RB > 0 && K > 0 && n_cu > 0, PK_ERR_ARG, "moe ffn plan: bad shape");
    const int grid = gu_RB * K;
    PK_CHECK(down_task == nullptr || n_out >= grid, PK_ERR_ARG, "moe ffn plan: %d outputs for %d tasks", n_out, grid);
    if (down_task)
        for (int t = 0; t < grid; ++t) down_task[t] = pk_moe_down_task(t, grid, n_cu);
    return pk_moe_ffn_supported(gu_RB, dn_RB, K, n_cu, dot != 0) ? 1 : 0;
}

int pk_launch_moe_ffn(const pk_moe_ffn_args &a, hipStream_t st) {
    constexpr int NW = MF_NW, GPW = MF_GPW, WPE = MF_WPE;
    PK_CHECK(a.rt.logits && a.rt.sel && a.rt.w_scaled && a.rt.E > 0 && a.rt.E <= 128 && a.K > 0 &&
                 a.K <= a.rt.E && a.rt.K == a.K,
             PK_ERR_ARG, "moe ffn: routing of K=%d over E=%d", a.K, a.rt.E);
    // (the routing state of more experts would not fit the registers of two
    // workgroups per CU: larger top-k runs as two launches)
    PK_CHECK(a.K <= 4, PK_ERR_UNSUPPORTED, "moe ffn: top-%d (at most 4 in one launch)", a.K);
    PK_CHECK(a.store && a.out && a.act_t && a.eo_t && a.epoch && a.status, PK_ERR_ARG, "moe ffn: missing buffers");
    PK_CHECK(a.dot ? a.xq != nullptr : a.x != nullptr, PK_ERR_ARG, "moe ffn: missing input");
    PK_CHECK(a.gu_NG > 0 && a.gu_NG <= NW * GPW && a.dn_NG > 0 && a.dn_NG <= NW * GPW && a.gu_O == a.gu_RB * 64 &&
                 a.dn_NG * 64 == a.gu_O / 2 && a.dn_RB * 64 >= a.dn_O && a.dn_RB <= a.gu_RB,
             PK_ERR_UNSUPPORTED, "moe ffn: shapes gate_up %d x %d groups, down %d x %d groups", a.gu_O, a.gu_NG,
             a.dn_O, a.dn_NG);
    PK_CHECK(a.n_cu > 0, PK_ERR_ARG, "moe ffn: n_cu %d", a.n_cu);
    // workgroups in their down task wait; they must leave room for the rest
    PK_CHECK(pk_moe_ffn_supported(a.gu_RB, a.dn_RB, a.K, a.n_cu, a.dot), PK_ERR_UNSUPPORTED,
             "moe ffn: %d down tasks do not leave a free slot among %d CUs x %d workgroups", a.dn_RB * a.K, a.n_cu,
             moe_ffn_wgs_per_cu(a.dot));
    const int grid = a.gu_RB * a.K;
    const size_t lds = MF_LDS;
    if (a.dot) hipLaunchKernelGGL((k_moe_ffn<true, 4, NW, GPW, WPE>), dim3(grid), dim3(NW * 64), lds, st, a);
    else hipLaunchKernelGGL((k_moe_ffn<false, 4, NW, GPW, WPE>), dim3(grid), dim3(NW * 64), lds, st, a);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────── reference-layout GEMV (any shape / group) ─────────────────
// One thread per (s, row). Same arithmetic as quant.h:259-319 including the
// scalar tail of a short last group; used for shapes the tiled layout does
// not cover (I % 64 != 0, group size != 64).
__global__ void k_i4_gemv_ref(float *y, const float *x, const uint8_t *q4, const float *s,
                              int S, int I, int O, int gs) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    const int si = blockIdx.y;
    if (o >= O || si >= S) return;
    const int rb = (I + 1) / 2, ng = (I + gs - 1) / gs;
    const uint8_t *w = q4 + (int64_t)o * rb;
    const float *xs = x + (int64_t)si * I;
    float a = 0.0f;
    for (int g = 0; g < ng; ++g) {
        const int g0 = g * gs, g1 = min(g0 + gs, I);
        int gi = g0;
        float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (; gi + 16 <= g1; gi += 16) {
            const uint8_t *p = w + (gi >> 1);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint8_t bt = p[j >> 1];
                const int nib = (j & 1) ? (bt >> 4) : (bt & 15);
                c[j] = __builtin_fmaf(xs[gi + j], (float)(nib - 8), c[j]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint8_t bt = p[4 + (j >> 1)];
                const int nib = (j & 1) ? (bt >> 4) : (bt & 15);
                c[j] = __builtin_fmaf(xs[gi + 8 + j], (float)(nib - 8), c[j]);
            }
        }
        const float b0 = c[0] + c[4], b1 = c[1] + c[5], b2 = c[2] + c[6], b3 = c[3] + c[7];
        float ga = (b0 + b2) + (b1 + b3);
        for (; gi < g1; gi += 2) {
            const uint8_t bt = w[gi >> 1];
            ga = __builtin_fmaf(xs[gi], (float)((int)(bt & 15) - 8), ga);
            if (gi + 1 < g1) ga = __builtin_fmaf(xs[gi + 1], (float)((int)(bt >> 4) - 8), ga);
        }
        a = __builtin_fmaf(ga, s[(int64_t)o * ng + g], a);
    }
    y[(int64_t)si * O + o] = a;
}

int pk_launch_i4_gemv_ref(float *y, const float *x, const uint8_t *q4, const float *s,
                          int S, int I, int O, int gs, hipStream_t st) {
    PK_CHECK(S > 0 && I > 0 && O > 0 && gs > 0, PK_ERR_ARG, "i4 gemv ref: bad shape");
    PK_CHECK(S <= 65535, PK_ERR_ARG, "i4 gemv ref: S=%d too large", S);
    hipLaunchKernelGGL(k_i4_gemv_ref, dim3((O + 127) / 128, S), dim3(128), 0, st,
                       y, x, q4, s, S, I, O, gs);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── repack ─────────────────────────
// Reference layout (q4 [O][I/2], s [O][I/64]) -> tiles + 16*scale.
// One thread per (row of the padded block, group).
__global__ void k_i4_repack(const uint8_t *q4, const float *s, int O, int I, int RB, int NG,
                            uint8_t *tiles, float *sc16) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)RB * 64 * NG) return;
    const int g = (int)(t % NG);
    const int row = (int)(t / NG);
    const int rb = row >> 6, r = row & 63;
    uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
    float scv = 0.0f;
    if (row < O) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(q4 + (int64_t)row * (I / 2) + g * 32);
        uint32_t v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = src[k] ^ 0x88888888u;
        lo = make_uint4(v[0], v[1], v[2], v[3]);
        hi = make_uint4(v[4], v[5], v[6], v[7]);
        scv = 16.0f * s[(int64_t)row * NG + g];
    }
    uint4 *dst = reinterpret_cast<uint4 *>(tiles + ((int64_t)rb * NG + g) * PK_TILE_BYTES);
    dst[r] = lo;
    dst[64 + r] = hi;
    sc16[((int64_t)rb * NG + g) * 64 + r] = scv;
}

int pk_launch_i4_repack(const uint8_t *q4, const float *s, int O, int I,
                        uint8_t *tiles, float *sc16, hipStream_t st) {
    PK_CHECK(I % 64 == 0 && O > 0, PK_ERR_UNSUPPORTED, "repack: I=%d not a multiple of 64", I);
    PK_CHECK(((uintptr_t)q4 & 3) == 0, PK_ERR_ARG, "repack: q4 not 4-byte aligned");
    const pk_i4_shape sh = pk_i4_make_shape(O, I);
    const int64_t n = (int64_t)sh.RB * 64 * sh.NG;
    hipLaunchKernelGGL(k_i4_repack, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       q4, s, O, I, sh.RB, sh.NG, tiles, sc16);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── quantizer ─────────────────────────
// convert.py:45-93: per (row, group) amax, scale = amax/7 (fp32, correctly
// rounded) or 1e-8, q = clip(rint(w/scale), -8, 7), low nibble = even column.
// One thread per (row, group); group_size <= 0 or >= I -> one group per row.
// Groups of odd length could share a byte with the next group: those are
// rare (odd gs) and handled by the per-row thread doing every group itself.
__global__ void k_quantize_i4(const float *w, int O, int I, int glen, int ng, int per_thread_row,
                              uint8_t *packed, float *scales) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int rbytes = (I + 1) / 2;
    int row, g_first, g_last;
    if (per_thread_row) {
        if (t >= O) return;
        row = (int)t; g_first = 0; g_last = ng;
    } else {
        if (t >= (int64_t)O * ng) return;
        row = (int)(t / ng); g_first = (int)(t % ng); g_last = g_first + 1;
    }
    const float *wr = w + (int64_t)row * I;
    uint8_t *pr = packed + (int64_t)row * rbytes;
    float *sr = scales + (int64_t)row * ng;
    for (int g = g_first; g < g_last; ++g) {
        const int a0 = g * glen, a1 = min(a0 + glen, I);
        float amax = 0.0f;
        for (int i = a0; i < a1; ++i) amax = fmaxf(amax, fabsf(wr[i]));
        sr[g] = amax > 1e-8f ? amax / 7.0f : 1e-8f;
    }
    // Column pairs (2c, 2c+1) -> byte c (convert.py:84-91). With an even group
    // length a thread's columns start on an even column; with an odd one the
    // thread owns the whole row. The last byte of an odd-width row keeps a
    // zero high nibble (convert.py:90-91).
    const int c0 = g_first * glen, c1 = min(g_last * glen, I);
    for (int i = c0; i < c1; i += 2) {
        float r0 = rintf(wr[i] / sr[i / glen]);
        r0 = fminf(fmaxf(r0, -8.0f), 7.0f);
        int n0 = ((int)r0 + 8) & 15, n1 = 0;
        if (i + 1 < I) {
            float r1 = rintf(wr[i + 1] / sr[(i + 1) / glen]);
            r1 = fminf(fmaxf(r1, -8.0f), 7.0f);
            n1 = ((int)r1 + 8) & 15;
        }
        pr[i >> 1] = (uint8_t)(n0 | (n1 << 4));
    }
}

int pk_launch_quantize_i4(const float *w, int O, int I, int gs, uint8_t *packed,
                          float *scales, hipStream_t st) {
    PK_CHECK(O > 0 && I > 0, PK_ERR_ARG, "quantize: bad shape");
    const int per_row_scale = (gs <= 0 || gs >= I);
    const int glen = per_row_scale ? I : gs;
    const int ng = per_row_scale ? 1 : (I + gs - 1) / gs;
    // an odd group length puts two groups in one byte: keep a row on one thread
    const int per_thread_row = (glen & 1) ? 1 : 0;
    const int64_t n = per_thread_row ? (int64_t)O : (int64_t)O * ng;
    hipLaunchKernelGGL(k_quantize_i4, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       w, O, I, glen, ng, per_thread_row, packed, scales);
    PK_HIP(hipGetLastError());
    return PK_OK;
}
