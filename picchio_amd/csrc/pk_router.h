// pk_router.h — one router logit with the MoE input's RMSNorm fused, shared
// by k_router_topk and the router workgroups of k_attn_oproj, so that the
// two produce the same bits.
#pragma once
#include "pk_dev.h"
#include "pk_i4_device.h"

constexpr int PK_ROUTER_U = 4;       // float4 per thread per chunk of the router row

// Router logit e of one token on rmsnorm(x) (moe_forward, picchio.c:1316-1324;
// rmsnorm, quant.h:396-402), without the bias, for a 256-thread block.
// The caller has loaded thread t's x[t + 256 k] (k < 12) into hv and the
// first chunk of the float4 rows (entry t + 256 u, u < PK_ROUTER_U; zeros
// past the row): xh of x, wf of router row e, xw of the norm weights nw. x
// itself (global or LDS) is read for later chunks, for the normalised
// slice that block e writes to hn, and for the integer-dot records (hq).
// The row's dot runs over thread t's entries t + 256 u in chunk order, then
// the wave tree and the block's four wave sums as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float pk_router_norm_logit(const float (&hv)[12], const float4 (&xh)[PK_ROUTER_U],
                                                      const float4 (&wf)[PK_ROUTER_U],
                                                      const float4 (&xw)[PK_ROUTER_U], const float *x,
                                                      const float *Rrow, const float *nw, int D, float eps, int e,
                                                      int E, float *hn, int32_t *hq, float *red, double *npart) {
    const int n4 = D >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *w4 = reinterpret_cast<const float4 *>(Rrow);
    const float4 *n4w = reinterpret_cast<const float4 *>(nw);
    const float rn = pk_rms_finish(hv, x, D, eps, npart);
    if (!hq) {
        const int span = (D + E - 1) / E;
        for (int i = e * span + threadIdx.x; i < min(D, (e + 1) * span); i += 256) hn[i] = x[i] * rn * nw[i];
    }
    float acc = 0.0f;
    for (int i0 = threadIdx.x; i0 < n4; i0 += 256 * PK_ROUTER_U) {
        float4 a[PK_ROUTER_U], w[PK_ROUTER_U], s[PK_ROUTER_U];
#pragma unroll
        for (int u = 0; u < PK_ROUTER_U; ++u) {
            const int i = i0 + u * 256;
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            const bool first = i0 == (int)threadIdx.x;
            a[u] = first ? xh[u] : (i < n4 ? x4[i] : z);
            w[u] = first ? wf[u] : (i < n4 ? w4[i] : z);
            s[u] = first ? xw[u] : (i < n4 ? n4w[i] : z);
        }
#pragma unroll
        for (int u = 0; u < PK_ROUTER_U; ++u) {
            if (i0 + u * 256 < n4) {
                const float4 xv = pk_norm4(a[u], rn, s[u]);
                acc = __builtin_fmaf(xv.x, w[u].x, acc);
                acc = __builtin_fmaf(xv.y, w[u].y, acc);
                acc = __builtin_fmaf(xv.z, w[u].z, acc);
                acc = __builtin_fmaf(xv.w, w[u].w, acc);
            }
        }
    }
    for (int i = (n4 << 2) + threadIdx.x; i < D; i += 256) acc = __builtin_fmaf(x[i] * rn * nw[i], Rrow[i], acc);
    acc = pk_wave_sum_f(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float v = (red[0] + red[1]) + (red[2] + red[3]);
    if (hq) {
        // the experts' input as half-group records of the integer-dot
        // arithmetic: one wave per 32 values, whole half-groups per
        // workgroup; hn is written here too
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const int nhg = (D + 31) >> 5, per = (nhg + E - 1) / E;
        for (int hg = e * per + wv; hg < min(nhg, (e + 1) * per); hg += 4) {
            const int i = hg * 32 + lane;
            const bool has = lane < 32 && i < D;
            const int ic = has ? i : 0;
            const float xv = x[ic] * rn * nw[ic];
            if (has) hn[i] = xv;
            pk_write_digits<1>(xv, has, hq + (int64_t)hg * PK_XQ_INTS);
        }
    }
    return v;
}
