// pk_i4_device.h — device helpers of the INT4 gs64 expert kernels.
//
// The arithmetic reproduces quant.h:259-319 (matmul_i4_gs, AVX2 branch):
//  * eight fp32 FMA chains per 64-column group, chain j taking columns
//    j, 8+j, ..., 56+j, folded with hsum256's tree (quant.h:94-103);
//  * nibbles decoded by v_cvt_off_f32_i4 (SDWA byte select) as q/16, the
//    1/16 being folded into the stored scales (x16, exact).
#pragma once
#include "pk_internal.h"

typedef uint32_t pk_u32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load (weights are read once per token: non-temporal).
__device__ __forceinline__ uint4 pk_load_nt(const uint4 *p) {
    const pk_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const pk_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ───────────────────────── nibble decode ─────────────────────────
// Low nibble of byte B of w, read as a signed 4-bit value, divided by 16.
template <int B>
__device__ __forceinline__ float pk_q16(uint32_t w) {
    float r;
    if constexpr (B == 0)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
            : "=v"(r) : "v"(w));
    else if constexpr (B == 1)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
            : "=v"(r) : "v"(w));
    else if constexpr (B == 2)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
            : "=v"(r) : "v"(w));
    else
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
            : "=v"(r) : "v"(w));
    return r;
}

// One 64-column group of one row: 32 stored bytes in two uint4 (columns 0..31
// and 32..63), x = the group's 64 inputs (wave-uniform). Returns partial/16.
// XP: any pointer to the 64 floats (global, constant or LDS address space).
template <typename XP>
__device__ __forceinline__ float pk_group_dot(uint4 a, uint4 b, XP xg) {
    float c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = 0.0f;
    const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        // dword d holds columns 8d..8d+7: byte k -> columns 8d+2k (low), 8d+2k+1 (high)
        const uint32_t w = wd[d], h = w >> 4;
        const XP xs = xg + 8 * d;
        c[0] = __builtin_fmaf(xs[0], pk_q16<0>(w), c[0]);
        c[1] = __builtin_fmaf(xs[1], pk_q16<0>(h), c[1]);
        c[2] = __builtin_fmaf(xs[2], pk_q16<1>(w), c[2]);
        c[3] = __builtin_fmaf(xs[3], pk_q16<1>(h), c[3]);
        c[4] = __builtin_fmaf(xs[4], pk_q16<2>(w), c[4]);
        c[5] = __builtin_fmaf(xs[5], pk_q16<2>(h), c[5]);
        c[6] = __builtin_fmaf(xs[6], pk_q16<3>(w), c[6]);
        c[7] = __builtin_fmaf(xs[7], pk_q16<3>(h), c[7]);
    }
    const float b0 = c[0] + c[4], b1 = c[1] + c[5], b2 = c[2] + c[6], b3 = c[3] + c[7];
    return (b0 + b2) + (b1 + b3);
}

// A pointer into the constant address space: wave-uniform loads through it
// are scalar loads (s_load, the scalar cache) whatever else the kernel
// writes. Only for data that no wave of the launch writes.
template <typename T>
using pk_cptr = const __attribute__((address_space(4))) T *;
template <typename T>
__device__ __forceinline__ pk_cptr<T> pk_const(const T *p) {
    return (pk_cptr<T>)(const __attribute__((address_space(1))) T *)p;
}

// 64 values held one per lane of a wave, read wave-uniformly: v[i] is
// lane (off + i)'s value (v_readlane: the operand lands in a scalar
// register). An input pointer for pk_group_dot / pk_dot_group when a wave
// has loaded its inputs itself instead of taking them from constant memory.
template <typename T>
struct pk_lanes {
    int v, off;
    __device__ __forceinline__ pk_lanes operator+(int d) const { return {v, off + d}; }
    __device__ __forceinline__ T operator[](int i) const {
        const int r = __builtin_amdgcn_readlane(v, off + i);
        if constexpr (sizeof(T) == 4 && T(0.5) != T(0)) return __int_as_float(r);
        else return r;
    }
};

// The row's value from its per-group partials in LDS (part[g][64], and the
// scales scl[g][64] for the fp32 chains), folded in group order: a = a + p_g
// (integer dot: the partials carry their scales) or a = fma(p_g, s_g, a)
// (quant.h:313). The LDS reads go out C at a time ahead of the chain.
template <bool DOT>
__device__ __forceinline__ float pk_fold_groups(const float *part, const float *scl, int NG) {
    const int lane = threadIdx.x & 63;
    constexpr int C = DOT ? 15 : 8;
    float acc = 0.0f;
    for (int g0 = 0; g0 < NG; g0 += C) {
        float p[C], q[C];
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int g = min(g0 + j, NG - 1);
            p[j] = part[g * 64 + lane];
            if constexpr (!DOT) q[j] = scl[g * 64 + lane];
        }
#pragma unroll
        for (int j = 0; j < C; ++j)
            if (g0 + j < NG) {
                if constexpr (DOT) acc = acc + p[j];
                else acc = __builtin_fmaf(p[j], q[j], acc);
            }
    }
    return acc;
}

// expf as the double exp rounded once to float: the correctly rounded value
// (but for double rounding in about 2^-29 of inputs), which is glibc's expf
// except where glibc's own result is not correctly rounded (~8e-5 of inputs).
__device__ __forceinline__ float pk_expf_cr(float x) { return (float)exp((double)x); }

__device__ __forceinline__ float pk_sigmoid(float v) { return 1.0f / (1.0f + pk_expf_cr(-v)); }

// GPT-OSS clamped SwiGLU of one (gate, up) pair (picchio.c:1416-1424).
__device__ __forceinline__ float pk_swiglu(float gate, float up, float lim, float alpha) {
    if (gate > lim) gate = lim;
    if (up > lim) up = lim;
    if (up < -lim) up = -lim;
    return (up + 1.0f) * gate * pk_sigmoid(alpha * gate);
}


// ───────────────────── router top-k of one token ─────────────────────
// Maximum of a 32-bit key over the wave with DPP (row shifts 1, 2, 4, 8,
// then the row broadcasts 15 and 31), read from lane 63: a handful of VALU
// steps instead of a chain of LDS permutes. 0 is the identity.
__device__ __forceinline__ uint32_t pk_wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Order-preserving key of a float (NaN and -0.0 handled by the caller):
// larger floats get larger unsigned keys, -inf the smallest above 0.
__device__ __forceinline__ uint32_t pk_fkey(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Selection round by round on one wave, the rule of moe_forward's top-k
// (picchio.c:1327-1339): repeated argmax with strict '>', so that the lowest
// index wins a tie (a wave maximum, then the lowest lane holding it by
// ballot; -0.0 counts as +0.0, NaN is never taken); when no logit is above
// -1e30 the reference leaves -1, here the index becomes 0 (inside the store)
// with the value -1e30. Lane l holds experts l and l + 64 (E <= 128).
// Returns round n's (index, logit), the same on every lane; rounds 0..n-1
// are taken out first.
// The logits as one wave holds them: lane l has experts l and l + 64
// (clamped, unconditional loads; entries past E are masked by the users).
struct pk_wave_logits {
    float v0, v1;
};
__device__ __forceinline__ pk_wave_logits pk_load_wave_logits(const float *logits, int E) {
    const int lane = threadIdx.x & 63;
    return {logits[min(lane, E - 1)], logits[min(lane + 64, E - 1)]};
}

__device__ __forceinline__ int pk_wave_topk_nth(const pk_wave_logits &lg, int E, int n, float *val) {
    const int lane = threadIdx.x & 63;
    const float v0 = lg.v0, v1 = lg.v1;
    const uint32_t k0 = (lane < E && v0 == v0) ? pk_fkey(v0 + 0.0f) : 0u;
    const uint32_t k1 = (lane + 64 < E && v1 == v1) ? pk_fkey(v1 + 0.0f) : 0u;
    const uint32_t floor_key = pk_fkey(-1e30f);
    bool t0 = false, t1 = false;
    int bi = 0;
    float bv = -1e30f;
    for (int k = 0; k <= n; ++k) {
        const uint32_t a0 = t0 ? 0u : k0, a1 = t1 ? 0u : k1;
        const uint32_t M = pk_wave_max_u32(max(a0, a1));
        if (M <= floor_key) {
            bi = 0;
            bv = -1e30f;
        } else {
            const uint64_t m0 = __ballot(a0 == M);
            bi = m0 ? __builtin_ctzll(m0) : 64 + __builtin_ctzll(__ballot(a1 == M));
            bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bi < 64 ? v0 : v1), bi & 63));
        }
        if (bi == lane) t0 = true;
        if (bi == lane + 64) t1 = true;
    }
    *val = bv;
    return bi;
}

__device__ __forceinline__ int pk_wave_topk_nth(const float *logits, int E, int n, float *val) {
    return pk_wave_topk_nth(pk_load_wave_logits(logits, E), E, n, val);
}

// Rounds 0..K-1 of the same selection in one pass: idx[k] / val[k] = round
// k's (index, logit), the same on every lane (KM: an upper bound of K).
template <int KM>
__device__ __forceinline__ void pk_wave_topk_all(const pk_wave_logits &lg, int E, int K, int *idx, float *val) {
    const int lane = threadIdx.x & 63;
    const float v0 = lg.v0, v1 = lg.v1;
    const uint32_t k0 = (lane < E && v0 == v0) ? pk_fkey(v0 + 0.0f) : 0u;
    const uint32_t k1 = (lane + 64 < E && v1 == v1) ? pk_fkey(v1 + 0.0f) : 0u;
    const uint32_t floor_key = pk_fkey(-1e30f);
    bool t0 = false, t1 = false;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        int bi = 0;
        float bv = -1e30f;
        if (k < K) {
            const uint32_t a0 = t0 ? 0u : k0, a1 = t1 ? 0u : k1;
            const uint32_t M = pk_wave_max_u32(max(a0, a1));
            if (M > floor_key) {
                const uint64_t m0 = __ballot(a0 == M);
                bi = m0 ? __builtin_ctzll(m0) : 64 + __builtin_ctzll(__ballot(a1 == M));
                bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bi < 64 ? v0 : v1), bi & 63));
            }
            if (bi == lane) t0 = true;
            if (bi == lane + 64) t1 = true;
        }
        idx[k] = bi;
        val[k] = bv;
    }
}

// Routing of one token from its logits, in the consumer of the router
// logits (picchio.c:1353, quant.h:406-412: max, expf, sum and division in
// routing order), with the arithmetic of k_router_topk's last block: ci[k] /
// ws[k] / wp[k] = round k's expert, its weight * routed_scale and its weight,
// the same on every lane.
// KM: an upper bound of rt.K (the arrays' length).
template <int KM = 16>
__device__ __forceinline__ void pk_wave_route(const pk_route_args &rt, const pk_wave_logits &lg, int *ci, float *ws,
                                              float *wp) {
    float m = -1e30f, cv[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        if (k < rt.K) {
            ci[k] = pk_wave_topk_nth(lg, rt.E, k, &cv[k]);
            if (cv[k] > m) m = cv[k];
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < rt.K) { cv[k] = pk_expf_cr(cv[k] - m); s += cv[k]; }
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < rt.K) {
            wp[k] = cv[k] / s;
            ws[k] = wp[k] * rt.routed_scale;
        }
}

// Where the expert kernels select their own experts, one wave also publishes
// the selection and the weights for the launches (and the host) after them.
template <int KM = 16>
__device__ __forceinline__ void pk_wave_route(const pk_route_args &rt, int *ci, float *ws, float *wp) {
    pk_wave_route<KM>(rt, pk_load_wave_logits(rt.logits, rt.E), ci, ws, wp);
}

template <int KM = 16>
__device__ __forceinline__ void pk_wave_route_publish(const pk_route_args &rt, const pk_wave_logits &lg) {
    int ci[KM];
    float ws[KM], wp[KM];
    pk_wave_route<KM>(rt, lg, ci, ws, wp);
    if ((threadIdx.x & 63) != 0) return;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < rt.K) {
            rt.sel[k] = ci[k];
            if (rt.w_soft) rt.w_soft[k] = wp[k];
            rt.w_scaled[k] = ws[k];
        }
}

template <int KM = 16>
__device__ __forceinline__ void pk_wave_route_publish(const pk_route_args &rt) {
    pk_wave_route_publish<KM>(rt, pk_load_wave_logits(rt.logits, rt.E));
}

// ─────────────── integer-dot arithmetic (opt-in to bit-exactness) ───────────────
// Not picchio's arithmetic: the expert GEMV on v_dot8c_i32_i4. An input row
// is cut into half-groups of 32 values; each has an exponent k (frexp of its
// largest magnitude, 0 if all are zero) and the integers A = rint(x 2^(18-k))
// (|A| <= 2^18) written as five balanced base-16 digits, A = sum_i d_i 16^i,
// d_i in [-8, 7] (which reach -559240 .. 489335: 2^19 would not fit). Record of a half-group (PK_XQ_INTS ints): dword 4i + w
// holds digit i of columns 8w .. 8w+7 (nibble n = column 8w+n), int 20 = k
// (PK_XQ_INTS ints with padding).
// The store holds each weight nibble as q ^ 8, the signed 4-bit q - 8
// (k_i4_repack), so per half-group and digit four v_dot8 give
// sum (q-8) d_i exactly, and
// C = sum_i 16^i P_i = sum (q-8) A exactly (|C| <= 2^26). The row's value is
// then sum over groups g and halves h of (16 s_g) 2^(k_h - 22) C_gh, folded
// in fp32 in a fixed order (pk_dot_group).
// 32 values of a half-group: lane src(c) = c * LS holds column c's value v
// (has: the lane holds one). Returns int `lane` of the record (lanes
// 0..PK_XQ_INTS-1).
template <int LS>
__device__ __forceinline__ int32_t pk_record_word(float v, bool has) {
    const int lane = threadIdx.x & 63;
    // the largest magnitude (non-negative floats order as their bits)
    const float m = __uint_as_float(pk_wave_max_u32(__float_as_uint(has ? fabsf(v) : 0.0f)));
    int k = 0;
    if (m > 0.0f) (void)frexpf(m, &k);
    int A = has ? (int)rintf(ldexpf(v, 18 - k)) : 0;
    // five balanced digits of A, packed one per nibble
    uint32_t dig = 0;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int d = ((A + 8) & 15) - 8;
        dig |= (uint32_t)(d & 15) << (4 * i);
        A = (A - d) >> 4;
    }
    // lane 4i + w gathers digit i of columns 8w .. 8w+7
    const int i = lane >> 2, w = lane & 3;
    uint32_t word = 0;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        const uint32_t src = (uint32_t)__shfl((int)dig, (8 * w + n) * LS, 64);
        word |= ((src >> (4 * (i < 5 ? i : 0))) & 15u) << (4 * n);
    }
    return lane < 20 ? (int32_t)word : lane == 20 ? k : 0;   // then padding
}

// The record of a half-group written to dst (lanes 0..PK_XQ_INTS-1 store):
// lane src(c) holds column c's value v (has: the lane holds one).
template <int LS>
__device__ __forceinline__ void pk_write_digits(float v, bool has, int32_t *dst) {
    const int32_t word = pk_record_word<LS>(v, has);
    if ((threadIdx.x & 63) < PK_XQ_INTS) dst[threadIdx.x & 63] = word;
}

// One 64-column group of one row on the integer dot: wa / wb = the stored
// nibbles (q ^ 8) of columns 0..31 / 32..63, x0 / x1 = the two half-group records
// (wave-uniform), s16 = the stored scale (16 s). Returns the group's value.
// XP: any pointer to the records (global, constant or LDS address space).
template <typename XP>
__device__ __forceinline__ float pk_dot_group(uint4 wa, uint4 wb, XP x0, XP x1, float s16) {
    float t = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 w = h ? wb : wa;
        const XP xq = h ? x1 : x0;
        const int w0 = (int)w.x, w1 = (int)w.y, w2 = (int)w.z, w3 = (int)w.w;
        int P[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            int p = __builtin_amdgcn_sdot8(w0, xq[4 * i + 0], 0, false);
            p = __builtin_amdgcn_sdot8(w1, xq[4 * i + 1], p, false);
            p = __builtin_amdgcn_sdot8(w2, xq[4 * i + 2], p, false);
            p = __builtin_amdgcn_sdot8(w3, xq[4 * i + 3], p, false);
            P[i] = p;
        }
        const int C = P[0] + 16 * (P[1] + 16 * (P[2] + 16 * (P[3] + 16 * P[4])));
        const float S = ldexpf(s16, xq[20] - 22);
        t = h ? __builtin_fmaf(S, (float)C, t) : S * (float)C;
    }
    return t;
}
