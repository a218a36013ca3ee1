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

__device__ __forceinline__ float pk_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

// GPT-OSS clamped SwiGLU of one (gate, up) pair (picchio.c:1416-1424).
__device__ __forceinline__ float pk_swiglu(float gate, float up, float lim, float alpha) {
    if (gate > lim) gate = lim;
    if (up > lim) up = lim;
    if (up < -lim) up = -lim;
    return (up + 1.0f) * gate * pk_sigmoid(alpha * gate);
}

