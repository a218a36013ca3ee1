// pk_dev.h — small device helpers shared by the dense and decode kernels.
#pragma once
#include "pk_internal.h"

// ───────────────────────── wave sums ─────────────────────────
// Sum over the 64 lanes of a wave (all active), every lane getting it. The
// tree is fixed: lane ^ 1, ^ 2, ^ 4, ^ 8 within each row of 16 lanes (own +
// partner at each step), then the four row sums r0..r3 as (r0 + r1) +
// (r2 + r3). The in-row steps are DPP moves (quad permutes and row
// rotations) and the row sums are lane reads: a few VALU cycles each
// instead of one LDS permute per step. Every kernel reduces with these, so
// the kernels that restate another's arithmetic keep its bits.
template <int CTRL>
__device__ __forceinline__ int pk_dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float pk_dpp_f(float v) {
    return __int_as_float(pk_dpp_i<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ double pk_dpp_d(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)pk_dpp_i<CTRL>((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)pk_dpp_i<CTRL>((int)(uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double pk_readlane_d(double v, int l) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// DPP controls: quad_perm [1,0,3,2] (lane ^ 1), [2,3,0,1] (lane ^ 2); row
// rotations by 4 and 12 (lane ^ 4 is +4 or -4 in the row), by 8 (lane ^ 8)
__device__ __forceinline__ float pk_wave_sum_f(float v) {
    v = v + pk_dpp_f<0xB1>(v);
    v = v + pk_dpp_f<0x4E>(v);
    const float p4 = pk_dpp_f<0x124>(v), m4 = pk_dpp_f<0x12C>(v);
    v = v + ((threadIdx.x & 4) ? m4 : p4);
    v = v + pk_dpp_f<0x128>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ double pk_wave_sum_d(double v) {
    v = v + pk_dpp_d<0xB1>(v);
    v = v + pk_dpp_d<0x4E>(v);
    const double p4 = pk_dpp_d<0x124>(v), m4 = pk_dpp_d<0x12C>(v);
    v = v + ((threadIdx.x & 4) ? m4 : p4);
    v = v + pk_dpp_d<0x128>(v);
    return (pk_readlane_d(v, 0) + pk_readlane_d(v, 16)) + (pk_readlane_d(v, 32) + pk_readlane_d(v, 48));
}

__device__ __forceinline__ double pk_dev_wave_sum_d(double v) { return pk_wave_sum_d(v); }

// Maximum over the wave (fmaxf: a NaN lane is ignored), every lane getting
// it; any tree gives the same value.
__device__ __forceinline__ float pk_wave_max_f(float v) {
    v = fmaxf(v, pk_dpp_f<0xB1>(v));
    v = fmaxf(v, pk_dpp_f<0x4E>(v));
    v = fmaxf(v, pk_dpp_f<0x124>(v));
    v = fmaxf(v, pk_dpp_f<0x128>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ───────────── range-checked loads through a buffer resource ─────────────
// A raw buffer resource over [base, base + bytes): a load at a byte offset
// at or past `bytes` returns zeros instead of touching memory, so that a
// kernel can issue a fixed number of loads per lane without guards (each
// guarded load would be waited for on its own) and without a 64-bit address
// per load. Offsets are 32-bit; each load is 4 or 16 bytes, at offsets that
// are multiples of its size, with `bytes` a multiple of 16 for the 16-byte
// form.
typedef __amdgpu_buffer_rsrc_t pk_buf_t;

__device__ __forceinline__ pk_buf_t pk_buf(const void *base, uint32_t bytes) {
    // word 3 = 0x00020000: 32-bit data format, the gfx9 raw-buffer setting
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// streaming (non-temporal) 16-byte load, for weights read once
__device__ __forceinline__ pk_f32x4 pk_buf_load4_nt(pk_buf_t r, uint32_t off) {
    const pk_i32x4 v = __builtin_bit_cast(pk_i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
    return __builtin_bit_cast(pk_f32x4, v);
}
__device__ __forceinline__ float4 pk_buf_load4(pk_buf_t r, uint32_t off) {
    const pk_f32x4 v = __builtin_bit_cast(pk_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float pk_buf_load_f32(pk_buf_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// RMSNorm scale of x[0..D) for a 256-thread block, every thread getting it:
// 1 / sqrtf((float)(sum x^2 / D) + eps) with a double sum (thread t adds
// x[t], x[t + 256], ... in order, then the wave tree and the block combine;
// every user shares this order, hence the same bits), so that a consumer can
// normalise its input on the fly: (x * r) * w.
//
// In two steps, so that a kernel can issue the loads of x before its weight
// loads and run the reduction while the weights stream in: pk_rms_load reads
// thread t's first NV values x[t + 256 k], pk_rms_finish adds them (and any
// further values, D > 256 NV; read as zeros with x_zero) and combines the
// block. pk_block_rms_scale does both in one call.
template <int NV>
__device__ __forceinline__ void pk_rms_load(const float *__restrict__ x, int D, float (&v)[NV]) {
    // buffer loads keep every load unconditional (entries past D read as
    // zero), so that all NV go out back to back: a guarded load is issued
    // and waited for on its own
    const pk_buf_t r = pk_buf(x, (uint32_t)D * 4u);
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = pk_buf_load_f32(r, ((uint32_t)threadIdx.x + 256u * k) * 4u);
}

template <int NV>
__device__ __forceinline__ float pk_rms_finish(const float (&v)[NV], const float *__restrict__ x, int D,
                                               float eps, double *part, bool x_zero = false) {
    // (entries past D hold zeros from pk_rms_load: adding 0 to the
    // non-negative sum leaves every bit of it unchanged)
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < NV; ++k) acc += (double)v[k] * (double)v[k];
    for (int i = threadIdx.x + 256 * NV; i < D; i += 256) {
        const double xi = x_zero ? 0.0 : (double)x[i];
        acc += xi * xi;
    }
    acc = pk_dev_wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    const double ms = (part[0] + part[1]) + (part[2] + part[3]);
    return 1.0f / sqrtf((float)(ms / D) + eps);
}

__device__ __forceinline__ float pk_block_rms_scale(const float *__restrict__ x, int D, float eps,
                                                    double *part) {
    float v[12];
    pk_rms_load(x, D, v);
    return pk_rms_finish(v, x, D, eps, part);
}

__device__ __forceinline__ float4 pk_norm4(float4 h, float r, float4 w) {
    return make_float4(h.x * r * w.x, h.y * r * w.y, h.z * r * w.z, h.w * r * w.w);
}
