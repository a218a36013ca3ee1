// pk_dev.h — small device helpers shared by the dense and decode kernels.
#pragma once
#include "pk_internal.h"

__device__ __forceinline__ double pk_dev_wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
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
