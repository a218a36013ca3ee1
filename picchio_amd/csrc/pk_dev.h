// pk_dev.h — small device helpers shared by the dense and decode kernels.
#pragma once
#include "pk_internal.h"

__device__ __forceinline__ double pk_dev_wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// RMSNorm scale of x[0..D) for a 256-thread block, every thread getting it:
// 1 / sqrtf((float)(sum x^2 / D) + eps) with k_rmsnorm's double sum (same
// per-thread partials, wave tree and block combine, hence the same bits), so
// a consumer can normalise its input on the fly: (x * r) * w.
__device__ __forceinline__ float pk_block_rms_scale(const float *__restrict__ x, int D, float eps,
                                                    double *part) {
    double acc = 0.0;
    for (int i = threadIdx.x; i < D; i += 256) acc += (double)x[i] * (double)x[i];
    acc = pk_dev_wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    const double ms = (part[0] + part[1]) + (part[2] + part[3]);
    return 1.0f / sqrtf((float)(ms / D) + eps);
}

__device__ __forceinline__ float4 pk_norm4(float4 h, float r, float4 w) {
    return make_float4(h.x * r * w.x, h.y * r * w.y, h.z * r * w.z, h.w * r * w.w);
}
