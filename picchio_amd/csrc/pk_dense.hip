// pk_dense.hip — fp32 / int8 GEMV, RMSNorm, router top-k, combine, and the
// on-device synthetic weight generator.
#include "pk_internal.h"
#include <algorithm>
#include "pk_dev.h"
#include "pk_i4_device.h"
#include "pk_synth.h"

// ───────────────────────── wave reductions ─────────────────────────
__device__ __forceinline__ float pk_wave_sum(float v) { return pk_wave_sum_f(v); }

// ───────────────────────── fp32 GEMV ─────────────────────────
// y[s][o] = x[s] . W[o] (+ bias[o]), matmul_f32 (quant.h:117-148). fp32 sum
// in a fixed tree order (not the reference's 8-lane order: within 1e-6
// relative, checked against the oracle). Every lane issues its loads for a
// chunk before the FMAs that consume them, so a row costs one or two memory
// round trips rather than one per float4.
constexpr int GEMV_U = 4;           // float4 per lane per chunk

// Large O: one wave per RPW rows, lanes stride the row in float4 (each load
// instruction reads 1 KiB contiguous).
// NORM: x is the raw residual row and nw the RMSNorm weight; the block
// normalises it on the fly (pk_block_rms_scale), fusing rmsnorm into the GEMV.
template <int RPW, bool NORM = false>
__global__ __launch_bounds__(256) void k_gemv_f32(float *__restrict__ y, const float *__restrict__ x,
                                                  const float *__restrict__ W,
                                                  const float *__restrict__ bias, int S, int I, int O,
                                                  const float *__restrict__ nw = nullptr, float eps = 0.f) {
    __shared__ double npart[4];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * RPW;
    const int s = blockIdx.y;
    const float *xs = x + (int64_t)s * I;
    const int n4 = I >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
    const float4 *nw4 = reinterpret_cast<const float4 *>(nw);
    float rn = 1.0f;
    if constexpr (NORM) rn = pk_block_rms_scale(xs, I, eps, npart);
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
    for (int i0 = lane; i0 < n4; i0 += 64 * GEMV_U) {
        float4 xv[GEMV_U];
        pk_f32x4 wv[RPW][GEMV_U];
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u) {
            const int i = i0 + u * 64;
            xv[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (NORM) xv[u] = i < n4 ? pk_norm4(xv[u], rn, nw4[i]) : xv[u];
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const int o = min(row0 + r, O - 1);
                wv[r][u] = i < n4 ? __builtin_nontemporal_load(
                                        reinterpret_cast<const pk_f32x4 *>(W + (int64_t)o * I) + i)
                                  : pk_f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u)
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                acc[r] = __builtin_fmaf(xv[u].x, wv[r][u].x, acc[r]);
                acc[r] = __builtin_fmaf(xv[u].y, wv[r][u].y, acc[r]);
                acc[r] = __builtin_fmaf(xv[u].z, wv[r][u].z, acc[r]);
                acc[r] = __builtin_fmaf(xv[u].w, wv[r][u].w, acc[r]);
            }
    }
    for (int i = (n4 << 2) + lane; i < I; i += 64) {
        const float xi = NORM ? xs[i] * rn * nw[i] : xs[i];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int o = min(row0 + r, O - 1);
            acc[r] = __builtin_fmaf(xi, W[(int64_t)o * I + i], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const float v = pk_wave_sum(acc[r]);
        const int o = row0 + r;
        if (lane == 0 && o < O) y[(int64_t)s * O + o] = bias ? v + bias[o] : v;
    }
}

// Small O: one workgroup per row, 256 threads split the row. With nw, xs is
// the raw row and is normalised on the fly with scale rn (x * rn * nw).
__device__ __forceinline__ float pk_row_dot_block(const float *__restrict__ xs,
                                                  const float *__restrict__ w, int I, float *red,
                                                  const float *__restrict__ nw = nullptr, float rn = 1.0f) {
    const int n4 = I >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    const float4 *nw4 = reinterpret_cast<const float4 *>(nw);
    float acc = 0.0f;
    for (int i0 = threadIdx.x; i0 < n4; i0 += 256 * GEMV_U) {
        float4 xv[GEMV_U], wv[GEMV_U];
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u) {
            const int i = i0 + u * 256;
            xv[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            if (nw && i < n4) xv[u] = pk_norm4(xv[u], rn, nw4[i]);
            wv[u] = i < n4 ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u) {
            acc = __builtin_fmaf(xv[u].x, wv[u].x, acc);
            acc = __builtin_fmaf(xv[u].y, wv[u].y, acc);
            acc = __builtin_fmaf(xv[u].z, wv[u].z, acc);
            acc = __builtin_fmaf(xv[u].w, wv[u].w, acc);
        }
    }
    for (int i = (n4 << 2) + threadIdx.x; i < I; i += 256)
        acc = __builtin_fmaf(nw ? xs[i] * rn * nw[i] : xs[i], w[i], acc);
    acc = pk_wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void k_gemv_f32_rows(float *__restrict__ y, const float *__restrict__ x,
                                                       const float *__restrict__ W,
                                                       const float *__restrict__ bias, int S, int I, int O,
                                                       const float *__restrict__ nw = nullptr, float eps = 0.f) {
    __shared__ float red[4];
    __shared__ double npart[4];
    const int o = blockIdx.x, s = blockIdx.y;
    const float rn = nw ? pk_block_rms_scale(x + (int64_t)s * I, I, eps, npart) : 1.0f;
    const float v = pk_row_dot_block(x + (int64_t)s * I, W + (int64_t)o * I, I, red, nw, rn);
    if (threadIdx.x == 0) y[(int64_t)s * O + o] = bias ? v + bias[o] : v;
}

// ───────────────── skinny fp32 GEMM on the matrix cores ─────────────────
// Y[s][o] = (residual ? Y[s][o] : 0) + (X[s] . W[o] + bias[o]) for s < S <= 32.
// A workgroup of 4 waves owns 64 output rows (16 per wave) over one K range.
// The 32 input rows' columns of the range pass through LDS once per
// workgroup (SK_ST steps of 32 columns per stage, double-buffered, staged a
// stage ahead by all threads), so that in L2 traffic the input rows cost
// half the weight bytes rather than twice (one read per 16 rows). Per 32
// columns a lane loads two float4 of its W row (o = o0 + 16 wave + lane % 16,
// columns k0 + 8 (lane / 16) .. +7: the four lane groups read 128 contiguous
// bytes of each row; W runs four steps ahead in a register ring), reads the
// same columns of its two input rows (s = lane % 16 and 16 + lane % 16) from
// LDS, then issues 16 v_mfma_f32_16x16x4_f32 (8 steps x 2 halves of the
// inputs); step i takes element i of every lane's 8 columns. Few output rows
// split K over grid.y workgroups: their partial tiles go to a workspace that
// k_gemm_splits adds in split order (deterministic). fp32 products and sums
// throughout (not the reference's 8-lane order: within 1e-6 relative,
// checked in tests).
typedef float pk_f32x4v __attribute__((ext_vector_type(4)));
constexpr int SK_WAVES = 4, SK_ROWS = 16 * SK_WAVES;
constexpr int SK_ST = 4;                  // 32-column steps per LDS stage
constexpr int SK_PAD = 36;                // floats per LDS input row (32 + 4: conflict-free 16-byte reads)

// TILED: W is the tile-order copy (pk_launch_tile_skinny): each weight load
// reads one contiguous kilobyte instead of sixteen 64-byte pieces of rows.
template <bool TILED>
__global__ __launch_bounds__(64 * SK_WAVES) void k_gemm_mfma32(float *__restrict__ Y, const float *__restrict__ X,
                                                               const float *__restrict__ W,
                                                               const float *__restrict__ bias, int S, int I,
                                                               int O, int residual, int kchunk,
                                                               float *__restrict__ ws) {
    __shared__ __attribute__((aligned(16))) float xs[2][SK_ST][32][SK_PAD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int o0 = blockIdx.x * SK_ROWS + 16 * wave;
    const int r16 = lane & 15, kq = lane >> 4;
    const float *wrow = W + (int64_t)min(o0 + r16, O - 1) * I;
    const int kb = blockIdx.y * kchunk, ke = min(I, kb + kchunk);
    const int nstage = (ke - kb + 32 * SK_ST - 1) / (32 * SK_ST);
    // stage loads: thread t carries float4 e = t + 256 u (u < 4) of the
    // stage's 32 rows x 128 columns: row e / 32, column 4 (e % 32)
    float4 xr[4];
    auto load_x = [&](int t) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = threadIdx.x + 64 * SK_WAVES * u, sr = e >> 5, c = kb + 128 * t + 4 * (e & 31);
            xr[u] = c < ke ? *reinterpret_cast<const float4 *>(X + (int64_t)min(sr, S - 1) * I + c)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = threadIdx.x + 64 * SK_WAVES * u, sr = e >> 5, c4 = e & 31;
            *reinterpret_cast<float4 *>(&xs[buf][c4 >> 3][sr][4 * (c4 & 7)]) = xr[u];
        }
    };
    // this lane's 8 columns of W at K0 (zero past ke)
    const int n_step = (I + 31) >> 5;
    const float *wtile = W + (int64_t)min(o0 >> 4, (O - 1) >> 4) * n_step * 512 + lane * 4;
    auto load_w = [&](int k0, float4 (&wv)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int k = k0 + 8 * kq + 4 * j;
            if (k < ke) {
                const float *src = TILED ? wtile + (int64_t)(k0 >> 5) * 512 + j * 256 : wrow + k;
                const pk_f32x4v t = __builtin_nontemporal_load(reinterpret_cast<const pk_f32x4v *>(src));
                wv[j] = make_float4(t.x, t.y, t.z, t.w);
            } else {
                wv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    pk_f32x4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float4 w0[2], w1[2], w2[2], w3[2];
    load_w(kb, w0);
    load_w(kb + 32, w1);
    load_w(kb + 64, w2);
    load_w(kb + 96, w3);
    load_x(0);
    store_x(0);
    __syncthreads();
    auto step = [&](int buf, int i, float4 (&wv)[2]) {
        const float *xa = &xs[buf][i][r16][8 * kq], *xb = &xs[buf][i][16 + r16][8 * kq];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float4 a = *reinterpret_cast<const float4 *>(xa + 4 * j);
            const float4 b = *reinterpret_cast<const float4 *>(xb + 4 * j);
            const float wv_[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
            const float av_[4] = {a.x, a.y, a.z, a.w};
            const float bv_[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av_[e], wv_[e], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(bv_[e], wv_[e], acc1, 0, 0, 0);
            }
        }
    };
    for (int t = 0; t < nstage; ++t) {
        const int buf = t & 1, k0 = kb + 128 * t;
        if (t + 1 < nstage) load_x(t + 1);
        // past ke the W ring holds zeros and the staged columns are zero
        step(buf, 0, w0);
        load_w(k0 + 128, w0);
        step(buf, 1, w1);
        load_w(k0 + 160, w1);
        step(buf, 2, w2);
        load_w(k0 + 192, w2);
        step(buf, 3, w3);
        load_w(k0 + 224, w3);
        if (t + 1 < nstage) store_x(buf ^ 1);
        __syncthreads();
    }
    // D layout of a 16x16 MFMA: lane l, element v -> input 4 (l / 16) + v, row l % 16
    const int orow = o0 + r16;
    if (orow >= O) return;
    const bool split = gridDim.y > 1;
    const float bv = !split && bias ? bias[orow] : 0.0f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
        const int srow = (v < 4 ? 0 : 16) + 4 * kq + (v & 3);
        if (srow >= S) continue;
        const float sum = v < 4 ? acc0[v] : acc1[v - 4];
        if (split) {
            ws[((int64_t)blockIdx.y * 32 + srow) * O + orow] = sum;
        } else {
            float *yp = Y + (int64_t)srow * O + orow;
            const float val = bias ? sum + bv : sum;
            *yp = residual ? *yp + val : val;
        }
    }
}

// The split-K partial tiles of k_gemm_mfma32 added in split order, + bias,
// (+ Y when residual).
__global__ __launch_bounds__(256) void k_gemm_splits(float *__restrict__ Y, const float *__restrict__ ws,
                                                     const float *__restrict__ bias, int S, int O, int splits,
                                                     int residual) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)S * O) return;
    const int srow = (int)(i / O), orow = (int)(i - (int64_t)srow * O);
    float sum = ws[(int64_t)srow * O + orow];
    for (int k = 1; k < splits; ++k) sum = sum + ws[((int64_t)k * 32 + srow) * O + orow];
    if (bias) sum = sum + bias[orow];
    Y[i] = residual ? Y[i] + sum : sum;
}

__global__ void k_tile_skinny(const float *__restrict__ W, int O, int I, float *__restrict__ Wt, int64_t n4) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n4) return;
    const int n_step = (I + 31) >> 5;
    const int64_t t = q >> 7;                                 // tile: 128 float4
    const int w = (int)(q & 127), j = w >> 6, l = w & 63;
    const int R = (int)(t / n_step), Sx = (int)(t - (int64_t)R * n_step);
    const int row = min(16 * R + (l & 15), O - 1), col = 32 * Sx + 8 * (l >> 4) + 4 * j;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (col < I) v = *reinterpret_cast<const float4 *>(W + (int64_t)row * I + col);
    reinterpret_cast<float4 *>(Wt)[q] = v;
}

int64_t pk_skinny_tile_floats(int O, int I) {
    return (int64_t)((O + 15) / 16) * ((I + 31) / 32) * 512;
}

int pk_launch_tile_skinny(const float *W, int O, int I, float *Wt, hipStream_t st) {
    PK_CHECK(W && Wt && O > 0 && I > 0 && (I & 3) == 0, PK_ERR_ARG, "tile skinny: O=%d I=%d", O, I);
    const int64_t n4 = pk_skinny_tile_floats(O, I) / 4;
    hipLaunchKernelGGL(k_tile_skinny, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, W, O, I, Wt, n4);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_gemm_skinny(float *y, const float *x, const float *W, const float *bias, int S, int I, int O,
                          int residual, hipStream_t st, float *ws, int64_t ws_floats, int *splits_out,
                          const float *Wt) {
    PK_CHECK(S > 0 && S <= 32 && I > 0 && O > 0, PK_ERR_ARG, "skinny gemm: bad shape");
    PK_CHECK(((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0 && (I & 3) == 0, PK_ERR_UNSUPPORTED,
             "skinny gemm: needs 16-byte aligned rows (I=%d)", I);
    const int rb = (O + SK_ROWS - 1) / SK_ROWS;
    // split K when the row blocks alone leave CUs idle: ~512 workgroups,
    // at least two LDS stages (256 columns) each, as the workspace allows
    int splits = 1, kchunk = (I + 127) / 128 * 128;
    if (ws && rb < 512) {
        const int want = std::min((512 + rb - 1) / rb, std::max(1, I / 256));
        const int cap = (int)std::min<int64_t>(want, ws_floats / ((int64_t)32 * O));
        if (cap > 1) {
            kchunk = ((I + cap - 1) / cap + 127) / 128 * 128;
            splits = (I + kchunk - 1) / kchunk;
        }
    }
    if (Wt)
        hipLaunchKernelGGL(k_gemm_mfma32<true>, dim3(rb, splits), dim3(64 * SK_WAVES), 0, st, y, x, Wt, bias, S, I,
                           O, residual, kchunk, ws);
    else
        hipLaunchKernelGGL(k_gemm_mfma32<false>, dim3(rb, splits), dim3(64 * SK_WAVES), 0, st, y, x, W, bias, S, I,
                           O, residual, kchunk, ws);
    PK_HIP(hipGetLastError());
    if (splits_out) *splits_out = splits;
    if (splits > 1 && !splits_out) {
        hipLaunchKernelGGL(k_gemm_splits, dim3((unsigned)(((int64_t)S * O + 255) / 256)), dim3(256), 0, st, y, ws,
                           bias, S, O, splits, residual);
        PK_HIP(hipGetLastError());
    }
    return PK_OK;
}

int pk_launch_gemv_f32(float *y, const float *x, const float *W, const float *bias,
                       int S, int I, int O, hipStream_t st, float *ws, int64_t ws_floats, const float *Wt) {
    PK_CHECK(S > 0 && I > 0 && O > 0 && S <= 65535, PK_ERR_ARG, "gemv f32: bad shape");
    PK_CHECK(((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0 && (I & 3) == 0,
             PK_ERR_UNSUPPORTED, "gemv f32: needs 16-byte aligned rows (I=%d)", I);
    if (S >= 4 && O >= 256) {
        // several inputs: one weight read per block of up to 32 inputs
        for (int s0 = 0; s0 < S; s0 += 32)
            PK_TRY(pk_launch_gemm_skinny(y + (int64_t)s0 * O, x + (int64_t)s0 * I, W, bias,
                                         S - s0 < 32 ? S - s0 : 32, I, O, 0, st, ws, ws_floats, nullptr, Wt));
        return PK_OK;
    }
    if (O <= 2048) {
        hipLaunchKernelGGL(k_gemv_f32_rows, dim3(O, S), dim3(256), 0, st, y, x, W, bias, S, I, O);
    } else {
        constexpr int RPW = 2;
        const int rows_per_block = 4 * RPW;
        hipLaunchKernelGGL((k_gemv_f32<RPW>), dim3((O + rows_per_block - 1) / rows_per_block, S),
                           dim3(256), 0, st, y, x, W, bias, S, I, O);
    }
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── int8 GEMV ─────────────────────────
// matmul_q8 (quant.h:152-186): fp32 accumulation of x*q, times the row scale.
__global__ __launch_bounds__(256) void k_gemv_q8(float *__restrict__ y, const float *__restrict__ x,
                                                 const int8_t *__restrict__ q,
                                                 const float *__restrict__ sc, int S, int I, int O) {
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int s = blockIdx.y;
    if (o >= O) return;
    const float *xs = x + (int64_t)s * I;
    const int8_t *w = q + (int64_t)o * I;
    float acc = 0.0f;
    const int n16 = I >> 4;
    for (int i = lane; i < n16; i += 64) {
        const pk_i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const pk_i32x4 *>(w) + i);
        const int32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc = __builtin_fmaf(xs[i * 16 + k * 4 + b], (float)(int8_t)(d[k] >> (8 * b)), acc);
    }
    for (int i = (n16 << 4) + lane; i < I; i += 64) acc = __builtin_fmaf(xs[i], (float)w[i], acc);
    const float v = pk_wave_sum(acc);
    if (lane == 0) y[(int64_t)s * O + o] = v * sc[o];
}

int pk_launch_gemv_f32_norm(float *y, const float *h, const float *nw, float eps, const float *W,
                            const float *bias, int I, int O, hipStream_t st) {
    PK_CHECK(I > 0 && O > 0 && nw, PK_ERR_ARG, "gemv f32 norm: bad shape");
    PK_CHECK(((uintptr_t)W & 15) == 0 && ((uintptr_t)h & 15) == 0 && ((uintptr_t)nw & 15) == 0 && (I & 3) == 0,
             PK_ERR_UNSUPPORTED, "gemv f32 norm: needs 16-byte aligned rows (I=%d)", I);
    if (O <= 2048) {
        hipLaunchKernelGGL(k_gemv_f32_rows, dim3(O, 1), dim3(256), 0, st, y, h, W, bias, 1, I, O, nw, eps);
    } else {
        constexpr int RPW = 2;
        hipLaunchKernelGGL((k_gemv_f32<RPW, true>), dim3((O + 4 * RPW - 1) / (4 * RPW), 1), dim3(256), 0, st, y,
                           h, W, bias, 1, I, O, nw, eps);
    }
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_gemv_q8(float *y, const float *x, const int8_t *q, const float *s,
                      int S, int I, int O, hipStream_t st) {
    PK_CHECK(S > 0 && I > 0 && O > 0 && S <= 65535, PK_ERR_ARG, "gemv q8: bad shape");
    PK_CHECK(((uintptr_t)q & 15) == 0 && (I & 15) == 0, PK_ERR_UNSUPPORTED,
             "gemv q8: needs I %% 16 == 0 and 16-byte aligned rows");
    hipLaunchKernelGGL(k_gemv_q8, dim3((O + 3) / 4, S), dim3(256), 0, st, y, x, q, s, S, I, O);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// Per-row INT4 (quant.h:191-253): fp32 sum of x*(nib-8), times the row scale.
__global__ __launch_bounds__(256) void k_gemv_i4_row(float *__restrict__ y, const float *__restrict__ x,
                                                     const uint8_t *__restrict__ q4,
                                                     const float *__restrict__ sc, int S, int I, int O) {
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int s = blockIdx.y;
    if (o >= O) return;
    const float *xs = x + (int64_t)s * I;
    const uint8_t *w = q4 + (int64_t)o * ((I + 1) / 2);
    float acc = 0.0f;
    for (int i = lane; i < I; i += 64) {
        const uint8_t b = w[i >> 1];
        const int nib = (i & 1) ? (b >> 4) : (b & 15);
        acc = __builtin_fmaf(xs[i], (float)(nib - 8), acc);
    }
    const float v = pk_wave_sum(acc);
    if (lane == 0) y[(int64_t)s * O + o] = v * sc[o];
}

int pk_launch_i4_rowscale_gemv(float *y, const float *x, const uint8_t *q4, const float *s,
                               int S, int I, int O, hipStream_t st) {
    PK_CHECK(S > 0 && I > 0 && O > 0 && S <= 65535, PK_ERR_ARG, "gemv i4 row: bad shape");
    hipLaunchKernelGGL(k_gemv_i4_row, dim3((O + 3) / 4, S), dim3(256), 0, st, y, x, q4, s, S, I, O);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── RMSNorm ─────────────────────────
// rmsnorm (quant.h:396-402): sum of x^2 in double (each term exact), one
// float rsqrt, out = (x * r) * w. Only the summation order of the double
// accumulator differs from the reference, far below float resolution.
__global__ __launch_bounds__(256) void k_rmsnorm(float *out, const float *x, const float *w, int D,
                                                 float eps) {
    __shared__ double part[4];
    const int t = blockIdx.x;
    const float *xr = x + (int64_t)t * D;
    // every load goes out before the reduction (clamped, unconditional)
    float v[12], wv[12];
    pk_rms_load(xr, D, v);
    pk_rms_load(w, D, wv);
    const float r = pk_rms_finish(v, xr, D, eps, part);
    float *o = out + (int64_t)t * D;
#pragma unroll
    for (int k = 0; k < 12; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i < D) o[i] = v[k] * r * wv[k];
    }
    for (int i = threadIdx.x + 256 * 12; i < D; i += 256) o[i] = xr[i] * r * w[i];
}

int pk_launch_rmsnorm(float *out, const float *x, const float *w, int D, float eps, int T,
                      hipStream_t st) {
    PK_CHECK(D > 0 && T > 0, PK_ERR_ARG, "rmsnorm: bad shape");
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(256), 0, st, out, x, w, D, eps);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── router top-k ─────────────────────────
// picchio.c:1330-1355: K rounds of argmax with strict '>' (ties -> lowest
// index, already-chosen experts skipped), softmax over the K raw logits
// (quant.h:406-412), weight_k * routed_scale for the combine (:1445).
// One wave per token; logits [T][E] -> sel [T][K], w [T][K].
__device__ __forceinline__ void topk_softmax_row(int t, const float *logits, int E, int K, float routed_scale,
                                                 int32_t *sel, float *w_scaled, float *w_soft) {
    const int lane = threadIdx.x;
    const float *lg = logits + (int64_t)t * E;
    // each lane holds experts lane, lane+64 (E <= 128)
    float v0 = lane < E ? lg[lane] : -INFINITY;
    float v1 = lane + 64 < E ? lg[lane + 64] : -INFINITY;
    bool t0 = lane >= E, t1 = lane + 64 >= E;
    int chosen[16];
    float val[16];
    for (int k = 0; k < K; ++k) {
        // best of this lane (lower index first on ties)
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
        chosen[k] = bi;
        val[k] = bv;
        if (bi == lane) t0 = true;
        if (bi == lane + 64) t1 = true;
    }
    if (lane == 0) {
        float m = -1e30f;
        for (int k = 0; k < K; ++k) if (val[k] > m) m = val[k];
        float e[16], s = 0.0f;
        for (int k = 0; k < K; ++k) { e[k] = pk_expf_cr(val[k] - m); s += e[k]; }
        for (int k = 0; k < K; ++k) {
            const float p = e[k] / s;
            sel[(int64_t)t * K + k] = chosen[k];
            if (w_soft) w_soft[(int64_t)t * K + k] = p;
            w_scaled[(int64_t)t * K + k] = p * routed_scale;
        }
    }
}

__global__ __launch_bounds__(64) void k_topk_softmax(const float *logits, int E, int K,
                                                     float routed_scale, int32_t *sel,
                                                     float *w_scaled, float *w_soft) {
    topk_softmax_row(blockIdx.x, logits, E, K, routed_scale, sel, w_scaled, w_soft);
}

// The same top-k for T rows and, in the launch's other blocks, the
// half-group records of x[0..n) (k_act_records' body): the two depend on
// nothing of each other, and one launch of both saves a dependent launch
// in the batched MoE on the integer dot.
__global__ __launch_bounds__(64) void k_topk_records(const float *logits, int T, int E, int K, float routed_scale,
                                                     int32_t *sel, float *w_scaled, const float *x, int n,
                                                     int32_t *rec) {
    if ((int)blockIdx.x < T) {
        topk_softmax_row(blockIdx.x, logits, E, K, routed_scale, sel, w_scaled, nullptr);
        return;
    }
    const int b = (int)blockIdx.x - T, lane = threadIdx.x;
    const int i = b * 32 + lane;
    const bool has = lane < 32 && i < n;
    pk_write_digits<1>(x[has ? i : 0], has, rec + (int64_t)b * PK_XQ_INTS);
}

// Router + top-k in one launch: block e computes logit e (one row per
// block), stores it device-coherently and counts itself in; the last block
// to arrive runs top-k + softmax (same arithmetic as k_topk_softmax) and
// re-arms the counter. (picchio.c:1316-1355)
__device__ __forceinline__ void pk_st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float pk_ld_dev(float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// With nw, x is the raw residual row: every block normalises it on the fly
// (rmsnorm fused, same bits) and block e also writes its slice of the
// normalised row to hn for the expert kernels that follow.
__global__ __launch_bounds__(256) void k_router_topk(const float *__restrict__ x, const float *__restrict__ R,
                                                     const float *__restrict__ b, int E, int D, int K,
                                                     float routed_scale, float *logits, int32_t *sel,
                                                     float *w_scaled, float *w_soft, uint32_t *counter,
                                                     const float *__restrict__ nw, float eps, float *hn,
                                                     int32_t *hq, uint32_t *epoch) {
    __shared__ float red[4];
    // a new epoch for the expert launch that follows (its hand-over tag)
    if (epoch && blockIdx.x == 0 && threadIdx.x == 0) *epoch = *epoch + 1u;
    __shared__ double npart[4];
    __shared__ int last;
    const int e = blockIdx.x;
    float v;
    float rn = 1.0f;
    // the inputs of this wave's first record go out with the others (read at
    // the end they would add a round trip to the launch)
    const int nhg = (D + 31) >> 5, per = (nhg + E - 1) / E;
    const int hg0 = e * per + (threadIdx.x >> 6);
    float rx = 0.0f, rw = 0.0f;
    if (hq && (int)(threadIdx.x >> 6) < per && hg0 < nhg) {
        const int i = hg0 * 32 + (threadIdx.x & 63);
        const int ic = ((threadIdx.x & 63) < 32 && i < D) ? i : 0;
        rx = x[ic];
        if (nw) rw = nw[ic];
    }
    if (nw) {
        const float4 *w4 = reinterpret_cast<const float4 *>(R + (int64_t)e * D);
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const float4 *n4w = reinterpret_cast<const float4 *>(nw);
        const int n4 = D >> 2;
        // the norm's inputs go out before the router row, so that the
        // reduction runs while the row is in flight
        float hv[12];
        pk_rms_load(x, D, hv);
        // (range-checked buffer loads, unconditional: a guarded load would
        // make the compiler wait for the row before the norm; entries past
        // it read as zero and are not used), then the first chunk's inputs
        const pk_buf_t wr = pk_buf(w4, (uint32_t)n4 * 16u), xr = pk_buf(x4, (uint32_t)n4 * 16u),
                       nr = pk_buf(n4w, (uint32_t)n4 * 16u);
        float4 wf[GEMV_U], xh[GEMV_U], xw[GEMV_U];
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u) {
            const uint32_t off = ((uint32_t)threadIdx.x + u * 256u) * 16u;
            wf[u] = pk_buf_load4(wr, off);
            xh[u] = pk_buf_load4(xr, off);
            xw[u] = pk_buf_load4(nr, off);
        }
        rn = pk_rms_finish(hv, x, D, eps, npart);
        if (!hq) {
            const int span = (D + E - 1) / E;
            for (int i = e * span + threadIdx.x; i < min(D, (e + 1) * span); i += 256) hn[i] = x[i] * rn * nw[i];
        }
        float acc = 0.0f;
        for (int i0 = threadIdx.x; i0 < n4; i0 += 256 * GEMV_U) {
            if (i0 != (int)threadIdx.x) {
#pragma unroll
                for (int u = 0; u < GEMV_U; ++u) {
                    const uint32_t off = ((uint32_t)i0 + u * 256u) * 16u;
                    wf[u] = pk_buf_load4(wr, off);
                    xh[u] = pk_buf_load4(xr, off);
                    xw[u] = pk_buf_load4(nr, off);
                }
            }
#pragma unroll
            for (int u = 0; u < GEMV_U; ++u) {
                const int i = i0 + u * 256;
                if (i < n4) {
                    const float4 xv = pk_norm4(xh[u], rn, xw[u]);
                    acc = __builtin_fmaf(xv.x, wf[u].x, acc);
                    acc = __builtin_fmaf(xv.y, wf[u].y, acc);
                    acc = __builtin_fmaf(xv.z, wf[u].z, acc);
                    acc = __builtin_fmaf(xv.w, wf[u].w, acc);
                }
            }
        }
        for (int i = (n4 << 2) + threadIdx.x; i < D; i += 256)
            acc = __builtin_fmaf(x[i] * rn * nw[i], R[(int64_t)e * D + i], acc);
        acc = pk_wave_sum(acc);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
        __syncthreads();
        v = (red[0] + red[1]) + (red[2] + red[3]);
    } else {
        v = pk_row_dot_block(x, R + (int64_t)e * D, D, red);
    }
    if (hq) {
        // the experts' input (the normalised row, or x) as half-group records
        // of the integer-dot arithmetic: one wave per 32 values, whole
        // half-groups per workgroup (with the norm, hn is written here too)
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        for (int hg = e * per + wv; hg < min(nhg, (e + 1) * per); hg += 4) {
            const int i = hg * 32 + lane;
            const bool has = lane < 32 && i < D;
            const int ic = has ? i : 0;
            const float xi = hg == hg0 ? rx : x[ic], wi = hg == hg0 ? rw : (nw ? nw[ic] : 0.0f);
            const float xv = nw ? xi * rn * wi : xi;
            if (has && nw) hn[i] = xv;
            pk_write_digits<1>(xv, has, hq + (int64_t)hg * PK_XQ_INTS);
        }
    }
    // without a counter the block only publishes its logit: the expert
    // kernels that follow run the top-k themselves (pk_route_args)
    if (!counter) {
        if (threadIdx.x == 0) logits[e] = v + b[e];
        return;
    }
    if (threadIdx.x == 0) {
        pk_st_dev(logits + e, v + b[e]);
        __builtin_amdgcn_s_waitcnt(0);
        last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(E - 1);
    }
    __syncthreads();
    if (!last || threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    float v0 = lane < E ? pk_ld_dev(logits + lane) : -INFINITY;
    float v1 = lane + 64 < E ? pk_ld_dev(logits + lane + 64) : -INFINITY;
    bool t0 = lane >= E, t1 = lane + 64 >= E;
    __shared__ int ci[16];
    __shared__ float cv[16];
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
        if (lane == 0) { ci[k] = bi; cv[k] = bv; }
        if (bi == lane) t0 = true;
        if (bi == lane + 64) t1 = true;
    }
    if (lane == 0) {
        float m = -1e30f;
        for (int k = 0; k < K; ++k) if (cv[k] > m) m = cv[k];
        float s = 0.0f;
        for (int k = 0; k < K; ++k) { cv[k] = pk_expf_cr(cv[k] - m); s += cv[k]; }
        for (int k = 0; k < K; ++k) {
            const float p = cv[k] / s;
            sel[k] = ci[k];
            if (w_soft) w_soft[k] = p;
            w_scaled[k] = p * routed_scale;
        }
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

int pk_launch_router_topk(const float *x, const float *R, const float *b, int E, int D, int K,
                          float routed_scale, float *logits, int32_t *sel, float *w_scaled,
                          float *w_soft, uint32_t *counter, hipStream_t st, const float *nw, float eps,
                          float *hn, int32_t *hq, uint32_t *epoch) {
    PK_CHECK(E > 0 && E <= 128 && K > 0 && K <= 16 && K <= E, PK_ERR_UNSUPPORTED,
             "router: E=%d K=%d outside 1..128 / 1..16", E, K);
    PK_CHECK(((uintptr_t)R & 15) == 0 && ((uintptr_t)x & 15) == 0 && (D & 3) == 0, PK_ERR_UNSUPPORTED,
             "router: needs 16-byte aligned rows");
    PK_CHECK(!nw || (hn && ((uintptr_t)nw & 15) == 0), PK_ERR_ARG, "router: fused norm needs hn");
    hipLaunchKernelGGL(k_router_topk, dim3(E), dim3(256), 0, st, x, R, b, E, D, K, routed_scale, logits,
                       sel, w_scaled, w_soft, counter, nw, eps, hn, hq, epoch);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// Batched router: logits [T][E] already computed.
int pk_launch_topk_batch(const float *logits, int T, int E, int K, float routed_scale,
                         int32_t *sel, float *w_scaled, float *w_soft, hipStream_t st) {
    PK_CHECK(E > 0 && E <= 128 && K > 0 && K <= 16 && K <= E, PK_ERR_UNSUPPORTED,
             "router: E=%d K=%d outside 1..128 / 1..16", E, K);
    hipLaunchKernelGGL(k_topk_softmax, dim3(T), dim3(64), 0, st, logits, E, K, routed_scale,
                       sel, w_scaled, w_soft);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// Batched router's top-k together with the records of the rows x [n floats]
// (k_topk_records): sel / w_scaled as pk_launch_topk_batch, rec as
// pk_launch_act_records.
int pk_launch_topk_records(const float *logits, int T, int E, int K, float routed_scale, int32_t *sel,
                           float *w_scaled, const float *x, int n, int32_t *rec, hipStream_t st) {
    PK_CHECK(E > 0 && E <= 128 && K > 0 && K <= 16 && K <= E, PK_ERR_UNSUPPORTED,
             "router: E=%d K=%d outside 1..128 / 1..16", E, K);
    PK_CHECK(T > 0 && n > 0 && n % 32 == 0, PK_ERR_ARG, "topk records: T=%d n=%d", T, n);
    hipLaunchKernelGGL(k_topk_records, dim3(T + n / 32), dim3(64), 0, st, logits, T, E, K, routed_scale, sel,
                       w_scaled, x, n, rec);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────────── combine ─────────────────────────
// moe_forward's accumulation (picchio.c:1387, :1445-1454): out = 0, then
// out = fma(w_k, eo_k, out) for k in routing order; optional residual add
// afterwards (forward_token, picchio.c:1714-1716): res + out.
__global__ void k_combine(float *out, const float *eo, const float *w, int K, int D,
                          const float *residual, float *res_out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= D) return;
    float o = 0.0f;
    for (int k = 0; k < K; ++k) o = __builtin_fmaf(w[k], eo[(int64_t)k * D + i], o);
    if (out) out[i] = o;
    if (res_out) res_out[i] = residual[i] + o;
}

int pk_launch_combine(float *out, const float *eo, const float *w, int K, int D,
                      const float *residual, float *res_out, hipStream_t st) {
    hipLaunchKernelGGL(k_combine, dim3((D + 255) / 256), dim3(256), 0, st, out, eo, w, K, D,
                       residual, res_out);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// dst += w * eo (expert_apply, picchio.c:1788); w read from device memory.
__global__ void k_axpy_dev(float *dst, const float *eo, const float *w, int D) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < D) dst[i] = __builtin_fmaf(w[0], eo[i], dst[i]);
}
__global__ void k_axpy(float *dst, const float *eo, float w, int D) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < D) dst[i] = __builtin_fmaf(w, eo[i], dst[i]);
}

int pk_launch_axpy(float *dst, const float *eo, float w, int D, hipStream_t st) {
    hipLaunchKernelGGL(k_axpy, dim3((D + 255) / 256), dim3(256), 0, st, dst, eo, w, D);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// ───────────────────── synthetic N(0,1)*std on the GPU ─────────────────────
// Same counter formula as pk_synth.h (SplitMix64 + Box-Muller in double);
// device log/sqrt/sin/cos may differ from glibc in the last double bit, which
// changes the rounded float in about one element per 10^9.
__global__ void k_fill_normal(float *out, int64_t n, uint64_t s, float std) {
    const int64_t pair = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * pair >= n) return;
    double n0, n1;
    pk_normal_pair(s, (uint64_t)pair, &n0, &n1);
    out[2 * pair] = (float)(n0 * (double)std);
    if (2 * pair + 1 < n) out[2 * pair + 1] = (float)(n1 * (double)std);
}

int pk_launch_fill_normal(float *out, int64_t n, uint64_t stream_seed, float std, hipStream_t st) {
    const int64_t pairs = (n + 1) / 2;
    hipLaunchKernelGGL(k_fill_normal, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, st,
                       out, n, stream_seed, std);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// The same values for a K cache region of n_pos positions, value f (f =
// pos * KVH * hd + kvh * hd + i, the position-major order) stored at its
// place in the chunk layout (pk_k_off).
__global__ void k_fill_normal_k(float *out, int n_pos, int ctx, int KVH, int hd, uint64_t s, float std) {
    const int64_t n = (int64_t)n_pos * KVH * hd;
    const int64_t pair = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * pair >= n) return;
    double nv[2];
    pk_normal_pair(s, (uint64_t)pair, &nv[0], &nv[1]);
    const int kv_dim = KVH * hd;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int64_t f = 2 * pair + k;
        if (f >= n) break;
        const int pos = (int)(f / kv_dim), i = (int)(f - (int64_t)pos * kv_dim);
        out[pk_k_off(pos, i / hd, i % hd, ctx, KVH, hd)] = (float)(nv[k] * (double)std);
    }
}

int pk_launch_fill_normal_k(float *out, int n_pos, int ctx, int KVH, int hd, uint64_t stream_seed, float std,
                            hipStream_t st) {
    PK_CHECK(n_pos >= 0 && n_pos <= ctx && hd % 4 == 0, PK_ERR_ARG, "k fill: %d positions of %d", n_pos, ctx);
    const int64_t pairs = ((int64_t)n_pos * KVH * hd + 1) / 2;
    if (pairs == 0) return PK_OK;
    hipLaunchKernelGGL(k_fill_normal_k, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, st, out, n_pos, ctx,
                       KVH, hd, stream_seed, std);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

__global__ void k_fill_const(float *out, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

int pk_launch_fill_const(float *out, int64_t n, float v, hipStream_t st) {
    hipLaunchKernelGGL(k_fill_const, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, v);
    PK_HIP(hipGetLastError());
    return PK_OK;
}
