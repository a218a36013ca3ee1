// pk_mfma.hip — expert-grouped prefill MoE on the int8 matrix cores (gfx950).
//
// forward_prefill (picchio.c:1829-1916) applies each expert to every token
// that chose it. With many tokens per expert that is a dense contraction, so
// here it runs as a grouped GEMM on v_mfma_i32_32x32x32_i8:
//
//  * Activations: each row x (one token's input, or one (token, expert)
//    pair's SwiGLU output) gets a power-of-two scale 2^(k-20), k the binary
//    exponent of max|x| (x = m 2^k, m in [0.5, 1)), and becomes the integers
//    A = rint(x 2^(20-k)), |A| <= 2^20, split exactly into three int8 limbs
//    A = a0 2^14 + a1 2^7 + a2 (a0, a1 in [-64, 64], a2 in [-64, 63]).
//  * Weights: the stored nibble (two's complement of q = nib-8) is placed in
//    the high half of a byte, i.e. the int8 value 16 q, with one mask.
//  * Per 64-column scale group the three MFMA accumulators give, exactly,
//    P_l = sum a_l (16 q); C = (P0 << 10) + (P1 << 3) + (P2 >> 4) = sum A q
//    (int32, |C| <= 2^29). The groups are folded in order in fp32,
//    acc = fma(16 s_g, (float) C_g, acc), and y = acc 2^(k-24) + bias.
// Integer parts are exact; the result differs from the reference's fp32
// arithmetic only by the 21-bit activation rounding (~1e-6 relative), and it
// is reproduced bit-for-bit by the oracle's restatement (po_moe_mfma_gemm).
#include "pk_engine.h"
#include "pk_i4_device.h"

namespace {

typedef int pk_v4i __attribute__((ext_vector_type(4)));
typedef int pk_v16i __attribute__((ext_vector_type(16)));

constexpr int TT = 32;        // tokens per tile (MFMA N)
constexpr int NWAVE = 4;      // waves per workgroup, 32 output rows each
constexpr int WG_ROWS = NWAVE * 32;

// Position of column u (0..15) of a 16-column chunk in the operand byte order
// produced by the weight expansion: low nibbles of bytes 0..3 (columns
// 0,2,4,6), high nibbles (1,3,5,7), then the same for bytes 4..7.
__device__ __forceinline__ int limb_pos(int u) {
    return (u & 8) + ((u & 1) << 2) + ((u & 7) >> 1);
}

// One row per workgroup: exponent k of max|x| and the three limb planes.
__global__ __launch_bounds__(256) void k_act_limbs(const float *__restrict__ x, int64_t x_stride, int cols,
                                                   int8_t *__restrict__ limbs, int64_t plane,
                                                   int32_t *__restrict__ exps, int permuted) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const float *xr = x + (int64_t)r * x_stride;
    float m = 0.0f;
    for (int i = threadIdx.x; i < cols; i += 256) m = fmaxf(m, fabsf(xr[i]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int k = 0;
    if (m > 0.0f) (void)frexpf(m, &k);
    if (threadIdx.x == 0) exps[r] = k;
    int8_t *l0 = limbs + (int64_t)r * cols;
    for (int i = threadIdx.x; i < cols; i += 256) {
        const int A = (int)rintf(ldexpf(xr[i], 20 - k));
        const int a0 = (A + 8192) >> 14;
        const int rem = A - (a0 << 14);
        const int a1 = (rem + 64) >> 7;
        const int a2 = rem - (a1 << 7);
        const int pos = permuted ? (i & ~15) + limb_pos(i & 15) : i;
        l0[pos] = (int8_t)a0;
        l0[plane + pos] = (int8_t)a1;
        l0[2 * plane + pos] = (int8_t)a2;
    }
}

// Stable grouping of the P = T*K (token, expert) pairs by expert, and the
// tile list: tile j = up to 32 consecutive pairs of one expert.
__global__ __launch_bounds__(1024) void k_group_pairs(const int32_t *__restrict__ sel, int P, int E,
                                                      int32_t *__restrict__ pairs, int32_t *__restrict__ tile_exp,
                                                      int32_t *__restrict__ tile_beg,
                                                      int32_t *__restrict__ tile_cnt, int32_t *n_tiles) {
    __shared__ int cnt[128], off[129];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int e = wave; e < E; e += nw) {
        int run = 0;
        for (int b = 0; b < P; b += 64) {
            const int i = b + lane;
            const bool hit = i < P && sel[i] == e;
            run += __popcll(__ballot(hit));
        }
        if (lane == 0) cnt[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        off[0] = 0;
        for (int e = 0; e < E; ++e) off[e + 1] = off[e] + cnt[e];
        int j = 0;
        for (int e = 0; e < E; ++e)
            for (int b = 0; b < cnt[e]; b += TT) {
                tile_exp[j] = e;
                tile_beg[j] = off[e] + b;
                tile_cnt[j] = min(TT, cnt[e] - b);
                ++j;
            }
        *n_tiles = j;
    }
    __syncthreads();
    for (int e = wave; e < E; e += nw) {
        int run = off[e];
        for (int b = 0; b < P; b += 64) {
            const int i = b + lane;
            const bool hit = i < P && sel[i] == e;
            const uint64_t m = __ballot(hit);
            if (hit) pairs[run + __popcll(m & lt)] = i;
            run += __popcll(m);
        }
    }
}

// Weights of one 64-column group for the lane's row: 16 stored bytes (32
// nibbles, half h of the group) -> two operands of 16 int8 (16 q each).
__device__ __forceinline__ void expand_w(uint4 w, pk_v4i &o0, pk_v4i &o1) {
    const uint32_t M = 0xF0F0F0F0u;
    o0 = pk_v4i{(int)((w.x << 4) & M), (int)(w.x & M), (int)((w.y << 4) & M), (int)(w.y & M)};
    o1 = pk_v4i{(int)((w.z << 4) & M), (int)(w.z & M), (int)((w.w << 4) & M), (int)(w.w & M)};
}

}  // namespace

// Grouped expert GEMM (pk_mfma_args in pk_engine.h): grid (max tiles,
// ceil(O / 128)), 256 threads. Tile j of expert e holds its up to 32 pairs;
// the activation row of pair p is p / x_div.
template <int EPI>
__global__ __launch_bounds__(256) void k_moe_mfma(pk_mfma_args a) {
    __shared__ __attribute__((aligned(16))) int8_t bsh[3][TT][64];
    __shared__ int tok_row[TT];
    __shared__ int tok_exp[TT];
    const int j = blockIdx.x;
    if (j >= *a.n_tiles) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = a.tile_exp[j], beg = a.tile_beg[j], cnt = a.tile_cnt[j];
    if (threadIdx.x < TT) {
        const int n = threadIdx.x;
        const int p = a.pairs[beg + (n < cnt ? n : 0)];
        const int row = p / a.x_div;
        tok_row[n] = row;
        tok_exp[n] = a.exps[row];
    }
    const uint8_t *base = a.base + (int64_t)(a.slot_base + e) * a.slot_stride;
    const int row0 = blockIdx.y * WG_ROWS + wave * 32;      // this wave's first output row
    const bool active = row0 < a.O;
    const int rb = row0 >> 6, r64 = (row0 & 63);             // HBM tile row block, offset in it
    const int h = lane >> 5, n = lane & 31;
    const uint4 *wt = reinterpret_cast<const uint4 *>(base + a.off_tiles + (int64_t)rb * a.NG * 2048 +
                                                      h * 1024 + 16 * (r64 + n));
    const float *sc = reinterpret_cast<const float *>(base + a.off_scales) + (int64_t)rb * a.NG * 64 +
                      r64 + 4 * h;
    __syncthreads();

    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    // cooperative activation-tile load: 384 chunks of 16 B (limb, token, quarter)
    const int c0 = threadIdx.x, c1 = threadIdx.x + 256;
    auto src = [&](int c, int g) -> const uint4 * {
        const int l = c >> 7, t = (c >> 2) & 31, q = c & 3;
        return reinterpret_cast<const uint4 *>(a.limbs + l * a.plane + (int64_t)tok_row[t] * a.lrow + g * 64 +
                                               q * 16);
    };
    // operands of group g are fetched while group g-1 computes
    uint4 v0 = *src(c0, 0), v1 = make_uint4(0, 0, 0, 0), w = make_uint4(0, 0, 0, 0);
    if (c1 < 384) v1 = *src(c1, 0);
    float4 s4[4];
    if (active) {
        w = wt[0];
#pragma unroll
        for (int b = 0; b < 4; ++b) s4[b] = *reinterpret_cast<const float4 *>(sc + 8 * b);
    }
    for (int g = 0; g < a.NG; ++g) {
        __syncthreads();                                     // previous group's LDS reads done
        reinterpret_cast<uint4 *>(&bsh[0][0][0])[c0] = v0;
        if (c1 < 384) reinterpret_cast<uint4 *>(&bsh[0][0][0])[c1] = v1;
        __syncthreads();
        const uint4 wc = w;
        float sc_g[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) sc_g[v] = (&s4[v >> 2].x)[v & 3];
        if (g + 1 < a.NG) {
            v0 = *src(c0, g + 1);
            if (c1 < 384) v1 = *src(c1, g + 1);
            if (active) {
                w = wt[(int64_t)(g + 1) * 128];
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    s4[b] = *reinterpret_cast<const float4 *>(sc + (g + 1) * 64 + 8 * b);
            }
        }
        if (!active) continue;
        pk_v4i A0, A1;
        expand_w(wc, A0, A1);
        pk_v16i P[3];
#pragma unroll
        for (int l = 0; l < 3; ++l) {
            const pk_v4i B0 = *reinterpret_cast<const pk_v4i *>(&bsh[l][n][32 * h]);
            const pk_v4i B1 = *reinterpret_cast<const pk_v4i *>(&bsh[l][n][32 * h + 16]);
            pk_v16i z = {};
            z = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B0, z, 0, 0, 0);
            P[l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B1, z, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int C = (P[0][v] << 10) + (P[1][v] << 3) + (P[2][v] >> 4);
            acc[v] = __builtin_fmaf(sc_g[v], (float)C, acc[v]);
        }
    }
    if (!active || n >= cnt) return;
    const int p = a.pairs[beg + n];
    const int k = tok_exp[n];
    const float *bias = a.off_bias >= 0 ? reinterpret_cast<const float *>(base + a.off_bias) : nullptr;
    float y[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = row0 + 8 * (v >> 2) + 4 * h + (v & 3);
        y[v] = ldexpf(acc[v], k - 24);
        if (bias) y[v] = y[v] + bias[row];
    }
    float *yr = a.y + (int64_t)p * a.y_stride;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int row = row0 + 8 * b + 4 * h;
        if constexpr (EPI == PK_EPI_SWIGLU) {
            float2 o;
            o.x = pk_swiglu(y[4 * b + 0], y[4 * b + 1], a.lim, a.alpha);
            o.y = pk_swiglu(y[4 * b + 2], y[4 * b + 3], a.lim, a.alpha);
            *reinterpret_cast<float2 *>(yr + (row >> 1)) = o;
        } else {
            *reinterpret_cast<float4 *>(yr + row) = make_float4(y[4 * b], y[4 * b + 1], y[4 * b + 2], y[4 * b + 3]);
        }
    }
}

int pk_launch_act_limbs(const float *x, int64_t x_stride, int rows, int cols, int8_t *limbs, int64_t plane,
                        int32_t *exps, int permuted, hipStream_t st) {
    PK_CHECK(rows > 0 && cols > 0 && (!permuted || cols % 16 == 0), PK_ERR_ARG, "act limbs: bad shape");
    hipLaunchKernelGGL(k_act_limbs, dim3(rows), dim3(256), 0, st, x, x_stride, cols, limbs, plane, exps,
                       permuted);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_group_pairs(const int32_t *sel, int P, int E, int32_t *pairs, int32_t *tile_exp,
                          int32_t *tile_beg, int32_t *tile_cnt, int32_t *n_tiles, hipStream_t st) {
    PK_CHECK(P > 0 && E > 0 && E <= 128, PK_ERR_ARG, "group pairs: P=%d E=%d", P, E);
    hipLaunchKernelGGL(k_group_pairs, dim3(1), dim3(1024), 0, st, sel, P, E, pairs, tile_exp, tile_beg,
                       tile_cnt, n_tiles);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_moe_mfma(const pk_mfma_args &a, int max_tiles, int epilogue, hipStream_t st) {
    PK_CHECK(a.O % 64 == 0 && a.NG > 0 && max_tiles > 0 && a.lrow % 64 == 0, PK_ERR_UNSUPPORTED,
             "mfma gemm: O=%d NG=%d", a.O, a.NG);
    const dim3 grid(max_tiles, (a.O + WG_ROWS - 1) / WG_ROWS);
    if (epilogue == PK_EPI_SWIGLU)
        hipLaunchKernelGGL(k_moe_mfma<PK_EPI_SWIGLU>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(k_moe_mfma<PK_EPI_PLAIN>, grid, dim3(256), 0, st, a);
    PK_HIP(hipGetLastError());
    return PK_OK;
}
