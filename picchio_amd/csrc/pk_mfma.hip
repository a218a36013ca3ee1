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
#include "pk_dev.h"

namespace {

typedef int pk_v4i __attribute__((ext_vector_type(4)));
typedef int pk_v16i __attribute__((ext_vector_type(16)));

constexpr int TT = 32;        // tokens per tile (MFMA N)
constexpr int NWAVE = 8;      // waves per workgroup, 32 output rows each
constexpr int NTHR = NWAVE * 64;
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
    m = pk_wave_max_f(m);
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
// tile list: tile j = up to 32 consecutive pairs of one expert. One
// workgroup: counts by LDS atomics, then each wave places the pairs of its
// experts in order with ballots (routing staged in LDS when it fits).
constexpr int GP_LDS = 16384;
__global__ __launch_bounds__(1024) void k_group_pairs(const int32_t *__restrict__ sel, int P, int E,
                                                      int32_t *__restrict__ pairs, int32_t *__restrict__ tile_exp,
                                                      int32_t *__restrict__ tile_beg,
                                                      int32_t *__restrict__ tile_cnt, int32_t *n_tiles, int tt) {
    __shared__ int cnt[128], off[129];
    __shared__ int s_sel[GP_LDS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const bool staged = P <= GP_LDS;
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int e = sel[i];
        if (staged) s_sel[i] = e;
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // offsets of the experts' pairs and of their tiles: one wave scans the
    // counts (lane l holds experts l and l + 64), then every expert writes its tiles
    __shared__ int toff[128];
    if (wave == 0) {
        const int c0 = lane < E ? cnt[lane] : 0, c1 = lane + 64 < E ? cnt[lane + 64] : 0;
        int p0 = c0, p1 = c1, q0 = (c0 + tt - 1) / tt, q1 = (c1 + tt - 1) / tt;
        for (int d = 1; d < 64; d <<= 1) {
            const int a = __shfl_up(p0, d, 64), b = __shfl_up(p1, d, 64);
            const int u = __shfl_up(q0, d, 64), v = __shfl_up(q1, d, 64);
            if (lane >= d) { p0 += a; p1 += b; q0 += u; q1 += v; }
        }
        const int pt = __shfl(p0, 63, 64), qt = __shfl(q0, 63, 64);   // first half's totals
        if (lane < E) { off[lane] = p0 - c0; toff[lane] = q0 - (c0 + tt - 1) / tt; }
        if (lane + 64 < E) { off[lane + 64] = pt + p1 - c1; toff[lane + 64] = qt + q1 - (c1 + tt - 1) / tt; }
        if (lane == 63) { off[E] = pt + p1; *n_tiles = qt + q1; }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
        for (int b = 0, j = toff[e]; b < cnt[e]; b += tt, ++j) {
            tile_exp[j] = e;
            tile_beg[j] = off[e] + b;
            tile_cnt[j] = min(tt, cnt[e] - b);
        }
    for (int e = wave; e < E; e += nw) {
        int run = off[e];
        for (int b = 0; b < P; b += 64) {
            const int i = b + lane;
            const bool hit = i < P && (staged ? s_sel[i] : sel[i]) == e;
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
// ceil(O / 256)), 512 threads. Tile j of expert e holds its up to 32 pairs;
// the activation row of pair p is p / x_div. Wave w computes output rows
// row0 .. row0+31 for the tile's 32 pairs. The K loop runs in stages of G
// scale groups: the stage's activation limbs and scales are staged in LDS
// (double-buffered, one barrier per stage) while the next stage's operands
// are fetched into registers.
constexpr int G = 3;                      // scale groups per stage (45 = 15 x 3)
constexpr int BROW = G * 64 + 16;         // LDS bytes per token row (padded: no bank conflicts)
constexpr int BCH = 3 * TT * G * 4;       // 16-byte activation chunks per stage

// Operands of stage st into registers: activation chunks (limb, token,
// 16-byte quarter of the stage's G groups), the stage's scales of the
// workgroup's 128 rows, and this lane's weight bytes of the G groups.
static_assert(G == 3 && NTHR == 512 && BCH == 2 * 512 + 128, "stage loads assume 3 groups, 512 threads");

__device__ __forceinline__ const uint4 *chunk_src(const pk_mfma_args &a, int st, const int *tok_row, int c) {
    const int l = c / (TT * G * 4), r = c - l * (TT * G * 4), t = r / (G * 4), q = r - t * (G * 4);
    return reinterpret_cast<const uint4 *>(a.limbs + l * a.plane + (int64_t)tok_row[t] * a.lrow +
                                           st * (G * 64) + q * 16);
}
__device__ __forceinline__ int chunk_dst(int c) {              // byte offset in one stage buffer
    const int l = c / (TT * G * 4), r = c - l * (TT * G * 4), t = r / (G * 4), q = r - t * (G * 4);
    return (l * TT + t) * BROW + q * 16;
}

// Operands of stage st into registers: activation chunks c = tid + 512 u
// (limb, token, 16-byte quarter of the stage's G groups; u = 2 only for
// tid < 128), the stage's scales of the workgroup's 256 rows (tid < 192),
// and this lane's weight bytes of the G groups.
#define MFMA_LOAD_STAGE(st)                                                                          \
    do {                                                                                             \
        const int t0_ = threadIdx.x;                                                                 \
        rb0 = *chunk_src(a, (st), tok_row, t0_);                                                     \
        rb1 = *chunk_src(a, (st), tok_row, t0_ + NTHR);                                              \
        if (t0_ < 128) rb2 = *chunk_src(a, (st), tok_row, t0_ + 2 * NTHR);                           \
        if (t0_ < G * (WG_ROWS / 4)) {                                                               \
            const int rr_ = rowW + (t0_ % (WG_ROWS / 4)) * 4;                                        \
            if (rr_ < a.O)                                                                           \
                rsv = *reinterpret_cast<const float4 *>(                                             \
                    scw + ((int64_t)(rr_ >> 6) * a.NG + (st) * G + t0_ / (WG_ROWS / 4)) * 64 +       \
                    (rr_ & 63));                                                                     \
        }                                                                                            \
        if (active) {                                                                                \
            rw0 = wt[(int64_t)((st) * G + 0) * 128];                                                 \
            rw1 = wt[(int64_t)((st) * G + 1) * 128];                                                 \
            rw2 = wt[(int64_t)((st) * G + 2) * 128];                                                 \
        }                                                                                            \
    } while (0)

#define MFMA_STORE_STAGE(buf)                                                                        \
    do {                                                                                             \
        const int t0_ = threadIdx.x;                                                                 \
        int8_t *bb_ = &bsh[buf][0][0][0];                                                            \
        *reinterpret_cast<uint4 *>(bb_ + chunk_dst(t0_)) = rb0;                                      \
        *reinterpret_cast<uint4 *>(bb_ + chunk_dst(t0_ + NTHR)) = rb1;                               \
        if (t0_ < 128) *reinterpret_cast<uint4 *>(bb_ + chunk_dst(t0_ + 2 * NTHR)) = rb2;            \
        if (t0_ < G * (WG_ROWS / 4))                                                                 \
            *reinterpret_cast<float4 *>(&ssh[buf][t0_ / (WG_ROWS / 4)][(t0_ % (WG_ROWS / 4)) * 4]) = rsv; \
    } while (0)

template <int EPI>
__global__ __launch_bounds__(NTHR, 4) void k_moe_mfma(pk_mfma_args a) {
    __shared__ __attribute__((aligned(16))) int8_t bsh[2][3][TT][BROW];
    __shared__ __attribute__((aligned(16))) float ssh[2][G][WG_ROWS];
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
    const int rowW = blockIdx.y * WG_ROWS;                   // workgroup's first output row
    const int row0 = rowW + wave * 32;                       // this wave's first output row
    const bool active = row0 < a.O;
    const int rb = row0 >> 6, r64 = (row0 & 63);
    const int h = lane >> 5, n = lane & 31;
    const uint4 *wt = reinterpret_cast<const uint4 *>(base + a.off_tiles + (int64_t)rb * a.NG * 2048 +
                                                      h * 1024 + 16 * (r64 + n));
    const float *scw = reinterpret_cast<const float *>(base + a.off_scales);
    const int n_stage = a.NG / G;
    // the epilogue's output row goes out now
    const float *bias = a.off_bias >= 0 ? reinterpret_cast<const float *>(base + a.off_bias) : nullptr;
    const int p_out = a.pairs[beg + min(n, cnt - 1)];
    __syncthreads();

    const uint4 z4 = make_uint4(0, 0, 0, 0);
    uint4 rb0 = z4, rb1 = z4, rb2 = z4, rw0 = z4, rw1 = z4, rw2 = z4;
    float4 rsv = make_float4(0.f, 0.f, 0.f, 0.f);
    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    MFMA_LOAD_STAGE(0);
    for (int st = 0; st < n_stage; ++st) {
        const int buf = st & 1;
        MFMA_STORE_STAGE(buf);
        const uint4 wc0 = rw0, wc1 = rw1, wc2 = rw2;
        __syncthreads();
        if (st + 1 < n_stage) MFMA_LOAD_STAGE(st + 1);
        if (!active) continue;
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            pk_v4i A0, A1;
            expand_w(gi == 0 ? wc0 : gi == 1 ? wc1 : wc2, A0, A1);
            // limb products low to high, each folded into the exact sum as it
            // arrives: C = (P0 << 10) + (P1 << 3) + (P2 >> 4) (two limb
            // results live at a time, not three)
            pk_v16i Cg;
#pragma unroll
            for (int l = 2; l >= 0; --l) {
                const int8_t *bp = &bsh[buf][l][n][gi * 64 + 32 * h];
                const pk_v4i B0 = *reinterpret_cast<const pk_v4i *>(bp);
                const pk_v4i B1 = *reinterpret_cast<const pk_v4i *>(bp + 16);
                pk_v16i z = {};
                z = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B0, z, 0, 0, 0);
                z = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B1, z, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    // (z << s) + C is one v_lshl_add_u32; two's complement
                    // arithmetic, so it is z 2^s + C for negative z too
                    if (l == 2) Cg[v] = z[v] >> 4;
                    else if (l == 1) Cg[v] = (int)(((uint32_t)z[v] << 3) + (uint32_t)Cg[v]);
                    else Cg[v] = (int)(((uint32_t)z[v] << 10) + (uint32_t)Cg[v]);
                }
            }
            const float *sp = &ssh[buf][gi][wave * 32 + 4 * h];
#pragma unroll
            for (int b4 = 0; b4 < 4; ++b4) {
                const float4 s4 = *reinterpret_cast<const float4 *>(sp + 8 * b4);
                const float sv4[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int v = 4 * b4 + i;
                    acc[v] = __builtin_fmaf(sv4[i], (float)Cg[v], acc[v]);
                }
            }
        }
    }
    if (!active || n >= cnt) return;
    float bv[16];
    if (bias) {
#pragma unroll
        for (int v = 0; v < 16; ++v) bv[v] = bias[row0 + 8 * (v >> 2) + 4 * h + (v & 3)];
    }
    const int k = tok_exp[n];
    float y[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        y[v] = ldexpf(acc[v], k - 24);
        if (bias) y[v] = y[v] + bv[v];
    }
    float *yr = a.y + (int64_t)p_out * a.y_stride;
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
                          int32_t *tile_beg, int32_t *tile_cnt, int32_t *n_tiles, hipStream_t st,
                          int tile_pairs) {
    PK_CHECK(P > 0 && E > 0 && E <= 128, PK_ERR_ARG, "group pairs: P=%d E=%d", P, E);
    hipLaunchKernelGGL(k_group_pairs, dim3(1), dim3(1024), 0, st, sel, P, E, pairs, tile_exp, tile_beg,
                       tile_cnt, n_tiles, tile_pairs > 0 ? tile_pairs : TT);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_moe_mfma(const pk_mfma_args &a, int max_tiles, int epilogue, hipStream_t st) {
    PK_CHECK(a.O % 64 == 0 && a.NG > 0 && a.NG % G == 0 && max_tiles > 0 && a.lrow % 64 == 0,
             PK_ERR_UNSUPPORTED, "mfma gemm: O=%d NG=%d (groups must be a multiple of %d)", a.O, a.NG, G);
    const dim3 grid(max_tiles, (a.O + WG_ROWS - 1) / WG_ROWS);
    if (epilogue == PK_EPI_SWIGLU)
        hipLaunchKernelGGL(k_moe_mfma<PK_EPI_SWIGLU>, grid, dim3(NTHR), 0, st, a);
    else
        hipLaunchKernelGGL(k_moe_mfma<PK_EPI_PLAIN>, grid, dim3(NTHR), 0, st, a);
    PK_HIP(hipGetLastError());
    return PK_OK;
}
