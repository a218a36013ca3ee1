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
#include <type_traits>

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
// tile list: tile j = up to tt consecutive pairs of one expert (with
// tile_grp: also the expert's first tile and tile count, tile_grp[2j] and
// [2j + 1]). Workgroup x (grid = E) places expert x. It counts every
// expert's pairs (LDS atomics; the offsets need them all) and scans the
// counts. Its waves then count their segment's pairs of x, and after a
// prefix over the 16 waves each wave places its pairs of x in order with
// ballots. No workgroup waits for another. (One workgroup placing every
// expert scanned the routing once per expert: for 8192 pairs and 32
// experts, 26 of its 33 µs.)
constexpr int GP_LDS = 16384;
__global__ __launch_bounds__(1024) void k_group_pairs(const int32_t *__restrict__ sel, int P, int E,
                                                      int32_t *__restrict__ pairs, int32_t *__restrict__ tile_exp,
                                                      int32_t *__restrict__ tile_beg,
                                                      int32_t *__restrict__ tile_cnt, int32_t *n_tiles, int tt,
                                                      int32_t *__restrict__ tile_grp) {
    __shared__ int cnt[128], off[129], toff[128], wcnt[16];
    __shared__ int s_sel[GP_LDS];
    const int x = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const bool staged = P <= GP_LDS;
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    if (staged && (int)blockDim.x * 16 >= GP_LDS) {
        // every load in flight at once (a loop would wait for each)
        int ev[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = threadIdx.x + u * blockDim.x;
            ev[u] = i < P ? sel[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = threadIdx.x + u * blockDim.x;
            if (i < P) {
                s_sel[i] = ev[u];
                if (ev[u] >= 0 && ev[u] < E) atomicAdd(&cnt[ev[u]], 1);
            }
        }
    } else {
        for (int i = threadIdx.x; i < P; i += blockDim.x) {
            const int e = sel[i];
            if (staged) s_sel[i] = e;
            if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    // offsets of the experts' pairs and of their tiles: one wave scans the
    // counts (lane l holds experts l and l + 64)
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
        if (lane == 63) {
            off[E] = pt + p1;
            if (x == 0) *n_tiles = qt + q1;
        }
    }
    __syncthreads();
    // expert x's tiles
    const int cx = cnt[x], nx = (cx + tt - 1) / tt;
    for (int k = threadIdx.x; k < nx; k += blockDim.x) {
        const int j = toff[x] + k;
        tile_exp[j] = x;
        tile_beg[j] = off[x] + k * tt;
        tile_cnt[j] = min(tt, cx - k * tt);
        if (tile_grp) {
            tile_grp[2 * j] = toff[x];
            tile_grp[2 * j + 1] = nx;
        }
    }
    // wave w's segment of the routing: its pairs of x, counted, then placed
    // after those of the waves before it
    const int seg = ((P + nw - 1) / nw + 63) & ~63;
    const int b0 = min(P, wave * seg), b1 = min(P, b0 + seg);
    auto sel_at = [&](int i) { return i < b1 ? (staged ? s_sel[i] : sel[i]) : -1; };
    int mine = 0;
    for (int b = b0; b < b1; b += 64) mine += __popcll(__ballot(sel_at(b + lane) == x));
    if (lane == 0) wcnt[wave] = mine;
    __syncthreads();
    int run = off[x];
    for (int w = 0; w < wave; ++w) run += wcnt[w];
    for (int b = b0; b < b1; b += 64) {
        const bool hit = sel_at(b + lane) == x;
        const uint64_t m = __ballot(hit);
        if (hit) pairs[run + __popcll(m & lt)] = b + lane;
        run += __popcll(m);
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

// ───────────── half-precision pair arithmetic (v_mfma_f32_32x32x16_f16) ─────────────
// The same grouped GEMM with the activations as two halves and fp32 sums:
//  * Activations: row x gets the factor 2^(15-k) (k the binary exponent of
//    max|x|, as above), x' = x 2^(15-k), |x'| <= 2^15, stored as hi = f16(x')
//    and lo = f16(x' - hi): hi + lo equals x' to ~2^-22 of |x'|.
//  * Weights: a stored nibble t (the two's complement of q) placed under the
//    exponent of 1024 reads 1024 + (t ^ 8) = 1032 + q; minus 1032 (packed
//    half adds) it is exactly q.
//  * Per 64-column group, 8 MFMAs (hi and lo over 4 x 16 columns) give
//    z = sum (hi + lo) q in fp32 (every product exact); the groups fold in
//    order, acc = fma(16 s_g, z_g, acc), and y = acc 2^(k-19) + bias.
// The MFMA adds in its own order, so this path is held to a tolerance
// against picchio's fp32 arithmetic (~1e-7 relative), not restated bit for
// bit. Per group and 32 x 32 tile it spends 16 VALU instructions on the
// fold (the int8 limbs need 80) and 44 on the weight expansion, shared by
// up to 64 pairs.
//
// Work items: (tile j of up to 64 pairs, row group r of 512 rows). The
// workgroup's 8 waves each take one 64-row block (two 32-row MFMA tiles) for
// both 32-pair halves of the tile (the second skipped when the tile holds
// at most 32 pairs). The MFMA runs with the activations as its first
// operand, so a lane's 16 results are 16 pairs of one output row: one scale
// per lane and row tile in the fold. Items i = r * n_tiles + j are dealt to
// the 8 XCDs (workgroup L runs on XCD L % 8) in contiguous runs, so that the
// workgroups resident on one XCD share an expert's weights in its L2.
namespace {
typedef _Float16 pk_v8h __attribute__((ext_vector_type(8)));
typedef float pk_v16f __attribute__((ext_vector_type(16)));

constexpr int FT = PK_F16_TILE;      // pairs per tile
constexpr int FW = 8;                // waves per workgroup
constexpr int FTHR = FW * 64;
constexpr int FROWS = FW * 64;       // rows per work item

// Stored position (0..7) of column u of an 8-column chunk: the expansion
// of one weight dword yields columns 0,4,1,5,2,6,3,7.
__device__ __forceinline__ int f16_pos(int u) { return ((u & 3) << 1) | (u >> 2); }

// 8 nibbles (columns 0..7 of a chunk, two's complement t) -> 8 halves q in
// the order above: ((w >> 4i) & M) ^ Y puts t ^ 8 = q + 8 under the
// exponent of 1024 in both halves of a dword (M = 0x000F000F,
// Y = 0x64086408; one three-input bit operation each when both are held in
// registers), then one packed half add per dword subtracts 1032.
__device__ __forceinline__ pk_v8h expand_f16(uint32_t w, uint32_t M, uint32_t Y) {
    typedef uint32_t pk_v4u __attribute__((ext_vector_type(4)));
    const pk_v4u p = {(w & M) ^ Y, ((w >> 4) & M) ^ Y, ((w >> 8) & M) ^ Y, ((w >> 12) & M) ^ Y};
    return __builtin_bit_cast(pk_v8h, p) + (_Float16)-1032.0f;
}
}  // namespace

// The clamped SwiGLU of picchio.c:1416-1424 with the hardware exp2 and
// reciprocal (1-2 ulp) in place of the correctly rounded expf: this path is
// held to a tolerance, and these few instructions replace a double-precision
// exp per pair.
__device__ __forceinline__ float swiglu_f16path(float gate, float up, float lim, float alpha) {
    if (gate > lim) gate = lim;
    if (up > lim) up = lim;
    if (up < -lim) up = -lim;
    const float e = __builtin_amdgcn_exp2f(-(alpha * gate) * 1.44269504088896341f);
    return (up + 1.0f) * gate * __builtin_amdgcn_rcpf(1.0f + e);
}

// One row per workgroup: exponent k of max|x|, the hi and lo planes (columns
// permuted by f16_pos inside each 8-column chunk).
// Rows of at most 4096 columns (16-byte aligned): the row is read once, two
// 8-column chunks per thread held in registers for the max and the split.
__global__ __launch_bounds__(256) void k_act_f16_reg(const float *__restrict__ x, int64_t x_stride, int cols,
                                                     uint16_t *__restrict__ xf, int64_t fplane,
                                                     int32_t *__restrict__ exps) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const float *xr = x + (int64_t)r * x_stride;
    const int nch = cols / 8;
    float4 v[2][2];
    float m = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = min((int)threadIdx.x + 256 * h, nch - 1);
        v[h][0] = *reinterpret_cast<const float4 *>(xr + 8 * c);
        v[h][1] = *reinterpret_cast<const float4 *>(xr + 8 * c + 4);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if ((int)threadIdx.x + 256 * h < nch)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                m = fmaxf(fmaxf(fmaxf(m, fabsf(v[h][q].x)), fmaxf(fabsf(v[h][q].y), fabsf(v[h][q].z))),
                          fabsf(v[h][q].w));
    m = pk_wave_max_f(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int k = 0;
    if (m > 0.0f) (void)frexpf(m, &k);
    if (threadIdx.x == 0) exps[r] = k;
    _Float16 *hr = reinterpret_cast<_Float16 *>(xf) + (int64_t)r * cols;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = (int)threadIdx.x + 256 * h;
        if (c >= nch) break;
        const float xs[8] = {v[h][0].x, v[h][0].y, v[h][0].z, v[h][0].w, v[h][1].x, v[h][1].y, v[h][1].z, v[h][1].w};
        pk_v8h hi, lo;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float vv = ldexpf(xs[u], 15 - k);
            const _Float16 vh = (_Float16)vv;
            hi[f16_pos(u)] = vh;
            lo[f16_pos(u)] = (_Float16)(vv - (float)vh);
        }
        *reinterpret_cast<pk_v8h *>(hr + 8 * c) = hi;
        *reinterpret_cast<pk_v8h *>(hr + fplane + 8 * c) = lo;
    }
}

__global__ __launch_bounds__(256) void k_act_f16(const float *__restrict__ x, int64_t x_stride, int cols,
                                                 uint16_t *__restrict__ xf, int64_t fplane,
                                                 int32_t *__restrict__ exps) {
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
    _Float16 *hr = reinterpret_cast<_Float16 *>(xf) + (int64_t)r * cols;
    for (int c = threadIdx.x; c < cols / 8; c += 256) {
        pk_v8h hi, lo;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float v = ldexpf(xr[8 * c + u], 15 - k);
            const _Float16 vh = (_Float16)v;
            hi[f16_pos(u)] = vh;
            lo[f16_pos(u)] = (_Float16)(v - (float)vh);
        }
        *reinterpret_cast<pk_v8h *>(hr + 8 * c) = hi;
        *reinterpret_cast<pk_v8h *>(hr + fplane + 8 * c) = lo;
    }
}

// Stage buffers: rings in LDS filled by direct global -> LDS loads (no
// registers), three stages ahead: activations and weights FR = 4 stages,
// scales FS = 8. Per stage and wave five load instructions, always issued,
// so that the wait for a stage is a fixed count of the wave's later loads.
//
// Schedule, per 64-column stage g and wave: fold stage g-1 into the
// accumulators | workgroup barrier | issue stage g+3, read this stage's
// scales and the next stage's weights, run the 32 MFMAs of stage g and,
// between them, expand the next stage's weights operand by operand as the
// MFMAs consume the current ones. Measured against a two-group schedule in
// which the waves of each SIMD alternate MFMA and fold/expand phases (two
// barriers per stage): 607-626 against 650-657 us per gate_up launch.
constexpr int FR = 4, FS = 8;
typedef __attribute__((address_space(3))) void pk_lds_void;

// 64 lanes x 16 (or 4) bytes from per-lane global addresses to LDS at
// lds + 16 (4) x lane; lds is the same for the whole wave. Issued as inline
// assembly: the compiler then does not pair these loads with the kernel's
// LDS reads (it would wait for every outstanding load before each read);
// the kernel's own waits order them instead. M0 carries the LDS address.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void pk_dma16(const void *src, void *lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(pk_lds_void *)lds);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m), "v"(src)
                 : "memory", "m0");
}
__device__ __forceinline__ void pk_dma4(const void *src, void *lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(pk_lds_void *)lds);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(m), "v"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
// s_waitcnt: at most N of the wave's vector-memory loads outstanding and no
// LDS read (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] at 15:14)
template <int N>
__device__ __forceinline__ void pk_wait_vm_lds() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}
// workgroup barrier after the wave's LDS reads are done; the compiler moves
// no instruction across it (memory accesses, MFMAs and VALU work stay in
// their stage)
__device__ __forceinline__ void pk_stage_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    pk_wait_vm_lds<63>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <int EPI>
__global__ __launch_bounds__(FTHR, 2) void k_moe_f16(pk_mfma_args a) {
    // activations [slot][hi, lo][token][64 halves: 8 chunks of 16 bytes, chunk q
    // of token t at position q ^ f(t), f(t) = (t ^ t / 8) % 8: any 16 tokens in a
    // row, even and odd apart, take distinct positions, so 16-byte reads of 8 or
    // 16 lanes hit distinct banks], weights [slot][wave][tile bytes],
    // scales [slot][row]
    // (one LDS block: after the last stage the output tile is staged in it)
    constexpr int B_BYTES = FR * 2 * FT * 64 * 2, W_BYTES = FR * FW * PK_TILE_BYTES, S_BYTES = FS * FROWS * 4;
    __shared__ __attribute__((aligned(16))) uint8_t lds[B_BYTES + W_BYTES + S_BYTES];
    auto &bring = *reinterpret_cast<_Float16 (*)[FR][2][FT][64]>(lds);
    auto &wring = *reinterpret_cast<uint8_t (*)[FR][FW][PK_TILE_BYTES]>(lds + B_BYTES);
    auto &sring = *reinterpret_cast<float (*)[FS][FROWS]>(lds + B_BYTES + W_BYTES);
    __shared__ int tok_row[FT], tok_exp[FT], tok_pair[FT];
    // this workgroup's item
    const int nt = *a.n_tiles;
    const int n_item = nt * ((a.O + FROWS - 1) / FROWS);
    const int run = (n_item + 7) >> 3;
    const int s = blockIdx.x >> 3;
    if (s >= run) return;
    const int item = (int)(blockIdx.x & 7) * run + s;
    if (item >= n_item) return;
    // item -> (row group, tile): row-group-major over all tiles, or (with
    // tile_grp) expert by expert and within an expert row-group-major over
    // its tiles, so that the workgroups resident on one XCD together share
    // the activation rows of their tiles as well as the expert's weights
    int rg, j;
    if (a.tile_grp) {
        const int RG = (a.O + FROWS - 1) / FROWS;
        const int p = item / RG;
        const int first = a.tile_grp[2 * p], n_e = a.tile_grp[2 * p + 1];
        const int local = item - RG * first;
        rg = local / n_e;
        j = first + (local - rg * n_e);
    } else {
        rg = item / nt;
        j = item - rg * nt;
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = a.tile_exp[j], beg = a.tile_beg[j], cnt = a.tile_cnt[j];
    if (threadIdx.x < FT) {
        const int t = threadIdx.x;
        const int pr = a.pairs[beg + (t < cnt ? t : 0)];
        const int row = pr / a.x_div;
        tok_row[t] = row;
        tok_exp[t] = a.exps[row];
        tok_pair[t] = pr;
    }
    const bool two = cnt > 32;                               // second 32-pair half in use
    const uint8_t *base = a.base + (int64_t)(a.slot_base + e) * a.slot_stride;
    const int RB = a.O >> 6;
    const int rb = (rg * FROWS >> 6) + wave;                 // this wave's 64-row block
    const bool active = rb < RB;
    const int rbc = min(rb, RB - 1);
    const int h = lane >> 5, n = lane & 31;
    const int NG = a.NG;
    uint32_t M = 0x000F000Fu, Y = 0x64086408u;
    asm volatile("" : "+v"(M), "+v"(Y));                    // held in registers (see expand_f16)
    __syncthreads();
    // this wave's loads per stage: activation rows 8 b .. 8 b + 7 of limb l for
    // b = 2 wave & 7 and b + 1 (l = wave / 4: waves 0..3 hi, 4..7 lo), its row
    // block's two weight halves and 64 scales
    const int blk = 8 * ((2 * wave) & 7);
    const int l = wave >> 2;
    const int ta = blk + (lane >> 3), tb = ta + 8, pos = lane & 7;
    const _Float16 *xb = reinterpret_cast<const _Float16 *>(a.xf) + l * a.fplane;
    const _Float16 *srca = xb + (int64_t)tok_row[ta] * a.frow + 8 * (pos ^ ((ta ^ (ta >> 3)) & 7));
    const _Float16 *srcb = xb + (int64_t)tok_row[tb] * a.frow + 8 * (pos ^ ((tb ^ (tb >> 3)) & 7));
    const uint8_t *wsrc = base + a.off_tiles + (int64_t)rbc * a.NG * PK_TILE_BYTES + 16 * lane;
    const float *ssrc = reinterpret_cast<const float *>(base + a.off_scales) + (int64_t)rbc * a.NG * 64 + lane;
    auto issue = [&](int g) {
        const int sl = g & (FR - 1);
        pk_dma16(srca + g * 64, &bring[sl][l][blk][0]);
        pk_dma16(srcb + g * 64, &bring[sl][l][blk + 8][0]);
        pk_dma16(wsrc + (int64_t)g * PK_TILE_BYTES, &wring[sl][wave][0]);
        pk_dma16(wsrc + (int64_t)g * PK_TILE_BYTES + 1024, &wring[sl][wave][1024]);
        pk_dma4(ssrc + g * 64, &sring[g & (FS - 1)][wave * 64]);
    };
    pk_v16f acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};   // [row tile][pair half]
    pk_v16f z00 = {}, z01 = {}, z10 = {}, z11 = {};           // the last stage's group sums
    pk_v8h A00, A01, A02, A03, A10, A11, A12, A13;           // the next stage's weights
    const int sw0 = (n ^ (n >> 3)) & 7;                      // f(n), f(32 + n)
    const int sw1 = (n ^ (4 + (n >> 3))) & 7;
    // weights (this wave's own loads) and scales of a stage, read into
    // registers ahead of the stage that uses them (the fold, the expansion)
    uint4 wr0 = make_uint4(0, 0, 0, 0), wr1 = wr0;
    float sr0 = 0.0f, sr1 = 0.0f;
    auto read_w = [&](int g) {
        const int sl = g & (FR - 1);
        wr0 = *reinterpret_cast<const uint4 *>(&wring[sl][wave][h * 1024 + 16 * n]);
        wr1 = *reinterpret_cast<const uint4 *>(&wring[sl][wave][h * 1024 + 512 + 16 * n]);
    };
    auto read_s = [&](int g) {                               // the lane's rows n and 32 + n
        sr0 = sring[g & (FS - 1)][wave * 64 + n];
        sr1 = sring[g & (FS - 1)][wave * 64 + 32 + n];
    };
    // weights -> MFMA operands
    auto expand = [&]() {
        A00 = expand_f16(wr0.x, M, Y); A01 = expand_f16(wr0.y, M, Y);
        A02 = expand_f16(wr0.z, M, Y); A03 = expand_f16(wr0.w, M, Y);
        A10 = expand_f16(wr1.x, M, Y); A11 = expand_f16(wr1.y, M, Y);
        A12 = expand_f16(wr1.z, M, Y); A13 = expand_f16(wr1.w, M, Y);
    };
    // Loads: stages 0..2 up front; after the barrier that opens stage g a
    // wave issues stage g+3 into the slot of stage g-1 (every wave's last read
    // of it came before that barrier), then waits for its own loads of stage
    // g+1 (those of g+2, g+3 may still run): so stage g+1 is in every wave's
    // LDS share before the barrier that opens it. Every wave passes NG
    // barriers. The wave's loads of a stage are in once at most those of the
    // `later` stages issued after it (5 each) are still outstanding.
    auto wait_stage = [&](int later) {
        asm volatile("" ::: "memory");
        if (later >= 2) pk_wait_vm_lds<10>();
        else if (later == 1) pk_wait_vm_lds<5>();
        else pk_wait_vm_lds<0>();
        asm volatile("" ::: "memory");
    };
    issue(0);
    if (NG > 1) issue(1);
    if (NG > 2) issue(2);
    wait_stage(min(2, NG - 1));                              // stage 0
    auto stage_loads = [&](int g) {
        if (g + 3 < NG) issue(g + 3);
        if (g + 1 < NG) wait_stage(min(g + 3, NG - 1) - (g + 1));   // stage g+1
    };
    const pk_v16f zero = {};
    // The stage loop for tiles with one (TWO false) or two 32-pair halves,
    // compiled apart so that neither carries the other's branches.
    auto stages = [&](auto two_c) {
        constexpr bool TWO = decltype(two_c)::value;
        // the stage's group sums for both row tiles (and pair halves): per
        // 16-column step m, the activation operands (hi, lo of each half) are
        // read from LDS two steps ahead of their MFMAs, so that the LDS latency
        // is covered by the MFMAs of the step in between
        auto mfma = [&](int g) {
            const int sl = g & (FR - 1);
            const _Float16 *bh = &bring[sl][0][n][0], *bl = &bring[sl][1][n][0];
            auto ld = [&](int m, pk_v8h &h0, pk_v8h &l0, pk_v8h &h1, pk_v8h &l1) {
                const int q0 = 8 * ((4 * h + m) ^ sw0);
                h0 = *reinterpret_cast<const pk_v8h *>(bh + q0);
                l0 = *reinterpret_cast<const pk_v8h *>(bl + q0);
                if constexpr (TWO) {
                    const int q1 = 8 * ((4 * h + m) ^ sw1);
                    h1 = *reinterpret_cast<const pk_v8h *>(bh + 32 * 64 + q1);
                    l1 = *reinterpret_cast<const pk_v8h *>(bl + 32 * 64 + q1);
                }
            };
            auto step = [&](bool first, const pk_v8h &A0, const pk_v8h &A1, const pk_v8h &h0, const pk_v8h &l0,
                            const pk_v8h &h1, const pk_v8h &l1) {
                z00 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h0, A0, first ? zero : z00, 0, 0, 0);
                z10 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h0, A1, first ? zero : z10, 0, 0, 0);
                z00 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l0, A0, z00, 0, 0, 0);
                z10 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l0, A1, z10, 0, 0, 0);
                if constexpr (TWO) {
                    z01 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h1, A0, first ? zero : z01, 0, 0, 0);
                    z11 = __builtin_amdgcn_mfma_f32_32x32x16_f16(h1, A1, first ? zero : z11, 0, 0, 0);
                    z01 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l1, A0, z01, 0, 0, 0);
                    z11 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l1, A1, z11, 0, 0, 0);
                }
            };
            // two operand sets alternate; after step m's MFMAs have issued (an
            // MFMA reads its operands at issue), its weight operands are
            // re-expanded from the next stage's weights (wr0 / wr1), so that
            // this VALU work issues between the MFMAs of the following steps
            pk_v8h xh0, xl0, xh1, xl1, yh0, yl0, yh1, yl1;
            ld(0, xh0, xl0, xh1, xl1);
            ld(1, yh0, yl0, yh1, yl1);
            step(true, A00, A10, xh0, xl0, xh1, xl1);
            A00 = expand_f16(wr0.x, M, Y); A10 = expand_f16(wr1.x, M, Y);
            ld(2, xh0, xl0, xh1, xl1);
            step(false, A01, A11, yh0, yl0, yh1, yl1);
            A01 = expand_f16(wr0.y, M, Y); A11 = expand_f16(wr1.y, M, Y);
            ld(3, yh0, yl0, yh1, yl1);
            step(false, A02, A12, xh0, xl0, xh1, xl1);
            A02 = expand_f16(wr0.z, M, Y); A12 = expand_f16(wr1.z, M, Y);
            step(false, A03, A13, yh0, yl0, yh1, yl1);
            A03 = expand_f16(wr0.w, M, Y); A13 = expand_f16(wr1.w, M, Y);
            // the expansion stays in this stage (the compiler may not sink it
            // to the next use), interleaved with the MFMAs above
            asm volatile("" : "+v"(A00), "+v"(A01), "+v"(A02), "+v"(A03), "+v"(A10), "+v"(A11), "+v"(A12),
                         "+v"(A13));
        };
        // acc += 16 s_g z_g in group order (the scales read by read_s)
        auto fold = [&]() {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                acc00[k] = __builtin_fmaf(sr0, z00[k], acc00[k]);
                acc10[k] = __builtin_fmaf(sr1, z10[k], acc10[k]);
                if constexpr (TWO) {
                    acc01[k] = __builtin_fmaf(sr0, z01[k], acc01[k]);
                    acc11[k] = __builtin_fmaf(sr1, z11[k], acc11[k]);
                }
            }
        };
        // per stage g: fold g-1 | barrier | loads, MFMA of g (expanding g+1)
        read_w(0);
        expand();
        for (int g = 0; g < NG; ++g) {
            if (g >= 1) fold();
            pk_stage_barrier();
            stage_loads(g);
            read_w(min(g + 1, NG - 1));
            read_s(g);
            mfma(g);
        }
        fold();
    };
    if (!active) {
        // no rows here: this wave's share of the loads and the barriers
        for (int g = 0; g < NG; ++g) {
            pk_stage_barrier();
            stage_loads(g);
        }
    } else if (two) {
        stages(std::true_type{});
    } else {
        stages(std::false_type{});
    }
    // Epilogue: the item's outputs go through LDS (every wave is past its last
    // read of the rings), [pair][output column of the item], so that each
    // lane then writes 16 contiguous bytes of a pair's row: a quarter of the
    // store instructions of writing the lanes' values in place, and each
    // wave's store covers whole 1 KB runs of rows.
    constexpr int OC = EPI == PK_EPI_SWIGLU ? FROWS / 2 : FROWS;   // output columns per item
    constexpr int OT = OC + 4;                                      // staged row (padded: banks)
    static_assert(FT * OT * 4 <= B_BYTES + W_BYTES + S_BYTES, "output tile exceeds the LDS block");
    float (*ot)[OT] = reinterpret_cast<float (*)[OT]>(lds);
    __syncthreads();
    if (active) {
        // lane (n, h) holds output row 32 rt + n of its block for the 16 pairs
        // 32 ts + 8 b + 4 h + i of the tile (element 4 b + i)
        const float *bias = a.off_bias >= 0 ? reinterpret_cast<const float *>(base + a.off_bias) : nullptr;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = rb * 64 + 32 * rt + n;
            const int lrow = wave * 64 + 32 * rt + n;                // row within the item
            const float bv = bias ? bias[row] : 0.0f;
#pragma unroll
            for (int ts = 0; ts < 2; ++ts) {
                if (ts == 1 && !two) break;
                const pk_v16f &c = rt ? (ts ? acc11 : acc10) : (ts ? acc01 : acc00);
                float y[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int tn = 32 * ts + 8 * (v >> 2) + 4 * h + (v & 3);
                    y[v] = ldexpf(c[v], tok_exp[tn] - 19);
                    if (bias) y[v] = y[v] + bv;
                }
                if constexpr (EPI == PK_EPI_SWIGLU) {
                    // rows 2i (gate, even lane) and 2i+1 (up, odd lane): the even
                    // lane finishes elements 0..7, the odd lane 8..15
                    const bool odd = n & 1;
#pragma unroll
                    for (int v = 0; v < 8; ++v) {
                        const float other = __shfl_xor(odd ? y[v] : y[v + 8], 1, 64);
                        const float mine = odd ? y[v + 8] : y[v];
                        const int va = odd ? v + 8 : v;
                        const int tn = 32 * ts + 8 * (va >> 2) + 4 * h + (va & 3);
                        ot[tn][lrow >> 1] = swiglu_f16path(odd ? other : mine, odd ? mine : other, a.lim, a.alpha);
                    }
                } else {
#pragma unroll
                    for (int v = 0; v < 16; ++v) ot[32 * ts + 8 * (v >> 2) + 4 * h + (v & 3)][lrow] = y[v];
                }
            }
        }
    }
    __syncthreads();
    // the item's valid output columns (rows of active waves), then per pair
    // of the tile its runs of 4 columns
    const int oc0 = (EPI == PK_EPI_SWIGLU ? rg * FROWS / 2 : rg * FROWS);
    const int noc = min(OC, (EPI == PK_EPI_SWIGLU ? a.O / 2 : a.O) - oc0);
    constexpr int Q = OC / 4;
    for (int k = threadIdx.x; k < cnt * Q; k += FTHR) {
        const int p = k / Q, c = 4 * (k - p * Q);
        if (c < noc)
            *reinterpret_cast<float4 *>(a.y + (int64_t)tok_pair[p] * a.y_stride + oc0 + c) =
                *reinterpret_cast<const float4 *>(&ot[p][c]);
    }
}

int pk_launch_act_f16(const float *x, int64_t x_stride, int rows, int cols, uint16_t *xf, int64_t fplane,
                      int32_t *exps, hipStream_t st) {
    PK_CHECK(rows > 0 && cols > 0 && cols % 8 == 0 && fplane >= (int64_t)rows * cols, PK_ERR_ARG,
             "act f16: bad shape");
    if (cols <= 4096 && ((uintptr_t)x & 15) == 0 && (x_stride & 3) == 0)
        hipLaunchKernelGGL(k_act_f16_reg, dim3(rows), dim3(256), 0, st, x, x_stride, cols, xf, fplane, exps);
    else
        hipLaunchKernelGGL(k_act_f16, dim3(rows), dim3(256), 0, st, x, x_stride, cols, xf, fplane, exps);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_moe_f16(const pk_mfma_args &a, int max_tiles, int epilogue, hipStream_t st) {
    PK_CHECK(a.O % 64 == 0 && a.O > 0 && a.NG > 0 && max_tiles > 0 && a.frow == a.NG * 64 && a.xf && a.fplane > 0,
             PK_ERR_UNSUPPORTED, "f16 grouped gemm: O=%d NG=%d", a.O, a.NG);
    // the epilogue writes 16-byte runs of output rows
    PK_CHECK((a.y_stride & 3) == 0 && ((uintptr_t)a.y & 15) == 0, PK_ERR_UNSUPPORTED,
             "f16 grouped gemm: output rows must be 16-byte aligned (stride %lld)", (long long)a.y_stride);
    const int64_t n = (int64_t)max_tiles * ((a.O + FROWS - 1) / FROWS);
    PK_CHECK(n < (1 << 30), PK_ERR_UNSUPPORTED, "f16 grouped gemm: %lld items", (long long)n);
    const dim3 grid((unsigned)((n + 7) & ~(int64_t)7));
    if (epilogue == PK_EPI_SWIGLU)
        hipLaunchKernelGGL(k_moe_f16<PK_EPI_SWIGLU>, grid, dim3(FTHR), 0, st, a);
    else
        hipLaunchKernelGGL(k_moe_f16<PK_EPI_PLAIN>, grid, dim3(FTHR), 0, st, a);
    PK_HIP(hipGetLastError());
    return PK_OK;
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
                          int tile_pairs, int32_t *tile_grp) {
    PK_CHECK(P > 0 && E > 0 && E <= 128, PK_ERR_ARG, "group pairs: P=%d E=%d", P, E);
    hipLaunchKernelGGL(k_group_pairs, dim3(E), dim3(1024), 0, st, sel, P, E, pairs, tile_exp, tile_beg,
                       tile_cnt, n_tiles, tile_pairs > 0 ? tile_pairs : TT, tile_grp);
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
