// pk_exact.hip — the prompt path's dense arithmetic in the reference's order.
//
// forward_prefill (picchio.c:1795-1932) runs the attention projections,
// the sink attention and the router on every prompt position. Here those
// steps follow the reference operation by operation, so that the prompt's
// hidden states (and the KV rows the decode steps read) carry no rounding
// of their own:
//  * matmul_f32 (quant.h:117-148, AVX2 branch) and matmul_q8 (quant.h:152-186),
//    also behind matmul_qt for those formats: per (row, output) eight fp32
//    FMA chains, chain j over columns j, 8+j, ..., folded with hsum256's tree
//    ((c0+c4)+(c2+c6))+((c1+c5)+(c3+c7)) (quant.h:94-103), then the ragged
//    tail as gcc builds quant.h:138 (a block of four products added one by
//    one, then contracted FMAs); bias and residual added afterwards as
//    gqa_attention (picchio.c:530-532, :613) and forward_token (:1691) do.
//  * gqa_attention's softmax with sink (picchio.c:569-607): in-order score
//    dots (products added one by one), the maximum over sink and scores,
//    the sum of expf terms in position order starting from the sink's, each
//    weight divided by the sum, and the value rows accumulated in position
//    order, oh = fma(w, v, oh).
//  * the prompt router (picchio.c:1840-1844): the dot starts at the bias and
//    adds the products one by one.
// expf is evaluated as the double exp rounded to float (pk_expf_cr), which
// equals glibc's expf except where glibc's result is not the correctly
// rounded one (about 8e-5 of inputs).
#include "pk_engine.h"
#include "pk_i4_device.h"

namespace {

// ───────────────────────── matmul_f32 for S rows ─────────────────────────
// grid (ceil(O / 32), ceil(S / 64)), 256 threads. Wave w owns outputs
// o0 + 8w .. +7 of the block; lane l = 8 g + j owns chain j of rows
// s0 + 8g .. +7 for those 8 outputs (64 accumulators). Column chunks of 64
// (8 chain steps) are staged in LDS as [step][j][row] and [step][j][output]
// so each lane reads its eight x and eight w values as two 16-byte loads.
constexpr int CH_KC = 64;                 // columns per staged chunk
constexpr int CH_ROWS = 64, CH_OUTS = 32;

// TW = int8_t: matmul_q8 (quant.h:152-186), the same chains over the weights
// converted to float, the tail as contracted FMAs, the sum times the row scale.
// VEC (fp32 weights, 16-byte aligned rows, ldx and I multiples of 4): each
// chunk's 64 x 64 inputs and 32 x 64 weights load as six float4 per thread,
// the next chunk's while the current one is multiplied (the scalar loops
// wait for every load on its own).
template <typename TW, bool VEC = false>
__global__ __launch_bounds__(256) void k_gemm_chain8(const float *__restrict__ X, int64_t ldx,
                                                     const TW *__restrict__ W, const float *__restrict__ rscale,
                                                     const float *__restrict__ bias, float *out, int64_t ldo,
                                                     int S, int I, int O, int add_res) {
    __shared__ __attribute__((aligned(16))) float xs[CH_KC / 8][8][CH_ROWS];
    __shared__ __attribute__((aligned(16))) float ws[CH_KC / 8][8][CH_OUTS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 7, g = lane >> 3;
    const int o0 = blockIdx.x * CH_OUTS, s0 = blockIdx.y * CH_ROWS;
    const int I8 = I & ~7;
    float acc[8][8];
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[m][i] = 0.0f;
    float4 xv4[4], wv4[2];
    // float4 e = tid + 256 u of the chunk: row e / 16, columns 4 (e % 16) .. +3
    auto load = [&](int c0) {
        const int nc = min(CH_KC, I8 - c0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = tid + 256 * u, r = e >> 4, c = 4 * (e & 15), sr = min(s0 + r, S - 1);
            const float4 v = *reinterpret_cast<const float4 *>(X + (int64_t)sr * ldx + c0 + min(c, nc - 4));
            xv4[u] = c < nc && s0 + r < S ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = tid + 256 * u, r = e >> 4, c = 4 * (e & 15), orow = min(o0 + r, O - 1);
            const float4 v =
                *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(W) + (int64_t)orow * I + c0 +
                                                  min(c, nc - 4));
            wv4[u] = c < nc && o0 + r < O ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    if constexpr (VEC)
        if (I8 > 0) load(0);
    for (int c0 = 0; c0 < I8; c0 += CH_KC) {
        const int nc = min(CH_KC, I8 - c0);    // a multiple of 8
        __syncthreads();
        if constexpr (VEC) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = tid + 256 * u, r = e >> 4, c = 4 * (e & 15);
                xs[c >> 3][(c & 7) + 0][r] = xv4[u].x;
                xs[c >> 3][(c & 7) + 1][r] = xv4[u].y;
                xs[c >> 3][(c & 7) + 2][r] = xv4[u].z;
                xs[c >> 3][(c & 7) + 3][r] = xv4[u].w;
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int e = tid + 256 * u, r = e >> 4, c = 4 * (e & 15);
                ws[c >> 3][(c & 7) + 0][r] = wv4[u].x;
                ws[c >> 3][(c & 7) + 1][r] = wv4[u].y;
                ws[c >> 3][(c & 7) + 2][r] = wv4[u].z;
                ws[c >> 3][(c & 7) + 3][r] = wv4[u].w;
            }
        } else {
            // X chunk: 64 rows x nc columns (zeros past S), 16 per thread
            for (int e = tid; e < CH_ROWS * CH_KC; e += 256) {
                const int r = e / CH_KC, c = e - r * CH_KC;
                const int s = s0 + r;
                xs[c >> 3][c & 7][r] = (c < nc && s < S) ? X[(int64_t)s * ldx + c0 + c] : 0.0f;
            }
            for (int e = tid; e < CH_OUTS * CH_KC; e += 256) {
                const int r = e / CH_KC, c = e - r * CH_KC;
                const int o = o0 + r;
                ws[c >> 3][c & 7][r] = (c < nc && o < O) ? (float)W[(int64_t)o * I + c0 + c] : 0.0f;
            }
        }
        __syncthreads();
        if constexpr (VEC)
            if (c0 + CH_KC < I8) load(c0 + CH_KC);
        for (int k = 0; k < nc / 8; ++k) {
            const float4 xa = *reinterpret_cast<const float4 *>(&xs[k][j][8 * g]);
            const float4 xb = *reinterpret_cast<const float4 *>(&xs[k][j][8 * g + 4]);
            const float4 wa = *reinterpret_cast<const float4 *>(&ws[k][j][8 * wave]);
            const float4 wb = *reinterpret_cast<const float4 *>(&ws[k][j][8 * wave + 4]);
            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int m = 0; m < 8; ++m)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[m][i] = __builtin_fmaf(xv[i], wv[m], acc[m][i]);
        }
    }
    // hsum256 across the eight chain lanes: lane j = 0 ends with the row value
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = acc[m][i];
            v = v + __shfl_xor(v, 4, 64);
            v = v + __shfl_xor(v, 2, 64);
            v = v + __shfl_xor(v, 1, 64);
            acc[m][i] = v;
        }
    if (j != 0) return;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int o = o0 + 8 * wave + m;
        if (o >= O) continue;
        const TW *wr = W + (int64_t)o * I;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int s = s0 + 8 * g + i;
            if (s >= S) continue;
            const float *xr = X + (int64_t)s * ldx;
            float a = acc[m][i];
            int c = I8;
            if constexpr (sizeof(TW) == 4) {
                if (I - c >= 4) {
                    const float p0 = xr[c] * wr[c], p1 = xr[c + 1] * wr[c + 1];
                    const float p2 = xr[c + 2] * wr[c + 2], p3 = xr[c + 3] * wr[c + 3];
                    a = a + p0; a = a + p1; a = a + p2; a = a + p3;
                    c += 4;
                }
            }
            for (; c < I; ++c) a = __builtin_fmaf(xr[c], (float)wr[c], a);
            if (rscale) a = a * rscale[o];
            if (bias) a = a + bias[o];
            float *y = out + (int64_t)s * ldo + o;
            *y = add_res ? *y + a : a;
        }
    }
}

// ───────────────────── gqa_attention of prompt rows ─────────────────────
// One wave per (head, row). Scores of the row's window into LDS, the max,
// the exp terms, their sum in position order (one lane), the weights, then
// lane i < hd accumulates column i of the values in position order.
__global__ __launch_bounds__(64) void k_attn_rows_exact(int pos_base, const float *qkv, int64_t qkv_stride,
                                                        const float *Kl, const float *Vl, int H, int KVH, int hd,
                                                        int ctx, int sliding, int window, const float *sinks,
                                                        float *att) {
    extern __shared__ float sc[];              // [window positions]
    __shared__ float s_sum;
    const int h = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const int pos = pos_base + r;
    int end = pos < ctx ? pos : ctx - 1;
    int start = 0;
    if (sliding) {
        start = end - window + 1;
        if (start < 0) start = 0;
    }
    const int n = end - start + 1;
    const int kv_dim = KVH * hd, kvh = h / (H / KVH);
    const float *qh = qkv + (int64_t)r * qkv_stride + h * hd;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int t = lane; t < n; t += 64) {
        // (the K cache's chunk layout: a position's float4 columns cs apart)
        const int tk = start + t;
        const int cs = pk_k_cs(tk, ctx);
        const float4 *kt = reinterpret_cast<const float4 *>(Kl + pk_k_off(tk, kvh, 0, ctx, KVH, hd));
        const float4 *q4 = reinterpret_cast<const float4 *>(qh);
        float dot = 0.0f;
        for (int i = 0; i < hd / 4; ++i) {
            const float4 k4 = kt[(int64_t)i * cs], qq = q4[i];
            float p;
            p = qq.x * k4.x; dot = dot + p;
            p = qq.y * k4.y; dot = dot + p;
            p = qq.z * k4.z; dot = dot + p;
            p = qq.w * k4.w; dot = dot + p;
        }
        sc[t] = dot * scale;
    }
    __syncthreads();
    // max over the sink and the scores (a comparison: order-free)
    float mx = -INFINITY;
    for (int t = lane; t < n; t += 64) mx = fmaxf(mx, sc[t]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float sink = sinks[h];
    if (sink > mx) mx = sink;
    for (int t = lane; t < n; t += 64) sc[t] = pk_expf_cr(sc[t] - mx);
    __syncthreads();
    if (lane == 0) {
        float sum = pk_expf_cr(sink - mx);
        for (int t = 0; t < n; ++t) sum += sc[t];
        s_sum = sum;
    }
    __syncthreads();
    const float sum = s_sum;
    for (int t = lane; t < n; t += 64) sc[t] = sc[t] / sum;
    __syncthreads();
    for (int i = lane; i < hd; i += 64) {
        const float *vc = Vl + (int64_t)start * kv_dim + kvh * hd + i;
        float o = 0.0f;
        for (int t = 0; t < n; ++t) o = __builtin_fmaf(sc[t], vc[(int64_t)t * kv_dim], o);
        att[(int64_t)r * H * hd + h * hd + i] = o;
    }
}

// ───────────────────────── prompt router ─────────────────────────
// logits[s][e] = bias[e] + x[s][0]*w[e][0] + ... in order (products
// rounded, then added). 128 threads: lane t takes expert t % E of row
// s0 + t / E; the router rows are staged transposed in LDS, 64 columns at a
// time, the input rows beside them.
constexpr int RS_KC = 64;

__global__ __launch_bounds__(128) void k_router_seq(const float *__restrict__ X, const float *__restrict__ R,
                                                    const float *__restrict__ bias, int S, int D, int E,
                                                    float *logits) {
    extern __shared__ float lds_rs[];
    const int rows = 128 / E;                  // rows per block (E <= 128)
    float *wt = lds_rs;                        // [RS_KC][E]
    float *xt = lds_rs + RS_KC * E;            // [rows][RS_KC]
    const int tid = threadIdx.x;
    const int e = tid % E, rr = tid / E;
    const int s = blockIdx.x * rows + rr;
    const bool live = rr < rows && s < S;
    float acc = live ? bias[e] : 0.0f;
    for (int c0 = 0; c0 < D; c0 += RS_KC) {
        const int nc = min(RS_KC, D - c0);
        __syncthreads();
        for (int q = tid; q < E * RS_KC; q += 128) {
            const int ee = q / RS_KC, c = q - ee * RS_KC;
            wt[c * E + ee] = c < nc ? R[(int64_t)ee * D + c0 + c] : 0.0f;
        }
        for (int q = tid; q < rows * RS_KC; q += 128) {
            const int r2 = q / RS_KC, c = q - r2 * RS_KC;
            const int s2 = blockIdx.x * rows + r2;
            xt[r2 * RS_KC + c] = (c < nc && s2 < S) ? X[(int64_t)s2 * D + c0 + c] : 0.0f;
        }
        __syncthreads();
        if (live)
            for (int c = 0; c < nc; ++c) {
                const float p = xt[rr * RS_KC + c] * wt[c * E + e];
                acc = acc + p;
            }
    }
    if (live) logits[(int64_t)s * E + e] = acc;
}

// The same sums with 16-byte loads (D % 4 == 0, aligned rows; 4 <= E <= 128):
// the next 64 columns of the router rows and of the block's input rows load
// into registers (at most 20 per thread, so that the load counter can wait
// for them in order) while the current ones are multiplied; in LDS each
// router row's chunk is contiguous, so a thread reads its 64 weights and
// its row's 64 inputs as float4, 32 at a time, before the dependent adds.
constexpr int RQ_P = RS_KC + 4;          // padded LDS row (floats)
__global__ __launch_bounds__(128) void k_router_seq4(const float *__restrict__ X, const float *__restrict__ R,
                                                     const float *__restrict__ bias, int S, int D, int E,
                                                     float *logits) {
    extern __shared__ float lds_rs[];
    const int rows = 128 / E;
    float *wt = lds_rs;                   // [E][RQ_P]
    float *xt = lds_rs + E * RQ_P;        // [rows][RQ_P]
    const int tid = threadIdx.x;
    const int e = tid % E, rr = tid / E;
    const int s = blockIdx.x * rows + rr;
    const bool live = rr < rows && s < S;
    float acc = live ? bias[e] : 0.0f;
    constexpr int WN = 16, XN = 4;        // float4 per thread: E * 16 / 128 and rows * 16 / 128
    const int nw4 = E * (RS_KC / 4), nx4 = rows * (RS_KC / 4);
    float4 wv[WN], xv[XN];
    auto load = [&](int c0) {
        const int nc4 = min(RS_KC, D - c0) / 4;
#pragma unroll
        for (int u = 0; u < WN; ++u) {
            const int q = min(tid + 128 * u, nw4 - 1), ee = q / (RS_KC / 4), c4 = q - ee * (RS_KC / 4);
            const float4 v = *reinterpret_cast<const float4 *>(R + (int64_t)ee * D + c0 + 4 * min(c4, nc4 - 1));
            wv[u] = c4 < nc4 ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < XN; ++u) {
            const int q = min(tid + 128 * u, nx4 - 1), r2 = q / (RS_KC / 4), c4 = q - r2 * (RS_KC / 4);
            const int s2 = min(blockIdx.x * rows + r2, S - 1);
            const float4 v = *reinterpret_cast<const float4 *>(X + (int64_t)s2 * D + c0 + 4 * min(c4, nc4 - 1));
            xv[u] = c4 < nc4 ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    load(0);
    // (the bias is waited for here: inside the loop the compiler would wait
    // for every outstanding load before the first add)
    asm volatile("" ::"v"(acc));
    for (int c0 = 0; c0 < D; c0 += RS_KC) {
        const int nc = min(RS_KC, D - c0);
        __syncthreads();                  // the previous chunk's reads are done
#pragma unroll
        for (int u = 0; u < WN; ++u) {
            const int q = tid + 128 * u, ee = q / (RS_KC / 4), c4 = q - ee * (RS_KC / 4);
            if (q < nw4) *reinterpret_cast<float4 *>(wt + ee * RQ_P + 4 * c4) = wv[u];
        }
#pragma unroll
        for (int u = 0; u < XN; ++u) {
            const int q = tid + 128 * u, r2 = q / (RS_KC / 4), c4 = q - r2 * (RS_KC / 4);
            if (q < nx4) *reinterpret_cast<float4 *>(xt + r2 * RQ_P + 4 * c4) = xv[u];
        }
        __syncthreads();
        if (c0 + RS_KC < D) load(c0 + RS_KC);
        if (live) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4 xa[8], wa[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    xa[j] = *reinterpret_cast<const float4 *>(xt + rr * RQ_P + 32 * h + 4 * j);
                    wa[j] = *reinterpret_cast<const float4 *>(wt + e * RQ_P + 32 * h + 4 * j);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float xs[4] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w};
                    const float ws[4] = {wa[j].x, wa[j].y, wa[j].z, wa[j].w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (32 * h + 4 * j + k < nc) {
                            const float p = xs[k] * ws[k];
                            acc = acc + p;
                        }
                }
            }
        }
    }
    if (live) logits[(int64_t)s * E + e] = acc;
}

}  // namespace

int pk_launch_gemm_chain8(const float *X, int64_t ldx, const float *W, const float *bias, float *out, int64_t ldo,
                          int S, int I, int O, bool add_res, hipStream_t st) {
    PK_CHECK(S > 0 && I > 0 && O > 0, PK_ERR_ARG, "gemm chain8: bad shape");
    PK_CHECK((S + CH_ROWS - 1) / CH_ROWS <= 65535, PK_ERR_UNSUPPORTED, "gemm chain8: %d rows", S);
    const bool vec = (ldx & 3) == 0 && (I & 3) == 0 && (((uintptr_t)X | (uintptr_t)W) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL((k_gemm_chain8<float, true>), dim3((O + CH_OUTS - 1) / CH_OUTS, (S + CH_ROWS - 1) / CH_ROWS),
                           dim3(256), 0, st, X, ldx, W, nullptr, bias, out, ldo, S, I, O, add_res ? 1 : 0);
    else
        hipLaunchKernelGGL((k_gemm_chain8<float, false>), dim3((O + CH_OUTS - 1) / CH_OUTS, (S + CH_ROWS - 1) / CH_ROWS),
                           dim3(256), 0, st, X, ldx, W, nullptr, bias, out, ldo, S, I, O, add_res ? 1 : 0);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_gemm_chain8_q8(const float *X, const int8_t *W, const float *scale, float *out, int S, int I, int O,
                             hipStream_t st) {
    PK_CHECK(S > 0 && I > 0 && O > 0 && scale, PK_ERR_ARG, "gemm chain8 q8: bad argument");
    PK_CHECK((S + CH_ROWS - 1) / CH_ROWS <= 65535, PK_ERR_UNSUPPORTED, "gemm chain8: %d rows", S);
    hipLaunchKernelGGL((k_gemm_chain8<int8_t, false>), dim3((O + CH_OUTS - 1) / CH_OUTS, (S + CH_ROWS - 1) / CH_ROWS),
                       dim3(256), 0, st, X, (int64_t)I, W, scale, nullptr, out, (int64_t)O, S, I, O, 0);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_attn_rows_exact(int pos_base, int n, const float *qkv, int64_t qkv_stride, const float *Kl,
                              const float *Vl, int H, int KVH, int hd, int ctx, int sliding, int window,
                              const float *sinks, float *att, hipStream_t st) {
    PK_CHECK(n > 0 && n <= 65535 && H % KVH == 0, PK_ERR_ARG, "attention rows: bad shape");
    const int last = pos_base + n - 1;
    int span = (last < ctx ? last : ctx - 1) + 1;
    if (sliding && span > window) span = window;
    PK_CHECK((size_t)span * 4 <= 64 * 1024, PK_ERR_UNSUPPORTED, "attention rows: window of %d positions", span);
    hipLaunchKernelGGL(k_attn_rows_exact, dim3(H, n), dim3(64), (size_t)span * 4, st, pos_base, qkv, qkv_stride,
                       Kl, Vl, H, KVH, hd, ctx, sliding, window, sinks, att);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_launch_router_seq(const float *X, const float *R, const float *bias, int S, int D, int E, float *logits,
                         hipStream_t st) {
    PK_CHECK(S > 0 && D > 0 && E > 0 && E <= 128, PK_ERR_ARG, "router: bad shape");
    if (E >= 4 && (D & 3) == 0 && (((uintptr_t)X | (uintptr_t)R) & 15) == 0) {
        const int rows = 128 / E;
        const size_t lds = ((size_t)E + rows) * RQ_P * 4;
        hipLaunchKernelGGL(k_router_seq4, dim3((S + rows - 1) / rows), dim3(128), lds, st, X, R, bias, S, D, E,
                           logits);
        PK_HIP(hipGetLastError());
        return PK_OK;
    }
    const int rows = 128 / E;
    const size_t lds = ((size_t)RS_KC * E + (size_t)rows * RS_KC) * 4;
    hipLaunchKernelGGL(k_router_seq, dim3((S + rows - 1) / rows), dim3(128), lds, st, X, R, bias, S, D, E, logits);
    PK_HIP(hipGetLastError());
    return PK_OK;
}
