// pk_decode.hip — GQA decode attention and the forward_token driver.
//
// One decode step (forward_token, picchio.c:1655-1756) on the GPU:
//   embed + RMSNorm -> per layer: QKV GEMV + bias, RoPE/YaRN + KV store,
//   sink/sliding-window attention (split over position chunks), O GEMV + bias
//   + residual, RMSNorm, MoE (router+top-k, gate_up+SwiGLU, down+combine+
//   residual) -> final RMSNorm -> lm_head GEMV with a fused greedy argmax.
// The token and position live in device memory (pk_dstate), so a captured
// step can be replayed for every token: the argmax writes the next token,
// appends it to the output list and advances the position.
#include "pk_engine.h"
#include "pk_dev.h"
#include "pk_tagged.h"

#include <math.h>
#include <vector>

namespace {

constexpr int ATT_CHUNK = 128;         // positions per attention partial

__device__ __forceinline__ float wave_sum(float v) { return pk_wave_sum_f(v); }

// Token row -> h (zeros for an out-of-range id, picchio.c:1476-1480), and
// hn = rmsnorm(h) (quant.h:396-402: double sum of squares).
__global__ __launch_bounds__(256) void k_embed_rmsnorm(const pk_dstate *st, const float *embed, int vocab,
                                                       float *h, float *hn, const float *w, int D,
                                                       float eps) {
    __shared__ double part[4];
    const int tok = st->tok;
    const bool ok = tok >= 0 && tok < vocab;
    const float *row = embed + (int64_t)(ok ? tok : 0) * D;
    // every load goes out before the reduction (clamped, unconditional)
    float v[12], wv[12];
    pk_rms_load(row, D, v);
    pk_rms_load(w, D, wv);
#pragma unroll
    for (int k = 0; k < 12; ++k) v[k] = ok ? v[k] : 0.0f;
    const float r = pk_rms_finish(v, row, D, eps, part, !ok);
#pragma unroll
    for (int k = 0; k < 12; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i < D) {
            h[i] = v[k];
            hn[i] = v[k] * r * wv[k];
        }
    }
    for (int i = threadIdx.x + 256 * 12; i < D; i += 256) {
        const float x = ok ? row[i] : 0.0f;
        h[i] = x;
        hn[i] = x * r * w[i];
    }
}

// Decode QKV projection with the in_ln rmsnorm, the biases, RoPE
// (picchio.c:455-473) and the KV store (picchio.c:492-498) fused. Each wave
// computes one row; waves (0,1) and (2,3) hold the two rows of one rotation,
// (head*hd + j, head*hd + j + hd/2) for q and k heads, or two adjacent v
// rows, and meet in LDS, where the first of the pair rotates them with the
// host-built table at the decode position and writes q / K / V. The first
// weight loads are issued before the norm reduction so that they overlap it.
constexpr int QKV_U = 12;              // float4 per lane loaded up front (2880 columns = 11.25)

__device__ __forceinline__ void qkv_fma4(float &a, float4 x, pk_f32x4 w) {
    a = __builtin_fmaf(x.x, w.x, a);
    a = __builtin_fmaf(x.y, w.y, a);
    a = __builtin_fmaf(x.z, w.z, a);
    a = __builtin_fmaf(x.w, w.w, a);
}

__global__ __launch_bounds__(256) void k_qkv_rope_norm(const pk_dstate *st, const float *__restrict__ h,
                                                       const float *__restrict__ nw, float eps,
                                                       const float *__restrict__ W, const float *__restrict__ b,
                                                       int D, int H, int KVH, int hd, int ctx, const float *rope,
                                                       float *qkv, float *Kl, float *Vl, uint32_t *att_epoch) {
    __shared__ double npart[4];
    // a new tag for the fused attention launch that follows
    if (att_epoch && blockIdx.x == 0 && threadIdx.x == 0) *att_epoch = *att_epoch + 1u;
    __shared__ float pv[4];
    __shared__ __attribute__((aligned(16))) float xn[4 * 64 * QKV_U];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int half = hd / 2;
    const int n_rot = (H + KVH) * half, n_pairs = n_rot + KVH * half;
    const int pi = blockIdx.x * 2 + (wave >> 1);
    const bool live = pi < n_pairs;
    int r0 = 0, head = 0, j = 0;
    if (live) {
        if (pi < n_rot) {
            head = pi / half;
            j = pi - head * half;
            r0 = head * hd + j;
        } else {
            r0 = (H + KVH) * hd + 2 * (pi - n_rot);
        }
    }
    const int r1 = pi < n_rot ? r0 + half : r0 + 1;
    const int row = live ? ((wave & 1) ? r1 : r0) : 0;
    const pk_f32x4 *w4 = reinterpret_cast<const pk_f32x4 *>(W + (int64_t)row * D);
    const int n4 = D >> 2;
    // Every load goes out at the start, unconditionally (range-checked buffer
    // loads; a guarded load is waited for on its own): the norm's inputs and weights
    // first, so that the reduction runs while the row's first QKV_U float4
    // per lane are in flight, then this row's weights. The block writes the
    // normalised input (x * r) * w once into LDS for its four rows; the sum
    // runs over i = lane + 64 u, u ascending. A wave past the last pair
    // reads row 0 and writes nothing.
    float hv[12], nv[12];
    pk_rms_load(h, D, hv);
    pk_rms_load(nw, D, nv);
    const pk_buf_t wr = pk_buf(w4, (uint32_t)n4 * 16u);
    pk_f32x4 wf[QKV_U];
#pragma unroll
    for (int u = 0; u < QKV_U; ++u) wf[u] = pk_buf_load4_nt(wr, (uint32_t)(lane + u * 64) * 16u);
    const int pos = st->pos, kv_dim = KVH * hd;
    const float b0 = b[r0], b1 = b[r1];
    float cs = 0.0f, sn = 0.0f;
    if (pi < n_rot) {
        cs = rope[((int64_t)pos * half + j) * 2 + 0];
        sn = rope[((int64_t)pos * half + j) * 2 + 1];
    }
    const float rn = pk_rms_finish(hv, h, D, eps, npart);
    // (entries past the row are zeros on both sides: x = 0 * r * 0 in LDS,
    // w = 0 from the range check, so their products add nothing)
#pragma unroll
    for (int k = 0; k < 12; ++k) xn[threadIdx.x + 256 * k] = hv[k] * rn * nv[k];
    __syncthreads();
    const float4 *xn4 = reinterpret_cast<const float4 *>(xn);
    float a = 0.0f;
#pragma unroll
    for (int u = 0; u < QKV_U; ++u) qkv_fma4(a, xn4[lane + u * 64], wf[u]);
    const float4 *h4 = reinterpret_cast<const float4 *>(h);
    const float4 *n4w = reinterpret_cast<const float4 *>(nw);
    for (int i0 = lane + 64 * QKV_U; live && i0 < n4; i0 += 256) {
        pk_f32x4 wv[4];
        float4 xv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * 64;
            wv[u] = i < n4 ? __builtin_nontemporal_load(w4 + i) : pk_f32x4{0.f, 0.f, 0.f, 0.f};
            xv[u] = i < n4 ? pk_norm4(h4[i], rn, n4w[i]) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) qkv_fma4(a, xv[u], wv[u]);
    }
    a = wave_sum(a);
    if (lane == 0) pv[wave] = a;
    __syncthreads();
    if (!live || (wave & 1) || lane != 0) return;
    const float v0 = pv[wave] + b0, v1 = pv[wave + 1] + b1;
    if (pi < n_rot) {
        const float q0 = __builtin_fmaf(v0, cs, -(v1 * sn));     // a*cs - b*sn (contracted)
        const float q1 = __builtin_fmaf(v0, sn, v1 * cs);        // a*sn + b*cs (contracted)
        qkv[r0] = q0;
        qkv[r1] = q1;
        if (head >= H) {
            Kl[pk_k_off(pos, head - H, j, ctx, KVH, hd)] = q0;
            Kl[pk_k_off(pos, head - H, j + half, ctx, KVH, hd)] = q1;
        }
    } else {
        qkv[r0] = v0;
        qkv[r1] = v1;
        const int c = r0 - (H + KVH) * hd;
        Vl[(int64_t)pos * kv_dim + c] = v0;
        Vl[(int64_t)pos * kv_dim + c + 1] = v1;
    }
}

// Position of row r: the decode step's (device state), or pos_base + r * step
// (step 1: consecutive prompt positions; step 0: sequences at one position).
__device__ __forceinline__ int row_pos(const pk_dstate *st, int pos_base, int step, int r) {
    return st ? st->pos : pos_base + r * step;
}

// RoPE (picchio.c:455-473) on q [H][hd] and k [KVH][hd] at the row's position
// with the host-built cos/sin table (attn_factor folded in), then kv_store
// (picchio.c:492-498): K/V rows of this layer at that position. grid.y = row;
// row r's cache starts kv_row * r floats after Kl / Vl.
// With ws (the split partial tiles [splits][32][qkv_stride] of a skinny
// GEMM over at most 32 rows), each value is first k_gemm_splits' sum of the
// row's partials + bias, written to qkv.
__device__ __forceinline__ float splits_sum(const float *ws, int splits, int r, int O, int col, const float *bias) {
    float sum = ws[(int64_t)r * O + col];
    for (int k = 1; k < splits; ++k) sum = sum + ws[((int64_t)k * 32 + r) * O + col];
    if (bias) sum = sum + bias[col];
    return sum;
}

__global__ void k_rope_kv(const pk_dstate *st, int pos_base, int pos_step, float *qkv, int64_t qkv_stride,
                          const float *rope, int H, int KVH, int hd, int ctx, float *Kl, float *Vl, int64_t kv_row,
                          const float *ws = nullptr, int splits = 1, const float *bias = nullptr) {
    const int pos = row_pos(st, pos_base, pos_step, blockIdx.y);
    const int r = blockIdx.y;
    qkv += (int64_t)blockIdx.y * qkv_stride;
    Kl += (int64_t)blockIdx.y * kv_row;
    Vl += (int64_t)blockIdx.y * kv_row;
    const int half = hd / 2;
    const int n_pairs = (H + KVH) * half;
    const int kv_dim = KVH * hd;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_pairs) {
        const int head = i / half, j = i - head * half;
        float *v = qkv + head * hd;                     // q heads then k heads
        const float cs = rope[((int64_t)pos * half + j) * 2 + 0];
        const float sn = rope[((int64_t)pos * half + j) * 2 + 1];
        const float a = ws ? splits_sum(ws, splits, r, (int)qkv_stride, head * hd + j, bias) : v[j];
        const float b = ws ? splits_sum(ws, splits, r, (int)qkv_stride, head * hd + j + half, bias) : v[j + half];
        const float r0 = __builtin_fmaf(a, cs, -(b * sn));   // a*cs - b*sn (contracted)
        const float r1 = __builtin_fmaf(a, sn, b * cs);      // a*sn + b*cs (contracted)
        v[j] = r0;
        v[j + half] = r1;
        if (head >= H) {
            Kl[pk_k_off(pos, head - H, j, ctx, KVH, hd)] = r0;
            Kl[pk_k_off(pos, head - H, j + half, ctx, KVH, hd)] = r1;
        }
    } else if (i < n_pairs + kv_dim) {
        const int c = i - n_pairs;
        float val;
        if (ws) {
            val = splits_sum(ws, splits, r, (int)qkv_stride, (H + KVH) * hd + c, bias);
            qkv[(H + KVH) * hd + c] = val;
        } else {
            val = qkv[(H + KVH) * hd + c];
        }
        Vl[(int64_t)pos * kv_dim + c] = val;
    }
}

// Window of picchio.c:556-567 for this layer at pos.
__device__ __forceinline__ void att_window(int pos, int ctx, int sliding, int window, int &start, int &end) {
    end = pos < ctx ? pos : ctx - 1;
    start = 0;
    if (sliding) {
        start = end - window + 1;
        if (start < 0) start = 0;
    }
}

// Attention partials: block (b, c, r) covers positions start+128c .. +127 of
// row r's window for gs of the G = H/KVH query heads that share one KV head
// (block b: KV head b / (G/gs), heads (b % (G/gs)) * gs ..), so each K and V
// row is read once per gs heads: gs = G at long contexts and large batches
// (one read per group), smaller when there would be too few blocks. Per head the arithmetic
// is fixed: scores are the reference's in-order dot (uncontracted products
// added one by one, picchio.c:573-577 as gcc builds it) times 1/sqrt(hd); the
// chunk max; p = exp(s - max) and its sum (lanes over t, t+64, then the wave
// tree); the exp-weighted V sum as hd/4 float4 columns x (128*4/hd) position
// groups summed in position order, the groups then added in order
// (flash-decoding partials).
//
// Threads (128 per half, one or two halves): half = tid / 128 takes heads
// [half*GH, half*GH + GH), GH = ceil(gs / halves); t = tid % 128 is the
// position for the scores and (column, group) for V.
//
// A window of one chunk is finished by its block (the combine's operations
// for one chunk). Otherwise the partials are stored device-coherently; the
// last of the row's chunk blocks to arrive at its (row, b) counter combines
// them (16 chunks' partials per load round) for the gs heads
// with the learned sinks (picchio.c:586-604: the sink joins the max and the
// denominator, not the value sum), writes att [row][h*hd..] and re-arms the
// counter.
constexpr int ATT_THREADS = 256;
constexpr int ATT_GH = 8;              // query heads per half-block (G <= 16)

// Block (bx, by, bz) of a (gdx, gdy, rows) grid: k_attn_part's own blocks,
// or the attention blocks of k_attn_oproj, which take the output as tagged
// words att_t (row 0, tag) instead of att.
template <int KD4>
__device__ __forceinline__ void attn_part_block(const pk_dstate *st, int pos_base, int pos_step, const float *qkv,
                                                int64_t qkv_stride, const float *Kl, const float *Vl, int64_t kv_row,
                                                int H, int KVH, int hd, int ctx, int sliding, int window,
                                                float *part, int max_chunks, const float *sinks, float *att,
                                                uint32_t *ctr, int gs, int bx, int by, int bz, int gdx, int gdy,
                                                uint64_t *att_t, uint32_t tag) {
    extern __shared__ __attribute__((aligned(16))) float att_lds[];
    const int G = gs;                         // heads of this block
    float *q = att_lds;                       // [G][hd]
    float *p = q + G * hd;                    // [G][128]
    float *vred = p;                          // [G][PG][hd] over p once the V sums have read it
    __shared__ float red[4][ATT_GH];
    __shared__ float mh[2 * ATT_GH];
    __shared__ float ssum[2 * ATT_GH];
    __shared__ int last;
    // Workgroups go to the 8 XCDs round-robin by linear id, each XCD with its
    // own L2: the SUB blocks that read the same (KV head, chunk) tile get ids
    // equal mod 8, so the tile comes from HBM once.
    const int SUB = (H / KVH) / gs;
    int b = bx, c = by;
    if (SUB > 1 && (KVH * gdy) % 8 == 0) {
        const int L = bx + gdx * by;
        const int q8 = L >> 3, p8 = L & 7;
        const int pp = (q8 / SUB) * 8 + p8;            // (KV head, chunk) pair
        c = pp / KVH;
        b = (pp - c * KVH) * SUB + q8 % SUB;
    }
    const int r = bz;
    const int kvh = b / SUB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = tid >> 7, tt = tid & 127;
    const int halves = blockDim.x >> 7, waves = blockDim.x >> 6;
    const int GH = (G + halves - 1) / halves;
    const int ja = half * GH, jn = min(G, ja + GH) - ja;    // this half's heads
    qkv += (int64_t)r * qkv_stride;
    part += (int64_t)r * H * max_chunks * (hd + 2);
    Kl += (int64_t)r * kv_row;
    Vl += (int64_t)r * kv_row;
    int start, end;
    att_window(row_pos(st, pos_base, pos_step, r), ctx, sliding, window, start, end);
    const int t0 = start + c * ATT_CHUNK;
    const int n = min(ATT_CHUNK, end - t0 + 1);
    if (n <= 0) return;
    const int kv_dim = KVH * hd, h0 = b * gs;
    // The query rows and this thread's K row (position tt; KD4 >= hd / 4
    // float4) go out before any wait, with the query rows' LDS copy behind
    // them; the V rows go out right after the scores, so that they arrive
    // during the softmax. Loads are unconditional: positions past the
    // chunk's last are clamped to it and their values are not used.
    float qv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) qv[k] = qkv[h0 * hd + min(tid + k * (int)blockDim.x, G * hd - 1)];
    const int D4 = hd >> 2;
    // (the K cache's chunk layout: float4 u of neighbouring positions adjacent)
    const int tk = t0 + min(tt, n - 1);
    const int kcs = pk_k_cs(tk, ctx);
    const float4 *kt4 = reinterpret_cast<const float4 *>(Kl + pk_k_off(tk, kvh, 0, ctx, KVH, hd));
    float4 kv[KD4];
#pragma unroll
    for (int u = 0; u < KD4; ++u) kv[u] = kt4[(int64_t)min(u, D4 - 1) * kcs];
    // (clamped like the loads: threads past G * hd write the last value
    // again; a guarded store would let its load sink behind the K loads)
#pragma unroll
    for (int k = 0; k < 4; ++k) q[min(tid + k * (int)blockDim.x, G * hd - 1)] = qv[k];
    for (int i = tid + 4 * blockDim.x; i < G * hd; i += blockDim.x) q[i] = qkv[h0 * hd + i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)hd);

    // scores of position tt for this half's heads (columns in order)
    float sc[ATT_GH];
#pragma unroll
    for (int jj = 0; jj < ATT_GH; ++jj) sc[jj] = -INFINITY;
    if (tt < n) {
        float dot[ATT_GH];
#pragma unroll
        for (int jj = 0; jj < ATT_GH; ++jj) dot[jj] = 0.0f;
        // (guards, not early exits, so that kv[] stays in registers)
#pragma unroll
        for (int u = 0; u < KD4; ++u) {
            if (u < D4) {
#pragma unroll
            for (int jj = 0; jj < ATT_GH; ++jj) {
                if (jj >= jn) break;
                const float *qq = q + (ja + jj) * hd + 4 * u;
                float pr;
                pr = qq[0] * kv[u].x; dot[jj] = dot[jj] + pr;
                pr = qq[1] * kv[u].y; dot[jj] = dot[jj] + pr;
                pr = qq[2] * kv[u].z; dot[jj] = dot[jj] + pr;
                pr = qq[3] * kv[u].w; dot[jj] = dot[jj] + pr;
            }
            }
        }
#pragma unroll
        for (int jj = 0; jj < ATT_GH; ++jj) sc[jj] = dot[jj] * scale;
    }
    // V rows: thread = (column group c4 of hd/4, position group g of PG) of
    // its half, positions g * PER + j, j < PER (PER = hd / 4 <= KD4). (Issued
    // with the K rows they cost registers: 3 instead of 4 blocks per SIMD,
    // slower at batch 1 and 32.)
    const int PG = ATT_CHUNK / D4, PER = ATT_CHUNK / PG;
    const int c4 = tt % D4, g = tt / D4;
    const float4 *v4 = reinterpret_cast<const float4 *>(Vl + (int64_t)t0 * kv_dim + kvh * hd) + c4;
    const int kv4 = kv_dim >> 2;
    float4 vv[KD4];
#pragma unroll
    for (int j = 0; j < KD4; ++j) vv[j] = v4[(int64_t)min(g * PER + min(j, PER - 1), n - 1) * kv4];
    // per-head chunk max over the half's two waves, then p = exp(s - m)
#pragma unroll
    for (int jj = 0; jj < ATT_GH; ++jj) {
        if (jj >= jn) break;
        const float m = pk_wave_max_f(sc[jj]);
        if (lane == 0) red[wave][jj] = m;
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < ATT_GH; ++jj) {
        if (jj >= jn) break;
        const float m = fmaxf(red[2 * half][jj], red[2 * half + 1][jj]);
        p[(ja + jj) * ATT_CHUNK + tt] = tt < n ? expf(sc[jj] - m) : 0.0f;
        if (tt == 0) mh[ja + jj] = m;
    }
    __syncthreads();
    // chunks of this row's window; with one, this block finishes the softmax
    const int nc = (end - start + 1 + ATT_CHUNK - 1) / ATT_CHUNK;
    // per-head sums: wave w takes heads w, w + waves, ...
    for (int j = wave; j < G; j += waves) {
        const float *pj = p + j * ATT_CHUNK;
        float sum = 0.0f;
        for (int t = lane; t < n; t += 64) sum += pj[t];
        sum = wave_sum(sum);
        if (lane == 0) {
            if (nc == 1) {
                ssum[j] = sum;
            } else {
                float *out = part + ((int64_t)(h0 + j) * max_chunks + c) * (hd + 2);
                __hip_atomic_store(out, mh[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(out + 1, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    // V sums over this thread's positions, in position order
    float4 acc[ATT_GH];
#pragma unroll
    for (int jj = 0; jj < ATT_GH; ++jj) acc[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < KD4; ++j) {
        const int t = g * PER + j;
        const bool ok = j < PER && t < n;
#pragma unroll
        for (int jj = 0; jj < ATT_GH; ++jj) {
            if (jj >= jn) break;
            const float pw = ok ? p[(ja + jj) * ATT_CHUNK + t] : 0.0f;
            acc[jj].x = __builtin_fmaf(pw, vv[j].x, acc[jj].x);
            acc[jj].y = __builtin_fmaf(pw, vv[j].y, acc[jj].y);
            acc[jj].z = __builtin_fmaf(pw, vv[j].z, acc[jj].z);
            acc[jj].w = __builtin_fmaf(pw, vv[j].w, acc[jj].w);
        }
    }
    __syncthreads();                          // every read of p is done: vred overwrites it
#pragma unroll
    for (int jj = 0; jj < ATT_GH; ++jj) {
        if (jj >= jn) break;
        *reinterpret_cast<float4 *>(&vred[((ja + jj) * PG + g) * hd + 4 * c4]) = acc[jj];
    }
    __syncthreads();
    if (nc == 1) {
        // the combine below with a single chunk, in its operations
        for (int idx = tid; idx < G * hd; idx += blockDim.x) {
            const int j = idx / hd, i = idx - j * hd, h = h0 + j;
            float o = 0.0f;
            for (int gg = 0; gg < PG; ++gg) o += vred[(j * PG + gg) * hd + i];
            const float M = fmaxf(sinks[h], mh[j]);
            const float e = expf(mh[j] - M);
            float S = expf(sinks[h] - M);
            S += ssum[j] * e;
            const float v = __builtin_fmaf(o, e, 0.0f) / S;
            if (att_t) pk_put_tagged(att_t + h * hd + i, tag, __float_as_uint(v));
            else att[(int64_t)r * H * hd + h * hd + i] = v;
        }
        return;
    }
    for (int idx = tid; idx < G * hd; idx += blockDim.x) {
        const int j = idx / hd, i = idx - j * hd;
        float o = 0.0f;
        for (int gg = 0; gg < PG; ++gg) o += vred[(j * PG + gg) * hd + i];
        float *out = part + ((int64_t)(h0 + j) * max_chunks + c) * (hd + 2);
        __hip_atomic_store(out + 2 + i, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // arrival: the last of the nc chunk blocks of (row, b) combines
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *cnt = ctr + (int64_t)r * gdx + b;
    if (tid == 0)
        last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(nc - 1);
    __syncthreads();
    if (!last) return;
    // every chunk's max and sum in one load round (LDS: the p region holds
    // G x 128 values); then per head the max M, the chunk factors
    // e_c = expf(m_c - M) and the denominator, in chunk order; the value
    // partials are read 16 chunks per round
    auto ld = [](const float *q) { return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto ld2 = [](const float *q) {
        const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t *>(q), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
    };
    constexpr int CB = 16;
    float *cm = p;                            // [G][nc] chunk maxima, then factors e_c
    float *cs = p + G * ATT_CHUNK;            // [G][nc] chunk sums (the V partials are stored)
    __shared__ float hS[2 * ATT_GH];
    // Windows of CB < nc <= CO chunks, or more outputs than threads: a thread
    // takes column pairs (i, i + 1) of a head, every chunk's two values in one
    // 8-byte load round, the first pair's round with the maxima and sums
    // (batch-32 full-context layers 167 -> 158 us; for short windows with an
    // output per thread the path below is faster: config 2 594 against 589 tok/s).
    constexpr int CO = 36;
    if (nc <= CO && (hd & 1) == 0 && (nc > CB || G * hd > (int)blockDim.x)) {
        const int np = G * hd / 2;            // column pairs
        float2 ov[CO];
        auto load_pair = [&](int pi) {
            const int j = pi / (hd / 2), i = 2 * (pi - j * (hd / 2));
            const float *ph = part + (int64_t)(h0 + j) * max_chunks * (hd + 2) + 2 + i;
#pragma unroll
            for (int u = 0; u < CO; ++u) ov[u] = u < nc ? ld2(ph + u * (hd + 2)) : make_float2(0.f, 0.f);
        };
        if (tid < np) load_pair(tid);
        for (int q0 = tid; q0 < G * nc; q0 += blockDim.x * 4) {
            float mv[4], sv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q = q0 + u * blockDim.x;
                const int j = q / nc, cc = q - j * nc;
                const float *pc = part + ((int64_t)(h0 + j) * max_chunks + cc) * (hd + 2);
                mv[u] = q < G * nc ? ld(pc) : 0.0f;
                sv[u] = q < G * nc ? ld(pc + 1) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q = q0 + u * blockDim.x;
                if (q < G * nc) { cm[q] = mv[u]; cs[q] = sv[u]; }
            }
        }
        __syncthreads();
        if (tid < G) {
            const int j = tid, h = h0 + j;
            float M = sinks[h];
            for (int cc = 0; cc < nc; ++cc) M = fmaxf(M, cm[j * nc + cc]);
            float S = expf(sinks[h] - M);
            for (int cc = 0; cc < nc; ++cc) {
                const float ec = expf(cm[j * nc + cc] - M);
                S += cs[j * nc + cc] * ec;
                cm[j * nc + cc] = ec;
            }
            hS[j] = S;
        }
        __syncthreads();
        for (int pi = tid; pi < np; pi += blockDim.x) {
            if (pi != tid) load_pair(pi);
            const int j = pi / (hd / 2), i = 2 * (pi - j * (hd / 2)), h = h0 + j;
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
            for (int u = 0; u < CO; ++u)
                if (u < nc) {
                    o0 = __builtin_fmaf(ov[u].x, cm[j * nc + u], o0);
                    o1 = __builtin_fmaf(ov[u].y, cm[j * nc + u], o1);
                }
            if (att_t) {
                pk_put_tagged(att_t + h * hd + i, tag, __float_as_uint(o0 / hS[j]));
                pk_put_tagged(att_t + h * hd + i + 1, tag, __float_as_uint(o1 / hS[j]));
            } else {
                att[(int64_t)r * H * hd + h * hd + i] = o0 / hS[j];
                att[(int64_t)r * H * hd + h * hd + i + 1] = o1 / hS[j];
            }
        }
    } else if (nc <= ATT_CHUNK) {
        for (int q0 = tid; q0 < G * nc; q0 += blockDim.x * 4) {
            float mv[4], sv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q = q0 + u * blockDim.x;
                const int j = q / nc, cc = q - j * nc;
                const float *pc = part + ((int64_t)(h0 + j) * max_chunks + cc) * (hd + 2);
                mv[u] = q < G * nc ? ld(pc) : 0.0f;
                sv[u] = q < G * nc ? ld(pc + 1) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q = q0 + u * blockDim.x;
                if (q < G * nc) { cm[q] = mv[u]; cs[q] = sv[u]; }
            }
        }
        __syncthreads();
        if (tid < G) {
            const int j = tid, h = h0 + j;
            float M = sinks[h];
            for (int cc = 0; cc < nc; ++cc) M = fmaxf(M, cm[j * nc + cc]);
            float S = expf(sinks[h] - M);
            for (int cc = 0; cc < nc; ++cc) {
                const float ec = expf(cm[j * nc + cc] - M);
                S += cs[j * nc + cc] * ec;
                cm[j * nc + cc] = ec;
            }
            hS[j] = S;
        }
        __syncthreads();
        for (int idx = tid; idx < G * hd; idx += blockDim.x) {
            const int j = idx / hd, i = idx - j * hd, h = h0 + j;
            const float *ph = part + (int64_t)h * max_chunks * (hd + 2);
            float o = 0.0f;
            for (int c0 = 0; c0 < nc; c0 += CB) {
                float ov[CB];
#pragma unroll
                for (int u = 0; u < CB; ++u) ov[u] = c0 + u < nc ? ld(ph + (c0 + u) * (hd + 2) + 2 + i) : 0.0f;
#pragma unroll
                for (int u = 0; u < CB; ++u)
                    if (c0 + u < nc) o = __builtin_fmaf(ov[u], cm[j * nc + c0 + u], o);
            }
            if (att_t) pk_put_tagged(att_t + h * hd + i, tag, __float_as_uint(o / hS[j]));
            else att[(int64_t)r * H * hd + h * hd + i] = o / hS[j];
        }
    } else {
        // windows longer than 128 chunks: the same arithmetic, reading the
        // partials 16 chunks per round in each pass
        for (int idx = tid; idx < G * hd; idx += blockDim.x) {
            const int j = idx / hd, i = idx - j * hd, h = h0 + j;
            const float *ph = part + (int64_t)h * max_chunks * (hd + 2);
            float M = sinks[h];
            for (int c0 = 0; c0 < nc; c0 += CB) {
                float mv[CB];
#pragma unroll
                for (int u = 0; u < CB; ++u) mv[u] = c0 + u < nc ? ld(ph + (c0 + u) * (hd + 2)) : -INFINITY;
#pragma unroll
                for (int u = 0; u < CB; ++u) M = fmaxf(M, mv[u]);
            }
            float S = expf(sinks[h] - M);
            for (int c0 = 0; c0 < nc; c0 += CB) {
                float mv[CB], sv[CB];
#pragma unroll
                for (int u = 0; u < CB; ++u) {
                    mv[u] = c0 + u < nc ? ld(ph + (c0 + u) * (hd + 2)) : 0.0f;
                    sv[u] = c0 + u < nc ? ld(ph + (c0 + u) * (hd + 2) + 1) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < CB; ++u)
                    if (c0 + u < nc) S += sv[u] * expf(mv[u] - M);
            }
            float o = 0.0f;
            for (int c0 = 0; c0 < nc; c0 += CB) {
                float mv[CB], ov[CB];
#pragma unroll
                for (int u = 0; u < CB; ++u) {
                    mv[u] = c0 + u < nc ? ld(ph + (c0 + u) * (hd + 2)) : 0.0f;
                    ov[u] = c0 + u < nc ? ld(ph + (c0 + u) * (hd + 2) + 2 + i) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < CB; ++u)
                    if (c0 + u < nc) o = __builtin_fmaf(ov[u], expf(mv[u] - M), o);
            }
            if (att_t) pk_put_tagged(att_t + h * hd + i, tag, __float_as_uint(o / S));
            else att[(int64_t)r * H * hd + h * hd + i] = o / S;
        }
    }
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KD4>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_part(const pk_dstate *st, int pos_base, int pos_step,
                                                           const float *qkv, int64_t qkv_stride, const float *Kl,
                                                           const float *Vl, int64_t kv_row, int H, int KVH,
                                                           int hd, int ctx, int sliding, int window, float *part,
                                                           int max_chunks, const float *sinks, float *att,
                                                           uint32_t *ctr, int gs) {
    attn_part_block<KD4>(st, pos_base, pos_step, qkv, qkv_stride, Kl, Vl, kv_row, H, KVH, hd, ctx, sliding, window,
                         part, max_chunks, sinks, att, ctr, gs, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x,
                         gridDim.y, nullptr, 0);
}

// y[o] += (W[o] . x + b[o])  — attention output projection + residual
// (picchio.c:615-616, :1690). One workgroup per 4 outputs (one per wave);
// grid.y = row of a batch (x [rows][I], y [rows][O]).
constexpr int RES_U = 16;              // float4 per lane loaded up front (4096 columns)
constexpr int ATT_RPW = 2;             // k_attn_oproj: output rows per wave

__global__ __launch_bounds__(256) void k_gemv_res(float *y, const float *__restrict__ x,
                                                  const float *__restrict__ W,
                                                  const float *__restrict__ b, int I, int O) {
    const int lane = threadIdx.x & 63;
    y += (int64_t)blockIdx.y * O;
    x += (int64_t)blockIdx.y * I;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= O) return;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const pk_f32x4 *w4 = reinterpret_cast<const pk_f32x4 *>(W + (int64_t)o * I);
    const int n4 = I >> 2;
    // the row's first RES_U float4 per lane in one round trip; the sum runs
    // over i = lane + 64 u, u ascending, as in the chunked loop after it
    // (range-checked buffer loads, all issued before the first use; entries
    // past the row read as zero and are not used)
    const pk_buf_t wr = pk_buf(w4, (uint32_t)n4 * 16u), xr = pk_buf(x4, (uint32_t)n4 * 16u);
    // the residual and the bias at entry (at the end each would cost a round trip)
    const float yo = y[o], bo = b[o];
    pk_f32x4 wv[RES_U];
    float4 xv[RES_U];
#pragma unroll
    for (int u = 0; u < RES_U; ++u) {
        xv[u] = pk_buf_load4(xr, (uint32_t)(lane + u * 64) * 16u);
        wv[u] = pk_buf_load4_nt(wr, (uint32_t)(lane + u * 64) * 16u);
    }
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < RES_U; ++u) {
        const int i = lane + u * 64;
        if (i < n4) qkv_fma4(acc, xv[u], wv[u]);
    }
    for (int i0 = lane + 64 * RES_U; i0 < n4; i0 += 64 * 4) {
        float4 xv[4];
        pk_f32x4 wc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * 64;
            xv[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            wc[u] = i < n4 ? __builtin_nontemporal_load(w4 + i) : pk_f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) qkv_fma4(acc, xv[u], wc[u]);
    }
    for (int i = (n4 << 2) + lane; i < I; i += 64) acc = __builtin_fmaf(x[i], W[(int64_t)o * I + i], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[o] = yo + (acc + bo);
}

// Decode attention and its output projection in one launch (one row,
// picchio.c:504-623 then :615-616, :1690). Blocks [0, gdx * gdy) are
// k_attn_part's blocks; they hand the attention row over as tagged words
// (pk_tagged.h, tag = *epoch, advanced by the QKV launch before). Each
// other block computes y[o] += W[o] . att + b[o] for 4 * ATT_RPW rows o
// (ATT_RPW per wave) with k_gemv_res's arithmetic per row: its weight rows
// go out at entry, so that they stream in while the attention runs, then
// the block reads the tagged row into LDS (one read per block: two rows
// per wave halve those reads) and finishes. The attention blocks wait for nothing
// (their chunk combine is a last-arrival count) and come first in dispatch
// order, so the waiting blocks cannot hold them back.
template <int KD4>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_oproj(const pk_dstate *st, const float *qkv, const float *Kl,
                                                            const float *Vl, int H, int KVH, int hd, int ctx,
                                                            int sliding, int window, float *part, int max_chunks,
                                                            const float *sinks, uint32_t *ctr, int gs, int gdx,
                                                            int gdy, uint64_t *att_t, const uint32_t *epoch,
                                                            uint32_t *status, float *y, const float *__restrict__ W,
                                                            const float *__restrict__ b, int O) {
    extern __shared__ __attribute__((aligned(16))) float att_lds[];
    const uint32_t tag = __builtin_amdgcn_readfirstlane(*epoch);
    const int n_att = gdx * gdy;
    if ((int)blockIdx.x < n_att) {
        const int bx = blockIdx.x % gdx, by = blockIdx.x / gdx;
        attn_part_block<KD4>(st, 0, 0, qkv, 0, Kl, Vl, 0, H, KVH, hd, ctx, sliding, window, part, max_chunks,
                             sinks, nullptr, ctr, gs, bx, by, 0, gdx, gdy, att_t, tag);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int o0 = (((int)blockIdx.x - n_att) * 4 + (threadIdx.x >> 6)) * ATT_RPW;   // this wave's rows
    const int I = H * hd, n4 = I >> 2;                 // I <= 64 * RES_U * 4, I % 4 == 0
    // the residual rows and biases first (read again at the end they would
    // cost a round trip of their own), then the weight rows
    float yv[ATT_RPW], bv[ATT_RPW];
#pragma unroll
    for (int k = 0; k < ATT_RPW; ++k) {
        yv[k] = y[min(o0 + k, O - 1)];
        bv[k] = b[min(o0 + k, O - 1)];
    }
    pk_f32x4 wv[ATT_RPW][RES_U];
#pragma unroll
    for (int k = 0; k < ATT_RPW; ++k) {
        const pk_buf_t wr = pk_buf(W + (int64_t)min(o0 + k, O - 1) * I, (uint32_t)n4 * 16u);
#pragma unroll
        for (int u = 0; u < RES_U; ++u) wv[k][u] = pk_buf_load4_nt(wr, (uint32_t)(lane + u * 64) * 16u);
    }
    // the attention row: RES_U / 4 tagged words per thread, polled until all
    // carry this launch's tag
    constexpr int TW = RES_U * 64 * 4 / ATT_THREADS;
    uint64_t tw[TW];
#pragma unroll
    for (int k = 0; k < TW; ++k) {
        const int i = threadIdx.x + k * ATT_THREADS;
        tw[k] = i < I ? __hip_atomic_load(att_t + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : (uint64_t)tag << 32;
    }
    const uint32_t bound = pk_poll_bound(status);
    for (uint32_t n = 0;; ++n) {
        bool stale = false;
#pragma unroll
        for (int k = 0; k < TW; ++k) stale |= (uint32_t)(tw[k] >> 32) != tag;
        if (!__any(stale)) break;
        if (n >= bound) {
            if (lane == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < TW; ++k)
            if ((uint32_t)(tw[k] >> 32) != tag)
                tw[k] = __hip_atomic_load(att_t + threadIdx.x + k * ATT_THREADS, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int k = 0; k < TW; ++k) {
        const int i = threadIdx.x + k * ATT_THREADS;
        if (i < I) att_lds[i] = __uint_as_float((uint32_t)tw[k]);
    }
    __syncthreads();
    const float4 *x4 = reinterpret_cast<const float4 *>(att_lds);
    float acc[ATT_RPW];
#pragma unroll
    for (int k = 0; k < ATT_RPW; ++k) acc[k] = 0.0f;
#pragma unroll
    for (int u = 0; u < RES_U; ++u) {
        const int i = lane + u * 64;
        if (i < n4) {
            const float4 xv = x4[i];
#pragma unroll
            for (int k = 0; k < ATT_RPW; ++k) qkv_fma4(acc[k], xv, wv[k][u]);
        }
    }
#pragma unroll
    for (int k = 0; k < ATT_RPW; ++k) {
        const float a = wave_sum(acc[k]);
        if (lane == 0 && o0 + k < O) y[o0 + k] = yv[k] + (a + bv[k]);
    }
}

// lm_head GEMV (fp32 or INT8 rows) and the greedy argmax of sample_logits
// (first maximum, picchio.c:1555-1560), in two launches: every block writes
// its rows' logits and its best (value, lowest index) pair; one workgroup
// then reduces the block pairs, writes the token, appends it to the output
// list and advances the position. (A single arrival counter for ~25k blocks
// serialised at L2 and cost more than the second launch.)
constexpr int LM_ROWS_PER_BLOCK = 8;      // 4 waves x 2 rows

__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

template <bool Q8>
__global__ __launch_bounds__(256) void k_lm_head(const float *__restrict__ x, const void *__restrict__ Wv,
                                                 const float *__restrict__ sc, int I, int O, float *logits,
                                                 float *bval, int32_t *bidx) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const int n4 = I >> 2;
    const int o0 = blockIdx.x * LM_ROWS_PER_BLOCK + wave * 2;
    float acc[2] = {0.0f, 0.0f};
    bool nan0 = false;                        // logit 0 is NaN (block 0, wave 0)
    if (Q8) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int8_t *w = reinterpret_cast<const int8_t *>(Wv) + (int64_t)min(o0 + r, O - 1) * I;
            for (int i = lane; i < I; i += 64) acc[r] = __builtin_fmaf(x[i], (float)w[i], acc[r]);
        }
    } else {
        const pk_f32x4 *w4[2];
#pragma unroll
        for (int r = 0; r < 2; ++r)
            w4[r] = reinterpret_cast<const pk_f32x4 *>(reinterpret_cast<const float *>(Wv) +
                                                       (int64_t)min(o0 + r, O - 1) * I);
        for (int i0 = lane; i0 < n4; i0 += 64 * 4) {
            float4 xv[4];
            pk_f32x4 wv[2][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * 64;
                xv[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int r = 0; r < 2; ++r)
                    wv[r][u] = i < n4 ? __builtin_nontemporal_load(w4[r] + i) : pk_f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    acc[r] = __builtin_fmaf(xv[u].x, wv[r][u].x, acc[r]);
                    acc[r] = __builtin_fmaf(xv[u].y, wv[r][u].y, acc[r]);
                    acc[r] = __builtin_fmaf(xv[u].z, wv[r][u].z, acc[r]);
                    acc[r] = __builtin_fmaf(xv[u].w, wv[r][u].w, acc[r]);
                }
        }
        for (int i = (n4 << 2) + lane; i < I; i += 64)
#pragma unroll
            for (int r = 0; r < 2; ++r)
                acc[r] = __builtin_fmaf(x[i], reinterpret_cast<const float *>(Wv)[(int64_t)min(o0 + r, O - 1) * I + i],
                                        acc[r]);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        float v = wave_sum(acc[r]);
        const int o = o0 + r;
        if (o < O) {
            if (Q8) v = v * sc[o];
            if (lane == 0 && logits) logits[o] = v;
            if (o == 0 && v != v) nan0 = true;
            better(bv, bi, v, o);
        }
    }
    if (lane == 0) { rv[wave] = bv; ri[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) better(bv, bi, rv[w], ri[w]);
        bval[blockIdx.x] = bv;
        bidx[blockIdx.x] = nan0 ? -1 : bi;     // -1: the argmax must keep index 0
    }
}

// One workgroup: the best of the block pairs, then the decode-state update.
__global__ __launch_bounds__(1024) void k_argmax_blocks(const float *bval, const int32_t *bidx, int nb,
                                                        pk_dstate *st, int32_t *out_toks, int out_cap) {
    __shared__ float rv[16];
    __shared__ int ri[16];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // the pairs in rounds of AM_U per thread, every load of a round issued
    // before the first comparison (range-checked: entries past nb are
    // skipped); better() picks the same pair in any order
    constexpr int AM_U = 32;
    const pk_buf_t vr = pk_buf(bval, (uint32_t)nb * 4u), ir = pk_buf(bidx, (uint32_t)nb * 4u);
    for (int b0 = 0; b0 < nb; b0 += AM_U * (int)blockDim.x) {
        float v[AM_U];
        int ix[AM_U];
#pragma unroll
        for (int u = 0; u < AM_U; ++u) {
            const uint32_t off = (uint32_t)(b0 + (int)threadIdx.x + u * (int)blockDim.x) * 4u;
            v[u] = pk_buf_load_f32(vr, off);
            ix[u] = __float_as_int(pk_buf_load_f32(ir, off));
        }
#pragma unroll
        for (int u = 0; u < AM_U; ++u)
            if (b0 + (int)threadIdx.x + u * (int)blockDim.x < nb) better(bv, bi, v[u], ix[u]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        better(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) { rv[threadIdx.x >> 6] = bv; ri[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) better(bv, bi, rv[w], ri[w]);
        // the reference's greedy scan (picchio.c:1555-1560) starts at index 0
        // and moves on a strictly greater value only: with logit 0 NaN it
        // keeps 0 (k_lm_head marks that case with index -1 in block 0)
        const int tok = (bi == 0x7fffffff || bidx[0] < 0) ? 0 : bi;
        if (st->n_out < out_cap) out_toks[st->n_out] = tok;
        st->n_out = st->n_out + 1;
        st->next = tok;
        st->tok = tok;
        st->pos = st->pos + 1;
    }
}

}  // namespace

// ───────────────────────── host side ─────────────────────────

int pk_decode_reserve(pk_engine *e) {
    if (e->dec_ready) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "decode buffers must exist before capturing a graph");
    const pk_cfg *c = &e->c;
    const int max_chunks = (c->ctx_len + ATT_CHUNK - 1) / ATT_CHUNK;
    PK_TRY(pk_dev_alloc(e, (void **)&e->attn_part, (int64_t)c->n_heads * max_chunks * (c->head_dim + 2) * 4));
    const int lm_blocks = (c->vocab + LM_ROWS_PER_BLOCK - 1) / LM_ROWS_PER_BLOCK;
    PK_TRY(pk_dev_alloc(e, (void **)&e->lm_bval, (int64_t)lm_blocks * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->lm_bidx, (int64_t)lm_blocks * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->dstate, sizeof(pk_dstate)));
    PK_HIP(hipMemsetAsync(e->dstate, 0, sizeof(pk_dstate), e->stream));
    // one pinned staging entry per position: host-set (tok, pos) copies stay
    // valid until the stream reaches them
    PK_HIP(hipHostMalloc((void **)&e->pin_state, (size_t)c->ctx_len * sizeof(pk_dstate), hipHostMallocDefault));
    e->dec_ready = true;
    return PK_OK;
}

int pk_check_model(pk_engine *e) {
    const pk_cfg *c = &e->c;
    PK_CHECK(e->have_globals, PK_ERR_MISSING, "embedding / lm_head / final norm not loaded");
    for (int l = 0; l < c->n_layers; ++l) {
        PK_CHECK(e->L[l].have_attn, PK_ERR_MISSING, "layer %d: attention weights not loaded", l);
        PK_CHECK(e->L[l].have_router, PK_ERR_MISSING, "layer %d: router not loaded", l);
        for (int x = 0; x < c->n_experts; ++x)
            PK_CHECK(e->expert_ready[(int64_t)l * c->n_experts + x], PK_ERR_MISSING,
                     "layer %d expert %d not loaded", l, x);
    }
    PK_CHECK(((c->n_heads + 2 * c->n_kv_heads) * c->head_dim) % 4 == 0 && c->hidden % 4 == 0,
             PK_ERR_UNSUPPORTED, "dimensions must be multiples of 4");
    return PK_OK;
}

extern "C" int pk_kv_layout(int ctx, int KVH, int hd, int64_t *k_off, int64_t n_out) {
    PK_CHECK(ctx > 0 && KVH > 0 && hd > 0 && hd % 4 == 0 && k_off, PK_ERR_ARG, "kv layout: ctx %d KVH %d hd %d", ctx,
             KVH, hd);
    const int64_t n = (int64_t)ctx * KVH * hd;
    PK_CHECK(n_out >= n, PK_ERR_ARG, "kv layout: %lld outputs for %lld values", (long long)n_out, (long long)n);
    for (int pos = 0; pos < ctx; ++pos)
        for (int h = 0; h < KVH; ++h)
            for (int i = 0; i < hd; ++i) k_off[((int64_t)pos * KVH + h) * hd + i] = pk_k_off(pos, h, i, ctx, KVH, hd);
    return PK_OK;
}

// Attention of layer l for n rows of normalised input xn: the decode token
// (st = device state, n = 1), prompt positions pos_base .. pos_base+n-1 of
// one sequence (pos_step 1, seq_step 0), or n sequences at one position
// (pos_step 0, seq_step 1). Writes K/V, qkv [n][(H+2KVH)hd], att [n][H hd]
// and adds the output projection into h [n][D] (residual).
int pk_attention_rows(pk_engine *e, int l, const pk_dstate *st, int pos_base, int pos_step, int seq0,
                      int seq_step, int n, const float *xn, float *qkv, float *part, float *att, float *h,
                      const float *norm_w, bool exact) {
    const pk_cfg *c = &e->c;
    const pk_layer_dev &d = e->L[l];
    const int H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim, D = c->hidden;
    const int kv_dim = KVH * hd, qkv_dim = (H + 2 * KVH) * hd;
    const int64_t kv_row = (int64_t)seq_step * e->seq_stride;
    float *Kl = e->K + seq0 * e->seq_stride + (int64_t)l * c->ctx_len * kv_dim;
    float *Vl = e->V + seq0 * e->seq_stride + (int64_t)l * c->ctx_len * kv_dim;
    const int ps = pk_prof_begin(e, PK_PROF_ATTENTION);
    if (norm_w) {
        // decode row: rmsnorm + QKV + bias + RoPE + KV store in one launch
        PK_CHECK(n == 1 && st, PK_ERR_ARG, "fused norm: the decode row");
        PK_CHECK(((uintptr_t)xn & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && (D & 3) == 0,
                 PK_ERR_UNSUPPORTED, "qkv: needs 16-byte aligned rows");
        const int n_pairs = (H + 2 * KVH) * hd / 2;
        hipLaunchKernelGGL(k_qkv_rope_norm, dim3((n_pairs + 1) / 2), dim3(256), 0, e->stream, st, xn, norm_w,
                           c->eps, d.wqkv, d.bqkv, D, H, KVH, hd, c->ctx_len, e->rope, qkv, Kl, Vl,
                           e->counters + PK_CTR_ATT_EPOCH);
        PK_HIP(hipGetLastError());
    } else {
        // 4..32 rows with the workspace: the split sums + bias go into the RoPE launch
        int splits = 1;
        const bool split_rope = !exact && e->skinny_ws && n >= 4 && n <= 32 && qkv_dim >= 256;
        if (exact)
            PK_TRY(pk_launch_gemm_chain8(xn, D, d.wqkv, d.bqkv, qkv, qkv_dim, n, D, qkv_dim, false, e->stream));
        else if (split_rope)
            PK_TRY(pk_launch_gemm_skinny(qkv, xn, d.wqkv, d.bqkv, n, D, qkv_dim, 0, e->stream, e->skinny_ws,
                                         PK_SKINNY_WS, &splits, pk_tiles_current(e) ? d.wqkv_t : nullptr));
        else
            PK_TRY(pk_launch_gemv_f32(qkv, xn, d.wqkv, d.bqkv, n, D, qkv_dim, e->stream, e->skinny_ws,
                                      e->skinny_ws ? PK_SKINNY_WS : 0, pk_tiles_current(e) ? d.wqkv_t : nullptr));
        const int n_rope = (H + KVH) * (hd / 2) + kv_dim;
        hipLaunchKernelGGL(k_rope_kv, dim3((n_rope + 255) / 256, n), dim3(256), 0, e->stream, st, pos_base,
                           pos_step, qkv, (int64_t)qkv_dim, e->rope, H, KVH, hd, c->ctx_len, Kl, Vl, kv_row,
                           splits > 1 ? e->skinny_ws : nullptr, splits, d.bqkv);
        PK_HIP(hipGetLastError());
    }
    const int sliding = c->layer_type[l] == 0;
    if (exact && !st && pos_step == 1 && seq_step == 0) {
        // prompt rows: softmax with sink and value sums in position order,
        // then the output projection's chains (when the window fits in LDS)
        const int last = pos_base + n - 1;
        int span = (last < c->ctx_len ? last : c->ctx_len - 1) + 1;
        if (sliding && span > c->sliding_window) span = c->sliding_window;
        if (span <= 16384) {
            PK_TRY(pk_launch_attn_rows_exact(pos_base, n, qkv, qkv_dim, Kl, Vl, H, KVH, hd, c->ctx_len, sliding,
                                             c->sliding_window, d.sinks, att, e->stream));
            PK_TRY(pk_launch_gemm_chain8(att, (int64_t)H * hd, d.wo, d.bo, h, D, n, H * hd, D, true, e->stream));
            return pk_prof_end(e, ps);
        }
    }
    const int max_chunks = (c->ctx_len + ATT_CHUNK - 1) / ATT_CHUNK;
    int chunks = st ? (e->att_pos_cap >= 0 ? e->att_pos_cap / ATT_CHUNK + 1 : max_chunks)
                    : (pos_base + (n - 1) * pos_step + ATT_CHUNK) / ATT_CHUNK;
    if (sliding) chunks = std::min(chunks, (c->sliding_window + ATT_CHUNK - 1) / ATT_CHUNK);
    chunks = std::min(chunks, max_chunks);
    const int G = H / KVH;
    PK_CHECK(H % KVH == 0 && G <= 2 * ATT_GH, PK_ERR_UNSUPPORTED, "attention: %d query heads per KV head", G);
    // heads per block: the most that still gives >= 1024 blocks (K/V read once
    // per gs heads), one head per 128-thread block when the grid is small
    int gs = 1;
    while (gs * 2 <= G && G % (gs * 2) == 0 && (int64_t)KVH * (G / (gs * 2)) * chunks * n >= 1024) gs *= 2;
    if (const char *v = getenv("PK_ATT_GS")) {
        const int f = atoi(v);
        if (f >= 1 && f <= G && G % f == 0) gs = f;
    }
    // the decode row with the norm fused into QKV: attention and output
    // projection in one launch (256-thread blocks: two heads per block)
    const bool fuse = norm_w && e->attn_fused && n == 1 && G % 2 == 0 && (H * hd) % 4 == 0 &&
                      H * hd <= 64 * RES_U * 4;
    if (fuse && gs < 2) gs = 2;
    // long windows in the one-launch form: all G heads of a KV head per
    // block (a quarter of the attention blocks ahead of the O-projection
    // blocks, each K/V row read once; config 4 at 4096 positions 383 against
    // 368 tok/s with two heads, 375 with four), two heads below 16 chunks
    if (fuse && chunks >= 16 && !getenv("PK_ATT_GS")) gs = G;
    PK_CHECK((int64_t)n * (H / gs) <= PK_CTR_ATTN_N, PK_ERR_UNSUPPORTED, "attention: %d rows x %d blocks", n,
             H / gs);
    // q, then p [gs][128] shared with the V partials [gs][PG][hd] (PG * hd = 512)
    const size_t att_lds = (size_t)gs * (hd + ATT_CHUNK * 4) * sizeof(float);
    // K / V rows held in registers: 16 float4 up to head_dim 64, else 32
    auto kern = hd <= 64 ? k_attn_part<16> : k_attn_part<32>;
    PK_CHECK(hd % 4 == 0 && hd <= 128, PK_ERR_UNSUPPORTED, "attention: head_dim %d", hd);
    if (fuse) {
        auto kf = hd <= 64 ? k_attn_oproj<16> : k_attn_oproj<32>;
        const int gdx = H / gs;
        const int rows_pb = 4 * ATT_RPW;
        const size_t lds = std::max(att_lds, (size_t)H * hd * sizeof(float));
        hipLaunchKernelGGL(kf, dim3(gdx * chunks + (D + rows_pb - 1) / rows_pb), dim3(ATT_THREADS), lds, e->stream, st, qkv, Kl, Vl,
                           H, KVH, hd, c->ctx_len, sliding, c->sliding_window, part, max_chunks, d.sinks,
                           e->counters + PK_CTR_ATTN, gs, gdx, chunks, e->att_t, e->counters + PK_CTR_ATT_EPOCH,
                           e->counters + PK_CTR_MOE_STATUS, h, d.wo, d.bo, D);
        PK_HIP(hipGetLastError());
        return pk_prof_end(e, ps);
    }
    // one 128-thread half per block while a thread's registers hold the
    // block's heads (both halves of a 256-thread block would read the same
    // K and V rows: batch-32 full-context layers 192 -> 167 us)
    const int thr = gs <= ATT_GH ? ATT_CHUNK : ATT_THREADS;
    hipLaunchKernelGGL(kern, dim3(H / gs, chunks, n), dim3(thr), att_lds,
                       e->stream, st, pos_base, pos_step,
                       qkv, (int64_t)qkv_dim, Kl, Vl, kv_row, H, KVH, hd, c->ctx_len, sliding, c->sliding_window,
                       part, max_chunks, d.sinks, att, e->counters + PK_CTR_ATTN, gs);
    PK_HIP(hipGetLastError());
    if (n >= 4) {
        // several rows: one read of wo per 32 rows
        for (int r0 = 0; r0 < n; r0 += 32)
            PK_TRY(pk_launch_gemm_skinny(h + (int64_t)r0 * D, att + (int64_t)r0 * H * hd, d.wo, d.bo,
                                         n - r0 < 32 ? n - r0 : 32, H * hd, D, 1, e->stream, e->skinny_ws,
                                         e->skinny_ws ? PK_SKINNY_WS : 0, nullptr,
                                         pk_tiles_current(e) ? d.wo_t : nullptr));
    } else {
        hipLaunchKernelGGL(k_gemv_res, dim3((D + 3) / 4, n), dim3(256), 0, e->stream, h, att, d.wo, d.bo,
                           H * hd, D);
        PK_HIP(hipGetLastError());
    }
    return pk_prof_end(e, ps);
}

// Sets the decode attention's position bound for one scope.
struct att_cap_scope {
    pk_engine *e;
    int old;
    att_cap_scope(pk_engine *eng, int cap) : e(eng), old(eng->att_pos_cap) { e->att_pos_cap = cap; }
    ~att_cap_scope() { e->att_pos_cap = old; }
};

// Decode attention of layer l on the residual row h (in_ln rmsnorm fused
// into the QKV GEMV); adds the output projection into h.
static int attention_layer(pk_engine *e, int l) {
    return pk_attention_rows(e, l, e->dstate, 0, 0, 0, 0, 1, e->h, e->qkv, e->attn_part, e->att, e->h,
                             e->L[l].in_ln);
}

// One forward_token step with tok/pos in device state; logits optional.
static int decode_step(pk_engine *e, float *logits_dev, int32_t *out_toks, int out_cap) {
    const pk_cfg *c = &e->c;
    const int D = c->hidden;
    hipLaunchKernelGGL(k_embed_rmsnorm, dim3(1), dim3(256), 0, e->stream, e->dstate, e->embed, c->vocab,
                       e->h, e->hn, e->L[0].in_ln, D, c->eps);
    PK_HIP(hipGetLastError());
    PK_TRY(pk_trace_vec(e, "embedding", -1, e->h, D));
    for (int l = 0; l < c->n_layers; ++l) {
        PK_TRY(attention_layer(e, l));
        PK_TRY(pk_trace_vec(e, "post_attention", l, e->h, D));
        // h += moe(rmsnorm(h)): the router normalises h and writes hn for the experts
        PK_TRY(pk_moe_layer(e, l, e->h, nullptr, e->h, e->h, e->L[l].post_ln));
        PK_TRY(pk_trace_vec(e, "post_moe", l, e->h, D));
    }
    PK_TRY(pk_launch_rmsnorm(e->hn, e->h, e->final_norm, D, c->eps, 1, e->stream));
    PK_TRY(pk_lm_head_step(e, e->hn, logits_dev, out_toks, out_cap));
    return pk_trace_top_logits(e, logits_dev ? logits_dev : e->logits);
}

// lm_head GEMV + greedy argmax of the normalised state hn for the token at
// dstate->pos: writes next/tok, advances pos, appends to out_toks.
int pk_lm_head_step(pk_engine *e, const float *hn, float *logits_dev, int32_t *out_toks, int out_cap) {
    const pk_cfg *c = &e->c;
    const int D = c->hidden;
    const int lm_blocks = (c->vocab + LM_ROWS_PER_BLOCK - 1) / LM_ROWS_PER_BLOCK;
    float *lg = logits_dev ? logits_dev : e->logits;
    const int ps = pk_prof_begin(e, PK_PROF_LM_HEAD);
    if (c->lm_head_fmt == PK_FMT_INT8)
        hipLaunchKernelGGL(k_lm_head<true>, dim3(lm_blocks), dim3(256), 0, e->stream, hn,
                           (const void *)e->lm_q8, e->lm_s, D, c->vocab, lg, e->lm_bval, e->lm_bidx);
    else
        hipLaunchKernelGGL(k_lm_head<false>, dim3(lm_blocks), dim3(256), 0, e->stream, hn,
                           (const void *)e->lm_f32, nullptr, D, c->vocab, lg, e->lm_bval, e->lm_bidx);
    PK_HIP(hipGetLastError());
    if (e->samp_on) {
        // sample_logits on the logits (picchio.c:1750): the draw updates the decode state
        PK_TRY(pk_launch_sample(e, lg, c->vocab, e->dstate, out_toks, out_cap, e->lm_bval, lm_blocks,
                                logits_dev != nullptr));
    } else {
        hipLaunchKernelGGL(k_argmax_blocks, dim3(1), dim3(1024), 0, e->stream, e->lm_bval, e->lm_bidx, lm_blocks,
                           e->dstate, out_toks, out_cap);
        PK_HIP(hipGetLastError());
    }
    return pk_prof_end(e, ps);
}

// tok / pos (and n_out = 0) for position pos through its pinned staging slot
int pk_set_state(pk_engine *e, int tok, int pos) {
    pk_dstate &s = e->pin_state[pos];
    s.tok = tok;
    s.pos = pos;
    s.n_out = 0;
    s.next = 0;
    PK_HIP(hipMemcpyAsync(e->dstate, &s, sizeof(s), hipMemcpyHostToDevice, e->stream));
    return PK_OK;
}

extern "C" int pk_gqa_attention(pk_engine *e, int layer, const float *x_dev, int pos, float *out_dev) {
    PK_CHECK(e && x_dev && out_dev, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    PK_CHECK(layer >= 0 && layer < c->n_layers, PK_ERR_ARG, "layer %d out of range", layer);
    PK_CHECK(e->L[layer].have_attn, PK_ERR_MISSING, "layer %d: attention weights not loaded", layer);
    PK_CHECK(pos >= 0, PK_ERR_ARG, "pos %d", pos);
    PK_CHECK(pos < c->ctx_len, PK_ERR_CONTEXT_FULL, "pos %d >= context %d", pos, c->ctx_len);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "gqa_attention: host position; not available while capturing");
    PK_TRY(pk_decode_reserve(e));
    PK_TRY(pk_set_state(e, 0, pos));
    PK_HIP(hipMemcpyAsync(e->hn, x_dev, (size_t)c->hidden * 4, hipMemcpyDeviceToDevice, e->stream));
    PK_HIP(hipMemsetAsync(e->h, 0, (size_t)c->hidden * 4, e->stream));
    att_cap_scope cap(e, pos);
    PK_TRY(pk_attention_rows(e, layer, e->dstate, 0, 0, 0, 0, 1, e->hn, e->qkv, e->attn_part, e->att,
                             e->h));                // h = 0 + attn(x)
    PK_HIP(hipMemcpyAsync(out_dev, e->h, (size_t)c->hidden * 4, hipMemcpyDeviceToDevice, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

extern "C" int pk_forward_token(pk_engine *e, int tok, int pos, int32_t *next_host, float *logits_dev) {
    PK_CHECK(e, PK_ERR_ARG, "engine is null");
    PK_CHECK(pos >= 0, PK_ERR_ARG, "pos %d", pos);
    PK_CHECK(pos < e->c.ctx_len, PK_ERR_CONTEXT_FULL, "pos %d >= context %d", pos, e->c.ctx_len);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "forward_token: use pk_generate inside graphs");
    PK_TRY(pk_check_model(e));
    PK_TRY(pk_decode_reserve(e));
    PK_TRY(pk_set_state(e, tok, pos));
    att_cap_scope cap(e, pos);
    PK_TRY(decode_step(e, logits_dev, nullptr, 0));
    if (next_host) {
        pk_dstate s{};
        PK_HIP(hipMemcpyAsync(&s, e->dstate, sizeof(s), hipMemcpyDeviceToHost, e->stream));
        PK_HIP(hipStreamSynchronize(e->stream));
        bool redo = false;
        PK_TRY(pk_wait_fallback(e, &redo));
        if (redo) return pk_forward_token(e, tok, pos, next_host, logits_dev);   // rewrites this position's K/V
        *next_host = s.next;
    }
    return PK_OK;
}

int pk_decode_token(pk_engine *e, int tok, int pos, int32_t *out_toks, int out_cap) {
    PK_TRY(pk_set_state(e, tok, pos));
    att_cap_scope cap(e, e->capturing ? e->att_pos_cap : pos);
    return decode_step(e, nullptr, out_toks, out_cap);
}

// Greedy generation as picchio runs a turn: the prompt through prefill_tokens
// (batched chunks, picchio.c:1936-1975), then n_steps - 1 forward_token steps
// replayed from one captured step graph that feeds itself (tok = last argmax,
// pos += 1). out[0] is the prompt's next token.
extern "C" int pk_generate(pk_engine *e, const int32_t *prompt, int n_prompt, int n_steps, int32_t *out) {
    PK_CHECK(e && prompt && out && n_prompt > 0 && n_steps >= 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(n_prompt + n_steps <= e->c.ctx_len, PK_ERR_CONTEXT_FULL,
             "%d prompt + %d steps exceed context %d", n_prompt, n_steps, e->c.ctx_len);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "generate: not available while capturing");
    PK_TRY(pk_check_model(e));
    PK_TRY(pk_decode_reserve(e));
    if (n_steps == 0) return PK_OK;
    int32_t *out_dev = nullptr;
    PK_TRY(pk_dev_alloc(e, (void **)&out_dev, (int64_t)n_steps * 4));
    int rc = PK_OK;
    bool redo = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    do {
        if (n_steps > 1) {
            if (hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
                rc = PK_ERR_HIP; break;
            }
            e->capturing = true;
            {
                // the replays reach positions n_prompt .. n_prompt + n_steps - 2
                att_cap_scope cap(e, n_prompt + n_steps - 1);
                rc = decode_step(e, nullptr, out_dev, n_steps);
            }
            e->capturing = false;
            hipError_t hr = hipStreamEndCapture(e->stream, &graph);
            if (rc != PK_OK) break;
            if (hr != hipSuccess || hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
                pk_set_error("generate: graph capture failed"); rc = PK_ERR_HIP; break;
            }
        }
        if ((rc = pk_prefill_run(e, 0, prompt, n_prompt, 0, out_dev, n_steps)) != PK_OK) break;
        for (int i = 0; i < n_steps - 1 && rc == PK_OK; ++i)
            if (hipGraphLaunch(exec, e->stream) != hipSuccess) { pk_set_error("generate: launch failed"); rc = PK_ERR_HIP; }
        if (rc != PK_OK) break;
        if (hipMemcpyAsync(out, out_dev, (size_t)n_steps * 4, hipMemcpyDeviceToHost, e->stream) != hipSuccess ||
            hipStreamSynchronize(e->stream) != hipSuccess) { rc = PK_ERR_HIP; break; }
        rc = pk_wait_fallback(e, &redo);
    } while (0);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipStreamSynchronize(e->stream);
    pk_dev_free(e, out_dev);
    e->device_bytes -= (int64_t)n_steps * 4;
    // the prompt's prefill rewrites every position the failed run wrote
    if (rc == PK_OK && redo) return pk_generate(e, prompt, n_prompt, n_steps, out);
    return rc;
}

// Timed decode: n_steps replays of the step graph from (tok, pos); the
// caller brackets the call with events. Returns tokens into out (host).
extern "C" int pk_decode_replay(pk_engine *e, int tok, int pos, int n_steps, int32_t *out) {
    PK_CHECK(e && out && n_steps > 0, PK_ERR_ARG, "bad argument");
    PK_CHECK(pos + n_steps <= e->c.ctx_len, PK_ERR_CONTEXT_FULL, "positions exceed context");
    PK_TRY(pk_check_model(e));
    PK_TRY(pk_decode_reserve(e));
    // The graph's attention grids cover positions 0..step_cap: captured
    // again, with the bound doubled, when a call goes past it
    const int need = pos + n_steps - 1;
    if (e->step_exec && need > e->step_cap) {
        PK_HIP(hipStreamSynchronize(e->stream));
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    if (!e->step_exec) {
        if (!e->step_out) {
            int32_t *od = nullptr;
            PK_TRY(pk_dev_alloc(e, (void **)&od, (int64_t)e->c.ctx_len * 4));
            e->step_out = od;
        }
        int64_t bound = 1024;
        while (bound <= need) bound *= 2;
        const int cap = (int)std::min<int64_t>(bound, e->c.ctx_len) - 1;
        hipGraph_t g = nullptr;
        PK_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
        e->capturing = true;
        int rc;
        {
            att_cap_scope scope(e, cap);
            rc = decode_step(e, nullptr, e->step_out, e->c.ctx_len);
        }
        e->capturing = false;
        hipError_t hr = hipStreamEndCapture(e->stream, &g);
        if (rc == PK_OK && hr == hipSuccess) hr = hipGraphInstantiate(&e->step_exec, g, nullptr, nullptr, 0);
        if (g) (void)hipGraphDestroy(g);            // every exit path after the capture
        PK_TRY(rc);
        if (hr != hipSuccess) {
            e->step_exec = nullptr;
            e->step_cap = -1;
            pk_set_error("decode step capture failed: %s", hipGetErrorString(hr));
            return PK_ERR_HIP;
        }
        e->step_cap = cap;
    }
    PK_TRY(pk_set_state(e, tok, pos));
    for (int i = 0; i < n_steps; ++i) PK_HIP(hipGraphLaunch(e->step_exec, e->stream));
    PK_HIP(hipMemcpyAsync(out, e->step_out, (size_t)n_steps * 4, hipMemcpyDeviceToHost, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    bool redo = false;
    PK_TRY(pk_wait_fallback(e, &redo));
    // from (tok, pos) again: every step rewrites its own position's K/V rows
    return redo ? pk_decode_replay(e, tok, pos, n_steps, out) : PK_OK;
}
