// pk_internal.h — shared definitions of the gfx950 expert-path library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/picchio_hip.h"

// Native vector types for non-temporal (streaming) 16-byte loads.
typedef float pk_f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t pk_i32x4 __attribute__((ext_vector_type(4)));

// K cache layout of one (sequence, layer) region: ctx positions x KVH * hd
// floats, the size of position-major rows. Positions go in chunks of 128
// (the last one ctx % 128 long); inside a chunk, KV head by KV head, then
// the head's float4 column u, then the chunk's positions. A position's
// float4 u sits next to its neighbours', so the attention's row reads (one
// lane per position, float4 u at a time) are contiguous across a wave.
constexpr int PK_K_CHUNK = 128;
// Positions in pos's chunk: the float4 stride between a position's columns.
__host__ __device__ inline int pk_k_cs(int pos, int ctx) {
    const int b = pos & ~(PK_K_CHUNK - 1);
    return ctx - b < PK_K_CHUNK ? ctx - b : PK_K_CHUNK;
}
// Offset in floats of element i (< hd) of KV head kvh at position pos (< ctx).
__host__ __device__ inline int64_t pk_k_off(int pos, int kvh, int i, int ctx, int KVH, int hd) {
    const int b = pos & ~(PK_K_CHUNK - 1), p = pos - b;
    return (int64_t)b * KVH * hd + ((int64_t)(kvh * (hd >> 2) + (i >> 2)) * pk_k_cs(pos, ctx) + p) * 4 + (i & 3);
}

// ───────────────────────── error plumbing ─────────────────────────
void pk_set_error(const char *fmt, ...);

#define PK_HIP(call)                                                          \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) {                                               \
            pk_set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), \
                         __FILE__, __LINE__);                                 \
            return PK_ERR_HIP;                                                \
        }                                                                     \
    } while (0)

#define PK_CHECK(cond, code, ...)                                             \
    do {                                                                      \
        if (!(cond)) {                                                        \
            pk_set_error(__VA_ARGS__);                                        \
            return (code);                                                    \
        }                                                                     \
    } while (0)

#define PK_TRY(expr)                                                          \
    do {                                                                      \
        int rc_ = (expr);                                                     \
        if (rc_ != PK_OK) return rc_;                                         \
    } while (0)

// ───────────────────── INT4 group-scaled HBM layout ─────────────────────
//
// The reference keeps an INT4 gs64 matrix row-major: uint8 [O][I/2] (low
// nibble = even column, value = nib - 8) and float scales [O][I/64]
// (convert.py:84-93). In HBM the library stores it as 64-row x 64-column
// tiles so that one wavefront load instruction reads 1 KiB contiguous:
//
//   tile (rb, g), rb = row block of 64 rows, g = 64-column scale group:
//     bytes [0, 1024):    lane r's 16 bytes = row rb*64+r, columns g*64 +  0..31
//     bytes [1024, 2048): lane r's 16 bytes = row rb*64+r, columns g*64 + 32..63
//   tiles ordered [rb][g]; every nibble is stored XOR 8, i.e. as the 4-bit
//   two's complement of (nib - 8), which v_cvt_off_f32_i4 reads as q/16.
//   scales: float [rb][g][64], each stored as 16 * scale (exact), so that
//   (partial sum of x*q/16) * (16*scale) == (partial sum of x*q) * scale.
//
// Rows beyond O are zero-padded (q = 0, scale = 0).
constexpr int PK_TILE_ROWS = 64;
constexpr int PK_GS = 64;
constexpr int PK_TILE_BYTES = PK_TILE_ROWS * PK_GS / 2;   // 2048

struct pk_i4_shape {
    int O, I;        // logical shape
    int RB, NG;      // row blocks of 64, groups of 64
    int64_t tile_bytes;   // RB*NG*2048
    int64_t scale_bytes;  // RB*NG*64*4
};

inline pk_i4_shape pk_i4_make_shape(int O, int I) {
    pk_i4_shape s;
    s.O = O; s.I = I;
    s.RB = (O + PK_TILE_ROWS - 1) / PK_TILE_ROWS;
    s.NG = I / PK_GS;
    s.tile_bytes = (int64_t)s.RB * s.NG * PK_TILE_BYTES;
    s.scale_bytes = (int64_t)s.RB * s.NG * PK_TILE_ROWS * 4;
    return s;
}

inline int64_t pk_align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// Expert slot layout inside the store (all experts of a model share it).
struct pk_expert_layout {
    pk_i4_shape gu, dn;          // gate_up [moe_inter][hidden], down [hidden][moe_inter/2]
    int64_t off_gu_tiles, off_gu_scales, off_dn_tiles, off_dn_scales;
    int64_t off_gu_bias, off_dn_bias;
    int64_t stride;              // bytes per expert slot
};

// ───────────────────────── device tensors ─────────────────────────
struct pk_qt {
    int fmt;           // PK_FMT_*
    int O, I;
    int gs;            // INT4 group size (0 = per-row)
    int tiled;         // INT4 gs64 in the tiled layout
    pk_i4_shape sh;
    void *data;        // F32 [O][I] / INT8 [O][I] / INT4 tiles or ref layout
    float *s;          // scales (INT8 per row, INT4 ref or tiled)
};

// ───────────────────────── kernel launchers ─────────────────────────
// All launchers queue on `st` and return PK_OK / PK_ERR_*.

// One INT4 GEMV "item" = one matrix applied to one input vector.
struct pk_i4_items {
    const uint8_t *base;       // store base (or matrix base when slots == null)
    int64_t slot_stride;       // bytes between expert slots
    int64_t off_tiles, off_scales, off_bias;  // offsets inside a slot (bias < 0: none)
    const int32_t *slots;      // [n_items] slot index (device), or null -> slot 0
    int32_t slot_base;         // added to every slot index (layer * n_experts)
    const float *x;            // input of item i at x + (i / x_div) * x_stride
    int64_t x_stride;
    int x_div = 1;             // items sharing one input row (token-major item lists)
    float *y;                  // output of item i at y + i * y_stride
    int64_t y_stride;
    int n_items;
    // integer-dot arithmetic (pk_dot_group): input half-group records of item i
    // at xq + (i / x_div) * xq_stride (ints); with xq set the launch runs on them
    const int32_t *xq = nullptr;
    int64_t xq_stride = 0;
    // SwiGLU epilogue: also the output's records, item i at yq + i * yq_stride
    // (one per 64-row block)
    int32_t *yq = nullptr;
    int64_t yq_stride = 0;
};

// ints per half-group record of the integer-dot expert arithmetic
// (pk_i4_device.h: five digit planes of 4 dwords, the exponent, padding)
constexpr int PK_XQ_INTS = 24;

enum pk_i4_epilogue { PK_EPI_PLAIN = 0, PK_EPI_SWIGLU = 1, PK_EPI_COMBINE = 2 };

struct pk_combine_args {
    const float *w;           // [n_items] routing weights (already * routed_scale), device
    float *out;               // [O] combined output
    const float *residual;    // optional: out = residual + combine
    uint32_t *counters;       // [RB] zero-initialised arrival counters (re-armed after use)
};

// Routing of one token selected inside an expert launch (see
// pk_launch_i4_gemv's route argument).
struct pk_route_args {
    const float *logits;      // [E] router logits (+ bias) of the token
    int E, K;
    float routed_scale;
    int32_t *sel;             // [K] outputs, written by one workgroup
    float *w_scaled, *w_soft; // [K] (w_soft optional)
};

// route (optional): the items are rounds 0..n_items-1 of the top-k of the
// router logits in route->logits, selected in the kernel; one workgroup
// writes route->sel / w_scaled / w_soft for the launches that follow.
int pk_launch_i4_gemv(const pk_i4_items &it, const pk_i4_shape &sh, int epilogue,
                      float swiglu_limit, float swiglu_alpha,
                      const pk_combine_args *comb, hipStream_t st,
                      const pk_route_args *route = nullptr);

// A token's routed experts in one launch (k_moe_ffn): gate_up + SwiGLU,
// down + combine, experts selected from rt.logits in the launch. Kept lean:
// every field a kernel argument reads stays in scalar registers.
struct pk_moe_ffn_args {
    const uint8_t *store;          // expert slots: slot (slot_base + e) at store + slot * slot_stride
    int64_t slot_stride;
    int slot_base;
    uint32_t gu_tiles, gu_scales, dn_tiles, dn_scales;   // byte offsets inside a slot
    int32_t gu_bias, dn_bias;      // byte offsets inside a slot, -1: no bias
    int gu_NG, gu_O, gu_RB;        // gate_up: O rows in RB row blocks of 64, NG groups of 64 columns
    int dn_NG, dn_O, dn_RB;        // down: its input is the gu_O / 2 = gu_RB * 32 activations
    int K;                         // routed experts (items)
    int n_cu;                      // compute units (placement of the down tasks)
    bool dot;                      // integer-dot arithmetic (xq) or picchio's fp32 chains (x)
    float lim, alpha;
    const float *x;                // input row (fp32 chains)
    const int32_t *xq;             // its half-group records (integer dot)
    float *out;                    // combined rows (+ residual)
    const float *residual;         // optional
    pk_route_args rt;
    // hand-over words (tag << 32 | bits), zero-initialised:
    uint64_t *act_t;               // [K][dot ? gu_RB * PK_XQ_INTS : gu_O / 2]
    uint64_t *eo_t;                // [K][dn_O]
    uint64_t *cont_t;              // k_moe_bal: [K x (gu_RB + dn_RB)][64] split row blocks' accumulators
    const uint32_t *epoch;         // the tag: advanced before each launch (router), never 0
    uint32_t *status;              // set to 1 if a wait gave up
};
int pk_launch_moe_ffn(const pk_moe_ffn_args &a, hipStream_t st);
// The same work with every CU streaming the same bytes (k_moe_bal, grid =
// a.n_cu workgroups, one per CU; pk_moe.hip). Supported: shape and CU count
// (the ranges) and one workgroup per CU fitting the kernel's resources.
int pk_launch_moe_bal(const pk_moe_ffn_args &a, hipStream_t st);
bool pk_moe_bal_supported(const pk_moe_ffn_args &a, int W);
bool pk_moe_bal_fits_cu(bool dot);
// Whether the one-launch experts can run on this device: every down task
// waits, so the down tasks must stay below the workgroups the device holds at
// once (n_cu x the kernel's occupancy per CU) — else the launcher refuses
// and the caller runs the two-launch form.
bool pk_moe_ffn_supported(int gu_RB, int dn_RB, int K, int n_cu, bool dot);

// The down task of k_moe_ffn's workgroup `task` (grid workgroups, n_cu CUs):
// the first down tasks go to the workgroups that have a CU to themselves
// (with grid <= 2 n_cu, workgroups n_cu.. share the CUs of workgroups 0..);
// with grid > 2 n_cu no workgroup is alone and the mapping is the identity.
// A permutation of [0, grid) for every n_cu >= 1.
__host__ __device__ inline int pk_moe_down_task(int task, int grid, int n_cu) {
    const int n2 = grid > n_cu ? grid - n_cu : 0;     // workgroups sharing a CU with a later one
    if (n2 >= n_cu) return task;
    if (task >= n2 && task < n_cu) return task - n2;
    if (task < n2) return n_cu - n2 + task;
    return task;
}

// Pairs grouped by expert into tiles (k_group_pairs): tile t = expert
// tile_exp[t], pairs[tile_beg[t] .. + tile_cnt[t]]; *n_tiles tiles (device).
struct pk_i4_tiles {
    const int32_t *pairs, *tile_exp, *tile_beg, *tile_cnt, *n_tiles;
};
// Integer-dot GEMV of every pair of every tile (at most 4 pairs per tile),
// each expert block loaded once per tile; outputs pair-indexed.
int pk_launch_i4_dot_tiles(const pk_i4_items &it, const pk_i4_tiles &tl, const pk_i4_shape &sh, int epilogue,
                           float lim, float alpha, int max_tiles, hipStream_t st);

// Half-group records (integer-dot arithmetic) of x[0..n), n % 32 == 0.
int pk_launch_act_records(const float *x, int n, int32_t *rec, hipStream_t st);

// Reference-layout INT4 gs GEMV, any I / group size (exact quant.h order).
int pk_launch_i4_gemv_ref(float *y, const float *x, const uint8_t *q4, const float *s,
                          int S, int I, int O, int gs, hipStream_t st);

int pk_launch_i4_repack(const uint8_t *q4, const float *s, int O, int I,
                        uint8_t *tiles, float *sc16, hipStream_t st);

int pk_launch_quantize_i4(const float *w, int O, int I, int gs, uint8_t *packed,
                          float *scales, hipStream_t st);

// ws / ws_floats (optional): workspace that lets the skinny GEMM split K
// (partial tiles [splits][32][O]); without it every row block takes all of K
// Wt (optional): W's copy in the skinny GEMM's tile order (pk_launch_tile_skinny), read instead of W
int pk_launch_gemv_f32(float *y, const float *x, const float *W, const float *bias,
                       int S, int I, int O, hipStream_t st, float *ws = nullptr, int64_t ws_floats = 0,
                       const float *Wt = nullptr);
// Y[s][o] = (residual ? Y[s][o] : 0) + X[s].W[o] + bias[o] for up to 32 inputs, one read of W.
// splits_out (optional): when K is split, the partial tiles stay in ws
// ([splits][32][O]) for the caller to add (*splits_out = splits, the sums
// and bias / residual not applied); 1 when y holds the result.
int pk_launch_gemm_skinny(float *y, const float *x, const float *W, const float *bias, int S, int I, int O,
                          int residual, hipStream_t st, float *ws = nullptr, int64_t ws_floats = 0,
                          int *splits_out = nullptr, const float *Wt = nullptr);
// W [O][I] (I % 4 == 0) copied into the skinny GEMM's tile order: a tile per
// 16 rows and 32 columns, 512 floats, holding what each lane of the wave
// that multiplies those rows reads at that column step, as two 1 KB halves
// (the lane's first, then its second four columns), so that every weight
// load of the GEMM is one contiguous kilobyte. Rows past O repeat row O - 1,
// columns past I are zero. Floats of the copy:
int64_t pk_skinny_tile_floats(int O, int I);
int pk_launch_tile_skinny(const float *W, int O, int I, float *Wt, hipStream_t st);
int pk_launch_gemv_q8(float *y, const float *x, const int8_t *q, const float *s,
                      int S, int I, int O, hipStream_t st);
int pk_launch_i4_rowscale_gemv(float *y, const float *x, const uint8_t *q4, const float *s,
                               int S, int I, int O, hipStream_t st);

// Router for one token: logits = R x + b, top-k by repeated argmax, softmax.
// nw (optional): x is the raw residual row, normalised in the kernel
// (rmsnorm fused); the normalised row is also written to hn.
// epoch (optional): incremented by one thread (k_moe_ffn's hand-over tag).
int pk_launch_router_topk(const float *x, const float *R, const float *b, int E, int D,
                          int K, float routed_scale, float *logits, int32_t *sel,
                          float *w_scaled, float *w_soft, uint32_t *counter,
                          hipStream_t st, const float *nw = nullptr, float eps = 0.f,
                          float *hn = nullptr, int32_t *hq = nullptr, uint32_t *epoch = nullptr);
// y = W . rmsnorm(h; nw, eps) + bias for one row (rmsnorm fused into the GEMV).
int pk_launch_gemv_f32_norm(float *y, const float *h, const float *nw, float eps, const float *W,
                            const float *bias, int I, int O, hipStream_t st);

int pk_launch_rmsnorm(float *out, const float *x, const float *w, int D, float eps,
                      int T, hipStream_t st);
