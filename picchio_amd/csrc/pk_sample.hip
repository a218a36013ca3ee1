// pk_sample.hip — next-token sampling on the device (sample_logits,
// picchio.c:1509-1649), so that a decode loop with temperature / top-k /
// top-p / repetition penalty never leaves the GPU.
//
// One workgroup of 1024 threads per draw. For a pass over the vocabulary
// wave w owns the w-th sixteenth, with 16 loads in flight per lane. Steps,
// in the reference's order:
//   1. repetition penalty: once per history entry (a token that appears c
//      times is divided / multiplied c times, as the reference's loop does);
//   2. temperature below 1e-6: the first maximum (greedy), no draw;
//   3. logits * (1 / T);
//   4. top-k threshold = the K-th largest value, by a radix select on
//      order-preserving keys (exact; ties at the threshold stay). After the
//      first 8-bit pass the entries in or above the threshold's bucket are
//      gathered into LDS when they fit, and the rest of the selection and the
//      index order of the kept entries are worked out there; otherwise the
//      passes stay in global memory and a ballot compaction keeps index order;
//   5. softmax, top-p over the probabilities > 1e-10, the draw.
// A logit below the top-k threshold becomes -1e30 and then exactly 0 in the
// reference, so its float sums equal the same sums over the kept entries in
// index order, one term at a time. Every sum here is made in that order by
// one lane: from LDS when at most SMALL entries are kept (every top-k up to
// 4096), else from global memory staged through LDS by the other waves. The
// top-p list is sorted descending with equal values by index (what glibc's
// merge sort leaves): in LDS for up to SMALL entries, beyond that chunk by
// chunk (a radix select on 64-bit (key, ~index) finds each chunk's bound) with
// the running sum carried across. The array left behind and the draw equal
// the reference's up to the device expf's last ulp.
// A serial sum over a 200k vocabulary costs about half a millisecond; the
// opt-in fast_sums mode makes those sums exact instead (64-bit integers of
// the values scaled by a power of two, rounded once), which any order gives:
// the top-p cut is the shortest descending prefix whose exact sum reaches
// top_p (a radix descent carrying counts and exact sums, ties by index) and
// the pick the first index whose exact running sum reaches the draw. The
// reference's float rounding (about sqrt(n) * 2^-24 relative) then separates
// the two, so over a flat distribution a cut or a pick moves now and then.
#include "pk_engine.h"

#include <cstddef>

namespace {

constexpr int SNT = 1024;                 // threads of the sampling workgroup
constexpr int NW = SNT / 64;              // its waves
constexpr int U = 16;                     // loads in flight per lane in a pass
constexpr int SMALL = 4096;               // kept entries handled in LDS in the reference's order
constexpr int CAND = 4096;                // top-k candidates gathered into LDS after the first radix pass
constexpr int FX_P = 62;                  // fixed-point bits for probabilities (sums <= ~1)

__device__ __forceinline__ uint32_t key_of(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float float_of(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// v * 2^S truncated to an integer, for 0 <= v with v * 2^S < 2^64 (exact
// whenever v >= 2^(23 - S)); zero, denormals and negatives give 0.
__device__ __forceinline__ uint64_t fx(float v, int S) {
    const uint32_t b = __float_as_uint(v);
    const int e = (int)(b >> 23) & 255;
    if (e == 0 || (b >> 31)) return 0;
    const uint64_t m = (b & 0x7fffffu) | 0x800000u;
    const int sh = e - 150 + S;
    if (sh >= 0) return m << sh;
    return sh <= -24 ? 0 : m >> (-sh);
}
// an exact integer sum back to float: one rounding, then the exact scaling
__device__ __forceinline__ float unfx(uint64_t q, int S) { return ldexpf((float)q, -S); }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int d) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, d, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), d, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
    const int lane = threadIdx.x & 63;
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t t = shfl_up_u64(v, d);
        if (lane >= d) v += t;
    }
    return v;
}
// Every thread of the workgroup calls these.
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t *s_q) {
    v = wave_sum_u64(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_q[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < NW; ++w) t += s_q[w];
    return t;
}
// The same network ordering by index ascending (values carried along).
__device__ __forceinline__ void bitonic_by_index(float *sv, int *si, int P) {
    const int half = P >> 1;
    for (int size = 2; size <= P; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < half; t += SNT) {
                const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
                const int ia = si[lo], ib = si[hi];
                const bool rev = (lo & size) != 0;
                if ((ia < ib) == rev) {
                    const float va = sv[lo];
                    sv[lo] = sv[hi]; sv[hi] = va;
                    si[lo] = ib; si[hi] = ia;
                }
            }
            __syncthreads();
        }
}

__device__ __forceinline__ float block_max(float v, float *s_red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = s_red[0];
    for (int w = 1; w < NW; ++w) m = fmaxf(m, s_red[w]);
    return m;
}
__device__ __forceinline__ int block_max_i(int v, int *s_redi) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_redi[threadIdx.x >> 6] = v;
    __syncthreads();
    int m = s_redi[0];
    for (int w = 1; w < NW; ++w) m = max(m, s_redi[w]);
    return m;
}

// This wave's share [b, e) of [0, n): 16 contiguous shares, multiples of 64.
struct seg_t { int b, e; };
__device__ __forceinline__ seg_t wave_seg(int n) {
    const int per = ((n + NW - 1) / NW + 63) & ~63;
    const int b = min(n, (int)(threadIdx.x >> 6) * per);
    return {b, min(n, b + per)};
}

// f(j, v, ok) for every j of this wave's share of src[0..n): 64-entry steps,
// U steps' loads issued before any is used (clamped, so every load is valid).
template <class F>
__device__ __forceinline__ void seg_for(const float *src, int n, F f) {
    const seg_t s = wave_seg(n);
    const int lane = threadIdx.x & 63;
    for (int base = s.b; base < s.e; base += 64 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = src[min(base + u * 64 + lane, n - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = base + u * 64 + lane;
            f(j, v[u], j < s.e);
        }
    }
}

// Entries of src[0..n) with keep(v), in index order, into dv / di as
// (map(v), j). Returns their number. Every thread of the workgroup calls it.
template <class Keep, class Map>
__device__ __forceinline__ int compact(const float *src, int n, Keep keep, Map map, float *dv, int *di, int *s_w) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int c = 0;
    seg_for(src, n, [&](int, float v, bool ok) { c += __popcll(__ballot(ok && keep(v))); });
    __syncthreads();
    if (lane == 0) s_w[wave] = c;
    __syncthreads();
    int off = 0, tot = 0;
    for (int w = 0; w < NW; ++w) {
        const int x = s_w[w];
        off += w < wave ? x : 0;
        tot += x;
    }
    const uint64_t lt = (1ull << lane) - 1ull;
    seg_for(src, n, [&](int j, float v, bool ok) {
        const bool p = ok && keep(v);
        const uint64_t m = __ballot(p);
        if (p) {
            const int o = off + __popcll(m & lt);
            dv[o] = map(v);
            di[o] = j;
        }
        off += __popcll(m);
    });
    __syncthreads();
    return tot;
}

// Bitonic network over LDS (sv, si)[0..P), P a power of two <= SMALL:
// value descending, then index ascending.
__device__ __forceinline__ void bitonic(float *sv, int *si, int P) {
    const int half = P >> 1;
    for (int size = 2; size <= P; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < half; t += SNT) {
                const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
                const float va = sv[lo], vb = sv[hi];
                const int ia = si[lo], ib = si[hi];
                const bool rev = (lo & size) != 0;     // second half of a merge runs backwards
                const bool a_first = va > vb || (va == vb && ia < ib);
                if (a_first == rev) {
                    sv[lo] = vb; sv[hi] = va;
                    si[lo] = ib; si[hi] = ia;
                }
            }
            __syncthreads();
        }
}

// Step 5 over kv / ki[0..n) in LDS (n <= SMALL), in the reference's order.
// Returns (to thread 0) the position picked, or -1; *r_out the draw.
__device__ __forceinline__ int finish_small(float *kv, int n, float top_p, pk_sampler_dev *sp, float *sv, int *si,
                            float *s_red, int *s_redi, float *s_sum, int *s_cut, float *r_out) {
    const int tid = threadIdx.x;
    float mx = -1e30f;
    for (int j = tid; j < n; j += SNT) mx = fmaxf(mx, kv[j]);
    mx = block_max(mx, s_red);
    for (int j = tid; j < n; j += SNT) kv[j] = expf(kv[j] - mx);
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        for (int j = 0; j < n; ++j) s = s + kv[j];
        *s_sum = s;
    }
    __syncthreads();
    const float sum = *s_sum;
    for (int j = tid; j < n; j += SNT) kv[j] = kv[j] / sum;
    __syncthreads();
    if (top_p < 1.0f && top_p > 0.0f) {
        int c = 0;
        for (int j = tid; j < n; j += SNT) c += kv[j] > 1e-10f ? 1 : 0;
        // the candidates' count: a block sum of c
        for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
        __syncthreads();
        if ((tid & 63) == 0) s_redi[tid >> 6] = c;
        __syncthreads();
        int na = 0;
        for (int w = 0; w < NW; ++w) na += s_redi[w];
        if (na > 1) {
            // sorting every entry puts the candidates (> 1e-10) first, in order
            int P = 1;
            while (P < n) P <<= 1;
            for (int j = tid; j < P; j += SNT) {
                sv[j] = j < n ? kv[j] : -INFINITY;
                si[j] = j < n ? j : 0x7fffffff;
            }
            __syncthreads();
            bitonic(sv, si, P);
            if (tid == 0) {
                float cum = 0.0f;
                int cut = na;
                for (int j = 0; j < na; ++j) {
                    cum = cum + sv[j];
                    if (cum >= top_p) { cut = j + 1; break; }
                }
                *s_cut = cut;
            }
            __syncthreads();
            for (int j = *s_cut + tid; j < na; j += SNT) kv[si[j]] = 0.0f;
            __syncthreads();
            if (tid == 0) {
                float s = 0.0f;
                for (int j = 0; j < n; ++j) s = s + kv[j];
                *s_sum = s;
            }
            __syncthreads();
            const float s2 = *s_sum;
            if (s2 > 0)
                for (int j = tid; j < n; j += SNT) kv[j] = kv[j] / s2;
            __syncthreads();
        }
    }
    int pick = -1;
    if (tid == 0) {
        uint64_t x = sp->rng;
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        sp->rng = x;
        const float r = (float)(x >> 33) / (float)(1ULL << 31);
        *r_out = r;
        float cum = 0.0f;
        for (int j = 0; j < n; ++j) {
            cum = cum + kv[j];
            if (cum >= r) { pick = j; break; }
        }
        if (pick < 0)
            for (int j = n - 1; j >= 0; --j)
                if (kv[j] > 0) { pick = j; break; }
    }
    return pick;
}

struct lds_hist {
    uint32_t c[NW][256];
    uint64_t s[NW][256];
};

// One lane adds src[0..n) one term at a time in index order (the reference's
// float sum) from LDS, while the other waves stage the next SMALL entries
// into the other half of buf. find: stop at the first index whose running sum
// is >= r. Leaves the sum in *s_out and that index (or -1) in *hit_out.
// Every thread of the workgroup calls it.
__device__ __forceinline__ void staged_seq(const float *src, int n, float *buf, bool find, float r,
                                           float *s_out, int *hit_out, int *s_flag) {
    const int tid = threadIdx.x;
    for (int j = tid; j < min(SMALL, n); j += SNT) buf[j] = src[j];
    __syncthreads();
    float s = 0.0f;
    int hit = -1;
    const int nb = (n + SMALL - 1) / SMALL;
    for (int b = 0; b < nb; ++b) {
        const float *cur = buf + (b & 1) * SMALL;
        float *nxt = buf + ((b + 1) & 1) * SMALL;
        if (tid >= 64) {
            const int o = (b + 1) * SMALL;
            for (int j = tid - 64; j < SMALL && o + j < n; j += SNT - 64) nxt[j] = src[o + j];
        } else if (tid == 0) {
            const int len = min(SMALL, n - b * SMALL);
            const float4 *c4 = reinterpret_cast<const float4 *>(cur);
            int k = 0;
            for (; k + 32 <= len; k += 32) {
                float4 t[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) t[u] = c4[(k >> 2) + u];
                const float s0 = s;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    s = s + t[u].x;
                    s = s + t[u].y;
                    s = s + t[u].z;
                    s = s + t[u].w;
                }
                if (find && s >= r) {
                    // the running sum only grows: the crossing is in these 32
                    s = s0;
                    for (int u = 0; u < 32; ++u) {
                        s = s + cur[k + u];
                        if (s >= r) { hit = b * SMALL + k + u; break; }
                    }
                    break;
                }
            }
            if (hit < 0)
                for (; k < len; ++k) {
                    s = s + cur[k];
                    if (find && s >= r) { hit = b * SMALL + k; break; }
                }
        }
        __syncthreads();
        if (find) {
            if (tid == 0) *s_flag = hit;
            __syncthreads();
            if (*s_flag >= 0) break;
        }
    }
    if (tid == 0) {
        *s_out = s;
        *hit_out = hit;
    }
    __syncthreads();
}

__device__ __forceinline__ uint64_t comp_key(float v, int j) {
    return ((uint64_t)key_of(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)j);
}

// Top-p in the reference's order over pv[0..n) (n > SMALL): the candidates
// (> 1e-10) are taken in descending (value, then index) order SMALL at a
// time: a radix select on 64-bit (key, ~index) finds each chunk's lower
// bound, the chunk is sorted in LDS and one lane continues the running float
// sum through it until it reaches top_p. Entries after the cut become 0; the
// rest is renormalised by the serial sum. Every thread calls it.
__device__ __forceinline__ void top_p_chunks(float *pv, int n, float top_p, lds_hist &H, float *sv, int *si,
                                             float *stage, int *s_redi, uint64_t *s_pfx, uint64_t *s_msk,
                                             uint32_t *s_k, int *s_cut, int *s_tp, float *s_sum, int *s_pick,
                                             int *s_flag) {
    const int tid = threadIdx.x, wave = tid >> 6;
    int c = 0;
    seg_for(pv, n, [&](int, float v, bool ok) { c += (ok && v > 1e-10f) ? 1 : 0; });
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    __syncthreads();
    if ((tid & 63) == 0) s_redi[wave] = c;
    __syncthreads();
    int m = 0;
    for (int w = 0; w < NW; ++w) m += s_redi[w];
    if (m <= 1) return;                                   // the reference's n_active > 1
    uint64_t bound = ~0ull;                               // chunks so far: composite keys >= bound
    uint64_t cut_ck = 0;
    bool found = false;
    __shared__ float s_cum;
    __shared__ int s_cnt;
    if (tid == 0) s_cum = 0.0f;
    for (int taken = 0; taken < m && !found;) {
        const int C = min(SMALL, m - taken);
        if (tid == 0) { *s_pfx = 0; *s_msk = 0; *s_k = (uint32_t)C; }
        for (int shift = 56; shift >= 0; shift -= 8) {
            for (int b = tid; b < NW * 256; b += SNT) (&H.c[0][0])[b] = 0;
            __syncthreads();
            const uint64_t prefix = *s_pfx, mask = *s_msk;
            seg_for(pv, n, [&](int j, float v, bool ok) {
                const uint64_t k = comp_key(v, j);
                if (ok && v > 1e-10f && k < bound && (k & mask) == prefix)
                    atomicAdd(&H.c[wave][(k >> shift) & 255u], 1u);
            });
            __syncthreads();
            if (tid < 256) {
                uint32_t cc = 0;
                for (int w = 0; w < NW; ++w) cc += H.c[w][tid];
                H.c[0][tid] = cc;
            }
            __syncthreads();
            if (tid == 0) {
                uint32_t k = *s_k;
                int d = 255;
                for (; d > 0; --d) {
                    if (k <= H.c[0][d]) break;
                    k -= H.c[0][d];
                }
                *s_k = k;
                *s_pfx = prefix | ((uint64_t)d << shift);
                *s_msk = mask | (255ull << shift);
                s_cnt = 0;
            }
            __syncthreads();
        }
        const uint64_t lo = *s_pfx;                       // the chunk: lo <= key < bound, C entries
        seg_for(pv, n, [&](int j, float v, bool ok) {
            const uint64_t k = comp_key(v, j);
            if (ok && v > 1e-10f && k >= lo && k < bound) {
                const int o = atomicAdd(&s_cnt, 1);        // below C: the keys are distinct
                if (o < SMALL) {
                    sv[o] = v;
                    si[o] = j;
                }
            }
        });
        __syncthreads();
        int P = 1;
        while (P < C) P <<= 1;
        for (int j = C + tid; j < P; j += SNT) { sv[j] = -INFINITY; si[j] = 0x7fffffff; }
        __syncthreads();
        bitonic(sv, si, P);
        if (tid == 0) {
            float cum = s_cum;
            int at = -1;
            for (int j = 0; j < C; ++j) {
                cum = cum + sv[j];
                if (cum >= top_p) { at = j; break; }
            }
            s_cum = cum;
            *s_cut = at < 0 ? -1 : si[at];
            *s_tp = at < 0 ? 0 : __float_as_int(sv[at]);
        }
        __syncthreads();
        if (*s_cut >= 0) {
            found = true;
            cut_ck = comp_key(__int_as_float(*s_tp), *s_cut);
        }
        taken += C;
        bound = lo;
        __syncthreads();
    }
    if (found)
        seg_for(pv, n, [&](int j, float v, bool ok) {
            if (ok && v > 1e-10f && comp_key(v, j) < cut_ck) pv[j] = 0.0f;
        });
    __syncthreads();
    staged_seq(pv, n, stage, false, 0.0f, s_sum, s_pick, s_flag);
    const float s2 = *s_sum;
    if (s2 > 0)
        seg_for(pv, n, [&](int j, float v, bool ok) {
            if (ok) pv[j] = v / s2;
        });
    __syncthreads();
}

// Top-p with exact sums over pv[0..n): the shortest descending prefix of the
// candidates (> 1e-10) whose exact sum reaches top_p, by a radix descent over
// keys carrying counts and exact sums per digit; ties at the cut value are
// taken by index. Every thread calls it.
__device__ __forceinline__ void top_p_exact_sums(float *pv, int n, float top_p, lds_hist &H, int *s_w,
                                                 uint64_t *s_q, uint32_t *s_prefix, uint32_t *s_mask,
                                                 uint32_t *s_k, uint64_t *s_acc, int *s_cut, int *s_tp) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t target = fx(top_p, FX_P) + ((fx(top_p, FX_P) == 0) ? 1 : 0);
    if (tid == 0) { *s_prefix = 0; *s_mask = 0; *s_acc = 0; *s_cut = 1; *s_tp = 1; }
    __syncthreads();
    for (int shift = 24; shift >= 0 && *s_tp; shift -= 8) {
        for (int b = tid; b < NW * 256; b += SNT) {
            (&H.c[0][0])[b] = 0;
            (&H.s[0][0])[b] = 0;
        }
        __syncthreads();
        const uint32_t prefix = *s_prefix, mask = *s_mask;
        seg_for(pv, n, [&](int, float v, bool ok) {
            const uint32_t k = key_of(v);
            if (ok && v > 1e-10f && (k & mask) == prefix) {
                atomicAdd(&H.c[wave][(k >> shift) & 255u], 1u);
                atomicAdd((unsigned long long *)&H.s[wave][(k >> shift) & 255u], (unsigned long long)fx(v, FX_P));
            }
        });
        __syncthreads();
        if (tid < 256) {
            uint32_t c = 0;
            uint64_t sm = 0;
            for (int w = 0; w < NW; ++w) { c += H.c[w][tid]; sm += H.s[w][tid]; }
            H.c[0][tid] = c;
            H.s[0][tid] = sm;
        }
        __syncthreads();
        if (tid == 0 && shift == 24) {
            uint32_t na = 0;
            for (int d = 0; d < 256; ++d) na += H.c[0][d];
            *s_tp = na > 1;                               // the reference's n_active > 1
        }
        if (tid == 0 && *s_cut) {
            uint64_t acc = *s_acc;
            int d = 255;
            for (; d >= 0; --d) {
                if (acc + H.s[0][d] >= target) break;
                acc += H.s[0][d];
            }
            if (d < 0) {
                *s_cut = 0;                               // the candidates never reach top_p: no cut
            } else {
                *s_acc = acc;
                *s_prefix = prefix | ((uint32_t)d << shift);
                *s_mask = mask | (255u << shift);
                if (shift == 0) *s_k = H.c[0][d];         // entries equal to the cut value
            }
        }
        __syncthreads();
    }
    if (*s_tp && *s_cut) {
        const float tau = float_of(*s_prefix);
        const uint64_t tq = fx(tau, FX_P);
        // tied entries kept, in index order: the first `keep` of them
        const int keep = (int)((target - *s_acc + tq - 1) / tq);
        const int ties = (int)*s_k;
        int off = 0;
        if (keep < ties) {
            int c = 0;
            seg_for(pv, n, [&](int, float v, bool ok) { c += __popcll(__ballot(ok && v == tau)); });
            __syncthreads();
            if (lane == 0) s_w[wave] = c;
            __syncthreads();
            for (int w = 0; w < wave; ++w) off += s_w[w];
        }
        const uint64_t lt = (1ull << lane) - 1ull;
        seg_for(pv, n, [&](int j, float v, bool ok) {
            const bool tie = ok && v == tau;
            const uint64_t m = __ballot(tie);
            if (ok && v > 1e-10f && (v < tau || (tie && off + __popcll(m & lt) >= keep))) pv[j] = 0.0f;
            off += __popcll(m);
        });
        __syncthreads();
    }
    if (*s_tp) {
        // renormalised (also when nothing was cut, as the reference does)
        uint64_t q2 = 0;
        seg_for(pv, n, [&](int, float v, bool ok) {
            if (ok) q2 += fx(v, FX_P);
        });
        const float s2 = unfx(block_sum_u64(q2, s_q), FX_P);
        if (s2 > 0)
            seg_for(pv, n, [&](int j, float v, bool ok) {
                if (ok) pv[j] = v / s2;
            });
        __syncthreads();
    }
}

// The first index of pv[0..n) whose exact cumulative sum reaches r (> 0):
// exact sums per wave share, then per 64 chunks of the chosen share, then the
// chosen chunk entry by entry. -1 when the total stays below r.
__device__ __forceinline__ int pick_exact_sums(const float *pv, int n, float r, uint64_t *s_q, int *s_wsel,
                                               uint64_t *s_run, int *s_pick) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t qw = 0;
    seg_for(pv, n, [&](int, float v, bool ok) {
        if (ok) qw += fx(v, FX_P);
    });
    qw = wave_sum_u64(qw);
    __syncthreads();
    if (lane == 0) s_q[wave] = qw;
    __syncthreads();
    const uint64_t R = fx(r, FX_P);
    if (tid == 0) {
        uint64_t run = 0;
        int w = 0;
        for (; w < NW; ++w) {
            if (run + s_q[w] >= R) break;
            run += s_q[w];
        }
        *s_wsel = w < NW ? w : -1;
        *s_run = run;
        *s_pick = -1;
    }
    __syncthreads();
    if (wave == *s_wsel) {
        const seg_t sg = wave_seg(n);
        const int cs = (sg.e - sg.b + 63) / 64;
        const int c0 = min(sg.e, sg.b + lane * cs), c1 = min(sg.e, c0 + cs);
        uint64_t ql = 0;
        for (int j = c0; j < c1; j += 16) {
            float t[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) t[u] = pv[min(j + u, c1 - 1)];
#pragma unroll
            for (int u = 0; u < 16; ++u) ql += j + u < c1 ? fx(t[u], FX_P) : 0;
        }
        const uint64_t incl = wave_incl_scan_u64(ql);
        const uint64_t run = *s_run;
        const uint64_t hit = __ballot(run + incl >= R);
        const int L = hit ? __ffsll((long long)hit) - 1 : 63;
        if (lane == L) {
            uint64_t acc = run + incl - ql;
            int pk = -1;
            for (int j = c0; j < c1; ++j) {
                acc += fx(pv[j], FX_P);
                if (acc >= R) { pk = j; break; }
            }
            *s_pick = pk;
        }
    }
    __syncthreads();
    return *s_pick;
}

// bmax[0..nb): optional maxima of disjoint blocks of lg as the GEMV wrote it
// (before the penalty, which only lowers values: an upper bound of the
// maximum, which is all the top-k window needs). write_back = 0: nobody
// reads lg afterwards, so a top-k draw leaves it as it is.
__global__ __launch_bounds__(SNT) void k_sample(float *lg, int V, pk_sampler_dev *sp, float *av, int *ai,
                                                pk_dstate *st, int32_t *out_toks, int out_cap,
                                                const float *bmax, int nb, int write_back) {
    // radix histograms (counts, exact sums) and the small path's sort share one block
    __shared__ __align__(16) uint64_t lds_raw[sizeof(lds_hist) / 8];
    // the small path's kept entries double as the staging buffer of the serial sums
    __shared__ __align__(16) float stage[2 * SMALL];
    __shared__ float s_red[NW];
    __shared__ int s_redi[NW], s_w[NW];
    __shared__ uint64_t s_q[NW];
    __shared__ uint32_t s_prefix, s_mask, s_k;
    __shared__ uint64_t s_pfx64, s_msk64;
    __shared__ int s_tok, s_cut, s_tp, s_wsel, s_pick, s_flag;
    __shared__ float s_sum, s_r;
    __shared__ uint64_t s_acc, s_run;
    lds_hist &H = *reinterpret_cast<lds_hist *>(lds_raw);
    float *sv = reinterpret_cast<float *>(lds_raw);
    int *si = reinterpret_cast<int *>(sv + SMALL);
    float *kv = stage;
    int *ki = reinterpret_cast<int *>(stage + SMALL);
    __shared__ float cv[CAND];                          // top-k candidates (value, index)
    __shared__ int ci[CAND];
    __shared__ int s_nc, s_cnt, s_win;
    __shared__ uint64_t s_q2[NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float T = sp->temperature, top_p = sp->top_p, rep = sp->rep_penalty;
    const int K = sp->top_k;

    // 1. repetition penalty: the first occurrence of each token applies it
    // as many times as the token occurs (counts in ai[], reset first)
    if (rep > 1.0f) {
        const int hl = min(sp->history_len, PK_HISTORY_CAP);
        for (int i = tid; i < hl; i += SNT) {
            const int t = sp->history[i];
            if (t >= 0 && t < V) ai[t] = 0;
        }
        __syncthreads();
        unsigned own = 0;
#pragma unroll
        for (int q = 0; q < PK_HISTORY_CAP / SNT; ++q) {
            const int i = tid + q * SNT;
            if (i < hl) {
                const int t = sp->history[i];
                if (t >= 0 && t < V && atomicAdd(&ai[t], 1) == 0) own |= 1u << q;
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PK_HISTORY_CAP / SNT; ++q)
            if (own & (1u << q)) {
                const int t = sp->history[tid + q * SNT];
                const int c = atomicAdd(&ai[t], 0);
                float v = lg[t];
                for (int r = 0; r < c; ++r) v = v > 0 ? v / rep : v * rep;
                lg[t] = v;
            }
        __syncthreads();
    }

    if (T < 1e-6f) {
        // 2. greedy: the first maximum (the reference moves on a strictly
        // greater value only, so ties and NaNs keep the earlier index)
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        seg_for(lg, V, [&](int j, float v, bool ok) {
            if (ok && (v > bv || (v == bv && j < bi))) { bv = v; bi = j; }
        });
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { s_red[wave] = bv; s_redi[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < NW; ++w)
                if (s_red[w] > bv || (s_red[w] == bv && s_redi[w] < bi)) { bv = s_red[w]; bi = s_redi[w]; }
            s_tok = (bi == 0x7fffffff || !(bv > lg[0])) ? 0 : bi;
        }
        __syncthreads();
    } else {
        // 3. temperature (applied as each pass reads, and stored with the kept entries)
        const float inv_t = 1.0f / T;
        const auto scaled = [inv_t](float v) { return v * inv_t; };

        // 4. top-k threshold: the K-th largest key, 8 bits per pass from the top.
        // After the first pass (sign and exponent) the entries whose top byte
        // reaches the threshold's are few for any real top-k; when at most CAND,
        // they are gathered into LDS and the later passes, the kept set and its
        // index order are worked out there.
        const bool use_k = K > 0 && K < V;
        int n = V;
        bool direct = false;                                  // kept entries already in kv / ki
        if (use_k) {
            if (tid == 0) { s_prefix = 0; s_mask = 0; s_k = (uint32_t)K; }
            // histogram totals into H.c[0], then the digit holding the K-th largest
            const auto radix_walk = [&](int shift) {
                __syncthreads();
                if (tid < 256) {
                    uint32_t c = 0;
                    for (int w = 0; w < NW; ++w) c += H.c[w][tid];
                    H.c[0][tid] = c;
                }
                __syncthreads();
                if (tid == 0) {
                    uint32_t k = s_k;
                    int d = 255;
                    for (; d > 0; --d) {
                        if (k <= H.c[0][d]) break;
                        k -= H.c[0][d];
                    }
                    s_k = k;
                    s_prefix = s_prefix | ((uint32_t)d << shift);
                    s_mask = s_mask | (255u << shift);
                    // entries at or above the new bucket: K - k above it, and the bucket
                    s_nc = (int)((uint32_t)K - k + H.c[0][d]);
                    s_cnt = 0;
                }
                __syncthreads();
            };
            // First 8 bits. The K-th largest nearly always lies within a few
            // binades of the maximum: the maximum key, then the counts of the 8
            // sign/exponent buckets at and below it in 16-bit fields of two
            // registers per lane (no atomics: a whole wave would hit the same
            // few LDS counters). Otherwise a full histogram pass.
            uint32_t mk = 0;
            if (bmax) {
                for (int b = tid; b < nb; b += SNT) mk = max(mk, key_of(bmax[b] * inv_t));
            } else {
                seg_for(lg, V, [&](int, float v, bool ok) {
                    if (ok) mk = max(mk, key_of(v * inv_t));
                });
            }
            for (int o = 32; o > 0; o >>= 1) mk = max(mk, (uint32_t)__shfl_xor((int)mk, o, 64));
            if (lane == 0) s_w[wave] = (int)mk;
            __syncthreads();
            mk = 0;
            for (int w = 0; w < NW; ++w) mk = max(mk, (uint32_t)s_w[w]);
            const uint32_t tb = mk >> 24;
            uint64_t lo = 0, hi = 0;
            seg_for(lg, V, [&](int, float v, bool ok) {
                const uint32_t d = tb - (key_of(v * inv_t) >> 24);
                const uint64_t inc = (ok && d < 8u) ? (1ull << (16u * (d & 3u))) : 0ull;
                lo += d < 4u ? inc : 0ull;
                hi += d < 4u ? 0ull : inc;
            });
            lo = wave_sum_u64(lo);                        // per wave at most V/16 per field
            hi = wave_sum_u64(hi);
            if (lane == 0) { s_q[wave] = lo; s_q2[wave] = hi; }
            __syncthreads();
            if (tid == 0) {
                uint32_t cum = 0, rank = 0;
                int i = 0;
                for (; i < 8; ++i) {
                    uint32_t c = 0;
                    for (int w = 0; w < NW; ++w)
                        c += (uint32_t)(((i < 4 ? s_q[w] : s_q2[w]) >> (16 * (i & 3))) & 0xffffu);
                    if (cum + c >= (uint32_t)K) {
                        rank = (uint32_t)K - cum;         // the K-th largest's rank inside bucket i
                        cum += c;
                        break;
                    }
                    cum += c;
                }
                s_win = i < 8 && (int)tb - i >= 0;
                if (s_win) {
                    s_k = rank;
                    s_prefix = (tb - (uint32_t)i) << 24;
                    s_mask = 0xff000000u;
                    s_nc = (int)cum;
                    s_cnt = 0;
                }
            }
            __syncthreads();
            if (!s_win) {
                for (int b = tid; b < NW * 256; b += SNT) (&H.c[0][0])[b] = 0;
                __syncthreads();
                seg_for(lg, V, [&](int, float v, bool ok) {
                    if (ok) atomicAdd(&H.c[wave][key_of(v * inv_t) >> 24], 1u);
                });
                radix_walk(24);
            }
            // the remaining 24 bits; as soon as the entries at or above the
            // current bucket fit in LDS they are gathered there and the rest runs on them
            bool in_lds = false;
            int nc = 0;
            for (int shift = 16; shift >= -8; shift -= 8) {
                if (!in_lds && s_nc <= CAND) {
                    nc = s_nc;
                    const uint32_t top = s_prefix;
                    seg_for(lg, V, [&](int j, float v, bool ok) {
                        const float x = v * inv_t;
                        if (ok && key_of(x) >= top) {
                            const int o = atomicAdd(&s_cnt, 1);   // below nc: counted by the passes
                            if (o < CAND) {
                                cv[o] = x;
                                ci[o] = j;
                            }
                        }
                    });
                    in_lds = true;
                    __syncthreads();
                }
                if (shift < 0) break;
                for (int b = tid; b < NW * 256; b += SNT) (&H.c[0][0])[b] = 0;
                __syncthreads();
                const uint32_t prefix = s_prefix, mask = s_mask;
                if (in_lds) {
                    for (int i = tid; i < nc; i += SNT) {
                        const uint32_t k = key_of(cv[i]);
                        if ((k & mask) == prefix) atomicAdd(&H.c[wave][(k >> shift) & 255u], 1u);
                    }
                } else {
                    seg_for(lg, V, [&](int, float v, bool ok) {
                        const uint32_t k = key_of(v * inv_t);
                        if (ok && (k & mask) == prefix) atomicAdd(&H.c[wave][(k >> shift) & 255u], 1u);
                    });
                }
                radix_walk(shift);
            }
            const float thr = float_of(s_prefix);
            // a zero threshold also keeps -0.0, whose key lies below the candidates'
            if (in_lds && thr != 0.0f) {
                // the kept candidates, then into index order
                if (tid == 0) s_cnt = 0;
                __syncthreads();
                for (int i = tid; i < nc; i += SNT)
                    if (!(cv[i] < thr)) {
                        const int o = atomicAdd(&s_cnt, 1);
                        kv[o] = cv[i];
                        ki[o] = ci[i];
                    }
                __syncthreads();
                n = s_cnt;
                int P = 1;
                while (P < n) P <<= 1;
                for (int j = n + tid; j < P; j += SNT) { kv[j] = 0.0f; ki[j] = 0x7fffffff; }
                __syncthreads();
                bitonic_by_index(kv, ki, P);
                direct = true;
            } else {
                n = compact(lg, V, [inv_t, thr](float v) { return !(v * inv_t < thr); }, scaled, av, ai, s_w);
            }
        }

        if (n <= SMALL) {
            // 5a. in LDS, the reference's order
            if (!direct) {
                for (int j = tid; j < n; j += SNT) {
                    kv[j] = use_k ? av[j] : lg[j] * inv_t;
                    ki[j] = use_k ? ai[j] : j;
                }
                __syncthreads();
            }
            const int pick = finish_small(kv, n, top_p, sp, sv, si, s_red, s_redi, &s_sum, &s_cut, &s_r);
            if (tid == 0) {
                // a draw of 0 takes the first vocabulary entry even when it was dropped
                s_tok = s_r <= 0.0f ? 0 : (pick >= 0 ? ki[pick] : -1);
            }
            __syncthreads();
            // the array as the reference leaves it: probabilities, 0 elsewhere
            if (use_k && write_back) {
                for (int i = tid; i < V; i += SNT) lg[i] = 0.0f;
                __syncthreads();
            }
            if (!use_k || write_back)
                for (int j = tid; j < n; j += SNT) lg[ki[j]] = kv[j];
        } else {
            // 5b. over pv[0..n) in global memory (av after top-k, else lg in place)
            float *pv = use_k ? av : lg;
            const bool fast = sp->fast_sums != 0;
            float mx = -1e30f;
            seg_for(pv, n, [&](int j, float v, bool ok) {
                if (!ok) return;
                if (!use_k) {
                    v = v * inv_t;
                    pv[j] = v;
                }
                mx = fmaxf(mx, v);
            });
            mx = block_max(mx, s_red);
            const int se = 63 - (32 - __clz(n));           // n values <= 1 sum below 2^63
            uint64_t q = 0;
            seg_for(pv, n, [&](int j, float v, bool ok) {
                if (!ok) return;
                const float e = expf(v - mx);
                pv[j] = e;
                q += fx(e, se);
            });
            float sum;
            if (fast) {
                sum = unfx(block_sum_u64(q, s_q), se);
            } else {
                __syncthreads();
                staged_seq(pv, n, stage, false, 0.0f, &s_sum, &s_pick, &s_flag);
                sum = s_sum;
            }
            seg_for(pv, n, [&](int j, float v, bool ok) {
                if (ok) pv[j] = v / sum;
            });
            __syncthreads();

            if (top_p < 1.0f && top_p > 0.0f) {
                if (fast)
                    top_p_exact_sums(pv, n, top_p, H, s_w, s_q, &s_prefix, &s_mask, &s_k, &s_acc, &s_cut, &s_tp);
                else
                    top_p_chunks(pv, n, top_p, H, sv, si, stage, s_redi, &s_pfx64, &s_msk64, &s_k, &s_cut,
                                 &s_tp, &s_sum, &s_pick, &s_flag);
            }

            // the draw
            if (tid == 0) {
                uint64_t x = sp->rng;
                x ^= x << 13;
                x ^= x >> 7;
                x ^= x << 17;
                sp->rng = x;
                s_r = (float)(x >> 33) / (float)(1ULL << 31);
            }
            __syncthreads();
            const float r = s_r;
            int pick;
            if (fast) {
                pick = pick_exact_sums(pv, n, r, s_q, &s_wsel, &s_run, &s_pick);
            } else {
                // the first index whose running float sum (in index order) reaches r
                staged_seq(pv, n, stage, true, r, &s_sum, &s_pick, &s_flag);
                pick = s_pick;
            }
            if (pick < 0) {
                // nothing reached r: the last entry with probability > 0
                int last = -1;
                seg_for(pv, n, [&](int j, float v, bool ok) {
                    if (ok && v > 0) last = max(last, j);
                });
                pick = block_max_i(last, s_redi);
            }
            // a draw of 0 takes the first vocabulary entry even when it was dropped
            if (tid == 0) s_tok = r <= 0.0f ? 0 : (pick >= 0 ? (use_k ? ai[pick] : pick) : -1);
            __syncthreads();
            if (use_k && write_back) {
                for (int i = tid; i < V; i += SNT) lg[i] = 0.0f;
                __syncthreads();
                for (int j = tid; j < n; j += SNT) lg[ai[j]] = av[j];
            }
        }
    }
    if (tid == 0) {
        const int tok = s_tok;
        // the reference appends every id it picks; its final fall-through 0 is not appended
        if (tok >= 0 && sp->history_len < PK_HISTORY_CAP) sp->history[sp->history_len++] = tok;
        const int t = tok < 0 ? 0 : tok;
        if (st) {
            if (st->n_out < out_cap) out_toks[st->n_out] = t;
            st->n_out = st->n_out + 1;
            st->next = t;
            st->tok = t;
            st->pos = st->pos + 1;
        }
        sp->last = t;
    }
}

// Prompt ids into the history in order (valid ids only, up to its capacity).
__global__ void k_seed_history(pk_sampler_dev *sp, const int32_t *ids, int n, int V) {
    if (threadIdx.x != 0) return;
    int hl = sp->history_len;
    for (int i = 0; i < n && hl < PK_HISTORY_CAP; ++i) {
        const int t = ids[i];
        if (t >= 0 && t < V) sp->history[hl++] = t;
    }
    sp->history_len = hl;
}

}  // namespace

int pk_sample_reserve(pk_engine *e, int vocab) {
    PK_CHECK(vocab >= 1, PK_ERR_ARG, "vocab %d", vocab);
    if (!e->samp) {
        PK_CHECK(!e->capturing, PK_ERR_ARG, "sampling: call pk_set_sampling before capturing");
        PK_TRY(pk_dev_alloc(e, (void **)&e->samp, sizeof(pk_sampler_dev)));
        pk_sampler_dev h{};
        h.top_p = 1.0f;
        h.rep_penalty = 1.0f;
        e->samp_params = h;
        PK_HIP(hipMemcpyAsync(e->samp, &h, sizeof(h), hipMemcpyHostToDevice, e->stream));
        PK_HIP(hipStreamSynchronize(e->stream));
    }
    if (vocab <= e->samp_cap) return PK_OK;
    PK_CHECK(!e->capturing, PK_ERR_ARG, "sampling: vocabulary %d beyond the scratch made before capture", vocab);
    PK_HIP(hipStreamSynchronize(e->stream));
    pk_dev_free(e, e->samp_av);
    pk_dev_free(e, e->samp_ai);
    e->device_bytes -= (int64_t)e->samp_cap * 8;
    e->samp_av = nullptr;
    e->samp_ai = nullptr;
    e->samp_cap = 0;
    PK_TRY(pk_dev_alloc(e, (void **)&e->samp_av, (int64_t)vocab * 4));
    PK_TRY(pk_dev_alloc(e, (void **)&e->samp_ai, (int64_t)vocab * 4));
    e->samp_cap = vocab;
    return PK_OK;
}

int pk_launch_sample(pk_engine *e, float *logits, int vocab, pk_dstate *st, int32_t *out_toks, int out_cap,
                     const float *block_max, int n_blocks, bool write_back) {
    PK_CHECK(e->samp && vocab >= 1 && vocab <= e->samp_cap, PK_ERR_ARG,
             "sampling: vocabulary %d, scratch for %d", vocab, e->samp_cap);
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(SNT), 0, e->stream, logits, vocab, e->samp, e->samp_av,
                       e->samp_ai, st, out_toks, out_cap, block_max, n_blocks, write_back ? 1 : 0);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

int pk_sample_seed_history(pk_engine *e, const int32_t *ids_dev, int n) {
    if (!e->samp_on || !(e->samp_params.rep_penalty > 1.0f) || n <= 0) return PK_OK;
    hipLaunchKernelGGL(k_seed_history, dim3(1), dim3(64), 0, e->stream, e->samp, ids_dev, n, e->c.vocab);
    PK_HIP(hipGetLastError());
    return PK_OK;
}

// Parameters into the device state; rng and history replaced only on reset
// (temperature .. top_k come before rng in the struct, so a short copy keeps them).
static int put_params(pk_engine *e, const pk_sampler_dev &p, bool reset) {
    PK_TRY(pk_sample_reserve(e, e->c.vocab > 0 ? e->c.vocab : 1));
    const size_t bytes = reset ? offsetof(pk_sampler_dev, history) : offsetof(pk_sampler_dev, rng);
    PK_HIP(hipMemcpyAsync(e->samp, &p, bytes, hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    e->samp_params = p;
    // greedy without a penalty is the lm_head's own argmax (no draw, no history use)
    const bool on = p.temperature >= 1e-6f || p.rep_penalty > 1.0f;
    if (on != e->samp_on && e->step_exec) {   // the captured step ends in the other kernel
        (void)hipGraphExecDestroy(e->step_exec);
        e->step_exec = nullptr;
        e->step_cap = -1;
    }
    e->samp_on = on;
    return PK_OK;
}

extern "C" int pk_set_sampling(pk_engine *e, float temperature, float top_p, int top_k, float rep_penalty,
                               uint64_t seed) {
    PK_CHECK(e, PK_ERR_ARG, "null argument");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_sampling: not available while capturing");
    pk_sampler_dev p{};
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.rep_penalty = rep_penalty;
    p.rng = seed;
    p.history_len = 0;
    p.fast_sums = e->samp ? e->samp_params.fast_sums : 0;
    return put_params(e, p, true);
}

extern "C" int pk_set_sampling_fast_sums(pk_engine *e, int on) {
    PK_CHECK(e, PK_ERR_ARG, "null argument");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_sampling_fast_sums: not available while capturing");
    PK_TRY(pk_sample_reserve(e, e->c.vocab > 0 ? e->c.vocab : 1));
    e->samp_params.fast_sums = on ? 1 : 0;
    PK_HIP(hipMemcpyAsync((char *)e->samp + offsetof(pk_sampler_dev, fast_sums), &e->samp_params.fast_sums, 4,
                          hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

extern "C" int pk_set_turn_sampling(pk_engine *e, float temperature, float top_p, int top_k) {
    PK_CHECK(e, PK_ERR_ARG, "null argument");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "set_turn_sampling: not available while capturing");
    PK_TRY(pk_sample_reserve(e, e->c.vocab > 0 ? e->c.vocab : 1));
    pk_sampler_dev p = e->samp_params;
    // the TURN header's defensive clamp (picchio.c:2737-2743)
    if (temperature < 0.0f) temperature = 0.0f;
    if (temperature > 5.0f) temperature = 5.0f;
    if (top_p <= 0.0f || top_p > 1.0f) top_p = 1.0f;
    if (top_k < 0) top_k = 0;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    return put_params(e, p, false);
}

extern "C" int pk_reset_history(pk_engine *e) {
    PK_CHECK(e, PK_ERR_ARG, "null argument");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "reset_history: not available while capturing");
    if (!e->samp) return PK_OK;
    static const int32_t zero = 0;
    PK_HIP(hipMemcpyAsync((char *)e->samp + offsetof(pk_sampler_dev, history_len), &zero, 4,
                          hipMemcpyHostToDevice, e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    return PK_OK;
}

extern "C" int pk_sample_logits(pk_engine *e, float *logits_dev, int vocab, int32_t *tok_host) {
    PK_CHECK(e && logits_dev && tok_host, PK_ERR_ARG, "null argument");
    PK_CHECK(vocab >= 1, PK_ERR_ARG, "vocab %d", vocab);
    PK_CHECK(!e->capturing, PK_ERR_ARG, "sample_logits: host result; not available while capturing");
    PK_TRY(pk_sample_reserve(e, vocab));
    PK_TRY(pk_launch_sample(e, logits_dev, vocab, nullptr, nullptr, 0, nullptr, 0, true));
    int32_t last = 0;
    PK_HIP(hipMemcpyAsync(&last, (char *)e->samp + offsetof(pk_sampler_dev, last), 4, hipMemcpyDeviceToHost,
                          e->stream));
    PK_HIP(hipStreamSynchronize(e->stream));
    *tok_host = last;
    return PK_OK;
}

extern "C" int pk_sampler_state(pk_engine *e, uint64_t *rng, int32_t *history, int cap, int *history_len) {
    PK_CHECK(e && rng && history_len, PK_ERR_ARG, "null argument");
    PK_CHECK(!e->capturing, PK_ERR_ARG, "sampler_state: not available while capturing");
    PK_TRY(pk_sample_reserve(e, e->c.vocab > 0 ? e->c.vocab : 1));
    pk_sampler_dev *h = new pk_sampler_dev;
    hipError_t rc = hipMemcpyAsync(h, e->samp, sizeof(*h), hipMemcpyDeviceToHost, e->stream);
    if (rc == hipSuccess) rc = hipStreamSynchronize(e->stream);
    if (rc == hipSuccess) {
        *rng = h->rng;
        *history_len = h->history_len;
        if (history)
            for (int i = 0; i < h->history_len && i < cap; ++i) history[i] = h->history[i];
    }
    delete h;
    PK_HIP(rc);
    return PK_OK;
}
