/* pk_synth.h — seeded synthetic weights and activations for the expert path.
 *
 * Counter-based generator: value i of a tensor depends only on (seed, tag, i),
 * so any thread layout produces the same bytes. SplitMix64 finaliser on the
 * counter gives two 53-bit uniforms per pair; Box-Muller in double precision
 * turns each pair into two N(0,1) samples, rounded once to float.
 *
 * Header-only C so the host engine and the CPU parity checker draw bit-identical
 * inputs from one definition.
 */
#ifndef PK_SYNTH_H
#define PK_SYNTH_H

#include <stdint.h>
#include <math.h>

/* Callable from device code too when compiled by hipcc. */
#if defined(__HIPCC__)
#define PK_SYNTH_FN static inline __host__ __device__
#else
#define PK_SYNTH_FN static inline
#endif

#ifdef __cplusplus
extern "C" {
#endif

PK_SYNTH_FN uint64_t pk_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Tensor kinds used to derive independent streams from one model seed. */
enum {
    PK_T_X = 1,          /* activations / token inputs        */
    PK_T_GU = 2,         /* expert gate_up weight             */
    PK_T_GU_B = 3,       /* expert gate_up bias               */
    PK_T_DOWN = 4,       /* expert down weight                */
    PK_T_DOWN_B = 5,     /* expert down bias                  */
    PK_T_ROUTER = 6,     /* router weight                     */
    PK_T_ROUTER_B = 7,   /* router bias                       */
    PK_T_WQ = 8, PK_T_WK = 9, PK_T_WV = 10, PK_T_WO = 11,
    PK_T_BQ = 12, PK_T_BK = 13, PK_T_BV = 14, PK_T_BO = 15,
    PK_T_SINKS = 16,
    PK_T_EMBED = 17,
    PK_T_LM_HEAD = 18,
    PK_T_IDS = 19        /* uniform token ids                 */
};

PK_SYNTH_FN uint64_t pk_stream(uint64_t seed, uint32_t kind, uint32_t layer,
                                 uint32_t index) {
    uint64_t tag = ((uint64_t)kind << 56) ^ ((uint64_t)layer << 36) ^ (uint64_t)index;
    return pk_mix64(seed ^ pk_mix64(tag));
}

/* Samples 2c and 2c+1 of stream `s`. */
PK_SYNTH_FN void pk_normal_pair(uint64_t s, uint64_t c, double *n0, double *n1) {
    uint64_t a = pk_mix64(s ^ pk_mix64(2 * c));
    uint64_t b = pk_mix64(s ^ pk_mix64(2 * c + 1));
    double u1 = (double)((a >> 11) + 1) * 0x1p-53;   /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1p-53;         /* [0, 1) */
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586 * u2;
    *n0 = r * cos(t);
    *n1 = r * sin(t);
}

/* out[i] = (float)(std * N_{first+i}) for i in [0, n). */
PK_SYNTH_FN void pk_fill_normal(float *out, int64_t n, uint64_t s, float std,
                                  int64_t first) {
    int64_t i = 0;
    while (i < n) {
        int64_t k = first + i;
        double n0, n1;
        pk_normal_pair(s, (uint64_t)(k >> 1), &n0, &n1);
        if ((k & 1) == 0) {
            out[i++] = (float)(n0 * (double)std);
            if (i < n) out[i++] = (float)(n1 * (double)std);
        } else {
            out[i++] = (float)(n1 * (double)std);
        }
    }
}

/* Uniform integer in [0, m). */
PK_SYNTH_FN int pk_uniform_int(uint64_t s, uint64_t c, int m) {
    uint64_t a = pk_mix64(s ^ pk_mix64(c));
    return (int)((a >> 11) % (uint64_t)m);
}

#ifdef __cplusplus
}
#endif
#endif /* PK_SYNTH_H */
