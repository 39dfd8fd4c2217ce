/*
 * Seeded synthetic inputs for the batch-1 decode path (header-only C99).
 *
 * Every tensor is a pure function of (base seed, tensor name, element index),
 * so any block can be generated independently and in parallel, on any host,
 * and the bytes come out identical.  The generator is SplitMix64 evaluated at
 * a counter: element i of stream s is mix(s + (i + 1) * 0x9E3779B97F4A7C15),
 * which is exactly the (i+1)-th output of a SplitMix64 seeded with s.
 *
 * Distributions:
 *   uniform  u = (z >> 11) * 2^-53 in [0, 1)             (double)
 *   range    lo + (hi - lo) * u, computed in double, rounded once to float
 *   normal   Box-Muller on stream elements 2i and 2i+1:
 *            mean + std * sqrt(-2 ln(1 - u1)) * cos(2 pi u2)  (double, rounded once)
 *   fp16     round-to-nearest-even of the float (synth_f32_to_f16)
 *
 * Block formats are GGUF's: Q4_0 (18 bytes per 32 weights, fp16 d then 16
 * bytes of nibbles, weight j = low nibble of byte j, weight j+16 = high
 * nibble) and Q6_K (210 bytes per 256 weights: ql[128], qh[64], int8
 * scales[16], fp16 d).
 *
 * Compile host code that uses this header with -ffp-contract=off so that
 * no multiply-add is fused and every host produces the same floats.
 */
#ifndef ADAFORGE_SYNTH_H
#define ADAFORGE_SYNTH_H

#include <math.h>
#include <stdint.h>
#include <string.h>

#define SYNTH_BASE_SEED 0x4D49333535ull
#define SYNTH_GAMMA 0x9E3779B97F4A7C15ull

static inline uint64_t synth_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Element i of the stream seeded with s. */
static inline uint64_t synth_at(uint64_t s, uint64_t i) {
    return synth_mix(s + (i + 1) * SYNTH_GAMMA);
}

/* FNV-1a over a name, folded into the base seed: one stream per tensor. */
static inline uint64_t synth_seed(uint64_t base, const char* name) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (const unsigned char* p = (const unsigned char*)name; *p; ++p) {
        h ^= *p;
        h *= 0x100000001B3ull;
    }
    return synth_mix(base ^ h);
}

static inline double synth_unit(uint64_t z) { return (double)(z >> 11) * (1.0 / 9007199254740992.0); }

static inline float synth_uniform(uint64_t s, uint64_t i, double lo, double hi) {
    return (float)(lo + (hi - lo) * synth_unit(synth_at(s, i)));
}

static inline double synth_normal_d(uint64_t s, uint64_t i) {
    double u1 = synth_unit(synth_at(s, 2 * i));
    double u2 = synth_unit(synth_at(s, 2 * i + 1));
    double r = sqrt(-2.0 * log(1.0 - u1));
    return r * cos(6.283185307179586476925286766559 * u2);
}

/* mean + std * N(0,1), computed in double and rounded once to float. */
static inline float synth_normal(uint64_t s, uint64_t i, double mean, double std) {
    return (float)(mean + std * synth_normal_d(s, i));
}

/* IEEE binary32 -> binary16, round to nearest, ties to even (subnormals, Inf, NaN kept). */
static inline uint16_t synth_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) { /* Inf or NaN */
        return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u | ((absx >> 13) & 0x3FFu) : 0u));
    }
    if (absx >= 0x477FF000u) { /* rounds to >= 65520: overflow to Inf */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (absx < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to zero (2^-25 itself ties to 0) */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); target unit 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t m = absx & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* carry may bump the exponent: correct */
    return (uint16_t)(sign | q);
}

/* ---- tensors ---------------------------------------------------------------- */

/* Q4_0 block b of a matrix stream: d ~ U[dlo, dhi] as fp16, 16 uniform random bytes. */
static inline void synth_q4_block(uint64_t s, uint64_t b, double dlo, double dhi, uint8_t* out18) {
    uint16_t d = synth_f32_to_f16(synth_uniform(s, 3 * b, dlo, dhi));
    out18[0] = (uint8_t)(d & 0xFF);
    out18[1] = (uint8_t)(d >> 8);
    uint64_t a = synth_at(s, 3 * b + 1), c = synth_at(s, 3 * b + 2);
    for (int j = 0; j < 8; ++j) out18[2 + j] = (uint8_t)(a >> (8 * j));
    for (int j = 0; j < 8; ++j) out18[10 + j] = (uint8_t)(c >> (8 * j));
}

/* The same block with a random sign on d (bit 0 of the stream element that draws |d|, which
 * the uniform draw does not use): GGUF's Q4_0 quantiser stores d = max / -8 for the block's
 * largest-magnitude weight, so real scales take both signs, and with both signs the -0.5 d mean
 * of a uniform nibble no longer gives every row of a matrix the same bias direction. */
static inline void synth_q4_block_signed(uint64_t s, uint64_t b, double dlo, double dhi, uint8_t* out18) {
    const uint64_t z = synth_at(s, 3 * b);
    uint16_t d = synth_f32_to_f16((float)(dlo + (dhi - dlo) * synth_unit(z)));
    if (z & 1u) d ^= 0x8000u;
    out18[0] = (uint8_t)(d & 0xFF);
    out18[1] = (uint8_t)(d >> 8);
    uint64_t a = synth_at(s, 3 * b + 1), c = synth_at(s, 3 * b + 2);
    for (int j = 0; j < 8; ++j) out18[2 + j] = (uint8_t)(a >> (8 * j));
    for (int j = 0; j < 8; ++j) out18[10 + j] = (uint8_t)(c >> (8 * j));
}

/* Q6_K super-block b: 192 uniform random code bytes (so every 6-bit code is
 * uniform in 0..63), 16 int8 sub-scales uniform in [-32, 31], d ~ U[dlo, dhi]. */
static inline void synth_q6_block(uint64_t s, uint64_t b, double dlo, double dhi, uint8_t* out210) {
    uint64_t base = 27 * b;
    for (int w = 0; w < 24; ++w) {
        uint64_t z = synth_at(s, base + (uint64_t)w);
        for (int j = 0; j < 8; ++j) out210[8 * w + j] = (uint8_t)(z >> (8 * j));
    }
    for (int w = 0; w < 2; ++w) {
        uint64_t z = synth_at(s, base + 24 + (uint64_t)w);
        for (int j = 0; j < 8; ++j) out210[192 + 8 * w + j] = (uint8_t)(int8_t)((int)((z >> (8 * j)) & 63u) - 32);
    }
    uint16_t d = synth_f32_to_f16(synth_uniform(s, base + 26, dlo, dhi));
    out210[208] = (uint8_t)(d & 0xFF);
    out210[209] = (uint8_t)(d >> 8);
}

#endif
