/*
 * Seeded random-init weights for the Qwen3 decode engine's test and bench
 * checkpoints (CPU, plain C, OpenMP).
 *
 * The benchmark configs call for "BF16 weights drawn N(0, 0.02) from seed 0".
 * torch.normal_ is not reproducible across machines or library versions, so
 * the draw is specified here as a counter-based stream that any machine with
 * the same C library reproduces bit for bit:
 *
 *   stream s   = mix64(seed * GAMMA + fnv1a64(tensor name))
 *   o_i        = mix64(s + i * GAMMA)        i = 1, 2, ...   (SplitMix64)
 *   pair j     : a = o_{2j+1}, b = o_{2j+2}
 *   u1 = ((a >> 11) + 1) * 2^-53  in (0, 1]
 *   u2 =  (b >> 11)      * 2^-53  in [0, 1)
 *   z0 = sqrt(-2 ln u1) * cos(2 pi u2),  z1 = sqrt(-2 ln u1) * sin(2 pi u2)
 *   element 2j = bf16(float(offset + z0 * std)), 2j+1 likewise with z1
 *   (offset 0 for weight matrices; 1 for perturbed norm gains in test models)
 *
 * Both roundings are round-to-nearest-even.  Each element depends only on
 * (seed, name, index), so the parallel fill is deterministic.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GAMMA 0x9E3779B97F4A7C15ULL

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

uint64_t q3seed_fnv1a64(const char *name) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (const unsigned char *p = (const unsigned char *)name; *p; ++p) {
        h ^= *p;
        h *= 0x100000001B3ULL;
    }
    return h;
}

uint64_t q3seed_stream(uint64_t seed, const char *name) {
    return mix64(seed * GAMMA + q3seed_fnv1a64(name));
}

/* Fill out[0..n) with bf16(float(offset + z * std)), z the N(0,1) stream of `stream`. */
void q3seed_fill_normal_bf16(uint64_t stream, uint16_t *out, int64_t n, double offset, double std) {
    const int64_t pairs = (n + 1) / 2;
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < pairs; ++j) {
        uint64_t a = mix64(stream + (uint64_t)(2 * j + 1) * GAMMA);
        uint64_t b = mix64(stream + (uint64_t)(2 * j + 2) * GAMMA);
        double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(b >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        double t = two_pi * u2;
        double z0 = offset + r * cos(t) * std;
        double z1 = offset + r * sin(t) * std;
        out[2 * j] = f32_to_bf16_rne((float)z0);
        if (2 * j + 1 < n) out[2 * j + 1] = f32_to_bf16_rne((float)z1);
    }
}

/* Fill out[0..n) with a constant bf16 bit pattern (norm gains = 1.0). */
void q3seed_fill_const_bf16(uint16_t *out, int64_t n, uint16_t bits) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = bits;
}

/* Uniform token ids in [0, vocab): o_i of the stream of (seed, row). */
void q3seed_prompt_ids(uint64_t seed, int64_t row, int64_t *out, int64_t n, int64_t vocab) {
    uint64_t s = mix64(seed * GAMMA + mix64((uint64_t)row + 0x5DEECE66DULL));
    for (int64_t i = 0; i < n; ++i) {
        uint64_t o = mix64(s + (uint64_t)(i + 1) * GAMMA);
        out[i] = (int64_t)(((o >> 32) * (uint64_t)vocab) >> 32);
    }
}
