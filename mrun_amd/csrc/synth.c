/* Seeded synthetic inputs (the generator spec is in include/mrun_synth.h). */
#include "mrun_synth.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define GAMMA 0x9E3779B97F4A7C15ull

uint64_t mrun_synth_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t mrun_synth_tensor_seed(uint64_t base, uint32_t config, uint32_t layer, uint32_t tensor) {
    uint64_t tag = ((uint64_t)config << 48) ^ ((uint64_t)layer << 24) ^ (uint64_t)tensor;
    return base ^ mrun_synth_mix64(tag);
}

uint64_t mrun_synth_draw(uint64_t seed, uint64_t n) { return mrun_synth_mix64(seed + (n + 1) * GAMMA); }

static inline double uniform(uint64_t seed, uint64_t n) {
    return (double)(mrun_synth_draw(seed, n) >> 11) * (1.0 / 9007199254740992.0);
}

double mrun_synth_normal(uint64_t seed, uint64_t i) {
    uint64_t b = i & ~1ull;
    double u1 = uniform(seed, b), u2 = uniform(seed, b + 1);
    double r = sqrt(-2.0 * log(1.0 - u1));
    double th = 6.283185307179586476925286766559 * u2;
    return (i & 1) ? r * sin(th) : r * cos(th);
}

static inline uint16_t bf16_of(double v) {
    float f = (float)v;
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float f32_of(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int mrun_synth_codes(uint64_t seed, int32_t bits, uint32_t *words, size_t n_words) {
    if (bits != 4 && bits != 8) return -1;
    const int per = 32 / bits;
    const int shift = 64 - bits;
#pragma omp parallel for schedule(static)
    for (size_t w = 0; w < n_words; w++) {
        uint32_t v = 0;
        for (int j = 0; j < per; j++) {
            uint64_t d = mrun_synth_draw(seed, (uint64_t)w * per + j);
            v |= (uint32_t)(d >> shift) << (bits * j);
        }
        words[w] = v;
    }
    return 0;
}

void mrun_synth_normal_bf16(uint64_t seed, float std, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) out[i] = bf16_of((double)std * mrun_synth_normal(seed, i));
}

void mrun_synth_scales_biases(uint64_t seed, uint16_t *scales, uint16_t *biases, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        uint16_t s = bf16_of(fabs(0.02 * mrun_synth_normal(seed, i)) / 7.5);
        scales[i] = s;
        if (biases) biases[i] = bf16_of(-8.0 * (double)f32_of(s));
    }
}

int mrun_synth_zipf_bias(uint64_t seed, int32_t experts, double s, double amp, uint16_t *bias,
                         int32_t *rank_out) {
    if (experts <= 0) return -1;
    int32_t *rank = malloc(sizeof(int32_t) * (size_t)experts);
    if (!rank) return -1;
    for (int32_t i = 0; i < experts; i++) rank[i] = i + 1;
    for (int32_t i = experts - 1; i > 0; i--) {
        uint64_t j = mrun_synth_draw(seed, (uint64_t)(experts - 1 - i)) % (uint64_t)(i + 1);
        int32_t t = rank[i];
        rank[i] = rank[j];
        rank[j] = t;
    }
    for (int32_t e = 0; e < experts; e++) {
        bias[e] = bf16_of(amp * pow((double)rank[e], -s));
        if (rank_out) rank_out[e] = rank[e];
    }
    free(rank);
    return 0;
}
