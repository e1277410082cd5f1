/* attn_synth.c -- synthetic bf16 inputs for the benchmark and tests (see attn_devutil.h). */
#include "attn_devutil.h"

#include <math.h>
#include <string.h>

uint16_t attn_synth_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7f800000u) == 0x7f800000u) /* Inf/NaN: truncate */
        return (uint16_t)(u >> 16);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static uint64_t synth_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void attn_synth_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t counter0,
                            double sigma) {
    const double two_pi = 6.283185307179586476925286766559;
    const double inv53 = 1.0 / 9007199254740992.0;
    long long nn = (long long)n;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < nn; i++) {
        uint64_t c = counter0 + (uint64_t)i;
        uint64_t a = synth_mix(seed + (2 * c + 1) * 0x9E3779B97F4A7C15ull);
        uint64_t b = synth_mix(seed + (2 * c + 2) * 0x9E3779B97F4A7C15ull);
        double u1 = ((double)(a >> 11) + 0.5) * inv53;
        double u2 = (double)(b >> 11) * inv53;
        double v = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = attn_synth_f32_to_bf16((float)(sigma * v));
    }
}

void attn_synth_lcg_bf16(uint32_t *state, uint16_t *out, size_t n) {
    uint32_t s = *state;
    for (size_t i = 0; i < n; i++) {
        s = s * 1664525u + 1013904223u;
        out[i] = attn_synth_f32_to_bf16((float)((s >> 8) & 0xffffu) / 32768.0f - 1.0f);
    }
    *state = s;
}
