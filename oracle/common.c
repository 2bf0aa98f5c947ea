/*
 * common.c — f16/bf16 conversion and the xorshift Rng.
 * TEST INFRASTRUCTURE ONLY (the oracle); see oracle.h.
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>

/* half 2.7.1 f16::from_f32: IEEE binary16 with round-to-nearest-even, quiet-NaN
 * payload kept (upper mantissa bits), overflow to infinity.  RIE relies on it at
 * quant/mod.rs:135-137, avx2.rs:253, model/cpu.rs:642, turbo.rs:162. */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | 0x0200u | (man >> 13));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t halfway = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t r = m >> shift;
        if (rem > halfway || (rem == halfway && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: man * 2^-24, exact in f32 */
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* half 2.7.1 bf16::from_f32 (round to nearest even, NaN kept quiet). */
uint16_t or_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t round_bit = 0x00008000u;
    if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0) return (uint16_t)((x >> 16) + 1u);
    return (uint16_t)(x >> 16);
}

/* kernels/mod.rs:421-434 → avx2.rs:243-256: _mm256_cvtps_ph(RNE) for 8-chunks and
 * half::f16::from_f32 for the tail; both are IEEE RNE. */
void or_f32_to_f16_slice(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = or_f32_to_f16(src[i]);
}

/* testing.rs:10-30 */
void or_rng_init(or_rng *r, uint64_t seed) { r->s = (seed * 0x9E3779B97F4A7C15ULL) | 1ULL; }

uint64_t or_rng_next(or_rng *r) {
    r->s ^= r->s << 13;
    r->s ^= r->s >> 7;
    r->s ^= r->s << 17;
    return r->s;
}

float or_rng_f32(or_rng *r) { return (float)(or_rng_next(r) >> 40) / (float)(1ULL << 24); }

float or_rng_sym(or_rng *r) { return or_rng_f32(r) * 2.0f - 1.0f; }

void or_free(void *p) { free(p); }
