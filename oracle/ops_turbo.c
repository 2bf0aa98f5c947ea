/*
 * ops_turbo.c — ops.rs (rmsnorm, silu, softmax, RoPE) and turbo.rs (TurboQuant
 * 4-bit KV rows) as RIE runs them on x86.
 * TEST INFRASTRUCTURE ONLY (the oracle); see oracle.h.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static inline float hsum8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    float a = s0 + s2, b = s1 + s3;
    return a + b;
}

/* ops.rs:7-14: out = (x*scale)*w with ss from the AVX2 dot_f32 */
void or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
    float ss = or_dot_f32(x, x, n) / (float)n;
    float scale = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* ops.rs:17-24: x *= (scale*w) — note the different association */
void or_rmsnorm_inplace(float *x, const float *w, size_t n, float eps) {
    float ss = or_dot_f32(x, x, n) / (float)n;
    float scale = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; i++) x[i] *= scale * w[i];
}

/* ops.rs:27-29 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops.rs:38-49 */
void or_softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* ops.rs:65-79: inv_freq[i] = base^(-2i/dim)·freq_scale (÷ factor) with libm powf */
void or_rope_inv_freq(size_t dim, float base, float freq_scale, const float *factors, size_t nfac, float *inv_freq) {
    size_t half = dim / 2;
    for (size_t i = 0; i < half; i++) {
        float f = powf(base, -2.0f * (float)i / (float)dim) * freq_scale;
        if (factors && i < nfac && factors[i] != 0.0f) f /= factors[i];
        inv_freq[i] = f;
    }
}

/* ops.rs:82-89 (mscale 1) */
void or_rope_table(const float *inv_freq, size_t half, size_t pos, float *cos_out, float *sin_out) {
    for (size_t i = 0; i < half; i++) {
        float theta = (float)pos * inv_freq[i];
        sin_out[i] = sinf(theta);
        cos_out[i] = cosf(theta);
    }
}

/* ops.rs:93-108 */
void or_rope_apply(float *x, size_t dim, int neox, const float *c, const float *s) {
    size_t half = dim / 2;
    if (neox) {
        for (size_t i = 0; i < half; i++) {
            float a = x[i], b = x[i + half];
            x[i] = a * c[i] - b * s[i];
            x[i + half] = a * s[i] + b * c[i];
        }
    } else {
        for (size_t i = 0; i < half; i++) {
            float a = x[2 * i], b = x[2 * i + 1];
            x[2 * i] = a * c[i] - b * s[i];
            x[2 * i + 1] = a * s[i] + b * c[i];
        }
    }
}

/* ---- turbo.rs ---------------------------------------------------------- */

static const int8_t KV_LEVELS_I8[16] = {-126, -95, -74, -58, -43, -30, -18, -6, 6, 18, 30, 43, 58, 74, 95, 126};

/* turbo.rs:52-58 */
size_t or_turbo_block_size(size_t d) {
    size_t b = 1;
    while (d % (b * 2) == 0 && b < 256) b *= 2;
    return b;
}

/* turbo.rs:136-138 */
size_t or_turbo_row_bytes(size_t d) { return 2 * (d / or_turbo_block_size(d)) + d / 2; }

/* turbo.rs:78-89 */
static float turbo_sign(uint64_t seed, size_t i) {
    uint64_t z = seed + (uint64_t)i * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return ((z ^ (z >> 31)) & 1u) == 0 ? 1.0f : -1.0f;
}

void or_turbo_signs(size_t d, uint64_t seed, float *signs) {
    for (size_t i = 0; i < d; i++) signs[i] = turbo_sign(seed, i);
}

/* turbo.rs:61-76 */
void or_fwht(float *x, size_t n) {
    for (size_t h = 1; h < n; h *= 2)
        for (size_t i = 0; i < n; i += 2 * h)
            for (size_t j = i; j < i + h; j++) {
                float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
    float s = 1.0f / sqrtf((float)n);
    for (size_t i = 0; i < n; i++) x[i] *= s;
}

/* turbo.rs:109-117 */
void or_turbo_rotate(float *x, size_t d, uint64_t seed) {
    size_t b = or_turbo_block_size(d);
    for (size_t i = 0; i < d; i++) x[i] *= turbo_sign(seed, i);
    for (size_t o = 0; o < d; o += b) or_fwht(x + o, b);
}

void or_turbo_rotate_inverse(float *x, size_t d, uint64_t seed) {
    size_t b = or_turbo_block_size(d);
    for (size_t o = 0; o < d; o += b) or_fwht(x + o, b);
    for (size_t i = 0; i < d; i++) x[i] *= turbo_sign(seed, i);
}

static void kv_levels(float c[16]) {
    for (int i = 0; i < 16; i++) c[i] = (float)KV_LEVELS_I8[i] / 46.0f;
}

/* turbo.rs:40-49 */
static uint8_t nearest(const float c[16], float v) {
    uint8_t i = 0;
    for (int k = 0; k < 15; k++) i += (uint8_t)(v > 0.5f * (c[k] + c[k + 1]));
    return i;
}

/* turbo.rs:140-164 */
void or_turbo_quantize_rotated(const float *y, size_t d, uint8_t *out) {
    size_t b = or_turbo_block_size(d), nb = d / b;
    float c[16];
    kv_levels(c);
    uint8_t *scales = out, *codes = out + 2 * nb;
    memset(codes, 0, d / 2);
    for (size_t bi = 0; bi < nb; bi++) {
        const float *yb = y + bi * b;
        float ss = 0.0f;
        for (size_t j = 0; j < b; j++) ss += yb[j] * yb[j];
        float rms = sqrtf(ss / (float)b);
        float inv = rms > 0.0f ? 1.0f / rms : 0.0f;
        float num = 0.0f, den = 0.0f;
        for (size_t j = 0; j < b; j++) {
            float v = yb[j];
            uint8_t q = nearest(c, v * inv);
            size_t g = bi * b + j;
            codes[(g / 32) * 16 + g % 16] |= (uint8_t)(q << ((g % 32) / 16 * 4));
            num += v * c[q];
            den += c[q] * c[q];
        }
        float s = den > 0.0f ? num / den : 0.0f;
        uint16_t h = or_f32_to_f16(s);
        scales[2 * bi] = (uint8_t)h;
        scales[2 * bi + 1] = (uint8_t)(h >> 8);
    }
}

/* turbo.rs:167-171 */
void or_turbo_quantize(const float *x, size_t d, uint64_t seed, uint8_t *out) {
    float tmp[512];
    memcpy(tmp, x, d * sizeof(float));
    or_turbo_rotate(tmp, d, seed);
    or_turbo_quantize_rotated(tmp, d, out);
}

static inline float scale_at(const uint8_t *row, size_t bi) {
    return or_f16_to_f32((uint16_t)(row[2 * bi] | ((uint16_t)row[2 * bi + 1] << 8)));
}

/* x86 dot_chunks, turbo.rs:279-294: lanes of 4 products, FMA with the chunk d */
static float dot_chunks_x86(const or_block_q8_0 *q, const uint8_t *codes, size_t nchunks) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t i = 0; i < nchunks; i++) {
        int x[32];
        for (int k = 0; k < 16; k++) {
            x[k] = KV_LEVELS_I8[codes[i * 16 + k] & 15];
            x[k + 16] = KV_LEVELS_I8[codes[i * 16 + k] >> 4];
        }
        for (int l = 0; l < 8; l++) {
            int32_t p = x[4 * l] * q[i].qs[4 * l] + x[4 * l + 1] * q[i].qs[4 * l + 1] + x[4 * l + 2] * q[i].qs[4 * l + 2] +
                        x[4 * l + 3] * q[i].qs[4 * l + 3];
            acc[l] = fmaf(q[i].d, (float)p, acc[l]);
        }
    }
    return hsum8(acc);
}

/* turbo.rs:180-193 */
float or_turbo_dot(const or_block_q8_0 *q, size_t d, const uint8_t *row) {
    size_t b = or_turbo_block_size(d), nb = d / b, cpb = b / 32;
    const uint8_t *codes = row + 2 * nb;
    float total = 0.0f;
    for (size_t bi = 0; bi < nb; bi++) total += scale_at(row, bi) * dot_chunks_x86(q + bi * cpb, codes + bi * cpb * 16, cpb);
    return total * (1.0f / 46.0f);
}

/* turbo.rs:224-250 with the x86 axpy_chunks (turbo.rs:297-311): y = fma(s, level, y) */
void or_turbo_axpy(float *y_rot, size_t d, float a, const uint8_t *row) {
    size_t b = or_turbo_block_size(d), nb = d / b;
    const uint8_t *codes = row + 2 * nb;
    for (size_t bi = 0; bi < nb; bi++) {
        float s = a * scale_at(row, bi) * (1.0f / 46.0f);
        float *yb = y_rot + bi * b;
        const uint8_t *cb = codes + bi * b / 2;
        for (size_t c = 0; c < b / 32; c++) {
            for (int k = 0; k < 16; k++) {
                yb[32 * c + k] = fmaf(s, (float)KV_LEVELS_I8[cb[16 * c + k] & 15], yb[32 * c + k]);
                yb[32 * c + 16 + k] = fmaf(s, (float)KV_LEVELS_I8[cb[16 * c + k] >> 4], yb[32 * c + 16 + k]);
            }
        }
    }
}

/* turbo.rs:253-257 */
void or_turbo_dequantize(const uint8_t *row, size_t d, uint64_t seed, float *out) {
    memset(out, 0, d * sizeof(float));
    or_turbo_axpy(out, d, 1.0f, row);
    or_turbo_rotate_inverse(out, d, seed);
}
