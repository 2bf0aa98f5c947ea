/*
 * quant.c — ggml block formats, activation quantizers and int8 block dots as RIE
 * runs them on an x86 host with AVX2+FMA+F16C.
 * TEST INFRASTRUCTURE ONLY (the oracle); see oracle.h.
 *
 * Lane model of the AVX2 kernels: mul_sum_i8 (avx2.rs:38-45) yields 8 int32
 * lanes, lane j holding the products of bytes 4j..4j+3 (maddubs pairs bytes,
 * madd pairs the int16 results).  The float accumulator keeps these 8 lanes
 * apart (one _mm256_fmadd_ps per block) and hsum_ps (avx2.rs:18-26) folds them
 * as ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static inline float f16_at(const uint8_t *b, size_t off) {
    return or_f16_to_f32((uint16_t)(b[off] | ((uint16_t)b[off + 1] << 8)));
}

/* avx2.rs:18-26 */
static inline float hsum8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    float a = s0 + s2, b = s1 + s3;
    return a + b;
}

/* quant/mod.rs:70-99 */
size_t or_block_size(int ty) {
    switch (ty) {
    case OR_F32: case OR_F16: case OR_BF16: return 1;
    case OR_Q4_0: case OR_Q4_1: case OR_Q5_0: case OR_Q5_1: case OR_Q8_0: return 32;
    default: return 256;
    }
}

size_t or_block_bytes(int ty) {
    switch (ty) {
    case OR_F32: return 4;
    case OR_F16: case OR_BF16: return 2;
    case OR_Q4_0: return 18;
    case OR_Q4_1: return 20;
    case OR_Q5_0: return 22;
    case OR_Q5_1: return 24;
    case OR_Q8_0: return 34;
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    default: return 0;
    }
}

size_t or_row_bytes(int ty, size_t n) { return n / or_block_size(ty) * or_block_bytes(ty); }

/* quant/mod.rs:118-124 */
int or_act_format(int ty) {
    switch (ty) {
    case OR_Q4_0: case OR_Q4_1: case OR_Q5_0: case OR_Q5_1: case OR_Q8_0: return OR_ACT_Q8_0;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_Q2_K: case OR_Q3_K: return OR_ACT_Q8K;
    default: return OR_ACT_F32;
    }
}

/* reference.rs:8-27 */
static void unpack_k4_scales(const uint8_t *q, uint8_t sc[8], uint8_t m[8]) {
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = q[j] & 63;
            m[j] = q[j + 4] & 63;
        } else {
            sc[j] = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
            m[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
        }
    }
}

/* reference.rs:31-51 */
static void unpack_q3k_scales(const uint8_t *s, int8_t out[16]) {
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    for (int i = 0; i < 3; i++)
        aux[i] = (uint32_t)s[4 * i] | ((uint32_t)s[4 * i + 1] << 8) | ((uint32_t)s[4 * i + 2] << 16) | ((uint32_t)s[4 * i + 3] << 24);
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | ((tmp & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    for (int i = 0; i < 4; i++)
        for (int k = 0; k < 4; k++) out[4 * i + k] = (int8_t)((uint8_t)(aux[i] >> (8 * k)) - 32);
}

/* reference.rs:53-215 */
static void dequantize_block(int ty, const uint8_t *b, float *y) {
    switch (ty) {
    case OR_Q4_0: {
        float d = f16_at(b, 0);
        const uint8_t *qs = b + 2;
        for (int j = 0; j < 16; j++) {
            y[j] = (float)((int)(qs[j] & 0xF) - 8) * d;
            y[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
        }
        break;
    }
    case OR_Q4_1: {
        float d = f16_at(b, 0), m = f16_at(b, 2);
        const uint8_t *qs = b + 4;
        for (int j = 0; j < 16; j++) {
            y[j] = (float)(qs[j] & 0xF) * d + m;
            y[j + 16] = (float)(qs[j] >> 4) * d + m;
        }
        break;
    }
    case OR_Q5_0: {
        float d = f16_at(b, 0);
        uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        const uint8_t *qs = b + 6;
        for (int j = 0; j < 16; j++) {
            uint32_t xh0 = ((qh >> j) << 4) & 0x10u;
            uint32_t xh1 = (qh >> (j + 12)) & 0x10u;
            y[j] = (float)((int)(((uint32_t)qs[j] & 0xFu) | xh0) - 16) * d;
            y[j + 16] = (float)((int)(((uint32_t)qs[j] >> 4) | xh1) - 16) * d;
        }
        break;
    }
    case OR_Q5_1: {
        float d = f16_at(b, 0), m = f16_at(b, 2);
        uint32_t qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
        const uint8_t *qs = b + 8;
        for (int j = 0; j < 16; j++) {
            uint32_t xh0 = ((qh >> j) << 4) & 0x10u;
            uint32_t xh1 = (qh >> (j + 12)) & 0x10u;
            y[j] = (float)(((uint32_t)qs[j] & 0xFu) | xh0) * d + m;
            y[j + 16] = (float)(((uint32_t)qs[j] >> 4) | xh1) * d + m;
        }
        break;
    }
    case OR_Q8_0: {
        float d = f16_at(b, 0);
        for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
        break;
    }
    case OR_Q2_K: {
        const uint8_t *scales = b, *q0 = b + 16;
        float d = f16_at(b, 80), min = f16_at(b, 82);
        int yi = 0, is = 0;
        for (int n = 0; n < 2; n++) {
            const uint8_t *q = q0 + n * 32;
            int shift = 0;
            for (int k = 0; k < 4; k++) {
                for (int half = 0; half < 2; half++) {
                    uint8_t sc = scales[is++];
                    float dl = d * (float)(sc & 0xF);
                    float ml = min * (float)(sc >> 4);
                    for (int l = 0; l < 16; l++) y[yi++] = dl * (float)((q[l + 16 * half] >> shift) & 3) - ml;
                }
                shift += 2;
            }
        }
        break;
    }
    case OR_Q3_K: {
        const uint8_t *hm = b, *q0 = b + 32;
        int8_t scales[16];
        unpack_q3k_scales(b + 96, scales);
        float d_all = f16_at(b, 108);
        uint8_t m = 1;
        int is = 0, yi = 0;
        for (int n = 0; n < 2; n++) {
            const uint8_t *q = q0 + n * 32;
            int shift = 0;
            for (int k = 0; k < 4; k++) {
                for (int half = 0; half < 2; half++) {
                    float dl = d_all * (float)scales[is++];
                    for (int l = 0; l < 16; l++) {
                        int idx = l + 16 * half;
                        int v = (int)((q[idx] >> shift) & 3) - ((hm[idx] & m) ? 0 : 4);
                        y[yi++] = dl * (float)v;
                    }
                }
                shift += 2;
                m = (uint8_t)(m << 1);
            }
        }
        break;
    }
    case OR_Q4_K: {
        float d = f16_at(b, 0), min = f16_at(b, 2);
        uint8_t sc[8], mn[8];
        unpack_k4_scales(b + 4, sc, mn);
        const uint8_t *q = b + 16;
        for (int j = 0; j < 4; j++) {
            float d1 = d * (float)sc[2 * j], m1 = min * (float)mn[2 * j];
            float d2 = d * (float)sc[2 * j + 1], m2 = min * (float)mn[2 * j + 1];
            for (int l = 0; l < 32; l++) {
                y[64 * j + l] = d1 * (float)(q[32 * j + l] & 0xF) - m1;
                y[64 * j + 32 + l] = d2 * (float)(q[32 * j + l] >> 4) - m2;
            }
        }
        break;
    }
    case OR_Q5_K: {
        float d = f16_at(b, 0), min = f16_at(b, 2);
        uint8_t sc[8], mn[8];
        unpack_k4_scales(b + 4, sc, mn);
        const uint8_t *qh = b + 16, *ql = b + 48;
        for (int j = 0; j < 4; j++) {
            float d1 = d * (float)sc[2 * j], m1 = min * (float)mn[2 * j];
            float d2 = d * (float)sc[2 * j + 1], m2 = min * (float)mn[2 * j + 1];
            uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
            for (int l = 0; l < 32; l++) {
                int h1 = (qh[l] & u1) ? 16 : 0, h2 = (qh[l] & u2) ? 16 : 0;
                y[64 * j + l] = d1 * (float)((ql[32 * j + l] & 0xF) + h1) - m1;
                y[64 * j + 32 + l] = d2 * (float)((ql[32 * j + l] >> 4) + h2) - m2;
            }
        }
        break;
    }
    case OR_Q6_K: {
        float d = f16_at(b, 208);
        for (int n = 0; n < 2; n++) {
            const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
            float *yy = y + 128 * n;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                yy[l] = d * (float)(int8_t)sc[is] * (float)q1;
                yy[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
                yy[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
                yy[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
            }
        }
        break;
    }
    default: break;
    }
}

/* quant/mod.rs:221-249 */
void or_dequantize_row(int ty, const uint8_t *src, float *dst, size_t n) {
    switch (ty) {
    case OR_F32:
        memcpy(dst, src, n * 4);
        return;
    case OR_F16:
        for (size_t i = 0; i < n; i++) dst[i] = or_f16_to_f32((uint16_t)(src[2 * i] | ((uint16_t)src[2 * i + 1] << 8)));
        return;
    case OR_BF16:
        for (size_t i = 0; i < n; i++) {
            uint32_t bits = ((uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 8)) << 16;
            memcpy(&dst[i], &bits, 4);
        }
        return;
    default: {
        size_t bs = or_block_size(ty), bb = or_block_bytes(ty);
        for (size_t i = 0; i < n / bs; i++) dequantize_block(ty, src + i * bb, dst + i * bs);
    }
    }
}

/* AVX2 quantizer, avx2.rs:153-184: amax by max_ps, d = amax/127, RNE conversion
 * (_mm256_cvtps_epi32 under the default MXCSR mode), clamp to ±127, and
 * s = d * Σ of the *unclamped* converted values. */
void or_quantize_q8_0(const float *x, or_block_q8_0 *out, size_t nb) {
    for (size_t bi = 0; bi < nb; bi++) {
        const float *p = x + bi * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(p[i]);
            amax = a > amax ? a : amax;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        int32_t isum = 0;
        for (int i = 0; i < 32; i++) {
            int32_t q = (int32_t)rintf(p[i] * id);
            isum += q;
            out[bi].qs[i] = (int8_t)(q < -127 ? -127 : (q > 127 ? 127 : q));
        }
        out[bi].d = d;
        out[bi].s = d * (float)isum;
    }
}

/* quant/mod.rs:175-189 (forced-scalar path, round half away from zero). */
void or_quantize_q8_0_scalar(const float *x, or_block_q8_0 *out, size_t nb) {
    for (size_t bi = 0; bi < nb; bi++) {
        const float *p = x + bi * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(p[i]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        int32_t sum = 0;
        for (int i = 0; i < 32; i++) {
            int32_t r = (int32_t)roundf(p[i] * id);
            r = r < -127 ? -127 : (r > 127 ? 127 : r);
            out[bi].qs[i] = (int8_t)r;
            sum += r;
        }
        out[bi].d = d;
        out[bi].s = d * (float)sum;
    }
}

/* quant/mod.rs:191-218: first strictly-largest |x| sets the signed max,
 * iscale = -127/max, round half away from zero, i16 bsums over 16, d = 1/iscale. */
void or_quantize_q8_k(const float *x, or_block_q8k *out, size_t nb) {
    for (size_t bi = 0; bi < nb; bi++) {
        const float *p = x + bi * 256;
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < 256; i++) {
            float a = fabsf(p[i]);
            if (a > amax) {
                amax = a;
                max = p[i];
            }
        }
        if (amax == 0.0f) {
            memset(&out[bi], 0, sizeof(or_block_q8k));
            continue;
        }
        float iscale = -127.0f / max;
        for (int i = 0; i < 256; i++) {
            int32_t r = (int32_t)roundf(iscale * p[i]);
            out[bi].qs[i] = (int8_t)(r < -127 ? -127 : (r > 127 ? 127 : r));
        }
        for (int j = 0; j < 16; j++) {
            int16_t s = 0;
            for (int i = 0; i < 16; i++) s = (int16_t)(s + out[bi].qs[j * 16 + i]);
            out[bi].bsums[j] = s;
        }
        out[bi].d = 1.0f / iscale;
    }
}

/* quantize::q4_0, quant/mod.rs:279-298 */
void or_quantize_weights_q4_0(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float max = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(xb[i]) > fabsf(max)) max = xb[i];
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = or_f32_to_f16(d);
        uint8_t *o = out + b * 18;
        o[0] = (uint8_t)h;
        o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; j++) {
            int q0 = (int)(xb[j] * id + 8.5f), q1 = (int)(xb[j + 16] * id + 8.5f);
            q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
            q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
            o[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* quantize::q8_0, quant/mod.rs:265-277 */
void or_quantize_weights_q8_0(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = or_f32_to_f16(d);
        uint8_t *o = out + b * 34;
        o[0] = (uint8_t)h;
        o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) {
            int r = (int)roundf(xb[j] * id);
            r = r < -127 ? -127 : (r > 127 ? 127 : r);
            o[2 + j] = (uint8_t)(int8_t)r;
        }
    }
}

/* ---------------------------------------------------------------------------
 * int8 block dots
 * ------------------------------------------------------------------------- */

/* avx2.rs:47-76: per-lane FMA of (d_w*d_a) with the lane's int32 partial. */
static float dot_q8_0_x86(const uint8_t *w, const or_block_q8_0 *a, size_t nb, int q4) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t bb = q4 ? 18 : 34;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * bb;
        int x[32];
        if (q4) {
            for (int j = 0; j < 16; j++) {
                x[j] = (int)(b[2 + j] & 0xF) - 8;
                x[j + 16] = (int)(b[2 + j] >> 4) - 8;
            }
        } else {
            for (int j = 0; j < 32; j++) x[j] = (int8_t)b[2 + j];
        }
        float d = f16_at(b, 0) * a[i].d;
        for (int l = 0; l < 8; l++) {
            int32_t s = x[4 * l] * a[i].qs[4 * l] + x[4 * l + 1] * a[i].qs[4 * l + 1] + x[4 * l + 2] * a[i].qs[4 * l + 2] +
                        x[4 * l + 3] * a[i].qs[4 * l + 3];
            acc[l] = fmaf(d, (float)s, acc[l]);
        }
    }
    return hsum8(acc);
}

static int32_t idot_q4_0(const uint8_t *b, const int8_t *aq) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        s += ((int)(b[2 + j] & 0xF) - 8) * aq[j];
        s += ((int)(b[2 + j] >> 4) - 8) * aq[j + 16];
    }
    return s;
}

static int32_t idot_q4_1(const uint8_t *b, const int8_t *aq) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        s += (int)(b[4 + j] & 0xF) * aq[j];
        s += (int)(b[4 + j] >> 4) * aq[j + 16];
    }
    return s;
}

static int32_t idot_q5(const uint8_t *b, const int8_t *aq, int with_min) {
    uint32_t qh;
    const uint8_t *qs;
    int off = with_min ? 0 : 16;
    if (with_min) {
        qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
        qs = b + 8;
    } else {
        qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        qs = b + 6;
    }
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
        s += ((int)(((uint32_t)qs[j] & 0xFu) | xh0) - off) * aq[j];
        s += ((int)(((uint32_t)qs[j] >> 4) | xh1) - off) * aq[j + 16];
    }
    return s;
}

static int32_t idot_q8_0(const uint8_t *b, const int8_t *aq) {
    int32_t s = 0;
    for (int j = 0; j < 32; j++) s += (int8_t)b[2 + j] * aq[j];
    return s;
}

/* reference.rs:295-319 integer parts: sumi = Σ sc·Σq·a, summ = Σ m·(bsum pair) */
static void idot_q4_k(const uint8_t *b, const or_block_q8k *a, int32_t *sumi_out, int32_t *summ_out) {
    uint8_t sc[8], mn[8];
    unpack_k4_scales(b + 4, sc, mn);
    const uint8_t *q = b + 16;
    int32_t sumi = 0, summ = 0;
    for (int j = 0; j < 4; j++) {
        int32_t s1 = 0, s2 = 0;
        for (int l = 0; l < 32; l++) {
            s1 += (int)(q[32 * j + l] & 0xF) * a->qs[64 * j + l];
            s2 += (int)(q[32 * j + l] >> 4) * a->qs[64 * j + 32 + l];
        }
        sumi += s1 * sc[2 * j] + s2 * sc[2 * j + 1];
    }
    for (int j = 0; j < 8; j++) summ += ((int32_t)a->bsums[2 * j] + a->bsums[2 * j + 1]) * mn[j];
    *sumi_out = sumi;
    *summ_out = summ;
}

static void idot_q5_k(const uint8_t *b, const or_block_q8k *a, int32_t *sumi_out, int32_t *summ_out) {
    uint8_t sc[8], mn[8];
    unpack_k4_scales(b + 4, sc, mn);
    const uint8_t *qh = b + 16, *ql = b + 48;
    int32_t sumi = 0, summ = 0;
    for (int j = 0; j < 4; j++) {
        uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        int32_t s1 = 0, s2 = 0;
        for (int l = 0; l < 32; l++) {
            int h1 = (qh[l] & u1) ? 16 : 0, h2 = (qh[l] & u2) ? 16 : 0;
            s1 += ((int)(ql[32 * j + l] & 0xF) + h1) * a->qs[64 * j + l];
            s2 += ((int)(ql[32 * j + l] >> 4) + h2) * a->qs[64 * j + 32 + l];
        }
        sumi += s1 * sc[2 * j] + s2 * sc[2 * j + 1];
    }
    for (int j = 0; j < 8; j++) summ += ((int32_t)a->bsums[2 * j] + a->bsums[2 * j + 1]) * mn[j];
    *sumi_out = sumi;
    *summ_out = summ;
}

/* reference.rs:352-385 integer part (the AVX2 form avx2.rs:109-151 computes the
 * same integer via Σ sc·Σ q6u·a − 32·Σ sc·bsum). */
static int32_t idot_q6_k(const uint8_t *b, const or_block_q8k *a) {
    int32_t sumi = 0;
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
        const int8_t *aq = a->qs + 128 * n;
        int32_t g[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            g[is] += q1 * aq[l];
            g[is + 2] += q2 * aq[l + 32];
            g[is + 4] += q3 * aq[l + 64];
            g[is + 6] += q4 * aq[l + 96];
        }
        for (int k = 0; k < 8; k++) sumi += g[k] * (int8_t)sc[k];
    }
    return sumi;
}

/* avx2.rs:186-203 */
float or_dot_f32(const float *a, const float *b, size_t n) {
    float acc0[8] = {0}, acc1[8] = {0};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; l++) {
            acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
            acc1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], acc1[l]);
        }
    float t[8];
    for (int l = 0; l < 8; l++) t[l] = acc0[l] + acc1[l];
    float s = hsum8(t);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* avx2.rs:205-224 */
float or_dot_f16_f32(const uint16_t *a, const float *b, size_t n) {
    float acc0[8] = {0}, acc1[8] = {0};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; l++) {
            acc0[l] = fmaf(or_f16_to_f32(a[i + l]), b[i + l], acc0[l]);
            acc1[l] = fmaf(or_f16_to_f32(a[i + 8 + l]), b[i + 8 + l], acc1[l]);
        }
    float t[8];
    for (int l = 0; l < 8; l++) t[l] = acc0[l] + acc1[l];
    float s = hsum8(t);
    for (; i < n; i++) s += or_f16_to_f32(a[i]) * b[i];
    return s;
}

/* avx2.rs:226-241 */
void or_axpy_f16(float *y, float alpha, const uint16_t *x, size_t n) {
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) y[i + l] = fmaf(or_f16_to_f32(x[i + l]), alpha, y[i + l]);
    for (; i < n; i++) y[i] += alpha * or_f16_to_f32(x[i]);
}

/* kernels/mod.rs:136-232 on an AVX2+FMA+F16C host. */
float or_vec_dot(int ty, const uint8_t *w, const void *act, size_t n) {
    switch (ty) {
    case OR_F32: {
        /* dot_f32_bytes (kernels/mod.rs:332-343): the aligned case (GGUF data is
         * 32-byte aligned) goes to the AVX2 dot_f32. */
        const float *x = (const float *)act;
        if (((uintptr_t)w & 3u) == 0) return or_dot_f32((const float *)(const void *)w, x, n);
        float s = 0.0f;
        for (size_t i = 0; i < n; i++) {
            float v;
            memcpy(&v, w + 4 * i, 4);
            s += v * x[i];
        }
        return s;
    }
    case OR_F16:
        return or_dot_f16_f32((const uint16_t *)(const void *)w, (const float *)act, n);
    case OR_BF16: {
        const float *x = (const float *)act;
        float s = 0.0f;
        for (size_t i = 0; i < n; i++) {
            uint32_t bits = ((uint32_t)w[2 * i] | ((uint32_t)w[2 * i + 1] << 8)) << 16;
            float v;
            memcpy(&v, &bits, 4);
            s += v * x[i];
        }
        return s;
    }
    case OR_Q8_0:
        return dot_q8_0_x86(w, (const or_block_q8_0 *)act, n / 32, 0);
    case OR_Q4_0:
        return dot_q8_0_x86(w, (const or_block_q8_0 *)act, n / 32, 1);
    case OR_Q4_1: { /* reference.rs:235-247 */
        const or_block_q8_0 *a = (const or_block_q8_0 *)act;
        float sum = 0.0f;
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = w + i * 20;
            int32_t s = idot_q4_1(b, a[i].qs);
            sum += f16_at(b, 0) * a[i].d * (float)s + f16_at(b, 2) * a[i].s;
        }
        return sum;
    }
    case OR_Q5_0: { /* reference.rs:249-264 */
        const or_block_q8_0 *a = (const or_block_q8_0 *)act;
        float sum = 0.0f;
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = w + i * 22;
            sum += f16_at(b, 0) * a[i].d * (float)idot_q5(b, a[i].qs, 0);
        }
        return sum;
    }
    case OR_Q5_1: { /* reference.rs:266-281 */
        const or_block_q8_0 *a = (const or_block_q8_0 *)act;
        float sum = 0.0f;
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = w + i * 24;
            sum += f16_at(b, 0) * a[i].d * (float)idot_q5(b, a[i].qs, 1) + f16_at(b, 2) * a[i].s;
        }
        return sum;
    }
    case OR_Q4_K: { /* avx2.rs:78-107 */
        const or_block_q8k *a = (const or_block_q8k *)act;
        float sum = 0.0f;
        for (size_t i = 0; i < n / 256; i++) {
            const uint8_t *b = w + i * 144;
            float d = f16_at(b, 0) * a[i].d;
            float dmin = f16_at(b, 2) * a[i].d;
            int32_t sumi, summ;
            idot_q4_k(b, &a[i], &sumi, &summ);
            sum += d * (float)sumi - dmin * (float)summ;
        }
        return sum;
    }
    case OR_Q5_K: { /* reference.rs:321-350 */
        const or_block_q8k *a = (const or_block_q8k *)act;
        float sum = 0.0f;
        for (size_t i = 0; i < n / 256; i++) {
            const uint8_t *b = w + i * 176;
            float d = f16_at(b, 0) * a[i].d;
            float dmin = f16_at(b, 2) * a[i].d;
            int32_t sumi, summ;
            idot_q5_k(b, &a[i], &sumi, &summ);
            sum += d * (float)sumi - dmin * (float)summ;
        }
        return sum;
    }
    case OR_Q6_K: { /* avx2.rs:109-151 */
        const or_block_q8k *a = (const or_block_q8k *)act;
        float sum = 0.0f;
        for (size_t i = 0; i < n / 256; i++) {
            const uint8_t *b = w + i * 210;
            float d = f16_at(b, 208) * a[i].d;
            sum += d * (float)idot_q6_k(b, &a[i]);
        }
        return sum;
    }
    case OR_Q2_K:
    case OR_Q3_K: { /* reference.rs:388-401 */
        const or_block_q8k *a = (const or_block_q8k *)act;
        size_t bb = or_block_bytes(ty);
        float tmp[256];
        float sum = 0.0f;
        for (size_t i = 0; i < n / 256; i++) {
            dequantize_block(ty, w + i * bb, tmp);
            float s = 0.0f;
            for (int j = 0; j < 256; j++) s += tmp[j] * (float)a[i].qs[j];
            sum += s * a[i].d;
        }
        return sum;
    }
    default:
        return 0.0f;
    }
}

void or_block_idots(int ty, const uint8_t *w, const void *act, size_t n, int32_t *out) {
    size_t bb = or_block_bytes(ty);
    if (or_block_size(ty) == 32) {
        const or_block_q8_0 *a = (const or_block_q8_0 *)act;
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = w + i * bb;
            switch (ty) {
            case OR_Q4_0: out[i] = idot_q4_0(b, a[i].qs); break;
            case OR_Q4_1: out[i] = idot_q4_1(b, a[i].qs); break;
            case OR_Q5_0: out[i] = idot_q5(b, a[i].qs, 0); break;
            case OR_Q5_1: out[i] = idot_q5(b, a[i].qs, 1); break;
            default: out[i] = idot_q8_0(b, a[i].qs); break;
            }
        }
    } else {
        const or_block_q8k *a = (const or_block_q8k *)act;
        for (size_t i = 0; i < n / 256; i++) {
            const uint8_t *b = w + i * bb;
            int32_t sumi = 0, summ = 0;
            if (ty == OR_Q4_K) idot_q4_k(b, &a[i], &sumi, &summ);
            else if (ty == OR_Q5_K) idot_q5_k(b, &a[i], &sumi, &summ);
            else if (ty == OR_Q6_K) sumi = idot_q6_k(b, &a[i]);
            out[2 * i] = sumi;
            out[2 * i + 1] = summ;
        }
    }
}
