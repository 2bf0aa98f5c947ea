// gemv_units.hpp — one lane's share of a GGUF weight row ("unit") for the
// decode GEMV kernels: raw loads, the matching activation slice, and the exact
// per-block integer dots (kernels/mod.rs:136-232 and quant/reference.rs:221-385
// in the reference define the arithmetic).  Shared by gemv.hip and the
// attention kernel's output-projection tail.
#pragma once

#include "common.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace rie {

constexpr uint32_t M4 = 0x0F0F0F0Fu;

// 6-bit scale and min j (0..7) of a Q4_K superblock from its 12 packed bytes
// (h1,h2,h3 little-endian), get_scale_min_k4 (crates/rie-core/src/quant/reference.rs:8-16).
__device__ __forceinline__ void q4k_scale_min(uint32_t h1, uint32_t h2, uint32_t h3, int j, int &sc, int &mn) {
    const int sh = 8 * (j & 3);
    const uint32_t b1 = (h1 >> sh) & 0xff, b2 = (h2 >> sh) & 0xff, b3 = (h3 >> sh) & 0xff;
    if (j < 4) {
        sc = b1 & 63;
        mn = b2 & 63;
    } else {
        sc = (b3 & 0xF) | ((b1 >> 6) << 4);
        mn = (b3 >> 4) | ((b2 >> 6) << 4);
    }
}

// ---- per-type units --------------------------------------------------------
// A unit is what one lane loads and dots at a time:
//   Q4_0/Q4_1/Q5_0/Q5_1/Q8_0 : two 32-value blocks (36/40/44/48/68 bytes, dword aligned when K % 64 == 0)
//   Q4_K/Q5_K                : a 64-value quarter of a superblock
//   Q6_K                     : two 32-value pieces of one 128-value half n of a
//                              superblock, values 128n + 32k + [0, 32) and
//                              128n + 32k + 64 + [0, 32) (k < 2), the low and high
//                              nibbles of the same 32 ql bytes and two bit planes of
//                              the half's 32 qh bytes: a lane's loaded bytes serve
//                              both pieces
//   Q2_K/Q3_K                : a 32-value eighth of a superblock
//   F32/F16/BF16             : 8 values
template <int TY>
struct ActSlice {
    uint32_t q[16];   // int8 activation codes of the unit (8 dwords for 32-value units)
    float d0, d1;     // Q8_0: block scales; Q8_K: d0 = superblock d
    float s0, s1;     // Q8_0: d·Σq per block (Q4_1 / Q5_1 minimum term)
    int i0, i1;       // Q8_0: Σq per block (Q4_0 / Q5_0 offsets)
    int16_t bs[4];    // Q8_K: the unit's 16-value sums
    float f[8];       // f32 activations
};

template <int TY>
__device__ __forceinline__ void load_act(ActSlice<TY> &a, int u, const ActQ8 &act, const float *actf, int K, int t = 0) {
    if constexpr (TY == T_Q4_0 || TY == T_Q4_1 || TY == T_Q5_0 || TY == T_Q5_1 || TY == T_Q8_0) {
        const size_t nb = (size_t)(K >> 5), b = (size_t)t * nb + 2 * u;
        const uint4 *ap = (const uint4 *)(act.qs + (size_t)t * K + 64 * u);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = ap[i];
            a.q[4 * i] = v.x; a.q[4 * i + 1] = v.y; a.q[4 * i + 2] = v.z; a.q[4 * i + 3] = v.w;
        }
        a.d0 = act.d[b];
        a.d1 = act.d[b + 1];
        if constexpr (TY == T_Q4_0 || TY == T_Q5_0) {
            a.i0 = act.isum[b];
            a.i1 = act.isum[b + 1];
        }
        if constexpr (TY == T_Q4_1 || TY == T_Q5_1) {
            a.s0 = act.s[b];
            a.s1 = act.s[b + 1];
        }
    } else if constexpr (TY == T_Q4_K || TY == T_Q5_K) {
        const int sb = u >> 2, qi = u & 3;
        const size_t nsb = (size_t)(K >> 8);
        const uint4 *ap = (const uint4 *)(act.qs + (size_t)t * K + 256 * sb + 64 * qi);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = ap[i];
            a.q[4 * i] = v.x; a.q[4 * i + 1] = v.y; a.q[4 * i + 2] = v.z; a.q[4 * i + 3] = v.w;
        }
        a.d0 = act.d[(size_t)t * nsb + sb];
#pragma unroll
        for (int i = 0; i < 4; i++) a.bs[i] = act.bsums[(size_t)t * (K >> 4) + 16 * sb + 4 * qi + i];
    } else if constexpr (TY == T_Q6_K) {
        // unit (n, k): values 128n + 32k + [0, 32) in q[0..7], +64 in q[8..15]
        const int sb = u >> 2, n = (u >> 1) & 1, k = u & 1;
        const int8_t *base = act.qs + (size_t)t * K + 256 * sb + 128 * n + 32 * k;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint4 *ap = (const uint4 *)(base + 64 * h);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint4 v = ap[i];
                a.q[8 * h + 4 * i] = v.x; a.q[8 * h + 4 * i + 1] = v.y; a.q[8 * h + 4 * i + 2] = v.z; a.q[8 * h + 4 * i + 3] = v.w;
            }
        }
        a.d0 = act.d[(size_t)t * (K >> 8) + sb];
        const size_t bi = (size_t)t * (K >> 4) + 16 * sb + 8 * n + 2 * k;  // the 16-value sums of the two pieces
        a.bs[0] = act.bsums[bi];
        a.bs[1] = act.bsums[bi + 1];
        a.bs[2] = act.bsums[bi + 4];
        a.bs[3] = act.bsums[bi + 5];
    } else if constexpr (TY == T_Q2_K || TY == T_Q3_K) {
        // unit (n, js) covers values 128n + 32js .. +32 of its superblock
        const int sb = u >> 3, r = u & 7;
        const uint4 *ap = (const uint4 *)(act.qs + (size_t)t * K + 256 * sb + 32 * r);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint4 v = ap[i];
            a.q[4 * i] = v.x; a.q[4 * i + 1] = v.y; a.q[4 * i + 2] = v.z; a.q[4 * i + 3] = v.w;
        }
        a.d0 = act.d[(size_t)t * (K >> 8) + sb];
        a.bs[0] = act.bsums[(size_t)t * (K >> 4) + 16 * sb + 2 * r];
        a.bs[1] = act.bsums[(size_t)t * (K >> 4) + 16 * sb + 2 * r + 1];
    } else {
        const f32x4 *xp = (const f32x4 *)(actf + (size_t)t * K + 8 * u);
        const f32x4 x0 = xp[0], x1 = xp[1];
        a.f[0] = x0.x; a.f[1] = x0.y; a.f[2] = x0.z; a.f[3] = x0.w;
        a.f[4] = x1.x; a.f[5] = x1.y; a.f[6] = x1.z; a.f[7] = x1.w;
    }
}

// Raw bytes of one unit, loaded unconditionally so that the loads of all rows
// of a pass are in flight together; dot_raw does the arithmetic afterwards.
template <int TY> struct Raw;
template <> struct Raw<T_Q4_0> { uint32_t w[9]; };
template <> struct Raw<T_Q4_1> { uint32_t w[10]; };
template <> struct Raw<T_Q5_0> { uint32_t w[11]; };
template <> struct Raw<T_Q5_1> { uint32_t w[12]; };
template <> struct Raw<T_Q8_0> { uint32_t w[17]; };
template <> struct Raw<T_Q4_K> { u32x4 hdr, v0, v1; };
template <> struct Raw<T_Q5_K> { u32x4 hdr, v0, v1, h0, h1; };
template <> struct Raw<T_Q6_K> { uint32_t ql[9], qh[9], sh_l, sh_h, sc0, sc1, d; };
template <> struct Raw<T_Q2_K> { uint32_t q[8], sc, dd; };
template <> struct Raw<T_Q3_K> { uint32_t q[9], hm[9], s[4], dd, sh; };
template <> struct Raw<T_F32> { f32x4 a, b; };
template <> struct Raw<T_F16> { u32x4 a; };
template <> struct Raw<T_BF16> { u32x4 a; };

template <int TY>
__device__ __forceinline__ int units_per_row(int K) {
    if (TY == T_Q2_K || TY == T_Q3_K) return K >> 5;
    if (TY == T_F32 || TY == T_F16 || TY == T_BF16) return K >> 3;
    return K >> 6;
}

// n dwords from the dword-aligned address below p (2-byte aligned rows)
template <int N>
__device__ __forceinline__ void load_dw_a2(const uint8_t *p, uint32_t (&w)[N], uint32_t &sh) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    sh = (uint32_t)(a & 3);
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = wload(q + i);
}

template <int TY>
__device__ __forceinline__ void load_raw(const uint8_t *__restrict__ row, int u, Raw<TY> &r) {
    if constexpr (TY == T_Q4_0 || TY == T_Q4_1 || TY == T_Q5_0 || TY == T_Q5_1 || TY == T_Q8_0) {
        constexpr int UB = TY == T_Q4_0 ? 36 : TY == T_Q4_1 ? 40 : TY == T_Q5_0 ? 44 : TY == T_Q5_1 ? 48 : 68;
        const uint32_t *wp = (const uint32_t *)(row + UB * u);
#pragma unroll
        for (int i = 0; i < UB / 4; i++) r.w[i] = wload(wp + i);
    } else if constexpr (TY == T_Q4_K) {
        const int sb = u >> 2, qi = u & 3;
        const uint8_t *b = row + 144 * sb;
        r.hdr = wload((const u32x4 *)b);
        r.v0 = wload((const u32x4 *)(b + 16 + 32 * qi));
        r.v1 = wload((const u32x4 *)(b + 32 + 32 * qi));
    } else if constexpr (TY == T_Q5_K) {
        const int sb = u >> 2, qi = u & 3;
        const uint8_t *b = row + 176 * sb;
        r.hdr = wload((const u32x4 *)b);
        r.h0 = wload((const u32x4 *)(b + 16));
        r.h1 = wload((const u32x4 *)(b + 32));
        r.v0 = wload((const u32x4 *)(b + 48 + 32 * qi));
        r.v1 = wload((const u32x4 *)(b + 64 + 32 * qi));
    } else if constexpr (TY == T_Q6_K) {
        const int sb = u >> 2, n = (u >> 1) & 1, k = u & 1;
        const uint8_t *b = row + 210 * sb;
        const uintptr_t al = (uintptr_t)(b + 64 * n + 32 * k), ah = (uintptr_t)(b + 128 + 32 * n);
        const uint32_t *ql = (const uint32_t *)(al & ~(uintptr_t)3), *qh = (const uint32_t *)(ah & ~(uintptr_t)3);
#pragma unroll
        for (int i = 0; i < 9; i++) {
            r.ql[i] = wload(ql + i);
            r.qh[i] = wload(qh + i);
        }
        r.sh_l = (uint32_t)(al & 3);
        r.sh_h = (uint32_t)(ah & 3);
        r.sc0 = wload((const uint16_t *)(b + 192 + 8 * n + 2 * k));      // scales of the first piece's 16-value halves
        r.sc1 = wload((const uint16_t *)(b + 192 + 8 * n + 2 * k + 4));  // and of the second piece's
        r.d = wload((const uint16_t *)(b + 208));
    } else if constexpr (TY == T_Q2_K) {
        // 84-byte superblocks: scales[16] | q[64] | d | dmin (dword aligned when K % 512 == 0 or the row starts so)
        const int sb = u >> 3, rr = u & 7, n = rr >> 2;
        const uint8_t *b = row + 84 * sb;
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = wload((const uint32_t *)(b + 16 + 32 * n) + i);
        r.sc = wload((const uint32_t *)(b + 4 * ((8 * n + 2 * (rr & 3)) >> 2)));
        r.dd = wload((const uint32_t *)(b + 80));
    } else if constexpr (TY == T_Q3_K) {
        // 110-byte superblocks: hmask[32] | q[64] | scales[12] | d (2-byte aligned)
        const int sb = u >> 3, rr = u & 7, n = rr >> 2;
        const uint8_t *b = row + 110 * sb;
        uint32_t sh;
        load_dw_a2<9>(b + 32 + 32 * n, r.q, sh);
        load_dw_a2<9>(b, r.hm, sh);
        load_dw_a2<4>(b + 96, r.s, sh);
        r.sh = sh;
        r.dd = wload((const uint16_t *)(b + 108));
    } else if constexpr (TY == T_F32) {
        r.a = wload((const f32x4 *)(row + 32 * u));
        r.b = wload((const f32x4 *)(row + 32 * u + 16));
    } else {
        r.a = wload((const u32x4 *)(row + 16 * u));
    }
}

// 8 × 4 nibble/bit-plane values of a 32-value half → int dot with 8 activation dwords
__device__ __forceinline__ int dot8(const uint32_t (&v)[8], const uint32_t *aq) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = sdot4(v[i], aq[i], s);
    return s;
}

// bit `bit` of each byte of w, moved to bit 4 (the 16s of a 5-bit code)
__device__ __forceinline__ uint32_t bits_to_16(uint32_t w, int bit) { return ((w >> bit) & 0x01010101u) << 4; }

// Q5_0/Q5_1 high bits: bit k of qh belongs to value k of the block (k < 32)
__device__ __forceinline__ uint32_t q5_hbits(uint32_t qh, int k0) {
    const uint32_t b = (qh >> k0) & 0xFu;  // values k0..k0+3
    return ((b & 1u) << 4) | ((b & 2u) << 11) | ((b & 4u) << 18) | ((b & 8u) << 25);
}

template <int TY>
__device__ __forceinline__ float dot_raw(const Raw<TY> &r, int u, const ActSlice<TY> &a) {
    if constexpr (TY == T_Q4_0) {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
#pragma unroll
        for (int i = 0; i < 4; i++) q[4 + i] = r.w[5 + i];
        int i0 = 0, i1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            i0 = sdot4(q[i] & M4, a.q[i], i0);
            i0 = sdot4((q[i] >> 4) & M4, a.q[4 + i], i0);
            i1 = sdot4(q[4 + i] & M4, a.q[8 + i], i1);
            i1 = sdot4((q[4 + i] >> 4) & M4, a.q[12 + i], i1);
        }
        i0 -= 8 * a.i0;
        i1 -= 8 * a.i1;
        const float r0 = h2f(r.w[0] & 0xffff) * a.d0 * (float)i0;
        return fmaf(h2f(r.w[4] >> 16) * a.d1, (float)i1, r0);
    } else if constexpr (TY == T_Q4_1) {
        // blocks of 20 bytes: d, m (f16) | 16 nibble bytes; value = q·d + m (reference.rs:235-247)
        int s[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int acc = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t q = r.w[5 * h + 1 + i];
                acc = sdot4(q & M4, a.q[8 * h + i], acc);
                acc = sdot4((q >> 4) & M4, a.q[8 * h + 4 + i], acc);
            }
            s[h] = acc;
        }
        const float b0 = h2f(r.w[0] & 0xffff) * a.d0 * (float)s[0] + h2f(r.w[0] >> 16) * a.s0;
        const float b1 = h2f(r.w[5] & 0xffff) * a.d1 * (float)s[1] + h2f(r.w[5] >> 16) * a.s1;
        return b0 + b1;
    } else if constexpr (TY == T_Q5_0 || TY == T_Q5_1) {
        // Q5_0: 22 bytes d | qh (u32) | 16 nibble bytes, value q − 16 (reference.rs:249-264)
        // Q5_1: 24 bytes d, m | qh | nibbles, value q·d + m (reference.rs:266-283)
        constexpr bool M = TY == T_Q5_1;
        int s[2];
        float dw[2], mw[2] = {0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t qh, q[4];
            if constexpr (M) {
                const int o = 6 * h;
                dw[h] = h2f(r.w[o] & 0xffff);
                mw[h] = h2f(r.w[o] >> 16);
                qh = r.w[o + 1];
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = r.w[o + 2 + i];
            } else if (h == 0) {
                dw[0] = h2f(r.w[0] & 0xffff);
                qh = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], 2);
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[i + 2], r.w[i + 1], 2);
            } else {
                dw[1] = h2f(r.w[5] >> 16);
                qh = r.w[6];
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = r.w[7 + i];
            }
            int acc = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc = sdot4((q[i] & M4) | q5_hbits(qh, 4 * i), a.q[8 * h + i], acc);
                acc = sdot4(((q[i] >> 4) & M4) | q5_hbits(qh, 16 + 4 * i), a.q[8 * h + 4 + i], acc);
            }
            s[h] = acc;
        }
        if constexpr (M) {
            const float b0 = dw[0] * a.d0 * (float)s[0] + mw[0] * a.s0;
            const float b1 = dw[1] * a.d1 * (float)s[1] + mw[1] * a.s1;
            return b0 + b1;
        } else {
            const float b0 = dw[0] * a.d0 * (float)(s[0] - 16 * a.i0);
            return fmaf(dw[1] * a.d1, (float)(s[1] - 16 * a.i1), b0);
        }
    } else if constexpr (TY == T_Q8_0) {
        int i0 = 0, i1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) i0 = sdot4(__builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2), a.q[i], i0);
#pragma unroll
        for (int i = 0; i < 8; i++) i1 = sdot4(r.w[9 + i], a.q[8 + i], i1);
        const float r0 = h2f(r.w[0] & 0xffff) * a.d0 * (float)i0;
        return fmaf(h2f(r.w[8] >> 16) * a.d1, (float)i1, r0);
    } else if constexpr (TY == T_Q4_K || TY == T_Q5_K) {
        const int qi = u & 3;
        int sc[2], mn[2];
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * qi, sc[0], mn[0]);
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * qi + 1, sc[1], mn[1]);
        const uint32_t v[8] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w, r.v1.x, r.v1.y, r.v1.z, r.v1.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = v[i] & M4;
            hi[i] = (v[i] >> 4) & M4;
        }
        if constexpr (TY == T_Q5_K) {  // high bits: bit 2qi / 2qi+1 of qh[l] (reference.rs:321-350)
            const uint32_t h[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                lo[i] |= bits_to_16(h[i], 2 * qi);
                hi[i] |= bits_to_16(h[i], 2 * qi + 1);
            }
        }
        const int s1 = dot8(lo, a.q), s2 = dot8(hi, a.q + 8);
        const int sumi = s1 * sc[0] + s2 * sc[1];
        const int summ = mn[0] * ((int)a.bs[0] + a.bs[1]) + mn[1] * ((int)a.bs[2] + a.bs[3]);
        return (h2f(r.hdr.x & 0xffff) * a.d0) * (float)sumi - (h2f(r.hdr.x >> 16) * a.d0) * (float)summ;
    } else if constexpr (TY == T_Q6_K) {
        // piece 0: low nibbles and qh bits 2k, 2k+1; piece 1: high nibbles and bits
        // 2k+4, 2k+5 (q6 = nibble | 2 bits << 4, value q6 − 32: reference.rs:352-385)
        const int hs = 2 * (u & 1);
        int d0l = 0, d0h = 0, d1l = 0, d1h = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t ql = __builtin_amdgcn_alignbyte(r.ql[j + 1], r.ql[j], r.sh_l);
            const uint32_t qh = __builtin_amdgcn_alignbyte(r.qh[j + 1], r.qh[j], r.sh_h);
            const uint32_t v0 = (ql & M4) | (((qh >> hs) & 0x03030303u) << 4);
            const uint32_t v1 = ((ql >> 4) & M4) | (((qh >> (hs + 4)) & 0x03030303u) << 4);
            if (j < 4) {
                d0l = sdot4(v0, a.q[j], d0l);
                d1l = sdot4(v1, a.q[8 + j], d1l);
            } else {
                d0h = sdot4(v0, a.q[j], d0h);
                d1h = sdot4(v1, a.q[8 + j], d1h);
            }
        }
        const int sumi = (int)(int8_t)(r.sc0 & 0xff) * (d0l - 32 * a.bs[0]) + (int)(int8_t)(r.sc0 >> 8) * (d0h - 32 * a.bs[1]) +
                         (int)(int8_t)(r.sc1 & 0xff) * (d1l - 32 * a.bs[2]) + (int)(int8_t)(r.sc1 >> 8) * (d1h - 32 * a.bs[3]);
        return h2f(r.d) * a.d0 * (float)sumi;
    } else if constexpr (TY == T_Q2_K) {
        // y = d·(sc & 15)·q − dmin·(sc >> 4) per 16 values (reference.rs:101-125); unit (n, js)
        const int js = u & 3;
        const uint32_t scb = r.sc >> (8 * ((2 * js) & 3));
        const int sc0 = scb & 0xff, sc1 = (scb >> 8) & 0xff;
        int dq0 = 0, dq1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t v = (r.q[i] >> (2 * js)) & 0x03030303u;
            if (i < 4) dq0 = sdot4(v, a.q[i], dq0);
            else dq1 = sdot4(v, a.q[i], dq1);
        }
        const int sumi = (sc0 & 15) * dq0 + (sc1 & 15) * dq1;
        const int summ = (sc0 >> 4) * (int)a.bs[0] + (sc1 >> 4) * (int)a.bs[1];
        const float d = h2f(r.dd & 0xffff) * a.d0, dmin = h2f(r.dd >> 16) * a.d0;
        return d * (float)sumi - dmin * (float)summ;
    } else if constexpr (TY == T_Q3_K) {
        // y = d·(sc − 32)·(q2 − 4·(hmask bit clear)) per 16 values (reference.rs:126-152)
        const int rr = u & 7, n = rr >> 2, js = rr & 3;
        const int hb = 4 * n + js;
        int dq0 = 0, dq1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t qw = __builtin_amdgcn_alignbyte(r.q[i + 1], r.q[i], r.sh);
            const uint32_t hw = __builtin_amdgcn_alignbyte(r.hm[i + 1], r.hm[i], r.sh);
            const uint32_t v = ((qw >> (2 * js)) & 0x03030303u) | (((hw >> hb) & 0x01010101u) << 2);  // q2 + 4·h
            if (i < 4) dq0 = sdot4(v, a.q[i], dq0);
            else dq1 = sdot4(v, a.q[i], dq1);
        }
        // 6-bit scales 8n + 2js and +1 (unpack_q3k_scales, reference.rs:31-51)
        const uint32_t s0 = __builtin_amdgcn_alignbyte(r.s[1], r.s[0], r.sh);
        const uint32_t s1 = __builtin_amdgcn_alignbyte(r.s[2], r.s[1], r.sh);
        const uint32_t t = __builtin_amdgcn_alignbyte(r.s[3], r.s[2], r.sh);
        const int k = 2 * n + (js >> 1);
        const uint32_t base = (k & 1) ? s1 : s0;
        const uint32_t aux = ((base >> (4 * (k >> 1))) & 0x0f0f0f0fu) | (((t >> (2 * k)) & 0x03030303u) << 4);
        const int bsh = 8 * ((2 * js) & 3);
        const int sc0 = (int)((aux >> bsh) & 0xff) - 32, sc1 = (int)((aux >> (bsh + 8)) & 0xff) - 32;
        const int sumi = sc0 * (dq0 - 4 * a.bs[0]) + sc1 * (dq1 - 4 * a.bs[1]);
        return h2f(r.dd) * a.d0 * (float)sumi;
    } else if constexpr (TY == T_F32) {
        float s = 0.0f;
        s = fmaf(r.a.x, a.f[0], s); s = fmaf(r.a.y, a.f[1], s); s = fmaf(r.a.z, a.f[2], s); s = fmaf(r.a.w, a.f[3], s);
        s = fmaf(r.b.x, a.f[4], s); s = fmaf(r.b.y, a.f[5], s); s = fmaf(r.b.z, a.f[6], s); s = fmaf(r.b.w, a.f[7], s);
        return s;
    } else if constexpr (TY == T_BF16) {
        const uint32_t wd[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s += __uint_as_float(wd[i] << 16) * a.f[2 * i];
            s += __uint_as_float(wd[i] & 0xffff0000u) * a.f[2 * i + 1];
        }
        return s;
    } else {
        const uint32_t wd[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s = fmaf(h2f(wd[i] & 0xffff), a.f[2 * i], s);
            s = fmaf(h2f(wd[i] >> 16), a.f[2 * i + 1], s);
        }
        return s;
    }
}

}  // namespace rie
