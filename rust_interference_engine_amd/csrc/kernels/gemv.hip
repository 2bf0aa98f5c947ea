// gemv.hip — decode matrix-vector products of ggml-block weights with int8
// activations (kernels/mod.rs:136-232 and quant/reference.rs:221-385 in the
// reference define the arithmetic), written for CDNA4 wavefronts.
//
// Weights stay in their native GGUF block bytes in HBM.  Each row is split into
// "units" that a lane can load with dword-aligned vector loads and reduce with
// v_dot4_i32_i8 (sdot4):
//   Q4_0 / Q8_0 : a pair of 32-blocks (36 / 68 bytes, dword aligned when K%64==0)
//   Q4_K        : one 64-value quarter of a 256-superblock (16-byte aligned)
//   Q6_K        : one 32-value eighth of a 210-byte superblock (2-byte aligned,
//                 realigned with v_alignbyte)
// LPR lanes of a wavefront share a row (64/LPR rows per wave), every weight byte
// is loaded once per launch (plain loads: see wload), and a lane's partial sums
// are reduced across the LPR lanes through LDS and cross-lane shuffles.  Per-block integer dot products are exact;
// only the float accumulation order differs from the CPU path.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"

#include <algorithm>
#include <cstdlib>

namespace rie {

constexpr int MAXT = 4;  // tokens processed per weight load
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

struct SegP {
    const uint8_t *w;
    size_t rb;
    int rows;
    float *out;
    int ld;
    int epi;
};

struct GemvP {
    SegP seg[3];
    int nseg;
    int total_rows;
    ActQ8 act;
    const float *actf;
    int n_tok, K;
    int glu;  // 0 none, 1 silu, 2 gelu-tanh (seg[0] = gate, seg[1] = up)
};

// ---------------------------------------------------------------------------
// Single-token decode GEMV.  A workgroup owns TR consecutive rows; LPR lanes
// (16..256) share a row so that each lane holds UPL ≤ 2 units.  The lane's
// activation slice is loaded into registers once and reused for every row of
// the workgroup; per-lane partial sums go to a padded LDS tile
// [row][LPR+DEC_PAD] and 8 threads per row add them.
// GLU: gate and up rows give h = act(g)·u, optionally quantized to Q8_0 in the
// epilogue (32 rows per half-wave) for the down projection.
// ---------------------------------------------------------------------------
struct DecP {
    SegP seg[3];
    int nseg, total_rows, K;
    int tr;          // rows per workgroup; a workgroup never spans two segments
    int blk_end[3];  // cumulative workgroup count at the end of each segment
    ActQ8 act;
    const float *actf;
    int glu;         // 0 none, 1 silu, 2 gelu
    ActQ8 hq;        // GLU: Q8_0 output of h when hq.qs != nullptr
    NormIn nin;      // nin.x != nullptr: the activation is RMSNorm(x)·w, quantized here
    // routed experts: seg 0 (and seg 1 for GLU) hold the stacked expert matrices;
    // rows [j·slot_rows, (j+1)·slot_rows) of the launch are rows of expert xsel[j]
    const int *xsel;
    int slot_rows;
    int act_per_slot;  // slot j reads activation row j (the down projection of expert j's hidden)
};

// ---- per-type units --------------------------------------------------------
// A unit is what one lane loads and dots at a time:
//   Q4_0/Q4_1/Q5_0/Q5_1/Q8_0 : two 32-value blocks (36/40/44/48/68 bytes, dword aligned when K % 64 == 0)
//   Q4_K/Q5_K                : a 64-value quarter of a superblock
//   Q2_K/Q3_K/Q6_K           : a 32-value eighth of a superblock
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
        const int sb = u >> 3, r = u & 7, n = r >> 2, k = r & 3;
        const uint4 *ap = (const uint4 *)(act.qs + (size_t)t * K + 256 * sb + 128 * n + 32 * k);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint4 v = ap[i];
            a.q[4 * i] = v.x; a.q[4 * i + 1] = v.y; a.q[4 * i + 2] = v.z; a.q[4 * i + 3] = v.w;
        }
        a.d0 = act.d[(size_t)t * (K >> 8) + sb];
        a.bs[0] = act.bsums[(size_t)t * (K >> 4) + 16 * sb + 8 * n + 2 * k];
        a.bs[1] = act.bsums[(size_t)t * (K >> 4) + 16 * sb + 8 * n + 2 * k + 1];
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
template <> struct Raw<T_Q6_K> { uint32_t ql[9], qh[9], sh_l, sh_h, scw, d; };
template <> struct Raw<T_Q2_K> { uint32_t q[8], sc, dd; };
template <> struct Raw<T_Q3_K> { uint32_t q[9], hm[9], s[4], dd, sh; };
template <> struct Raw<T_F32> { f32x4 a, b; };
template <> struct Raw<T_F16> { u32x4 a; };
template <> struct Raw<T_BF16> { u32x4 a; };

template <int TY>
__device__ __forceinline__ int units_per_row(int K) {
    if (TY == T_Q6_K || TY == T_Q2_K || TY == T_Q3_K) return K >> 5;
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
        const int sb = u >> 3, rr = u & 7, n = rr >> 2, k = rr & 3;
        const uint8_t *b = row + 210 * sb;
        const uintptr_t al = (uintptr_t)(b + 64 * n + 32 * (k & 1)), ah = (uintptr_t)(b + 128 + 32 * n);
        const uint32_t *ql = (const uint32_t *)(al & ~(uintptr_t)3), *qh = (const uint32_t *)(ah & ~(uintptr_t)3);
#pragma unroll
        for (int i = 0; i < 9; i++) {
            r.ql[i] = wload(ql + i);
            r.qh[i] = wload(qh + i);
        }
        r.sh_l = (uint32_t)(al & 3);
        r.sh_h = (uint32_t)(ah & 3);
        r.scw = wload((const uint16_t *)(b + 192 + 8 * n + 2 * k));
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
        const int k = u & 3;
        const int sh = k >= 2 ? 4 : 0, hs = 2 * k;
        int dl = 0, dh = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t ql = __builtin_amdgcn_alignbyte(r.ql[j + 1], r.ql[j], r.sh_l);
            const uint32_t qh = __builtin_amdgcn_alignbyte(r.qh[j + 1], r.qh[j], r.sh_h);
            const uint32_t v = ((ql >> sh) & M4) | (((qh >> hs) & 0x03030303u) << 4);
            if (j < 4) dl = sdot4(v, a.q[j], dl);
            else dh = sdot4(v, a.q[j], dh);
        }
        const int sumi = (int)(int8_t)(r.scw & 0xff) * (dl - 32 * a.bs[0]) + (int)(int8_t)(r.scw >> 8) * (dh - 32 * a.bs[1]);
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

// ---------------------------------------------------------------------------
// Small-batch GEMV (2 ≤ n_tok ≤ 8, and prompt batches of types without an MFMA
// kernel): LPR lanes share a row, each unit's weight bytes are loaded once and
// dotted with up to MAXT tokens' activations.
// ---------------------------------------------------------------------------
template <int TY, int LPR>
__global__ __launch_bounds__(256) void gemv_kernel(GemvP p) {
    constexpr int RPW = 64 / LPR;  // rows per wavefront
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, l = lane % LPR;
    const int n_waves = gridDim.x * 4;
    const int U = units_per_row<TY>(p.K);
    for (int rg = blockIdx.x * 4 + (threadIdx.x >> 6); rg * RPW < p.total_rows; rg += n_waves) {
        const int r = rg * RPW + sub;
        const bool valid = r < p.total_rows;
        // segment lookup without dynamic indexing of the kernel-argument struct
        int rr = r;
        const uint8_t *sw = p.seg[0].w;
        size_t srb = p.seg[0].rb;
        float *sout = p.seg[0].out;
        int sld = p.seg[0].ld, sepi = p.seg[0].epi;
        if (!p.glu && p.nseg > 1 && rr >= p.seg[0].rows) {
            rr -= p.seg[0].rows;
            if (p.nseg > 2 && rr >= p.seg[1].rows) {
                rr -= p.seg[1].rows;
                sw = p.seg[2].w; srb = p.seg[2].rb; sout = p.seg[2].out; sld = p.seg[2].ld; sepi = p.seg[2].epi;
            } else {
                sw = p.seg[1].w; srb = p.seg[1].rb; sout = p.seg[1].out; sld = p.seg[1].ld; sepi = p.seg[1].epi;
            }
        }
        for (int t0 = 0; t0 < p.n_tok; t0 += MAXT) {
            const int nt = min(MAXT, p.n_tok - t0);
            float acc[MAXT] = {0.f, 0.f, 0.f, 0.f};
            float acc2[MAXT] = {0.f, 0.f, 0.f, 0.f};
            if (valid) {
                const uint8_t *row = sw + (size_t)rr * srb;
                const uint8_t *row2 = p.glu ? p.seg[1].w + (size_t)rr * p.seg[1].rb : nullptr;
                for (int u = l; u < U; u += LPR) {
                    Raw<TY> w1, w2;
                    load_raw<TY>(row, u, w1);
                    if (p.glu) load_raw<TY>(row2, u, w2);
#pragma unroll
                    for (int tt = 0; tt < MAXT; tt++) {
                        if (tt >= nt) break;
                        ActSlice<TY> a;
                        load_act<TY>(a, u, p.act, p.actf, p.K, t0 + tt);
                        acc[tt] += dot_raw<TY>(w1, u, a);
                        if (p.glu) acc2[tt] += dot_raw<TY>(w2, u, a);
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < MAXT; tt++) {
                acc[tt] = wave_sum(acc[tt], LPR);
                if (p.glu) acc2[tt] = wave_sum(acc2[tt], LPR);
            }
            if (valid && l == 0) {
#pragma unroll
                for (int tt = 0; tt < MAXT; tt++) {
                    if (tt >= nt) break;
                    float *o = sout + (size_t)(t0 + tt) * sld + rr;
                    if (p.glu) {
                        const float g = acc[tt];
                        *o = (p.glu == 2 ? gelu_tanh_f(g) : silu_f(g)) * acc2[tt];
                    } else if (sepi == EPI_ADD) {
                        *o += acc[tt];
                    } else {
                        *o = acc[tt];
                    }
                }
            }
        }
    }
}

// rows whose loads a wave keeps in flight together (register budget ≈ R × unit bytes)
#ifndef RIE_DEC_ROWS_SMALL
#define RIE_DEC_ROWS_SMALL 4  // units of ≤ 48 bytes: Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q4_K, F16, BF16
#endif
#ifndef RIE_DEC_ROWS_LARGE
#define RIE_DEC_ROWS_LARGE 2  // Q8_0, Q3_K, Q5_K, Q6_K, F32
#endif
template <int TY>
constexpr int dec_rows_per_pass() {
    return (TY == T_Q8_0 || TY == T_Q6_K || TY == T_F32 || TY == T_Q5_K || TY == T_Q3_K) ? RIE_DEC_ROWS_LARGE : RIE_DEC_ROWS_SMALL;
}

constexpr int DEC_PAD = 8;  // LDS row padding of the partial-sum tile

// NT threads (256 or 512): one pass of NT/LPR row groups × R rows covers a
// 32-row tile in a single pass (all of a workgroup's loads issued up front).
template <int TY, int LPR, int UPL, bool GLU, int R, int NT>
__global__ __launch_bounds__(NT) void gemv_dec_kernel(DecP p) {
    constexpr int GROUPS = NT / LPR;
    constexpr int STRIDE = LPR + DEC_PAD;
    constexpr int NW = GLU ? 2 : 1;
    extern __shared__ float red[];  // [NW][tr][STRIDE], then tr floats of h
    const int tid = threadIdx.x;
    const int grp = LPR >= 64 ? __builtin_amdgcn_readfirstlane(tid / LPR) : tid / LPR;
    const int l = tid % LPR;
    const int U = units_per_row<TY>(p.K);
    ActSlice<TY> a[UPL];
    bool valid[UPL];
    int uu[UPL];
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        valid[k] = l + LPR * k < U;
        uu[k] = valid[k] ? l + LPR * k : U - 1;  // idle lanes load a real unit and drop it
    }
    // workgroup → (segment, first row): uniform, so the segment's fields are scalar
    const int bid = blockIdx.x;
    const int sg = (!GLU && p.nseg > 1 && bid >= p.blk_end[0]) ? ((p.nseg > 2 && bid >= p.blk_end[1]) ? 2 : 1) : 0;
    const int row0 = (bid - (sg ? p.blk_end[sg - 1] : 0)) * p.tr;
    const int seg_rows = p.seg[sg].rows;
    const int last = seg_rows - 1;
    const uint8_t *wbase = p.seg[sg].w;
    const uint8_t *wbase2 = GLU ? p.seg[1].w : nullptr;
    const size_t rb = p.seg[sg].rb;
    int slot = 0;
    if (p.xsel) {  // a workgroup's rows lie in one slot (slot_rows is a multiple of the tile)
        slot = row0 / p.slot_rows;
        const size_t off = ((size_t)p.xsel[slot] - (size_t)slot) * (size_t)p.slot_rows * rb;
        wbase += off;
        if constexpr (GLU) wbase2 += ((size_t)p.xsel[slot] - (size_t)slot) * (size_t)p.slot_rows * p.seg[1].rb;
    }
    Raw<TY> raw[NW][R][UPL];
    auto load_pass = [&](int base) {
#pragma unroll
        for (int k = 0; k < R; k++) {
            const int r = min(row0 + base + k, last);
            const uint8_t *row = wbase + (size_t)r * rb;
#pragma unroll
            for (int u = 0; u < UPL; u++) load_raw<TY>(row, uu[u], raw[0][k][u]);
            if constexpr (GLU) {
                const uint8_t *row2 = wbase2 + (size_t)r * p.seg[1].rb;
#pragma unroll
                for (int u = 0; u < UPL; u++) load_raw<TY>(row2, uu[u], raw[1][k][u]);
            }
        }
    };
    const int base0 = grp * R;
    if (base0 < p.tr) load_pass(base0);  // in flight while the activation is prepared
    bool have_act = false;
    if constexpr (TY == T_Q4_0 || TY == T_Q8_0) {
        if (p.nin.x) {
            // The activation is Q8_0(RMSNorm(x)·w), made here once per workgroup:
            // thread τ normalizes values 16τ..16τ+15 (a 32-block is a thread pair)
            // into LDS, then every lane reads its slice (quantizer: quant.hip).
            __shared__ __align__(16) int8_t s_q[4096];
            __shared__ float s_d[128], s_red[NT / 64];
            __shared__ int s_i[128];
            const int K = p.K, nthr = K >> 4;
            const bool act = tid < nthr;
            float4 xv[4], gv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = gv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float ss = 0.0f;
            if (act) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    xv[i] = ((const float4 *)(p.nin.x + 16 * tid))[i];
                    gv[i] = ((const float4 *)(p.nin.w + 16 * tid))[i];
                    ss = fmaf(xv[i].x, xv[i].x, ss);
                    ss = fmaf(xv[i].y, xv[i].y, ss);
                    ss = fmaf(xv[i].z, xv[i].z, ss);
                    ss = fmaf(xv[i].w, xv[i].w, ss);
                }
            }
            ss = wave_sum(ss, 64);
            if ((tid & 63) == 0) s_red[tid >> 6] = ss;
            __syncthreads();
            const float scale = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)K + p.nin.eps);
            float y[16];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                y[4 * i] = xv[i].x * scale * gv[i].x;
                y[4 * i + 1] = xv[i].y * scale * gv[i].y;
                y[4 * i + 2] = xv[i].z * scale * gv[i].z;
                y[4 * i + 3] = xv[i].w * scale * gv[i].w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(y[i]));
            amax = fmaxf(amax, xor_f<1>(amax));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t w4[4];
            int isum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t v = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    int q = (int)rintf(y[4 * j + e] * id);
                    q = q < -127 ? -127 : (q > 127 ? 127 : q);
                    isum += q;
                    v |= ((uint32_t)(q & 0xff)) << (8 * e);
                }
                w4[j] = v;
            }
            isum += xor_i<1>(isum);
            if (act) {
                *(uint4 *)(s_q + 16 * tid) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
                if ((tid & 1) == 0) {
                    s_d[tid >> 1] = d;
                    s_i[tid >> 1] = isum;
                }
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const uint4 *src = (const uint4 *)(s_q + 64 * uu[k]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint4 v = src[i];
                    a[k].q[4 * i] = v.x;
                    a[k].q[4 * i + 1] = v.y;
                    a[k].q[4 * i + 2] = v.z;
                    a[k].q[4 * i + 3] = v.w;
                }
                a[k].d0 = s_d[2 * uu[k]];
                a[k].d1 = s_d[2 * uu[k] + 1];
                a[k].i0 = s_i[2 * uu[k]];
                a[k].i1 = s_i[2 * uu[k] + 1];
            }
            have_act = true;
        }
    }
    if (!have_act) {
#pragma unroll
        for (int k = 0; k < UPL; k++)
            if (valid[k]) load_act<TY>(a[k], uu[k], p.act, p.actf, p.K, p.act_per_slot ? slot : 0);
    }
    for (int base = base0; base < p.tr; base += GROUPS * R) {
        if (base != base0) load_pass(base);
#pragma unroll
        for (int wv = 0; wv < NW; wv++)
#pragma unroll
            for (int k = 0; k < R; k++) {
                float s = 0.0f;
#pragma unroll
                for (int u = 0; u < UPL; u++) {
                    const float x = dot_raw<TY>(raw[wv][k][u], uu[u], a[u]);
                    s += valid[u] ? x : 0.0f;
                }
                red[(wv * p.tr + base + k) * STRIDE + l] = s;
            }
    }
    __syncthreads();
    // 8 threads per row add its LPR partials
    float *hv = red + NW * p.tr * STRIDE;
    const int s8 = tid & 7;
    for (int i = tid >> 3; i < ((p.tr + NT / 8 - 1) & ~(NT / 8 - 1)); i += NT / 8) {
        float sum = 0.0f, sum2 = 0.0f;
        if (i < p.tr) {
            for (int j = s8; j < LPR; j += 8) sum += red[i * STRIDE + j];
            if constexpr (GLU)
                for (int j = s8; j < LPR; j += 8) sum2 += red[(p.tr + i) * STRIDE + j];
        }
        xor_up<1, 4>([&](auto oc) {
            sum += xor_f<decltype(oc)::value>(sum);
            sum2 += xor_f<decltype(oc)::value>(sum2);
        });
        const int r = row0 + i;
        if (s8 == 0 && i < p.tr && r < seg_rows) {
            float v = sum;
            if constexpr (GLU) v = (p.glu == 2 ? gelu_tanh_f(sum) : silu_f(sum)) * sum2;
            float *out = p.seg[sg].out;
            if (p.seg[sg].epi == EPI_ADD) out[r] += v;
            else out[r] = v;
            hv[i] = v;
        }
    }
    if (!(GLU && p.hq.qs)) return;
    // Q8_0 of h (ops: avx2 quantizer semantics), one half-wave per 32 rows
    __syncthreads();
    if (tid < p.tr) {
        const int r = row0 + tid;
        const float y = r < seg_rows ? hv[tid] : 0.0f;
        float amax = fabsf(y);
        amax = xmax_f<32>(amax);
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int q = (int)rintf(y * id);
        const int qc = q < -127 ? -127 : (q > 127 ? 127 : q);
        int su = q, scl = qc;
        su = xsum_i<32>(su);
        scl = xsum_i<32>(scl);
        if (r < seg_rows) {
            p.hq.qs[r] = (int8_t)qc;
            if ((r & 31) == 0) {
                p.hq.d[r >> 5] = d;
                if (p.hq.s) p.hq.s[r >> 5] = d * (float)su;
                if (p.hq.isum) p.hq.isum[r >> 5] = scl;
            }
        }
    }
}

static int dec_units(int ty, int K) {
    if (ty == T_Q6_K || ty == T_Q2_K || ty == T_Q3_K) return K / 32;
    if (ty == T_F32 || ty == T_F16 || ty == T_BF16) return K / 8;
    return K / 64;
}

// Rows-per-workgroup multiplier override (0 = automatic), for launch-shape sweeps.
static int dec_tile_override() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("RIE_HIP_GEMV_TILE");
        v = e ? atoi(e) : 0;
    }
    return v;
}

// Rows per pass override for Q4_0 (tuning): 0 default, 1 eight rows for the
// gate/up kernel with the Q8_0 hidden, 2 eight rows for every Q4_0 launch.
static int dec_r8_mode() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("RIE_HIP_DEC_R8");
        v = e ? atoi(e) : 0;
    }
    return v;
}

template <int TY, int R>
static bool launch_dec_r(DecP p, hipStream_t st) {
    const int U = dec_units(TY, p.K);
    int lpr = 16;
    while (lpr < U && lpr < 256) lpr *= 2;
    const int upl = (U + lpr - 1) / lpr;
    if (upl > 2) return false;
    int pass = (256 / lpr) * R;  // rows per pass of a 256-thread workgroup
    int m, nt = 256;
    if (p.glu && p.hq.qs) {
        if (p.total_rows % 32) return false;
        // whole Q8_0 blocks of h per workgroup, in one pass: 512 or 1024 threads
        if (pass < 32) {
            nt = 256 * (32 / pass);
            pass = 32;
        }
        m = 1;
        if (nt > 1024) return false;
    } else {
        const int ov = dec_tile_override();
        m = ov > 0 ? ov : std::max(1, std::min(4, p.total_rows / (pass * 1024)));
    }
    p.tr = pass * m;
    if (p.xsel && p.slot_rows % p.tr) {  // a workgroup must not straddle two experts
        p.tr = pass;
        if (p.slot_rows % p.tr || (p.glu && p.hq.qs && p.tr % 32)) return false;
    }
    const size_t lds = ((size_t)(p.glu ? 2 : 1) * p.tr * (lpr + DEC_PAD) + p.tr) * sizeof(float);
    if (lds > 64 * 1024) return false;
    int blocks = 0;
    const int nseg = p.glu ? 1 : p.nseg;
    for (int i = 0; i < 3; i++) {
        if (i < nseg) blocks += (p.seg[i].rows + p.tr - 1) / p.tr;
        p.blk_end[i] = blocks;
    }
#define RIE_DEC(L, UP)                                                                                            \
    do {                                                                                                          \
        if (p.glu && nt == 512) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 512>), dim3(blocks), dim3(512), lds, st, p);    \
        else if (p.glu && nt == 1024) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 1024>), dim3(blocks), dim3(1024), lds, st, p); \
        else if (p.glu) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 256>), dim3(blocks), dim3(256), lds, st, p);      \
        else hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, false, R, 256>), dim3(blocks), dim3(256), lds, st, p);                \
    } while (0)
    if (upl == 1) {
        switch (lpr) {
        case 16: RIE_DEC(16, 1); break;
        case 32: RIE_DEC(32, 1); break;
        case 64: RIE_DEC(64, 1); break;
        case 128: RIE_DEC(128, 1); break;
        default: RIE_DEC(256, 1); break;
        }
    } else {
        RIE_DEC(256, 2);
    }
#undef RIE_DEC
    return true;
}

template <int TY>
static bool launch_dec_t(const DecP &p, hipStream_t st) {
    if constexpr (TY == T_Q4_0) {
        const int m = dec_r8_mode();
        if (m == 2 || (m == 1 && p.glu && p.hq.qs)) return launch_dec_r<TY, 8>(p, st);
    }
    return launch_dec_r<TY, dec_rows_per_pass<TY>()>(p, st);
}

static bool dispatch_dec(int ty, const DecP &p, hipStream_t st) {
    switch (ty) {
    case T_Q4_0: return launch_dec_t<T_Q4_0>(p, st);
    case T_Q4_1: return launch_dec_t<T_Q4_1>(p, st);
    case T_Q5_0: return launch_dec_t<T_Q5_0>(p, st);
    case T_Q5_1: return launch_dec_t<T_Q5_1>(p, st);
    case T_Q8_0: return launch_dec_t<T_Q8_0>(p, st);
    case T_Q2_K: return launch_dec_t<T_Q2_K>(p, st);
    case T_Q3_K: return launch_dec_t<T_Q3_K>(p, st);
    case T_Q4_K: return launch_dec_t<T_Q4_K>(p, st);
    case T_Q5_K: return launch_dec_t<T_Q5_K>(p, st);
    case T_Q6_K: return launch_dec_t<T_Q6_K>(p, st);
    case T_F32: return launch_dec_t<T_F32>(p, st);
    case T_F16: return launch_dec_t<T_F16>(p, st);
    case T_BF16: return launch_dec_t<T_BF16>(p, st);
    default: return false;
    }
}

bool gemv_supported(int ty, size_t K) {
    switch (ty) {
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: return K % 64 == 0;
    case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: return K % 256 == 0;
    case T_F32: case T_F16: case T_BF16: return K % 8 == 0;
    default: return false;
    }
}

template <int TY>
static void launch_t(const GemvP &p, hipStream_t st) {
    const int U = dec_units(TY, p.K);
    int lpr = 64;
    if (U <= 8) lpr = 8;
    else if (U <= 16) lpr = 16;
    else if (U <= 32) lpr = 32;
    const int rpw = 64 / lpr;
    const int waves = (p.total_rows + rpw - 1) / rpw;
    int blocks = (waves + 3) / 4;
    if (blocks > 4096) blocks = 4096;
    switch (lpr) {
    case 8: hipLaunchKernelGGL((gemv_kernel<TY, 8>), dim3(blocks), dim3(256), 0, st, p); break;
    case 16: hipLaunchKernelGGL((gemv_kernel<TY, 16>), dim3(blocks), dim3(256), 0, st, p); break;
    case 32: hipLaunchKernelGGL((gemv_kernel<TY, 32>), dim3(blocks), dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((gemv_kernel<TY, 64>), dim3(blocks), dim3(256), 0, st, p); break;
    }
}

static bool dispatch(int ty, const GemvP &p, hipStream_t st) {
    switch (ty) {
    case T_Q4_0: launch_t<T_Q4_0>(p, st); return true;
    case T_Q4_1: launch_t<T_Q4_1>(p, st); return true;
    case T_Q5_0: launch_t<T_Q5_0>(p, st); return true;
    case T_Q5_1: launch_t<T_Q5_1>(p, st); return true;
    case T_Q8_0: launch_t<T_Q8_0>(p, st); return true;
    case T_Q2_K: launch_t<T_Q2_K>(p, st); return true;
    case T_Q3_K: launch_t<T_Q3_K>(p, st); return true;
    case T_Q4_K: launch_t<T_Q4_K>(p, st); return true;
    case T_Q5_K: launch_t<T_Q5_K>(p, st); return true;
    case T_Q6_K: launch_t<T_Q6_K>(p, st); return true;
    case T_F32: launch_t<T_F32>(p, st); return true;
    case T_F16: launch_t<T_F16>(p, st); return true;
    case T_BF16: launch_t<T_BF16>(p, st); return true;
    default: return false;
    }
}

// The operands a weight type reads must exist: a missing activation array is a
// host-side error, never a launch.
static bool operands_ok(int ty, const ActQ8 &act, const float *act_f32) {
    switch (act_format(ty)) {
    case ACT_F32: return act_f32 != nullptr;
    case ACT_Q8_0:
        return act.qs && act.d && ((ty != T_Q4_0 && ty != T_Q5_0) || act.isum) && ((ty != T_Q4_1 && ty != T_Q5_1) || act.s);
    default: return act.qs && act.d && act.bsums;
    }
}

bool gemv_norm_ok(int ty, size_t K) { return (ty == T_Q4_0 || ty == T_Q8_0) && K % 64 == 0 && K >= 64 && K <= 4096; }

bool launch_gemv(const GemvSeg *segs, int nseg, const ActQ8 &act, const float *act_f32, int n_tok, int K, hipStream_t st,
                 const NormIn *nin) {
    if (n_tok < 1) return false;
    if (nin && (n_tok != 1 || !nin->x || !nin->w)) return false;
    for (int s = 0; s < nseg; s++)
        if (nin && !gemv_norm_ok(segs[s].w.ty, (size_t)K)) return false;
    // segments of one launch must share a weight type; split otherwise
    int i = 0;
    while (i < nseg) {
        int j = i + 1;
        while (j < nseg && j - i < 3 && segs[j].w.ty == segs[i].w.ty) j++;
        GemvP p{};
        p.nseg = j - i;
        p.total_rows = 0;
        for (int s = i; s < j; s++) {
            if (!gemv_supported(segs[s].w.ty, K) || segs[s].w.cols != (size_t)K || !segs[s].w.data || !segs[s].out ||
                !operands_ok(segs[s].w.ty, act, act_f32))
                return false;
            p.seg[s - i] = SegP{segs[s].w.data, segs[s].w.rb(), (int)segs[s].w.rows, segs[s].out, segs[s].ld, segs[s].epi};
            p.total_rows += (int)segs[s].w.rows;
        }
        p.act = act;
        p.actf = act_f32;
        p.n_tok = n_tok;
        p.K = K;
        p.glu = 0;
        bool done = false;
        if (n_tok == 1) {
            DecP d{};
            for (int s = 0; s < p.nseg; s++) d.seg[s] = p.seg[s];
            d.nseg = p.nseg;
            d.total_rows = p.total_rows;
            d.K = K;
            d.act = act;
            d.actf = act_f32;
            if (nin) d.nin = *nin;
            done = dispatch_dec(segs[i].w.ty, d, st);
        }
        if (!done && (nin || !dispatch(segs[i].w.ty, p, st))) return false;
        i = j;
    }
    return true;
}

bool launch_gemv_experts(const DevWeight &stacked, int slot_rows, const int *sel, int n_slots, const ActQ8 &act,
                         const float *act_f32, bool act_per_slot, int K, float *out, hipStream_t st) {
    if (!gemv_supported(stacked.ty, (size_t)K) || stacked.cols != (size_t)K || !stacked.data || !out || !sel || n_slots < 1 ||
        slot_rows < 1 || stacked.rows % (size_t)slot_rows || !operands_ok(stacked.ty, act, act_f32))
        return false;
    DecP d{};
    d.seg[0] = SegP{stacked.data, stacked.rb(), slot_rows * n_slots, out, slot_rows * n_slots, EPI_STORE};
    d.nseg = 1;
    d.total_rows = slot_rows * n_slots;
    d.K = K;
    d.act = act;
    d.actf = act_f32;
    d.xsel = sel;
    d.slot_rows = slot_rows;
    d.act_per_slot = act_per_slot;
    return dispatch_dec(stacked.ty, d, st);
}

bool launch_gemv_glu_experts(const DevWeight &gate, const DevWeight &up, int ff, const int *sel, int n_slots, const ActQ8 &act,
                             const float *act_f32, int K, float *h, int gelu, const ActQ8 *hq, hipStream_t st) {
    if (gate.ty != up.ty || !gemv_supported(gate.ty, (size_t)K) || gate.cols != (size_t)K || up.cols != (size_t)K ||
        gate.rows != up.rows || gate.rows % (size_t)ff || !gate.data || !up.data || !h || !sel || n_slots < 1 ||
        !operands_ok(gate.ty, act, act_f32))
        return false;
    DecP d{};
    d.seg[0] = SegP{gate.data, gate.rb(), ff * n_slots, h, ff * n_slots, EPI_STORE};
    d.seg[1] = SegP{up.data, up.rb(), ff * n_slots, h, ff * n_slots, EPI_STORE};
    d.nseg = 2;
    d.total_rows = ff * n_slots;
    d.K = K;
    d.act = act;
    d.actf = act_f32;
    d.glu = gelu ? 2 : 1;
    if (hq) d.hq = *hq;
    d.xsel = sel;
    d.slot_rows = ff;
    return dispatch_dec(gate.ty, d, st);
}

bool launch_gemv_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, const float *act_f32, int n_tok, int K, float *h,
                     int ld, int gelu, const ActQ8 *hq, hipStream_t st, const NormIn *nin) {
    if (nin && (n_tok != 1 || !nin->x || !nin->w || !gemv_norm_ok(gate.ty, (size_t)K))) return false;
    if (gate.ty != up.ty || gate.rows != up.rows || !gemv_supported(gate.ty, K) || gate.cols != (size_t)K || up.cols != (size_t)K ||
        !gate.data || !up.data || !h || n_tok < 1 || !operands_ok(gate.ty, act, act_f32))
        return false;
    GemvP p{};
    p.nseg = 2;
    p.seg[0] = SegP{gate.data, gate.rb(), (int)gate.rows, h, ld, EPI_STORE};
    p.seg[1] = SegP{up.data, up.rb(), (int)up.rows, h, ld, EPI_STORE};
    p.total_rows = (int)gate.rows;
    p.act = act;
    p.actf = act_f32;
    p.n_tok = n_tok;
    p.K = K;
    p.glu = gelu ? 2 : 1;
    if (n_tok == 1) {
        DecP d{};
        d.seg[0] = p.seg[0];
        d.seg[1] = p.seg[1];
        d.nseg = 2;
        d.total_rows = p.total_rows;
        d.K = K;
        d.act = act;
        d.actf = act_f32;
        d.glu = p.glu;
        if (hq) d.hq = *hq;
        if (nin) d.nin = *nin;
        if (dispatch_dec(gate.ty, d, st)) return true;
    }
    if (hq || nin) return false;  // the batched kernel neither quantizes h nor normalizes
    return dispatch(gate.ty, p, st);
}

}  // namespace rie
