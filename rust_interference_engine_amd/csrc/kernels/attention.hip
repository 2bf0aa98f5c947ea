// attention.hip — per-head Q/K preparation with KV-cache append, and causal
// grouped-query attention over an f16, Q8_0 or TurboQuant-4 cache, for gfx950.
//
// Reference semantics (crates/rie-core/src): model/cpu.rs:267-328 (bias, per-head
// RMSNorm, RoPE, q·attn_scale after RoPE, KV append at slot (pos0+t) % slots),
// model/cpu.rs:550-634 (attention), model/cpu.rs:636-658 (Q8_0 rows),
// turbo.rs:91-250 (rotation, 4-bit codes, rotated-domain dot/axpy).
//
// Cache layout in HBM, per layer: [kv_head][slot][row]
//   f16    : row = hd × f16
//   Q8_0   : row = hd/32 × 34-byte ggml blocks (f16 d + 32 int8)
//   Turbo4 : codes [kv_head][slot][hd/2] (Q4_0 nibble order) plus a separate
//            f16 scale array [kv_head][slot] (one rotation block for hd=128),
//            so code rows stay 16-byte aligned.
// Attention splits each query's context into n_split ranges (flash-decoding):
// every workgroup handles one (token, kv head, range) and accumulates V with
// lanes over (head, dim).  Prompt tokens: the group's query heads sit in LDS,
// the online softmax runs per tile, and a combine kernel merges the ranges,
// undoes the TurboQuant rotation and quantizes the result to Q8_0 for the
// output projection.  A single token: one launch does the query/key
// preparation, the KV append, the attention and (in the last workgroup of each
// KV head) the range merge.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"

#include <algorithm>

namespace rie {

// Lloyd–Max levels of the 4-bit Turbo4 codes as int8 (turbo.rs:126-127), and the
// same 16 bytes as four little-endian dwords for v_perm table lookups
constexpr int8_t KV_LEVELS_I8[16] = {-126, -95, -74, -58, -43, -30, -18, -6, 6, 18, 30, 43, 58, 74, 95, 126};
constexpr uint32_t kv_level_word(int i) {
    return (uint32_t)(uint8_t)KV_LEVELS_I8[4 * i] | ((uint32_t)(uint8_t)KV_LEVELS_I8[4 * i + 1] << 8) |
           ((uint32_t)(uint8_t)KV_LEVELS_I8[4 * i + 2] << 16) | ((uint32_t)(uint8_t)KV_LEVELS_I8[4 * i + 3] << 24);
}
constexpr uint32_t KV_LV0 = kv_level_word(0), KV_LV1 = kv_level_word(1), KV_LV2 = kv_level_word(2), KV_LV3 = kv_level_word(3);

// four table lookups: byte i of s (each 0..15) → byte s_i of the 16-byte table t0..t3
// (v_perm selects among 8 bytes; selector 12 gives 0x00 and 13 gives 0xFF, which
// makes the byte mask of s_i ≥ 8)
__device__ __forceinline__ uint32_t lut16(uint32_t s, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t s7 = s & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, s7), hi = __builtin_amdgcn_perm(t3, t2, s7);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((s >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
    return (hi & m) | (lo & ~m);
}

__host__ __device__ constexpr int turbo_block(int d) {
    int b = 1;
    while (d % (b * 2) == 0 && b < 256) b *= 2;
    return b;
}

// One wavefront prepares one head vector of token t at position pos: bias,
// per-head RMSNorm (q, k), RoPE (q, k); a query is scaled and written to q_dst,
// a key/value row is appended to the cache (and K to k_out when set).  With
// mirror set, the encoded row (and its Turbo4 scales) is also written there as
// one cache row of a one-row cache: [row bytes | f16 scales at KV_MIRROR_SC].
// xs, ys: this wave's LDS scratch, 256 floats each; s_inv: 8 floats.
// HD > 0: the head size as a compile-time constant (HD = a.hd).
constexpr int KV_MIRROR_SC = 512;  // byte offset of the scales in a mirror row
// KVT ≥ 0: the cache type as a compile-time constant (KVT = a.kv_type).
template <int HD, int KVT = -1>
__device__ void prep_head_wave(const HeadPrepArgs &a, int kind, int h, int t, int pos, float *q_dst, float *xs, float *ys,
                               float *s_inv, uint8_t *mirror = nullptr) {
    const int lane = threadIdx.x & 63;
    const int hd = HD > 0 ? HD : a.hd;
    const int qd = a.n_head * hd, kvd = a.n_kv * hd;
    const float *src;
    const float *bias;
    const float *nw;
    if (kind == 0) {
        src = a.q + (size_t)t * qd + h * hd; bias = a.bq; nw = a.q_norm;
    } else if (kind == 1) {
        src = a.k + (size_t)t * kvd + h * hd; bias = a.bk; nw = a.k_norm;
    } else {
        src = a.v + (size_t)t * kvd + h * hd; bias = a.bv; nw = nullptr;
    }
    // this lane's elements e = lane + 64k and their RoPE table entries, loads issued together
    const int half = a.rope_dim / 2;
    const float *ct = a.cos_t + (size_t)pos * half;
    const float *st = a.sin_t + (size_t)pos * half;
    float xr[4], cr[4], sr[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        xr[k] = cr[k] = sr[k] = 0.0f;
        if (e < hd) {
            xr[k] = src[e];
            if (kind < 2 && e < a.rope_dim) {
                const int i = a.neox ? (e < half ? e : e - half) : (e >> 1);
                cr[k] = ct[i];
                sr[k] = st[i];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        if (e < hd) xs[e] = bias ? xr[k] + bias[h * hd + e] : xr[k];
    }
    wave_sync();
    if (kind < 2) {
        if (nw) {  // ops.rs:17-24: x *= scale·w
            float ss = 0.0f;
            for (int e = lane; e < hd; e += 64) ss = fmaf(xs[e], xs[e], ss);
            ss = wave_sum(ss, 64);
            const float scale = 1.0f / sqrtf(ss / (float)hd + a.eps);
            for (int e = lane; e < hd; e += 64) xs[e] = xs[e] * (scale * nw[e]);
            wave_sync();
        }
        // RoPE, ops.rs:93-108, with the host-computed cos/sin table row of this position
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = lane + 64 * k;
            if (e >= hd) break;
            float y = xs[e];
            if (e < a.rope_dim) {
                if (a.neox) {
                    const int i = e < half ? e : e - half;
                    const float x0 = xs[i], x1 = xs[i + half];
                    y = e < half ? x0 * cr[k] - x1 * sr[k] : x0 * sr[k] + x1 * cr[k];
                } else {
                    const int i = e >> 1;
                    const float x0 = xs[2 * i], x1 = xs[2 * i + 1];
                    y = (e & 1) == 0 ? x0 * cr[k] - x1 * sr[k] : x0 * sr[k] + x1 * cr[k];
                }
            }
            ys[e] = y;
        }
        wave_sync();
        for (int e = lane; e < hd; e += 64) xs[e] = ys[e];
        wave_sync();
    }
    if (kind == 0) {
        for (int e = lane; e < hd; e += 64) q_dst[e] = xs[e] * a.attn_scale;
        return;
    }
    if (a.k_out && kind == 1)
        for (int e = lane; e < hd; e += 64) a.k_out[(size_t)t * kvd + h * hd + e] = xs[e];
    const int slot = pos % a.slots;
    const size_t row = (size_t)h * a.slots + slot;
    uint8_t *cache = kind == 1 ? a.k_cache : a.v_cache;
    const int kvt = KVT >= 0 ? KVT : a.kv_type;
    if (kvt == 0) {
        uint16_t *dst = (uint16_t *)cache + row * hd;
        for (int e = lane; e < hd; e += 64) {
            const uint16_t hb = f2h(xs[e]);
            dst[e] = hb;
            if (mirror) ((uint16_t *)mirror)[e] = hb;
        }
    } else if (kvt == 1) {
        // store_q8_0 (cpu.rs:637-647): round half away from zero, f16 scale
        uint8_t *dst = cache + row * (size_t)(hd / 32 * 34);
        for (int e0 = 0; e0 < hd; e0 += 64) {
            const int e = e0 + lane;
            const float x = e < hd ? xs[e] : 0.0f;
            float amax = fabsf(x);
            amax = xmax_f<32>(amax);
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int q = (int)roundf(x * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            if (e < hd) {
                const int off = (e >> 5) * 34;
                dst[off + 2 + (e & 31)] = (uint8_t)(int8_t)q;
                if (mirror) mirror[off + 2 + (e & 31)] = (uint8_t)(int8_t)q;
                if ((e & 31) == 0) {
                    const uint16_t hb = f2h(d);
                    dst[off] = (uint8_t)hb;
                    dst[off + 1] = (uint8_t)(hb >> 8);
                    if (mirror) {
                        mirror[off] = (uint8_t)hb;
                        mirror[off + 1] = (uint8_t)(hb >> 8);
                    }
                }
            }
        }
    } else {
        // TurboQuant-4 (turbo.rs:140-171): signs, block FWHT, RMS codes, LS scale
        for (int e = lane; e < hd; e += 64) xs[e] *= a.turbo_signs[e];
        wave_sync();
        const int b = turbo_block(hd);
#pragma unroll
        for (int hstep = 1; hstep < b; hstep *= 2) {
            for (int k = lane; k < hd / 2; k += 64) {
                const int blk = k / (b / 2), kk = k % (b / 2);
                const int j = blk * b + (kk / hstep) * 2 * hstep + (kk % hstep);
                const float x0 = xs[j], x1 = xs[j + hstep];
                xs[j] = x0 + x1;
                xs[j + hstep] = x0 - x1;
            }
            wave_sync();
        }
        const float s = 1.0f / sqrtf((float)b);
        for (int e = lane; e < hd; e += 64) xs[e] *= s;
        wave_sync();
        float c[16];
#pragma unroll
        for (int i = 0; i < 16; i++) c[i] = (float)KV_LEVELS_I8[i] / 46.0f;
        uint8_t *codes = cache + row * (size_t)(hd / 2);
        uint16_t *scales = (kind == 1 ? a.k_scale : a.v_scale) + row * (size_t)(hd / b);
        uint8_t *qv = (uint8_t *)ys;  // 256 code bytes
        // The per-block sums run in the reference's order, sequential f32 adds over the
        // block's values (turbo.rs:148-164): every lane forms its values' products at
        // once (the same roundings as the reference's x·x and x·c), then one chain of
        // adds, the same in every lane, reads them in element order with readlane.
        // chain(p, fin): Σ over each block of p(e) in order e = 0, 1, …; fin(block, sum)
        // at the end of every block.
        float xv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = lane + 64 * k < hd ? xs[lane + 64 * k] : 0.0f;
        auto chain = [&](const float (&pv)[4], auto fin) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (64 * k >= hd) break;
                const int pk = __float_as_int(pv[k]);
#pragma unroll
                for (int l = 0; l < 64; l++) {
                    const int e = 64 * k + l;
                    if (e >= hd) break;  // hd = 32: half a chunk
                    acc = acc + __int_as_float(__builtin_amdgcn_readlane(pk, l));
                    if (((e + 1) & (b - 1)) == 0) {
                        fin(e / b, acc);
                        acc = 0.0f;
                    }
                }
            }
        };
        float sq[4];
#pragma unroll
        for (int k = 0; k < 4; k++) sq[k] = xv[k] * xv[k];
        chain(sq, [&](int bk, float ss) {
            const float rms = sqrtf(ss / (float)b);
            if (lane == 0) s_inv[bk] = rms > 0.0f ? 1.0f / rms : 0.0f;
        });
        wave_sync();
        float px[4], pc[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = lane + 64 * k;
            px[k] = pc[k] = 0.0f;
            if (e < hd) {
                const float v = xv[k] * s_inv[e / b];
                int q = 0;
#pragma unroll
                for (int i = 0; i < 15; i++) q += v > 0.5f * (c[i] + c[i + 1]) ? 1 : 0;
                qv[e] = (uint8_t)q;
                float cq = c[0];
#pragma unroll
                for (int i = 1; i < 16; i++) cq = q == i ? c[i] : cq;
                px[k] = xv[k] * cq;
                pc[k] = cq * cq;
            }
        }
        wave_sync();
        for (int i = lane; i < hd / 2; i += 64) {  // byte i holds values g (low) and g+16 (high) of its 32-chunk
            const int g = (i / 16) * 32 + (i % 16);
            codes[i] = (uint8_t)(qv[g] | (qv[g + 16] << 4));
            if (mirror) mirror[i] = (uint8_t)(qv[g] | (qv[g + 16] << 4));
        }
        // least-squares scale Σx·c / Σc² per block (the two sums of one sequential loop);
        // the numerators wait in LDS past the codes (lane 0 writes and reads them)
        float *nums = ys + 128;
        chain(px, [&](int bk, float num) {
            if (lane == 0) nums[bk] = num;
        });
        chain(pc, [&](int bk, float den) {
            if (lane == 0) {
                const uint16_t hb = f2h(den > 0.0f ? nums[bk] / den : 0.0f);
                scales[bk] = hb;
                if (mirror) ((uint16_t *)(mirror + KV_MIRROR_SC))[bk] = hb;
            }
        });
    }
}

// The same preparation with the head vector in registers (no LDS round trips):
// HD ∈ {64, 128, 256} with full rotary and an f16 or Q8_0 cache.  Lane l holds
// elements l + 64k; the NEOX partner e ± HD/2 is in the same lane (HD ≥ 128) or
// lane l ^ 32 (HD = 64), the interleaved partner e ^ 1 in lane l ^ 1.  The
// arithmetic is prep_head_wave's, operation for operation.
__device__ __forceinline__ bool prep_fast_ok(const HeadPrepArgs &a, int hd) {
    return (hd == 64 || hd == 128 || hd == 256) && a.rope_dim == hd && a.kv_type != 2;
}
// The loads of one head vector's preparation (the vector, its bias, norm weights
// and rotary factors), issued apart from the arithmetic so that a caller can put
// other loads in flight behind them.  kind and h are wave-uniform.
template <int HD>
struct PrepIn {
    static constexpr int NE = HD / 64;
    float x[NE], c[NE], sn[NE], b[NE], nw[NE];
};
template <int HD>
__device__ __forceinline__ void prep_load_fast(const HeadPrepArgs &a, int kind, int h, int pos, PrepIn<HD> &in) {
    constexpr int NE = HD / 64, half = HD / 2;
    const int lane = threadIdx.x & 63;
    const float *src = kind == 0 ? a.q + h * HD : (kind == 1 ? a.k : a.v) + h * HD;
    const float *bias = kind == 0 ? a.bq : kind == 1 ? a.bk : a.bv;
    const float *nw = kind == 0 ? a.q_norm : kind == 1 ? a.k_norm : nullptr;
    const float *ct = a.cos_t + (size_t)pos * half, *st = a.sin_t + (size_t)pos * half;
#pragma unroll
    for (int k = 0; k < NE; k++) {
        const int e = lane + 64 * k;
        in.x[k] = src[e];
        const int i = a.neox ? (e < half ? e : e - half) : (e >> 1);
        in.c[k] = kind < 2 ? ct[i] : 0.0f;
        in.sn[k] = kind < 2 ? st[i] : 0.0f;
        in.b[k] = bias ? bias[h * HD + e] : 0.0f;
        in.nw[k] = (kind < 2 && nw) ? nw[e] : 0.0f;
    }
}

template <int HD>
__device__ void prep_finish_fast(const HeadPrepArgs &a, int kind, int h, int pos, const PrepIn<HD> &in, float *q_dst, uint8_t *mirror) {
    constexpr int NE = HD / 64, half = HD / 2;
    const int lane = threadIdx.x & 63;
    const float *bias = kind == 0 ? a.bq : kind == 1 ? a.bk : a.bv;
    const float *nw = kind == 0 ? a.q_norm : kind == 1 ? a.k_norm : nullptr;
    float x[NE], c[NE], sn[NE];
#pragma unroll
    for (int k = 0; k < NE; k++) {
        x[k] = in.x[k];
        c[k] = in.c[k];
        sn[k] = in.sn[k];
    }
    if (bias)
#pragma unroll
        for (int k = 0; k < NE; k++) x[k] = x[k] + in.b[k];
    if (kind < 2) {
        if (nw) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < NE; k++) ss = fmaf(x[k], x[k], ss);
            ss = xsum_f<64>(ss);
            const float scale = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
            for (int k = 0; k < NE; k++) x[k] = x[k] * (scale * in.nw[k]);
        }
        float y[NE];
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int e = lane + 64 * k;
            if (a.neox) {
                float x0, x1;  // elements i and i + half of the pair
                if constexpr (HD == 64) {
                    const float o = xor_f<32>(x[k]);
                    x0 = e < half ? x[k] : o;
                    x1 = e < half ? o : x[k];
                } else {
                    constexpr int KH = NE / 2;  // element e ± half sits KH slots away in this lane
                    x0 = k < KH ? x[k] : x[k - KH];
                    x1 = k < KH ? x[k + KH] : x[k];
                }
                y[k] = e < half ? x0 * c[k] - x1 * sn[k] : x0 * sn[k] + x1 * c[k];
            } else {
                const float o = xor_f<1>(x[k]);
                const float x0 = (e & 1) ? o : x[k], x1 = (e & 1) ? x[k] : o;
                y[k] = (e & 1) == 0 ? x0 * c[k] - x1 * sn[k] : x0 * sn[k] + x1 * c[k];
            }
        }
#pragma unroll
        for (int k = 0; k < NE; k++) x[k] = y[k];
    }
    if (kind == 0) {
#pragma unroll
        for (int k = 0; k < NE; k++) q_dst[lane + 64 * k] = x[k] * a.attn_scale;
        return;
    }
    if (a.k_out && kind == 1)
#pragma unroll
        for (int k = 0; k < NE; k++) a.k_out[h * HD + lane + 64 * k] = x[k];
    const size_t row = (size_t)h * a.slots + pos % a.slots;
    uint8_t *cache = kind == 1 ? a.k_cache : a.v_cache;
    if (a.kv_type == 0) {
        uint16_t *dst = (uint16_t *)cache + row * HD;
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const uint16_t hb = f2h(x[k]);
            dst[lane + 64 * k] = hb;
            if (mirror) ((uint16_t *)mirror)[lane + 64 * k] = hb;
        }
    } else {  // store_q8_0 (cpu.rs:637-647): round half away from zero, f16 scale
        uint8_t *dst = cache + row * (size_t)(HD / 32 * 34);
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int e = lane + 64 * k;
            const float amax = xmax_f<32>(fabsf(x[k]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int q = (int)roundf(x[k] * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            const int off = (e >> 5) * 34;
            dst[off + 2 + (e & 31)] = (uint8_t)(int8_t)q;
            if (mirror) mirror[off + 2 + (e & 31)] = (uint8_t)(int8_t)q;
            if ((e & 31) == 0) {
                const uint16_t hb = f2h(d);
                dst[off] = (uint8_t)hb;
                dst[off + 1] = (uint8_t)(hb >> 8);
                if (mirror) {
                    mirror[off] = (uint8_t)hb;
                    mirror[off + 1] = (uint8_t)(hb >> 8);
                }
            }
        }
    }
}

// one wavefront per (head vector, token); the query is rewritten in place.
// HD, KVT > 0 / ≥ 0: head size and cache type as compile-time constants (the
// Turbo4 rotation's butterfly indices then cost no integer divisions)
template <int HD, int KVT>
__global__ __launch_bounds__(64) void head_prep_kernel(HeadPrepArgs a) {
    const int t = blockIdx.y;
    const int hh = blockIdx.x;
    const int pos0 = a.d_pos0 ? *a.d_pos0 : a.pos0;
    __shared__ float xs[256];
    __shared__ float ys[256];
    __shared__ float s_inv[8];
    int kind, h;
    if (hh < a.n_head) {
        kind = 0; h = hh;
    } else if (hh < a.n_head + a.n_kv) {
        kind = 1; h = hh - a.n_head;
    } else {
        kind = 2; h = hh - a.n_head - a.n_kv;
    }
    prep_head_wave<HD, KVT>(a, kind, h, t, pos0 + t, a.q + (size_t)t * a.n_head * a.hd + h * a.hd, xs, ys, s_inv);
}

template <int HD>
static void launch_head_prep_hd(const HeadPrepArgs &a, dim3 grid, hipStream_t st) {
    switch (a.kv_type) {
    case 0: hipLaunchKernelGGL((head_prep_kernel<HD, 0>), grid, dim3(64), 0, st, a); break;
    case 1: hipLaunchKernelGGL((head_prep_kernel<HD, 1>), grid, dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((head_prep_kernel<HD, 2>), grid, dim3(64), 0, st, a); break;
    }
}

void launch_head_prep(const HeadPrepArgs &a, hipStream_t st) {
    const dim3 grid(a.n_head + 2 * a.n_kv, a.n_tok);
    switch (a.hd) {
    case 64: launch_head_prep_hd<64>(a, grid, st); break;
    case 128: launch_head_prep_hd<128>(a, grid, st); break;
    case 256: launch_head_prep_hd<256>(a, grid, st); break;
    default: hipLaunchKernelGGL((head_prep_kernel<0, -1>), grid, dim3(64), 0, st, a); break;
    }
}

// ---- attention over the cache ---------------------------------------------------
// A workgroup owns one (range, kv head, token).  SUB = hd/8 lanes (rounded up to
// a power of two) share a cache position, each lane holding 8 dims (16 bytes of
// an f16 row); PP = 256/SUB positions per pass, NP passes per tile, with the K
// and V loads of the whole tile issued together.  Per-position scores are
// reduced over the SUB lanes with DPP, the online softmax runs one wavefront per
// query head, and each lane accumulates its 8 dims of V for every query head of
// the group; the position slots are summed at the end.
constexpr int ATT_NP = 4;

__device__ __forceinline__ float softcap_f(float v, float cap) { return cap > 0.0f ? cap * tanhf(v / cap) : v; }

// 8 dims [d0, d0+8) of a row of the cache as floats (f16 / Q8_0 / Turbo4 levels·scale)
template <int KVT>
struct KvChunk {
    uint4 raw;      // f16: 8 halves; Q8_0: 8 codes in x,y; Turbo4: 8 code bytes in x,y
    uint32_t sc;    // Q8_0 block d or Turbo4 block scale (f16 bits)
};

template <int KVT>
__device__ __forceinline__ void load_chunk(const uint8_t *cache, const uint16_t *scales, size_t row, int hd, int d0, int tb,
                                           KvChunk<KVT> &c) {
    if constexpr (KVT == 0) {
        c.raw = *(const uint4 *)(cache + (row * hd + d0) * 2);
        c.sc = 0;
    } else if constexpr (KVT == 1) {
        const uint8_t *blk = cache + row * (size_t)(hd / 32) * 34 + (d0 / 32) * 34;
        const uint8_t *q = blk + 2 + (d0 % 32);
        const uint32_t lo = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
        const uint32_t hi = (uint32_t)q[4] | ((uint32_t)q[5] << 8) | ((uint32_t)q[6] << 16) | ((uint32_t)q[7] << 24);
        c.raw = make_uint4(lo, hi, 0, 0);
        c.sc = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
    } else {
        const uint2 v = *(const uint2 *)(cache + row * (size_t)(hd / 2) + (d0 / 32) * 16 + (d0 % 16));
        c.raw = make_uint4(v.x, v.y, 0, 0);
        c.sc = scales[row * (size_t)(hd / tb) + d0 / tb];
    }
}

// Turbo4: 8 codes of the chunk → 8 int8 levels packed in two dwords
__device__ __forceinline__ void turbo_levels8(const KvChunk<2> &c, bool hi, uint32_t out[2]) {
    const uint32_t w[2] = {c.raw.x, c.raw.y};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t codes = (hi ? (w[h] >> 4) : w[h]) & 0x0F0F0F0Fu;  // one code per byte
        out[h] = lut16(codes, KV_LV0, KV_LV1, KV_LV2, KV_LV3);
    }
}

template <int KVT>
__device__ __forceinline__ void chunk_values(const KvChunk<KVT> &c, int d0, float v[8]) {
    if constexpr (KVT == 0) {
        const uint32_t w[4] = {c.raw.x, c.raw.y, c.raw.z, c.raw.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = h2f(w[i] & 0xffff);
            v[2 * i + 1] = h2f(w[i] >> 16);
        }
    } else if constexpr (KVT == 1) {
        const float d = h2f(c.sc);
        const uint32_t w[2] = {c.raw.x, c.raw.y};
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = d * (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xff);
    } else {
        const float s = h2f(c.sc) * (1.0f / 46.0f);
        uint32_t lv[2];
        turbo_levels8(c, (d0 % 32) >= 16, lv);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = s * (float)(int8_t)((lv[i >> 2] >> (8 * (i & 3))) & 0xff);
    }
}

// The same 8 values as level·scale: the levels (Q8_0 codes, Turbo4 int8 levels) as
// floats and the chunk's one scale (Q8_0 d, Turbo4 scale/46)
template <int KVT>
__device__ __forceinline__ float chunk_levels(const KvChunk<KVT> &c, int d0, float v[8]) {
    static_assert(KVT == 1 || KVT == 2, "quantized caches");
    uint32_t lv[2];
    if constexpr (KVT == 1) {
        lv[0] = c.raw.x;
        lv[1] = c.raw.y;
    } else {
        turbo_levels8(c, (d0 % 32) >= 16, lv);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)(int8_t)((lv[i >> 2] >> (8 * (i & 3))) & 0xff);
    return KVT == 1 ? h2f(c.sc) : h2f(c.sc) * (1.0f / 46.0f);
}

// Scores of ATT_NP positions × MG query heads: each lane's partial dot over its 8
// dims, summed over the SUB lanes of the position (every lane of the group gets
// the sum).  Q8_0 / Turbo4 caches: per-block integer dots (cpu.rs: int32 block
// sums) over the 4 lanes of a block, scaled by d_k·d_q.
template <int KVT, int SUB, int MG, int NP = ATT_NP>
__device__ __forceinline__ void tile_scores(const KvChunk<KVT> (&kc)[NP], const float (&qf)[MG][8], const uint32_t (&qq)[MG][2],
                                            const float (&qdd)[MG], int c, bool cact, int d0, float (&sc)[NP][MG]) {
#pragma unroll
    for (int n = 0; n < NP; n++) {
        float kf[8];
        if constexpr (KVT == 0) chunk_values<0>(kc[n], d0, kf);
#pragma unroll
        for (int j = 0; j < MG; j++) {
            float part = 0.0f;
            if constexpr (KVT == 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) part = fmaf(kf[i], qf[j][i], part);
            } else {
                uint32_t kw[2];
                if constexpr (KVT == 1) {
                    kw[0] = kc[n].raw.x;
                    kw[1] = kc[n].raw.y;
                } else {
                    turbo_levels8(kc[n], (d0 % 32) >= 16, kw);
                }
                const int isum = quad_sum_i(sdot4(kw[1], qq[j][1], sdot4(kw[0], qq[j][0], 0)));
                const float ks = KVT == 1 ? h2f(kc[n].sc) : h2f(kc[n].sc) * (1.0f / 46.0f);
                part = (c & 3) == 0 ? (KVT == 1 ? ks * qdd[j] : qdd[j] * ks) * (float)isum : 0.0f;
            }
            if (!cact) part = 0.0f;
            sc[n][j] = group_sum<SUB>(part);
        }
    }
}

// The group's query heads (in qs_f, f32) → Turbo4 rotation and Q8_0 codes
// (cpu.rs:585-598) for quantized caches, then this lane's registers.  256 threads.
template <int KVT, int MG>
__device__ __forceinline__ void query_registers(const AttnArgs &a, int G, int hd, int tb, int d0, float *qs_f, int8_t *qs_i, float *qs_d,
                                                float (&qf)[MG][8], uint32_t (&qq)[MG][2], float (&qdd)[MG]) {
    const int tid = threadIdx.x;
    if constexpr (KVT != 0) {
        if constexpr (KVT == 2) {
            // every head of the group at once, one barrier per butterfly stage; the
            // signs (exact ±1 factors) are applied as the first stage reads its
            // operands and 1/√tb as the last stage writes, the same roundings as
            // sign pass, stages, scale pass
            const float sq = 1.0f / sqrtf((float)tb);
            for (int hstep = 1; hstep < tb; hstep *= 2) {
                for (int k = tid; k < G * hd / 2; k += 256) {
                    const int j = k / (hd / 2), kh = k % (hd / 2);
                    const int blk = kh / (tb / 2), kk = kh % (tb / 2);
                    const int e = blk * tb + (kk / hstep) * 2 * hstep + (kk % hstep);
                    float *x = qs_f + j * hd;
                    float x0 = x[e], x1 = x[e + hstep];
                    if (hstep == 1) {
                        x0 *= a.turbo_signs[e];
                        x1 *= a.turbo_signs[e + hstep];
                    }
                    float y0 = x0 + x1, y1 = x0 - x1;
                    if (2 * hstep == tb) {
                        y0 *= sq;
                        y1 *= sq;
                    }
                    x[e] = y0;
                    x[e + hstep] = y1;
                }
                __syncthreads();
            }
        }
        // RNE Q8_0 quantization of each 32-block, half a wave per block
        const int hw = tid >> 5, j = tid & 31;
        for (int bi = hw; bi < G * hd / 32; bi += 8) {
            const float y = qs_f[bi * 32 + j];
            float amax = fabsf(y);
            amax = xmax_f<32>(amax);
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int q = (int)rintf(y * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            qs_i[bi * 32 + j] = (int8_t)q;
            if (j == 0) qs_d[bi] = d;
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < MG; j++) {
        const int jj = j < G ? j : 0;
        if constexpr (KVT == 0) {
#pragma unroll
            for (int i = 0; i < 8; i++) qf[j][i] = qs_f[jj * hd + d0 + i];
            qq[j][0] = qq[j][1] = 0;
            qdd[j] = 0.0f;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) qf[j][i] = 0.0f;
            qq[j][0] = *(const uint32_t *)(qs_i + jj * hd + d0);
            qq[j][1] = *(const uint32_t *)(qs_i + jj * hd + d0 + 4);
            qdd[j] = qs_d[(jj * hd) / 32 + d0 / 32];
        }
    }
}

// K and V chunks of NP positions tile + pi + PP·n (rows past r1 repeat row r0);
// LOADK false: V only (the K rows are loaded in the matrix-core layout instead)
template <int KVT, int PP, int NP = ATT_NP, bool LOADK = true>
__device__ __forceinline__ void load_tile(const AttnArgs &a, size_t kv_row0, int tile, int pi, int r0, int r1, int hd, int d0, int tb,
                                          KvChunk<KVT> (&kc)[NP], KvChunk<KVT> (&vc)[NP], bool (&ok)[NP]) {
#pragma unroll
    for (int n = 0; n < NP; n++) {
        const int pos = tile + pi + PP * n;
        ok[n] = pos < r1;
        const int q = ok[n] ? pos : r0;
        const size_t row = kv_row0 + (size_t)(q < a.slots ? q : q % a.slots);
        if constexpr (LOADK) load_chunk<KVT>(a.k_cache, a.k_scale, row, hd, d0, tb, kc[n]);
        load_chunk<KVT>(a.v_cache, a.v_scale, row, hd, d0, tb, vc[n]);
    }
}

// ---- Turbo4 scores on int8 matrix cores (head size 128, the range kernel) ----
// The 16 positions of a wave's tile (slot 4w + s, pass n: position tile + 4w + s +
// 16n) are the rows r = 4n + s of v_mfma_i32_16x16x32_i8, one MFMA per 32-value
// chunk c: A = the K rows' levels (lane l: row l % 16, chunk values 8·(l / 16) ..
// +7, i.e. bytes 16c + 8·(l/16 & 1) of the code row, high nibbles for l/16 ≥ 2),
// B = the rotated Q8_0 query codes (lane l: query head l % 16 of the slice, the
// same 8 chunk values), D = the exact int32 chunk dots Σ LEVEL[code]·q8 of
// dot_rotated_4 (turbo.rs:178-193; lane l: head l % 16, rows 4·(l/16) + i).
// score = Σ_c (d_q,c · scale/46) · dot_c, as the VALU path forms each chunk's term.
typedef int att_v4i __attribute__((ext_vector_type(4)));
struct KTileMF {
    uint2 w[4];      // the A row's code bytes of chunks 0..3
    uint32_t sc[4];  // f16 scales of the lane's output rows 4·(l/16) + i
};
__device__ __forceinline__ int ktile_row_pos(int tile, int wv, int r) { return tile + 4 * wv + (r & 3) + 16 * (r >> 2); }
__device__ __forceinline__ void load_k_mfma(const AttnArgs &a, size_t kv_row0, int tile, int wv, int lane, int r0, int r1, KTileMF &k) {
    const int kg = lane >> 4;
    const int pos = ktile_row_pos(tile, wv, lane & 15);
    const int q = pos < r1 ? pos : r0;
    const size_t row = kv_row0 + (size_t)(q < a.slots ? q : q % a.slots);
    const uint8_t *src = a.k_cache + row * 64 + 8 * (kg & 1);
#pragma unroll
    for (int c = 0; c < 4; c++) k.w[c] = *(const uint2 *)(src + 16 * c);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int op = ktile_row_pos(tile, wv, 4 * kg + i);
        const int oq = op < r1 ? op : r0;
        k.sc[i] = a.k_scale[kv_row0 + (size_t)(oq < a.slots ? oq : oq % a.slots)];  // one scale per row (block 128)
    }
}
// the new position's row from the LDS mirror (row bytes, then the f16 scale at KV_MIRROR_SC)
__device__ __forceinline__ void k_mfma_mirror(int tile, int wv, int lane, int p, const uint8_t *mirror, KTileMF &k) {
    const int kg = lane >> 4;
    if (ktile_row_pos(tile, wv, lane & 15) == p) {
#pragma unroll
        for (int c = 0; c < 4; c++) k.w[c] = *(const uint2 *)(mirror + 16 * c + 8 * (kg & 1));
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (ktile_row_pos(tile, wv, 4 * kg + i) == p) k.sc[i] = *(const uint16_t *)(mirror + KV_MIRROR_SC);
}
// scores of the wave's 16 positions × MG heads, handed to the slot layout through
// LDS (sc_s: [64 rows][MG]); sc[n][j] for this lane's slot s, pass n, head j
template <int MG>
__device__ __forceinline__ void mfma_scores(const KTileMF &k, const long (&qb)[4], const float (&qdc)[4], int wv, int lane, float *sc_s,
                                            float (&sc)[ATT_NP][MG]) {
    const int kg = lane >> 4, hh = lane & 15;
    att_v4i I[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t c0 = (kg >= 2 ? (k.w[c].x >> 4) : k.w[c].x) & 0x0F0F0F0Fu;
        const uint32_t c1 = (kg >= 2 ? (k.w[c].y >> 4) : k.w[c].y) & 0x0F0F0F0Fu;
        const long av = (long)(((unsigned long)lut16(c1, KV_LV0, KV_LV1, KV_LV2, KV_LV3) << 32) |
                               (unsigned long)lut16(c0, KV_LV0, KV_LV1, KV_LV2, KV_LV3));
        const att_v4i z = {0, 0, 0, 0};
        I[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, qb[c], z, 0, 0, 0);
    }
    if (hh < MG) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float ks = h2f(k.sc[i]) * (1.0f / 46.0f);
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) acc += (qdc[c] * ks) * (float)I[c][i];
            sc_s[(16 * wv + 4 * kg + i) * MG + hh] = acc;
        }
    }
    wave_sync();
    const int s = (lane >> 4);  // the slot within the wave (16 lanes per cache row at head size 128)
#pragma unroll
    for (int n = 0; n < ATT_NP; n++)
#pragma unroll
        for (int j = 0; j < MG; j++) sc[n][j] = sc_s[(16 * wv + 4 * n + s) * MG + j];
    wave_sync();
}

// Prompt tokens: one workgroup per (range, kv head, token); per tile of positions
// the scores go through LDS, the online softmax runs one wavefront per query head,
// and the V accumulation is per lane; the position slots are summed at the end.
template <int KVT, int SUB, int MG>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
    constexpr int PP = 256 / SUB;  // position slots per pass
    constexpr int TP = PP * ATT_NP;  // positions per tile
    const int s_idx = blockIdx.x, g = blockIdx.y, t = blockIdx.z;
    const int tid = threadIdx.x;
    const int hd = a.hd;
    const int G = a.n_head / a.n_kv;
    const int qd = a.n_head * hd;
    const int pos0 = a.d_pos0 ? *a.d_pos0 : a.pos0;
    const int p = pos0 + t;
    const int start = a.window > 0 ? max(0, p + 1 - a.window) : 0;
    const int len = p + 1 - start;
    const int chunk = (len + a.n_split - 1) / a.n_split;
    const int r0 = start + s_idx * chunk;
    const int r1 = min(start + (s_idx + 1) * chunk, p + 1);
    const int pi = tid / SUB, c = tid % SUB;
    const bool cact = c < hd / 8;
    const int d0 = cact ? 8 * c : 0;
    const int tb = turbo_block(hd);

    __shared__ float qs_f[MG * 256];   // query heads of the group (f32; rotated for Turbo4)
    __shared__ __align__(16) int8_t qs_i[MG * 256];  // their Q8_0 codes (Q8_0 / Turbo4 caches)
    __shared__ float qs_d[MG * 8];     // Q8_0 block scales
    __shared__ float sc[MG][TP];       // scores → probabilities of one tile
    __shared__ float m_run[MG], l_run[MG], alpha[MG];

    const size_t kv_row0 = (size_t)g * a.slots;
    KvChunk<KVT> kc[ATT_NP], vc[ATT_NP];
    bool ok[ATT_NP];
    if (r0 < r1) load_tile<KVT, PP>(a, kv_row0, r0, pi, r0, r1, hd, d0, tb, kc, vc, ok);  // overlaps the query load
    for (int i = tid; i < G * hd; i += 256) qs_f[i] = a.q[(size_t)t * qd + (size_t)g * G * hd + i];
    if (tid < MG) {
        m_run[tid] = -INFINITY;
        l_run[tid] = 0.0f;
    }
    __syncthreads();
    float qf[MG][8];
    uint32_t qq[MG][2];
    float qdd[MG];
    query_registers<KVT, MG>(a, G, hd, tb, d0, qs_f, qs_i, qs_d, qf, qq, qdd);
    float o[MG][8];
#pragma unroll
    for (int j = 0; j < MG; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) o[j][i] = 0.0f;

    for (int tile = r0; tile < r1; tile += TP) {
        if (tile != r0) load_tile<KVT, PP>(a, kv_row0, tile, pi, r0, r1, hd, d0, tb, kc, vc, ok);
        float s4[ATT_NP][MG];
        tile_scores<KVT, SUB, MG>(kc, qf, qq, qdd, c, cact, d0, s4);
#pragma unroll
        for (int n = 0; n < ATT_NP; n++)
#pragma unroll
            for (int j = 0; j < MG; j++)
                if (c == 0 && j < G) sc[j][pi + PP * n] = ok[n] ? softcap_f(s4[n][j], a.softcap) : -INFINITY;
        __syncthreads();
        // ---- online softmax: one wavefront per head ----
        const int wv = tid >> 6, lane = tid & 63;
        for (int j = wv; j < G; j += 4) {
            float mx = -INFINITY;
            for (int i = lane; i < TP; i += 64) mx = fmaxf(mx, sc[j][i]);
            mx = wave_max(mx, 64);
            const float m_new = fmaxf(m_run[j], mx);
            float sum = 0.0f;
            for (int i = lane; i < TP; i += 64) {
                const float pv = expf(sc[j][i] - m_new);
                sc[j][i] = pv;
                sum += pv;
            }
            sum = wave_sum(sum, 64);
            if (lane == 0) {
                const float al = expf(m_run[j] - m_new);
                alpha[j] = al;
                l_run[j] = l_run[j] * al + sum;
                m_run[j] = m_new;
            }
        }
        __syncthreads();
        // ---- V: o[j] = alpha[j]·o[j] + Σ_pos p[j][pos]·v[pos] over this lane's 8 dims ----
#pragma unroll
        for (int j = 0; j < MG; j++) {
            const float al = j < G ? alpha[j] : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) o[j][i] *= al;
        }
#pragma unroll
        for (int n = 0; n < ATT_NP; n++) {
            float vv[8];
            chunk_values<KVT>(vc[n], d0, vv);
#pragma unroll
            for (int j = 0; j < MG; j++) {
                const float w = j < G ? sc[j][pi + PP * n] : 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) o[j][i] = fmaf(w, vv[i], o[j][i]);
            }
        }
        __syncthreads();
    }
    // ---- sum the position slots: inside the wave, then over the 4 waves in LDS ----
    xor_up<SUB, 32>([&](auto oc) {
#pragma unroll
        for (int j = 0; j < MG; j++)
#pragma unroll
            for (int i = 0; i < 8; i++) o[j][i] += xor_f<decltype(oc)::value>(o[j][i]);
    });
    float *wsum = qs_f;  // MG·256 floats: reused, the query now lives in registers
    const int wv = tid >> 6, lane = tid & 63;
    __syncthreads();
    for (int w = 0; w < 4; w++) {
        if (wv == w && lane < SUB && cact) {
#pragma unroll
            for (int j = 0; j < MG; j++)
                if (j < G)
#pragma unroll
                    for (int i = 0; i < 8; i++) wsum[j * hd + d0 + i] = (w == 0 ? 0.0f : wsum[j * hd + d0 + i]) + o[j][i];
        }
        __syncthreads();
    }
    float *part = a.part + (((size_t)t * a.n_head + (size_t)g * G) * a.n_split) * (hd + 2);
    for (int i = tid; i < G * hd; i += 256) {
        const int j = i / hd, d = i % hd;
        part[((size_t)j * a.n_split + s_idx) * (hd + 2) + d] = wsum[i];
    }
    if (tid < G) {
        float *pp = part + ((size_t)tid * a.n_split + s_idx) * (hd + 2);
        pp[hd] = m_run[tid];
        pp[hd + 1] = l_run[tid];
    }
}

// ---- single token (decode) ----------------------------------------------------------
// One launch per layer, grid (n_split, n_kv · slices per group).  The workgroup
// prepares its query heads itself (bias, RMSNorm, RoPE, scale); the workgroup whose range holds
// the new position also prepares, encodes and appends that position's K and V row
// and uses its LDS copy of the encoded row.  Each SUB-lane position slot keeps its
// own online softmax state in registers (no LDS or barrier inside the tile loop);
// the slots are merged by shuffles within the wave and through LDS across the 4
// waves.  The last workgroup of each head slice to finish merges the ranges, undoes
// the Turbo4 rotation and writes att (f32 and Q8_0).

// The G merged, normalized query heads h0 .. h0 + G - 1 in o_s (LDS) → the inverse
// Turbo4 rotation, att (f32) and its Q8_0 codes; NT threads (every thread calls it).
template <int HD, int G, int NT>
__device__ void att_finish(const AttnArgs &a, int h0, float *o_s) {
    const int tid = threadIdx.x;
    constexpr int hd = HD;
    if (a.kv_type == 2) {  // o ← Rᵀ o per head: block FWHT, then signs (turbo.rs:114-117)
        const int b = turbo_block(hd);
        for (int hstep = 1; hstep < b; hstep *= 2) {
            for (int k = tid; k < G * hd / 2; k += NT) {
                const int j = k / (hd / 2), kh = k % (hd / 2);
                const int blk = kh / (b / 2), kk = kh % (b / 2);
                const int e = j * hd + blk * b + (kk / hstep) * 2 * hstep + (kk % hstep);
                const float x0 = o_s[e], x1 = o_s[e + hstep];
                o_s[e] = x0 + x1;
                o_s[e + hstep] = x0 - x1;
            }
            __syncthreads();
        }
        const float sq = 1.0f / sqrtf((float)b);
        for (int i = tid; i < G * hd; i += NT) o_s[i] = o_s[i] * sq * a.turbo_signs[i % hd];
        __syncthreads();
    }
    const size_t base = (size_t)h0 * hd;
    for (int i = tid; i < G * hd; i += NT) a.att[base + i] = o_s[i];
    if (a.att_fmt == ACT_Q8_0) {  // hd % 32 == 0: the group's values are whole blocks
        // 16 lanes per block, values j and j + 16 in lane j (max and integer sums
        // are exact in any order, so the codes are those of the reference's quantizer)
        const int hb = tid >> 4, j = tid & 15;
        for (int bi = hb; bi < G * hd / 32; bi += NT / 16) {
            const float y0 = o_s[bi * 32 + j], y1 = o_s[bi * 32 + j + 16];
            float amax = fmaxf(fabsf(y0), fabsf(y1));
            amax = xmax_f<16>(amax);
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int q0 = (int)rintf(y0 * id), q1 = (int)rintf(y1 * id);
            const int c0 = q0 < -127 ? -127 : (q0 > 127 ? 127 : q0);
            const int c1 = q1 < -127 ? -127 : (q1 > 127 ? 127 : q1);
            int su = q0 + q1, scl = c0 + c1;
            su = xsum_i<16>(su);
            scl = xsum_i<16>(scl);
            const size_t e = base + bi * 32 + j;
            a.att_q.qs[e] = (int8_t)c0;
            a.att_q.qs[e + 16] = (int8_t)c1;
            if (j == 0) {
                const size_t blk = e / 32;
                a.att_q.d[blk] = d;
                if (a.att_q.s) a.att_q.s[blk] = d * (float)su;
                if (a.att_q.isum) a.att_q.isum[blk] = scl;
            }
        }
    }
}

// Merge of the n_split range partials of query heads h0 .. h0 + G - 1 by the last
// workgroup (256 threads).
// The single-token path keeps scores and running maxima in log2 units (scores
// scaled by log2 e), so every exponential is one v_exp_f32.
template <int HD, int G>
__device__ void combine_group(const AttnArgs &a, int h0, float *o_s, float *wts, float *Ls) {
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    constexpr int hd = HD;
    const int ns = a.n_split;
    const size_t prow = (size_t)hd + 2;
    const float *part0 = a.part + (size_t)h0 * ns * prow;
    constexpr int n_out = G * hd;
    constexpr int NO = (n_out + 255) / 256;     // outputs per thread
    constexpr int NPF = NO < 2 ? NO : 2;        // of which the first batch is loaded before the weights
    constexpr int CB = 16;                      // ranges per batch of loads
    float pre[NPF][CB];
#pragma unroll
    for (int r = 0; r < NPF; r++) {
        const int i = min(tid + 256 * r, n_out - 1);
        const float *src = part0 + (size_t)(i / hd) * ns * prow + i % hd;
#pragma unroll
        for (int b = 0; b < CB; b++) pre[r][b] = ld_coh(src + (size_t)min(b, ns - 1) * prow);
    }
    for (int j = wv; j < G; j += 4) {  // range weights, one wave per head
        const float *part = part0 + (size_t)j * ns * prow;
        float mv[ATT_MAX_SPLIT / 64], lv[ATT_MAX_SPLIT / 64];
#pragma unroll
        for (int k = 0; k < ATT_MAX_SPLIT / 64; k++) {
            const int s = min(lane + 64 * k, ns - 1);
            mv[k] = ld_coh(part + (size_t)s * prow + hd);
            lv[k] = ld_coh(part + (size_t)s * prow + hd + 1);
        }
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < ATT_MAX_SPLIT / 64; k++) m = fmaxf(m, mv[k]);
        m = wave_max(m, 64);
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < ATT_MAX_SPLIT / 64; k++) {
            const int s = lane + 64 * k;
            // zero past ns: the sums below run over whole batches of CB ranges
            // without a branch per range (the clamped partials they then read are
            // finite, so each such term adds an exact zero)
            const float w = (s < ns && lv[k] > 0.0f) ? exp2_hw(mv[k] - m) : 0.0f;
            wts[j * ATT_MAX_SPLIT + s] = w;
            L += s < ns ? lv[k] * w : 0.0f;
        }
        L = wave_sum(L, 64);
        if (lane == 0) Ls[j] = L;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NO; r++) {
        const int i = min(tid + 256 * r, n_out - 1);
        const int j = i / hd;
        const float *src = part0 + (size_t)j * ns * prow + i % hd;
        const float *w = wts + j * ATT_MAX_SPLIT;
        float v[CB];
#pragma unroll
        for (int b = 0; b < CB; b++) v[b] = r < NPF ? pre[r < NPF ? r : 0][b] : ld_coh(src + (size_t)min(b, ns - 1) * prow);
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < CB; b++) acc = fmaf(v[b], w[b], acc);
        for (int s0 = CB; s0 < ns; s0 += CB) {  // ns is a power of two: whole batches
#pragma unroll
            for (int b = 0; b < CB; b++) v[b] = ld_coh(src + (size_t)(s0 + b) * prow);
#pragma unroll
            for (int b = 0; b < CB; b++) acc = fmaf(v[b], w[s0 + b], acc);
        }
        if (tid + 256 * r < n_out) o_s[i] = acc * (1.0f / Ls[j]);
    }
    __syncthreads();
    att_finish<HD, G, 256>(a, h0, o_s);
}

// The same merge for a compile-time range count NS: a thread takes output pairs
// (d, d + 1), one 64-bit agent-scope load per range brings both partial values, and
// every range's load of a batch (at most 64 in flight per thread) is issued before
// the range weights are formed, so a merge over 64 ranges waits for one round trip
// to the coherence point instead of one per 16 ranges.  The sums run over the
// ranges in the same order as combine_group's, with the same weights.
template <int HD, int G, int NS>
__device__ void combine_group_ns(const AttnArgs &a, int h0, float *o_s, float *wts, float *Ls) {
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    static_assert(NS <= 64 && HD % 2 == 0, "one lane per range in the weight pass; pairs of outputs");
    constexpr int hd = HD;
    constexpr size_t prow = (size_t)hd + 2;  // even: every pair (d, d + 1) is 8-byte aligned
    const float *part0 = a.part + (size_t)h0 * NS * prow;
    constexpr int NPAIR = G * hd / 2;
    constexpr int PT = (NPAIR + 255) / 256;                      // pairs per thread
    constexpr int CP = PT * NS <= 64 ? PT : (NS >= 64 ? 1 : 64 / NS);  // pairs per batch of loads
    constexpr int NB = (PT + CP - 1) / CP;
    uint64_t v[CP][NS];
    auto issue = [&](int bt) {
#pragma unroll
        for (int c = 0; c < CP; c++) {
            const int i = 2 * min(tid + 256 * (bt * CP + c), NPAIR - 1);
            const float *src = part0 + (size_t)(i / hd) * NS * prow + i % hd;
#pragma unroll
            for (int s = 0; s < NS; s++)
                v[c][s] = __hip_atomic_load((const uint64_t *)(src + (size_t)s * prow), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    issue(0);
    for (int j = wv; j < G; j += 4) {  // range weights, one wave per head, while the partials are in flight
        const float *part = part0 + (size_t)j * NS * prow;
        float mv = -INFINITY, lv = 0.0f;
        if (lane < NS) {
            mv = ld_coh(part + (size_t)lane * prow + hd);
            lv = ld_coh(part + (size_t)lane * prow + hd + 1);
        }
        const float m = wave_max(mv, 64);
        const float w = (lane < NS && lv > 0.0f) ? exp2_hw(mv - m) : 0.0f;
        if (lane < NS) wts[j * ATT_MAX_SPLIT + lane] = w;
        const float L = wave_sum(lane < NS ? lv * w : 0.0f, 64);
        if (lane == 0) Ls[j] = L;
    }
    __syncthreads();
#pragma unroll
    for (int bt = 0; bt < NB; bt++) {
        if (bt) issue(bt);
#pragma unroll
        for (int c = 0; c < CP; c++) {
            const int pi = tid + 256 * (bt * CP + c);
            const int i = 2 * min(pi, NPAIR - 1), j = i / hd;
            const float *w = wts + j * ATT_MAX_SPLIT;
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                acc0 = fmaf(__uint_as_float((uint32_t)v[c][s]), w[s], acc0);
                acc1 = fmaf(__uint_as_float((uint32_t)(v[c][s] >> 32)), w[s], acc1);
            }
            if (pi < NPAIR) {
                o_s[i] = acc0 * (1.0f / Ls[j]);
                o_s[i + 1] = acc1 * (1.0f / Ls[j]);
            }
        }
    }
    __syncthreads();
    att_finish<HD, G, 256>(a, h0, o_s);
}

// G query heads share a KV head; a workgroup takes H of them (H divides G), so the
// grid is (n_split, n_kv · G / H): blockIdx.y = g · (G / H) + the head slice.
template <int KVT, int HD, int G, int H>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnArgs a, HeadPrepArgs hp) {
    static_assert(G % H == 0, "the head slices tile the group");
    constexpr int SUB = HD / 8;      // lanes per cache row (8 dims each)
    constexpr int MG = H;
    constexpr int PP = 256 / SUB;    // position slots
    constexpr int TP = PP * ATT_NP;  // positions per tile
    const int s_idx = blockIdx.x, g = blockIdx.y / (G / H);
    const int h0 = g * G + (blockIdx.y % (G / H)) * H;  // first query head of the slice
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    constexpr int hd = HD;
    const int p = a.d_pos0 ? *a.d_pos0 : a.pos0;
    const int start = a.window > 0 ? max(0, p + 1 - a.window) : 0;
    const int len = p + 1 - start;
    const int chunk = (len + a.n_split - 1) / a.n_split;
    const int r0 = start + s_idx * chunk;
    const int r1 = min(start + (s_idx + 1) * chunk, p + 1);
    const int pi = tid / SUB, c = tid % SUB;
    constexpr bool cact = true;
    const int d0 = 8 * c;
    constexpr int tb = turbo_block(hd);
    const bool own = r0 <= p && p < r1;  // this range holds the new position

    __shared__ float qs_f[MG * 256];
    __shared__ __align__(16) int8_t qs_i[MG * 256];
    __shared__ float qs_d[MG * 8];
    __shared__ __align__(16) uint8_t mirror[2][KV_MIRROR_SC + 16];  // the new position's encoded K and V rows
    __shared__ float pscr[4][520];                                   // per-wave prep scratch
    __shared__ float wo_s[4][MG * 256];                              // per-wave merged slot states
    __shared__ float wm_s[4][MG], wl_s[4][MG];

    const size_t kv_row0 = (size_t)g * a.slots;
    KvChunk<KVT> kc[ATT_NP], vc[ATT_NP];
    bool ok[ATT_NP];
    // Preparation items: the H query heads, then (range owner only) the new
    // position's K and V; wave w takes items w, w + 4, ...  When a group is split
    // into slices, each slice's range owner writes the same encoded row to the
    // cache (identical bytes) and keeps its own LDS copy.  On the register path
    // every item's loads are issued first (clamped to a valid item, so the count
    // of loads in flight is fixed), then the K/V tile's, and the arithmetic runs
    // while the tile is in flight.
    const int wvu = __builtin_amdgcn_readfirstlane(wv);
    const int nv = H + (own ? 2 : 0);
    const bool fast = prep_fast_ok(hp, hd);
    constexpr int NI = (H + 2 + 3) / 4;
    PrepIn<HD> pin[NI];
    if (fast) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int v = min(wvu + 4 * i, nv - 1), kind = v < H ? 0 : v - H + 1;
            prep_load_fast<HD>(hp, kind, kind == 0 ? h0 + v : g, p, pin[i]);
        }
    }
    constexpr bool MFK = KVT == 2 && HD == 128;  // Turbo4 scores on int8 matrix cores
    load_tile<KVT, PP, ATT_NP, !MFK>(a, kv_row0, r0, pi, r0, r1, hd, d0, tb, kc, vc, ok);  // every row index is in range (mod slots)
    KTileMF kt;
    if constexpr (MFK) load_k_mfma(a, kv_row0, r0, wv, lane, r0, r1, kt);
    if (fast) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int v = wvu + 4 * i, kind = v < H ? 0 : v - H + 1;
            if (v < nv) prep_finish_fast<HD>(hp, kind, kind == 0 ? h0 + v : g, p, pin[i], qs_f + v * hd, kind == 0 ? nullptr : mirror[kind - 1]);
        }
    } else {
        for (int v = wv; v < nv; v += 4) {
            const int kind = v < H ? 0 : v - H + 1;
            prep_head_wave<HD, KVT>(hp, kind, kind == 0 ? h0 + v : g, 0, p, qs_f + v * hd, pscr[wv], pscr[wv] + 256, pscr[wv] + 512,
                               kind == 0 ? nullptr : mirror[kind - 1]);
        }
    }
    __syncthreads();
    float qf[MG][8];
    uint32_t qq[MG][2];
    float qdd[MG];
    query_registers<KVT, MG>(a, H, hd, tb, d0, qs_f, qs_i, qs_d, qf, qq, qdd);
    long qb[4] = {0, 0, 0, 0};  // MFK: B operands, lane l: head l % 16, chunk values 8·(l/16)..+7
    float qdc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    __shared__ float sc_s[MFK ? 64 * MG : 1];
    if constexpr (MFK) {
        const int hh = lane & 15, kg = lane >> 4;
        if (hh < H) {
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                qb[cc] = *(const long *)(qs_i + hh * hd + 32 * cc + 8 * kg);
                qdc[cc] = qs_d[hh * 4 + cc];
            }
        }
    }

    float m_s[MG], l_s[MG], o[MG][8];
#pragma unroll
    for (int j = 0; j < MG; j++) {
        m_s[j] = -INFINITY;
        l_s[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) o[j][i] = 0.0f;
    }
    const bool softcap = a.softcap > 0.0f;
    for (int tile = r0; tile < r1; tile += TP) {
        if (tile != r0) {
            load_tile<KVT, PP, ATT_NP, !MFK>(a, kv_row0, tile, pi, r0, r1, hd, d0, tb, kc, vc, ok);
            if constexpr (MFK) load_k_mfma(a, kv_row0, tile, wv, lane, r0, r1, kt);
        }
        if (own && tile + TP >= r1) {
#pragma unroll
            for (int n = 0; n < ATT_NP; n++)
                if (tile + pi + PP * n == p) {
                    if constexpr (!MFK) load_chunk<KVT>(mirror[0], (const uint16_t *)(mirror[0] + KV_MIRROR_SC), 0, hd, d0, tb, kc[n]);
                    load_chunk<KVT>(mirror[1], (const uint16_t *)(mirror[1] + KV_MIRROR_SC), 0, hd, d0, tb, vc[n]);
                }
            if constexpr (MFK) k_mfma_mirror(tile, wv, lane, p, mirror[0], kt);
        }
        float sc[ATT_NP][MG];
        if constexpr (MFK) mfma_scores<MG>(kt, qb, qdc, wv, lane, sc_s, sc);
        else tile_scores<KVT, SUB, MG>(kc, qf, qq, qdd, c, cact, d0, sc);
        if (softcap) {  // uniform
#pragma unroll
            for (int n = 0; n < ATT_NP; n++)
#pragma unroll
                for (int j = 0; j < MG; j++) sc[n][j] = softcap_f(sc[n][j], a.softcap);
        }
        // Online softmax of this slot's positions, per head.  The running maximum moves
        // only when a score exceeds it by 8 (log2 units): probabilities stay ≤ 2⁸, and
        // the rescale of the state runs only in tiles where some lane's maximum moved.
        float mnew[MG];
        bool grow = false;
#pragma unroll
        for (int j = 0; j < MG; j++) {
            float mx = -INFINITY;
#pragma unroll
            for (int n = 0; n < ATT_NP; n++) {
                sc[n][j] = ok[n] ? sc[n][j] * LOG2E_F : -INFINITY;
                mx = fmaxf(mx, sc[n][j]);
            }
            mnew[j] = mx > m_s[j] + 8.0f ? mx : m_s[j];
            grow |= mnew[j] != m_s[j];
        }
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int j = 0; j < MG; j++) {
                const float al = mnew[j] != -INFINITY ? exp2_hw(m_s[j] - mnew[j]) : 1.0f;
                l_s[j] = l_s[j] * al;
                m_s[j] = mnew[j];
#pragma unroll
                for (int i = 0; i < 8; i++) o[j][i] *= al;
            }
        }
        float pw[ATT_NP][MG];
#pragma unroll
        for (int j = 0; j < MG; j++) {
            const bool any = m_s[j] != -INFINITY;
            float sum = 0.0f;
#pragma unroll
            for (int n = 0; n < ATT_NP; n++) {
                pw[n][j] = any ? exp2_hw(sc[n][j] - m_s[j]) : 0.0f;
                sum += pw[n][j];
            }
            l_s[j] = l_s[j] + sum;
        }
#pragma unroll
        for (int n = 0; n < ATT_NP; n++) {
            float vv[8];
            if constexpr (KVT == 0) {
                chunk_values<KVT>(vc[n], d0, vv);
#pragma unroll
                for (int j = 0; j < MG; j++)
#pragma unroll
                    for (int i = 0; i < 8; i++) o[j][i] = fmaf(pw[n][j], vv[i], o[j][i]);
            } else {  // the chunk's scale goes on the probability (axpy_rotated_4's weight)
                const float vs = chunk_levels<KVT>(vc[n], d0, vv);
#pragma unroll
                for (int j = 0; j < MG; j++) {
                    const float w = pw[n][j] * vs;
#pragma unroll
                    for (int i = 0; i < 8; i++) o[j][i] = fmaf(w, vv[i], o[j][i]);
                }
            }
        }
    }
    // ---- merge the slots of the wave (lane groups SUB apart) ----
    xor_up<SUB, 32>([&](auto oc) {
        constexpr int off = decltype(oc)::value;
#pragma unroll
        for (int j = 0; j < MG; j++) {
            if constexpr (off >= 16) {  // lane pairs by permlane swaps: f(lower lane's slot, upper lane's slot)
                float m0, m1, l0, l1;
                pair_f<off>(m_s[j], m0, m1);
                pair_f<off>(l_s[j], l0, l1);
                const float M = fmaxf(m0, m1);
                const bool any = M != -INFINITY;
                const float a0 = any ? exp2_hw(m0 - M) : 0.0f, a1 = any ? exp2_hw(m1 - M) : 0.0f;
                l_s[j] = l0 * a0 + l1 * a1;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float o0, o1;
                    pair_f<off>(o[j][i], o0, o1);
                    o[j][i] = o0 * a0 + o1 * a1;
                }
                m_s[j] = M;
            } else {
                const float mo = xor_f<off>(m_s[j]), lo = xor_f<off>(l_s[j]);
                const float M = fmaxf(m_s[j], mo);
                const bool any = M != -INFINITY;
                const float a1 = any ? exp2_hw(m_s[j] - M) : 0.0f, a2 = any ? exp2_hw(mo - M) : 0.0f;
                l_s[j] = l_s[j] * a1 + lo * a2;
#pragma unroll
                for (int i = 0; i < 8; i++) o[j][i] = o[j][i] * a1 + xor_f<off>(o[j][i]) * a2;
                m_s[j] = M;
            }
        }
    });
    if (lane < SUB && cact) {
#pragma unroll
        for (int j = 0; j < MG; j++)
#pragma unroll
            for (int i = 0; i < 8; i++) wo_s[wv][j * hd + d0 + i] = o[j][i];
    }
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < MG; j++) {
            wm_s[wv][j] = m_s[j];
            wl_s[wv][j] = l_s[j];
        }
    }
    __syncthreads();
    // ---- merge the 4 waves; store this range's partial (agent-coherent) ----
    const int ns = a.n_split;
    float *part = a.part + (size_t)h0 * ns * (hd + 2);
    for (int i = tid; i < H * hd; i += 256) {
        const int j = i / hd, d = i % hd;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm_s[w][j]);
        float O = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float aw = M != -INFINITY ? exp2_hw(wm_s[w][j] - M) : 0.0f;
            O = fmaf(wo_s[w][j * hd + d], aw, O);
            L = fmaf(wl_s[w][j], aw, L);
        }
        float *pp = part + ((size_t)j * ns + s_idx) * (hd + 2);
        st_coh(pp + d, O);
        if (d == 0) {
            st_coh(pp + hd, M);
            st_coh(pp + hd + 1, L);
        }
    }
    __shared__ int s_last;
    // Publication of the partials.  They are agent-scope atomic stores (written
    // through to the device coherence point), every thread waits for their
    // completion before the barrier, and the merge reads them only with
    // agent-scope atomic loads (read from that point), so the arrival count is a
    // relaxed agent-scope add issued after the barrier, and the last arrival's
    // loads issue after the add has returned.  An agent-scope release or acquire
    // would add a write-back or an invalidation of the whole L2 of the XCD
    // (buffer_wbl2 / buffer_inv), which only plain stores and loads need.
    wait_vmem();
    __syncthreads();
    if (tid == 0) {
        int *cnt = a.counters + blockIdx.y * ATT_CNT_STRIDE;  // one 128-byte line per head slice: no contention between slices
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == ns - 1;
        if (old == ns - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    switch (ns) {  // the decode's range counts (powers of two, 4..64)
    case 4: combine_group_ns<HD, H, 4>(a, h0, qs_f, wo_s[0], wm_s[0]); break;
    case 8: combine_group_ns<HD, H, 8>(a, h0, qs_f, wo_s[0], wm_s[0]); break;
    case 16: combine_group_ns<HD, H, 16>(a, h0, qs_f, wo_s[0], wm_s[0]); break;
    case 32: combine_group_ns<HD, H, 32>(a, h0, qs_f, wo_s[0], wm_s[0]); break;
    case 64: combine_group_ns<HD, H, 64>(a, h0, qs_f, wo_s[0], wm_s[0]); break;
    default: combine_group<HD, H>(a, h0, qs_f, wo_s[0], wm_s[0]); break;
    }
}

// Short contexts (attention_splits returns one range): one workgroup of ATT_HEAD_NT
// threads per query head reads every position of its KV head, so there are no range
// partials and no cross-workgroup arrival count (at a few hundred positions the
// range form's chain of partial stores, release, acquire and reloads costs as much as
// the pass over the cache).  The query heads of a group read the same K/V rows:
// blockIdx.x = j · n_kv + g, so with 8 KV heads the heads of group g share one XCD
// (workgroups are placed on the 8 XCDs round-robin by index) and the repeated reads
// hit its L2; placement affects speed only.  Every workgroup's range holds the new
// position, so each prepares, encodes and appends its K and V row (the workgroups of
// a group write identical bytes) and reads its own LDS copy of it.  Each SUB-lane
// position slot keeps its own online softmax state in registers; the slots are
// merged by lane swaps within a wave and through LDS across the waves.
constexpr int ATT_HEAD_NT = 1024;
constexpr int ATT_HEAD_NP = 8;  // positions per slot per tile
template <int KVT, int HD>
__global__ __launch_bounds__(ATT_HEAD_NT) void attn_decode_head_kernel(AttnArgs a, HeadPrepArgs hp) {
    constexpr int NT = ATT_HEAD_NT, NW = NT / 64;
    constexpr int SUB = HD / 8;   // lanes per cache row (8 dims each)
    constexpr int PP = NT / SUB;  // position slots
    constexpr int NP = ATT_HEAD_NP;
    constexpr int TP = PP * NP;   // positions per tile
    constexpr int hd = HD;
    constexpr int tb = turbo_block(HD);
    const int G = a.n_head / a.n_kv;
    const int g = blockIdx.x % a.n_kv, h = g * G + blockIdx.x / a.n_kv;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int p = a.d_pos0 ? *a.d_pos0 : a.pos0;
    const int r0 = a.window > 0 ? max(0, p + 1 - a.window) : 0;
    const int r1 = p + 1;
    const int pi = tid / SUB, c = tid % SUB;
    const int d0 = 8 * c;

    __shared__ float qs_f[HD];
    __shared__ __align__(16) int8_t qs_i[HD];
    __shared__ float qs_d[HD / 32];
    __shared__ __align__(16) uint8_t mirror[2][KV_MIRROR_SC + 16];  // the new position's encoded K and V rows
    __shared__ float pscr[3][520];                                   // prep scratch of waves 0-2
    __shared__ float wo_s[NW][HD];                                   // per-wave merged slot states
    __shared__ float wm_s[NW], wl_s[NW];
    __shared__ float o_s[HD];

    const size_t kv_row0 = (size_t)g * a.slots;
    KvChunk<KVT> kc[NP], vc[NP];
    bool ok[NP];
    // Preparation items: 0 the query head, 1 and 2 the new position's K and V, one per
    // wave of waves 0-2.  On the register path every wave issues an item's loads (the
    // waves past 2 item 2's, unused), so every wave has the same loads in flight ahead
    // of its tile, and the arithmetic runs while the tile is in flight.
    const int wvu = __builtin_amdgcn_readfirstlane(wv);
    const int item = min(wvu, 2);
    const bool fast = prep_fast_ok(hp, hd);
    PrepIn<HD> pin;
    if (fast) prep_load_fast<HD>(hp, item, item == 0 ? h : g, p, pin);
    load_tile<KVT, PP, NP>(a, kv_row0, r0, pi, r0, r1, hd, d0, tb, kc, vc, ok);  // every row index is in range (mod slots)
    if (wvu < 3) {
        if (fast)
            prep_finish_fast<HD>(hp, item, item == 0 ? h : g, p, pin, qs_f, item == 0 ? nullptr : mirror[item - 1]);
        else
            prep_head_wave<HD, KVT>(hp, item, item == 0 ? h : g, 0, p, qs_f, pscr[item], pscr[item] + 256, pscr[item] + 512,
                                    item == 0 ? nullptr : mirror[item - 1]);
    }
    __syncthreads();
    float qf[1][8];
    uint32_t qq[1][2];
    float qdd[1];
    query_registers<KVT, 1>(a, 1, hd, tb, d0, qs_f, qs_i, qs_d, qf, qq, qdd);

    float m_s = -INFINITY, l_s = 0.0f, o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = 0.0f;
    const bool softcap = a.softcap > 0.0f;
    for (int tile = r0; tile < r1; tile += TP) {
        if (tile != r0) load_tile<KVT, PP, NP>(a, kv_row0, tile, pi, r0, r1, hd, d0, tb, kc, vc, ok);
        if (tile + TP >= r1) {
#pragma unroll
            for (int n = 0; n < NP; n++)
                if (tile + pi + PP * n == p) {
                    load_chunk<KVT>(mirror[0], (const uint16_t *)(mirror[0] + KV_MIRROR_SC), 0, hd, d0, tb, kc[n]);
                    load_chunk<KVT>(mirror[1], (const uint16_t *)(mirror[1] + KV_MIRROR_SC), 0, hd, d0, tb, vc[n]);
                }
        }
        float sc[NP][1];
        tile_scores<KVT, SUB, 1, NP>(kc, qf, qq, qdd, c, true, d0, sc);
        if (softcap) {  // uniform
#pragma unroll
            for (int n = 0; n < NP; n++) sc[n][0] = softcap_f(sc[n][0], a.softcap);
        }
        // online softmax of this slot's positions (log2 units); the running maximum
        // moves only when a score exceeds it by 8, and the state is rescaled only in
        // tiles where some lane's maximum moved
        float mx = -INFINITY;
#pragma unroll
        for (int n = 0; n < NP; n++) {
            sc[n][0] = ok[n] ? sc[n][0] * LOG2E_F : -INFINITY;
            mx = fmaxf(mx, sc[n][0]);
        }
        const float mnew = mx > m_s + 8.0f ? mx : m_s;
        if (__builtin_amdgcn_ballot_w64(mnew != m_s)) {
            const float al = mnew != -INFINITY ? exp2_hw(m_s - mnew) : 1.0f;
            l_s = l_s * al;
            m_s = mnew;
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] *= al;
        }
        float pw[NP];
        {
            const bool any = m_s != -INFINITY;
            float sum = 0.0f;
#pragma unroll
            for (int n = 0; n < NP; n++) {
                pw[n] = any ? exp2_hw(sc[n][0] - m_s) : 0.0f;
                sum += pw[n];
            }
            l_s = l_s + sum;
        }
#pragma unroll
        for (int n = 0; n < NP; n++) {
            float vv[8];
            if constexpr (KVT == 0) {
                chunk_values<KVT>(vc[n], d0, vv);
#pragma unroll
                for (int i = 0; i < 8; i++) o[i] = fmaf(pw[n], vv[i], o[i]);
            } else {  // the chunk's scale goes on the probability (axpy_rotated_4's weight)
                const float w = pw[n] * chunk_levels<KVT>(vc[n], d0, vv);
#pragma unroll
                for (int i = 0; i < 8; i++) o[i] = fmaf(w, vv[i], o[i]);
            }
        }
    }
    // ---- merge the slots of the wave (lane groups SUB apart) ----
    xor_up<SUB, 32>([&](auto oc) {
        constexpr int off = decltype(oc)::value;
        if constexpr (off >= 16) {  // lane pairs by permlane swaps: f(lower lane's slot, upper lane's slot)
            float m0, m1, l0, l1;
            pair_f<off>(m_s, m0, m1);
            pair_f<off>(l_s, l0, l1);
            const float M = fmaxf(m0, m1);
            const bool any = M != -INFINITY;
            const float a0 = any ? exp2_hw(m0 - M) : 0.0f, a1 = any ? exp2_hw(m1 - M) : 0.0f;
            l_s = l0 * a0 + l1 * a1;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float o0, o1;
                pair_f<off>(o[i], o0, o1);
                o[i] = o0 * a0 + o1 * a1;
            }
            m_s = M;
        } else {
            const float mo = xor_f<off>(m_s), lo = xor_f<off>(l_s);
            const float M = fmaxf(m_s, mo);
            const bool any = M != -INFINITY;
            const float a1 = any ? exp2_hw(m_s - M) : 0.0f, a2 = any ? exp2_hw(mo - M) : 0.0f;
            l_s = l_s * a1 + lo * a2;
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = o[i] * a1 + xor_f<off>(o[i]) * a2;
            m_s = M;
        }
    });
    if (lane < SUB) {
#pragma unroll
        for (int i = 0; i < 8; i++) wo_s[wv][d0 + i] = o[i];
    }
    if (lane == 0) {
        wm_s[wv] = m_s;
        wl_s[wv] = l_s;
    }
    __syncthreads();
    // ---- merge the waves, normalize ----
    if (tid < hd) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, wm_s[w]);
        float O = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float aw = M != -INFINITY ? exp2_hw(wm_s[w] - M) : 0.0f;
            O = fmaf(wo_s[w][tid], aw, O);
            L = fmaf(wl_s[w], aw, L);
        }
        o_s[tid] = O * (1.0f / L);
    }
    __syncthreads();
    att_finish<HD, 1, NT>(a, h, o_s);
}

// merge the ranges of one (token, head); undo the rotation; quantize to Q8_0
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int hd = a.hd;
    __shared__ float o_s[256];
    __shared__ float wts[ATT_MAX_SPLIT];
    __shared__ float acc_s[256];
    __shared__ float s_L;
    const float *part = a.part + ((size_t)t * a.n_head + h) * a.n_split * (hd + 2);
    if (tid < 64) {
        float m = -INFINITY;
        for (int s = tid; s < a.n_split; s += 64) m = fmaxf(m, part[(size_t)s * (hd + 2) + hd]);
        m = wave_max(m, 64);
        float L = 0.0f;
        for (int s = tid; s < a.n_split; s += 64) {
            const float ms = part[(size_t)s * (hd + 2) + hd], ls = part[(size_t)s * (hd + 2) + hd + 1];
            const float w = ls > 0.0f ? expf(ms - m) : 0.0f;
            wts[s] = w;
            L += ls * w;
        }
        L = wave_sum(L, 64);
        if (tid == 0) s_L = L;
    }
    __syncthreads();
    const float invL = 1.0f / s_L;
    // nh thread groups of hd threads, group k takes splits k, k+nh, …
    const int nh = hd <= 128 ? 256 / hd : 1;
    const int grp = tid / hd, d = tid % hd;
    float o = 0.0f;
    if (grp < nh) {
#pragma unroll 4
        for (int s = grp; s < a.n_split; s += nh) o = fmaf(part[(size_t)s * (hd + 2) + d], wts[s], o);
    }
    if (grp == 1 && grp < nh) acc_s[d] = o;
    __syncthreads();
    for (int k = 2; k < nh; k++) {  // more than two groups (hd ≤ 64): add in order
        if (grp == k) acc_s[d] += o;
        __syncthreads();
    }
    if (grp == 0) o_s[d] = (nh > 1 ? o + acc_s[d] : o) * invL;
    for (int dd = 256 + tid; dd < hd; dd += 256) {  // hd > 256 is rejected by the host; kept for clarity
        float x = 0.0f;
        for (int s = 0; s < a.n_split; s++) x = fmaf(part[(size_t)s * (hd + 2) + dd], wts[s], x);
        o_s[dd] = x * invL;
    }
    __syncthreads();
    if (a.kv_type == 2) {  // o ← Rᵀ o: block FWHT, then signs (turbo.rs:114-117)
        const int b = turbo_block(hd);
        for (int hstep = 1; hstep < b; hstep *= 2) {
            for (int k = tid; k < hd / 2; k += 256) {
                const int blk = k / (b / 2), kk = k % (b / 2);
                const int j = blk * b + (kk / hstep) * 2 * hstep + (kk % hstep);
                const float x0 = o_s[j], x1 = o_s[j + hstep];
                o_s[j] = x0 + x1;
                o_s[j + hstep] = x0 - x1;
            }
            __syncthreads();
        }
        const float s = 1.0f / sqrtf((float)b);
        for (int d = tid; d < hd; d += 256) o_s[d] = o_s[d] * s * a.turbo_signs[d];
        __syncthreads();
    }
    const size_t qd = (size_t)a.n_head * hd;
    for (int d = tid; d < hd; d += 256) a.att[(size_t)t * qd + (size_t)h * hd + d] = o_s[d];
    if (a.att_fmt == ACT_Q8_0) {
        const int hw = tid >> 5, j = tid & 31;
        for (int bi = hw; bi < hd / 32; bi += 8) {
            const float y = o_s[bi * 32 + j];
            float amax = fabsf(y);
            amax = xmax_f<32>(amax);
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int q = (int)rintf(y * id);
            const int qc = q < -127 ? -127 : (q > 127 ? 127 : q);
            int su = q, scl = qc;
            su = xsum_i<32>(su);
            scl = xsum_i<32>(scl);
            const size_t e = (size_t)t * qd + (size_t)h * hd + bi * 32 + j;
            a.att_q.qs[e] = (int8_t)qc;
            if (j == 0) {
                const size_t blk = e / 32;
                a.att_q.d[blk] = d;
                if (a.att_q.s) a.att_q.s[blk] = d * (float)su;
                if (a.att_q.isum) a.att_q.isum[blk] = scl;
            }
        }
    }
}

template <int KVT, int SUB>
static void launch_split_g(const AttnArgs &a, int G, dim3 grid, hipStream_t st) {
    if (G <= 2) hipLaunchKernelGGL((attn_split_kernel<KVT, SUB, 2>), grid, dim3(256), 0, st, a);
    else if (G <= 4) hipLaunchKernelGGL((attn_split_kernel<KVT, SUB, 4>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((attn_split_kernel<KVT, SUB, 8>), grid, dim3(256), 0, st, a);
}

// Query heads per decode workgroup: groups of 6 or 8 are split in two slices, which
// halves the registers and LDS per workgroup and doubles the workgroups per range
// (the two slices read the same K/V rows; they sit n_split blocks apart, on the
// same XCD when n_split is a multiple of 8, so the second read is an L2 hit).
static int decode_heads_per_wg(int G) { return (G == 6 || G == 8) ? G / 2 : G; }

template <int KVT, int HD>
static void launch_decode_g(const AttnArgs &a, const HeadPrepArgs &hp, int G, dim3 grid, hipStream_t st) {
    const bool split = decode_heads_per_wg(G) != G;
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 1, 1>), grid, dim3(256), 0, st, a, hp); break;
    case 2: hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 2, 2>), grid, dim3(256), 0, st, a, hp); break;
    case 3: hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 3, 3>), grid, dim3(256), 0, st, a, hp); break;
    case 4: hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 4, 4>), grid, dim3(256), 0, st, a, hp); break;
    case 5: hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 5, 5>), grid, dim3(256), 0, st, a, hp); break;
    case 6:
        if (split) hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 6, 3>), grid, dim3(256), 0, st, a, hp);
        else hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 6, 6>), grid, dim3(256), 0, st, a, hp);
        break;
    case 7: hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 7, 7>), grid, dim3(256), 0, st, a, hp); break;
    default:
        if (split) hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 8, 4>), grid, dim3(256), 0, st, a, hp);
        else hipLaunchKernelGGL((attn_decode_kernel<KVT, HD, 8, 8>), grid, dim3(256), 0, st, a, hp);
        break;
    }
}

template <int KVT>
static void launch_decode_kvt(const AttnArgs &a, const HeadPrepArgs &hp, dim3 grid, hipStream_t st) {
    const int G = a.n_head / a.n_kv;
    switch (a.hd) {
    case 64: launch_decode_g<KVT, 64>(a, hp, G, grid, st); break;
    case 128: launch_decode_g<KVT, 128>(a, hp, G, grid, st); break;
    default: launch_decode_g<KVT, 256>(a, hp, G, grid, st); break;
    }
}

static int lanes_per_row(int hd) { return hd <= 16 ? 2 : hd <= 32 ? 4 : hd <= 64 ? 8 : hd <= 128 ? 16 : 32; }

template <int KVT>
static void launch_kvt(const AttnArgs &a, dim3 grid, hipStream_t st) {
    const int G = a.n_head / a.n_kv;
    switch (lanes_per_row(a.hd)) {
    case 2: launch_split_g<KVT, 2>(a, G, grid, st); break;
    case 4: launch_split_g<KVT, 4>(a, G, grid, st); break;
    case 8: launch_split_g<KVT, 8>(a, G, grid, st); break;
    case 16: launch_split_g<KVT, 16>(a, G, grid, st); break;
    default: launch_split_g<KVT, 32>(a, G, grid, st); break;
    }
}

int attention_splits(int n_tok, int n_kv, int max_len, int hd, bool fused) {
    if (n_tok > 1) return std::max(1, std::min(32, 2048 / std::max(1, n_tok * n_kv)));
    // one workgroup per query head while the context fits one tile of that kernel
    // (512 positions at head size 128); with a second tile, a second round trip to
    // memory, it loses to ranges, and so does a larger tile (more threads per CU do
    // not fit the registers, fewer threads with more positions each are slower)
    if (fused && hd > 0 && max_len <= (ATT_HEAD_NT / (hd / 8)) * ATT_HEAD_NP) return 1;
    // single token: about 64 positions per range, the count rounded up to a power
    // of two (so that a captured graph serves a span of context lengths), at most
    // 64 ranges: past 4096 positions the ranges grow instead, since the merge reads
    // every range's partial through one workgroup (at 32K positions, 64 ranges take
    // the attention from 94 to 47 µs per layer against 256)
    const int want = (max_len + 63) / 64;
    int ns = 4;
    while (ns < want && ns < 64) ns *= 2;
    return ns;
}

void launch_attention(const AttnArgs &a, hipStream_t st) {
    if (launch_attention_prompt_mfma(a, st)) return;
    const dim3 grid(a.n_split, a.n_kv, a.n_tok);
    switch (a.kv_type) {
    case 0: launch_kvt<0>(a, grid, st); break;
    case 1: launch_kvt<1>(a, grid, st); break;
    default: launch_kvt<2>(a, grid, st); break;
    }
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.n_head, a.n_tok), dim3(256), 0, st, a);
}

void launch_attention_combine(const AttnArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.n_head, a.n_tok), dim3(256), 0, st, a);
}

bool attention_fused_ok(const AttnArgs &a) {
    const int G = a.n_kv > 0 ? a.n_head / a.n_kv : 0;
    // the range merge reads whole batches of 16 ranges past the first: n_split a power of two
    return a.n_tok == 1 && a.counters && (a.hd == 64 || a.hd == 128 || a.hd == 256) && G >= 1 && G <= 8 && a.n_head == G * a.n_kv &&
           a.n_split >= 1 && a.n_split <= ATT_MAX_SPLIT && (a.n_split & (a.n_split - 1)) == 0;
}

template <int KVT>
static void launch_decode_head_kvt(const AttnArgs &a, const HeadPrepArgs &hp, hipStream_t st) {
    const dim3 grid(a.n_head), block(ATT_HEAD_NT);
    switch (a.hd) {
    case 64: hipLaunchKernelGGL((attn_decode_head_kernel<KVT, 64>), grid, block, 0, st, a, hp); break;
    case 128: hipLaunchKernelGGL((attn_decode_head_kernel<KVT, 128>), grid, block, 0, st, a, hp); break;
    default: hipLaunchKernelGGL((attn_decode_head_kernel<KVT, 256>), grid, block, 0, st, a, hp); break;
    }
}

bool launch_attention_fused(const AttnArgs &a, const HeadPrepArgs &hp, hipStream_t st) {
    if (!attention_fused_ok(a) || hp.n_tok != 1) return false;
    if (a.n_split == 1) {  // one range: one workgroup per query head, no cross-workgroup merge
        switch (a.kv_type) {
        case 0: launch_decode_head_kvt<0>(a, hp, st); break;
        case 1: launch_decode_head_kvt<1>(a, hp, st); break;
        default: launch_decode_head_kvt<2>(a, hp, st); break;
        }
        return true;
    }
    const int G = a.n_head / a.n_kv;
    const dim3 grid(a.n_split, a.n_kv * (G / decode_heads_per_wg(G)), 1);
    switch (a.kv_type) {
    case 0: launch_decode_kvt<0>(a, hp, grid, st); break;
    case 1: launch_decode_kvt<1>(a, hp, grid, st); break;
    default: launch_decode_kvt<2>(a, hp, grid, st); break;
    }
    return true;
}

}  // namespace rie
