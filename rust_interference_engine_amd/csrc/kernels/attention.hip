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
// every workgroup handles one (token, kv head, range), keeps the group's query
// heads in LDS, scores a tile of positions with one lane per position, runs an
// online softmax and accumulates V with lanes over (head, dim).  A combine
// kernel merges the ranges, undoes the TurboQuant rotation, and quantizes the
// result to Q8_0 for the output projection.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"

#include <algorithm>

namespace rie {

__constant__ int8_t KV_LEVELS_I8[16] = {-126, -95, -74, -58, -43, -30, -18, -6, 6, 18, 30, 43, 58, 74, 95, 126};

__device__ __forceinline__ int turbo_block(int d) {
    int b = 1;
    while (d % (b * 2) == 0 && b < 256) b *= 2;
    return b;
}

// one wavefront per (head vector, token); x lives in LDS during the transform
__global__ __launch_bounds__(64) void head_prep_kernel(HeadPrepArgs a) {
    const int t = blockIdx.y;
    const int hh = blockIdx.x;
    const int lane = threadIdx.x;
    const int hd = a.hd;
    const int pos0 = a.d_pos0 ? *a.d_pos0 : a.pos0;
    const int pos = pos0 + t;
    const int qd = a.n_head * hd, kvd = a.n_kv * hd;
    __shared__ float xs[256];
    __shared__ float ys[256];
    int kind;  // 0 q, 1 k, 2 v
    int h;
    const float *src;
    const float *bias;
    const float *nw;
    if (hh < a.n_head) {
        kind = 0; h = hh; src = a.q + (size_t)t * qd + h * hd; bias = a.bq; nw = a.q_norm;
    } else if (hh < a.n_head + a.n_kv) {
        kind = 1; h = hh - a.n_head; src = a.k + (size_t)t * kvd + h * hd; bias = a.bk; nw = a.k_norm;
    } else {
        kind = 2; h = hh - a.n_head - a.n_kv; src = a.v + (size_t)t * kvd + h * hd; bias = a.bv; nw = nullptr;
    }
    for (int e = lane; e < hd; e += 64) {
        float x = src[e];
        if (bias) x += bias[h * hd + e];
        xs[e] = x;
    }
    __syncthreads();
    if (kind < 2) {
        if (nw) {  // ops.rs:17-24: x *= scale·w
            float ss = 0.0f;
            for (int e = lane; e < hd; e += 64) ss = fmaf(xs[e], xs[e], ss);
            ss = wave_sum(ss, 64);
            const float scale = 1.0f / sqrtf(ss / (float)hd + a.eps);
            for (int e = lane; e < hd; e += 64) xs[e] = xs[e] * (scale * nw[e]);
            __syncthreads();
        }
        // RoPE, ops.rs:93-108, with the host-computed cos/sin table row of this position
        const int half = a.rope_dim / 2;
        const float *ct = a.cos_t + (size_t)pos * half;
        const float *st = a.sin_t + (size_t)pos * half;
        for (int e = lane; e < hd; e += 64) {
            float y = xs[e];
            if (e < a.rope_dim) {
                if (a.neox) {
                    const int i = e < half ? e : e - half;
                    const float x0 = xs[i], x1 = xs[i + half];
                    y = e < half ? x0 * ct[i] - x1 * st[i] : x0 * st[i] + x1 * ct[i];
                } else {
                    const int i = e >> 1;
                    const float x0 = xs[2 * i], x1 = xs[2 * i + 1];
                    y = (e & 1) == 0 ? x0 * ct[i] - x1 * st[i] : x0 * st[i] + x1 * ct[i];
                }
            }
            ys[e] = y;
        }
        __syncthreads();
        for (int e = lane; e < hd; e += 64) xs[e] = ys[e];
        __syncthreads();
    }
    if (kind == 0) {
        float *dst = a.q + (size_t)t * qd + h * hd;
        for (int e = lane; e < hd; e += 64) dst[e] = xs[e] * a.attn_scale;
        return;
    }
    if (a.k_out && kind == 1)
        for (int e = lane; e < hd; e += 64) a.k_out[(size_t)t * kvd + h * hd + e] = xs[e];
    const int slot = pos % a.slots;
    const size_t row = (size_t)h * a.slots + slot;
    uint8_t *cache = kind == 1 ? a.k_cache : a.v_cache;
    if (a.kv_type == 0) {
        uint16_t *dst = (uint16_t *)cache + row * hd;
        for (int e = lane; e < hd; e += 64) dst[e] = f2h(xs[e]);
    } else if (a.kv_type == 1) {
        // store_q8_0 (cpu.rs:637-647): round half away from zero, f16 scale
        uint8_t *dst = cache + row * (size_t)(hd / 32 * 34);
        for (int e0 = 0; e0 < hd; e0 += 64) {
            const int e = e0 + lane;
            const float x = e < hd ? xs[e] : 0.0f;
            float amax = fabsf(x);
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int q = (int)roundf(x * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            if (e < hd) {
                uint8_t *blk = dst + (e >> 5) * 34;
                blk[2 + (e & 31)] = (uint8_t)(int8_t)q;
                if ((e & 31) == 0) {
                    const uint16_t hb = f2h(d);
                    blk[0] = (uint8_t)hb;
                    blk[1] = (uint8_t)(hb >> 8);
                }
            }
        }
    } else {
        // TurboQuant-4 (turbo.rs:140-171): signs, block FWHT, RMS codes, LS scale
        for (int e = lane; e < hd; e += 64) xs[e] *= a.turbo_signs[e];
        __syncthreads();
        const int b = turbo_block(hd);
        for (int hstep = 1; hstep < b; hstep *= 2) {
            for (int k = lane; k < hd / 2; k += 64) {
                const int blk = k / (b / 2), kk = k % (b / 2);
                const int j = blk * b + (kk / hstep) * 2 * hstep + (kk % hstep);
                const float x0 = xs[j], x1 = xs[j + hstep];
                xs[j] = x0 + x1;
                xs[j + hstep] = x0 - x1;
            }
            __syncthreads();
        }
        const float s = 1.0f / sqrtf((float)b);
        for (int e = lane; e < hd; e += 64) xs[e] *= s;
        __syncthreads();
        float c[16];
#pragma unroll
        for (int i = 0; i < 16; i++) c[i] = (float)KV_LEVELS_I8[i] / 46.0f;
        uint8_t *codes = cache + row * (size_t)(hd / 2);
        uint16_t *scales = (kind == 1 ? a.k_scale : a.v_scale) + row * (size_t)(hd / b);
        __shared__ float s_inv[8];
        __shared__ uint8_t qv[256];
        const int nbk = hd / b;
        if (lane < nbk) {  // sequential f32 sums, the reference's order
            float ss = 0.0f;
            for (int j = 0; j < b; j++) ss += xs[lane * b + j] * xs[lane * b + j];
            const float rms = sqrtf(ss / (float)b);
            s_inv[lane] = rms > 0.0f ? 1.0f / rms : 0.0f;
        }
        __syncthreads();
        for (int e = lane; e < hd; e += 64) {
            const float v = xs[e] * s_inv[e / b];
            uint8_t q = 0;
#pragma unroll
            for (int k = 0; k < 15; k++) q += (uint8_t)(v > 0.5f * (c[k] + c[k + 1]));
            qv[e] = q;
        }
        __syncthreads();
        for (int i = lane; i < hd / 2; i += 64) {  // byte i holds values g (low) and g+16 (high) of its 32-chunk
            const int g = (i / 16) * 32 + (i % 16);
            codes[i] = (uint8_t)(qv[g] | (qv[g + 16] << 4));
        }
        if (lane < nbk) {
            float num = 0.0f, den = 0.0f;
            for (int j = 0; j < b; j++) {
                const float cq = c[qv[lane * b + j]];
                num += xs[lane * b + j] * cq;
                den += cq * cq;
            }
            scales[lane] = f2h(den > 0.0f ? num / den : 0.0f);
        }
    }
}

void launch_head_prep(const HeadPrepArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(head_prep_kernel, dim3(a.n_head + 2 * a.n_kv, a.n_tok), dim3(64), 0, st, a);
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
        uint32_t r = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t byte = (w[h] >> (8 * i)) & 0xff;
            const uint32_t code = hi ? (byte >> 4) : (byte & 15);
            r |= ((uint32_t)(uint8_t)KV_LEVELS_I8[code]) << (8 * i);
        }
        out[h] = r;
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

    for (int i = tid; i < G * hd; i += 256) qs_f[i] = a.q[(size_t)t * qd + (size_t)g * G * hd + i];
    if (tid < MG) {
        m_run[tid] = -INFINITY;
        l_run[tid] = 0.0f;
    }
    __syncthreads();
    if constexpr (KVT != 0) {
        // the query is rotated (Turbo4) and quantized to Q8_0 once (cpu.rs:585-598)
        if constexpr (KVT == 2) {
            for (int j = 0; j < G; j++) {
                float *x = qs_f + j * hd;
                for (int e = tid; e < hd; e += 256) x[e] *= a.turbo_signs[e];
                __syncthreads();
                for (int hstep = 1; hstep < tb; hstep *= 2) {
                    for (int k = tid; k < hd / 2; k += 256) {
                        const int blk = k / (tb / 2), kk = k % (tb / 2);
                        const int jj = blk * tb + (kk / hstep) * 2 * hstep + (kk % hstep);
                        const float x0 = x[jj], x1 = x[jj + hstep];
                        x[jj] = x0 + x1;
                        x[jj + hstep] = x0 - x1;
                    }
                    __syncthreads();
                }
                const float sq = 1.0f / sqrtf((float)tb);
                for (int e = tid; e < hd; e += 256) x[e] *= sq;
                __syncthreads();
            }
        }
        // RNE Q8_0 quantization of each 32-block, half a wave per block
        const int hw = tid >> 5, j = tid & 31;
        for (int bi = hw; bi < G * hd / 32; bi += 8) {
            const float y = qs_f[bi * 32 + j];
            float amax = fabsf(y);
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int q = (int)rintf(y * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            qs_i[bi * 32 + j] = (int8_t)q;
            if (j == 0) qs_d[bi] = d;
        }
        __syncthreads();
    }
    // this lane's 8 query dims of every head of the group
    float qf[MG][8];
    uint32_t qq[MG][2];
    float qdd[MG];
#pragma unroll
    for (int j = 0; j < MG; j++) {
        const int jj = j < G ? j : 0;
        if constexpr (KVT == 0) {
#pragma unroll
            for (int i = 0; i < 8; i++) qf[j][i] = qs_f[jj * hd + d0 + i];
        } else {
            qq[j][0] = *(const uint32_t *)(qs_i + jj * hd + d0);
            qq[j][1] = *(const uint32_t *)(qs_i + jj * hd + d0 + 4);
            qdd[j] = qs_d[(jj * hd) / 32 + d0 / 32];
        }
    }
    float o[MG][8];
#pragma unroll
    for (int j = 0; j < MG; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) o[j][i] = 0.0f;

    const size_t kv_row0 = (size_t)g * a.slots;
    for (int tile = r0; tile < r1; tile += TP) {
        // ---- K and V of the tile, all loads in flight together ----
        KvChunk<KVT> kc[ATT_NP], vc[ATT_NP];
        bool ok[ATT_NP];
#pragma unroll
        for (int n = 0; n < ATT_NP; n++) {
            const int pos = tile + pi + PP * n;
            ok[n] = pos < r1;
            const size_t row = kv_row0 + (size_t)((ok[n] ? pos : r0) % a.slots);
            load_chunk<KVT>(a.k_cache, a.k_scale, row, hd, d0, tb, kc[n]);
            load_chunk<KVT>(a.v_cache, a.v_scale, row, hd, d0, tb, vc[n]);
        }
        // ---- scores: partial dot over 8 dims, summed over the SUB lanes ----
#pragma unroll
        for (int n = 0; n < ATT_NP; n++) {
#pragma unroll
            for (int j = 0; j < MG; j++) {
                float part = 0.0f;
                if constexpr (KVT == 0) {
                    float kf[8];
                    chunk_values<0>(kc[n], d0, kf);
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
                    // the block's integer dot is exact over its 4 lanes (cpu.rs: per-block int32 sums)
                    const int isum = quad_sum_i(sdot4(kw[1], qq[j][1], sdot4(kw[0], qq[j][0], 0)));
                    const float ks = KVT == 1 ? h2f(kc[n].sc) : h2f(kc[n].sc) * (1.0f / 46.0f);
                    part = (cact && (c & 3) == 0) ? (KVT == 1 ? ks * qdd[j] : qdd[j] * ks) * (float)isum : 0.0f;
                }
                if (!cact) part = 0.0f;
                const float sum = group_sum<SUB>(part);
                if (c == 0 && j < G) sc[j][pi + PP * n] = ok[n] ? softcap_f(sum, a.softcap) : -INFINITY;
            }
        }
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
#pragma unroll
    for (int off = SUB; off < 64; off <<= 1)
#pragma unroll
        for (int j = 0; j < MG; j++)
#pragma unroll
            for (int i = 0; i < 8; i++) o[j][i] += __shfl_xor(o[j][i], off, 64);
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
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int q = (int)rintf(y * id);
            const int qc = q < -127 ? -127 : (q > 127 ? 127 : q);
            int su = q, scl = qc;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) {
                su += __shfl_xor(su, o, 64);
                scl += __shfl_xor(scl, o, 64);
            }
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

template <int KVT>
static void launch_split_kvt(const AttnArgs &a, dim3 grid, hipStream_t st) {
    const int G = a.n_head / a.n_kv;
    const int sub = a.hd <= 16 ? 2 : a.hd <= 32 ? 4 : a.hd <= 64 ? 8 : a.hd <= 128 ? 16 : 32;
    switch (sub) {
    case 2: launch_split_g<KVT, 2>(a, G, grid, st); break;
    case 4: launch_split_g<KVT, 4>(a, G, grid, st); break;
    case 8: launch_split_g<KVT, 8>(a, G, grid, st); break;
    case 16: launch_split_g<KVT, 16>(a, G, grid, st); break;
    default: launch_split_g<KVT, 32>(a, G, grid, st); break;
    }
}

int attention_splits(int n_tok, int n_kv, int max_len) {
    if (n_tok > 1) return std::max(1, std::min(32, 2048 / std::max(1, n_tok * n_kv)));
    // decode: at least 32 ranges, and ranges of at most 256 positions
    return std::min(ATT_MAX_SPLIT, std::max(32, (max_len + 255) / 256));
}

void launch_attention(const AttnArgs &a, hipStream_t st) {
    const dim3 grid(a.n_split, a.n_kv, a.n_tok);
    switch (a.kv_type) {
    case 0: launch_split_kvt<0>(a, grid, st); break;
    case 1: launch_split_kvt<1>(a, grid, st); break;
    default: launch_split_kvt<2>(a, grid, st); break;
    }
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.n_head, a.n_tok), dim3(256), 0, st, a);
}

}  // namespace rie
