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
constexpr int ATT_TILE = 256;
constexpr int MAXG = 8;

__device__ __forceinline__ void turbo_levels32(const uint8_t *codes, int8_t out[32]) {
    // 16 code bytes → 32 int8 levels in value order (low nibbles 0..15, high 16..31)
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint8_t c = codes[i];
        out[i] = KV_LEVELS_I8[c & 15];
        out[i + 16] = KV_LEVELS_I8[c >> 4];
    }
}

__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
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

    __shared__ float qs_f[MAXG * 256];       // query heads of the group (f32)
    __shared__ int8_t qs_i[MAXG * 256];      // Q8_0 query codes (Q8_0 / Turbo4 caches)
    __shared__ float qs_d[MAXG * 8];         // Q8_0 query block scales
    __shared__ float sc[MAXG][ATT_TILE];     // scores → probabilities of one tile
    __shared__ float m_run[MAXG], l_run[MAXG], alpha[MAXG];

    for (int i = tid; i < G * hd; i += 256) qs_f[i] = a.q[(size_t)t * qd + (size_t)g * G * hd + i];
    if (tid < MAXG) {
        m_run[tid] = -INFINITY;
        l_run[tid] = 0.0f;
    }
    __syncthreads();
    if (a.kv_type != 0) {
        // the query is rotated (Turbo4) and quantized to Q8_0 once (cpu.rs:585-598)
        if (a.kv_type == 2) {
            // rotation: signs then FWHT per block, one head per loop iteration
            const int b = turbo_block(hd);
            for (int j = 0; j < G; j++) {
                float *x = qs_f + j * hd;
                for (int e = tid; e < hd; e += 256) x[e] *= a.turbo_signs[e];
                __syncthreads();
                for (int hstep = 1; hstep < b; hstep *= 2) {
                    for (int k = tid; k < hd / 2; k += 256) {
                        const int blk = k / (b / 2), kk = k % (b / 2);
                        const int jj = blk * b + (kk / hstep) * 2 * hstep + (kk % hstep);
                        const float x0 = x[jj], x1 = x[jj + hstep];
                        x[jj] = x0 + x1;
                        x[jj + hstep] = x0 - x1;
                    }
                    __syncthreads();
                }
                const float s = 1.0f / sqrtf((float)b);
                for (int e = tid; e < hd; e += 256) x[e] *= s;
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

    // V accumulation: an item is (head j, 8-dim chunk c); NI items, P groups of
    // positions; each thread owns one (item, group) and 8 accumulators.
    const int NI = G * (hd / 8);
    const int P = max(1, 256 / NI);
    const int item = tid % NI, pg = tid / NI;
    const bool v_active = tid < NI * P;
    const int vj = item / (hd / 8), vc = item % (hd / 8);
    float o8[8];
#pragma unroll
    for (int i = 0; i < 8; i++) o8[i] = 0.0f;

    const size_t kv_row0 = (size_t)g * a.slots;
    const size_t q8rb = (size_t)(hd / 32) * 34;
    const int tb = turbo_block(hd);
    for (int tile = r0; tile < r1; tile += ATT_TILE) {
        const int nt = min(ATT_TILE, r1 - tile);
        // ---- scores, one lane per position ----
        if (tid < nt) {
            const int slot = (tile + tid) % a.slots;
            const size_t row = kv_row0 + slot;
            float sj[MAXG];
#pragma unroll
            for (int j = 0; j < MAXG; j++) sj[j] = 0.0f;
            if (a.kv_type == 0) {
                const uint4 *kr = (const uint4 *)(a.k_cache + row * hd * 2);
                for (int c = 0; c < hd / 8; c++) {
                    const uint4 kv = kr[c];
                    const uint32_t w4[4] = {kv.x, kv.y, kv.z, kv.w};
                    float kf[8];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        kf[2 * i] = h2f(w4[i] & 0xffff);
                        kf[2 * i + 1] = h2f(w4[i] >> 16);
                    }
                    for (int j = 0; j < G; j++) {
                        const float *qq = qs_f + j * hd + c * 8;
#pragma unroll
                        for (int i = 0; i < 8; i++) sj[j] = fmaf(kf[i], qq[i], sj[j]);
                    }
                }
            } else if (a.kv_type == 1) {
                const uint8_t *kr = a.k_cache + row * q8rb;
                for (int bi = 0; bi < hd / 32; bi++) {
                    const uint8_t *blk = kr + bi * 34;
                    const float dk = h2f(blk[0] | (blk[1] << 8));
                    int8_t kq[32];
#pragma unroll
                    for (int i = 0; i < 32; i++) kq[i] = (int8_t)blk[2 + i];
                    for (int j = 0; j < G; j++) {
                        const int8_t *qq = qs_i + j * hd + bi * 32;
                        int acc = 0;
#pragma unroll
                        for (int i = 0; i < 32; i++) acc += (int)kq[i] * qq[i];
                        sj[j] = fmaf(dk * qs_d[(j * hd) / 32 + bi], (float)acc, sj[j]);
                    }
                }
            } else {
                const uint8_t *kr = a.k_cache + row * (size_t)(hd / 2);
                for (int bi = 0; bi < hd / 32; bi++) {
                    int8_t lv[32];
                    turbo_levels32(kr + bi * 16, lv);
                    const float ks = h2f(a.k_scale[row * (hd / tb) + (bi * 32) / tb]);
                    for (int j = 0; j < G; j++) {
                        const int8_t *qq = qs_i + j * hd + bi * 32;
                        int acc = 0;
#pragma unroll
                        for (int i = 0; i < 32; i++) acc += (int)lv[i] * qq[i];
                        sj[j] = fmaf(qs_d[(j * hd) / 32 + bi] * ks * (1.0f / 46.0f), (float)acc, sj[j]);
                    }
                }
            }
            for (int j = 0; j < G; j++) {
                float v = sj[j];
                if (a.softcap > 0.0f) v = a.softcap * tanhf(v / a.softcap);
                sc[j][tid] = v;
            }
        }
        __syncthreads();
        // ---- online softmax: one wavefront per head ----
        const int wv = tid >> 6, lane = tid & 63;
        for (int j = wv; j < G; j += 4) {
            float mx = -INFINITY;
            for (int i = lane; i < nt; i += 64) mx = fmaxf(mx, sc[j][i]);
            mx = wave_max(mx, 64);
            const float m_new = fmaxf(m_run[j], mx);
            float sum = 0.0f;
            for (int i = lane; i < nt; i += 64) {
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
        // ---- V accumulation: 16-byte V-row loads per (item, position) ----
        if (v_active) {
            const float al = alpha[vj];
#pragma unroll
            for (int i = 0; i < 8; i++) o8[i] *= al;
            for (int pi = pg; pi < nt; pi += P) {
                const size_t row = kv_row0 + (tile + pi) % a.slots;
                const float pw = sc[vj][pi];
                float vv[8];
                if (a.kv_type == 0) {
                    const uint4 w4 = *(const uint4 *)(a.v_cache + (row * hd + vc * 8) * 2);
                    const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        vv[2 * i] = h2f(ww[i] & 0xffff);
                        vv[2 * i + 1] = h2f(ww[i] >> 16);
                    }
                } else if (a.kv_type == 1) {
                    const uint8_t *blk = a.v_cache + row * q8rb + (vc * 8 / 32) * 34;
                    const float dv = h2f(blk[0] | (blk[1] << 8));
#pragma unroll
                    for (int i = 0; i < 8; i++) vv[i] = dv * (float)(int8_t)blk[2 + (vc * 8) % 32 + i];
                } else {
                    const int d0 = vc * 8;
                    const uint8_t *cb = a.v_cache + row * (size_t)(hd / 2) + (d0 / 32) * 16 + (d0 % 16);
                    const bool hi = (d0 % 32) >= 16;
                    const float vs = h2f(a.v_scale[row * (hd / tb) + d0 / tb]) * (1.0f / 46.0f);
#pragma unroll
                    for (int i = 0; i < 8; i++) vv[i] = vs * (float)KV_LEVELS_I8[hi ? (cb[i] >> 4) : (cb[i] & 15)];
                }
#pragma unroll
                for (int i = 0; i < 8; i++) o8[i] = fmaf(pw, vv[i], o8[i]);
            }
        }
        __syncthreads();
    }
    // ---- reduce the position groups, write this range's partial ----
    float *red = &sc[0][0];  // reuse the score tile: P·NI·8 ≤ 8·256 floats
    if (v_active && pg > 0)
#pragma unroll
        for (int i = 0; i < 8; i++) red[((pg - 1) * NI + item) * 8 + i] = o8[i];
    __syncthreads();
    float *part = a.part + (((size_t)t * a.n_head + (size_t)g * G) * a.n_split) * (hd + 2);
    if (v_active && pg == 0) {
        for (int q = 1; q < P; q++)
#pragma unroll
            for (int i = 0; i < 8; i++) o8[i] += red[((q - 1) * NI + item) * 8 + i];
        float *dst = part + ((size_t)vj * a.n_split + s_idx) * (hd + 2) + vc * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) dst[i] = o8[i];
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
    __shared__ float wts[64];
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
    for (int d = tid; d < hd; d += 256) {
        float o = 0.0f;
        for (int s = 0; s < a.n_split; s++) {
            const float w = wts[s];
            if (w != 0.0f) o = fmaf(part[(size_t)s * (hd + 2) + d], w, o);
        }
        o_s[d] = o * invL;
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

void launch_attention(const AttnArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(attn_split_kernel, dim3(a.n_split, a.n_kv, a.n_tok), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.n_head, a.n_tok), dim3(256), 0, st, a);
}

}  // namespace rie
