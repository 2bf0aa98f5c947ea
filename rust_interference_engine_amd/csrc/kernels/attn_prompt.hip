// attn_prompt.hip — causal grouped-query attention of a prompt batch over an f16
// KV cache on CDNA4 f16 matrix cores (flash-attention form, one pass, no range
// partials).  Reference semantics: crates/rie-core/src/model/cpu.rs:550-634
// (scores q·k in f32 over positions start..=pos, optional softcap, softmax,
// out = Σ p·v), with the KV rows at slot pos % slots (cpu.rs:304, 577).
//
// Accuracy: K and V are f16 in the cache, so a product with an f16 operand is
// exact in the f32 accumulator.  The query (f32) is split into q_hi + q_lo
// (two f16 values whose sum carries 22 significant bits) and so is each
// probability p, so every score and every output is an f32-accurate sum of
// exact products; only the summation order differs from the CPU path.
//
// Work split: a workgroup (4 waves) owns one KV head and a block of query rows;
// each wave owns 32 tokens of one query head.  Scores are computed transposed,
// Sᵀ = K·Qᵀ (v_mfma_f32_32x32x16_f16: lane l holds token l mod 32 and 16 cache
// positions), so the online softmax state of a token lives in one lane (plus
// one exchange with the other half-wave), and the output is Oᵀ = Vᵀ·Pᵀ with the
// MFMA's k index mapped onto the positions each lane already holds.  K tiles
// sit row-major in LDS, V tiles transposed ([dim][position]); the next tile's
// loads are in flight while the current one is computed.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"

namespace rie {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int PT = 32;         // cache positions per tile
constexpr int VROW = PT * 2 + 16;  // bytes per transposed V row in LDS (padded)

__device__ __forceinline__ half8 split_hi(const float (&x)[8], half8 &lo) {
    half8 hi;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        hi[i] = (_Float16)x[i];
        lo[i] = (_Float16)(x[i] - (float)hi[i]);
    }
    return hi;
}

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

template <int HD>
__global__ __launch_bounds__(256) void attn_prompt_f16_kernel(AttnArgs a) {
    constexpr int KS = HD / 16;          // 16-dim k-steps of the score product
    constexpr int DT = HD / 32;          // 32-dim output tiles
    constexpr int KROW = HD * 2 + 16;    // bytes per K row in LDS (padded)
    constexpr int NCH = (PT * HD / 8 + 255) / 256;  // 16-byte chunks per thread per tile (K and V each)
    __shared__ __align__(16) uint8_t k_s[PT * KROW];
    __shared__ __align__(16) uint8_t v_s[HD * VROW];

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, h = lane >> 5, col = lane & 31;
    const int G = a.n_head / a.n_kv;
    const int wpt = G < 4 ? G : 4;        // waves per 32-token block (query heads side by side)
    const int tbw = 4 / wpt;              // 32-token blocks per workgroup
    const int hgroups = (G + 3) / 4;      // workgroups per KV head for one token range
    const int tr = gridDim.x - 1 - blockIdx.x;  // the longest rows first
    const int g = blockIdx.y / hgroups, hg = blockIdx.y % hgroups;
    const int j = hg * 4 + wv % wpt;      // query head within the group
    const int tb = tr * tbw + wv / wpt;   // this wave's 32-token block
    const bool wave_on = wv < wpt * tbw && j < G && tb * 32 < a.n_tok;
    const int pos0 = a.pos0;
    const int hd = HD, qd = a.n_head * HD;
    const int head = g * G + j;

    // token of this lane and its visible positions [start_t, pos_t]
    const int t = tb * 32 + col;
    const bool tok_ok = wave_on && t < a.n_tok;
    const int pos_t = pos0 + t;
    const int start_t = a.window > 0 ? max(0, pos_t + 1 - a.window) : 0;

    // workgroup position range
    const int t_first = tr * tbw * 32;
    const int t_last = min(a.n_tok, (tr + 1) * tbw * 32) - 1;
    const int p_hi = pos0 + t_last;
    const int p_lo = a.window > 0 ? max(0, pos0 + t_first + 1 - a.window) : 0;
    const int k0 = p_lo & ~(PT - 1);
    const int n_tiles = (p_hi - k0) / PT + 1;
    // wave-uniform bounds of its tokens' visible positions
    const int w_tmin = tb * 32, w_tmax = min(a.n_tok, tb * 32 + 32) - 1;
    const int w_pmax = pos0 + w_tmax;
    const int w_smin = a.window > 0 ? max(0, pos0 + w_tmin + 1 - a.window) : 0;

    // query fragments: token col of the block, dims 16s + 8h .. +8 (f32 → hi + lo)
    half8 qh[KS], ql[KS];
    {
        const int tq = tok_ok ? t : (a.n_tok - 1);
        const float *qrow = a.q + (size_t)tq * qd + (size_t)(wave_on ? head : 0) * hd;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const f32x4 x0 = *(const f32x4 *)(qrow + 16 * s + 8 * h);
            const f32x4 x1 = *(const f32x4 *)(qrow + 16 * s + 8 * h + 4);
            const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            qh[s] = split_hi(x, ql[s]);
        }
    }

    const uint8_t *kc = a.k_cache + (size_t)g * a.slots * (HD * 2);
    const uint8_t *vc = a.v_cache + (size_t)g * a.slots * (HD * 2);
    u32x4 kr[NCH], vr[NCH];
    auto fetch = [&](int tile) {
        const int P0 = k0 + tile * PT;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int ch = tid + 256 * c;
            const int pos = min(P0 + ch / (HD / 8), p_hi);  // rows past the range repeat a valid one
            const int slot = pos < a.slots ? pos : pos % a.slots;
            const size_t off = (size_t)slot * (HD * 2) + (ch % (HD / 8)) * 16;
            if (ch < PT * HD / 8) {
                kr[c] = *(const u32x4 *)(kc + off);
                vr[c] = *(const u32x4 *)(vc + off);
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int ch = tid + 256 * c;
            if (ch < PT * HD / 8) {
                const int p = ch / (HD / 8), d8 = (ch % (HD / 8)) * 8;
                *(u32x4 *)(k_s + p * KROW + d8 * 2) = kr[c];
                const uint32_t w[4] = {vr[c][0], vr[c][1], vr[c][2], vr[c][3]};
#pragma unroll
                for (int i = 0; i < 8; i++)
                    *(uint16_t *)(v_s + (d8 + i) * VROW + p * 2) = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
            }
        }
    };

    float m = -INFINITY, l_half = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[d][v] = 0.0f;

    fetch(0);
    stage();
    __syncthreads();
    for (int tile = 0; tile < n_tiles; tile++) {
        const int P0 = k0 + tile * PT;
        if (tile + 1 < n_tiles) fetch(tile + 1);
        const bool work = wave_on && P0 <= w_pmax && P0 + PT - 1 >= w_smin;
        if (work) {
            // Sᵀ[pos][tok] = Σ_d K[pos][d]·q[tok][d]
            f32x16 s = {};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const half8 kf = as_half8(*(const u32x4 *)(k_s + col * KROW + (16 * ks + 8 * h) * 2));
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qh[ks], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, ql[ks], s, 0, 0, 0);
            }
            // lane: token col, positions P0 + 8(v/4) + 4h + v%4
            float mx = -INFINITY;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int p = P0 + 8 * (v >> 2) + 4 * h + (v & 3);
                const bool ok = tok_ok && p >= start_t && p <= pos_t;
                float x = s[v];
                if (a.softcap > 0.0f) x = a.softcap * tanhf(x / a.softcap);
                s[v] = ok ? x * LOG2E_F : -INFINITY;
                mx = fmaxf(mx, s[v]);
            }
            mx = fmaxf(mx, xor_f<32>(mx));
            const float m_new = fmaxf(m, mx);
            const bool any = m_new != -INFINITY;
            const float alpha = any ? exp2_hw(m - m_new) : 1.0f;
            float pv[16], psum = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                pv[v] = any ? exp2_hw(s[v] - m_new) : 0.0f;
                psum += pv[v];
            }
            l_half = l_half * alpha + psum;
            m = m_new;
            half8 ph[2], pl[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                float x[8];
#pragma unroll
                for (int i = 0; i < 8; i++) x[i] = pv[8 * u + i];
                ph[u] = split_hi(x, pl[u]);
            }
            // Oᵀ[dim][tok] = alpha·Oᵀ + Σ_pos Vᵀ[dim][pos]·P[tok][pos]; k-slot 8h + i of step u
            // is position 16u + 4h + i (i < 4) or 16u + 8 + 4h + (i − 4)
#pragma unroll
            for (int d = 0; d < DT; d++) {
#pragma unroll
                for (int v = 0; v < 16; v++) o[d][v] *= alpha;
                const uint8_t *vrow = v_s + (32 * d + col) * VROW;
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint2 lo4 = *(const uint2 *)(vrow + (16 * u + 4 * h) * 2);
                    const uint2 hi4 = *(const uint2 *)(vrow + (16 * u + 8 + 4 * h) * 2);
                    u32x4 vv;
                    vv[0] = lo4.x;
                    vv[1] = lo4.y;
                    vv[2] = hi4.x;
                    vv[3] = hi4.y;
                    const half8 vf = as_half8(vv);
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, ph[u], o[d], 0, 0, 0);
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pl[u], o[d], 0, 0, 0);
                }
            }
        }
        __syncthreads();
        if (tile + 1 < n_tiles) {
            stage();
            __syncthreads();
        }
    }
    if (!wave_on) return;
    const float l_tot = l_half + xor_f<32>(l_half);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    // lane: token col, dims 32d + 8(v/4) + 4h + v%4
#pragma unroll
    for (int d = 0; d < DT; d++) {
        float y[16];
#pragma unroll
        for (int v = 0; v < 16; v++) y[v] = o[d][v] * inv;
        if (tok_ok) {
            float *dst = a.att + (size_t)t * qd + (size_t)head * hd + 32 * d + 4 * h;
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                f32x4 w4;
#pragma unroll
                for (int e = 0; e < 4; e++) w4[e] = y[4 * q4 + e];
                *(f32x4 *)(dst + 8 * q4) = w4;
            }
        }
        if (a.att_fmt == ACT_Q8_0) {  // one 32-dim block: 16 values here, 16 in the other half-wave
            float amax = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; v++) amax = fmaxf(amax, fabsf(y[v]));
            amax = fmaxf(amax, xor_f<32>(amax));
            const float dq = amax / 127.0f;
            const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
            int su = 0, scl = 0;
            uint32_t packed[4];
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int q = (int)rintf(y[4 * q4 + e] * id);
                    const int qc = q < -127 ? -127 : (q > 127 ? 127 : q);
                    su += q;
                    scl += qc;
                    w |= ((uint32_t)(qc & 0xff)) << (8 * e);
                }
                packed[q4] = w;
            }
            su += xor_i<32>(su);
            scl += xor_i<32>(scl);
            if (tok_ok) {
                const size_t e0 = (size_t)t * qd + (size_t)head * hd + 32 * d;
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) *(uint32_t *)(a.att_q.qs + e0 + 8 * q4 + 4 * h) = packed[q4];
                if (h == 0) {
                    const size_t blk = e0 / 32;
                    a.att_q.d[blk] = dq;
                    if (a.att_q.s) a.att_q.s[blk] = dq * (float)su;
                    if (a.att_q.isum) a.att_q.isum[blk] = scl;
                }
            }
        }
    }
}

}  // namespace

bool attention_prompt_mfma_ok(const AttnArgs &a) {
    const int G = a.n_kv > 0 ? a.n_head / a.n_kv : 0;
    return a.kv_type == 0 && a.n_tok > 1 && !a.d_pos0 && (a.hd == 32 || a.hd == 64 || a.hd == 96 || a.hd == 128) && G >= 1 &&
           G <= 8 && a.n_head == G * a.n_kv && (a.att_fmt != ACT_Q8_0 || (a.att_q.qs && a.att_q.d));
}

bool launch_attention_prompt_mfma(const AttnArgs &a, hipStream_t st) {
    if (!attention_prompt_mfma_ok(a)) return false;
    const int G = a.n_head / a.n_kv;
    const int wpt = G < 4 ? G : 4, tbw = 4 / wpt, hgroups = (G + 3) / 4;
    const dim3 grid((a.n_tok + 32 * tbw - 1) / (32 * tbw), a.n_kv * hgroups);
    switch (a.hd) {
    case 32: hipLaunchKernelGGL(attn_prompt_f16_kernel<32>, grid, dim3(256), 0, st, a); break;
    case 64: hipLaunchKernelGGL(attn_prompt_f16_kernel<64>, grid, dim3(256), 0, st, a); break;
    case 96: hipLaunchKernelGGL(attn_prompt_f16_kernel<96>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(attn_prompt_f16_kernel<128>, grid, dim3(256), 0, st, a); break;
    }
    return true;
}

}  // namespace rie
