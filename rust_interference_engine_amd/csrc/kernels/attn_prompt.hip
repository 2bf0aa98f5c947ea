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
// Turbo4 caches (KVT = 2, head dim 128, one rotation block per row): attention
// runs in the rotated domain as the reference's does (cpu.rs:584-632, turbo.rs:
// 178-250).  The query is rotated and quantized to Q8_0 first (turbo_query_kernel,
// bitwise the reference's codes), and its dequantized values d·q8 take the place of
// q.  Key and value tiles are the int8 Lloyd–Max levels of their codes (exact in
// f16); a key row's scale/46 multiplies its scores, a value row's scale/46 its
// probabilities before the P·V product (axpy_rotated_4's factor), and the output
// goes back through the inverse rotation (FWHT, 1/√128, signs) in the epilogue.
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

#include <algorithm>
#include <type_traits>

namespace rie {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int PT = 32;         // cache positions per tile
constexpr int VROW = PT * 2 + 8;   // bytes per transposed V row in LDS (padded: 8-row steps shift by 16 banks)

// Lloyd–Max levels of the Turbo4 codes as int8 (turbo.rs:126-127), four per
// dword for v_perm lookups
constexpr int8_t TQ_LEVELS[16] = {-126, -95, -74, -58, -43, -30, -18, -6, 6, 18, 30, 43, 58, 74, 95, 126};
constexpr uint32_t tq_word(int i) {
    return (uint32_t)(uint8_t)TQ_LEVELS[4 * i] | ((uint32_t)(uint8_t)TQ_LEVELS[4 * i + 1] << 8) |
           ((uint32_t)(uint8_t)TQ_LEVELS[4 * i + 2] << 16) | ((uint32_t)(uint8_t)TQ_LEVELS[4 * i + 3] << 24);
}
// four codes (one per byte, 0..15) → their int8 levels (one per byte)
__device__ __forceinline__ uint32_t tq_levels4(uint32_t codes) {
    const uint32_t s7 = codes & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(tq_word(1), tq_word(0), s7), hi = __builtin_amdgcn_perm(tq_word(3), tq_word(2), s7);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((codes >> 3) & 0x01010101u) | 0x0C0C0C0Cu);  // 0xFF where code ≥ 8
    return (hi & m) | (lo & ~m);
}
// byte e of a dword of int8 levels as the bits of an f16 (exact: |level| ≤ 126)
__device__ __forceinline__ uint32_t tq_f16(uint32_t lv, int e) {
    const _Float16 h = (_Float16)(float)(int)(int8_t)((lv >> (8 * e)) & 0xff);
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

typedef float f32x8 __attribute__((ext_vector_type(8)));
// x = hi + lo with hi = x rounded to 11 significant bits in f32 (exact in f16, so
// its conversion cannot round) and lo = x − hi exactly, then rounded to f16
// (|lo| ≤ 2^-11·|x|).  Rounding x to f16 and computing lo from that value instead
// is not safe: the compiler may convert x twice with different instructions
// (v_cvt_f16_f32 for lo, v_cvt_pk_f16_f32 for the packed hi), and values just
// above a rounding midpoint have come out of the two on opposite sides, an error
// of one f16 ulp of x.
__device__ __forceinline__ half8 split_hi(const float (&x)[8], half8 &lo) {
    f32x8 hi, r;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        hi[i] = __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, x[i]) + 0x1000u) & 0xFFFFE000u);
        r[i] = x[i] - hi[i];
    }
    lo = __builtin_convertvector(r, half8);
    return __builtin_convertvector(hi, half8);
}

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

// LDS bytes of one wave group's K and transposed V tile (+ the rows' score and
// probability factors of a Turbo4 tile)
template <int HD, int KVT = 0>
constexpr int tile_bytes() { return PT * (HD * 2 + 16) + HD * VROW + (KVT == 2 ? 2 * PT * 4 : 0); }
// merge scratch of NW groups: running maxima and sums, then one 32-dim output tile per group
template <int NW>
constexpr int merge_bytes() { return NW > 1 ? 2 * NW * 256 * 4 + (NW - 1) * 256 * 16 * 4 : 0; }
template <int HD, int NW, int KVT = 0>
constexpr int prompt_lds_bytes() {
    return 2 * NW * tile_bytes<HD, KVT>() > merge_bytes<NW>() ? 2 * NW * tile_bytes<HD, KVT>() : merge_bytes<NW>();
}

// NW groups of 4 waves: group q handles the tiles q, q + NW, …, and the groups'
// online-softmax states are merged through LDS at the end.
template <int HD, int NW, int KVT>
__global__ __launch_bounds__(256 * NW) void attn_prompt_f16_kernel(AttnArgs a) {
    static_assert(KVT == 0 || (KVT == 2 && HD == 128), "Turbo4 tiles: one 128-dim rotation block per row");
    constexpr int KS = HD / 16;          // 16-dim k-steps of the score product
    constexpr int DT = HD / 32;          // 32-dim output tiles
    constexpr int KROW = HD * 2 + 16;    // bytes per K row in LDS (padded)
    constexpr int NCH = (PT * HD / 8 + 255) / 256;  // 16-byte chunks per thread per tile (K and V each)
    constexpr int RB = KVT == 2 ? HD / 2 : HD * 2;   // cache row bytes
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int TB = tile_bytes<HD, KVT>();
    const int grp = threadIdx.x >> 8;
    uint8_t *const tiles = lds + grp * 2 * TB;  // this group's two tile buffers: K rows, then Vᵀ rows

    const int tid = threadIdx.x & 255, wv = tid >> 6, lane = tid & 63, h = lane >> 5, col = lane & 31;
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

    // workgroup position range, and of it the tiles [t_lo, t_hi) of KV split blockIdx.z
    const int t_first = tr * tbw * 32;
    const int t_last = min(a.n_tok, (tr + 1) * tbw * 32) - 1;
    const int p_hi = pos0 + t_last;
    const int p_lo = a.window > 0 ? max(0, pos0 + t_first + 1 - a.window) : 0;
    const int k0 = p_lo & ~(PT - 1);
    const int n_all = (p_hi - k0) / PT + 1;
    const int per = (n_all + (int)gridDim.z - 1) / (int)gridDim.z;
    const int t_lo = min(n_all, (int)blockIdx.z * per), t_hi = min(n_all, t_lo + per);
    const int n_tiles = t_hi;
    // wave-uniform bounds of its tokens' visible positions
    const int w_tmin = tb * 32, w_tmax = min(a.n_tok, tb * 32 + 32) - 1;
    const int w_pmax = pos0 + w_tmax;
    const int w_smin = a.window > 0 ? max(0, pos0 + w_tmin + 1 - a.window) : 0;
    const int w_pmin = pos0 + w_tmin;                                            // the first token's position
    const int w_smax = a.window > 0 ? max(0, pos0 + w_tmax + 1 - a.window) : 0;  // the last token's window start
    const bool w_full = wave_on && tb * 32 + 31 < a.n_tok;                        // all 32 tokens exist

    // query fragments: token col of the block, dims 16s + 8h .. +8 (f32 → hi + lo)
    half8 qh[KS], ql[KS];
    {
        const int tq = tok_ok ? t : (a.n_tok - 1);
        const float *qrow = a.q + (size_t)tq * qd + (size_t)(wave_on ? head : 0) * hd;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const f32x4 x0 = *(const f32x4 *)(qrow + 16 * s + 8 * h);
            const f32x4 x1 = *(const f32x4 *)(qrow + 16 * s + 8 * h + 4);
            float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            qh[s] = split_hi(x, ql[s]);
        }
    }

    const uint8_t *kc = a.k_cache + (size_t)g * a.slots * RB;
    const uint8_t *vc = a.v_cache + (size_t)g * a.slots * RB;
    const uint16_t *ksc = KVT == 2 ? a.k_scale + (size_t)g * a.slots : nullptr;
    const uint16_t *vsc = KVT == 2 ? a.v_scale + (size_t)g * a.slots : nullptr;
    // one tile in flight in registers: f16 K as 16-byte row chunks and V as two
    // positions × 8 dims; Turbo4 K as 8 code bytes of a row, V as 4 code bytes of two
    // rows, and the row scale of position tid (K) or tid − 32 (V)
    struct Regs {
        u32x4 k[NCH];
        u32x4 v[2];
        uint32_t sc;
    };
    // Every lane issues the same loads (indices past the tile's data repeat valid
    // ones, and ring slots wrap without a branch: slots ≥ 32 = the tile length).
    auto fetch = [&](int tile, Regs &r) {
        const int P0 = k0 + tile * PT;
        const int slot0 = P0 % a.slots;
        const int span = p_hi - P0;  // positions past p_hi repeat row p_hi
        auto slot = [&](int off) {
            const int s0 = slot0 + min(off, span);
            return (size_t)(s0 >= a.slots ? s0 - a.slots : s0);
        };
        auto row = [&](int off) { return slot(off) * RB; };
        if constexpr (KVT == 2) {
            const uint2 kk = *(const uint2 *)(kc + row(tid >> 3) + 8 * (tid & 7));  // position tid/8, bytes 8·(tid%8)..+8
            r.k[0] = u32x4{kk.x, kk.y, 0u, 0u};
#pragma unroll
            for (int rr = 0; rr < 2; rr++)  // positions 2·(tid/16) + rr, bytes 4·(tid%16)..+4
                r.v[rr][0] = *(const uint32_t *)(vc + row(2 * (tid >> 4) + rr) + 4 * (tid & 15));
            r.sc = tid < 32 ? ksc[slot(tid)] : vsc[slot(min(tid - 32, PT - 1))];
        } else {
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                const int ch = min(tid + 256 * c, PT * HD / 8 - 1);
                r.k[c] = *(const u32x4 *)(kc + row(ch / (HD / 8)) + (ch % (HD / 8)) * 16);
            }
            const int vi = min(tid, 2 * HD - 1);  // positions 2·(vi % 16) + {0, 1}, dims 8·(vi / 16) .. +8
#pragma unroll
            for (int rr = 0; rr < 2; rr++) r.v[rr] = *(const u32x4 *)(vc + row(2 * (vi & 15) + rr) + (vi >> 4) * 16);
        }
    };
    auto stage = [&](const Regs &r, int buf) {
        uint8_t *kb = tiles + buf * TB, *vb = kb + PT * KROW;
        if constexpr (KVT == 2) {
            // K row tid/8: code bytes 8c..8c+8 (c = tid%8) of chunk c/2 hold dims
            // 32(c/2) + 8(c%2) + 0..7 (low nibbles) and the same + 16 (high nibbles)
            const int pos = tid >> 3, c = tid & 7;
            const uint32_t w[2] = {r.k[0][0], r.k[0][1]};
#pragma unroll
            for (int half = 0; half < 2; half++) {
                uint32_t lv[2];
#pragma unroll
                for (int q = 0; q < 2; q++) lv[q] = tq_levels4((half ? (w[q] >> 4) : w[q]) & 0x0F0F0F0Fu);
                u32x4 hv;
#pragma unroll
                for (int q = 0; q < 4; q++) hv[q] = tq_f16(lv[q >> 1], 2 * (q & 1)) | (tq_f16(lv[q >> 1], 2 * (q & 1) + 1) << 16);
                *(u32x4 *)(kb + pos * KROW + (32 * (c >> 1) + 8 * (c & 1) + 16 * half) * 2) = hv;
            }
            // Vᵀ: code bytes 4j..4j+4 (j = tid%16) of positions 2·(tid/16) + {0, 1}: dims
            // 32(j/4) + 4(j%4) + 0..3 and the same + 16, one dword = the two positions
            const int pp = tid >> 4, j = tid & 15;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const uint32_t l0 = tq_levels4((half ? (r.v[0][0] >> 4) : r.v[0][0]) & 0x0F0F0F0Fu);
                const uint32_t l1 = tq_levels4((half ? (r.v[1][0] >> 4) : r.v[1][0]) & 0x0F0F0F0Fu);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int dim = 32 * (j >> 2) + 4 * (j & 3) + 16 * half + e;
                    *(uint32_t *)(vb + dim * VROW + 4 * pp) = tq_f16(l0, e) | (tq_f16(l1, e) << 16);
                }
            }
            // per-position factors: score × scale_k/46 (in log2 units), probability ×
            // scale_v/46 × 2^8 (undone in the epilogue; it keeps the f16 halves of small
            // weighted probabilities out of the subnormal range)
            float *fac = (float *)(vb + HD * VROW);
            if (tid < 2 * PT) fac[tid] = h2f(r.sc) * (tid < PT ? LOG2E_F / 46.0f : 256.0f / 46.0f);
            return;
        }
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int ch = tid + 256 * c;
            if (ch < PT * HD / 8) *(u32x4 *)(kb + (ch / (HD / 8)) * KROW + (ch % (HD / 8)) * 16) = r.k[c];
        }
        if (tid < 2 * HD) {  // Vᵀ[dim][pos]: one dword = the two positions of one dim
            uint8_t *dst = vb + 8 * (tid >> 4) * VROW + 4 * (tid & 15);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t w0 = r.v[0][i >> 1], w1 = r.v[1][i >> 1];
                const uint32_t pair = (i & 1) ? ((w0 >> 16) | (w1 & 0xFFFF0000u)) : ((w0 & 0xFFFFu) | (w1 << 16));
                *(uint32_t *)(dst + i * VROW) = pair;
            }
        }
    };

    const uint8_t *k_s = tiles, *v_s = tiles + PT * KROW;  // rebound per tile below
    float m = -INFINITY, l_half = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[d][v] = 0.0f;

    // group tile i is T(i) = t_lo + grp + i·NW; buffer i & 1 holds T(i) during iteration
    // i, and the register sets hold T(i+1) and T(i+2) (issued two iterations before
    // their use)
    const int n_iter = (t_hi - t_lo + NW - 1) / NW;
    // Loads are issued unconditionally (tile indices past the end repeat the last
    // tile; an empty split loads tile 0) so that every wait for a register set is an
    // exact count of the loads issued after it.
    Regs ra, rb;
    const int last = max(n_tiles - 1, 0);
    fetch(min(t_lo + grp, last), ra);
    stage(ra, 0);
    fetch(min(t_lo + grp + NW, last), rb);
    fetch(min(t_lo + grp + 2 * NW, last), ra);
    __syncthreads();
    auto body = [&](int it, Regs &x) {
        const int tile = t_lo + grp + it * NW;
        stage(x, (it + 1) & 1);
        fetch(min(tile + 3 * NW, last), x);
        k_s = tiles + (it & 1) * TB;
        v_s = k_s + PT * KROW;
        const float *fk = (const float *)(v_s + HD * VROW), *fv = fk + PT;  // Turbo4 row factors
        const int P0 = k0 + tile * PT;
        const bool work = tile < n_tiles && wave_on && P0 <= w_pmax && P0 + PT - 1 >= w_smin;
        if (work) {
            // Sᵀ[pos][tok] = Σ_d K[pos][d]·q[tok][d]; the hi and lo halves of q in two chains
            f32x16 s = {}, s2 = {};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const half8 kf = as_half8(*(const u32x4 *)(k_s + col * KROW + (16 * ks + 8 * h) * 2));
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qh[ks], s, 0, 0, 0);
                s2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, ql[ks], s2, 0, 0, 0);
            }
            if constexpr (KVT == 2) {
#pragma unroll
                for (int v = 0; v < 16; v++) s[v] = (s[v] + s2[v]) * fk[8 * (v >> 2) + 4 * h + (v & 3)];
            } else {
#pragma unroll
                for (int v = 0; v < 16; v++) s[v] = (s[v] + s2[v]) * LOG2E_F;
            }
            // lane: token col, positions P0 + 8(v/4) + 4h + v%4; scores in log2 units (q carries log2 e)
            if (a.softcap > 0.0f) {
                const float cl = a.softcap * LOG2E_F;  // the cap in the same units
#pragma unroll
                for (int v = 0; v < 16; v++) s[v] = cl * tanhf(s[v] / cl);
            }
            if (!(w_full && P0 + PT - 1 <= w_pmin && P0 >= w_smax)) {  // a tile that is not visible to every token
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int p = P0 + 8 * (v >> 2) + 4 * h + (v & 3);
                    s[v] = (tok_ok && p >= start_t && p <= pos_t) ? s[v] : -INFINITY;
                }
            }
            float mx = s[0];
#pragma unroll
            for (int v = 1; v < 16; v++) mx = fmaxf(mx, s[v]);
            mx = fmaxf(mx, xor_f<32>(mx));
            // The reference maximum m moves only when a score exceeds it by more than
            // 2^8, so probabilities stay ≤ 256 and the accumulators are rescaled rarely
            // (exact either way: m cancels in O / l).
            // (Turbo4: 2^2, so a weighted probability ≤ 4·scale_v·2^8/46 stays an f16 for row
            // scales — the rotated row's RMS — up to 2944)
            const bool grow = mx > m + (KVT == 2 ? 2.0f : 8.0f);
            if (__builtin_amdgcn_ballot_w64(grow)) {
                const float m_new = grow ? mx : m;
                const float alpha = grow ? exp2_hw(m - m_new) : 1.0f;  // m = −inf: 0
                l_half *= alpha;
#pragma unroll
                for (int d = 0; d < DT; d++)
#pragma unroll
                    for (int v = 0; v < 16; v++) o[d][v] *= alpha;
                m = m_new;
            }
            const float mref = m == -INFINITY ? 0.0f : m;  // no visible position yet: every p is 0
            float pv[16];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                pv[v] = exp2_hw(s[v] - mref);
                l_half += pv[v];
            }
            if constexpr (KVT == 2) {  // the value rows' scale/46 (l keeps the plain probabilities)
#pragma unroll
                for (int v = 0; v < 16; v++) pv[v] *= fv[8 * (v >> 2) + 4 * h + (v & 3)];
            }
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
    };
    // an even number of steps (the last one may be idle), so that the loop has one
    // entry path per register set and every wait count is exact
    for (int it = 0; it < n_iter; it += 2) {
        body(it, rb);
        body(it + 1, ra);
    }
    if constexpr (NW > 1) {  // merge the groups' states into group 0 (the tile buffers are free now)
        float *ms = (float *)lds, *ls = ms + NW * 256, *os = ls + NW * 256;
        ms[grp * 256 + tid] = m;
        ls[grp * 256 + tid] = l_half;
        __syncthreads();
        float M = -INFINITY;
#pragma unroll
        for (int q = 0; q < NW; q++) M = fmaxf(M, ms[q * 256 + tid]);
        const float sc = (M == -INFINITY || m == -INFINITY) ? 0.0f : exp2_hw(m - M);
        float L = 0.0f;
#pragma unroll
        for (int q = 0; q < NW; q++) {
            const float mq = ms[q * 256 + tid];
            L += (M == -INFINITY || mq == -INFINITY) ? 0.0f : ls[q * 256 + tid] * exp2_hw(mq - M);
        }
        l_half = L;
        m = M;  // o and l are relative to the merged maximum from here on
#pragma unroll
        for (int d = 0; d < DT; d++) {
            if (grp > 0)
#pragma unroll
                for (int v = 0; v < 16; v++) os[((grp - 1) * 256 + tid) * 16 + v] = o[d][v] * sc;
            __syncthreads();
            if (grp == 0) {
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    float acc = o[d][v] * sc;
#pragma unroll
                    for (int q = 1; q < NW; q++) acc += os[((q - 1) * 256 + tid) * 16 + v];
                    o[d][v] = acc;
                }
            }
            __syncthreads();
        }
        if (grp > 0) return;
    }
    if (!wave_on) return;
    const float l_tot = l_half + xor_f<32>(l_half);
    if (gridDim.z > 1) {
        // KV split: this range's partial (unnormalized output, maximum in natural-log
        // units, sum) in the layout attn_combine_kernel merges: [t][head][split][hd + 2]
        if (tok_ok) {
            float *pp = a.part + (((size_t)t * a.n_head + head) * gridDim.z + blockIdx.z) * (hd + 2);
            const float osc = KVT == 2 ? 1.0f / 256.0f : 1.0f;
#pragma unroll
            for (int d = 0; d < DT; d++)
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    f32x4 w4;
#pragma unroll
                    for (int e = 0; e < 4; e++) w4[e] = o[d][4 * q4 + e] * osc;
                    *(f32x4 *)(pp + 32 * d + 8 * q4 + 4 * h) = w4;
                }
            if (h == 0) {
                pp[hd] = m == -INFINITY ? -INFINITY : m * LN2_F;
                pp[hd + 1] = l_tot;
            }
        }
        return;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    // lane: token col, dims 32d + 8(v/4) + 4h + v%4
    if constexpr (KVT == 2) {
        // Rᵀ o (turbo.rs:113-117): the normalized FWHT of the rotated output (stages of
        // distance 1, 2, …, 64 as fwht runs them: x[j] = a + b, x[j+h] = a − b), then the
        // signs.  Distance 4 is the half-wave (lane ± 32), the others are in the lane.
        float x[DT][16];
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v++) x[d][v] = o[d][v] * (inv * (1.0f / 256.0f));
        auto bfly = [](float &lo, float &hi) {
            const float p = lo, q = hi;
            lo = p + q;
            hi = p - q;
        };
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v += 2) bfly(x[d][v], x[d][v + 1]);
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                if (!(v & 2)) bfly(x[d][v], x[d][v + 2]);
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float other = xor_f<32>(x[d][v]);
                x[d][v] = h == 0 ? x[d][v] + other : other - x[d][v];
            }
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                if (!(v & 4)) bfly(x[d][v], x[d][v + 4]);
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                if (!(v & 8)) bfly(x[d][v], x[d][v + 8]);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            bfly(x[0][v], x[1][v]);
            bfly(x[2 % DT][v], x[3 % DT][v]);
        }
#pragma unroll
        for (int v = 0; v < 16; v++) {
            bfly(x[0][v], x[2 % DT][v]);
            bfly(x[1 % DT][v], x[3 % DT][v]);
        }
        const float nrm = 1.0f / sqrtf((float)HD);
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int v = 0; v < 16; v++) o[d][v] = x[d][v] * nrm * a.turbo_signs[32 * d + 8 * (v >> 2) + 4 * h + (v & 3)];
    }
#pragma unroll
    for (int d = 0; d < DT; d++) {
        float y[16];
#pragma unroll
        for (int v = 0; v < 16; v++) y[v] = KVT == 2 ? o[d][v] : o[d][v] * inv;
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

template <int HD, int NW, int KVT>
void launch_nw(const AttnArgs &a, dim3 grid, hipStream_t st) {
    constexpr int lds = prompt_lds_bytes<HD, NW, KVT>();
    static const bool attr = hipFuncSetAttribute((const void *)attn_prompt_f16_kernel<HD, NW, KVT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess;
    (void)attr;
    hipLaunchKernelGGL((attn_prompt_f16_kernel<HD, NW, KVT>), grid, dim3(256 * NW), lds, st, a);
}

// Turbo4 query of one (token, head) per wave (turbo.rs:103-112, then the x86
// Q8_0 quantizer, kernels/avx2.rs:153-184, as cpu.rs:584-600 prepares it): lane l
// holds dims 2l, 2l+1; signs, the FWHT stages of distance 1 (in the lane) and
// 2..64 (lane exchanges), ×1/√128, then Q8_0 per 32 dims (16 lanes); writes d·q8.
__global__ __launch_bounds__(64) void turbo_query_kernel(const float *__restrict__ q, int qd, const float *__restrict__ signs,
                                                        float *__restrict__ qhat) {
    const int t = blockIdx.y, hq = blockIdx.x, lane = threadIdx.x;
    const size_t base = (size_t)t * qd + (size_t)hq * 128;
    float x0 = q[base + 2 * lane] * signs[2 * lane], x1 = q[base + 2 * lane + 1] * signs[2 * lane + 1];
    {
        const float a = x0, b = x1;
        x0 = a + b;
        x1 = a - b;
    }
    auto stage = [&](auto oc) {
        constexpr int o = decltype(oc)::value;  // lane distance; dim distance 2·o
        const float p0 = xor_f<o>(x0), p1 = xor_f<o>(x1);
        const bool lo = (lane & o) == 0;
        x0 = lo ? x0 + p0 : p0 - x0;
        x1 = lo ? x1 + p1 : p1 - x1;
    };
    stage(std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 2>{});
    stage(std::integral_constant<int, 4>{});
    stage(std::integral_constant<int, 8>{});
    stage(std::integral_constant<int, 16>{});
    stage(std::integral_constant<int, 32>{});
    const float s = 1.0f / sqrtf(128.0f);
    x0 *= s;
    x1 *= s;
    float amax = fmaxf(fabsf(x0), fabsf(x1));
    amax = fmaxf(amax, xor_f<1>(amax));
    amax = fmaxf(amax, xor_f<2>(amax));
    amax = fmaxf(amax, xor_f<4>(amax));
    amax = fmaxf(amax, xor_f<8>(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int c0 = max(-127, min(127, (int)rintf(x0 * id))), c1 = max(-127, min(127, (int)rintf(x1 * id)));
    qhat[base + 2 * lane] = d * (float)c0;
    qhat[base + 2 * lane + 1] = d * (float)c1;
}

}  // namespace

bool attention_prompt_mfma_ok(const AttnArgs &a) {
    const int G = a.n_kv > 0 ? a.n_head / a.n_kv : 0;
    const bool cache_ok = a.kv_type == 0 || (a.kv_type == 2 && a.hd == 128 && a.turbo_signs && a.k_scale && a.v_scale && a.part);
    return cache_ok && a.n_tok > 1 && !a.d_pos0 && a.slots >= 32 && (a.hd == 32 || a.hd == 64 || a.hd == 96 || a.hd == 128) && G >= 1 &&
           G <= 8 && a.n_head == G * a.n_kv && (a.att_fmt != ACT_Q8_0 || (a.att_q.qs && a.att_q.d));
}

// KV splits of a launch: long rows are split over grid.z workgroups (at least 16
// tiles of 32 positions each, up to about two workgroups per CU, at most 16) whose
// partials attn_combine_kernel merges.  Rows under 1024 positions keep one pass:
// at a 512-token prompt from position 0, two splits (8 tiles each) and the merge
// launch measured 29.3 k tok/s against 31.1 k.
static int prompt_kv_splits(const AttnArgs &a, const dim3 &grid) {
    const int longest = (a.pos0 + a.n_tok - 1) / PT + 1;  // tiles of the last query row (no window)
    const int by_work = longest / 16, by_grid = 512 / (int)(grid.x * grid.y);
    return std::max(1, std::min(16, std::min(by_work, by_grid)));
}

bool launch_attention_prompt_mfma(const AttnArgs &a, hipStream_t st) {
    if (!attention_prompt_mfma_ok(a)) return false;
    const int G = a.n_head / a.n_kv;
    const int wpt = G < 4 ? G : 4, tbw = 4 / wpt, hgroups = (G + 3) / 4;
    dim3 grid((a.n_tok + 32 * tbw - 1) / (32 * tbw), a.n_kv * hgroups);
    const int S = a.window > 0 ? 1 : prompt_kv_splits(a, grid);
    grid.z = S;
    AttnArgs b = a;
    b.n_split = S;
    // partials [t][head][split][hd + 2] at the start of the range-partial buffer; the
    // Turbo4 path's rotated, quantized queries after them
    float *qhat = a.part + (S > 1 ? (size_t)a.n_tok * a.n_head * S * (a.hd + 2) : 0);
    if (a.kv_type == 2) {
        hipLaunchKernelGGL(turbo_query_kernel, dim3(a.n_head, a.n_tok), dim3(64), 0, st, a.q, a.n_head * 128, a.turbo_signs, qhat);
        b.q = qhat;
        launch_nw<128, 2, 2>(b, grid, st);
    } else {
        switch (a.hd) {
        case 32: launch_nw<32, 2, 0>(b, grid, st); break;
        case 64: launch_nw<64, 2, 0>(b, grid, st); break;
        case 96: launch_nw<96, 2, 0>(b, grid, st); break;
        default: launch_nw<128, 2, 0>(b, grid, st); break;
        }
    }
    if (S > 1) launch_attention_combine(b, st);
    return true;
}

}  // namespace rie
