// gemm.hip — prompt-batch matmul on CDNA4 int8 MFMA (Q4_0 / Q8_0 weights ×
// Q8_0 activations), the batched counterpart of vec_dot / vec_dot_x4
// (crates/rie-core/src/kernels/mod.rs:136-284, kernels/matmul.rs:119-241).
//
// One wavefront computes 32 weight rows × 32·NT tokens.  Per 32-value block b:
//   I[t][r]  = Σ_k a_q[t][k]·(w_q[r][k] − 8)      v_mfma_i32_32x32x32_i8, exact
//   S[t][r]  = d_a[t][b]·d_w[r][b]                v_mfma_f32_32x32x2_f32 (rank-1)
//   acc      = fma((float)I, S, acc)              VALU
// so each block contributes (d_w·d_a)·isum exactly as the reference's block dot
// does; only the order of the f32 sum over blocks differs.  Weights stay in
// their ggml layout: a lane loads its row's 2-block unit (36 / 68 bytes, dword
// aligned), unpacks the nibbles of its 16-value half and subtracts 8 bytewise.
//
// Operand lane layout (checked by the parity tests): lane l supplies row
// (l mod 32) and values 16·(l/32)..+16 of the block, for A (tokens) and B
// (weights) alike; the 32×32 result holds column l mod 32 (weight row) and rows
// 8·(v/4) + 4·(l/32) + v mod 4 (v = 0..15).  Tokens are permuted onto A's rows
// so that lane l's 16 results are the 16 consecutive tokens 16·(l/32) + v.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"

#include <algorithm>

namespace rie {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int GEMM_WAVES = 4;                  // row tiles per workgroup
constexpr int GEMM_ROWS = 32 * GEMM_WAVES;     // rows per workgroup

struct GemmP {
    const uint8_t *w[3];
    size_t rb[3];
    int rows[3];
    float *out[3];
    int ld[3];
    int epi[3];
    int nseg;
    int rg_end[3];  // cumulative row groups (GEMM_ROWS rows) at the end of each segment
    int n_rg;       // row groups in total
    int n_tg;       // token groups
    int glu;        // 0 none; 1 silu / 2 gelu-tanh: seg 0 gate, seg 1 up, out[0] = h
    const int8_t *qs;
    const float *d;
    int n_tok, K;
};

// weight unit: blocks b and b+1 of one row (36 or 68 bytes from a dword boundary)
template <int TY>
struct WUnit {
    uint32_t w[TY == T_Q4_0 ? 9 : 17];
};

template <int TY>
__device__ __forceinline__ void load_wunit(const uint8_t *row, int b, WUnit<TY> &u) {
    const uint32_t *p = (const uint32_t *)(row + (size_t)b * (TY == T_Q4_0 ? 18 : 34));
#pragma unroll
    for (int i = 0; i < (TY == T_Q4_0 ? 9 : 17); i++) u.w[i] = wload(p + i);
}

// B operand (16 signed values of this lane's half) and d of block (b + j)
template <int TY>
__device__ __forceinline__ v4i unpack_w(const WUnit<TY> &u, int j, int h, float &dw) {
    v4i r;
    if constexpr (TY == T_Q4_0) {
        uint32_t q[4];
        if (j == 0) {
            dw = h2f(u.w[0] & 0xffff);
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(u.w[i + 1], u.w[i], 2);
        } else {
            dw = h2f(u.w[4] >> 16);
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = u.w[5 + i];
        }
        const uint32_t sh = 4u * (uint32_t)h;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t nib = (q[i] >> sh) & 0x0F0F0F0Fu;
            r[i] = (int)((nib + 0x78787878u) ^ 0x80808080u);  // bytewise q − 8
        }
    } else {
        if (j == 0) {
            dw = h2f(u.w[0] & 0xffff);
#pragma unroll
            for (int i = 0; i < 4; i++) r[i] = (int)__builtin_amdgcn_alignbyte(u.w[4 * h + i + 1], u.w[4 * h + i], 2);
        } else {
            dw = h2f(u.w[8] >> 16);
#pragma unroll
            for (int i = 0; i < 4; i++) r[i] = (int)u.w[9 + 4 * h + i];
        }
    }
    return r;
}

template <int TY, int NT, bool GLU>
__global__ __launch_bounds__(256) void gemm_kernel(GemmP p) {
    constexpr int NW = GLU ? 2 : 1;
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    // workgroups of one row group share an XCD (id mod 8) and are dispatched together
    const int bid = blockIdx.x;
    const int xcd = bid & 7, u = bid >> 3;
    const int tg = u % p.n_tg;
    const int rg = (u / p.n_tg) * 8 + xcd;
    if (rg >= p.n_rg) return;
    const int sg = (!GLU && p.nseg > 1 && rg >= p.rg_end[0]) ? ((p.nseg > 2 && rg >= p.rg_end[1]) ? 2 : 1) : 0;
    const int row0 = (rg - (sg ? p.rg_end[sg - 1] : 0)) * GEMM_ROWS + wv * 32;
    const int rows = p.rows[sg];
    if (row0 >= rows) return;  // no barriers in this kernel: idle waves leave early
    const int h = l >> 5, m = l & 31;
    const int r = min(row0 + m, rows - 1);
    const uint8_t *wrow[NW];
    wrow[0] = p.w[sg] + (size_t)r * p.rb[sg];
    if constexpr (GLU) wrow[1] = p.w[1] + (size_t)r * p.rb[1];
    // A rows: token of row m of each 32-token tile
    const int tok_m = 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
    const int t0 = tg * 32 * NT;
    const int K = p.K, nb = K >> 5;
    const int8_t *arow[NT];
    const float *drow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tok = min(t0 + 32 * t + tok_m, p.n_tok - 1);
        arow[t] = p.qs + (size_t)tok * K + 16 * h;
        drow[t] = p.d + (size_t)tok * nb;
    }
    float acc[NW][NT][16];
#pragma unroll
    for (int a = 0; a < NW; a++)
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][t][v] = 0.0f;
    const v16i zi = {0};
    const v16f zf = {0};

    // software pipeline: the next unit's loads are in flight during this unit's math
    WUnit<TY> wu[NW], wn[NW];
    v4i av[NT][2], an[NT][2];
    float da[NT][2], dn[NT][2];
    auto load_unit = [&](int b, WUnit<TY> *W, v4i (*A)[2], float (*D)[2]) {
#pragma unroll
        for (int a = 0; a < NW; a++) load_wunit<TY>(wrow[a], b, W[a]);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            A[t][0] = *(const v4i *)(arow[t] + 32 * b);
            A[t][1] = *(const v4i *)(arow[t] + 32 * b + 32);
            D[t][0] = drow[t][b];
            D[t][1] = drow[t][b + 1];
        }
    };
    load_unit(0, wu, av, da);
    for (int b = 0; b < nb; b += 2) {
        if (b + 2 < nb) load_unit(b + 2, wn, an, dn);
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int a = 0; a < NW; a++) {
                float dw;
                const v4i bw = unpack_w<TY>(wu[a], j, h, dw);
                const float bs = l < 32 ? dw : 0.0f;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[t][j], bw, zi, 0, 0, 0);
                    const float as = l < 32 ? da[t][j] : 0.0f;
                    const v16f S = __builtin_amdgcn_mfma_f32_32x32x2f32(as, bs, zf, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[a][t][v] = fmaf((float)I[v], S[v], acc[a][t][v]);
                }
            }
        }
        if (b + 2 < nb) {
#pragma unroll
            for (int a = 0; a < NW; a++) wu[a] = wn[a];
#pragma unroll
            for (int t = 0; t < NT; t++) {
                av[t][0] = an[t][0];
                av[t][1] = an[t][1];
                da[t][0] = dn[t][0];
                da[t][1] = dn[t][1];
            }
        }
    }
    // ---- epilogue: lane holds weight row row0 + m for tokens t0 + 32t + 16h + v ----
    const int row = row0 + m;
    if (row >= rows) return;
    float *out = p.out[sg];
    const int ld = p.ld[sg];
    const int epi = p.epi[sg];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int tok = t0 + 32 * t + 16 * h + v;
            if (tok < p.n_tok) {
                float y = acc[0][t][v];
                if constexpr (GLU) {
                    const float g = acc[0][t][v];
                    y = (p.glu == 2 ? gelu_tanh_f(g) : silu_f(g)) * acc[NW - 1][t][v];
                }
                float *o = out + (size_t)tok * ld + row;
                if (epi == EPI_ADD) *o += y;
                else *o = y;
            }
        }
}

bool gemm_supported(int ty, size_t K) { return (ty == T_Q4_0 || ty == T_Q8_0) && K % 64 == 0 && K >= 64; }

template <int TY, int NT, bool GLU>
static void launch_t(GemmP p, hipStream_t st) {
    p.n_tg = (p.n_tok + 32 * NT - 1) / (32 * NT);
    const int slots = (p.n_rg + 7) / 8;
    hipLaunchKernelGGL((gemm_kernel<TY, NT, GLU>), dim3(slots * 8 * p.n_tg), dim3(256), 0, st, p);
}

static bool operands_ok(const ActQ8 &act) { return act.qs && act.d; }

static void set_groups(GemmP &p, int nseg) {
    int acc = 0;
    for (int i = 0; i < 3; i++) {
        if (i < nseg) acc += (p.rows[i] + GEMM_ROWS - 1) / GEMM_ROWS;
        p.rg_end[i] = acc;
    }
    p.n_rg = acc;
}

bool launch_gemm(const GemvSeg *segs, int nseg, const ActQ8 &act, int n_tok, int K, hipStream_t st) {
    if (nseg < 1 || nseg > 3 || n_tok < 1 || !operands_ok(act)) return false;
    const int ty = segs[0].w.ty;
    GemmP p{};
    for (int i = 0; i < nseg; i++) {
        const GemvSeg &s = segs[i];
        if (s.w.ty != ty || !gemm_supported(s.w.ty, K) || s.w.cols != (size_t)K || !s.w.data || !s.out) return false;
        p.w[i] = s.w.data;
        p.rb[i] = s.w.rb();
        p.rows[i] = (int)s.w.rows;
        p.out[i] = s.out;
        p.ld[i] = s.ld;
        p.epi[i] = s.epi;
    }
    p.nseg = nseg;
    set_groups(p, nseg);
    p.glu = 0;
    p.qs = act.qs;
    p.d = act.d;
    p.n_tok = n_tok;
    p.K = K;
    if (ty == T_Q4_0) launch_t<T_Q4_0, 4, false>(p, st);
    else launch_t<T_Q8_0, 4, false>(p, st);
    return true;
}

bool launch_gemm_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, int n_tok, int K, float *h, int ld, int gelu,
                     float *scratch, hipStream_t st) {
    (void)scratch;
    if (n_tok < 1 || !operands_ok(act) || gate.ty != up.ty || !gemm_supported(gate.ty, K) || gate.cols != (size_t)K ||
        up.cols != (size_t)K || gate.rows != up.rows || !gate.data || !up.data || !h)
        return false;
    GemmP p{};
    p.w[0] = gate.data;
    p.w[1] = up.data;
    p.rb[0] = gate.rb();
    p.rb[1] = up.rb();
    p.rows[0] = p.rows[1] = (int)gate.rows;
    p.out[0] = h;
    p.ld[0] = ld;
    p.epi[0] = EPI_STORE;
    p.nseg = 1;
    set_groups(p, 1);
    p.glu = gelu ? 2 : 1;
    p.qs = act.qs;
    p.d = act.d;
    p.n_tok = n_tok;
    p.K = K;
    if (gate.ty == T_Q4_0) launch_t<T_Q4_0, 2, true>(p, st);
    else launch_t<T_Q8_0, 2, true>(p, st);
    return true;
}

}  // namespace rie
