// gemm.hip — prompt-batch matmul on CDNA4 int8 MFMA (Q4_0 / Q8_0 weights ×
// Q8_0 activations), the batched counterpart of vec_dot / vec_dot_x4
// (crates/rie-core/src/kernels/mod.rs:136-284, kernels/matmul.rs:119-241).
//
// One wavefront computes 32 weight rows × 32·NT tokens.  Per 32-value block b:
//   I[t][r]  = Σ_k a_q[t][k]·(w_q[r][k] − 8)      v_mfma_i32_32x32x32_i8, exact
//   S[t][r]  = d_a[t][b]·d_w[r][b]                v_mfma_f32_32x32x1f32 (outer product;
//                                                  two blocks' S per instruction)
//   acc      = fma((float)I, S, acc)              VALU
// (Q4_0 codes enter the MFMA as 16·(w_q − 8) and d_w as d_w/16: the same I·S)
// so each block contributes (d_w·d_a)·isum exactly as the reference's block dot
// does; only the order of the f32 sum over blocks differs.  Weights stay in
// their ggml layout: a lane loads its row's 2-block unit (36 / 68 bytes, dword
// aligned) per stage and writes its codes to LDS as int8, for Q4_0 with the
// nibbles unpacked to 16·(q − 8) and the 1/16 on the block scale (once per
// workgroup, not per wave).
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
typedef float v32f __attribute__((ext_vector_type(32)));


struct GemmP {
    const uint8_t *w[3];
    size_t rb[3];
    int rows[3];
    float *out[3];
    int ld[3];
    int epi[3];
    int nseg;
    int rg_end[3];  // cumulative row groups (64 rows) at the end of each segment
    int n_rg;       // row groups in total
    int n_tg;       // token groups
    int glu;        // 0 none; 1 silu / 2 gelu-tanh: seg 0 gate, seg 1 up, out[0] = h
    const int8_t *qs;
    const float *d;
    int n_tok, K;
    int grouped;    // expert groups: one matrix per expert (grp), 64-token tiles from its table
    GroupTiles grp;
    // K split (one segment, not gated or grouped): split 0 runs the segment's
    // epilogue on its partial sum, split i > 0 stores its partial to part[i-1]
    // ([n_tok][ld], stride part_stride floats), which a second launch adds to the
    // output in split order
    int ks;
    float *part;
    size_t part_stride;
};

// A workgroup's token rows: tokens [r0, r_end) of the batch, or gathered rows
// [r0, r_end) of expert e (e < 0: a tile past the grouping's count).  Returned by
// value: the reference-parameter form kept the struct in scratch memory.
struct GTileRows {
    int r0, r_end, e;
};
__device__ __forceinline__ GTileRows gtile_rows(const GemmP &p, int tg, int bn) {
    if (!p.grouped) return GTileRows{tg * bn, p.n_tok, 0};
    if (tg >= *p.grp.n_tiles) return GTileRows{0, 0, -1};
    const int e = p.grp.tile_e[tg], r0 = p.grp.tile_r0[tg];
    return GTileRows{r0, min(p.grp.off[e + 1], r0 + bn), e};
}
__device__ __forceinline__ int gact_row(const GemmP &p, int r) { return p.grouped && p.grp.amap ? p.grp.amap[r] : r; }
__device__ __forceinline__ int gout_row(const GemmP &p, int r) { return p.grouped && p.grp.omap ? p.grp.omap[r] : r; }

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

// ---- LDS-tiled kernel ---------------------------------------------------------
// Workgroup tile: 64 weight rows × 128 tokens, 4 waves as 2 (rows) × 2 (tokens),
// each wave 32 rows × 64 tokens.  Per stage of KC = 4 blocks (128 values of K)
// the workgroup stages the activation codes and scales and the weight codes
// (nibbles kept packed, 16 B/block for Q4_0) and scales in LDS; the next
// stage's global loads are in flight while the current stage is multiplied.
constexpr int G_BM = 64, G_KC = 4;  // G_KC: 32-value blocks per LDS stage
constexpr int G_AST = G_KC * 32 + 16;  // activation row stride in LDS (bytes, padded)

template <int TY>
struct GemmLds {
    static constexpr int QB = 32;                       // weight codes per block in LDS: int8 (Q4_0 unpacked as 16·(q − 8))
    static constexpr int WST = G_KC * QB + 16;          // weight row stride (bytes, padded)
};

// BN tokens per workgroup tile: 128 (two 32-token tiles per wave) or 64 (one)
template <int TY, bool GLU, int BN>
struct __align__(16) GemmStage {
    static constexpr int NW = GLU ? 2 : 1;
    int8_t a[BN * G_AST];
    float da[BN * G_KC];
    uint8_t wq[NW][G_BM * GemmLds<TY>::WST];
    float dw[NW][G_BM * G_KC];
};

// registers holding one stage's global loads before they are written to LDS
template <int TY, bool GLU, int BN>
struct StageRegs {
    static constexpr int NW = GLU ? 2 : 1;
    v4i a[BN / 32];  // the thread's part of its token's 128-byte chunk
    float4 da;
    WUnit<TY> w;
};

// tokA: the activation row of the thread's token (tid / (256/BN)); tokD: of token tid
// (tid < BN); woff: the expert's byte offset in a grouped launch
template <int TY, bool GLU, int BN>
__device__ __forceinline__ void stage_load(const GemmP &p, int sg, int row0, int tokA, int tokD, size_t woff, int b0, int tid,
                                           StageRegs<TY, GLU, BN> &R) {
    const int K = p.K, nb = K >> 5;
    {   // activation codes: thread → (token, part of its 128-byte chunk)
        constexpr int TPT = 256 / BN, NV = 128 / TPT / 16;  // threads per token, 16-byte loads per thread
        const v4i *src = (const v4i *)(p.qs + (size_t)tokA * K + 32 * b0 + 16 * NV * (tid % TPT));
#pragma unroll
        for (int i = 0; i < NV; i++) R.a[i] = src[i];
    }
    if (tid < BN) R.da = *(const float4 *)(p.d + (size_t)tokD * nb + b0);
    {   // weights: thread → (matrix, row, 2-block unit)
        const int nw = GLU ? (tid >> 7) : 0;
        const int idx = tid & 127;
        const int row = min(row0 + (idx >> 1), p.rows[GLU ? 0 : sg] - 1);
        if (GLU || tid < 128) {
            const int s = GLU ? nw : sg;
            load_wunit<TY>(p.w[s] + woff + (size_t)row * p.rb[s], b0 + 2 * (idx & 1), R.w);
        }
    }
}

template <int TY, bool GLU, int BN>
__device__ __forceinline__ void stage_store(GemmStage<TY, GLU, BN> &S, int tid, const StageRegs<TY, GLU, BN> &R) {
    {
        constexpr int TPT = 256 / BN, NV = 128 / TPT / 16;
        v4i *dst = (v4i *)(S.a + (tid / TPT) * G_AST + 16 * NV * (tid % TPT));
#pragma unroll
        for (int i = 0; i < NV; i++) dst[i] = R.a[i];
    }
    if (tid < BN) *(float4 *)(S.da + tid * G_KC) = R.da;
    if (GLU || tid < 128) {
        const int nw = GLU ? (tid >> 7) : 0;
        const int idx = tid & 127, row = idx >> 1, u = idx & 1;
        constexpr int QB = GemmLds<TY>::QB, WST = GemmLds<TY>::WST;
        uint8_t *wq = S.wq[nw] + row * WST + 2 * u * QB;
        float *dw = S.dw[nw] + row * G_KC + 2 * u;
        if constexpr (TY == T_Q4_0) {
            // nibbles → int8 16·(q − 8) once per workgroup: bytes 0..15 of a block are
            // values 0..15 (low nibbles), bytes 16..31 values 16..31 (high nibbles).
            // q ^ 8 is q − 8 as a 4-bit two's complement number, so with every nibble
            // flipped by one XOR, a nibble moved into (or left in) the high half of its
            // byte, low half zero, is the int8 16·(q − 8): 4 instructions per 8 codes.
            // The block's product is then 16·I exactly (|16·I| < 2²⁴) and its weight
            // scale carries the 1/16 (a power of two: d_a·d_w/16 and the fma with 16·I
            // round exactly as d_a·d_w and I do).
            uint32_t q[8];
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(R.w.w[i + 1], R.w.w[i], 2) ^ 0x88888888u;
#pragma unroll
            for (int i = 0; i < 4; i++) q[4 + i] = R.w.w[5 + i] ^ 0x88888888u;
            auto lo16 = [](uint32_t v) { return (v << 4) & 0xF0F0F0F0u; };
            auto hi16 = [](uint32_t v) { return v & 0xF0F0F0F0u; };
#pragma unroll
            for (int b = 0; b < 2; b++) {
                *(uint4 *)(wq + 32 * b) = make_uint4(lo16(q[4 * b]), lo16(q[4 * b + 1]), lo16(q[4 * b + 2]), lo16(q[4 * b + 3]));
                *(uint4 *)(wq + 32 * b + 16) = make_uint4(hi16(q[4 * b]), hi16(q[4 * b + 1]), hi16(q[4 * b + 2]), hi16(q[4 * b + 3]));
            }
            dw[0] = h2f(R.w.w[0] & 0xffff) * 0.0625f;
            dw[1] = h2f(R.w.w[4] >> 16) * 0.0625f;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) ((uint32_t *)wq)[i] = __builtin_amdgcn_alignbyte(R.w.w[i + 1], R.w.w[i], 2);
#pragma unroll
            for (int i = 0; i < 8; i++) ((uint32_t *)wq)[8 + i] = R.w.w[9 + i];
            dw[0] = h2f(R.w.w[0] & 0xffff);
            dw[1] = h2f(R.w.w[8] >> 16);
        }
    }
}

template <int TY, bool GLU, int NT>
__global__ __launch_bounds__(256, (!GLU && NT == 1) ? 3 : 2) void gemm_kernel(GemmP p) {  // one-tile non-gated: three waves per SIMD
    constexpr int NW = GLU ? 2 : 1;
    constexpr int BN = 64 * NT;  // tokens per workgroup tile: NT 32-token tiles per wave, 2 waves along tokens
    constexpr int QB = GemmLds<TY>::QB, WST = GemmLds<TY>::WST;
    __shared__ GemmStage<TY, GLU, BN> st[2];
    const int tid = threadIdx.x;
    const int wv = tid >> 6, l = tid & 63;
    const int wr = wv >> 1, wc = wv & 1;
    // workgroups of one row group share an XCD (id mod 8) and are dispatched together
    // (the K splits of one tile are neighbours in u: the same XCD)
    const int bid = blockIdx.x;
    const int xcd = bid & 7, uk = bid >> 3;
    const int ksi = uk % p.ks, u = uk / p.ks;
    const int tg = u % p.n_tg;
    const int rg = (u / p.n_tg) * 8 + xcd;
    if (rg >= p.n_rg) return;  // whole workgroup: uniform
    const int sg = (!GLU && p.nseg > 1 && rg >= p.rg_end[0]) ? ((p.nseg > 2 && rg >= p.rg_end[1]) ? 2 : 1) : 0;
    const int row0 = (rg - (sg ? p.rg_end[sg - 1] : 0)) * G_BM;
    const GTileRows tr = gtile_rows(p, tg, BN);
    if (tr.e < 0) return;  // whole workgroup: uniform
    const size_t woff = p.grouped ? (size_t)tr.e * p.grp.wstride : 0;
    const int tokA = gact_row(p, min(tr.r0 + tid / (256 / BN), tr.r_end - 1));
    const int tokD = gact_row(p, min(tr.r0 + tid % BN, tr.r_end - 1));
    const int h = l >> 5, m = l & 31;
    const int tok_m = 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
    const int wrow = wr * 32 + m;  // this lane's weight row in the tile (B operand / result column)
    int arow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) arow[t] = wc * 32 * NT + 32 * t + tok_m;

    float acc[NW][NT][16];
#pragma unroll
    for (int a = 0; a < NW; a++)
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][t][v] = 0.0f;
    const v16i zi = {0};
    const v32f zf32 = {0};

    // Stage ring: LDS holds stages s (being multiplied) and s + 1; two register sets
    // hold the global loads of stages s + 1 and s + 2, so a stage's loads are issued
    // two stages before their LDS store.  Load indices past the last stage repeat the
    // last stage and the step count is even, so every load is unconditional and the
    // compiler's wait for a register set counts exactly the loads issued after it.
    // this workgroup's stages: [k0, k0 + n_stages) of the K / 128 (its K split)
    const int all_stages = p.K / (32 * G_KC);
    const int k0 = ksi * all_stages / p.ks;
    const int n_stages = (ksi + 1) * all_stages / p.ks - k0;
    const int last_stage = n_stages - 1;
    StageRegs<TY, GLU, BN> ra, rb;
    stage_load<TY, GLU, BN>(p, sg, row0, tokA, tokD, woff, k0 * G_KC, tid, ra);
    stage_store<TY, GLU, BN>(st[0], tid, ra);
    stage_load<TY, GLU, BN>(p, sg, row0, tokA, tokD, woff, (k0 + min(1, last_stage)) * G_KC, tid, rb);
    __syncthreads();
    // Per stage: all operands of the stage's KC blocks from LDS, then the
    // P = KC·NT·NW tile products in a software pipeline: the MFMAs of product
    // q+1 are issued before the VALU epilogue of product q.
    constexpr int P = G_KC * NT * NW;
    // rl: receives stage s + 2; rs: holds stage s + 1, stored to LDS after stage s
    auto body = [&](int s, StageRegs<TY, GLU, BN> &rl, const StageRegs<TY, GLU, BN> &rs) {
        stage_load<TY, GLU, BN>(p, sg, row0, tokA, tokD, woff, (k0 + min(s + 2, last_stage)) * G_KC, tid, rl);
        if (s < n_stages) {  // workgroup-uniform; the idle step of an odd stage count skips it
            const GemmStage<TY, GLU, BN> &S = st[s & 1];
            v4i bw[G_KC][NW], av[G_KC][NT];
#pragma unroll
            for (int j = 0; j < G_KC; j++) {
#pragma unroll
                for (int a = 0; a < NW; a++) {
                    const uint4 q = *(const uint4 *)(S.wq[a] + wrow * WST + j * QB + 16 * h);
                    bw[j][a] = v4i{(int)q.x, (int)q.y, (int)q.z, (int)q.w};
                }
#pragma unroll
                for (int t = 0; t < NT; t++) av[j][t] = *(const v4i *)(S.a + arow[t] * G_AST + 32 * j + 16 * h);
            }
            // scale operands of the product pairs (2i, 2i + 1): lane half h supplies
            // product 2i + h's, for the two-block outer product v_mfma_f32_32x32x1f32
            // (block h's 32×32 result in registers 16h..16h+15, laid out as a single
            // block's); one such MFMA per two products halves the scale-MFMA cycles
            float sa[P / 2], sb[P / 2];
#pragma unroll
            for (int i = 0; i < P / 2; i++) {
                const int qh = 2 * i + h;
                const int jh = qh / (NT * NW), th = (qh / NW) % NT, ah = qh % NW;
                const int arh = wc * 32 * NT + 32 * th + tok_m;
                sa[i] = S.da[arh * G_KC + jh];
                sb[i] = S.dw[ah][wrow * G_KC + jh];
            }
            v16i Iq[2];
            v32f Sp[2];
            // The MFMAs of product q take an (empty asm) dependency on the finished
            // accumulators of product q-2: at most two result pairs are live, and the
            // MFMAs of q overlap the VALU epilogue of q-1.
            auto issue = [&](int q) {
                const int j = q / (NT * NW), t = (q / NW) % NT, a = q % NW;
                v4i aop = av[j][t];
                if (q >= 2) {
                    const int t2 = ((q - 2) / NW) % NT, a2 = (q - 2) % NW;
                    const float *d = acc[a2][t2];
                    asm volatile("" : "+v"(aop) : "v"(d[0]), "v"(d[1]), "v"(d[2]), "v"(d[3]), "v"(d[4]), "v"(d[5]), "v"(d[6]), "v"(d[7]),
                                 "v"(d[8]), "v"(d[9]), "v"(d[10]), "v"(d[11]), "v"(d[12]), "v"(d[13]), "v"(d[14]), "v"(d[15]));
                }
                Iq[q & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bw[j][a], zi, 0, 0, 0);
                if ((q & 1) == 0) Sp[(q >> 1) & 1] = __builtin_amdgcn_mfma_f32_32x32x1f32(sa[q >> 1], sb[q >> 1], zf32, 0, 0, 0);
            };
            issue(0);
#pragma unroll
            for (int q = 0; q < P; q++) {
                if (q + 1 < P) issue(q + 1);
                // scheduling fences: the epilogue of q stays between the MFMAs of q + 1 and
                // those of q + 2, so it runs while the matrix core works on q + 1 (left to
                // itself the scheduler moves each epilogue right behind its own MFMAs and
                // fills the latency with s_nop)
                __builtin_amdgcn_sched_barrier(0);
                const int t = (q / NW) % NT, a = q % NW;
#pragma unroll
                for (int v = 0; v < 16; v++)
                    acc[a][t][v] = fmaf((float)Iq[q & 1][v], Sp[(q >> 1) & 1][16 * (q & 1) + v], acc[a][t][v]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (s + 1 < n_stages) stage_store<TY, GLU, BN>(st[(s + 1) & 1], tid, rs);
        __syncthreads();
    };
    for (int s = 0; s < n_stages; s += 2) {
        body(s, ra, rb);
        body(s + 1, rb, ra);
    }
    // ---- epilogue: lane holds weight row row0 + wrow for tokens t0 + wc·64 + 32t + 16h + v ----
    const int rows = p.rows[sg];
    const int row = row0 + wrow;
    if (row >= rows) return;
    const int ld = p.ld[sg];
    float *out = ksi ? p.part + (size_t)(ksi - 1) * p.part_stride : p.out[sg];
    const int epi = ksi ? EPI_STORE : p.epi[sg];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = tr.r0 + wc * 32 * NT + 32 * t + 16 * h + v;
            if (r < tr.r_end) {
                float y = acc[0][t][v];
                if constexpr (GLU) y = (p.glu == 2 ? gelu_tanh_f(acc[0][t][v]) : silu_f(acc[0][t][v])) * acc[NW - 1][t][v];
                float *o = out + (size_t)gout_row(p, r) * ld + row;
                if (epi == EPI_ADD) *o += y;
                else *o = y;
            }
        }
}

bool gemm_supported(int ty, size_t K) {
    return ((ty == T_Q4_0 || ty == T_Q8_0) && K % (32 * G_KC) == 0 && K > 0) || gemm_kq_supported(ty, K);
}

// out[t·ld + r] += part[0][…] + … + part[n_part−1][…] for r < rows, in split order
__global__ __launch_bounds__(256) void gemm_add_parts_kernel(float *__restrict__ out, const float *__restrict__ part, size_t stride,
                                                             int n_part, int rows, int ld) {
    const int r = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (r >= rows) return;
    const size_t i = (size_t)t * ld + r;
    float v = out[i];
    for (int k = 0; k < n_part; k++) v += part[(size_t)k * stride + i];
    out[i] = v;
}

// 128-token tiles unless that leaves fewer than two workgroups per CU (256 CUs),
// then 64-token tiles (one 32-token tile per wave); the gated pair always 64.
// One segment with a long K (≥ 48 stages of 128) whose 128-token tiles number
// under 512 keeps the 128-token tiles and splits K in 2 or 4 (each split ≥ 16
// stages) while part holds the extra splits' partial sums (part_cap floats).
template <int TY, bool GLU>
static void launch_t(GemmP p, hipStream_t st, const GroupTiles *grp, float *part, size_t part_cap) {
    const int slots = (p.n_rg + 7) / 8;
    const int tiles128 = slots * 8 * ((p.n_tok + 127) / 128);
    const int n_st = p.K / (32 * G_KC);
    p.ks = 1;
    if (!GLU && !grp && p.nseg == 1 && part && n_st >= 48 && p.n_tok > 64) {
        const size_t plane = (size_t)p.n_tok * p.ld[0];
        while (p.ks < 4 && tiles128 * p.ks < 512 && n_st / (2 * p.ks) >= 16 && (size_t)(2 * p.ks - 1) * plane <= part_cap) p.ks *= 2;
        p.part = part;
        p.part_stride = plane;
    }
    int nt = 2;
    if (GLU || (p.ks == 1 && tiles128 < 512 && p.n_tok > 64)) nt = 1;  // GLU: two register sets of 128-token stages do not fit
    p.n_tg = (p.n_tok + 64 * nt - 1) / (64 * nt);
    if (grp) {  // 64-token tiles from the grouping's table
        static_assert(GROUP_BN == 64, "grouped tiles are one 32-token tile per wave");
        nt = 1;
        p.grouped = 1;
        p.grp = *grp;
        p.n_tg = grp->max_tiles;
    }
    const dim3 grid(slots * 8 * p.n_tg * p.ks);
    if constexpr (!GLU) {
        if (nt == 2) hipLaunchKernelGGL((gemm_kernel<TY, GLU, 2>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((gemm_kernel<TY, GLU, 1>), grid, dim3(256), 0, st, p);
        if (p.ks > 1)
            hipLaunchKernelGGL(gemm_add_parts_kernel, dim3((p.rows[0] + 255) / 256, p.n_tok), dim3(256), 0, st, p.out[0], p.part,
                               p.part_stride, p.ks - 1, p.rows[0], p.ld[0]);
        return;
    }
    hipLaunchKernelGGL((gemm_kernel<TY, GLU, 1>), grid, dim3(256), 0, st, p);
}

void launch_gemm_add_parts(float *out, const float *part, size_t stride, int n_part, int rows, int ld, int n_tok, hipStream_t st) {
    hipLaunchKernelGGL(gemm_add_parts_kernel, dim3((rows + 255) / 256, n_tok), dim3(256), 0, st, out, part, stride, n_part, rows, ld);
}

static bool operands_ok(const ActQ8 &act) { return act.qs && act.d; }

static void set_groups(GemmP &p, int nseg) {
    int acc = 0;
    for (int i = 0; i < 3; i++) {
        if (i < nseg) acc += (p.rows[i] + G_BM - 1) / G_BM;
        p.rg_end[i] = acc;
    }
    p.n_rg = acc;
}

bool launch_gemm(const GemvSeg *segs, int nseg, const ActQ8 &act, int n_tok, int K, hipStream_t st, const GroupTiles *grp, float *part,
                 size_t part_cap) {
    if (nseg < 1 || nseg > 3 || n_tok < 1 || !operands_ok(act) || (grp && (nseg != 1 || grp->max_tiles < 1))) return false;
    const int ty = segs[0].w.ty;
    if (gemm_kq_supported(ty, K)) return launch_gemm_kq(segs, nseg, act, n_tok, K, st, grp, part, part_cap);
    if (grp && grp->bn != GROUP_BN) return false;  // this kernel's grouped tiles are 64 tokens
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
    if (ty == T_Q4_0) launch_t<T_Q4_0, false>(p, st, grp, part, part_cap);
    else launch_t<T_Q8_0, false>(p, st, grp, part, part_cap);
    return true;
}

bool launch_gemm_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, int n_tok, int K, float *h, int ld, int gelu,
                     float *scratch, hipStream_t st, const GroupTiles *grp) {
    (void)scratch;
    if (grp && grp->max_tiles < 1) return false;
    if (gemm_kq_supported(gate.ty, K)) return launch_gemm_kq_glu(gate, up, act, n_tok, K, h, ld, gelu, st, grp);
    if (grp && grp->bn != GROUP_BN) return false;  // this kernel's grouped tiles are 64 tokens
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
    if (gate.ty == T_Q4_0) launch_t<T_Q4_0, true>(p, st, grp, nullptr, 0);
    else launch_t<T_Q8_0, true>(p, st, grp, nullptr, 0);
    return true;
}

}  // namespace rie
