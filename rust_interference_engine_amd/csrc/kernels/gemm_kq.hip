// gemm_kq.hip — prompt-batch matmul of Q4_K weights × Q8_K activations on CDNA4
// int8 MFMA, the batched counterpart of the Q4_K block dot (the x86 prefill tiles
// of kernels/mod.rs:238-296 cover Q4_K; kernels/avx2.rs dot_q4_k 78-107).
//
// Per 256-value superblock b, for activation row t and weight row r:
//   y += (f16(d_r)·d_t)·Σ_j sc_j·Σ_{32} q4·q8 − (f16(dmin_r)·d_t)·Σ_j m_j·(bsum_2j + bsum_2j+1)
// * the eight 32-value sub-block dots are v_mfma_i32_32x32x32_i8 (exact);
// * Σ_j sc_j·I_j is an exact int32 sum (|.| < 2^25);
// * Σ_j m_j·bs_j (< 2^21, exact in f32) and the scale products d·d_t, dmin·d_t are
//   v_mfma_f32_32x32x2_f32 rank-1 / rank-2 products;
// so the superblock's two integer sums equal the reference's exactly and only the
// f32 accumulation over superblocks differs in order.
//
// Workgroup tile: 64 weight rows × 64 tokens, 4 waves as 2 × 2 (32 rows × 32
// tokens each).  A stage is half a superblock (4 sub-blocks, 128 values): the
// activation codes, the superblock's activation scale and 32-value sums, the
// weight nibbles of the half and the row's d, dmin and unpacked 6-bit scales and
// mins go to LDS; the next stage's global loads are in flight meanwhile.
// Operand lane layout as in gemm.hip: lane l supplies row l mod 32 and values
// 16·(l/32)..+16; tokens are permuted onto the A rows so that lane l's 16
// results are the 16 consecutive tokens 16·(l/32) + v.
//
// Q6_K weights × Q8_K activations (kernels/avx2.rs dot_q6_k 109-151): per
// superblock y += (f16(d_r)·d_t)·Σ_k sc_k·Σ_{16} (q6−32)·q8.  The codes are
// unpacked once per stage into int8 q6−32 in LDS (four at a time); each
// 16-value sub-block dot is one v_mfma_i32_32x32x16_i8 (exact), Σ_k sc_k·D_k
// accumulates in int32 with 24-bit multiply-adds (|.| < 2^27), and the
// superblock's float product is the rank-1 f32 MFMA of d_t and d_r.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"
#include "../gemv_units.hpp"

#include <type_traits>

namespace rie {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 half8k __attribute__((ext_vector_type(8)));

struct KqP {
    const uint8_t *w[3];
    size_t rb[3];
    int rows[3];
    float *out[3];
    int ld[3];
    int epi[3];
    int nseg;
    int rg_end[3];  // cumulative 64-row groups at the end of each segment
    int n_rg, n_tg;
    int glu;        // 0 none; 1 silu / 2 gelu-tanh: seg 0 gate, seg 1 up, out[0] = h
    const int8_t *qs;
    const float *d;
    const int16_t *bsums;
    int n_tok, K;
    int grouped;     // expert groups: one matrix per expert (grp), token tiles from its table
    GroupTiles grp;
    // K split (Q6_K, one segment, not grouped): split i takes superblocks
    // [i·nsb/ks, (i+1)·nsb/ks); split 0 runs the segment's epilogue on its partial
    // sum, split i > 0 stores its partial to part[i-1] ([n_tok][ld], stride
    // part_stride floats), which a second launch adds to the output in split order
    int ks;
    float *part;
    size_t part_stride;
};

constexpr int KQ_BM = 64, KQ_BN = 64;
static_assert(KQ_BN == GROUP_BN, "grouped tiles are built for this token tile");
// Q4_K tiles of BN = 32 tokens (groupings of Q4_K experts, a few dozen rows each)
// are 128 weight rows tall: the four waves stand along the rows
template <int BN> constexpr int kq_bm() { return BN == 64 ? 64 : 128; }

// A workgroup's token rows: tokens [r0, r_end) of the batch, or gathered rows
// [r0, r_end) of expert e (e < 0: a tile past the grouping's count, nothing to
// do).  Returned by value: the reference-parameter form kept it in scratch memory.
struct TileRows {
    int r0, r_end, e;
};
template <int BN = KQ_BN>
__device__ __forceinline__ TileRows tile_rows(const KqP &p, int tg) {
    if (!p.grouped) return TileRows{tg * BN, p.n_tok, 0};
    if (tg >= *p.grp.n_tiles) return TileRows{0, 0, -1};
    const int e = p.grp.tile_e[tg], r0 = p.grp.tile_r0[tg];
    return TileRows{r0, min(p.grp.off[e + 1], r0 + BN), e};
}
__device__ __forceinline__ int act_row(const KqP &p, int r) { return p.grouped && p.grp.amap ? p.grp.amap[r] : r; }
__device__ __forceinline__ int out_row(const KqP &p, int r) { return p.grouped && p.grp.omap ? p.grp.omap[r] : r; }
constexpr int KA_ST = 128 + 16;  // activation bytes per token in LDS (one half superblock, padded)
constexpr int KW_ST = 64 + 16;   // weight nibble bytes per row in LDS (one half superblock, padded)

// BN = 32 keeps the 6-bit scales and mins as bytes, so that two 128-row stages of
// the gated pair fit two workgroups in a CU's LDS.
template <bool GLU, int BN = KQ_BN>
struct __align__(16) KqStage {
    static constexpr int NW = GLU ? 2 : 1, BM = kq_bm<BN>();
    using ScT = std::conditional_t<BN == 64, int, uint8_t>;
    using MnT = std::conditional_t<BN == 64, float, uint8_t>;
    int8_t a[BN * KA_ST];
    float da[BN];
    float bs[BN * 8];              // the superblock's 32-value activation sums (both halves hold all 8)
    uint8_t wq[NW][BM * KW_ST];
    float wd[NW][BM], wdm[NW][BM];
    ScT wsc[NW][BM * 8];           // 6-bit scales of the 8 sub-blocks
    MnT wm[NW][BM * 8];            // 6-bit mins
};

template <bool GLU, int BN = KQ_BN>
struct KqRegs {
    static constexpr int NA = BN == 64 ? 2 : 1, NQ = (BN == 32 && GLU) ? 4 : 2;
    v4i a[NA];        // 32 (BN 64) or 16 (BN 32) activation bytes of the thread's token
    float da;
    v4i bs[2];        // the token's 16 bsums (int16)
    v4i wq[NQ];       // 32 nibble bytes of the thread's row (64, both units, in the 32-token gated form)
    v4i hdr;          // d, dmin, scales[12]
};

// stage loads for half hs of superblock sb
// tokA: the activation row of the thread's token (tid/4, or tid/8 for BN 32); tokD: of
// token tid (tid < BN); woff: the expert's byte offset in a grouped launch
template <bool GLU, int BN = KQ_BN>
__device__ __forceinline__ void kq_load(const KqP &p, int sg, int row0, int tokA, int tokD, size_t woff, int sb, int hs, int tid,
                                        KqRegs<GLU, BN> &R) {
    const int K = p.K, nsb = K >> 8;
    if constexpr (BN == 64) {
        const v4i *src = (const v4i *)(p.qs + (size_t)tokA * K + 256 * sb + 128 * hs + 32 * (tid & 3));
        R.a[0] = src[0];
        R.a[1] = src[1];
    } else {
        R.a[0] = *(const v4i *)(p.qs + (size_t)tokA * K + 256 * sb + 128 * hs + 16 * (tid & 7));
    }
    if (tid < BN) {
        R.da = p.d[(size_t)tokD * nsb + sb];
        const v4i *bsrc = (const v4i *)(p.bsums + (size_t)tokD * (K >> 4) + 16 * sb);
        R.bs[0] = bsrc[0];
        R.bs[1] = bsrc[1];
    }
    if constexpr (BN == 32 && GLU) {  // thread → (matrix, row): both units of the half
        const int nw = tid >> 7;
        const int row = min(row0 + (tid & 127), p.rows[0] - 1);
        const uint8_t *blk = p.w[nw] + woff + (size_t)row * p.rb[nw] + 144 * (size_t)sb;
        const v4i *q = (const v4i *)(blk + 16 + 64 * hs);
#pragma unroll
        for (int i = 0; i < 4; i++) R.wq[i] = wload(q + i);
        R.hdr = wload((const v4i *)blk);
    } else if (GLU || BN == 32 || tid < 128) {  // thread → (matrix, row, unit)
        const int nw = (GLU && BN == 64) ? (tid >> 7) : 0, idx = BN == 64 ? (tid & 127) : tid, u = idx & 1;
        const int s = GLU ? nw : sg;
        const int row = min(row0 + (idx >> 1), p.rows[GLU ? 0 : sg] - 1);
        const uint8_t *blk = p.w[s] + woff + (size_t)row * p.rb[s] + 144 * (size_t)sb;
        const v4i *q = (const v4i *)(blk + 16 + 64 * hs + 32 * u);
        R.wq[0] = wload(q);
        R.wq[1] = wload(q + 1);
        R.hdr = wload((const v4i *)blk);
    }
}

template <bool GLU, int BN = KQ_BN>
__device__ __forceinline__ void kq_store(KqStage<GLU, BN> &S, int tid, const KqRegs<GLU, BN> &R) {
    if constexpr (BN == 64) {
        v4i *dst = (v4i *)(S.a + (tid >> 2) * KA_ST + 32 * (tid & 3));
        dst[0] = R.a[0];
        dst[1] = R.a[1];
    } else {
        *(v4i *)(S.a + (tid >> 3) * KA_ST + 16 * (tid & 7)) = R.a[0];
    }
    if (tid < BN) {
        S.da[tid] = R.da;
        const uint32_t w[8] = {(uint32_t)R.bs[0][0], (uint32_t)R.bs[0][1], (uint32_t)R.bs[0][2], (uint32_t)R.bs[0][3],
                               (uint32_t)R.bs[1][0], (uint32_t)R.bs[1][1], (uint32_t)R.bs[1][2], (uint32_t)R.bs[1][3]};
#pragma unroll
        for (int j = 0; j < 8; j++)  // bsum_2j + bsum_2j+1 = the two int16 halves of dword j
            S.bs[tid * 8 + j] = (float)((int)(int16_t)(w[j] & 0xffff) + (int)(int16_t)(w[j] >> 16));
    }
    if (GLU || BN == 32 || tid < 128) {
        int nw, row, u;
        if constexpr (BN == 32 && GLU) {
            nw = tid >> 7;
            row = tid & 127;
            u = 0;
            v4i *dst = (v4i *)(S.wq[nw] + row * KW_ST);
#pragma unroll
            for (int i = 0; i < 4; i++) dst[i] = R.wq[i];
        } else {
            nw = (GLU && BN == 64) ? (tid >> 7) : 0;
            const int idx = BN == 64 ? (tid & 127) : tid;
            row = idx >> 1;
            u = idx & 1;
            v4i *dst = (v4i *)(S.wq[nw] + row * KW_ST + 32 * u);
            dst[0] = R.wq[0];
            dst[1] = R.wq[1];
        }
        if (u == 0) {
            const uint32_t h0 = (uint32_t)R.hdr[0], h1 = (uint32_t)R.hdr[1], h2 = (uint32_t)R.hdr[2], h3 = (uint32_t)R.hdr[3];
            S.wd[nw][row] = h2f(h0 & 0xffff);
            S.wdm[nw][row] = h2f(h0 >> 16);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                q4k_scale_min(h1, h2, h3, j, sc, mn);  // get_scale_min_k4 (quant/reference.rs:8-16)
                S.wsc[nw][row * 8 + j] = (typename KqStage<GLU, BN>::ScT)sc;
                S.wm[nw][row * 8 + j] = (typename KqStage<GLU, BN>::MnT)mn;
            }
        }
    }
}

// c + a·b for |a|, |b| < 2^23 on the full-rate 24-bit multiplier (v_mul_i32_i24,
// folded into v_mad_i32_i24 where the compiler can); a 32-bit product would be the
// quarter-rate v_mul_lo_u32.  Plain code, not inline asm: b is an MFMA result, and
// the compiler inserts the wait states between an MFMA and a VALU read of its
// result only for instructions it generates itself.
__device__ __forceinline__ int mad24(int a, int b, int c) { return c + __mul24(a, b); }

template <bool GLU, int BN = KQ_BN>
__global__ __launch_bounds__(256) void gemm_q4k_kernel(KqP p) {
    constexpr int NW = GLU ? 2 : 1, BM = kq_bm<BN>(), WC = BN / 32;  // waves along the tokens
    __shared__ KqStage<GLU, BN> st[2];
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    const int wr = wv / WC, wc = wv % WC;
    // workgroups of one row group share an XCD (id mod 8); the K splits of one tile
    // (non-gated 64-token tiles only) are neighbours in u (the same XCD)
    constexpr bool KSPLIT = !GLU && BN == 64;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, uk = bid >> 3;
    const int ksi = KSPLIT ? uk % p.ks : 0, u = KSPLIT ? uk / p.ks : uk;
    const int tg = u % p.n_tg;
    const int rg = (u / p.n_tg) * 8 + xcd;
    if (rg >= p.n_rg) return;  // whole workgroup: uniform
    const int sg = (!GLU && p.nseg > 1 && rg >= p.rg_end[0]) ? ((p.nseg > 2 && rg >= p.rg_end[1]) ? 2 : 1) : 0;
    const int row0 = (rg - (sg ? p.rg_end[sg - 1] : 0)) * BM;
    const TileRows tr = tile_rows<BN>(p, tg);
    if (tr.e < 0) return;  // whole workgroup: uniform
    const size_t woff = p.grouped ? (size_t)tr.e * p.grp.wstride : 0;
    const int tokA = act_row(p, min(tr.r0 + (tid >> (BN == 64 ? 2 : 3)), tr.r_end - 1));
    const int tokD = act_row(p, min(tr.r0 + (tid & (BN - 1)), tr.r_end - 1));
    const int h = l >> 5, m = l & 31;
    const int tok_m = 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
    const int wrow = wr * 32 + m;   // this lane's weight row (B operand / result column)
    const int arow = wc * 32 + tok_m;  // this lane's token row of the A operands
    const v16i zi = {0};
    const v16f zf = {0};
    const v32f zf32 = {0};

    float acc[NW][16];
    int s1[NW][16];
#pragma unroll
    for (int a = 0; a < NW; a++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            acc[a][v] = 0.0f;
            s1[a][v] = 0;
        }
    // this workgroup's superblocks [sb0, sb0 + n_stages / 2) (its K split)
    const int nsb = p.K >> 8;
    const int sb0 = KSPLIT ? ksi * nsb / p.ks : 0;
    const int n_stages = KSPLIT ? ((ksi + 1) * nsb / p.ks - sb0) * 2 : nsb * 2;
    KqRegs<GLU, BN> R;
    kq_load<GLU, BN>(p, sg, row0, tokA, tokD, woff, sb0, 0, tid, R);
    kq_store<GLU, BN>(st[0], tid, R);
    __syncthreads();
    for (int s = 0; s < n_stages; s++) {
        const int hs = s & 1;
        if (s + 1 < n_stages) kq_load<GLU, BN>(p, sg, row0, tokA, tokD, woff, sb0 + ((s + 1) >> 1), (s + 1) & 1, tid, R);
        const KqStage<GLU, BN> &S = st[s & 1];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const v4i av = *(const v4i *)(S.a + arow * KA_ST + 32 * j + 16 * h);
#pragma unroll
            for (int a = 0; a < NW; a++) {
                const uint4 q = *(const uint4 *)(S.wq[a] + wrow * KW_ST + 32 * (j >> 1) + 16 * h);
                const uint32_t sh = 4u * (uint32_t)(j & 1);
                const v4i bw = {(int)((q.x >> sh) & 0x0F0F0F0Fu), (int)((q.y >> sh) & 0x0F0F0F0Fu), (int)((q.z >> sh) & 0x0F0F0F0Fu),
                                (int)((q.w >> sh) & 0x0F0F0F0Fu)};
                const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bw, zi, 0, 0, 0);
                const int sc = (int)S.wsc[a][wrow * 8 + 4 * hs + j];  // |sc| < 64, |I| < 2^16
#pragma unroll
                for (int v = 0; v < 16; v++) s1[a][v] = mad24(sc, I[v], s1[a][v]);
            }
        }
        if (hs == 1) {  // end of the superblock: the min term and the two scale products
#pragma unroll
            for (int a = 0; a < NW; a++) {
                // Σ_j m_j·bs_j exactly on one f16 MFMA: k-slots 2j, 2j + 1 hold the base-64
                // digits of the block sum (bs = 64·hi + lo, |bs| ≤ 32·127) against m_j and
                // 64·m_j; every product and partial sum is an integer below 2^24.  Lane half h
                // supplies sub-blocks 4h..4h+3.
                half8k ab, bb;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int j = 4 * h + q;
                    const int bsj = (int)S.bs[arow * 8 + j];
                    const float mj = (float)S.wm[a][wrow * 8 + j];
                    ab[2 * q] = (_Float16)(float)(bsj & 63);
                    ab[2 * q + 1] = (_Float16)(float)(bsj >> 6);
                    bb[2 * q] = (_Float16)mj;
                    bb[2 * q + 1] = (_Float16)(64.0f * mj);
                }
                const v16f s2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ab, bb, zf, 0, 0, 0);
                // d·d_a and dmin·d_a in one two-block outer product (block 0: lanes 0-31, d;
                // block 1: lanes 32-63, dmin)
                const v32f pp = __builtin_amdgcn_mfma_f32_32x32x1f32(S.da[arow], h == 0 ? S.wd[a][wrow] : S.wdm[a][wrow], zf32, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    acc[a][v] += pp[v] * (float)s1[a][v] - pp[16 + v] * s2[v];
                    s1[a][v] = 0;
                }
            }
        }
        if (s + 1 < n_stages) kq_store<GLU, BN>(st[(s + 1) & 1], tid, R);
        __syncthreads();
    }
    // ---- epilogue: lane holds weight row row0 + wrow for tokens t0 + wc·32 + 16h + v ----
    const int rows = p.rows[sg];
    const int row = row0 + wrow;
    if (row >= rows) return;
    float *out = (KSPLIT && ksi) ? p.part + (size_t)(ksi - 1) * p.part_stride : p.out[sg];
    const int ld = p.ld[sg];
    const int epi = (KSPLIT && ksi) ? EPI_STORE : p.epi[sg];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int r = tr.r0 + wc * 32 + 16 * h + v;
        if (r < tr.r_end) {
            float y = acc[0][v];
            if constexpr (GLU) y = (p.glu == 2 ? gelu_tanh_f(acc[0][v]) : silu_f(acc[0][v])) * acc[NW - 1][v];
            float *o = out + (size_t)out_row(p, r) * ld + row;
            if (epi == EPI_ADD) *o += y;
            else *o = y;
        }
    }
}

// ---- Q6_K ----------------------------------------------------------------
constexpr int K6_ST = 128 + 16;  // weight code bytes per row in LDS (one half superblock, padded)

struct __align__(16) K6Stage {
    int8_t a[KQ_BN * KA_ST];
    float da[KQ_BN];
    int8_t wq[KQ_BM * K6_ST];  // q6 − 32 of the half, in value order
    float wd[KQ_BM];
    int wsc[KQ_BM * 8];        // the half's 8 signed sub-block scales
};

struct K6Regs {
    v4i a[2];
    float da;
    uint32_t lo[3], hi[3], qh[3];  // 8 bytes each from a 2-byte aligned address (+1 dword)
    uint32_t sc[3];                // the half's 8 scale bytes
    uint32_t d;
    uint32_t sh_l, sh_h, sh_q, sh_s;
};

// 3 dwords from the dword-aligned address at or below p; sh = p's offset in the first
__device__ __forceinline__ void ld3_a2(const uint8_t *p, uint32_t (&w)[3], uint32_t &sh) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    sh = (uint32_t)(a & 3);
#pragma unroll
    for (int i = 0; i < 3; i++) w[i] = wload(q + i);
}

// thread → (row tid/4, part tid%4): values l + 32i of the half, l in 8·part..+8, i = 0..3
__device__ __forceinline__ void k6_load(const KqP &p, int sg, int row0, int tokA, int tokD, size_t woff, int sb, int hs, int tid,
                                        K6Regs &R) {
    const int K = p.K, nsb = K >> 8;
    {
        const v4i *src = (const v4i *)(p.qs + (size_t)tokA * K + 256 * sb + 128 * hs + 32 * (tid & 3));
        R.a[0] = src[0];
        R.a[1] = src[1];
    }
    if (tid < KQ_BN) R.da = p.d[(size_t)tokD * nsb + sb];
    const int row = min(row0 + (tid >> 2), p.rows[sg] - 1), part = tid & 3;
    const uint8_t *blk = p.w[sg] + woff + (size_t)row * p.rb[sg] + 210 * (size_t)sb;
    ld3_a2(blk + 64 * hs + 8 * part, R.lo, R.sh_l);
    ld3_a2(blk + 64 * hs + 32 + 8 * part, R.hi, R.sh_h);
    ld3_a2(blk + 128 + 32 * hs + 8 * part, R.qh, R.sh_q);
    if (part == 0) {
        ld3_a2(blk + 192 + 8 * hs, R.sc, R.sh_s);
        R.d = wload((const uint16_t *)(blk + 208));
    }
}

__device__ __forceinline__ void k6_store(K6Stage &S, int tid, const K6Regs &R) {
    {
        v4i *dst = (v4i *)(S.a + (tid >> 2) * KA_ST + 32 * (tid & 3));
        dst[0] = R.a[0];
        dst[1] = R.a[1];
    }
    if (tid < KQ_BN) S.da[tid] = R.da;
    const int row = tid >> 2, part = tid & 3;
    const uint32_t lo[2] = {__builtin_amdgcn_alignbyte(R.lo[1], R.lo[0], R.sh_l), __builtin_amdgcn_alignbyte(R.lo[2], R.lo[1], R.sh_l)};
    const uint32_t hi[2] = {__builtin_amdgcn_alignbyte(R.hi[1], R.hi[0], R.sh_h), __builtin_amdgcn_alignbyte(R.hi[2], R.hi[1], R.sh_h)};
    const uint32_t qh[2] = {__builtin_amdgcn_alignbyte(R.qh[1], R.qh[0], R.sh_q), __builtin_amdgcn_alignbyte(R.qh[2], R.qh[1], R.sh_q)};
    // value l + 32i: low nibble of ql[l] (i = 0), ql[l + 32] (i = 1), high nibbles (i = 2, 3);
    // bits 2i, 2i+1 of qh[l] on top (quant/reference.rs:190-212).  Four codes per dword:
    // (q | 0x80) − 32, then bit 7 flipped back, is the int8 q − 32 without cross-byte borrows.
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t *src = (i & 1) ? hi : lo;
        const int sl = 4 * (i >> 1), sq = 2 * i;
        uint32_t w[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t q = ((src[k] >> sl) & 0x0F0F0F0Fu) | (((qh[k] >> sq) & 0x03030303u) << 4);
            w[k] = ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
        }
        *(uint2 *)(S.wq + row * K6_ST + 32 * i + 8 * part) = make_uint2(w[0], w[1]);
    }
    if (part == 0) {
        const uint32_t s0 = __builtin_amdgcn_alignbyte(R.sc[1], R.sc[0], R.sh_s), s1 = __builtin_amdgcn_alignbyte(R.sc[2], R.sc[1], R.sh_s);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            S.wsc[row * 8 + k] = (int)(int8_t)(s0 >> (8 * k));
            S.wsc[row * 8 + 4 + k] = (int)(int8_t)(s1 >> (8 * k));
        }
        S.wd[row] = h2f(R.d);
    }
}

__global__ __launch_bounds__(256) void gemm_q6k_kernel(KqP p) {
    __shared__ K6Stage st[2];
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    const int wr = wv >> 1, wc = wv & 1;
    // workgroups of one row group share an XCD (id mod 8); the K splits of one tile
    // are neighbours in u (the same XCD)
    const int bid = blockIdx.x;
    const int xcd = bid & 7, uk = bid >> 3;
    const int ksi = uk % p.ks, u = uk / p.ks;
    const int tg = u % p.n_tg;
    const int rg = (u / p.n_tg) * 8 + xcd;
    if (rg >= p.n_rg) return;  // whole workgroup: uniform
    const int sg = (p.nseg > 1 && rg >= p.rg_end[0]) ? ((p.nseg > 2 && rg >= p.rg_end[1]) ? 2 : 1) : 0;
    const int row0 = (rg - (sg ? p.rg_end[sg - 1] : 0)) * KQ_BM;
    const TileRows tr = tile_rows(p, tg);
    if (tr.e < 0) return;  // whole workgroup: uniform
    const size_t woff = p.grouped ? (size_t)tr.e * p.grp.wstride : 0;
    const int tokA = act_row(p, min(tr.r0 + (tid >> 2), tr.r_end - 1));
    const int tokD = act_row(p, min(tr.r0 + (tid & 63), tr.r_end - 1));
    const int h = l >> 5, m = l & 31;
    const int tok_m = 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
    const int wrow = wr * 32 + m;
    const int arow = wc * 32 + tok_m;
    const v16i zi = {0};
    const v16f zf = {0};
    float acc[16];
    int s1[16];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        acc[v] = 0.0f;
        s1[v] = 0;
    }
    // this workgroup's superblocks [sb0, sb0 + n_stages / 2) (its K split)
    const int nsb = p.K >> 8;
    const int sb0 = ksi * nsb / p.ks;
    const int n_stages = ((ksi + 1) * nsb / p.ks - sb0) * 2;
    K6Regs R;
    k6_load(p, sg, row0, tokA, tokD, woff, sb0, 0, tid, R);
    k6_store(st[0], tid, R);
    __syncthreads();
    for (int s = 0; s < n_stages; s++) {
        const int hs = s & 1;
        if (s + 1 < n_stages) k6_load(p, sg, row0, tokA, tokD, woff, sb0 + ((s + 1) >> 1), (s + 1) & 1, tid, R);
        const K6Stage &S = st[s & 1];
#pragma unroll
        for (int k = 0; k < 8; k++) {  // 16-value sub-blocks of the half
            const long av = *(const long *)(S.a + arow * KA_ST + 16 * k + 8 * h);
            const long bw = *(const long *)(S.wq + wrow * K6_ST + 16 * k + 8 * h);
            const v16i D = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, bw, zi, 0, 0, 0);
            const int sc = S.wsc[wrow * 8 + k];
#pragma unroll
            for (int v = 0; v < 16; v++) s1[v] = mad24(sc, D[v], s1[v]);
        }
        if (hs == 1) {  // end of the superblock: (d_r·d_t)·Σ sc·D
            const v16f p1 = __builtin_amdgcn_mfma_f32_32x32x2f32(h == 0 ? S.da[arow] : 0.0f, h == 0 ? S.wd[wrow] : 0.0f, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                acc[v] = fmaf(p1[v], (float)s1[v], acc[v]);
                s1[v] = 0;
            }
        }
        if (s + 1 < n_stages) k6_store(st[(s + 1) & 1], tid, R);
        __syncthreads();
    }
    const int rows = p.rows[sg];
    const int row = row0 + wrow;
    if (row >= rows) return;
    float *out = ksi ? p.part + (size_t)(ksi - 1) * p.part_stride : p.out[sg];
    const int ld = p.ld[sg];
    const int epi = ksi ? EPI_STORE : p.epi[sg];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int r = tr.r0 + wc * 32 + 16 * h + v;
        if (r < tr.r_end) {
            float *o = out + (size_t)out_row(p, r) * ld + row;
            if (epi == EPI_ADD) *o += acc[v];
            else *o = acc[v];
        }
    }
}

void kq_groups(KqP &p, int nseg, const GroupTiles *grp, int bm = KQ_BM) {
    int acc = 0;
    for (int i = 0; i < 3; i++) {
        if (i < nseg) acc += (p.rows[i] + bm - 1) / bm;
        p.rg_end[i] = acc;
    }
    p.n_rg = acc;
    p.n_tg = (p.n_tok + KQ_BN - 1) / KQ_BN;
    if (grp) {
        p.grouped = 1;
        p.grp = *grp;
        p.n_tg = grp->max_tiles;
    }
}

// The non-gated 64-token form splits K as k6_launch does (below).
template <bool GLU, int BN = KQ_BN>
void kq_launch(KqP p, hipStream_t st, float *part = nullptr, size_t part_cap = 0) {
    const int slots = (p.n_rg + 7) / 8;
    const int tiles = slots * 8 * p.n_tg, nsb = p.K >> 8;
    p.ks = 1;
    if (!GLU && BN == 64 && !p.grouped && p.nseg == 1 && part && p.n_tok > 64) {
        const size_t plane = (size_t)p.n_tok * p.ld[0];
        while (p.ks < 4 && tiles * p.ks < 512 && nsb / (2 * p.ks) >= 4 && (size_t)(2 * p.ks - 1) * plane <= part_cap) p.ks *= 2;
        p.part = part;
        p.part_stride = plane;
    }
    hipLaunchKernelGGL((gemm_q4k_kernel<GLU, BN>), dim3(tiles * p.ks), dim3(256), 0, st, p);
    if (p.ks > 1) launch_gemm_add_parts(p.out[0], p.part, p.part_stride, p.ks - 1, p.rows[0], p.ld[0], p.n_tok, st);
}

// A single ungrouped segment whose tiles number under 512 splits K in 2 or 4
// (each split ≥ 4 superblocks) while part holds the extra splits' partial sums
// (part_cap floats); the partials are added by a second launch.
void k6_launch(KqP p, hipStream_t st, float *part, size_t part_cap) {
    const int slots = (p.n_rg + 7) / 8;
    const int tiles = slots * 8 * p.n_tg, nsb = p.K >> 8;
    p.ks = 1;
    if (!p.grouped && p.nseg == 1 && part && p.n_tok > 64) {
        const size_t plane = (size_t)p.n_tok * p.ld[0];
        while (p.ks < 4 && tiles * p.ks < 512 && nsb / (2 * p.ks) >= 4 && (size_t)(2 * p.ks - 1) * plane <= part_cap) p.ks *= 2;
        p.part = part;
        p.part_stride = plane;
    }
    hipLaunchKernelGGL(gemm_q6k_kernel, dim3(tiles * p.ks), dim3(256), 0, st, p);
    if (p.ks > 1) launch_gemm_add_parts(p.out[0], p.part, p.part_stride, p.ks - 1, p.rows[0], p.ld[0], p.n_tok, st);
}

}  // namespace

bool gemm_kq_supported(int ty, size_t K) { return (ty == T_Q4_K || ty == T_Q6_K) && K % 256 == 0 && K > 0; }

bool launch_gemm_kq(const GemvSeg *segs, int nseg, const ActQ8 &act, int n_tok, int K, hipStream_t st, const GroupTiles *grp, float *part,
                    size_t part_cap) {
    if (nseg < 1 || nseg > 3 || n_tok < 1 || !act.qs || !act.d || (grp && (nseg != 1 || grp->max_tiles < 1))) return false;
    const int ty = segs[0].w.ty;
    if (ty == T_Q4_K && !act.bsums) return false;
    KqP p{};
    for (int i = 0; i < nseg; i++) {
        const GemvSeg &s = segs[i];
        if (s.w.ty != ty || !gemm_kq_supported(s.w.ty, K) || s.w.cols != (size_t)K || !s.w.data || !s.out) return false;
        p.w[i] = s.w.data;
        p.rb[i] = s.w.rb();
        p.rows[i] = (int)s.w.rows;
        p.out[i] = s.out;
        p.ld[i] = s.ld;
        p.epi[i] = s.epi;
    }
    p.nseg = nseg;
    p.n_tok = n_tok;
    p.K = K;
    p.qs = act.qs;
    p.d = act.d;
    p.bsums = act.bsums;
    if (grp && grp->bn != KQ_BN && (grp->bn != 32 || ty != T_Q4_K)) return false;
    const bool t32 = grp && grp->bn == 32;  // 32-token tiles of a Q4_K expert grouping
    kq_groups(p, nseg, grp, t32 ? kq_bm<32>() : KQ_BM);
    if (ty == T_Q6_K) k6_launch(p, st, part, part_cap);
    else if (t32) kq_launch<false, 32>(p, st);
    else kq_launch<false>(p, st, part, part_cap);
    return true;
}

bool launch_gemm_kq_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, int n_tok, int K, float *h, int ld, int gelu,
                        hipStream_t st, const GroupTiles *grp) {
    if (grp && grp->max_tiles < 1) return false;
    if (n_tok < 1 || !act.qs || !act.d || !act.bsums || gate.ty != up.ty || gate.ty != T_Q4_K || !gemm_kq_supported(gate.ty, K) ||
        gate.cols != (size_t)K || up.cols != (size_t)K || gate.rows != up.rows || !gate.data || !up.data || !h)
        return false;
    KqP p{};
    p.w[0] = gate.data;
    p.w[1] = up.data;
    p.rb[0] = gate.rb();
    p.rb[1] = up.rb();
    p.rows[0] = p.rows[1] = (int)gate.rows;
    p.out[0] = h;
    p.ld[0] = ld;
    p.epi[0] = EPI_STORE;
    p.nseg = 1;
    p.glu = gelu ? 2 : 1;
    p.n_tok = n_tok;
    p.K = K;
    p.qs = act.qs;
    p.d = act.d;
    p.bsums = act.bsums;
    if (grp && grp->bn != KQ_BN && grp->bn != 32) return false;
    const bool t32 = grp && grp->bn == 32;  // 32-token tiles of a Q4_K expert grouping
    kq_groups(p, 1, grp, t32 ? kq_bm<32>() : KQ_BM);
    if (t32) kq_launch<true, 32>(p, st);
    else kq_launch<true>(p, st);
    return true;
}

}  // namespace rie
