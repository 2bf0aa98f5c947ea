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
#include "../moe_route.hpp"
#include "../gemv_units.hpp"

#include <algorithm>
#include <cstdlib>

namespace rie {

constexpr int MAXT = 4;  // tokens processed per weight load
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
    int tpg;  // tokens per blockIdx.y group (batched GEMV)
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
    int n_xsel;        // experts in the stacked matrices: a selection is clamped below it
    int act_per_slot;  // slot j reads activation row j (the down projection of expert j's hidden)
    RouteEpi route;    // F32 router of one token: the last workgroup routes it (route.cnt != nullptr)
};

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
        const int t_end = min(p.n_tok, ((int)blockIdx.y + 1) * p.tpg);
        for (int t0 = (int)blockIdx.y * p.tpg; t0 < t_end; t0 += MAXT) {
            const int nt = min(MAXT, t_end - t0);
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

// rows whose loads a wave keeps in flight together (register budget ≈ R × unit
// bytes): 4 for units of ≤ 48 bytes (Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q4_K, F16,
// BF16), 2 for Q8_0, Q3_K, Q5_K, Q6_K, F32
template <int TY>
constexpr int dec_rows_per_pass() {
    return (TY == T_Q8_0 || TY == T_Q6_K || TY == T_F32 || TY == T_Q5_K || TY == T_Q3_K) ? 2 : 4;
}

constexpr int DEC_PAD = 8;  // LDS row padding of the partial-sum tile

// NT threads (256 or 512): one pass of NT/LPR row groups × R rows covers a
// 32-row tile in a single pass (all of a workgroup's loads issued up front).
// One 16-value group gi of a Q8_K superblock (the 16 lanes of a 16-lane row hold
// one superblock): the superblock's first strictly largest |y| (DPP within the
// row, the lower index winning ties), iscale = −127/max, round-half-away codes,
// the group's sum, d = 1/iscale (quant/mod.rs:191-218).  Writes the codes, the
// group sum and (first lane of the row) d into the LDS copy of the activation.
__device__ __forceinline__ void q8k_group_to_lds(const float (&y)[16], int gi, int8_t *s_q, int16_t *s_bs, float *s_d) {
    float am = 0.0f, mv = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < 16; e++)
        if (fabsf(y[e]) > am) {
            am = fabsf(y[e]);
            mv = y[e];
            idx = 16 * gi + e;
        }
    auto merge = [&](float oa, float om, int oi) {
        if (oa > am || (oa == am && oi < idx)) {
            am = oa;
            mv = om;
            idx = oi;
        }
    };
    merge(dpp_f<DPP_QUAD_XOR1>(am), dpp_f<DPP_QUAD_XOR1>(mv), dpp_i<DPP_QUAD_XOR1>(idx));
    merge(dpp_f<DPP_QUAD_XOR2>(am), dpp_f<DPP_QUAD_XOR2>(mv), dpp_i<DPP_QUAD_XOR2>(idx));
    merge(dpp_f<DPP_ROW_ROR4>(am), dpp_f<DPP_ROW_ROR4>(mv), dpp_i<DPP_ROW_ROR4>(idx));
    merge(dpp_f<DPP_ROW_ROR8>(am), dpp_f<DPP_ROW_ROR8>(mv), dpp_i<DPP_ROW_ROR8>(idx));
    uint32_t w4[4] = {0u, 0u, 0u, 0u};
    int bsum = 0;
    float dsb = 0.0f;
    if (am != 0.0f) {
        const float iscale = -127.0f / mv;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            int q = (int)roundf(iscale * y[e]);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            bsum += q;
            w4[e >> 2] |= ((uint32_t)(q & 0xff)) << (8 * (e & 3));
        }
        dsb = 1.0f / iscale;
    }
    *(uint4 *)(s_q + 16 * gi) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    s_bs[gi] = (int16_t)bsum;
    if ((gi & 15) == 0) s_d[gi >> 4] = dsb;
}
constexpr int QK_PRO_MAX = 8192;  // widest activation the quantize-only Q8_K prologue holds in LDS

// PRO8 (Q4_0/Q8_0 weights with a norm input): the activation is made in the
// prologue; a separate instance, so that every load before the prologue is
// unconditional and the compiler's wait for x does not cover the weight stream.
// PROQ (K-quant weights, an activation to quantize without a norm): the same for
// Q8_K(x), widths up to QK_PRO_MAX.
template <int TY, int LPR, int UPL, bool GLU, int R, int NT, bool PRO8, bool PROQ = false>
__device__ __forceinline__ void dec_body(const DecP &p, const int bid) {
    constexpr bool KQ = TY == T_Q2_K || TY == T_Q3_K || TY == T_Q4_K || TY == T_Q5_K || TY == T_Q6_K;
    static_assert(!PRO8 || TY == T_Q4_0 || TY == T_Q8_0 || KQ, "the norm prologue serves Q4_0/Q8_0 (Q8_0) and K-quant (Q8_K) weights");
    static_assert(!PROQ || ((TY == T_Q2_K || TY == T_Q3_K || TY == T_Q4_K || TY == T_Q5_K || TY == T_Q6_K) && !GLU),
                  "the quantize-only prologue serves K-quant weights");
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
        // the routing writes every selection below the expert count; the clamp keeps
        // the weight stream inside the stacked matrices whatever the ids hold
        const int e = min((unsigned)p.xsel[slot], (unsigned)(p.n_xsel - 1));
        const size_t off = ((size_t)e - (size_t)slot) * (size_t)p.slot_rows * rb;
        wbase += off;
        if constexpr (GLU) wbase2 += ((size_t)e - (size_t)slot) * (size_t)p.slot_rows * p.seg[1].rb;
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
    // EPI_ADD over long rows (256 lanes per row, quantized weights, no prologue:
    // the down projection): the residual value of the first row this thread adds to
    // in the epilogue (8 threads per row, rows tid/8, tid/8 + NT/8, …) is requested
    // at entry, so the epilogue's read-modify-write is not one more memory round
    // trip after the reduction.  A row has one writer in the launch, so the early
    // value is the one the add uses.  (In the other instances it measured no gain.)
    constexpr bool EP_PRE = !GLU && !PRO8 && !PROQ && LPR == 256 && TY != T_F32;
    const int ep_i0 = tid >> 3;
    const bool ep_pre = EP_PRE && p.seg[sg].epi == EPI_ADD && (tid & 7) == 0 && ep_i0 < p.tr && row0 + ep_i0 < seg_rows;
    const float ep_res = ep_pre ? p.seg[sg].out[row0 + ep_i0] : 0.0f;
    // PRO8: x and the norm weight are requested before the weight stream, and the
    // prologue's barriers order LDS only, so the activation is made while the
    // weights are in flight (loads complete in issue order, and a full
    // __syncthreads() would wait for the whole stream).
    // SPLIT (512 threads): waves 0-3 make the activation before they request any
    // weights, and meet through LDS arrival counts instead of workgroup barriers;
    // waves 4-7 request their weights at once and wait for the count.  A wave stalls
    // on issuing loads while its CU's memory pipeline is full, and everything after
    // the loads in program order waits with it: with every wave's weight loads
    // ahead of the prologue, the activation was ready 8 µs (median) into the
    // gate/up launch, against ~2 µs for the x loads alone.
    constexpr bool SPLIT = PRO8 && !KQ && NT >= 512;
    constexpr bool ROUTER = TY == T_F32 && !GLU;  // may carry the MoE routing (p.route)
    __shared__ int s_arrive;  // SPLIT: arrivals of waves 0-3 (4: norm sums, 8: activation)
    if constexpr (SPLIT) {
        if (tid == 0) s_arrive = 0;
        lds_barrier();  // at entry, before any load
    }
    float4 xv[4], gv[4];  // values 16τ..16τ+15 of x and of the norm weight
    float4 kx[4];         // K-quant norm: x at 4τ + 1024k (the standalone Q8_K quantizer's sum order)
    if constexpr (PRO8) {
        const float *xr = p.nin.x + ((KQ && p.xsel && p.act_per_slot) ? (size_t)slot * p.K : 0);
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = gv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (KQ) {
#pragma unroll
            for (int k = 0; k < 4; k++)
                kx[k] = (tid < 256 && 4 * tid + 1024 * k < p.K) ? *(const float4 *)(xr + 4 * tid + 1024 * k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (tid < (p.K >> 4)) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xv[i] = ((const float4 *)(xr + 16 * tid))[i];
                gv[i] = ((const float4 *)(p.nin.w + 16 * tid))[i];
            }
        }
        // unconditional (rows are clamped): a group without rows here drops its loads
        if (!SPLIT || tid >= 256) load_pass(base0);
    }
    constexpr int QG = PROQ ? (QK_PRO_MAX / 16 + NT - 1) / NT : 1;  // PROQ: 16-value groups per thread
    float4 xq[QG][4];  // PROQ: groups τ + NT·g of x
    if constexpr (PROQ) {
        const float *xr = p.nin.x + ((p.xsel && p.act_per_slot) ? (size_t)slot * p.K : 0);
#pragma unroll
        for (int g = 0; g < QG; g++) {
            const int gi = tid + NT * g;
#pragma unroll
            for (int i = 0; i < 4; i++)
                xq[g][i] = gi < (p.K >> 4) ? ((const float4 *)(xr + 16 * gi))[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        load_pass(base0);  // unconditional, as above
    }
    // F32 weights with a norm input up to 4096 wide (the MoE router): x and the norm
    // weight are requested before the weight stream, as in the PRO8 prologue, so the
    // prologue's loads do not wait behind the weights (loads complete in issue order)
    constexpr int FX = 4;  // float4 of x per thread for the sum of squares
    float4 fx[FX], ux[UPL][2], uw[UPL][2];
    const bool f32pro = TY == T_F32 && p.nin.x && p.nin.w && p.K <= 4096;
    if constexpr (TY == T_F32) {
        if (f32pro) {
#pragma unroll
            for (int k = 0; k < FX; k++) {
                const int i0 = p.nin.order16 ? 16 * tid + 4 * k : 4 * tid + 1024 * k;
                const bool in = tid < 256 && (p.nin.order16 ? 16 * tid : i0) < p.K;
                fx[k] = in ? *(const float4 *)(p.nin.x + i0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const float4 *xp = (const float4 *)(p.nin.x + 8 * uu[k]), *wp = (const float4 *)(p.nin.w + 8 * uu[k]);
                ux[k][0] = xp[0];
                ux[k][1] = xp[1];
                uw[k][0] = wp[0];
                uw[k][1] = wp[1];
            }
        }
    }
    if constexpr (!PRO8 && !PROQ) {
        if (base0 < p.tr) load_pass(base0);  // in flight while the activation is prepared
    }
    bool have_act = false;
    if constexpr (PRO8 && KQ) {
        // The activation is Q8_K(RMSNorm(x)·w), made here once per workgroup from the
        // loads issued ahead of the weight stream, with the standalone quantizer's
        // arithmetic (quant/mod.rs:191-218): the norm's partial sums in rms_scale_wg's
        // order (the first 256 threads, float4 at 4τ + 1024k; a missing k adds an
        // exact zero), then 16 threads per superblock (q8k_group_to_lds).  The
        // barriers order LDS only, so no wave waits for its weight loads here.
        __shared__ __align__(16) int8_t s_q[4096];
        __shared__ float s_d[16], s_red[4];
        __shared__ __align__(16) int16_t s_bs[256];
        const int K = p.K;
        float ss = 0.0f;
        if (tid < 256) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                ss = fmaf(kx[k].x, kx[k].x, ss);
                ss = fmaf(kx[k].y, kx[k].y, ss);
                ss = fmaf(kx[k].z, kx[k].z, ss);
                ss = fmaf(kx[k].w, kx[k].w, ss);
            }
        }
        ss = wave_sum(ss, 64);
        if ((tid & 63) == 0 && tid < 256) s_red[tid >> 6] = ss;
        lds_barrier();
        const float scale = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)K + p.nin.eps);
        if (tid < (K >> 4)) {  // whole 16-lane rows
            float y[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                y[4 * i] = xv[i].x * scale * gv[i].x;
                y[4 * i + 1] = xv[i].y * scale * gv[i].y;
                y[4 * i + 2] = xv[i].z * scale * gv[i].z;
                y[4 * i + 3] = xv[i].w * scale * gv[i].w;
            }
            q8k_group_to_lds(y, tid, s_q, s_bs, s_d);
        }
        lds_barrier();
        ActQ8 la;
        la.qs = s_q;
        la.d = s_d;
        la.bsums = s_bs;
#pragma unroll
        for (int k = 0; k < UPL; k++)
            if (valid[k]) load_act<TY>(a[k], uu[k], la, nullptr, K, 0);
        have_act = true;
    } else if constexpr (PRO8) {
        {
            // The activation is Q8_0(RMSNorm(x)·w), made here once per workgroup:
            // thread τ normalizes values 16τ..16τ+15 (a 32-block is a thread pair)
            // into LDS, then every lane reads its slice (quantizer: quant.hip).
            __shared__ __align__(16) int8_t s_q[4096];
            __shared__ float s_d[128], s_red[NT / 64];
            __shared__ int s_i[128];
            const int K = p.K, nthr = K >> 4;
            const bool act = tid < nthr;
            if (!SPLIT || tid < 256) {  // SPLIT: waves 0-3 only (wave-uniform)
                float ss = 0.0f;
                if (act) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        ss = fmaf(xv[i].x, xv[i].x, ss);
                        ss = fmaf(xv[i].y, xv[i].y, ss);
                        ss = fmaf(xv[i].z, xv[i].z, ss);
                        ss = fmaf(xv[i].w, xv[i].w, ss);
                    }
                }
                ss = wave_sum(ss, 64);
                if ((tid & 63) == 0) s_red[tid >> 6] = ss;
                if constexpr (SPLIT) {
                    lds_arrive(&s_arrive);
                    lds_wait_count(&s_arrive, 4);
                } else {
                    lds_barrier();
                }
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
                if constexpr (SPLIT) {
                    lds_arrive(&s_arrive);
                    load_pass(base0);  // waves 0-3 request their weights now
                } else {
                    lds_barrier();
                }
            }  // prologue waves
            if constexpr (SPLIT) lds_wait_count(&s_arrive, 8);
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
    } else if constexpr (PROQ) {
        // Q8_K(x) of the whole activation in LDS, groups quantized as the standalone
        // quantizer does (q8k_group_to_lds); LDS-only barriers, as in PRO8
        __shared__ __align__(16) int8_t s_qk[QK_PRO_MAX];
        __shared__ float s_dk[QK_PRO_MAX / 256];
        __shared__ __align__(16) int16_t s_bsk[QK_PRO_MAX / 16];
        const int K = p.K;
        lds_barrier();  // the previous workgroup-local use of the LDS copy is over
#pragma unroll
        for (int g = 0; g < QG; g++) {
            const int gi = tid + NT * g;
            if (gi < (K >> 4)) {  // whole 16-lane rows (K % 256 == 0)
                float y[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    y[4 * i] = xq[g][i].x;
                    y[4 * i + 1] = xq[g][i].y;
                    y[4 * i + 2] = xq[g][i].z;
                    y[4 * i + 3] = xq[g][i].w;
                }
                q8k_group_to_lds(y, gi, s_qk, s_bsk, s_dk);
            }
        }
        lds_barrier();
        ActQ8 la;
        la.qs = s_qk;
        la.d = s_dk;
        la.bsums = s_bsk;
#pragma unroll
        for (int k = 0; k < UPL; k++)
            if (valid[k]) load_act<TY>(a[k], uu[k], la, nullptr, K, 0);
        have_act = true;
    } else if constexpr (TY == T_Q2_K || TY == T_Q3_K || TY == T_Q4_K || TY == T_Q5_K || TY == T_Q6_K) {
        if (p.nin.x) {
            // The activation is Q8_K(RMSNorm(x)·w), made here once per workgroup in
            // LDS, in the layout of the global buffer, with the arithmetic of the
            // standalone quantizer (quant/mod.rs:191-218): the norm's partial sums
            // in rms_scale_wg's order (the first 256 threads, float4 at 4τ + 1024k);
            // then 16 threads per superblock, 16 values each: the first strictly
            // largest |y| (DPP within the 16-lane row, the lower index winning
            // ties), iscale = −127/max, round-half-away codes, the thread's 16-value
            // sum, d = 1/iscale.  Every code equals the standalone kernel's.
            // Without a norm weight the prologue only quantizes (y = x·1·1 = x,
            // exactly), reading the workgroup's slot row when activations are per
            // slot (an expert's hidden).
            __shared__ __align__(16) int8_t s_q[4096];
            __shared__ float s_d[16], s_red[4];
            __shared__ __align__(16) int16_t s_bs[256];
            const int K = p.K;
            const bool norm = p.nin.w != nullptr;
            const float *xr = p.nin.x + ((p.xsel && p.act_per_slot) ? (size_t)slot * K : 0);
            float ss = 0.0f;
            if (norm && tid < 256)
                for (int i = tid * 4; i < K; i += 1024) {
                    const float4 v = *(const float4 *)(xr + i);
                    ss = fmaf(v.x, v.x, ss);
                    ss = fmaf(v.y, v.y, ss);
                    ss = fmaf(v.z, v.z, ss);
                    ss = fmaf(v.w, v.w, ss);
                }
            ss = wave_sum(ss, 64);
            if ((tid & 63) == 0 && tid < 256) s_red[tid >> 6] = ss;
            __syncthreads();
            const float scale = norm ? 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)K + p.nin.eps) : 1.0f;
            if (tid < (K >> 4)) {  // whole 16-lane rows
                float y[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 xv = ((const float4 *)(xr + 16 * tid))[i];
                    const float4 gv = norm ? ((const float4 *)(p.nin.w + 16 * tid))[i] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
                    y[4 * i] = xv.x * scale * gv.x;
                    y[4 * i + 1] = xv.y * scale * gv.y;
                    y[4 * i + 2] = xv.z * scale * gv.z;
                    y[4 * i + 3] = xv.w * scale * gv.w;
                }
                q8k_group_to_lds(y, tid, s_q, s_bs, s_d);
            }
            __syncthreads();
            ActQ8 la;
            la.qs = s_q;
            la.d = s_d;
            la.bsums = s_bs;
#pragma unroll
            for (int k = 0; k < UPL; k++)
                if (valid[k]) load_act<TY>(a[k], uu[k], la, nullptr, K, 0);
            have_act = true;
        }
    }
    if constexpr (TY == T_F32) {
        if (f32pro) {  // the same arithmetic on the early loads; the barrier orders LDS only
            __shared__ float s_red2[4];
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < FX; k++) {
                ss = fmaf(fx[k].x, fx[k].x, ss);
                ss = fmaf(fx[k].y, fx[k].y, ss);
                ss = fmaf(fx[k].z, fx[k].z, ss);
                ss = fmaf(fx[k].w, fx[k].w, ss);
            }
            ss = wave_sum(ss, 64);
            if ((tid & 63) == 0 && tid < 256) s_red2[tid >> 6] = ss;
            lds_barrier();
            const float scale = 1.0f / sqrtf(((s_red2[0] + s_red2[1]) + (s_red2[2] + s_red2[3])) / (float)p.K + p.nin.eps);
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const float4 x0 = ux[k][0], x1 = ux[k][1], w0 = uw[k][0], w1 = uw[k][1];
                a[k].f[0] = x0.x * scale * w0.x; a[k].f[1] = x0.y * scale * w0.y;
                a[k].f[2] = x0.z * scale * w0.z; a[k].f[3] = x0.w * scale * w0.w;
                a[k].f[4] = x1.x * scale * w1.x; a[k].f[5] = x1.y * scale * w1.y;
                a[k].f[6] = x1.z * scale * w1.z; a[k].f[7] = x1.w * scale * w1.w;
            }
            have_act = true;
        } else if (p.nin.x) {
            // The activation is RMSNorm(x)·w in f32, bit for bit the rows of the
            // standalone kernel it replaces: the scale from that kernel's partial
            // sums (the first 256 threads; q8_0_rows_kernel's 16 consecutive values
            // per thread and 4096-value pass, or rms_scale_wg's float4 at
            // 4τ + 1024k), then (x·scale)·w per value.
            __shared__ float s_red[4];
            const int K = p.K;
            float ss = 0.0f;
            if (tid < 256) {
                const int step = p.nin.order16 ? 4096 : 1024;
                for (int i0 = p.nin.order16 ? 16 * tid : 4 * tid; i0 < K; i0 += step)
                    for (int k = 0; k < (p.nin.order16 ? 4 : 1); k++) {
                        const float4 v = *(const float4 *)(p.nin.x + i0 + 4 * k);
                        ss = fmaf(v.x, v.x, ss);
                        ss = fmaf(v.y, v.y, ss);
                        ss = fmaf(v.z, v.z, ss);
                        ss = fmaf(v.w, v.w, ss);
                    }
            }
            ss = wave_sum(ss, 64);
            if ((tid & 63) == 0 && tid < 256) s_red[tid >> 6] = ss;
            __syncthreads();
            const float scale = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)K + p.nin.eps);
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const float4 *xp = (const float4 *)(p.nin.x + 8 * uu[k]), *wp = (const float4 *)(p.nin.w + 8 * uu[k]);
                const float4 x0 = xp[0], x1 = xp[1], w0 = wp[0], w1 = wp[1];
                a[k].f[0] = x0.x * scale * w0.x; a[k].f[1] = x0.y * scale * w0.y;
                a[k].f[2] = x0.z * scale * w0.z; a[k].f[3] = x0.w * scale * w0.w;
                a[k].f[4] = x1.x * scale * w1.x; a[k].f[5] = x1.y * scale * w1.y;
                a[k].f[6] = x1.z * scale * w1.z; a[k].f[7] = x1.w * scale * w1.w;
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
        // the 8 lanes of the row (DPP: the same pairings as a 1, 2, 4 butterfly)
        sum = xsum_f<8>(sum);
        sum2 = xsum_f<8>(sum2);
        const int r = row0 + i;
        if (s8 == 0 && i < p.tr && r < seg_rows) {
            float v = sum;
            if constexpr (GLU) v = (p.glu == 2 ? gelu_tanh_f(sum) : silu_f(sum)) * sum2;
            float *out = p.seg[sg].out;
            if (p.seg[sg].epi == EPI_ADD) out[r] = (ep_pre && i == ep_i0 ? ep_res : out[r]) + v;
            else if (ROUTER && p.route.cnt) st_coh(out + r, v);  // read by the routing workgroup
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

// The router GEMV's last workgroup routes the token.  The logits are agent-scope
// atomic stores (written through to the device coherence point); every thread
// waits for their completion before the barrier, so the arrival count is a
// relaxed agent-scope add, and the last workgroup to arrive re-arms the counter
// and runs the routing in its first wave, reading the logits with agent-scope
// atomic loads.  No release or acquire: those add a write-back or invalidation of
// the whole L2 of the XCD, which only plain stores and loads need.
__device__ __forceinline__ void route_last_workgroup(const DecP &p) {
    __shared__ int s_last;
    wait_vmem();
    __syncthreads();  // the workgroup's logits are stored
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(p.route.cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (int)gridDim.x - 1;
        if (s_last) __hip_atomic_store(p.route.cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_last && threadIdx.x < 64)
        moe_route_wave<true>(p.seg[0].out, p.route.n_exp, p.route.k, p.route.norm_topk, p.route.unit_weights, p.route.sel, p.route.wgt);
}

template <int TY, int LPR, int UPL, bool GLU, int R, int NT, bool PRO8 = false, bool PROQ = false>
__global__ __launch_bounds__(NT, NT == 512 ? 4 : 1) void gemv_dec_kernel(DecP p) {  // 512 threads: two workgroups per CU
    dec_body<TY, LPR, UPL, GLU, R, NT, PRO8, PROQ>(p, blockIdx.x);
    if constexpr (TY == T_F32 && !GLU) {
        if (p.route.cnt) route_last_workgroup(p);
    }
}

// Q4_K and Q6_K segments of one activation in one launch (Q/K and V of a Q4_K_M
// layer): the first n1 workgroups run the Q4_K rows, the others the Q6_K rows.
// Each half is the single-type kernel's body with its own tile; with a norm input
// both halves make the Q8_K activation in their prologue.
template <int L1, int L2, bool PRO = false>
__global__ __launch_bounds__(256) void gemv_dec_k46_kernel(DecP p1, DecP p2, int n1) {
    if ((int)blockIdx.x < n1) dec_body<T_Q4_K, L1, 1, false, dec_rows_per_pass<T_Q4_K>(), 256, PRO>(p1, blockIdx.x);
    else dec_body<T_Q6_K, L2, 1, false, dec_rows_per_pass<T_Q6_K>(), 256, PRO>(p2, blockIdx.x - n1);
}

static int dec_units(int ty, int K) {
    if (ty == T_Q2_K || ty == T_Q3_K) return K / 32;
    if (ty == T_F32 || ty == T_F16 || ty == T_BF16) return K / 8;
    return K / 64;
}

// tile and grid of a decode GEMV launch: lanes per row, units per lane, threads,
// LDS bytes and workgroups (p.tr and p.blk_end are filled in)
template <int TY, int R>
static bool plan_dec(DecP &p, int &lpr, int &upl, int &nt, size_t &lds, int &blocks) {
    const int U = dec_units(TY, p.K);
    lpr = 16;
    while (lpr < U && lpr < 256) lpr *= 2;
    upl = (U + lpr - 1) / lpr;
    if (upl > 2) return false;
    int pass = (256 / lpr) * R;  // rows per pass of a 256-thread workgroup
    int m;
    nt = 256;
    if (p.glu && p.hq.qs) {
        if (p.total_rows % 32) return false;
        // whole Q8_0 blocks of h per workgroup, in one pass: 512 or 1024 threads.
        // 64 rows (one workgroup per CU) where 32-row workgroups would number more
        // than the 256 CUs: a CU's second workgroup would request its activation
        // behind the first one's weight stream
        const int want = (!p.xsel && p.total_rows % 64 == 0 && p.total_rows / 32 > 256) ? 64 : 32;
        if (pass < want) {
            nt = 256 * (want / pass);
            pass = want;
        }
        m = 1;
        if (nt > 1024) return false;
    } else {
        m = std::max(1, std::min(4, p.total_rows / (pass * 1024)));
    }
    p.tr = pass * m;
    if (p.xsel && p.slot_rows % p.tr) {  // a workgroup must not straddle two experts
        p.tr = pass;
        if (p.slot_rows % p.tr || (p.glu && p.hq.qs && p.tr % 32)) return false;
    }
    lds = ((size_t)(p.glu ? 2 : 1) * p.tr * (lpr + DEC_PAD) + p.tr) * sizeof(float);
    if (lds > 64 * 1024) return false;
    blocks = 0;
    const int nseg = p.glu ? 1 : p.nseg;
    for (int i = 0; i < 3; i++) {
        if (i < nseg) blocks += (p.seg[i].rows + p.tr - 1) / p.tr;
        p.blk_end[i] = blocks;
    }
    return true;
}

template <int TY, int R>
static bool launch_dec_r(DecP p, hipStream_t st) {
    int lpr, upl, nt, blocks;
    size_t lds;
    if (!plan_dec<TY, R>(p, lpr, upl, nt, lds, blocks)) return false;
    constexpr bool Q8PRO = TY == T_Q4_0 || TY == T_Q8_0;
    constexpr bool KPRO = TY == T_Q2_K || TY == T_Q3_K || TY == T_Q4_K || TY == T_Q5_K || TY == T_Q6_K;
    const bool pro = Q8PRO && p.nin.x;
    const bool prok = KPRO && p.nin.x && p.nin.w && p.K <= 4096 && nt == 256;  // RMSNorm + Q8_K in the prologue
    const bool proq = KPRO && p.nin.x && !p.nin.w && !p.glu && nt == 256 && upl == 1 && lpr >= 32 && p.K <= QK_PRO_MAX;
#define RIE_DEC_P(L, UP, PR)                                                                                          \
    do {                                                                                                              \
        if (p.glu && nt == 512) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 512, PR>), dim3(blocks), dim3(512), lds, st, p);    \
        else if (p.glu && nt == 1024) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 1024, PR>), dim3(blocks), dim3(1024), lds, st, p); \
        else if (p.glu) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 256, PR>), dim3(blocks), dim3(256), lds, st, p);      \
        else hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, false, R, 256, PR>), dim3(blocks), dim3(256), lds, st, p);                \
    } while (0)
#define RIE_DEC_PK(L, UP)                                                                                               \
    do {                                                                                                                \
        if (p.glu) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, true, R, 256, true>), dim3(blocks), dim3(256), lds, st, p);   \
        else hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, false, R, 256, true>), dim3(blocks), dim3(256), lds, st, p);        \
    } while (0)
#define RIE_DEC(L, UP)                                                                                                  \
    do {                                                                                                                \
        if constexpr (Q8PRO) {                                                                                          \
            if (pro) RIE_DEC_P(L, UP, true);                                                                            \
            else RIE_DEC_P(L, UP, false);                                                                               \
        } else if constexpr (KPRO && UP == 1 && L >= 32) {                                                              \
            if (prok) RIE_DEC_PK(L, UP);                                                                                \
            else if (proq) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, 1, false, R, 256, false, true>), dim3(blocks), dim3(256), lds, st, p); \
            else RIE_DEC_P(L, UP, false);                                                                               \
        } else if constexpr (KPRO) {                                                                                    \
            if (prok) RIE_DEC_PK(L, UP);                                                                                \
            else RIE_DEC_P(L, UP, false);                                                                               \
        } else {                                                                                                        \
            RIE_DEC_P(L, UP, false);                                                                                    \
        }                                                                                                               \
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
#undef RIE_DEC_P
#undef RIE_DEC_PK
    return true;
}

// Q4_K segments (p1) and Q6_K segments (p2) of one activation in one launch
static bool launch_dec_k46(DecP p1, DecP p2, hipStream_t st) {
    int l1, u1, n1t, b1, l2, u2, n2t, b2;
    size_t lds1, lds2;
    if (!plan_dec<T_Q4_K, dec_rows_per_pass<T_Q4_K>()>(p1, l1, u1, n1t, lds1, b1) ||
        !plan_dec<T_Q6_K, dec_rows_per_pass<T_Q6_K>()>(p2, l2, u2, n2t, lds2, b2))
        return false;
    if (u1 != 1 || u2 != 1 || n1t != 256 || n2t != 256 || l2 != l1) return false;
    const size_t lds = std::max(lds1, lds2);
    const dim3 grid(b1 + b2), block(256);
    // with a norm input both halves make RMSNorm + Q8_K in the early-load prologue
    const bool pro = p1.nin.x && p1.nin.w && p2.nin.x && p2.nin.w && p1.K <= 4096;
#define RIE_K46(A, B)                                                                                            \
    do {                                                                                                         \
        if (pro) hipLaunchKernelGGL((gemv_dec_k46_kernel<A, B, true>), grid, block, lds, st, p1, p2, b1);        \
        else hipLaunchKernelGGL((gemv_dec_k46_kernel<A, B, false>), grid, block, lds, st, p1, p2, b1);           \
    } while (0)
    switch (l1) {
    case 32: RIE_K46(32, 32); return true;
    case 64: RIE_K46(64, 64); return true;
    case 128: RIE_K46(128, 128); return true;
    default: return false;
    }
#undef RIE_K46
}

// Non-gated dense launches of Q4_0/Q8_0 rows with R rows per lane and pass
// below the type's default (the same kernel body, smaller workgroup tiles).
template <int TY, int R>
static bool launch_dec_small(DecP p, hipStream_t st) {
    int lpr, upl, nt, blocks;
    size_t lds;
    if (!plan_dec<TY, R>(p, lpr, upl, nt, lds, blocks) || nt != 256) return false;
    const bool pro = p.nin.x != nullptr;
#define RIE_DS(L, UP)                                                                                                      \
    do {                                                                                                                   \
        if (pro) hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, false, R, 256, true>), dim3(blocks), dim3(256), lds, st, p);  \
        else hipLaunchKernelGGL((gemv_dec_kernel<TY, L, UP, false, R, 256, false>), dim3(blocks), dim3(256), lds, st, p);     \
    } while (0)
    if (upl == 1) {
        switch (lpr) {
        case 16: RIE_DS(16, 1); break;
        case 32: RIE_DS(32, 1); break;
        case 64: RIE_DS(64, 1); break;
        case 128: RIE_DS(128, 1); break;
        default: RIE_DS(256, 1); break;
        }
    } else {
        RIE_DS(256, 2);
    }
#undef RIE_DS
    return true;
}

// workgroups of the launch for R rows per pass (0 when that tile does not apply)
template <int TY, int R>
static int dec_blocks(DecP p) {
    int lpr, upl, nt, blocks;
    size_t lds;
    return plan_dec<TY, R>(p, lpr, upl, nt, lds, blocks) ? blocks : 0;
}

template <int TY>
static bool launch_dec_t(const DecP &p, hipStream_t st) {
    constexpr int R = dec_rows_per_pass<TY>();
    if constexpr (TY == T_Q4_0 || TY == T_Q8_0) {
        // Dense non-gated launches whose default tile leaves CUs without a
        // workgroup (fewer than 256: wo at hidden 2048 has 64 workgroups of 32
        // rows) take the largest smaller tile that reaches 256 workgroups, or the
        // smallest.  (A smaller tile only to even out the CUs' loads, e.g. Q/K/V at
        // hidden 4096 as 768 workgroups instead of 384, measured slower.)
        if (!p.glu && !p.xsel && !p.route.cnt) {
            const int b0 = dec_blocks<TY, R>(p);
            if (b0 > 0 && b0 < 256) {
                const int b1 = dec_blocks<TY, R / 2>(p);
                if constexpr (R >= 4) {
                    if (b1 > 0 && b1 < 256 && dec_blocks<TY, R / 4>(p) > b1 && launch_dec_small<TY, R / 4>(p, st)) return true;
                }
                if (b1 > b0 && launch_dec_small<TY, R / 2>(p, st)) return true;
            }
        }
    }
    return launch_dec_r<TY, R>(p, st);
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
    // few rows (a router, a small projection): the tokens are split over
    // blockIdx.y as well, in groups of a multiple of 4, up to ~1024 workgroups
    GemvP q = p;
    int groups = 1;
    if (blocks < 512 && p.n_tok > 16) groups = std::min((p.n_tok + 15) / 16, std::max(1, 1024 / blocks));
    q.tpg = ((p.n_tok + groups - 1) / groups + 3) / 4 * 4;
    groups = (p.n_tok + q.tpg - 1) / q.tpg;
    const dim3 grid(blocks, groups);
    switch (lpr) {
    case 8: hipLaunchKernelGGL((gemv_kernel<TY, 8>), grid, dim3(256), 0, st, q); break;
    case 16: hipLaunchKernelGGL((gemv_kernel<TY, 16>), grid, dim3(256), 0, st, q); break;
    case 32: hipLaunchKernelGGL((gemv_kernel<TY, 32>), grid, dim3(256), 0, st, q); break;
    default: hipLaunchKernelGGL((gemv_kernel<TY, 64>), grid, dim3(256), 0, st, q); break;
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

bool gemv_norm_ok(int ty, size_t K) {
    if (ty == T_Q4_0 || ty == T_Q8_0) return K % 64 == 0 && K >= 64 && K <= 4096;
    if (ty == T_Q2_K || ty == T_Q3_K || ty == T_Q4_K || ty == T_Q5_K || ty == T_Q6_K) return K % 256 == 0 && K >= 256 && K <= 4096;
    return false;
}

bool gemv_norm_f32_ok(int ty, size_t K) { return ty == T_F32 && K % 16 == 0 && K >= 16; }

bool gemv_quant_ok(int ty, size_t K) {
    return (ty == T_Q2_K || ty == T_Q3_K || ty == T_Q4_K || ty == T_Q5_K || ty == T_Q6_K) && K % 256 == 0 && K >= 256 &&
           K <= (size_t)QK_PRO_MAX;
}

bool launch_gemv(const GemvSeg *segs, int nseg, const ActQ8 &act, const float *act_f32, int n_tok, int K, hipStream_t st,
                 const NormIn *nin) {
    if (n_tok < 1) return false;
    if (nin && (n_tok != 1 || !nin->x)) return false;
    for (int s = 0; s < nseg; s++) {
        if (nin && nin->w && !gemv_norm_ok(segs[s].w.ty, (size_t)K) && !gemv_norm_f32_ok(segs[s].w.ty, (size_t)K)) return false;
        // without a norm weight only the Q8_K prologue applies (it then quantizes x as it is)
        if (nin && !nin->w && !gemv_quant_ok(segs[s].w.ty, (size_t)K)) return false;
    }
    // one token, Q4_K segments followed by Q6_K ones (the Q4_K_M attention): one launch
    if (n_tok == 1 && nseg >= 2) {
        int k = 0;
        while (k < nseg && segs[k].w.ty == T_Q4_K) k++;
        bool mixed = k > 0 && k < nseg;
        for (int s = k; s < nseg; s++) mixed = mixed && segs[s].w.ty == T_Q6_K;
        for (int s = 0; s < nseg && mixed; s++)
            mixed = gemv_supported(segs[s].w.ty, K) && segs[s].w.cols == (size_t)K && segs[s].w.data && segs[s].out &&
                    operands_ok(segs[s].w.ty, act, act_f32);
        if (mixed) {
            DecP d[2]{};
            for (int s = 0; s < nseg; s++) {
                DecP &dd = d[s < k ? 0 : 1];
                dd.seg[dd.nseg++] = SegP{segs[s].w.data, segs[s].w.rb(), (int)segs[s].w.rows, segs[s].out, segs[s].ld, segs[s].epi};
                dd.total_rows += (int)segs[s].w.rows;
            }
            for (auto &dd : d) {
                dd.K = K;
                dd.act = act;
                dd.actf = act_f32;
                if (nin) dd.nin = *nin;
            }
            if (launch_dec_k46(d[0], d[1], st)) return true;
        }
    }
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

bool launch_gemv_route(const GemvSeg &seg, const ActQ8 &act, const float *act_f32, int K, const NormIn *nin, const RouteEpi &route,
                       hipStream_t st) {
    // F32 router weights only (the instances that carry the routing epilogue); n_exp ≤ 512
    if (seg.w.ty != T_F32 || !route.cnt || !route.sel || !route.wgt || route.n_exp < 1 || route.n_exp > 512 || route.k < 1 ||
        route.k > route.n_exp || route.k > 64 || seg.w.rows != (size_t)route.n_exp || seg.epi != EPI_STORE ||
        !gemv_supported(seg.w.ty, K) || seg.w.cols != (size_t)K || !seg.w.data || !seg.out)
        return false;
    if (nin && (!nin->x || !nin->w || !gemv_norm_f32_ok(seg.w.ty, (size_t)K))) return false;
    DecP d{};
    d.seg[0] = SegP{seg.w.data, seg.w.rb(), (int)seg.w.rows, seg.out, seg.ld, EPI_STORE};
    d.nseg = 1;
    d.total_rows = (int)seg.w.rows;
    d.K = K;
    d.act = act;
    d.actf = act_f32;
    if (nin) d.nin = *nin;
    d.route = route;
    return dispatch_dec(T_F32, d, st);
}

bool launch_gemv_experts(const DevWeight &stacked, int slot_rows, const int *sel, int n_slots, const ActQ8 &act,
                         const float *act_f32, bool act_per_slot, int K, float *out, hipStream_t st, const NormIn *nin) {
    // with nin: the K-quant prologue quantizes (and with nin->w normalizes) the activation itself
    if (nin && (!nin->x || act_format(stacked.ty) != ACT_Q8K ||
                !(nin->w ? gemv_norm_ok(stacked.ty, (size_t)K) : gemv_quant_ok(stacked.ty, (size_t)K))))
        return false;
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
    d.n_xsel = (int)(stacked.rows / (size_t)slot_rows);
    d.act_per_slot = act_per_slot;
    if (nin) d.nin = *nin;
    return dispatch_dec(stacked.ty, d, st);
}

bool launch_gemv_glu_experts(const DevWeight &gate, const DevWeight &up, int ff, const int *sel, int n_slots, const ActQ8 &act,
                             const float *act_f32, int K, float *h, int gelu, const ActQ8 *hq, hipStream_t st, const NormIn *nin) {
    if (nin && (!nin->x || !nin->w || !gemv_norm_ok(gate.ty, (size_t)K))) return false;
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
    if (nin) d.nin = *nin;
    d.xsel = sel;
    d.slot_rows = ff;
    d.n_xsel = (int)(gate.rows / (size_t)ff);
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
