// kernels.hpp — host-side launchers of the gfx950 kernels.
#pragma once

#include "common.hpp"

namespace rie {

// ---- quant.hip ----
// ref_order: the norm's Σx² in the reference's summation order (kernels/avx2.rs:
// dot_f32), bitwise the reference's normalized row for the same input row (a
// serial sum: for rows that are identical on both sides, the first layer's).
void launch_rmsnorm_quant(const float *x, int ldx, const float *w, float eps, int n_rows, int E, float *xn, int fmt, const ActQ8 &act,
                          hipStream_t st, bool ref_order = false);
void launch_rmsnorm(const float *x, int ldx, const float *w, float eps, int n_rows, int E, float *out, int ldo, int inplace_assoc,
                    hipStream_t st, bool ref_order = false);
void launch_embed(const uint32_t *tokens, int n, const DevWeight &table, float scale, float *x, hipStream_t st);

// ---- gemv.hip ----
// Output epilogues of one GEMV segment.
enum Epi : int { EPI_STORE = 0, EPI_ADD = 1 };
struct GemvSeg {
    DevWeight w;
    float *out;   // out[t*ld + r]
    int ld;
    int epi;
};
// y_seg = W_seg · act for up to 3 segments sharing one activation batch (n_tok rows).
// Returns false when a weight type/shape has no kernel.
// nin (single token, Q4_0/Q8_0 weights, K ≤ 4096): the kernel computes the
// activation itself as Q8_0(RMSNorm(x)·w) — no separate normalization launch;
// K-quant weights likewise as Q8_K, and with nin->w == nullptr as Q8_K(x).
struct NormIn {
    const float *x;   // residual row [K]
    const float *w;   // norm weight [K]
    float eps;
    // F32 weights only: the order of the scale's partial sums, that of the
    // standalone kernel whose rows the prologue replaces: 1 = q8_0_rows_kernel
    // (thread τ: values 16τ..16τ+15 of each 4096-value pass), 0 = rms_scale_wg
    // (float4 at 4τ + 1024k)
    int order16;
};
bool gemv_norm_ok(int ty, size_t K);
// K-quant weights with nin->w == nullptr: the prologue quantizes x to Q8_K (K ≤ 8192)
bool gemv_quant_ok(int ty, size_t K);
// F32 weights with nin: the activation is RMSNorm(x)·w in f32, equal to the standalone norm's rows
bool gemv_norm_f32_ok(int ty, size_t K);
bool launch_gemv(const GemvSeg *segs, int nseg, const ActQ8 &act, const float *act_f32, int n_tok, int K, hipStream_t st,
                 const NormIn *nin = nullptr);
// h = act(gate·x) ⊙ (up·x) for gated feed-forward blocks (gelu selects GELU-tanh).
// hq (n_tok == 1, Q8_0 down projection): also quantize h to Q8_0 in the epilogue;
// returns false (nothing launched) when that is not possible.
bool launch_gemv_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, const float *act_f32, int n_tok, int K, float *h,
                     int ld, int gelu, const ActQ8 *hq, hipStream_t st, const NormIn *nin = nullptr);
bool gemv_supported(int ty, size_t K);
// Routing of one token by the router GEMV's last workgroup (F32 router weights):
// the logits go to seg.out as usual, then sel/wgt receive the token's top-k
// (the routing kernel's results).  cnt: one int, zero before the first launch,
// re-armed by each launch.  False (nothing launched) when not applicable.
struct RouteEpi {
    int *cnt = nullptr;
    int n_exp = 0, k = 0, norm_topk = 0, unit_weights = 0;
    int *sel = nullptr;
    float *wgt = nullptr;
};

// ---- attention.hip ----
struct HeadPrepArgs {
    float *q;            // [n][qd] in/out (rotated, scaled)
    const float *k;      // [n][kvd]
    const float *v;      // [n][kvd]
    const float *bq, *bk, *bv;        // optional biases
    const float *q_norm, *k_norm;     // optional per-head RMSNorm weights [hd]
    const float *cos_t, *sin_t;       // rope tables [n_ctx][rope_dim/2]
    int n_tok, pos0, n_head, n_kv, hd, rope_dim, neox;
    float eps, attn_scale;
    int kv_type;                      // 0 f16, 1 q8_0, 2 turbo4
    uint8_t *k_cache, *v_cache;       // layer base: [n_kv][slots][row]
    uint16_t *k_scale, *v_scale;      // turbo4 only: [n_kv][slots] f16 scales
    int slots;
    const int *d_pos0;                // optional device-resident pos0 (graph replay)
    const float *turbo_signs;         // [hd]
    float *k_out;                     // optional: K after norm/RoPE, [n][kvd] (parity hooks)
};
void launch_head_prep(const HeadPrepArgs &a, hipStream_t st);

struct AttnArgs {
    const float *q;              // [n][qd]
    const uint8_t *k_cache, *v_cache;
    const uint16_t *k_scale, *v_scale;
    int n_tok, pos0, n_head, n_kv, hd, slots, window, kv_type;
    float softcap;               // 0 = none
    float *part;                 // [n][n_head][n_split][hd + 2]
    int n_split;
    float *att;                  // [n][qd] f32 output
    ActQ8 att_q;                 // optional Q8_0 quantization of att (qs/d/s/isum) when att_fmt == ACT_Q8_0
    int att_fmt;
    const int *d_pos0;
    const float *turbo_signs;
    int *counters;               // fused single-token path: [n_head · ATT_CNT_STRIDE] zeroed ints, left zeroed
};
constexpr int ATT_CNT_STRIDE = 32;  // ints between the arrival counters of the head slices
void launch_attention(const AttnArgs &a, hipStream_t st);
// Single token: Q/K prep, KV append, attention and the range merge in one launch
// (hp describes the raw Q/K/V rows; hp.q is only read).  False when not applicable.
bool attention_fused_ok(const AttnArgs &a);
bool launch_attention_fused(const AttnArgs &a, const HeadPrepArgs &hp, hipStream_t st);
// ---- attn_prompt.hip ----
// Prompt batches over an f16 cache on f16 matrix cores (one launch, no range
// partials); false when the shape or cache type is not covered.
bool attention_prompt_mfma_ok(const AttnArgs &a);
bool launch_attention_prompt_mfma(const AttnArgs &a, hipStream_t st);
// Merge of a.n_split range partials per (token, head) [t][head][split][hd + 2]
// (maximum in natural-log units), the inverse Turbo4 rotation, f32 att and Q8_0.
void launch_attention_combine(const AttnArgs &a, hipStream_t st);
// number of context ranges (n_split) for a launch whose longest query sees max_len
// positions; fused: a single token on the one-launch path (attention_fused_ok), which
// takes one range (one workgroup per query head) at short contexts
constexpr int ATT_MAX_SPLIT = 256;
int attention_splits(int n_tok, int n_kv, int max_len, int hd, bool fused);

// ---- misc.hip ----
// cnt: one zeroed int (left zeroed) for the one-launch form, where the last workgroup
// reduces the partials; nullptr: two launches
void launch_argmax(const float *x, int n, int *partial_idx, float *partial_val, int n_part, uint32_t *out_idx, hipStream_t st,
                   int *cnt = nullptr);
// The same, as one step of greedy decoding replayed in a graph: the token also goes
// to gen[step[1] + 1] (when below gen_cap), then step[0] (position) and step[1]
// (index of the step) advance by one.
void launch_argmax_step(const float *x, int n, int *partial_idx, float *partial_val, int n_part, uint32_t *out_idx, uint32_t *gen,
                        int *step, int gen_cap, hipStream_t st, int *cnt = nullptr);
// The same argmax with its partials in the library's static device array (no
// allocation); n in 1..ARGMAX_SCRATCH_PARTS·ARGMAX_SCRATCH_PER_PART, else throws.
// Calls that overlap on one GPU share the array and race.
constexpr int ARGMAX_SCRATCH_PARTS = 1024, ARGMAX_SCRATCH_PER_PART = 1024;
void launch_argmax_noalloc(const float *x, int n, uint32_t *out_idx, hipStream_t st);
void launch_add_inplace(float *x, const float *y, size_t n, float scale, hipStream_t st);
void launch_scale(float *x, size_t n, float div, hipStream_t st);
void launch_set_int(int *p, int v, hipStream_t st);
void launch_softcap(float *x, size_t n, float cap, hipStream_t st);
void launch_quant_only(const float *x, int ldx, int n_rows, int K, int fmt, const ActQ8 &act, hipStream_t st);
// MoE routing: softmax over n_exp logits per token, top-k with index tie-break, renorm.
// (sel, wgt) of each token are stored in ascending expert order.
void launch_moe_route(const float *logits, int n_tok, int n_exp, int k, int norm_topk, int unit_weights, int *sel, float *wgt,
                      hipStream_t st);
// out[t] (= or +=) Σ_j w[t·k+j]·y[t·k+j] over the k routed experts (cpu.rs:502-513)
void launch_moe_combine(const float *y, const float *w, int n_tok, int k, int E, float *out, int epi, hipStream_t st);
void launch_moe_gather(const float *x, const int *rows, int n, int E, float *xg, hipStream_t st);
void launch_moe_scatter_add(const float *yg, const int *rows, const float *w, int n, int E, float *out, hipStream_t st);
void launch_moe_shared_add(const float *ys, const float *gate_inp, const float *x, int n_tok, int E, float *out, hipStream_t st);
// Routed experts of one token (stacked expert tensors, expert ids on the device):
// out rows [j·slot_rows, (j+1)·slot_rows) = expert sel[j]'s rows · act (act row j
// when act_per_slot); the GLU variant writes h [n_slots][ff].
// With nin (Q8_K weight types): every workgroup quantizes its activation row from
// nin->x itself (normalized first when nin->w is given).
bool launch_gemv_route(const GemvSeg &seg, const ActQ8 &act, const float *act_f32, int K, const NormIn *nin, const RouteEpi &route,
                       hipStream_t st);
bool launch_gemv_experts(const DevWeight &stacked, int slot_rows, const int *sel, int n_slots, const ActQ8 &act,
                         const float *act_f32, bool act_per_slot, int K, float *out, hipStream_t st,
                         const NormIn *nin = nullptr);
// With nin (gemv_norm_ok types) every workgroup forms the activation from RMSNorm(x)·w itself.
bool launch_gemv_glu_experts(const DevWeight &gate, const DevWeight &up, int ff, const int *sel, int n_slots, const ActQ8 &act,
                             const float *act_f32, int K, float *h, int gelu, const ActQ8 *hq, hipStream_t st,
                             const NormIn *nin = nullptr);

// ---- grouped expert GEMMs (prompt batches of MoE layers, moe_ffn cpu.rs:487-524) ----
// The routed (token, slot) pairs of a batch, grouped by expert on the device: gathered
// row r of expert e lies in [off[e], off[e+1]); token tiles of bn rows (GROUP_BN, or 32
// for Q4_K experts) list their expert and first row.  A grouped GEMM runs one weight matrix per expert (expert e's at
// w + e·wstride) over that expert's rows only; its activation row for gathered row r is
// amap[r] (or r), its output row omap[r] (or r).
constexpr int GROUP_BN = 64;
struct GroupTiles {
    const int *tile_e = nullptr, *tile_r0 = nullptr, *n_tiles = nullptr, *off = nullptr;
    const int *amap = nullptr, *omap = nullptr;
    size_t wstride = 0;
    int max_tiles = 0;  // grid bound: token tiles of the largest possible grouping
    int bn = GROUP_BN;  // rows per token tile (32: the Q4_K GEMMs' 128 × 32 tiles)
};
// sel [n_tok·k] (ascending experts per token) → off [n_exp+1], row_tok / row_slot
// [n_tok·k] (token t and pair index t·k + j of each gathered row), the tile table
// (tile_e / tile_r0 [max_tiles], *n_tiles).  One workgroup; n_exp ≤ 512.
void launch_moe_group(const int *sel, int n_tok, int k, int n_exp, int *off, int *row_tok, int *row_slot, int *tile_e, int *tile_r0,
                      int *n_tiles, int bn, hipStream_t st);
int moe_group_max_tiles(int n_tok, int k, int n_exp, int bn = GROUP_BN);

// ---- gemm_kq.hip (prefill, Q4_K × Q8_K on int8 MFMA; reached through gemm.hip) ----
bool gemm_kq_supported(int ty, size_t K);
// part (part_cap floats): partial sums of a K split (Q6_K, one ungrouped segment)
bool launch_gemm_kq(const GemvSeg *segs, int nseg, const ActQ8 &act, int n_tok, int K, hipStream_t st, const GroupTiles *grp = nullptr,
                    float *part = nullptr, size_t part_cap = 0);
// out[t·ld + r] += part[0][t·ld + r] + … + part[n_part−1][…] (planes stride floats
// apart) for r < rows, t < n_tok, in split order
void launch_gemm_add_parts(float *out, const float *part, size_t stride, int n_part, int rows, int ld, int n_tok, hipStream_t st);
bool launch_gemm_kq_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, int n_tok, int K, float *h, int ld, int gelu,
                        hipStream_t st, const GroupTiles *grp = nullptr);

// ---- gemm.hip (prefill, int8 MFMA) ----
bool gemm_supported(int ty, size_t K);
// grp: one segment per expert group (the segment's rows are one expert's; see GroupTiles)
// part (part_cap floats): room for the partial sums of a K split (see launch_t)
bool launch_gemm(const GemvSeg *segs, int nseg, const ActQ8 &act, int n_tok, int K, hipStream_t st, const GroupTiles *grp = nullptr,
                 float *part = nullptr, size_t part_cap = 0);
bool launch_gemm_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, int n_tok, int K, float *h, int ld, int gelu,
                     float *scratch, hipStream_t st, const GroupTiles *grp = nullptr);

}  // namespace rie
