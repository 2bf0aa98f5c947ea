// backend.hpp — the HIP implementation of RIE's Backend contract
// (trait Backend, model/mod.rs:303-320 in the reference).
#pragma once

#include "../common.hpp"
#include "../kernels.hpp"
#include "model.hpp"

#include <memory>
#include <string>
#include <map>
#include <vector>

namespace rie {

struct BackendConfig {
    size_t n_ctx = 4096;
    size_t max_batch = 64;
    int kv_type = 0;      // 0 f16, 1 q8_0, 2 turbo4
    int device = 0;
    bool use_graph = true;  // capture the single-token decode step in a HIP graph
};

class HipBackend {
  public:
    HipBackend(const uint8_t *gguf, size_t len, const BackendConfig &cfg);
    ~HipBackend();
    HipBackend(const HipBackend &) = delete;
    HipBackend &operator=(const HipBackend &) = delete;

    const std::string &name() const { return name_; }
    size_t max_batch() const { return max_batch_; }
    size_t n_ctx() const { return n_ctx_; }
    int kv_type() const { return kv_type_; }
    size_t kv_bytes() const { return kv_bytes_; }
    size_t weight_bytes() const { return blob_len_; }
    const ModelConfig &config() const { return m_.cfg; }

    // Backend::forward: logits of the last token ([V]) or of all tokens ([n·V]).
    void forward(const uint32_t *tokens, size_t n, size_t pos, bool all_logits, float *logits, size_t logits_len);
    // Backend::hidden: final normalized rows of the last forward (copied on request).
    const float *hidden(size_t *rows);

    // Engine-side greedy decoding on the device (sampler.rs::argmax, first max).
    uint32_t forward_argmax(const uint32_t *tokens, size_t n, size_t pos);
    // n_gen greedy steps: feeds the last argmax token at pos, pos+1, ...; writes the
    // fed tokens to out (out[0] = the token chosen by the previous forward).
    void generate_greedy(size_t pos, size_t n_gen, uint32_t *out);
    void synchronize();

    // debugging / parity hooks
    void set_capture(bool on);
    void set_attention_ranges(bool on) { attn_ranges_only_ = on; }  // single token: range kernel at every context length
    bool capture(size_t layer, int what, float *out, size_t len);
    void kv_layer(size_t layer, int which, uint8_t *out, size_t len, uint8_t *scales_out, size_t scales_len);
    size_t kv_row_bytes() const;
    // TurboQuant rotation blocks per head vector: head_dim / largest power of two ≤ 256 dividing it
    size_t turbo_blocks() const {
        size_t b = 1, d = m_.cfg.head_dim;
        while (d % (b * 2) == 0 && b < 256) b *= 2;
        return d / b;
    }
    hipStream_t stream() const { return st_; }
    // kernel time probe: runs the decode step `reps` times eagerly and times each
    // kernel family with events (ms per launch, summed per family)
    struct KernelTime {
        std::string name;
        double ms = 0;   // summed over launches
        int launches = 0;
    };
    std::vector<KernelTime> profile_decode(size_t pos, int reps);
    // Average duration (µs) of the single-token gate/up/SwiGLU launch, cycling
    // through every layer's weights; *bytes = algorithmic bytes of one launch.
    double time_ffn_glu(int reps, size_t *bytes);

  private:
    struct DevLayer {
        const float *attn_norm, *ffn_norm, *q_norm, *k_norm, *bq, *bk, *bv, *post_attn_norm, *post_ffn_norm;
        DevWeight wq, wk, wv, wo, gate, up, down, router, sh_gate, sh_up, sh_down;
        const float *sh_gate_inp;
        bool moe;
        size_t n_used, ff;
        bool norm_topk, unit_weights;
        uint8_t *k_cache, *v_cache;
        uint16_t *k_scale, *v_scale;
        size_t slots;
    };

    DevWeight dev(const HostWeight &w) const;
    const float *dev_vec(const HostWeight &w);
    void run_layers(int n, size_t pos0, const int *d_pos0, bool all_logits, int n_split);
    void prepare(const float *x, const float *norm, int n, int K, const DevWeight *const *ws, int nw, bool want_f32,
                 bool ref_order = false);
    void matmul(const GemvSeg *segs, int nseg, int n, int K, const ActQ8 *act_q8_0 = nullptr);
    void ffn_dense(const DevLayer &L, int n, float *out_resid, int epi);
    // writes the block's output to d_o_, or (true returned) adds it to d_x_ itself
    bool ffn_moe(const DevLayer &L, int n, bool direct);
    void expert_ffn(const DevWeight &g, const DevWeight &u, const DevWeight &dn, const float *x, int m, float *y);
    void head(int first, int m);
    void check_launch(const char *what);
    void decode_step_graph(size_t pos);
    void greedy_step_graph(size_t pos);
    // context ranges per (token, kv head) in attention; the same for every batch size so
    // a token's attention does not depend on how its batch was formed
    int splits_for(size_t n, size_t pos) const;  // attention context ranges of a launch

    HostModel m_;
    std::string name_;
    size_t n_ctx_, max_batch_;
    int kv_type_;
    size_t kv_bytes_ = 0;
    bool use_graph_;
    hipStream_t st_ = nullptr;
    int device_ = 0;

    uint8_t *d_blob_ = nullptr;
    size_t blob_len_ = 0;
    uint64_t blob_base_off_ = 0;
    std::vector<void *> allocs_;
    std::vector<DevLayer> layers_;
    DevWeight embd_, out_w_;
    const float *out_norm_ = nullptr;
    float *d_cos_ = nullptr, *d_sin_ = nullptr, *d_cos_swa_ = nullptr, *d_sin_swa_ = nullptr, *d_signs_ = nullptr;

    // scratch
    uint32_t *d_tokens_ = nullptr, *d_next_ = nullptr, *d_gen_ = nullptr;
    int *d_pos_ = nullptr;
    float *d_x_ = nullptr, *d_xn_ = nullptr, *d_q_ = nullptr, *d_k_ = nullptr, *d_v_ = nullptr, *d_att_ = nullptr, *d_h_ = nullptr,
          *d_o_ = nullptr, *d_logits_ = nullptr, *d_part_ = nullptr, *d_amax_val_ = nullptr, *d_gemm_ws_ = nullptr;
    size_t gemm_ws_cap_ = 0;  // floats at d_gemm_ws_
    int *d_amax_idx_ = nullptr, *d_amax_cnt_ = nullptr;
    int *d_attn_cnt_ = nullptr;  // per-KV-head arrival counters of the fused single-token attention
    int *d_route_cnt_ = nullptr;  // arrival counter of the router GEMV that routes one token
    ActQ8 act0_, actk_;  // Q8_0 and Q8_K batches
    ActQ8 act_h_;        // Q8_0 of the single-token FFN hidden
    size_t kmax_ = 0, ff_max_ = 0, part_floats_ = 0;
    size_t n_used_max_ = 0;  // largest clamped routed-expert count of any MoE layer
    // MoE scratch
    float *d_router_ = nullptr, *d_moe_w_ = nullptr, *d_moe_y_ = nullptr;
    float *d_moe_xn_ = nullptr, *d_moe_xg_ = nullptr, *d_moe_yg_ = nullptr, *d_moe_rw_ = nullptr;
    int *d_moe_sel_ = nullptr, *d_moe_rows_ = nullptr;
    int *d_moe_off_ = nullptr, *d_moe_rtok_ = nullptr, *d_moe_rslot_ = nullptr, *d_moe_tile_e_ = nullptr, *d_moe_tile_r0_ = nullptr,
        *d_moe_ntiles_ = nullptr;
    int moe_max_tiles_ = 0;
    bool moe_grouped_ok(const DevLayer &L) const;
    float *d_kcap_ = nullptr;  // K after norm/RoPE when capturing
    int n_amax_part_ = 64;

    size_t hidden_rows_ = 0;
    int head_first_ = 0;        // first batch row of the last head launch
    bool head_normed_ = true;   // d_xn_ holds the head's normalized rows (else Backend::hidden forms them)
    std::vector<float> hidden_host_;
    bool capture_ = false;
    bool attn_ranges_only_ = false;
    std::vector<std::vector<std::vector<float>>> cap_;  // [what][layer]
    size_t cur_layer_ = 0;                               // layer run_layers is in (capture bookkeeping)

    // per-launch event marks while profiling (eager path only)
    void mark(const char *name);
    bool profiling_ = false;
    std::vector<std::pair<const char *, hipEvent_t>> marks_;
    hipEvent_t mark0_ = nullptr;

    struct DecodeGraph {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        // the head's state as captured: every replay leaves d_x_/d_xn_ as the
        // captured launches do, so Backend::hidden must see these values again
        bool head_normed = true;
        int head_first = 0;
    };
    std::map<int, DecodeGraph> graphs_;  // by attention range count
    std::map<int, DecodeGraph> greedy_graphs_;  // the same with the advancing argmax (generate_greedy)
    bool in_capture_ = false;
};

}  // namespace rie
