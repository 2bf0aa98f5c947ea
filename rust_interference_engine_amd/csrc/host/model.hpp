// model.hpp — GGUF image parsing and the model description the HIP backend
// consumes: hyper-parameters (ModelConfig, model/config.rs:55-93 in the
// reference) and the tensor table (Model::load, model/mod.rs:112-247).
#pragma once

#include "../common.hpp"

#include <map>
#include <string>
#include <vector>

namespace rie {

struct KV {
    uint32_t type = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    size_t arr_len = 0;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    int ty = 0;
    uint64_t offset = 0;  // absolute offset in the image
    uint64_t size = 0;
    size_t rows() const;
    size_t cols() const { return (size_t)dims[0]; }
};

// gguf.rs:212-269: header, metadata, tensor table, data at align(general.alignment|32)
struct Gguf {
    std::map<std::string, KV> kv;
    std::vector<TensorInfo> tensors;
    std::map<std::string, size_t> index;
    uint64_t data_start = 0;
    const uint8_t *base = nullptr;
    size_t len = 0;

    static Gguf parse(const uint8_t *p, size_t len);  // throws Error
    const KV *get(const std::string &k) const;
    const TensorInfo *tensor(const std::string &name) const;
};

enum Arch { A_LLAMA, A_QWEN2, A_QWEN3, A_PHI3, A_GEMMA, A_GEMMA2, A_GEMMA3, A_GRANITE, A_QWEN3MOE, A_QWEN2MOE };

struct ModelConfig {
    Arch arch = A_LLAMA;
    std::string arch_name, name;
    size_t n_vocab = 0, n_embd = 0, n_layer = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ff = 0, ctx_train = 0;
    size_t rope_dim = 0;
    bool rope_neox = false;
    float rms_eps = 1e-5f, rope_base = 10000.0f, rope_freq_scale = 1.0f;
    bool has_rope_swa = false;
    float rope_base_swa = 10000.0f;
    bool gelu = false;
    float embd_scale = 1.0f, attn_scale = 1.0f, residual_scale = 1.0f, logit_scale = 1.0f;
    float attn_softcap = 0.0f, final_softcap = 0.0f;  // 0 = none
    size_t swa_window = 0, swa_pattern = 0;
    size_t n_expert = 0, n_expert_used = 2, n_ff_exp = 0;
    bool expert_norm_topk = true;

    size_t q_dim() const { return n_head * head_dim; }
    size_t kv_dim() const { return n_head_kv * head_dim; }
    bool is_swa(size_t il) const { return swa_window > 0 && swa_pattern > 0 && (il % swa_pattern) < swa_pattern - 1; }
    static ModelConfig from_gguf(const Gguf &g);  // throws Error
};

// A weight as a view into the GGUF image: offset relative to data_start.
struct HostWeight {
    int ty = -1;
    size_t rows = 0, cols = 0;
    uint64_t off = 0;  // absolute offset in the image
    bool present() const { return ty >= 0; }
    size_t rb() const { return row_bytes(ty, cols); }
    HostWeight slice_rows(size_t start, size_t n) const {
        HostWeight w = *this;
        w.rows = n;
        w.off = off + start * rb();
        return w;
    }
};

struct HostLayer {
    HostWeight attn_norm, ffn_norm, q_norm, k_norm, bq, bk, bv, post_attn_norm, post_ffn_norm;
    HostWeight wq, wk, wv, wo;
    bool moe = false;
    HostWeight gate, up, down;                  // dense, or stacked experts
    HostWeight router, shexp_gate, shexp_up, shexp_down, shexp_gate_inp;
    size_t n_used = 0;
    bool norm_topk = true, unit_weights = false;
};

struct HostModel {
    ModelConfig cfg;
    HostWeight token_embd, output, output_norm, rope_factors;
    std::vector<HostLayer> layers;
    static HostModel load(const Gguf &g);  // throws Error
};

}  // namespace rie
