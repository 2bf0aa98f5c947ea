// model.cpp — GGUF reader and model description for the HIP backend.
// Restates the reference's gguf.rs:193-269, model/config.rs:106-247 and
// model/mod.rs:101-247 with the same error classes (Format / Unsupported /
// Missing) and messages.
#include "model.hpp"

#include <cmath>
#include <cstring>

namespace rie {

static Error fmt_err(const std::string &m) { return Error{E_FORMAT, "invalid model file: " + m}; }
static Error unsup(const std::string &m) { return Error{E_UNSUPPORTED, "unsupported: " + m}; }
static Error missing(const std::string &m) { return Error{E_MISSING, "missing: " + m}; }

size_t TensorInfo::rows() const {
    uint64_t n = 1;
    for (auto d : dims) n *= d;
    return (size_t)(n / dims[0]);
}

namespace {
struct Reader {
    const uint8_t *p;
    size_t len, pos = 0;
    const uint8_t *take(size_t n) {
        if (pos + n > len) throw fmt_err("unexpected end of file at byte " + std::to_string(pos));
        const uint8_t *s = p + pos;
        pos += n;
        return s;
    }
    template <class T>
    T get() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string str() {
        uint64_t n = get<uint64_t>();
        if (n > len) throw fmt_err("string length " + std::to_string(n) + " out of range");
        const uint8_t *s = take((size_t)n);
        return std::string((const char *)s, (size_t)n);
    }
    void value(uint32_t ty, KV &kv, int depth) {
        switch (ty) {
        case 0: kv.u = get<uint8_t>(); kv.i = (int64_t)kv.u; break;
        case 1: kv.i = get<int8_t>(); kv.u = (uint64_t)kv.i; break;
        case 2: kv.u = get<uint16_t>(); kv.i = (int64_t)kv.u; break;
        case 3: kv.i = get<int16_t>(); kv.u = (uint64_t)kv.i; break;
        case 4: kv.u = get<uint32_t>(); kv.i = (int64_t)kv.u; break;
        case 5: kv.i = get<int32_t>(); kv.u = (uint64_t)kv.i; break;
        case 6: kv.f = get<float>(); kv.i = (int64_t)kv.f; kv.u = (uint64_t)kv.i; break;
        case 7: kv.u = get<uint8_t>() != 0; kv.i = (int64_t)kv.u; break;
        case 8: kv.s = str(); break;
        case 9: {
            if (depth > 4) throw fmt_err("array nesting too deep");
            uint32_t et = get<uint32_t>();
            uint64_t n = get<uint64_t>();
            if (n > len) throw fmt_err("array length " + std::to_string(n) + " out of range");
            kv.arr_len = (size_t)n;
            KV tmp;
            for (uint64_t i = 0; i < n; i++) value(et, tmp, depth + 1);
            break;
        }
        case 10: kv.u = get<uint64_t>(); kv.i = (int64_t)kv.u; break;
        case 11: kv.i = get<int64_t>(); kv.u = (uint64_t)kv.i; break;
        case 12: kv.f = get<double>(); kv.i = (int64_t)kv.f; kv.u = (uint64_t)kv.i; break;
        default: throw fmt_err("unknown metadata value type " + std::to_string(ty));
        }
        if (ty != 6 && ty != 12 && ty != 8 && ty != 9) kv.f = (ty == 1 || ty == 3 || ty == 5 || ty == 11) ? (double)kv.i : (double)kv.u;
    }
};

bool valid_type(uint32_t id) {
    switch (id) {
    case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 10: case 11: case 12: case 13: case 14: case 30: return true;
    default: return false;
    }
}
}  // namespace

Gguf Gguf::parse(const uint8_t *p, size_t len) {
    Gguf g;
    g.base = p;
    g.len = len;
    Reader r{p, len};
    if (r.get<uint32_t>() != 0x46554747u) throw fmt_err("not a GGUF file (bad magic)");
    uint32_t version = r.get<uint32_t>();
    if (version < 2 || version > 3) throw unsup("GGUF version " + std::to_string(version) + " (only v2 and v3 are supported)");
    uint64_t n_t = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = r.str();
        KV kv;
        kv.type = r.get<uint32_t>();
        r.value(kv.type, kv, 0);
        g.kv[key] = kv;  // later keys replace earlier ones (HashMap insert)
    }
    uint64_t align = 32;
    if (auto a = g.get("general.alignment"); a && a->type != 6 && a->type != 12 && a->type != 8 && a->type != 9 && a->u > 0)
        align = a->u;
    std::vector<TensorInfo> infos;
    for (uint64_t i = 0; i < n_t; i++) {
        TensorInfo t;
        t.name = r.str();
        uint32_t nd = r.get<uint32_t>();
        if (nd == 0 || nd > 4) throw fmt_err("tensor " + t.name + " has " + std::to_string(nd) + " dims");
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(r.get<uint64_t>());
        uint32_t id = r.get<uint32_t>();
        if (!valid_type(id)) throw unsup("tensor " + t.name + " uses ggml type id " + std::to_string(id));
        t.ty = (int)id;
        t.offset = r.get<uint64_t>();
        infos.push_back(std::move(t));
    }
    g.data_start = (r.pos + align - 1) / align * align;
    for (auto &t : infos) {
        uint64_t n = 1;
        for (auto d : t.dims) n *= d;
        if (t.dims[0] % block_size(t.ty) != 0) throw fmt_err("tensor " + t.name + ": row length " + std::to_string(t.dims[0]) + " not a multiple of block size");
        t.size = n / block_size(t.ty) * block_bytes(t.ty);
        t.offset += g.data_start;
        if (t.offset + t.size > len) throw fmt_err("tensor " + t.name + " extends past end of file");
        g.index[t.name] = g.tensors.size();
        g.tensors.push_back(t);
    }
    return g;
}

const KV *Gguf::get(const std::string &k) const {
    auto it = kv.find(k);
    return it == kv.end() ? nullptr : &it->second;
}

const TensorInfo *Gguf::tensor(const std::string &name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
}

// ---- config.rs:106-247 -------------------------------------------------------------
static bool is_int(const KV *k) { return k && k->type != 6 && k->type != 12 && k->type != 8 && k->type != 9; }
static bool get_u(const Gguf &g, const std::string &key, uint64_t &out) {
    const KV *k = g.get(key);
    if (!is_int(k)) return false;
    if ((k->type == 1 || k->type == 3 || k->type == 5 || k->type == 11) && k->i < 0) return false;
    out = k->u;
    return true;
}
static bool get_f(const Gguf &g, const std::string &key, float &out) {
    const KV *k = g.get(key);
    if (!k || k->type == 8 || k->type == 9) return false;
    out = (float)k->f;
    return true;
}

ModelConfig ModelConfig::from_gguf(const Gguf &g) {
    ModelConfig c;
    const KV *ak = g.get("general.architecture");
    if (!ak || ak->type != 8) throw missing("general.architecture");
    c.arch_name = ak->s;
    static const std::map<std::string, Arch> names = {{"llama", A_LLAMA}, {"mistral", A_LLAMA}, {"qwen2", A_QWEN2}, {"qwen3", A_QWEN3},
                                                      {"phi3", A_PHI3}, {"gemma", A_GEMMA}, {"gemma2", A_GEMMA2}, {"gemma3", A_GEMMA3},
                                                      {"granite", A_GRANITE}, {"qwen3moe", A_QWEN3MOE}, {"qwen2moe", A_QWEN2MOE}};
    auto it = names.find(c.arch_name);
    if (it == names.end())
        throw unsup("architecture '" + c.arch_name + "' (supported: llama, mistral, qwen2, qwen3, phi3, gemma, gemma2, gemma3, granite, qwen3moe, qwen2moe)");
    c.arch = it->second;
    if (auto n = g.get("general.name"); n && n->type == 8) c.name = n->s;
    const std::string a = c.arch_name + ".";
    uint64_t v;
    auto req = [&](const char *k) -> size_t {
        if (!get_u(g, a + k, v)) throw missing("metadata " + a + k);
        return (size_t)v;
    };
    c.n_embd = req("embedding_length");
    c.n_layer = req("block_count");
    c.n_head = req("attention.head_count");
    c.n_head_kv = get_u(g, a + "attention.head_count_kv", v) ? (size_t)v : c.n_head;
    c.head_dim = get_u(g, a + "attention.key_length", v) ? (size_t)v : c.n_embd / c.n_head;
    if (get_u(g, a + "attention.value_length", v) && v != c.head_dim)
        throw unsup("value head dim " + std::to_string(v) + " != key head dim " + std::to_string(c.head_dim));
    if (get_u(g, a + "feed_forward_length", v) || get_u(g, a + "expert_feed_forward_length", v)) c.n_ff = (size_t)v;
    else throw missing("metadata " + a + "feed_forward_length");
    if (auto tk = g.get("tokenizer.ggml.tokens"); tk && tk->type == 9) c.n_vocab = tk->arr_len;
    else if (get_u(g, a + "vocab_size", v)) c.n_vocab = (size_t)v;
    else throw missing("vocabulary");
    if (!get_f(g, a + "attention.layer_norm_rms_epsilon", c.rms_eps)) c.rms_eps = 1e-5f;
    c.ctx_train = get_u(g, a + "context_length", v) ? (size_t)v : 4096;
    c.rope_dim = get_u(g, a + "rope.dimension_count", v) ? (size_t)v : c.head_dim;
    if (!get_f(g, a + "rope.freq_base", c.rope_base)) c.rope_base = 10000.0f;
    float f;
    if (auto st = g.get(a + "rope.scaling.type"); st && st->type == 8 && st->s == "linear" && get_f(g, a + "rope.scaling.factor", f) && f > 0)
        c.rope_freq_scale = 1.0f / f;
    if (get_f(g, a + "rope.scale_linear", f) && f > 0) c.rope_freq_scale = 1.0f / f;
    c.rope_neox = !(c.arch == A_LLAMA || c.arch == A_GRANITE);
    c.n_expert = get_u(g, a + "expert_count", v) ? (size_t)v : 0;
    c.n_expert_used = get_u(g, a + "expert_used_count", v) ? (size_t)v : 2;
    c.n_ff_exp = get_u(g, a + "expert_feed_forward_length", v) ? (size_t)v : c.n_ff;
    if (const KV *nk = g.get(a + "expert_weights_norm")) c.expert_norm_topk = nk->u != 0;
    else c.expert_norm_topk = c.arch != A_QWEN2MOE;
    const bool gemma = c.arch == A_GEMMA || c.arch == A_GEMMA2 || c.arch == A_GEMMA3;
    c.gelu = gemma;
    c.embd_scale = gemma ? std::sqrt((float)c.n_embd) : 1.0f;
    c.attn_scale = 1.0f / std::sqrt((float)c.head_dim);
    if (c.arch == A_GEMMA2) {
        if (!get_f(g, a + "attn_logit_softcapping", c.attn_softcap)) c.attn_softcap = 50.0f;
        if (!get_f(g, a + "final_logit_softcapping", c.final_softcap)) c.final_softcap = 30.0f;
        c.swa_window = get_u(g, a + "attention.sliding_window", v) ? (size_t)v : 4096;
        c.swa_pattern = 2;
        if (c.n_layer == 46) c.attn_scale = 1.0f / std::sqrt((float)(c.n_embd / c.n_head));
    } else if (c.arch == A_GEMMA3) {
        c.swa_window = get_u(g, a + "attention.sliding_window", v) ? (size_t)v : 1024;
        c.swa_pattern = 6;
        c.has_rope_swa = true;
        c.rope_base_swa = 10000.0f;
        if (c.n_layer == 62) c.attn_scale = 1.0f / std::sqrt((float)(c.n_embd / c.n_head));
        if (!get_f(g, a + "final_logit_softcapping", c.final_softcap)) c.final_softcap = 0.0f;
        if (!get_f(g, a + "attn_logit_softcapping", c.attn_softcap)) c.attn_softcap = 0.0f;
    } else if (c.arch == A_GRANITE) {
        if (!get_f(g, a + "embedding_scale", c.embd_scale)) c.embd_scale = 1.0f;
        if (!get_f(g, a + "residual_scale", c.residual_scale)) c.residual_scale = 1.0f;
        if (!get_f(g, a + "logit_scale", c.logit_scale)) c.logit_scale = 1.0f;
        float s;
        if (get_f(g, a + "attention.scale", s)) c.attn_scale = s;
    }
    if (c.n_head_kv == 0 || c.n_head % c.n_head_kv != 0)
        throw fmt_err("n_head " + std::to_string(c.n_head) + " not divisible by n_head_kv " + std::to_string(c.n_head_kv));
    if (c.rope_dim > c.head_dim || c.rope_dim % 2 != 0) throw fmt_err("invalid rope dimension " + std::to_string(c.rope_dim));
    return c;
}

// ---- model/mod.rs:101-247 --------------------------------------------------------------
static HostWeight weight_of(const TensorInfo &t) {
    const bool stacked_ok = t.name.find("_exps") != std::string::npos && t.dims.size() == 3;
    if (t.dims.size() > 2 && !stacked_ok)
        for (size_t i = 2; i < t.dims.size(); i++)
            if (t.dims[i] != 1) throw unsup("tensor " + t.name + " has an unsupported shape");
    HostWeight w;
    w.ty = t.ty;
    w.rows = t.rows();
    w.cols = t.cols();
    w.off = t.offset;
    return w;
}

HostModel HostModel::load(const Gguf &g) {
    HostModel m;
    m.cfg = ModelConfig::from_gguf(g);
    const ModelConfig &c = m.cfg;
    auto get = [&](const std::string &n) -> HostWeight {
        const TensorInfo *t = g.tensor(n);
        if (!t) throw missing("tensor " + n);
        return weight_of(*t);
    };
    auto opt = [&](const std::string &n) -> HostWeight {
        const TensorInfo *t = g.tensor(n);
        return t ? weight_of(*t) : HostWeight{};
    };
    m.token_embd = get("token_embd.weight");
    if (m.token_embd.cols != c.n_embd)
        throw fmt_err("token_embd has " + std::to_string(m.token_embd.cols) + " columns, expected " + std::to_string(c.n_embd));
    m.output = opt("output.weight");
    if (!m.output.present()) m.output = m.token_embd;
    m.output_norm = get("output_norm.weight");
    m.rope_factors = opt("rope_freqs.weight");
    if (!m.rope_factors.present()) m.rope_factors = opt("rope_factors_short.weight");
    const size_t qd = c.q_dim(), kvd = c.kv_dim();
    for (size_t il = 0; il < c.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        HostLayer L;
        HostWeight qkv = opt(p + "attn_qkv.weight");
        if (qkv.present()) {
            if (qkv.rows != qd + 2 * kvd)
                throw fmt_err("fused qkv has " + std::to_string(qkv.rows) + " rows, expected " + std::to_string(qd + 2 * kvd));
            L.wq = qkv.slice_rows(0, qd);
            L.wk = qkv.slice_rows(qd, kvd);
            L.wv = qkv.slice_rows(qd + kvd, kvd);
        } else {
            L.wq = get(p + "attn_q.weight");
            L.wk = get(p + "attn_k.weight");
            L.wv = get(p + "attn_v.weight");
        }
        HostWeight router = opt(p + "ffn_gate_inp.weight");
        if (router.present()) {
            const size_t ne = c.n_expert, ff = c.n_ff_exp;
            if (ne == 0 || router.rows != ne || router.cols != c.n_embd)
                throw fmt_err(p + "ffn_gate_inp: shape " + std::to_string(router.rows) + "x" + std::to_string(router.cols));
            L.moe = true;
            L.router = router;
            auto stacked = [&](const std::string &n, size_t rows, size_t cols) {
                HostWeight w = get(p + n);
                if (w.rows != rows * ne || w.cols != cols) throw fmt_err(p + n + ": unexpected shape");
                return w;
            };
            L.gate = stacked("ffn_gate_exps.weight", ff, c.n_embd);
            L.up = stacked("ffn_up_exps.weight", ff, c.n_embd);
            L.down = stacked("ffn_down_exps.weight", c.n_embd, ff);
            L.shexp_gate = opt(p + "ffn_gate_shexp.weight");
            if (L.shexp_gate.present()) {
                L.shexp_up = get(p + "ffn_up_shexp.weight");
                L.shexp_down = get(p + "ffn_down_shexp.weight");
            }
            L.shexp_gate_inp = opt(p + "ffn_gate_inp_shexp.weight");
            L.n_used = std::min(std::max(c.n_expert_used, (size_t)1), ne);
            L.norm_topk = c.expert_norm_topk;
            const KV *gk = g.get("rie.expert_gating");
            L.unit_weights = gk && gk->type == 8 && gk->s == "unit";
        } else {
            HostWeight gw = opt(p + "ffn_gate.weight");
            if (gw.present()) {
                L.gate = gw;
                L.up = get(p + "ffn_up.weight");
            } else {
                HostWeight up = get(p + "ffn_up.weight");
                if (up.rows != 2 * c.n_ff) throw unsup("layer " + std::to_string(il) + ": missing ffn_gate and ffn_up is not fused");
                L.gate = up.slice_rows(0, c.n_ff);
                L.up = up.slice_rows(c.n_ff, c.n_ff);
            }
            L.down = get(p + "ffn_down.weight");
            const HostWeight *ws[3] = {&L.gate, &L.up, &L.down};
            const char *nm[3] = {"ffn_gate", "ffn_up", "ffn_down"};
            size_t er[3] = {c.n_ff, c.n_ff, c.n_embd}, ec[3] = {c.n_embd, c.n_embd, c.n_ff};
            for (int i = 0; i < 3; i++)
                if (ws[i]->rows != er[i] || ws[i]->cols != ec[i]) throw fmt_err(p + nm[i] + ": unexpected shape");
        }
        L.attn_norm = get(p + "attn_norm.weight");
        L.wo = get(p + "attn_output.weight");
        L.bq = opt(p + "attn_q.bias");
        L.bk = opt(p + "attn_k.bias");
        L.bv = opt(p + "attn_v.bias");
        L.q_norm = opt(p + "attn_q_norm.weight");
        L.k_norm = opt(p + "attn_k_norm.weight");
        L.post_attn_norm = opt(p + "post_attention_norm.weight");
        L.ffn_norm = opt(p + "ffn_norm.weight");
        if (!L.ffn_norm.present()) throw missing("tensor " + p + "ffn_norm.weight");
        L.post_ffn_norm = opt(p + "post_ffw_norm.weight");
        const HostWeight *chk[4] = {&L.wq, &L.wk, &L.wv, &L.wo};
        size_t er[4] = {qd, kvd, kvd, c.n_embd}, ec[4] = {c.n_embd, c.n_embd, c.n_embd, qd};
        const char *nm[4] = {"attn_q", "attn_k", "attn_v", "attn_output"};
        for (int i = 0; i < 4; i++)
            if (chk[i]->rows != er[i] || chk[i]->cols != ec[i])
                throw fmt_err(p + nm[i] + ": shape " + std::to_string(chk[i]->rows) + "x" + std::to_string(chk[i]->cols));
        if (L.q_norm.present() && L.q_norm.rows * L.q_norm.cols != c.head_dim)
            throw unsup("q_norm over " + std::to_string(L.q_norm.rows * L.q_norm.cols) + " elements (expected per-head " + std::to_string(c.head_dim) + ")");
        m.layers.push_back(L);
    }
    if (m.output.cols != c.n_embd || m.output.rows < c.n_vocab)
        throw fmt_err("output matrix " + std::to_string(m.output.rows) + "x" + std::to_string(m.output.cols) + " does not cover vocabulary");
    return m;
}

}  // namespace rie
