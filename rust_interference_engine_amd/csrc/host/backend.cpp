// backend.cpp — HipBackend: the per-token forward loop of RIE
// (CpuBackend::forward_impl, model/cpu.rs:210-409 in the reference) on one
// MI355X.  The GGUF tensor data is uploaded once, unchanged, into one HBM
// buffer; every weight is a view into it.  A forward call is a fixed sequence
// of stream-ordered kernel launches; the single-token decode step is captured
// once in a HIP graph whose only per-step inputs live in device memory
// ({pos} and the token id), so greedy decoding never returns to the host.
#include "backend.hpp"

#include "../kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace rie {

static Error rt_err(const std::string &m) { return Error{E_RUNTIME, m}; }

template <class T>
static T *dalloc(std::vector<void *> &list, size_t count) {
    void *p = nullptr;
    size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    RIE_HIP_CHECK(hipMalloc(&p, bytes));
    RIE_HIP_CHECK(hipMemset(p, 0, bytes));
    list.push_back(p);
    return (T *)p;
}

static bool gemv_type_ok(int ty, size_t K) { return gemv_supported(ty, K); }

HipBackend::HipBackend(const uint8_t *gguf, size_t len, const BackendConfig &cfg) {
    Gguf g = Gguf::parse(gguf, len);
    m_ = HostModel::load(g);
    const ModelConfig &c = m_.cfg;
    n_ctx_ = std::max<size_t>(cfg.n_ctx, 1);
    max_batch_ = std::min(std::max<size_t>(cfg.max_batch, 1), n_ctx_);
    use_graph_ = cfg.use_graph;
    device_ = cfg.device;
    int kv = cfg.kv_type;
    // cpu.rs:103-108: Q8_0 needs hd%32==0, Turbo4 needs hd%32==0 and hd<=512
    if (kv == 1 && c.head_dim % 32 != 0) kv = 0;
    if (kv == 2 && (c.head_dim % 32 != 0 || c.head_dim > 512)) kv = 0;
    kv_type_ = kv;
    if (c.head_dim % 8 != 0) throw Error{E_UNSUPPORTED, "unsupported: head dim " + std::to_string(c.head_dim) + " (not a multiple of 8) on the HIP backend"};
    if (c.head_dim > 256) throw Error{E_UNSUPPORTED, "unsupported: head dim " + std::to_string(c.head_dim) + " on the HIP backend"};
    if (c.n_head / c.n_head_kv > 8) throw Error{E_UNSUPPORTED, "unsupported: more than 8 query heads per KV head"};

    // shape/type checks: every matrix needs a kernel
    auto need = [&](const HostWeight &w, const char *what) {
        if (!w.present()) return;
        if (!gemv_type_ok(w.ty, w.cols))
            throw Error{E_UNSUPPORTED, std::string("unsupported: ") + what + " of type " + type_name(w.ty) + " with " +
                                           std::to_string(w.cols) + " columns on the HIP backend"};
    };
    for (auto &L : m_.layers) {
        need(L.wq, "attn_q"); need(L.wk, "attn_k"); need(L.wv, "attn_v"); need(L.wo, "attn_output");
        need(L.gate, "ffn_gate"); need(L.up, "ffn_up"); need(L.down, "ffn_down"); need(L.router, "ffn_gate_inp");
        if (L.moe) {
            need(L.shexp_gate, "ffn_gate_shexp"); need(L.shexp_up, "ffn_up_shexp"); need(L.shexp_down, "ffn_down_shexp");
            if (m_.cfg.n_expert > 512 || L.n_used > 64)
                throw Error{E_UNSUPPORTED, "unsupported: more than 512 experts or 64 experts per token on the HIP backend"};
        }
        for (const HostWeight *nw : {&L.attn_norm, &L.ffn_norm, &L.q_norm, &L.k_norm, &L.bq, &L.bk, &L.bv, &L.post_attn_norm, &L.post_ffn_norm})
            if (nw->present() && nw->ty != T_F32) throw Error{E_UNSUPPORTED, "unsupported: non-F32 norm/bias vectors"};
    }
    need(m_.output, "output");
    {
        int et = m_.token_embd.ty;
        if (block_bytes(et) == 0)  // every ggml type of the reference has an embedding dequantizer here
            throw Error{E_UNSUPPORTED, std::string("unsupported: token_embd of type ") + type_name(et)};
    }

    RIE_HIP_CHECK(hipSetDevice(device_));
    RIE_HIP_CHECK(hipStreamCreateWithFlags(&st_, hipStreamNonBlocking));
    hipDeviceProp_t prop;
    RIE_HIP_CHECK(hipGetDeviceProperties(&prop, device_));
    name_ = std::string("HIP ") + prop.gcnArchName + " (" + std::to_string(prop.multiProcessorCount) + " CUs)";

    // ---- weights: the GGUF data region, once, unchanged ----
    blob_base_off_ = g.data_start;
    blob_len_ = len - g.data_start;
    RIE_HIP_CHECK(hipMalloc(&d_blob_, blob_len_ + 4096));  // slack for realigning vector loads at the end
    RIE_HIP_CHECK(hipMemcpy(d_blob_, gguf + g.data_start, blob_len_, hipMemcpyHostToDevice));
    RIE_HIP_CHECK(hipMemset(d_blob_ + blob_len_, 0, 4096));

    const size_t hd = c.head_dim, E = c.n_embd, qd = c.q_dim(), kvd = c.kv_dim();
    embd_ = dev(m_.token_embd);
    out_w_ = dev(m_.output.rows > c.n_vocab ? m_.output.slice_rows(0, c.n_vocab) : m_.output);
    out_norm_ = dev_vec(m_.output_norm);
    ff_max_ = 0;
    for (auto &L : m_.layers) {
        DevLayer D{};
        D.attn_norm = dev_vec(L.attn_norm);
        D.ffn_norm = dev_vec(L.ffn_norm);
        D.q_norm = dev_vec(L.q_norm);
        D.k_norm = dev_vec(L.k_norm);
        D.bq = dev_vec(L.bq);
        D.bk = dev_vec(L.bk);
        D.bv = dev_vec(L.bv);
        D.post_attn_norm = dev_vec(L.post_attn_norm);
        D.post_ffn_norm = dev_vec(L.post_ffn_norm);
        D.wq = dev(L.wq); D.wk = dev(L.wk); D.wv = dev(L.wv); D.wo = dev(L.wo);
        D.gate = dev(L.gate); D.up = dev(L.up); D.down = dev(L.down);
        D.moe = L.moe;
        if (L.moe) {
            D.router = dev(L.router);
            if (L.shexp_gate.present()) {
                D.sh_gate = dev(L.shexp_gate);
                D.sh_up = dev(L.shexp_up);
                D.sh_down = dev(L.shexp_down);
            }
            D.sh_gate_inp = dev_vec(L.shexp_gate_inp);
            D.n_used = L.n_used;
            D.ff = c.n_ff_exp;
            D.norm_topk = L.norm_topk;
            D.unit_weights = L.unit_weights;
            // the shared expert's hidden goes through the same scratch as the routed ones
            // (cpu.rs:134-140 sizes its buffers over dense, expert and shared-expert widths)
            if (D.sh_gate.data) ff_max_ = std::max(ff_max_, D.sh_gate.rows);
            n_used_max_ = std::max(n_used_max_, D.n_used);
        } else {
            D.ff = L.gate.rows;
        }
        ff_max_ = std::max(ff_max_, D.ff);
        layers_.push_back(D);
    }

    // ---- KV cache: [layer][kv_head][slot][row] ----
    const size_t rb = kv_row_bytes();
    for (size_t il = 0; il < c.n_layer; il++) {
        DevLayer &D = layers_[il];
        D.slots = c.is_swa(il) ? std::min(c.swa_window + max_batch_, n_ctx_) : n_ctx_;
        const size_t rows = c.n_head_kv * D.slots;
        D.k_cache = dalloc<uint8_t>(allocs_, rows * rb);
        D.v_cache = dalloc<uint8_t>(allocs_, rows * rb);
        kv_bytes_ += 2 * rows * rb;
        if (kv_type_ == 2) {  // one f16 scale per rotation block (turbo.rs:133-138)
            D.k_scale = dalloc<uint16_t>(allocs_, rows * turbo_blocks());
            D.v_scale = dalloc<uint16_t>(allocs_, rows * turbo_blocks());
            kv_bytes_ += 4 * rows * turbo_blocks();
        }
    }

    // ---- RoPE tables from libm powf/sinf/cosf, as ops.rs:65-89 computes them ----
    {
        const size_t half = c.rope_dim / 2;
        auto table = [&](float base, float fscale, bool factors, float *&dc, float *&ds) {
            std::vector<float> inv(std::max<size_t>(half, 1));
            std::vector<float> fac;
            if (factors && m_.rope_factors.present()) {
                fac.resize(m_.rope_factors.rows * m_.rope_factors.cols);
                std::memcpy(fac.data(), gguf + m_.rope_factors.off, fac.size() * 4);
            }
            for (size_t i = 0; i < half; i++) {
                float f = powf(base, -2.0f * (float)i / (float)c.rope_dim) * fscale;
                if (i < fac.size() && fac[i] != 0.0f) f /= fac[i];
                inv[i] = f;
            }
            std::vector<float> cs(n_ctx_ * std::max<size_t>(half, 1)), sn(cs.size());
            for (size_t p = 0; p < n_ctx_; p++)
                for (size_t i = 0; i < half; i++) {
                    const float th = (float)p * inv[i];
                    sn[p * half + i] = sinf(th);
                    cs[p * half + i] = cosf(th);
                }
            dc = dalloc<float>(allocs_, cs.size());
            ds = dalloc<float>(allocs_, sn.size());
            RIE_HIP_CHECK(hipMemcpy(dc, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
            RIE_HIP_CHECK(hipMemcpy(ds, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
        };
        table(c.rope_base, c.rope_freq_scale, true, d_cos_, d_sin_);
        if (c.has_rope_swa) table(c.rope_base_swa, 1.0f, false, d_cos_swa_, d_sin_swa_);
    }
    // TurboQuant sign pattern (turbo.rs:78-89) for KV_SEED
    {
        std::vector<float> s(hd);
        const uint64_t seed = 0x75426F5175616E74ULL;
        for (size_t i = 0; i < hd; i++) {
            uint64_t z = seed + (uint64_t)i * 0x9E3779B97F4A7C15ULL;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
            s[i] = ((z ^ (z >> 31)) & 1u) == 0 ? 1.0f : -1.0f;
        }
        d_signs_ = dalloc<float>(allocs_, hd);
        RIE_HIP_CHECK(hipMemcpy(d_signs_, s.data(), hd * 4, hipMemcpyHostToDevice));
    }

    // ---- scratch ----
    const size_t mb = max_batch_;
    kmax_ = std::max({E, qd, ff_max_});
    d_tokens_ = dalloc<uint32_t>(allocs_, mb);
    d_next_ = dalloc<uint32_t>(allocs_, 1);
    d_gen_ = dalloc<uint32_t>(allocs_, std::max<size_t>(n_ctx_, 1));
    d_pos_ = dalloc<int>(allocs_, 4);
    d_x_ = dalloc<float>(allocs_, mb * E);
    d_xn_ = dalloc<float>(allocs_, mb * kmax_);
    d_q_ = dalloc<float>(allocs_, mb * qd);
    d_k_ = dalloc<float>(allocs_, mb * kvd);
    d_v_ = dalloc<float>(allocs_, mb * kvd);
    d_kcap_ = dalloc<float>(allocs_, mb * kvd);
    d_att_ = dalloc<float>(allocs_, mb * qd);
    d_o_ = dalloc<float>(allocs_, mb * E);
    // partial sums of K-split prompt GEMMs (up to three planes of a batch's E-wide
    // outputs, at most 64 MiB): only batches above 64 tokens split
    gemm_ws_cap_ = mb > 64 ? std::min<size_t>(3 * mb * E, (size_t)1 << 24) : 0;
    if (gemm_ws_cap_) d_gemm_ws_ = dalloc<float>(allocs_, gemm_ws_cap_);
    // routed experts per token as the layers run them (clamped to [1, n_expert], model/mod.rs:176)
    const size_t nu = std::max<size_t>(n_used_max_, 1);
    d_h_ = dalloc<float>(allocs_, mb * ff_max_ * nu);
    d_logits_ = dalloc<float>(allocs_, mb * c.n_vocab);
    const size_t kq = mb * kmax_ * nu;
    act0_.qs = dalloc<int8_t>(allocs_, kq);
    act0_.d = dalloc<float>(allocs_, kq / 32);
    act0_.s = dalloc<float>(allocs_, kq / 32);
    act0_.isum = dalloc<int32_t>(allocs_, kq / 32);
    // Q8_0 of the single-token FFN hidden, written by the gate/up kernel while
    // it still reads act0_
    const size_t hrows = nu;  // routed experts of one token
    act_h_.qs = dalloc<int8_t>(allocs_, hrows * ff_max_);
    act_h_.d = dalloc<float>(allocs_, hrows * ff_max_ / 32 + 1);
    act_h_.s = dalloc<float>(allocs_, hrows * ff_max_ / 32 + 1);
    act_h_.isum = dalloc<int32_t>(allocs_, hrows * ff_max_ / 32 + 1);
    actk_.qs = dalloc<int8_t>(allocs_, kq);
    actk_.d = dalloc<float>(allocs_, kq / 256 + 1);
    actk_.bsums = dalloc<int16_t>(allocs_, kq / 16);
    part_floats_ = (size_t)std::max<size_t>(32 * mb, ATT_MAX_SPLIT) * c.n_head * (hd + 2);
    d_part_ = dalloc<float>(allocs_, part_floats_);
    d_attn_cnt_ = dalloc<int>(allocs_, c.n_head * ATT_CNT_STRIDE);  // one per head slice: at most one per query head
    d_route_cnt_ = dalloc<int>(allocs_, 64);  // the router GEMV's arrival counter (one-token routing)
    d_amax_idx_ = dalloc<int>(allocs_, n_amax_part_);
    d_amax_val_ = dalloc<float>(allocs_, n_amax_part_);
    d_amax_cnt_ = dalloc<int>(allocs_, 1);  // arrival counter of the one-launch argmax
    if (c.n_expert) {
        d_router_ = dalloc<float>(allocs_, mb * c.n_expert);
        d_moe_w_ = dalloc<float>(allocs_, mb * nu);
        d_moe_sel_ = dalloc<int>(allocs_, mb * nu);
        d_moe_y_ = dalloc<float>(allocs_, mb * nu * E);
        d_moe_xn_ = dalloc<float>(allocs_, mb * E);
        d_moe_xg_ = dalloc<float>(allocs_, mb * E);
        d_moe_yg_ = dalloc<float>(allocs_, mb * E);
        d_moe_rows_ = dalloc<int>(allocs_, mb * nu);
        d_moe_rw_ = dalloc<float>(allocs_, mb * nu);
        // device-side grouping of prompt batches (grouped expert GEMMs)
        moe_max_tiles_ = moe_group_max_tiles((int)mb, (int)nu, (int)c.n_expert, 32);  // the smaller tiles' bound
        d_moe_off_ = dalloc<int>(allocs_, c.n_expert + 1);
        d_moe_rtok_ = dalloc<int>(allocs_, mb * nu);
        d_moe_rslot_ = dalloc<int>(allocs_, mb * nu);
        d_moe_tile_e_ = dalloc<int>(allocs_, moe_max_tiles_);
        d_moe_tile_r0_ = dalloc<int>(allocs_, moe_max_tiles_);
        d_moe_ntiles_ = dalloc<int>(allocs_, 1);
    }
    cap_.resize(10);
    RIE_HIP_CHECK(hipDeviceSynchronize());
}

HipBackend::~HipBackend() {
    if (st_) (void)hipStreamSynchronize(st_);
    for (auto *m : {&graphs_, &greedy_graphs_})
        for (auto &kv : *m) {
            (void)hipGraphExecDestroy(kv.second.exec);
            (void)hipGraphDestroy(kv.second.graph);
        }
    for (void *p : allocs_) (void)hipFree(p);
    if (d_blob_) (void)hipFree(d_blob_);
    if (st_) (void)hipStreamDestroy(st_);
}

DevWeight HipBackend::dev(const HostWeight &w) const {
    DevWeight d;
    if (!w.present()) return d;
    d.ty = w.ty;
    d.rows = w.rows;
    d.cols = w.cols;
    d.data = d_blob_ + (w.off - blob_base_off_);
    return d;
}

const float *HipBackend::dev_vec(const HostWeight &w) {
    if (!w.present()) return nullptr;
    return (const float *)(const void *)(d_blob_ + (w.off - blob_base_off_));
}

size_t HipBackend::kv_row_bytes() const {
    const size_t hd = m_.cfg.head_dim;
    if (kv_type_ == 0) return hd * 2;
    if (kv_type_ == 1) return hd / 32 * 34;
    return hd / 2;
}

void HipBackend::check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw rt_err(std::string("HIP launch failed in ") + what + ": " + hipGetErrorString(e));
}

// QuantActs::prepare (matmul.rs:34-71): quantize x (optionally RMS-normalized)
// once per activation format the given weights consume.
// ref_order: the norm sums in the reference's order (see launch_rmsnorm_quant).
void HipBackend::prepare(const float *x, const float *norm, int n, int K, const DevWeight *const *ws, int nw, bool want_f32,
                         bool ref_order) {
    bool need[3] = {want_f32, false, false};
    for (int i = 0; i < nw; i++)
        if (ws[i] && ws[i]->ty >= 0) need[act_format(ws[i]->ty)] = true;
    const float eps = m_.cfg.rms_eps;
    bool wrote_f32 = false;
    if (need[ACT_Q8_0]) {
        launch_rmsnorm_quant(x, K, norm, eps, n, K, need[ACT_F32] ? d_xn_ : nullptr, ACT_Q8_0, act0_, st_, ref_order);
        wrote_f32 = need[ACT_F32];
    }
    if (need[ACT_Q8K]) {
        launch_rmsnorm_quant(x, K, norm, eps, n, K, (need[ACT_F32] && !wrote_f32) ? d_xn_ : nullptr, ACT_Q8K, actk_, st_, ref_order);
        wrote_f32 = wrote_f32 || need[ACT_F32];
    }
    if (need[ACT_F32] && !wrote_f32) {
        if (norm) launch_rmsnorm(x, K, norm, eps, n, K, d_xn_, K, 0, st_, ref_order);
        else RIE_HIP_CHECK(hipMemcpyAsync(d_xn_, x, (size_t)n * K * 4, hipMemcpyDeviceToDevice, st_));
    }
    check_launch("prepare");
}

// matmul_multi (matmul.rs:136-176): decode-sized batches stream the weights
// through the GEMV kernels; prompt batches go to the int8 MFMA GEMM.
void HipBackend::matmul(const GemvSeg *segs, int nseg, int n, int K, const ActQ8 *act_q8_0) {
    // runs of segments that read the same activation batch share one launch
    int i = 0;
    while (i < nseg) {
        const int fmt = act_format(segs[i].w.ty);
        int j = i + 1;
        while (j < nseg && act_format(segs[j].w.ty) == fmt) j++;
        const ActQ8 &a = fmt == ACT_Q8K ? actk_ : (act_q8_0 ? *act_q8_0 : act0_);
        // prompt batches: one GEMM launch per run of segments of one weight type
        int s = i;
        while (n > 8 && s < j && gemm_supported(segs[s].w.ty, K)) {
            int e = s + 1;
            while (e < j && e - s < 3 && segs[e].w.ty == segs[s].w.ty) e++;
            if (!launch_gemm(&segs[s], e - s, a, n, K, st_, nullptr, d_gemm_ws_, gemm_ws_cap_)) break;
            s = e;
        }
        if (s < j && !launch_gemv(&segs[s], j - s, a, d_xn_, n, K, st_))
            throw Error{E_UNSUPPORTED, std::string("unsupported: matmul of type ") + type_name(segs[s].w.ty)};
        i = j;
    }
    check_launch("matmul");
}

void HipBackend::ffn_dense(const DevLayer &L, int n, float *out, int epi) {
    const ModelConfig &c = m_.cfg;
    const int E = (int)c.n_embd, ff = (int)L.ff;
    const DevWeight *ws[2] = {&L.gate, &L.up};
    // single token with Q4_0/Q8_0 or K-quant gate/up: the gate/up kernel normalizes x itself
    const bool self_norm = n == 1 && !capture_ && L.ffn_norm && L.gate.ty == L.up.ty && gemv_norm_ok(L.gate.ty, E);
    const NormIn nin{d_x_, L.ffn_norm, c.rms_eps};
    if (!self_norm) {
        prepare(d_x_, L.ffn_norm, n, E, ws, 2, false);
        mark("rmsnorm_quant");
    }
    const ActQ8 &a = act_format(L.gate.ty) == ACT_Q8K ? actk_ : act0_;
    bool done = false;
    if (n > 8 && gemm_supported(L.gate.ty, E)) done = launch_gemm_glu(L.gate, L.up, a, n, E, d_h_, ff, c.gelu, nullptr, st_);
    const int fmt = act_format(L.down.ty);
    // single-token Q8_0 down projection: the gate/up kernel quantizes h itself
    bool h_quantized = false;
    if (!done && n == 1 && fmt == ACT_Q8_0 && ff % 32 == 0)
        h_quantized = done = launch_gemv_glu(L.gate, L.up, a, d_xn_, n, E, d_h_, ff, c.gelu, &act_h_, st_, self_norm ? &nin : nullptr);
    if (!done && !launch_gemv_glu(L.gate, L.up, a, d_xn_, n, E, d_h_, ff, c.gelu, nullptr, st_, self_norm ? &nin : nullptr))
        throw Error{E_UNSUPPORTED, "unsupported: gated FFN weights"};
    check_launch("ffn glu");
    mark("matmul_gate_up_glu");
    GemvSeg s{L.down, out, E, epi};
    // (K-quant down weights keep the standalone quantizer: the quantize-only prologue
    // over the 8192-value hidden of the Llama-3.2-3B shape measured 670 against 690
    // tok/s, its 32 KB of x per workgroup on every workgroup's critical path)
    if (!h_quantized) {
        if (fmt == ACT_F32) RIE_HIP_CHECK(hipMemcpyAsync(d_xn_, d_h_, (size_t)n * ff * 4, hipMemcpyDeviceToDevice, st_));
        else launch_quant_only(d_h_, ff, n, ff, fmt, fmt == ACT_Q8K ? actk_ : act0_, st_);
        mark("quant");
    }
    matmul(&s, 1, n, ff, h_quantized ? &act_h_ : nullptr);
    mark("matmul_down");
}

void HipBackend::run_layers(int n, size_t pos0, const int *d_pos0, bool all_logits, int n_split) {
    const ModelConfig &c = m_.cfg;
    const int E = (int)c.n_embd, qd = (int)c.q_dim(), kvd = (int)c.kv_dim(), hd = (int)c.head_dim;
    launch_embed(d_tokens_, n, embd_, c.embd_scale, d_x_, st_);
    check_launch("embed");
    mark("embed");
    for (size_t il = 0; il < c.n_layer; il++) {
        const DevLayer &L = layers_[il];
        const bool swa = c.is_swa(il);
        cur_layer_ = il;
        // ---- attention block ----
        const DevWeight *ws[3] = {&L.wq, &L.wk, &L.wv};
        // single token with Q4_0/Q8_0 or K-quant Q/K/V of one activation format:
        // the GEMV normalizes and quantizes x itself
        const int qkv_fmt = act_format(L.wq.ty);
        // The first layer's input rows are the embedding rows, the same bits as the
        // reference's: its norm sums in the reference's order (a standalone launch), so
        // its activation codes are the reference's too.  Later layers' inputs already
        // carry f32 reduction-order differences, and their norms use wide sums.
        const bool first = il == 0;
        const bool self_norm = n == 1 && !capture_ && !first && L.attn_norm && gemv_norm_ok(L.wq.ty, E) &&
                               gemv_norm_ok(L.wk.ty, E) && gemv_norm_ok(L.wv.ty, E) && act_format(L.wk.ty) == qkv_fmt &&
                               act_format(L.wv.ty) == qkv_fmt;
        const NormIn nin{d_x_, L.attn_norm, c.rms_eps};
        if (!self_norm) {
            prepare(d_x_, L.attn_norm, n, E, ws, 3, false, first);
            mark("rmsnorm_quant");
        }
        GemvSeg qkv[3] = {{L.wq, d_q_, qd, EPI_STORE}, {L.wk, d_k_, kvd, EPI_STORE}, {L.wv, d_v_, kvd, EPI_STORE}};
        if (self_norm) {
            if (!launch_gemv(qkv, 3, qkv_fmt == ACT_Q8K ? actk_ : act0_, d_xn_, n, E, st_, &nin))
                throw rt_err("normalizing Q/K/V GEMV launch failed");
            check_launch("matmul");
        } else {
            matmul(qkv, 3, n, E);
        }
        mark("matmul_qkv");
        if (capture_ && !in_capture_) {
            RIE_HIP_CHECK(hipStreamSynchronize(st_));
        }
        HeadPrepArgs hp{};
        hp.q = d_q_;
        hp.k = d_k_;
        hp.v = d_v_;
        hp.bq = L.bq; hp.bk = L.bk; hp.bv = L.bv;
        hp.q_norm = L.q_norm; hp.k_norm = L.k_norm;
        hp.cos_t = (swa && d_cos_swa_) ? d_cos_swa_ : d_cos_;
        hp.sin_t = (swa && d_sin_swa_) ? d_sin_swa_ : d_sin_;
        hp.n_tok = n; hp.pos0 = (int)pos0; hp.n_head = (int)c.n_head; hp.n_kv = (int)c.n_head_kv; hp.hd = hd;
        hp.rope_dim = (int)c.rope_dim; hp.neox = c.rope_neox;
        hp.eps = c.rms_eps; hp.attn_scale = c.attn_scale;
        hp.kv_type = kv_type_;
        hp.k_cache = L.k_cache; hp.v_cache = L.v_cache; hp.k_scale = L.k_scale; hp.v_scale = L.v_scale;
        hp.slots = (int)L.slots;
        hp.d_pos0 = d_pos0;
        hp.turbo_signs = d_signs_;
        hp.k_out = (capture_ && !in_capture_) ? d_kcap_ : nullptr;
        if (capture_ && !in_capture_) {
            cap_[5].resize(c.n_layer);
            cap_[5][il].resize((size_t)n * kvd);
            RIE_HIP_CHECK(hipMemcpy(cap_[5][il].data(), d_v_, (size_t)n * kvd * 4, hipMemcpyDeviceToHost));
        }
        const int wo_fmt = act_format(L.wo.ty);
        AttnArgs aa{};
        aa.q = d_q_;
        aa.k_cache = L.k_cache; aa.v_cache = L.v_cache; aa.k_scale = L.k_scale; aa.v_scale = L.v_scale;
        aa.n_tok = n; aa.pos0 = (int)pos0; aa.n_head = (int)c.n_head; aa.n_kv = (int)c.n_head_kv; aa.hd = hd;
        aa.slots = (int)L.slots; aa.window = swa ? (int)c.swa_window : 0; aa.kv_type = kv_type_;
        aa.softcap = c.attn_softcap;
        aa.part = d_part_;
        aa.n_split = n_split;
        aa.att = d_att_;
        aa.att_fmt = wo_fmt == ACT_Q8_0 ? ACT_Q8_0 : -1;
        aa.att_q = act0_;
        aa.d_pos0 = d_pos0;
        aa.turbo_signs = d_signs_;
        aa.counters = d_attn_cnt_;
        // single token: prep, append, attention and range merge in one launch
        const bool fused_attn = n == 1 && attention_fused_ok(aa);
        // capture also runs the standalone prep before the fused launch, for its
        // query rows; that prep works on the query in place, so the raw rows are
        // put back for the fused kernel (which rewrites the same cache row, same bytes)
        if (!fused_attn || (capture_ && !in_capture_)) {
            std::vector<float> raw_q;
            if (fused_attn) {
                RIE_HIP_CHECK(hipStreamSynchronize(st_));
                raw_q.resize((size_t)n * qd);
                RIE_HIP_CHECK(hipMemcpy(raw_q.data(), d_q_, (size_t)n * qd * 4, hipMemcpyDeviceToHost));
            }
            launch_head_prep(hp, st_);
            check_launch("head_prep");
            mark("head_prep_kv_append");
            if (capture_ && !in_capture_) {  // the prepared query exists in memory only on this path
                RIE_HIP_CHECK(hipStreamSynchronize(st_));
                cap_[3].resize(c.n_layer);
                cap_[3][il].resize((size_t)n * qd);
                RIE_HIP_CHECK(hipMemcpy(cap_[3][il].data(), d_q_, (size_t)n * qd * 4, hipMemcpyDeviceToHost));
            }
            if (fused_attn) RIE_HIP_CHECK(hipMemcpy(d_q_, raw_q.data(), (size_t)n * qd * 4, hipMemcpyHostToDevice));
        }
        if (fused_attn) {
            if (!launch_attention_fused(aa, hp, st_)) throw rt_err("fused attention launch rejected");
        } else {
            launch_attention(aa, st_);
        }
        check_launch("attention");
        mark("attention");
        if (capture_ && !in_capture_) {
            RIE_HIP_CHECK(hipStreamSynchronize(st_));
            cap_[4].resize(c.n_layer);
            cap_[4][il].resize((size_t)n * kvd);
            RIE_HIP_CHECK(hipMemcpy(cap_[4][il].data(), d_kcap_, (size_t)n * kvd * 4, hipMemcpyDeviceToHost));
            cap_[2].resize(c.n_layer);
            cap_[2][il].resize((size_t)n * qd);
            RIE_HIP_CHECK(hipMemcpy(cap_[2][il].data(), d_att_, (size_t)n * qd * 4, hipMemcpyDeviceToHost));
        }
        // one token, K-quant wo: its GEMV quantizes the attention output itself (Q8_K prologue without a norm)
        const bool wo_self_q = n == 1 && !capture_ && wo_fmt == ACT_Q8K && gemv_quant_ok(L.wo.ty, qd);
        if (wo_fmt == ACT_Q8K && !wo_self_q) launch_quant_only(d_att_, qd, n, qd, ACT_Q8K, actk_, st_);
        if (wo_fmt == ACT_F32) RIE_HIP_CHECK(hipMemcpyAsync(d_xn_, d_att_, (size_t)n * qd * 4, hipMemcpyDeviceToDevice, st_));
        const bool direct = !L.post_attn_norm && c.residual_scale == 1.0f;
        GemvSeg so{L.wo, direct ? d_x_ : d_o_, E, direct ? EPI_ADD : EPI_STORE};
        if (wo_self_q) {
            const NormIn qin{d_att_, nullptr, 0.0f, 0};
            if (!launch_gemv(&so, 1, actk_, d_xn_, 1, qd, st_, &qin)) throw rt_err("quantizing wo GEMV launch failed");
            check_launch("matmul");
        } else {
            matmul(&so, 1, n, qd);
        }
        mark("matmul_wo");
        if (!direct) {
            if (L.post_attn_norm) launch_rmsnorm(d_o_, E, L.post_attn_norm, c.rms_eps, n, E, d_o_, E, 1, st_);
            launch_add_inplace(d_x_, d_o_, (size_t)n * E, c.residual_scale, st_);
        }
        if (capture_ && !in_capture_) {
            RIE_HIP_CHECK(hipStreamSynchronize(st_));
            cap_[0].resize(c.n_layer);
            cap_[0][il].resize((size_t)n * E);
            RIE_HIP_CHECK(hipMemcpy(cap_[0][il].data(), d_x_, (size_t)n * E * 4, hipMemcpyDeviceToHost));
        }
        // ---- feed-forward block ----
        const bool fdirect = !L.post_ffn_norm && c.residual_scale == 1.0f;
        if (L.moe) {
            if (!ffn_moe(L, n, fdirect)) {
                if (L.post_ffn_norm) launch_rmsnorm(d_o_, E, L.post_ffn_norm, c.rms_eps, n, E, d_o_, E, 1, st_);
                launch_add_inplace(d_x_, d_o_, (size_t)n * E, c.residual_scale, st_);
            }
        } else {
            ffn_dense(L, n, fdirect ? d_x_ : d_o_, fdirect ? EPI_ADD : EPI_STORE);
            if (capture_ && !in_capture_) {
                RIE_HIP_CHECK(hipStreamSynchronize(st_));
                cap_[6].resize(c.n_layer);
                cap_[6][il].resize((size_t)n * L.ff);
                RIE_HIP_CHECK(hipMemcpy(cap_[6][il].data(), d_h_, (size_t)n * L.ff * 4, hipMemcpyDeviceToHost));
            }
            if (!fdirect) {
                if (L.post_ffn_norm) launch_rmsnorm(d_o_, E, L.post_ffn_norm, c.rms_eps, n, E, d_o_, E, 1, st_);
                launch_add_inplace(d_x_, d_o_, (size_t)n * E, c.residual_scale, st_);
            }
        }
        check_launch("layer");
        if (capture_ && !in_capture_) {
            RIE_HIP_CHECK(hipStreamSynchronize(st_));
            cap_[1].resize(c.n_layer);
            cap_[1][il].resize((size_t)n * E);
            RIE_HIP_CHECK(hipMemcpy(cap_[1][il].data(), d_x_, (size_t)n * E * 4, hipMemcpyDeviceToHost));
        }
    }
    const int first = all_logits ? 0 : n - 1;
    head(first, n - first);
}

// output head (cpu.rs:388-407): final RMSNorm of the requested rows, logits
void HipBackend::head(int first, int m) {
    const ModelConfig &c = m_.cfg;
    const int E = (int)c.n_embd;
    const DevWeight *ws[1] = {&out_w_};
    const int fmt = act_format(out_w_.ty);
    const float *xr = d_x_ + (size_t)first * E;
    GemvSeg s{out_w_, d_logits_, (int)c.n_vocab, EPI_STORE};
    head_first_ = first;
    // one row, Q8_0/Q8_K head: the head GEMV normalizes and quantizes the row
    // itself; Backend::hidden then forms the normalized row on demand
    const NormIn nin{xr, out_norm_, c.rms_eps};
    head_normed_ = !(m == 1 && !capture_ && fmt != ACT_F32 && gemv_norm_ok(out_w_.ty, E) &&
                     launch_gemv(&s, 1, fmt == ACT_Q8K ? actk_ : act0_, d_xn_, 1, E, st_, &nin));
    if (head_normed_) {  // the normalized rows are kept in d_xn_ for Backend::hidden
        if (fmt == ACT_F32) {
            launch_rmsnorm(xr, E, out_norm_, c.rms_eps, m, E, d_xn_, E, 0, st_);
        } else {
            launch_rmsnorm_quant(xr, E, out_norm_, c.rms_eps, m, E, d_xn_, fmt, fmt == ACT_Q8K ? actk_ : act0_, st_);
        }
        mark("rmsnorm_quant");
        matmul(&s, 1, m, E);
    }
    (void)ws;
    mark("matmul_output");
    const size_t total = (size_t)m * c.n_vocab;
    if (c.logit_scale != 1.0f) launch_scale(d_logits_, total, c.logit_scale, st_);
    if (c.final_softcap > 0.0f) launch_softcap(d_logits_, total, c.final_softcap, st_);
    check_launch("head");
}

static DevWeight slice_rows(const DevWeight &w, size_t r0, size_t rows) {
    DevWeight s = w;
    s.data = w.data + r0 * w.rb();
    s.rows = rows;
    return s;
}

// y = down(act(gate·x) ⊙ up·x) for m rows of x (dense_ffn, cpu.rs:431-467); x is
// already normalized, so the activations are only quantized.
void HipBackend::expert_ffn(const DevWeight &g, const DevWeight &u, const DevWeight &dn, const float *x, int m, float *y) {
    const ModelConfig &c = m_.cfg;
    const int E = (int)c.n_embd, ff = (int)g.rows;
    const DevWeight *ws[2] = {&g, &u};
    prepare(x, nullptr, m, E, ws, 2, false);
    const ActQ8 &a = act_format(g.ty) == ACT_Q8K ? actk_ : act0_;
    bool done = false;
    if (m > 8 && gemm_supported(g.ty, E)) done = launch_gemm_glu(g, u, a, m, E, d_h_, ff, c.gelu, nullptr, st_);
    if (!done && !launch_gemv_glu(g, u, a, d_xn_, m, E, d_h_, ff, c.gelu, nullptr, st_))
        throw Error{E_UNSUPPORTED, "unsupported: expert FFN weights"};
    const int fmt = act_format(dn.ty);
    if (fmt == ACT_F32) RIE_HIP_CHECK(hipMemcpyAsync(d_xn_, d_h_, (size_t)m * ff * 4, hipMemcpyDeviceToDevice, st_));
    else launch_quant_only(d_h_, ff, m, ff, fmt, fmt == ACT_Q8K ? actk_ : act0_, st_);
    GemvSeg s{dn, y, E, EPI_STORE};
    matmul(&s, 1, m, ff);
}

// moe_ffn (cpu.rs:469-524): router logits → softmax/top-k (on the device) → the
// routed experts' outputs weighted and summed in ascending expert order into
// d_o_, plus the optionally gated shared expert.  One token: everything stays on
// the device (graph replay); prompt batches read the routing back and run each
// selected expert once over its gathered tokens.
// direct: the caller's residual add is a plain x += y (no post-norm, scale 1); a
// single token without a shared expert then combines straight into x, and the
// return value says so (x + y is what the add kernel computes at scale 1).
bool HipBackend::ffn_moe(const DevLayer &L, int n, bool direct) {
    const ModelConfig &c = m_.cfg;
    const int E = (int)c.n_embd, ne = (int)c.n_expert, k = (int)L.n_used, ff = (int)L.ff;
    const bool shared = L.sh_gate.data != nullptr;
    // One token without a shared expert: the router GEMV and the experts' gate/up
    // normalize x in their prologues (the same values as the standalone norm's
    // rows and codes), so neither the norm launch nor the row copy runs.
    const bool self_norm = n == 1 && !capture_ && !shared && L.ffn_norm && L.gate.ty == L.up.ty &&
                           (gemv_norm_f32_ok(L.router.ty, E) || gemv_norm_ok(L.router.ty, E)) && gemv_norm_ok(L.gate.ty, E);
    // the router's f32 rows follow the kernel prepare() would have made them with
    const NormIn nin{d_x_, L.ffn_norm, c.rms_eps, act_format(L.gate.ty) == ACT_Q8_0 ? 1 : 0};
    if (!self_norm) {
        const DevWeight *ws[4] = {&L.router, &L.gate, &L.up, shared ? &L.sh_gate : nullptr};
        prepare(d_x_, L.ffn_norm, n, E, ws, 4, true);  // f32 rows for the router, gathers and the shared gate
    }
    mark("rmsnorm_quant");
    GemvSeg rs{L.router, d_router_, ne, EPI_STORE};
    // one token, F32 router: its last workgroup also routes the token (no routing launch)
    RouteEpi re;
    re.cnt = d_route_cnt_;
    re.n_exp = ne;
    re.k = k;
    re.norm_topk = L.norm_topk;
    re.unit_weights = L.unit_weights;
    re.sel = d_moe_sel_;
    re.wgt = d_moe_w_;
    const bool routed = n == 1 && !capture_ &&
                        launch_gemv_route(rs, act_format(L.router.ty) == ACT_Q8K ? actk_ : act0_, d_xn_, E, self_norm ? &nin : nullptr, re, st_);
    if (routed) {
        check_launch("router");
    } else if (self_norm) {
        if (!launch_gemv(&rs, 1, act_format(L.router.ty) == ACT_Q8K ? actk_ : act0_, d_xn_, 1, E, st_, &nin))
            throw rt_err("normalizing router GEMV launch failed");
    } else {
        matmul(&rs, 1, n, E);
    }
    if (capture_ && !in_capture_) {  // router logits before the softmax
        RIE_HIP_CHECK(hipStreamSynchronize(st_));
        cap_[7].resize(c.n_layer);
        cap_[7][cur_layer_].resize((size_t)n * ne);
        RIE_HIP_CHECK(hipMemcpy(cap_[7][cur_layer_].data(), d_router_, (size_t)n * ne * 4, hipMemcpyDeviceToHost));
    }
    if (!routed) launch_moe_route(d_router_, n, ne, k, L.norm_topk, L.unit_weights, d_moe_sel_, d_moe_w_, st_);
    check_launch("moe route");
    if (capture_ && !in_capture_) {  // the routing the device applied: selected experts (int bits) and weights
        RIE_HIP_CHECK(hipStreamSynchronize(st_));
        for (int w = 8; w < 10; w++) {
            cap_[w].resize(c.n_layer);
            cap_[w][cur_layer_].resize((size_t)n * k);
        }
        RIE_HIP_CHECK(hipMemcpy(cap_[8][cur_layer_].data(), d_moe_sel_, (size_t)n * k * 4, hipMemcpyDeviceToHost));
        RIE_HIP_CHECK(hipMemcpy(cap_[9][cur_layer_].data(), d_moe_w_, (size_t)n * k * 4, hipMemcpyDeviceToHost));
    }
    mark("moe_route");
    if (!self_norm) RIE_HIP_CHECK(hipMemcpyAsync(d_moe_xn_, d_xn_, (size_t)n * E * 4, hipMemcpyDeviceToDevice, st_));
    if (n == 1) {
        const ActQ8 &ax = act_format(L.gate.ty) == ACT_Q8K ? actk_ : act0_;
        const int dfmt = act_format(L.down.ty);
        const NormIn *gn = self_norm ? &nin : nullptr;
        bool hq = dfmt == ACT_Q8_0 && ff % 32 == 0 &&
                  launch_gemv_glu_experts(L.gate, L.up, ff, d_moe_sel_, k, ax, d_xn_, E, d_h_, c.gelu, &act_h_, st_, gn);
        if (!hq && !launch_gemv_glu_experts(L.gate, L.up, ff, d_moe_sel_, k, ax, d_xn_, E, d_h_, c.gelu, nullptr, st_, gn))
            throw Error{E_UNSUPPORTED, "unsupported: routed expert weights"};
        mark("moe_gate_up_glu");
        // Q8_K down weights: the down GEMV quantizes its expert's hidden row in its
        // prologue (the standalone quantizer's codes) instead of a quantizer launch;
        // capture mode keeps the launch (a bitwise check of this form)
        const bool hpro = !hq && !capture_ && dfmt == ACT_Q8K && gemv_quant_ok(L.down.ty, ff);
        if (!hq && dfmt != ACT_F32 && !hpro) launch_quant_only(d_h_, ff, k, ff, dfmt, dfmt == ACT_Q8K ? actk_ : act0_, st_);
        const ActQ8 &ah = hq ? act_h_ : (dfmt == ACT_Q8K ? actk_ : act0_);
        const NormIn hn{d_h_, nullptr, 0.0f, 0};
        if (!launch_gemv_experts(L.down, E, d_moe_sel_, k, ah, d_h_, true, ff, d_moe_y_, st_, hpro ? &hn : nullptr))
            throw Error{E_UNSUPPORTED, "unsupported: routed expert down weights"};
        mark("moe_down");
        if (direct && !shared && !capture_) {  // capture keeps the two-step form (a bitwise check of this one)
            launch_moe_combine(d_moe_y_, d_moe_w_, 1, k, E, d_x_, EPI_ADD, st_);
            check_launch("moe");
            mark("moe_combine");
            return true;
        }
        launch_moe_combine(d_moe_y_, d_moe_w_, 1, k, E, d_o_, EPI_STORE, st_);
    } else if (moe_grouped_ok(L)) {
        // Prompt batch, on the device: the routed pairs grouped by expert, one grouped
        // GEMM launch for every expert's gate/up (activation rows gathered through the
        // token map, hidden rows in gathered order), the hidden's quantization, one for
        // every expert's down projection (rows scattered to their pair slots), and the
        // per-token combine in ascending expert order (cpu.rs:487-513).
        // Q4_K experts: 32-token tiles (128 rows × 32 tokens per workgroup), since a
        // prompt's experts hold a few dozen rows each; other types: GROUP_BN
        const int bn = L.gate.ty == T_Q4_K && L.down.ty == T_Q4_K ? 32 : GROUP_BN;
        launch_moe_group(d_moe_sel_, n, k, ne, d_moe_off_, d_moe_rtok_, d_moe_rslot_, d_moe_tile_e_, d_moe_tile_r0_, d_moe_ntiles_, bn, st_);
        check_launch("moe group");
        GroupTiles g;
        g.bn = bn;
        g.tile_e = d_moe_tile_e_;
        g.tile_r0 = d_moe_tile_r0_;
        g.n_tiles = d_moe_ntiles_;
        g.off = d_moe_off_;
        g.amap = d_moe_rtok_;
        g.max_tiles = moe_group_max_tiles(n, k, ne, bn);
        DevWeight ge = L.gate, ue = L.up, de = L.down;  // expert 0's matrices; the others follow at wstride
        ge.rows = ue.rows = (size_t)ff;
        de.rows = (size_t)E;
        g.wstride = (size_t)ff * L.gate.rb();
        const ActQ8 &ax = act_format(L.gate.ty) == ACT_Q8K ? actk_ : act0_;
        if (!launch_gemm_glu(ge, ue, ax, n * k, E, d_h_, ff, c.gelu, nullptr, st_, &g)) throw rt_err("grouped expert gate/up launch rejected");
        check_launch("moe gate/up");
        mark("moe_gate_up_glu");
        const int dfmt = act_format(L.down.ty);
        const ActQ8 &ah = dfmt == ACT_Q8K ? actk_ : act0_;
        launch_quant_only(d_h_, ff, n * k, ff, dfmt, ah, st_);
        GroupTiles g2 = g;
        g2.amap = nullptr;
        g2.omap = d_moe_rslot_;
        g2.wstride = (size_t)E * L.down.rb();
        GemvSeg sd{de, d_moe_y_, E, EPI_STORE};
        if (!launch_gemm(&sd, 1, ah, n * k, ff, st_, &g2)) throw rt_err("grouped expert down launch rejected");
        check_launch("moe down");
        mark("moe_down");
        if (direct && !shared && !capture_) {
            launch_moe_combine(d_moe_y_, d_moe_w_, n, k, E, d_x_, EPI_ADD, st_);
            check_launch("moe");
            mark("moe_combine");
            return true;
        }
        launch_moe_combine(d_moe_y_, d_moe_w_, n, k, E, d_o_, EPI_STORE, st_);
    } else {
        std::vector<int> sel((size_t)n * k);
        std::vector<float> w((size_t)n * k);
        RIE_HIP_CHECK(hipMemcpyAsync(sel.data(), d_moe_sel_, sel.size() * 4, hipMemcpyDeviceToHost, st_));
        RIE_HIP_CHECK(hipMemcpyAsync(w.data(), d_moe_w_, w.size() * 4, hipMemcpyDeviceToHost, st_));
        RIE_HIP_CHECK(hipStreamSynchronize(st_));
        // tokens of each expert, experts in ascending order (cpu.rs:489-501)
        std::vector<std::vector<std::pair<int, float>>> assign(ne);
        for (int t = 0; t < n; t++)
            for (int j = 0; j < k; j++) {
                const int ex = sel[(size_t)t * k + j];
                if (ex < 0 || ex >= ne) throw rt_err("expert routing produced an invalid expert id");
                assign[ex].emplace_back(t, w[(size_t)t * k + j]);
            }
        std::vector<int> rows;
        std::vector<float> rw;
        std::vector<int> off(ne + 1, 0);
        for (int ex = 0; ex < ne; ex++) {
            off[ex] = (int)rows.size();
            for (auto &tw : assign[ex]) {
                rows.push_back(tw.first);
                rw.push_back(tw.second);
            }
        }
        off[ne] = (int)rows.size();
        RIE_HIP_CHECK(hipMemcpyAsync(d_moe_rows_, rows.data(), rows.size() * 4, hipMemcpyHostToDevice, st_));
        RIE_HIP_CHECK(hipMemcpyAsync(d_moe_rw_, rw.data(), rw.size() * 4, hipMemcpyHostToDevice, st_));
        RIE_HIP_CHECK(hipMemsetAsync(d_o_, 0, (size_t)n * E * 4, st_));
        for (int ex = 0; ex < ne; ex++) {
            const int m = off[ex + 1] - off[ex];
            if (!m) continue;
            launch_moe_gather(d_moe_xn_, d_moe_rows_ + off[ex], m, E, d_moe_xg_, st_);
            expert_ffn(slice_rows(L.gate, (size_t)ex * ff, ff), slice_rows(L.up, (size_t)ex * ff, ff),
                       slice_rows(L.down, (size_t)ex * E, E), d_moe_xg_, m, d_moe_yg_);
            launch_moe_scatter_add(d_moe_yg_, d_moe_rows_ + off[ex], d_moe_rw_ + off[ex], m, E, d_o_, st_);
        }
        RIE_HIP_CHECK(hipStreamSynchronize(st_));  // the host vectors above are read by the async copies
    }
    if (shared) {
        expert_ffn(L.sh_gate, L.sh_up, L.sh_down, d_moe_xn_, n, d_moe_yg_);
        launch_moe_shared_add(d_moe_yg_, L.sh_gate_inp, d_moe_xn_, n, E, d_o_, st_);
    }
    check_launch("moe");
    mark("moe_combine");
    return false;
}

// The device-grouped prompt path needs the int8 MFMA GEMMs for the experts' matrices:
// a gated pair (Q4_0, Q8_0 or Q4_K) and a down projection with a GEMM.
bool HipBackend::moe_grouped_ok(const DevLayer &L) const {
    const size_t E = m_.cfg.n_embd, ff = L.ff;
    const int gt = L.gate.ty;
    return L.gate.ty == L.up.ty && (gt == T_Q4_0 || gt == T_Q8_0 || gt == T_Q4_K) && gemm_supported(gt, E) &&
           gemm_supported(L.down.ty, ff) && d_moe_off_ != nullptr;
}

void HipBackend::forward(const uint32_t *tokens, size_t n, size_t pos, bool all_logits, float *logits, size_t logits_len) {
    const ModelConfig &c = m_.cfg;
    hidden_rows_ = 0;
    if (n == 0) throw rt_err("empty batch");
    if (n > max_batch_) throw rt_err("batch of " + std::to_string(n) + " tokens exceeds max batch " + std::to_string(max_batch_));
    if (pos + n > n_ctx_) throw rt_err("context window full (" + std::to_string(n_ctx_) + " tokens)");
    for (size_t t = 0; t < n; t++)
        if (tokens[t] >= m_.token_embd.rows) throw rt_err("token id " + std::to_string(tokens[t]) + " out of range");
    const size_t m = all_logits ? n : 1;
    if (logits_len < m * c.n_vocab) throw rt_err("logits buffer too small");
    RIE_HIP_CHECK(hipSetDevice(device_));
    RIE_HIP_CHECK(hipMemcpyAsync(d_tokens_, tokens, n * 4, hipMemcpyHostToDevice, st_));
    if (n == 1 && use_graph_ && !capture_) {
        decode_step_graph(pos);
    } else {
        run_layers((int)n, pos, nullptr, all_logits, splits_for(n, pos));
    }
    RIE_HIP_CHECK(hipMemcpyAsync(logits, d_logits_, m * c.n_vocab * 4, hipMemcpyDeviceToHost, st_));
    RIE_HIP_CHECK(hipStreamSynchronize(st_));
    hidden_rows_ = m;
}

// The decode step as a graph: kernels read pos from d_pos_ and the token from
// d_tokens_[0].  One graph per attention range count (it grows with the context).
void HipBackend::decode_step_graph(size_t pos) {
    // the position travels as a kernel argument (copied at launch), so queued
    // steps never share a host-side slot
    launch_set_int(d_pos_, (int)pos, st_);
    check_launch("set pos");
    const int ns = splits_for(1, pos);
    auto it = graphs_.find(ns);
    if (it == graphs_.end()) {
        DecodeGraph dg;
        in_capture_ = true;
        RIE_HIP_CHECK(hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal));
        try {
            run_layers(1, 0, d_pos_, false, ns);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(st_, &g);
            if (g) (void)hipGraphDestroy(g);
            in_capture_ = false;
            throw;
        }
        RIE_HIP_CHECK(hipStreamEndCapture(st_, &dg.graph));
        in_capture_ = false;
        dg.head_normed = head_normed_;
        dg.head_first = head_first_;
        RIE_HIP_CHECK(hipGraphInstantiate(&dg.exec, dg.graph, nullptr, nullptr, 0));
        it = graphs_.emplace(ns, dg).first;
    }
    RIE_HIP_CHECK(hipGraphLaunch(it->second.exec, st_));
    head_normed_ = it->second.head_normed;
    head_first_ = it->second.head_first;
}

// One greedy step as a graph (per attention range count): run_layers at the
// device-resident position d_pos_[0], then the advancing argmax.
void HipBackend::greedy_step_graph(size_t pos) {
    const int ns = splits_for(1, pos);
    auto it = greedy_graphs_.find(ns);
    if (it == greedy_graphs_.end()) {
        DecodeGraph dg;
        in_capture_ = true;
        RIE_HIP_CHECK(hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal));
        try {
            run_layers(1, 0, d_pos_, false, ns);
            launch_argmax_step(d_logits_, (int)m_.cfg.n_vocab, d_amax_idx_, d_amax_val_, n_amax_part_, d_tokens_, d_gen_, d_pos_,
                               (int)std::max<size_t>(n_ctx_, 1), st_, d_amax_cnt_);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(st_, &g);
            if (g) (void)hipGraphDestroy(g);
            in_capture_ = false;
            throw;
        }
        RIE_HIP_CHECK(hipStreamEndCapture(st_, &dg.graph));
        in_capture_ = false;
        dg.head_normed = head_normed_;
        dg.head_first = head_first_;
        RIE_HIP_CHECK(hipGraphInstantiate(&dg.exec, dg.graph, nullptr, nullptr, 0));
        it = greedy_graphs_.emplace(ns, dg).first;
    }
    RIE_HIP_CHECK(hipGraphLaunch(it->second.exec, st_));
    head_normed_ = it->second.head_normed;
    head_first_ = it->second.head_first;
}

int HipBackend::splits_for(size_t n, size_t pos) const {
    const ModelConfig &c = m_.cfg;
    AttnArgs probe{};  // the shape fields attention_fused_ok looks at
    probe.n_tok = (int)n;
    probe.n_head = (int)c.n_head;
    probe.n_kv = (int)c.n_head_kv;
    probe.hd = (int)c.head_dim;
    probe.counters = d_attn_cnt_;
    probe.n_split = 1;
    return attention_splits((int)n, (int)c.n_head_kv, (int)(pos + n), (int)c.head_dim,
                            attention_fused_ok(probe) && !attn_ranges_only_);
}

const float *HipBackend::hidden(size_t *rows) {
    *rows = hidden_rows_;
    if (!hidden_rows_) return nullptr;
    if (!head_normed_) {  // the head normalized its row in its prologue: form it here (the same kernel as the head's rows)
        const ModelConfig &c = m_.cfg;
        const int E = (int)c.n_embd, fmt = act_format(out_w_.ty);
        RIE_HIP_CHECK(hipSetDevice(device_));
        launch_rmsnorm_quant(d_x_ + (size_t)head_first_ * E, E, out_norm_, c.rms_eps, (int)hidden_rows_, E, d_xn_, fmt,
                             fmt == ACT_Q8K ? actk_ : act0_, st_);
        check_launch("hidden rows");
        head_normed_ = true;
    }
    hidden_host_.resize(hidden_rows_ * m_.cfg.n_embd);
    RIE_HIP_CHECK(hipMemcpyAsync(hidden_host_.data(), d_xn_, hidden_host_.size() * 4, hipMemcpyDeviceToHost, st_));
    RIE_HIP_CHECK(hipStreamSynchronize(st_));
    return hidden_host_.data();
}

uint32_t HipBackend::forward_argmax(const uint32_t *tokens, size_t n, size_t pos) {
    const ModelConfig &c = m_.cfg;
    hidden_rows_ = 0;
    if (n == 0) throw rt_err("empty batch");
    if (n > max_batch_) throw rt_err("batch of " + std::to_string(n) + " tokens exceeds max batch " + std::to_string(max_batch_));
    if (pos + n > n_ctx_) throw rt_err("context window full (" + std::to_string(n_ctx_) + " tokens)");
    for (size_t t = 0; t < n; t++)
        if (tokens[t] >= m_.token_embd.rows) throw rt_err("token id " + std::to_string(tokens[t]) + " out of range");
    RIE_HIP_CHECK(hipSetDevice(device_));
    RIE_HIP_CHECK(hipMemcpyAsync(d_tokens_, tokens, n * 4, hipMemcpyHostToDevice, st_));
    if (n == 1 && use_graph_ && !capture_) {
        decode_step_graph(pos);
    } else {
        run_layers((int)n, pos, nullptr, false, splits_for(n, pos));
    }
    launch_argmax(d_logits_, (int)c.n_vocab, d_amax_idx_, d_amax_val_, n_amax_part_, d_tokens_, st_, d_amax_cnt_);
    check_launch("argmax");
    uint32_t tok = 0;
    RIE_HIP_CHECK(hipMemcpyAsync(&tok, d_tokens_, 4, hipMemcpyDeviceToHost, st_));
    RIE_HIP_CHECK(hipStreamSynchronize(st_));
    hidden_rows_ = 1;
    return tok;
}

// greedy steps without host round trips: each step's argmax is written to
// d_tokens_[0] (the next step's input) and appended to d_gen_.
void HipBackend::generate_greedy(size_t pos, size_t n_gen, uint32_t *out) {
    if (pos + n_gen > n_ctx_) throw rt_err("context window full (" + std::to_string(n_ctx_) + " tokens)");
    if (n_gen == 0) return;
    const ModelConfig &c = m_.cfg;
    RIE_HIP_CHECK(hipSetDevice(device_));
    if (use_graph_ && !capture_) {
        // every step one graph launch: the layers, the head and the argmax, which
        // records the token, feeds it to the next step and advances the position
        RIE_HIP_CHECK(hipMemcpyAsync(d_gen_, d_tokens_, 4, hipMemcpyDeviceToDevice, st_));
        launch_set_int(d_pos_, (int)pos, st_);
        launch_set_int(d_pos_ + 1, 0, st_);
        check_launch("greedy setup");
        for (size_t i = 0; i < n_gen; i++) greedy_step_graph(pos + i);
        RIE_HIP_CHECK(hipMemcpyAsync(out, d_gen_, n_gen * 4, hipMemcpyDeviceToHost, st_));
        RIE_HIP_CHECK(hipStreamSynchronize(st_));
        hidden_rows_ = 1;
        return;
    }
    for (size_t i = 0; i < n_gen; i++) {
        RIE_HIP_CHECK(hipMemcpyAsync(d_gen_ + i, d_tokens_, 4, hipMemcpyDeviceToDevice, st_));
        if (use_graph_ && !capture_) {
            decode_step_graph(pos + i);
        } else {
            run_layers(1, pos + i, nullptr, false, splits_for(1, pos + i));
        }
        launch_argmax(d_logits_, (int)c.n_vocab, d_amax_idx_, d_amax_val_, n_amax_part_, d_tokens_, st_, d_amax_cnt_);
        check_launch("argmax");
    }
    RIE_HIP_CHECK(hipMemcpyAsync(out, d_gen_, n_gen * 4, hipMemcpyDeviceToHost, st_));
    RIE_HIP_CHECK(hipStreamSynchronize(st_));
    hidden_rows_ = 1;
}

void HipBackend::synchronize() { RIE_HIP_CHECK(hipStreamSynchronize(st_)); }

void HipBackend::set_capture(bool on) {
    capture_ = on;
    for (auto &v : cap_) v.clear();
}

bool HipBackend::capture(size_t layer, int what, float *out, size_t len) {
    if (what < 0 || what >= (int)cap_.size() || layer >= cap_[what].size()) return false;
    const auto &v = cap_[what][layer];
    if (v.empty() || len < v.size()) return false;
    std::memcpy(out, v.data(), v.size() * 4);
    return true;
}

void HipBackend::kv_layer(size_t layer, int which, uint8_t *out, size_t len, uint8_t *scales_out, size_t scales_len) {
    if (layer >= layers_.size()) throw rt_err("layer out of range");
    const DevLayer &D = layers_[layer];
    const size_t bytes = m_.cfg.n_head_kv * D.slots * kv_row_bytes();
    if (len < bytes) throw rt_err("buffer too small");
    RIE_HIP_CHECK(hipStreamSynchronize(st_));
    RIE_HIP_CHECK(hipMemcpy(out, which ? D.v_cache : D.k_cache, bytes, hipMemcpyDeviceToHost));
    if (kv_type_ == 2 && scales_out) {
        const size_t sb = m_.cfg.n_head_kv * D.slots * 2 * turbo_blocks();
        if (scales_len < sb) throw rt_err("buffer too small");
        RIE_HIP_CHECK(hipMemcpy(scales_out, which ? D.v_scale : D.k_scale, sb, hipMemcpyDeviceToHost));
    }
}

void HipBackend::mark(const char *name) {
    if (!profiling_) return;
    hipEvent_t e;
    RIE_HIP_CHECK(hipEventCreate(&e));
    RIE_HIP_CHECK(hipEventRecord(e, st_));
    marks_.emplace_back(name, e);
}

double HipBackend::time_ffn_glu(int reps, size_t *bytes) {
    const ModelConfig &c = m_.cfg;
    const int E = (int)c.n_embd;
    if (reps < 1) throw rt_err("reps must be positive");
    for (const auto &L : layers_)
        if (L.moe) throw Error{E_UNSUPPORTED, "unsupported: gate/up timing of a MoE layer"};
    RIE_HIP_CHECK(hipSetDevice(device_));
    const DevLayer &L0 = layers_[0];
    const DevWeight *ws[2] = {&L0.gate, &L0.up};
    prepare(d_x_, L0.ffn_norm, 1, E, ws, 2, false);
    const int fmt_in = act_format(L0.gate.ty);
    const ActQ8 &a = fmt_in == ACT_Q8K ? actk_ : act0_;
    auto one_pass = [&](size_t *b) {
        for (const auto &L : layers_) {
            const int ff = (int)L.ff;
            // the same launch as a decode step (ffn_dense)
            const bool self_norm = L.ffn_norm && L.gate.ty == L.up.ty && gemv_norm_ok(L.gate.ty, E);
            const NormIn nin{d_x_, L.ffn_norm, c.rms_eps};
            const bool hq = act_format(L.down.ty) == ACT_Q8_0 && ff % 32 == 0;
            bool done = hq && launch_gemv_glu(L.gate, L.up, a, d_xn_, 1, E, d_h_, ff, c.gelu, &act_h_, st_, self_norm ? &nin : nullptr);
            if (!done && !launch_gemv_glu(L.gate, L.up, a, d_xn_, 1, E, d_h_, ff, c.gelu, nullptr, st_, self_norm ? &nin : nullptr))
                throw Error{E_UNSUPPORTED, "unsupported: gated FFN weights"};
            if (b && !*b) {  // weights + activation read + hidden (and its Q8_0) written
                size_t in = self_norm ? (size_t)E * 8  // residual row and norm weight, f32
                            : fmt_in == ACT_F32 ? (size_t)E * 4
                            : fmt_in == ACT_Q8_0 ? (size_t)E + (size_t)E / 32 * (L.gate.ty == T_Q4_0 ? 8 : 4)
                                                 : (size_t)E + (size_t)E / 256 * 4 + (size_t)E / 16 * 2;
                *b = L.gate.rows * L.gate.rb() + L.up.rows * L.up.rb() + in + (size_t)ff * 4 + (done ? (size_t)ff + (size_t)ff / 32 * 12 : 0);
            }
        }
    };
    size_t b = 0;
    one_pass(&b);  // warm-up
    check_launch("ffn glu timing");
    hipEvent_t e0, e1;
    RIE_HIP_CHECK(hipEventCreate(&e0));
    RIE_HIP_CHECK(hipEventCreate(&e1));
    RIE_HIP_CHECK(hipEventRecord(e0, st_));
    for (int r = 0; r < reps; r++) one_pass(nullptr);
    RIE_HIP_CHECK(hipEventRecord(e1, st_));
    RIE_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0;
    RIE_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *bytes = b;
    return (double)ms * 1e3 / ((double)reps * layers_.size());
}

// One eager decode step per repetition at position pos, with an event after
// every launch on the backend's stream; returns per-kernel-family totals.
std::vector<HipBackend::KernelTime> HipBackend::profile_decode(size_t pos, int reps) {
    if (pos + 1 > n_ctx_) throw rt_err("context window full");
    std::vector<KernelTime> out;
    RIE_HIP_CHECK(hipSetDevice(device_));
    for (int r = 0; r < reps; r++) {
        profiling_ = true;
        marks_.clear();
        RIE_HIP_CHECK(hipEventCreate(&mark0_));
        RIE_HIP_CHECK(hipEventRecord(mark0_, st_));
        try {
            run_layers(1, pos, nullptr, false, splits_for(1, pos));
        } catch (...) {
            profiling_ = false;
            throw;
        }
        profiling_ = false;
        RIE_HIP_CHECK(hipStreamSynchronize(st_));
        hipEvent_t prev = mark0_;
        for (auto &m : marks_) {
            float ms = 0;
            RIE_HIP_CHECK(hipEventElapsedTime(&ms, prev, m.second));
            auto it = std::find_if(out.begin(), out.end(), [&](const KernelTime &k) { return k.name == m.first; });
            if (it == out.end()) {
                out.push_back(KernelTime{m.first, 0, 0});
                it = out.end() - 1;
            }
            it->ms += ms;
            it->launches += 1;
            prev = m.second;
        }
        (void)hipEventDestroy(mark0_);
        for (auto &m : marks_) (void)hipEventDestroy(m.second);
        marks_.clear();
    }
    return out;
}

}  // namespace rie
