// capi.cpp — the extern "C" boundary (include/rie_hip.h).  Every entry point
// catches C++ exceptions and turns them into an error code plus message, like
// the reference's FFI does with catch_unwind (crates/rie-ffi/src/lib.rs:146).
#include "../../../include/rie_hip.h"

#include "../kernels.hpp"
#include "backend.hpp"
#include "synth.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <vector>

using rie::Error;
using rie::HipBackend;

struct rie_hip_backend {
    HipBackend *b;
};

static void write_err(char *err, size_t len, const std::string &m) {
    if (!err || !len) return;
    size_t n = std::min(len - 1, m.size());
    std::memcpy(err, m.data(), n);
    err[n] = 0;
}

template <class F>
static int32_t guarded(char *err, size_t err_len, F &&f) {
    try {
        f();
        return RIE_HIP_OK;
    } catch (const Error &e) {
        write_err(err, err_len, e.msg);
        return e.code;
    } catch (const std::exception &e) {
        write_err(err, err_len, std::string("internal error: ") + e.what());
        return RIE_HIP_ERR_RUNTIME;
    } catch (...) {
        write_err(err, err_len, "internal error");
        return RIE_HIP_ERR_RUNTIME;
    }
}

extern "C" {

rie_hip_config rie_hip_default_config(void) {
    rie_hip_config c;
    c.n_ctx = 4096;
    c.max_batch = 64;
    c.kv_type = RIE_HIP_KV_F16;
    c.device = 0;
    c.use_graph = 1;
    return c;
}

rie_hip_backend *rie_hip_create(const uint8_t *gguf, size_t gguf_len, const rie_hip_config *cfg, int32_t *err_code, char *err,
                                size_t err_len) {
    rie_hip_backend *h = nullptr;
    int32_t rc = guarded(err, err_len, [&] {
        if (!gguf) throw Error{rie::E_IO, "null GGUF image"};
        rie_hip_config c = cfg ? *cfg : rie_hip_default_config();
        rie::BackendConfig bc;
        bc.n_ctx = (size_t)std::max(c.n_ctx, 1);
        bc.max_batch = (size_t)std::max(c.max_batch, 1);
        bc.kv_type = c.kv_type;
        bc.device = c.device;
        bc.use_graph = c.use_graph != 0;
        h = new rie_hip_backend{new HipBackend(gguf, gguf_len, bc)};
    });
    if (err_code) *err_code = rc;
    return rc == RIE_HIP_OK ? h : nullptr;
}

void rie_hip_destroy(rie_hip_backend *b) {
    if (!b) return;
    try {
        delete b->b;
    } catch (...) {
    }
    delete b;
}

size_t rie_hip_name(const rie_hip_backend *b, char *buf, size_t buf_len) {
    const std::string &n = b->b->name();
    write_err(buf, buf_len, n);
    return n.size();
}

size_t rie_hip_max_batch(const rie_hip_backend *b) { return b->b->max_batch(); }
size_t rie_hip_n_ctx(const rie_hip_backend *b) { return b->b->n_ctx(); }
size_t rie_hip_n_vocab(const rie_hip_backend *b) { return b->b->config().n_vocab; }
size_t rie_hip_n_embd(const rie_hip_backend *b) { return b->b->config().n_embd; }
int32_t rie_hip_kv_type(const rie_hip_backend *b) { return b->b->kv_type(); }
size_t rie_hip_kv_bytes(const rie_hip_backend *b) { return b->b->kv_bytes(); }
size_t rie_hip_weight_bytes(const rie_hip_backend *b) { return b->b->weight_bytes(); }
size_t rie_hip_kv_row_bytes(const rie_hip_backend *b) { return b->b->kv_row_bytes(); }

int32_t rie_hip_forward(rie_hip_backend *b, const uint32_t *tokens, size_t n, size_t pos, int32_t all_logits, float *logits,
                        size_t logits_len, char *err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!logits && logits_len) throw Error{rie::E_RUNTIME, "null logits buffer"};
        if (n && !tokens) throw Error{rie::E_RUNTIME, "null tokens"};
        b->b->forward(tokens, n, pos, all_logits != 0, logits, logits_len);
    });
}

const float *rie_hip_hidden(rie_hip_backend *b, size_t *rows) {
    size_t r = 0;
    const float *p = nullptr;
    try {
        p = b->b->hidden(&r);
    } catch (...) {
        p = nullptr;
        r = 0;
    }
    if (rows) *rows = r;
    return p;
}

int32_t rie_hip_forward_argmax(rie_hip_backend *b, const uint32_t *tokens, size_t n, size_t pos, uint32_t *next, char *err,
                               size_t err_len) {
    return guarded(err, err_len, [&] {
        if (n && !tokens) throw Error{rie::E_RUNTIME, "null tokens"};
        uint32_t t = b->b->forward_argmax(tokens, n, pos);
        if (next) *next = t;
    });
}

int32_t rie_hip_generate_greedy(rie_hip_backend *b, size_t pos, size_t n_gen, uint32_t *out, char *err, size_t err_len) {
    return guarded(err, err_len, [&] { b->b->generate_greedy(pos, n_gen, out); });
}

int32_t rie_hip_bench(rie_hip_backend *b, size_t n_prompt, size_t n_gen, double *pp_tps, double *tg_tps, char *err, size_t err_len) {
    return guarded(err, err_len, [&] {
        HipBackend &be = *b->b;
        const uint32_t nv = (uint32_t)be.config().n_vocab;
        if (n_prompt < 1) n_prompt = 1;
        std::vector<uint32_t> toks(n_prompt);
        for (size_t i = 0; i < n_prompt; i++) toks[i] = ((uint32_t)i * 7919u + 13u) % nv;
        const size_t nb = be.max_batch();
        auto eval = [&](size_t count) -> uint32_t {
            uint32_t next = 0;
            for (size_t pos = 0; pos < count; pos += nb) {
                const size_t end = std::min(pos + nb, count);
                next = be.forward_argmax(toks.data() + pos, end - pos, pos);
            }
            return next;
        };
        eval(std::min<size_t>(n_prompt, 8));  // warm-up
        be.synchronize();
        auto t0 = std::chrono::steady_clock::now();
        eval(n_prompt);
        be.synchronize();
        auto t1 = std::chrono::steady_clock::now();
        std::vector<uint32_t> gen(std::max<size_t>(n_gen, 1));
        if (n_gen) be.generate_greedy(n_prompt, n_gen, gen.data());
        be.synchronize();
        auto t2 = std::chrono::steady_clock::now();
        const double pp = std::chrono::duration<double>(t1 - t0).count();
        const double tg = std::chrono::duration<double>(t2 - t1).count();
        if (pp_tps) *pp_tps = (double)n_prompt / pp;
        if (tg_tps) *tg_tps = n_gen ? (double)n_gen / tg : 0.0;
    });
}

int32_t rie_hip_synth_tiny(const char *arch, int32_t wtype, rie_hip_synth_spec *out) { return rie::synth_tiny(arch, wtype, out); }
int32_t rie_hip_synth_preset(const char *name, int32_t wtype, rie_hip_synth_spec *out) { return rie::synth_preset(name, wtype, out); }

size_t rie_hip_synth_build(const rie_hip_synth_spec *spec, uint8_t **out, int32_t n_threads) {
    try {
        size_t n = 0;
        *out = rie::synth_build(*spec, n_threads, &n);
        return n;
    } catch (...) {
        return 0;
    }
}

void rie_hip_free(void *p) { free(p); }

int32_t rie_hip_quantize(int32_t ty, const float *x, size_t n, uint8_t *out) {
    return rie::synth_quantize(ty, x, n, out) ? RIE_HIP_OK : RIE_HIP_ERR_UNSUPPORTED;
}

int32_t rie_hip_set_capture(rie_hip_backend *b, int32_t on) {
    return guarded(nullptr, 0, [&] { b->b->set_capture(on != 0); });
}

int32_t rie_hip_set_attention_ranges(rie_hip_backend *b, int32_t on) {
    return guarded(nullptr, 0, [&] { b->b->set_attention_ranges(on != 0); });
}

int32_t rie_hip_capture(rie_hip_backend *b, size_t layer, int32_t what, float *out, size_t len) {
    return guarded(nullptr, 0, [&] {
        if (!b->b->capture(layer, what, out, len)) throw Error{rie::E_RUNTIME, "nothing captured"};
    });
}

int32_t rie_hip_kv_layer(rie_hip_backend *b, size_t layer, int32_t which, uint8_t *out, size_t len, uint8_t *scales_out,
                         size_t scales_len) {
    return guarded(nullptr, 0, [&] { b->b->kv_layer(layer, which, out, len, scales_out, scales_len); });
}

int32_t rie_hip_profile_decode(rie_hip_backend *b, size_t pos, int32_t reps, char *names, size_t names_len, double *ms,
                               int32_t *launches, size_t max_entries, size_t *n_entries) {
    return guarded(nullptr, 0, [&] {
        auto v = b->b->profile_decode(pos, reps);
        std::string all;
        size_t i = 0;
        for (; i < v.size() && i < max_entries; i++) {
            all += v[i].name + "\n";
            ms[i] = v[i].ms;
            launches[i] = v[i].launches;
        }
        write_err(names, names_len, all);
        *n_entries = i;
    });
}

int32_t rie_hip_time_ffn_glu(rie_hip_backend *b, int32_t reps, double *avg_us, size_t *bytes_per_launch) {
    return guarded(nullptr, 0, [&] { *avg_us = b->b->time_ffn_glu(reps, bytes_per_launch); });
}

// ---- kernel entry points ----
int32_t rie_hip_k_rmsnorm_quant(const float *x, const float *w, float eps, int32_t n, int32_t k, int32_t fmt, float *xn, int8_t *qs,
                                float *d, float *s, int32_t *isum, int16_t *bsums) {
    return guarded(nullptr, 0, [&] {
        if ((fmt == rie::ACT_Q8_0 && k % 32) || (fmt == rie::ACT_Q8K && k % 256) || (fmt != rie::ACT_Q8_0 && fmt != rie::ACT_Q8K))
            throw Error{rie::E_RUNTIME, "bad format/size"};
        rie::ActQ8 a;
        a.qs = qs;
        a.d = d;
        a.s = s;
        a.isum = isum;
        a.bsums = bsums;
        rie::launch_rmsnorm_quant(x, k, w, eps, n, k, xn, fmt, a, 0, true);
        RIE_HIP_CHECK(hipGetLastError());
        RIE_HIP_CHECK(hipDeviceSynchronize());
    });
}

static rie::DevWeight mkw(int32_t ty, const uint8_t *w, int32_t rows, int32_t k) {
    rie::DevWeight dw;
    dw.ty = ty;
    dw.rows = (size_t)rows;
    dw.cols = (size_t)k;
    dw.data = w;
    return dw;
}

// The kernels read whole aligned words around each block, up to 4 KiB past a
// matrix's last row (the backend's weight upload carries that slack).  A caller's
// buffer may end at the last row, so the kernel entry points run on a copy with
// the slack; the copy is freed when the call returns.
struct PaddedWeight {
    uint8_t *data = nullptr;
    PaddedWeight(int32_t ty, const uint8_t *w, int32_t rows, int32_t k) {
        if (!w || rows < 1 || k < 1 || !rie::block_bytes(ty) || k % (int32_t)rie::block_size(ty)) throw Error{rie::E_UNSUPPORTED, "unsupported weight type/shape"};
        const size_t bytes = (size_t)rows * rie::row_bytes(ty, (size_t)k);
        RIE_HIP_CHECK(hipMalloc(&data, bytes + 4096));
        RIE_HIP_CHECK(hipMemset(data + bytes, 0, 4096));
        RIE_HIP_CHECK(hipMemcpy(data, w, bytes, hipMemcpyDeviceToDevice));
    }
    ~PaddedWeight() {
        if (data) (void)hipFree(data);
    }
    PaddedWeight(const PaddedWeight &) = delete;
    PaddedWeight &operator=(const PaddedWeight &) = delete;
};

int32_t rie_hip_k_gemv(int32_t ty, const uint8_t *w, int32_t rows, int32_t k, const int8_t *qs, const float *d, const float *s,
                       const int32_t *isum, const int16_t *bsums, const float *act_f32, int32_t n_tok, float *out) {
    return guarded(nullptr, 0, [&] {
        rie::ActQ8 a;
        a.qs = const_cast<int8_t *>(qs);
        a.d = const_cast<float *>(d);
        a.s = const_cast<float *>(s);
        a.isum = const_cast<int32_t *>(isum);
        a.bsums = const_cast<int16_t *>(bsums);
        PaddedWeight pw(ty, w, rows, k);
        rie::GemvSeg sg{mkw(ty, pw.data, rows, k), out, rows, rie::EPI_STORE};
        if (!rie::launch_gemv(&sg, 1, a, act_f32, n_tok, k, 0)) throw Error{rie::E_UNSUPPORTED, "unsupported weight type/shape"};
        RIE_HIP_CHECK(hipGetLastError());
        RIE_HIP_CHECK(hipDeviceSynchronize());
    });
}

int32_t rie_hip_k_gemm(int32_t ty, const uint8_t *w, int32_t rows, int32_t k, const int8_t *qs, const float *d, const float *s,
                       const int32_t *isum, const int16_t *bsums, int32_t n_tok, float *out) {
    return guarded(nullptr, 0, [&] {
        rie::ActQ8 a;
        a.qs = const_cast<int8_t *>(qs);
        a.d = const_cast<float *>(d);
        a.s = const_cast<float *>(s);
        a.isum = const_cast<int32_t *>(isum);
        a.bsums = const_cast<int16_t *>(bsums);
        PaddedWeight pw(ty, w, rows, k);
        rie::GemvSeg sg{mkw(ty, pw.data, rows, k), out, rows, rie::EPI_STORE};
        // room for the partial sums of a K split (up to three planes, capped at
        // 64 MiB like the backend's workspace), only where a split can happen:
        // Q4_0/Q8_0 weights with at least 48 stages of 128 values, or Q4_K/Q6_K with
        // at least 8 superblocks, over 64 tokens
        const bool can_split = ((ty == rie::T_Q4_0 || ty == rie::T_Q8_0) && k / 128 >= 48 && n_tok > 64) ||
                               ((ty == rie::T_Q4_K || ty == rie::T_Q6_K) && k / 256 >= 8 && n_tok > 64);
        const size_t cap = can_split ? std::min<size_t>(3 * (size_t)n_tok * (size_t)std::max(rows, 0), (size_t)1 << 24) : 0;
        float *part = nullptr;
        if (cap) RIE_HIP_CHECK(hipMalloc(&part, cap * sizeof(float)));
        const bool ok = rie::gemm_supported(ty, (size_t)k) && rie::launch_gemm(&sg, 1, a, n_tok, k, 0, nullptr, part, cap);
        hipError_t e = hipGetLastError();
        hipError_t e2 = hipDeviceSynchronize();
        if (part) (void)hipFree(part);
        if (!ok) throw Error{rie::E_UNSUPPORTED, "no GEMM kernel for this weight type/shape"};
        RIE_HIP_CHECK(e);
        RIE_HIP_CHECK(e2);
    });
}

int32_t rie_hip_k_moe_route(const float *logits, int32_t n_tok, int32_t n_exp, int32_t k, int32_t norm_topk, int32_t unit_weights,
                            int32_t *sel, float *wgt) {
    return guarded(nullptr, 0, [&] {
        if (n_tok < 1 || n_exp < 1 || n_exp > 512 || k < 1 || k > n_exp || k > 64 || !logits || !sel || !wgt)
            throw Error{rie::E_RUNTIME, "bad routing sizes"};
        rie::launch_moe_route(logits, n_tok, n_exp, k, norm_topk, unit_weights, sel, wgt, 0);
        RIE_HIP_CHECK(hipGetLastError());
        RIE_HIP_CHECK(hipDeviceSynchronize());
    });
}

int32_t rie_hip_k_argmax(const float *x, int32_t n, uint32_t *out_idx) {
    return guarded(nullptr, 0, [&] {
        // 64 partial indices, 64 partial values and the arrival counter of the
        // one-launch form (the backend's), in one zeroed allocation
        void *buf = nullptr;
        RIE_HIP_CHECK(hipMalloc(&buf, 129 * 4));
        hipError_t e = hipMemset(buf, 0, 129 * 4);
        if (e == hipSuccess) {
            int *pi = (int *)buf;
            float *pv = (float *)buf + 64;
            rie::launch_argmax(x, n, pi, pv, 64, out_idx, 0, (int *)buf + 128);
            e = hipGetLastError();
        }
        hipError_t e2 = hipDeviceSynchronize();
        (void)hipFree(buf);
        RIE_HIP_CHECK(e);
        RIE_HIP_CHECK(e2);
    });
}

int32_t rie_hip_k_argmax_noalloc(const float *x, int32_t n, uint32_t *out_idx, void *stream, char *err, size_t err_len) {
    return guarded(err, err_len, [&] {
        rie::launch_argmax_noalloc(x, n, out_idx, (hipStream_t)stream);
        RIE_HIP_CHECK(hipGetLastError());
        if (!stream) RIE_HIP_CHECK(hipDeviceSynchronize());
    });
}

}  // extern "C"
