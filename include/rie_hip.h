/*
 * rie_hip.h — C ABI of the MI355X (gfx950) backend for RIE's per-token forward
 * loop (librie_hip.so).
 *
 * The backend entry points mirror the reference's `trait Backend`
 * (crates/rie-core/src/model/mod.rs:303-320) one for one, so a Rust
 * `impl Backend for HipBackend` over these symbols is a drop-in for the seam
 * that `rie bench`, `rie run` and rie-server already call
 * (crates/rie-cli/src/main.rs:246-262, crates/rie-server/src/lib.rs:602-640,
 * crates/rie-ffi/src/lib.rs:96-129).  Conventions follow rie.h
 * (crates/rie-ffi/include/rie.h:17-73): NULL / negative return on failure with
 * the message written into a caller buffer, no exceptions across the ABI.
 *
 * Thread-safety: one host thread drives a handle at a time (Backend: Send).
 * forward() is synchronous: it returns after the logits are in host memory.
 */
#ifndef RIE_HIP_H
#define RIE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes: one per variant of the reference's Error enum
 * (crates/rie-core/src/error.rs:5-15). */
#define RIE_HIP_OK 0
#define RIE_HIP_ERR_IO (-1)
#define RIE_HIP_ERR_FORMAT (-2)
#define RIE_HIP_ERR_UNSUPPORTED (-3)
#define RIE_HIP_ERR_MISSING (-4)
#define RIE_HIP_ERR_RUNTIME (-5)

/* KV cache formats (KvType, crates/rie-core/src/model/cpu.rs:12-36). */
#define RIE_HIP_KV_F16 0
#define RIE_HIP_KV_Q8_0 1
#define RIE_HIP_KV_TURBO4 2

typedef struct rie_hip_backend rie_hip_backend;

typedef struct rie_hip_config {
    int32_t n_ctx;     /* KV capacity in positions (the caller applies min(n_ctx, ctx_train)) */
    int32_t max_batch; /* tokens per forward (CpuBackend max_batch, clamped to [1, n_ctx]) */
    int32_t kv_type;   /* RIE_HIP_KV_*; falls back to f16 like CpuBackend::with_kv_type */
    int32_t device;    /* HIP device ordinal */
    int32_t use_graph; /* 1: replay the single-token decode step as a HIP graph */
} rie_hip_config;

rie_hip_config rie_hip_default_config(void);

/* Construct a backend from a GGUF image held in host memory (the reference's
 * GgufFile::data(), crates/rie-core/src/gguf.rs:271-276).  Tensor data is copied
 * once to HBM in its native ggml block layout; the image may be released after
 * the call.  Replaces CpuBackend::with_kv_type (model/cpu.rs:100-177) /
 * GpuBackend::new (crates/rie-gpu/src/lib.rs:236-624).  Returns NULL on failure;
 * *err_code (if non-NULL) receives the RIE_HIP_ERR_* class. */
rie_hip_backend *rie_hip_create(const uint8_t *gguf, size_t gguf_len, const rie_hip_config *cfg, int32_t *err_code, char *err,
                                size_t err_len);
void rie_hip_destroy(rie_hip_backend *b);

/* Backend::name (model/mod.rs:305): copies a NUL-terminated name, returns its length. */
size_t rie_hip_name(const rie_hip_backend *b, char *buf, size_t buf_len);
/* Backend::max_batch (model/mod.rs:307) */
size_t rie_hip_max_batch(const rie_hip_backend *b);
/* Backend::n_ctx (model/mod.rs:309) */
size_t rie_hip_n_ctx(const rie_hip_backend *b);
/* Backend::forward (model/mod.rs:310-313; CpuBackend semantics model/cpu.rs:210-409):
 * evaluate tokens[0..n) at positions pos..pos+n; writes the last token's logits
 * (n_vocab floats) or, with all_logits, n·n_vocab floats.  Errors (RUNTIME):
 * empty batch, n > max_batch, pos+n > n_ctx, token id out of range, logits buffer
 * too small (checked before any work is done). */
int32_t rie_hip_forward(rie_hip_backend *b, const uint32_t *tokens, size_t n, size_t pos, int32_t all_logits, float *logits,
                        size_t logits_len, char *err, size_t err_len);
/* Backend::hidden (model/mod.rs:314-319): final normalized hidden rows of the last
 * forward (rows × n_embd), valid until the next call; NULL when none. */
const float *rie_hip_hidden(rie_hip_backend *b, size_t *rows);

/* ---- model facts ---- */
size_t rie_hip_n_vocab(const rie_hip_backend *b);
size_t rie_hip_n_embd(const rie_hip_backend *b);
int32_t rie_hip_kv_type(const rie_hip_backend *b);
size_t rie_hip_kv_bytes(const rie_hip_backend *b);
size_t rie_hip_weight_bytes(const rie_hip_backend *b);

/* ---- engine-side greedy decoding on the device (Engine::bench / eval_next,
 * crates/rie-core/src/engine.rs:384-392, 540-564; sampler.rs:199-209 argmax with
 * first-max tie-break).  No per-token logits readback. ---- */
/* forward(tokens, pos) then argmax of the last logits row; returns 0 and *next. */
int32_t rie_hip_forward_argmax(rie_hip_backend *b, const uint32_t *tokens, size_t n, size_t pos, uint32_t *next, char *err,
                               size_t err_len);
/* n_gen greedy steps continuing from the token chosen by the previous
 * forward_argmax/generate call, at positions pos, pos+1, ...; out[i] receives the
 * token fed at step i. */
int32_t rie_hip_generate_greedy(rie_hip_backend *b, size_t pos, size_t n_gen, uint32_t *out, char *err, size_t err_len);
/* Engine::bench (engine.rs:540-564): prompt ids (i·7919+13) mod V, warm-up on the
 * first 8, one prompt evaluation in chunks of max_batch, then n_gen greedy steps.
 * Returns prompt and generation throughput in tokens/s. */
int32_t rie_hip_bench(rie_hip_backend *b, size_t n_prompt, size_t n_gen, double *pp_tps, double *tg_tps, char *err, size_t err_len);

/* ---- synthetic GGUF images (`rie bench --synthetic`, crates/rie-core/src/testing.rs:95-383) ---- */
typedef struct rie_hip_synth_spec {
    char arch[32];
    uint32_t n_vocab, n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, rope_dim, ctx;
    int32_t wtype, embd_type;
    int32_t tied_output, qkv_bias, qk_norm, post_norms, fused;
    uint32_t swa_window, n_expert, n_expert_used, n_ff_exp, n_ff_shexp;
    int32_t chat_template; /* 0 none, 1 chatml, 2 llama3 */
    uint64_t seed;
    /* workload mode: 0 = the reference's random-byte weights (testing.rs:46-91);
     * 1 = N(0, 0.02) values quantized with quantize::q4_0 / Q8_0 (quant/mod.rs:262-298),
     *     unit norms, rope_base below */
    int32_t mode;
    float rope_base;
    int32_t output_type; /* mode 1: type of output.weight (-1 = embd_type) */
    /* mode 1 per-tensor mix: 0 = every matrix wtype; 1 = Q4_K_M: attn_v Q6_K, ffn_down
     * Q6_K in the layers llama.cpp's Q4_K_M gives more bits (i < n/8, i >= 7n/8,
     * (i - n/8) % 3 == 2), wtype elsewhere */
    int32_t mix;
} rie_hip_synth_spec;

/* SyntheticSpec::tiny (testing.rs:127-154) / preset (testing.rs:157-212); 0 or -1. */
int32_t rie_hip_synth_tiny(const char *arch, int32_t wtype, rie_hip_synth_spec *out);
int32_t rie_hip_synth_preset(const char *name, int32_t wtype, rie_hip_synth_spec *out);
/* SyntheticSpec::build (testing.rs:229-383): writes the GGUF image to a buffer
 * owned by the library (release with rie_hip_free); returns its size, 0 on error. */
size_t rie_hip_synth_build(const rie_hip_synth_spec *spec, uint8_t **out, int32_t n_threads);
void rie_hip_free(void *p);
/* The generator's weight quantizers: n values of x to ggml blocks of type ty
 * (Q4_0 and Q8_0 are quantize::q4_0 / quantize::q8_0, quant/mod.rs:262-298;
 * Q4_K and Q6_K, which the reference has no quantizer for, are min/max
 * quantizers of this library).  0, or RIE_HIP_ERR_UNSUPPORTED for other types
 * or n not a multiple of the block size. */
int32_t rie_hip_quantize(int32_t ty, const float *x, size_t n, uint8_t *out);

/* ---- parity hooks (no counterpart in the reference; for tests and debugging) ---- */
/* Keep per-layer copies of intermediate f32 tensors during forward (slow path):
 * what = 0 x after attention, 1 x after FFN, 2 attention output, 3 q after
 * RoPE/scale, 4 k after norm/RoPE, 5 v, 6 FFN gated hidden, 7 MoE router logits,
 * 8 the experts the device routing selected ([n][k] int32 bit patterns, ascending),
 * 9 their combination weights ([n][k]). */
int32_t rie_hip_set_capture(rie_hip_backend *b, int32_t on);
/* on = 1: single-token attention always splits the context into ranges merged
 * across workgroups, also at the short contexts where it otherwise runs one
 * workgroup per query head over the whole cache (so tests can check both kernels
 * on the same positions); on = 0: automatic (the default). */
int32_t rie_hip_set_attention_ranges(rie_hip_backend *b, int32_t on);
int32_t rie_hip_capture(rie_hip_backend *b, size_t layer, int32_t what, float *out, size_t len);
/* Raw KV cache of one layer: which 0 = K, 1 = V; [kv_head][slot][row bytes];
 * Turbo4 scales ([kv_head][slot] f16) go to scales_out. */
int32_t rie_hip_kv_layer(rie_hip_backend *b, size_t layer, int32_t which, uint8_t *out, size_t len, uint8_t *scales_out,
                         size_t scales_len);
size_t rie_hip_kv_row_bytes(const rie_hip_backend *b);
/* Time one eager decode step at pos, reps times, with a HIP event after every
 * launch on the backend's stream; per kernel family: summed ms and launch count.
 * names receives the family names separated by newlines. */
int32_t rie_hip_profile_decode(rie_hip_backend *b, size_t pos, int32_t reps, char *names, size_t names_len, double *ms,
                               int32_t *launches, size_t max_entries, size_t *n_entries);

/* Average duration in microseconds of the single-token gate/up/SwiGLU launch
 * (dense_ffn's gate·x, up·x and silu product, model/cpu.rs:431-467, as one
 * kernel), timed with HIP events on the backend's stream while cycling through
 * every layer's weights reps times; *bytes_per_launch = weight bytes of gate
 * and up + activation read + hidden written.  No counterpart in the reference:
 * it measures the dominant decode kernel for the roofline report. */
int32_t rie_hip_time_ffn_glu(rie_hip_backend *b, int32_t reps, double *avg_us, size_t *bytes_per_launch);

/* ---- kernel entry points on device pointers (stream 0, synchronous) ---- */
/* RMSNorm (w may be NULL: quantize only) + Q8_0 (fmt 1) or Q8_K (fmt 2) quantization
 * of n rows of k values (ops.rs:7-14 with the sum of squares in the order of
 * kernels/avx2.rs:186-203; quant/mod.rs:191-218, kernels/avx2.rs:153-184).  Outputs:
 * Q8_0: qs [n][k], d/s/isum [n][k/32]; Q8_K: qs [n][k], d [n][k/256], bsums [n][k/16]. */
int32_t rie_hip_k_rmsnorm_quant(const float *x, const float *w, float eps, int32_t n, int32_t k, int32_t fmt, float *xn, int8_t *qs,
                                float *d, float *s, int32_t *isum, int16_t *bsums);
/* out[t*rows + r] = W[r] · act[t] for one ggml weight matrix (kernels/mod.rs:136-232).
 * w may end at its last row: the kernels read whole aligned words around each
 * block, up to 4 KiB past the matrix, so these entry points run on a padded copy
 * of w (allocated and freed inside the call). */
int32_t rie_hip_k_gemv(int32_t ty, const uint8_t *w, int32_t rows, int32_t k, const int8_t *qs, const float *d, const float *s,
                       const int32_t *isum, const int16_t *bsums, const float *act_f32, int32_t n_tok, float *out);
/* the int8 MFMA prompt GEMM on the same operands (n_tok > 8) */
int32_t rie_hip_k_gemm(int32_t ty, const uint8_t *w, int32_t rows, int32_t k, const int8_t *qs, const float *d, const float *s,
                       const int32_t *isum, const int16_t *bsums, int32_t n_tok, float *out);
/* MoE routing of n_tok tokens (moe_ffn's routing, model/cpu.rs:487-501): softmax
 * over each token's n_exp router logits (ops.rs:38-49), the k most probable
 * experts with the lower index first on ties (NaN probabilities compare Equal, so
 * a token whose probabilities are NaN takes experts 0..k-1), weights p/Σ_top p
 * (norm_topk), p, or 1 (unit_weights).  sel/wgt [n_tok][k] receive each token's
 * choices in ascending expert order.  1 ≤ k ≤ min(n_exp, 64), n_exp ≤ 512; other
 * sizes return RIE_HIP_ERR_RUNTIME. */
int32_t rie_hip_k_moe_route(const float *logits, int32_t n_tok, int32_t n_exp, int32_t k, int32_t norm_topk, int32_t unit_weights,
                            int32_t *sel, float *wgt);
/* greedy argmax (sampler.rs:199-209) of n floats */
int32_t rie_hip_k_argmax(const float *x, int32_t n, uint32_t *out_idx);
/* The same argmax without allocating device memory.  No counterpart in the
 * reference: for callers that cannot call hipMalloc (code under HIP stream or
 * graph capture, tight serving loops, harnesses that forbid allocation).  The
 * partial maxima live in a fixed 8 KiB array of the library's static device
 * memory (one copy per GPU, held until the process ends), so n must be in
 * 1..1048576 (1024 partials of up to 1024 values); larger or empty inputs return
 * RIE_HIP_ERR_RUNTIME with the reason in err.  stream: a hipStream_t to launch on
 * (the call returns once the two kernels are queued, without synchronizing, so
 * it can be recorded under capture), or NULL: the null stream, and the call
 * returns after the result is written.  The first call on a device looks up the
 * array's address (hipGetSymbolAddress), so make it outside capture.  Calls that
 * overlap on one GPU (several streams or host threads) share that array and race. */
int32_t rie_hip_k_argmax_noalloc(const float *x, int32_t n, uint32_t *out_idx, void *stream, char *err, size_t err_len);

#ifdef __cplusplus
}
#endif
#endif
