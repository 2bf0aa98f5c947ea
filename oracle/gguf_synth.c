/*
 * gguf_synth.c — GGUF v3 writer/reader (gguf.rs) and the synthetic model
 * generator behind `rie bench --synthetic` (testing.rs), restated byte for byte.
 * TEST INFRASTRUCTURE ONLY (the oracle); see oracle.h.
 */
#include "oracle.h"
#include "oracle_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- growable byte buffer ------------------------------------------------ */
typedef struct {
    uint8_t *p;
    size_t len, cap;
} buf_t;

static void buf_reserve(buf_t *b, size_t extra) {
    if (b->len + extra <= b->cap) return;
    size_t nc = b->cap ? b->cap : 4096;
    while (nc < b->len + extra) nc *= 2;
    b->p = (uint8_t *)realloc(b->p, nc);
    b->cap = nc;
}
static void put(buf_t *b, const void *src, size_t n) {
    buf_reserve(b, n);
    memcpy(b->p + b->len, src, n);
    b->len += n;
}
static void put_u32(buf_t *b, uint32_t v) { put(b, &v, 4); }
static void put_u64(buf_t *b, uint64_t v) { put(b, &v, 8); }
static void put_str(buf_t *b, const char *s) {
    put_u64(b, (uint64_t)strlen(s));
    put(b, s, strlen(s));
}
static void pad_to(buf_t *b, size_t align) {
    size_t n = (b->len + align - 1) / align * align;
    buf_reserve(b, n - b->len);
    memset(b->p + b->len, 0, n - b->len);
    b->len = n;
}

/* GgufWriter (gguf.rs:335-437): kv pairs are buffered as encoded bytes, tensor
 * data is kept in order. */
typedef struct {
    buf_t kv;
    uint64_t n_kv;
    buf_t tinfo_names; /* not used: tensors are written directly below */
    size_t n_t, cap_t;
    char **names;
    uint64_t (*dims)[4];
    uint32_t *ndims;
    int *types;
    uint8_t **data;
    size_t *sizes;
} writer_t;

static void kv_key(writer_t *w, const char *key, uint32_t ty) {
    put_str(&w->kv, key);
    put_u32(&w->kv, ty);
    w->n_kv++;
}
static void kv_u32(writer_t *w, const char *key, uint32_t v) {
    kv_key(w, key, 4);
    put_u32(&w->kv, v);
}
static void kv_f32(writer_t *w, const char *key, float v) {
    kv_key(w, key, 6);
    put(&w->kv, &v, 4);
}
static void kv_str(writer_t *w, const char *key, const char *v) {
    kv_key(w, key, 8);
    put_str(&w->kv, v);
}

static void add_tensor(writer_t *w, const char *name, const uint64_t *dims, uint32_t nd, int ty, uint8_t *data) {
    if (w->n_t == w->cap_t) {
        w->cap_t = w->cap_t ? w->cap_t * 2 : 64;
        w->names = (char **)realloc(w->names, w->cap_t * sizeof(char *));
        w->dims = (uint64_t(*)[4])realloc(w->dims, w->cap_t * sizeof(*w->dims));
        w->ndims = (uint32_t *)realloc(w->ndims, w->cap_t * sizeof(uint32_t));
        w->types = (int *)realloc(w->types, w->cap_t * sizeof(int));
        w->data = (uint8_t **)realloc(w->data, w->cap_t * sizeof(uint8_t *));
        w->sizes = (size_t *)realloc(w->sizes, w->cap_t * sizeof(size_t));
    }
    uint64_t n = 1;
    for (uint32_t i = 0; i < nd; i++) {
        w->dims[w->n_t][i] = dims[i];
        n *= dims[i];
    }
    w->names[w->n_t] = strdup(name);
    w->ndims[w->n_t] = nd;
    w->types[w->n_t] = ty;
    w->data[w->n_t] = data;
    w->sizes[w->n_t] = (size_t)(n / or_block_size(ty) * or_block_bytes(ty));
    w->n_t++;
}

/* gguf.rs:407-436 */
static size_t writer_finish(writer_t *w, uint8_t **out) {
    buf_t o = {0};
    size_t total = w->kv.len + 1024;
    for (size_t i = 0; i < w->n_t; i++) total += w->sizes[i] + 64 + strlen(w->names[i]);
    buf_reserve(&o, total);
    put_u32(&o, 0x46554747u);
    put_u32(&o, 3);
    put_u64(&o, (uint64_t)w->n_t);
    put_u64(&o, w->n_kv);
    put(&o, w->kv.p, w->kv.len);
    uint64_t offset = 0;
    for (size_t i = 0; i < w->n_t; i++) {
        put_str(&o, w->names[i]);
        put_u32(&o, w->ndims[i]);
        for (uint32_t d = 0; d < w->ndims[i]; d++) put_u64(&o, w->dims[i][d]);
        put_u32(&o, (uint32_t)w->types[i]);
        put_u64(&o, offset);
        offset += (w->sizes[i] + 31) / 32 * 32;
    }
    pad_to(&o, 32);
    for (size_t i = 0; i < w->n_t; i++) {
        put(&o, w->data[i], w->sizes[i]);
        pad_to(&o, 32);
        free(w->data[i]);
        free(w->names[i]);
    }
    free(w->kv.p);
    free(w->names);
    free(w->dims);
    free(w->ndims);
    free(w->types);
    free(w->data);
    free(w->sizes);
    *out = o.p;
    return o.len;
}

/* ---- random_weight, testing.rs:33-91 --------------------------------------- */
static const size_t *scale_offsets(int ty, size_t *n) {
    static const size_t o0[] = {0}, o02[] = {0, 2}, o8082[] = {80, 82}, o108[] = {108}, o208[] = {208};
    switch (ty) {
    case OR_Q4_0: case OR_Q5_0: case OR_Q8_0: *n = 1; return o0;
    case OR_Q4_1: case OR_Q5_1: case OR_Q4_K: case OR_Q5_K: *n = 2; return o02;
    case OR_Q2_K: *n = 2; return o8082;
    case OR_Q3_K: *n = 1; return o108;
    case OR_Q6_K: *n = 1; return o208;
    default: *n = 0; return NULL;
    }
}

void or_random_weight(or_rng *r, int ty, size_t rows, size_t cols, float gain, uint8_t *out) {
    size_t n = rows * cols;
    if (ty == OR_F32 || ty == OR_F16 || ty == OR_BF16) {
        float sc = 0.1f * gain;
        for (size_t i = 0; i < n; i++) {
            float v = or_rng_sym(r) * sc;
            if (ty == OR_F32) memcpy(out + 4 * i, &v, 4);
            else {
                uint16_t h = ty == OR_F16 ? or_f32_to_f16(v) : or_f32_to_bf16(v);
                out[2 * i] = (uint8_t)h;
                out[2 * i + 1] = (uint8_t)(h >> 8);
            }
        }
        return;
    }
    size_t nblocks = n / or_block_size(ty), bb = or_block_bytes(ty), total = nblocks * bb;
    size_t i = 0;
    for (; i + 8 <= total; i += 8) {
        uint64_t v = or_rng_next(r);
        memcpy(out + i, &v, 8);
    }
    if (i < total) {
        uint64_t v = or_rng_next(r);
        memcpy(out + i, &v, total - i);
    }
    float k;
    switch (ty) {
    case OR_Q4_0: case OR_Q4_1: k = 0.01f; break;
    case OR_Q5_0: case OR_Q5_1: k = 0.005f; break;
    case OR_Q8_0: k = 0.001f; break;
    case OR_Q2_K: k = 0.004f; break;
    case OR_Q3_K: k = 0.003f; break;
    case OR_Q4_K: k = 0.001f; break;
    case OR_Q5_K: k = 0.0007f; break;
    case OR_Q6_K: k = 0.0001f; break;
    default: k = 0.01f;
    }
    float scale = gain * k;
    size_t nofs;
    const size_t *offs = scale_offsets(ty, &nofs);
    int signed_first = ty == OR_Q4_0 || ty == OR_Q5_0 || ty == OR_Q8_0 || ty == OR_Q3_K || ty == OR_Q6_K;
    int min_second = ty == OR_Q4_1 || ty == OR_Q5_1;
    for (size_t b = 0; b < nblocks; b++) {
        for (size_t si = 0; si < nofs; si++) {
            float v = (or_rng_f32(r) * 0.5f + 0.5f) * scale;
            if (si == 0 && signed_first && or_rng_f32(r) < 0.3f) v = -v;
            if (si == 1 && min_second) v = -v * 8.0f;
            uint16_t h = or_f32_to_f16(v);
            out[b * bb + offs[si]] = (uint8_t)h;
            out[b * bb + offs[si] + 1] = (uint8_t)(h >> 8);
        }
    }
}

/* ---- SyntheticSpec, testing.rs:95-212 -------------------------------------- */
static int is_kquant(int t) { return t == OR_Q4_K || t == OR_Q5_K || t == OR_Q6_K || t == OR_Q2_K || t == OR_Q3_K; }

int or_synth_tiny(const char *arch, int wtype, or_synth_spec *s) {
    memset(s, 0, sizeof(*s));
    snprintf(s->arch, sizeof(s->arch), "%s", arch);
    s->n_vocab = 384;
    s->n_embd = 256;
    s->n_layer = 2;
    s->n_head = 4;
    s->n_head_kv = 2;
    s->head_dim = 64;
    s->n_ff = 512;
    s->rope_dim = 64;
    s->ctx = 256;
    s->wtype = wtype;
    s->embd_type = or_block_size(wtype) > 1 ? OR_Q8_0 : wtype;
    s->tied_output = 0;
    s->qkv_bias = strcmp(arch, "qwen2") == 0;
    s->qk_norm = strcmp(arch, "qwen3") == 0 || strcmp(arch, "gemma3") == 0;
    s->post_norms = strcmp(arch, "gemma2") == 0 || strcmp(arch, "gemma3") == 0;
    s->fused = strcmp(arch, "phi3") == 0;
    s->swa_window = (strcmp(arch, "gemma2") == 0 || strcmp(arch, "gemma3") == 0) ? 5 : 0;
    s->n_expert = (strcmp(arch, "qwen3moe") == 0 || strcmp(arch, "qwen2moe") == 0) ? 8 : 0;
    s->n_expert_used = 2;
    s->n_ff_exp = 256;
    s->n_ff_shexp = strcmp(arch, "qwen2moe") == 0 ? 256 : 0;
    s->chat_template = 0;
    s->seed = 1;
    return 0;
}

int or_synth_preset(const char *name, int wtype, or_synth_spec *s) {
    static const struct {
        const char *name, *arch;
        uint32_t v, e, l, h, kv, hd, ff;
        int tied;
    } P[] = {
        {"llama-3.2-1b", "llama", 128256, 2048, 16, 32, 8, 64, 8192, 1},
        {"llama-3.2-3b", "llama", 128256, 3072, 28, 24, 8, 128, 8192, 1},
        {"qwen2.5-0.5b", "qwen2", 151936, 896, 24, 14, 2, 64, 4864, 1},
        {"qwen2.5-1.5b", "qwen2", 151936, 1536, 28, 12, 2, 128, 8960, 1},
        {"qwen3-0.6b", "qwen3", 151936, 1024, 28, 16, 8, 128, 3072, 1},
        {"qwen3-1.7b", "qwen3", 151936, 2048, 28, 16, 8, 128, 6144, 1},
        {"qwen3-4b", "qwen3", 151936, 2560, 36, 32, 8, 128, 9728, 1},
        {"gemma-3-1b", "gemma3", 262144, 1152, 26, 4, 1, 256, 6912, 1},
        {"phi-4-mini", "phi3", 200064, 3072, 32, 24, 8, 128, 8192, 1},
        {"smollm2-360m", "llama", 49152, 960, 32, 15, 5, 64, 2560, 1},
        {"qwen3-30b-a3b", "qwen3moe", 151936, 2048, 48, 32, 4, 128, 6144, 0},
    };
    for (size_t i = 0; i < sizeof(P) / sizeof(P[0]); i++) {
        if (strcmp(P[i].name, name) != 0) continue;
        or_synth_tiny(P[i].arch, wtype, s);
        s->n_vocab = P[i].v;
        s->n_embd = P[i].e;
        s->n_layer = P[i].l;
        s->n_head = P[i].h;
        s->n_head_kv = P[i].kv;
        s->head_dim = P[i].hd;
        s->n_ff = P[i].ff;
        s->rope_dim = strcmp(P[i].arch, "phi3") == 0 ? 96 : P[i].hd;
        s->ctx = 4096;
        s->swa_window = strcmp(P[i].arch, "gemma3") == 0 ? 512 : 0;
        if (strcmp(P[i].arch, "qwen3moe") == 0) {
            s->n_expert = 128;
            s->n_expert_used = 8;
            s->n_ff_exp = 768;
        }
        s->tied_output = P[i].tied;
        s->embd_type = or_block_size(wtype) > 1 ? OR_Q6_K : wtype;
        if (P[i].e % 256 != 0 || P[i].ff % 256 != 0) {
            if (is_kquant(wtype)) s->wtype = OR_Q8_0;
            if (s->embd_type == OR_Q6_K) s->embd_type = OR_Q8_0;
        }
        return 0;
    }
    return -1;
}

static uint8_t *mat(or_rng *r, uint64_t rows, uint64_t cols, int ty) {
    size_t sz = (size_t)(rows * cols / or_block_size(ty) * or_block_bytes(ty));
    uint8_t *p = (uint8_t *)malloc(sz ? sz : 1);
    or_random_weight(r, ty, (size_t)rows, (size_t)cols, 1.0f, p);
    return p;
}

static uint8_t *norm_vec(or_rng *r, size_t n) {
    float *p = (float *)malloc(n * 4);
    for (size_t i = 0; i < n; i++) p[i] = 1.0f + 0.1f * or_rng_sym(r);
    return (uint8_t *)p;
}

static uint8_t *f32_vec(or_rng *r, size_t n, float sc) {
    float *p = (float *)malloc(n * 4);
    for (size_t i = 0; i < n; i++) p[i] = or_rng_sym(r) * sc;
    return (uint8_t *)p;
}

/* testing.rs:229-383 */
size_t or_synth_build(const or_synth_spec *sp, uint8_t **out) {
    or_rng rng;
    or_rng_init(&rng, sp->seed);
    writer_t w;
    memset(&w, 0, sizeof(w));
    const char *a = sp->arch;
    char key[256], val[256];
#define K(suffix) (snprintf(key, sizeof(key), "%s." suffix, a), key)
    kv_str(&w, "general.architecture", a);
    snprintf(val, sizeof(val), "synthetic-%s", a);
    kv_str(&w, "general.name", val);
    kv_u32(&w, K("embedding_length"), sp->n_embd);
    kv_u32(&w, K("block_count"), sp->n_layer);
    kv_u32(&w, K("attention.head_count"), sp->n_head);
    kv_u32(&w, K("attention.head_count_kv"), sp->n_head_kv);
    kv_u32(&w, K("attention.key_length"), sp->head_dim);
    kv_u32(&w, K("attention.value_length"), sp->head_dim);
    kv_u32(&w, K("feed_forward_length"), sp->n_ff);
    kv_u32(&w, K("context_length"), sp->ctx);
    kv_u32(&w, K("rope.dimension_count"), sp->rope_dim);
    kv_f32(&w, K("rope.freq_base"), 10000.0f);
    kv_f32(&w, K("attention.layer_norm_rms_epsilon"), 1e-6f);
    if (sp->n_expert > 0) {
        kv_u32(&w, K("expert_count"), sp->n_expert);
        kv_u32(&w, K("expert_used_count"), sp->n_expert_used);
        kv_u32(&w, K("expert_feed_forward_length"), sp->n_ff_exp);
    }
    if (sp->swa_window > 0) kv_u32(&w, K("attention.sliding_window"), sp->swa_window);
    if (strcmp(a, "granite") == 0) {
        kv_f32(&w, "granite.embedding_scale", 12.0f);
        kv_f32(&w, "granite.residual_scale", 0.22f);
        kv_f32(&w, "granite.logit_scale", 8.0f);
        kv_f32(&w, "granite.attention.scale", 0.0078125f * 8.0f);
    }
    if (strcmp(a, "gemma3") == 0) kv_f32(&w, "gemma3.rope.freq_base", 1000000.0f);
#undef K
    /* vocabulary: <unk> <s> </s> + 256 byte tokens + specials + pieces + filler */
    size_t nv = sp->n_vocab;
    char **toks = (char **)calloc(nv + 300, sizeof(char *));
    int32_t *types = (int32_t *)calloc(nv + 300, sizeof(int32_t));
    size_t nt = 0;
#define PUSH(s, t)                    \
    do {                              \
        toks[nt] = strdup(s);         \
        types[nt] = (t);              \
        nt++;                         \
    } while (0)
    PUSH("<unk>", 2);
    PUSH("<s>", 3);
    PUSH("</s>", 3);
    for (int b = 0; b < 256; b++) {
        char t[16];
        snprintf(t, sizeof(t), "<0x%02X>", b);
        PUSH(t, 6);
    }
    if (sp->chat_template == 1) {
        PUSH("<|im_start|>", 3);
        PUSH("<|im_end|>", 3);
    } else if (sp->chat_template == 2) {
        PUSH("<|start_header_id|>", 3);
        PUSH("<|end_header_id|>", 3);
        PUSH("<|eot_id|>", 3);
    }
    static const char *pieces[] = {"\xe2\x96\x81the", "\xe2\x96\x81" "a", "\xe2\x96\x81phone", "\xe2\x96\x81" "fast",
                                   "in", "er", "\xe2\x96\x81", "e", "t", "h", "o", "n"};
    for (size_t i = 0; i < 12; i++)
        if (nt < nv) PUSH(pieces[i], 1);
    char **all = toks;
    if (nt < nv) {
        all = (char **)realloc(toks, nv * sizeof(char *));
        types = (int32_t *)realloc(types, nv * sizeof(int32_t));
        toks = all;
    }
    while (nt < nv) {
        char t[32];
        snprintf(t, sizeof(t), "[tok%zu]", nt);
        PUSH(t, 1);
    }
#undef PUSH
    for (size_t i = nv; i < nt; i++) free(toks[i]);
    nt = nv < nt ? nv : nt;
    kv_str(&w, "tokenizer.ggml.model", "llama");
    kv_key(&w, "tokenizer.ggml.tokens", 9);
    put_u32(&w.kv, nt ? 8u : 4u);
    put_u64(&w.kv, nt);
    for (size_t i = 0; i < nt; i++) put_str(&w.kv, toks[i]);
    kv_key(&w, "tokenizer.ggml.scores", 9);
    put_u32(&w.kv, nv ? 6u : 4u);
    put_u64(&w.kv, nv);
    for (size_t i = 0; i < nv; i++) {
        float f = -(float)i;
        put(&w.kv, &f, 4);
    }
    kv_key(&w, "tokenizer.ggml.token_type", 9);
    put_u32(&w.kv, nt ? 5u : 4u);
    put_u64(&w.kv, nt);
    for (size_t i = 0; i < nt; i++) put(&w.kv, &types[i], 4);
    kv_u32(&w, "tokenizer.ggml.bos_token_id", 1);
    kv_u32(&w, "tokenizer.ggml.eos_token_id", 2);
    kv_u32(&w, "tokenizer.ggml.unknown_token_id", 0);
    if (sp->chat_template == 1)
        kv_str(&w, "tokenizer.chat_template",
               "{% for m in messages %}<|im_start|>{{ m.role }}\n{{ m.content }}<|im_end|>\n{% endfor %}");
    else if (sp->chat_template == 2)
        kv_str(&w, "tokenizer.chat_template", "<|start_header_id|>{{ role }}<|end_header_id|>\n\n{{ content }}<|eot_id|>");
    for (size_t i = 0; i < nt; i++) free(toks[i]);
    free(toks);
    free(types);

    uint64_t e = sp->n_embd, ff = sp->n_ff, qd = (uint64_t)sp->n_head * sp->head_dim,
             kvd = (uint64_t)sp->n_head_kv * sp->head_dim, hd = sp->head_dim;
    int wt = sp->wtype;
    uint64_t d2[4];
#define T2(name, c0, c1, ty, data)              \
    do {                                        \
        d2[0] = (c0);                           \
        d2[1] = (c1);                           \
        add_tensor(&w, name, d2, 2, ty, data);  \
    } while (0)
#define T1(name, c0, ty, data)                  \
    do {                                        \
        d2[0] = (c0);                           \
        add_tensor(&w, name, d2, 1, ty, data);  \
    } while (0)
    uint8_t *embd = mat(&rng, sp->n_vocab, e, sp->embd_type);
    T2("token_embd.weight", e, sp->n_vocab, sp->embd_type, embd);
    T1("output_norm.weight", e, OR_F32, norm_vec(&rng, sp->n_embd));
    if (!sp->tied_output) {
        uint8_t *o = mat(&rng, sp->n_vocab, e, sp->embd_type);
        T2("output.weight", e, sp->n_vocab, sp->embd_type, o);
    }
    char nm[128];
    for (uint32_t il = 0; il < sp->n_layer; il++) {
#define P(s) (snprintf(nm, sizeof(nm), "blk.%u.%s", il, s), nm)
        T1(P("attn_norm.weight"), e, OR_F32, norm_vec(&rng, sp->n_embd));
        if (sp->fused) {
            T2(P("attn_qkv.weight"), e, qd + 2 * kvd, wt, mat(&rng, qd + 2 * kvd, e, wt));
        } else {
            uint8_t *q = mat(&rng, qd, e, wt);
            T2(P("attn_q.weight"), e, qd, wt, q);
            uint8_t *k = mat(&rng, kvd, e, wt);
            T2(P("attn_k.weight"), e, kvd, wt, k);
            uint8_t *v = mat(&rng, kvd, e, wt);
            T2(P("attn_v.weight"), e, kvd, wt, v);
        }
        if (sp->qkv_bias) {
            T1(P("attn_q.bias"), qd, OR_F32, f32_vec(&rng, qd, 0.1f));
            T1(P("attn_k.bias"), kvd, OR_F32, f32_vec(&rng, kvd, 0.1f));
            T1(P("attn_v.bias"), kvd, OR_F32, f32_vec(&rng, kvd, 0.1f));
        }
        if (sp->qk_norm) {
            T1(P("attn_q_norm.weight"), hd, OR_F32, norm_vec(&rng, sp->head_dim));
            T1(P("attn_k_norm.weight"), hd, OR_F32, norm_vec(&rng, sp->head_dim));
        }
        T2(P("attn_output.weight"), qd, e, wt, mat(&rng, e, qd, wt));
        if (sp->post_norms) {
            T1(P("post_attention_norm.weight"), e, OR_F32, norm_vec(&rng, sp->n_embd));
            T1(P("post_ffw_norm.weight"), e, OR_F32, norm_vec(&rng, sp->n_embd));
        }
        T1(P("ffn_norm.weight"), e, OR_F32, norm_vec(&rng, sp->n_embd));
        if (sp->n_expert > 0) {
            uint64_t ne = sp->n_expert, fx = sp->n_ff_exp;
            uint8_t *router = f32_vec(&rng, (size_t)(ne * e), 0.5f);
            T2(P("ffn_gate_inp.weight"), e, ne, OR_F32, router);
            uint64_t d3[3];
            d3[0] = e; d3[1] = fx; d3[2] = ne;
            add_tensor(&w, P("ffn_gate_exps.weight"), d3, 3, wt, mat(&rng, fx * ne, e, wt));
            add_tensor(&w, P("ffn_up_exps.weight"), d3, 3, wt, mat(&rng, fx * ne, e, wt));
            d3[0] = fx; d3[1] = e;
            add_tensor(&w, P("ffn_down_exps.weight"), d3, 3, wt, mat(&rng, e * ne, fx, wt));
            if (sp->n_ff_shexp > 0) {
                uint64_t fs = sp->n_ff_shexp;
                T2(P("ffn_gate_shexp.weight"), e, fs, wt, mat(&rng, fs, e, wt));
                T2(P("ffn_up_shexp.weight"), e, fs, wt, mat(&rng, fs, e, wt));
                T2(P("ffn_down_shexp.weight"), fs, e, wt, mat(&rng, e, fs, wt));
                T1(P("ffn_gate_inp_shexp.weight"), e, OR_F32, f32_vec(&rng, sp->n_embd, 0.3f));
            }
        } else if (sp->fused) {
            T2(P("ffn_up.weight"), e, 2 * ff, wt, mat(&rng, 2 * ff, e, wt));
            T2(P("ffn_down.weight"), ff, e, wt, mat(&rng, e, ff, wt));
        } else {
            T2(P("ffn_gate.weight"), e, ff, wt, mat(&rng, ff, e, wt));
            T2(P("ffn_up.weight"), e, ff, wt, mat(&rng, ff, e, wt));
            T2(P("ffn_down.weight"), ff, e, wt, mat(&rng, e, ff, wt));
        }
#undef P
    }
#undef T1
#undef T2
    return writer_finish(&w, out);
}

/* ---- GGUF reader, gguf.rs:193-269 ------------------------------------------- */
typedef struct {
    const uint8_t *p;
    size_t len, pos;
    int err;
} rd_t;

static const uint8_t *take(rd_t *r, size_t n) {
    if (r->err || r->pos + n > r->len) {
        r->err = 1;
        return NULL;
    }
    const uint8_t *s = r->p + r->pos;
    r->pos += n;
    return s;
}
static uint64_t rd_u(rd_t *r, size_t n) {
    const uint8_t *s = take(r, n);
    uint64_t v = 0;
    if (s) memcpy(&v, s, n);
    return v;
}

static int skip_value(rd_t *r, uint32_t ty, or_kv *kv, int depth) {
    switch (ty) {
    case 0: case 1: case 7: kv->u = rd_u(r, 1); kv->i = ty == 1 ? (int8_t)kv->u : (int64_t)kv->u; kv->f = (double)kv->i; break;
    case 2: case 3: kv->u = rd_u(r, 2); kv->i = ty == 3 ? (int16_t)kv->u : (int64_t)kv->u; kv->f = (double)kv->i; break;
    case 4: case 5: kv->u = rd_u(r, 4); kv->i = ty == 5 ? (int32_t)kv->u : (int64_t)kv->u; kv->f = (double)kv->i; break;
    case 6: {
        uint32_t b = (uint32_t)rd_u(r, 4);
        float f;
        memcpy(&f, &b, 4);
        kv->f = f;
        kv->i = (int64_t)f;
        kv->u = (uint64_t)kv->i;
        break;
    }
    case 10: case 11: kv->u = rd_u(r, 8); kv->i = (int64_t)kv->u; kv->f = ty == 11 ? (double)kv->i : (double)kv->u; break;
    case 12: {
        uint64_t b = rd_u(r, 8);
        memcpy(&kv->f, &b, 8);
        kv->i = (int64_t)kv->f;
        kv->u = (uint64_t)kv->i;
        break;
    }
    case 8: {
        uint64_t n = rd_u(r, 8);
        if (n > r->len) return -1;
        kv->str = (const char *)take(r, (size_t)n);
        kv->str_len = (size_t)n;
        break;
    }
    case 9: {
        if (depth > 4) return -1;
        uint32_t et = (uint32_t)rd_u(r, 4);
        uint64_t n = rd_u(r, 8);
        if (n > r->len) return -1;
        kv->arr_len = (size_t)n;
        kv->arr_type = et;
        or_kv tmp;
        for (uint64_t i = 0; i < n && !r->err; i++) {
            memset(&tmp, 0, sizeof(tmp));
            if (skip_value(r, et, &tmp, depth + 1)) return -1;
        }
        break;
    }
    default: return -1;
    }
    return r->err ? -1 : 0;
}

int or_gguf_parse(const uint8_t *p, size_t len, or_gguf *g, char *err, size_t err_len) {
    memset(g, 0, sizeof(*g));
    rd_t r = {p, len, 0, 0};
    if (rd_u(&r, 4) != 0x46554747u) {
        snprintf(err, err_len, "invalid model file: not a GGUF file (bad magic)");
        return -2;
    }
    uint32_t version = (uint32_t)rd_u(&r, 4);
    if (version < 2 || version > 3) {
        snprintf(err, err_len, "unsupported: GGUF version %u (only v2 and v3 are supported)", version);
        return -3;
    }
    uint64_t n_t = rd_u(&r, 8), n_kv = rd_u(&r, 8);
    if (r.err || n_kv > len || n_t > len) {
        snprintf(err, err_len, "invalid model file: truncated header");
        return -2;
    }
    g->kv = (or_kv *)calloc(n_kv ? n_kv : 1, sizeof(or_kv));
    g->n_kv = (size_t)n_kv;
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t kl = rd_u(&r, 8);
        const uint8_t *ks = take(&r, (size_t)kl);
        if (!ks) break;
        g->kv[i].key = (const char *)ks;
        g->kv[i].key_len = (size_t)kl;
        g->kv[i].type = (uint32_t)rd_u(&r, 4);
        if (skip_value(&r, g->kv[i].type, &g->kv[i], 0)) {
            snprintf(err, err_len, "invalid model file: bad metadata value");
            return -2;
        }
    }
    uint64_t align = 32;
    const or_kv *al = or_gguf_get(g, "general.alignment");
    if (al && al->u > 0) align = al->u;
    g->tensors = (or_tensor *)calloc(n_t ? n_t : 1, sizeof(or_tensor));
    g->n_tensors = (size_t)n_t;
    for (uint64_t i = 0; i < n_t; i++) {
        uint64_t nl = rd_u(&r, 8);
        const uint8_t *ns = take(&r, (size_t)nl);
        uint32_t nd = (uint32_t)rd_u(&r, 4);
        if (r.err || nd == 0 || nd > 4) {
            snprintf(err, err_len, "invalid model file: tensor has %u dims", nd);
            return -2;
        }
        or_tensor *t = &g->tensors[i];
        size_t cl = nl < sizeof(t->name) - 1 ? (size_t)nl : sizeof(t->name) - 1;
        memcpy(t->name, ns, cl);
        t->name[cl] = 0;
        t->n_dims = nd;
        for (uint32_t d = 0; d < nd; d++) t->dims[d] = rd_u(&r, 8);
        t->type = (int)rd_u(&r, 4);
        t->offset = rd_u(&r, 8);
        if (or_block_bytes(t->type) == 0) {
            snprintf(err, err_len, "unsupported: tensor %s uses ggml type id %d", t->name, t->type);
            return -3;
        }
    }
    if (r.err) {
        snprintf(err, err_len, "invalid model file: unexpected end of file");
        return -2;
    }
    uint64_t data_start = (r.pos + align - 1) / align * align;
    for (size_t i = 0; i < g->n_tensors; i++) {
        or_tensor *t = &g->tensors[i];
        uint64_t n = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) n *= t->dims[d];
        if (t->dims[0] % or_block_size(t->type) != 0) {
            snprintf(err, err_len, "invalid model file: tensor %s: row length not a multiple of block size", t->name);
            return -2;
        }
        t->size = n / or_block_size(t->type) * or_block_bytes(t->type);
        t->offset += data_start;
        if (t->offset + t->size > len) {
            snprintf(err, err_len, "invalid model file: tensor %s extends past end of file", t->name);
            return -2;
        }
        t->data = p + t->offset;
        t->cols = t->dims[0];
        t->rows = n / t->dims[0];
    }
    g->data_start = data_start;
    return 0;
}

void or_gguf_free(or_gguf *g) {
    free(g->kv);
    free(g->tensors);
    memset(g, 0, sizeof(*g));
}

/* later keys replace earlier ones, like the HashMap insert in gguf.rs:232 */
const or_kv *or_gguf_get(const or_gguf *g, const char *key) {
    size_t kl = strlen(key);
    for (size_t i = g->n_kv; i-- > 0;)
        if (g->kv[i].key_len == kl && memcmp(g->kv[i].key, key, kl) == 0) return &g->kv[i];
    return NULL;
}

const or_tensor *or_gguf_tensor(const or_gguf *g, const char *name) {
    for (size_t i = 0; i < g->n_tensors; i++)
        if (strcmp(g->tensors[i].name, name) == 0) return &g->tensors[i];
    return NULL;
}
