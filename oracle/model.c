/*
 * model.c — ModelConfig::from_gguf, Model::load, CpuBackend::forward_impl and
 * the Engine loops (eval_tokens / eval_next / bench) restated for x86.
 * TEST INFRASTRUCTURE ONLY (the oracle); see oracle.h.
 *
 * Reference files (crates/rie-core/src): model/config.rs:106-247,
 * model/mod.rs:101-247, model/cpu.rs:93-658, engine.rs:250-272/384-392/540-564,
 * sampler.rs:199-209, kernels/matmul.rs:28-241.
 */
#include "oracle.h"
#include "oracle_internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

enum { A_LLAMA, A_QWEN2, A_QWEN3, A_PHI3, A_GEMMA, A_GEMMA2, A_GEMMA3, A_GRANITE, A_QWEN3MOE, A_QWEN2MOE };

typedef struct {
    int ty;
    size_t rows, cols;
    const uint8_t *data;
} weight_t;

typedef struct {
    weight_t gate, up, down;
} dense_t;

typedef struct {
    weight_t router;
    dense_t *experts;
    size_t n_exp, n_used;
    int norm_topk, unit_weights, has_shared;
    dense_t shared;
    float *shared_gate;
} moe_t;

typedef struct {
    float *attn_norm, *bq, *bk, *bv, *q_norm, *k_norm, *post_attn_norm, *ffn_norm, *post_ffn_norm;
    weight_t wq, wk, wv, wo;
    int is_moe;
    dense_t dense;
    moe_t moe;
} layer_t;

struct or_model {
    int arch;
    size_t n_vocab, n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, ctx_train, rope_dim;
    float rms_eps, rope_base, rope_freq_scale, rope_base_swa;
    int has_rope_swa, rope_neox, gelu;
    float embd_scale, attn_scale, residual_scale, logit_scale;
    int has_attn_softcap, has_final_softcap;
    float attn_softcap, final_softcap;
    size_t swa_window, swa_pattern, n_expert, n_expert_used, n_ff_exp;
    int expert_norm_topk;
    weight_t token_embd, output;
    float *output_norm, *rope_factors;
    size_t n_rope_factors;
    layer_t *layers;
    or_gguf g;
};

static int is_swa(const or_model *m, size_t il) {
    return m->swa_window > 0 && m->swa_pattern > 0 && (il % m->swa_pattern) < m->swa_pattern - 1;
}

/* ---- config.rs:106-247 ---------------------------------------------------- */
static int get_u64(const or_gguf *g, const char *arch, const char *k, uint64_t *out) {
    char key[256];
    snprintf(key, sizeof(key), "%s.%s", arch, k);
    const or_kv *kv = or_gguf_get(g, key);
    if (!kv || kv->type == 6 || kv->type == 12 || kv->type == 8 || kv->type == 9) return 0;
    if ((kv->type == 1 || kv->type == 3 || kv->type == 5 || kv->type == 11) && kv->i < 0) return 0;
    *out = kv->u;
    return 1;
}
static int get_f32(const or_gguf *g, const char *key, float *out) {
    const or_kv *kv = or_gguf_get(g, key);
    if (!kv || kv->type == 8 || kv->type == 9) return 0;
    *out = (float)kv->f;
    return 1;
}
static int get_f32a(const or_gguf *g, const char *arch, const char *k, float *out) {
    char key[256];
    snprintf(key, sizeof(key), "%s.%s", arch, k);
    return get_f32(g, key, out);
}

static float *vec_of(const or_tensor *t) {
    size_t n = (size_t)(t->rows * t->cols);
    float *v = (float *)malloc(n * sizeof(float));
    or_dequantize_row(t->type, t->data, v, n);
    return v;
}

static weight_t wt_of(const or_tensor *t) {
    weight_t w = {t->type, (size_t)t->rows, (size_t)t->cols, t->data};
    return w;
}

static weight_t slice_rows(weight_t w, size_t start, size_t n) {
    weight_t s = w;
    s.rows = n;
    s.data = w.data + start * or_row_bytes(w.ty, w.cols);
    return s;
}

static void set_err(char *err, size_t len, const char *msg) {
    if (err && len) snprintf(err, len, "%s", msg);
}

or_model *or_model_load(const uint8_t *gguf, size_t len, char *err, size_t err_len) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    if (or_gguf_parse(gguf, len, &m->g, err, err_len)) {
        free(m);
        return NULL;
    }
    or_gguf *g = &m->g;
    char ebuf[256];
    const or_kv *ak = or_gguf_get(g, "general.architecture");
    if (!ak || ak->type != 8) {
        set_err(err, err_len, "missing: general.architecture");
        goto fail;
    }
    char arch[64];
    snprintf(arch, sizeof(arch), "%.*s", (int)ak->str_len, ak->str);
    static const char *names[] = {"llama", "qwen2", "qwen3", "phi3", "gemma", "gemma2", "gemma3", "granite", "qwen3moe", "qwen2moe"};
    m->arch = -1;
    for (int i = 0; i < 10; i++)
        if (strcmp(arch, names[i]) == 0) m->arch = i;
    if (strcmp(arch, "mistral") == 0) m->arch = A_LLAMA;
    if (m->arch < 0) {
        snprintf(ebuf, sizeof(ebuf), "unsupported: architecture '%s'", arch);
        set_err(err, err_len, ebuf);
        goto fail;
    }
    uint64_t v;
#define REQ(k, dst)                                                            \
    do {                                                                       \
        if (!get_u64(g, arch, k, &v)) {                                        \
            snprintf(ebuf, sizeof(ebuf), "missing: metadata %s.%s", arch, k);   \
            set_err(err, err_len, ebuf);                                       \
            goto fail;                                                         \
        }                                                                      \
        dst = (size_t)v;                                                       \
    } while (0)
    REQ("embedding_length", m->n_embd);
    REQ("block_count", m->n_layer);
    REQ("attention.head_count", m->n_head);
#undef REQ
    m->n_head_kv = get_u64(g, arch, "attention.head_count_kv", &v) ? (size_t)v : m->n_head;
    m->head_dim = get_u64(g, arch, "attention.key_length", &v) ? (size_t)v : m->n_embd / m->n_head;
    if (get_u64(g, arch, "attention.value_length", &v) && v != m->head_dim) {
        set_err(err, err_len, "unsupported: value head dim != key head dim");
        goto fail;
    }
    if (get_u64(g, arch, "feed_forward_length", &v) || get_u64(g, arch, "expert_feed_forward_length", &v)) m->n_ff = (size_t)v;
    else {
        set_err(err, err_len, "missing: metadata feed_forward_length");
        goto fail;
    }
    const or_kv *tk = or_gguf_get(g, "tokenizer.ggml.tokens");
    if (tk && tk->type == 9) m->n_vocab = tk->arr_len;
    else if (get_u64(g, arch, "vocab_size", &v)) m->n_vocab = (size_t)v;
    else {
        set_err(err, err_len, "missing: vocabulary");
        goto fail;
    }
    if (!get_f32a(g, arch, "attention.layer_norm_rms_epsilon", &m->rms_eps)) m->rms_eps = 1e-5f;
    m->ctx_train = get_u64(g, arch, "context_length", &v) ? (size_t)v : 4096;
    m->rope_dim = get_u64(g, arch, "rope.dimension_count", &v) ? (size_t)v : m->head_dim;
    if (!get_f32a(g, arch, "rope.freq_base", &m->rope_base)) m->rope_base = 10000.0f;
    m->rope_freq_scale = 1.0f;
    {
        char key[256];
        snprintf(key, sizeof(key), "%s.rope.scaling.type", arch);
        const or_kv *st = or_gguf_get(g, key);
        float f;
        if (st && st->type == 8 && st->str_len == 6 && memcmp(st->str, "linear", 6) == 0 &&
            get_f32a(g, arch, "rope.scaling.factor", &f) && f > 0.0f)
            m->rope_freq_scale = 1.0f / f;
        if (get_f32a(g, arch, "rope.scale_linear", &f) && f > 0.0f) m->rope_freq_scale = 1.0f / f;
    }
    m->rope_neox = m->arch != A_LLAMA && m->arch != A_GRANITE;
    m->n_expert = get_u64(g, arch, "expert_count", &v) ? (size_t)v : 0;
    m->n_expert_used = get_u64(g, arch, "expert_used_count", &v) ? (size_t)v : 2;
    m->n_ff_exp = get_u64(g, arch, "expert_feed_forward_length", &v) ? (size_t)v : m->n_ff;
    {
        char key[256];
        snprintf(key, sizeof(key), "%s.expert_weights_norm", arch);
        const or_kv *nk = or_gguf_get(g, key);
        m->expert_norm_topk = nk ? (nk->type == 7 ? (int)nk->u : nk->u != 0) : m->arch != A_QWEN2MOE;
    }
    int gemma = m->arch == A_GEMMA || m->arch == A_GEMMA2 || m->arch == A_GEMMA3;
    m->gelu = gemma;
    m->embd_scale = gemma ? sqrtf((float)m->n_embd) : 1.0f;
    m->attn_scale = 1.0f / sqrtf((float)m->head_dim);
    m->residual_scale = 1.0f;
    m->logit_scale = 1.0f;
    if (m->arch == A_GEMMA2) {
        m->has_attn_softcap = 1;
        if (!get_f32a(g, arch, "attn_logit_softcapping", &m->attn_softcap)) m->attn_softcap = 50.0f;
        m->has_final_softcap = 1;
        if (!get_f32a(g, arch, "final_logit_softcapping", &m->final_softcap)) m->final_softcap = 30.0f;
        m->swa_window = get_u64(g, arch, "attention.sliding_window", &v) ? (size_t)v : 4096;
        m->swa_pattern = 2;
        if (m->n_layer == 46) m->attn_scale = 1.0f / sqrtf((float)(m->n_embd / m->n_head));
    } else if (m->arch == A_GEMMA3) {
        m->swa_window = get_u64(g, arch, "attention.sliding_window", &v) ? (size_t)v : 1024;
        m->swa_pattern = 6;
        m->has_rope_swa = 1;
        m->rope_base_swa = 10000.0f;
        if (m->n_layer == 62) m->attn_scale = 1.0f / sqrtf((float)(m->n_embd / m->n_head));
        m->has_final_softcap = get_f32a(g, arch, "final_logit_softcapping", &m->final_softcap);
        m->has_attn_softcap = get_f32a(g, arch, "attn_logit_softcapping", &m->attn_softcap);
    } else if (m->arch == A_GRANITE) {
        if (!get_f32a(g, arch, "embedding_scale", &m->embd_scale)) m->embd_scale = 1.0f;
        if (!get_f32a(g, arch, "residual_scale", &m->residual_scale)) m->residual_scale = 1.0f;
        if (!get_f32a(g, arch, "logit_scale", &m->logit_scale)) m->logit_scale = 1.0f;
        float s;
        if (get_f32a(g, arch, "attention.scale", &s)) m->attn_scale = s;
    }
    if (m->n_head % m->n_head_kv != 0 || m->rope_dim > m->head_dim || m->rope_dim % 2 != 0) {
        set_err(err, err_len, "invalid model file: bad head configuration");
        goto fail;
    }

    /* model/mod.rs:112-247 */
    const or_tensor *t = or_gguf_tensor(g, "token_embd.weight");
    if (!t) {
        set_err(err, err_len, "missing: tensor token_embd.weight");
        goto fail;
    }
    m->token_embd = wt_of(t);
    if (m->token_embd.cols != m->n_embd) {
        set_err(err, err_len, "invalid model file: token_embd columns");
        goto fail;
    }
    t = or_gguf_tensor(g, "output.weight");
    m->output = t ? wt_of(t) : m->token_embd;
    t = or_gguf_tensor(g, "output_norm.weight");
    if (!t) {
        set_err(err, err_len, "missing: tensor output_norm.weight");
        goto fail;
    }
    m->output_norm = vec_of(t);
    t = or_gguf_tensor(g, "rope_freqs.weight");
    if (!t) t = or_gguf_tensor(g, "rope_factors_short.weight");
    if (t) {
        m->rope_factors = vec_of(t);
        m->n_rope_factors = (size_t)(t->rows * t->cols);
    }
    size_t qd = m->n_head * m->head_dim, kvd = m->n_head_kv * m->head_dim;
    m->layers = (layer_t *)calloc(m->n_layer, sizeof(layer_t));
    char nm[128];
#define TN(s) (snprintf(nm, sizeof(nm), "blk.%zu.%s", il, s), or_gguf_tensor(g, nm))
#define NEED(dst, s)                                                   \
    do {                                                               \
        const or_tensor *tt_ = TN(s);                                  \
        if (!tt_) {                                                    \
            snprintf(ebuf, sizeof(ebuf), "missing: tensor %s", nm);    \
            set_err(err, err_len, ebuf);                               \
            goto fail;                                                 \
        }                                                              \
        dst = wt_of(tt_);                                              \
    } while (0)
#define OPTV(dst, s)                     \
    do {                                 \
        const or_tensor *tt_ = TN(s);    \
        dst = tt_ ? vec_of(tt_) : NULL;  \
    } while (0)
    for (size_t il = 0; il < m->n_layer; il++) {
        layer_t *L = &m->layers[il];
        const or_tensor *qkv = TN("attn_qkv.weight");
        if (qkv) {
            weight_t f = wt_of(qkv);
            L->wq = slice_rows(f, 0, qd);
            L->wk = slice_rows(f, qd, kvd);
            L->wv = slice_rows(f, qd + kvd, kvd);
        } else {
            NEED(L->wq, "attn_q.weight");
            NEED(L->wk, "attn_k.weight");
            NEED(L->wv, "attn_v.weight");
        }
        const or_tensor *router = TN("ffn_gate_inp.weight");
        if (router) {
            size_t ne = m->n_expert, ff = m->n_ff_exp;
            L->is_moe = 1;
            L->moe.router = wt_of(router);
            weight_t ga, ua, da;
            NEED(ga, "ffn_gate_exps.weight");
            NEED(ua, "ffn_up_exps.weight");
            NEED(da, "ffn_down_exps.weight");
            L->moe.n_exp = ne;
            L->moe.experts = (dense_t *)calloc(ne, sizeof(dense_t));
            for (size_t x = 0; x < ne; x++) {
                L->moe.experts[x].gate = slice_rows(ga, x * ff, ff);
                L->moe.experts[x].up = slice_rows(ua, x * ff, ff);
                L->moe.experts[x].down = slice_rows(da, x * m->n_embd, m->n_embd);
            }
            const or_tensor *sg = TN("ffn_gate_shexp.weight");
            if (sg) {
                L->moe.has_shared = 1;
                L->moe.shared.gate = wt_of(sg);
                NEED(L->moe.shared.up, "ffn_up_shexp.weight");
                NEED(L->moe.shared.down, "ffn_down_shexp.weight");
            }
            OPTV(L->moe.shared_gate, "ffn_gate_inp_shexp.weight");
            size_t nu = m->n_expert_used;
            L->moe.n_used = nu < 1 ? 1 : (nu > ne ? ne : nu);
            L->moe.norm_topk = m->expert_norm_topk;
            const or_kv *gk = or_gguf_get(g, "rie.expert_gating");
            L->moe.unit_weights = gk && gk->type == 8 && gk->str_len == 4 && memcmp(gk->str, "unit", 4) == 0;
        } else {
            const or_tensor *gt = TN("ffn_gate.weight");
            if (gt) {
                L->dense.gate = wt_of(gt);
                NEED(L->dense.up, "ffn_up.weight");
            } else {
                weight_t up;
                NEED(up, "ffn_up.weight");
                L->dense.gate = slice_rows(up, 0, m->n_ff);
                L->dense.up = slice_rows(up, m->n_ff, m->n_ff);
            }
            NEED(L->dense.down, "ffn_down.weight");
        }
        const or_tensor *an = TN("attn_norm.weight");
        if (!an) {
            set_err(err, err_len, "missing: attn_norm");
            goto fail;
        }
        L->attn_norm = vec_of(an);
        NEED(L->wo, "attn_output.weight");
        OPTV(L->bq, "attn_q.bias");
        OPTV(L->bk, "attn_k.bias");
        OPTV(L->bv, "attn_v.bias");
        OPTV(L->q_norm, "attn_q_norm.weight");
        OPTV(L->k_norm, "attn_k_norm.weight");
        OPTV(L->post_attn_norm, "post_attention_norm.weight");
        OPTV(L->ffn_norm, "ffn_norm.weight");
        if (!L->ffn_norm) {
            set_err(err, err_len, "missing: ffn_norm");
            goto fail;
        }
        OPTV(L->post_ffn_norm, "post_ffw_norm.weight");
    }
#undef TN
#undef NEED
#undef OPTV
    if (m->output.cols != m->n_embd || m->output.rows < m->n_vocab) {
        set_err(err, err_len, "invalid model file: output matrix does not cover vocabulary");
        goto fail;
    }
    return m;
fail:
    or_model_free(m);
    return NULL;
}

void or_model_free(or_model *m) {
    if (!m) return;
    if (m->layers) {
        for (size_t il = 0; il < m->n_layer; il++) {
            layer_t *L = &m->layers[il];
            free(L->attn_norm); free(L->bq); free(L->bk); free(L->bv); free(L->q_norm); free(L->k_norm);
            free(L->post_attn_norm); free(L->ffn_norm); free(L->post_ffn_norm);
            free(L->moe.experts); free(L->moe.shared_gate);
        }
        free(m->layers);
    }
    free(m->output_norm);
    free(m->rope_factors);
    or_gguf_free(&m->g);
    free(m);
}

void or_model_config(const or_model *m, int64_t *out, size_t n) {
    int64_t v[20] = {(int64_t)m->n_vocab, (int64_t)m->n_embd, (int64_t)m->n_layer, (int64_t)m->n_head,
                     (int64_t)m->n_head_kv, (int64_t)m->head_dim, (int64_t)m->n_ff, (int64_t)m->rope_dim,
                     m->rope_neox, (int64_t)m->n_expert, (int64_t)m->n_expert_used, (int64_t)m->n_ff_exp,
                     (int64_t)m->ctx_train, m->arch, (int64_t)m->output.ty, (int64_t)m->token_embd.ty,
                     (int64_t)m->swa_window, (int64_t)m->swa_pattern, m->gelu, 0};
    for (size_t i = 0; i < n && i < 20; i++) out[i] = v[i];
}

/* ---- QuantActs (matmul.rs:18-97) ------------------------------------------ */
typedef struct {
    size_t n_tok, k;
    const float *f32;
    or_block_q8_0 *q8_0;
    or_block_q8k *q8k;
    size_t cap0, capk;
} acts_t;

typedef struct {
    const float *x;
    acts_t *a;
    int fmt;
} qctx;

static void quant_task(size_t t, int tid, void *c) {
    (void)tid;
    qctx *q = (qctx *)c;
    size_t k = q->a->k;
    if (q->fmt == OR_ACT_Q8_0) or_quantize_q8_0(q->x + t * k, q->a->q8_0 + t * (k / 32), k / 32);
    else or_quantize_q8_k(q->x + t * k, q->a->q8k + t * (k / 256), k / 256);
}

static void acts_prepare(or_pool *pool, acts_t *a, const float *x, size_t n_tok, size_t k, const weight_t **ws, size_t nw) {
    a->n_tok = n_tok;
    a->k = k;
    int have[3] = {0, 0, 0};
    for (size_t i = 0; i < nw; i++) {
        int f = or_act_format(ws[i]->ty);
        if (have[f]) continue;
        have[f] = 1;
        if (f == OR_ACT_F32) {
            a->f32 = x;
        } else if (f == OR_ACT_Q8_0) {
            size_t need = n_tok * (k / 32);
            if (need > a->cap0) {
                free(a->q8_0);
                a->q8_0 = (or_block_q8_0 *)aligned_alloc(16, need * sizeof(or_block_q8_0));
                a->cap0 = need;
            }
            qctx c = {x, a, f};
            or_pool_for(pool, n_tok, 1, quant_task, &c);
        } else {
            size_t need = n_tok * (k / 256);
            if (need > a->capk) {
                free(a->q8k);
                a->q8k = (or_block_q8k *)aligned_alloc(16, need * sizeof(or_block_q8k));
                a->capk = need;
            }
            qctx c = {x, a, f};
            or_pool_for(pool, n_tok, 1, quant_task, &c);
        }
    }
}

static const void *act_row(const acts_t *a, int fmt, size_t t) {
    if (fmt == OR_ACT_F32) return a->f32 + t * a->k;
    if (fmt == OR_ACT_Q8_0) return a->q8_0 + t * (a->k / 32);
    return a->q8k + t * (a->k / 256);
}

/* matmul_multi / compute_rows (matmul.rs:136-241).  The x4 tiles of the AVX2
 * path give bit-identical results to vec_dot (same per-lane FMA order), so the
 * generic row×token loop reproduces every tiling. */
typedef struct {
    const weight_t *w;
    float *out;
    size_t ld, chunk, n_chunks;
} plan_t;

typedef struct {
    plan_t *p;
    size_t np;
    const acts_t *a;
} mmctx;

static void mm_task(size_t c, int tid, void *ctx) {
    (void)tid;
    mmctx *m = (mmctx *)ctx;
    size_t pi = 0;
    while (c >= m->p[pi].n_chunks) {
        c -= m->p[pi].n_chunks;
        pi++;
    }
    const plan_t *p = &m->p[pi];
    const weight_t *w = p->w;
    size_t r0 = c * p->chunk, r1 = r0 + p->chunk < w->rows ? r0 + p->chunk : w->rows;
    int fmt = or_act_format(w->ty);
    size_t rb = or_row_bytes(w->ty, w->cols);
    for (size_t r = r0; r < r1; r++)
        for (size_t t = 0; t < m->a->n_tok; t++)
            p->out[t * p->ld + r] = or_vec_dot(w->ty, w->data + r * rb, act_row(m->a, fmt, t), w->cols);
}

static void matmul_multi(or_pool *pool, const acts_t *a, const weight_t **ws, float **outs, const size_t *lds, size_t nj) {
    plan_t p[8];
    size_t total = 0, nt = (size_t)or_pool_threads(pool);
    for (size_t j = 0; j < nj; j++) {
        size_t rows = ws[j]->rows;
        size_t target = rows / (nt * 8);
        if (target < 16) target = 16;
        size_t chunk = (target + 3) / 4 * 4;
        p[j].w = ws[j];
        p[j].out = outs[j];
        p[j].ld = lds[j];
        p[j].chunk = chunk;
        p[j].n_chunks = (rows + chunk - 1) / chunk;
        total += p[j].n_chunks;
    }
    mmctx c = {p, nj, a};
    or_pool_for(pool, total, 1, mm_task, &c);
}

static void matmul1(or_pool *pool, const acts_t *a, const weight_t *w, float *out) {
    size_t ld = w->rows;
    matmul_multi(pool, a, &w, &out, &ld, 1);
}

/* ---- backend ---------------------------------------------------------------- */
typedef struct {
    uint16_t *k, *v;   /* f16: [kv_head][slot][hd] */
    uint8_t *kq, *vq;  /* Q8_0 / Turbo4 rows */
    size_t slots;
} cache_t;

struct or_backend {
    or_model *m;
    or_pool *pool;
    size_t n_ctx, max_batch;
    int kv;
    cache_t *cache;
    float *inv_freq, *inv_freq_swa;
    float *x, *xn, *q, *k, *v, *att, *o, *gate, *up, *scores, *cos_t, *sin_t, *cos_swa, *sin_swa;
    float *moe_logits, *xg, *yg, *ys;
    acts_t acts;
    size_t hidden_rows;
    int capture;
    float **cap[8];
};

static size_t kv_row_bytes(const or_backend *b) {
    size_t hd = b->m->head_dim;
    return b->kv == OR_KV_TURBO4 ? or_turbo_row_bytes(hd) : or_row_bytes(OR_Q8_0, hd);
}

/* cpu.rs:100-177 */
or_backend *or_backend_new(or_model *m, size_t n_ctx, size_t max_batch, int kv, int n_threads) {
    or_backend *b = (or_backend *)calloc(1, sizeof(or_backend));
    b->m = m;
    b->pool = or_pool_new(n_threads);
    if (max_batch < 1) max_batch = 1;
    if (max_batch > (n_ctx > 1 ? n_ctx : 1)) max_batch = n_ctx > 1 ? n_ctx : 1;
    b->n_ctx = n_ctx;
    b->max_batch = max_batch;
    size_t hd = m->head_dim;
    if (kv == OR_KV_Q8_0 && hd % 32 != 0) kv = OR_KV_F16;
    if (kv == OR_KV_TURBO4 && (hd % 32 != 0 || hd > 512)) kv = OR_KV_F16;
    b->kv = kv;
    b->cache = (cache_t *)calloc(m->n_layer, sizeof(cache_t));
    for (size_t il = 0; il < m->n_layer; il++) {
        size_t slots = n_ctx;
        if (is_swa(m, il)) {
            slots = m->swa_window + max_batch;
            if (slots > n_ctx) slots = n_ctx;
        }
        b->cache[il].slots = slots;
        size_t rows = m->n_head_kv * slots;
        if (kv == OR_KV_F16) {
            b->cache[il].k = (uint16_t *)calloc(rows * hd, 2);
            b->cache[il].v = (uint16_t *)calloc(rows * hd, 2);
        } else {
            size_t rb = kv_row_bytes(b);
            b->cache[il].kq = (uint8_t *)calloc(rows * rb, 1);
            b->cache[il].vq = (uint8_t *)calloc(rows * rb, 1);
        }
    }
    size_t half = m->rope_dim / 2;
    b->inv_freq = (float *)malloc((half ? half : 1) * 4);
    or_rope_inv_freq(m->rope_dim, m->rope_base, m->rope_freq_scale, m->rope_factors, m->n_rope_factors, b->inv_freq);
    if (m->has_rope_swa) {
        b->inv_freq_swa = (float *)malloc((half ? half : 1) * 4);
        or_rope_inv_freq(m->rope_dim, m->rope_base_swa, 1.0f, NULL, 0, b->inv_freq_swa);
    }
    size_t ff_max = m->n_ff;
    int any = 0;
    for (size_t il = 0; il < m->n_layer; il++) {
        layer_t *L = &m->layers[il];
        size_t f;
        if (L->is_moe) {
            f = m->n_ff_exp;
            if (L->moe.has_shared && L->moe.shared.gate.rows > f) f = L->moe.shared.gate.rows;
        } else f = L->dense.gate.rows;
        if (!any || f > ff_max) ff_max = f;
        any = 1;
    }
    size_t e = m->n_embd, qd = m->n_head * hd, kvd = m->n_head_kv * hd, mb = max_batch;
    b->x = (float *)calloc(mb * e, 4);
    b->xn = (float *)calloc(mb * e, 4);
    b->q = (float *)calloc(mb * qd, 4);
    b->k = (float *)calloc(mb * kvd, 4);
    b->v = (float *)calloc(mb * kvd, 4);
    b->att = (float *)calloc(mb * qd, 4);
    b->o = (float *)calloc(mb * e, 4);
    b->gate = (float *)calloc(mb * ff_max, 4);
    b->up = (float *)calloc(mb * ff_max, 4);
    b->moe_logits = (float *)calloc(mb * (m->n_expert ? m->n_expert : 1), 4);
    b->xg = (float *)calloc(mb * e, 4);
    b->yg = (float *)calloc(mb * e, 4);
    b->ys = (float *)calloc(mb * e, 4);
    b->scores = (float *)calloc((size_t)or_pool_threads(b->pool) * n_ctx, 4);
    b->cos_t = (float *)calloc(mb * (half ? half : 1), 4);
    b->sin_t = (float *)calloc(mb * (half ? half : 1), 4);
    b->cos_swa = (float *)calloc(mb * (half ? half : 1), 4);
    b->sin_swa = (float *)calloc(mb * (half ? half : 1), 4);
    return b;
}

static void free_capture(or_backend *b) {
    for (int w = 0; w < 8; w++) {
        if (!b->cap[w]) continue;
        for (size_t il = 0; il < b->m->n_layer; il++)
            if (b->cap[w][il]) free((char *)b->cap[w][il] - 16);
        free(b->cap[w]);
        b->cap[w] = NULL;
    }
}

void or_backend_free(or_backend *b) {
    if (!b) return;
    for (size_t il = 0; il < b->m->n_layer; il++) {
        free(b->cache[il].k); free(b->cache[il].v); free(b->cache[il].kq); free(b->cache[il].vq);
    }
    free(b->cache);
    free(b->inv_freq); free(b->inv_freq_swa);
    free(b->x); free(b->xn); free(b->q); free(b->k); free(b->v); free(b->att); free(b->o); free(b->gate); free(b->up);
    free(b->moe_logits); free(b->xg); free(b->yg); free(b->ys); free(b->scores);
    free(b->cos_t); free(b->sin_t); free(b->cos_swa); free(b->sin_swa);
    free(b->acts.q8_0); free(b->acts.q8k);
    free_capture(b);
    or_pool_free(b->pool);
    free(b);
}

int or_backend_kv_type(const or_backend *b) { return b->kv; }

size_t or_backend_kv_bytes(const or_backend *b) {
    size_t tot = 0;
    for (size_t il = 0; il < b->m->n_layer; il++) {
        size_t rows = b->m->n_head_kv * b->cache[il].slots;
        tot += b->kv == OR_KV_F16 ? rows * b->m->head_dim * 2 * 2 : rows * kv_row_bytes(b) * 2;
    }
    return tot;
}

const uint8_t *or_kv_layer(const or_backend *b, size_t layer, int which, size_t *bytes) {
    const cache_t *c = &b->cache[layer];
    size_t rows = b->m->n_head_kv * c->slots;
    if (b->kv == OR_KV_F16) {
        *bytes = rows * b->m->head_dim * 2;
        return (const uint8_t *)(which ? c->v : c->k);
    }
    *bytes = rows * kv_row_bytes(b);
    return which ? c->vq : c->kq;
}

void or_set_capture(or_backend *b, int on) {
    free_capture(b);
    b->capture = on;
}

const float *or_capture(const or_backend *b, size_t layer, int what, size_t *len) {
    if (!b->cap[what] || layer >= b->m->n_layer) return NULL;
    const float *p = b->cap[what][layer];
    if (!p) return NULL;
    *len = (size_t)((const int64_t *)(const void *)p)[-2];
    return p;
}

static void cap_store(or_backend *b, int what, size_t il, const float *src, size_t n) {
    if (!b->capture) return;
    if (!b->cap[what]) b->cap[what] = (float **)calloc(b->m->n_layer, sizeof(float *));
    free(b->cap[what][il] ? (char *)b->cap[what][il] - 16 : NULL);
    char *mem = (char *)malloc(16 + n * 4);
    ((int64_t *)(void *)mem)[0] = (int64_t)n;
    memcpy(mem + 16, src, n * 4);
    b->cap[what][il] = (float *)(void *)(mem + 16);
}

/* attention (cpu.rs:550-634), one (token, head) task */
typedef struct {
    or_backend *b;
    const cache_t *c;
    size_t n_tok, pos0, window;
} attctx;

static void store_q8_0(const float *x, uint8_t *dst, size_t n) {
    for (size_t bi = 0; bi < n / 32; bi++) {
        const float *xb = x + bi * 32;
        uint8_t *ob = dst + bi * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = or_f32_to_f16(d);
        ob[0] = (uint8_t)h;
        ob[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) {
            int r = (int)roundf(xb[i] * id);
            r = r < -127 ? -127 : (r > 127 ? 127 : r);
            ob[2 + i] = (uint8_t)(int8_t)r;
        }
    }
}

static void axpy_q8_0(float *y, float a, const uint8_t *row, size_t n) {
    for (size_t bi = 0; bi < n / 32; bi++) {
        const uint8_t *b = row + bi * 34;
        float s = a * or_f16_to_f32((uint16_t)(b[0] | ((uint16_t)b[1] << 8)));
        for (int i = 0; i < 32; i++) y[bi * 32 + i] += s * (float)(int8_t)b[2 + i];
    }
}

static void att_task(size_t task, int tid, void *vctx) {
    attctx *A = (attctx *)vctx;
    or_backend *b = A->b;
    const or_model *m = b->m;
    size_t n_head = m->n_head, hd = m->head_dim, qd = n_head * hd;
    size_t group = n_head / m->n_head_kv;
    size_t t = task / n_head, h = task % n_head, g = h / group;
    size_t p = A->pos0 + t;
    size_t start = A->window > 0 ? (p + 1 > A->window ? p + 1 - A->window : 0) : 0;
    size_t len = p + 1 - start;
    const float *qh = b->q + t * qd + h * hd;
    float *sc = b->scores + (size_t)tid * b->n_ctx;
    size_t slots = A->c->slots;
    size_t rb = kv_row_bytes(b);
    float qrot[512];
    or_block_q8_0 qq[16];
    size_t nqb = hd / 32;
    if (b->kv == OR_KV_TURBO4) {
        memcpy(qrot, qh, hd * 4);
        or_turbo_rotate(qrot, hd, OR_TURBO_KV_SEED);
        or_quantize_q8_0(qrot, qq, nqb);
    } else if (b->kv == OR_KV_Q8_0) {
        or_quantize_q8_0(qh, qq, nqb);
    }
    float max = -INFINITY;
    for (size_t i = 0; i < len; i++) {
        size_t row = g * slots + (start + i) % slots;
        float v;
        if (b->kv == OR_KV_F16) v = or_dot_f16_f32(A->c->k + row * hd, qh, hd);
        else if (b->kv == OR_KV_Q8_0) v = or_vec_dot(OR_Q8_0, A->c->kq + row * rb, qq, hd);
        else v = or_turbo_dot(qq, hd, A->c->kq + row * rb);
        if (m->has_attn_softcap) v = m->attn_softcap * tanhf(v / m->attn_softcap);
        sc[i] = v;
        max = fmaxf(max, v);
    }
    float sum = 0.0f;
    for (size_t i = 0; i < len; i++) {
        sc[i] = expf(sc[i] - max);
        sum += sc[i];
    }
    float inv = 1.0f / sum;
    float *o = b->att + t * qd + h * hd;
    memset(o, 0, hd * 4);
    for (size_t i = 0; i < len; i++) {
        size_t row = g * slots + (start + i) % slots;
        if (b->kv == OR_KV_F16) or_axpy_f16(o, sc[i] * inv, A->c->v + row * hd, hd);
        else if (b->kv == OR_KV_Q8_0) axpy_q8_0(o, sc[i] * inv, A->c->vq + row * rb, hd);
        else or_turbo_axpy(o, hd, sc[i] * inv, A->c->vq + row * rb);
    }
    if (b->kv == OR_KV_TURBO4) or_turbo_rotate_inverse(o, hd, OR_TURBO_KV_SEED);
}

typedef struct {
    float *out;
    const float *x, *w;
    size_t e;
    float eps;
} rmsctx;

static void rms_task(size_t t, int tid, void *c) {
    (void)tid;
    rmsctx *r = (rmsctx *)c;
    or_rmsnorm(r->out + t * r->e, r->x + t * r->e, r->w, r->e, r->eps);
}

/* cpu.rs:538-548 */
static void par_rmsnorm(or_pool *pool, float *out, const float *x, const float *w, size_t n, size_t e, float eps) {
    rmsctx c = {out, x, w, e, eps};
    if (n == 1) {
        or_rmsnorm(out, x, w, e, eps);
        return;
    }
    or_pool_for(pool, n, 1, rms_task, &c);
}

static float gelu_tanh(float x) {
    const float k = 0.7978846f;
    return 0.5f * x * (1.0f + tanhf(k * x * (1.0f + 0.044715f * x * x)));
}

/* cpu.rs:433-467 */
static void dense_ffn(or_backend *b, const dense_t *d, const float *x, size_t n, float *out) {
    const or_model *m = b->m;
    size_t e = d->gate.cols, ff = d->gate.rows;
    const weight_t *ws[2] = {&d->gate, &d->up};
    acts_prepare(b->pool, &b->acts, x, n, e, ws, 2);
    float *outs[2] = {b->gate, b->up};
    size_t lds[2] = {ff, ff};
    matmul_multi(b->pool, &b->acts, ws, outs, lds, 2);
    for (size_t i = 0; i < n * ff; i++) {
        float gv = b->gate[i];
        b->gate[i] = (m->gelu ? gelu_tanh(gv) : or_silu(gv)) * b->up[i];
    }
    const weight_t *wd = &d->down;
    acts_prepare(b->pool, &b->acts, b->gate, n, ff, &wd, 1);
    matmul1(b->pool, &b->acts, &d->down, out);
}

/* The routing of one token, cpu.rs:492-500: softmax in place (ops.rs:38-49),
 * sort descending by probability with the comparator
 * `l[b].partial_cmp(&l[a]).unwrap_or(Equal).then(a.cmp(&b))` (a NaN pair compares
 * Equal and falls back to the index), then the top k with weights p/norm, where
 * norm is the sum of the top k in sorted order (norm_topk) or 1, or 1 for unit
 * weights.  choice/w receive the k experts in sorted order. */
static void route_token(float *l, size_t ne, size_t k, int norm_topk, int unit_weights, size_t *choice, float *w) {
    or_softmax(l, ne);
    size_t *idx = (size_t *)malloc(ne * sizeof(size_t));
    for (size_t i = 0; i < ne; i++) idx[i] = i;
    for (size_t i = 1; i < ne; i++) { /* insertion sort: stable, deterministic */
        size_t cur = idx[i], j = i;
        while (j > 0) {
            size_t pv = idx[j - 1];
            int before;
            if (l[cur] > l[pv]) before = 1;
            else if (l[cur] < l[pv]) before = 0;
            else before = cur < pv; /* Equal, or unordered (NaN) */
            if (!before) break;
            idx[j] = pv;
            j--;
        }
        idx[j] = cur;
    }
    float norm = 1.0f;
    if (norm_topk) {
        norm = 0.0f;
        for (size_t q = 0; q < k; q++) norm += l[idx[q]];
    }
    for (size_t q = 0; q < k; q++) {
        choice[q] = idx[q];
        w[q] = unit_weights ? 1.0f : l[idx[q]] / norm;
    }
    free(idx);
}

void or_moe_route(const float *logits, size_t n_tok, size_t n_exp, size_t k, int norm_topk, int unit_weights, int32_t *sel,
                  float *wgt) {
    float *l = (float *)malloc(n_exp * sizeof(float));
    size_t *ch = (size_t *)malloc(k * sizeof(size_t));
    float *w = (float *)malloc(k * sizeof(float));
    for (size_t t = 0; t < n_tok; t++) {
        memcpy(l, logits + t * n_exp, n_exp * sizeof(float));
        route_token(l, n_exp, k, norm_topk, unit_weights, ch, w);
        /* ascending expert order: the order in which moe_ffn adds the experts' outputs */
        for (size_t q = 0; q < k; q++) {
            size_t rank = 0;
            for (size_t r = 0; r < k; r++) rank += ch[r] < ch[q];
            sel[t * k + rank] = (int32_t)ch[q];
            wgt[t * k + rank] = w[q];
        }
    }
    free(l); free(ch); free(w);
}

/* cpu.rs:473-524 */
static void moe_ffn(or_backend *b, const moe_t *mo, const float *x, size_t n, float *out, size_t il) {
    size_t e = mo->router.cols, ne = mo->router.rows;
    const weight_t *wr = &mo->router;
    acts_prepare(b->pool, &b->acts, x, n, e, &wr, 1);
    matmul1(b->pool, &b->acts, &mo->router, b->moe_logits);
    if (b->capture) cap_store(b, 7, il, b->moe_logits, n * ne); /* router logits, before the softmax */
    /* per-expert token lists */
    size_t *cnt = (size_t *)calloc(ne, sizeof(size_t));
    size_t *tok = (size_t *)malloc(ne * n * sizeof(size_t));
    float *wgt = (float *)malloc(ne * n * sizeof(float));
    size_t *idx = (size_t *)malloc(ne * sizeof(size_t));
    float *tw = (float *)malloc(ne * sizeof(float));
    for (size_t t = 0; t < n; t++) {
        route_token(b->moe_logits + t * ne, ne, mo->n_used, mo->norm_topk, mo->unit_weights, idx, tw);
        for (size_t k = 0; k < mo->n_used; k++) {
            size_t i = idx[k];
            tok[i * n + cnt[i]] = t;
            wgt[i * n + cnt[i]] = tw[k];
            cnt[i]++;
        }
    }
    memset(out, 0, n * e * 4);
    for (size_t ex = 0; ex < ne; ex++) {
        size_t k = cnt[ex];
        if (!k) continue;
        for (size_t j = 0; j < k; j++) memcpy(b->xg + j * e, x + tok[ex * n + j] * e, e * 4);
        dense_ffn(b, &mo->experts[ex], b->xg, k, b->yg);
        for (size_t j = 0; j < k; j++) {
            float w = wgt[ex * n + j];
            float *o = out + tok[ex * n + j] * e;
            const float *y = b->yg + j * e;
            for (size_t i = 0; i < e; i++) o[i] += w * y[i];
        }
    }
    if (mo->has_shared) {
        dense_ffn(b, &mo->shared, x, n, b->ys);
        for (size_t t = 0; t < n; t++) {
            const float *xt = x + t * e;
            float scale = mo->shared_gate ? 1.0f / (1.0f + expf(-or_dot_f32(mo->shared_gate, xt, e))) : 1.0f;
            for (size_t i = 0; i < e; i++) out[t * e + i] += scale * b->ys[t * e + i];
        }
    }
    free(cnt); free(tok); free(wgt); free(idx); free(tw);
}

static void residual_add(float *x, const float *y, size_t n, float scale) {
    if (scale == 1.0f)
        for (size_t i = 0; i < n; i++) x[i] += y[i];
    else
        for (size_t i = 0; i < n; i++) x[i] += y[i] * scale;
}

/* cpu.rs:210-409 */
int or_forward(or_backend *b, const uint32_t *tokens, size_t n, size_t pos0, int all_logits, float *logits,
               size_t logits_len, char *err, size_t err_len) {
    or_model *m = b->m;
    char ebuf[256];
    b->hidden_rows = 0;
    if (n == 0) {
        set_err(err, err_len, "empty batch");
        return -5;
    }
    if (n > b->max_batch) {
        snprintf(ebuf, sizeof(ebuf), "batch of %zu tokens exceeds max batch %zu", n, b->max_batch);
        set_err(err, err_len, ebuf);
        return -5;
    }
    if (pos0 + n > b->n_ctx) {
        snprintf(ebuf, sizeof(ebuf), "context window full (%zu tokens)", b->n_ctx);
        set_err(err, err_len, ebuf);
        return -5;
    }
    size_t e = m->n_embd, hd = m->head_dim, qd = m->n_head * hd, kvd = m->n_head_kv * hd, half = m->rope_dim / 2;
    size_t erb = or_row_bytes(m->token_embd.ty, e);
    for (size_t t = 0; t < n; t++) {
        if (tokens[t] >= m->token_embd.rows) {
            snprintf(ebuf, sizeof(ebuf), "token id %u out of range", tokens[t]);
            set_err(err, err_len, ebuf);
            return -5;
        }
        float *row = b->x + t * e;
        or_dequantize_row(m->token_embd.ty, m->token_embd.data + (size_t)tokens[t] * erb, row, e);
        if (m->embd_scale != 1.0f)
            for (size_t i = 0; i < e; i++) row[i] *= m->embd_scale;
    }
    for (size_t t = 0; t < n; t++) {
        or_rope_table(b->inv_freq, half, pos0 + t, b->cos_t + t * half, b->sin_t + t * half);
        if (b->inv_freq_swa) or_rope_table(b->inv_freq_swa, half, pos0 + t, b->cos_swa + t * half, b->sin_swa + t * half);
    }
    for (size_t il = 0; il < m->n_layer; il++) {
        layer_t *L = &m->layers[il];
        int swa = is_swa(m, il);
        par_rmsnorm(b->pool, b->xn, b->x, L->attn_norm, n, e, m->rms_eps);
        const weight_t *ws[3] = {&L->wq, &L->wk, &L->wv};
        acts_prepare(b->pool, &b->acts, b->xn, n, e, ws, 3);
        float *outs[3] = {b->q, b->k, b->v};
        size_t lds[3] = {qd, kvd, kvd};
        matmul_multi(b->pool, &b->acts, ws, outs, lds, 3);
        for (size_t t = 0; t < n; t++) {
            if (L->bq) for (size_t i = 0; i < qd; i++) b->q[t * qd + i] += L->bq[i];
            if (L->bk) for (size_t i = 0; i < kvd; i++) b->k[t * kvd + i] += L->bk[i];
            if (L->bv) for (size_t i = 0; i < kvd; i++) b->v[t * kvd + i] += L->bv[i];
        }
        const float *cs = (swa && b->inv_freq_swa) ? b->cos_swa : b->cos_t;
        const float *sn = (swa && b->inv_freq_swa) ? b->sin_swa : b->sin_t;
        for (size_t t = 0; t < n; t++) {
            const float *ct = cs + t * half, *st = sn + t * half;
            for (size_t h = 0; h < m->n_head; h++) {
                float *qh = b->q + t * qd + h * hd;
                if (L->q_norm) or_rmsnorm_inplace(qh, L->q_norm, hd, m->rms_eps);
                or_rope_apply(qh, m->rope_dim, m->rope_neox, ct, st);
                for (size_t i = 0; i < hd; i++) qh[i] *= m->attn_scale;
            }
            for (size_t h = 0; h < m->n_head_kv; h++) {
                float *kh = b->k + t * kvd + h * hd;
                if (L->k_norm) or_rmsnorm_inplace(kh, L->k_norm, hd, m->rms_eps);
                or_rope_apply(kh, m->rope_dim, m->rope_neox, ct, st);
            }
        }
        cache_t *c = &b->cache[il];
        size_t rb = b->kv == OR_KV_F16 ? 0 : kv_row_bytes(b);
        for (size_t t = 0; t < n; t++) {
            size_t slot = (pos0 + t) % c->slots;
            for (size_t h = 0; h < m->n_head_kv; h++) {
                const float *ks = b->k + t * kvd + h * hd, *vs = b->v + t * kvd + h * hd;
                size_t row = h * c->slots + slot;
                if (b->kv == OR_KV_F16) {
                    or_f32_to_f16_slice(ks, c->k + row * hd, hd);
                    or_f32_to_f16_slice(vs, c->v + row * hd, hd);
                } else if (b->kv == OR_KV_Q8_0) {
                    store_q8_0(ks, c->kq + row * rb, hd);
                    store_q8_0(vs, c->vq + row * rb, hd);
                } else {
                    or_turbo_quantize(ks, hd, OR_TURBO_KV_SEED, c->kq + row * rb);
                    or_turbo_quantize(vs, hd, OR_TURBO_KV_SEED, c->vq + row * rb);
                }
            }
        }
        if (b->capture) {
            cap_store(b, 3, il, b->q, n * qd);
            cap_store(b, 4, il, b->k, n * kvd);
            cap_store(b, 5, il, b->v, n * kvd);
        }
        attctx A = {b, c, n, pos0, swa ? m->swa_window : 0};
        or_pool_for(b->pool, n * m->n_head, 1, att_task, &A);
        if (b->capture) cap_store(b, 2, il, b->att, n * qd);
        const weight_t *wo = &L->wo;
        acts_prepare(b->pool, &b->acts, b->att, n, qd, &wo, 1);
        matmul1(b->pool, &b->acts, &L->wo, b->o);
        if (L->post_attn_norm)
            for (size_t t = 0; t < n; t++) or_rmsnorm_inplace(b->o + t * e, L->post_attn_norm, e, m->rms_eps);
        residual_add(b->x, b->o, n * e, m->residual_scale);
        if (b->capture) cap_store(b, 0, il, b->x, n * e);

        par_rmsnorm(b->pool, b->xn, b->x, L->ffn_norm, n, e, m->rms_eps);
        if (L->is_moe) moe_ffn(b, &L->moe, b->xn, n, b->o, il);
        else {
            dense_ffn(b, &L->dense, b->xn, n, b->o);
            if (b->capture) cap_store(b, 6, il, b->gate, n * L->dense.gate.rows);
        }
        if (L->post_ffn_norm)
            for (size_t t = 0; t < n; t++) or_rmsnorm_inplace(b->o + t * e, L->post_ffn_norm, e, m->rms_eps);
        residual_add(b->x, b->o, n * e, m->residual_scale);
        if (b->capture) cap_store(b, 1, il, b->x, n * e);
    }
    size_t first = all_logits ? 0 : n - 1, mrows = n - first, nv = m->n_vocab;
    for (size_t t = 0; t < mrows; t++) or_rmsnorm(b->xn + t * e, b->x + (first + t) * e, m->output_norm, e, m->rms_eps);
    if (logits_len < mrows * nv) {
        set_err(err, err_len, "logits buffer too small");
        return -5;
    }
    b->hidden_rows = mrows;
    weight_t out_w = m->output.rows > nv ? slice_rows(m->output, 0, nv) : m->output;
    const weight_t *ow = &out_w;
    acts_prepare(b->pool, &b->acts, b->xn, mrows, e, &ow, 1);
    matmul1(b->pool, &b->acts, &out_w, logits);
    if (m->logit_scale != 1.0f)
        for (size_t i = 0; i < mrows * nv; i++) logits[i] /= m->logit_scale;
    if (m->has_final_softcap)
        for (size_t i = 0; i < mrows * nv; i++) logits[i] = m->final_softcap * tanhf(logits[i] / m->final_softcap);
    return 0;
}

const float *or_hidden(const or_backend *b, size_t *rows) {
    *rows = b->hidden_rows;
    return b->hidden_rows ? b->xn : NULL;
}

/* sampler.rs:199-209: first index of the strict maximum */
uint32_t or_argmax(const float *x, size_t n) {
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return (uint32_t)best;
}

static float top2_margin(const float *x, size_t n) {
    float a = -INFINITY, bb = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (x[i] > a) {
            bb = a;
            a = x[i];
        } else if (x[i] > bb) bb = x[i];
    }
    return a - bb;
}

/* eval_tokens chunking (engine.rs:250-272) from a reset cache, then eval_next
 * steps with greedy argmax as in Engine::bench (engine.rs:540-564). */
int or_greedy(or_backend *b, const uint32_t *prompt, size_t n_prompt, size_t n_batch, size_t n_gen, uint32_t *out_tokens,
              float *out_margin, float *out_logits_first, char *err, size_t err_len) {
    size_t nv = b->m->n_vocab;
    float *logits = (float *)malloc(nv * 4);
    if (n_batch == 0 || n_batch > b->max_batch) n_batch = b->max_batch;
    size_t pos = 0;
    int rc = 0;
    while (pos < n_prompt) {
        size_t end = pos + n_batch < n_prompt ? pos + n_batch : n_prompt;
        rc = or_forward(b, prompt + pos, end - pos, pos, 0, logits, nv, err, err_len);
        if (rc) goto done;
        pos = end;
    }
    if (out_logits_first) memcpy(out_logits_first, logits, nv * 4);
    for (size_t i = 0; i < n_gen; i++) {
        uint32_t tok = or_argmax(logits, nv);
        out_tokens[i] = tok;
        if (out_margin) out_margin[i] = top2_margin(logits, nv);
        rc = or_forward(b, &tok, 1, pos, 0, logits, nv, err, err_len);
        if (rc) goto done;
        pos++;
    }
done:
    free(logits);
    return rc;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int or_bench(or_backend *b, size_t n_prompt, size_t n_gen, double *pp_tps, double *tg_tps, char *err, size_t err_len) {
    size_t nv = b->m->n_vocab;
    if (n_prompt < 1) n_prompt = 1;
    uint32_t *toks = (uint32_t *)malloc(n_prompt * 4);
    for (size_t i = 0; i < n_prompt; i++) toks[i] = (uint32_t)(((uint32_t)i * 7919u + 13u) % (uint32_t)nv);
    float *logits = (float *)malloc(nv * 4);
    int rc = 0;
    size_t warm = n_prompt < 8 ? n_prompt : 8;
    for (size_t pos = 0; pos < warm; pos += b->max_batch) {
        size_t end = pos + b->max_batch < warm ? pos + b->max_batch : warm;
        if ((rc = or_forward(b, toks + pos, end - pos, pos, 0, logits, nv, err, err_len))) goto done;
    }
    double t0 = now_s();
    for (size_t pos = 0; pos < n_prompt; pos += b->max_batch) {
        size_t end = pos + b->max_batch < n_prompt ? pos + b->max_batch : n_prompt;
        if ((rc = or_forward(b, toks + pos, end - pos, pos, 0, logits, nv, err, err_len))) goto done;
    }
    double pp = now_s() - t0;
    double t1 = now_s();
    uint32_t tok = or_argmax(logits, nv);
    for (size_t i = 0; i < n_gen; i++) {
        if ((rc = or_forward(b, &tok, 1, n_prompt + i, 0, logits, nv, err, err_len))) goto done;
        tok = or_argmax(logits, nv);
    }
    double tg = now_s() - t1;
    *pp_tps = (double)n_prompt / pp;
    *tg_tps = n_gen ? (double)n_gen / tg : 0.0;
done:
    free(toks);
    free(logits);
    return rc;
}
