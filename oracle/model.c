/*
 * model.c -- restatement of the streaming transformer and the two backbone steps.
 *
 * TEST INFRASTRUCTURE ONLY (see svl_oracle.h).
 *
 *   Transformer / KvCache / Layer   SVL/nn/transformer.rs:43-551
 *   Linear dispatch (Dense | Q8_0)  SVL/nn/mod.rs:55-100
 *   LanguageModel::step (STT)       SVL/stt/model.rs:196-276
 *   Recognizer::step token feedback SVL/stt/mod.rs:551-566
 *   FlowLm::step backbone (TTS)     SVL/tts/flow_lm.rs:45-126, 162-181
 *   FlowLm::step heads (TTS)        SVL/tts/flow_lm.rs:181-185 (flow.c)
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

int svlo_attention_strided(const float* q, const float* k, const float* v, float* out, size_t b,
                           size_t h, size_t t, size_t d, size_t kvh, size_t n, size_t kv_sb,
                           size_t kv_sh, size_t kv_sr, size_t position, size_t first_key,
                           size_t context);

static __thread char g_err[512];
const char* svlo_last_error(void) { return g_err; }
static int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

/* ---- linear ------------------------------------------------------------------------- */

enum { LIN_NONE = 0, LIN_DENSE = 1, LIN_Q8_0 = 2, LIN_Q4K = 3, LIN_Q4_0 = 4 };

typedef struct {
    int kind;
    size_t out, in;
    float* w;
    svlo_block_q8_0* q8;
    svlo_block_q4k* q4;
    svlo_block_q4_0* q40;
} linear_t;

static void linear_free(linear_t* l) {
    free(l->w);
    free(l->q8);
    free(l->q4);
    free(l->q40);
    memset(l, 0, sizeof(*l));
}

/* SVL/nn/mod.rs:90-100: Dense goes through kernels::matvec row by row (the reference uses
 * candle's gemm for several rows; per-row matvec differs from it only in summation order);
 * Quantized goes through candle's QMatMul: each input row quantized to the weights' dot
 * type, then one vec_dot per output [candle hypothesis]. */
static void linear_forward(const linear_t* L, const float* x, size_t rows, float* y) {
    int threads = svlo_get_threads();
    if (L->kind == LIN_DENSE) {
        for (size_t r = 0; r < rows; ++r) svlo_matvec(x + r * L->in, L->w, NULL, y + r * L->out, L->out, L->in);
    } else if (L->kind == LIN_Q8_0) {
        size_t nb = L->in / SVLO_QK8_0;
        svlo_block_q8_0* xb = (svlo_block_q8_0*)malloc(sizeof(svlo_block_q8_0) * nb);
        for (size_t r = 0; r < rows; ++r) {
            svlo_quantize_q8_0(x + r * L->in, xb, L->in);
            float* yr = y + r * L->out;
#pragma omp parallel for schedule(static, 128) num_threads(threads)
            for (long o = 0; o < (long)L->out; ++o) yr[o] = svlo_vec_dot_q8_0(L->in, L->q8 + (size_t)o * nb, xb);
        }
        free(xb);
    } else if (L->kind == LIN_Q4_0) {
        /* BlockQ4_0's VecDotType is BlockQ8_0: the row is quantized as for Q8_0 weights */
        size_t nb = L->in / SVLO_QK8_0;
        svlo_block_q8_0* xb = (svlo_block_q8_0*)malloc(sizeof(svlo_block_q8_0) * nb);
        for (size_t r = 0; r < rows; ++r) {
            svlo_quantize_q8_0(x + r * L->in, xb, L->in);
            float* yr = y + r * L->out;
#pragma omp parallel for schedule(static, 128) num_threads(threads)
            for (long o = 0; o < (long)L->out; ++o) yr[o] = svlo_vec_dot_q4_0_q8_0(L->in, L->q40 + (size_t)o * nb, xb);
        }
        free(xb);
    } else if (L->kind == LIN_Q4K) {
        size_t nb = L->in / SVLO_QK_K;
        svlo_block_q8k* xb = (svlo_block_q8k*)malloc(sizeof(svlo_block_q8k) * nb);
        for (size_t r = 0; r < rows; ++r) {
            svlo_quantize_q8k(x + r * L->in, xb, L->in);
            float* yr = y + r * L->out;
#pragma omp parallel for schedule(static, 128) num_threads(threads)
            for (long o = 0; o < (long)L->out; ++o) yr[o] = svlo_vec_dot_q4k_q8k(L->in, L->q4 + (size_t)o * nb, xb);
        }
        free(xb);
    }
}

/* ---- tensors -------------------------------------------------------------------------- */

typedef struct {
    const svlo_tensor* t;
    size_t n;
} tensors_t;

static const svlo_tensor* find(const tensors_t* ts, const char* name) {
    for (size_t i = 0; i < ts->n; ++i)
        if (ts->t[i].name && strcmp(ts->t[i].name, name) == 0) return &ts->t[i];
    return NULL;
}

static size_t numel(const svlo_tensor* t) {
    size_t n = 1;
    for (int i = 0; i < t->ndim; ++i) n *= (size_t)t->shape[i];
    return n;
}

/* f32 copy of a dense tensor with `n` elements (as candle's VarBuilder converts to f32). */
static float* load_f32(const tensors_t* ts, const char* name, size_t n, int* rc) {
    const svlo_tensor* t = find(ts, name);
    if (!t) { *rc = fail("missing tensor %s", name); return NULL; }
    if (numel(t) != n) { *rc = fail("tensor %s: %zu elements, expected %zu", name, numel(t), n); return NULL; }
    float* out = (float*)malloc(sizeof(float) * n);
    if (t->dtype == SVLO_F32) memcpy(out, t->data, sizeof(float) * n);
    else if (t->dtype == SVLO_BF16) svlo_bf16_to_f32_n((const uint16_t*)t->data, out, n);
    else if (t->dtype == SVLO_F16) for (size_t i = 0; i < n; ++i) out[i] = svlo_f16_to_f32(((const uint16_t*)t->data)[i]);
    else { free(out); *rc = fail("tensor %s: dense dtype expected", name); return NULL; }
    return out;
}

/* SVL/nn/mod.rs:76-87 `Linear::from_weight`: quantized when asked and in % block == 0. */
static int load_linear(const tensors_t* ts, const char* name, size_t out, size_t in, int quantize, linear_t* L) {
    memset(L, 0, sizeof(*L));
    L->out = out;
    L->in = in;
    const svlo_tensor* t = find(ts, name);
    if (!t) return fail("missing tensor %s", name);
    if (t->ndim != 2 || (size_t)t->shape[0] != out || (size_t)t->shape[1] != in)
        return fail("tensor %s: shape mismatch (expected [%zu, %zu])", name, out, in);
    if (t->dtype == SVLO_Q8_0) {
        if (in % SVLO_QK8_0) return fail("tensor %s: Q8_0 needs in %% 32 == 0", name);
        size_t nb = out * in / SVLO_QK8_0;
        L->kind = LIN_Q8_0;
        L->q8 = (svlo_block_q8_0*)malloc(sizeof(svlo_block_q8_0) * nb);
        memcpy(L->q8, t->data, sizeof(svlo_block_q8_0) * nb);
        return 0;
    }
    if (t->dtype == SVLO_Q4_0) {
        if (in % SVLO_QK4_0) return fail("tensor %s: Q4_0 needs in %% 32 == 0", name);
        size_t nb = out * in / SVLO_QK4_0;
        L->kind = LIN_Q4_0;
        L->q40 = (svlo_block_q4_0*)malloc(sizeof(svlo_block_q4_0) * nb);
        memcpy(L->q40, t->data, sizeof(svlo_block_q4_0) * nb);
        return 0;
    }
    if (t->dtype == SVLO_Q4K) {
        if (in % SVLO_QK_K) return fail("tensor %s: Q4K needs in %% 256 == 0", name);
        size_t nb = out * in / SVLO_QK_K;
        L->kind = LIN_Q4K;
        L->q4 = (svlo_block_q4k*)malloc(sizeof(svlo_block_q4k) * nb);
        memcpy(L->q4, t->data, sizeof(svlo_block_q4k) * nb);
        return 0;
    }
    int rc = 0;
    float* w = load_f32(ts, name, out * in, &rc);
    if (!w) return rc;
    if (quantize == SVLO_Q8_0 && in % SVLO_QK8_0 == 0) {
        L->kind = LIN_Q8_0;
        L->q8 = (svlo_block_q8_0*)malloc(sizeof(svlo_block_q8_0) * out * in / SVLO_QK8_0);
#pragma omp parallel for schedule(static) num_threads(svlo_get_threads())
        for (long r = 0; r < (long)out; ++r) svlo_quantize_q8_0(w + r * in, L->q8 + r * (in / SVLO_QK8_0), in);
        free(w);
    } else if (quantize == SVLO_Q4_0 && in % SVLO_QK4_0 == 0) {
        L->kind = LIN_Q4_0;
        L->q40 = (svlo_block_q4_0*)malloc(sizeof(svlo_block_q4_0) * out * in / SVLO_QK4_0);
#pragma omp parallel for schedule(static) num_threads(svlo_get_threads())
        for (long r = 0; r < (long)out; ++r) svlo_quantize_q4_0(w + r * in, L->q40 + r * (in / SVLO_QK4_0), in);
        free(w);
    } else if (quantize == SVLO_Q4K && in % SVLO_QK_K == 0) {
        L->kind = LIN_Q4K;
        L->q4 = (svlo_block_q4k*)malloc(sizeof(svlo_block_q4k) * out * in / SVLO_QK_K);
#pragma omp parallel for schedule(static) num_threads(svlo_get_threads())
        for (long r = 0; r < (long)out; ++r) svlo_quantize_q4k(w + r * in, L->q4 + r * (in / SVLO_QK_K), in);
        free(w);
    } else {
        L->kind = LIN_DENSE;
        L->w = w;
    }
    return 0;
}

/* ---- model ------------------------------------------------------------------------------ */

typedef struct {
    float *n1w, *n1b, *n2w, *n2b;
    float *ls1, *ls2;
    linear_t in_proj, out_proj, ff1, ff2;
} layer_t;

struct svlo_model {
    svlo_config cfg;
    layer_t* layers;
    float* inv_freq; /* unused copy kept for inspection */
    /* STT */
    float* text_emb;
    float** emb;
    float* out_norm_w;
    float* out_norm_b;
    linear_t text_linear;
    linear_t* extra_heads; /* extra_heads_num dense [extra_heads_dim, d] */
    /* TTS */
    linear_t input_linear, z_proj;
    float* bos;
    svlo_flow* flow; /* flow head + out_eos, or NULL (flow_dim 0) */
};

const svlo_flow* svlo_model_flow(const svlo_model* m) { return m->flow; }

void svlo_model_destroy(svlo_model* m) {
    if (!m) return;
    if (m->layers) {
        for (int i = 0; i < m->cfg.num_layers; ++i) {
            layer_t* L = &m->layers[i];
            free(L->n1w); free(L->n1b); free(L->n2w); free(L->n2b); free(L->ls1); free(L->ls2);
            linear_free(&L->in_proj); linear_free(&L->out_proj); linear_free(&L->ff1); linear_free(&L->ff2);
        }
        free(m->layers);
    }
    free(m->inv_freq);
    free(m->text_emb);
    if (m->emb) {
        for (int i = 0; i < m->cfg.n_q; ++i) free(m->emb[i]);
        free(m->emb);
    }
    free(m->out_norm_w);
    free(m->out_norm_b);
    linear_free(&m->text_linear);
    if (m->extra_heads) {
        for (int i = 0; i < m->cfg.extra_heads_num; ++i) linear_free(&m->extra_heads[i]);
        free(m->extra_heads);
    }
    linear_free(&m->input_linear);
    linear_free(&m->z_proj);
    free(m->bos);
    svlo_flow_destroy(m->flow);
    free(m);
}

/* SVL/nn/transformer.rs:107-125, 204-219, 267-279, 300-316, 417-436 (tensor names and shapes). */
int svlo_model_create(const svlo_config* cfg, const svlo_tensor* tensors, size_t n, svlo_model** out) {
    *out = NULL;
    const svlo_config* c = cfg;
    if (c->d_model <= 0 || c->num_layers <= 0 || c->num_heads <= 0 || c->num_kv_heads <= 0 ||
        c->head_dim <= 0 || c->head_dim % 2 || c->num_heads % c->num_kv_heads || c->ff_hidden <= 0)
        return fail("invalid transformer config");
    tensors_t ts = {tensors, n};
    svlo_model* m = (svlo_model*)calloc(1, sizeof(svlo_model));
    m->cfg = *cfg;
    const char* pre = c->kind == SVLO_MODEL_TRANSFORMER ? "" : "transformer.";
    size_t d = (size_t)c->d_model, hd = (size_t)c->head_dim;
    size_t qdim = (size_t)c->num_heads * hd, kvdim = (size_t)c->num_kv_heads * hd;
    int rc = 0;
    char name[256];
    m->layers = (layer_t*)calloc((size_t)c->num_layers, sizeof(layer_t));
    for (int i = 0; i < c->num_layers && rc == 0; ++i) {
        layer_t* L = &m->layers[i];
#define LOADV(dst, fmtname, count)                                          \
    do {                                                                    \
        snprintf(name, sizeof(name), fmtname, pre, i);                      \
        dst = load_f32(&ts, name, count, &rc);                              \
        if (!dst) goto done;                                                \
    } while (0)
        if (c->norm_kind == SVLO_NORM_RMS) {
            LOADV(L->n1w, "%slayers.%d.norm1.alpha", d);
            LOADV(L->n2w, "%slayers.%d.norm2.alpha", d);
        } else {
            LOADV(L->n1w, "%slayers.%d.norm1.weight", d);
            LOADV(L->n1b, "%slayers.%d.norm1.bias", d);
            LOADV(L->n2w, "%slayers.%d.norm2.weight", d);
            LOADV(L->n2b, "%slayers.%d.norm2.bias", d);
        }
        if (c->layer_scale) {
            LOADV(L->ls1, "%slayers.%d.layer_scale_1.scale", d);
            LOADV(L->ls2, "%slayers.%d.layer_scale_2.scale", d);
        }
#undef LOADV
        /* in_proj_weight (moshi) or in_proj.weight (Pocket TTS), transformer.rs:304-309 */
        snprintf(name, sizeof(name), "%slayers.%d.self_attn.in_proj_weight", pre, i);
        if (!find(&ts, name)) snprintf(name, sizeof(name), "%slayers.%d.self_attn.in_proj.weight", pre, i);
        if ((rc = load_linear(&ts, name, qdim + 2 * kvdim, d, c->quantize, &L->in_proj))) goto done;
        snprintf(name, sizeof(name), "%slayers.%d.self_attn.out_proj.weight", pre, i);
        if ((rc = load_linear(&ts, name, d, qdim, c->quantize, &L->out_proj))) goto done;
        size_t F = (size_t)c->ff_hidden;
        if (c->ff_kind == SVLO_FF_GATED) {
            snprintf(name, sizeof(name), "%slayers.%d.gating.linear_in.weight", pre, i);
            if ((rc = load_linear(&ts, name, 2 * F, d, c->quantize, &L->ff1))) goto done;
            snprintf(name, sizeof(name), "%slayers.%d.gating.linear_out.weight", pre, i);
            if ((rc = load_linear(&ts, name, d, F, c->quantize, &L->ff2))) goto done;
        } else {
            snprintf(name, sizeof(name), "%slayers.%d.linear1.weight", pre, i);
            if ((rc = load_linear(&ts, name, F, d, c->quantize, &L->ff1))) goto done;
            snprintf(name, sizeof(name), "%slayers.%d.linear2.weight", pre, i);
            if ((rc = load_linear(&ts, name, d, F, c->quantize, &L->ff2))) goto done;
        }
    }
    if (rc) goto done;
    if (c->kind == SVLO_MODEL_STT) {
        /* SVL/stt/model.rs:224-231 */
        if (c->n_q <= 0 || c->card <= 0 || c->text_card <= 0) { rc = fail("invalid STT config"); goto done; }
        m->text_emb = load_f32(&ts, "text_emb.weight", (size_t)(c->text_card + 1) * d, &rc);
        if (!m->text_emb) goto done;
        m->emb = (float**)calloc((size_t)c->n_q, sizeof(float*));
        for (int i = 0; i < c->n_q; ++i) {
            snprintf(name, sizeof(name), "emb.%d.weight", i);
            m->emb[i] = load_f32(&ts, name, (size_t)(c->card + 1) * d, &rc);
            if (!m->emb[i]) goto done;
        }
        m->out_norm_w = load_f32(&ts, "out_norm.alpha", d, &rc);
        if (!m->out_norm_w) goto done;
        if ((rc = load_linear(&ts, "text_linear.weight", (size_t)c->text_card, d, c->quantize, &m->text_linear))) goto done;
        /* SVL/stt/model.rs:217-222: extra_heads.{i} are dense Linear [extra_heads_dim, d]
         * without bias, never quantized */
        if (c->extra_heads_num < 0 || (c->extra_heads_num > 0 && c->extra_heads_dim <= 0)) {
            rc = fail("invalid extra heads config");
            goto done;
        }
        if (c->extra_heads_num > 0) {
            m->extra_heads = (linear_t*)calloc((size_t)c->extra_heads_num, sizeof(linear_t));
            for (int i = 0; i < c->extra_heads_num; ++i) {
                snprintf(name, sizeof(name), "extra_heads.%d.weight", i);
                if ((rc = load_linear(&ts, name, (size_t)c->extra_heads_dim, d, 0, &m->extra_heads[i]))) goto done;
            }
        }
    } else if (c->kind == SVLO_MODEL_TTS) {
        /* SVL/tts/flow_lm.rs:72-74, 97-115: these linears are always dense (Linear::new) */
        if (c->latent_dim <= 0) { rc = fail("invalid TTS config"); goto done; }
        if ((rc = load_linear(&ts, "input_linear.weight", d, (size_t)c->latent_dim, 0, &m->input_linear))) goto done;
        m->out_norm_w = load_f32(&ts, "out_norm.weight", d, &rc);
        if (!m->out_norm_w) goto done;
        m->out_norm_b = load_f32(&ts, "out_norm.bias", d, &rc);
        if (!m->out_norm_b) goto done;
        if (c->z_dim > 0)
            if ((rc = load_linear(&ts, "z_proj.weight", (size_t)c->z_dim, d, 0, &m->z_proj))) goto done;
        m->bos = load_f32(&ts, "bos_emb", (size_t)c->latent_dim, &rc);
        if (!m->bos) goto done;
        if (c->flow_dim > 0) {
            /* SVL/tts/flow_lm.rs:107-113: the heads read z, of width z_dim or d_model */
            int cond = c->z_dim > 0 ? c->z_dim : c->d_model;
            if (svlo_flow_create(c->flow_dim, c->flow_depth, c->flow_kind, c->latent_dim, cond, tensors, n, &m->flow)) {
                rc = fail("%s", svlo_flow_last_error());
                goto done;
            }
        }
    }
done:
    if (rc) {
        svlo_model_destroy(m);
        return rc;
    }
    *out = m;
    return 0;
}

int svlo_model_linear_weight(const svlo_model* m, const char* name, float* out, size_t n) {
    const linear_t* L = NULL;
    int layer = -1;
    char which[64];
    if (strcmp(name, "text_linear") == 0) L = &m->text_linear;
    else if (strcmp(name, "input_linear") == 0) L = &m->input_linear;
    else if (sscanf(name, "%d.%63s", &layer, which) == 2 && layer >= 0 && layer < m->cfg.num_layers) {
        const layer_t* ly = &m->layers[layer];
        if (strcmp(which, "in_proj") == 0) L = &ly->in_proj;
        else if (strcmp(which, "out_proj") == 0) L = &ly->out_proj;
        else if (strcmp(which, "ff1") == 0) L = &ly->ff1;
        else if (strcmp(which, "ff2") == 0) L = &ly->ff2;
    }
    if (!L || L->kind == LIN_NONE) return fail("unknown linear %s", name);
    if (n != L->out * L->in) return fail("size mismatch");
    if (L->kind == LIN_DENSE) memcpy(out, L->w, sizeof(float) * n);
    else if (L->kind == LIN_Q8_0) svlo_dequantize_q8_0(L->q8, out, n);
    else if (L->kind == LIN_Q4_0) svlo_dequantize_q4_0(L->q40, out, n);
    else svlo_dequantize_q4k(L->q4, out, n);
    return 0;
}

/* ---- KV cache: SVL/nn/transformer.rs:467-551 ----------------------------------------- */

typedef struct {
    float *k, *v; /* [b][kvh][cap][hd] */
    size_t cap, len, start;
} kvcache_t;

struct svlo_state {
    const svlo_model* m;
    int32_t b;
    kvcache_t* caches;
    int64_t position;
};

svlo_state* svlo_state_create(const svlo_model* m, int32_t batch) {
    svlo_state* s = (svlo_state*)calloc(1, sizeof(svlo_state));
    s->m = m;
    s->b = batch > 0 ? batch : 1;
    s->caches = (kvcache_t*)calloc((size_t)m->cfg.num_layers, sizeof(kvcache_t));
    return s;
}

void svlo_state_destroy(svlo_state* s) {
    if (!s) return;
    for (int i = 0; i < s->m->cfg.num_layers; ++i) {
        free(s->caches[i].k);
        free(s->caches[i].v);
    }
    free(s->caches);
    free(s);
}

svlo_state* svlo_state_duplicate(const svlo_state* s) {
    svlo_state* c = svlo_state_create(s->m, s->b);
    c->position = s->position;
    size_t kvh = (size_t)s->m->cfg.num_kv_heads, hd = (size_t)s->m->cfg.head_dim;
    for (int i = 0; i < s->m->cfg.num_layers; ++i) {
        c->caches[i] = s->caches[i];
        if (s->caches[i].k) {
            size_t bytes = sizeof(float) * (size_t)s->b * kvh * s->caches[i].cap * hd;
            c->caches[i].k = (float*)malloc(bytes);
            c->caches[i].v = (float*)malloc(bytes);
            memcpy(c->caches[i].k, s->caches[i].k, bytes);
            memcpy(c->caches[i].v, s->caches[i].v, bytes);
        }
    }
    return c;
}

int64_t svlo_state_position(const svlo_state* s) { return s->position; }

/* KvCache::append: k_new, v_new [b][kvh][t][hd].  Returns the visible view (offset into the
 * buffers, count) and the absolute position of its first key. */
static void kv_append(kvcache_t* c, const float* kn, const float* vn, size_t b, size_t kvh, size_t t,
                      size_t hd, size_t window, size_t* off, size_t* count, size_t* first_key) {
    if (c->len + t > c->cap) {
        size_t keep = window ? (c->len < window ? c->len : window) : c->len;
        size_t drop = c->len - keep;
        size_t ncap;
        if (window) ncap = 2 * window + t;
        else {
            ncap = 2 * c->cap;
            if (ncap < keep + t) ncap = keep + t;
            if (ncap < 64) ncap = 64;
        }
        float* nk = (float*)calloc(b * kvh * ncap * hd, sizeof(float));
        float* nv = (float*)calloc(b * kvh * ncap * hd, sizeof(float));
        if (c->k && keep > 0) {
            for (size_t m = 0; m < b * kvh; ++m) {
                memcpy(nk + m * ncap * hd, c->k + (m * c->cap + drop) * hd, sizeof(float) * keep * hd);
                memcpy(nv + m * ncap * hd, c->v + (m * c->cap + drop) * hd, sizeof(float) * keep * hd);
            }
        }
        free(c->k);
        free(c->v);
        c->k = nk;
        c->v = nv;
        c->cap = ncap;
        c->start += drop;
        c->len = keep;
    }
    for (size_t m = 0; m < b * kvh; ++m) {
        memcpy(c->k + (m * c->cap + c->len) * hd, kn + m * t * hd, sizeof(float) * t * hd);
        memcpy(c->v + (m * c->cap + c->len) * hd, vn + m * t * hd, sizeof(float) * t * hd);
    }
    c->len += t;
    size_t visible = window ? (c->len < window + t - 1 ? c->len : window + t - 1) : c->len;
    *off = c->len - visible;
    *count = visible;
    *first_key = c->start + *off;
}

int svlo_state_cache_info(const svlo_state* s, int layer, int64_t* len, int64_t* start) {
    if (layer < 0 || layer >= s->m->cfg.num_layers) return fail("layer out of range");
    *len = (int64_t)s->caches[layer].len;
    *start = (int64_t)s->caches[layer].start;
    return 0;
}

int svlo_state_cache_copy(const svlo_state* s, int layer, float* k, float* v) {
    if (layer < 0 || layer >= s->m->cfg.num_layers) return fail("layer out of range");
    const kvcache_t* c = &s->caches[layer];
    size_t hd = (size_t)s->m->cfg.head_dim, kvh = (size_t)s->m->cfg.num_kv_heads;
    for (size_t m = 0; m < (size_t)s->b * kvh; ++m) {
        memcpy(k + m * c->len * hd, c->k + m * c->cap * hd, sizeof(float) * c->len * hd);
        memcpy(v + m * c->len * hd, c->v + m * c->cap * hd, sizeof(float) * c->len * hd);
    }
    return 0;
}

/* TransformerState::from_layer_caches, SVL/nn/transformer.rs:81-103. */
svlo_state* svlo_state_from_layer_caches(const svlo_model* m, int32_t batch, int64_t len,
                                         const float* const* ks, const float* const* vs) {
    svlo_state* s = svlo_state_create(m, batch);
    size_t kvh = (size_t)m->cfg.num_kv_heads, hd = (size_t)m->cfg.head_dim;
    size_t window = m->cfg.context > 0 ? (size_t)m->cfg.context : 0;
    for (int i = 0; i < m->cfg.num_layers; ++i) {
        size_t off, cnt, fk;
        if (len > 0) kv_append(&s->caches[i], ks[i], vs[i], (size_t)s->b, kvh, (size_t)len, hd, window, &off, &cnt, &fk);
    }
    s->position = len;
    return s;
}

/* ---- forward ----------------------------------------------------------------------------- */

static void norm_rows(const svlo_model* m, const float* w, const float* b, const float* x, float* y, size_t rows) {
    size_t d = (size_t)m->cfg.d_model;
    if (m->cfg.norm_kind == SVLO_NORM_RMS) svlo_rms_norm(x, w, y, rows, d, m->cfg.norm_eps);
    else svlo_layer_norm(x, w, b, y, rows, d, m->cfg.norm_eps);
}

/* Layer::forward, SVL/nn/transformer.rs:222-250, with Attention::forward :318-345 and
 * FeedForwardLayer::forward :438-464.  x is [b][t][d], updated in place. */
static int layer_forward(const svlo_model* m, const layer_t* L, kvcache_t* cache, float* x, size_t b,
                         size_t t, const float* cos_t, const float* sin_t, size_t position) {
    const svlo_config* c = &m->cfg;
    size_t d = (size_t)c->d_model, H = (size_t)c->num_heads, KVH = (size_t)c->num_kv_heads, hd = (size_t)c->head_dim;
    size_t rows = b * t, qkvw = (H + 2 * KVH) * hd;
    size_t window = c->context > 0 ? (size_t)c->context : 0;
    float* h = (float*)malloc(sizeof(float) * rows * d);
    float* qkv = (float*)malloc(sizeof(float) * rows * qkvw);
    float* q = (float*)malloc(sizeof(float) * b * H * t * hd);
    float* kn = (float*)malloc(sizeof(float) * b * KVH * t * hd);
    float* vn = (float*)malloc(sizeof(float) * b * KVH * t * hd);
    float* att = (float*)malloc(sizeof(float) * rows * H * hd);
    float* upd = (float*)malloc(sizeof(float) * rows * d);
    norm_rows(m, L->n1w, L->n1b, x, h, rows);
    linear_forward(&L->in_proj, h, rows, qkv);
    /* split: q heads, then k heads, then v heads (transformer.rs:330-338) */
    for (size_t bi = 0; bi < b; ++bi)
        for (size_t ti = 0; ti < t; ++ti) {
            const float* r = qkv + (bi * t + ti) * qkvw;
            for (size_t hh = 0; hh < H; ++hh)
                memcpy(q + ((bi * H + hh) * t + ti) * hd, r + hh * hd, sizeof(float) * hd);
            for (size_t hh = 0; hh < KVH; ++hh) {
                memcpy(kn + ((bi * KVH + hh) * t + ti) * hd, r + (H + hh) * hd, sizeof(float) * hd);
                memcpy(vn + ((bi * KVH + hh) * t + ti) * hd, r + (H + KVH + hh) * hd, sizeof(float) * hd);
            }
        }
    svlo_rope_i(q, cos_t, sin_t, b * H, t, hd);
    svlo_rope_i(kn, cos_t, sin_t, b * KVH, t, hd);
    size_t off, count, first_key;
    kv_append(cache, kn, vn, b, KVH, t, hd, window, &off, &count, &first_key);
    if (svlo_attention_strided(q, cache->k + off * hd, cache->v + off * hd, att, b, H, t, hd, KVH, count,
                               KVH * cache->cap * hd, cache->cap * hd, hd, position, first_key, window))
        return fail("attention: shape error");
    linear_forward(&L->out_proj, att, rows, upd);
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < d; ++i) {
            float u = upd[r * d + i];
            if (L->ls1) u = u * L->ls1[i];
            x[r * d + i] = x[r * d + i] + u;
        }
    norm_rows(m, L->n2w, L->n2b, x, h, rows);
    size_t F = (size_t)c->ff_hidden;
    if (c->ff_kind == SVLO_FF_GATED) {
        float* hid = (float*)malloc(sizeof(float) * rows * 2 * F);
        float* prod = (float*)malloc(sizeof(float) * rows * F);
        linear_forward(&L->ff1, h, rows, hid);
        for (size_t r = 0; r < rows; ++r)
            for (size_t j = 0; j < F; ++j) {
                float g = svlo_silu(hid[r * 2 * F + j]);
                prod[r * F + j] = g * hid[r * 2 * F + F + j];
            }
        linear_forward(&L->ff2, prod, rows, upd);
        free(hid);
        free(prod);
    } else {
        float* hid = (float*)malloc(sizeof(float) * rows * F);
        linear_forward(&L->ff1, h, rows, hid);
        if (c->ff_kind == SVLO_FF_PLAIN_ERF) {
            for (size_t j = 0; j < rows * F; ++j) hid[j] = svlo_gelu_erf(hid[j]);
        } else {
            svlo_gelu_tanh_n(hid, rows * F);
        }
        linear_forward(&L->ff2, hid, rows, upd);
        free(hid);
    }
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < d; ++i) {
            float u = upd[r * d + i];
            if (L->ls2) u = u * L->ls2[i];
            x[r * d + i] = x[r * d + i] + u;
        }
    free(h); free(qkv); free(q); free(kn); free(vn); free(att); free(upd);
    return 0;
}

/* Transformer::forward_block, SVL/nn/transformer.rs:156-186.  xs [b][t][d] in place. */
static int forward_block(const svlo_model* m, svlo_state* s, float* xs, size_t t) {
    if (t == 0) return 0;
    size_t hd = (size_t)m->cfg.head_dim;
    float* cs = (float*)malloc(sizeof(float) * t * hd / 2);
    float* sn = (float*)malloc(sizeof(float) * t * hd / 2);
    svlo_rope_tables((size_t)s->position, t, hd, m->cfg.max_period, cs, sn);
    int rc = 0;
    for (int i = 0; i < m->cfg.num_layers && rc == 0; ++i)
        rc = layer_forward(m, &m->layers[i], &s->caches[i], xs, (size_t)s->b, t, cs, sn, (size_t)s->position);
    free(cs);
    free(sn);
    if (rc == 0) s->position += (int64_t)t;
    return rc;
}

/* Transformer::forward, SVL/nn/transformer.rs:139-154: blocks of `context` steps. */
int svlo_transformer_forward(const svlo_model* m, svlo_state* s, const float* xs, int64_t t, float* ys) {
    size_t b = (size_t)s->b, d = (size_t)m->cfg.d_model, T = (size_t)t;
    size_t blk = (m->cfg.context > 0 && T > (size_t)m->cfg.context) ? (size_t)m->cfg.context : T;
    if (T == 0) return 0;
    float* buf = (float*)malloc(sizeof(float) * b * blk * d);
    for (size_t start = 0; start < T; start += blk) {
        size_t len = T - start < blk ? T - start : blk;
        for (size_t bi = 0; bi < b; ++bi) memcpy(buf + bi * len * d, xs + (bi * T + start) * d, sizeof(float) * len * d);
        int rc = forward_block(m, s, buf, len);
        if (rc) { free(buf); return rc; }
        for (size_t bi = 0; bi < b; ++bi) memcpy(ys + (bi * T + start) * d, buf + bi * len * d, sizeof(float) * len * d);
    }
    free(buf);
    return 0;
}

/* LanguageModel::step, SVL/stt/model.rs:239-276. */
int svlo_stt_step(const svlo_model* m, svlo_state* s, uint32_t text_token, const uint32_t* audio,
                  uint32_t* out_token, float* out_logits, float* out_probs) {
    const svlo_config* c = &m->cfg;
    if (c->kind != SVLO_MODEL_STT) return fail("not an STT model");
    if (s->b != 1) return fail("stt_step: batch 1 only");
    if (text_token > (uint32_t)c->text_card) return fail("text token %u out of range", text_token);
    size_t d = (size_t)c->d_model;
    float* x = (float*)malloc(sizeof(float) * d);
    float* y = (float*)malloc(sizeof(float) * d);
    float* logits = (float*)malloc(sizeof(float) * (size_t)c->text_card);
    memcpy(x, m->text_emb + (size_t)text_token * d, sizeof(float) * d);
    for (int i = 0; i < c->n_q; ++i) {
        if (audio[i] > (uint32_t)c->card) {
            free(x); free(y); free(logits);
            return fail("audio token %u out of range", audio[i]);
        }
        const float* e = m->emb[i] + (size_t)audio[i] * d;
        for (size_t j = 0; j < d; ++j) x[j] = x[j] + e[j];
    }
    int rc = svlo_transformer_forward(m, s, x, 1, y);
    if (rc == 0) {
        svlo_rms_norm(y, m->out_norm_w, x, 1, d, 1e-8f);
        linear_forward(&m->text_linear, x, 1, logits);
        *out_token = svlo_argmax(logits, (size_t)c->text_card);
        if (out_logits) memcpy(out_logits, logits, sizeof(float) * (size_t)c->text_card);
        /* SVL/stt/model.rs:259-271: per extra head, softmax of its logits, probability 0 */
        if (out_probs && c->extra_heads_num > 0) {
            float* hl = (float*)malloc(sizeof(float) * (size_t)c->extra_heads_dim);
            for (int h = 0; h < c->extra_heads_num; ++h) {
                linear_forward(&m->extra_heads[h], x, 1, hl);
                out_probs[h] = svlo_softmax_first(hl, (size_t)c->extra_heads_dim);
            }
            free(hl);
        }
    }
    free(x); free(y); free(logits);
    return rc;
}

/* Recognizer::step token feedback, SVL/stt/mod.rs:551-566. */
int svlo_stt_greedy(const svlo_model* m, svlo_state* s, int64_t n, const uint32_t* audio,
                    uint32_t* out_tokens, float* out_last_logits, float* out_probs) {
    const svlo_config* c = &m->cfg;
    uint32_t* initial = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)c->n_q);
    for (int i = 0; i < c->n_q; ++i) initial[i] = (uint32_t)c->card;
    uint32_t text = (uint32_t)c->text_card;
    int rc = 0;
    for (int64_t i = 0; i < n && rc == 0; ++i) {
        const uint32_t* a = (s->position == 0) ? initial : audio + (size_t)i * (size_t)c->n_q;
        uint32_t tok = 0;
        rc = svlo_stt_step(m, s, text, a, &tok, (i == n - 1) ? out_last_logits : NULL,
                           out_probs ? out_probs + (size_t)i * (size_t)c->extra_heads_num : NULL);
        out_tokens[i] = tok;
        text = tok;
    }
    free(initial);
    return rc;
}

/* FlowLm::step backbone part, SVL/tts/flow_lm.rs:169-180. */
int svlo_tts_backbone_step(const svlo_model* m, svlo_state* s, const float* latent, float* out_z) {
    const svlo_config* c = &m->cfg;
    if (c->kind != SVLO_MODEL_TTS) return fail("not a TTS model");
    if (s->b != 1) return fail("tts step: batch 1 only");
    size_t d = (size_t)c->d_model;
    float* x = (float*)malloc(sizeof(float) * d);
    float* y = (float*)malloc(sizeof(float) * d);
    linear_forward(&m->input_linear, latent ? latent : m->bos, 1, x);
    int rc = svlo_transformer_forward(m, s, x, 1, y);
    if (rc == 0) {
        svlo_layer_norm(y, m->out_norm_w, m->out_norm_b, x, 1, d, 1e-5f);
        if (c->z_dim > 0) linear_forward(&m->z_proj, x, 1, out_z);
        else memcpy(out_z, x, sizeof(float) * d);
    }
    free(x);
    free(y);
    return rc;
}

/* FlowLm::step (SVL/tts/flow_lm.rs:162-185) after the sampler's noise draw (:187-203, the
 * caller's): the backbone's z, the end-of-speech logit of out_eos(z), the flow head's decode
 * of the noise conditioned on z. */
int svlo_tts_step(const svlo_model* m, svlo_state* s, const float* latent, const float* noise, int decode_steps,
                  float* out_latent, float* out_eos_logit) {
    if (!m->flow) return fail("the model has no flow head");
    const svlo_config* c = &m->cfg;
    size_t zd = (size_t)(c->z_dim > 0 ? c->z_dim : c->d_model);
    float* z = (float*)malloc(sizeof(float) * zd);
    int rc = svlo_tts_backbone_step(m, s, latent, z);
    if (rc == 0) {
        if (out_eos_logit) *out_eos_logit = svlo_flow_eos_logit(m->flow, z);
        svlo_flow_decode(m->flow, z, noise, decode_steps, out_latent);
    }
    free(z);
    return rc;
}
