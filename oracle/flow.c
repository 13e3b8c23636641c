/*
 * flow.c -- restatement of Pocket TTS's flow head and end-of-speech head, the part of
 * FlowLm::step after the backbone (SVL/tts/flow_lm.rs:181-184, 206-387).
 *
 * TEST INFRASTRUCTURE ONLY (see svl_oracle.h).  Batch 1, f32, the reference's CPU path:
 *   * every Linear is a single f32 row through the reference's matvec (`dot` + bias,
 *     SVL/nn/mod.rs:90-100, SVL/nn/kernels/matvec.rs:174-202) -> svlo_matvec;
 *   * SiLU is the reference's own kernel (SVL/nn/kernels/activation.rs:70-74) -> svlo_silu;
 *   * candle_nn::ops::layer_norm (ResBlock's in_ln) -> svlo_layer_norm;
 *   * the other norms are composed of candle tensor ops, restated op for op
 *     [candle hypothesis]: `sum_keepdim` adds the row in index order with one f32
 *     accumulator (the scalar CPU reduction); `t * c`, `t / c`, `t + c` with an f64 constant
 *     are candle's affine `v * (f32)mul + (f32)add` (Div by c multiplies by (f32)(1 / c));
 *     `mean_keepdim` is the sum times (f32)(1 / n); `sqrt` and `recip` are the correctly rounded
 *     f32 operations; cos / sin are the C library's cosf / sinf (Rust's f32::cos / f32::sin
 *     call the platform libm).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

struct svlo_flow {
    int dim, depth, kind, latent, cond, n_time;
    /* TimestepEmbedder (flow_lm.rs:313-349) per time condition */
    float *freqs[2], *t1w[2], *t1b[2], *t2w[2], *t2b[2], *talpha[2];
    float *cw, *cb;   /* cond_embed [dim][cond] */
    float *iw, *ib;   /* input_proj [dim][latent] */
    float **lnw, **lnb, **m1w, **m1b, **m2w, **m2b, **mw, **mb; /* ResBlock j (flow_lm.rs:351-387) */
    float *fmw, *fmb; /* final_layer.adaLN_modulation.1 [2 dim][dim] */
    float *flw, *flb; /* final_layer.linear [latent][dim] */
    float *ew, *eb;   /* out_eos [1][cond], [1] (flow_lm.rs:109-112) */
};

static char g_flow_err[256];
const char* svlo_flow_last_error(void) { return g_flow_err; }

static const svlo_tensor* ffind(const svlo_tensor* ts, size_t n, const char* name) {
    for (size_t i = 0; i < n; ++i)
        if (ts[i].name && strcmp(ts[i].name, name) == 0) return &ts[i];
    return NULL;
}

/* f32 copy of a dense tensor of `count` elements (VarBuilder::get converts to f32). */
static float* fload(const svlo_tensor* ts, size_t n, const char* name, size_t count, int* rc) {
    if (*rc) return NULL;
    const svlo_tensor* t = ffind(ts, n, name);
    size_t have = 1;
    if (t)
        for (int i = 0; i < t->ndim; ++i) have *= (size_t)t->shape[i];
    if (!t || have != count) {
        snprintf(g_flow_err, sizeof(g_flow_err), t ? "tensor %s: %zu elements, expected %zu" : "missing tensor %s",
                 name, have, count);
        *rc = -1;
        return NULL;
    }
    float* out = (float*)malloc(sizeof(float) * count);
    if (t->dtype == SVLO_F32) memcpy(out, t->data, sizeof(float) * count);
    else if (t->dtype == SVLO_BF16) svlo_bf16_to_f32_n((const uint16_t*)t->data, out, count);
    else if (t->dtype == SVLO_F16) for (size_t i = 0; i < count; ++i) out[i] = svlo_f16_to_f32(((const uint16_t*)t->data)[i]);
    else {
        free(out);
        snprintf(g_flow_err, sizeof(g_flow_err), "tensor %s: dense dtype expected", name);
        *rc = -1;
        return NULL;
    }
    return out;
}

/* FlowKind::num_time_conditions (SVL/tts/config.rs:187-195). */
static int time_conditions(int kind) {
    return kind == SVLO_FLOW_LSD ? 2 : (kind == SVLO_FLOW_MATCHING ? 1 : 0);
}

void svlo_flow_destroy(svlo_flow* f) {
    if (!f) return;
    for (int i = 0; i < 2; ++i) {
        free(f->freqs[i]); free(f->t1w[i]); free(f->t1b[i]); free(f->t2w[i]); free(f->t2b[i]); free(f->talpha[i]);
    }
    free(f->cw); free(f->cb); free(f->iw); free(f->ib);
    for (int j = 0; j < f->depth; ++j) {
        if (f->lnw) free(f->lnw[j]);
        if (f->lnb) free(f->lnb[j]);
        if (f->m1w) free(f->m1w[j]);
        if (f->m1b) free(f->m1b[j]);
        if (f->m2w) free(f->m2w[j]);
        if (f->m2b) free(f->m2b[j]);
        if (f->mw) free(f->mw[j]);
        if (f->mb) free(f->mb[j]);
    }
    free(f->lnw); free(f->lnb); free(f->m1w); free(f->m1b); free(f->m2w); free(f->m2b); free(f->mw); free(f->mb);
    free(f->fmw); free(f->fmb); free(f->flw); free(f->flb); free(f->ew); free(f->eb);
    free(f);
}

/* FlowHead::new (flow_lm.rs:232-251), TimestepEmbedder::new (:322-331), ResBlock::new
 * (:359-368) and out_eos (:109-112): tensor names under "flow_net." and "out_eos.". */
int svlo_flow_create(int dim, int depth, int kind, int latent, int cond, const svlo_tensor* ts, size_t n,
                     svlo_flow** out) {
    *out = NULL;
    if (dim <= 0 || depth < 0 || latent <= 0 || cond <= 0 || kind < 0 || kind > SVLO_FLOW_POINTWISE) {
        snprintf(g_flow_err, sizeof(g_flow_err), "invalid flow head config");
        return -1;
    }
    svlo_flow* f = (svlo_flow*)calloc(1, sizeof(svlo_flow));
    f->dim = dim;
    f->depth = depth;
    f->kind = kind;
    f->latent = latent;
    f->cond = cond;
    f->n_time = time_conditions(kind);
    const size_t D = (size_t)dim;
    int rc = 0;
    char nm[160];
    for (int i = 0; i < f->n_time; ++i) {
        snprintf(nm, sizeof nm, "flow_net.time_embed.%d.freqs", i);
        f->freqs[i] = fload(ts, n, nm, 128, &rc);
        snprintf(nm, sizeof nm, "flow_net.time_embed.%d.mlp.0.weight", i);
        f->t1w[i] = fload(ts, n, nm, D * 256, &rc);
        snprintf(nm, sizeof nm, "flow_net.time_embed.%d.mlp.0.bias", i);
        f->t1b[i] = fload(ts, n, nm, D, &rc);
        snprintf(nm, sizeof nm, "flow_net.time_embed.%d.mlp.2.weight", i);
        f->t2w[i] = fload(ts, n, nm, D * D, &rc);
        snprintf(nm, sizeof nm, "flow_net.time_embed.%d.mlp.2.bias", i);
        f->t2b[i] = fload(ts, n, nm, D, &rc);
        snprintf(nm, sizeof nm, "flow_net.time_embed.%d.mlp.3.alpha", i);
        f->talpha[i] = fload(ts, n, nm, D, &rc);
    }
    f->cw = fload(ts, n, "flow_net.cond_embed.weight", D * cond, &rc);
    f->cb = fload(ts, n, "flow_net.cond_embed.bias", D, &rc);
    f->iw = fload(ts, n, "flow_net.input_proj.weight", D * latent, &rc);
    f->ib = fload(ts, n, "flow_net.input_proj.bias", D, &rc);
    f->lnw = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->lnb = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->m1w = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->m1b = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->m2w = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->m2b = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->mw = (float**)calloc((size_t)depth + 1, sizeof(float*));
    f->mb = (float**)calloc((size_t)depth + 1, sizeof(float*));
    for (int j = 0; j < depth; ++j) {
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.in_ln.weight", j);
        f->lnw[j] = fload(ts, n, nm, D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.in_ln.bias", j);
        f->lnb[j] = fload(ts, n, nm, D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.mlp.0.weight", j);
        f->m1w[j] = fload(ts, n, nm, D * D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.mlp.0.bias", j);
        f->m1b[j] = fload(ts, n, nm, D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.mlp.2.weight", j);
        f->m2w[j] = fload(ts, n, nm, D * D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.mlp.2.bias", j);
        f->m2b[j] = fload(ts, n, nm, D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.adaLN_modulation.1.weight", j);
        f->mw[j] = fload(ts, n, nm, 3 * D * D, &rc);
        snprintf(nm, sizeof nm, "flow_net.res_blocks.%d.adaLN_modulation.1.bias", j);
        f->mb[j] = fload(ts, n, nm, 3 * D, &rc);
    }
    f->fmw = fload(ts, n, "flow_net.final_layer.adaLN_modulation.1.weight", 2 * D * D, &rc);
    f->fmb = fload(ts, n, "flow_net.final_layer.adaLN_modulation.1.bias", 2 * D, &rc);
    f->flw = fload(ts, n, "flow_net.final_layer.linear.weight", (size_t)latent * D, &rc);
    f->flb = fload(ts, n, "flow_net.final_layer.linear.bias", (size_t)latent, &rc);
    f->ew = fload(ts, n, "out_eos.weight", (size_t)cond, &rc);
    f->eb = fload(ts, n, "out_eos.bias", 1, &rc);
    if (rc) {
        svlo_flow_destroy(f);
        return rc;
    }
    *out = f;
    return 0;
}

/* Sum of x[0..n) with one f32 accumulator, index order (candle's scalar CPU sum_keepdim)
 * [candle hypothesis]. */
static float seq_sum(const float* x, size_t n) {
    float acc = 0.0f;
    for (size_t i = 0; i < n; ++i) acc += x[i];
    return acc;
}

/* candle affine `v * mul + add` in f32. */
static inline float affine(float v, float mul, float add) {
    float p = v * mul;
    return p + add;
}

/* TimestepEmbedder::forward (flow_lm.rs:333-348): args = freqs * t; [cos(args), sin(args)];
 * linear2(silu(linear1(.))); then the "RMSNorm" that divides by the unbiased variance:
 * xs * recip(sqrt(sum((xs - mean)^2) / (n - 1) + 1e-5)) * alpha. */
void svlo_flow_time_embed(const svlo_flow* f, int i, float t, float* out) {
    const size_t D = (size_t)f->dim;
    float emb[256];
    for (int k = 0; k < 128; ++k) {
        float a = affine(f->freqs[i][k], t, 0.0f);
        emb[k] = cosf(a);
        emb[128 + k] = sinf(a);
    }
    float* h = (float*)malloc(sizeof(float) * D);
    float* c = (float*)malloc(sizeof(float) * D);
    svlo_matvec(emb, f->t1w[i], f->t1b[i], h, D, 256);
    svlo_silu_n(h, D);
    svlo_matvec(h, f->t2w[i], f->t2b[i], out, D, D);
    const double n = (double)D;
    float mean = affine(seq_sum(out, D), (float)(1.0 / n), 0.0f);
    for (size_t k = 0; k < D; ++k) {
        float v = out[k] - mean;
        c[k] = v * v;
    }
    float var = affine(seq_sum(c, D), (float)(1.0 / (n - 1.0)), 0.0f);
    float r = 1.0f / sqrtf(affine(var, 1.0f, 1e-5f));
    for (size_t k = 0; k < D; ++k) {
        float v = out[k] * r;
        out[k] = v * f->talpha[i][k];
    }
    free(h);
    free(c);
}

/* The time conditioning FlowHead::forward adds to the condition (flow_lm.rs:256-266): the
 * embeddings summed in order, divided by their count. */
void svlo_flow_time_mean(const svlo_flow* f, const float* times, float* out) {
    const size_t D = (size_t)f->dim;
    float* e = (float*)malloc(sizeof(float) * D);
    for (int i = 0; i < f->n_time; ++i) {
        svlo_flow_time_embed(f, i, times[i], i == 0 ? out : e);
        if (i > 0)
            for (size_t k = 0; k < D; ++k) out[k] = out[k] + e[k];
    }
    const float inv = (float)(1.0 / (double)f->n_time);
    for (size_t k = 0; k < D; ++k) out[k] = affine(out[k], inv, 0.0f);
    free(e);
}

/* layer_norm_no_affine (flow_lm.rs:220-225): (xs - mean) / sqrt(mean((xs - mean)^2) + eps). */
static void layer_norm_no_affine(const float* x, float* y, size_t n, float eps) {
    float mean = affine(seq_sum(x, n), (float)(1.0 / (double)n), 0.0f);
    float* sq = (float*)malloc(sizeof(float) * n);
    for (size_t k = 0; k < n; ++k) {
        float v = x[k] - mean;
        y[k] = v;
        sq[k] = v * v;
    }
    float var = affine(seq_sum(sq, n), (float)(1.0 / (double)n), 0.0f);
    float s = sqrtf(affine(var, 1.0f, eps));
    for (size_t k = 0; k < n; ++k) y[k] = y[k] / s;
    free(sq);
}

/* modulate (flow_lm.rs:227-230): x * (1 + scale) + shift, with `scale + 1.0` an affine. */
static void modulate(float* x, const float* shift, const float* scale, size_t n) {
    for (size_t k = 0; k < n; ++k) {
        float s1 = affine(scale[k], 1.0f, 1.0f);
        float v = x[k] * s1;
        x[k] = v + shift[k];
    }
}

/* FlowHead::forward (flow_lm.rs:253-283) for the condition `cond` [cond], the flow times and
 * the sample xs [latent] -> out [latent].  `tmean` (the time conditioning of `times`) may be
 * given precomputed; NULL computes it. */
void svlo_flow_forward(const svlo_flow* f, const float* cond, const float* times, const float* tmean,
                       const float* xs, float* out) {
    const size_t D = (size_t)f->dim;
    float* y = (float*)malloc(sizeof(float) * D);
    float* sy = (float*)malloc(sizeof(float) * D);
    float* h = (float*)malloc(sizeof(float) * D);
    float* a = (float*)malloc(sizeof(float) * D);
    float* g = (float*)malloc(sizeof(float) * D);
    float* hn = (float*)malloc(sizeof(float) * D);
    float* m = (float*)malloc(sizeof(float) * 3 * D);
    svlo_matvec(cond, f->cw, f->cb, y, D, (size_t)f->cond);
    if (f->n_time > 0) {
        float* t = (float*)malloc(sizeof(float) * D);
        if (tmean) memcpy(t, tmean, sizeof(float) * D);
        else svlo_flow_time_mean(f, times, t);
        for (size_t k = 0; k < D; ++k) y[k] = y[k] + t[k];
        free(t);
    }
    for (size_t k = 0; k < D; ++k) sy[k] = svlo_silu(y[k]);
    svlo_matvec(xs, f->iw, f->ib, h, D, (size_t)f->latent);
    for (int j = 0; j < f->depth; ++j) {
        /* ResBlock::forward (flow_lm.rs:370-386): chunk(3) = shift, scale, gate */
        svlo_matvec(sy, f->mw[j], f->mb[j], m, 3 * D, D);
        svlo_layer_norm(h, f->lnw[j], f->lnb[j], hn, 1, D, 1e-6f);
        modulate(hn, m, m + D, D);
        svlo_matvec(hn, f->m1w[j], f->m1b[j], a, D, D);
        svlo_silu_n(a, D);
        svlo_matvec(a, f->m2w[j], f->m2b[j], g, D, D);
        for (size_t k = 0; k < D; ++k) {
            float v = m[2 * D + k] * g[k];
            h[k] = h[k] + v;
        }
    }
    /* final layer: chunk(2) = shift, scale */
    svlo_matvec(sy, f->fmw, f->fmb, m, 2 * D, D);
    layer_norm_no_affine(h, hn, D, 1e-6f);
    modulate(hn, m, m + D, D);
    svlo_matvec(hn, f->flw, f->flb, out, (size_t)f->latent, D);
    free(y); free(sy); free(h); free(a); free(g); free(hn); free(m);
}

/* FlowHead::decode (flow_lm.rs:286-309): noise [latent] -> latent [latent]. */
void svlo_flow_decode(const svlo_flow* f, const float* cond, const float* noise, int steps, float* out) {
    const size_t L = (size_t)f->latent;
    if (steps < 1) steps = 1;
    float* flow = (float*)malloc(sizeof(float) * L);
    if (f->kind == SVLO_FLOW_LSD || f->kind == SVLO_FLOW_MATCHING) {
        memcpy(out, noise, sizeof(float) * L);
        const float inv = (float)(1.0 / (double)steps);
        for (int i = 0; i < steps; ++i) {
            float times[2];
            if (f->kind == SVLO_FLOW_LSD) {
                times[0] = (float)i / (float)steps;
                times[1] = (float)(i + 1) / (float)steps;
            } else {
                times[0] = (float)i / (float)steps;
            }
            svlo_flow_forward(f, cond, times, NULL, out, flow);
            for (size_t k = 0; k < L; ++k) out[k] = out[k] + affine(flow[k], inv, 0.0f);
        }
    } else if (f->kind == SVLO_FLOW_DRIFTING) {
        svlo_flow_forward(f, cond, NULL, NULL, noise, out);
    } else {
        svlo_flow_forward(f, cond, NULL, NULL, noise, flow);
        for (size_t k = 0; k < L; ++k) out[k] = noise[k] + flow[k];
    }
    free(flow);
}

/* out_eos (flow_lm.rs:181): Linear with bias over z [cond]. */
float svlo_flow_eos_logit(const svlo_flow* f, const float* z) {
    float y;
    svlo_matvec(z, f->ew, f->eb, &y, 1, (size_t)f->cond);
    return y;
}
