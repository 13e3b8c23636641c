/*
 * rvq.c -- restatement of Mimi's split residual vector quantizer, encoding only
 * (SVL/stt/model.rs:84-174: Quantizer, ResidualQuantizer, Codebook).
 *
 * TEST INFRASTRUCTURE ONLY (see svl_oracle.h).
 *
 *   * Codebook::new (model.rs:144-153): embedding = embedding_sum / max(cluster_usage, 1e-5)
 *     element by element; half_norms = sum over the 256 dims of embedding^2, then / 2.0
 *     ([candle hypothesis] the sum in element order, `/ 2.0` as candle's affine x * 0.5 + 0.0).
 *   * ResidualQuantizer::encode (model.rs:125-134): residual = input_proj(x) (a 1x1 convolution
 *     512 -> 256 without bias), then per codebook: indices = Codebook::encode(residual);
 *     residual -= embedding[indices].
 *   * Codebook::encode (model.rs:157-166): dot = residual . embedding^T, then the argmin over the
 *     entries of half_norms - dot ([candle hypothesis] argmin: the first index of the minimum).
 *   * Quantizer::encode (model.rs:101-104): the first quantizer (1 codebook) and the rest
 *     (n_q - 1 codebooks) both encode the same input; the codes are concatenated.
 * The products -- the 1x1 convolution and the dots -- go through candle's matmul in the
 * reference, whose summation order is the CPU-feature-specific order of the gemm crate; here
 * they use the reference's own 16-lane dot (SVL/nn/kernels/mod.rs:66-91, svlo_dot), so that the
 * GPU can follow one stated order.  Codes can differ from the reference's only where two entries'
 * scores lie within the products' rounding of each other.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

struct svlo_rvq {
    int n_q, bins;
    float* w[2];   /* input_proj of the first and the rest quantizer, [256][512] */
    float* emb;    /* [n_q][bins][256], stage order: first's codebook, then the rest's */
    float* hn;     /* [n_q][bins] */
};

void svlo_rvq_destroy(svlo_rvq* q) {
    if (!q) return;
    free(q->w[0]);
    free(q->w[1]);
    free(q->emb);
    free(q->hn);
    free(q);
}

/* SVL/stt/model.rs:144-153 */
static void codebook_prepare(const float* sums, const float* usage, int bins, float* emb, float* hn) {
    for (int e = 0; e < bins; ++e) {
        const float u = fmaxf(usage[e], 1e-5f);
        float s = 0.0f;
        for (int d = 0; d < SVLO_RVQ_DIM; ++d) {
            const float v = sums[(size_t)e * SVLO_RVQ_DIM + d] / u;
            emb[(size_t)e * SVLO_RVQ_DIM + d] = v;
            const float sq = v * v;
            s = s + sq;
        }
        hn[e] = s * 0.5f + 0.0f;
    }
}

svlo_rvq* svlo_rvq_create(int n_q, int bins, const float* w_first, const float* w_rest, const float* sums,
                          const float* usage) {
    if (n_q < 1 || bins < 1 || !w_first || !w_rest || !sums || !usage) return NULL;
    svlo_rvq* q = (svlo_rvq*)calloc(1, sizeof(*q));
    if (!q) return NULL;
    q->n_q = n_q;
    q->bins = bins;
    const size_t wn = (size_t)SVLO_RVQ_DIM * SVLO_RVQ_IN;
    q->w[0] = (float*)malloc(wn * 4);
    q->w[1] = (float*)malloc(wn * 4);
    q->emb = (float*)malloc((size_t)n_q * bins * SVLO_RVQ_DIM * 4);
    q->hn = (float*)malloc((size_t)n_q * bins * 4);
    if (!q->w[0] || !q->w[1] || !q->emb || !q->hn) {
        svlo_rvq_destroy(q);
        return NULL;
    }
    memcpy(q->w[0], w_first, wn * 4);
    memcpy(q->w[1], w_rest, wn * 4);
    for (int s = 0; s < n_q; ++s)
        codebook_prepare(sums + (size_t)s * bins * SVLO_RVQ_DIM, usage + (size_t)s * bins, bins,
                         q->emb + (size_t)s * bins * SVLO_RVQ_DIM, q->hn + (size_t)s * bins);
    return q;
}

void svlo_rvq_codebook(const svlo_rvq* q, int stage, float* emb, float* half_norms) {
    if (emb) memcpy(emb, q->emb + (size_t)stage * q->bins * SVLO_RVQ_DIM, (size_t)q->bins * SVLO_RVQ_DIM * 4);
    if (half_norms) memcpy(half_norms, q->hn + (size_t)stage * q->bins, (size_t)q->bins * 4);
}

/* SVL/stt/model.rs:157-166: the first index of the minimum of half_norms - residual . e */
static uint32_t nearest(const svlo_rvq* q, int stage, const float* r) {
    const float* emb = q->emb + (size_t)stage * q->bins * SVLO_RVQ_DIM;
    const float* hn = q->hn + (size_t)stage * q->bins;
    uint32_t best = 0;
    float mn = 0.0f;
    for (int e = 0; e < q->bins; ++e) {
        const float sc = hn[e] - svlo_dot(r, emb + (size_t)e * SVLO_RVQ_DIM, SVLO_RVQ_DIM);
        if (e == 0 || sc < mn) {
            mn = sc;
            best = (uint32_t)e;
        }
    }
    return best;
}

/* latents [batch][512][frames] (channel first), codes [batch][frames][n_q] */
void svlo_rvq_encode(const svlo_rvq* q, size_t batch, size_t frames, const float* latents, uint32_t* codes) {
    float x[SVLO_RVQ_IN], r[SVLO_RVQ_DIM];
    for (size_t b = 0; b < batch; ++b)
        for (size_t t = 0; t < frames; ++t) {
            for (int c = 0; c < SVLO_RVQ_IN; ++c) x[c] = latents[(b * SVLO_RVQ_IN + c) * frames + t];
            uint32_t* out = codes + (b * frames + t) * q->n_q;
            for (int part = 0; part < 2; ++part) {
                const int stages = part == 0 ? 1 : q->n_q - 1;
                const int stage0 = part == 0 ? 0 : 1;
                /* SVL/stt/model.rs:126: input_proj, a 1x1 convolution without bias */
                for (int o = 0; o < SVLO_RVQ_DIM; ++o)
                    r[o] = svlo_dot(q->w[part] + (size_t)o * SVLO_RVQ_IN, x, SVLO_RVQ_IN);
                for (int k = 0; k < stages; ++k) {
                    const int stage = stage0 + k;
                    const uint32_t idx = nearest(q, stage, r);
                    out[stage] = idx;
                    const float* e = q->emb + ((size_t)stage * q->bins + idx) * SVLO_RVQ_DIM;
                    for (int d = 0; d < SVLO_RVQ_DIM; ++d) r[d] = r[d] - e[d];
                }
            }
        }
}
