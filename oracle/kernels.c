/*
 * kernels.c -- restatement of the reference's own CPU kernels (SVL/nn/kernels/{mod,matvec,attention,activation}.rs) and of
 * the candle-nn ops the step calls.
 *
 * TEST INFRASTRUCTURE ONLY (see svl_oracle.h).  Build with -ffp-contract=off: every fused
 * multiply-add below is an explicit fmaf(), exactly where the reference's `mul_add::<FMA>`
 * fuses (SVL/nn/kernels/mod.rs:60-64).
 */
#include <math.h>
#include <string.h>
#include <stdlib.h>
#include <omp.h>

#include "svl_oracle.h"

static int g_fma = 1;
static int g_threads = 4;

void svlo_set_fma(int fma) { g_fma = fma ? 1 : 0; }
int svlo_get_fma(void) { return g_fma; }
void svlo_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }
int svlo_get_threads(void) { return g_threads; }

/* SVL/nn/kernels/mod.rs:60-64 `mul_add::<FMA>` */
static inline float mul_add(float a, float b, float c) { return g_fma ? fmaf(a, b, c) : a * b + c; }

/* SVL/nn/kernels/mod.rs:66-91 `dot`: 16 independent lanes, scalar tail, pairwise lane sum. */
float svlo_dot(const float* a, const float* b, size_t n) {
    enum { LANES = 16 };
    float acc[LANES];
    memset(acc, 0, sizeof(acc));
    size_t chunks = n / LANES;
    for (size_t c = 0; c < chunks; ++c)
        for (int i = 0; i < LANES; ++i) acc[i] = mul_add(a[c * LANES + i], b[c * LANES + i], acc[i]);
    float sum = 0.0f;
    for (size_t i = chunks * LANES; i < n; ++i) {
        float p = a[i] * b[i];
        sum += p;
    }
    int width = LANES;
    while (width > 1) {
        width /= 2;
        for (int i = 0; i < width; ++i) acc[i] += acc[i + width];
    }
    return acc[0] + sum;
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* SVL/nn/kernels/mod.rs:93-121 `exp_parts`: Cody-Waite reduction x = k ln2 + r with a split
 * ln2, then expm1(r) by its degree-8 Taylor polynomial in Horner form. */
static inline void exp_parts(float x, float* two_k, float* expm1_r) {
    const float LN2_HI = 0.69314575f;
    const float LN2_LO = 1.4286068e-6f;
    const float ROUND = 12582912.0f;
    const float LOG2E = 1.44269504088896340736f;
    float shifted = mul_add(x, LOG2E, ROUND);
    float k = shifted - ROUND;
    int32_t k_int = (int32_t)(f2u(shifted) - f2u(ROUND));
    float r = mul_add(-k, LN2_LO, mul_add(-k, LN2_HI, x));
    static const float C[7] = {1.0f / 5040.0f, 1.0f / 720.0f, 1.0f / 120.0f, 1.0f / 24.0f,
                               1.0f / 6.0f,    0.5f,           1.0f};
    float p = 1.0f / 40320.0f;
    for (int i = 0; i < 7; ++i) p = mul_add(p, r, C[i]);
    *two_k = u2f(((uint32_t)(k_int + 127)) << 23);
    *expm1_r = p * r;
}

static inline float clampf(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* SVL/nn/kernels/mod.rs:123-131 `exp`. */
float svlo_exp(float x) {
    float two_k, e;
    exp_parts(clampf(x, -87.0f, 88.0f), &two_k, &e);
    float y = mul_add(two_k, e, two_k);
    if (x > 88.72f) y = INFINITY;
    return x < -87.0f ? 0.0f : y;
}

/* SVL/nn/kernels/activation.rs:70-74 `silu` = x / (1 + exp(-x)). */
float svlo_silu(float x) { return x / (1.0f + svlo_exp(-x)); }

/* SVL/nn/kernels/activation.rs:76-82 `gelu_tanh` = x sigmoid(2y),
 * y = 0.7978846 * mul_add(0.044715 x, x^2, x). */
float svlo_gelu_tanh(float x) {
    const float SQRT_2_OVER_PI = 0.7978846f;
    float a = 0.044715f * x;
    float x2 = x * x;
    float y = SQRT_2_OVER_PI * mul_add(a, x2, x);
    return x / (1.0f + svlo_exp(-2.0f * y));
}

/* [candle hypothesis] Tensor::gelu_erf (SVL/nn/transformer.rs:446-447) for f32: evaluated in f64
 * as (erf(v / sqrt 2) + 1) * 0.5 * v with the C library's erf, rounded to f32. */
float svlo_gelu_erf(float x) {
    const double v = (double)x;
    return (float)((erf(v / 1.4142135623730951) + 1.0) * 0.5 * v);
}

void svlo_silu_n(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = svlo_silu(x[i]);
}
void svlo_gelu_tanh_n(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = svlo_gelu_tanh(x[i]);
}

/* SVL/nn/kernels/matvec.rs:174-202 `MatVec::run`: rows split in tasks of
 * clamp(n / (4 threads), 8, 256), each row a `dot`, then the bias added. */
void svlo_matvec(const float* x, const float* w, const float* bias, float* y, size_t n, size_t k) {
    long rows = (long)(n / (4 * (size_t)g_threads));
    if (rows < 8) rows = 8;
    if (rows > 256) rows = 256;
    long tasks = ((long)n + rows - 1) / rows;
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
    for (long tsk = 0; tsk < tasks; ++tsk) {
        size_t r0 = (size_t)(tsk * rows), r1 = r0 + (size_t)rows;
        if (r1 > n) r1 = n;
        for (size_t r = r0; r < r1; ++r) {
            y[r] = svlo_dot(x, w + r * k, k);
            if (bias) y[r] += bias[r];
        }
    }
}

/* SVL/nn/kernels/attention.rs:139-168 `attend`. */
static void attend(const float* q, const float* keys, size_t kstride, const float* values,
                   size_t vstride, size_t count, size_t d, float scale, float* out, float* wbuf) {
    if (count == 0) return;
    for (size_t j = 0; j < count; ++j) wbuf[j] = scale * svlo_dot(q, keys + j * kstride, d);
    float mx = wbuf[0];
    for (size_t j = 1; j < count; ++j) {
        float w = wbuf[j];
        mx = (mx != mx) ? w : (w != w ? mx : (w > mx ? w : mx));
    }
    for (size_t j = 0; j < count; ++j) wbuf[j] = svlo_exp(wbuf[j] - mx);
    float sum = 0.0f;
    for (size_t j = 0; j < count; ++j) sum += wbuf[j];
    for (size_t j = 0; j < count; ++j) {
        float w = wbuf[j] / sum;
        const float* v = values + j * vstride;
        for (size_t i = 0; i < d; ++i) out[i] = mul_add(w, v[i], out[i]);
    }
}

/* SVL/nn/kernels/attention.rs:81-136 with explicit strides for k and v
 * ([b][kvh][row] strides; rows contiguous). */
int svlo_attention_strided(const float* q, const float* k, const float* v, float* out, size_t b,
                           size_t h, size_t t, size_t d, size_t kvh, size_t n, size_t kv_sb,
                           size_t kv_sh, size_t kv_sr, size_t position, size_t first_key,
                           size_t context) {
    if (kvh == 0 || h % kvh != 0) return -1;
    size_t ctx = context ? context : (size_t)-1;
    float scale = powf((float)d, -0.5f);
    memset(out, 0, sizeof(float) * b * t * h * d);
    long total = (long)(b * t * h);
    int parallel = b * t * h * n * d >= (1u << 16);
#pragma omp parallel num_threads(parallel ? g_threads : 1)
    {
        float* wbuf = (float*)malloc(sizeof(float) * (n ? n : 1));
#pragma omp for schedule(dynamic, 4)
        for (long index = 0; index < total; ++index) {
            size_t batch = (size_t)index / (t * h), rest = (size_t)index % (t * h);
            size_t step = rest / h, head = rest % h;
            size_t kv_head = head / (h / kvh);
            size_t query = position + step;
            size_t lo = ctx - 1 > query ? 0 : query - (ctx - 1);
            if (lo < first_key) lo = first_key;
            size_t first = lo - first_key;
            size_t end = query + 1 > first_key ? query + 1 - first_key : 0;
            if (end > n) end = n;
            size_t count = end > first ? end - first : 0;
            const float* qq = q + ((batch * h + head) * t + step) * d;
            const float* kk = k + batch * kv_sb + kv_head * kv_sh + first * kv_sr;
            const float* vv = v + batch * kv_sb + kv_head * kv_sh + first * kv_sr;
            attend(qq, kk, kv_sr, vv, kv_sr, count, d, scale, out + (size_t)index * d, wbuf);
        }
        free(wbuf);
    }
    return 0;
}

int svlo_attention(const float* q, const float* k, const float* v, float* out, size_t b, size_t h,
                   size_t t, size_t d, size_t kvh, size_t n, size_t position, size_t first_key,
                   size_t context) {
    return svlo_attention_strided(q, k, v, out, b, h, t, d, kvh, n, kvh * n * d, n * d, d,
                                  position, first_key, context);
}

/* Order of the norm statistics' sums (svlo_set_norm_order).
 *
 * SVLO_NORM_ORDER_ELEMENT (default) is candle-nn's CPU RmsNorm / LayerNorm: one f32
 * accumulator per row, x_0, x_1, ... added in index order (`Iterator::sum::<f32>` and a plain
 * `for v in src` loop; Rust never reassociates float adds).  [candle hypothesis]
 *
 * SVLO_NORM_ORDER_BLOCKED is the order of the GPU kernels: 64 strided partials (partial l sums
 * x[l], x[l+64], ... sequentially), then a butterfly over the partials (p[l] + p[l ^ o] for
 * o = 32, 16, 8, 4, 2, 1; every lane ends with the same value, lane 0's is returned).  The two
 * orders differ by rounding only; tests/ measure what that does to logits and greedy tokens. */
static int g_norm_order = SVLO_NORM_ORDER_ELEMENT;

void svlo_set_norm_order(int order) {
    g_norm_order = order == SVLO_NORM_ORDER_BLOCKED ? SVLO_NORM_ORDER_BLOCKED : SVLO_NORM_ORDER_ELEMENT;
}
int svlo_get_norm_order(void) { return g_norm_order; }

static float row_sum(const float* x, size_t n, int squares) {
    if (g_norm_order == SVLO_NORM_ORDER_ELEMENT) {
        float acc = 0.0f;
        for (size_t i = 0; i < n; ++i) {
            float v = x[i];
            if (squares) v = v * v;
            acc += v;
        }
        return acc;
    }
    float p[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (size_t i = (size_t)l; i < n; i += 64) {
            float v = x[i];
            if (squares) v = v * v;
            acc += v;
        }
        p[l] = acc;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        float q[64];
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ o];
        memcpy(p, q, sizeof(p));
    }
    return p[0];
}

/* [candle hypothesis] candle-nn ops::rms_norm CPU: m = sqrt(sum(x^2) / dim + eps),
 * y = x / m * alpha (sum in the order selected above).  Call sites SVL/nn/transformer.rs:286,
 * SVL/stt/model.rs:252. */
void svlo_rms_norm(const float* x, const float* alpha, float* y, size_t rows, size_t dim, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float* s = x + r * dim;
        float* d = y + r * dim;
        float sum2 = row_sum(s, dim, 1);
        float m = sqrtf(sum2 / (float)dim + eps);
        for (size_t i = 0; i < dim; ++i) {
            float t = s[i] / m;
            d[i] = t * alpha[i];
        }
    }
}

/* [candle hypothesis] candle-nn ops::layer_norm CPU: mean = sum(x) / dim,
 * var = sum(x^2) / dim - mean^2, y = (x - mean) * (1 / sqrt(var + eps)) * w + b (sums in the
 * order selected above).  Call sites SVL/nn/transformer.rs:284, SVL/tts/flow_lm.rs:176. */
void svlo_layer_norm(const float* x, const float* w, const float* b, float* y, size_t rows,
                     size_t dim, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float* s = x + r * dim;
        float* d = y + r * dim;
        float sum = row_sum(s, dim, 0);
        float sum2 = row_sum(s, dim, 1);
        float mean = sum / (float)dim;
        float mm = mean * mean;
        float var = sum2 / (float)dim - mm;
        float inv_std = 1.0f / sqrtf(var + eps);
        for (size_t i = 0; i < dim; ++i) {
            float t = (s[i] - mean) * inv_std;
            t = t * w[i];
            d[i] = t + b[i];
        }
    }
}

/* [candle hypothesis] candle-nn rotary_emb::rope_i CPU: interleaved pairs (2i, 2i+1) of every
 * row of x [bh][t][d], with cos/sin [t][d/2].  Call site SVL/nn/transformer.rs:339-340. */
void svlo_rope_i(float* x, const float* cos_t, const float* sin_t, size_t bh, size_t t, size_t d) {
    for (size_t m = 0; m < bh; ++m) {
        float* s = x + m * t * d;
        for (size_t io2 = 0; io2 < t * d / 2; ++io2) {
            size_t i = 2 * io2;
            float a = s[i], b = s[i + 1];
            float c = cos_t[io2], sn = sin_t[io2];
            float ac = a * c, bs = b * sn, as = a * sn, bc = b * c;
            s[i] = ac - bs;
            s[i + 1] = as + bc;
        }
    }
}

/* SVL/nn/transformer.rs:114-118 (inv_freq in f64, cast to f32) and :161-172 (positions as f32
 * times inv_freq, then cos and sin). */
void svlo_rope_tables(size_t position, size_t t, size_t head_dim, double max_period, float* cos_t,
                      float* sin_t) {
    size_t half = head_dim / 2;
    for (size_t s = 0; s < t; ++s) {
        float pos = (float)(position + s);
        for (size_t i = 0; i < half; ++i) {
            float inv = (float)exp(-(log(max_period)) * 2.0 * (double)i / (double)head_dim);
            float f = pos * inv;
            cos_t[s * half + i] = cosf(f);
            sin_t[s * half + i] = sinf(f);
        }
    }
}

/* [candle hypothesis] argmax over the last dim: the first index of the maximum. */
uint32_t svlo_argmax(const float* x, size_t n) {
    uint32_t best = 0;
    float mx = x[0];
    for (size_t i = 1; i < n; ++i)
        if (x[i] > mx) {
            mx = x[i];
            best = (uint32_t)i;
        }
    return best;
}

/* [candle hypothesis] candle-nn ops::softmax_last_dim on the CPU, as LanguageModel::step applies it
 * to each extra head's logits (SVL/stt/model.rs:262-268): the maximum in index order starting
 * from x[0], exp(x_i - max) with the C library's expf (Rust's f32::exp), their sum in index
 * order from zero, then element 0 divided by the sum (the step keeps only `.i(0)`). */
float svlo_softmax_first(const float* x, size_t n) {
    float mx = x[0];
    for (size_t i = 1; i < n; ++i) mx = fmaxf(mx, x[i]);
    float sum = 0.0f, first = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float e = expf(x[i] - mx);
        if (i == 0) first = e;
        sum += e;
    }
    return first / sum;
}
