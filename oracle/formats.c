/*
 * formats.c -- f16/bf16 conversion and the candle GGML block formats (Q8_0, Q4_0, Q4K, Q8K).
 *
 * TEST INFRASTRUCTURE ONLY (see svl_oracle.h).
 *
 * The block layouts are the GGML ones that candle-core 0.11.1 stores for
 * `QTensor::quantize(&weight, GgmlDType::Q8_0)` (call site SVL/nn/mod.rs:77-86).  candle's
 * source is not present here, so the arithmetic below is a [candle hypothesis] restated from
 * the published GGML/candle algorithms; each function names what pins it in tests/.
 */
#include <math.h>
#include <string.h>

#include "svl_oracle.h"

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16, round to nearest even (half 2.7.1 `f16::from_f32`, Cargo.lock:1063).
 * Pinned in tests by an exhaustive f16 round trip and numpy's float16 cast. */
uint16_t svlo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m >> shift;
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1u);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float svlo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    if (exp == 0x1fu) return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 0x1p-24f;
        return u2f(sign | f2u(v));
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* bfloat16, round to nearest even, NaN kept quiet (half 2.7.1 `bf16::from_f32`). */
uint16_t svlo_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t round_bit = 0x8000u;
    if ((x & round_bit) && (x & (3u * round_bit - 1u))) return (uint16_t)((x >> 16) + 1u);
    return (uint16_t)(x >> 16);
}

float svlo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void svlo_f32_to_f16_n(const float* x, uint16_t* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = svlo_f32_to_f16(x[i]);
}
void svlo_f32_to_bf16_n(const float* x, uint16_t* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = svlo_f32_to_bf16(x[i]);
}
void svlo_bf16_to_f32_n(const uint16_t* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = svlo_bf16_to_f32(x[i]);
}

/* Rust `f as i8` / `f as i32`: saturating, NaN -> 0. */
static inline int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}
static inline int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (-2147483647 - 1);
    return (int32_t)v;
}
/* Rust f32::max / f32::min: a NaN operand yields the other operand. */
static inline float rmax(float a, float b) { return a != a ? b : (b != b ? a : (a > b ? a : b)); }
static inline float rmin(float a, float b) { return a != a ? b : (b != b ? a : (a < b ? a : b)); }

/* ---- Q8_0 ---------------------------------------------------------------------------
 * [candle hypothesis] BlockQ8_0::from_float: per 32 values, amax = max|x|, d = amax / 127,
 * id = 1/d (0 when d == 0), stored d as f16, q = round(x * id) (half away from zero, as
 * f32::round), saturating to i8. */
void svlo_quantize_q8_0(const float* x, svlo_block_q8_0* y, size_t k) {
    size_t nb = k / SVLO_QK8_0;
    for (size_t i = 0; i < nb; ++i) {
        const float* xs = x + i * SVLO_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < SVLO_QK8_0; ++j) amax = rmax(amax, fabsf(xs[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = svlo_f32_to_f16(d);
        for (int j = 0; j < SVLO_QK8_0; ++j) y[i].qs[j] = sat_i8(roundf(xs[j] * id));
    }
}

/* Dequantization is the closed form q * f32(d) (exact: one rounding of an exact product). */
void svlo_dequantize_q8_0(const svlo_block_q8_0* x, float* y, size_t k) {
    size_t nb = k / SVLO_QK8_0;
    for (size_t i = 0; i < nb; ++i) {
        float d = svlo_f16_to_f32(x[i].d);
        for (int j = 0; j < SVLO_QK8_0; ++j) y[i * SVLO_QK8_0 + j] = (float)x[i].qs[j] * d;
    }
}

/* [candle hypothesis] BlockQ8_0::vec_dot_unopt (the variant a default x86-64 build without the
 * `avx` target feature compiles): exact i32 block sums, each scaled as
 * (sum as f32 * d_w) * d_x and accumulated sequentially in f32.  `w` are the weight blocks,
 * `x` the activation blocks (candle's matmul passes `vec_dot(k, rhs_col, lhs_row)`). */
float svlo_vec_dot_q8_0(size_t n, const svlo_block_q8_0* w, const svlo_block_q8_0* x) {
    size_t nb = n / SVLO_QK8_0;
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; ++i) {
        int32_t s = 0;
        for (int j = 0; j < SVLO_QK8_0; ++j) s += (int32_t)w[i].qs[j] * (int32_t)x[i].qs[j];
        float t = (float)s * svlo_f16_to_f32(w[i].d);
        t = t * svlo_f16_to_f32(x[i].d);
        sumf += t;
    }
    return sumf;
}

/* ---- Q4_0 ---------------------------------------------------------------------------
 * [candle hypothesis] BlockQ4_0 (GGML quantize_row_q4_0 / dequantize_row_q4_0 as candle's
 * k_quants restate them): per 32 values, `max` = the value of largest magnitude (the first one
 * on ties: `if amax < |x|`), d = max / -8, id = 1 / d (0 if d = 0), d stored as f16; the code
 * of x is min(15, (x * id + 8.5) as u8) (Rust's saturating, truncating cast); byte j holds
 * element j in its low nibble and element j + 16 in its high nibble; value = (code - 8) * d. */

/* Rust `v as u8`: NaN -> 0, saturating to [0, 255], truncation toward zero. */
static inline uint8_t cast_u8(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}

void svlo_quantize_q4_0(const float* x, svlo_block_q4_0* y, size_t k) {
    size_t nb = k / SVLO_QK4_0;
    for (size_t i = 0; i < nb; ++i) {
        const float* xs = x + i * SVLO_QK4_0;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < SVLO_QK4_0; ++j) {
            float a = fabsf(xs[j]);
            if (amax < a) {
                amax = a;
                max = xs[j];
            }
        }
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = svlo_f32_to_f16(d);
        for (int j = 0; j < SVLO_QK4_0 / 2; ++j) {
            float x0 = xs[j] * id, x1 = xs[SVLO_QK4_0 / 2 + j] * id;
            uint8_t q0 = cast_u8(x0 + 8.5f), q1 = cast_u8(x1 + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            y[i].qs[j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

void svlo_dequantize_q4_0(const svlo_block_q4_0* x, float* y, size_t k) {
    size_t nb = k / SVLO_QK4_0;
    for (size_t i = 0; i < nb; ++i) {
        float d = svlo_f16_to_f32(x[i].d);
        for (int j = 0; j < SVLO_QK4_0 / 2; ++j) {
            y[i * SVLO_QK4_0 + j] = (float)((x[i].qs[j] & 0x0F) - 8) * d;
            y[i * SVLO_QK4_0 + j + SVLO_QK4_0 / 2] = (float)((x[i].qs[j] >> 4) - 8) * d;
        }
    }
}

/* [candle hypothesis] BlockQ4_0::vec_dot_unopt against Q8_0 activations: the exact i32 sum of
 * (code - 8) * q over the block, then sumf += ((f32)sum * d_w) * d_x in block order. */
float svlo_vec_dot_q4_0_q8_0(size_t n, const svlo_block_q4_0* w, const svlo_block_q8_0* x) {
    size_t nb = n / SVLO_QK4_0;
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; ++i) {
        int32_t s = 0;
        for (int j = 0; j < SVLO_QK4_0 / 2; ++j) {
            int32_t v0 = (int32_t)(w[i].qs[j] & 0x0F) - 8, v1 = (int32_t)(w[i].qs[j] >> 4) - 8;
            s += v0 * (int32_t)x[i].qs[j] + v1 * (int32_t)x[i].qs[j + SVLO_QK4_0 / 2];
        }
        float t = (float)s * svlo_f16_to_f32(w[i].d);
        t = t * svlo_f16_to_f32(x[i].d);
        sumf += t;
    }
    return sumf;
}

/* ---- Q4K ------------------------------------------------------------------------------ */

/* GGML get_scale_min_k4: 6-bit scale and min of sub-block j from the packed 12 bytes. */
static inline void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static inline int32_t nearest_int(float v) { return sat_i32(roundf(v)); }

/* Rust total_cmp on non-NaN floats orders -0.0 before +0.0. */
static inline int total_lt(float a, float b) {
    int32_t ia = (int32_t)f2u(a), ib = (int32_t)f2u(b);
    ia ^= (int32_t)(((uint32_t)(ia >> 31)) >> 1);
    ib ^= (int32_t)(((uint32_t)(ib >> 31)) >> 1);
    return ia < ib;
}

/* [candle hypothesis] make_qkx1_quants(nmax, ntry, x): iterative scale/min fit of a 32-value
 * sub-block; returns (scale, -min). */
static void make_qkx1_quants(int nmax, int ntry, const float* x, int n, float* scale_out,
                             float* min_out) {
    uint8_t L[32];
    memset(L, 0, sizeof(L));
    float mn = x[0], mx = x[0];
    for (int i = 1; i < n; ++i)
        if (total_lt(x[i], mn)) mn = x[i]; /* min_by: first minimum */
    for (int i = 1; i < n; ++i)
        if (!total_lt(x[i], mx)) mx = x[i]; /* max_by: last maximum */
    if (mx == mn) {
        *scale_out = 0.0f;
        *min_out = 0.0f;
        return;
    }
    mn = rmin(mn, 0.0f);
    float iscale = (float)nmax / (mx - mn);
    float scale = 1.0f / iscale;
    for (int itry = 0; itry < ntry; ++itry) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; ++i) {
            int32_t li = nearest_int(iscale * (x[i] - mn));
            if (li < 0) li = 0;
            if (li > nmax) li = nmax;
            if ((uint8_t)li != L[i]) {
                L[i] = (uint8_t)li;
                did_change = 1;
            }
            sumlx += (x[i] - mn) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)L[i];
        mn = sum / (float)n;
        if (mn > 0.0f) mn = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *scale_out = scale;
    *min_out = -mn;
}

/* [candle hypothesis] BlockQ4K::from_float. */
void svlo_quantize_q4k(const float* x, svlo_block_q4k* y, size_t k) {
    size_t nb = k / SVLO_QK_K;
    for (size_t ib = 0; ib < nb; ++ib) {
        const float* xb = x + ib * SVLO_QK_K;
        svlo_block_q4k* b = &y[ib];
        float mins[8], scales[8];
        for (int j = 0; j < 8; ++j) make_qkx1_quants(15, 5, xb + 32 * j, 32, &scales[j], &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) max_scale = rmax(scales[j], max_scale);
        for (int j = 0; j < 8; ++j) max_min = rmax(mins[j], max_min);
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        memset(b->scales, 0, sizeof(b->scales));
        for (int j = 0; j < 8; ++j) {
            int32_t lsi = nearest_int(inv_scale * scales[j]);
            int32_t lmi = nearest_int(inv_min * mins[j]);
            uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
            uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
            if (j < 4) {
                b->scales[j] = ls;
                b->scales[j + 4] = lm;
            } else {
                b->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                b->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                b->scales[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        b->d = svlo_f32_to_f16(max_scale / 63.0f);
        b->dmin = svlo_f32_to_f16(max_min / 63.0f);
        uint8_t L[SVLO_QK_K];
        memset(L, 0, sizeof(L));
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            get_scale_min_k4(j, b->scales, &sc, &m);
            float d = svlo_f16_to_f32(b->d) * (float)sc;
            if (d != 0.0f) {
                float dm = svlo_f16_to_f32(b->dmin) * (float)m;
                for (int ii = 0; ii < 32; ++ii) {
                    int32_t l = nearest_int((xb[32 * j + ii] + dm) / d);
                    if (l < 0) l = 0;
                    if (l > 15) l = 15;
                    L[32 * j + ii] = (uint8_t)l;
                }
            }
        }
        for (int j = 0; j < SVLO_QK_K; j += 64)
            for (int l = 0; l < 32; ++l)
                b->qs[(j / 64) * 32 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    }
}

/* Q4K dequantization closed form: y = (d * sc) * q - (dmin * m), evaluated unfused. */
void svlo_dequantize_q4k(const svlo_block_q4k* x, float* y, size_t k) {
    size_t nb = k / SVLO_QK_K;
    for (size_t ib = 0; ib < nb; ++ib) {
        const svlo_block_q4k* b = &x[ib];
        float d = svlo_f16_to_f32(b->d);
        float mn = svlo_f16_to_f32(b->dmin);
        float* out = y + ib * SVLO_QK_K;
        int is = 0;
        for (int j = 0; j < SVLO_QK_K; j += 64) {
            const uint8_t* q = b->qs + j / 2;
            uint8_t sc, m;
            get_scale_min_k4(is, b->scales, &sc, &m);
            float d1 = d * (float)sc, m1 = mn * (float)m;
            get_scale_min_k4(is + 1, b->scales, &sc, &m);
            float d2 = d * (float)sc, m2 = mn * (float)m;
            for (int l = 0; l < 32; ++l) {
                float t = d1 * (float)(q[l] & 0xF);
                out[j + l] = t - m1;
            }
            for (int l = 0; l < 32; ++l) {
                float t = d2 * (float)(q[l] >> 4);
                out[j + 32 + l] = t - m2;
            }
            is += 2;
        }
    }
}

/* [candle hypothesis] BlockQ8K::from_float: per 256 values, max = the value of largest
 * magnitude (first one on ties), iscale = -128 / max, q = min(round(iscale * x), 127),
 * bsums over groups of 16, d = 1 / iscale. */
void svlo_quantize_q8k(const float* x, svlo_block_q8k* y, size_t k) {
    size_t nb = k / SVLO_QK_K;
    for (size_t i = 0; i < nb; ++i) {
        const float* xs = x + i * SVLO_QK_K;
        float mx = 0.0f, amax = 0.0f;
        for (int j = 0; j < SVLO_QK_K; ++j) {
            float a = fabsf(xs[j]);
            if (amax < a) {
                amax = a;
                mx = xs[j];
            }
        }
        if (amax == 0.0f) {
            y[i].d = 0.0f;
            memset(y[i].qs, 0, sizeof(y[i].qs));
        } else {
            float iscale = -128.0f / mx;
            for (int j = 0; j < SVLO_QK_K; ++j) {
                float v = roundf(iscale * xs[j]);
                y[i].qs[j] = sat_i8(rmin(v, 127.0f));
            }
            y[i].d = 1.0f / iscale;
        }
        for (int j = 0; j < SVLO_QK_K / 16; ++j) {
            int32_t s = 0;
            for (int ii = 0; ii < 16; ++ii) s += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)s;
        }
    }
}

/* [candle hypothesis] BlockQ4K::vec_dot_unopt against Q8K activations: integer sub-block
 * sums scaled by the 6-bit scales in 8 i32 lanes, mins applied through the Q8K bsums, f32
 * lane sums accumulated across blocks and added at the end. */
float svlo_vec_dot_q4k_q8k(size_t n, const svlo_block_q4k* w, const svlo_block_q8k* x) {
    size_t nb = n / SVLO_QK_K;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (size_t ib = 0; ib < nb; ++ib) {
        const svlo_block_q4k* b = &w[ib];
        const svlo_block_q8k* a = &x[ib];
        int8_t aux8[SVLO_QK_K];
        for (int j = 0; j < 4; ++j) {
            for (int l = 0; l < 32; ++l) aux8[64 * j + l] = (int8_t)(b->qs[32 * j + l] & 0xF);
            for (int l = 0; l < 32; ++l) aux8[64 * j + 32 + l] = (int8_t)(b->qs[32 * j + l] >> 4);
        }
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4(j, b->scales, &scales[j], &mins[j]);
        int32_t sumi = 0;
        for (int j = 0; j < 16; ++j) sumi += (int32_t)a->bsums[j] * (int32_t)mins[j / 2];
        int32_t aux32[8] = {0};
        int pos = 0;
        for (int s = 0; s < 8; ++s) {
            int32_t scale = scales[s];
            for (int g = 0; g < 4; ++g) {
                for (int l = 0; l < 8; ++l) {
                    int16_t p = (int16_t)((int16_t)a->qs[pos + l] * (int16_t)aux8[pos + l]);
                    aux32[l] += scale * (int32_t)p;
                }
                pos += 8;
            }
        }
        float d = svlo_f16_to_f32(b->d) * a->d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        float dmin = svlo_f16_to_f32(b->dmin) * a->d;
        sumf -= dmin * (float)sumi;
    }
    float s8 = 0.0f;
    for (int l = 0; l < 8; ++l) s8 += sums[l];
    return sumf + s8;
}
