/*
 * svl_oracle.h -- CPU restatement of semantic-voice-local's streaming-transformer step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle and the reported CPU
 * baseline.  Only tests/, the smoke check and the benchmark's CPU-baseline leg may load it;
 * the product library (libsvl) never links or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.  Paths are
 * relative to the reference repository; SVL = crates/semantic-voice-local/src.
 * Functions that restate candle-core / candle-nn 0.11.1 internals (Cargo.lock:226-229,
 * 283-286), whose sources are not available here, are marked [candle hypothesis]: they follow
 * the published GGML block formats and candle's documented CPU algorithms and are pinned by
 * closed forms, invariants and brute-force checks in tests/, not by candle itself.
 */
#ifndef SVL_ORACLE_H
#define SVL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- formats (candle-core quantized k_quants; half 2.7.1) ------------------------------ */

#define SVLO_QK8_0 32
#define SVLO_QK4_0 32
#define SVLO_QK_K 256

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } svlo_block_q8_0;                 /* 34 B */
typedef struct { uint16_t d; uint8_t qs[16]; } svlo_block_q4_0;                /* 18 B */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } svlo_block_q4k; /* 144 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } svlo_block_q8k;   /* 292 B */
#pragma pack(pop)

uint16_t svlo_f32_to_f16(float x);
float svlo_f16_to_f32(uint16_t h);
uint16_t svlo_f32_to_bf16(float x);
float svlo_bf16_to_f32(uint16_t h);
void svlo_f32_to_f16_n(const float* x, uint16_t* y, size_t n);
void svlo_f32_to_bf16_n(const float* x, uint16_t* y, size_t n);
void svlo_bf16_to_f32_n(const uint16_t* x, float* y, size_t n);

void svlo_quantize_q8_0(const float* x, svlo_block_q8_0* y, size_t k);
void svlo_dequantize_q8_0(const svlo_block_q8_0* x, float* y, size_t k);
float svlo_vec_dot_q8_0(size_t n, const svlo_block_q8_0* w, const svlo_block_q8_0* x);
void svlo_quantize_q4_0(const float* x, svlo_block_q4_0* y, size_t k);
void svlo_dequantize_q4_0(const svlo_block_q4_0* x, float* y, size_t k);
float svlo_vec_dot_q4_0_q8_0(size_t n, const svlo_block_q4_0* w, const svlo_block_q8_0* x);

void svlo_quantize_q4k(const float* x, svlo_block_q4k* y, size_t k);
void svlo_dequantize_q4k(const svlo_block_q4k* x, float* y, size_t k);
void svlo_quantize_q8k(const float* x, svlo_block_q8k* y, size_t k);
float svlo_vec_dot_q4k_q8k(size_t n, const svlo_block_q4k* w, const svlo_block_q8k* x);

/* ---- the reference's own CPU kernels (SVL/nn/kernels) -------------------------------- */

/* fma != 0 selects the FMA variant chosen at run time on AVX2+FMA CPUs (kernels/mod.rs:10-35). */
void svlo_set_fma(int fma);
int svlo_get_fma(void);
void svlo_set_threads(int threads);
int svlo_get_threads(void);

float svlo_dot(const float* a, const float* b, size_t n);
float svlo_exp(float x);
float svlo_silu(float x);
float svlo_gelu_tanh(float x);
float svlo_gelu_erf(float x);
void svlo_silu_n(float* x, size_t n);
void svlo_gelu_tanh_n(float* x, size_t n);
void svlo_matvec(const float* x, const float* w, const float* bias, float* y, size_t n, size_t k);
/* q [b,h,t,d]; k,v [b,kvh,n,d] contiguous; out [b,t,h,d].  Returns 0, or -1 on shape error. */
int svlo_attention(const float* q, const float* k, const float* v, float* out, size_t b, size_t h,
                   size_t t, size_t d, size_t kvh, size_t n, size_t position, size_t first_key,
                   size_t context /* 0 = none */);

/* ---- candle-nn ops [candle hypothesis] ------------------------------------------------ */

/* Summation order of the norm statistics: element order (candle's CPU ops, the default) or the
 * blocked order of the GPU kernels. */
enum { SVLO_NORM_ORDER_ELEMENT = 0, SVLO_NORM_ORDER_BLOCKED = 1 };
void svlo_set_norm_order(int order);
int svlo_get_norm_order(void);
void svlo_rms_norm(const float* x, const float* alpha, float* y, size_t rows, size_t dim, float eps);
void svlo_layer_norm(const float* x, const float* w, const float* b, float* y, size_t rows,
                     size_t dim, float eps);
/* x [b,h,t,d] in place; cos/sin [t, d/2] */
void svlo_rope_i(float* x, const float* cos_t, const float* sin_t, size_t bh, size_t t, size_t d);
void svlo_rope_tables(size_t position, size_t t, size_t head_dim, double max_period, float* cos_t,
                      float* sin_t);
uint32_t svlo_argmax(const float* x, size_t n);
/* softmax over x[0..n) (candle-nn softmax_last_dim), returning its first element */
float svlo_softmax_first(const float* x, size_t n);

/* ---- Mimi's split residual vector quantizer, encoding (rvq.c) ------------------------- */

#define SVLO_RVQ_IN 512   /* latent channels */
#define SVLO_RVQ_DIM 256  /* codebook dims (ResidualQuantizer::DIM) */
typedef struct svlo_rvq svlo_rvq;
/* w_first / w_rest: input_proj weights [256][512]; sums [n_q][bins][256] and usage [n_q][bins]:
 * the codebooks' embedding_sum and cluster_usage, the first quantizer's codebook first, then the
 * rest's in order. */
svlo_rvq* svlo_rvq_create(int n_q, int bins, const float* w_first, const float* w_rest, const float* sums,
                          const float* usage);
void svlo_rvq_destroy(svlo_rvq* q);
/* the prepared embedding [bins][256] and half norms [bins] of codebook `stage` */
void svlo_rvq_codebook(const svlo_rvq* q, int stage, float* emb, float* half_norms);
/* latents [batch][512][frames] -> codes [batch][frames][n_q] */
void svlo_rvq_encode(const svlo_rvq* q, size_t batch, size_t frames, const float* latents, uint32_t* codes);

/* ---- model ------------------------------------------------------------------------------ */

enum { SVLO_F32 = 0, SVLO_BF16 = 1, SVLO_F16 = 2, SVLO_Q8_0 = 3, SVLO_Q4K = 4, SVLO_Q4_0 = 5 };
enum { SVLO_NORM_LAYER = 0, SVLO_NORM_RMS = 1 };
enum { SVLO_FF_PLAIN = 0, SVLO_FF_GATED = 1, SVLO_FF_PLAIN_ERF = 2 };
enum { SVLO_MODEL_TRANSFORMER = 0, SVLO_MODEL_STT = 1, SVLO_MODEL_TTS = 2 };
/* FlowKind (SVL/tts/config.rs:170-185) */
enum { SVLO_FLOW_LSD = 0, SVLO_FLOW_MATCHING = 1, SVLO_FLOW_DRIFTING = 2, SVLO_FLOW_POINTWISE = 3 };

typedef struct {
    int32_t kind;          /* SVLO_MODEL_* */
    int32_t d_model, num_layers, num_heads, num_kv_heads, head_dim;
    int32_t ff_kind, ff_hidden;
    int32_t norm_kind;
    float norm_eps;
    int32_t layer_scale;
    int32_t context;       /* 0 = unlimited */
    double max_period;
    int32_t quantize;      /* 0: linears as given; SVLO_Q8_0/SVLO_Q4K: quantize dense linears */
    /* STT */
    int32_t card, n_q, text_card;
    /* TTS */
    int32_t latent_dim, z_dim; /* z_dim 0 = no z_proj */
    int32_t extra_heads_num, extra_heads_dim; /* STT VAD heads (0: none) */
    int32_t flow_dim, flow_depth, flow_kind;  /* TTS flow head (0 = none), SVLO_FLOW_* */
} svlo_config;

typedef struct {
    const char* name;
    int32_t dtype;
    int32_t ndim;
    int64_t shape[4];
    const void* data;
} svlo_tensor;

typedef struct svlo_model svlo_model;
typedef struct svlo_state svlo_state;

int svlo_model_create(const svlo_config* cfg, const svlo_tensor* tensors, size_t n, svlo_model** out);
void svlo_model_destroy(svlo_model* m);
const char* svlo_last_error(void);
/* Dequantized (or converted) f32 copy of a linear weight as the model holds it. */
int svlo_model_linear_weight(const svlo_model* m, const char* name, float* out, size_t n);

svlo_state* svlo_state_create(const svlo_model* m, int32_t batch);
svlo_state* svlo_state_duplicate(const svlo_state* s);
void svlo_state_destroy(svlo_state* s);
int64_t svlo_state_position(const svlo_state* s);
/* Visible cache length and first absolute position of layer `layer` (as KvCache::current). */
int svlo_state_cache_info(const svlo_state* s, int layer, int64_t* len, int64_t* start);
/* Copies layer caches [b, kvh, len, hd] for k and v. */
int svlo_state_cache_copy(const svlo_state* s, int layer, float* k, float* v);
/* Rebuilds a state from per-layer caches covering positions 0..len. */
svlo_state* svlo_state_from_layer_caches(const svlo_model* m, int32_t batch, int64_t len,
                                         const float* const* ks, const float* const* vs);

/* xs [b, t, d] -> ys [b, t, d] */
int svlo_transformer_forward(const svlo_model* m, svlo_state* s, const float* xs, int64_t t, float* ys);
/* batch 1: text token + n_q audio tokens -> argmax; logits (text_card) and the extra heads'
 * first-class probabilities (extra_heads_num) optional */
int svlo_stt_step(const svlo_model* m, svlo_state* s, uint32_t text_token, const uint32_t* audio,
                  uint32_t* out_token, float* out_logits, float* out_probs);
/* Recognizer loop: n steps, audio [n * n_q]; step 0 of a fresh state sees `card` tokens; text
 * token = previous argmax, initially text_card. */
int svlo_stt_greedy(const svlo_model* m, svlo_state* s, int64_t n, const uint32_t* audio,
                    uint32_t* out_tokens, float* out_last_logits, float* out_probs /* [n][heads] */);
/* latent [latent_dim] or NULL (bos) -> z [z_dim or d_model] */
int svlo_tts_backbone_step(const svlo_model* m, svlo_state* s, const float* latent, float* out_z);
/* FlowLm::step (SVL/tts/flow_lm.rs:162-185) with the noise the sampler drew: latent or NULL
 * (bos), noise [latent_dim] -> next latent [latent_dim] and the end-of-speech logit. */
int svlo_tts_step(const svlo_model* m, svlo_state* s, const float* latent, const float* noise, int decode_steps,
                  float* out_latent, float* out_eos_logit);

/* ---- turns (turns.c): the recognizer's word events and TurnDetector ---------------------- */
typedef struct {
    float threshold;
    int32_t frames, head;
    int64_t above;        /* consecutive frames above the threshold */
    int32_t in_turn;      /* words came since the last end of turn */
    int32_t pending;      /* the recognizer holds word tokens not yet emitted */
} svlo_turn;
void svlo_turn_init(svlo_turn* t, float threshold, int frames, int head);
int svlo_turn_word(svlo_turn* t);
int svlo_turn_activity(svlo_turn* t, const float* probs, int n);
int svlo_turn_step(svlo_turn* t, uint32_t token, const float* probs, int n);

/* ---- flow head (flow.c): FlowHead / TimestepEmbedder / ResBlock / out_eos -------------- */
typedef struct svlo_flow svlo_flow;
int svlo_flow_create(int dim, int depth, int kind, int latent, int cond, const svlo_tensor* ts, size_t n,
                     svlo_flow** out);
void svlo_flow_destroy(svlo_flow* f);
const char* svlo_flow_last_error(void);
const svlo_flow* svlo_model_flow(const svlo_model* m);
/* TimestepEmbedder i at time t -> [dim]; the mean of the embeddings of `times` -> [dim] */
void svlo_flow_time_embed(const svlo_flow* f, int i, float t, float* out);
void svlo_flow_time_mean(const svlo_flow* f, const float* times, float* out);
/* FlowHead::forward: cond [cond], times, tmean [dim] or NULL, xs [latent] -> out [latent] */
void svlo_flow_forward(const svlo_flow* f, const float* cond, const float* times, const float* tmean,
                       const float* xs, float* out);
/* FlowHead::decode: noise [latent] -> latent [latent] */
void svlo_flow_decode(const svlo_flow* f, const float* cond, const float* noise, int steps, float* out);
float svlo_flow_eos_logit(const svlo_flow* f, const float* z);

#ifdef __cplusplus
}
#endif
#endif
