/*
 * svl.h -- C ABI of the MI355X streaming-transformer step (libsvl.so).
 *
 * A drop-in for the per-frame decode step of semantic-voice-local's streaming transformer:
 * the Kyutai STT language-model step and the Pocket-TTS flow-LM backbone step.  Reference
 * paths are relative to the reference repository; SVL = crates/semantic-voice-local/src.
 *
 * Conventions (mirroring the crate's Rust API):
 *  - Every function returns 0 on success, a negative svl_status on error (the message is in
 *    svl_last_error(), thread-local), mirroring `Result<T, Error>` (SVL/error.rs:1-32), or
 *    SVL_UNSUPPORTED (positive) when the request is valid for the reference but outside what
 *    these kernels cover: the caller then runs the reference's own path, as the reference's
 *    kernels return `Ok(None)` to fall back (SVL/nn/kernels/matvec.rs:12-17,
 *    SVL/nn/kernels/attention.rs:21-23).  Nothing was created or changed in that case.
 *  - Work enqueued by the *_async functions reports its errors at svl_state_synchronize.
 *  - svl_model is immutable after creation and may be shared by host threads, as
 *    `Stt: Send + Sync` (SVL/stt/mod.rs:159).  svl_state is per stream and used by one host
 *    thread at a time, as `&mut TransformerState` (SVL/nn/transformer.rs:139).
 *  - Host buffers belong to the caller.  svl_model_create copies (and repacks) the weights to
 *    the GPU and keeps no host pointer.  Output buffers are caller-provided.
 *  - Each state owns one HIP stream.  The *_async functions only enqueue work on it and take
 *    device pointers; svl_state_synchronize waits for it.  The other entry points take host
 *    pointers and return once their outputs are in host memory, like `to_scalar`
 *    (SVL/stt/model.rs:258).
 */
#ifndef SVL_H
#define SVL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SVL/error.rs:3-30: Config, InvalidInput, Candle (tensor/device), Io; and the kernels'
 * `None` (fall back to the reference's path, SVL/nn/kernels/matvec.rs:12-17). */
typedef enum {
    SVL_UNSUPPORTED = 1,
    SVL_OK = 0,
    SVL_ERR_CONFIG = -1,
    SVL_ERR_INVALID_INPUT = -2,
    SVL_ERR_DEVICE = -3,
    SVL_ERR_IO = -4,
} svl_status;

/* Weight dtypes: dense, or candle QTensor block formats (GgmlDType::Q8_0 = 34-byte blocks
 * {f16 d; i8 qs[32]}, GgmlDType::Q4K = 144-byte blocks {f16 d, dmin; u8 scales[12];
 * u8 qs[128]}, GgmlDType::Q4_0 = 18-byte blocks {f16 d; u8 qs[16]}: byte j holds the 4-bit code
 * of element j (low nibble) and of element j + 16 (high nibble), value (code - 8) * d),
 * row-major [out][in / block].  SVL_I64: integer metadata (voice states' offsets). */
typedef enum { SVL_F32 = 0, SVL_BF16 = 1, SVL_F16 = 2, SVL_Q8_0 = 3, SVL_Q4K = 4, SVL_Q4_0 = 5, SVL_I64 = 6 } svl_dtype;

typedef enum { SVL_NORM_LAYER = 0, SVL_NORM_RMS = 1 } svl_norm;          /* transformer.rs:12-16 */
/* transformer.rs:18-24: linear2(gelu(linear1(x))) with the tanh GELU, the gated SiLU, or the plain
 * feed-forward with erf GELU (`exact_gelu`, the Kyutai STT Mimi's transformers, mimi.rs:47-48) */
typedef enum { SVL_FF_PLAIN_GELU = 0, SVL_FF_GATED_SILU = 1, SVL_FF_PLAIN_GELU_ERF = 2 } svl_ff;
typedef enum { SVL_MODEL_TRANSFORMER = 0, SVL_MODEL_STT = 1, SVL_MODEL_TTS = 2 } svl_model_kind;
/* FlowKind (SVL/tts/config.rs:170-195): LSD (two flow times), flow matching (one), drifting and
 * pointwise (none). */
typedef enum { SVL_FLOW_LSD = 0, SVL_FLOW_MATCHING = 1, SVL_FLOW_DRIFTING = 2, SVL_FLOW_POINTWISE = 3 } svl_flow_kind;

/* TransformerConfig (SVL/nn/transformer.rs:26-41) plus the heads of the two backbones
 * (SttConfig, SVL/stt/model.rs:16-34; FlowLmConfig's latent/z dims, SVL/tts/flow_lm.rs:45-126). */
typedef struct {
    int32_t kind;          /* svl_model_kind */
    int32_t d_model, num_layers, num_heads, num_kv_heads, head_dim;
    int32_t ff_kind;       /* svl_ff */
    int32_t ff_hidden;
    int32_t norm_kind;     /* svl_norm */
    float norm_eps;
    int32_t layer_scale;   /* 0/1: layers.{i}.layer_scale_{1,2}.scale */
    int32_t context;       /* attention window; 0 = unlimited */
    double max_period;     /* RoPE base */
    int32_t quantize;      /* 0, SVL_Q8_0, SVL_Q4_0 or SVL_Q4K: dense linears are quantized on the
                              GPU at creation (Linear::from_weight, SVL/nn/mod.rs:76-87, with
                              the block type chosen here instead of its fixed Q8_0) */
    int32_t card, n_q, text_card;    /* STT */
    int32_t latent_dim, z_dim;       /* TTS (z_dim 0: no z_proj) */
    int32_t kv_dtype;      /* SVL_F32 (default) or SVL_BF16: element type of the KV ring buffers */
    int32_t extra_heads_num, extra_heads_dim;  /* STT extra (VAD) heads, SttConfig's
                              extra_heads_num_heads / extra_heads_dim (SVL/stt/model.rs:217-222):
                              dense "extra_heads.{i}.weight" [dim][d_model], never quantized;
                              0 = none */
    int32_t flow_dim, flow_depth, flow_kind;  /* TTS flow head (FlowHeadConfig dim / depth /
                              type, SVL/tts/config.rs:197-204) and end-of-speech head: tensors
                              "flow_net.*" and "out_eos.*" (SVL/tts/flow_lm.rs:107-113, 232-251),
                              dense; flow_dim 0 = backbone only */
} svl_config;

/* One named tensor (the reference's safetensors names, e.g.
 * "transformer.layers.3.self_attn.in_proj_weight", "emb.7.weight", "text_linear.weight"). */
typedef struct {
    const char* name;
    int32_t dtype;         /* svl_dtype */
    int32_t ndim;          /* <= 5 */
    int64_t shape[5];
    const void* data;      /* host pointer */
} svl_tensor;

typedef struct svl_model svl_model;
typedef struct svl_state svl_state;

const char* svl_last_error(void);
int svl_device_count(int* count);

/* Transformer::new + LanguageModel::new / FlowLm::new (SVL/nn/transformer.rs:107-125,
 * SVL/stt/model.rs:196-233, SVL/tts/flow_lm.rs:45-126) on GPU `device`. */
int svl_model_create(const svl_config* cfg, const svl_tensor* tensors, size_t count, int device,
                     svl_model** out);
void svl_model_destroy(svl_model* model);

/* The weight of linear `name` ("text_linear", "input_linear", "<layer>.in_proj",
 * "<layer>.out_proj", "<layer>.ff1", "<layer>.ff2") as the GPU holds it: `f32` receives the
 * dequantized (or converted) values computed by the GPU's dequantization kernel
 * ([out][in] f32), `blocks` the candle block bytes rebuilt from the device copy (quantized
 * linears only).  Either pointer may be NULL. */
int svl_model_linear_weight(const svl_model* model, const char* name, float* f32, size_t f32_count,
                            void* blocks, size_t block_bytes);

/* Transformer::init_state (SVL/nn/transformer.rs:127-136) for `batch` lockstep streams.  Each
 * stream has its own position (the reference's state has one position for the whole batch,
 * transformer.rs:55; streams stepped together from a fresh state share it).  `capacity` bounds
 * the positions of an unlimited-context model (ignored with a window: the ring buffer then has
 * `context` slots). */
int svl_state_create(const svl_model* model, int32_t batch, int32_t capacity, svl_state** out);
/* TransformerState::duplicate (SVL/nn/transformer.rs:64-73). */
int svl_state_duplicate(const svl_state* state, svl_state** out);
/* TransformerState::from_layer_caches (SVL/nn/transformer.rs:81-103) for stream `stream`:
 * per layer keys/values [num_kv_heads][len][head_dim] f32 covering positions 0..len. */
int svl_state_load_stream(svl_state* state, int32_t stream, int64_t len, const float* const* keys,
                          const float* const* values);
/* Voice::load (SVL/tts/voice.rs:103-143): a voice state in upstream Pocket TTS's safetensors
 * layout -- per layer i, "transformer.layers.{i}.self_attn/cache" f32 or bf16 [2, 1, time,
 * num_kv_heads, head_dim] (keys then values), "/offset" SVL_I64 [1] (the cached length; older
 * exports: the length of "/current_end", else `time`) and "/pad" SVL_I64 (must be 0) -- loaded
 * into stream `stream` as by svl_state_load_stream.  Batched (batch > 1) states are
 * SVL_UNSUPPORTED. */
int svl_state_load_voice(svl_state* state, int32_t stream, const svl_tensor* tensors, size_t count);
/* TransformerState::layer_caches (SVL/nn/transformer.rs:76-78) for one stream and layer: the
 * visible keys/values [num_kv_heads][*len][head_dim] f32 (pass NULL buffers to query *len and
 * *first, the absolute position of the first one). */
int svl_state_layer_cache(const svl_state* state, int32_t stream, int32_t layer, float* keys,
                          float* values, int64_t* len, int64_t* first);
int svl_state_positions(const svl_state* state, int64_t* positions /* [batch] */);
int svl_state_reset(svl_state* state);
void svl_state_destroy(svl_state* state);
/* Waits for the state's stream; reports the errors of the *_async work enqueued since the last
 * call (SVL_ERR_INVALID_INPUT for an out-of-range token id). */
int svl_state_synchronize(svl_state* state);
/* The state's HIP stream (hipStream_t), for callers that time or order work around it. */
void* svl_state_stream(const svl_state* state);

/* Transformer::forward (SVL/nn/transformer.rs:139-154): xs [batch][t][d_model] f32 ->
 * ys [batch][t][d_model] f32 (host).  With an unlimited context (a prompt prefill, as
 * FlowLm::prompt_text / prompt_voice, SVL/tts/flow_lm.rs:137-158) up to 256 positions run as one
 * pass of the step's kernels (each position a row, attending causally within the block); a
 * windowed model runs one position at a time. */
int svl_transformer_forward(const svl_model* model, svl_state* state, const float* xs, int64_t t,
                            float* ys);

/* LanguageModel::step (SVL/stt/model.rs:239-276) for every stream: text_tokens [batch],
 * audio_tokens [batch][n_q] -> out_tokens [batch] (argmax, first index on ties) and optionally
 * out_logits [batch][text_card] f32.  Host pointers. */
int svl_stt_step(const svl_model* model, svl_state* state, const uint32_t* text_tokens,
                 const uint32_t* audio_tokens, uint32_t* out_tokens, float* out_logits);

/* LanguageModel::step with its Prediction (SVL/stt/model.rs:189-193, 239-276): as svl_stt_step,
 * and out_probs [batch][extra_heads_num] receives, per extra head, the probability of its first
 * class (softmax of the head's logits over the out_norm'ed output, index 0; the VAD heads'
 * "no speech").  out_probs may be NULL. */
int svl_stt_step_heads(const svl_model* model, svl_state* state, const uint32_t* text_tokens,
                       const uint32_t* audio_tokens, uint32_t* out_tokens, float* out_logits,
                       float* out_probs);

/* Recognizer::step's token loop (SVL/stt/mod.rs:551-566) for n_steps steps with no host round
 * trip: the text token of a step is the previous step's argmax (text_card before the first
 * step of a stream), and a stream's first step (position 0) sees `card` for every audio
 * token.  audio_tokens [n_steps][batch][n_q], out_tokens [n_steps][batch].  Host pointers. */
int svl_stt_recognize(const svl_model* model, svl_state* state, int64_t n_steps,
                      const uint32_t* audio_tokens, uint32_t* out_tokens);
/* The same, enqueued on the state's stream; device pointers; returns without waiting.  The
 * audio token ids are checked on the device: an id past `card` raises the state's error flag
 * (the step then reads the table's last row) and svl_state_synchronize returns
 * SVL_ERR_INVALID_INPUT, as the synchronous call does for the same input up front. */
int svl_stt_recognize_async(const svl_model* model, svl_state* state, int64_t n_steps,
                            const uint32_t* d_audio_tokens, uint32_t* d_out_tokens);
/* svl_stt_recognize with the extra heads' first-class probabilities of every step
 * (Prediction::extra_head_probabilities, SVL/stt/model.rs:259-271, as the recognizer's turn
 * detection reads them, SVL/stt/mod.rs:327-350): out_probs [n_steps][batch][extra_heads_num].
 * Host pointers. */
int svl_stt_recognize_heads(const svl_model* model, svl_state* state, int64_t n_steps,
                            const uint32_t* audio_tokens, uint32_t* out_tokens, float* out_probs);
/* The same with device pointers, enqueued on the state's stream; d_out_probs may be NULL. */
int svl_stt_recognize_heads_async(const svl_model* model, svl_state* state, int64_t n_steps,
                                  const uint32_t* d_audio_tokens, uint32_t* d_out_tokens,
                                  float* d_out_probs);

/* TurnDetector's parameters (SVL/stt/mod.rs:283-325): `threshold` (default 0.5), `frames`
 * (consecutive frames above it that end a turn; default 1, values below 1 count as 1) and `head`
 * (the extra head whose first-class probability is read; TurnDetector::HEAD = 2). */
typedef struct {
    float threshold;
    int32_t frames;
    int32_t head;
} svl_turn_config;

/* svl_stt_recognize_heads with the end-of-turn signal computed on the device: for every step and
 * stream, out_turn_ends [n_steps][batch] = TurnDetector::update (SVL/stt/mod.rs:327-350) over
 * the step's events in the recognizer's order (:566-589): the VoiceActivity event of the extra
 * heads' probabilities (when the model has extra heads), then the Word events -- a padding token
 * (0 = end of padding, 3 = padding) after pending word tokens (ids above 3) emits them; the
 * tokenizer is taken to decode such a run to at least one word.  The recognizer's pending word
 * tokens and the detector's state are kept per stream in the state (cleared by svl_state_reset);
 * the detector's part changes only in calls that ask for turn ends.  out_probs may be NULL.  The
 * probabilities are within a few ulp of the C library's softmax, so a frame whose probability is
 * that close to the threshold may count differently.  Host pointers. */
int svl_stt_recognize_turns(const svl_model* model, svl_state* state, int64_t n_steps, const uint32_t* audio_tokens,
                            const svl_turn_config* turn, uint32_t* out_tokens, float* out_probs,
                            int32_t* out_turn_ends);
/* The same with device pointers, enqueued on the state's stream; d_out_probs may be NULL. */
int svl_stt_recognize_turns_async(const svl_model* model, svl_state* state, int64_t n_steps,
                                  const uint32_t* d_audio_tokens, const svl_turn_config* turn,
                                  uint32_t* d_out_tokens, float* d_out_probs, int32_t* d_out_turn_ends);

/* svl_stt_recognize without any allocation: no counterpart in the reference; for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The device copies of the audio and output tokens go through a
 * library-owned scratch of 2 MiB per GPU instead of buffers allocated per call, so
 * n_steps * batch * (n_q + 1) * 4 bytes must fit in it (SVL_ERR_INVALID_INPUT otherwise), and
 * every position must be covered by the model's precomputed RoPE table (65536 positions).
 * Calls on one GPU share its scratch; the library runs them one at a time.  Host pointers. */
int svl_stt_recognize_noalloc(const svl_model* model, svl_state* state, int64_t n_steps,
                              const uint32_t* audio_tokens, uint32_t* out_tokens);

/* FlowLm::step's backbone (SVL/tts/flow_lm.rs:169-180) for every stream: latent
 * [batch][latent_dim] f32, or NULL for the learnt `bos_emb` -> z [batch][z_dim or d_model]. */
int svl_tts_backbone_step(const svl_model* model, svl_state* state, const float* latent,
                          float* out_z);

/* FlowLm::step (SVL/tts/flow_lm.rs:162-185) for every stream: the backbone on latent
 * [batch][latent_dim] (NULL: the learnt bos_emb), the end-of-speech logit out_eos(z) and the
 * flow head's decode of `noise` [batch][latent_dim] in `decode_steps` steps (<= 0 counts as 1)
 * -> out_latent [batch][latent_dim], out_eos_logit [batch] (may be NULL) and out_eos [batch]
 * (logit > eos_threshold; may be NULL).  The noise is the caller's draw (Sampling's temperature
 * and clamp, `sample_noise`, :187-203), so that the caller's RNG stream is kept.  Host pointers.
 * The first call with a given decode_steps computes and keeps that count's time conditioning
 * (it waits for the state's stream once). */
int svl_tts_step(const svl_model* model, svl_state* state, const float* latent, const float* noise,
                 int32_t decode_steps, float eos_threshold, float* out_latent, float* out_eos_logit,
                 int32_t* out_eos);
/* The same with device pointers, enqueued on the state's stream: no host round trip per frame
 * (the reference reads the logit back with to_vec1, :181).  d_latent may be the previous call's
 * d_out_latent; d_out_eos_logit may be NULL. */
int svl_tts_step_async(const svl_model* model, svl_state* state, const float* d_latent, const float* d_noise,
                       int32_t decode_steps, float* d_out_latent, float* d_out_eos_logit);

/* ---- the STT audio-token producer's quantizer ----------------------------------------------- */

/* Mimi's split residual vector quantizer, encoding only (SVL/stt/model.rs:84-174;
 * Quantizer::new, :93-98, binds `n_q` codebooks of `bins` entries).  Tensors (f32, bf16 or f16):
 *   rvq_first.input_proj.weight, rvq_rest.input_proj.weight        [256, 512, 1] or [256, 512]
 *   rvq_first.vq.layers.0._codebook.embedding_sum                   [bins, 256]
 *   rvq_first.vq.layers.0._codebook.cluster_usage                   [bins]
 *   rvq_rest.vq.layers.<i>._codebook.{embedding_sum, cluster_usage} for i < n_q - 1
 * (the names under the checkpoint's `quantizer.` prefix, SVL/stt/mod.rs:196). */
typedef struct svl_rvq svl_rvq;
int svl_rvq_create(const svl_tensor* tensors, size_t count, int32_t n_q, int32_t bins, int device,
                   svl_rvq** out);
void svl_rvq_destroy(svl_rvq* rvq);
/* Quantizer::encode (:101-104): latents [batch][512][frames] f32 -> codes [batch][frames][n_q].
 * Host pointers. */
int svl_rvq_encode(svl_rvq* rvq, int32_t batch, int32_t frames, const float* latents, uint32_t* codes);
/* The same on device buffers, enqueued on the quantizer's stream; svl_rvq_synchronize waits. */
int svl_rvq_encode_async(svl_rvq* rvq, int32_t batch, int32_t frames, const float* d_latents,
                         uint32_t* d_codes);
int svl_rvq_synchronize(svl_rvq* rvq);

#ifdef __cplusplus
}
#endif
#endif
