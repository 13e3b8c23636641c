// libsvl: the C ABI of include/svl.h on top of the step kernels.
//
// Reference (crates/semantic-voice-local/src = SVL) behaviour mirrored here:
//   Transformer / Layer / Attention / FeedForwardLayer   SVL/nn/transformer.rs:106-465
//   Linear::from_weight (quantize at load)               SVL/nn/mod.rs:76-87
//   LanguageModel::step / Recognizer::step               SVL/stt/model.rs:239-276, SVL/stt/mod.rs:551-566
//   FlowLm::step backbone                                SVL/tts/flow_lm.rs:162-181
//   FlowLm::step heads: out_eos, FlowHead::decode         SVL/tts/flow_lm.rs:181-185, 206-387
//   TransformerState duplicate / from_layer_caches       SVL/nn/transformer.rs:58-104
// The KV cache is a ring of `context` slots per layer (or `capacity` slots without a window):
// key j of a stream lives in slot j % slots.  The reference's compacting cache
// (transformer.rs:467-551) exposes exactly the last `context` keys to a one-step query, which
// is the ring's content.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/svl.h"
#include "../../include/svl_bench.h"
#include "flow_head.h"
#include "kernels.h"
#include "rvq.h"

using namespace svl;

namespace {

thread_local std::string g_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                                          \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess)                                                                      \
      return set_error(SVL_ERR_DEVICE, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                       __FILE__, __LINE__);                                                    \
  } while (0)

#define TRY(expr)          \
  do {                     \
    int rc_ = (expr);      \
    if (rc_ != 0) return rc_; \
  } while (0)

struct Layer {
  float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
  float *ls1 = nullptr, *ls2 = nullptr;
  LinearDev in_proj, out_proj, ff1, ff2;
};

const svl_tensor* find_tensor(const svl_tensor* ts, size_t n, const std::string& name) {
  for (size_t i = 0; i < n; ++i)
    if (ts[i].name && name == ts[i].name) return &ts[i];
  return nullptr;
}

size_t numel(const svl_tensor* t) {
  if (t->ndim < 0 || t->ndim > 5) return 0;  // svl_tensor::shape holds 5 dimensions
  size_t n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= (size_t)t->shape[i];
  return n;
}

size_t dtype_bytes(int dtype) { return dtype == SVL_F32 ? 4 : 2; }

}  // namespace

struct svl_model {
  svl_config cfg{};
  int device = 0;
  std::vector<void*> allocs;
  std::vector<Layer> layers;
  // RoPE cos/sin of every position below rope_len: [rope_len][head_dim / 2][2], computed on
  // the host with the C library's cosf/sinf (SVL/nn/transformer.rs:114-118, 161-172) and
  // grown by doubling up to rope_cap positions (65536 by default: 32 MiB at head_dim 128).
  // Superseded tables stay allocated until the model is destroyed, since kernels already
  // enqueued may still read them; all of them together hold fewer than 2 rope_cap rows.
  // Positions from rope_cap on get their rows per call, in the state (prepare_rope).
  mutable std::mutex rope_mu;
  mutable float* rope = nullptr;
  mutable int64_t rope_len = 0;
  mutable std::vector<void*> rope_old;
  int64_t rope_cap = 65536;
  // STT
  void* text_emb = nullptr;
  void* emb = nullptr;  // n_q tables back to back
  int tables_bf16 = 0;
  float* out_norm_w = nullptr;
  float* out_norm_b = nullptr;
  LinearDev text_linear;
  LinearDev extra_heads;  // the extra heads' weights stacked: [extra_heads_num * extra_heads_dim][d]
  // TTS
  LinearDev input_linear, z_proj;
  float* bos = nullptr;
  // TTS flow head (FlowHead, SVL/tts/flow_lm.rs:206-387) and out_eos (:109-112), f32
  struct Flow {
    int dim = 0, depth = 0, kind = 0, n_time = 0, latent = 0, cond = 0;
    int mod_rows = 0;           // depth * 3 dim (ResBlock modulations) + 2 dim (final layer)
    FhLinear ce;                // cond_embed rows [0, dim) and out_eos row dim, stacked
    FhLinear in;                // input_proj
    FhLinear mod;               // every adaLN_modulation.1 stacked (they share the input silu(y))
    std::vector<FhLinear> m1, m2;
    std::vector<float*> lnw, lnb;
    FhLinear fl;                // final_layer.linear
    FhLinear t1[2], t2[2];      // TimestepEmbedder mlp.0 / mlp.2
    float* talpha[2] = {nullptr, nullptr};
    std::vector<float> freqs[2];  // host copies: the embedders' cos/sin are computed on the host
    // time conditioning of each flow step, by step count: [steps][dim] (computed on first use)
    std::map<int, float*> tmean;
  } flow;
  mutable std::mutex flow_mu;
  hipStream_t stream = nullptr;  // used at creation only

  ~svl_model() {
    hipSetDevice(device);
    for (void* p : allocs) hipFree(p);
    for (void* p : rope_old) hipFree(p);
    if (rope) hipFree(rope);
    if (stream) hipStreamDestroy(stream);
  }

  int alloc(void** p, size_t bytes) {
    HIP_TRY(hipMalloc(p, bytes ? bytes : 16));
    allocs.push_back(*p);
    return 0;
  }
};

struct Program {
  std::vector<Phase> phases;
  Phase* dev = nullptr;  // device copy
  size_t smem = 0;       // dynamic LDS of the largest phase
};

struct svl_state {
  const svl_model* m = nullptr;
  int B = 1;
  int slots = 0;  // ring slots per stream and layer
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;
  std::vector<void*> kc, vc;  // per layer [B][KVH][slots][hd]
  int* pos = nullptr;
  std::vector<int64_t> pos_host;
  int* attn_order = nullptr;     // [B] streams by visible keys, longest first (attention units)
  std::vector<int> order_host, order_tmp;
  uint32_t* fb_tok = nullptr;
  float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr, *z = nullptr;
  float* in = nullptr;        // TTS latent staging [B][latent_dim]
  // TTS flow head: cond_embed + out_eos [B][dim + 1], modulations [B][mod_rows], residual stream
  // and MLP hidden [B][dim], the sample and the noise [B][latent_dim]
  float *fh_ce = nullptr, *fh_mod = nullptr, *fh_h = nullptr, *fh_a = nullptr, *fh_x = nullptr, *fh_noise = nullptr;
  float* xlogits = nullptr;   // STT extra heads: logits [B][nh * hd]
  float* xprob = nullptr;     //                  first-class probabilities [B][nh]
  uint32_t* turn_state = nullptr;  // STT: pending word tokens and turn detector per stream [B], then
                                   // the detector's threshold, frames and head of the current call
  float* fwd = nullptr;       // transformer forward staging (input then output)
  size_t fwd_cap = 0;
  uint32_t* tok_in = nullptr; // explicit tokens staging [B] + [B][n_q]
  void* stage = nullptr;      // STT: next step's audio embedding rows [B][n_q][d]
  int8_t* xqb = nullptr;      // batched Q8_0 path: quantized input rows [width / 128][B][128]
  float* xdqb = nullptr;      //                    and their block scales [B][width / 32]
  uint32_t* tok_out = nullptr;  // [B] tokens, then the bad-token flag (EmbedArgs::bad_token)
  // RoPE rows of positions at or past the model table's cap, computed for each call
  float* rope_ovf = nullptr;     // device [ovf_rows][head_dim]
  int64_t ovf_rows = 0;
  int* rope_delta = nullptr;     // device [B]: a stream's position p reads row p + delta
  float* ovf_host = nullptr;     // pinned staging of the rows and deltas
  size_t ovf_host_bytes = 0;
  hipEvent_t ovf_copied = nullptr;  // the last staging copy has been read
  // step programs and the grid barrier of the persistent kernel
  Program stt, tts, fwd_prog;
  SyncState* sync = nullptr;
  unsigned gen = 0;
  int grid = 0;
  bool persistent = true;
  // split attention (per-phase launches of few streams): up to split_max units per head, one per
  // split_keys visible keys; per-head rows of tagged scores [B * H][slots] and the tag of the last
  // split launch (split_gen); split_used: a split launch ran since the last check of the abort flag
  int split_max = 1, split_min = 2, split_keys = 0;  // split_min: the fewest units whose LDS fits
  uint64_t* split_scores = nullptr;
  unsigned split_gen = 0;
  bool split_used = false;
  size_t lds_budget = 0;  // dynamic LDS a step launch may request on this device
  // Prefill (Transformer::forward with T > 1 positions, unlimited context): the positions of a
  // block run as the batch rows of a shadow state whose ring is this state's (kv_group rows per
  // stream), so that one pass of the step's phases processes the whole block.
  int kv_group = 1;
  bool owns_stream = true;
  svl_state* shadow = nullptr;
  std::vector<int> pos_stage;  // host staging of positions uploaded by a call (waited for in it)

  ~svl_state() {
    hipSetDevice(m->device);
    if (stream) hipStreamSynchronize(stream);
    delete shadow;
    for (void* p : allocs) hipFree(p);
    if (rope_ovf) hipFree(rope_ovf);
    if (ovf_host) hipHostFree(ovf_host);
    if (ovf_copied) hipEventDestroy(ovf_copied);
    if (stream && owns_stream) hipStreamDestroy(stream);
  }
  int alloc(void** p, size_t bytes) {
    HIP_TRY(hipMalloc(p, bytes ? bytes : 16));
    allocs.push_back(*p);
    return 0;
  }
};

// Mimi's split residual vector quantizer (encoding): input projections, prepared codebooks and the
// work buffers of a call, on its own stream.
struct svl_rvq {
  int device = 0, n_q = 0, bins = 0;
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;
  float* w = nullptr;               // input_proj of the first and the rest quantizer [2][256][512]
  float *emb = nullptr, *hn = nullptr;  // codebooks [n_q][bins][256] and half norms [n_q][bins]
  // per-call work for up to rows_cap rows: projections [2][rows][256], residuals [2][rows][256],
  // keys [n_q][rows], and the staging of the host-pointer call
  int64_t rows_cap = 0;
  float *proj = nullptr, *res = nullptr, *lat = nullptr;
  unsigned long long* keys = nullptr;
  uint32_t* codes = nullptr;

  ~svl_rvq() {
    hipSetDevice(device);
    if (stream) hipStreamSynchronize(stream);
    free_work();
    for (void* p : allocs) hipFree(p);
    if (stream) hipStreamDestroy(stream);
  }
  void free_work() {
    for (void* p : {(void*)proj, (void*)res, (void*)lat, (void*)keys, (void*)codes})
      if (p) hipFree(p);
    proj = res = lat = nullptr;
    keys = nullptr;
    codes = nullptr;
    rows_cap = 0;
  }
};

namespace {

// Copies a dense tensor of n elements to device memory dst as f32 (converted on the GPU from
// bf16/f16).
int copy_f32_on(hipStream_t stream, const svl_tensor* t, size_t n, void* dst) {
  if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor");
  if (numel(t) != n)
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: %zu elements, expected %zu", t->name, numel(t), n);
  if (t->dtype == SVL_F32) {
    HIP_TRY(hipMemcpy(dst, t->data, n * 4, hipMemcpyHostToDevice));
  } else if (t->dtype == SVL_BF16 || t->dtype == SVL_F16) {
    void* tmp;
    HIP_TRY(hipMalloc(&tmp, n * 2));
    HIP_TRY(hipMemcpy(tmp, t->data, n * 2, hipMemcpyHostToDevice));
    hipError_t e = t->dtype == SVL_BF16 ? launch_bf16_to_f32((const uint16_t*)tmp, (float*)dst, n, stream)
                                         : launch_f16_to_f32((const uint16_t*)tmp, (float*)dst, n, stream);
    hipError_t e2 = hipStreamSynchronize(stream);
    hipFree(tmp);
    HIP_TRY(e);
    HIP_TRY(e2);
  } else {
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: dense dtype expected", t->name);
  }
  return 0;
}

int copy_f32(svl_model* m, const svl_tensor* t, size_t n, void* dst) { return copy_f32_on(m->stream, t, n, dst); }

// Uploads a dense tensor as f32 into a new model allocation.
int upload_f32(svl_model* m, const svl_tensor* t, size_t n, float** out) {
  if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor");
  if (numel(t) != n)
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: %zu elements, expected %zu", t->name, numel(t), n);
  void* dst;
  TRY(m->alloc(&dst, n * 4));
  TRY(copy_f32(m, t, n, dst));
  *out = (float*)dst;
  return 0;
}

int load_vec(svl_model* m, const svl_tensor* ts, size_t n, const std::string& name, size_t count, float** out) {
  const svl_tensor* t = find_tensor(ts, n, name);
  if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", name.c_str());
  return upload_f32(m, t, count, out);
}

// Linear::from_weight (SVL/nn/mod.rs:76-87): candle blocks are repacked; dense weights are
// quantized on the GPU when `quantize` asks for it and the input width is a multiple of the
// block, kept dense (f32 or bf16) otherwise.
int load_linear(svl_model* m, const svl_tensor* ts, size_t n, const std::string& name, int out_f, int in_f,
                int quantize, LinearDev* L) {
  const svl_tensor* t = find_tensor(ts, n, name);
  if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", name.c_str());
  if (t->ndim != 2 || t->shape[0] != out_f || t->shape[1] != in_f)
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: shape mismatch (expected [%d, %d])", name.c_str(), out_f, in_f);
  L->out = out_f;
  L->in = in_f;
  const size_t count = (size_t)out_f * in_f;
  if (t->dtype == SVL_Q4K) {
    if (in_f % 256) return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: Q4K needs in %% 256 == 0", name.c_str());
    const size_t bytes = count / 256 * 144;
    void *w, *tmp;
    TRY(m->alloc(&w, bytes));
    HIP_TRY(hipMalloc(&tmp, bytes));
    HIP_TRY(hipMemcpy(tmp, t->data, bytes, hipMemcpyHostToDevice));
    hipError_t e = launch_q4k_from_blocks((const uint8_t*)tmp, out_f, in_f, (uint8_t*)w, m->stream);
    hipError_t e2 = hipStreamSynchronize(m->stream);
    hipFree(tmp);
    HIP_TRY(e);
    HIP_TRY(e2);
    L->fmt = FMT_Q4K;
    L->w = w;
    return 0;
  }
  if (t->dtype == SVL_Q4_0) {
    if (in_f % 32) return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: Q4_0 needs in %% 32 == 0", name.c_str());
    void *qs, *d, *tmp;
    TRY(m->alloc(&qs, count / 2));
    TRY(m->alloc(&d, count / 32 * 2));
    HIP_TRY(hipMalloc(&tmp, count / 32 * 18));
    HIP_TRY(hipMemcpy(tmp, t->data, count / 32 * 18, hipMemcpyHostToDevice));
    hipError_t e = launch_q4_0_from_blocks((const uint8_t*)tmp, out_f, in_f, (uint8_t*)qs, (uint16_t*)d, m->stream);
    hipError_t e2 = hipStreamSynchronize(m->stream);
    hipFree(tmp);
    HIP_TRY(e);
    HIP_TRY(e2);
    L->fmt = FMT_Q4_0;
    L->w = qs;
    L->scale = (uint16_t*)d;
    return 0;
  }
  if (t->dtype == SVL_Q8_0) {
    if (in_f % 32) return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: Q8_0 needs in %% 32 == 0", name.c_str());
    void *qs, *d, *tmp;
    TRY(m->alloc(&qs, count));
    TRY(m->alloc(&d, count / 32 * 2));
    HIP_TRY(hipMalloc(&tmp, count / 32 * 34));
    HIP_TRY(hipMemcpy(tmp, t->data, count / 32 * 34, hipMemcpyHostToDevice));
    hipError_t e = launch_q8_from_blocks((const uint8_t*)tmp, out_f, in_f, (int8_t*)qs, (uint16_t*)d, m->stream);
    hipError_t e2 = hipStreamSynchronize(m->stream);
    hipFree(tmp);
    HIP_TRY(e);
    HIP_TRY(e2);
    L->fmt = FMT_Q8_0;
    L->w = qs;
    L->scale = (uint16_t*)d;
    return 0;
  }
  if (t->dtype != SVL_F32 && t->dtype != SVL_BF16 && t->dtype != SVL_F16)
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: unsupported dtype %d", name.c_str(), t->dtype);
  if (quantize == SVL_Q4K && in_f % 256 == 0) {
    float* f = nullptr;
    TRY(upload_f32(m, t, count, &f));
    void* w;
    TRY(m->alloc(&w, count / 256 * 144));
    HIP_TRY(launch_q4k_quantize(f, out_f, in_f, (uint8_t*)w, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    // the f32 staging copy is released right away
    m->allocs.pop_back();
    m->allocs.pop_back();
    hipFree(f);
    m->allocs.push_back(w);
    L->fmt = FMT_Q4K;
    L->w = w;
    return 0;
  }
  if (quantize == SVL_Q4_0 && in_f % 32 == 0) {
    float* f = nullptr;
    TRY(upload_f32(m, t, count, &f));
    void *qs, *d;
    TRY(m->alloc(&qs, count / 2));
    TRY(m->alloc(&d, count / 32 * 2));
    HIP_TRY(launch_q4_0_quantize(f, out_f, in_f, (uint8_t*)qs, (uint16_t*)d, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    // the f32 staging copy is released right away
    m->allocs.pop_back();
    m->allocs.pop_back();
    m->allocs.pop_back();
    hipFree(f);
    m->allocs.push_back(qs);
    m->allocs.push_back(d);
    L->fmt = FMT_Q4_0;
    L->w = qs;
    L->scale = (uint16_t*)d;
    return 0;
  }
  if (quantize == SVL_Q8_0 && in_f % 32 == 0) {
    float* f = nullptr;
    TRY(upload_f32(m, t, count, &f));
    void *qs, *d;
    TRY(m->alloc(&qs, count));
    TRY(m->alloc(&d, count / 32 * 2));
    HIP_TRY(launch_q8_quantize(f, out_f, in_f, (int8_t*)qs, (uint16_t*)d, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    // the f32 staging copy is released right away
    m->allocs.pop_back();
    m->allocs.pop_back();
    m->allocs.pop_back();
    hipFree(f);
    m->allocs.push_back(qs);
    m->allocs.push_back(d);
    L->fmt = FMT_Q8_0;
    L->w = qs;
    L->scale = (uint16_t*)d;
    return 0;
  }
  if (t->dtype == SVL_BF16) {
    if (in_f % 8) return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: bf16 rows need in %% 8 == 0", name.c_str());
    void* w;
    TRY(m->alloc(&w, count * 2));
    if (in_f % 128 == 0) {  // chain-packed for the weight waves
      void* tmp;
      HIP_TRY(hipMalloc(&tmp, count * 2));
      hipError_t e = hipMemcpy(tmp, t->data, count * 2, hipMemcpyHostToDevice);
      if (e == hipSuccess) e = launch_chain_pack(tmp, 1, out_f, in_f, w, 1, m->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
      hipFree(tmp);
      HIP_TRY(e);
      L->fmt = FMT_BF16C;
    } else {
      HIP_TRY(hipMemcpy(w, t->data, count * 2, hipMemcpyHostToDevice));
      L->fmt = FMT_BF16;
    }
    L->w = w;
    return 0;
  }
  if (in_f % 4) return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: f32 rows need in %% 4 == 0", name.c_str());
  float* f = nullptr;
  TRY(upload_f32(m, t, count, &f));
  if (in_f % 64 == 0) {  // chain-packed for the weight waves
    void* w;
    TRY(m->alloc(&w, count * 4));
    HIP_TRY(launch_chain_pack(f, 0, out_f, in_f, w, 0, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    // the row-major staging copy is released right away
    m->allocs.pop_back();
    m->allocs.pop_back();
    hipFree(f);
    m->allocs.push_back(w);
    L->fmt = FMT_F32C;
    L->w = w;
    return 0;
  }
  L->fmt = FMT_F32;
  L->w = f;
  return 0;
}

// Embedding table `name` ([count] values) copied to `dst` on the device, kept bf16 when every
// table is bf16 and converted to f32 otherwise.
int load_table(svl_model* m, const svl_tensor* ts, size_t n, const std::string& name, size_t count, void* dst) {
  const svl_tensor* t = find_tensor(ts, n, name);
  if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", name.c_str());
  if (numel(t) != count)
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: %zu elements, expected %zu", name.c_str(), numel(t), count);
  if (m->tables_bf16) {
    HIP_TRY(hipMemcpy(dst, t->data, count * 2, hipMemcpyHostToDevice));
    return 0;
  }
  if (t->dtype == SVL_F32) {
    HIP_TRY(hipMemcpy(dst, t->data, count * 4, hipMemcpyHostToDevice));
    return 0;
  }
  if (t->dtype != SVL_BF16 && t->dtype != SVL_F16)
    return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: dense dtype expected", name.c_str());
  void* tmp;
  HIP_TRY(hipMalloc(&tmp, count * 2));
  hipError_t e = hipMemcpy(tmp, t->data, count * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = t->dtype == SVL_BF16 ? launch_bf16_to_f32((const uint16_t*)tmp, (float*)dst, count, m->stream)
                             : launch_f16_to_f32((const uint16_t*)tmp, (float*)dst, count, m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  hipFree(tmp);
  HIP_TRY(e);
  return 0;
}

// inv_freq[i] = exp(-ln(max_period) * 2 i / head_dim) in f64, then f32
// (SVL/nn/transformer.rs:114-118).
std::vector<float> rope_inv_freq(const svl_config& c) {
  std::vector<float> inv(c.head_dim / 2);
  for (int i = 0; i < c.head_dim / 2; ++i)
    inv[i] = (float)std::exp(-(std::log(c.max_period)) * 2.0 * (double)i / (double)c.head_dim);
  return inv;
}

// cos and sin of the f32 angle (f32)p * inv_freq[i] with the C library's cosf / sinf, as the
// reference computes them (SVL/nn/transformer.rs:161-172): row p is [head_dim / 2][cos, sin].
void rope_row(const std::vector<float>& inv, int64_t p, float* row) {
  for (size_t i = 0; i < inv.size(); ++i) {
    const float f = (float)p * inv[i];
    row[2 * i] = ::cosf(f);
    row[2 * i + 1] = ::sinf(f);
  }
}

// Makes the model's RoPE table cover positions [0, min(needed, rope_cap)).
int ensure_rope(const svl_model* m, int64_t needed) {
  std::lock_guard<std::mutex> lock(m->rope_mu);
  needed = std::min(needed, m->rope_cap);
  if (needed <= m->rope_len) return 0;
  int64_t len = m->rope_len ? m->rope_len : std::min<int64_t>(4096, m->rope_cap);
  while (len < needed) len = std::min(2 * len, m->rope_cap);
  const std::vector<float> inv = rope_inv_freq(m->cfg);
  const int hd = m->cfg.head_dim;
  std::vector<float> tab((size_t)len * hd);
  const int nt = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> workers;
  for (int w = 0; w < nt; ++w)
    workers.emplace_back([&, w] {
      for (int64_t p = w; p < len; p += nt) rope_row(inv, p, tab.data() + (size_t)p * hd);
    });
  for (auto& t : workers) t.join();
  void* d;
  HIP_TRY(hipMalloc(&d, tab.size() * 4));
  hipError_t e = hipMemcpy(d, tab.data(), tab.size() * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    hipFree(d);
    HIP_TRY(e);
  }
  if (m->rope) m->rope_old.push_back(m->rope);
  m->rope = (float*)d;
  m->rope_len = len;
  return 0;
}

// LanguageModel::new's extra heads (SVL/stt/model.rs:217-222): extra_heads.{i}.weight, dense
// [extra_heads_dim][d] without bias, loaded unquantized (Linear::load(.., false)).  The heads are
// stacked into one linear of extra_heads_num * extra_heads_dim rows: each output row is its own
// dot product, so stacking changes no arithmetic.
int load_extra_heads(svl_model* m, const svl_tensor* ts, size_t n) {
  const svl_config& c = m->cfg;
  const int nh = c.extra_heads_num, hd = c.extra_heads_dim, d = c.d_model;
  if (nh == 0) return 0;
  if (nh < 0 || nh > 256 || hd <= 0 || hd > 4096)
    return set_error(SVL_ERR_CONFIG, "extra heads: need 0 <= extra_heads_num <= 256 and 1 <= extra_heads_dim <= 4096");
  int dtype = -1;
  std::vector<const svl_tensor*> parts(nh);
  for (int i = 0; i < nh; ++i) {
    const std::string name = "extra_heads." + std::to_string(i) + ".weight";
    const svl_tensor* t = find_tensor(ts, n, name);
    if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", name.c_str());
    if (t->ndim != 2 || t->shape[0] != hd || t->shape[1] != d)
      return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: shape mismatch (expected [%d, %d])", name.c_str(), hd, d);
    if (t->dtype != SVL_F32 && t->dtype != SVL_BF16 && t->dtype != SVL_F16)
      return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: the extra heads are dense (f32, bf16 or f16)", name.c_str());
    if (dtype >= 0 && t->dtype != dtype)
      return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: the extra heads must share one dtype", name.c_str());
    dtype = t->dtype;
    parts[i] = t;
  }
  const size_t esz = dtype == SVL_F32 ? 4 : 2, one = (size_t)hd * d * esz;
  std::vector<unsigned char> stacked(one * nh);
  for (int i = 0; i < nh; ++i) memcpy(stacked.data() + one * i, parts[i]->data, one);
  svl_tensor all{};
  all.name = "extra_heads";
  all.dtype = dtype;
  all.ndim = 2;
  all.shape[0] = (int64_t)nh * hd;
  all.shape[1] = d;
  all.data = stacked.data();
  return load_linear(m, &all, 1, "extra_heads", nh * hd, d, 0, &m->extra_heads);
}

// Dense f32 linears with bias, stacked row-wise in the order of `parts` ({prefix, rows}: tensors
// prefix + ".weight" [rows][in] and prefix + ".bias" [rows]), chain-packed when in % 64 == 0.
int load_fh_linear(svl_model* m, const svl_tensor* ts, size_t n, const std::vector<std::pair<std::string, int>>& parts,
                   int in, FhLinear* L) {
  int rows = 0;
  for (const auto& p : parts) rows += p.second;
  const size_t count = (size_t)rows * in;
  void *rm = nullptr, *bias = nullptr;
  TRY(m->alloc(&bias, (size_t)rows * 4));
  HIP_TRY(hipMalloc(&rm, count * 4));
  std::unique_ptr<void, void (*)(void*)> rm_guard(rm, [](void* p) { hipFree(p); });
  size_t r0 = 0;
  for (const auto& p : parts) {
    const std::string wn = p.first + ".weight", bn = p.first + ".bias";
    const svl_tensor* w = find_tensor(ts, n, wn);
    if (!w) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", wn.c_str());
    if (w->ndim != 2 || w->shape[0] != p.second || w->shape[1] != in)
      return set_error(SVL_ERR_INVALID_INPUT, "tensor %s: shape mismatch (expected [%d, %d])", wn.c_str(), p.second, in);
    TRY(copy_f32(m, w, (size_t)p.second * in, (float*)rm + r0 * in));
    const svl_tensor* b = find_tensor(ts, n, bn);
    if (!b) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", bn.c_str());
    TRY(copy_f32(m, b, (size_t)p.second, (float*)bias + r0));
    r0 += (size_t)p.second;
  }
  void* w;
  TRY(m->alloc(&w, count * 4));
  if (in % 64 == 0) {
    HIP_TRY(launch_chain_pack(rm, 0, rows, in, w, 0, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    L->packed = 1;
  } else {
    HIP_TRY(hipMemcpy(w, rm, count * 4, hipMemcpyDeviceToDevice));
    L->packed = 0;
  }
  L->w = (const float*)w;
  L->b = (const float*)bias;
  L->out = rows;
  L->in = in;
  return 0;
}

// FlowHead::new (SVL/tts/flow_lm.rs:232-251) with its TimestepEmbedders (:322-331) and ResBlocks
// (:359-368), and out_eos (:109-112), which reads the same z as cond_embed.
int load_flow(svl_model* m, const svl_tensor* ts, size_t n) {
  const svl_config& c = m->cfg;
  svl_model::Flow& F = m->flow;
  F.dim = c.flow_dim;
  F.depth = c.flow_depth;
  F.kind = c.flow_kind;
  F.n_time = c.flow_kind == SVL_FLOW_LSD ? 2 : (c.flow_kind == SVL_FLOW_MATCHING ? 1 : 0);
  F.latent = c.latent_dim;
  F.cond = c.z_dim > 0 ? c.z_dim : c.d_model;
  const int D = F.dim;
  F.mod_rows = F.depth * 3 * D + 2 * D;
  const std::string p = "flow_net.";
  TRY(load_fh_linear(m, ts, n, {{p + "cond_embed", D}, {"out_eos", 1}}, F.cond, &F.ce));
  TRY(load_fh_linear(m, ts, n, {{p + "input_proj", D}}, F.latent, &F.in));
  std::vector<std::pair<std::string, int>> mods;
  for (int j = 0; j < F.depth; ++j) mods.push_back({p + "res_blocks." + std::to_string(j) + ".adaLN_modulation.1", 3 * D});
  mods.push_back({p + "final_layer.adaLN_modulation.1", 2 * D});
  TRY(load_fh_linear(m, ts, n, mods, D, &F.mod));
  F.m1.resize(F.depth);
  F.m2.resize(F.depth);
  F.lnw.resize(F.depth);
  F.lnb.resize(F.depth);
  for (int j = 0; j < F.depth; ++j) {
    const std::string r = p + "res_blocks." + std::to_string(j) + ".";
    TRY(load_fh_linear(m, ts, n, {{r + "mlp.0", D}}, D, &F.m1[j]));
    TRY(load_fh_linear(m, ts, n, {{r + "mlp.2", D}}, D, &F.m2[j]));
    TRY(load_vec(m, ts, n, r + "in_ln.weight", D, &F.lnw[j]));
    TRY(load_vec(m, ts, n, r + "in_ln.bias", D, &F.lnb[j]));
  }
  TRY(load_fh_linear(m, ts, n, {{p + "final_layer.linear", F.latent}}, D, &F.fl));
  for (int i = 0; i < F.n_time; ++i) {
    const std::string t = p + "time_embed." + std::to_string(i) + ".";
    TRY(load_fh_linear(m, ts, n, {{t + "mlp.0", D}}, 256, &F.t1[i]));
    TRY(load_fh_linear(m, ts, n, {{t + "mlp.2", D}}, D, &F.t2[i]));
    TRY(load_vec(m, ts, n, t + "mlp.3.alpha", D, &F.talpha[i]));
    float* fr = nullptr;
    TRY(load_vec(m, ts, n, t + "freqs", 128, &fr));
    F.freqs[i].resize(128);
    HIP_TRY(hipMemcpy(F.freqs[i].data(), fr, 128 * 4, hipMemcpyDeviceToHost));
  }
  return 0;
}

// Configuration errors (what the reference itself rejects or cannot build) are SVL_ERR_CONFIG;
// valid configurations outside what these kernels cover are SVL_UNSUPPORTED, for the caller to
// run the reference's own path (the reference's kernels return None: SVL/nn/kernels/matvec.rs:12-17).
int check_config(const svl_config* c) {
  if (c->d_model <= 0 || c->num_layers <= 0 || c->num_heads <= 0 || c->num_kv_heads <= 0 || c->head_dim <= 0)
    return set_error(SVL_ERR_CONFIG, "invalid transformer dimensions");
  if (c->num_heads % c->num_kv_heads) return set_error(SVL_ERR_CONFIG, "num_heads must be a multiple of num_kv_heads");
  if (c->ff_hidden <= 0) return set_error(SVL_ERR_CONFIG, "ff_hidden must be positive");
  if (c->norm_kind != SVL_NORM_LAYER && c->norm_kind != SVL_NORM_RMS) return set_error(SVL_ERR_CONFIG, "unknown norm");
  if (c->ff_kind != SVL_FF_PLAIN_GELU && c->ff_kind != SVL_FF_GATED_SILU && c->ff_kind != SVL_FF_PLAIN_GELU_ERF)
    return set_error(SVL_ERR_CONFIG, "unknown feed-forward");
  if (c->context < 0) return set_error(SVL_ERR_CONFIG, "context must be >= 0");
  if (c->kv_dtype != SVL_F32 && c->kv_dtype != SVL_BF16) return set_error(SVL_ERR_CONFIG, "kv_dtype must be F32 or BF16");
  if (c->quantize != 0 && c->quantize != SVL_Q8_0 && c->quantize != SVL_Q4_0 && c->quantize != SVL_Q4K)
    return set_error(SVL_ERR_CONFIG, "quantize must be 0, Q8_0, Q4_0 or Q4K");
  if (c->kind == SVL_MODEL_STT && (c->n_q <= 0 || c->card <= 0 || c->text_card <= 0))
    return set_error(SVL_ERR_CONFIG, "invalid STT heads");
  if (c->kind == SVL_MODEL_TTS && c->latent_dim <= 0) return set_error(SVL_ERR_CONFIG, "invalid TTS latent_dim");
  // shapes the kernels do not cover
  if (c->head_dim != 64 && c->head_dim != 128) return set_error(SVL_UNSUPPORTED, "head_dim must be 64 or 128");
  if (c->d_model % 32) return set_error(SVL_UNSUPPORTED, "d_model must be a multiple of 32");
  if (c->ff_hidden % 32) return set_error(SVL_UNSUPPORTED, "ff_hidden must be a multiple of 32");
  if ((c->num_heads * c->head_dim) % 32) return set_error(SVL_UNSUPPORTED, "attention width must be a multiple of 32");
  // a GEMV input row is held by 512 row-wave threads, 16 elements each (8 for normalized rows)
  if (c->d_model > 4096) return set_error(SVL_UNSUPPORTED, "d_model must be <= 4096");
  if (c->ff_hidden > 8192 || c->num_heads * c->head_dim > 8192)
    return set_error(SVL_UNSUPPORTED, "ff_hidden and num_heads * head_dim must be <= 8192");
  // the ring buffer of a stream and layer (attention stages a head's scores over it in LDS)
  if (c->context > kMaxRingSlots) return set_error(SVL_UNSUPPORTED, "context must be <= %d", kMaxRingSlots);
  if (c->kind == SVL_MODEL_STT && c->n_q > 64) return set_error(SVL_UNSUPPORTED, "n_q must be <= 64");
  if (c->kind == SVL_MODEL_TTS && c->latent_dim % 4) return set_error(SVL_UNSUPPORTED, "latent_dim must be a multiple of 4");
  if (c->kind == SVL_MODEL_TTS && c->flow_dim != 0) {
    if (c->flow_dim < 0 || c->flow_depth < 0 || c->flow_kind < SVL_FLOW_LSD || c->flow_kind > SVL_FLOW_POINTWISE)
      return set_error(SVL_ERR_CONFIG, "invalid flow head config");
    const int cond = c->z_dim > 0 ? c->z_dim : c->d_model;
    if (c->flow_dim > kFhMaxWidth || cond > kFhMaxWidth || c->latent_dim > kFhMaxWidth)
      return set_error(SVL_UNSUPPORTED, "flow head widths must be <= %d", kFhMaxWidth);
  }
  return 0;
}

int create_model(const svl_config* cfg, const svl_tensor* ts, size_t n, svl_model* m) {
  const svl_config& c = *cfg;
  TRY(check_config(cfg));
  HIP_TRY(hipStreamCreate(&m->stream));
  const std::string pre = c.kind == SVL_MODEL_TRANSFORMER ? "" : "transformer.";
  const int d = c.d_model, hd = c.head_dim;
  const int qdim = c.num_heads * hd, kvdim = c.num_kv_heads * hd;
  m->layers.resize(c.num_layers);
  for (int i = 0; i < c.num_layers; ++i) {
    Layer& L = m->layers[i];
    const std::string p = pre + "layers." + std::to_string(i) + ".";
    if (c.norm_kind == SVL_NORM_RMS) {
      TRY(load_vec(m, ts, n, p + "norm1.alpha", d, &L.n1w));
      TRY(load_vec(m, ts, n, p + "norm2.alpha", d, &L.n2w));
    } else {
      TRY(load_vec(m, ts, n, p + "norm1.weight", d, &L.n1w));
      TRY(load_vec(m, ts, n, p + "norm1.bias", d, &L.n1b));
      TRY(load_vec(m, ts, n, p + "norm2.weight", d, &L.n2w));
      TRY(load_vec(m, ts, n, p + "norm2.bias", d, &L.n2b));
    }
    if (c.layer_scale) {
      TRY(load_vec(m, ts, n, p + "layer_scale_1.scale", d, &L.ls1));
      TRY(load_vec(m, ts, n, p + "layer_scale_2.scale", d, &L.ls2));
    }
    std::string inp = p + "self_attn.in_proj_weight";
    if (!find_tensor(ts, n, inp)) inp = p + "self_attn.in_proj.weight";
    TRY(load_linear(m, ts, n, inp, qdim + 2 * kvdim, d, c.quantize, &L.in_proj));
    TRY(load_linear(m, ts, n, p + "self_attn.out_proj.weight", d, qdim, c.quantize, &L.out_proj));
    if (c.ff_kind == SVL_FF_GATED_SILU) {
      TRY(load_linear(m, ts, n, p + "gating.linear_in.weight", 2 * c.ff_hidden, d, c.quantize, &L.ff1));
      TRY(load_linear(m, ts, n, p + "gating.linear_out.weight", d, c.ff_hidden, c.quantize, &L.ff2));
    } else {
      TRY(load_linear(m, ts, n, p + "linear1.weight", c.ff_hidden, d, c.quantize, &L.ff1));
      TRY(load_linear(m, ts, n, p + "linear2.weight", d, c.ff_hidden, c.quantize, &L.ff2));
    }
  }
  TRY(ensure_rope(m, m->rope_cap));  // the whole table up front: steps never allocate for it
  if (c.kind == SVL_MODEL_STT) {
    bool all_bf16 = true;
    const svl_tensor* te = find_tensor(ts, n, "text_emb.weight");
    if (!te) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor text_emb.weight");
    all_bf16 = te->dtype == SVL_BF16;
    for (int i = 0; i < c.n_q && all_bf16; ++i) {
      const svl_tensor* t = find_tensor(ts, n, "emb." + std::to_string(i) + ".weight");
      all_bf16 = t && t->dtype == SVL_BF16;
    }
    m->tables_bf16 = all_bf16 ? 1 : 0;
    const size_t esz = m->tables_bf16 ? 2 : 4;
    const size_t rows = (size_t)(c.card + 1) * d;
    TRY(m->alloc(&m->text_emb, (size_t)(c.text_card + 1) * d * esz));
    TRY(load_table(m, ts, n, "text_emb.weight", (size_t)(c.text_card + 1) * d, m->text_emb));
    TRY(m->alloc(&m->emb, rows * c.n_q * esz));
    for (int i = 0; i < c.n_q; ++i)
      TRY(load_table(m, ts, n, "emb." + std::to_string(i) + ".weight", rows, (char*)m->emb + rows * i * esz));
    TRY(load_vec(m, ts, n, "out_norm.alpha", d, &m->out_norm_w));
    TRY(load_linear(m, ts, n, "text_linear.weight", c.text_card, d, c.quantize, &m->text_linear));
    TRY(load_extra_heads(m, ts, n));
  } else if (c.kind == SVL_MODEL_TTS) {
    // input_linear, z_proj: always dense (Linear::new, SVL/tts/flow_lm.rs:72-74)
    TRY(load_linear(m, ts, n, "input_linear.weight", d, c.latent_dim, 0, &m->input_linear));
    TRY(load_vec(m, ts, n, "out_norm.weight", d, &m->out_norm_w));
    TRY(load_vec(m, ts, n, "out_norm.bias", d, &m->out_norm_b));
    if (c.z_dim > 0) TRY(load_linear(m, ts, n, "z_proj.weight", c.z_dim, d, 0, &m->z_proj));
    TRY(load_vec(m, ts, n, "bos_emb", c.latent_dim, &m->bos));
    if (c.flow_dim > 0) TRY(load_flow(m, ts, n));
  }
  HIP_TRY(hipDeviceSynchronize());
  return 0;
}

const LinearDev* find_linear(const svl_model* m, const char* name) {
  if (!strcmp(name, "text_linear")) return m->cfg.kind == SVL_MODEL_STT ? &m->text_linear : nullptr;
  if (!strcmp(name, "extra_heads")) return m->cfg.kind == SVL_MODEL_STT && m->cfg.extra_heads_num > 0 ? &m->extra_heads : nullptr;
  if (!strcmp(name, "input_linear")) return m->cfg.kind == SVL_MODEL_TTS ? &m->input_linear : nullptr;
  if (!strcmp(name, "z_proj")) return m->cfg.z_dim > 0 ? &m->z_proj : nullptr;
  int layer = -1;
  char which[64] = {0};
  if (sscanf(name, "%d.%63s", &layer, which) != 2 || layer < 0 || layer >= m->cfg.num_layers) return nullptr;
  const Layer& L = m->layers[layer];
  if (!strcmp(which, "in_proj")) return &L.in_proj;
  if (!strcmp(which, "out_proj")) return &L.out_proj;
  if (!strcmp(which, "ff1")) return &L.ff1;
  if (!strcmp(which, "ff2")) return &L.ff2;
  return nullptr;
}

int norm_code(const svl_config& c) { return c.norm_kind == SVL_NORM_RMS ? NORM_RMS : NORM_LAYER; }

Phase gemv_phase(const svl_state* s, const LinearDev& L) {
  Phase ph{};
  ph.kind = PH_GEMV;
  ph.g.L = L;
  ph.g.B = s->B;
  return ph;
}

// A Q8_0 linear of a lockstep batch of at least kBatchMfma streams runs as two phases: the
// input rows are normalized and quantized once (PH_QUANT, one unit per stream), then an MFMA
// GEMM reads every weight block once per 64 streams (PH_QGEMM; its weight scales travel as f16
// pairs, so the input width must be a multiple of 64).  Otherwise one GEMV phase.
void add_gemv(const svl_state* s, std::vector<Phase>& out, Phase ph) {
  if (ph.g.L.fmt == FMT_Q8_0 && s->B >= kBatchMfma && ph.g.L.in % 64 == 0) {
    ph.g.xq = s->xqb;
    ph.g.xdq = s->xdqb;
    Phase q = ph;
    q.kind = PH_QUANT;
    q.units = s->B;
    out.push_back(q);
    ph.kind = PH_QGEMM;
    plan_qgemm(ph.g, s->grid, &ph.units);
    out.push_back(ph);
    return;
  }
  plan_gemv(ph.g, s->grid, &ph.units);
  out.push_back(ph);
}

// The layers of one step (Layer::forward, SVL/nn/transformer.rs:222-250): s->x in, s->x out.
// The last layer's feed-forward output advances the positions: no later phase of the step
// reads them.
void build_layers(const svl_model* m, const svl_state* s, std::vector<Phase>& out) {
  const svl_config& c = m->cfg;
  const int d = c.d_model, hd = c.head_dim, H = c.num_heads, KVH = c.num_kv_heads;
  const int kv_bf16 = c.kv_dtype == SVL_BF16;
  for (int i = 0; i < c.num_layers; ++i) {
    const Layer& L = m->layers[i];
    // norm1 -> in_proj -> RoPE(q, k) -> q buffer and KV ring
    Phase g = gemv_phase(s, L.in_proj);
    g.g.x = s->x;
    g.g.x_stride = d;
    g.g.norm = norm_code(c);
    g.g.nw = L.n1w;
    g.g.nb = L.n1b;
    g.g.eps = c.norm_eps;
    g.g.epi = EPI_QKV_ROPE;
    g.g.pos = s->pos;
    g.g.rope = nullptr;  // set per launch (the table grows)
    g.g.rope_cap = (int)m->rope_cap;
    g.g.rope_ovf = nullptr;
    g.g.rope_delta = s->rope_delta;
    g.g.H = H;
    g.g.KVH = KVH;
    g.g.hd = hd;
    g.g.q_out = s->q;
    g.g.kc = s->kc[i];
    g.g.vc = s->vc[i];
    g.g.cap = s->slots;
    g.g.kv_bf16 = kv_bf16;
    g.g.kv_group = s->kv_group;
    add_gemv(s, out, g);
    // attention over the ring
    Phase a{};
    a.at.q = s->q;
    a.at.kc = s->kc[i];
    a.at.vc = s->vc[i];
    a.at.pos = s->pos;
    a.at.B = s->B;
    a.at.H = H;
    a.at.KVH = KVH;
    a.at.hd = hd;
    a.at.cap = s->slots;
    a.at.window = c.context;
    a.at.kv_bf16 = kv_bf16;
    a.at.scale = std::pow((float)hd, -0.5f);  // (d as f32).powf(-0.5), attention.rs:100
    a.at.out = s->att;
    a.at.order = s->attn_order;
    a.at.kv_group = s->kv_group;
    // two heads per unit once the batch has at least two units per workgroup without pairing
    // (SVL_ATTN_PAIRS=1 forces pairs, for tests)
    const char* pairs = getenv("SVL_ATTN_PAIRS");
    a.at.hpu = H % 2 == 0 && (s->B * H >= 2 * s->grid || (pairs && !strcmp(pairs, "1"))) ? 2 : 1;
    a.kind = PH_ATTN;
    if (a.at.hpu == 2 && phase_smem(a) > s->lds_budget) a.at.hpu = 1;  // two heads' scores do not fit
    a.units = s->B * H / a.at.hpu;
    out.push_back(a);
    // out_proj + residual (layer scale if any)
    Phase o = gemv_phase(s, L.out_proj);
    o.g.x = s->att;
    o.g.x_stride = H * hd;
    o.g.norm = NORM_NONE;
    o.g.epi = EPI_RESID;
    o.g.resid = s->x;
    o.g.resid_stride = d;
    o.g.lscale = L.ls1;
    add_gemv(s, out, o);
    // norm2 -> feed-forward in (SiLU gate or GELU)
    Phase f = gemv_phase(s, L.ff1);
    f.g.x = s->x;
    f.g.x_stride = d;
    f.g.norm = norm_code(c);
    f.g.nw = L.n2w;
    f.g.nb = L.n2b;
    f.g.eps = c.norm_eps;
    f.g.y = s->h;
    f.g.y_stride = c.ff_hidden;
    if (c.ff_kind == SVL_FF_GATED_SILU) {
      f.g.epi = EPI_SILU_GATE;
      f.g.ff_hidden = c.ff_hidden;
    } else {
      f.g.epi = c.ff_kind == SVL_FF_PLAIN_GELU_ERF ? EPI_GELU_ERF : EPI_GELU;
    }
    add_gemv(s, out, f);
    // feed-forward out + residual
    Phase f2 = gemv_phase(s, L.ff2);
    f2.g.x = s->h;
    f2.g.x_stride = c.ff_hidden;
    f2.g.norm = NORM_NONE;
    f2.g.epi = EPI_RESID;
    f2.g.resid = s->x;
    f2.g.resid_stride = d;
    f2.g.lscale = L.ls2;
    f2.g.pos = s->pos;
    f2.g.advance_pos = i == c.num_layers - 1;
    add_gemv(s, out, f2);
  }
}

int upload_program(svl_state* s, Program& p) {
  p.smem = 0;
  for (const Phase& ph : p.phases) p.smem = std::max(p.smem, phase_smem(ph));
  void* d;
  TRY(s->alloc(&d, p.phases.size() * sizeof(Phase)));
  HIP_TRY(hipMemcpy(d, p.phases.data(), p.phases.size() * sizeof(Phase), hipMemcpyHostToDevice));
  p.dev = (Phase*)d;
  return 0;
}

// Writes the current RoPE table pointers into the program's in_proj phases (host and device
// copies) when they changed.
int refresh_rope(svl_state* s, Program& p, const float* rope) {
  bool changed = false;
  for (Phase& ph : p.phases)
    if ((ph.kind == PH_GEMV || ph.kind == PH_QGEMM) && ph.g.epi == EPI_QKV_ROPE &&
        (ph.g.rope != rope || ph.g.rope_ovf != s->rope_ovf)) {
      ph.g.rope = rope;
      ph.g.rope_ovf = s->rope_ovf;
      changed = true;
    }
  if (changed)
    HIP_TRY(hipMemcpyAsync(p.dev, p.phases.data(), p.phases.size() * sizeof(Phase), hipMemcpyHostToDevice, s->stream));
  return 0;
}

// Builds the STT, TTS and forward programs of a state (SVL/stt/model.rs:239-276,
// SVL/tts/flow_lm.rs:169-180, SVL/nn/transformer.rs:139-186).
int build_programs(const svl_model* m, svl_state* s) {
  const svl_config& c = m->cfg;
  const int d = c.d_model;
  if (c.kind == SVL_MODEL_STT) {
    std::vector<Phase>& P = s->stt.phases;
    Phase e{};
    e.kind = PH_EMBED;
    e.e.text_emb = m->text_emb;
    e.e.emb = m->emb;
    e.e.tables_bf16 = m->tables_bf16;
    e.e.d = d;
    e.e.n_q = c.n_q;
    e.e.card = c.card;
    e.e.text_card = c.text_card;
    e.e.B = s->B;
    e.e.fb_tok = s->fb_tok;
    e.e.initial_at_zero = 1;
    e.e.pos = s->pos;
    e.e.x = s->x;
    e.e.stage = s->stage;
    e.e.bad_token = s->tok_out + s->B;
    e.units = s->B * ((d + kRowThreads - 1) / kRowThreads);
    P.push_back(e);
    build_layers(m, s, P);
    // the first attention phase (16 of 256 workgroups busy) also gathers the next step's
    // audio embedding rows
    for (Phase& ph : P) {
      if (ph.kind == PH_ATTN) {
        ph.e = e.e;
        ph.units += s->B * c.n_q;
        break;
      }
    }
    Phase t = gemv_phase(s, m->text_linear);
    t.g.x = s->x;
    t.g.x_stride = d;
    t.g.norm = NORM_RMS;
    t.g.nw = m->out_norm_w;
    t.g.eps = 1e-8f;  // SVL/stt/model.rs:252
    t.g.epi = EPI_STORE;
    t.g.y = s->logits;
    t.g.y_stride = c.text_card;
    add_gemv(s, P, t);
    if (c.extra_heads_num > 0) {
      // the extra heads' logits from the same normalized output (SVL/stt/model.rs:259-266)
      Phase xh = gemv_phase(s, m->extra_heads);
      xh.g.x = s->x;
      xh.g.x_stride = d;
      xh.g.norm = NORM_RMS;
      xh.g.nw = m->out_norm_w;
      xh.g.eps = 1e-8f;
      xh.g.epi = EPI_STORE;
      xh.g.y = s->xlogits;
      xh.g.y_stride = c.extra_heads_num * c.extra_heads_dim;
      add_gemv(s, P, xh);
    }
    Phase am{};
    am.kind = PH_ARGMAX;
    am.am.logits = s->logits;
    am.am.B = s->B;
    am.am.V = c.text_card;
    am.am.fb_tok = s->fb_tok;
    am.am.xlogits = s->xlogits;
    am.am.nh = c.extra_heads_num;
    am.am.hd = c.extra_heads_dim;
    am.am.xprob = s->xprob;
    am.am.turn_state = s->turn_state;
    am.units = s->B;
    P.push_back(am);
    TRY(upload_program(s, s->stt));
  }
  if (c.kind == SVL_MODEL_TTS) {
    std::vector<Phase>& P = s->tts.phases;
    Phase in = gemv_phase(s, m->input_linear);
    in.g.x = s->in;
    in.g.x_stride = c.latent_dim;
    in.g.norm = NORM_NONE;
    in.g.epi = EPI_STORE;
    in.g.y = s->x;
    in.g.y_stride = d;
    add_gemv(s, P, in);
    build_layers(m, s, P);
    if (c.z_dim > 0) {
      Phase z = gemv_phase(s, m->z_proj);
      z.g.x = s->x;
      z.g.x_stride = d;
      z.g.norm = NORM_LAYER;
      z.g.nw = m->out_norm_w;
      z.g.nb = m->out_norm_b;
      z.g.eps = 1e-5f;  // SVL/tts/flow_lm.rs:176
      z.g.epi = EPI_STORE;
      z.g.y = s->z;
      z.g.y_stride = c.z_dim;
      add_gemv(s, P, z);
    } else {
      Phase n{};
      n.kind = PH_NORM;
      n.nm.x = s->x;
      n.nm.x_stride = d;
      n.nm.y = s->z;
      n.nm.y_stride = d;
      n.nm.B = s->B;
      n.nm.d = d;
      n.nm.norm = NORM_LAYER;
      n.nm.w = m->out_norm_w;
      n.nm.b = m->out_norm_b;
      n.nm.eps = 1e-5f;
      n.units = s->B;
      P.push_back(n);
    }
    TRY(upload_program(s, s->tts));
  }
  {
    // Transformer::forward one position at a time (causal attention makes this the reference's
    // block forward, transformer.rs:139-186): x[b] = in[b][t]; layers; out[b][t] = x[b].
    std::vector<Phase>& P = s->fwd_prog.phases;
    Phase ci{};
    ci.kind = PH_COPY_IN;
    ci.cp.y = s->x;
    ci.cp.y_stride = d;
    ci.cp.B = s->B;
    ci.cp.n = d;
    ci.units = s->B * ((d + kRowThreads - 1) / kRowThreads);
    P.push_back(ci);
    build_layers(m, s, P);
    Phase co = ci;
    co.kind = PH_COPY_OUT;
    co.cp.x = s->x;
    co.cp.x_stride = d;
    P.push_back(co);
    TRY(upload_program(s, s->fwd_prog));
  }
  return 0;
}

// RoPE rows for the next `steps` positions of every stream: the model's table below its cap;
// past it, this call's rows are computed into the state's overflow buffer (stream b's position
// p at row p + delta[b]), so a long stream holds only the rows of one call.
int prepare_rope(svl_state* s, int64_t steps, int64_t top) {
  const svl_model* m = s->m;
  TRY(ensure_rope(m, top));
  if (top <= m->rope_cap) return 0;
  const int hd = m->cfg.head_dim;
  std::vector<int> delta(s->B, 0);
  int64_t rows = 0;
  for (int b = 0; b < s->B; ++b) {
    const int64_t r0 = std::max(s->pos_host[b], m->rope_cap), r1 = s->pos_host[b] + steps;
    delta[b] = (int)(rows - r0);
    rows += std::max<int64_t>(0, r1 - r0);
  }
  if (rows > s->ovf_rows) {
    // kernels already enqueued may read the old rows
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (s->rope_ovf) HIP_TRY(hipFree(s->rope_ovf));
    s->rope_ovf = nullptr;
    s->ovf_rows = 0;
    int64_t cap = 64;
    while (cap < rows) cap *= 2;
    void* d;
    HIP_TRY(hipMalloc(&d, (size_t)cap * hd * 4));
    s->rope_ovf = (float*)d;
    s->ovf_rows = cap;
  }
  const size_t bytes = (size_t)rows * hd * 4 + (size_t)s->B * 4;
  if (s->ovf_copied) HIP_TRY(hipEventSynchronize(s->ovf_copied));  // the staging is free again
  if (bytes > s->ovf_host_bytes) {
    if (s->ovf_host) HIP_TRY(hipHostFree(s->ovf_host));
    s->ovf_host = nullptr;
    s->ovf_host_bytes = 0;
    void* h;
    HIP_TRY(hipHostMalloc(&h, 2 * bytes));
    s->ovf_host = (float*)h;
    s->ovf_host_bytes = 2 * bytes;
  }
  if (!s->ovf_copied) HIP_TRY(hipEventCreateWithFlags(&s->ovf_copied, hipEventDisableTiming));
  const std::vector<float> inv = rope_inv_freq(m->cfg);
  for (int b = 0; b < s->B; ++b)
    for (int64_t p = std::max(s->pos_host[b], m->rope_cap); p < s->pos_host[b] + steps; ++p)
      rope_row(inv, p, s->ovf_host + (size_t)(p + delta[b]) * hd);
  memcpy(s->ovf_host + (size_t)rows * hd, delta.data(), (size_t)s->B * 4);
  HIP_TRY(hipMemcpyAsync(s->rope_ovf, s->ovf_host, (size_t)rows * hd * 4, hipMemcpyHostToDevice, s->stream));
  HIP_TRY(hipMemcpyAsync(s->rope_delta, s->ovf_host + (size_t)rows * hd, (size_t)s->B * 4, hipMemcpyHostToDevice,
                         s->stream));
  HIP_TRY(hipEventRecord(s->ovf_copied, s->stream));
  return 0;
}

// Validates that every stream has room for `steps` more positions and prepares their RoPE rows.
int check_room(svl_state* s, int64_t steps) {
  int64_t top = 0;
  for (int64_t p : s->pos_host) {
    if (s->m->cfg.context == 0 && p + steps > s->slots)
      return set_error(SVL_ERR_INVALID_INPUT, "state capacity %d exceeded (position %lld + %lld steps)", s->slots,
                       (long long)p, (long long)steps);
    top = std::max(top, p + steps);
  }
  if (top >= ((int64_t)1 << 31)) return set_error(SVL_ERR_INVALID_INPUT, "position beyond 2^31");
  return prepare_rope(s, steps, top);
}

// Attention units take the streams longest first, so that the workgroups that get a second
// round of units get short ones (visible keys grow with the position up to the window; the
// order of the streams does not change while they step together).
int refresh_attn_order(svl_state* s) {
  const int64_t window = s->m->cfg.context;
  std::vector<int>& order = s->order_tmp;  // sized at creation: no allocation per call
  for (int b = 0; b < s->B; ++b) order[b] = b;
  auto visible = [&](int b) { return window > 0 ? std::min(s->pos_host[b] + 1, window) : s->pos_host[b] + 1; };
  // longest first, ties in stream order (an in-place sort)
  std::sort(order.begin(), order.end(), [&](int x, int y) {
    const int64_t vx = visible(x), vy = visible(y);
    return vx != vy ? vx > vy : x < y;
  });
  if (order == s->order_host) return 0;
  std::copy(order.begin(), order.end(), s->order_host.begin());
  HIP_TRY(hipMemcpyAsync(s->attn_order, s->order_host.data(), (size_t)s->B * sizeof(int), hipMemcpyHostToDevice,
                         s->stream));
  return 0;
}

// 32-bit words of a state's split score rows.
size_t split_score_words(const svl_state* s) { return (size_t)s->B * s->m->cfg.num_heads * s->slots * 2; }

// Units per head of the attention launches of step `step` of a call (1: the unsplit unit): the
// largest power of two up to split_max with split_keys visible keys per unit for the longest
// stream, and at least split_min once the head is split at all.
int attn_split(const svl_state* s, int64_t step) {
  if (s->split_max < 2) return 1;
  const int64_t window = s->m->cfg.context;
  int64_t L = 0;
  for (int64_t q : s->pos_host) L = std::max(L, window > 0 ? std::min(q + step + 1, window) : q + step + 1);
  int S = 1;
  while (S < s->split_max && (int64_t)2 * S * s->split_keys <= L) S *= 2;
  return S > 1 ? std::max(S, s->split_min) : 1;
}

// One split attention launch, tagged split_gen + 1 (the rows are cleared to tag 0 before the tags
// would wrap).
int launch_split(svl_state* s, const Phase& ph, const StepParams& P, int step, int S) {
  if (s->split_gen >= (1u << 31)) {
    HIP_TRY(launch_fill_u32((uint32_t*)s->split_scores, 0u, split_score_words(s), s->stream));
    s->split_gen = 0;
  }
  Phase a = ph;
  a.at.split_tag = ++s->split_gen;
  s->split_used = true;
  HIP_TRY(launch_attn_split(a, P, step, S, s->split_scores, s->stream));
  return 0;
}

// Runs `n_steps` steps of program `p` on the state's stream: one persistent launch, or one
// launch per phase.
int run_program(svl_state* s, Program& p, StepParams P, int64_t n_steps) {
  TRY(refresh_attn_order(s));
  const float* rope;
  {
    std::lock_guard<std::mutex> lock(s->m->rope_mu);
    rope = s->m->rope;
  }
  TRY(refresh_rope(s, p, rope));
  P.prog = p.dev;
  P.nphase = (int)p.phases.size();
  P.sync = s->sync;
  P.pos = s->pos;
  P.B = s->B;
  if (s->persistent) {
    const unsigned need = (unsigned)(P.nphase * n_steps);
    if ((uint64_t)s->gen + need >= (1u << 31)) {
      HIP_TRY(hipMemsetAsync(s->sync, 0, sizeof(SyncState), s->stream));
      s->gen = 0;
    }
    P.n_steps = (int)n_steps;
    P.gen0 = s->gen;
    HIP_TRY(launch_step_program(P, program_families(p.phases.data(), P.nphase), s->grid, p.smem, s->stream));
    s->gen += need;
  } else {
    P.n_steps = (int)n_steps;  // the units see the launch's step count (next-step gathers)
    for (int64_t step = 0; step < n_steps; ++step) {
      const int S = attn_split(s, step);
      for (int i = 0; i < P.nphase; ++i) {
        if (S > 1 && p.phases[i].kind == PH_ATTN) TRY(launch_split(s, p.phases[i], P, (int)step, S));
        else HIP_TRY(launch_phase(p.phases[i], P, (int)step, p.smem, s->stream));
      }
    }
  }
  for (auto& q : s->pos_host) q += n_steps;
  return 0;
}

// After a synchronization: reports (and clears) a grid barrier that gave up waiting.
int check_abort(svl_state* s) {
  if (!s->persistent && !s->split_used) return 0;
  unsigned flag = 0;
  HIP_TRY(hipMemcpy(&flag, &s->sync->abort_flag[0], sizeof(flag), hipMemcpyDeviceToHost));
  s->split_used = false;
  if (flag) {
    HIP_TRY(hipMemset(s->sync, 0, sizeof(SyncState)));
    s->gen = 0;
    if (s->split_scores) HIP_TRY(hipMemset(s->split_scores, 0, split_score_words(s) * 4));
    s->split_gen = 0;
    return set_error(SVL_ERR_DEVICE, "a grid barrier or attention meeting of the step timed out; the state is undefined");
  }
  return 0;
}

// A state for `batch` streams; with `kv_parent`, a prefill shadow: `batch` = kv_group rows per
// stream of kv_parent, sharing its rings and stream (kv_parent outlives it).
int make_state(const svl_model* m, int32_t batch, int32_t capacity, svl_state** out, svl_state* kv_parent = nullptr,
               int kv_group = 1) {
  const svl_config& c = m->cfg;
  if (batch <= 0) return set_error(SVL_ERR_INVALID_INPUT, "batch must be positive");
  if (batch > kMaxBatch) return set_error(SVL_UNSUPPORTED, "batch must be <= %d", kMaxBatch);
  int slots = kv_parent ? kv_parent->slots : (c.context > 0 ? c.context : capacity);
  if (slots <= 0) return set_error(SVL_ERR_INVALID_INPUT, "an unlimited-context model needs a positive capacity");
  if (slots > kMaxRingSlots) return set_error(SVL_UNSUPPORTED, "capacity must be <= %d", kMaxRingSlots);
  HIP_TRY(hipSetDevice(m->device));
  std::unique_ptr<svl_state> holder(new svl_state());
  svl_state* s = holder.get();
  s->m = m;
  s->B = batch;
  s->slots = slots;
  s->kv_group = kv_parent ? kv_group : 1;
  s->grid = step_program_grid(m->device);
  const char* mode = getenv("SVL_STEP_LAUNCH");
  // one launch per phase by default (kernel boundaries order the phases); SVL_STEP_LAUNCH=persistent
  // runs the steps of a call in one cooperative launch with grid barriers instead
  s->persistent = mode && !strcmp(mode, "persistent");
  auto fail = [](int rc) { return rc; };  // the holder frees the state
  if (s->grid <= 0) return fail(set_error(SVL_ERR_DEVICE, "cannot query the compute unit count"));
  int max_lds = 0;
  if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, m->device) != hipSuccess || max_lds <= 0)
    return fail(set_error(SVL_ERR_DEVICE, "cannot query the LDS size"));
  s->lds_budget = (size_t)max_lds - kStaticLdsReserve;
  if (kv_parent) {
    s->stream = kv_parent->stream;
    s->owns_stream = false;
  } else if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) {
    return fail(set_error(SVL_ERR_DEVICE, "hipStreamCreate failed"));
  }
  const size_t kvb = (size_t)batch * c.num_kv_heads * slots * c.head_dim * (c.kv_dtype == SVL_BF16 ? 2 : 4);
  s->kc.resize(c.num_layers);
  s->vc.resize(c.num_layers);
  int rc = 0;
  if (kv_parent) {
    s->kc = kv_parent->kc;
    s->vc = kv_parent->vc;
  }
  for (int i = 0; i < c.num_layers && !rc && !kv_parent; ++i) {
    rc = s->alloc(&s->kc[i], kvb);
    if (!rc) rc = s->alloc(&s->vc[i], kvb);
    if (!rc && hipMemsetAsync(s->kc[i], 0, kvb, s->stream) != hipSuccess) rc = set_error(SVL_ERR_DEVICE, "memset");
    if (!rc && hipMemsetAsync(s->vc[i], 0, kvb, s->stream) != hipSuccess) rc = set_error(SVL_ERR_DEVICE, "memset");
  }
  const int qdim = c.num_heads * c.head_dim;
  const int width = std::max(std::max(c.d_model, qdim), c.ff_hidden);
  void* p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * sizeof(int)), s->pos = (int*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * sizeof(int)), s->attn_order = (int*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * 4), s->fb_tok = (uint32_t*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * c.d_model * 4), s->x = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * qdim * 4), s->q = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * qdim * 4), s->att = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * width * 4), s->h = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * std::max(c.text_card, 1) * 4), s->logits = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * std::max(c.d_model, c.z_dim) * 4), s->z = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * std::max(c.latent_dim, 1) * 4), s->in = (float*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * (1 + std::max(c.n_q, 0)) * 4), s->tok_in = (uint32_t*)p;
  if (!rc && c.kind == SVL_MODEL_STT)
    rc = s->alloc(&p, (size_t)batch * c.n_q * c.d_model * (m->tables_bf16 ? 2 : 4)), s->stage = p;
  if (!rc && c.kind == SVL_MODEL_STT) rc = s->alloc(&p, (size_t)(batch + 3) * 4), s->turn_state = (uint32_t*)p;
  if (!rc && c.kind == SVL_MODEL_STT && c.extra_heads_num > 0) {
    rc = s->alloc(&p, (size_t)batch * c.extra_heads_num * c.extra_heads_dim * 4), s->xlogits = (float*)p;
    if (!rc) rc = s->alloc(&p, (size_t)batch * c.extra_heads_num * 4), s->xprob = (float*)p;
  }
  if (!rc && batch >= kBatchMfma) {
    const int wmax = std::max(std::max(c.d_model, c.num_heads * c.head_dim), c.ff_hidden);
    rc = s->alloc(&p, (size_t)batch * ((wmax + 127) / 128 * 128)), s->xqb = (int8_t*)p;
    if (!rc) rc = s->alloc(&p, (size_t)batch * (wmax / 32) * 4), s->xdqb = (float*)p;
  }
  if (!rc && c.kind == SVL_MODEL_TTS && c.flow_dim > 0) {
    const svl_model::Flow& F = m->flow;
    rc = s->alloc(&p, (size_t)batch * (F.dim + 1) * 4), s->fh_ce = (float*)p;
    // the modulation rows also hold the time embedders' outputs while a step count's time
    // conditioning is computed (n_time * dim <= 2 dim <= mod_rows)
    if (!rc) rc = s->alloc(&p, (size_t)batch * F.mod_rows * 4), s->fh_mod = (float*)p;
    if (!rc) rc = s->alloc(&p, (size_t)batch * F.dim * 4), s->fh_h = (float*)p;
    if (!rc) rc = s->alloc(&p, (size_t)batch * F.dim * 4), s->fh_a = (float*)p;
    if (!rc) rc = s->alloc(&p, (size_t)batch * F.latent * 4), s->fh_x = (float*)p;
    if (!rc) rc = s->alloc(&p, (size_t)batch * F.latent * 4), s->fh_noise = (float*)p;
  }
  if (!rc) rc = s->alloc(&p, (size_t)(batch + 1) * 4), s->tok_out = (uint32_t*)p;
  if (!rc) rc = s->alloc(&p, (size_t)batch * sizeof(int)), s->rope_delta = (int*)p;
  if (!rc) rc = s->alloc(&p, sizeof(SyncState)), s->sync = (SyncState*)p;
  if (!rc && hipMemsetAsync(s->sync, 0, sizeof(SyncState), s->stream) != hipSuccess) rc = set_error(SVL_ERR_DEVICE, "memset");
  if (!rc) {
    // split attention while B * H units leave most CUs idle (SVL_ATTN_SPLIT: keys per split unit,
    // 0 = never split)
    const char* sp = getenv("SVL_ATTN_SPLIT");
    s->split_keys = sp ? std::max(atoi(sp), 0) : kSplitKeys;
    const int nh = batch * c.num_heads, kv_bf16 = c.kv_dtype == SVL_BF16 ? 1 : 0;
    int S = kMaxSplit;
    while (S > 1 && nh * S > s->grid) S /= 2;
    if (s->persistent || kv_parent || s->split_keys == 0 || (c.head_dim != 64 && c.head_dim != 128) ||
        split_smem(slots, c.head_dim, kv_bf16, S) > s->lds_budget)
      S = 1;
    s->split_max = S;
    // fewer units hold more value columns each
    s->split_min = 2;
    while (s->split_min < S && split_smem(slots, c.head_dim, kv_bf16, s->split_min) > s->lds_budget) s->split_min *= 2;
    if (S > 1) {
      rc = s->alloc(&p, (size_t)nh * slots * 8), s->split_scores = (uint64_t*)p;
      if (!rc && hipMemsetAsync(s->split_scores, 0, (size_t)nh * slots * 8, s->stream) != hipSuccess)
        rc = set_error(SVL_ERR_DEVICE, "memset");
    }
  }
  if (!rc) rc = build_programs(m, s);
  if (rc) return fail(rc);
  for (const Program* p : {&s->stt, &s->tts, &s->fwd_prog})
    if (p->smem > s->lds_budget)
      return fail(set_error(SVL_UNSUPPORTED, "a step phase needs %zu bytes of LDS, more than the %zu available (window %d)",
                            p->smem, s->lds_budget, s->slots));
  s->pos_host.assign(batch, 0);
  s->order_tmp.assign(batch, 0);
  s->order_host.assign(batch, -1);  // differs from any order: the first run uploads it
  if (launch_fill_i32(s->pos, 0, batch, s->stream) != hipSuccess ||
      launch_fill_i32(s->rope_delta, 0, batch, s->stream) != hipSuccess ||
      launch_fill_u32(s->tok_out, 0u, batch + 1, s->stream) != hipSuccess ||
      (s->turn_state && launch_fill_u32(s->turn_state, 0u, batch + 3, s->stream) != hipSuccess) ||
      launch_fill_u32(s->fb_tok, (uint32_t)std::max(c.text_card, 0), batch, s->stream) != hipSuccess ||
      hipStreamSynchronize(s->stream) != hipSuccess)
    return fail(set_error(SVL_ERR_DEVICE, "state initialisation failed"));
  *out = holder.release();
  return 0;
}

// The time conditioning of every flow step for `steps` steps (SVL/tts/flow_lm.rs:256-266,
// 286-309): [steps][dim], computed once per step count on the state's stream and kept in the
// model.  The embedders' cos/sin rows are the C library's cosf/sinf of freqs * t, as Rust's
// f32::cos / f32::sin compute them on the host (:333-337).
int flow_tmean(svl_state* s, int steps, const float** out) {
  svl_model* m = const_cast<svl_model*>(s->m);  // the cache is guarded by flow_mu
  svl_model::Flow& F = m->flow;
  std::lock_guard<std::mutex> lock(m->flow_mu);
  auto it = F.tmean.find(steps);
  if (it != F.tmean.end()) {
    *out = it->second;
    return 0;
  }
  const int D = F.dim;
  std::vector<float> emb((size_t)steps * F.n_time * 256);
  for (int i = 0; i < steps; ++i) {
    // LSD: (s, t) = (i / steps, (i + 1) / steps); flow matching: t = i / steps
    const float times[2] = {(float)i / (float)steps, (float)(i + 1) / (float)steps};
    for (int e = 0; e < F.n_time; ++e) {
      float* row = emb.data() + ((size_t)i * F.n_time + e) * 256;
      for (int k = 0; k < 128; ++k) {
        const float pr = F.freqs[e][k] * times[e];
        const float a = pr + 0.0f;
        row[k] = cosf(a);
        row[128 + k] = sinf(a);
      }
    }
  }
  void *dtab = nullptr, *demb = nullptr;
  HIP_TRY(hipMalloc(&dtab, (size_t)steps * D * 4));
  std::unique_ptr<void, void (*)(void*)> tab_guard(dtab, [](void* p) { hipFree(p); });
  HIP_TRY(hipMalloc(&demb, emb.size() * 4));
  std::unique_ptr<void, void (*)(void*)> emb_guard(demb, [](void* p) { hipFree(p); });
  HIP_TRY(hipMemcpyAsync(demb, emb.data(), emb.size() * 4, hipMemcpyHostToDevice, s->stream));
  for (int i = 0; i < steps; ++i) {
    for (int e = 0; e < F.n_time; ++e) {
      FhArgs a{};
      a.B = 1;
      a.L = F.t1[e];
      a.x = (const float*)demb + ((size_t)i * F.n_time + e) * 256;
      a.x_stride = 256;
      a.y = s->fh_a;
      a.y_stride = D;
      HIP_TRY(launch_fh_gemv(a, FH_PLAIN, FH_BIAS_SILU, s->stream));
      a = FhArgs{};
      a.B = 1;
      a.L = F.t2[e];
      a.x = s->fh_a;
      a.x_stride = D;
      a.y = s->fh_mod + (size_t)e * D;
      a.y_stride = D;
      HIP_TRY(launch_fh_gemv(a, FH_PLAIN, FH_BIAS, s->stream));
    }
    HIP_TRY(launch_fh_time_norm(s->fh_mod, F.talpha, F.n_time, D, (float)(1.0 / D), (float)(1.0 / (D - 1.0)),
                                (float)(1.0 / F.n_time), (float*)dtab + (size_t)i * D, s->stream));
  }
  HIP_TRY(hipStreamSynchronize(s->stream));  // the host table is released on return
  F.tmean[steps] = (float*)dtab;
  m->allocs.push_back(tab_guard.release());
  *out = (const float*)dtab;
  return 0;
}

// FlowLm::step after the backbone (SVL/tts/flow_lm.rs:181-185): z (s->z) -> the end-of-speech
// logits (s->fh_ce[b][dim]) and the decoded sample (s->fh_x) from the noise in s->fh_noise.
int run_flow_head(svl_state* s, int steps) {
  const svl_model::Flow& F = s->m->flow;
  steps = std::max(steps, 1);  // FlowHead::decode: steps.max(1)
  const float* tmean = nullptr;
  if (F.n_time > 0) TRY(flow_tmean(s, steps, &tmean));
  const int D = F.dim, B = s->B;
  FhArgs a{};
  a.B = B;
  a.L = F.ce;
  a.x = s->z;
  a.x_stride = F.cond;
  a.y = s->fh_ce;
  a.y_stride = D + 1;
  HIP_TRY(launch_fh_gemv(a, FH_PLAIN, FH_BIAS, s->stream));
  HIP_TRY(hipMemcpyAsync(s->fh_x, s->fh_noise, (size_t)B * F.latent * 4, hipMemcpyDeviceToDevice, s->stream));
  // LSD and flow matching integrate `steps` Euler steps; drifting and pointwise run the head once
  const bool euler = F.kind == SVL_FLOW_LSD || F.kind == SVL_FLOW_MATCHING;
  const int n = euler ? steps : 1;
  for (int i = 0; i < n; ++i) {
    FhArgs g{};
    g.B = B;
    g.L = F.mod;
    g.x = s->fh_ce;
    g.x_stride = D + 1;
    g.x2 = tmean ? tmean + (size_t)i * D : nullptr;
    g.y = s->fh_mod;
    g.y_stride = F.mod_rows;
    HIP_TRY(launch_fh_gemv(g, FH_SILU_Y, FH_BIAS, s->stream));
    g = FhArgs{};
    g.B = B;
    g.L = F.in;
    g.x = s->fh_x;
    g.x_stride = F.latent;
    g.y = s->fh_h;
    g.y_stride = D;
    HIP_TRY(launch_fh_gemv(g, FH_PLAIN, FH_BIAS, s->stream));
    for (int j = 0; j < F.depth; ++j) {
      const float* mj = s->fh_mod + (size_t)j * 3 * D;  // chunk(3): shift, scale, gate
      g = FhArgs{};
      g.B = B;
      g.L = F.m1[j];
      g.x = s->fh_h;
      g.x_stride = D;
      g.lnw = F.lnw[j];
      g.lnb = F.lnb[j];
      g.shift = mj;
      g.scale = mj + D;
      g.mod_stride = F.mod_rows;
      g.eps = 1e-6f;  // SVL/tts/flow_lm.rs:378
      g.y = s->fh_a;
      g.y_stride = D;
      HIP_TRY(launch_fh_gemv(g, FH_LN_MOD, FH_BIAS_SILU, s->stream));
      g = FhArgs{};
      g.B = B;
      g.L = F.m2[j];
      g.x = s->fh_a;
      g.x_stride = D;
      g.gate = mj + 2 * D;
      g.mod_stride = F.mod_rows;
      g.y = s->fh_h;
      g.y_stride = D;
      HIP_TRY(launch_fh_gemv(g, FH_PLAIN, FH_GATE_RES, s->stream));
    }
    const float* mf = s->fh_mod + (size_t)F.depth * 3 * D;  // chunk(2): shift, scale
    g = FhArgs{};
    g.B = B;
    g.L = F.fl;
    g.x = s->fh_h;
    g.x_stride = D;
    g.shift = mf;
    g.scale = mf + D;
    g.mod_stride = F.mod_rows;
    g.eps = 1e-6f;  // SVL/tts/flow_lm.rs:277
    g.inv_k = (float)(1.0 / D);
    g.y = s->fh_x;
    g.y_stride = F.latent;
    g.inv_steps = (float)(1.0 / steps);
    g.noise = s->fh_noise;
    g.noise_stride = F.latent;
    const int epi = euler ? FH_FLOW : (F.kind == SVL_FLOW_DRIFTING ? FH_BIAS : FH_POINTWISE);
    HIP_TRY(launch_fh_gemv(g, FH_LN0_MOD, epi, s->stream));
  }
  return 0;
}

StepParams stt_params(const svl_state* s, const uint32_t* d_audio, const uint32_t* d_text, uint32_t* d_out,
                       float* d_prob = nullptr, int32_t* d_turn = nullptr) {
  StepParams P{};
  P.out_turn = d_turn;
  P.out_prob = d_prob;
  P.prob_stride = (size_t)s->B * std::max(s->m->cfg.extra_heads_num, 0);
  P.audio = d_audio;
  P.audio_stride = (size_t)s->B * s->m->cfg.n_q;
  P.text = d_text;
  P.text_stride = (size_t)s->B;
  P.out_tok = d_out;
  P.out_stride = (size_t)s->B;
  return P;
}

}  // namespace

// ---- scratch of the allocation-free entry point ----------------------------------------------
// svl_stt_recognize_noalloc stages its audio tokens and output tokens in this array instead of
// buffers allocated per call.  Each GPU holds its own copy until the process ends; host code
// uses the address hipGetSymbolAddress returns for the current device, never the array's name
// (a host-side stand-in).
constexpr size_t kNoAllocScratchBytes = (size_t)2 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;  // calls share their device's scratch: they run one at a time
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on `device` (current), looked up on the first call there.
int scratch_on(int device, unsigned char** out) {
  if (device < 0 || device >= kMaxScratchDevices) return set_error(SVL_ERR_DEVICE, "device %d out of range", device);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(SVL_ERR_DEVICE, "no device address for the scratch array");
    g_scratch_ptr[device] = p;
  }
  *out = (unsigned char*)g_scratch_ptr[device];
  return 0;
}

// Runs an entry point's body; a C++ exception (a failed host allocation, most likely) becomes an
// error code instead of crossing the C boundary.
template <class F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const std::bad_alloc&) {
    return set_error(SVL_ERR_DEVICE, "host memory allocation failed");
  } catch (const std::exception& e) {
    return set_error(SVL_ERR_DEVICE, "internal error: %s", e.what());
  } catch (...) {
    return set_error(SVL_ERR_DEVICE, "internal error");
  }
}

}  // namespace

extern "C" {

const char* svl_last_error(void) { return g_error.c_str(); }

static int rvq_create_impl(const svl_tensor* ts, size_t n, int32_t n_q, int32_t bins, int device, svl_rvq** out) {
  if (!out) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  *out = nullptr;
  if (n_q < 1 || bins < 1 || bins > (1 << 24)) return set_error(SVL_ERR_CONFIG, "n_q and bins must be positive");
  if (!ts && n) return set_error(SVL_ERR_INVALID_INPUT, "null tensors");
  HIP_TRY(hipSetDevice(device));
  std::unique_ptr<svl_rvq> q(new svl_rvq());
  q->device = device;
  q->n_q = n_q;
  q->bins = bins;
  HIP_TRY(hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking));
  auto alloc = [&](void** p, size_t bytes) -> int {
    HIP_TRY(hipMalloc(p, bytes));
    q->allocs.push_back(*p);
    return 0;
  };
  const size_t wn = (size_t)kRvqDim * kRvqIn, entries = (size_t)n_q * bins;
  void* p;
  TRY(alloc(&p, 2 * wn * 4));
  q->w = (float*)p;
  TRY(alloc(&p, entries * kRvqDim * 4));
  q->emb = (float*)p;
  TRY(alloc(&p, entries * 4));
  q->hn = (float*)p;
  const char* parts[2] = {"rvq_first", "rvq_rest"};
  for (int part = 0; part < 2; ++part) {
    const std::string name = std::string(parts[part]) + ".input_proj.weight";
    const svl_tensor* t = find_tensor(ts, n, name);
    if (!t) return set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s", name.c_str());
    TRY(copy_f32_on(q->stream, t, wn, q->w + part * wn));
  }
  // the codebooks' sums and usages, staged and prepared on the GPU
  float *sums = nullptr, *usage = nullptr;
  HIP_TRY(hipMalloc((void**)&sums, entries * kRvqDim * 4));
  int rc = 0;
  if (hipMalloc((void**)&usage, entries * 4) != hipSuccess) rc = set_error(SVL_ERR_DEVICE, "hipMalloc failed");
  for (int stage = 0; stage < n_q && !rc; ++stage) {
    const std::string pre = stage == 0 ? "rvq_first.vq.layers.0._codebook."
                                       : "rvq_rest.vq.layers." + std::to_string(stage - 1) + "._codebook.";
    const svl_tensor* es = find_tensor(ts, n, pre + "embedding_sum");
    const svl_tensor* us = find_tensor(ts, n, pre + "cluster_usage");
    if (!es || !us) {
      rc = set_error(SVL_ERR_INVALID_INPUT, "missing tensor %s%s", pre.c_str(), es ? "cluster_usage" : "embedding_sum");
      break;
    }
    rc = copy_f32_on(q->stream, es, (size_t)bins * kRvqDim, sums + (size_t)stage * bins * kRvqDim);
    if (!rc) rc = copy_f32_on(q->stream, us, (size_t)bins, usage + (size_t)stage * bins);
  }
  if (!rc && launch_rvq_prepare(sums, usage, entries, q->emb, q->hn, q->stream) != hipSuccess)
    rc = set_error(SVL_ERR_DEVICE, "codebook preparation failed");
  if (!rc && hipStreamSynchronize(q->stream) != hipSuccess) rc = set_error(SVL_ERR_DEVICE, "codebook preparation failed");
  hipFree(sums);
  if (usage) hipFree(usage);
  TRY(rc);
  *out = q.release();
  return 0;
}

// Work buffers for `rows` rows (waits for the stream before replacing smaller ones).
static int rvq_reserve(svl_rvq* q, int64_t rows) {
  if (rows <= q->rows_cap) return 0;
  HIP_TRY(hipStreamSynchronize(q->stream));
  q->free_work();
  const int64_t cap = std::max<int64_t>(rows, 64);
  HIP_TRY(hipMalloc((void**)&q->proj, (size_t)cap * 2 * kRvqDim * 4));
  HIP_TRY(hipMalloc((void**)&q->res, (size_t)cap * 2 * kRvqDim * 4));
  HIP_TRY(hipMalloc((void**)&q->lat, (size_t)cap * kRvqIn * 4));
  HIP_TRY(hipMalloc((void**)&q->keys, (size_t)cap * q->n_q * 8));
  HIP_TRY(hipMalloc((void**)&q->codes, (size_t)cap * q->n_q * 4));
  q->rows_cap = cap;
  return 0;
}

static int rvq_encode_async_impl(svl_rvq* q, int32_t batch, int32_t frames, const float* d_lat, uint32_t* d_codes) {
  if (!q || (!d_lat && batch * (int64_t)frames > 0) || (!d_codes && batch * (int64_t)frames > 0))
    return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (batch < 0 || frames < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative batch or frames");
  const int64_t rows = (int64_t)batch * frames;
  if (rows == 0) return 0;
  if (rows > (1 << 20)) return set_error(SVL_ERR_INVALID_INPUT, "at most 2^20 frames a call");
  HIP_TRY(hipSetDevice(q->device));
  TRY(rvq_reserve(q, rows));
  const int r = (int)rows;
  HIP_TRY(launch_fill_u32((uint32_t*)q->keys, 0xffffffffu, (size_t)rows * q->n_q * 2, q->stream));
  HIP_TRY(launch_rvq_project(d_lat, batch, frames, q->w, q->w + (size_t)kRvqDim * kRvqIn, q->proj, q->stream));
  for (int k = 0; k < std::max(q->n_q - 1, 1); ++k)
    HIP_TRY(launch_rvq_stage(k, q->n_q, r, q->bins, q->emb, q->hn, q->proj, q->res, q->keys, q->stream));
  HIP_TRY(launch_rvq_codes(q->keys, r, q->n_q, d_codes, q->stream));
  return 0;
}

static int rvq_encode_impl(svl_rvq* q, int32_t batch, int32_t frames, const float* lat, uint32_t* codes) {
  if (!q || ((!lat || !codes) && batch * (int64_t)frames > 0)) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (batch < 0 || frames < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative batch or frames");
  const int64_t rows = (int64_t)batch * frames;
  if (rows == 0) return 0;
  if (rows > (1 << 20)) return set_error(SVL_ERR_INVALID_INPUT, "at most 2^20 frames a call");
  HIP_TRY(hipSetDevice(q->device));
  TRY(rvq_reserve(q, rows));
  HIP_TRY(hipMemcpyAsync(q->lat, lat, (size_t)rows * kRvqIn * 4, hipMemcpyHostToDevice, q->stream));
  TRY(rvq_encode_async_impl(q, batch, frames, q->lat, q->codes));
  HIP_TRY(hipMemcpyAsync(codes, q->codes, (size_t)rows * q->n_q * 4, hipMemcpyDeviceToHost, q->stream));
  HIP_TRY(hipStreamSynchronize(q->stream));
  return 0;
}

static int device_count_impl(int* count) {
  HIP_TRY(hipGetDeviceCount(count));
  return 0;
}

static int bench_copy_impl(int device, const void* src, void* dst, size_t bytes, void* stream) {
  if ((bytes % 16) || ((uintptr_t)src % 16) || ((uintptr_t)dst % 16))
    return set_error(SVL_ERR_INVALID_INPUT, "copy needs 16-byte multiples and alignment");
  if (bytes && (!src || !dst)) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(launch_copy(src, dst, bytes, (hipStream_t)stream));
  return 0;
}

static int bench_read_impl(int device, const void* src, size_t bytes, int blocks, int threads, uint32_t* out,
                           void* stream) {
  if ((bytes % 16) || ((uintptr_t)src % 16)) return set_error(SVL_ERR_INVALID_INPUT, "read needs 16-byte multiples and alignment");
  if (blocks < 1 || blocks > 65536 || threads < 64 || threads > 1024 || threads % 64)
    return set_error(SVL_ERR_INVALID_INPUT, "grid %d x %d: 1 .. 65536 workgroups of 64 .. 1024 threads (multiple of 64)",
                     blocks, threads);
  if (!out || (bytes && !src)) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(launch_read(src, bytes, blocks, threads, out, (hipStream_t)stream));
  return 0;
}

static int bench_row_stats_impl(int device, const float* x, int rows, int k, int norm, float* out, void* stream) {
  if (!x || !out || rows <= 0) return set_error(SVL_ERR_INVALID_INPUT, "null argument or no rows");
  if (k < 4 || k > 4096 || k % 4) return set_error(SVL_ERR_INVALID_INPUT, "row length %d: 4 .. 4096, a multiple of 4", k);
  if (norm != SVL_NORM_LAYER && norm != SVL_NORM_RMS) return set_error(SVL_ERR_INVALID_INPUT, "unknown norm %d", norm);
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(launch_row_stats(x, rows, k, norm == SVL_NORM_LAYER ? NORM_LAYER : NORM_RMS, out, (hipStream_t)stream));
  return 0;
}

static int bench_activation_impl(int device, int kind, const float* x, size_t n, float* y, void* stream) {
  if ((!x || !y) && n) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (kind < 0 || kind > 3) return set_error(SVL_ERR_INVALID_INPUT, "unknown function %d", kind);
  if (n > ((size_t)1 << 31)) return set_error(SVL_ERR_INVALID_INPUT, "at most 2^31 values");
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(launch_activation(kind, x, n, y, (hipStream_t)stream));
  return 0;
}

static int model_create_impl(const svl_config* cfg, const svl_tensor* tensors, size_t count, int device, svl_model** out) {
  if (!cfg || !out || (!tensors && count)) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  *out = nullptr;
  TRY(check_config(cfg));
  int ndev = 0;
  HIP_TRY(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) return set_error(SVL_ERR_DEVICE, "device %d not available (%d devices)", device, ndev);
  HIP_TRY(hipSetDevice(device));
  std::unique_ptr<svl_model> m(new svl_model());
  m->cfg = *cfg;
  m->device = device;
  if (const char* cap = getenv("SVL_ROPE_TABLE_POSITIONS"))  // smaller tables exercise the per-call rows in tests
    m->rope_cap = std::min<int64_t>(std::max<int64_t>(atoll(cap), 16), (int64_t)1 << 30);
  TRY(create_model(cfg, tensors, count, m.get()));
  *out = m.release();
  return 0;
}

void svl_model_destroy(svl_model* model) { delete model; }

static int model_linear_weight_impl(const svl_model* m, const char* name, float* f32, size_t f32_count, void* blocks,
                            size_t block_bytes) {
  if (!m || !name) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  const LinearDev* L = find_linear(m, name);
  if (!L) return set_error(SVL_ERR_INVALID_INPUT, "unknown linear %s", name);
  HIP_TRY(hipSetDevice(m->device));
  const size_t n = (size_t)L->out * L->in;
  if (f32) {
    if (f32_count != n) return set_error(SVL_ERR_INVALID_INPUT, "f32 buffer holds %zu values, need %zu", f32_count, n);
    float* tmp;
    HIP_TRY(hipMalloc(&tmp, n * 4));
    hipError_t e = launch_dequant(*L, tmp, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e == hipSuccess) e = hipMemcpy(f32, tmp, n * 4, hipMemcpyDeviceToHost);
    hipFree(tmp);
    HIP_TRY(e);
  }
  if (blocks && L->fmt == FMT_Q4K) {
    if (block_bytes != n / 256 * 144) return set_error(SVL_ERR_INVALID_INPUT, "block buffer size mismatch");
    uint8_t* tmp;
    HIP_TRY(hipMalloc(&tmp, block_bytes));
    hipError_t e = launch_q4k_to_blocks((const uint8_t*)L->w, L->out, L->in, tmp, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e == hipSuccess) e = hipMemcpy(blocks, tmp, block_bytes, hipMemcpyDeviceToHost);
    hipFree(tmp);
    HIP_TRY(e);
  } else if (blocks && L->fmt == FMT_Q4_0) {
    if (block_bytes != n / 32 * 18) return set_error(SVL_ERR_INVALID_INPUT, "block buffer size mismatch");
    uint8_t* tmp;
    HIP_TRY(hipMalloc(&tmp, block_bytes));
    hipError_t e = launch_q4_0_to_blocks((const uint8_t*)L->w, L->scale, L->out, L->in, tmp, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e == hipSuccess) e = hipMemcpy(blocks, tmp, block_bytes, hipMemcpyDeviceToHost);
    hipFree(tmp);
    HIP_TRY(e);
  } else if (blocks) {
    if (L->fmt != FMT_Q8_0) return set_error(SVL_ERR_INVALID_INPUT, "linear %s is not quantized", name);
    if (block_bytes != n / 32 * 34) return set_error(SVL_ERR_INVALID_INPUT, "block buffer size mismatch");
    uint8_t* tmp;
    HIP_TRY(hipMalloc(&tmp, block_bytes));
    hipError_t e = launch_q8_to_blocks((const int8_t*)L->w, L->scale, L->out, L->in, tmp, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e == hipSuccess) e = hipMemcpy(blocks, tmp, block_bytes, hipMemcpyDeviceToHost);
    hipFree(tmp);
    HIP_TRY(e);
  }
  return 0;
}

static int state_create_impl(const svl_model* model, int32_t batch, int32_t capacity, svl_state** out) {
  if (!model || !out) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  *out = nullptr;
  return make_state(model, batch, capacity, out);
}

static int state_duplicate_impl(const svl_state* s, svl_state** out) {
  if (!s || !out) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  svl_state* c = nullptr;
  TRY(make_state(s->m, s->B, s->slots, &c));
  const svl_config& cfg = s->m->cfg;
  const size_t kvb = (size_t)s->B * cfg.num_kv_heads * s->slots * cfg.head_dim * (cfg.kv_dtype == SVL_BF16 ? 2 : 4);
  hipError_t e = hipStreamSynchronize(s->stream);
  for (int i = 0; i < cfg.num_layers && e == hipSuccess; ++i) {
    e = hipMemcpyAsync(c->kc[i], s->kc[i], kvb, hipMemcpyDeviceToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->vc[i], s->vc[i], kvb, hipMemcpyDeviceToDevice, c->stream);
  }
  if (e == hipSuccess) e = hipMemcpyAsync(c->pos, s->pos, s->B * sizeof(int), hipMemcpyDeviceToDevice, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(c->fb_tok, s->fb_tok, s->B * 4, hipMemcpyDeviceToDevice, c->stream);
  if (e == hipSuccess && s->turn_state)
    e = hipMemcpyAsync(c->turn_state, s->turn_state, s->B * 4, hipMemcpyDeviceToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    delete c;
    return set_error(SVL_ERR_DEVICE, "state copy failed: %s", hipGetErrorString(e));
  }
  c->pos_host = s->pos_host;
  *out = c;
  return 0;
}

static int state_load_stream_impl(svl_state* s, int32_t stream, int64_t len, const float* const* keys,
                          const float* const* values) {
  if (!s || (len > 0 && (!keys || !values))) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (stream < 0 || stream >= s->B) return set_error(SVL_ERR_INVALID_INPUT, "stream %d out of range", stream);
  if (len < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative length");
  const svl_config& c = s->m->cfg;
  if (c.context == 0 && len > s->slots)
    return set_error(SVL_ERR_INVALID_INPUT, "cache length %lld exceeds the state capacity %d", (long long)len, s->slots);
  HIP_TRY(hipSetDevice(s->m->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  const int KVH = c.num_kv_heads, hd = c.head_dim, S = s->slots;
  const size_t per = (size_t)KVH * S * hd;
  std::vector<float> hk(per, 0.0f), hv(per, 0.0f);
  float* tmp;
  HIP_TRY(hipMalloc(&tmp, per * 4));
  const int64_t keep = len < S ? len : S;
  hipError_t e = hipSuccess;
  const int esz = c.kv_dtype == SVL_BF16 ? 2 : 4;
  for (int i = 0; i < c.num_layers && e == hipSuccess; ++i) {
    for (int kv = 0; kv < 2 && e == hipSuccess; ++kv) {
      const float* src = kv == 0 ? keys[i] : values[i];
      std::vector<float>& h = kv == 0 ? hk : hv;
      std::fill(h.begin(), h.end(), 0.0f);
      for (int g = 0; g < KVH; ++g)
        for (int64_t j = len - keep; j < len; ++j)
          memcpy(&h[((size_t)g * S + (size_t)(j % S)) * hd], src + ((size_t)g * len + j) * hd, (size_t)hd * 4);
      e = hipMemcpyAsync(tmp, h.data(), per * 4, hipMemcpyHostToDevice, s->stream);
      void* dst = (char*)(kv == 0 ? s->kc[i] : s->vc[i]) + (size_t)stream * per * esz;
      if (e == hipSuccess) e = launch_f32_to_kv(tmp, dst, c.kv_dtype == SVL_BF16, per, s->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    }
  }
  int p32 = (int)len;
  if (e == hipSuccess) e = hipMemcpyAsync(s->pos + stream, &p32, sizeof(int), hipMemcpyHostToDevice, s->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  hipFree(tmp);
  HIP_TRY(e);
  s->pos_host[stream] = len;
  return 0;
}

// Voice::load (SVL/tts/voice.rs:103-143): the state after a voice prompt as upstream Pocket TTS
// saves it -- per layer i, "transformer.layers.{i}.self_attn/cache" [2, batch, time, heads,
// head_dim] (keys, then values), "/offset" (the cached length; older exports: the length of
// "/current_end", else `time`) and "/pad" (must be zero) -- loaded into stream `stream` as
// TransformerState::from_layer_caches does.
static int state_load_voice_impl(svl_state* s, int32_t stream, const svl_tensor* ts, size_t n) {
  if (!s || (n && !ts)) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  const svl_config& c = s->m->cfg;
  const std::string pre = "transformer.layers.", suf = ".self_attn/cache";
  std::vector<const svl_tensor*> caches(c.num_layers, nullptr);
  std::vector<int64_t> lens(c.num_layers, -1);
  size_t found = 0;
  auto to_i64 = [](const svl_tensor* t, int64_t* v) -> bool {
    if (!t || !t->data || numel(t) < 1) return false;
    if (t->dtype == SVL_I64) *v = ((const int64_t*)t->data)[0];
    else if (t->dtype == SVL_F32) *v = (int64_t)((const float*)t->data)[0];
    else return false;
    return true;
  };
  for (size_t i = 0; i < n; ++i) {
    if (!ts[i].name) continue;
    const std::string name = ts[i].name;
    if (name.size() <= pre.size() + suf.size() || name.compare(0, pre.size(), pre) ||
        name.compare(name.size() - suf.size(), suf.size(), suf))
      continue;
    const std::string idx = name.substr(pre.size(), name.size() - pre.size() - suf.size());
    char* end = nullptr;
    const long layer = strtol(idx.c_str(), &end, 10);
    if (idx.empty() || *end || layer < 0) return set_error(SVL_ERR_INVALID_INPUT, "bad tensor name %s", name.c_str());
    if (layer >= c.num_layers) return set_error(SVL_ERR_INVALID_INPUT, "%s: the model has %d layers", name.c_str(), c.num_layers);
    const svl_tensor* t = &ts[i];
    if (t->ndim != 5 || t->shape[0] != 2 || t->shape[3] != c.num_kv_heads || t->shape[4] != c.head_dim)
      return set_error(SVL_ERR_INVALID_INPUT, "%s: expected [2, batch, time, %d, %d]", name.c_str(), c.num_kv_heads,
                       c.head_dim);
    if (t->dtype != SVL_F32 && t->dtype != SVL_BF16)
      return set_error(SVL_ERR_INVALID_INPUT, "%s: f32 or bf16 cache expected", name.c_str());
    if (t->shape[1] != 1) return set_error(SVL_UNSUPPORTED, "%s: voice states of batch %lld", name.c_str(), (long long)t->shape[1]);
    const std::string module = name.substr(0, name.size() - std::string("/cache").size());
    int64_t len = t->shape[2], v = 0;
    if (to_i64(find_tensor(ts, n, module + "/offset"), &v)) len = v;
    else if (const svl_tensor* ce = find_tensor(ts, n, module + "/current_end")) len = ce->ndim > 0 ? ce->shape[0] : 0;
    const svl_tensor* pad = find_tensor(ts, n, module + "/pad");
    if (pad && pad->data) {
      for (size_t k = 0; k < numel(pad); ++k) {
        const int64_t pv = pad->dtype == SVL_I64 ? ((const int64_t*)pad->data)[k] : (int64_t)((const float*)pad->data)[k];
        if (pv != 0) return set_error(SVL_ERR_INVALID_INPUT, "padded (batched) voice states are not supported");
      }
    }
    if (len < 0 || len > t->shape[2]) return set_error(SVL_ERR_INVALID_INPUT, "%s: offset %lld past the cache", name.c_str(), (long long)len);
    if (!caches[layer]) ++found;
    caches[layer] = t;
    lens[layer] = len;
  }
  if (found == 0) return set_error(SVL_ERR_INVALID_INPUT, "not a voice state");
  if (found != (size_t)c.num_layers) return set_error(SVL_ERR_INVALID_INPUT, "voice state has %zu of %d layers", found, c.num_layers);
  const int64_t len = lens[0];
  for (int64_t l : lens)
    if (l != len) return set_error(SVL_ERR_INVALID_INPUT, "voice state layers of different lengths");
  // [2][1][time][heads][hd] -> keys / values [heads][len][hd] f32
  const size_t kvh = c.num_kv_heads, hd = c.head_dim;
  std::vector<std::vector<float>> kh(c.num_layers), vh(c.num_layers);
  std::vector<const float*> kp(c.num_layers), vp(c.num_layers);
  for (int l = 0; l < c.num_layers; ++l) {
    const svl_tensor* t = caches[l];
    const size_t T = t->shape[2];
    kh[l].resize(kvh * len * hd);
    vh[l].resize(kvh * len * hd);
    for (int kv = 0; kv < 2; ++kv)
      for (int64_t j = 0; j < len; ++j)
        for (size_t h = 0; h < kvh; ++h)
          for (size_t e = 0; e < hd; ++e) {
            const size_t src = (((size_t)kv * T + j) * kvh + h) * hd + e;
            const float v = t->dtype == SVL_F32 ? ((const float*)t->data)[src]
                                                : [&] {
                                                    uint32_t u = (uint32_t)((const uint16_t*)t->data)[src] << 16;
                                                    float f;
                                                    memcpy(&f, &u, 4);
                                                    return f;
                                                  }();
            (kv ? vh : kh)[l][(h * len + j) * hd + e] = v;
          }
    kp[l] = kh[l].data();
    vp[l] = vh[l].data();
  }
  return state_load_stream_impl(s, stream, len, kp.data(), vp.data());
}

static int state_layer_cache_impl(const svl_state* s, int32_t stream, int32_t layer, float* keys, float* values, int64_t* len,
                          int64_t* first) {
  if (!s) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  const svl_config& c = s->m->cfg;
  if (stream < 0 || stream >= s->B || layer < 0 || layer >= c.num_layers)
    return set_error(SVL_ERR_INVALID_INPUT, "stream or layer out of range");
  const int64_t p = s->pos_host[stream];
  const int64_t L = p < s->slots ? p : s->slots;
  if (len) *len = L;
  if (first) *first = p - L;
  if (!keys && !values) return 0;
  HIP_TRY(hipSetDevice(s->m->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  const int KVH = c.num_kv_heads, hd = c.head_dim, S = s->slots;
  const size_t per = (size_t)KVH * S * hd;
  const int esz = c.kv_dtype == SVL_BF16 ? 2 : 4;
  std::vector<float> h(per);
  float* tmp;
  HIP_TRY(hipMalloc(&tmp, per * 4));
  hipError_t e = hipSuccess;
  for (int kv = 0; kv < 2 && e == hipSuccess; ++kv) {
    float* dst = kv == 0 ? keys : values;
    if (!dst) continue;
    const void* src = (const char*)(kv == 0 ? s->kc[layer] : s->vc[layer]) + (size_t)stream * per * esz;
    e = launch_kv_to_f32(src, c.kv_dtype == SVL_BF16, tmp, per, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e == hipSuccess) e = hipMemcpy(h.data(), tmp, per * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) break;
    for (int g = 0; g < KVH; ++g)
      for (int64_t j = 0; j < L; ++j)
        memcpy(dst + ((size_t)g * L + j) * hd, &h[((size_t)g * S + (size_t)((p - L + j) % S)) * hd], (size_t)hd * 4);
  }
  hipFree(tmp);
  HIP_TRY(e);
  return 0;
}

static int state_positions_impl(const svl_state* s, int64_t* positions) {
  if (!s || !positions) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  for (int b = 0; b < s->B; ++b) positions[b] = s->pos_host[b];
  return 0;
}

static int state_reset_impl(svl_state* s) {
  if (!s) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  HIP_TRY(hipSetDevice(s->m->device));
  HIP_TRY(launch_fill_i32(s->pos, 0, s->B, s->stream));
  HIP_TRY(launch_fill_u32(s->fb_tok, (uint32_t)std::max(s->m->cfg.text_card, 0), s->B, s->stream));
  HIP_TRY(launch_fill_u32(s->tok_out + s->B, 0u, 1, s->stream));
  if (s->turn_state) HIP_TRY(launch_fill_u32(s->turn_state, 0u, s->B, s->stream));
  HIP_TRY(hipStreamSynchronize(s->stream));
  s->pos_host.assign(s->B, 0);
  return 0;
}

void svl_state_destroy(svl_state* s) { delete s; }

static int state_synchronize_impl(svl_state* s) {
  if (!s) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  HIP_TRY(hipSetDevice(s->m->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  TRY(check_abort(s));
  // token ids of the *_async calls are validated on the device (the host never sees them)
  uint32_t bad = 0;
  HIP_TRY(hipMemcpy(&bad, s->tok_out + s->B, 4, hipMemcpyDeviceToHost));
  if (bad) {
    HIP_TRY(launch_fill_u32(s->tok_out + s->B, 0u, 1, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return set_error(SVL_ERR_INVALID_INPUT,
                     "an asynchronous call read a token id past its embedding table (the step used the last "
                     "row); its outputs are not the model's");
  }
  return 0;
}

void* svl_state_stream(const svl_state* s) { return s ? (void*)s->stream : nullptr; }

// Positions of one Transformer::forward block run together at most (rows of the prefill shadow).
constexpr int kPrefillBlock = 256;

// One block of Transformer::forward (SVL/nn/transformer.rs:139-154) for positions t0 .. t0 + tb - 1
// of every stream of an unlimited-context state: the shadow state's batch rows b * tb + i are
// position pos[b] + t0 + i of stream b; they write their keys and values into stream b's ring
// slots and attend to the keys up to their own position (the causal mask of the block), so that
// one pass of the step's phases is the block's forward, each row with the arithmetic of a single
// step.  din / dout: [B][t][d] on the device.
static int prefill_block(svl_state* s, const float* din, float* dout, int64_t t, int64_t t0, int tb, int* pos_stage) {
  const svl_model* m = s->m;
  const int d = m->cfg.d_model, B = s->B;
  if (!s->shadow || s->shadow->B != B * tb) {
    delete s->shadow;
    s->shadow = nullptr;
    svl_state* sh = nullptr;
    TRY(make_state(m, B * tb, s->slots, &sh, s, tb));
    s->shadow = sh;
    for (Phase& ph : sh->fwd_prog.phases)
      if (ph.kind == PH_COPY_IN || ph.kind == PH_COPY_OUT) {
        ph.cp.x_stride = d;
        ph.cp.y_stride = d;
      }
    HIP_TRY(hipMemcpyAsync(sh->fwd_prog.dev, sh->fwd_prog.phases.data(), sh->fwd_prog.phases.size() * sizeof(Phase),
                           hipMemcpyHostToDevice, sh->stream));
  }
  svl_state* sh = s->shadow;
  const size_t rows = (size_t)B * tb;
  if (sh->fwd_cap < 2 * rows * d * 4) {
    void* p;
    TRY(sh->alloc(&p, 2 * rows * d * 4));
    sh->fwd = (float*)p;
    sh->fwd_cap = 2 * rows * d * 4;
  }
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < tb; ++i) {
      sh->pos_host[(size_t)b * tb + i] = s->pos_host[b] + t0 + i;
      pos_stage[(size_t)b * tb + i] = (int)(s->pos_host[b] + t0 + i);
    }
  HIP_TRY(hipMemcpyAsync(sh->pos, pos_stage, rows * sizeof(int), hipMemcpyHostToDevice, sh->stream));
  TRY(check_room(sh, 1));
  float* sin = sh->fwd;
  float* sout = sh->fwd + rows * d;
  HIP_TRY(hipMemcpy2DAsync(sin, (size_t)tb * d * 4, din + (size_t)t0 * d, (size_t)t * d * 4, (size_t)tb * d * 4, B,
                           hipMemcpyDeviceToDevice, sh->stream));
  StepParams P{};
  P.fwd_in = sin;
  P.fwd_out = sout;
  P.fwd_T = 1;
  TRY(run_program(sh, sh->fwd_prog, P, 1));
  HIP_TRY(hipMemcpy2DAsync(dout + (size_t)t0 * d, (size_t)t * d * 4, sout, (size_t)tb * d * 4, (size_t)tb * d * 4, B,
                           hipMemcpyDeviceToDevice, sh->stream));
  return 0;
}

static int transformer_forward_impl(const svl_model* m, svl_state* s, const float* xs, int64_t t, float* ys) {
  if (!m || !s || (t > 0 && (!xs || !ys))) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  if (t < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative length");
  if (t == 0) return 0;
  TRY(check_room(s, t));
  HIP_TRY(hipSetDevice(m->device));
  const int d = m->cfg.d_model;
  const size_t bytes = (size_t)s->B * t * d * 4;
  if (s->fwd_cap < 2 * bytes) {
    void* p;
    TRY(s->alloc(&p, 2 * bytes));
    s->fwd = (float*)p;
    s->fwd_cap = 2 * bytes;
  }
  float* din = s->fwd;
  float* dout = s->fwd + (size_t)s->B * t * d;
  HIP_TRY(hipMemcpyAsync(din, xs, bytes, hipMemcpyHostToDevice, s->stream));
  // Blocks of positions when nothing is evicted from the ring meanwhile (unlimited context: the
  // ring holds every position); a windowed ring has no room for a block's later keys.
  const int tmax = std::min<int64_t>(kPrefillBlock, kMaxBatch / s->B);
  if (m->cfg.context == 0 && t > 1 && tmax > 1) {
    const int64_t nblk = (t + tmax - 1) / tmax;
    const int tb = (int)((t + nblk - 1) / nblk);  // equal blocks but the last
    s->pos_stage.resize((size_t)(nblk + 1) * s->B * tb + s->B);
    int64_t t0 = 0;
    for (int64_t k = 0; k < nblk; ++k, t0 += tb)
      TRY(prefill_block(s, din, dout, t, t0, (int)std::min<int64_t>(tb, t - t0), s->pos_stage.data() + (size_t)k * s->B * tb));
    int* np = s->pos_stage.data() + (size_t)nblk * s->B * tb;
    for (int b = 0; b < s->B; ++b) {
      s->pos_host[b] += t;
      np[b] = (int)s->pos_host[b];
    }
    HIP_TRY(hipMemcpyAsync(s->pos, np, (size_t)s->B * sizeof(int), hipMemcpyHostToDevice, s->stream));
  } else {
    // one position at a time: the copy phases read column `step` of [B][T][d]
    for (Phase& ph : s->fwd_prog.phases)
      if (ph.kind == PH_COPY_IN || ph.kind == PH_COPY_OUT) {
        ph.cp.x_stride = (int)(t * d);
        ph.cp.y_stride = ph.kind == PH_COPY_IN ? d : (int)(t * d);
      }
    HIP_TRY(hipMemcpyAsync(s->fwd_prog.dev, s->fwd_prog.phases.data(), s->fwd_prog.phases.size() * sizeof(Phase),
                           hipMemcpyHostToDevice, s->stream));
    StepParams P{};
    P.fwd_in = din;
    P.fwd_out = dout;
    P.fwd_T = (int)t;
    TRY(run_program(s, s->fwd_prog, P, t));
  }
  HIP_TRY(hipMemcpyAsync(ys, dout, bytes, hipMemcpyDeviceToHost, s->stream));
  HIP_TRY(hipStreamSynchronize(s->stream));
  return check_abort(s);
}

static int stt_step_impl(const svl_model* m, svl_state* s, const uint32_t* text_tokens, const uint32_t* audio_tokens,
                 uint32_t* out_tokens, float* out_logits) {
  return svl_stt_step_heads(m, s, text_tokens, audio_tokens, out_tokens, out_logits, nullptr);
}

static int stt_step_heads_impl(const svl_model* m, svl_state* s, const uint32_t* text_tokens, const uint32_t* audio_tokens,
                       uint32_t* out_tokens, float* out_logits, float* out_probs) {
  if (!m || !s || !text_tokens || !audio_tokens || !out_tokens) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  const svl_config& c = m->cfg;
  if (c.kind != SVL_MODEL_STT) return set_error(SVL_ERR_CONFIG, "not an STT model");
  for (int b = 0; b < s->B; ++b) {
    if (text_tokens[b] > (uint32_t)c.text_card)
      return set_error(SVL_ERR_INVALID_INPUT, "text token %u out of range", text_tokens[b]);
    for (int i = 0; i < c.n_q; ++i)
      if (audio_tokens[(size_t)b * c.n_q + i] > (uint32_t)c.card)
        return set_error(SVL_ERR_INVALID_INPUT, "audio token %u out of range", audio_tokens[(size_t)b * c.n_q + i]);
  }
  TRY(check_room(s, 1));
  HIP_TRY(hipSetDevice(m->device));
  uint32_t* dtext = s->tok_in;
  uint32_t* daudio = s->tok_in + s->B;
  HIP_TRY(hipMemcpyAsync(dtext, text_tokens, (size_t)s->B * 4, hipMemcpyHostToDevice, s->stream));
  HIP_TRY(hipMemcpyAsync(daudio, audio_tokens, (size_t)s->B * c.n_q * 4, hipMemcpyHostToDevice, s->stream));
  // LanguageModel::step takes the caller's tokens as they are (no first-step rule).
  s->stt.phases[0].e.initial_at_zero = 0;
  HIP_TRY(hipMemcpyAsync(s->stt.dev, s->stt.phases.data(), sizeof(Phase), hipMemcpyHostToDevice, s->stream));
  int rc = run_program(s, s->stt, stt_params(s, daudio, dtext, s->tok_out), 1);
  s->stt.phases[0].e.initial_at_zero = 1;
  HIP_TRY(hipMemcpyAsync(s->stt.dev, s->stt.phases.data(), sizeof(Phase), hipMemcpyHostToDevice, s->stream));
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(out_tokens, s->tok_out, (size_t)s->B * 4, hipMemcpyDeviceToHost, s->stream));
  if (out_logits)
    HIP_TRY(hipMemcpyAsync(out_logits, s->logits, (size_t)s->B * c.text_card * 4, hipMemcpyDeviceToHost, s->stream));
  if (out_probs && c.extra_heads_num > 0)
    HIP_TRY(hipMemcpyAsync(out_probs, s->xprob, (size_t)s->B * c.extra_heads_num * 4, hipMemcpyDeviceToHost,
                           s->stream));
  HIP_TRY(hipStreamSynchronize(s->stream));
  return check_abort(s);
}

static int stt_recognize_async_impl(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* d_audio_tokens,
                            uint32_t* d_out_tokens) {
  return svl_stt_recognize_heads_async(m, s, n_steps, d_audio_tokens, d_out_tokens, nullptr);
}

// The turn detector's parameters of a call, written after the streams' states (kernel arguments
// carry the values: nothing on the host has to outlive the call).
int set_turn_config(svl_state* s, const svl_turn_config* turn) {
  uint32_t th;
  memcpy(&th, &turn->threshold, 4);
  HIP_TRY(launch_fill_u32(s->turn_state + s->B, th, 1, s->stream));
  HIP_TRY(launch_fill_u32(s->turn_state + s->B + 1, (uint32_t)std::max(turn->frames, 1), 1, s->stream));  // frames.max(1)
  HIP_TRY(launch_fill_u32(s->turn_state + s->B + 2, (uint32_t)turn->head, 1, s->stream));
  return 0;
}

static int stt_recognize_heads_async_impl(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* d_audio_tokens,
                                  uint32_t* d_out_tokens, float* d_out_probs, const svl_turn_config* turn = nullptr,
                                  int32_t* d_out_turn = nullptr) {
  if (!m || !s || (n_steps > 0 && (!d_audio_tokens || !d_out_tokens)))
    return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  if (m->cfg.kind != SVL_MODEL_STT) return set_error(SVL_ERR_CONFIG, "not an STT model");
  if (n_steps < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative step count");
  if (n_steps == 0) return 0;
  TRY(check_room(s, n_steps));
  HIP_TRY(hipSetDevice(m->device));
  if (d_out_turn) TRY(set_turn_config(s, turn));
  return run_program(s, s->stt,
                     stt_params(s, d_audio_tokens, nullptr, d_out_tokens, m->cfg.extra_heads_num > 0 ? d_out_probs : nullptr,
                                d_out_turn),
                     n_steps);
}

static int stt_recognize_impl(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                      uint32_t* out_tokens) {
  return svl_stt_recognize_heads(m, s, n_steps, audio_tokens, out_tokens, nullptr);
}

static int stt_recognize_heads_impl(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                            uint32_t* out_tokens, float* out_probs, const svl_turn_config* turn = nullptr,
                            int32_t* out_turn = nullptr) {
  if (!m || !s || (n_steps > 0 && (!audio_tokens || !out_tokens))) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  const svl_config& c = m->cfg;
  if (c.kind != SVL_MODEL_STT) return set_error(SVL_ERR_CONFIG, "not an STT model");
  if (n_steps < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative step count");
  if (n_steps == 0) return 0;
  const size_t na = (size_t)n_steps * s->B * c.n_q;
  for (size_t i = 0; i < na; ++i)
    if (audio_tokens[i] > (uint32_t)c.card) return set_error(SVL_ERR_INVALID_INPUT, "audio token %u out of range", audio_tokens[i]);
  TRY(check_room(s, n_steps));
  HIP_TRY(hipSetDevice(m->device));
  const size_t np = out_probs ? (size_t)n_steps * s->B * std::max(c.extra_heads_num, 0) : 0;
  uint32_t *da, *dout;
  float* dprob = nullptr;
  const size_t nt = (size_t)n_steps * s->B;
  if (out_turn) TRY(set_turn_config(s, turn));
  HIP_TRY(hipMalloc(&da, na * 4));
  // the output tokens, then the turn ends when asked for
  hipError_t e = hipMalloc(&dout, nt * 4 * (out_turn ? 2 : 1));
  int32_t* dturn = out_turn ? (int32_t*)(dout + nt) : nullptr;
  if (e == hipSuccess && np) {
    e = hipMalloc(&dprob, np * 4);
    if (e != hipSuccess) hipFree(dout);
  }
  if (e != hipSuccess) {
    hipFree(da);
    HIP_TRY(e);
  }
  int rc = 0;
  e = hipMemcpyAsync(da, audio_tokens, na * 4, hipMemcpyHostToDevice, s->stream);
  if (e == hipSuccess) rc = run_program(s, s->stt, stt_params(s, da, nullptr, dout, dprob, dturn), n_steps);
  if (e == hipSuccess && rc == 0) e = hipMemcpyAsync(out_tokens, dout, nt * 4, hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess && rc == 0 && dturn) e = hipMemcpyAsync(out_turn, dturn, nt * 4, hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess && rc == 0 && np) e = hipMemcpyAsync(out_probs, dprob, np * 4, hipMemcpyDeviceToHost, s->stream);
  hipError_t e2 = hipStreamSynchronize(s->stream);
  hipFree(da);
  hipFree(dout);
  if (dprob) hipFree(dprob);
  if (rc) return rc;
  HIP_TRY(e);
  HIP_TRY(e2);
  return check_abort(s);
}

static int bench_phase_impl(const svl_model* m, svl_state* s, int program, int phase, int reps, float* us_per_launch,
                            int* info) {
  if (!m || !s || !us_per_launch || !info) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  Program* p = program == 0 ? &s->stt : (program == 1 ? &s->tts : nullptr);
  if (!p || p->phases.empty()) return set_error(SVL_ERR_INVALID_INPUT, "no such program for this model");
  if (phase < 0 || phase >= (int)p->phases.size() || reps <= 0)
    return set_error(SVL_ERR_INVALID_INPUT, "phase %d of %zu, reps %d", phase, p->phases.size(), reps);
  const Phase& ph = p->phases[phase];
  info[0] = ph.kind;
  info[1] = (ph.kind == PH_GEMV || ph.kind == PH_QUANT || ph.kind == PH_QGEMM) ? ph.g.L.fmt : -1;
  info[2] = (ph.kind == PH_GEMV || ph.kind == PH_QUANT || ph.kind == PH_QGEMM) ? ph.g.L.out : 0;
  info[3] = (ph.kind == PH_GEMV || ph.kind == PH_QUANT || ph.kind == PH_QGEMM) ? ph.g.L.in : 0;
  info[4] = ph.units;
  info[5] = ph.kind == PH_ATTN ? ph.at.hpu : 0;  // heads per unit (a split launch: 1 head, split over units)
  if (ph.kind == PH_GEMV && ph.g.epi == EPI_QKV_ROPE) TRY(check_room(s, 1));
  HIP_TRY(hipSetDevice(m->device));
  TRY(refresh_attn_order(s));
  const float* rope;
  {
    std::lock_guard<std::mutex> lock(m->rope_mu);
    rope = m->rope;
  }
  TRY(refresh_rope(s, *p, rope));
  // the embedding phase reads token ids: the state's own token staging (zeros are valid ids)
  HIP_TRY(launch_fill_u32(s->tok_in, 0u, (size_t)s->B * (1 + std::max(m->cfg.n_q, 0)), s->stream));
  StepParams P = stt_params(s, s->tok_in + s->B, s->tok_in, nullptr);
  P.prog = p->dev;
  P.nphase = (int)p->phases.size();
  P.sync = s->sync;
  P.pos = s->pos;
  P.B = s->B;
  P.n_steps = 1;
  // an attention phase launches as the step would at the state's positions (split or not)
  const int split = ph.kind == PH_ATTN ? attn_split(s, 0) : 1;
  auto one = [&]() -> int {
    if (split > 1) return launch_split(s, ph, P, 0, split);
    HIP_TRY(launch_phase(ph, P, 0, p->smem, s->stream));
    return 0;
  };
  TRY(one());  // warm-up
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  hipError_t e = hipEventCreate(&e1);
  if (e != hipSuccess) {
    hipEventDestroy(e0);
    HIP_TRY(e);
  }
  e = hipEventRecord(e0, s->stream);
  int rc = 0;
  for (int r = 0; r < reps && e == hipSuccess && !rc; ++r) rc = one();
  if (rc) {
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return rc;
  }
  if (e == hipSuccess) e = hipEventRecord(e1, s->stream);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  HIP_TRY(e);
  *us_per_launch = ms * 1000.0f / (float)reps;
  return 0;
}

static int stt_recognize_noalloc_impl(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                                      uint32_t* out_tokens) {
  if (!m || !s || (n_steps > 0 && (!audio_tokens || !out_tokens))) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  const svl_config& c = m->cfg;
  if (c.kind != SVL_MODEL_STT) return set_error(SVL_ERR_CONFIG, "not an STT model");
  if (n_steps < 0) return set_error(SVL_ERR_INVALID_INPUT, "negative step count");
  if (n_steps == 0) return 0;
  const size_t na = (size_t)n_steps * s->B * c.n_q, nt = (size_t)n_steps * s->B;
  if ((na + nt) * 4 > kNoAllocScratchBytes)
    return set_error(SVL_ERR_INVALID_INPUT, "%lld steps x %d streams x (%d + 1) token ids exceed the %zu-byte scratch",
                     (long long)n_steps, s->B, c.n_q, kNoAllocScratchBytes);
  for (size_t i = 0; i < na; ++i)
    if (audio_tokens[i] > (uint32_t)c.card) return set_error(SVL_ERR_INVALID_INPUT, "audio token %u out of range", audio_tokens[i]);
  int64_t top = 0;
  for (int64_t p : s->pos_host) top = std::max(top, p + n_steps);
  {
    std::lock_guard<std::mutex> lock(m->rope_mu);
    if (top > m->rope_len)
      return set_error(SVL_ERR_INVALID_INPUT, "positions up to %lld: the RoPE table covers %lld (later rows are prepared "
                       "per call by svl_stt_recognize)", (long long)top, (long long)m->rope_len);
  }
  TRY(check_room(s, n_steps));  // capacity only: the table covers every position
  HIP_TRY(hipSetDevice(m->device));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  unsigned char* base;
  TRY(scratch_on(m->device, &base));
  uint32_t* da = (uint32_t*)base;
  uint32_t* dout = da + na;
  HIP_TRY(hipMemcpyAsync(da, audio_tokens, na * 4, hipMemcpyHostToDevice, s->stream));
  TRY(run_program(s, s->stt, stt_params(s, da, nullptr, dout, nullptr), n_steps));
  HIP_TRY(hipMemcpyAsync(out_tokens, dout, nt * 4, hipMemcpyDeviceToHost, s->stream));
  HIP_TRY(hipStreamSynchronize(s->stream));
  return check_abort(s);
}

static int tts_backbone_step_impl(const svl_model* m, svl_state* s, const float* latent, float* out_z) {
  if (!m || !s || !out_z) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  const svl_config& c = m->cfg;
  if (c.kind != SVL_MODEL_TTS) return set_error(SVL_ERR_CONFIG, "not a TTS model");
  TRY(check_room(s, 1));
  HIP_TRY(hipSetDevice(m->device));
  const int d = c.d_model, ld = c.latent_dim;
  if (latent) {
    HIP_TRY(hipMemcpyAsync(s->in, latent, (size_t)s->B * ld * 4, hipMemcpyHostToDevice, s->stream));
  } else {
    for (int b = 0; b < s->B; ++b)
      HIP_TRY(hipMemcpyAsync(s->in + (size_t)b * ld, m->bos, (size_t)ld * 4, hipMemcpyDeviceToDevice, s->stream));
  }
  TRY(run_program(s, s->tts, StepParams{}, 1));
  const int zd = c.z_dim > 0 ? c.z_dim : d;
  HIP_TRY(hipMemcpyAsync(out_z, s->z, (size_t)s->B * zd * 4, hipMemcpyDeviceToHost, s->stream));
  HIP_TRY(hipStreamSynchronize(s->stream));
  return check_abort(s);
}

// FlowLm::step (SVL/tts/flow_lm.rs:162-185).  `host`: the pointers are host memory and the
// call returns with the outputs there; otherwise device pointers, enqueued only.
static int tts_step_impl(const svl_model* m, svl_state* s, const float* latent, const float* noise, int32_t steps,
                         bool host, float* out_latent, float* out_eos_logit) {
  if (!m || !s || !noise || !out_latent) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  if (s->m != m) return set_error(SVL_ERR_INVALID_INPUT, "state belongs to another model");
  const svl_config& c = m->cfg;
  if (c.kind != SVL_MODEL_TTS) return set_error(SVL_ERR_CONFIG, "not a TTS model");
  if (c.flow_dim <= 0) return set_error(SVL_ERR_CONFIG, "the model has no flow head (flow_dim 0)");
  TRY(check_room(s, 1));
  HIP_TRY(hipSetDevice(m->device));
  const int ld = c.latent_dim;
  const size_t lb = (size_t)s->B * ld * 4;
  const hipMemcpyKind in_kind = host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
  const hipMemcpyKind out_kind = host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  if (latent) {
    HIP_TRY(hipMemcpyAsync(s->in, latent, lb, in_kind, s->stream));
  } else {
    for (int b = 0; b < s->B; ++b)
      HIP_TRY(hipMemcpyAsync(s->in + (size_t)b * ld, m->bos, (size_t)ld * 4, hipMemcpyDeviceToDevice, s->stream));
  }
  HIP_TRY(hipMemcpyAsync(s->fh_noise, noise, lb, in_kind, s->stream));
  TRY(run_program(s, s->tts, StepParams{}, 1));
  TRY(run_flow_head(s, steps));
  HIP_TRY(hipMemcpyAsync(out_latent, s->fh_x, lb, out_kind, s->stream));
  if (out_eos_logit)
    HIP_TRY(hipMemcpy2DAsync(out_eos_logit, 4, s->fh_ce + m->flow.dim, (size_t)(m->flow.dim + 1) * 4, 4, s->B, out_kind,
                             s->stream));
  if (!host) return 0;
  HIP_TRY(hipStreamSynchronize(s->stream));
  return check_abort(s);
}

static int tts_step_sync_impl(const svl_model* m, svl_state* s, const float* latent, const float* noise, int32_t steps,
                              float eos_threshold, float* out_latent, float* out_eos_logit, int32_t* out_eos) {
  if (!s) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
  std::vector<float> logits((size_t)s->B);
  TRY(tts_step_impl(m, s, latent, noise, steps, true, out_latent, logits.data()));
  for (int b = 0; b < s->B; ++b) {
    if (out_eos_logit) out_eos_logit[b] = logits[b];
    if (out_eos) out_eos[b] = logits[b] > eos_threshold ? 1 : 0;  // SVL/tts/flow_lm.rs:184
  }
  return 0;
}



// The C entry points: no C++ exception crosses the boundary.
int svl_device_count(int* count) {
  return guarded([&] { return device_count_impl(count); });
}

int svl_bench_copy(int device, const void* src, void* dst, size_t bytes, void* stream) {
  return guarded([&] { return bench_copy_impl(device, src, dst, bytes, stream); });
}

int svl_bench_read(int device, const void* src, size_t bytes, int blocks, int threads, uint32_t* out, void* stream) {
  return guarded([&] { return bench_read_impl(device, src, bytes, blocks, threads, out, stream); });
}

int svl_bench_activation(int device, int kind, const float* x, size_t n, float* y, void* stream) {
  return guarded([&] { return bench_activation_impl(device, kind, x, n, y, stream); });
}

int svl_bench_row_stats(int device, const float* x, int rows, int k, int norm, float* out, void* stream) {
  return guarded([&] { return bench_row_stats_impl(device, x, rows, k, norm, out, stream); });
}

int svl_rvq_create(const svl_tensor* tensors, size_t count, int32_t n_q, int32_t bins, int device, svl_rvq** out) {
  return guarded([&] { return rvq_create_impl(tensors, count, n_q, bins, device, out); });
}

void svl_rvq_destroy(svl_rvq* rvq) { delete rvq; }

int svl_rvq_encode(svl_rvq* rvq, int32_t batch, int32_t frames, const float* latents, uint32_t* codes) {
  return guarded([&] { return rvq_encode_impl(rvq, batch, frames, latents, codes); });
}

int svl_rvq_encode_async(svl_rvq* rvq, int32_t batch, int32_t frames, const float* d_latents, uint32_t* d_codes) {
  return guarded([&] { return rvq_encode_async_impl(rvq, batch, frames, d_latents, d_codes); });
}

int svl_rvq_synchronize(svl_rvq* rvq) {
  return guarded([&] {
    if (!rvq) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
    HIP_TRY(hipSetDevice(rvq->device));
    HIP_TRY(hipStreamSynchronize(rvq->stream));
    return 0;
  });
}

int svl_model_create(const svl_config* cfg, const svl_tensor* tensors, size_t count, int device, svl_model** out) {
  return guarded([&] { return model_create_impl(cfg, tensors, count, device, out); });
}

int svl_model_linear_weight(const svl_model* m, const char* name, float* f32, size_t f32_count, void* blocks,
                            size_t block_bytes) {
  return guarded([&] { return model_linear_weight_impl(m, name, f32, f32_count, blocks, block_bytes); });
}

int svl_state_create(const svl_model* model, int32_t batch, int32_t capacity, svl_state** out) {
  return guarded([&] { return state_create_impl(model, batch, capacity, out); });
}

int svl_state_duplicate(const svl_state* s, svl_state** out) {
  return guarded([&] { return state_duplicate_impl(s, out); });
}

int svl_state_load_stream(svl_state* s, int32_t stream, int64_t len, const float* const* keys,
                          const float* const* values) {
  return guarded([&] { return state_load_stream_impl(s, stream, len, keys, values); });
}

int svl_state_layer_cache(const svl_state* s, int32_t stream, int32_t layer, float* keys, float* values, int64_t* len,
                          int64_t* first) {
  return guarded([&] { return state_layer_cache_impl(s, stream, layer, keys, values, len, first); });
}

int svl_state_positions(const svl_state* s, int64_t* positions) {
  return guarded([&] { return state_positions_impl(s, positions); });
}

int svl_state_reset(svl_state* s) {
  return guarded([&] { return state_reset_impl(s); });
}

int svl_state_synchronize(svl_state* s) {
  return guarded([&] { return state_synchronize_impl(s); });
}

int svl_transformer_forward(const svl_model* m, svl_state* s, const float* xs, int64_t t, float* ys) {
  return guarded([&] { return transformer_forward_impl(m, s, xs, t, ys); });
}

int svl_stt_step(const svl_model* m, svl_state* s, const uint32_t* text_tokens, const uint32_t* audio_tokens,
                 uint32_t* out_tokens, float* out_logits) {
  return guarded([&] { return stt_step_impl(m, s, text_tokens, audio_tokens, out_tokens, out_logits); });
}

int svl_stt_step_heads(const svl_model* m, svl_state* s, const uint32_t* text_tokens, const uint32_t* audio_tokens,
                       uint32_t* out_tokens, float* out_logits, float* out_probs) {
  return guarded([&] { return stt_step_heads_impl(m, s, text_tokens, audio_tokens, out_tokens, out_logits, out_probs); });
}

int svl_stt_recognize_async(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* d_audio_tokens,
                            uint32_t* d_out_tokens) {
  return guarded([&] { return stt_recognize_async_impl(m, s, n_steps, d_audio_tokens, d_out_tokens); });
}

int svl_stt_recognize_heads_async(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* d_audio_tokens,
                                  uint32_t* d_out_tokens, float* d_out_probs) {
  return guarded([&] { return stt_recognize_heads_async_impl(m, s, n_steps, d_audio_tokens, d_out_tokens, d_out_probs); });
}

int svl_stt_recognize(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                      uint32_t* out_tokens) {
  return guarded([&] { return stt_recognize_impl(m, s, n_steps, audio_tokens, out_tokens); });
}

int svl_stt_recognize_heads(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                            uint32_t* out_tokens, float* out_probs) {
  return guarded([&] { return stt_recognize_heads_impl(m, s, n_steps, audio_tokens, out_tokens, out_probs); });
}

int svl_tts_backbone_step(const svl_model* m, svl_state* s, const float* latent, float* out_z) {
  return guarded([&] { return tts_backbone_step_impl(m, s, latent, out_z); });
}
int svl_bench_phase(const svl_model* m, svl_state* s, int program, int phase, int reps, float* us_per_launch,
                    int* info) {
  return guarded([&] { return bench_phase_impl(m, s, program, phase, reps, us_per_launch, info); });
}

int svl_stt_recognize_noalloc(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                              uint32_t* out_tokens) {
  return guarded([&] { return stt_recognize_noalloc_impl(m, s, n_steps, audio_tokens, out_tokens); });
}

int svl_stt_recognize_turns(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* audio_tokens,
                            const svl_turn_config* turn, uint32_t* out_tokens, float* out_probs, int32_t* out_turn_ends) {
  return guarded([&] {
    if (!turn || !out_turn_ends) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
    return stt_recognize_heads_impl(m, s, n_steps, audio_tokens, out_tokens, out_probs, turn, out_turn_ends);
  });
}

int svl_stt_recognize_turns_async(const svl_model* m, svl_state* s, int64_t n_steps, const uint32_t* d_audio_tokens,
                                  const svl_turn_config* turn, uint32_t* d_out_tokens, float* d_out_probs,
                                  int32_t* d_out_turn_ends) {
  return guarded([&] {
    if (!turn || !d_out_turn_ends) return set_error(SVL_ERR_INVALID_INPUT, "null argument");
    return stt_recognize_heads_async_impl(m, s, n_steps, d_audio_tokens, d_out_tokens, d_out_probs, turn,
                                          d_out_turn_ends);
  });
}

int svl_state_load_voice(svl_state* s, int32_t stream, const svl_tensor* tensors, size_t count) {
  return guarded([&] { return state_load_voice_impl(s, stream, tensors, count); });
}

int svl_tts_step(const svl_model* m, svl_state* s, const float* latent, const float* noise, int32_t decode_steps,
                 float eos_threshold, float* out_latent, float* out_eos_logit, int32_t* out_eos) {
  return guarded([&] {
    return tts_step_sync_impl(m, s, latent, noise, decode_steps, eos_threshold, out_latent, out_eos_logit, out_eos);
  });
}

int svl_tts_step_async(const svl_model* m, svl_state* s, const float* d_latent, const float* d_noise,
                       int32_t decode_steps, float* d_out_latent, float* d_out_eos_logit) {
  return guarded([&] {
    return tts_step_impl(m, s, d_latent, d_noise, decode_steps, false, d_out_latent, d_out_eos_logit);
  });
}

}  // extern "C"
