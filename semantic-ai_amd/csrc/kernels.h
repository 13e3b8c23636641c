// Launch interface of the step kernels (host side).  Internal to libsvl.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svl {

enum WeightFmt { FMT_F32 = 0, FMT_BF16 = 1, FMT_Q8_0 = 3, FMT_Q4K = 4, FMT_F32C = 5, FMT_BF16C = 6, FMT_Q4_0 = 7 };
enum NormKind { NORM_NONE = 0, NORM_LAYER = 1, NORM_RMS = 2 };
enum Epilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU_GATE = 2, EPI_QKV_ROPE = 3, EPI_GELU = 4, EPI_GELU_ERF = 5 };

// One linear layer as held on the device.
//   FMT_F32 / FMT_BF16: w = [out][in] row-major.
//   FMT_F32C / FMT_BF16C: chain-packed dense weights, for in % (16 E) == 0 with E = 4 (f32) or
//     8 (bf16) elements per 16 bytes: element (row, 16 c + l) is at
//     ((row * in / (16 E) + c / E) * 16 + l) * E + c % E, i.e. the 16 lane chains of a row are
//     interleaved 16 bytes at a time.
//   FMT_Q8_0: w = int8 quants [out][in]; scale = f16 block scales [out][in/32].
//   FMT_Q4_0: w = candle's Q4_0 code bytes [out][in/2]: the 16 bytes of block blk of a row at
//     byte 16 blk, byte j holding the code of element j in its low nibble and of element j + 16
//     in its high nibble (value = (code - 8) * d); scale = f16 block scales [out][in/32].
//   FMT_Q4K: w = 144-byte super-blocks [out][in/256]: f16 d, f16 dmin and the 12 bytes of packed
//     6-bit sub-block scales and mins exactly as candle's BlockQ4K holds them, then the 128 quant
//     bytes with each 32-byte group lane-grouped: byte 4 l + g of a group is candle's byte
//     8 g + l of it, so that one dword holds the four values that i32 lane l of the vec_dot
//     adds for the group's two sub-blocks (low and high nibbles).
struct LinearDev {
  int fmt = FMT_F32;
  int out = 0, in = 0;
  void* w = nullptr;
  uint16_t* scale = nullptr;
};

struct GemvArgs {
  LinearDev L;
  int B;               // batch rows
  int ipw;             // work items per unit (rows, or gate/value pairs for the SiLU gate)
  int parts;           // units per batch row = ceil(items / ipw)
  int maxb;            // Q8_0 / Q4K: weight blocks per weight-wave thread and unit
                       // (1 .. kWBlocks, Q4K 1 .. kQ4Blocks)
  const float* x;      // input [B][x_stride]
  int x_stride;
  int norm;            // NormKind applied to x in the prologue
  const float* nw;
  const float* nb;
  float eps;
  int epi;             // Epilogue
  float* y;            // STORE/SILU/GELU: [B][y_stride]
  int y_stride;
  float* resid;        // RESID: resid[b][row] += y (* lscale[row])
  int resid_stride;
  const float* lscale;
  int ff_hidden;       // SILU: gate rows j, value rows j + ff_hidden
  // QKV_ROPE
  int* pos;            // [B] positions (read by QKV_ROPE, advanced when advance_pos)
  const float* rope;   // [rope_cap][hd/2][cos, sin] computed on the host (positions < rope_cap)
  int rope_cap;
  const float* rope_ovf;    // positions >= rope_cap: row p + rope_delta[b] of this call's rows
  const int* rope_delta;    // [B]
  int H, KVH, hd;
  float* q_out;        // [B][H*hd]
  void* kc;            // [B][KVH][cap][hd]
  void* vc;
  int cap;
  int kv_bf16;
  int kv_group;        // > 1: batch rows b share the ring of stream b / kv_group (positions of one
                       // stream processed together, prefill); 0 or 1: one ring per batch row
  int advance_pos;
  // batched Q8_0 path (PH_QUANT / PH_QGEMM): the quantized input rows of the whole batch
  int8_t* xq;          // [ceil(L.in / 128)][B][128]: chunk-major, so that a chunk of all rows is contiguous
  float* xdq;          // [B][L.in / 32] (f16-rounded block scales)
};

struct AttnArgs {
  const float* q;      // [B][H*hd]
  const void* kc;
  const void* vc;
  int* pos;
  int B, H, KVH, hd, cap, window;  // window 0 = unlimited
  int kv_bf16;
  float scale;
  float* out;          // [B][H*hd]
  int hpu;             // heads per unit (1 or 2); units = B * H / hpu
  const int* order;    // [B] the stream of units k H / hpu .. (k + 1) H / hpu - 1
  int kv_group;        // as GemvArgs::kv_group
  // split launches (launch_attn_split): the tag that marks this launch's entries in the score
  // rows (distinct from the tags of the state's earlier launches)
  unsigned split_tag;
};

struct EmbedArgs {
  const void* text_emb;     // [text_card+1][d]
  const void* emb;          // n_q tables back to back, [n_q][card+1][d]
  int tables_bf16;
  int d, n_q, card, text_card, B;
  const uint32_t* text_tok; // [B] explicit tokens, or null: use fb_tok
  uint32_t* fb_tok;         // [B] feedback tokens (previous argmax)
  const uint32_t* audio;    // [B][n_q]
  int initial_at_zero;      // a stream at position 0 sees `card` audio tokens
  int* pos;
  float* x;                 // [B][d]
  void* stage;              // [B][n_q][d] table rows of the next step's audio tokens, gathered
                            // during the previous step (table element type), or null
  uint32_t* bad_token;      // set to 1 when a token id is past its table (the id is clamped)
};

struct ArgmaxArgs {
  const float* logits;      // [B][V]
  int B, V;
  uint32_t* fb_tok;         // [B]
  uint32_t* out;            // [B] or null
  // STT extra heads: softmax over each head's hd logits, element 0 (nh = 0: none)
  const float* xlogits;     // [B][nh * hd]
  int nh, hd;
  float* xprob;             // [B][nh], the last step's probabilities
  // per stream: bit 0 = the recognizer holds word tokens not yet emitted, bit 1 = the turn
  // detector's in_turn, bits 2.. = its count of consecutive frames above the threshold; then the
  // detector's parameters of the current call: threshold (f32 bits), frames (>= 1), head
  uint32_t* turn_state;     // [B + 3]
};

struct NormArgs {           // y[b] = norm(x[b]) (TTS out_norm without z_proj)
  const float* x;
  int x_stride;
  float* y;
  int y_stride;
  int B, d, norm;
  const float* w;
  const float* b;
  float eps;
};

struct CopyArgs {           // y[b][0..n) = x[b][0..n)
  const float* x;
  int x_stride;
  float* y;
  int y_stride;
  int B, n;
  int advance;              // step-indexed source/destination (see StepParams)
};

// One phase of a step program: a unit function applied to `units` work units.
enum PhaseKind { PH_EMBED = 0, PH_GEMV = 1, PH_ATTN = 2, PH_ARGMAX = 4, PH_NORM = 5, PH_COPY_IN = 6, PH_COPY_OUT = 7,
                 PH_QUANT = 8, PH_QGEMM = 9 };

struct Phase {
  int kind;
  int units;
  GemvArgs g;
  AttnArgs at;
  EmbedArgs e;
  ArgmaxArgs am;
  NormArgs nm;
  CopyArgs cp;
};

// Grid barrier counters (device memory, zeroed at creation): 8 group counters and a top
// counter, each in its own 128-byte line, the release generation, and an abort flag.
struct SyncState {
  unsigned group[8][32];
  unsigned top[32];
  unsigned release[32];
  unsigned abort_flag[32];
};

// Per-launch inputs of a step program run for n_steps steps.
struct StepParams {
  const Phase* prog;
  int nphase;
  int n_steps;
  int* pos;                      // [B] stream positions (the persistent kernel caches them per step in LDS)
  int B;
  SyncState* sync;
  unsigned gen0;                 // barriers completed by earlier launches on this state
  const uint32_t* audio;         // step s: audio + s * audio_stride
  size_t audio_stride;
  const uint32_t* text;          // step s: text + s * text_stride, or null (feedback)
  size_t text_stride;
  uint32_t* out_tok;             // step s: out_tok + s * out_stride, or null
  size_t out_stride;
  float* out_prob;               // step s: out_prob + s * prob_stride (extra heads), or null
  size_t prob_stride;
  const float* fwd_in;           // [B][T][d], step s reads column s
  float* fwd_out;
  int fwd_T;
  int32_t* out_turn;             // step s: out_turn + s * B (turn ends), or null: no turn detector
};

constexpr int kStepThreads = 1024;                       // workgroup of the step kernels
constexpr int kRowThreads = 512;                         // row waves: threads [0, 512)
constexpr int kWeightThreads = kStepThreads - kRowThreads;  // weight waves: threads [512, 1024)
constexpr int kWBlocks = 6;                              // Q8_0 blocks per weight-wave thread and unit
constexpr int kDenseBatch = 16;                          // 16-byte loads in flight per dense weight-wave thread
constexpr int kQ4Blocks = 2;                             // Q4K super-blocks per weight-wave thread and unit
constexpr int kQ4Terms = 9;   // f32 terms per Q4K super-block and row: 8 lane sums and the min term
constexpr int kQ4TermStride = 12;  // LDS floats per (row, super-block): the 9 terms in three 16-byte words
constexpr int kBatchMfma = 16;   // lockstep batches from this size run their Q8_0 linears as MFMA GEMMs
constexpr int kTileRows = 32;    // output rows (16 gate/value pairs) of a GEMM unit (or 16)
constexpr int kTileBatch = 64;   // batch rows of a GEMM unit
constexpr int kMaxBatch = 1024;
constexpr int kMaxRingSlots = 12000;  // KV ring slots per stream and layer (attention keeps a head's scores in LDS)
constexpr size_t kStaticLdsReserve = 8192;  // static LDS of the step kernels (barrier state, positions)
constexpr int kGemmChunk = 4;    // Q8_0 blocks (128 bytes of K) per LDS stage of a GEMM unit
constexpr int kGemmStages = 8;   // LDS stages of a GEMM unit
// A GEMM stage: weights [kTileRows][128] | activations [kTileBatch][128] | weight scales
// [kTileRows][4] f16 (two 4-byte direct loads per row) | activation scales [kTileBatch][4] f32.  The
// operand rows come in groups of 8 (one wave's 1 KB direct load), each group kGemmGroupBytes
// apart: the 128 bytes between groups put rows j and j + 8 of an MFMA operand in different banks.
constexpr int kGemmGroupBytes = 1152;
constexpr int kGemmStageBytes = kTileRows / 8 * kGemmGroupBytes + kTileBatch / 8 * kGemmGroupBytes + kTileRows * kGemmChunk * 2 +
                                kTileBatch * kGemmChunk * 4;
static_assert(kGemmStageBytes % 16 == 0 && (kTileRows / 8 * kGemmGroupBytes + kTileBatch / 8 * kGemmGroupBytes + kTileRows * kGemmChunk * 2) % 16 == 0,
              "16-byte aligned stages and activation scales");
constexpr int kSyncChunks = 2;   // stages consumed between two row-wave barriers
// s_waitcnt immediates (vmcnt only) of the GEMM: at a barrier the chunks of the interval being
// consumed and of the next one (read ahead) have landed, the kGemmStages - 3 kSyncChunks chunks after
// them may still be in flight (1, 2 or 3 loads per wave and chunk), or none
constexpr int vm_wait_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
constexpr int kVmWait2 = vm_wait_imm(2 * (kGemmStages - 3 * kSyncChunks));
constexpr int kVmWait3 = vm_wait_imm(3 * (kGemmStages - 3 * kSyncChunks));
constexpr int kVmWait1 = vm_wait_imm(1 * (kGemmStages - 3 * kSyncChunks));
constexpr int kVmWait0 = vm_wait_imm(0);
constexpr int kAttnChunkBytes = 16384;  // K or V rows per LDS stage of an attention unit
constexpr int kAttnStages = 6;
constexpr int kMaxSplit = 16;  // units per head of a split attention launch
constexpr int kSplitKeys = 32;  // visible keys per split unit (the split starts at 2 kSplitKeys keys)
// A split attention unit's LDS:
//   * the V columns of its hd / S dims as rows of keys (f32 words, bf16 widened; split_row_words
//     words a row: 16 keys of slack for the chains' read-ahead, and a row stride of 16 bytes past
//     a multiple of 256, so that the lanes' 16-byte reads of their rows fall in different banks);
//   * the staging of those columns as they arrive ([key][hd / S] in pieces of split_piece_bytes,
//     rounds of 256 pieces by four waves);
//   * the weights [cap + kSplitSlack] and 32 words of slots.
constexpr int kSplitSlack = 48;
__host__ __device__ constexpr int split_row_words(int cap) { return (cap + 16 + 63) / 64 * 64 + 4; }
__host__ __device__ constexpr int split_piece_bytes(int hd, int kv_bf16, int S) {
  return (hd / S) * (kv_bf16 ? 2 : 4) % 16 == 0 ? 16 : 4;
}
__host__ __device__ constexpr size_t split_rows_bytes(int cap, int hd, int S) {
  return (size_t)(hd / S) * split_row_words(cap) * 4;
}
__host__ __device__ constexpr size_t split_stage_bytes(int cap, int hd, int kv_bf16, int S) {
  return ((size_t)cap * ((hd / S) * (kv_bf16 ? 2 : 4) / split_piece_bytes(hd, kv_bf16, S)) + 255) / 256 * 256 *
         split_piece_bytes(hd, kv_bf16, S);
}
__host__ __device__ constexpr size_t split_smem(int cap, int hd, int kv_bf16, int S) {
  return split_rows_bytes(cap, hd, S) + split_stage_bytes(cap, hd, kv_bf16, S) + (size_t)(cap + kSplitSlack + 32) * 4 + 64;
}
constexpr int kAttnVmWait = vm_wait_imm(2 * (kAttnStages - 2 * kSyncChunks));  // two direct loads per wave and chunk

// Unit families of a step program.  The persistent kernel is compiled for a few family sets, so
// that a program is run by a kernel holding only the registers of the units it has.
enum UnitFamily : unsigned {
  FAM_Q8 = 1,     // Q8_0 and Q4_0 GEMV (row waves + weight waves)
  FAM_Q4K = 2,    // Q4K GEMV (row waves + weight waves)
  FAM_DENSE = 4,  // f32 / bf16 GEMV
  FAM_BATCH = 8,  // batched Q8_0: activation quantization + MFMA GEMM
  FAM_ALL = 15,
};
unsigned program_families(const Phase* phases, int n);
hipError_t launch_step_program(const StepParams& p, unsigned families, int grid, size_t smem, hipStream_t s);
hipError_t launch_phase(const Phase& ph, const StepParams& p, int step, size_t smem, hipStream_t s);
// An attention phase with each (stream, head) split over S units (S = 2, 4, 8 or 16; S divides
// the head dim): `scores` [B * H][cap] tagged entries (tag << 32 | f32 bits), ph.at.split_tag as
// in AttnArgs.  Per-phase launches only (the units of a head exchange scores within the launch).
hipError_t launch_attn_split(const Phase& ph, const StepParams& p, int step, int S, uint64_t* scores, hipStream_t s);
int step_program_grid(int device);
size_t phase_smem(const Phase& ph);
// Fills the unit layout of a GEMV phase (ipw, parts, maxb, units) for `grid` workgroups.
void plan_gemv(GemvArgs& g, int grid, int* units);
// Unit layout of a batched Q8_0 GEMM phase (units = row tiles x batch tiles; parts = row tiles):
// 32-row tiles, or 16-row tiles when they put no more units on the busiest of `grid` workgroups.
void plan_qgemm(GemvArgs& g, int grid, int* units);

hipError_t launch_q8_quantize(const float* w, int rows, int K, int8_t* qs, uint16_t* d, hipStream_t s);
hipError_t launch_q8_from_blocks(const uint8_t* blocks, int rows, int K, int8_t* qs, uint16_t* d, hipStream_t s);
hipError_t launch_q8_to_blocks(const int8_t* qs, const uint16_t* d, int rows, int K, uint8_t* blocks, hipStream_t s);
hipError_t launch_q4_0_quantize(const float* w, int rows, int K, uint8_t* qs, uint16_t* d, hipStream_t s);
hipError_t launch_q4_0_from_blocks(const uint8_t* blocks, int rows, int K, uint8_t* qs, uint16_t* d, hipStream_t s);
hipError_t launch_q4_0_to_blocks(const uint8_t* qs, const uint16_t* d, int rows, int K, uint8_t* blocks, hipStream_t s);
hipError_t launch_q4k_quantize(const float* w, int rows, int K, uint8_t* blocks, hipStream_t s);
hipError_t launch_q4k_from_blocks(const uint8_t* candle, int rows, int K, uint8_t* blocks, hipStream_t s);
hipError_t launch_q4k_to_blocks(const uint8_t* blocks, int rows, int K, uint8_t* candle, hipStream_t s);
// Row-major [rows][K] f32 or bf16 (src_bf16) -> chain-packed FMT_F32C (dst_bf16 = 0) or FMT_BF16C.
hipError_t launch_chain_pack(const void* src, int src_bf16, int rows, int K, void* dst, int dst_bf16, hipStream_t s);
hipError_t launch_dequant(const LinearDev& L, float* out, hipStream_t s);
hipError_t launch_f16_to_f32(const uint16_t* x, float* y, size_t n, hipStream_t s);
hipError_t launch_bf16_to_f32(const uint16_t* x, float* y, size_t n, hipStream_t s);
hipError_t launch_kv_to_f32(const void* src, int kv_bf16, float* dst, size_t n, hipStream_t s);
hipError_t launch_f32_to_kv(const float* src, void* dst, int kv_bf16, size_t n, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s);
// y = exp / SiLU / GELU-tanh / erf GELU (kind 0 .. 3) of x, as the step kernels evaluate them.
hipError_t launch_activation(int kind, const float* x, size_t n, float* y, hipStream_t s);
hipError_t launch_fill_i32(int* p, int v, size_t n, hipStream_t s);
hipError_t launch_copy(const void* src, void* dst, size_t bytes, hipStream_t s);
// out[0 .. blocks * threads): one word per thread of a bare streaming read of src[0, bytes)
hipError_t launch_read(const void* src, size_t bytes, int blocks, int threads, uint32_t* out, hipStream_t s);
hipError_t launch_row_stats(const float* x, int rows, int K, int norm, float* out, hipStream_t s);

}  // namespace svl
