// Launch interface of the step kernels (host side).  Internal to libsvl.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svl {

enum WeightFmt { FMT_F32 = 0, FMT_BF16 = 1, FMT_Q8_0 = 3, FMT_Q4K = 4 };
enum NormKind { NORM_NONE = 0, NORM_LAYER = 1, NORM_RMS = 2 };
enum Epilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU_GATE = 2, EPI_QKV_ROPE = 3, EPI_GELU = 4 };

// One linear layer as held on the device.
//   FMT_F32 / FMT_BF16: w = [out][in] row-major.
//   FMT_Q8_0: w = int8 quants [out][in]; scale = f16 block scales [out][in/32].
//   FMT_Q4K: w = 144-byte candle blocks [out][in/256] (kept as given).
struct LinearDev {
  int fmt = FMT_F32;
  int out = 0, in = 0;
  void* w = nullptr;
  uint16_t* scale = nullptr;
};

struct GemvArgs {
  LinearDev L;
  int B;               // batch rows (grid.y)
  int ipw;             // work items per workgroup (set by launch_gemv)
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
  const float* rope;   // [positions][hd/2][cos, sin] computed on the host
  int H, KVH, hd;
  float* q_out;        // [B][H*hd]
  void* kc;            // [B][KVH][cap][hd]
  void* vc;
  int cap;
  int kv_bf16;
  int advance_pos;
};

struct AttnArgs {
  const float* q;      // [B][H*hd]
  const void* kc;
  const void* vc;
  const int* pos;
  int B, H, KVH, hd, cap, window;  // window 0 = unlimited
  int kv_bf16;
  float scale;
  float* scores;       // [B][H][cap] scratch: scaled q.k of the visible keys
  float* out;          // [B][H*hd]
};

struct EmbedArgs {
  const void* text_emb;     // [text_card+1][d]
  const void* emb;          // n_q tables back to back, [n_q][card+1][d]
  int tables_bf16;
  int d, n_q, card, text_card, B;
  const uint32_t* text_tok; // [B] or null: use fb_tok
  const uint32_t* fb_tok;   // [B] feedback tokens (previous argmax)
  const uint32_t* audio;    // [B][n_q]
  int initial_at_zero;      // a stream at position 0 sees `card` audio tokens
  const int* pos;
  float* x;                 // [B][d]
};

hipError_t launch_gemv(const GemvArgs& a, hipStream_t s);
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);
hipError_t launch_embed(const EmbedArgs& a, hipStream_t s);
hipError_t launch_norm(const float* x, int x_stride, float* y, int y_stride, int B, int d, int norm,
                       const float* w, const float* b, float eps, hipStream_t s);
// argmax over logits [B][V]; writes fb_tok[b] and, when out is not null, out[b]; advances pos.
hipError_t launch_argmax(const float* logits, int B, int V, uint32_t* fb_tok, uint32_t* out, int* pos,
                         hipStream_t s);
hipError_t launch_q8_quantize(const float* w, int rows, int K, int8_t* qs, uint16_t* d, hipStream_t s);
hipError_t launch_q8_from_blocks(const uint8_t* blocks, int rows, int K, int8_t* qs, uint16_t* d, hipStream_t s);
hipError_t launch_q8_to_blocks(const int8_t* qs, const uint16_t* d, int rows, int K, uint8_t* blocks, hipStream_t s);
hipError_t launch_dequant(const LinearDev& L, float* out, hipStream_t s);
hipError_t launch_f16_to_f32(const uint16_t* x, float* y, size_t n, hipStream_t s);
hipError_t launch_bf16_to_f32(const uint16_t* x, float* y, size_t n, hipStream_t s);
hipError_t launch_kv_to_f32(const void* src, int kv_bf16, float* dst, size_t n, hipStream_t s);
hipError_t launch_f32_to_kv(const float* src, void* dst, int kv_bf16, size_t n, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s);
hipError_t launch_fill_i32(int* p, int v, size_t n, hipStream_t s);

}  // namespace svl
