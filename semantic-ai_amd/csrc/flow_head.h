// Launch interface of the TTS flow-head kernels (flow_head.hip).  Internal to libsvl.
//
// The flow head (SimpleMLPAdaLN, SVL/tts/flow_lm.rs:206-387) and the end-of-speech head
// (:181) are small dense f32 linears (width 512 for Pocket TTS) applied to one row per stream,
// each with a bias and a fused elementwise prologue or epilogue.  One launch per linear: every
// workgroup builds the (normalized, modulated) input row in LDS, then each 16-lane group of a
// wave computes one output row with the reference's 16-lane dot (SVL/nn/kernels/mod.rs:66-91).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svl {

// A dense f32 linear with bias.  packed: chain-packed rows (FMT_F32C layout, in % 64 == 0):
// the 16-byte vector ((row * in / 64 + k) * 16 + l) holds elements 64 k + 16 j + l, j = 0..3,
// of lane chain l; otherwise row-major [out][in].
struct FhLinear {
  const float* w = nullptr;
  const float* b = nullptr;
  int out = 0, in = 0;
  int packed = 0;
};

enum FhPro {
  FH_PLAIN = 0,    // x
  FH_SILU_Y = 1,   // silu(x + x2), x2 optional (the condition plus the time conditioning)
  FH_LN_MOD = 2,   // modulate(layer_norm(x, lnw, lnb, eps), shift, scale)  (candle-nn layer_norm)
  FH_LN0_MOD = 3,  // modulate(layer_norm_no_affine(x, eps), shift, scale)   (tensor ops)
};

enum FhEpi {
  FH_BIAS = 0,       // y = dot + b
  FH_BIAS_SILU = 1,  // y = silu(dot + b)
  FH_GATE_RES = 2,   // y = y + gate * (dot + b)
  FH_FLOW = 3,       // y = y + ((dot + b) * inv_steps + 0)
  FH_POINTWISE = 4,  // y = noise + (dot + b)
};

struct FhArgs {
  FhLinear L;
  int B;
  const float* x;      // input rows [B][x_stride]
  int x_stride;
  const float* x2;     // FH_SILU_Y: added to every row, or null
  const float* lnw;    // FH_LN_MOD
  const float* lnb;
  const float* shift;  // FH_LN_MOD / FH_LN0_MOD: rows [B][mod_stride]
  const float* scale;
  const float* gate;   // FH_GATE_RES
  int mod_stride;
  float eps;
  float inv_k;         // (f32)(1 / in): the mean's factor of layer_norm_no_affine
  float* y;            // output rows [B][y_stride]
  int y_stride;
  float inv_steps;     // FH_FLOW
  const float* noise;  // FH_POINTWISE: [B][noise_stride]
  int noise_stride;
};

constexpr int kFhMaxWidth = 4096;  // widest input row of a flow-head linear

hipError_t launch_fh_gemv(const FhArgs& a, int pro, int epi, hipStream_t s);

// The time conditioning of one flow step (SVL/tts/flow_lm.rs:256-266, 333-348): e [n][dim] the
// embedders' linear2 outputs, alpha[i] their norm scales -> out [dim] =
// (sum_i e_i * recip(sqrt(var_i + 1e-5)) * alpha_i) * inv_n, var_i the unbiased variance.
hipError_t launch_fh_time_norm(const float* e, const float* const* alpha, int n, int dim, float inv_dim,
                               float inv_dim_m1, float inv_n, float* out, hipStream_t s);

}  // namespace svl
