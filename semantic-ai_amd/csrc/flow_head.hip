// Kernels of the TTS flow head and end-of-speech head (SVL/tts/flow_lm.rs:181, 206-387).
//
// Numerics follow the reference's CPU path operation for operation (bit-identical to the
// oracle's restatement in oracle/flow.c):
//   * each Linear is the reference's matvec: the 16-lane FMA dot, the pairwise lane sum, the
//     scalar tail, then `+ bias` (SVL/nn/kernels/mod.rs:66-91, matvec.rs:174-202);
//   * SiLU is the reference's own (SVL/nn/kernels/activation.rs:70-74);
//   * ResBlock's in_ln is candle-nn's layer_norm: sum and sum of squares in one index-order pass,
//     mean = sum / n, var = sum2 / n - mean^2, (x - mean) * (1 / sqrt(var + eps)) * w + b;
//   * layer_norm_no_affine and the timestep embedder's norm are candle tensor ops: index-order
//     sums, `* (f32)(1 / n) + 0` for the means and for `/ (n - 1)`, `v * 1 + eps`, sqrt, recip or
//     division;
//   * modulate is `x * (scale * 1 + 1) + shift`, the flow update `x + (flow * (1 / steps) + 0)`.
// All code is compiled with -ffp-contract=off: products are fused only where fmaf() is written.
#include "flow_head.h"
#include "device_math.h"

namespace svl {
namespace {

constexpr int kFhThreads = 256;
constexpr int kFhRowsPerGroup = kFhThreads / 16;  // one output row per 16-lane group

// x[0] + x[1] + ... + x[n-1] with one f32 accumulator, reading LDS four values at a time.
__device__ __forceinline__ float seq_sum(const float* x, int n) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  float acc = 0.0f;
  int i = 0;
  for (; i + 4 <= n; i += 4) {
    const v4 v = *(const v4*)(x + i);
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  }
  for (; i < n; ++i) acc = acc + x[i];
  return acc;
}

// candle-nn layer_norm's statistics: one pass, `sum += v; sum2 += v * v` in index order.
__device__ __forceinline__ void seq_sum_and_squares(const float* x, int n, float& s, float& s2) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  float a = 0.0f, q = 0.0f;
  int i = 0;
  for (; i + 4 <= n; i += 4) {
    const v4 v = *(const v4*)(x + i);
    float p;
    a = a + v.x; p = v.x * v.x; q = q + p;
    a = a + v.y; p = v.y * v.y; q = q + p;
    a = a + v.z; p = v.z * v.z; q = q + p;
    a = a + v.w; p = v.w * v.w; q = q + p;
  }
  for (; i < n; ++i) {
    const float v = x[i];
    a = a + v;
    const float p = v * v;
    q = q + p;
  }
  s = a;
  s2 = q;
}

// modulate (flow_lm.rs:227-230)
__device__ __forceinline__ float modulate(float x, float shift, float scale) {
  const float s1a = scale * 1.0f;
  const float s1 = s1a + 1.0f;
  const float v = x * s1;
  return v + shift;
}

// The input row of stream b in LDS (xin[0, K)).  Every thread of the workgroup returns after
// the row is complete.
template <int PRO>
__device__ __forceinline__ void build_input(const FhArgs& a, int b, float* xin, float* sq, float* red) {
  const int K = a.L.in, t = threadIdx.x;
  const float* x = a.x + (size_t)b * a.x_stride;
  if (PRO == FH_PLAIN) {
    for (int k = t; k < K; k += kFhThreads) xin[k] = x[k];
    __syncthreads();
    return;
  }
  if (PRO == FH_SILU_Y) {
    for (int k = t; k < K; k += kFhThreads) {
      float v = x[k];
      if (a.x2) v = v + a.x2[k];
      xin[k] = ref_silu(v);
    }
    __syncthreads();
    return;
  }
  for (int k = t; k < K; k += kFhThreads) xin[k] = x[k];
  __syncthreads();
  const float* shift = a.shift + (size_t)b * a.mod_stride;
  const float* scale = a.scale + (size_t)b * a.mod_stride;
  if (PRO == FH_LN_MOD) {
    if (t == 0) seq_sum_and_squares(xin, K, red[0], red[1]);
    __syncthreads();
    const float mean = red[0] / (float)K;
    const float mm = mean * mean;
    const float var = red[1] / (float)K - mm;
    const float inv_std = 1.0f / sqrtf(var + a.eps);
    for (int k = t; k < K; k += kFhThreads) {
      float v = xin[k] - mean;
      v = v * inv_std;
      v = v * a.lnw[k];
      v = v + a.lnb[k];
      xin[k] = modulate(v, shift[k], scale[k]);
    }
  } else {  // FH_LN0_MOD
    if (t == 0) {
      const float s = seq_sum(xin, K);
      const float mp = s * a.inv_k;
      red[0] = mp + 0.0f;
    }
    __syncthreads();
    const float mean = red[0];
    for (int k = t; k < K; k += kFhThreads) {
      const float c = xin[k] - mean;
      sq[k] = c * c;
    }
    __syncthreads();
    if (t == 0) {
      const float s2 = seq_sum(sq, K);
      const float vp = s2 * a.inv_k;
      const float var = vp + 0.0f;
      const float ve = var * 1.0f;
      red[1] = sqrtf(ve + a.eps);
    }
    __syncthreads();
    const float sd = red[1];
    for (int k = t; k < K; k += kFhThreads) {
      const float c = xin[k] - mean;
      xin[k] = modulate(c / sd, shift[k], scale[k]);
    }
  }
  __syncthreads();
}

// Grid: (ceil(out / 16), B) workgroups of 256 threads; 16-lane group g of the workgroup computes
// row blockIdx.x * 16 + g of stream blockIdx.y.
template <int PRO, int EPI>
__global__ __launch_bounds__(kFhThreads) void fh_gemv_kernel(FhArgs a) {
  __shared__ __attribute__((aligned(16))) float xin[kFhMaxWidth];
  __shared__ __attribute__((aligned(16))) float sq[PRO == FH_LN0_MOD ? kFhMaxWidth : 4];
  __shared__ float red[2];
  const int b = blockIdx.y;
  build_input<PRO>(a, b, xin, sq, red);
  const int l = threadIdx.x & 15;
  const int row = blockIdx.x * kFhRowsPerGroup + (threadIdx.x >> 4);
  if (row >= a.L.out) return;  // a whole 16-lane group; no barrier follows
  const int K = a.L.in;
  float acc = 0.0f, tail = 0.0f;
  if (a.L.packed) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    const v4* w4 = (const v4*)a.L.w + (size_t)row * (K / 64) * 16 + l;
    const int kn = K / 64;
    int k = 0;
    for (; k + 4 <= kn; k += 4) {
      v4 w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = w4[(size_t)(k + u) * 16];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float* xs = xin + 64 * (k + u) + l;
        acc = fmaf(xs[0], w[u].x, acc);
        acc = fmaf(xs[16], w[u].y, acc);
        acc = fmaf(xs[32], w[u].z, acc);
        acc = fmaf(xs[48], w[u].w, acc);
      }
    }
    for (; k < kn; ++k) {
      const v4 w = w4[(size_t)k * 16];
      const float* xs = xin + 64 * k + l;
      acc = fmaf(xs[0], w.x, acc);
      acc = fmaf(xs[16], w.y, acc);
      acc = fmaf(xs[32], w.z, acc);
      acc = fmaf(xs[48], w.w, acc);
    }
  } else {
    const float* w = a.L.w + (size_t)row * K;
    const int chunks = K / 16;
    for (int c = 0; c < chunks; ++c) acc = fmaf(xin[16 * c + l], w[16 * c + l], acc);
    if (l == 0)
      for (int i = chunks * 16; i < K; ++i) {
        const float p = xin[i] * w[i];
        tail = tail + p;
      }
  }
  const float s = row16_pairwise_sum(acc);
  if (l != 0) return;
  float y = s + tail;
  y = y + a.L.b[row];
  float* out = a.y + (size_t)b * a.y_stride + row;
  if (EPI == FH_BIAS) {
    *out = y;
  } else if (EPI == FH_BIAS_SILU) {
    *out = ref_silu(y);
  } else if (EPI == FH_GATE_RES) {
    const float v = a.gate[(size_t)b * a.mod_stride + row] * y;
    *out = *out + v;
  } else if (EPI == FH_FLOW) {
    const float p = y * a.inv_steps;
    const float v = p + 0.0f;
    *out = *out + v;
  } else {  // FH_POINTWISE
    *out = a.noise[(size_t)b * a.noise_stride + row] + y;
  }
}

// One workgroup; thread 0 runs the index-order sums.
__global__ __launch_bounds__(kFhThreads) void fh_time_norm_kernel(const float* e, const float* alpha0,
                                                                  const float* alpha1, int n, int dim, float inv_dim,
                                                                  float inv_dim_m1, float inv_n, float* out) {
  __shared__ __attribute__((aligned(16))) float v[kFhMaxWidth];
  __shared__ __attribute__((aligned(16))) float sq[kFhMaxWidth];
  __shared__ float red[2];
  const int t = threadIdx.x;
  for (int i = 0; i < n; ++i) {
    const float* ei = e + (size_t)i * dim;
    for (int k = t; k < dim; k += kFhThreads) v[k] = ei[k];
    __syncthreads();
    if (t == 0) {
      const float mp = seq_sum(v, dim) * inv_dim;
      red[0] = mp + 0.0f;
    }
    __syncthreads();
    const float mean = red[0];
    for (int k = t; k < dim; k += kFhThreads) {
      const float c = v[k] - mean;
      sq[k] = c * c;
    }
    __syncthreads();
    if (t == 0) {
      const float vp = seq_sum(sq, dim) * inv_dim_m1;
      const float var = vp + 0.0f;
      const float ve = var * 1.0f;
      red[1] = 1.0f / sqrtf(ve + 1e-5f);
    }
    __syncthreads();
    const float r = red[1];
    const float* al = i == 0 ? alpha0 : alpha1;
    for (int k = t; k < dim; k += kFhThreads) {
      const float p = v[k] * r;
      const float q = p * al[k];
      out[k] = i == 0 ? q : out[k] + q;
    }
    __syncthreads();
  }
  for (int k = t; k < dim; k += kFhThreads) {
    const float p = out[k] * inv_n;
    out[k] = p + 0.0f;
  }
}

template <int PRO>
hipError_t launch_pro(const FhArgs& a, int epi, dim3 grid, hipStream_t s) {
  switch (epi) {
    case FH_BIAS: hipLaunchKernelGGL((fh_gemv_kernel<PRO, FH_BIAS>), grid, dim3(kFhThreads), 0, s, a); break;
    case FH_BIAS_SILU: hipLaunchKernelGGL((fh_gemv_kernel<PRO, FH_BIAS_SILU>), grid, dim3(kFhThreads), 0, s, a); break;
    case FH_GATE_RES: hipLaunchKernelGGL((fh_gemv_kernel<PRO, FH_GATE_RES>), grid, dim3(kFhThreads), 0, s, a); break;
    case FH_FLOW: hipLaunchKernelGGL((fh_gemv_kernel<PRO, FH_FLOW>), grid, dim3(kFhThreads), 0, s, a); break;
    case FH_POINTWISE: hipLaunchKernelGGL((fh_gemv_kernel<PRO, FH_POINTWISE>), grid, dim3(kFhThreads), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fh_gemv(const FhArgs& a, int pro, int epi, hipStream_t s) {
  if (a.L.in <= 0 || a.L.in > kFhMaxWidth || a.L.out <= 0 || a.B <= 0) return hipErrorInvalidValue;
  if (a.L.packed && a.L.in % 64) return hipErrorInvalidValue;
  const dim3 grid((a.L.out + kFhRowsPerGroup - 1) / kFhRowsPerGroup, a.B);
  switch (pro) {
    case FH_PLAIN: return launch_pro<FH_PLAIN>(a, epi, grid, s);
    case FH_SILU_Y: return launch_pro<FH_SILU_Y>(a, epi, grid, s);
    case FH_LN_MOD: return launch_pro<FH_LN_MOD>(a, epi, grid, s);
    case FH_LN0_MOD: return launch_pro<FH_LN0_MOD>(a, epi, grid, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fh_time_norm(const float* e, const float* const* alpha, int n, int dim, float inv_dim,
                               float inv_dim_m1, float inv_n, float* out, hipStream_t s) {
  if (n < 1 || n > 2 || dim <= 0 || dim > kFhMaxWidth) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fh_time_norm_kernel, dim3(1), dim3(kFhThreads), 0, s, e, alpha[0], n > 1 ? alpha[1] : alpha[0], n,
                     dim, inv_dim, inv_dim_m1, inv_n, out);
  return hipGetLastError();
}

}  // namespace svl
