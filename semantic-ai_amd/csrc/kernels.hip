// Step kernels for gfx950 (MI355X): batch-row GEMV with fused prologue (norm + Q8_0 activation
// quantization) and fused epilogues (residual, SiLU gate, GELU, RoPE + KV ring write),
// single-query split-K attention over the KV ring, embedding gather-sum, argmax, and the
// weight-format kernels used at model creation.
//
// Numerics follow the reference's CPU path (crates/semantic-voice-local/src, "SVL"):
//   * Q8_0 matmul as candle's quantized CPU matmul: the activation row is quantized to Q8_0
//     blocks (d = amax/127 stored as f16, q = round(x / d) via x * (1/d)); every weight block
//     contributes (exact i32 dot as f32 * d_w) * d_x; blocks are summed in f32.
//   * SiLU / GELU-tanh / exp exactly as SVL/nn/kernels/{activation,mod}.rs.
//   * RMSNorm / LayerNorm as candle-nn's CPU ops (x / m * alpha; (x - mean) * inv_std * w + b).
//   * interleaved RoPE (candle-nn rope_i), attention visibility of SVL/nn/transformer.rs:385.
// Only the order of f32 summations differs from the CPU path.
#include "kernels.h"
#include "device_math.h"

namespace svl {

constexpr int kThreads = 256;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// Row statistics in the order shared with the oracle: 64 strided partials (lane l sums
// x[l], x[l+64], ... sequentially), then a butterfly over the partials (offsets 32 .. 1).
// Every lane of every wave computes the same value, so no cross-wave exchange is needed.

__device__ __forceinline__ float blocked_sum(const float* xs, int K, bool squares) {
  const int lane = threadIdx.x % kWave;
  float acc = 0.0f;
  for (int i = lane; i < K; i += kWave) {
    float v = xs[i];
    if (squares) v = v * v;
    acc = acc + v;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o, kWave);
  return acc;
}

// Normalizes xs[0..K) in LDS in place: candle-nn rms_norm (x / m * alpha,
// m = sqrt(sum(x^2) / K + eps)) or layer_norm ((x - mean) * (1 / sqrt(var + eps)) * w + b,
// var = sum(x^2) / K - mean^2).  Callers synchronize before and after.
__device__ void norm_lds(float* xs, int K, int norm, const float* nw, const float* nb, float eps) {
  if (norm == NORM_RMS) {
    const float s2 = blocked_sum(xs, K, true);
    const float m = sqrtf(s2 / (float)K + eps);
    __syncthreads();
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
      float t = xs[i] / m;
      xs[i] = t * nw[i];
    }
  } else {
    const float s = blocked_sum(xs, K, false);
    const float s2 = blocked_sum(xs, K, true);
    const float mean = s / (float)K;
    const float mm = mean * mean;
    const float var = s2 / (float)K - mm;
    const float inv_std = 1.0f / sqrtf(var + eps);
    __syncthreads();
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
      float t = (xs[i] - mean) * inv_std;
      t = t * nw[i];
      xs[i] = t + nb[i];
    }
  }
}

// Q8_0 activation quantization of xs[0..K) into xq (int8) and xdq (the f16-rounded block
// scales as f32): candle's BlockQ8_0::from_float.  A half-wave owns one block per iteration
// (lane = element); the shuffles stay inside the half.
__device__ void quantize_lds(const float* xs, int K, int8_t* xq, float* xdq) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int nwaves = blockDim.x / kWave;
  const int nb = K / 32;
  for (int blk = wave * 2 + lane / 32; blk < nb; blk += nwaves * 2) {
    float v = xs[blk * 32 + (lane % 32)];
    float amax = half_max(fabsf(v));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    xq[blk * 32 + (lane % 32)] = (int8_t)sat_i8(roundf(v * id));
    if ((lane % 32) == 0) xdq[blk] = f16_to_f32(f32_to_f16(d));
  }
}

// Loads one batch row of the input into LDS and applies the prologue norm.
__device__ void stage_input(const GemvArgs& a, int b, float* xs) {
  const int K = a.L.in;
  const float* x = a.x + (size_t)b * a.x_stride;
  for (int i = threadIdx.x; i < K; i += blockDim.x) xs[i] = x[i];
  __syncthreads();
  if (a.norm != NORM_NONE) {
    norm_lds(xs, K, a.norm, a.nw, a.nb, a.eps);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// Epilogues.  `item` is the workgroup-local work item; `y` its row value and `yp` the value of
// the RoPE partner row (row ^ 1), both from the workgroup's row results.

__device__ __forceinline__ void epilogue(const GemvArgs& a, int b, int row, float y, float yp, float yv) {
  switch (a.epi) {
    case EPI_STORE:
      a.y[(size_t)b * a.y_stride + row] = y;
      break;
    case EPI_GELU:
      a.y[(size_t)b * a.y_stride + row] = ref_gelu_tanh(y);
      break;
    case EPI_SILU_GATE: {
      // FeedForwardLayer::forward gated branch (SVL/nn/transformer.rs:453-461): silu(gate) * value
      float g = ref_silu(y);
      a.y[(size_t)b * a.y_stride + row] = g * yv;
      break;
    }
    case EPI_RESID: {
      float u = y;
      if (a.lscale) u = u * a.lscale[row];
      float* r = a.resid + (size_t)b * a.resid_stride + row;
      *r = *r + u;
      break;
    }
    case EPI_QKV_ROPE: {
      // split q | k | v (transformer.rs:330-338); interleaved RoPE on q and k (rope_i); k, v
      // into the ring slot of the current position.
      const int qdim = a.H * a.hd, kvdim = a.KVH * a.hd;
      const int p = a.pos[b];
      const int region = row < qdim ? 0 : (row < qdim + kvdim ? 1 : 2);
      const int rr = region == 0 ? row : (region == 1 ? row - qdim : row - qdim - kvdim);
      const int head = rr / a.hd, dim = rr % a.hd;
      float out = y;
      if (region < 2) {
        const float* cs = a.rope + ((size_t)p * (a.hd / 2) + dim / 2) * 2;
        const float c = cs[0], s = cs[1];
        if ((dim & 1) == 0) {
          float t0 = y * c, t1 = yp * s;
          out = t0 - t1;
        } else {
          float t0 = yp * s, t1 = y * c;
          out = t0 + t1;
        }
      }
      if (region == 0) {
        a.q_out[(size_t)b * qdim + rr] = out;
      } else {
        size_t idx = (((size_t)b * a.KVH + head) * a.cap + (size_t)(p % a.cap)) * a.hd + dim;
        void* base = region == 1 ? a.kc : a.vc;
        if (a.kv_bf16) ((uint16_t*)base)[idx] = f32_to_bf16(out);
        else ((float*)base)[idx] = out;
      }
      break;
    }
  }
}

// Physical row of workgroup-local row r: the SiLU gate takes `ni` gate rows then their `ni`
// value rows (j + ff_hidden).
__device__ __forceinline__ int phys_row(const GemvArgs& a, int i0, int ni, int r) {
  if (a.epi == EPI_SILU_GATE) return r < ni ? i0 + r : i0 + (r - ni) + a.ff_hidden;
  return i0 + r;
}

__device__ __forceinline__ void run_epilogues(const GemvArgs& a, int b, int i0, int ni, const float* Y) {
  const int t = threadIdx.x;
  if (t < ni) {
    const float y = Y[t];
    const float yp = a.epi == EPI_QKV_ROPE ? Y[t ^ 1] : 0.0f;
    const float yv = a.epi == EPI_SILU_GATE ? Y[ni + t] : 0.0f;
    epilogue(a, b, i0 + t, y, yp, yv);
  }
  if (a.advance_pos && blockIdx.x == 0 && t == 0) a.pos[b] += 1;
}

// ---------------------------------------------------------------------------------------------
// Q8_0 GEMV (candle's quantized CPU matmul, SVL/nn/mod.rs:97): every block term is
// (exact i32 dot as f32 * d_w) * d_x, and each row sums its terms in block order
// (BlockQ8_0::vec_dot_unopt).  A workgroup owns `ipw` work items; its weight blocks are loaded
// before the prologue (they do not depend on the input), one 32-byte block per thread and
// round, the terms go to LDS, and one thread per row adds them up in order.

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <int MAXB>
__global__ __launch_bounds__(kThreads) void gemv_q8_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.L.in, nb = K / 32;
  const int b = blockIdx.y;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int items = silu ? a.ff_hidden : a.L.out;
  const int i0 = blockIdx.x * a.ipw;
  const int ni = min(a.ipw, items - i0);
  const int NR = silu ? 2 * ni : ni;
  const int total = NR * nb;
  const int ts = nb + 1;  // padded term-row stride
  float* xs = (float*)smem;                   // K
  int8_t* xq = (int8_t*)(xs + K);             // K
  float* xdq = (float*)(xq + K);              // nb
  float* T = xdq + nb;                        // NR * (nb + 1)
  float* Y = T + 2 * a.ipw * ts;              // NR

  const int8_t* wq = (const int8_t*)a.L.w;
  v4i wa[MAXB], wb[MAXB];
  uint16_t wd[MAXB];
#pragma unroll
  for (int k = 0; k < MAXB; ++k) {
    const int idx = threadIdx.x + k * kThreads;
    if (idx < total) {
      const int r = idx / nb, blk = idx - r * nb;
      const size_t row = (size_t)phys_row(a, i0, ni, r);
      const v4i* p = (const v4i*)(wq + row * K + (size_t)blk * 32);
      wa[k] = __builtin_nontemporal_load(p);
      wb[k] = __builtin_nontemporal_load(p + 1);
      wd[k] = a.L.scale[row * nb + blk];
    }
  }
  stage_input(a, b, xs);
  quantize_lds(xs, K, xq, xdq);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < MAXB; ++k) {
    const int idx = threadIdx.x + k * kThreads;
    if (idx < total) {
      const int r = idx / nb, blk = idx - r * nb;
      const v4i xa = *(const v4i*)(xq + blk * 32);
      const v4i xb = *(const v4i*)(xq + blk * 32 + 16);
      int s = sdot4(wa[k].x, xa.x, 0);
      s = sdot4(wa[k].y, xa.y, s);
      s = sdot4(wa[k].z, xa.z, s);
      s = sdot4(wa[k].w, xa.w, s);
      s = sdot4(wb[k].x, xb.x, s);
      s = sdot4(wb[k].y, xb.y, s);
      s = sdot4(wb[k].z, xb.z, s);
      s = sdot4(wb[k].w, xb.w, s);
      float t = (float)s * f16_to_f32(wd[k]);
      T[r * ts + blk] = t * xdq[blk];
    }
  }
  __syncthreads();
  if (threadIdx.x < NR) {
    const float* tr = T + threadIdx.x * ts;
    float acc = 0.0f;
    for (int blk = 0; blk < nb; ++blk) acc = acc + tr[blk];
    Y[threadIdx.x] = acc;
  }
  __syncthreads();
  run_epilogues(a, b, i0, ni, Y);
}

// ---------------------------------------------------------------------------------------------
// Dense GEMV (f32 or bf16 weights): the reference's matvec (SVL/nn/kernels/matvec.rs:239-246)
// row by row with its 16-lane dot (kernels/mod.rs:66-91): 16 threads per row, thread i
// accumulating x[16c + i] * w[16c + i] with FMA over c, then the pairwise lane sum and the
// scalar tail.  A workgroup owns 16 rows (8 gate/value pairs for the SiLU gate).

template <bool BF16W>
__global__ __launch_bounds__(kThreads) void gemv_dense_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.L.in;
  const int b = blockIdx.y;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int items = silu ? a.ff_hidden : a.L.out;
  const int i0 = blockIdx.x * a.ipw;
  const int ni = min(a.ipw, items - i0);
  const int NR = silu ? 2 * ni : ni;
  float* xs = (float*)smem;   // K
  float* Y = xs + K;          // 16
  stage_input(a, b, xs);
  const int g = threadIdx.x / 16, li = threadIdx.x % 16;
  const int chunks = K / 16;
  if (g < NR) {
    const size_t row = (size_t)phys_row(a, i0, ni, g);
    float acc = 0.0f;
    if (BF16W) {
      const uint16_t* w = (const uint16_t*)a.L.w + row * K + li;
      int c = 0;
      for (; c + 8 <= chunks; c += 8) {
        uint16_t wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) wv[u] = __builtin_nontemporal_load(w + (size_t)(c + u) * 16);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(xs[(c + u) * 16 + li], bf16_to_f32(wv[u]), acc);
      }
      for (; c < chunks; ++c) acc = fmaf(xs[c * 16 + li], bf16_to_f32(w[(size_t)c * 16]), acc);
    } else {
      const float* w = (const float*)a.L.w + row * K + li;
      int c = 0;
      for (; c + 8 <= chunks; c += 8) {
        float wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) wv[u] = __builtin_nontemporal_load(w + (size_t)(c + u) * 16);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(xs[(c + u) * 16 + li], wv[u], acc);
      }
      for (; c < chunks; ++c) acc = fmaf(xs[c * 16 + li], w[(size_t)c * 16], acc);
    }
    // pairwise lane sum: acc[i] += acc[i + width] for width 8, 4, 2, 1
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o, 16);
    if (li == 0) {
      float tail = 0.0f;
      for (int i = chunks * 16; i < K; ++i) {
        float wv = BF16W ? bf16_to_f32(((const uint16_t*)a.L.w)[row * K + i]) : ((const float*)a.L.w)[row * K + i];
        float p = xs[i] * wv;
        tail = tail + p;
      }
      Y[g] = acc + tail;
    }
  }
  __syncthreads();
  run_epilogues(a, b, i0, ni, Y);
}

static int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

hipError_t launch_gemv(const GemvArgs& a0, hipStream_t s) {
  GemvArgs a = a0;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int items = silu ? a.ff_hidden : a.L.out;
  const int K = a.L.in;
  if (a.L.fmt == FMT_Q8_0) {
    const int nb = K / 32;
    // As many items per workgroup as keep 16 rows, 8 blocks per thread and 256 workgroups.
    int ipw = silu ? 8 : 16;
    while (ipw > 2 && ((silu ? 2 * ipw : ipw) * nb > 8 * kThreads || items / ipw < 256)) ipw /= 2;
    a.ipw = ipw;
    const int NR = silu ? 2 * ipw : ipw;
    const int maxb = pow2_at_least((NR * nb + kThreads - 1) / kThreads);
    const size_t smem = (size_t)K * 4 + K + (size_t)nb * 4 + (size_t)2 * ipw * (nb + 1) * 4 + (size_t)NR * 4 + 64;
    dim3 grid((items + ipw - 1) / ipw, a.B);
    switch (maxb) {
      case 1: hipLaunchKernelGGL((gemv_q8_kernel<1>), grid, dim3(kThreads), smem, s, a); break;
      case 2: hipLaunchKernelGGL((gemv_q8_kernel<2>), grid, dim3(kThreads), smem, s, a); break;
      case 4: hipLaunchKernelGGL((gemv_q8_kernel<4>), grid, dim3(kThreads), smem, s, a); break;
      case 8: hipLaunchKernelGGL((gemv_q8_kernel<8>), grid, dim3(kThreads), smem, s, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (a.L.fmt == FMT_F32 || a.L.fmt == FMT_BF16) {
    a.ipw = silu ? 8 : 16;
    const size_t smem = (size_t)K * 4 + 16 * 4 + 64;
    dim3 grid((items + a.ipw - 1) / a.ipw, a.B);
    if (a.L.fmt == FMT_BF16) hipLaunchKernelGGL((gemv_dense_kernel<true>), grid, dim3(kThreads), smem, s, a);
    else hipLaunchKernelGGL((gemv_dense_kernel<false>), grid, dim3(kThreads), smem, s, a);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------------
// Attention (SVL/nn/kernels/attention.rs:103-168): the query at position p attends to keys
// max(0, p - window + 1) ..= p (transformer.rs:385) in the ring.  Same order of operations as
// the reference's `attend`:
//   attn_scores:    w_j = scale * dot(q, k_j) with the 16-lane dot       (parallel over keys)
//   attn_softmax_v: max, e_j = exp(w_j - max), sum_j e_j in key order, then
//                   out = sum over keys in order of mul_add(e_j / sum, v_j, out)

template <bool BF16KV>
__device__ __forceinline__ float kv_at(const void* base, size_t idx) {
  if (BF16KV) return bf16_to_f32(((const uint16_t*)base)[idx]);
  return ((const float*)base)[idx];
}

constexpr int kKeysPerScoreBlock = 64;

template <int HD, bool BF16KV>
__global__ __launch_bounds__(kThreads) void attn_scores_kernel(AttnArgs a) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int p = a.pos[b];
  const int L = a.window > 0 ? min(p + 1, a.window) : p + 1;
  const int first = p + 1 - L;
  const int g = threadIdx.x / 16, li = threadIdx.x % 16;
  const int kvh = h / (a.H / a.KVH);
  constexpr int C = HD / 16;
  float q[C];
  const float* qp = a.q + (size_t)b * a.H * HD + (size_t)h * HD + li;
#pragma unroll
  for (int c = 0; c < C; ++c) q[c] = qp[c * 16];
  const size_t head_base = ((size_t)b * a.KVH + kvh) * (size_t)a.cap;
  for (int jj = blockIdx.x * kKeysPerScoreBlock + g; jj < min(L, (int)(blockIdx.x + 1) * kKeysPerScoreBlock); jj += 16) {
    const int j = first + jj;
    const size_t base = (head_base + (size_t)(j % a.cap)) * HD + li;
    float kv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) kv[c] = kv_at<BF16KV>(a.kc, base + c * 16);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) acc = fmaf(q[c], kv[c], acc);
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o, 16);
    if (li == 0) a.scores[((size_t)b * a.H + h) * a.cap + jj] = a.scale * (acc + 0.0f);
  }
}

template <int HD, bool BF16KV>
__global__ __launch_bounds__(kWave) void attn_softmax_v_kernel(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* w = (float*)smem;  // L weights
  __shared__ float s_sum;
  const int h = blockIdx.y, b = blockIdx.z;
  const int p = a.pos[b];
  const int L = a.window > 0 ? min(p + 1, a.window) : p + 1;
  const int first = p + 1 - L;
  const int lane = threadIdx.x;
  const float* sc = a.scores + ((size_t)b * a.H + h) * a.cap;
  float mx = -__builtin_huge_valf();
  for (int j = lane; j < L; j += kWave) {
    float v = sc[j];
    w[j] = v;
    mx = fmaxf(mx, v);
  }
  mx = wave_max(mx);
  for (int j = lane; j < L; j += kWave) w[j] = ref_exp(w[j] - mx);
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int j = 0; j < L; ++j) sum = sum + w[j];
    s_sum = sum;
  }
  __syncthreads();
  const float sum = s_sum;
  for (int j = lane; j < L; j += kWave) w[j] = w[j] / sum;
  __syncthreads();
  if (lane < 32) {
    const int d = blockIdx.x * 32 + lane;
    const int kvh = h / (a.H / a.KVH);
    const size_t head_base = ((size_t)b * a.KVH + kvh) * (size_t)a.cap;
    float acc = 0.0f;
    int j = 0;
    for (; j + 8 <= L; j += 8) {
      float vv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) vv[u] = kv_at<BF16KV>(a.vc, (head_base + (size_t)((first + j + u) % a.cap)) * HD + d);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = fmaf(w[j + u], vv[u], acc);
    }
    for (; j < L; ++j) acc = fmaf(w[j], kv_at<BF16KV>(a.vc, (head_base + (size_t)((first + j) % a.cap)) * HD + d), acc);
    a.out[(size_t)b * a.H * HD + (size_t)h * HD + d] = acc;
  }
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
  const int lmax = a.cap;
  dim3 gs((lmax + kKeysPerScoreBlock - 1) / kKeysPerScoreBlock, a.H, a.B);
  dim3 gv(a.hd / 32, a.H, a.B);
  const size_t smem = (size_t)lmax * 4 + 64;
  if (a.hd == 128) {
    if (a.kv_bf16) {
      hipLaunchKernelGGL((attn_scores_kernel<128, true>), gs, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((attn_softmax_v_kernel<128, true>), gv, dim3(kWave), smem, s, a);
    } else {
      hipLaunchKernelGGL((attn_scores_kernel<128, false>), gs, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((attn_softmax_v_kernel<128, false>), gv, dim3(kWave), smem, s, a);
    }
  } else if (a.hd == 64) {
    if (a.kv_bf16) {
      hipLaunchKernelGGL((attn_scores_kernel<64, true>), gs, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((attn_softmax_v_kernel<64, true>), gv, dim3(kWave), smem, s, a);
    } else {
      hipLaunchKernelGGL((attn_scores_kernel<64, false>), gs, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((attn_softmax_v_kernel<64, false>), gv, dim3(kWave), smem, s, a);
    }
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Embedding gather-sum (SVL/stt/model.rs:246-250): x = text_emb[t] + emb_0[a_0] + ... in that
// order, f32 adds.  Token ids past the table are clamped (the host validates its own inputs).

__global__ void embed_kernel(EmbedArgs a) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.d) return;
  uint32_t t = a.text_tok ? a.text_tok[b] : a.fb_tok[b];
  t = t > (uint32_t)a.text_card ? (uint32_t)a.text_card : t;
  const bool initial = a.initial_at_zero && a.pos[b] == 0;
  const size_t rows = (size_t)a.card + 1;
  float x;
  if (a.tables_bf16) x = bf16_to_f32(((const uint16_t*)a.text_emb)[(size_t)t * a.d + i]);
  else x = ((const float*)a.text_emb)[(size_t)t * a.d + i];
  const uint32_t* au = a.audio + (size_t)b * a.n_q;
  for (int c0 = 0; c0 < a.n_q; c0 += 8) {
    float e[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = c0 + u;
      e[u] = 0.0f;
      if (c < a.n_q) {
        uint32_t tok = initial ? (uint32_t)a.card : au[c];
        tok = tok > (uint32_t)a.card ? (uint32_t)a.card : tok;
        const size_t idx = ((size_t)c * rows + tok) * a.d + i;
        e[u] = a.tables_bf16 ? bf16_to_f32(((const uint16_t*)a.emb)[idx]) : ((const float*)a.emb)[idx];
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (c0 + u < a.n_q) x = x + e[u];
  }
  a.x[(size_t)b * a.d + i] = x;
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t s) {
  dim3 grid((a.d + 255) / 256, a.B);
  hipLaunchKernelGGL(embed_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void norm_kernel(const float* x, int x_stride, float* y, int y_stride,
                                                        int d, int norm, const float* w, const float* nb, float eps) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* xs = (float*)smem;
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < d; i += kThreads) xs[i] = x[(size_t)b * x_stride + i];
  __syncthreads();
  norm_lds(xs, d, norm, w, nb, eps);
  __syncthreads();
  for (int i = threadIdx.x; i < d; i += kThreads) y[(size_t)b * y_stride + i] = xs[i];
}

hipError_t launch_norm(const float* x, int x_stride, float* y, int y_stride, int B, int d, int norm,
                       const float* w, const float* b, float eps, hipStream_t s) {
  size_t smem = (size_t)d * 4 + 64;
  hipLaunchKernelGGL(norm_kernel, dim3(B), dim3(kThreads), smem, s, x, x_stride, y, y_stride, d, norm, w, b, eps);
  return hipGetLastError();
}

// Argmax over the last dim, first index on ties.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, int V, uint32_t* fb_tok, uint32_t* out,
                                                      int* pos) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int b = blockIdx.x;
  const float* lg = logits + (size_t)b * V;
  float best = -__builtin_huge_valf();
  int idx = 0x7fffffff;
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    float v = lg[i];
    if (idx == 0x7fffffff || v > best) {
      best = v;
      idx = i;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    float ov = __shfl_xor(best, o, kWave);
    int oi = __shfl_xor(idx, o, kWave);
    if (oi != 0x7fffffff && (idx == 0x7fffffff || ov > best || (ov == best && oi < idx))) {
      best = ov;
      idx = oi;
    }
  }
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int nw = blockDim.x / kWave;
    float bv = sv[0];
    int bi = si[0];
    for (int w = 1; w < nw; ++w) {
      if (si[w] != 0x7fffffff && (bi == 0x7fffffff || sv[w] > bv || (sv[w] == bv && si[w] < bi))) {
        bv = sv[w];
        bi = si[w];
      }
    }
    if (bi == 0x7fffffff) bi = 0;
    fb_tok[b] = (uint32_t)bi;
    if (out) out[b] = (uint32_t)bi;
    if (pos) pos[b] += 1;
  }
}

hipError_t launch_argmax(const float* logits, int B, int V, uint32_t* fb_tok, uint32_t* out, int* pos,
                         hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(B), dim3(1024), 0, s, logits, V, fb_tok, out, pos);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Weight formats.

// candle BlockQ8_0::from_float on the GPU: one thread per 32-value block.
__global__ void q8_quantize_kernel(const float* w, size_t nblocks, int8_t* qs, uint16_t* d) {
  size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  const float* x = w + blk * 32;
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
  float dd = amax / 127.0f;
  float id = dd != 0.0f ? 1.0f / dd : 0.0f;
  d[blk] = f32_to_f16(dd);
  for (int j = 0; j < 32; ++j) qs[blk * 32 + j] = (int8_t)sat_i8(roundf(x[j] * id));
}

hipError_t launch_q8_quantize(const float* w, int rows, int K, int8_t* qs, uint16_t* d, hipStream_t s) {
  size_t nb = (size_t)rows * (K / 32);
  hipLaunchKernelGGL(q8_quantize_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, w, nb, qs, d);
  return hipGetLastError();
}

// 34-byte candle blocks -> split quants and scales.
__global__ void q8_from_blocks_kernel(const uint8_t* blocks, size_t nblocks, int8_t* qs, uint16_t* d) {
  size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  const uint8_t* p = blocks + blk * 34;
  d[blk] = (uint16_t)(p[0] | (p[1] << 8));
  for (int j = 0; j < 32; ++j) qs[blk * 32 + j] = (int8_t)p[2 + j];
}

hipError_t launch_q8_from_blocks(const uint8_t* blocks, int rows, int K, int8_t* qs, uint16_t* d, hipStream_t s) {
  size_t nb = (size_t)rows * (K / 32);
  hipLaunchKernelGGL(q8_from_blocks_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, blocks, nb, qs, d);
  return hipGetLastError();
}

__global__ void q8_to_blocks_kernel(const int8_t* qs, const uint16_t* d, size_t nblocks, uint8_t* blocks) {
  size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  uint8_t* p = blocks + blk * 34;
  p[0] = (uint8_t)(d[blk] & 0xff);
  p[1] = (uint8_t)(d[blk] >> 8);
  for (int j = 0; j < 32; ++j) p[2 + j] = (uint8_t)qs[blk * 32 + j];
}

hipError_t launch_q8_to_blocks(const int8_t* qs, const uint16_t* d, int rows, int K, uint8_t* blocks, hipStream_t s) {
  size_t nb = (size_t)rows * (K / 32);
  hipLaunchKernelGGL(q8_to_blocks_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, qs, d, nb, blocks);
  return hipGetLastError();
}

// Dequantization: Q8_0 closed form q * f32(d); dense bf16 widening; f32 copy.
__global__ void dequant_kernel(LinearDev L, float* out) {
  size_t n = (size_t)L.out * L.in;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (L.fmt == FMT_Q8_0) out[i] = (float)((const int8_t*)L.w)[i] * f16_to_f32(L.scale[i / 32]);
  else if (L.fmt == FMT_BF16) out[i] = bf16_to_f32(((const uint16_t*)L.w)[i]);
  else out[i] = ((const float*)L.w)[i];
}

hipError_t launch_dequant(const LinearDev& L, float* out, hipStream_t s) {
  size_t n = (size_t)L.out * L.in;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, L, out);
  return hipGetLastError();
}

__global__ void f16_to_f32_kernel(const uint16_t* x, float* y, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = f16_to_f32(x[i]);
}
__global__ void bf16_to_f32_kernel(const uint16_t* x, float* y, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = bf16_to_f32(x[i]);
}
__global__ void f32_to_bf16_kernel(const float* x, uint16_t* y, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = f32_to_bf16(x[i]);
}
__global__ void copy_f32_kernel(const float* x, float* y, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = x[i];
}

hipError_t launch_f16_to_f32(const uint16_t* x, float* y, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}
hipError_t launch_bf16_to_f32(const uint16_t* x, float* y, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}
hipError_t launch_kv_to_f32(const void* src, int kv_bf16, float* dst, size_t n, hipStream_t s) {
  if (kv_bf16) return launch_bf16_to_f32((const uint16_t*)src, dst, n, s);
  hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const float*)src, dst, n);
  return hipGetLastError();
}
hipError_t launch_f32_to_kv(const float* src, void* dst, int kv_bf16, size_t n, hipStream_t s) {
  if (kv_bf16)
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, (uint16_t*)dst, n);
  else
    hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, (float*)dst, n);
  return hipGetLastError();
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
__global__ void fill_i32_kernel(int* p, int v, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}
hipError_t launch_fill_i32(int* p, int v, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}

}  // namespace svl
