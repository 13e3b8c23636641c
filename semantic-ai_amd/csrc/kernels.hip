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
constexpr int kWaves = kThreads / kWave;

// ---------------------------------------------------------------------------------------------
// GEMV prologue: x (one batch row) -> LDS, optional norm, optional Q8_0 quantization.

__device__ __forceinline__ void block_sum2(float& a, float& b, float* red) {
  a = wave_sum(a);
  b = wave_sum(b);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    red[wave] = a;
    red[kWaves + wave] = b;
  }
  __syncthreads();
  a = 0.0f;
  b = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    a += red[w];
    b += red[kWaves + w];
  }
  __syncthreads();
}

// Normalizes xs[0..K) in LDS in place (candle-nn rms_norm / layer_norm CPU formulas).
__device__ void norm_lds(float* xs, int K, int norm, const float* nw, const float* nb, float eps,
                         float* red) {
  float s = 0.0f, s2 = 0.0f;
  for (int i = threadIdx.x; i < K; i += kThreads) {
    float v = xs[i];
    s += v;
    float p = v * v;
    s2 += p;
  }
  block_sum2(s, s2, red);
  if (norm == NORM_RMS) {
    float m = sqrtf(s2 / (float)K + eps);
    for (int i = threadIdx.x; i < K; i += kThreads) {
      float t = xs[i] / m;
      xs[i] = t * nw[i];
    }
  } else {
    float mean = s / (float)K;
    float mm = mean * mean;
    float var = s2 / (float)K - mm;
    float inv_std = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < K; i += kThreads) {
      float t = (xs[i] - mean) * inv_std;
      t = t * nw[i];
      xs[i] = t + nb[i];
    }
  }
  __syncthreads();
}

// Q8_0 activation quantization of xs[0..K) into xq (int8) and xdq (the f16-rounded block
// scales as f32).  Each half-wave quantizes one 32-value block: lane = element.
__device__ void quantize_lds(const float* xs, int K, int8_t* xq, float* xdq) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int nb = K / 32;
  // A half-wave owns one block per iteration; shuffles stay inside the half.
  for (int blk = wave * 2 + lane / 32; blk < nb; blk += kWaves * 2) {
    float v = xs[blk * 32 + (lane % 32)];
    float amax = half_max(fabsf(v));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    xq[blk * 32 + (lane % 32)] = (int8_t)sat_i8(roundf(v * id));
    if ((lane % 32) == 0) xdq[blk] = f16_to_f32(f32_to_f16(d));
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------
// GEMV main loops.  Each wave computes R consecutive work items; a work item is one output
// row, or for the SiLU gate a (gate row j, value row j + F) pair.

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <int NR>
__device__ __forceinline__ void dot_rows_q8(const LinearDev& L, const int* rows, const int8_t* xq,
                                            const float* xdq, float* acc) {
  const int lane = threadIdx.x % kWave;
  const int K = L.in, nb = K / 32;
  const int8_t* wq = (const int8_t*)L.w;
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
  for (int b = lane; b < nb; b += kWave) {
    v4i wa[NR], wb[NR];
    uint16_t wd[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const v4i* p = (const v4i*)(wq + (size_t)rows[r] * K + (size_t)b * 32);
      wa[r] = __builtin_nontemporal_load(p);
      wb[r] = __builtin_nontemporal_load(p + 1);
      wd[r] = L.scale[(size_t)rows[r] * nb + b];
    }
    const v4i xa = *(const v4i*)(xq + b * 32);
    const v4i xb = *(const v4i*)(xq + b * 32 + 16);
    const float dx = xdq[b];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      int s = sdot4(wa[r].x, xa.x, 0);
      s = sdot4(wa[r].y, xa.y, s);
      s = sdot4(wa[r].z, xa.z, s);
      s = sdot4(wa[r].w, xa.w, s);
      s = sdot4(wb[r].x, xb.x, s);
      s = sdot4(wb[r].y, xb.y, s);
      s = sdot4(wb[r].z, xb.z, s);
      s = sdot4(wb[r].w, xb.w, s);
      float t = (float)s * f16_to_f32(wd[r]);
      t = t * dx;
      acc[r] = acc[r] + t;
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);
}

template <int NR>
__device__ __forceinline__ void dot_rows_bf16(const LinearDev& L, const int* rows, const float* xs,
                                              float* acc) {
  const int lane = threadIdx.x % kWave;
  const int K = L.in, nc = K / 8;
  const uint16_t* w = (const uint16_t*)L.w;
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
  for (int c = lane; c < nc; c += kWave) {
    v4u wv[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) wv[r] = __builtin_nontemporal_load((const v4u*)(w + (size_t)rows[r] * K) + c);
    const float4 x0 = *(const float4*)(xs + c * 8);
    const float4 x1 = *(const float4*)(xs + c * 8 + 4);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float a = acc[r];
      a = fmaf(u2f(wv[r].x << 16), x0.x, a);
      a = fmaf(u2f(wv[r].x & 0xffff0000u), x0.y, a);
      a = fmaf(u2f(wv[r].y << 16), x0.z, a);
      a = fmaf(u2f(wv[r].y & 0xffff0000u), x0.w, a);
      a = fmaf(u2f(wv[r].z << 16), x1.x, a);
      a = fmaf(u2f(wv[r].z & 0xffff0000u), x1.y, a);
      a = fmaf(u2f(wv[r].w << 16), x1.z, a);
      a = fmaf(u2f(wv[r].w & 0xffff0000u), x1.w, a);
      acc[r] = a;
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);
}

template <int NR>
__device__ __forceinline__ void dot_rows_f32(const LinearDev& L, const int* rows, const float* xs,
                                             float* acc) {
  const int lane = threadIdx.x % kWave;
  const int K = L.in, nc = K / 4;
  const float* w = (const float*)L.w;
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
  for (int c = lane; c < nc; c += kWave) {
    v4f wv[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) wv[r] = __builtin_nontemporal_load((const v4f*)(w + (size_t)rows[r] * K) + c);
    const float4 x0 = *(const float4*)(xs + c * 4);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float a = acc[r];
      a = fmaf(wv[r].x, x0.x, a);
      a = fmaf(wv[r].y, x0.y, a);
      a = fmaf(wv[r].z, x0.z, a);
      a = fmaf(wv[r].w, x0.w, a);
      acc[r] = a;
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);
}

// Applies the epilogue to physical row `row` with value `v`; `vp` is the value of the RoPE
// partner row (row ^ 1) for EPI_QKV_ROPE.
__device__ __forceinline__ void epilogue_row(const GemvArgs& a, int b, int row, float v, float vp) {
  switch (a.epi) {
    case EPI_STORE:
      a.y[(size_t)b * a.y_stride + row] = v;
      break;
    case EPI_GELU:
      a.y[(size_t)b * a.y_stride + row] = ref_gelu_tanh(v);
      break;
    case EPI_RESID: {
      float u = v;
      if (a.lscale) u = u * a.lscale[row];
      float* r = a.resid + (size_t)b * a.resid_stride + row;
      *r = *r + u;
      break;
    }
    case EPI_QKV_ROPE: {
      const int qdim = a.H * a.hd, kvdim = a.KVH * a.hd;
      const int p = a.pos[b];
      int region = row < qdim ? 0 : (row < qdim + kvdim ? 1 : 2);
      int rr = region == 0 ? row : (region == 1 ? row - qdim : row - qdim - kvdim);
      int head = rr / a.hd, dim = rr % a.hd;
      float out = v;
      if (region < 2) {
        float theta = (float)p * a.inv_freq[dim / 2];
        float c = cosf(theta), s = sinf(theta);
        if ((dim & 1) == 0) {
          float t0 = v * c, t1 = vp * s;
          out = t0 - t1;
        } else {
          float t0 = vp * s, t1 = v * c;
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

template <int FMT, int NR>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.L.in;
  float* xs = (float*)smem;                         // K floats
  int8_t* xq = (int8_t*)(xs + K);                   // K bytes
  float* xdq = (float*)(xq + K);                    // K/32 floats
  float* red = xdq + (K / 32);                      // 2 * kWaves floats
  const int b = blockIdx.y;
  const float* x = a.x + (size_t)b * a.x_stride;
  for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = x[i];
  __syncthreads();
  if (a.norm != NORM_NONE) norm_lds(xs, K, a.norm, a.nw, a.nb, a.eps, red);
  if (FMT == FMT_Q8_0) quantize_lds(xs, K, xq, xdq);

  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int items = a.epi == EPI_SILU_GATE ? a.ff_hidden : a.L.out;
  const int item0 = (blockIdx.x * kWaves + wave) * NR;
  if (item0 < items) {
    constexpr int NROWS = NR;  // rows per item group (SiLU handled with two passes)
    int rows[NROWS];
    float acc[NROWS], acc2[NROWS];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      int it = item0 + r < items ? item0 + r : items - 1;
      rows[r] = it;
    }
    if (FMT == FMT_Q8_0) dot_rows_q8<NR>(a.L, rows, xq, xdq, acc);
    else if (FMT == FMT_BF16) dot_rows_bf16<NR>(a.L, rows, xs, acc);
    else dot_rows_f32<NR>(a.L, rows, xs, acc);
    if (a.epi == EPI_SILU_GATE) {
#pragma unroll
      for (int r = 0; r < NR; ++r) rows[r] += a.ff_hidden;
      if (FMT == FMT_Q8_0) dot_rows_q8<NR>(a.L, rows, xq, xdq, acc2);
      else if (FMT == FMT_BF16) dot_rows_bf16<NR>(a.L, rows, xs, acc2);
      else dot_rows_f32<NR>(a.L, rows, xs, acc2);
    }
    if (lane < NR && item0 + lane < items) {
      float v = 0.0f, vp = 0.0f, v2 = 0.0f;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (r == lane) v = acc[r];
        if (r == (lane ^ 1)) vp = acc[r];
        if (a.epi == EPI_SILU_GATE && r == lane) v2 = acc2[r];
      }
      if (a.epi == EPI_SILU_GATE) {
        float g = ref_silu(v);
        a.y[(size_t)b * a.y_stride + item0 + lane] = g * v2;
      } else {
        epilogue_row(a, b, item0 + lane, v, vp);
      }
    }
  }
  if (a.advance_pos && blockIdx.x == 0 && threadIdx.x == 0) a.pos[b] += 1;
}

static size_t gemv_smem(int K) { return (size_t)K * 4 + K + (K / 32) * 4 + 2 * kWaves * 4 + 16; }

template <int FMT>
static hipError_t launch_gemv_fmt(const GemvArgs& a, hipStream_t s) {
  const int items = a.epi == EPI_SILU_GATE ? a.ff_hidden : a.L.out;
  // Rows per wave: enough waves to cover the GPU, and pairs for RoPE.
  int nr = items >= 4 * 4096 ? 4 : (items >= 2 * 4096 || a.epi == EPI_QKV_ROPE ? 2 : 1);
  if (a.epi == EPI_QKV_ROPE && nr < 2) nr = 2;
  dim3 block(kThreads);
  size_t smem = gemv_smem(a.L.in);
  if (nr == 4) {
    dim3 grid((items + kWaves * 4 - 1) / (kWaves * 4), a.B);
    hipLaunchKernelGGL((gemv_kernel<FMT, 4>), grid, block, smem, s, a);
  } else if (nr == 2) {
    dim3 grid((items + kWaves * 2 - 1) / (kWaves * 2), a.B);
    hipLaunchKernelGGL((gemv_kernel<FMT, 2>), grid, block, smem, s, a);
  } else {
    dim3 grid((items + kWaves - 1) / kWaves, a.B);
    hipLaunchKernelGGL((gemv_kernel<FMT, 1>), grid, block, smem, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs& a, hipStream_t s) {
  switch (a.L.fmt) {
    case FMT_Q8_0: return launch_gemv_fmt<FMT_Q8_0>(a, s);
    case FMT_BF16: return launch_gemv_fmt<FMT_BF16>(a, s);
    case FMT_F32: return launch_gemv_fmt<FMT_F32>(a, s);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------------------------
// Attention: one query per (stream, head) over the visible keys of the ring buffer, split in
// chunks of keys across workgroups (grid (nsplit, H, B)); each half-wave runs an online
// softmax over its keys, the workgroup merges its half-waves, and attn_combine merges splits.
// Visible keys of the query at position p: max(0, p - window + 1) ..= p
// (SVL/nn/transformer.rs:385, SVL/nn/kernels/attention.rs:107-113).

template <int DPL, bool BF16KV>
__device__ __forceinline__ void load_row(const void* base, size_t off, float* out) {
  if (BF16KV) {
    const uint16_t* p = (const uint16_t*)base + off;
    if (DPL == 4) {
      uint2 u = *(const uint2*)p;
      out[0] = u2f(u.x << 16); out[1] = u2f(u.x & 0xffff0000u);
      out[2] = u2f(u.y << 16); out[3] = u2f(u.y & 0xffff0000u);
    } else {
      uint32_t u = *(const uint32_t*)p;
      out[0] = u2f(u << 16); out[1] = u2f(u & 0xffff0000u);
    }
  } else {
    const float* p = (const float*)base + off;
    if (DPL == 4) {
      float4 v = *(const float4*)p;
      out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
      float2 v = *(const float2*)p;
      out[0] = v.x; out[1] = v.y;
    }
  }
}

template <int HD, bool BF16KV>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(AttnArgs a) {
  constexpr int DPL = HD / 32;
  __shared__ float sm[8], sl[8];
  __shared__ float so[8][HD];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int hw = threadIdx.x / 32, l32 = threadIdx.x % 32;
  const int p = a.pos[b];
  const int L = a.window > 0 ? min(p + 1, a.window) : p + 1;
  const int first = p + 1 - L;
  const int k0 = first + split * a.chunk;
  const int k1 = min(k0 + a.chunk, p + 1);
  const int kvh = h / (a.H / a.KVH);
  float q[DPL];
  const float* qp = a.q + (size_t)b * a.H * HD + (size_t)h * HD + l32 * DPL;
#pragma unroll
  for (int i = 0; i < DPL; ++i) q[i] = qp[i];
  float m = -__builtin_huge_valf(), l = 0.0f, o[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) o[i] = 0.0f;
  const size_t head_base = ((size_t)b * a.KVH + kvh) * (size_t)a.cap;
  for (int j = k0 + hw; j < k1; j += 8) {
    const size_t off = (head_base + (size_t)(j % a.cap)) * HD + l32 * DPL;
    float kv[DPL], vv[DPL];
    load_row<DPL, BF16KV>(a.kc, off, kv);
    load_row<DPL, BF16KV>(a.vc, off, vv);
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) d = fmaf(q[i], kv[i], d);
    float s = a.scale * half_sum(d);
    float mn = fmaxf(m, s);
    float c = ref_exp(m - mn);
    float e = ref_exp(s - mn);
    l = l * c + e;
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] = fmaf(e, vv[i], o[i] * c);
    m = mn;
  }
  if (l32 == 0) {
    sm[hw] = m;
    sl[hw] = l;
  }
#pragma unroll
  for (int i = 0; i < DPL; ++i) so[hw][l32 * DPL + i] = o[i];
  __syncthreads();
  const size_t pidx = ((size_t)b * a.H + h) * a.nsplit + split;
  if (threadIdx.x < HD) {
    float M = sm[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) M = fmaxf(M, sm[w]);
    float lsum = 0.0f, osum = 0.0f;
    if (M != -__builtin_huge_valf()) {
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        float f = ref_exp(sm[w] - M);
        lsum += sl[w] * f;
        osum += so[w][threadIdx.x] * f;
      }
    }
    a.po[pidx * HD + threadIdx.x] = osum;
    if (threadIdx.x == 0) {
      a.pm[pidx] = M;
      a.pl[pidx] = lsum;
    }
  }
}

template <int HD>
__global__ void attn_combine_kernel(AttnArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int p = a.pos[b];
  const int L = a.window > 0 ? min(p + 1, a.window) : p + 1;
  const int ns = (L + a.chunk - 1) / a.chunk;
  const size_t base = ((size_t)b * a.H + h) * a.nsplit;
  float M = -__builtin_huge_valf();
  for (int s = 0; s < ns; ++s) M = fmaxf(M, a.pm[base + s]);
  float lsum = 0.0f, osum = 0.0f;
  for (int s = 0; s < ns; ++s) {
    float f = ref_exp(a.pm[base + s] - M);
    lsum += a.pl[base + s] * f;
    osum += a.po[(base + s) * HD + d] * f;
  }
  a.out[(size_t)b * a.H * HD + (size_t)h * HD + d] = lsum > 0.0f ? osum / lsum : 0.0f;
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, a.H, a.B);
  if (a.hd == 128) {
    if (a.kv_bf16) hipLaunchKernelGGL((attn_partial_kernel<128, true>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((attn_partial_kernel<128, false>), grid, dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL((attn_combine_kernel<128>), dim3(a.H, a.B), dim3(128), 0, s, a);
  } else if (a.hd == 64) {
    if (a.kv_bf16) hipLaunchKernelGGL((attn_partial_kernel<64, true>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((attn_partial_kernel<64, false>), grid, dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL((attn_combine_kernel<64>), dim3(a.H, a.B), dim3(64), 0, s, a);
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
  float x;
  if (a.tables_bf16) x = bf16_to_f32(((const uint16_t*)a.text_emb)[(size_t)t * a.d + i]);
  else x = ((const float*)a.text_emb)[(size_t)t * a.d + i];
  for (int c = 0; c < a.n_q; ++c) {
    uint32_t tok = initial ? (uint32_t)a.card : a.audio[(size_t)b * a.n_q + c];
    tok = tok > (uint32_t)a.card ? (uint32_t)a.card : tok;
    float e;
    if (a.tables_bf16) e = bf16_to_f32(((const uint16_t*)a.emb[c])[(size_t)tok * a.d + i]);
    else e = ((const float*)a.emb[c])[(size_t)tok * a.d + i];
    x = x + e;
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
  float* red = xs + d;
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < d; i += kThreads) xs[i] = x[(size_t)b * x_stride + i];
  __syncthreads();
  norm_lds(xs, d, norm, w, nb, eps, red);
  for (int i = threadIdx.x; i < d; i += kThreads) y[(size_t)b * y_stride + i] = xs[i];
}

hipError_t launch_norm(const float* x, int x_stride, float* y, int y_stride, int B, int d, int norm,
                       const float* w, const float* b, float eps, hipStream_t s) {
  size_t smem = (size_t)d * 4 + 2 * kWaves * 4;
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
