// Work units of the decode step, run by one 1024-thread workgroup each.  The same functions
// back the one-kernel-per-phase launches and the persistent step-program kernel.
//
// Numerics follow the reference's CPU path (crates/semantic-voice-local/src = SVL) operation
// for operation, so results are bit-identical to the CPU restatement in oracle/:
//   * Q8_0 matmul as candle's quantized CPU matmul: the activation row is quantized to Q8_0
//     (d = amax / 127 kept as f16, q = round(x * (1 / d))); each weight block contributes
//     (exact i32 dot as f32 * d_w) * d_x, added in block order.
//   * dense matvec with the reference's 16-lane dot (SVL/nn/kernels/mod.rs:66-91).
//   * attention with the reference's two passes (SVL/nn/kernels/attention.rs:139-168).
//   * SiLU / GELU-tanh / exp as SVL/nn/kernels/{activation,mod}.rs (FMA variant).
//   * RMSNorm / LayerNorm statistics in a 64-way blocked order (see blocked_sum).
//
// Data one workgroup writes and another reads within a launch (activations, KV ring, scores,
// logits, tokens, positions) goes through agent-scope coherent loads and stores (the `sc1`
// cache policy on gfx950), so no cache-wide fence is needed at phase boundaries.
#pragma once

#include "device_math.h"
#include "kernels.h"

namespace svl {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---- global memory accesses ----------------------------------------------------------------------
// Every device pointer the units receive is global memory; it is addressed as such (global_load /
// global_store rather than flat accesses, whose completion the compiler has to wait for
// conservatively).

#define SVL_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ const SVL_GLOBAL T* gbl(const T* p) {
  return (const SVL_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ SVL_GLOBAL T* gbl(T* p) {
  return (SVL_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  return *gbl(p);
}
template <typename T>
__device__ __forceinline__ T ldg_stream(const T* p) {  // read once: non-temporal
  return __builtin_nontemporal_load(gbl(p));
}

// Coherent accesses: data one workgroup writes and another reads within a launch.
template <typename T>
__device__ __forceinline__ T ld_co(const T* p) {
  return __hip_atomic_load(gbl(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_co(T* p, T v) {
  __hip_atomic_store(gbl(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool BF16KV>
__device__ __forceinline__ float kv_ld(const void* base, size_t idx) {
  if (BF16KV) return bf16_to_f32(ld_co((const uint16_t*)base + idx));
  return ld_co((const float*)base + idx);
}

// ---- rows, norms, activation quantization ---------------------------------------------------------
// A row of K <= 8192 activations is held in registers, thread t owning elements t + 1024 u.

constexpr int kPerThread = 8192 / kStepThreads;

// v[u] = x[t + 1024 u] (coherent loads, all in flight together); 0 past K.  Every load is
// issued (past K at the clamped address x[K - 1]) so that the number of loads in flight is
// known at compile time and waiting for the row never waits for loads issued after it.
__device__ __forceinline__ void load_row(const float* x, int K, float (&v)[kPerThread]) {
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int i = threadIdx.x + u * kStepThreads;
    v[u] = ld_co(x + min(i, K - 1));
  }
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int i = threadIdx.x + u * kStepThreads;
    if (i >= K) v[u] = 0.0f;
  }
}

__device__ __forceinline__ void store_row(const float (&v)[kPerThread], int K, float* xs) {
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    if (u * kStepThreads >= K) break;  // uniform
    const int i = threadIdx.x + u * kStepThreads;
    if (i < K) xs[i] = v[u];
  }
}

// Lane 0 ends with the oracle's butterfly over 64 partials: for o = 32, 16, ..., 1, lane l < o
// adds lane l + o (the lanes whose results reach lane 0).
__device__ __forceinline__ float lane0_tree_sum(float v) {
  v = v + __shfl_down(v, 32, kWave);
  v = v + swizzle<0x401F>(v);  // lane ^ 16
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xf, 0xf, false));  // row_shl:8
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xf, 0xf, false));  // row_shl:4
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x102, 0xf, 0xf, false));  // row_shl:2
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xf, 0xf, false));  // row_shl:1
  return v;
}

// Sums of x[i] and of x[i]^2 over a row in the order shared with the oracle: 64 strided partials
// (lane l adds x[l], x[l+64], ... in order), then the butterfly over the partials (offsets
// 32 .. 1).  Run by one wave; the totals are valid in lane 0.
template <bool PLAIN>
__device__ __forceinline__ void blocked_sums(const float* xs, int K, float& s, float& s2) {
  const int lane = threadIdx.x % kWave;
  constexpr int U = 16;
  float a = 0.0f, a2 = 0.0f;
  int i = lane;
  for (; i + (U - 1) * kWave < K; i += U * kWave) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = xs[i + u * kWave];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (PLAIN) a = a + v[u];
      const float t = v[u] * v[u];
      a2 = a2 + t;
    }
  }
  for (; i < K; i += kWave) {
    const float v = xs[i];
    if (PLAIN) a = a + v;
    const float t = v * v;
    a2 = a2 + t;
  }
  s = PLAIN ? lane0_tree_sum(a) : 0.0f;
  s2 = lane0_tree_sum(a2);
}

// Norm weights of the elements a thread owns, loaded ahead of the row statistics.
struct NormW {
  float w[kPerThread], b[kPerThread];
};

__device__ __forceinline__ void load_norm_weights(int norm, const float* nw, const float* nb, int K, NormW& o) {
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) o.w[u] = ldg(nw + min((int)threadIdx.x + u * kStepThreads, K - 1));
  if (norm == NORM_LAYER) {
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) o.b[u] = ldg(nb + min((int)threadIdx.x + u * kStepThreads, K - 1));
  }
}

// candle-nn rms_norm (x / m * alpha, m = sqrt(sum(x^2) / K + eps)) or layer_norm
// ((x - mean) * (1 / sqrt(var + eps)) * w + b, var = sum(x^2) / K - mean^2) of the row in v,
// in place.  xs (K floats) and stats (2 floats) are LDS scratch; wave 0 computes the
// statistics.
__device__ __forceinline__ void norm_regs(float (&v)[kPerThread], int K, int norm, const NormW& nw, float eps, float* xs,
                                          float* stats) {
  store_row(v, K, xs);
  lds_barrier();
  if (threadIdx.x < kWave) {
    float s, s2;
    if (norm == NORM_LAYER) blocked_sums<true>(xs, K, s, s2);
    else blocked_sums<false>(xs, K, s, s2);
    if (threadIdx.x == 0) {
      if (norm == NORM_RMS) {
        stats[0] = sqrtf(s2 / (float)K + eps);
      } else {
        const float mean = s / (float)K;
        const float mm = mean * mean;
        const float var = s2 / (float)K - mm;
        stats[0] = mean;
        stats[1] = 1.0f / sqrtf(var + eps);
      }
    }
  }
  lds_barrier();
  const float s0 = stats[0], s1 = stats[1];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    if (u * kStepThreads >= K) break;  // uniform
    if (norm == NORM_RMS) {
      const float t = v[u] / s0;
      v[u] = t * nw.w[u];
    } else {
      float t = (v[u] - s0) * s1;
      t = t * nw.w[u];
      v[u] = t + nw.b[u];
    }
  }
}

// candle BlockQ8_0::from_float of the row in v into xq (int8, LDS) and xdq (the f16-rounded
// block scales as f32, LDS): amax = max(0, |x_i|...), d = amax / 127, id = 1 / d (0 if d = 0),
// q_i = round(x_i * id).  The 32 elements of a block are held by the 32 lanes of a half-wave;
// after the half-wave maximum, lane u of each half computes d and id of the block of element
// group u, and every lane takes id back from that lane.
__device__ __forceinline__ void quantize_regs(const float (&v)[kPerThread], int K, int8_t* xq, float* xdq) {
  const int hl = threadIdx.x & 31;
  float mine = 0.0f;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    if (u * kStepThreads >= K) break;  // uniform
    const float m = __uint_as_float(half_max_bits(__float_as_uint(fmaxf(fabsf(v[u]), 0.0f))));
    if (hl == u) mine = m;
  }
  const float dm = mine / 127.0f;
  const float idm = dm != 0.0f ? 1.0f / dm : 0.0f;
  const int own = (threadIdx.x & ~31) + hl * kStepThreads;  // first element of lane hl's block
  if (hl < kPerThread && own < K) xdq[own / 32] = f16_to_f32(f32_to_f16(dm));
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    if (u * kStepThreads >= K) break;  // uniform
    const float id = half_lane(idm, u);
    const int i = threadIdx.x + u * kStepThreads;
    if (i < K) xq[i] = (int8_t)sat_i8(roundf(v[u] * id));
  }
}

// acc = 0; acc += t[i] for i = 0 .. n-1 in order, reading t (16-byte aligned, in LDS) 16 values
// ahead of the additions.
__device__ __forceinline__ float ordered_sum(const float* t, int n) {
  typedef float v4f_t __attribute__((ext_vector_type(4)));
  const v4f_t* t4 = (const v4f_t*)t;
  const int n16 = n / 16;
  float acc = 0.0f;
  v4f_t cur[4], nxt[4];
  if (n16 > 0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) cur[u] = t4[u];
  }
  for (int c = 0; c < n16; ++c) {
    if (c + 1 < n16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) nxt[u] = t4[(c + 1) * 4 + u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc = acc + cur[u].x;
      acc = acc + cur[u].y;
      acc = acc + cur[u].z;
      acc = acc + cur[u].w;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) cur[u] = nxt[u];
  }
  for (int i = n16 * 16; i < n; ++i) acc = acc + t[i];
  return acc;
}

// ---- GEMV epilogues ---------------------------------------------------------------------------
// Inputs of an item's epilogue that live in global memory (RoPE cos/sin, the old residual) are
// loaded when the unit starts, so they arrive with the weights.

struct EpiIn {
  float a = 0.0f, b = 0.0f;  // QKV_ROPE: cos, sin; RESID: old residual
};

__device__ __forceinline__ EpiIn gemv_epi_prefetch(const GemvArgs& a, int b, int row, int p) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  EpiIn e;
  if (a.epi == EPI_QKV_ROPE) {
    // q rows, then k rows; v rows (no rotation) read an unused but valid entry
    const int qdim = a.H * a.hd;
    const int rr = row < qdim ? row : row - qdim;
    const v2f cs = ldg((const v2f*)(a.rope + ((size_t)p * (a.hd / 2) + (rr % a.hd) / 2) * 2));
    e.a = cs.x;
    e.b = cs.y;
  } else if (a.epi == EPI_RESID) {
    e.a = ld_co(a.resid + (size_t)b * a.resid_stride + row);
  }
  return e;
}

__device__ __forceinline__ void gemv_epilogue(const GemvArgs& a, int b, int row, int p, const EpiIn& in, float y,
                                              float yp, float yv) {
  switch (a.epi) {
    case EPI_STORE:
      st_co(a.y + (size_t)b * a.y_stride + row, y);
      break;
    case EPI_GELU:
      st_co(a.y + (size_t)b * a.y_stride + row, ref_gelu_tanh(y));
      break;
    case EPI_SILU_GATE: {
      // FeedForwardLayer::forward, gated (SVL/nn/transformer.rs:453-461): silu(gate) * value
      float g = ref_silu(y);
      st_co(a.y + (size_t)b * a.y_stride + row, g * yv);
      break;
    }
    case EPI_RESID: {
      float u = y;
      if (a.lscale) u = u * ldg(a.lscale + row);
      st_co(a.resid + (size_t)b * a.resid_stride + row, in.a + u);
      break;
    }
    case EPI_QKV_ROPE: {
      // split q | k | v (transformer.rs:330-338); interleaved RoPE of q and k (rope_i); k and v
      // into the ring slot of the current position.
      const int qdim = a.H * a.hd, kvdim = a.KVH * a.hd;
      const int region = row < qdim ? 0 : (row < qdim + kvdim ? 1 : 2);
      const int rr = region == 0 ? row : (region == 1 ? row - qdim : row - qdim - kvdim);
      const int head = rr / a.hd, dim = rr % a.hd;
      float out = y;
      if (region < 2) {
        const float c = in.a, s = in.b;
        if ((dim & 1) == 0) {
          float t0 = y * c, t1 = yp * s;
          out = t0 - t1;
        } else {
          float t0 = yp * s, t1 = y * c;
          out = t0 + t1;
        }
      }
      if (region == 0) {
        st_co(a.q_out + (size_t)b * qdim + rr, out);
      } else {
        const size_t idx = (((size_t)b * a.KVH + head) * a.cap + (size_t)(p % a.cap)) * a.hd + dim;
        void* base = region == 1 ? a.kc : a.vc;
        if (a.kv_bf16) st_co((uint16_t*)base + idx, f32_to_bf16(out));
        else st_co((float*)base + idx, out);
      }
      break;
    }
  }
}

__device__ __forceinline__ int gemv_phys_row(const GemvArgs& a, int i0, int ni, int r) {
  if (a.epi == EPI_SILU_GATE) return r < ni ? i0 + r : i0 + (r - ni) + a.ff_hidden;
  return i0 + r;
}

__device__ __forceinline__ void gemv_finish(const GemvArgs& a, int b, int part, int i0, int ni, int p, const EpiIn& in,
                                            const float* Y) {
  const int t = threadIdx.x;
  if (t < ni) {
    const float y = Y[t];
    const float yp = a.epi == EPI_QKV_ROPE ? Y[t ^ 1] : 0.0f;
    const float yv = a.epi == EPI_SILU_GATE ? Y[ni + t] : 0.0f;
    gemv_epilogue(a, b, i0 + t, p, in, y, yp, yv);
  }
  if (a.advance_pos && part == 0 && t == 0) st_co(a.pos + b, p + 1);
}

__device__ __forceinline__ int gemv_items(const GemvArgs& a) {
  return a.epi == EPI_SILU_GATE ? a.ff_hidden : a.L.out;
}

// Row stride of the per-block terms in LDS: 16-byte aligned, padded.
__device__ __forceinline__ int term_stride(int nb) { return ((nb + 3) & ~3) + 4; }

// ---- Q8_0 GEMV unit ---------------------------------------------------------------------------
// Candle's quantized CPU matmul (SVL/nn/mod.rs:97; BlockQ8_0::vec_dot_unopt): terms
// (exact i32 block dot as f32 * d_w) * d_x, each row adding its terms in block order.  The
// unit's weight blocks (one 32-byte block per thread and round) are loaded before the input is
// staged, since they do not depend on it.

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <int MAXB>
__device__ __forceinline__ void gemv_q8_unit(const GemvArgs& a, int unit, const int* spos, unsigned char* smem) {
  const int K = a.L.in, nb = K / 32;
  const int b = unit / a.parts, part = unit % a.parts;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int i0 = part * a.ipw;
  const int ni = min(a.ipw, gemv_items(a) - i0);
  const int NR = silu ? 2 * ni : ni;
  const int total = NR * nb;
  const int ts = term_stride(nb);
  const int p = spos[b];
  float* xs = (float*)smem;             // K
  int8_t* xq = (int8_t*)(xs + K);       // K
  float* xdq = (float*)(xq + K);        // nb (+ pad to 16 bytes)
  float* T = xdq + ((nb + 3) & ~3);     // 2 * ipw * ts
  float* Y = T + 2 * a.ipw * ts;        // 2 * ipw (first 2 floats: norm statistics)

  // The epilogue inputs, the row and its norm weights are requested before the weight blocks:
  // loads complete in order, so the norm and the quantization run while the weights stream in.
  const EpiIn in = gemv_epi_prefetch(a, b, i0 + min((int)threadIdx.x, ni - 1), p);
  NormW nwt;
  if (a.norm != NORM_NONE) load_norm_weights(a.norm, a.nw, a.nb, K, nwt);
  float v[kPerThread];
  load_row(a.x + (size_t)b * a.x_stride, K, v);
  __builtin_amdgcn_sched_barrier(0);
  const int8_t* wq = (const int8_t*)a.L.w;
  v4i wa[MAXB], wb[MAXB];
  uint32_t wd[MAXB];
  // block k of this thread: index threadIdx.x + 1024 k = r * nb + blk, stepped without division
  int rk[MAXB], bk[MAXB];
  {
    int r = threadIdx.x / nb, blk = threadIdx.x - (threadIdx.x / nb) * nb;
    const int dr = kStepThreads / nb, db = kStepThreads - dr * nb;
#pragma unroll
    for (int k = 0; k < MAXB; ++k) {
      rk[k] = r;
      bk[k] = blk;
      r += dr;
      blk += db;
      if (blk >= nb) {
        blk -= nb;
        ++r;
      }
    }
  }
  // Every thread issues MAXB block loads (past the unit's blocks: the unit's first block again),
  // so their number is known at compile time.
#pragma unroll
  for (int k = 0; k < MAXB; ++k) {
    const bool live = (int)threadIdx.x + k * kStepThreads < total;
    const int r = live ? rk[k] : 0, blk = live ? bk[k] : 0;
    const size_t row = (size_t)gemv_phys_row(a, i0, ni, r);
    const v4i* wp = (const v4i*)(wq + row * K + (size_t)blk * 32);
    wa[k] = ldg_stream(wp);
    wb[k] = ldg_stream(wp + 1);
    wd[k] = ldg(a.L.scale + row * nb + blk);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (a.norm != NORM_NONE) norm_regs(v, K, a.norm, nwt, a.eps, xs, Y);
  quantize_regs(v, K, xq, xdq);
  lds_barrier();
#pragma unroll
  for (int k = 0; k < MAXB; ++k) {
    const int idx = threadIdx.x + k * kStepThreads;
    if (idx < total) {
      const int r = rk[k], blk = bk[k];
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
      float t = (float)s * f16_to_f32((uint16_t)wd[k]);
      T[r * ts + blk] = t * xdq[blk];
    }
  }
  lds_barrier();
  if ((int)threadIdx.x < NR) Y[threadIdx.x] = ordered_sum(T + threadIdx.x * ts, nb);
  lds_barrier();
  gemv_finish(a, b, part, i0, ni, p, in, Y);
}

// ---- dense GEMV unit ----------------------------------------------------------------------------
// The reference's matvec (SVL/nn/kernels/matvec.rs:239-246) with its 16-lane dot
// (kernels/mod.rs:66-91): 16 threads per row, thread i accumulating x[16c + i] * w[16c + i]
// with FMA over c, then the pairwise lane sum and the scalar tail.  Up to 64 rows per unit
// (32 gate/value pairs for the SiLU gate).

template <bool BF16W>
__device__ __forceinline__ void gemv_dense_unit(const GemvArgs& a, int unit, const int* spos, unsigned char* smem) {
  const int K = a.L.in;
  const int b = unit / a.parts, part = unit % a.parts;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int i0 = part * a.ipw;
  const int ni = min(a.ipw, gemv_items(a) - i0);
  const int NR = silu ? 2 * ni : ni;
  const int p = spos[b];
  float* xs = (float*)smem;   // K
  float* Y = xs + K;          // kStepThreads / 16 (first 2 floats: norm statistics)
  EpiIn in;
  if ((int)threadIdx.x < ni) in = gemv_epi_prefetch(a, b, i0 + threadIdx.x, p);
  NormW nwt;
  if (a.norm != NORM_NONE) load_norm_weights(a.norm, a.nw, a.nb, K, nwt);
  float v[kPerThread];
  load_row(a.x + (size_t)b * a.x_stride, K, v);
  if (a.norm != NORM_NONE) {
    norm_regs(v, K, a.norm, nwt, a.eps, xs, Y);
    lds_barrier();  // every read of xs by the statistics is done
  }
  store_row(v, K, xs);
  lds_barrier();
  const int g = threadIdx.x / 16, li = threadIdx.x % 16;
  const int chunks = K / 16;
  if (g < NR) {
    const size_t row = (size_t)gemv_phys_row(a, i0, ni, g);
    float acc = 0.0f;
    int c = 0;
    if (BF16W) {
      const uint16_t* w = (const uint16_t*)a.L.w + row * K + li;
      for (; c + 16 <= chunks; c += 16) {
        uint16_t wv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) wv[u] = ldg_stream(w + (size_t)(c + u) * 16);
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = fmaf(xs[(c + u) * 16 + li], bf16_to_f32(wv[u]), acc);
      }
      for (; c < chunks; ++c) acc = fmaf(xs[c * 16 + li], bf16_to_f32(ldg(w + (size_t)c * 16)), acc);
    } else {
      const float* w = (const float*)a.L.w + row * K + li;
      for (; c + 16 <= chunks; c += 16) {
        float wv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) wv[u] = ldg_stream(w + (size_t)(c + u) * 16);
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = fmaf(xs[(c + u) * 16 + li], wv[u], acc);
      }
      for (; c < chunks; ++c) acc = fmaf(xs[c * 16 + li], ldg(w + (size_t)c * 16), acc);
    }
    // pairwise lane sum: acc[i] += acc[i + width] for width 8, 4, 2, 1
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o, 16);
    if (li == 0) {
      float tail = 0.0f;
      for (int i = chunks * 16; i < K; ++i) {
        const float wv = BF16W ? bf16_to_f32(ldg((const uint16_t*)a.L.w + row * K + i)) : ldg((const float*)a.L.w + row * K + i);
        float pr = xs[i] * wv;
        tail = tail + pr;
      }
      Y[g] = acc + tail;
    }
  }
  lds_barrier();
  gemv_finish(a, b, part, i0, ni, p, in, Y);
}

__device__ __forceinline__ void gemv_unit(const GemvArgs& a, int unit, const int* spos, unsigned char* smem) {
  if (a.L.fmt == FMT_Q8_0) {
    switch (a.maxb) {
      case 1: gemv_q8_unit<1>(a, unit, spos, smem); break;
      case 2: gemv_q8_unit<2>(a, unit, spos, smem); break;
      case 3: gemv_q8_unit<3>(a, unit, spos, smem); break;
      default: gemv_q8_unit<4>(a, unit, spos, smem); break;
    }
  } else if (a.L.fmt == FMT_BF16) {
    gemv_dense_unit<true>(a, unit, spos, smem);
  } else {
    gemv_dense_unit<false>(a, unit, spos, smem);
  }
}

// ---- attention units ----------------------------------------------------------------------------
// The query at position p attends to keys max(0, p - window + 1) ..= p (transformer.rs:385) in
// the ring, in the reference's order (attention.rs:139-168):
//   scores:    w_j = scale * dot(q, k_j) with the 16-lane dot; 64 keys per unit, one per
//              16-thread group.  Units are chunk-major (chunk = unit / (B * H)), so once a
//              chunk is past every stream's keys the workgroup has no more work in the phase.
//   softmax_v: max, e_j = exp(w_j - max), sum of e_j in key order, then
//              out = sum over keys in order of mul_add(e_j / sum, v_j, out).  One unit per
//              (stream, head); wave w produces dims [32w, 32w + 32).

constexpr int kKeysPerUnit = kStepThreads / 16;

__device__ __forceinline__ int visible_keys(const AttnArgs& a, int p) {
  return a.window > 0 ? min(p + 1, a.window) : p + 1;
}

// Returns false when no later unit of this phase has keys to score.
template <int HD, bool BF16KV>
__device__ __forceinline__ bool attn_scores_unit(const AttnArgs& a, int unit, const int* spos) {
  const int chunk = unit / (a.B * a.H);
  const int bh = unit % (a.B * a.H);
  const int b = bh / a.H, h = bh % a.H;
  const int p = spos[b];
  const int L = visible_keys(a, p);
  if (chunk * kKeysPerUnit >= L) {
    int lmax = 0;
    for (int i = 0; i < a.B; ++i) lmax = max(lmax, visible_keys(a, spos[i]));
    return chunk * kKeysPerUnit < lmax;
  }
  const int jj = chunk * kKeysPerUnit + threadIdx.x / 16;
  const int li = threadIdx.x % 16;
  constexpr int C = HD / 16;
  const int kvh = h / (a.H / a.KVH);
  const float* qp = a.q + (size_t)b * a.H * HD + (size_t)h * HD + li;
  float q[C], kv[C];
  const bool live = jj < L;
  const int j = p + 1 - L + jj;
  const size_t base = ((((size_t)b * a.KVH + kvh) * (size_t)a.cap) + (size_t)(live ? j % a.cap : 0)) * HD + li;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    q[c] = ld_co(qp + c * 16);
    kv[c] = kv_ld<BF16KV>(a.kc, base + c * 16);
  }
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) acc = fmaf(q[c], kv[c], acc);
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o, 16);
  if (live && li == 0) st_co(a.scores + ((size_t)b * a.H + h) * a.cap + jj, a.scale * (acc + 0.0f));
  return true;
}

template <int HD, bool BF16KV>
__device__ __forceinline__ void attn_softmax_v_unit(const AttnArgs& a, int unit, const int* spos, unsigned char* smem) {
  float* w = (float*)smem;                     // L weights (16-byte aligned)
  float* sum_slot = w + ((a.cap + 3) & ~3);    // 1
  const int h = unit % a.H, b = unit / a.H;
  const int p = spos[b];
  const int L = visible_keys(a, p);
  const int first = p + 1 - L;
  const float* sc = a.scores + ((size_t)b * a.H + h) * a.cap;
  for (int j0 = 0; j0 < L; j0 += 8 * kStepThreads) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + threadIdx.x + u * kStepThreads;
      if (j < L) v[u] = ld_co(sc + j);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + threadIdx.x + u * kStepThreads;
      if (j < L) w[j] = v[u];
    }
  }
  lds_barrier();
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (wave == 0) {
    float mx = -__builtin_huge_valf();
    for (int j = lane; j < L; j += kWave) mx = fmaxf(mx, w[j]);
    mx = wave_max(mx);
    for (int j = lane; j < L; j += kWave) w[j] = ref_exp(w[j] - mx);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes done before lane 0 reads them
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) sum_slot[0] = ordered_sum(w, L);
  }
  lds_barrier();
  const float sum = sum_slot[0];
  for (int j = threadIdx.x; j < L; j += kStepThreads) w[j] = w[j] / sum;
  lds_barrier();
  if (wave < HD / 32 && lane < 32) {
    const int d = wave * 32 + lane;
    const int kvh = h / (a.H / a.KVH);
    const size_t head_base = ((size_t)b * a.KVH + kvh) * (size_t)a.cap;
    constexpr int CH = 16;
    float acc = 0.0f;
    float cur[CH], nxt[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u)
      cur[u] = u < L ? kv_ld<BF16KV>(a.vc, (head_base + (size_t)((first + u) % a.cap)) * HD + d) : 0.0f;
    for (int j = 0; j < L; j += CH) {
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int jn = j + CH + u;
        nxt[u] = jn < L ? kv_ld<BF16KV>(a.vc, (head_base + (size_t)((first + jn) % a.cap)) * HD + d) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < CH; ++u)
        if (j + u < L) acc = fmaf(w[j + u], cur[u], acc);
#pragma unroll
      for (int u = 0; u < CH; ++u) cur[u] = nxt[u];
    }
    st_co(a.out + (size_t)b * a.H * HD + (size_t)h * HD + d, acc);
  }
}

__device__ __forceinline__ bool attn_scores_dispatch(const AttnArgs& a, int unit, const int* spos) {
  if (a.hd == 128) {
    if (a.kv_bf16) return attn_scores_unit<128, true>(a, unit, spos);
    return attn_scores_unit<128, false>(a, unit, spos);
  }
  if (a.kv_bf16) return attn_scores_unit<64, true>(a, unit, spos);
  return attn_scores_unit<64, false>(a, unit, spos);
}

__device__ __forceinline__ void attn_softmax_v_dispatch(const AttnArgs& a, int unit, const int* spos, unsigned char* smem) {
  if (a.hd == 128) {
    if (a.kv_bf16) attn_softmax_v_unit<128, true>(a, unit, spos, smem);
    else attn_softmax_v_unit<128, false>(a, unit, spos, smem);
  } else {
    if (a.kv_bf16) attn_softmax_v_unit<64, true>(a, unit, spos, smem);
    else attn_softmax_v_unit<64, false>(a, unit, spos, smem);
  }
}

// ---- embedding, argmax, norm, copies ----------------------------------------------------------

// SVL/stt/model.rs:246-250: x = text_emb[t] + emb_0[a_0] + ... in that order, f32 adds.  Token
// ids past the tables are clamped (the host validates its own inputs).  Units: B x d / 1024.
__device__ __forceinline__ void embed_unit(const EmbedArgs& a, const uint32_t* text, const uint32_t* audio, int unit, const int* spos) {
  const int chunks = (a.d + kStepThreads - 1) / kStepThreads;
  const int b = unit / chunks;
  const int i = (unit % chunks) * kStepThreads + threadIdx.x;
  if (i >= a.d) return;
  const bool initial = a.initial_at_zero && spos[b] == 0;
  const uint32_t* au = audio + (size_t)b * a.n_q;
  uint32_t t = text ? ldg(text + b) : ld_co(a.fb_tok + b);
  t = t > (uint32_t)a.text_card ? (uint32_t)a.text_card : t;
  const size_t rows = (size_t)a.card + 1;
  float x = a.tables_bf16 ? bf16_to_f32(ldg((const uint16_t*)a.text_emb + (size_t)t * a.d + i))
                          : ldg((const float*)a.text_emb + (size_t)t * a.d + i);
  constexpr int G = 16;  // codebooks per round: tokens, then rows, then the adds in order
  for (int c0 = 0; c0 < a.n_q; c0 += G) {
    uint32_t tok[G];
    float e[G];
#pragma unroll
    for (int u = 0; u < G; ++u) tok[u] = c0 + u < a.n_q ? (initial ? (uint32_t)a.card : ldg(au + c0 + u)) : 0u;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      if (c0 + u < a.n_q) {
        const uint32_t tk = tok[u] > (uint32_t)a.card ? (uint32_t)a.card : tok[u];
        const size_t idx = ((size_t)(c0 + u) * rows + tk) * a.d + i;
        e[u] = a.tables_bf16 ? bf16_to_f32(ldg((const uint16_t*)a.emb + idx)) : ldg((const float*)a.emb + idx);
      }
    }
#pragma unroll
    for (int u = 0; u < G; ++u)
      if (c0 + u < a.n_q) x = x + e[u];
  }
  st_co(a.x + (size_t)b * a.d + i, x);
}

// argmax over logits[b] (first index of the maximum); unit = stream.
__device__ __forceinline__ void argmax_unit(const ArgmaxArgs& a, uint32_t* out, int unit, unsigned char* smem) {
  float* sv = (float*)smem;
  int* si = (int*)(sv + 16);
  const int b = unit;
  const float* lg = a.logits + (size_t)b * a.V;
  float best = -__builtin_huge_valf();
  int idx = 0x7fffffff;
  constexpr int R = 8;
  for (int i0 = 0; i0 < a.V; i0 += R * kStepThreads) {
    float v[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int i = i0 + threadIdx.x + u * kStepThreads;
      if (i < a.V) v[u] = ld_co(lg + i);
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int i = i0 + threadIdx.x + u * kStepThreads;
      if (i < a.V && (idx == 0x7fffffff || v[u] > best)) {
        best = v[u];
        idx = i;
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(idx, o, kWave);
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
  lds_barrier();
  if (threadIdx.x == 0) {
    float bv = sv[0];
    int bi = si[0];
    for (int w = 1; w < kStepThreads / kWave; ++w) {
      if (si[w] != 0x7fffffff && (bi == 0x7fffffff || sv[w] > bv || (sv[w] == bv && si[w] < bi))) {
        bv = sv[w];
        bi = si[w];
      }
    }
    if (bi == 0x7fffffff) bi = 0;
    st_co(a.fb_tok + b, (uint32_t)bi);
    if (out) st_co(out + b, (uint32_t)bi);
  }
}

// y[b] = norm(x[b]); unit = stream.
__device__ __forceinline__ void norm_unit(const NormArgs& a, int unit, unsigned char* smem) {
  float* xs = (float*)smem;
  NormW nwt;
  load_norm_weights(a.norm, a.w, a.b, a.d, nwt);
  float v[kPerThread];
  load_row(a.x + (size_t)unit * a.x_stride, a.d, v);
  norm_regs(v, a.d, a.norm, nwt, a.eps, xs, xs + a.d);
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int i = threadIdx.x + u * kStepThreads;
    if (i < a.d) st_co(a.y + (size_t)unit * a.y_stride + i, v[u]);
  }
}

// y[b][0..n) = x[b][0..n); unit = (stream, 1024-element chunk).
__device__ __forceinline__ void copy_unit(const float* x, int x_stride, float* y, int y_stride, int n, int unit) {
  const int chunks = (n + kStepThreads - 1) / kStepThreads;
  const int b = unit / chunks;
  const int i = (unit % chunks) * kStepThreads + threadIdx.x;
  if (i < n) st_co(y + (size_t)b * y_stride + i, ld_co(x + (size_t)b * x_stride + i));
}

// Runs work unit `unit` of phase `ph` for step `step` of a launch; `spos` holds the streams'
// positions at the start of the step.  Returns false when the workgroup has no later unit in
// this phase.
__device__ __forceinline__ bool run_unit(const Phase& ph, const StepParams& P, int step, int unit, const int* spos,
                                         unsigned char* smem) {
  switch (ph.kind) {
    case PH_EMBED: {
      const uint32_t* text = P.text ? P.text + (size_t)step * P.text_stride : nullptr;
      embed_unit(ph.e, text, P.audio + (size_t)step * P.audio_stride, unit, spos);
      break;
    }
    case PH_GEMV:
      gemv_unit(ph.g, unit, spos, smem);
      break;
    case PH_ATTN_SCORES:
      return attn_scores_dispatch(ph.at, unit, spos);
    case PH_ATTN_SOFTMAX_V:
      attn_softmax_v_dispatch(ph.at, unit, spos, smem);
      break;
    case PH_ARGMAX:
      argmax_unit(ph.am, P.out_tok ? P.out_tok + (size_t)step * P.out_stride : nullptr, unit, smem);
      break;
    case PH_NORM:
      norm_unit(ph.nm, unit, smem);
      break;
    case PH_COPY_IN:
      copy_unit(P.fwd_in + (size_t)step * ph.cp.n, ph.cp.x_stride, ph.cp.y, ph.cp.y_stride, ph.cp.n, unit);
      break;
    case PH_COPY_OUT:
      copy_unit(ph.cp.x, ph.cp.x_stride, P.fwd_out + (size_t)step * ph.cp.n, ph.cp.y_stride, ph.cp.n, unit);
      break;
  }
  return true;
}

}  // namespace svl
