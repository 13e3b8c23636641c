// Work units of the decode step.  The same functions back the persistent step-program kernel
// and the one-kernel-per-phase launches.
//
// Numerics follow the reference's CPU path (crates/semantic-voice-local/src = SVL) operation
// for operation, so results are bit-identical to the CPU restatement in oracle/:
//   * Q8_0 matmul as candle's quantized CPU matmul: the activation row is quantized to Q8_0
//     (d = amax / 127 kept as f16, q = round(x * (1 / d))); each weight block contributes
//     (exact i32 dot as f32 * d_w) * d_x, added in block order.
//   * dense matvec with the reference's 16-lane dot (SVL/nn/kernels/mod.rs:66-91).
//   * attention with the reference's two passes (SVL/nn/kernels/attention.rs:139-168).
//   * SiLU / GELU-tanh / exp as SVL/nn/kernels/{activation,mod}.rs (FMA variant).
//   * RMSNorm / LayerNorm statistics as candle-nn's CPU ops: one f32 accumulator per sum, the
//     elements added in index order (see element_stats).
//
// Data one workgroup writes and another reads within a launch (activations, KV ring, scores,
// logits, tokens, positions) goes through agent-scope coherent loads and stores (the `sc1`
// cache policy on gfx950), so no cache-wide fence is needed at phase boundaries.
//
// Workgroup roles.  A workgroup is 16 waves.  The row waves (threads [0, 512)) run every
// unit's dependent chain -- input row, norm, quantization, row sums, epilogues, attention,
// embedding, argmax -- and the grid barrier.  The weight waves (threads [512, 1024)) only
// stream Q8_0 weight blocks into registers and compute the block dot products.  Weight waves
// never join a workgroup barrier: they request the next unit's blocks as soon as the current
// unit's dot products are written, and issuing those loads may wait on the memory system for
// microseconds, during which the row waves go on with the epilogue, the grid barrier and the
// next input row.  The groups hand over through counters in LDS (WgSync); the Q8_0 GEMV units
// a workgroup runs are numbered in program order ("items"):
//   xq_parts  += 1 per row wave once its part of item i's quantized input row is in LDS,
//   t_parts   += 1 per weight wave once its block terms of item i are in LDS.
// Row waves synchronize among themselves with a counter barrier (RowSync).
#pragma once

#include "device_math.h"
#include "exact_sum.h"
#include "kernels.h"

namespace svl {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---- global memory accesses ----------------------------------------------------------------------
// Every device pointer the units receive is global memory; it is addressed as such (global_load /
// global_store rather than flat accesses, whose completion the compiler has to wait for
// conservatively).

#define SVL_GLOBAL __attribute__((address_space(1)))
#define SVL_CONST __attribute__((address_space(4)))

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
// Uniform read of memory that no kernel writes while a launch runs (the step program):
// scalar loads.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const SVL_CONST T*)p;
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

// ---- workgroup roles and LDS hand-over -----------------------------------------------------------

constexpr int kRowWaves = kRowThreads / kWave;
constexpr int kWeightWaves = kWeightThreads / kWave;

struct WgSync {
  unsigned r_arrive;   // row-wave barrier arrivals
  unsigned xq_parts;   // row waves done quantizing an item's input row
  unsigned t_parts;    // weight waves done with an item's block terms
  unsigned r_issued;   // row waves that have requested an item's input row
  unsigned g_arrive;   // row waves whose stores of the phase are complete (grid barrier)
  unsigned g_release;  // grid barriers of the launch this workgroup has passed
  unsigned stop;       // raised when a wait gave up or the grid barrier aborted
  unsigned w_staged;   // weight waves whose staged weight loads have landed (dense, one item per launch)
  float stats[2];      // a row's norm statistics (sum of squares, sum), published by row wave 0
};

constexpr unsigned kLdsSpinLimit = 1u << 22;

__device__ __forceinline__ unsigned lds_ld(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits until *ctr reaches `target` (counters only grow; the comparison is wrap-safe).  Returns
// false once `stop` is raised, or after the spin limit (which raises it).  Long waits (LONG)
// sleep between polls so that the waiting wave leaves the SIMD and LDS to the others.
template <bool LONG = false>
__device__ __forceinline__ bool lds_wait(const unsigned* ctr, unsigned target, unsigned* stop) {
  unsigned spins = 0;
  while ((int)(lds_ld(ctr) - target) < 0) {
    if ((++spins & 15) == 0) {  // one LDS round trip per poll; the abort flag every 16th
      if (lds_ld(stop)) return false;
      if (spins > kLdsSpinLimit) {
        __hip_atomic_store(stop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return false;
      }
    }
    if (LONG) __builtin_amdgcn_s_sleep(2);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  return true;
}

// This wave's LDS writes complete, then lane 0 adds one to *ctr.
__device__ __forceinline__ void lds_signal(unsigned* ctr) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if ((threadIdx.x & (kWave - 1)) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// LDS writes of this wave are visible to its own later reads (LDS operations of a wave complete
// in order; this keeps the compiler from moving reads above the writes).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The hardware workgroup barrier after this wave's LDS accesses (outstanding global loads,
// direct-to-LDS ones included, stay in flight).  It waits for every wave of the workgroup that
// has not ended.
__device__ __forceinline__ void hw_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

// Barrier of the row waves.  Every row wave calls sync() the same number of times.  Two kinds:
//   * hw: the hardware barrier (~50 cycles), which every wave of the workgroup that has not ended
//     must pass: for launches whose weight waves have ended (or that have none).
//   * otherwise a counter in LDS (~500 cycles), for launches whose weight waves stream weights
//     meanwhile: they are held up by their own requests for as long as the bytes take to arrive,
//     and could not take part in a hardware barrier promptly.
struct RowSync {
  WgSync* ws;
  unsigned epoch;
  bool hw = false;
  __device__ __forceinline__ void sync() {
    if (hw) {
      hw_barrier();
      return;
    }
    lds_signal(&ws->r_arrive);
    epoch += kRowWaves;
    lds_wait(&ws->r_arrive, epoch, &ws->stop);
  }
  // The same barrier for waits of microseconds: waiting waves sleep between polls, leaving the
  // SIMD to the wave that works.
  __device__ __forceinline__ void sync_long() {
    if (hw) {
      hw_barrier();
      return;
    }
    lds_signal(&ws->r_arrive);
    epoch += kRowWaves;
    lds_wait<true>(&ws->r_arrive, epoch, &ws->stop);
  }
};

// Clears the workgroup's LDS counters; the one full-workgroup barrier of a launch.
__device__ __forceinline__ void init_wg_sync(WgSync* ws) {
  if (threadIdx.x == 0) {
    ws->r_arrive = 0;
    ws->xq_parts = 0;
    ws->t_parts = 0;
    ws->r_issued = 0;
    ws->g_arrive = 0;
    ws->g_release = 0;
    ws->stop = 0;
    ws->w_staged = 0;
  }
  __syncthreads();  // the only full-workgroup barrier: nothing is in flight yet
}

// ---- rows, norms, activation quantization ---------------------------------------------------------
// A row of K <= 8192 activations is held in registers by the row waves, thread t owning
// elements t + 512 u for u < KP, KP = row_slots(K) (a compile-time count, so that no branch
// merges the register arrays).  Slots past K read the clamped address x[K - 1] and hold 0.

constexpr int kMaxSlots = 8192 / kRowThreads;

__host__ __device__ constexpr int row_slots(int K) {
  return K <= 2 * kRowThreads ? 2 : (K <= 4 * kRowThreads ? 4 : (K <= 8 * kRowThreads ? 8 : kMaxSlots));
}

// v[u] = x[t + 512 u] (coherent loads, all in flight together); 0 past K.  When `issued` is
// given, the wave counts itself there once its loads are requested.
template <int KP>
__device__ __forceinline__ void load_row(const float* x, int K, float (&v)[KP], unsigned* issued = nullptr) {
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    const int i = threadIdx.x + u * kRowThreads;
    v[u] = ld_co(x + min(i, K - 1));
  }
  if (issued) {
    __builtin_amdgcn_sched_barrier(0);
    lds_signal(issued);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    const int i = threadIdx.x + u * kRowThreads;
    v[u] = i < K ? v[u] : 0.0f;
  }
}

template <int KP>
__device__ __forceinline__ void store_row(const float (&v)[KP], int K, float* xs) {
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    const int i = threadIdx.x + u * kRowThreads;
    if (i < K) xs[i] = v[u];
  }
}

static_assert(kSumThreads == kRowThreads, "the row waves sum the norm statistics");

// Row statistics in element order, as candle-nn's CPU RmsNorm / LayerNorm compute them: one f32
// accumulator per sum, x_0, x_1, ... added in index order.  The row is staged in LDS contiguously:
// xs[0, staged_floats(K)) the values (LayerNorm only; RMSNorm uses that space as the summing
// scratch) and xs[staged_floats(K), ...) the squares fl(x_i * x_i).  RMSNorm's sum of squares
// takes the exact parallel path of exact_sum.h over all row waves; LayerNorm runs the two
// sequential chains in one instruction stream (lane 0 over the squares, lane 1 over the values)
// while the other row waves sleep at the barrier.  s2 = sum of squares, s = sum of values
// (LayerNorm).  U = slabs of 2048 elements (K <= 2048 U).
__host__ __device__ constexpr int norm_scratch_floats(int K) { return 2 * staged_floats(K); }

template <int U>
__device__ __forceinline__ void element_stats(float* xs, int K, int norm, RowSync& rs, float& s, float& s2) {
  rs.sync();  // the row is staged
  const float* sq = xs + staged_floats(K);
  if (norm == NORM_RMS) {
    s2 = block_exact_sum_squares<U>(sq, K, (unsigned char*)xs, rs);
    s = 0.0f;
    if (threadIdx.x == 0) rs.ws->stats[0] = s2;
    return;
  }
  if (threadIdx.x < 2) rs.ws->stats[threadIdx.x] = ordered_sum_from(threadIdx.x == 1 ? xs : sq, K, 0.0f);
  rs.sync_long();
  s2 = rs.ws->stats[0];
  s = rs.ws->stats[1];
}

// Norm weights of the elements a thread owns, loaded ahead of the row statistics.
template <int KP>
struct NormW {
  float w[KP], b[KP];
};

template <int KP>
__device__ __forceinline__ void load_norm_weights(int norm, const float* nw, const float* nb, int K, NormW<KP>& o) {
#pragma unroll
  for (int u = 0; u < KP; ++u) o.w[u] = ldg(nw + min((int)threadIdx.x + u * kRowThreads, K - 1));
#pragma unroll
  for (int u = 0; u < KP; ++u) o.b[u] = norm == NORM_LAYER ? ldg(nb + min((int)threadIdx.x + u * kRowThreads, K - 1)) : 0.0f;
}

// candle-nn rms_norm (x / m * alpha, m = sqrt(sum(x^2) / K + eps)) or layer_norm
// ((x - mean) * (1 / sqrt(var + eps)) * w + b, var = sum(x^2) / K - mean^2) of the row in v,
// in place.  xs (2 K floats) is LDS scratch.
template <int KP>
__device__ __forceinline__ void norm_regs(float (&v)[KP], int K, int norm, const NormW<KP>& nw, float eps, float* xs,
                                          RowSync& rs) {
  constexpr int U = (KP + 3) / 4;  // K <= 512 KP
  float* sq = xs + staged_floats(K);
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    const int i = threadIdx.x + u * kRowThreads;
    if (i < K) {
      if (norm == NORM_LAYER) xs[i] = v[u];
      sq[i] = v[u] * v[u];
    }
  }
  float s, s2;
  element_stats<U>(xs, K, norm, rs, s, s2);
  float s0, s1 = 0.0f;
  if (norm == NORM_RMS) {
    s0 = sqrtf(s2 / (float)K + eps);
  } else {
    const float mean = s / (float)K;
    const float mm = mean * mean;
    const float var = s2 / (float)K - mm;
    s0 = mean;
    s1 = 1.0f / sqrtf(var + eps);
  }
  if (norm == NORM_RMS) {
#pragma unroll
    for (int u = 0; u < KP; ++u) {
      const float t = v[u] / s0;
      v[u] = t * nw.w[u];
    }
  } else {
#pragma unroll
    for (int u = 0; u < KP; ++u) {
      float t = (v[u] - s0) * s1;
      t = t * nw.w[u];
      v[u] = t + nw.b[u];
    }
  }
}

// ---- rows in 4-element chunks (Q8_0 activation quantization) -------------------------------------
// The Q8_0 paths hold the input row as 4-element chunks: thread t owns elements 4 c .. 4 c + 3 of
// chunks c = t + 512 u, u < KU = chunk_slots(K); a Q8_0 block (32 elements) is the chunks of 8
// consecutive lanes, so that its maximum takes three lane exchanges and each element costs a few
// instructions.  Chunks past K / 4 hold 0.

typedef float v4f __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int chunk_slots(int K) { return (K + 4 * kRowThreads - 1) / (4 * kRowThreads); }

// v[u] = the chunk's four elements: one 16-byte coherent (agent scope, the sc1 cache policy)
// buffer load per chunk over the row x (16-byte aligned), all in flight together.  When `issued`
// is given, the wave counts itself there once its loads are requested.
template <int KU>
__device__ __forceinline__ void load_row4(const float* x, int K, v4f (&v)[KU], unsigned* issued = nullptr) {
  const int nc = K / 4;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, K * 4, 0x00020000);
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int c = min((int)threadIdx.x + u * kRowThreads, nc - 1);
    v[u] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, 16 * c, 0, 16));
  }
  if (issued) {
    __builtin_amdgcn_sched_barrier(0);
    lds_signal(issued);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int u = 0; u < KU; ++u)
    if ((int)threadIdx.x + u * kRowThreads >= nc) v[u] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
}

template <int KU>
struct NormW4 {
  v4f w[KU], b[KU];
};

template <int KU>
__device__ __forceinline__ void load_norm_weights4(int norm, const float* nw, const float* nb, int K, NormW4<KU>& o) {
  const int nc = K / 4;
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int c = min((int)threadIdx.x + u * kRowThreads, nc - 1);
    o.w[u] = ldg((const v4f*)nw + c);
    o.b[u] = norm == NORM_LAYER ? ldg((const v4f*)nb + c) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }
}

// norm_regs on the chunked row: the same statistics, the same per-element arithmetic.
template <int KU>
__device__ __forceinline__ void norm_row4(v4f (&v)[KU], int K, int norm, const NormW4<KU>& nw, float eps, float* xs,
                                          RowSync& rs) {
  const int nc = K / 4;  // K <= 2048 KU
  float* sq = xs + staged_floats(K);
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int c = threadIdx.x + u * kRowThreads;
    if (c < nc) {
      if (norm == NORM_LAYER) *(v4f*)(xs + 4 * c) = v[u];
      *(v4f*)(sq + 4 * c) = v[u] * v[u];
    }
  }
  float s, s2;
  element_stats<KU>(xs, K, norm, rs, s, s2);
  if (norm == NORM_RMS) {
    const float s0 = sqrtf(s2 / (float)K + eps);
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float t = v[u][e] / s0;
        v[u][e] = t * nw.w[u][e];
      }
  } else {
    const float mean = s / (float)K;
    const float mm = mean * mean;
    const float var = s2 / (float)K - mm;
    const float s1 = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = (v[u][e] - mean) * s1;
        t = t * nw.w[u][e];
        v[u][e] = t + nw.b[u][e];
      }
  }
}

// candle BlockQ8_0::from_float of the chunked row into xq (int8, LDS) and xdq (the f16-rounded
// block scales as f32, LDS): amax = max(0, |x_i|...), d = amax / 127, id = 1 / d (0 if d = 0),
// q_i = round(x_i * id).  The block maximum runs over 8 lanes (after each lane's maximum of its
// four elements); every lane then computes its block's d and id and writes its four quantized
// elements as one word; lane 0 of the 8 writes the block scale.
// With `xsum` (Q4_0 weights), lane 0 of the 8 also writes the block's sum of quantized values
// (exact), which the Q4_0 dot subtracts 8 times: sum (code - 8) q = sum code q - 8 sum q.
template <int KU>
__device__ __forceinline__ void quantize_row4(const v4f (&v)[KU], int K, int8_t* xq, float* xdq, int* xsum = nullptr) {
  const int nc = K / 4;
  uint32_t m[KU];
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const uint32_t a0 = __float_as_uint(fmaxf(fabsf(v[u].x), 0.0f)), a1 = __float_as_uint(fmaxf(fabsf(v[u].y), 0.0f));
    const uint32_t a2 = __float_as_uint(fmaxf(fabsf(v[u].z), 0.0f)), a3 = __float_as_uint(fmaxf(fabsf(v[u].w), 0.0f));
    m[u] = max(max(a0, a1), max(a2, a3));
  }
#pragma unroll
  for (int u = 0; u < KU; ++u) m[u] = max(m[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m[u], 0xB1, 0xf, 0xf, false));
#pragma unroll
  for (int u = 0; u < KU; ++u) m[u] = max(m[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m[u], 0x4E, 0xf, 0xf, false));
#pragma unroll
  for (int u = 0; u < KU; ++u) m[u] = max(m[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m[u], 0x141, 0xf, 0xf, false));
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int c = threadIdx.x + u * kRowThreads;
    if (c >= nc) continue;  // uniform per 8 lanes (nc is a multiple of 8)
    const float dm = __uint_as_float(m[u]) / 127.0f;
    const float idm = dm != 0.0f ? 1.0f / dm : 0.0f;
    if ((c & 7) == 0) xdq[c / 8] = f16_to_f32(f32_to_f16(dm));
    const uint32_t q0 = (uint32_t)sat_i8(roundf(v[u].x * idm)) & 0xffu;
    const uint32_t q1 = (uint32_t)sat_i8(roundf(v[u].y * idm)) & 0xffu;
    const uint32_t q2 = (uint32_t)sat_i8(roundf(v[u].z * idm)) & 0xffu;
    const uint32_t q3 = (uint32_t)sat_i8(roundf(v[u].w * idm)) & 0xffu;
    const uint32_t word = q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
    ((uint32_t*)xq)[c] = word;
    if (xsum) {  // uniform
      int bs = __builtin_amdgcn_sdot4((int)word, 0x01010101, 0, false);
      bs += __builtin_amdgcn_update_dpp(0, bs, 0xB1, 0xf, 0xf, false);
      bs += __builtin_amdgcn_update_dpp(0, bs, 0x4E, 0xf, 0xf, false);
      bs += __builtin_amdgcn_update_dpp(0, bs, 0x141, 0xf, 0xf, false);
      if ((c & 7) == 0) xsum[c / 8] = bs;
    }
  }
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
    const float* tab = p < a.rope_cap ? a.rope + (size_t)p * a.hd : a.rope_ovf + (size_t)(p + ldg(a.rope_delta + b)) * a.hd;
    const v2f cs = ldg((const v2f*)(tab + (rr % a.hd) / 2 * 2));
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
    case EPI_GELU_ERF:
      st_co(a.y + (size_t)b * a.y_stride + row, ref_gelu_erf(y));
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
        const size_t kb = a.kv_group > 1 ? (size_t)(b / a.kv_group) : (size_t)b;  // the ring's stream
        const size_t idx = ((kb * a.KVH + head) * a.cap + (size_t)(p % a.cap)) * a.hd + dim;
        void* base = region == 1 ? a.kc : a.vc;
        if (a.kv_bf16) st_co((uint16_t*)base + idx, f32_to_bf16(out));
        else st_co((float*)base + idx, out);
      }
      break;
    }
  }
}

__device__ __forceinline__ int gemv_phys_row(int epi, int ff_hidden, int i0, int ni, int r) {
  if (epi == EPI_SILU_GATE) return r < ni ? i0 + r : i0 + (r - ni) + ff_hidden;
  return i0 + r;
}

__device__ __forceinline__ int gemv_items(const GemvArgs& a) {
  return a.epi == EPI_SILU_GATE ? a.ff_hidden : a.L.out;
}

// Epilogue of a unit's ni items by row threads t < ni.
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

// Q4K terms are stored block-major, T[blk * ts + r] with an odd stride ts = 2 ipw + 1, so that
// the row threads (consecutive r) and the weight-wave threads (consecutive blk) both access LDS
// without bank conflicts.
__device__ __forceinline__ int term_stride(int ipw) { return 2 * ipw + 1; }

// Q8_0 terms are stored row-major, T[r * rs + blk] with rs = q8_row_stride(nb): a multiple of 4
// (16-byte rows) with 4 words of padding, so that the rows' 16-byte reads fall in different banks.
__host__ __device__ inline int q8_row_stride(int nb) { return ((nb + 3) & ~3) + 4; }

// acc = 0; acc += T[r * rs + blk] for blk = 0 .. nb-1 in order; each batch of 32 terms is read
// (as 16-byte vectors) before its additions, the last partial batch too.
__device__ __forceinline__ float ordered_row_sum(const float* T, int rs, int r, int nb) {
  typedef float v4f_t __attribute__((ext_vector_type(4)));
  const v4f_t* t4 = (const v4f_t*)(T + r * rs);
  float acc = 0.0f;
  int blk = 0;
  for (; blk + 32 <= nb; blk += 32) {
    v4f_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = t4[blk / 4 + u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc = acc + v[u].x;
      acc = acc + v[u].y;
      acc = acc + v[u].z;
      acc = acc + v[u].w;
    }
  }
  if (blk < nb) {  // the last partial batch (vectors past the row's last read its last vector)
    v4f_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = t4[min(blk / 4 + u, (nb - 1) / 4)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int b0 = blk + 4 * u;
      acc = b0 < nb ? acc + v[u].x : acc;
      acc = b0 + 1 < nb ? acc + v[u].y : acc;
      acc = b0 + 2 < nb ? acc + v[u].z : acc;
      acc = b0 + 3 < nb ? acc + v[u].w : acc;
    }
  }
  return acc;
}

// ---- Q8_0 GEMV ------------------------------------------------------------------------------------
// Candle's quantized CPU matmul (SVL/nn/mod.rs:97; BlockQ8_0::vec_dot_unopt): terms
// (exact i32 block dot as f32 * d_w) * d_x, each row adding its terms in block order.  A unit
// is `ipw` items (rows, or gate/value row pairs of the SiLU gate) of one batch row.

struct Q8Geom {
  int K, nb, b, part, i0, ni, NR, total, ts;
};

__device__ __forceinline__ Q8Geom q8_geom(int K, int items, int ipw, int parts, bool silu, int unit) {
  Q8Geom g;
  g.K = K;
  g.nb = K / 32;
  g.b = unit / parts;
  g.part = unit - g.b * parts;
  g.i0 = g.part * ipw;
  g.ni = min(ipw, items - g.i0);
  g.NR = silu ? 2 * g.ni : g.ni;
  g.total = g.NR * g.nb;
  g.ts = term_stride(ipw);
  return g;
}

// LDS of a Q8_0 / Q4_0 unit: xs [norm_scratch_floats(K)] f32 | xq [K] int8 | xdq [nb, padded to 4]
// f32 | xsum [nb, padded to 4] i32 (Q4_0) | T [2 ipw][q8_row_stride(nb)] f32 | Y [2 ipw] f32.
struct Q8Lds {
  float* xs;
  int8_t* xq;
  float* xdq;
  int* xsum;
  float* T;
  float* Y;
};

__device__ __forceinline__ Q8Lds q8_lds(unsigned char* smem, int K, int nb, int ipw) {
  Q8Lds l;
  l.xs = (float*)smem;
  l.xq = (int8_t*)(l.xs + norm_scratch_floats(K));
  l.xdq = (float*)(l.xq + K);
  l.xsum = (int*)(l.xdq + ((nb + 3) & ~3));
  l.T = (float*)(l.xsum + ((nb + 3) & ~3));
  l.Y = l.T + 2 * ipw * q8_row_stride(nb);
  return l;
}

// Row-wave part of Q8_0 GEMV item `item`: input row, norm, quantization, then (once the weight
// waves have written the terms) the ordered row sums and the epilogue.
template <int KP>
__device__ __forceinline__ void gemv_q8_rows(const GemvArgs& a, int unit, const int* spos, unsigned char* smem,
                                             RowSync& rs, unsigned item) {
  const Q8Geom g = q8_geom(a.L.in, gemv_items(a), a.ipw, a.parts, a.epi == EPI_SILU_GATE, unit);
  const Q8Lds l = q8_lds(smem, g.K, g.nb, a.ipw);
  constexpr int KU = chunk_slots(KP * kRowThreads);
  // rows wider than 4096 (row_slots 16) are never normalized (d_model <= 4096)
  constexpr bool kNorm = KP <= 8;
  NormW4<kNorm ? KU : 1> nwt;
  if (kNorm && a.norm != NORM_NONE) load_norm_weights4(a.norm, a.nw, a.nb, g.K, nwt);
  v4f v[KU];
  load_row4(a.x + (size_t)g.b * a.x_stride, g.K, v, &rs.ws->r_issued);
  const int p = (a.epi == EPI_QKV_ROPE || a.advance_pos ? spos[g.b] : 0);
  const EpiIn in = gemv_epi_prefetch(a, g.b, g.i0 + min((int)threadIdx.x, g.ni - 1), p);
  if constexpr (kNorm) {
    if (a.norm != NORM_NONE) norm_row4(v, g.K, a.norm, nwt, a.eps, l.xs, rs);
  }
  // the weight waves have read the previous item's quantized row
  lds_wait(&rs.ws->t_parts, item * kWeightWaves, &rs.ws->stop);
  quantize_row4(v, g.K, l.xq, l.xdq, a.L.fmt == FMT_Q4_0 ? l.xsum : nullptr);
  lds_signal(&rs.ws->xq_parts);
  // one thread per row adds the row's terms in block order once every term is written
  const bool many = g.NR > kWave;  // uniform
  if (many || threadIdx.x < kWave) {
    lds_wait(&rs.ws->t_parts, (item + 1) * kWeightWaves, &rs.ws->stop);
    if ((int)threadIdx.x < g.NR) l.Y[threadIdx.x] = ordered_row_sum(l.T, q8_row_stride(g.nb), threadIdx.x, g.nb);
  }
  if (many) {
    rs.sync();
  } else {
    if (threadIdx.x >= kWave) return;
    wave_lds_fence();
  }
  gemv_finish(a, g.b, g.part, g.i0, g.ni, p, in, l.Y);
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Weight-wave state of one item: the item's geometry and this thread's weight blocks.
struct WItem {
  Q8Geom g;
  int ipw;
  int maxb;
  int q4;  // Q4_0 weights: one 16-byte load of codes per block (wa)
  v4i wa[kWBlocks], wb[kWBlocks];
  uint32_t wd[kWBlocks];
};

// Requests this weight-wave thread's blocks of unit `unit` of GEMV phase `ph` (descriptor read
// with scalar loads).  Block k of thread w is index w + 512 k = r * nb + blk of the unit.
// The geometry the requests need: K, items (output rows, or gate/value pairs: then also the offset
// of the value rows), rows per unit, units per batch row, blocks per thread, the epilogue kind.
__device__ __forceinline__ void w_issue_at(const int8_t* wq, const uint16_t* sc, int K, int items, int ipw, int parts,
                                           int maxb, int epi, int unit, WItem& it, int q4 = 0) {
  const int ff_hidden = items;  // read by gemv_phys_row for the SiLU gate only, where items = ff_hidden
  it.ipw = ipw;
  it.maxb = maxb;
  it.q4 = q4;
  it.g = q8_geom(K, items, ipw, parts, epi == EPI_SILU_GATE, unit);
  const int nb = it.g.nb;
  const int w = threadIdx.x - kRowThreads;
  int r = w / nb, blk = w - r * nb;
  const int dr = kWeightThreads / nb, db = kWeightThreads - dr * nb;
#pragma unroll
  for (int k = 0; k < kWBlocks; ++k) {
    if (k >= it.maxb) break;  // uniform
    if (w + k * kWeightThreads < it.g.total) {
      const size_t row = (size_t)gemv_phys_row(epi, ff_hidden, it.g.i0, it.g.ni, r);
      if (q4) {  // uniform
        it.wa[k] = ldg_stream((const v4i*)(wq + row * (K / 2) + (size_t)blk * 16));
      } else {
        const v4i* wp = (const v4i*)(wq + row * K + (size_t)blk * 32);
        it.wa[k] = ldg_stream(wp);
        it.wb[k] = ldg_stream(wp + 1);
      }
      it.wd[k] = ldg_stream(sc + row * nb + blk);
    }
    r += dr;
    blk += db;
    if (blk >= nb) {
      blk -= nb;
      ++r;
    }
  }
}

__device__ __forceinline__ void w_issue(const Phase* ph, int unit, WItem& it) {
  const int epi = ld_const(&ph->g.epi);
  const int items = epi == EPI_SILU_GATE ? ld_const(&ph->g.ff_hidden) : ld_const(&ph->g.L.out);
  w_issue_at((const int8_t*)ld_const(&ph->g.L.w), (const uint16_t*)ld_const(&ph->g.L.scale), ld_const(&ph->g.L.in),
             items, ld_const(&ph->g.ipw), ld_const(&ph->g.parts), ld_const(&ph->g.maxb), epi, unit, it,
             ld_const(&ph->g.L.fmt) == FMT_Q4_0);
}

// The item's block terms T[r][blk] = ((f32)(sum qw * qx) * d_w) * d_x into LDS; for Q4_0 weights
// qw = code - 8, and the exact sum is sum code * qx - 8 sum qx.
__device__ __forceinline__ void w_terms(const WItem& it, unsigned char* smem) {
  const Q8Lds l = q8_lds(smem, it.g.K, it.g.nb, it.ipw);
  const int rs = q8_row_stride(it.g.nb);
  const int nb = it.g.nb;
  const int w = threadIdx.x - kRowThreads;
  int r = w / nb, blk = w - r * nb;
  const int dr = kWeightThreads / nb, db = kWeightThreads - dr * nb;
#pragma unroll
  for (int k = 0; k < kWBlocks; ++k) {
    if (k >= it.maxb) break;  // uniform
    if (w + k * kWeightThreads < it.g.total) {
      const v4i xa = *(const v4i*)(l.xq + blk * 32);
      const v4i xb = *(const v4i*)(l.xq + blk * 32 + 16);
      int s;
      if (it.q4) {  // uniform: low nibbles are elements 0-15, high nibbles 16-31
        const int m = 0x0F0F0F0F;
        s = sdot4(it.wa[k].x & m, xa.x, 0);
        s = sdot4(it.wa[k].y & m, xa.y, s);
        s = sdot4(it.wa[k].z & m, xa.z, s);
        s = sdot4(it.wa[k].w & m, xa.w, s);
        s = sdot4((it.wa[k].x >> 4) & m, xb.x, s);
        s = sdot4((it.wa[k].y >> 4) & m, xb.y, s);
        s = sdot4((it.wa[k].z >> 4) & m, xb.z, s);
        s = sdot4((it.wa[k].w >> 4) & m, xb.w, s);
        s -= 8 * l.xsum[blk];
      } else {
        s = sdot4(it.wa[k].x, xa.x, 0);
        s = sdot4(it.wa[k].y, xa.y, s);
        s = sdot4(it.wa[k].z, xa.z, s);
        s = sdot4(it.wa[k].w, xa.w, s);
        s = sdot4(it.wb[k].x, xb.x, s);
        s = sdot4(it.wb[k].y, xb.y, s);
        s = sdot4(it.wb[k].z, xb.z, s);
        s = sdot4(it.wb[k].w, xb.w, s);
      }
      const float t = (float)s * f16_to_f32((uint16_t)it.wd[k]);
      l.T[r * rs + blk] = t * l.xdq[blk];
    }
    r += dr;
    blk += db;
    if (blk >= nb) {
      blk -= nb;
      ++r;
    }
  }
}

// ---- Q4K GEMV ------------------------------------------------------------------------------------
// Candle's Q4K x Q8K CPU matmul (BlockQ4K::vec_dot_unopt against the activation row quantized by
// BlockQ8K::from_float).  Per weight super-block and row, the i32 lane sums
// aux[l] = sum over sub-blocks s of sc_s * (sum over g of q4 * q8 at element 32 s + 8 g + l) and
// the min term sumi = sum over 16-groups j of bsum_j * m_{j/2} are exact; the row adds
// (d_w * d_x) * (f32)aux[l] to lane sum l and subtracts (dmin_w * d_x) * (f32)sumi, super-block
// by super-block, and ends with min_sum + (((s_0 + s_1) + ...) + s_7).  The weight waves write
// the nine f32 terms of every (row, super-block) into LDS; the row waves add them in order.

// LDS of a Q4K unit: xs [norm_scratch_floats(K)] f32 | xq [K] int8 (lane-grouped) | xd [nb, padded to 4] f32 |
// bs [nb][16] i32 | T [nb][ts][kQ4TermStride] f32 (16-byte aligned) | Y [2 ipw] f32.
// A (row, super-block)'s nine terms are contiguous, so that they move as three 16-byte words.
struct Q4Lds {
  float* xs;
  int8_t* xq;
  float* xd;
  int* bs;
  float* T;
  float* Y;
};

__device__ __forceinline__ Q4Lds q4_lds(unsigned char* smem, int K, int nb, int ts) {
  Q4Lds l;
  l.xs = (float*)smem;
  l.xq = (int8_t*)(l.xs + norm_scratch_floats(K));
  l.xd = (float*)(l.xq + K);
  l.bs = (int*)(l.xd + ((nb + 3) & ~3));
  l.T = (float*)(((size_t)(l.bs + nb * 16) + 15) & ~(size_t)15);
  l.Y = l.T + nb * ts * kQ4TermStride;
  return l;
}

__device__ __forceinline__ Q8Geom q4_geom(int K, int items, int ipw, int parts, bool silu, int unit) {
  Q8Geom g = q8_geom(K, items, ipw, parts, silu, unit);
  g.nb = K / 256;
  g.total = g.NR * g.nb;
  return g;
}

// Byte offset of element e (< 32) of a 32-value group in the lane-grouped order.
__host__ __device__ constexpr int q4k_lane_pos(int e) { return ((e & 7) << 2) | (e >> 3); }

// BlockQ8K::from_float of the chunked row (chunks c = t + 512 u of 4 elements): per 256 values,
// mx = the value of largest magnitude (the first one on ties), iscale = -128 / mx,
// q = min(round(iscale * x), 127), d = 1 / iscale (all zero when the block is); bs = sums of 16
// consecutive quants.  A super-block is the 64 chunks of one wave and slot, so its maximum and
// first index stay within the wave (no barrier); a 16-sum is the chunks of 4 lanes.
template <int KU>
__device__ __forceinline__ void q8k_quantize4(const v4f (&v)[KU], int K, int8_t* xq, float* xd, int* bs) {
  const int nc = K / 4, lane = threadIdx.x % kWave;
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int c = threadIdx.x + u * kRowThreads;
    if (c - lane >= nc) break;  // uniform per wave (nc is a multiple of 64)
    const uint32_t a0 = __float_as_uint(fabsf(v[u].x)), a1 = __float_as_uint(fabsf(v[u].y));
    const uint32_t a2 = __float_as_uint(fabsf(v[u].z)), a3 = __float_as_uint(fabsf(v[u].w));
    const uint32_t lm = max(max(a0, a1), max(a2, a3));
    const uint32_t hm = half_max_bits(lm);
    const uint32_t best = max((uint32_t)__builtin_amdgcn_readlane((int)hm, 0), (uint32_t)__builtin_amdgcn_readlane((int)hm, 32));
    // the first element of the largest magnitude: the first lane holding one, its first element
    const int first = (int)__builtin_ctzll(__ballot(lm == best));
    const float own = a0 == best ? v[u].x : (a1 == best ? v[u].y : (a2 == best ? v[u].z : v[u].w));
    const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(own), first));
    const float iscale = best != 0 ? -128.0f / mx : 0.0f;
    const float xs[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
    int qs = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = best != 0 ? sat_i8(fminf(roundf(iscale * xs[k]), 127.0f)) : 0;
      qs += q;
      const int i = 4 * c + k;
      xq[(i & ~31) | q4k_lane_pos(i & 31)] = (int8_t)q;
    }
    qs += __builtin_amdgcn_update_dpp(0, qs, 0xB1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
    qs += __builtin_amdgcn_update_dpp(0, qs, 0x4E, 0xf, 0xf, false);  // quad_perm [2, 3, 0, 1]
    if ((c & 3) == 0) bs[c >> 2] = qs;
    if (lane == 0) xd[c >> 6] = best != 0 ? 1.0f / iscale : 0.0f;
  }
}

// acc over the nine term rows of row r: lane sums l < 8 in super-block order, the min term
// subtracted in super-block order, then min_sum + (((s_0 + s_1) + ...) + s_7).
__device__ __forceinline__ float q4k_row_sum(const float* T, int ts, int r, int nb) {
  const float* t = T + (size_t)r * kQ4TermStride;
  float s[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  float mins = 0.0f;
  for (int blk = 0; blk < nb; ++blk) {
    const float* tb = t + (size_t)blk * ts * kQ4TermStride;
    const float4 a = *(const float4*)tb, b = *(const float4*)(tb + 4);
    const float v[kQ4Terms] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, tb[8]};
#pragma unroll
    for (int c = 0; c < 8; ++c) s[c] = s[c] + v[c];
    mins = mins - v[8];
  }
  float s8 = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) s8 = s8 + s[c];
  return mins + s8;
}

// Row-wave part of Q4K GEMV item `item` (the Q8_0 item's flow with the Q8K quantizer).
template <int KP>
__device__ __forceinline__ void gemv_q4k_rows(const GemvArgs& a, int unit, const int* spos, unsigned char* smem,
                                              RowSync& rs, unsigned item) {
  const Q8Geom g = q4_geom(a.L.in, gemv_items(a), a.ipw, a.parts, a.epi == EPI_SILU_GATE, unit);
  const Q4Lds l = q4_lds(smem, g.K, g.nb, g.ts);
  constexpr int KU = chunk_slots(KP * kRowThreads);
  constexpr bool kNorm = KP <= 8;  // rows wider than 4096 are never normalized (d_model <= 4096)
  NormW4<kNorm ? KU : 1> nwt;
  if (kNorm && a.norm != NORM_NONE) load_norm_weights4(a.norm, a.nw, a.nb, g.K, nwt);
  v4f v[KU];
  load_row4(a.x + (size_t)g.b * a.x_stride, g.K, v, &rs.ws->r_issued);
  const int p = (a.epi == EPI_QKV_ROPE || a.advance_pos ? spos[g.b] : 0);
  const EpiIn in = gemv_epi_prefetch(a, g.b, g.i0 + min((int)threadIdx.x, g.ni - 1), p);
  if constexpr (kNorm) {
    if (a.norm != NORM_NONE) norm_row4(v, g.K, a.norm, nwt, a.eps, l.xs, rs);
  }
  // the weight waves have read the previous item's quantized row
  lds_wait(&rs.ws->t_parts, item * kWeightWaves, &rs.ws->stop);
  q8k_quantize4(v, g.K, l.xq, l.xd, l.bs);
  lds_signal(&rs.ws->xq_parts);
  const bool many = g.NR > kWave;  // uniform
  if (many || threadIdx.x < kWave) {
    lds_wait(&rs.ws->t_parts, (item + 1) * kWeightWaves, &rs.ws->stop);
    if ((int)threadIdx.x < g.NR) l.Y[threadIdx.x] = q4k_row_sum(l.T, g.ts, threadIdx.x, g.nb);
  }
  if (many) {
    rs.sync();
  } else {
    if (threadIdx.x >= kWave) return;
    wave_lds_fence();
  }
  gemv_finish(a, g.b, g.part, g.i0, g.ni, p, in, l.Y);
}

// Weight-wave state of one Q4K item: per super-block slot the 16-byte header and the 128 quant
// bytes.
struct WItemQ4 {
  Q8Geom g;
  int ipw;
  int maxb;
  v4i h[kQ4Blocks];
  v4i q[kQ4Blocks][8];
};

__device__ __forceinline__ void w_issue_q4k_at(const unsigned char* wb, int K, int items, int ipw, int parts, int maxb,
                                               int epi, int unit, WItemQ4& it) {
  const int ff_hidden = items;  // read by gemv_phys_row for the SiLU gate only, where items = ff_hidden
  it.ipw = ipw;
  it.maxb = maxb;
  it.g = q4_geom(K, items, ipw, parts, epi == EPI_SILU_GATE, unit);
  const int nb = it.g.nb;
  const int w = threadIdx.x - kRowThreads;
  int r = w / nb, blk = w - r * nb;
  const int dr = kWeightThreads / nb, db = kWeightThreads - dr * nb;
#pragma unroll
  for (int k = 0; k < kQ4Blocks; ++k) {
    if (k >= it.maxb) break;  // uniform
    if (w + k * kWeightThreads < it.g.total) {
      const size_t row = (size_t)gemv_phys_row(epi, ff_hidden, it.g.i0, it.g.ni, r);
      const v4i* bp = (const v4i*)(wb + (row * nb + blk) * 144);
      it.h[k] = ldg(bp);
#pragma unroll
      for (int j = 0; j < 8; ++j) it.q[k][j] = ldg_stream(bp + 1 + j);
    }
    r += dr;
    blk += db;
    if (blk >= nb) {
      blk -= nb;
      ++r;
    }
  }
}

__device__ __forceinline__ void w_issue_q4k(const Phase* ph, int unit, WItemQ4& it) {
  const int epi = ld_const(&ph->g.epi);
  const int items = epi == EPI_SILU_GATE ? ld_const(&ph->g.ff_hidden) : ld_const(&ph->g.L.out);
  w_issue_q4k_at((const unsigned char*)ld_const(&ph->g.L.w), ld_const(&ph->g.L.in), items, ld_const(&ph->g.ipw),
                 ld_const(&ph->g.parts), ld_const(&ph->g.maxb), epi, unit, it);
}

__device__ __forceinline__ int q4k_lane(const v4i& a, const v4i& b, int l) {
  switch (l) {
    case 0: return a.x;
    case 1: return a.y;
    case 2: return a.z;
    case 3: return a.w;
    case 4: return b.x;
    case 5: return b.y;
    case 6: return b.z;
    default: return b.w;
  }
}

// The item's terms: T[blk][l][r] = (d_w * d_x) * (f32)aux[l] for l < 8 and
// T[blk][8][r] = (dmin_w * d_x) * (f32)sumi.
__device__ __forceinline__ void w_terms_q4k(const WItemQ4& it, unsigned char* smem) {
  const Q4Lds l = q4_lds(smem, it.g.K, it.g.nb, it.g.ts);
  const int nb = it.g.nb;
  const int w = threadIdx.x - kRowThreads;
  int r = w / nb, blk = w - r * nb;
  const int dr = kWeightThreads / nb, db = kWeightThreads - dr * nb;
#pragma unroll
  for (int k = 0; k < kQ4Blocks; ++k) {
    if (k >= it.maxb) break;  // uniform
    if (w + k * kWeightThreads < it.g.total) {
      // get_scale_min_k4 for all eight sub-blocks, four bytes at a time
      const uint32_t s0 = (uint32_t)it.h[k].y, s1 = (uint32_t)it.h[k].z, s2 = (uint32_t)it.h[k].w;
      const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, mn_lo = s1 & 0x3F3F3F3Fu;
      const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | (((s0 >> 6) & 0x03030303u) << 4);
      const uint32_t mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | (((s1 >> 6) & 0x03030303u) << 4);
      const int* xw = (const int*)(l.xq + blk * 256);
      int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t scw = j < 2 ? sc_lo : sc_hi;
        const int sa = (int)((scw >> (16 * (j & 1))) & 0xFF);      // sub-block 2 j
        const int sb = (int)((scw >> (16 * (j & 1) + 8)) & 0xFF);  // sub-block 2 j + 1
        const v4i xa0 = *(const v4i*)(xw + 16 * j), xa1 = *(const v4i*)(xw + 16 * j + 4);
        const v4i xb0 = *(const v4i*)(xw + 16 * j + 8), xb1 = *(const v4i*)(xw + 16 * j + 12);
#pragma unroll
        for (int ln = 0; ln < 8; ++ln) {
          const uint32_t dw = (uint32_t)q4k_lane(it.q[k][2 * j], it.q[k][2 * j + 1], ln);
          const int lo = (int)(dw & 0x0F0F0F0Fu), hi = (int)((dw >> 4) & 0x0F0F0F0Fu);
          aux[ln] += sa * sdot4(lo, q4k_lane(xa0, xa1, ln), 0) + sb * sdot4(hi, q4k_lane(xb0, xb1, ln), 0);
        }
      }
      const int* bs = l.bs + blk * 16;
      int sumi = 0;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int s = jj / 2;
        const uint32_t mw = s < 4 ? mn_lo : mn_hi;
        sumi += bs[jj] * (int)((mw >> (8 * (s & 3))) & 0xFF);
      }
      const float xd = l.xd[blk];
      const uint32_t hd = (uint32_t)it.h[k].x;
      const float d = f16_to_f32((uint16_t)(hd & 0xFFFF)) * xd;
      const float dm = f16_to_f32((uint16_t)(hd >> 16)) * xd;
      float* T = l.T + ((size_t)blk * it.g.ts + r) * kQ4TermStride;
      *(float4*)T = float4{d * (float)aux[0], d * (float)aux[1], d * (float)aux[2], d * (float)aux[3]};
      *(float4*)(T + 4) = float4{d * (float)aux[4], d * (float)aux[5], d * (float)aux[6], d * (float)aux[7]};
      T[8] = dm * (float)sumi;
    }
    r += dr;
    blk += db;
    if (blk >= nb) {
      blk -= nb;
      ++r;
    }
  }
}

// GEMV phases whose units the row waves and the weight waves share (quantized weights).
__device__ __forceinline__ bool is_split_gemv(const Phase* ph) {
  if (ld_const(&ph->kind) != PH_GEMV) return false;
  const int fmt = ld_const(&ph->g.L.fmt);
  return fmt == FMT_Q8_0 || fmt == FMT_Q4_0 || fmt == FMT_Q4K || fmt == FMT_F32C || fmt == FMT_BF16C;
}

// ---- batched Q8_0 GEMM (lockstep batches; row waves) ----------------------------------------------
// The same arithmetic as the Q8_0 GEMV, with the int8 block dots of a tile of 32 output rows x 64
// batch rows done by v_mfma_i32_16x16x32_i8 (one instruction per 16 x 16 sub-tile and block:
// K = 32 is exactly one block).  Per block and output, ((f32)dot * d_w) * d_x is added to the
// output's sum in block order, as in the GEMV.  The activations are quantized once per batch
// row by a PH_QUANT phase before the GEMM phase.
//
// Operand layouts of v_mfma_i32_16x16x32_i8 (one 64-lane wave): lane l supplies row l % 16 of A
// (and column l % 16 of B) at k = 8 (l / 16) .. 8 (l / 16) + 7 as 8 packed int8; it receives
// D[4 (l / 16) + i][l % 16], i = 0 .. 3.

// Quantizes x[b] (after the norm, if any) into xq[b] / xdq[b]; unit = batch row.
template <int KP>
__device__ __forceinline__ void quant_unit(const GemvArgs& a, int b, unsigned char* smem, RowSync& rs) {
  const int K = a.L.in, nb = K / 32;
  float* xs = (float*)smem;  // norm scratch
  int8_t* xq = (int8_t*)(xs + norm_scratch_floats(K));
  float* xdq = (float*)(xq + K);
  constexpr int KU = chunk_slots(KP * kRowThreads);
  constexpr bool kNorm = KP <= 8;
  NormW4<kNorm ? KU : 1> nwt;
  if (kNorm && a.norm != NORM_NONE) load_norm_weights4(a.norm, a.nw, a.nb, K, nwt);
  v4f v[KU];
  load_row4(a.x + (size_t)b * a.x_stride, K, v);
  if constexpr (kNorm) {
    if (a.norm != NORM_NONE) norm_row4(v, K, a.norm, nwt, a.eps, xs, rs);
  }
  quantize_row4(v, K, xq, xdq);
  rs.sync();
  // chunk-major: the 128-byte chunk c of every batch row is one contiguous run of B x 128 bytes, so
  // that the GEMM units' concurrent reads of a chunk spread over the L2 channels
  for (int i = threadIdx.x; i < K / 4; i += kRowThreads) {
    const int c = i / 32, w = i % 32;
    st_co((uint32_t*)(a.xq + ((size_t)c * a.B + b) * 128) + w, ((const uint32_t*)xq)[i]);
  }
  for (int i = threadIdx.x; i < nb; i += kRowThreads) st_co(a.xdq + (size_t)b * nb + i, xdq[i]);
}

typedef long v_i8x8;

// One GEMM unit: output rows of row tile `part`, batch rows of batch tile `bt`.  K is streamed in
// chunks of kGemmChunk blocks through a ring of kGemmStages LDS stages, filled by direct
// global -> LDS loads issued kGemmStages - 1 chunks ahead (W and X rows with their 16-byte
// segments XOR-swizzled by row, so that the MFMA operand reads spread over the banks).  Wave w
// computes the 16 x 16 sub-tile of tile rows 16 (w / 4) .. and batch rows 16 (w % 4) ..; the
// results meet in LDS for the epilogues.
#define SVL_LDS __attribute__((address_space(3)))

// Lane i's BYTES at src land at dst_wave_base + i * BYTES (dst is wave-uniform); a 2-byte load
// fills the low half of the 4-byte slot dst_wave_base + 4 i.  CO: coherent (agent scope) load, for
// data written by other workgroups during the launch.
template <int BYTES, bool CO>
__device__ __forceinline__ void lds_dma(const void* src, unsigned char* dst_wave_base) {
  const SVL_GLOBAL void* g = (const SVL_GLOBAL void*)src;
  SVL_LDS void* l = (SVL_LDS void*)dst_wave_base;
  if constexpr (BYTES == 16) {
    if constexpr (CO) __builtin_amdgcn_global_load_lds(g, l, 16, 0, 16);
    else __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
  } else if constexpr (BYTES == 4) {
    if constexpr (CO) __builtin_amdgcn_global_load_lds(g, l, 4, 0, 16);
    else __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0);
  } else {
    static_assert(BYTES == 2, "2, 4 or 16 bytes per lane");
    if constexpr (CO) __builtin_amdgcn_global_load_lds(g, l, 2, 0, 16);
    else __builtin_amdgcn_global_load_lds(g, l, 2, 0, 0);
  }
}

struct GemmStage {
  unsigned char* w;   // [kTileRows][128] int8, swizzled
  unsigned char* x;   // [kTileBatch][128] int8, swizzled
  uint32_t* dw;       // [kTileRows][kGemmChunk / 2] f16 pairs
  float* dx;          // [kTileBatch][kGemmChunk]
};

__device__ __forceinline__ GemmStage gemm_stage(unsigned char* smem, int s) {
  unsigned char* base = smem + kTileRows * kTileBatch * 4 + s * kGemmStageBytes;
  GemmStage g;
  g.w = base;
  g.x = base + kTileRows / 8 * kGemmGroupBytes;
  g.dw = (uint32_t*)(g.x + kTileBatch / 8 * kGemmGroupBytes);
  g.dx = (float*)(g.dw + kTileRows * kGemmChunk / 2);
  return g;
}

// Byte offset of 16-byte segment `seg` of row j in a swizzled 128-byte row.
__device__ __forceinline__ int swz(int j, int seg) {
  return j * 128 + (j >> 3) * 128 + ((seg ^ (j & 7)) << 4);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t u4c(const u32x4& v, int q) { return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w; }

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(size_t)(const SVL_LDS void*)p; }

// RowSync::sync for the GEMM loop, its LDS accesses written out so that the compiler does not
// wait for the direct loads in flight before them (it cannot tell the counters from the stages).
// Prior LDS reads of the wave have completed (gemm_wait waits for them).
__device__ __forceinline__ void gemm_sync(RowSync& rs) {
  if (rs.hw) {
    asm volatile("s_barrier" : : : "memory");
    return;
  }
  const uint32_t ctr = lds_addr(&rs.ws->r_arrive), stop = lds_addr(&rs.ws->stop);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    const uint32_t one = 1;
    asm volatile("ds_add_u32 %0, %1" : : "v"(ctr), "v"(one) : "memory");
  }
  rs.epoch += kRowWaves;
  unsigned spins = 0;
  for (;;) {
    uint32_t v, st;
    asm volatile(
        "ds_read_b32 %0, %2\n\t"
        "ds_read_b32 %1, %3\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v), "=&v"(st)
        : "v"(ctr), "v"(stop)
        : "memory");
    v = __builtin_amdgcn_readfirstlane(v);
    st = __builtin_amdgcn_readfirstlane(st);
    if ((int)(v - rs.epoch) >= 0 || st) break;
    if (++spins > kLdsSpinLimit) {
      const uint32_t one = 1;
      asm volatile("ds_write_b32 %0, %1" : : "v"(stop), "v"(one) : "memory");
      break;
    }
  }
}

struct GemmOps {
  v_i8x8 a[4], b[4];  // A (weight) and B (activation) fragments of blocks 0-3
  u32x4 dw[2];        // weight scales as f16 pairs: rows 4g, 4g + 1, then rows 4g + 2, 4g + 3
  v4f dx;             // activation scales of the lane's column, blocks 0-3
};

struct GemmAddr {
  uint32_t a[4], b[4], w, x;
};

__device__ __forceinline__ GemmAddr gemm_addr(const GemmStage& st, int ja, int jb, int g, int r0) {
  GemmAddr p;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int seg = 2 * kk + g / 2, inner = 8 * (g & 1);
    p.a[kk] = lds_addr(st.w) + swz(ja, seg) + inner;
    p.b[kk] = lds_addr(st.x) + swz(jb, seg) + inner;
  }
  p.w = lds_addr(st.dw) + (r0 + 4 * g) * 8;
  p.x = lds_addr(st.dx) + jb * (kGemmChunk * 4);
  return p;
}

// One lane's operands of a chunk, issued by gemm_issue and completed by gemm_wait, whose operands
// are the same registers: in between the wave computes the chunk before.  Direct loads land in the
// LDS stages meanwhile, which is why the reads are written out: the compiler would wait for every
// direct load in flight before a read it issued itself.
__device__ __forceinline__ void gemm_issue(const GemmAddr& p, GemmOps& o) {
  asm volatile(
      "ds_read_b64 %0, %11\n\t"
      "ds_read_b64 %1, %12\n\t"
      "ds_read_b64 %2, %13\n\t"
      "ds_read_b64 %3, %14\n\t"
      "ds_read_b64 %4, %15\n\t"
      "ds_read_b64 %5, %16\n\t"
      "ds_read_b64 %6, %17\n\t"
      "ds_read_b64 %7, %18\n\t"
      "ds_read_b128 %8, %19\n\t"
      "ds_read_b128 %9, %19 offset:16\n\t"
      "ds_read_b128 %10, %20"
      : "=&v"(o.a[0]), "=&v"(o.a[1]), "=&v"(o.a[2]), "=&v"(o.a[3]), "=&v"(o.b[0]), "=&v"(o.b[1]), "=&v"(o.b[2]),
        "=&v"(o.b[3]), "=&v"(o.dw[0]), "=&v"(o.dw[1]), "=&v"(o.dx)
      : "v"(p.a[0]), "v"(p.a[1]), "v"(p.a[2]), "v"(p.a[3]), "v"(p.b[0]), "v"(p.b[1]), "v"(p.b[2]), "v"(p.b[3]),
        "v"(p.w), "v"(p.x)
      : "memory");
}

// The registers are operands so that they stay where the reads land until the wait.
__device__ __forceinline__ void gemm_wait(const GemmOps& o) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               :
               : "v"(o.a[0]), "v"(o.a[1]), "v"(o.a[2]), "v"(o.a[3]), "v"(o.b[0]), "v"(o.b[1]), "v"(o.b[2]),
                 "v"(o.b[3]), "v"(o.dw[0]), "v"(o.dw[1]), "v"(o.dx)
               : "memory");
}

// The block products of a chunk (independent MFMAs).
__device__ __forceinline__ void gemm_mfma(const GemmOps& o, v4i (&cc)[kGemmChunk]) {
#pragma unroll
  for (int kk = 0; kk < kGemmChunk; ++kk)
    cc[kk] = __builtin_amdgcn_mfma_i32_16x16x32_i8(o.a[kk], o.b[kk], v4i{0, 0, 0, 0}, 0, 0, 0);
}

// The chunk's terms ((f32)dot * d_w) * d_x added to the lane's four outputs in block order; nk
// (uniform) blocks of the chunk are in K.
__device__ __forceinline__ void gemm_terms(const GemmOps& o, const v4i (&cc)[kGemmChunk], int nk, float (&acc)[4]) {
  const float dxs[4] = {o.dx.x, o.dx.y, o.dx.z, o.dx.w};
#pragma unroll
  for (int kk = 0; kk < kGemmChunk; ++kk) {
    if (kk >= nk) break;  // uniform
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t dwp = u4c(o.dw[i >> 1], (i & 1) * 2 + (kk >> 1));
      const float dw = f16_to_f32((uint16_t)(kk & 1 ? dwp >> 16 : dwp & 0xFFFF));
      const float t = (float)cc[kk][i] * dw;
      acc[i] = acc[i] + t * dxs[kk];
    }
  }
}

template <int TR>  // tile rows: 32 (waves 0-7 compute) or 16 (waves 0-3 compute)
__device__ __forceinline__ void qgemm_unit(const GemvArgs& a, int unit, const int* spos, unsigned char* smem,
                                           RowSync& rs) {
  const int K = a.L.in, nb = K / 32;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int part = unit % a.parts, bt = unit / a.parts;
  const int i0 = part * a.ipw;
  const int ni = min(a.ipw, gemv_items(a) - i0);
  const int NR = silu ? 2 * ni : ni;  // tile rows in use
  const int b0 = bt * kTileBatch;
  const int nbat = min(kTileBatch, a.B - b0);
  float* Y = (float*)smem;            // [kTileRows][kTileBatch]
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  // ---- loads of one chunk: wave w brings X rows 8w..8w+7.  TR = 32: waves 0-3 W rows 8w..8w+7,
  // wave 4 the weight scales (lane l: the f16 pair of blocks 2 (l % 2), + 1 of row l / 2), waves
  // 6-7 the activation scales of batch rows 32 (w - 6) .. (two loads).  TR = 16: waves 0-1 W rows
  // 8w..8w+7, wave 2 the weight scales, waves 4-7 the activation scales of batch rows 16 (w - 4) ..
  // Rows past the tile load the last row in use; blocks past K load the last block (pair) in K
  // (their results are never used).  The pairs are 4-byte aligned: K / 32 is even on this path.
  const int lrow = 8 * wave + lane / 8, lslot = lane % 8;
  const int8_t* xsrc = a.xq + (size_t)(b0 + min(lrow, nbat - 1)) * 128;  // + chunk * B * 128
  const int8_t* wsrc = (const int8_t*)a.L.w +
                       (size_t)gemv_phys_row(a.epi, a.ff_hidden, i0, ni, min(wave < TR / 8 ? lrow : 0, NR - 1)) * K;
  const int srow = lane / 2, sblk = 2 * (lane % 2);  // f16 pairs: blocks sblk, sblk + 1 of row srow
  const uint16_t* dwsrc = a.L.scale + (size_t)gemv_phys_row(a.epi, a.ff_hidden, i0, ni, min(srow, NR - 1)) * nb;
  const int xrow0 = (TR == 32 ? 32 * (wave & 1) : 16 * (wave & 3)) + lane / 4;
  const float* dxsrc0 = a.xdq + (size_t)(b0 + min(xrow0, nbat - 1)) * nb;
  const float* dxsrc1 = a.xdq + (size_t)(b0 + min(xrow0 + 16, nbat - 1)) * nb;
  auto issue = [&](int c) {
    const GemmStage st = gemm_stage(smem, c % kGemmStages);
    const int seg = lslot ^ (lrow & 7);
    const int off = min(128 * c + 16 * seg, K - 16);
    lds_dma<16, true>(xsrc + (size_t)(off / 128) * a.B * 128 + off % 128, st.x + wave * kGemmGroupBytes);
    const int k = min(kGemmChunk * c + sblk, nb - 2);  // weight scales
    const int kx = min(kGemmChunk * c + lane % 4, nb - 1);                  // activation scales
    if constexpr (TR == 32) {
      if (wave < 4) {
        lds_dma<16, false>(wsrc + off, st.w + wave * kGemmGroupBytes);
      } else if (wave < 6) {
        if (wave == 4) lds_dma<4, false>(dwsrc + k, (unsigned char*)st.dw);
      } else {
        lds_dma<4, true>(dxsrc0 + kx, (unsigned char*)st.dx + (wave - 6) * 512);
        lds_dma<4, true>(dxsrc1 + kx, (unsigned char*)st.dx + (wave - 6) * 512 + 256);
      }
    } else {
      if (wave < 2) lds_dma<16, false>(wsrc + off, st.w + wave * kGemmGroupBytes);
      else if (wave == 2) lds_dma<4, false>(dwsrc + k, (unsigned char*)st.dw);
      else if (wave >= 4) lds_dma<4, true>(dxsrc0 + kx, (unsigned char*)st.dx + (wave - 4) * 256);
    }
  };
  const int nch = (nb + kGemmChunk - 1) / kGemmChunk;
  constexpr int S = kSyncChunks, AHEAD = kGemmStages - kSyncChunks;  // chunks per sync, chunks issued ahead
  static_assert(S == 2 && kGemmStages >= 3 * S, "a barrier certifies the interval and the next one");
  __builtin_amdgcn_s_waitcnt(kVmWait0);  // no older stores interleave with the counted loads
  for (int c = 0; c < min(AHEAD, nch); ++c) issue(c);
  const int r0 = 16 * (wave / 4), c0 = 16 * (wave % 4);
  const int g = lane / 16, ja = r0 + lane % 16, jb = c0 + lane % 16;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // Chunk k is computed from the registers its reads landed in while the reads of chunk k + 1 are in
  // flight (even chunks in `ra`, odd ones in `rb`).  The barrier of interval c certifies the chunks
  // up to c + 3, so the read-ahead of c + 2 may be issued before the next barrier.
  GemmOps ra, rb;
  auto chunk = [&](int k, GemmOps& cur, GemmOps& nxt) {
    if (k >= nch) return;  // uniform
    if (k + 1 < nch) gemm_issue(gemm_addr(gemm_stage(smem, (k + 1) % kGemmStages), ja, jb, g, r0), nxt);
    v4i cc[kGemmChunk];
    gemm_mfma(cur, cc);
    gemm_terms(cur, cc, min(kGemmChunk, nb - kGemmChunk * k), acc);  // uniform block count
    if (k + 1 < nch) gemm_wait(nxt);
  };
  for (int c = 0; c < nch; c += S) {
    // this wave's loads of chunks .. c + 3 have landed (later chunks may still be in flight)
    if (c + AHEAD <= nch) {
      if (TR == 32 && wave >= 6) __builtin_amdgcn_s_waitcnt(kVmWait3);
      else if (TR == 16 && wave == 3) __builtin_amdgcn_s_waitcnt(kVmWait1);
      else if (TR == 32 && wave == 5) __builtin_amdgcn_s_waitcnt(kVmWait1);
      else __builtin_amdgcn_s_waitcnt(kVmWait2);
    } else {
      __builtin_amdgcn_s_waitcnt(kVmWait0);
    }
    gemm_sync(rs);  // chunks .. c + 3 are in LDS everywhere; every wave is done reading the chunks before c
#pragma unroll
    for (int u = 0; u < S; ++u)
      if (c + AHEAD + u < nch) issue(c + AHEAD + u);
    if (wave < TR / 4) {  // uniform
      if (c == 0) {
        gemm_issue(gemm_addr(gemm_stage(smem, 0), ja, jb, g, r0), ra);
        gemm_wait(ra);
      }
      chunk(c, ra, rb);
      chunk(c + 1, rb, ra);
    }
  }
  if (wave < TR / 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) Y[(r0 + 4 * g + i) * kTileBatch + jb] = acc[i];
  }
  rs.sync();
  // epilogues: item t of the tile for batch row b0 + j
  for (int e = threadIdx.x; e < ni * nbat; e += kRowThreads) {
    const int t = e % ni, j = e / ni;
    const int b = b0 + j, row = i0 + t, p = a.epi == EPI_QKV_ROPE ? spos[b] : 0;
    const float y = Y[t * kTileBatch + j];
    const float yp = a.epi == EPI_QKV_ROPE ? Y[(t ^ 1) * kTileBatch + j] : 0.0f;
    const float yv = silu ? Y[(ni + t) * kTileBatch + j] : 0.0f;
    const EpiIn in = gemv_epi_prefetch(a, b, row, p);
    gemv_epilogue(a, b, row, p, in, y, yp, yv);
  }
  if (a.advance_pos && part == 0)
    for (int j = threadIdx.x; j < nbat; j += kRowThreads) st_co(a.pos + b0 + j, spos[b0 + j] + 1);
}

// ---- dense GEMV unit (row waves) -----------------------------------------------------------------
// The reference's matvec (SVL/nn/kernels/matvec.rs:239-246) with its 16-lane dot
// (kernels/mod.rs:66-91): 16 threads per row, thread i accumulating x[16c + i] * w[16c + i]
// with FMA over c, then the pairwise lane sum and the scalar tail.  32 rows per unit (16
// gate/value pairs for the SiLU gate).

template <bool BF16W, int KP>
__device__ __forceinline__ void gemv_dense_unit(const GemvArgs& a, int unit, const int* spos, unsigned char* smem,
                                                RowSync& rs) {
  const int K = a.L.in;
  const int b = unit / a.parts, part = unit % a.parts;
  const bool silu = a.epi == EPI_SILU_GATE;
  const int i0 = part * a.ipw;
  const int ni = min(a.ipw, gemv_items(a) - i0);
  const int NR = silu ? 2 * ni : ni;
  float* xs = (float*)smem;   // norm scratch, then the normalized row
  float* Y = xs + norm_scratch_floats(K);  // kRowThreads / 16
  constexpr bool kNorm = KP <= 8;  // rows wider than 4096 are never normalized (d_model <= 4096)
  NormW<kNorm ? KP : 1> nwt;
  if (kNorm && a.norm != NORM_NONE) load_norm_weights(a.norm, a.nw, a.nb, K, nwt);
  float v[KP];
  load_row(a.x + (size_t)b * a.x_stride, K, v);
  const int p = a.epi == EPI_QKV_ROPE || a.advance_pos ? spos[b] : 0;
  const EpiIn in = gemv_epi_prefetch(a, b, i0 + min((int)threadIdx.x, ni - 1), p);
  if constexpr (kNorm) {
    if (a.norm != NORM_NONE) {
      norm_regs(v, K, a.norm, nwt, a.eps, xs, rs);
      rs.sync();  // every read of xs by the statistics is done
    }
  }
  store_row(v, K, xs);
  rs.sync();
  const int g = threadIdx.x / 16, li = threadIdx.x % 16;
  const int chunks = K / 16;
  if (g < NR) {
    const size_t row = (size_t)gemv_phys_row(a.epi, a.ff_hidden, i0, ni, g);
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
    acc = row16_pairwise_sum(acc);
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
  rs.sync();
  gemv_finish(a, b, part, i0, ni, p, in, Y);
}

// ---- dense GEMV, chain-packed weights (row waves + weight waves) ---------------------------------
// The reference's matvec with its 16-lane dot (SVL/nn/kernels/matvec.rs:239-246,
// kernels/mod.rs:66-91): lane l of a row accumulates x[16 c + l] * w[16 c + l] over c with FMA,
// then the pairwise lane sum.  The weights are packed so that one weight-wave thread owns one
// lane chain of one row and reads it with 16-byte loads (FMT_F32C / FMT_BF16C); the row waves
// put the normalized input into LDS chain-major (xT[l][c], rows padded by 4 floats against bank
// conflicts).  A unit has up to 2 x 32 rows; the weight waves take them 32 at a time.

__device__ __forceinline__ int dense_chain_stride(int K) { return K / 16 + 4; }

struct DenseLds {
  float* xs;  // [norm_scratch_floats(K)] norm scratch
  float* xT;  // [16][K / 16 + 4]
  float* Y;   // [2 ipw]
};

// Without a norm on the input the norm scratch is left out.
__device__ __forceinline__ DenseLds dense_lds(unsigned char* smem, int K, bool norm) {
  DenseLds l;
  l.xs = (float*)smem;
  l.xT = l.xs + (norm ? norm_scratch_floats(K) : 0);
  l.Y = l.xT + 16 * dense_chain_stride(K);
  return l;
}

// A dense unit whose lane chains are longer than the loads a chain thread keeps in flight
// (kDenseBatch), whose rows are whole KiB and whose LDS with the rows staged stays within
// kDenseLdsCap stages them after Y [2 ipw]: every weight wave requests its share of the rows at
// once, instead of each row's 16 chain threads streaming their own loads (few rows per unit leave
// most weight threads idle).  Shorter chains already have their whole row in flight.
constexpr int kDenseLdsCap = 144 * 1024;
__host__ __device__ constexpr int dense_base_bytes(int K, int ipw, bool norm) {
  return (norm ? norm_scratch_floats(K) * 4 : 0) + 16 * (K / 16 + 4) * 4 + 2 * ipw * 4 + 64 + 16;
}
__host__ __device__ constexpr int dense_stage_bytes(int K, int ipw, int nr_max, bool bf16, bool norm) {
  return K / (bf16 ? 128 : 64) > kDenseBatch && (K * (bf16 ? 2 : 4)) % 1024 == 0 &&
                 dense_base_bytes(K, ipw, norm) + nr_max * K * (bf16 ? 2 : 4) <= kDenseLdsCap
             ? nr_max * K * (bf16 ? 2 : 4)
             : 0;
}
__device__ __forceinline__ unsigned char* dense_stage(const DenseLds& l, int ipw) {
  return (unsigned char*)(((size_t)(l.Y + 2 * ipw) + 15) & ~(size_t)15);
}

template <int KP>
__device__ __forceinline__ void store_row_chains(const float (&v)[KP], int K, float* xT) {
  const int stride = dense_chain_stride(K);
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    const int i = threadIdx.x + u * kRowThreads;
    if (i < K) xT[(i & 15) * stride + (i >> 4)] = v[u];
  }
}

// Row-wave part of dense item `item`: input row, norm, the chain-major copy for the weight waves,
// then (once they have written the row results) the epilogue.
template <int KP>
__device__ __forceinline__ void gemv_dense_rows(const GemvArgs& a, int unit, const int* spos, unsigned char* smem,
                                                RowSync& rs, unsigned item) {
  const int K = a.L.in;
  const Q8Geom g = q8_geom(K, gemv_items(a), a.ipw, a.parts, a.epi == EPI_SILU_GATE, unit);
  const DenseLds l = dense_lds(smem, K, a.norm != NORM_NONE);
  constexpr bool kNorm = KP <= 8;
  NormW<kNorm ? KP : 1> nwt;
  if (kNorm && a.norm != NORM_NONE) load_norm_weights(a.norm, a.nw, a.nb, K, nwt);
  float v[KP];
  load_row(a.x + (size_t)g.b * a.x_stride, K, v, &rs.ws->r_issued);
  const int p = (a.epi == EPI_QKV_ROPE || a.advance_pos ? spos[g.b] : 0);
  const EpiIn in = gemv_epi_prefetch(a, g.b, g.i0 + min((int)threadIdx.x, g.ni - 1), p);
  if constexpr (kNorm) {
    if (a.norm != NORM_NONE) norm_regs(v, K, a.norm, nwt, a.eps, l.xs, rs);
  }
  // the weight waves are done with the previous item's input and results
  lds_wait(&rs.ws->t_parts, item * kWeightWaves, &rs.ws->stop);
  store_row_chains(v, K, l.xT);
  lds_signal(&rs.ws->xq_parts);
  if ((int)(threadIdx.x & ~(kWave - 1)) >= g.ni && threadIdx.x != 0) return;  // waves without epilogue rows
  lds_wait(&rs.ws->t_parts, (item + 1) * kWeightWaves, &rs.ws->stop);
  gemv_finish(a, g.b, g.part, g.i0, g.ni, p, in, l.Y);
}

// Weight-wave part of a dense item: issue the first loads of the thread's lane chain as soon as
// the row waves have requested the input row, wait for the chain-major input, then stream the
// chain (kDenseBatch loads in flight), sum the 16 lanes and write the row result.  With STAGE (a
// launch of one item per workgroup) and a unit that fits, the unit's rows are first staged in LDS
// by all weight waves and the chains read them there (the same loads in the same order).
template <bool BF16W, bool STAGE = false>
__device__ __forceinline__ bool w_dense_at(const unsigned char* wbase, int K, int items, int ipw, int parts, int epi,
                                           bool norm, int unit, WgSync* ws, unsigned char* smem, unsigned item) {
  constexpr int EPL = BF16W ? 8 : 4;  // elements per 16-byte load
  const int ff_hidden = items;  // read by gemv_phys_row for the SiLU gate only, where items = ff_hidden
  const Q8Geom g = q8_geom(K, items, ipw, parts, epi == EPI_SILU_GATE, unit);
  const DenseLds l = dense_lds(smem, K, norm);
  const int stride = dense_chain_stride(K);
  const int NL = K / (16 * EPL);  // loads per chain
  const int w = threadIdx.x - kRowThreads;
  const int rr = w / 16, lane16 = w % 16;
  const int rowb = K * (BF16W ? 2 : 4);
  const bool staged = STAGE && item == 0 &&
                      dense_stage_bytes(K, ipw, epi == EPI_SILU_GATE ? 2 * ipw : ipw, BF16W, norm) > 0;  // uniform
  unsigned char* W = dense_stage(l, ipw);
  if (staged) {
    // 1 KiB pieces of the unit's rows (row r at W + r rowb), piece p by weight wave p % 8
    const int wave = __builtin_amdgcn_readfirstlane(w / kWave), lane = w % kWave;
    const int ppr = rowb / 1024, np = g.NR * ppr;
    for (int pc = wave; pc < np; pc += kWeightWaves) {
      const int r = pc / ppr, q = pc - r * ppr;
      const size_t row = (size_t)gemv_phys_row(epi, ff_hidden, g.i0, g.ni, r);
      lds_dma<16, false>(wbase + row * rowb + q * 1024 + lane * 16, W + pc * 1024);
    }
    __builtin_amdgcn_s_waitcnt(kVmWait0);  // this wave's pieces have landed
    lds_signal(&ws->w_staged);
    if (!lds_wait<true>(&ws->w_staged, kWeightWaves, &ws->stop)) return false;
  }
  bool ready = false;
  for (int r0 = 0; r0 < g.NR; r0 += 32) {
    const int r = r0 + rr;
    const size_t row = staged ? (size_t)min(r, g.NR - 1) : (size_t)gemv_phys_row(epi, ff_hidden, g.i0, g.ni, min(r, g.NR - 1));
    // load k at src[16 k]: in the staged rows, or in global memory
    const v4i* src = (const v4i*)(wbase + (row * NL * 16 + lane16) * 16);
    const SVL_LDS v4i* lsrc = (const SVL_LDS v4i*)(W + (row * NL * 16 + lane16) * 16);
    // load k of the chain: from the staged rows (LDS) or streamed from global memory
    auto wload = [&](int k) -> v4i { return staged ? lsrc[16 * k] : ldg_stream(src + 16 * k); };
    v4i buf[kDenseBatch];
#pragma unroll
    for (int u = 0; u < kDenseBatch; ++u) buf[u] = wload(min(u, NL - 1));
    if (!ready) {
      if (!lds_wait<true>(&ws->xq_parts, (item + 1) * kRowWaves, &ws->stop)) return false;
      ready = true;
    }
    const float* xc = l.xT + lane16 * stride;
    float acc = 0.0f;
    const bool stream = NL > kDenseBatch;  // uniform: more loads than fit in flight
    for (int k0 = 0; k0 < NL; k0 += kDenseBatch) {
#pragma unroll
      for (int u = 0; u < kDenseBatch; ++u) {
        const int k = k0 + u;
        if (k < NL) {  // uniform
        const v4i wv = buf[u];
        if (stream) buf[u] = wload(min(k + kDenseBatch, NL - 1));
        float xv[EPL];
        if constexpr (BF16W) {
          const float4 x0 = *(const float4*)(xc + k * 8), x1 = *(const float4*)(xc + k * 8 + 4);
          xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w;
          xv[4] = x1.x; xv[5] = x1.y; xv[6] = x1.z; xv[7] = x1.w;
          const uint32_t wd[4] = {(uint32_t)wv.x, (uint32_t)wv.y, (uint32_t)wv.z, (uint32_t)wv.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            acc = fmaf(xv[e], __uint_as_float(e & 1 ? (wd[e / 2] & 0xFFFF0000u) : (wd[e / 2] << 16)), acc);
        } else {
          const float4 x0 = *(const float4*)(xc + k * 4);
          xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w;
          acc = fmaf(xv[0], __int_as_float(wv.x), acc);
          acc = fmaf(xv[1], __int_as_float(wv.y), acc);
          acc = fmaf(xv[2], __int_as_float(wv.z), acc);
          acc = fmaf(xv[3], __int_as_float(wv.w), acc);
        }
        }
      }
    }
    acc = row16_pairwise_sum(acc);
    if (lane16 == 0 && r < g.NR) l.Y[r] = acc;
  }
  if (!ready && !lds_wait<true>(&ws->xq_parts, (item + 1) * kRowWaves, &ws->stop)) return false;
  return true;
}

template <bool BF16W>
__device__ __forceinline__ bool w_dense(const Phase* ph, int unit, WgSync* ws, unsigned char* smem, unsigned item) {
  const int epi = ld_const(&ph->g.epi);
  const int items = epi == EPI_SILU_GATE ? ld_const(&ph->g.ff_hidden) : ld_const(&ph->g.L.out);
  return w_dense_at<BF16W>((const unsigned char*)ld_const(&ph->g.L.w), ld_const(&ph->g.L.in), items,
                           ld_const(&ph->g.ipw), ld_const(&ph->g.parts), epi, ld_const(&ph->g.norm) != NORM_NONE, unit, ws,
                           smem, item);
}

__device__ __forceinline__ bool is_chained_dense(int fmt) { return fmt == FMT_F32C || fmt == FMT_BF16C; }

// ---- attention unit (row waves) ------------------------------------------------------------------
// One unit per (stream, head).  The query at position p attends to keys
// max(0, p - window + 1) ..= p (transformer.rs:385) in the ring, in the reference's order
// (attention.rs:139-168): w_j = scale * dot(q, k_j) with the 16-lane dot (16 threads per key),
// max, e_j = exp(w_j - max), the sum of e_j in key order, then out = sum over keys in order of
// mul_add(e_j / sum, v_j, out), thread d owning dim d.  K and then V rows stream through
// kAttnStages LDS stages of kAttnChunkBytes by direct loads issued kAttnStages - 1 chunks ahead;
// the LDS reads of the stages are written out (see gemm_issue).

__device__ __forceinline__ int visible_keys(const AttnArgs& a, int p) {
  return a.window > 0 ? min(p + 1, a.window) : p + 1;
}

__device__ __forceinline__ void lds_write_f32(uint32_t addr, float v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}

// v[i] = the f32 (BF16: the widened bf16) at LDS byte addr + i * STEP, i < N (N = 4 or 8).
template <int N, int STEP, bool BF16>
__device__ __forceinline__ void lds_read_strided(uint32_t addr, float (&v)[N]) {
  uint32_t r[8];
  if constexpr (N == 8 && !BF16) {
    asm volatile(
        "ds_read_b32 %0, %8\n\tds_read_b32 %1, %8 offset:%9\n\tds_read_b32 %2, %8 offset:%10\n\t"
        "ds_read_b32 %3, %8 offset:%11\n\tds_read_b32 %4, %8 offset:%12\n\tds_read_b32 %5, %8 offset:%13\n\t"
        "ds_read_b32 %6, %8 offset:%14\n\tds_read_b32 %7, %8 offset:%15\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(addr), "i"(STEP), "i"(2 * STEP), "i"(3 * STEP), "i"(4 * STEP), "i"(5 * STEP), "i"(6 * STEP),
          "i"(7 * STEP)
        : "memory");
  } else if constexpr (N == 8) {
    asm volatile(
        "ds_read_u16 %0, %8\n\tds_read_u16 %1, %8 offset:%9\n\tds_read_u16 %2, %8 offset:%10\n\t"
        "ds_read_u16 %3, %8 offset:%11\n\tds_read_u16 %4, %8 offset:%12\n\tds_read_u16 %5, %8 offset:%13\n\t"
        "ds_read_u16 %6, %8 offset:%14\n\tds_read_u16 %7, %8 offset:%15\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(addr), "i"(STEP), "i"(2 * STEP), "i"(3 * STEP), "i"(4 * STEP), "i"(5 * STEP), "i"(6 * STEP),
          "i"(7 * STEP)
        : "memory");
  } else if constexpr (!BF16) {
    static_assert(N == 4, "4 or 8 values");
    asm volatile(
        "ds_read_b32 %0, %4\n\tds_read_b32 %1, %4 offset:%5\n\tds_read_b32 %2, %4 offset:%6\n\t"
        "ds_read_b32 %3, %4 offset:%7\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(addr), "i"(STEP), "i"(2 * STEP), "i"(3 * STEP)
        : "memory");
  } else {
    static_assert(N == 4, "4 or 8 values");
    asm volatile(
        "ds_read_u16 %0, %4\n\tds_read_u16 %1, %4 offset:%5\n\tds_read_u16 %2, %4 offset:%6\n\t"
        "ds_read_u16 %3, %4 offset:%7\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(addr), "i"(STEP), "i"(2 * STEP), "i"(3 * STEP)
        : "memory");
  }
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = BF16 ? __uint_as_float(r[i] << 16) : __uint_as_float(r[i]);
}

// The values phase's operands of 16 keys in one round trip: wv = 16 consecutive f32 at waddr
// (16-byte aligned), vv[i] = the f32 (BF16: the widened bf16) at vaddr + i * STEP.
template <int STEP, bool BF16>
__device__ __forceinline__ void lds_read_wv16(uint32_t waddr, uint32_t vaddr, float (&wv)[16], float (&vv)[16]) {
  float4 w0, w1, w2, w3;
  uint32_t r[16];
#define SVL_V16(OP)                                                                                              \
  asm volatile("ds_read_b128 %0, %20\n\tds_read_b128 %1, %20 offset:16\n\t"                                     \
               "ds_read_b128 %2, %20 offset:32\n\tds_read_b128 %3, %20 offset:48\n\t"                           \
               OP " %4, %21\n\t" OP " %5, %21 offset:%22\n\t" OP " %6, %21 offset:%23\n\t"                      \
               OP " %7, %21 offset:%24\n\t" OP " %8, %21 offset:%25\n\t" OP " %9, %21 offset:%26\n\t"           \
               OP " %10, %21 offset:%27\n\t" OP " %11, %21 offset:%28\n\t" OP " %12, %21 offset:%29\n\t"        \
               OP " %13, %21 offset:%30\n\t" OP " %14, %21 offset:%31\n\t" OP " %15, %21 offset:%32\n\t"        \
               OP " %16, %21 offset:%33\n\t" OP " %17, %21 offset:%34\n\t" OP " %18, %21 offset:%35\n\t"        \
               OP " %19, %21 offset:%36\n\ts_waitcnt lgkmcnt(0)"                                                  \
               : "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3), "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]),    \
                 "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]),       \
                 "=&v"(r[11]), "=&v"(r[12]), "=&v"(r[13]), "=&v"(r[14]), "=&v"(r[15])                            \
               : "v"(waddr), "v"(vaddr), "i"(STEP), "i"(2 * STEP), "i"(3 * STEP), "i"(4 * STEP), "i"(5 * STEP),  \
                 "i"(6 * STEP), "i"(7 * STEP), "i"(8 * STEP), "i"(9 * STEP), "i"(10 * STEP), "i"(11 * STEP),      \
                 "i"(12 * STEP), "i"(13 * STEP), "i"(14 * STEP), "i"(15 * STEP)                                   \
               : "memory")
  if constexpr (BF16) SVL_V16("ds_read_u16");
  else SVL_V16("ds_read_b32");
#undef SVL_V16
  const float4 ws[4] = {w0, w1, w2, w3};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wv[4 * i] = ws[i].x;
    wv[4 * i + 1] = ws[i].y;
    wv[4 * i + 2] = ws[i].z;
    wv[4 * i + 3] = ws[i].w;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) vv[i] = BF16 ? __uint_as_float(r[i] << 16) : __uint_as_float(r[i]);
}

// Eight consecutive f32 at a 16-byte aligned LDS byte address.
__device__ __forceinline__ void lds_read8_f32(uint32_t addr, float (&v)[8]) {
  float4 x, y;
  asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(x), "=&v"(y)
               : "v"(addr)
               : "memory");
  v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
}

// HPU heads of one stream per unit (1, or 2 for large batches): chunk row r holds head r % HPU,
// key r / HPU of the chunk, so that a thread's scores stay with one head; the weighted sums of
// head hh run on waves [hh HD / 64, (hh + 1) HD / 64).
template <int HD, bool BF16KV, int HPU>
__device__ __forceinline__ void attn_unit(const AttnArgs& a, int unit, const int* spos, unsigned char* smem, RowSync& rs) {
  constexpr int RB = HD * (BF16KV ? 2 : 4);   // bytes of a K or V row
  constexpr int R = kAttnChunkBytes / RB;     // rows per stage
  constexpr int RH = R / HPU;                 // keys per stage and head
  constexpr int C = HD / 16;
  static_assert(RH % 16 == 0 && HPU * HD <= kRowThreads, "stage rows per head");
  // the descriptor's fields are read once: the written-out LDS accesses below count as memory
  // clobbers, after which the compiler would read the descriptor again (and wait for every load
  // in flight before using the value)
  const int cap = a.cap, H = a.H, KVH = a.KVH;
  const float scale = a.scale;
  const void* kc = a.kc;
  const void* vc = a.vc;
  float* out = a.out;
  const int wstride = ((cap + 7) & ~7) + 8;  // reads of w run up to 7 past the last key
  float* w = (float*)(smem + kAttnStages * kAttnChunkBytes);  // HPU x L weights (16-byte aligned)
  float* slot = w + HPU * wstride;  // [0, HPU): sums; [4, 4 + 32): score maxima of the 32 groups
  // a single stream needs no order lookup (one dependent load less before the position)
  const int h0 = (unit % (H / HPU)) * HPU, b = a.B == 1 ? 0 : ldg(a.order + unit / (H / HPU));
  // the query is requested with the position (the prologue needs only the position)
  const int li = threadIdx.x % 16, grp = threadIdx.x / 16;
  const int hs = grp % HPU;  // this thread's head for the scores
  float q[C];
  {
    const float* qp = a.q + (size_t)b * H * HD + (size_t)(h0 + hs) * HD + li;
    __builtin_amdgcn_s_waitcnt(kVmWait0);  // no older store interleaves with the counted loads
#pragma unroll
    for (int c = 0; c < C; ++c) q[c] = ld_co(qp + c * 16);
  }
  const int p = spos[b];
  const int L = visible_keys(a, p);
  const int first = p + 1 - L;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const int nch = (L + RH - 1) / RH;
  // This thread's two 16-byte pieces of every chunk: piece o is byte o * 8192 + 1024 wave + 16 lane
  // of the chunk, i.e. row (that / RB), column (that % RB); the row is key (row / HPU) of head
  // h0 + row % HPU.
  const int off0 = wave * 1024 + lane * 16, off1 = off0 + 8192;
  const int row0 = off0 / RB, col0 = off0 % RB, row1 = off1 / RB, col1 = off1 % RB;
  const size_t kb = a.kv_group > 1 ? (size_t)(b / a.kv_group) : (size_t)b;  // the ring's stream
  const size_t base0 = (kb * KVH + (h0 + row0 % HPU) / (H / KVH)) * (size_t)cap;
  const size_t base1 = (kb * KVH + (h0 + row1 % HPU) / (H / KVH)) * (size_t)cap;
  auto issue = [&](const void* kv, int c) {
    unsigned char* st = smem + (c % kAttnStages) * kAttnChunkBytes;
    const int j0 = min(c * RH + row0 / HPU, L - 1), j1 = min(c * RH + row1 / HPU, L - 1);
    const unsigned char* g = (const unsigned char*)kv;
    lds_dma<16, true>(g + (base0 + (size_t)((first + j0) % cap)) * RB + col0, st + wave * 1024);
    lds_dma<16, true>(g + (base1 + (size_t)((first + j1) % cap)) * RB + col1, st + 8192 + wave * 1024);
  };
  constexpr int S = kSyncChunks, AHEAD = kAttnStages - kSyncChunks;  // chunks per sync, chunks issued ahead
  auto wait_chunks = [&](int c) {  // this wave's pieces of chunks c .. c + S - 1 have landed
    if (c + AHEAD <= nch) __builtin_amdgcn_s_waitcnt(kAttnVmWait);
    else __builtin_amdgcn_s_waitcnt(kVmWait0);
  };
  // ---- scores w_j = scale * dot16(q, k_j): 16 threads per key (thread i accumulating dims
  // i, i + 16, ... with FMA, then the pairwise lane sum); group grp takes rows grp, grp + 32, ...
  float* ws = w + hs * wstride;
  float mx = -__builtin_huge_valf();  // running maximum of this thread's scores
  for (int c = 0; c < min(AHEAD, nch); ++c) issue(kc, c);
  for (int c0 = 0; c0 < nch; c0 += S) {
    wait_chunks(c0);
    gemm_sync(rs);  // chunks c0 .. are in LDS everywhere; every wave is done with the chunks before
#pragma unroll
    for (int u = 0; u < S; ++u)
      if (c0 + AHEAD + u < nch) issue(kc, c0 + AHEAD + u);
#pragma unroll 1
    for (int pass = 0; pass < S * R / 32; ++pass) {
      const int c = c0 + pass / (R / 32);
      if (c >= nch) break;  // uniform
      const uint32_t st = lds_addr(smem + (c % kAttnStages) * kAttnChunkBytes);
      const int r = (pass % (R / 32)) * 32 + grp, jj = c * RH + r / HPU;
      float kv[C];
      lds_read_strided<C, 16 * (BF16KV ? 2 : 4), BF16KV>(st + r * RB + li * (BF16KV ? 2 : 4), kv);
      float acc = 0.0f;
#pragma unroll
      for (int cc = 0; cc < C; ++cc) acc = fmaf(q[cc], kv[cc], acc);
      acc = row16_pairwise_sum(acc);
      if (jj < L && li == 0) {
        const float sc = scale * (acc + 0.0f);
        lds_write_f32(lds_addr(ws + jj), sc);
        mx = fmaxf(mx, sc);
      }
    }
  }
  // ---- softmax: max (exact in any order), e_j = exp(w_j - max), the sum of e_j in key order,
  // e_j / sum
  if (li == 0) lds_write_f32(lds_addr(slot + 4 + grp), mx);
  __builtin_amdgcn_s_waitcnt(kVmWait0);
  gemm_sync(rs);
  float mxh[HPU];
#pragma unroll
  for (int hh = 0; hh < HPU; ++hh) {
    mxh[hh] = -__builtin_huge_valf();
#pragma unroll
    for (int gg = hh; gg < 32; gg += HPU) mxh[hh] = fmaxf(mxh[hh], slot[4 + gg]);
  }
#pragma unroll
  for (int hh = 0; hh < HPU; ++hh)
    for (int j = threadIdx.x; j < L; j += kRowThreads) w[hh * wstride + j] = ref_exp(w[hh * wstride + j] - mxh[hh]);
  rs.sync();
  if (lane == 0 && wave < HPU) slot[wave] = ordered_sum_from(w + wave * wstride, L, 0.0f);
  rs.sync();
#pragma unroll
  for (int hh = 0; hh < HPU; ++hh) {
    const float sum = slot[hh];
    for (int j = threadIdx.x; j < L; j += kRowThreads) w[hh * wstride + j] = w[hh * wstride + j] / sum;
  }
  rs.sync();
  // ---- out_d = mul_add(w_j, v_jd, out_d) over keys in order; thread hh HD + d owns dim d of
  // head h0 + hh
  for (int c = 0; c < min(AHEAD, nch); ++c) issue(vc, c);
  float acc = 0.0f;
  const int hv = min((int)threadIdx.x / HD, HPU - 1), d = threadIdx.x % HD;
  const float* wv_h = w + hv * wstride;
  for (int c0 = 0; c0 < nch; c0 += S) {
    wait_chunks(c0);
    gemm_sync(rs);
#pragma unroll
    for (int u = 0; u < S; ++u)
      if (c0 + AHEAD + u < nch) issue(vc, c0 + AHEAD + u);
#pragma unroll 1
    for (int u = 0; u < S; ++u) {
      const int c = c0 + u;
      if (c >= nch || wave >= HPU * HD / kWave) break;  // uniform
      const uint32_t st = lds_addr(smem + (c % kAttnStages) * kAttnChunkBytes) + hv * RB + d * (BF16KV ? 2 : 4);
#pragma unroll
      for (int r0 = 0; r0 < RH; r0 += 16) {
        if (c * RH + r0 >= L) break;  // uniform
        float wv[16], vv[16];
        lds_read_wv16<HPU * RB, BF16KV>(lds_addr(wv_h + c * RH + r0), st + r0 * HPU * RB, wv, vv);
        if (c * RH + r0 + 16 <= L) {  // uniform
#pragma unroll
          for (int k = 0; k < 16; ++k) acc = fmaf(wv[k], vv[k], acc);
        } else {
#pragma unroll
          for (int k = 0; k < 16; ++k)
            if (c * RH + r0 + k < L) acc = fmaf(wv[k], vv[k], acc);
        }
      }
    }
  }
  if ((int)threadIdx.x < HPU * HD) st_co(out + (size_t)b * H * HD + (size_t)(h0 + hv) * HD + d, acc);
}

// Compile-time attention variant of (head_dim, bf16 cache, heads per unit); 0 = chosen at run time.
__host__ __device__ constexpr int attn_variant(int hd, int kv_bf16, int hpu) {
  return 1 + (hd == 128 ? 1 : 0) + (kv_bf16 ? 2 : 0) + (hpu == 2 ? 4 : 0);
}

template <int AV>
__device__ __forceinline__ void attn_dispatch(const AttnArgs& a, int unit, const int* spos, unsigned char* smem,
                                              RowSync& rs) {
  if constexpr (AV != 0) {
    constexpr int c = AV - 1;
    attn_unit<(c & 1) ? 128 : 64, (c & 2) != 0, (c & 4) ? 2 : 1>(a, unit, spos, smem, rs);
    return;
  }
  if (a.hpu == 2) {
    if (a.hd == 128) {
      if (a.kv_bf16) attn_unit<128, true, 2>(a, unit, spos, smem, rs);
      else attn_unit<128, false, 2>(a, unit, spos, smem, rs);
    } else {
      if (a.kv_bf16) attn_unit<64, true, 2>(a, unit, spos, smem, rs);
      else attn_unit<64, false, 2>(a, unit, spos, smem, rs);
    }
  } else if (a.hd == 128) {
    if (a.kv_bf16) attn_unit<128, true, 1>(a, unit, spos, smem, rs);
    else attn_unit<128, false, 1>(a, unit, spos, smem, rs);
  } else {
    if (a.kv_bf16) attn_unit<64, true, 1>(a, unit, spos, smem, rs);
    else attn_unit<64, false, 1>(a, unit, spos, smem, rs);
  }
}

// ---- embedding, argmax, norm, copies (row waves) -------------------------------------------------

__device__ __forceinline__ float table_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ float table_f32(float v) { return v; }

// Element i of the text token's row plus the rows of the n_q codebooks' tokens, added in that
// order.  The raw elements (bf16 bits or f32) of the text row and of 32 codebooks are requested
// before any is used, so that no load waits for another.  Past n_q the last codebook's row is read
// again.
template <typename E>
__device__ __forceinline__ float embed_sum(const EmbedArgs& a, const uint32_t* stok, int b, int i, bool staged) {
  constexpr int G = 32;
  const size_t rows = (size_t)a.card + 1;
  const E te = ldg((const E*)a.text_emb + (size_t)stok[0] * a.d + i);
  const E* base = (const E*)(staged ? a.stage : a.emb);
  float x = 0.0f;
  for (int c0 = 0; c0 < a.n_q; c0 += G) {
    E e[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int c = min(c0 + u, a.n_q - 1);
      // staged: the rows were copied next to each other during the previous step
      const size_t row = staged ? (size_t)b * a.n_q + c : (size_t)c * rows + stok[1 + c];
      e[u] = ld_co(base + row * a.d + i);
    }
    if (c0 == 0) x = table_f32(te);
#pragma unroll
    for (int u = 0; u < G; ++u) x = c0 + u < a.n_q ? x + table_f32(e[u]) : x;
  }
  return a.n_q > 0 ? x : table_f32(te);
}

// SVL/stt/model.rs:246-250: x = text_emb[t] + emb_0[a_0] + ... in that order, f32 adds.  Token
// ids past the tables raise the state's bad-token flag (reported as invalid input when the
// caller synchronizes) and are clamped, so that every access stays in the tables.  Units:
// B x d / 512.
// The stream's tokens are staged in LDS first, then every table row is requested at once.  When
// `staged`, the audio rows are read from the copies gathered during the previous step (random
// table rows cost an address-translation miss each; the copies are contiguous).
__device__ __forceinline__ void embed_unit(const EmbedArgs& a, const uint32_t* text, const uint32_t* audio, int unit,
                                           const int* spos, bool staged, unsigned char* smem, RowSync& rs) {
  uint32_t* stok = (uint32_t*)smem;  // [0]: text token, [1 + c]: token of codebook c
  const int chunks = (a.d + kRowThreads - 1) / kRowThreads;
  const int b = unit / chunks;
  const bool initial = a.initial_at_zero && spos[b] == 0;
  if ((int)threadIdx.x <= a.n_q) {
    uint32_t t;
    uint32_t lim;
    if (threadIdx.x == 0) {
      t = text ? ldg(text + b) : ld_co(a.fb_tok + b);
      lim = (uint32_t)a.text_card;
    } else {
      t = initial ? (uint32_t)a.card : ldg(audio + (size_t)b * a.n_q + threadIdx.x - 1);
      lim = (uint32_t)a.card;
    }
    if (t > lim) {
      if (a.bad_token && unit % chunks == 0) st_co(a.bad_token, 1u);
      t = lim;
    }
    stok[threadIdx.x] = t;
  }
  rs.sync();
  const int i = (unit % chunks) * kRowThreads + threadIdx.x;
  if (i >= a.d) return;
  const float x = a.tables_bf16 ? embed_sum<uint16_t>(a, stok, b, i, staged) : embed_sum<float>(a, stok, b, i, staged);
  st_co(a.x + (size_t)b * a.d + i, x);
}

// Copies the table rows of step `step`'s audio tokens of stream b, codebook c (unit = b * n_q + c)
// into a.stage, for the next step's embedding.  Positions only grow within a launch, so a later
// step never has a stream at position 0.
__device__ __forceinline__ void gather_unit(const EmbedArgs& a, const uint32_t* audio, int unit) {
  const int b = unit / a.n_q, c = unit % a.n_q;
  uint32_t tok = ldg(audio + (size_t)b * a.n_q + c);
  tok = tok > (uint32_t)a.card ? (uint32_t)a.card : tok;
  const int words = a.d * (a.tables_bf16 ? 2 : 4) / 4;  // d is a multiple of 32
  const uint32_t* src = (const uint32_t*)((const char*)a.emb + ((size_t)c * (a.card + 1) + tok) * (size_t)words * 4);
  uint32_t* dst = (uint32_t*)((char*)a.stage + ((size_t)b * a.n_q + c) * (size_t)words * 4);
  for (int i = threadIdx.x; i < words; i += kRowThreads) st_co(dst + i, ldg(src + i));
}

// argmax over logits[b] (first index of the maximum); unit = stream.
// The recognizer's word events and TurnDetector::update (SVL/stt/mod.rs:327-350, 566-589) for one
// step of stream b: the step's VoiceActivity event (when the model has extra heads), then its Word
// events -- a padding token (END_OF_PADDING 0 or PADDING 3) after pending word tokens (> 3) emits
// them (the tokenizer is taken to decode a pending run to at least one word).  `prob` is the
// probability at the detector's head.  Returns whether the step ends a turn.  The detector's part
// of the state changes only when `turns` (a call that reads turn ends), the recognizer's always.
__device__ __forceinline__ int turn_update(uint32_t& st, uint32_t token, bool turns, bool activity, float prob,
                                           float threshold, int frames) {
  bool pending = st & 1u, in_turn = (st >> 1) & 1u;
  uint32_t above = st >> 2;
  int end = 0;
  if (turns && activity) {
    above = prob > threshold ? min(above + 1u, 0x3fffffffu) : 0u;
    if (in_turn && above >= (uint32_t)frames) {
      in_turn = false;
      end = 1;
    }
  }
  if (token == 0u || token == 3u) {
    if (pending) {
      pending = false;
      if (turns) in_turn = true;
    }
  } else if (token > 3u) {
    pending = true;
  }
  st = (pending ? 1u : 0u) | (in_turn ? 2u : 0u) | (above << 2);
  return end;
}


__device__ __forceinline__ void argmax_unit(const ArgmaxArgs& a, uint32_t* out, float* out_prob, int unit,
                                            unsigned char* smem, RowSync& rs, int32_t* turn_out = nullptr) {
  float* sv = (float*)smem;
  int* si = (int*)(sv + kRowWaves);
  const int b = unit;
  const float* lg = a.logits + (size_t)b * a.V;
  float best = -__builtin_huge_valf();
  int idx = 0x7fffffff;
  constexpr int R = 16;
  for (int i0 = 0; i0 < a.V; i0 += R * kRowThreads) {
    float v[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int i = i0 + threadIdx.x + u * kRowThreads;
      if (i < a.V) v[u] = ld_co(lg + i);
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int i = i0 + threadIdx.x + u * kRowThreads;
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
  rs.sync();
  if (threadIdx.x == 0) {
    float bv = sv[0];
    int bi = si[0];
    for (int w = 1; w < kRowWaves; ++w) {
      if (si[w] != 0x7fffffff && (bi == 0x7fffffff || sv[w] > bv || (sv[w] == bv && si[w] < bi))) {
        bv = sv[w];
        bi = si[w];
      }
    }
    if (bi == 0x7fffffff) bi = 0;
    st_co(a.fb_tok + b, (uint32_t)bi);
    if (out) st_co(out + b, (uint32_t)bi);
    ((int*)(si + kRowWaves))[1] = bi;  // for the turn update below
  }
  // Extra heads (SVL/stt/model.rs:259-271): thread kWave + h takes head h's logits through
  // candle-nn's softmax_last_dim as the oracle restates it -- the maximum in index order from
  // element 0, exp(l_i - max), their sum in index order from zero -- and keeps element 0.
  const int h = (int)threadIdx.x - kWave;
  if (h >= 0 && h < a.nh) {
    const float* l = a.xlogits + ((size_t)b * a.nh + h) * a.hd;
    float mx = ld_co(l);
    for (int i = 1; i < a.hd; ++i) mx = fmaxf(mx, ld_co(l + i));
    float sum = 0.0f, first = 0.0f;
    for (int i = 0; i < a.hd; ++i) {
      const float e = expf(ld_co(l + i) - mx);
      if (i == 0) first = e;
      sum = sum + e;
    }
    const float p = first / sum;
    st_co(a.xprob + (size_t)b * a.nh + h, p);
    if (out_prob) st_co(out_prob + (size_t)b * a.nh + h, p);
    if (turn_out && h == (int)ld_const(a.turn_state + a.B + 2)) ((float*)(si + kRowWaves))[0] = p;
  }
  if (a.turn_state) {
    rs.sync();  // the token and the head's probability are in LDS (after si)
    if (threadIdx.x == 0) {
      uint32_t st = ld_co(a.turn_state + b);
      const float threshold = __uint_as_float(ld_const(a.turn_state + a.B));
      const int frames = (int)ld_const(a.turn_state + a.B + 1), head = (int)ld_const(a.turn_state + a.B + 2);
      const bool activity = a.nh > 0, at_head = head >= 0 && head < a.nh;
      const float* tp = (const float*)(si + kRowWaves);
      const int end = turn_update(st, (uint32_t)((const int*)tp)[1], turn_out != nullptr, activity,
                                  at_head ? tp[0] : 0.0f, threshold, frames);
      st_co(a.turn_state + b, st);
      if (turn_out) st_co(turn_out + b, (int32_t)end);
    }
  }
}

// y[b] = norm(x[b]); unit = stream.
template <int KP>
__device__ __forceinline__ void norm_unit(const NormArgs& a, int unit, unsigned char* smem, RowSync& rs) {
  float* xs = (float*)smem;
  NormW<KP> nwt;
  load_norm_weights(a.norm, a.w, a.b, a.d, nwt);
  float v[KP];
  load_row(a.x + (size_t)unit * a.x_stride, a.d, v);
  norm_regs(v, a.d, a.norm, nwt, a.eps, xs, rs);
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    const int i = threadIdx.x + u * kRowThreads;
    if (i < a.d) st_co(a.y + (size_t)unit * a.y_stride + i, v[u]);
  }
}

// y[b][0..n) = x[b][0..n); unit = (stream, 512-element chunk).
__device__ __forceinline__ void copy_unit(const float* x, int x_stride, float* y, int y_stride, int n, int unit) {
  const int chunks = (n + kRowThreads - 1) / kRowThreads;
  const int b = unit / chunks;
  const int i = (unit % chunks) * kRowThreads + threadIdx.x;
  if (i < n) st_co(y + (size_t)b * y_stride + i, ld_co(x + (size_t)b * x_stride + i));
}

// Row-wave part of work unit `unit` of phase `ph` for step `step` of a launch; `spos` holds
// the streams' positions at the start of the step, `item` counts the workgroup's Q8_0 GEMV
// units.
// Phase kinds compiled into a kernel, one bit per PhaseKind.
__host__ __device__ constexpr unsigned kind_bit(int k) { return 1u << k; }
constexpr unsigned kAllKinds = 0x3FFu;
constexpr unsigned kMiscKinds = kind_bit(PH_EMBED) | kind_bit(PH_ARGMAX) | kind_bit(PH_NORM) | kind_bit(PH_COPY_IN) |
                                kind_bit(PH_COPY_OUT);

template <unsigned F, unsigned KM = kAllKinds, int V = 0>
__device__ __forceinline__ void run_unit(const Phase& ph, const StepParams& P, int step, int unit, const int* spos,
                                         unsigned char* smem, RowSync& rs, unsigned& item) {
  if ((F & FAM_Q8) && ph.kind == PH_GEMV && (ph.g.L.fmt == FMT_Q8_0 || ph.g.L.fmt == FMT_Q4_0)) {
    if constexpr (V != 0) gemv_q8_rows<V>(ph.g, unit, spos, smem, rs, item);
    else switch (row_slots(ph.g.L.in)) {
      case 2: gemv_q8_rows<2>(ph.g, unit, spos, smem, rs, item); break;
      case 4: gemv_q8_rows<4>(ph.g, unit, spos, smem, rs, item); break;
      case 8: gemv_q8_rows<8>(ph.g, unit, spos, smem, rs, item); break;
      default: gemv_q8_rows<kMaxSlots>(ph.g, unit, spos, smem, rs, item); break;
    }
    ++item;
    return;
  }
  if ((F & FAM_DENSE) && ph.kind == PH_GEMV && is_chained_dense(ph.g.L.fmt)) {
    if constexpr (V != 0) gemv_dense_rows<V>(ph.g, unit, spos, smem, rs, item);
    else switch (row_slots(ph.g.L.in)) {
      case 2: gemv_dense_rows<2>(ph.g, unit, spos, smem, rs, item); break;
      case 4: gemv_dense_rows<4>(ph.g, unit, spos, smem, rs, item); break;
      case 8: gemv_dense_rows<8>(ph.g, unit, spos, smem, rs, item); break;
      default: gemv_dense_rows<kMaxSlots>(ph.g, unit, spos, smem, rs, item); break;
    }
    ++item;
    return;
  }
  if ((F & FAM_Q4K) && ph.kind == PH_GEMV && ph.g.L.fmt == FMT_Q4K) {
    if constexpr (V != 0) gemv_q4k_rows<V>(ph.g, unit, spos, smem, rs, item);
    else switch (row_slots(ph.g.L.in)) {
      case 2: gemv_q4k_rows<2>(ph.g, unit, spos, smem, rs, item); break;
      case 4: gemv_q4k_rows<4>(ph.g, unit, spos, smem, rs, item); break;
      case 8: gemv_q4k_rows<8>(ph.g, unit, spos, smem, rs, item); break;
      default: gemv_q4k_rows<kMaxSlots>(ph.g, unit, spos, smem, rs, item); break;
    }
    ++item;
    return;
  }
  rs.sync();  // the previous unit's readers of LDS are done
  switch (ph.kind) {
    case PH_EMBED: {
      if constexpr (!(KM & kind_bit(PH_EMBED))) break;
      const uint32_t* text = P.text ? P.text + (size_t)step * P.text_stride : nullptr;
      const bool staged = ph.e.stage != nullptr && step > 0 && !P.text;
      embed_unit(ph.e, text, P.audio + (size_t)step * P.audio_stride, unit, spos, staged, smem, rs);
      break;
    }
    case PH_GEMV:
      if constexpr (!(F & FAM_DENSE) || !(KM & kind_bit(PH_GEMV))) break;
      switch (row_slots(ph.g.L.in)) {
        case 2:
          if (ph.g.L.fmt == FMT_BF16) gemv_dense_unit<true, 2>(ph.g, unit, spos, smem, rs);
          else gemv_dense_unit<false, 2>(ph.g, unit, spos, smem, rs);
          break;
        case 4:
          if (ph.g.L.fmt == FMT_BF16) gemv_dense_unit<true, 4>(ph.g, unit, spos, smem, rs);
          else gemv_dense_unit<false, 4>(ph.g, unit, spos, smem, rs);
          break;
        case 8:
          if (ph.g.L.fmt == FMT_BF16) gemv_dense_unit<true, 8>(ph.g, unit, spos, smem, rs);
          else gemv_dense_unit<false, 8>(ph.g, unit, spos, smem, rs);
          break;
        default:
          if (ph.g.L.fmt == FMT_BF16) gemv_dense_unit<true, kMaxSlots>(ph.g, unit, spos, smem, rs);
          else gemv_dense_unit<false, kMaxSlots>(ph.g, unit, spos, smem, rs);
          break;
      }
      break;
    case PH_ATTN: {
      if constexpr (!(KM & kind_bit(PH_ATTN))) break;
      const int heads = ph.at.B * ph.at.H / ph.at.hpu;
      if (unit < heads) attn_dispatch<V>(ph.at, unit, spos, smem, rs);
      else if (step + 1 < P.n_steps && !P.text) gather_unit(ph.e, P.audio + (size_t)(step + 1) * P.audio_stride, unit - heads);
      break;
    }
    case PH_QUANT:
      if constexpr (!(F & FAM_BATCH) || !(KM & kind_bit(PH_QUANT))) break;
      if constexpr (V != 0) quant_unit<V>(ph.g, unit, smem, rs);
      else switch (row_slots(ph.g.L.in)) {
        case 2: quant_unit<2>(ph.g, unit, smem, rs); break;
        case 4: quant_unit<4>(ph.g, unit, smem, rs); break;
        case 8: quant_unit<8>(ph.g, unit, smem, rs); break;
        default: quant_unit<kMaxSlots>(ph.g, unit, smem, rs); break;
      }
      break;
    case PH_QGEMM:
      if constexpr (!(F & FAM_BATCH) || !(KM & kind_bit(PH_QGEMM))) break;
      if ((ph.g.epi == EPI_SILU_GATE ? 2 * ph.g.ipw : ph.g.ipw) == kTileRows) qgemm_unit<kTileRows>(ph.g, unit, spos, smem, rs);
      else qgemm_unit<kTileRows / 2>(ph.g, unit, spos, smem, rs);
      break;
    case PH_ARGMAX:
      if constexpr (!(KM & kind_bit(PH_ARGMAX))) break;
      argmax_unit(ph.am, P.out_tok ? P.out_tok + (size_t)step * P.out_stride : nullptr,
                  P.out_prob ? P.out_prob + (size_t)step * P.prob_stride : nullptr, unit, smem, rs,
                  P.out_turn ? P.out_turn + (size_t)step * P.B : nullptr);
      break;
    case PH_NORM:
      if constexpr (!(KM & kind_bit(PH_NORM))) break;
      switch (row_slots(ph.nm.d)) {  // d_model <= 4096
        case 2: norm_unit<2>(ph.nm, unit, smem, rs); break;
        case 4: norm_unit<4>(ph.nm, unit, smem, rs); break;
        default: norm_unit<8>(ph.nm, unit, smem, rs); break;
      }
      break;
    case PH_COPY_IN:
      if constexpr (!(KM & kind_bit(PH_COPY_IN))) break;
      copy_unit(P.fwd_in + (size_t)step * ph.cp.n, ph.cp.x_stride, ph.cp.y, ph.cp.y_stride, ph.cp.n, unit);
      break;
    case PH_COPY_OUT:
      if constexpr (!(KM & kind_bit(PH_COPY_OUT))) break;
      copy_unit(ph.cp.x, ph.cp.x_stride, P.fwd_out + (size_t)step * ph.cp.n, ph.cp.y_stride, ph.cp.n, unit);
      break;
  }
}

// Weight waves of a launch: the quantized GEMV units of this workgroup in program order
// (steps x phases x units u = blockIdx.x + k * gridDim.x).  Advances (step, p, u) to the next
// one; false when there is none.
__device__ __forceinline__ bool w_next(const StepParams& P, int& step, int& p, int& u) {
  if (p >= 0) {
    u += gridDim.x;
    if (u < ld_const(&P.prog[p].units)) return true;
  }
  for (;;) {
    if (++p >= P.nphase) {
      p = 0;
      if (++step >= P.n_steps) return false;
    }
    if (is_split_gemv(P.prog + p) && (int)blockIdx.x < ld_const(&P.prog[p].units)) {
      u = blockIdx.x;
      return true;
    }
  }
}

// The weight-wave loop: request an item's blocks, wait for its quantized row, write its terms.
template <unsigned F>
__device__ __forceinline__ void weight_waves(const StepParams& P, WgSync* ws, unsigned char* smem) {
  int step = 0, p = -1, u = 0;
  unsigned item = 0;
  while (w_next(P, step, p, u)) {
    // the blocks are requested right after the row waves have requested the item's input row,
    // so that neither the row nor the row waves' stores and barrier traffic queue behind them
    if (!lds_wait<true>(&ws->r_issued, (item + 1) * kRowWaves, &ws->stop)) return;
    const int fmt = ld_const(&P.prog[p].g.L.fmt);
    if ((F & FAM_DENSE) && is_chained_dense(fmt)) {
      const bool ok = fmt == FMT_BF16C ? w_dense<true>(P.prog + p, u, ws, smem, item)
                                       : w_dense<false>(P.prog + p, u, ws, smem, item);
      if (!ok) return;
    } else if ((F & FAM_Q4K) && (!(F & FAM_Q8) || fmt == FMT_Q4K)) {
      WItemQ4 it4;
      w_issue_q4k(P.prog + p, u, it4);
      if (!lds_wait<true>(&ws->xq_parts, (item + 1) * kRowWaves, &ws->stop)) return;
      w_terms_q4k(it4, smem);
    } else if constexpr ((F & FAM_Q8) != 0) {
      WItem it;
      w_issue(P.prog + p, u, it);
      if (!lds_wait<true>(&ws->xq_parts, (item + 1) * kRowWaves, &ws->stop)) return;
      w_terms(it, smem);
    }
    lds_signal(&ws->t_parts);
    ++item;
  }
}

}  // namespace svl
