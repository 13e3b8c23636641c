// Decode-step kernels for gfx950 (MI355X).
//
// A decode step is a program of phases (embedding, the GEMVs of each layer, attention, output
// head, argmax; see the work units in step_units.h).  It runs either
//   * as one persistent kernel for many steps: every workgroup walks the program, takes the
//     work units u = blockIdx.x, blockIdx.x + gridDim.x, ... of each phase and meets the others
//     at a grid barrier between phases (all workgroups are co-resident: cooperative launch of
//     one workgroup per CU), or
//   * as one kernel launch per phase (the same units, one workgroup per unit).
#include <algorithm>

#include "kernels.h"
#include "step_units.h"

namespace svl {

// ---- grid barrier -------------------------------------------------------------------------------
// Hierarchical arrive: each workgroup adds to the counter of its group (blockIdx % 8), the last
// arriver of a group adds to the top counter, the last group publishes the generation.  Counters
// only grow (generation g completes when group counters reach g * members), so nothing is reset
// between barriers or launches.  All data a workgroup wrote in the phase was stored with
// agent-scope stores, and waited for before arriving.  A bounded spin sets the abort flag instead
// of hanging; every workgroup then leaves the kernel.

constexpr unsigned kSpinLimit = 1u << 22;

__device__ __forceinline__ bool grid_barrier(SyncState* s, unsigned gen) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int s_ok;
  if (threadIdx.x == 0) {
    const unsigned g = blockIdx.x & 7u;
    const unsigned members = gridDim.x / 8u + (g < (gridDim.x & 7u) ? 1u : 0u);
    const unsigned ngroups = gridDim.x < 8u ? gridDim.x : 8u;
    const unsigned old = __hip_atomic_fetch_add(gbl(&s->group[g][0]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1u == members * gen) {
      const unsigned t = __hip_atomic_fetch_add(gbl(&s->top[0]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t + 1u == ngroups * gen) __hip_atomic_store(gbl(&s->release[0]), gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    int ok = 1;
    unsigned spins = 0;
    while (__hip_atomic_load(gbl(&s->release[0]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gen) {
      if (__hip_atomic_load(gbl(&s->abort_flag[0]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        ok = 0;
        break;
      }
      if (++spins > kSpinLimit) {
        __hip_atomic_store(gbl(&s->abort_flag[0]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
    }
    s_ok = ok;
  }
  __syncthreads();
  return s_ok != 0;
}

// Positions of the streams at the start of the step, cached in LDS (the last layer advances
// them; no later phase of the step reads them).
__device__ __forceinline__ void load_positions(const StepParams& P, int* spos) {
  for (int b = threadIdx.x; b < P.B; b += kStepThreads) spos[b] = ld_co(P.pos + b);
  lds_barrier();
}

// The program's phase descriptors are copied into LDS once per phase, so the units read their
// arguments from LDS.
constexpr int kPhaseWords = sizeof(Phase) / 4;
static_assert(sizeof(Phase) % 4 == 0 && kPhaseWords <= kStepThreads, "phase descriptor size");

__device__ __forceinline__ void load_phase(const Phase* src, uint32_t* dst) {
  lds_barrier();
  if (threadIdx.x < kPhaseWords) dst[threadIdx.x] = ldg((const uint32_t*)src + threadIdx.x);
  lds_barrier();
}

__global__ __launch_bounds__(kStepThreads) void step_program_kernel(StepParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int spos[kMaxBatch];
  __shared__ __align__(16) uint32_t ph_words[kPhaseWords];
  const Phase& ph = *(const Phase*)ph_words;
  unsigned gen = P.gen0;
  for (int step = 0; step < P.n_steps; ++step) {
    load_positions(P, spos);
    for (int p = 0; p < P.nphase; ++p) {
      load_phase(P.prog + p, ph_words);
      for (int u = blockIdx.x; u < ph.units; u += gridDim.x) {
        lds_barrier();
        if (!run_unit(ph, P, step, u, spos, smem)) break;
      }
      if (!grid_barrier(P.sync, ++gen)) return;
    }
  }
}

__global__ __launch_bounds__(kStepThreads) void phase_kernel(const Phase* d_ph, StepParams P, int step) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int spos[kMaxBatch];
  __shared__ __align__(16) uint32_t ph_words[kPhaseWords];
  const Phase& ph = *(const Phase*)ph_words;
  load_phase(d_ph, ph_words);
  load_positions(P, spos);
  run_unit(ph, P, step, blockIdx.x, spos, smem);
}

hipError_t launch_step_program(const StepParams& p, int grid, size_t smem, hipStream_t s) {
  StepParams args = p;
  void* kargs[] = {&args};
  return hipLaunchCooperativeKernel((const void*)step_program_kernel, dim3(grid), dim3(kStepThreads), kargs,
                                    (unsigned)smem, s);
}

hipError_t launch_phase(const Phase* d_ph, int units, const StepParams& p, int step, size_t smem, hipStream_t s) {
  if (units <= 0) return hipSuccess;
  hipLaunchKernelGGL(phase_kernel, dim3(units), dim3(kStepThreads), smem, s, d_ph, p, step);
  return hipGetLastError();
}

int step_program_grid(int device) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) return 0;
  return cus;
}

// ---- planning ---------------------------------------------------------------------------------

static int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

void plan_gemv(GemvArgs& g, int grid, int* units) {
  const bool silu = g.epi == EPI_SILU_GATE;
  const int items = silu ? g.ff_hidden : g.L.out;
  if (g.L.fmt == FMT_Q8_0) {
    const int nb = g.L.in / 32;
    // About one unit per workgroup and batch row, at most 4 weight blocks per thread.
    int ipw = (items + grid - 1) / grid;
    if (g.epi == EPI_QKV_ROPE && (ipw & 1)) ++ipw;
    const int per_row = silu ? 2 : 1;
    if (ipw > kStepThreads / per_row) ipw = kStepThreads / per_row;  // one thread per row in the sums
    while (ipw > 1 && per_row * ipw * nb > 4 * kStepThreads) ipw = (g.epi == EPI_QKV_ROPE) ? ((ipw / 2 + 1) & ~1) : ipw / 2;
    if (g.epi == EPI_QKV_ROPE && ipw < 2) ipw = 2;
    g.ipw = ipw;
    g.maxb = (per_row * ipw * nb + kStepThreads - 1) / kStepThreads;
    if (g.maxb > 4) g.maxb = 4;
  } else {
    g.ipw = silu ? kStepThreads / 32 : kStepThreads / 16;
    g.maxb = 0;
  }
  g.parts = (items + g.ipw - 1) / g.ipw;
  *units = g.parts * g.B;
}

size_t phase_smem(const Phase& ph) {
  switch (ph.kind) {
    case PH_GEMV: {
      const GemvArgs& g = ph.g;
      const int K = g.L.in;
      if (g.L.fmt == FMT_Q8_0) {
        const int nb = K / 32, nb4 = (nb + 3) & ~3, ts = nb4 + 4;
        return (size_t)K * 4 + K + (size_t)nb4 * 4 + (size_t)2 * g.ipw * ts * 4 + (size_t)2 * g.ipw * 4 + 64;
      }
      return (size_t)K * 4 + (kStepThreads / 16) * 4 + 64;
    }
    case PH_ATTN_SOFTMAX_V:
      return (size_t)(((ph.at.cap + 3) & ~3) + 4) * 4 + 64;
    case PH_ARGMAX:
      return 32 * 4 + 64;
    case PH_NORM:
      return (size_t)ph.nm.d * 4 + 64;
    default:
      return 64;
  }
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

// Plain streaming copy (calibration of the HBM traffic counters): grid-stride 16-byte moves.
__global__ __launch_bounds__(256) void copy_kernel(const v4i* src, v4i* dst, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    __builtin_nontemporal_store(ldg_stream(src + i), gbl(dst + i));
}

hipError_t launch_copy(const void* src, void* dst, size_t bytes, hipStream_t s) {
  const size_t n = bytes / 16;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, s, (const v4i*)src, (v4i*)dst, n);
  return hipGetLastError();
}

}  // namespace svl
