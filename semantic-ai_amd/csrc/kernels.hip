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

// ---- grid barrier (row waves) ----------------------------------------------------------------------
// Each row wave waits for its own stores of the phase and counts itself in LDS; the first row
// wave then adds one to the counter of the workgroup's group (blockIdx % 8) without waiting for
// the result, polls the group counters until each has reached generation x members, and
// releases the other row waves through LDS.  Counters only grow, so nothing is reset between
// barriers or launches (the host clears them long before 32-bit wrap).  A bounded spin sets the
// abort flag instead of hanging; every workgroup then leaves the kernel.

constexpr unsigned kSpinLimit = 1u << 22;

__device__ __forceinline__ unsigned group_members(unsigned g) {
  return gridDim.x / 8u + (g < (gridDim.x & 7u) ? 1u : 0u);
}

// Row waves only; `n` counts the grid barriers of this launch (1, 2, ...).  False when the
// launch is aborting.
__device__ __forceinline__ bool grid_barrier(SyncState* s, unsigned gen, unsigned n, WgSync* ws) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete
  lds_signal(&ws->g_arrive);
  if (threadIdx.x >= kWave) return lds_wait<true>(&ws->g_release, n, &ws->stop);
  const int lane = threadIdx.x;
  if (!lds_wait(&ws->g_arrive, n * kRowWaves, &ws->stop)) return false;
  if (lane == 0) __hip_atomic_fetch_add(gbl(&s->group[blockIdx.x & 7u][0]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned ngroups = gridDim.x < 8u ? gridDim.x : 8u;
  const unsigned target = lane < (int)ngroups ? group_members(lane) * gen : 0u;
  const unsigned* ctr = lane < (int)ngroups ? &s->group[lane][0] : &s->abort_flag[0];
  bool ok = true;
  unsigned spins = 0;
  for (;;) {
    const unsigned v = __hip_atomic_load(gbl(ctr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned ab = __hip_atomic_load(gbl(&s->abort_flag[0]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool waiting = lane < (int)ngroups && (int)(v - target) < 0;
    if (ab || lds_ld(&ws->stop)) {
      ok = false;
      break;
    }
    if (!__any(waiting)) break;
    if (++spins > kSpinLimit) {
      if (lane == 0) __hip_atomic_store(gbl(&s->abort_flag[0]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = false;
      break;
    }
  }
  if (lane == 0) {
    if (ok) __hip_atomic_store(&ws->g_release, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(&ws->stop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  return ok;
}

// Positions of the streams at the start of the step, cached in LDS (the last layer advances
// them; no later phase of the step reads them).  Row waves.
__device__ __forceinline__ void load_positions(const StepParams& P, int* spos) {
  for (int b = threadIdx.x; b < P.B; b += kRowThreads) spos[b] = ld_co(P.pos + b);
}

// The phase descriptors are read with scalar loads from the program (read-only during a launch),
// so the compiler may read a field again instead of keeping it in registers.
__device__ __forceinline__ const Phase& phase_at(const Phase* prog, int p) {
  return *(const Phase*)(const SVL_CONST Phase*)(prog + p);
}

__device__ __forceinline__ void init_wg_sync(WgSync* ws) {
  if (threadIdx.x == 0) {
    ws->r_arrive = 0;
    ws->xq_parts = 0;
    ws->t_parts = 0;
    ws->r_issued = 0;
    ws->g_arrive = 0;
    ws->g_release = 0;
    ws->stop = 0;
  }
  __syncthreads();  // the only full-workgroup barrier: nothing is in flight yet
}

__global__ __launch_bounds__(kStepThreads) void step_program_kernel(StepParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int spos[kMaxBatch];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  if (threadIdx.x >= kRowThreads) {
    weight_waves(P, &ws, smem);
    return;
  }
  RowSync rs{&ws, 0u};
  unsigned gen = P.gen0;
  unsigned item = 0;
  for (int step = 0; step < P.n_steps; ++step) {
    load_positions(P, spos);
    rs.sync();
    for (int p = 0; p < P.nphase; ++p) {
      const Phase& ph = phase_at(P.prog, p);
      for (int u = blockIdx.x; u < ph.units; u += gridDim.x) run_unit(ph, P, step, u, spos, smem, rs, item);
      ++gen;
      if (!grid_barrier(P.sync, gen, gen - P.gen0, &ws)) return;
    }
  }
}

__global__ __launch_bounds__(kStepThreads) void phase_kernel(const Phase* d_ph, StepParams P, int step) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int spos[kMaxBatch];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  if (threadIdx.x >= kRowThreads) {
    if (is_q8_gemv(d_ph)) {
      WItem it;
      if (!lds_wait<true>(&ws.r_issued, kRowWaves, &ws.stop)) return;
      w_issue(d_ph, blockIdx.x, it);
      if (!lds_wait(&ws.xq_parts, kRowWaves, &ws.stop)) return;
      w_terms(it, smem);
      lds_signal(&ws.t_parts);
    }
    return;
  }
  RowSync rs{&ws, 0u};
  load_positions(P, spos);
  rs.sync();
  unsigned item = 0;
  run_unit(phase_at(d_ph, 0), P, step, blockIdx.x, spos, smem, rs, item);
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

void plan_gemv(GemvArgs& g, int grid, int* units) {
  const bool silu = g.epi == EPI_SILU_GATE;
  const int items = silu ? g.ff_hidden : g.L.out;
  if (g.L.fmt == FMT_Q8_0) {
    const int nb = g.L.in / 32;
    // About one unit per workgroup and batch row; at most kWBlocks weight blocks per weight-wave
    // thread and one row-wave thread per row for the row sums.
    int ipw = (items + grid - 1) / grid;
    if (g.epi == EPI_QKV_ROPE && (ipw & 1)) ++ipw;
    const int per_row = silu ? 2 : 1;
    if (ipw > kRowThreads / per_row) ipw = kRowThreads / per_row;
    while (ipw > 1 && per_row * ipw * nb > kWBlocks * kWeightThreads) ipw = (g.epi == EPI_QKV_ROPE) ? ((ipw / 2 + 1) & ~1) : ipw / 2;
    if (g.epi == EPI_QKV_ROPE && ipw < 2) ipw = 2;
    g.ipw = ipw;
    g.maxb = (per_row * ipw * nb + kWeightThreads - 1) / kWeightThreads;
    if (g.maxb > kWBlocks) g.maxb = kWBlocks;
  } else {
    g.ipw = silu ? kRowThreads / 32 : kRowThreads / 16;
    g.maxb = 0;
  }
  g.parts = (items + g.ipw - 1) / g.ipw;
  *units = g.parts * g.B;
}

void plan_qgemm(GemvArgs& g, int* units) {
  const bool silu = g.epi == EPI_SILU_GATE;
  const int items = silu ? g.ff_hidden : g.L.out;
  g.ipw = silu ? kTileRows / 2 : kTileRows;
  g.parts = (items + g.ipw - 1) / g.ipw;
  g.maxb = 0;
  *units = g.parts * ((g.B + kTileBatch - 1) / kTileBatch);
}

size_t phase_smem(const Phase& ph) {
  switch (ph.kind) {
    case PH_GEMV: {
      const GemvArgs& g = ph.g;
      const int K = g.L.in;
      if (g.L.fmt == FMT_Q8_0) {
        const int nb = K / 32, nb4 = (nb + 3) & ~3, ts = 2 * g.ipw + 1;
        return (size_t)K * 4 + K + (size_t)nb4 * 4 + (size_t)nb * ts * 4 + (size_t)2 * g.ipw * 4 + 64;
      }
      return (size_t)K * 4 + (kRowThreads / 16) * 4 + 64;
    }
    case PH_ATTN:
      return (size_t)(((ph.at.cap + 3) & ~3) + 4) * 4 + 64;
    case PH_ARGMAX:
      return 32 * 4 + 64;
    case PH_NORM:
      return (size_t)ph.nm.d * 4 + 64;
    case PH_EMBED:
      return (size_t)(ph.e.n_q + 1) * 4 + 64;
    case PH_QUANT: {
      const int K = ph.g.L.in, nb4 = (K / 32 + 3) & ~3;
      return (size_t)K * 4 + K + (size_t)nb4 * 4 + 64;
    }
    case PH_QGEMM:
      return (size_t)kTileRows * kTileBatch * 4 + 64;
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
