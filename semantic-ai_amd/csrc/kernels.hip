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
    // lanes < ngroups read the group counters, the others the abort flag
    const unsigned v = __hip_atomic_load(gbl(ctr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool waiting = lane < (int)ngroups && (int)(v - target) < 0;
    if (__any(lane >= (int)ngroups && v != 0u) || lds_ld(&ws->stop)) {
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

template <unsigned F>
__global__ __launch_bounds__(kStepThreads) void step_program_kernel(StepParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int spos[kMaxBatch];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  if (threadIdx.x >= kRowThreads) {
    if constexpr ((F & (FAM_Q8 | FAM_Q4K | FAM_DENSE)) != 0) weight_waves<F>(P, &ws, smem);
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
      for (int u = blockIdx.x; u < ph.units; u += gridDim.x) run_unit<F>(ph, P, step, u, spos, smem, rs, item);
      ++gen;
      if (!grid_barrier(P.sync, gen, gen - P.gen0, &ws)) return;
    }
  }
}

// One phase of a step.  The descriptor travels in the kernel arguments: its fields are read from
// the argument segment, with no dependent load of a descriptor pointer first.  F and KM select
// the unit code compiled in (one GEMV family, or a group of phase kinds), so that each launch
// runs a compact kernel.
// Requests every 64-byte line of the first 832 bytes of the kernel arguments at once and waits for
// them, so that the scalar loads of descriptor fields that follow hit the scalar cache instead of
// going to memory one after another.
__device__ __forceinline__ void touch_kernel_args() {
  const void* k = (const void*)__builtin_amdgcn_kernarg_segment_ptr();
  unsigned d0, d1, d2, d3, d4, d5, d6, d7, d8, d9, d10, d11, d12;
  asm volatile(
      "s_load_dword %0, %13, 0x0\n\t"
      "s_load_dword %1, %13, 0x40\n\t"
      "s_load_dword %2, %13, 0x80\n\t"
      "s_load_dword %3, %13, 0xc0\n\t"
      "s_load_dword %4, %13, 0x100\n\t"
      "s_load_dword %5, %13, 0x140\n\t"
      "s_load_dword %6, %13, 0x180\n\t"
      "s_load_dword %7, %13, 0x1c0\n\t"
      "s_load_dword %8, %13, 0x200\n\t"
      "s_load_dword %9, %13, 0x240\n\t"
      "s_load_dword %10, %13, 0x280\n\t"
      "s_load_dword %11, %13, 0x2c0\n\t"
      "s_load_dword %12, %13, 0x300\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7), "=&s"(d8),
        "=&s"(d9), "=&s"(d10), "=&s"(d11), "=&s"(d12)
      : "s"(k)
      : "memory");
}

template <unsigned F, unsigned KM, int V>
__global__ __launch_bounds__(kStepThreads) void phase_kernel(const Phase ph, StepParams P, int step) {
  static_assert(sizeof(Phase) + sizeof(StepParams) + sizeof(int) <= 0x340, "kernel arguments past the touched lines");
  touch_kernel_args();
  const Phase* d_ph = &ph;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  if (threadIdx.x >= kRowThreads) {
    if constexpr ((F & (FAM_Q8 | FAM_Q4K | FAM_DENSE)) != 0) {
      if (is_split_gemv(d_ph)) {
        if (!lds_wait<true>(&ws.r_issued, kRowWaves, &ws.stop)) return;
        if constexpr (F == FAM_DENSE) {
          const int fmt = ld_const(&d_ph->g.L.fmt);
          const bool ok = fmt == FMT_BF16C ? w_dense<true>(d_ph, blockIdx.x, &ws, smem, 0)
                                           : w_dense<false>(d_ph, blockIdx.x, &ws, smem, 0);
          if (!ok) return;
        } else if constexpr (F == FAM_Q4K) {
          WItemQ4 it;
          w_issue_q4k(d_ph, blockIdx.x, it);
          if (!lds_wait(&ws.xq_parts, kRowWaves, &ws.stop)) return;
          w_terms_q4k(it, smem);
        } else {
          WItem it;
          w_issue(d_ph, blockIdx.x, it);
          if (!lds_wait(&ws.xq_parts, kRowWaves, &ws.stop)) return;
          w_terms(it, smem);
        }
        lds_signal(&ws.t_parts);
      }
    }
    return;
  }
  // the weight waves have ended unless the unit is a split GEMV (they wait in LDS meanwhile)
  RowSync rs{&ws, 0u, !is_split_gemv(d_ph)};
  unsigned item = 0;
  // Units read the positions from memory where they need them: only the step's last phase that
  // reads them advances them, and launches are ordered on the stream.
  run_unit<F, KM, V>(phase_at(d_ph, 0), P, step, blockIdx.x, P.pos, smem, rs, item);
}

// A GEMV phase whose weight waves stream the weights (Q8_0, Q4K, chain-packed dense) launched
// with the fields its first loads depend on as leading scalar arguments, which the hardware
// preloads into SGPRs (-amdgpu-kernarg-preload-count): the input row and the weight requests go
// out at wave start instead of after a scalar load of the argument segment.  `hx` input rows,
// `hw` / `hsc` weights and Q8_0 / Q4_0 block scales, `hnw` norm weights, `hparts` = units per batch
// row | batch rows << 16, `hepn` = epilogue | norm kind << 8 | blocks per weight thread << 16 |
// (bf16 dense weights, or Q4_0 codes) << 24, `hxs` input row stride.  Workgroup w runs unit
// (w % B) * parts + w / B: the batch rows of one slice of weight rows run side by side, so that
// their weights come from L2 after the first read (lockstep batches, prefill blocks).
template <unsigned F, int V>
__global__ __launch_bounds__(kStepThreads) void gemv_phase_kernel(const float* hx, const void* hw, const void* hsc,
                                                                  const float* hnw, int hin, int hipw, int hparts,
                                                                  int hitems, int hepn, int hxs, const Phase ph,
                                                                  StepParams P, int step) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  const int epi = hepn & 0xff, maxb = (hepn >> 16) & 0xff;
  const int nparts = hparts & 0xffff, nbatch = hparts >> 16;
  const int unit = nbatch > 1 ? (int)(blockIdx.x % nbatch) * nparts + (int)(blockIdx.x / nbatch) : (int)blockIdx.x;
  hparts = nparts;
  if (threadIdx.x >= kRowThreads) {
    if (!lds_wait<true>(&ws.r_issued, kRowWaves, &ws.stop)) return;
    if constexpr (F == FAM_Q8) {
      WItem it;
      w_issue_at((const int8_t*)hw, (const uint16_t*)hsc, hin, hitems, hipw, hparts, maxb, epi, unit, it,
                 (hepn >> 24) & 1);
      if (!lds_wait(&ws.xq_parts, kRowWaves, &ws.stop)) return;
      w_terms(it, smem);
    } else if constexpr (F == FAM_Q4K) {
      WItemQ4 it;
      w_issue_q4k_at((const unsigned char*)hw, hin, hitems, hipw, hparts, maxb, epi, unit, it);
      if (!lds_wait(&ws.xq_parts, kRowWaves, &ws.stop)) return;
      w_terms_q4k(it, smem);
    } else {
      const bool nrm = ((hepn >> 8) & 0xff) != NORM_NONE;
      const bool ok = (hepn >> 24) ? w_dense_at<true, true>((const unsigned char*)hw, hin, hitems, hipw, hparts, epi, nrm,
                                                            unit, &ws, smem, 0)
                                   : w_dense_at<false, true>((const unsigned char*)hw, hin, hitems, hipw, hparts, epi, nrm,
                                                             unit, &ws, smem, 0);
      if (!ok) return;
    }
    lds_signal(&ws.t_parts);
    return;
  }
  RowSync rs{&ws, 0u};  // LDS barriers: the weight waves stream meanwhile
  GemvArgs a = ph.g;
  a.x = hx;
  a.x_stride = hxs;
  a.L.in = hin;
  a.ipw = hipw;
  a.parts = hparts;
  a.epi = epi;
  a.norm = (hepn >> 8) & 0xff;
  a.nw = hnw;
  if (epi == EPI_SILU_GATE) a.ff_hidden = hitems;
  else a.L.out = hitems;
  if constexpr (F == FAM_Q8) gemv_q8_rows<V>(a, unit, P.pos, smem, rs, 0u);
  else if constexpr (F == FAM_Q4K) gemv_q4k_rows<V>(a, unit, P.pos, smem, rs, 0u);
  else gemv_dense_rows<V>(a, unit, P.pos, smem, rs, 0u);
}

// An attention phase launched like gemv_phase_kernel: the query, K / V ring, position and order
// pointers, ring slots, window, batch and head units as preloaded scalar arguments.  Units past
// `hheads` gather the next step's audio embedding rows (the first attention phase of an STT step).
template <int AV>
__global__ __launch_bounds__(kStepThreads) void attn_phase_kernel(const float* hq, const void* hkc, const void* hvc,
                                                                  const int* hpos, const int* horder, int hcap,
                                                                  int hwindow, int hB, int hheads, const Phase ph,
                                                                  StepParams P, int step) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  if (threadIdx.x >= kRowThreads) return;
  RowSync rs{&ws, 0u, true};
  const int unit = blockIdx.x;
  if (unit < hheads) {
    AttnArgs a = ph.at;
    a.q = hq;
    a.kc = hkc;
    a.vc = hvc;
    a.pos = (int*)hpos;
    a.order = horder;
    a.cap = hcap;
    a.window = hwindow;
    a.B = hB;
    attn_dispatch<AV>(a, unit, hpos, smem, rs);
  } else if (step + 1 < P.n_steps && !P.text) {
    gather_unit(ph.e, P.audio + (size_t)(step + 1) * P.audio_stride, unit - hheads);
  }
}

// The batched Q8_0 phases (activation quantization, MFMA GEMM) launched the same way.  PH_QUANT:
// `hp0` input rows, `hp1` norm weights, `hp2` / `hp3` quantized rows and their scales; PH_QGEMM:
// `hp0` / `hp1` quantized rows and scales, `hp2` / `hp3` quants and block scales of the weights.
// `hepn` = epilogue | norm kind << 8 | phase kind << 24.
template <int V>
__global__ __launch_bounds__(kStepThreads) void batch_phase_kernel(const void* hp0, const void* hp1, const void* hp2,
                                                                   const void* hp3, int hin, int hipw, int hparts,
                                                                   int hitems, int hepn, int hxs, const Phase ph,
                                                                   StepParams P, int step) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  if (threadIdx.x >= kRowThreads) return;
  RowSync rs{&ws, 0u, true};
  GemvArgs a = ph.g;
  const int epi = hepn & 0xff;
  a.L.in = hin;
  a.ipw = hipw;
  a.parts = hparts;
  a.epi = epi;
  if (epi == EPI_SILU_GATE) a.ff_hidden = hitems;
  else a.L.out = hitems;
  if ((hepn >> 24) == PH_QUANT) {
    a.x = (const float*)hp0;
    a.x_stride = hxs;
    a.nw = (const float*)hp1;
    a.norm = (hepn >> 8) & 0xff;
    a.xq = (int8_t*)hp2;
    a.xdq = (float*)hp3;
    quant_unit<V>(a, blockIdx.x, smem, rs);
  } else {
    a.xq = (int8_t*)hp0;
    a.xdq = (float*)hp1;
    a.L.w = (void*)hp2;
    a.L.scale = (uint16_t*)hp3;
    if ((epi == EPI_SILU_GATE ? 2 * hipw : hipw) == kTileRows) qgemm_unit<kTileRows>(a, blockIdx.x, P.pos, smem, rs);
    else qgemm_unit<kTileRows / 2>(a, blockIdx.x, P.pos, smem, rs);
  }
}

template <int AV>
void (*attn_phase_kernel_at(int v))(const float*, const void*, const void*, const int*, const int*, int, int, int, int,
                                    const Phase, StepParams, int) {
  if constexpr (AV > 8) {
    return nullptr;
  } else {
    return v == AV ? attn_phase_kernel<AV> : attn_phase_kernel_at<AV + 1>(v);
  }
}

unsigned program_families(const Phase* phases, int n) {
  unsigned f = 0;
  for (int i = 0; i < n; ++i) {
    const Phase& ph = phases[i];
    if (ph.kind == PH_GEMV)
      f |= ph.g.L.fmt == FMT_Q8_0 || ph.g.L.fmt == FMT_Q4_0 ? FAM_Q8 : (ph.g.L.fmt == FMT_Q4K ? FAM_Q4K : FAM_DENSE);
    if (ph.kind == PH_QUANT || ph.kind == PH_QGEMM) f |= FAM_BATCH;
  }
  return f;
}

hipError_t launch_step_program(const StepParams& p, unsigned families, int grid, size_t smem, hipStream_t s) {
  StepParams args = p;
  void* kargs[] = {&args};
  const void* k;
  if ((families & ~(unsigned)FAM_Q8) == 0) k = (const void*)step_program_kernel<FAM_Q8>;
  else if ((families & ~(unsigned)(FAM_Q8 | FAM_BATCH)) == 0) k = (const void*)step_program_kernel<FAM_Q8 | FAM_BATCH>;
  else if ((families & ~(unsigned)FAM_Q4K) == 0) k = (const void*)step_program_kernel<FAM_Q4K>;
  else if ((families & ~(unsigned)FAM_DENSE) == 0) k = (const void*)step_program_kernel<FAM_DENSE>;
  else k = (const void*)step_program_kernel<FAM_ALL>;
  return hipLaunchCooperativeKernel(k, dim3(grid), dim3(kStepThreads), kargs, (unsigned)smem, s);
}

// The preloaded-argument GEMV kernel of a family for inputs of `slots` row slots.
template <unsigned F>
void (*gemv_slots_kernel(int slots))(const float*, const void*, const void*, const float*, int, int, int, int, int, int,
                                     const Phase, StepParams, int) {
  switch (slots) {
    case 2: return gemv_phase_kernel<F, 2>;
    case 4: return gemv_phase_kernel<F, 4>;
    case 8: return gemv_phase_kernel<F, 8>;
    default: return gemv_phase_kernel<F, kMaxSlots>;
  }
}

// The kernel of a GEMV family for inputs of `slots` row slots (2, 4, 8 or 16).
template <unsigned F, unsigned KM>
void (*slots_kernel(int slots))(const Phase, StepParams, int) {
  switch (slots) {
    case 2: return phase_kernel<F, KM, 2>;
    case 4: return phase_kernel<F, KM, 4>;
    case 8: return phase_kernel<F, KM, 8>;
    default: return phase_kernel<F, KM, kMaxSlots>;
  }
}

template <int AV>
void (*attn_kernel_at(int v))(const Phase, StepParams, int) {
  if constexpr (AV > 8) {
    return nullptr;
  } else {
    return v == AV ? phase_kernel<0u, kind_bit(PH_ATTN), AV> : attn_kernel_at<AV + 1>(v);
  }
}

hipError_t launch_phase(const Phase& ph, const StepParams& p, int step, size_t smem, hipStream_t s) {
  if (ph.units <= 0) return hipSuccess;
  void (*k)(const Phase, StepParams, int);
  if (ph.kind == PH_GEMV && (ph.g.L.fmt == FMT_Q8_0 || ph.g.L.fmt == FMT_Q4_0 || ph.g.L.fmt == FMT_Q4K ||
                             ph.g.L.fmt == FMT_F32C || ph.g.L.fmt == FMT_BF16C)) {
    const GemvArgs& g = ph.g;
    void (*kq)(const float*, const void*, const void*, const float*, int, int, int, int, int, int, const Phase,
               StepParams, int);
    if (g.L.fmt == FMT_Q8_0 || g.L.fmt == FMT_Q4_0) kq = gemv_slots_kernel<FAM_Q8>(row_slots(g.L.in));
    else if (g.L.fmt == FMT_Q4K) kq = gemv_slots_kernel<FAM_Q4K>(row_slots(g.L.in));
    else kq = gemv_slots_kernel<FAM_DENSE>(row_slots(g.L.in));
    const int items = g.epi == EPI_SILU_GATE ? g.ff_hidden : g.L.out;
    const int epn = g.epi | (g.norm << 8) | (g.maxb << 16) | ((g.L.fmt == FMT_BF16C || g.L.fmt == FMT_Q4_0 ? 1 : 0) << 24);
    hipLaunchKernelGGL(kq, dim3(ph.units), dim3(kStepThreads), smem, s, g.x, (const void*)g.L.w, (const void*)g.L.scale,
                       g.nw, g.L.in, g.ipw, g.parts | (g.B << 16), items, epn, g.x_stride, ph, p, step);
    return hipGetLastError();
  }
  if (ph.kind == PH_QUANT || ph.kind == PH_QGEMM) {
    const GemvArgs& g = ph.g;
    void (*kb)(const void*, const void*, const void*, const void*, int, int, int, int, int, int, const Phase,
               StepParams, int);
    switch (row_slots(g.L.in)) {
      case 2: kb = batch_phase_kernel<2>; break;
      case 4: kb = batch_phase_kernel<4>; break;
      case 8: kb = batch_phase_kernel<8>; break;
      default: kb = batch_phase_kernel<kMaxSlots>; break;
    }
    const bool quant = ph.kind == PH_QUANT;
    const int items = g.epi == EPI_SILU_GATE ? g.ff_hidden : g.L.out;
    const int epn = g.epi | (g.norm << 8) | (ph.kind << 24);
    hipLaunchKernelGGL(kb, dim3(ph.units), dim3(kStepThreads), smem, s, quant ? (const void*)g.x : (const void*)g.xq,
                       quant ? (const void*)g.nw : (const void*)g.xdq, quant ? (const void*)g.xq : (const void*)g.L.w,
                       quant ? (const void*)g.xdq : (const void*)g.L.scale, g.L.in, g.ipw, g.parts, items, epn,
                       g.x_stride, ph, p, step);
    return hipGetLastError();
  }
  if (ph.kind == PH_ATTN) {
    const AttnArgs& a = ph.at;
    const int hd = a.hd == 128 ? 128 : 64;
    auto ka = attn_phase_kernel_at<1>(attn_variant(hd, a.kv_bf16, a.hpu));
    hipLaunchKernelGGL(ka, dim3(ph.units), dim3(kStepThreads), smem, s, a.q, a.kc, a.vc, (const int*)p.pos, a.order,
                       a.cap, a.window, a.B, a.B * a.H / a.hpu, ph, p, step);
    return hipGetLastError();
  }
  switch (ph.kind) {
    case PH_GEMV:
      if (ph.g.L.fmt == FMT_Q8_0 || ph.g.L.fmt == FMT_Q4_0) k = slots_kernel<FAM_Q8, 0u>(row_slots(ph.g.L.in));
      else if (ph.g.L.fmt == FMT_Q4K) k = slots_kernel<FAM_Q4K, 0u>(row_slots(ph.g.L.in));
      else k = slots_kernel<FAM_DENSE, kind_bit(PH_GEMV)>(row_slots(ph.g.L.in));
      break;
    case PH_QUANT:
    case PH_QGEMM:
      k = slots_kernel<FAM_BATCH, kind_bit(PH_QUANT) | kind_bit(PH_QGEMM)>(row_slots(ph.g.L.in));
      break;
    case PH_ATTN: {
      const int hd = ph.at.hd == 128 ? 128 : 64;
      k = attn_kernel_at<1>(attn_variant(hd, ph.at.kv_bf16, ph.at.hpu));
      break;
    }
    default: k = phase_kernel<0u, kMiscKinds, 0>; break;
  }
  hipLaunchKernelGGL(k, dim3(ph.units), dim3(kStepThreads), smem, s, ph, p, step);
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
  if (g.L.fmt == FMT_Q8_0 || g.L.fmt == FMT_Q4_0) {
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
  } else if (g.L.fmt == FMT_Q4K) {
    // The same with 256-value super-blocks, at most kQ4Blocks of them per weight-wave thread.
    const int nb = g.L.in / 256;
    int ipw = (items + grid - 1) / grid;
    if (g.epi == EPI_QKV_ROPE && (ipw & 1)) ++ipw;
    const int per_row = silu ? 2 : 1;
    if (ipw > kRowThreads / per_row) ipw = kRowThreads / per_row;
    while (ipw > 1 && per_row * ipw * nb > kQ4Blocks * kWeightThreads) ipw = (g.epi == EPI_QKV_ROPE) ? ((ipw / 2 + 1) & ~1) : ipw / 2;
    if (g.epi == EPI_QKV_ROPE && ipw < 2) ipw = 2;
    g.ipw = ipw;
    g.maxb = (per_row * ipw * nb + kWeightThreads - 1) / kWeightThreads;
    if (g.maxb > kQ4Blocks) g.maxb = kQ4Blocks;
  } else if (g.L.fmt == FMT_F32C || g.L.fmt == FMT_BF16C) {
    // About one unit per workgroup over all batch rows, at most 64 rows (two weight-wave passes):
    // a single row spreads over the workgroups; many rows (lockstep batches, prefill blocks) take
    // up to 64 rows per unit, each unit's weights read once per batch row.
    const int per_row = silu ? 2 : 1;
    int ipw = (int)(((int64_t)items * g.B + grid - 1) / grid);
    if (g.epi == EPI_QKV_ROPE && (ipw & 1)) ++ipw;
    if (ipw > 64 / per_row) ipw = 64 / per_row;
    g.ipw = ipw;
    g.maxb = 0;
  } else {
    g.ipw = silu ? kRowThreads / 32 : kRowThreads / 16;
    g.maxb = 0;
  }
  g.parts = (items + g.ipw - 1) / g.ipw;
  *units = g.parts * g.B;
}

void plan_qgemm(GemvArgs& g, int grid, int* units) {
  const bool silu = g.epi == EPI_SILU_GATE;
  const int items = silu ? g.ff_hidden : g.L.out;
  const int btiles = (g.B + kTileBatch - 1) / kTileBatch;
  // a unit's time depends little on its rows (it is bound by the per-chunk latency), so 16-row
  // tiles are used only when they add no unit to the busiest workgroup
  auto busiest_units = [&](int tr) {
    const int ipw = silu ? tr / 2 : tr;
    const int u = (items + ipw - 1) / ipw * btiles;
    return (u + grid - 1) / grid;
  };
  const int tr = busiest_units(kTileRows / 2) <= busiest_units(kTileRows) ? kTileRows / 2 : kTileRows;
  g.ipw = silu ? tr / 2 : tr;
  g.parts = (items + g.ipw - 1) / g.ipw;
  g.maxb = 0;
  *units = g.parts * btiles;
}

size_t phase_smem(const Phase& ph) {
  switch (ph.kind) {
    case PH_GEMV: {
      const GemvArgs& g = ph.g;
      const int K = g.L.in;
      if (g.L.fmt == FMT_Q8_0 || g.L.fmt == FMT_Q4_0) {
        const int nb = K / 32, nb4 = (nb + 3) & ~3;
        return (size_t)norm_scratch_floats(K) * 4 + K + (size_t)nb4 * 8 + (size_t)2 * g.ipw * q8_row_stride(nb) * 4 +
               (size_t)2 * g.ipw * 4 + 64;
      }
      if (g.L.fmt == FMT_Q4K) {
        const int nb = K / 256, nb4 = (nb + 3) & ~3, ts = 2 * g.ipw + 1;
        return (size_t)norm_scratch_floats(K) * 4 + K + (size_t)nb4 * 4 + (size_t)nb * 16 * 4 +
               (size_t)nb * ts * kQ4TermStride * 4 + 16 + (size_t)2 * g.ipw * 4 + 64;
      }
      if (g.L.fmt == FMT_F32C || g.L.fmt == FMT_BF16C)
        return (size_t)dense_base_bytes(K, g.ipw, g.norm != NORM_NONE) +
               (size_t)dense_stage_bytes(K, g.ipw, g.epi == EPI_SILU_GATE ? 2 * g.ipw : g.ipw, g.L.fmt == FMT_BF16C,
                                         g.norm != NORM_NONE);
      return (size_t)norm_scratch_floats(K) * 4 + (kRowThreads / 16) * 4 + 64;
    }
    case PH_ATTN:
      return (size_t)kAttnStages * kAttnChunkBytes + (size_t)(ph.at.hpu * (((ph.at.cap + 7) & ~7) + 8) + 4 + 32) * 4 + 64;
    case PH_ARGMAX:
      return 32 * 4 + 64;
    case PH_NORM:
      return (size_t)norm_scratch_floats(ph.nm.d) * 4 + 64;
    case PH_EMBED:
      return (size_t)(ph.e.n_q + 1) * 4 + 64;
    case PH_QUANT: {
      const int K = ph.g.L.in, nb4 = (K / 32 + 3) & ~3;
      return (size_t)norm_scratch_floats(K) * 4 + K + (size_t)nb4 * 4 + 64;
    }
    case PH_QGEMM:
      return (size_t)kTileRows * kTileBatch * 4 + (size_t)kGemmStages * kGemmStageBytes + 64;
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

// ---- Q4_0 ---------------------------------------------------------------------------------------
// candle BlockQ4_0::from_float on the GPU: one thread per 32-value block.  max = the value of
// largest magnitude (the first on ties), d = max / -8, id = 1 / d (0 if d = 0), code =
// min(15, (x * id + 8.5) as u8) with Rust's saturating truncation.
__device__ __forceinline__ uint32_t cast_u8(float v) {
  if (v != v || v <= 0.0f) return 0u;
  if (v >= 255.0f) return 255u;
  return (uint32_t)v;
}

__global__ void q4_0_quantize_kernel(const float* w, size_t nblocks, uint8_t* qs, uint16_t* d) {
  size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  const float* x = w + blk * 32;
  float amax = 0.0f, mx = 0.0f;
  for (int j = 0; j < 32; ++j) {
    const float a = fabsf(x[j]);
    if (amax < a) {
      amax = a;
      mx = x[j];
    }
  }
  const float dd = mx / -8.0f;
  const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
  d[blk] = f32_to_f16(dd);
  for (int j = 0; j < 16; ++j) {
    const float x0 = x[j] * id, x1 = x[j + 16] * id;
    const uint32_t q0 = min(15u, cast_u8(x0 + 8.5f)), q1 = min(15u, cast_u8(x1 + 8.5f));
    qs[blk * 16 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

hipError_t launch_q4_0_quantize(const float* w, int rows, int K, uint8_t* qs, uint16_t* d, hipStream_t s) {
  size_t nb = (size_t)rows * (K / 32);
  hipLaunchKernelGGL(q4_0_quantize_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, w, nb, qs, d);
  return hipGetLastError();
}

// 18-byte candle blocks <-> split codes and scales.
__global__ void q4_0_from_blocks_kernel(const uint8_t* blocks, size_t nblocks, uint8_t* qs, uint16_t* d) {
  size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  const uint8_t* p = blocks + blk * 18;
  d[blk] = (uint16_t)(p[0] | (p[1] << 8));
  for (int j = 0; j < 16; ++j) qs[blk * 16 + j] = p[2 + j];
}

hipError_t launch_q4_0_from_blocks(const uint8_t* blocks, int rows, int K, uint8_t* qs, uint16_t* d, hipStream_t s) {
  size_t nb = (size_t)rows * (K / 32);
  hipLaunchKernelGGL(q4_0_from_blocks_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, blocks, nb, qs, d);
  return hipGetLastError();
}

__global__ void q4_0_to_blocks_kernel(const uint8_t* qs, const uint16_t* d, size_t nblocks, uint8_t* blocks) {
  size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  uint8_t* p = blocks + blk * 18;
  p[0] = (uint8_t)(d[blk] & 0xff);
  p[1] = (uint8_t)(d[blk] >> 8);
  for (int j = 0; j < 16; ++j) p[2 + j] = qs[blk * 16 + j];
}

hipError_t launch_q4_0_to_blocks(const uint8_t* qs, const uint16_t* d, int rows, int K, uint8_t* blocks, hipStream_t s) {
  size_t nb = (size_t)rows * (K / 32);
  hipLaunchKernelGGL(q4_0_to_blocks_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, qs, d, nb, blocks);
  return hipGetLastError();
}

// ---- Q4K ----------------------------------------------------------------------------------------
// Device layout: candle's 144-byte BlockQ4K with the quant bytes of each 32-byte group
// lane-grouped (device byte 4 l + g = candle byte 8 g + l; see q4k_lane_pos).

__device__ __forceinline__ int32_t sat_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483647.0f) return 2147483647;
  if (v <= -2147483648.0f) return (-2147483647 - 1);
  return (int32_t)v;
}
__device__ __forceinline__ int32_t nearest_int(float v) { return sat_i32(roundf(v)); }
// f32::max / f32::min (a NaN operand yields the other one).
__device__ __forceinline__ float rmax(float a, float b) { return a != a ? b : (b != b ? a : (a > b ? a : b)); }
__device__ __forceinline__ float rmin(float a, float b) { return a != a ? b : (b != b ? a : (a < b ? a : b)); }
// a < b under f32::total_cmp (-0.0 orders before +0.0).
__device__ __forceinline__ bool total_lt(float a, float b) {
  int32_t ia = __float_as_int(a), ib = __float_as_int(b);
  ia ^= (int32_t)(((uint32_t)(ia >> 31)) >> 1);
  ib ^= (int32_t)(((uint32_t)(ib >> 31)) >> 1);
  return ia < ib;
}

// GGML get_scale_min_k4: the 6-bit scale and min of sub-block j from the 12 packed bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& d, int& m) {
  if (j < 4) {
    d = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// make_qkx1_quants(nmax = 15, ntry = 5) of 32 values: iterative least-squares fit of a scale
// and a (non-positive) offset; returns scale and -offset.
__device__ void qkx1_fit(const float* x, float& scale_out, float& min_out) {
  constexpr int n = 32, nmax = 15, ntry = 5;
  uint8_t L[n];
  for (int i = 0; i < n; ++i) L[i] = 0;
  float mn = x[0], mx = x[0];
  for (int i = 1; i < n; ++i)
    if (total_lt(x[i], mn)) mn = x[i];  // first minimum
  for (int i = 1; i < n; ++i)
    if (!total_lt(x[i], mx)) mx = x[i];  // last maximum
  if (mx == mn) {
    scale_out = 0.0f;
    min_out = 0.0f;
    return;
  }
  mn = rmin(mn, 0.0f);
  float iscale = (float)nmax / (mx - mn);
  float scale = 1.0f / iscale;
  for (int itry = 0; itry < ntry; ++itry) {
    float sumlx = 0.0f;
    int32_t suml2 = 0;
    bool changed = false;
    for (int i = 0; i < n; ++i) {
      int32_t li = nearest_int(iscale * (x[i] - mn));
      li = li < 0 ? 0 : (li > nmax ? nmax : li);
      if ((uint8_t)li != L[i]) {
        L[i] = (uint8_t)li;
        changed = true;
      }
      sumlx += (x[i] - mn) * (float)li;
      suml2 += li * li;
    }
    scale = sumlx / (float)suml2;
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)L[i];
    mn = sum / (float)n;
    if (mn > 0.0f) mn = 0.0f;
    iscale = 1.0f / scale;
    if (!changed) break;
  }
  scale_out = scale;
  min_out = -mn;
}

// candle BlockQ4K::from_float on the GPU: one thread per 256-value super-block.
__global__ void q4k_quantize_kernel(const float* w, size_t nblocks, uint8_t* out) {
  const size_t blk = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blk >= nblocks) return;
  const float* xb = w + blk * 256;
  uint8_t* b = out + blk * 144;
  float mins[8], scales[8];
  for (int j = 0; j < 8; ++j) qkx1_fit(xb + 32 * j, scales[j], mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; ++j) max_scale = rmax(scales[j], max_scale);
  for (int j = 0; j < 8; ++j) max_min = rmax(mins[j], max_min);
  const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  uint8_t sc[12];
  for (int j = 0; j < 12; ++j) sc[j] = 0;
  for (int j = 0; j < 8; ++j) {
    const int32_t lsi = nearest_int(inv_scale * scales[j]);
    const int32_t lmi = nearest_int(inv_min * mins[j]);
    const uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
    const uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
    if (j < 4) {
      sc[j] = ls;
      sc[j + 4] = lm;
    } else {
      sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
      sc[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  const uint16_t dh = f32_to_f16(max_scale / 63.0f), mh = f32_to_f16(max_min / 63.0f);
  b[0] = (uint8_t)(dh & 0xFF);
  b[1] = (uint8_t)(dh >> 8);
  b[2] = (uint8_t)(mh & 0xFF);
  b[3] = (uint8_t)(mh >> 8);
  for (int j = 0; j < 12; ++j) b[4 + j] = sc[j];
  const float dd = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t L[256];
  for (int i = 0; i < 256; ++i) L[i] = 0;
  for (int j = 0; j < 8; ++j) {
    int s, m;
    scale_min_k4(j, sc, s, m);
    const float d = dd * (float)s;
    if (d != 0.0f) {
      const float dm = dmin * (float)m;
      for (int ii = 0; ii < 32; ++ii) {
        int32_t l = nearest_int((xb[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : (l > 15 ? 15 : l));
      }
    }
  }
  // candle byte 32 g + e of group g holds L[64 g + e] | L[64 g + 32 + e] << 4
  for (int g = 0; g < 4; ++g)
    for (int e = 0; e < 32; ++e)
      b[16 + 32 * g + q4k_lane_pos(e)] = (uint8_t)(L[64 * g + e] | (L[64 * g + 32 + e] << 4));
}

hipError_t launch_q4k_quantize(const float* w, int rows, int K, uint8_t* blocks, hipStream_t s) {
  const size_t nb = (size_t)rows * (K / 256);
  hipLaunchKernelGGL(q4k_quantize_kernel, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, s, w, nb, blocks);
  return hipGetLastError();
}

// candle blocks <-> device blocks (the quant bytes regrouped, everything else as it is).
__global__ void q4k_regroup_kernel(const uint8_t* src, size_t nblocks, uint8_t* dst, bool to_device) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= nblocks * 144) return;
  const size_t blk = i / 144;
  const int o = (int)(i - blk * 144);
  int t = o;
  if (o >= 16) {
    const int g = (o - 16) / 32, e = (o - 16) % 32;
    t = 16 + 32 * g + q4k_lane_pos(e);
  }
  if (to_device) dst[blk * 144 + t] = src[i];
  else dst[i] = src[blk * 144 + t];
}

hipError_t launch_q4k_from_blocks(const uint8_t* candle, int rows, int K, uint8_t* blocks, hipStream_t s) {
  const size_t nb = (size_t)rows * (K / 256);
  hipLaunchKernelGGL(q4k_regroup_kernel, dim3((unsigned)((nb * 144 + 255) / 256)), dim3(256), 0, s, candle, nb, blocks, true);
  return hipGetLastError();
}

hipError_t launch_q4k_to_blocks(const uint8_t* blocks, int rows, int K, uint8_t* candle, hipStream_t s) {
  const size_t nb = (size_t)rows * (K / 256);
  hipLaunchKernelGGL(q4k_regroup_kernel, dim3((unsigned)((nb * 144 + 255) / 256)), dim3(256), 0, s, blocks, nb, candle, false);
  return hipGetLastError();
}

// Q4K closed form of element e (< 256) of a device block: (d * sc) * q - dmin * m, unfused.
__device__ float q4k_value(const uint8_t* b, int e) {
  const float d = f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
  const float dmin = f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
  const int g = e / 64, hi = (e % 64) >= 32, ee = e % 32;
  const uint8_t byte = b[16 + 32 * g + q4k_lane_pos(ee)];
  const int q = hi ? byte >> 4 : byte & 0xF;
  int s, m;
  scale_min_k4(2 * g + hi, b + 4, s, m);
  const float d1 = d * (float)s, m1 = dmin * (float)m;
  const float t = d1 * (float)q;
  return t - m1;
}

// Position of element (row, col) of a [rows][K] matrix in the chain-packed layout with E elements
// per 16 bytes.
__host__ __device__ inline size_t chain_index(size_t row, int col, int K, int E) {
  const int l = col % 16, c = col / 16;
  return ((row * (K / (16 * E)) + c / E) * 16 + l) * E + c % E;
}

__global__ void chain_pack_kernel(const void* src, int src_bf16, size_t n, int K, void* dst, int dst_bf16) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const size_t row = i / K;
  const int col = (int)(i % K);
  const size_t o = chain_index(row, col, K, dst_bf16 ? 8 : 4);
  if (dst_bf16) {
    ((uint16_t*)dst)[o] = src_bf16 ? ((const uint16_t*)src)[i] : f32_to_bf16(((const float*)src)[i]);
  } else {
    ((float*)dst)[o] = src_bf16 ? bf16_to_f32(((const uint16_t*)src)[i]) : ((const float*)src)[i];
  }
}

hipError_t launch_chain_pack(const void* src, int src_bf16, int rows, int K, void* dst, int dst_bf16, hipStream_t s) {
  const size_t n = (size_t)rows * K;
  hipLaunchKernelGGL(chain_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, src_bf16, n, K, dst,
                     dst_bf16);
  return hipGetLastError();
}

// Dequantization: Q8_0 closed form q * f32(d); Q4K closed form; dense bf16 widening; f32 copy.
__global__ void dequant_kernel(LinearDev L, float* out) {
  size_t n = (size_t)L.out * L.in;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (L.fmt == FMT_Q8_0) out[i] = (float)((const int8_t*)L.w)[i] * f16_to_f32(L.scale[i / 32]);
  else if (L.fmt == FMT_Q4_0) {
    const size_t blk = i / 32;
    const int e = (int)(i % 32);
    const uint8_t byte = ((const uint8_t*)L.w)[blk * 16 + (e & 15)];
    const int code = e < 16 ? (byte & 0xF) : (byte >> 4);
    out[i] = (float)(code - 8) * f16_to_f32(L.scale[blk]);
  }
  else if (L.fmt == FMT_Q4K) out[i] = q4k_value((const uint8_t*)L.w + (i / 256) * 144, (int)(i % 256));
  else if (L.fmt == FMT_BF16) out[i] = bf16_to_f32(((const uint16_t*)L.w)[i]);
  else if (L.fmt == FMT_BF16C) out[i] = bf16_to_f32(((const uint16_t*)L.w)[chain_index(i / L.in, (int)(i % L.in), L.in, 8)]);
  else if (L.fmt == FMT_F32C) out[i] = ((const float*)L.w)[chain_index(i / L.in, (int)(i % L.in), L.in, 4)];
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

// The norm statistics of rows of x exactly as the step's norm prologues compute them (values
// staged by the row waves, element-order sums): out[r] = {sum of squares, sum} (the sum for
// LayerNorm only).  One workgroup of row waves per row.
template <int KP>
__global__ __launch_bounds__(kRowThreads) void row_stats_kernel(const float* x, int K, int norm, float* out) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  RowSync rs{&ws, 0u, true};  // a workgroup of row waves only
  float v[KP];
  load_row(x + (size_t)blockIdx.x * K, K, v);
  NormW<KP> nw;
#pragma unroll
  for (int u = 0; u < KP; ++u) nw.w[u] = 1.0f, nw.b[u] = 0.0f;
  norm_regs(v, K, norm, nw, 1e-5f, (float*)smem, rs);
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = ws.stats[0];
    out[2 * blockIdx.x + 1] = norm == NORM_LAYER ? ws.stats[1] : 0.0f;
  }
}

hipError_t launch_row_stats(const float* x, int rows, int K, int norm, float* out, hipStream_t s) {
  const size_t smem = (size_t)norm_scratch_floats(K) * 4;
  switch (row_slots(K)) {
    case 2: hipLaunchKernelGGL(row_stats_kernel<2>, dim3(rows), dim3(kRowThreads), smem, s, x, K, norm, out); break;
    case 4: hipLaunchKernelGGL(row_stats_kernel<4>, dim3(rows), dim3(kRowThreads), smem, s, x, K, norm, out); break;
    default: hipLaunchKernelGGL(row_stats_kernel<8>, dim3(rows), dim3(kRowThreads), smem, s, x, K, norm, out); break;
  }
  return hipGetLastError();
}

__global__ void activation_kernel(int kind, const float* x, size_t n, float* y) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  y[i] = kind == 0 ? ref_exp(v) : kind == 1 ? ref_silu(v) : kind == 2 ? ref_gelu_tanh(v) : ref_gelu_erf(v);
}

hipError_t launch_activation(int kind, const float* x, size_t n, float* y, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(activation_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kind, x, n, y);
  return hipGetLastError();
}

hipError_t launch_copy(const void* src, void* dst, size_t bytes, hipStream_t s) {
  const size_t n = bytes / 16;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, s, (const v4i*)src, (v4i*)dst, n);
  return hipGetLastError();
}

// A bare streaming read: n 16-byte pieces, four non-temporal loads in flight per thread, folded
// into one word per thread so that the loads stay live (out[thread] = xor of two words of each
// piece the thread read).
__global__ void __launch_bounds__(1024) read_kernel(const v4i* __restrict__ x, size_t n, uint32_t* out) {
  const size_t nt = (size_t)gridDim.x * blockDim.x, g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  size_t i = g;
  for (; i + 3 * nt < n; i += 4 * nt) {
    v4i a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = __builtin_nontemporal_load(x + i + u * nt);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= (uint32_t)a[u].x ^ (uint32_t)a[u].w;
  }
  for (; i < n; i += nt) {
    const v4i a = __builtin_nontemporal_load(x + i);
    acc ^= (uint32_t)a.x ^ (uint32_t)a.w;
  }
  out[g] = acc;
}

hipError_t launch_read(const void* src, size_t bytes, int blocks, int threads, uint32_t* out, hipStream_t s) {
  hipLaunchKernelGGL(read_kernel, dim3((unsigned)blocks), dim3((unsigned)threads), 0, s, (const v4i*)src, bytes / 16, out);
  return hipGetLastError();
}

}  // namespace svl
