// Mimi's split residual vector quantizer, encoding (SVL/stt/model.rs:84-174), for gfx950.
//
// The codebook products use the 16-lane dot of the reference's own matvec kernel
// (SVL/nn/kernels/mod.rs:66-91): lane i of a 16-lane row accumulates dims i, i + 16, ... by FMA,
// then the rows' pairwise lane sum, then + 0.0 (the scalar tail's empty sum).  A stage is one
// launch: each workgroup takes kRvqBlock entries and kRvqTile rows, forms the rows' residuals in
// LDS, scores its entries against them and folds its per-row minimum into a 64-bit key per row
// (the score's order-preserving bits, then the entry index), so that the smallest key over all
// workgroups is the first index of the minimum score.
#include "device_math.h"
#include "rvq.h"

namespace svl {

namespace {

__global__ __launch_bounds__(256) void rvq_prepare_kernel(const float* sums, const float* usage, size_t entries,
                                                          float* emb, float* hn) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= entries) return;
  const float u = fmaxf(usage[e], 1e-5f);  // cluster_usage.maximum(1e-5)
  float s = 0.0f;
  for (int d = 0; d < kRvqDim; ++d) {
    const float v = sums[e * kRvqDim + d] / u;
    emb[e * kRvqDim + d] = v;
    const float sq = v * v;
    s = s + sq;
  }
  hn[e] = s * 0.5f + 0.0f;  // sum(D::Minus1) / 2.0
}

// Grid (kRvqDim / 32, rows, 2): 32 outputs of one row and part per workgroup of 512 threads.
__global__ __launch_bounds__(512) void rvq_project_kernel(const float* latents, int frames, const float* w_first,
                                                          const float* w_rest, int rows, float* proj) {
  __shared__ float x[kRvqIn];
  const int row = blockIdx.y, part = blockIdx.z;
  const int b = row / frames, t = row % frames;
  x[threadIdx.x] = latents[((size_t)b * kRvqIn + threadIdx.x) * frames + t];
  __syncthreads();
  const int li = threadIdx.x % 16, o = blockIdx.x * 32 + threadIdx.x / 16;
  const float* w = (part ? w_rest : w_first) + (size_t)o * kRvqIn;
  float acc = 0.0f;
#pragma unroll 8
  for (int u = 0; u < kRvqIn / 16; ++u) acc = fmaf(w[li + 16 * u], x[li + 16 * u], acc);
  acc = row16_pairwise_sum(acc);
  if (li == 0) proj[((size_t)part * rows + row) * kRvqDim + o] = acc + 0.0f;
}

// Bits of a float whose unsigned order is the float order (non-NaN).
__device__ __forceinline__ uint32_t order_bits(float f) {
  const uint32_t u = __float_as_uint(f + 0.0f);  // -0 as +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Grid (ceil(bins / kRvqBlock), ceil(rows / kRvqTile), chains), 512 threads.
__global__ __launch_bounds__(512) void rvq_stage_kernel(int k, int rows, int bins, const float* emb, const float* hn,
                                                        const float* proj, float* res_g, unsigned long long* keys) {
  __shared__ float res[kRvqTile][kRvqDim];
  __shared__ float sc[kRvqTile][kRvqBlock];
  const int chain = k == 0 ? (int)blockIdx.z : 1;  // 0: the first quantizer, 1: the rest
  const int stage = chain == 0 ? 0 : 1 + k;
  const int eb = blockIdx.x, r0 = blockIdx.y * kRvqTile, nr = min(kRvqTile, rows - r0);
  // ---- residuals of the tile's rows
  for (int i = threadIdx.x; i < nr * kRvqDim; i += blockDim.x) {
    const int r = i / kRvqDim, d = i % kRvqDim, row = r0 + r;
    float v;
    if (k == 0) {
      v = proj[((size_t)chain * rows + row) * kRvqDim + d];
    } else {
      const uint32_t idx = min((uint32_t)keys[(size_t)(stage - 1) * rows + row], (uint32_t)(bins - 1));
      v = res_g[((size_t)((k - 1) & 1) * rows + row) * kRvqDim + d] - emb[((size_t)(stage - 1) * bins + idx) * kRvqDim + d];
    }
    res[r][d] = v;
    if (chain == 1 && eb == 0) res_g[((size_t)(k & 1) * rows + row) * kRvqDim + d] = v;
  }
  __syncthreads();
  // ---- scores half_norm - residual . entry: group g of 16 lanes takes entries g and g + 32
  const int li = threadIdx.x % 16, g = threadIdx.x / 16;
  for (int ee = g; ee < kRvqBlock; ee += 32) {
    const int e = min(eb * kRvqBlock + ee, bins - 1);
    const float* ev = emb + ((size_t)stage * bins + e) * kRvqDim;
    float ent[kRvqDim / 16];
#pragma unroll
    for (int u = 0; u < kRvqDim / 16; ++u) ent[u] = ev[li + 16 * u];
    const float h = hn[(size_t)stage * bins + e];
    for (int r = 0; r < nr; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int u = 0; u < kRvqDim / 16; ++u) acc = fmaf(res[r][li + 16 * u], ent[u], acc);
      acc = row16_pairwise_sum(acc);
      if (li == 0) sc[r][ee] = h - (acc + 0.0f);
    }
  }
  __syncthreads();
  // ---- the first minimum of each row over the block's entries, folded into the row's key
  if ((int)threadIdx.x < nr) {
    const int r = threadIdx.x, n = min(kRvqBlock, bins - eb * kRvqBlock);
    int best = 0;
    float mn = sc[r][0];
    for (int ee = 1; ee < n; ++ee)
      if (sc[r][ee] < mn) {
        mn = sc[r][ee];
        best = ee;
      }
    const unsigned long long key = (unsigned long long)order_bits(mn) << 32 | (unsigned)(eb * kRvqBlock + best);
    atomicMin(&keys[(size_t)stage * rows + r0 + r], key);
  }
}

__global__ void rvq_codes_kernel(const unsigned long long* keys, int rows, int n_q, uint32_t* codes) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n_q) return;
  const int row = i / n_q, q = i % n_q;
  codes[i] = (uint32_t)keys[(size_t)q * rows + row];
}

}  // namespace

hipError_t launch_rvq_prepare(const float* sums, const float* usage, size_t entries, float* emb, float* hn,
                              hipStream_t s) {
  if (entries == 0) return hipSuccess;
  hipLaunchKernelGGL(rvq_prepare_kernel, dim3((unsigned)((entries + 255) / 256)), dim3(256), 0, s, sums, usage, entries,
                     emb, hn);
  return hipGetLastError();
}

hipError_t launch_rvq_project(const float* latents, int batch, int frames, const float* w_first, const float* w_rest,
                              float* proj, hipStream_t s) {
  const int rows = batch * frames;
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(rvq_project_kernel, dim3(kRvqDim / 32, rows, 2), dim3(512), 0, s, latents, frames, w_first, w_rest,
                     rows, proj);
  return hipGetLastError();
}

hipError_t launch_rvq_stage(int k, int n_q, int rows, int bins, const float* emb, const float* hn, const float* proj,
                            float* res, unsigned long long* keys, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const unsigned chains = k == 0 ? (n_q > 1 ? 2u : 1u) : 1u;
  hipLaunchKernelGGL(rvq_stage_kernel, dim3((bins + kRvqBlock - 1) / kRvqBlock, (rows + kRvqTile - 1) / kRvqTile, chains),
                     dim3(512), 0, s, k, rows, bins, emb, hn, proj, res, keys);
  return hipGetLastError();
}

hipError_t launch_rvq_codes(const unsigned long long* keys, int rows, int n_q, uint32_t* codes, hipStream_t s) {
  const int n = rows * n_q;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(rvq_codes_kernel, dim3((n + 255) / 256), dim3(256), 0, s, keys, rows, n_q, codes);
  return hipGetLastError();
}

}  // namespace svl
