// Device-side scalar helpers shared by the step kernels.
//
// Everything here is compiled with -ffp-contract=off: a product is fused into an add only where
// fmaf() is written, which is where the reference's CPU kernels fuse (`mul_add::<FMA>`,
// SVL/nn/kernels/mod.rs:60-64).  The library targets gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svl {

constexpr int kWave = 64;

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// IEEE binary16 <-> f32 with the hardware conversions (v_cvt_f32_f16 / v_cvt_f16_f32: exact
// widening and round-to-nearest-even narrowing, f16 subnormals kept -- the `half` crate's
// f16::to_f32 / from_f32 for every non-NaN value).
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// The empty asm keeps the f32 value opaque: otherwise the compiler folds a preceding product into
// a mixed-precision FMA with a +0 addend (v_fma_mixlo_f16 x, c, 0), which turns a -0 product
// (candle's Q4_0 scale 0 / -8 of an all-zero block) into +0.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  __asm__ volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  if ((x & 0x8000u) && (x & 0x17fffu)) return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

// Rust `f as i8`: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i8(float v) {
  if (v != v) return 0;
  return v >= 127.0f ? 127 : (v <= -128.0f ? -128 : (int)v);
}

// The reference's branch-free exp (SVL/nn/kernels/mod.rs:93-131), FMA variant: Cody-Waite
// reduction with a split ln2 and a degree-8 Taylor expm1, clamped to [-87, 88].
__device__ __forceinline__ float ref_exp(float x) {
  const float LN2_HI = 0.69314575f, LN2_LO = 1.4286068e-6f, ROUND = 12582912.0f;
  const float LOG2E = 1.44269504088896340736f;
  float xc = x < -87.0f ? -87.0f : x;
  xc = xc > 88.0f ? 88.0f : xc;
  float shifted = fmaf(xc, LOG2E, ROUND);
  float k = shifted - ROUND;
  int32_t k_int = (int32_t)(f2u(shifted) - f2u(ROUND));
  float r = fmaf(-k, LN2_LO, fmaf(-k, LN2_HI, xc));
  float p = 1.0f / 40320.0f;
  p = fmaf(p, r, 1.0f / 5040.0f);
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  float two_k = u2f(((uint32_t)(k_int + 127)) << 23);
  float y = fmaf(two_k, p * r, two_k);
  if (x > 88.72f) y = __builtin_huge_valf();
  return x < -87.0f ? 0.0f : y;
}

// SVL/nn/kernels/activation.rs:70-82.
__device__ __forceinline__ float ref_silu(float x) { return x / (1.0f + ref_exp(-x)); }
__device__ __forceinline__ float ref_gelu_tanh(float x) {
  float a = 0.044715f * x;
  float x2 = x * x;
  float y = 0.7978846f * fmaf(a, x2, x);
  return x / (1.0f + ref_exp(-2.0f * y));
}
// Tensor::gelu_erf (SVL/nn/transformer.rs:446-447) as candle evaluates it for f32 [candle
// hypothesis]: in f64, (erf(v / sqrt 2) + 1) * 0.5 * v, rounded to f32; erf is the device
// library's f64 erf.
__device__ __forceinline__ float ref_gelu_erf(float x) {
  const double v = (double)x;
  return (float)((erf(v / 1.4142135623730951) + 1.0) * 0.5 * v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
// Lane 0 of each 16-lane row ends with the pairwise tree a[i] = a[i] + a[i + w], w = 8, 4, 2, 1,
// over the row's values: rotating the row by w and adding gives lane 0 the same operands at every
// node (up to their order, and a + b == b + a exactly).  DPP row_ror:w = 0x120 + w.
__device__ __forceinline__ float row16_pairwise_sum(float v) {
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// Lane moves inside a wave.  DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] =
// 0x4E, row_half_mirror (lane i of 8 <- 7 - i) = 0x141, row_mirror (lane i of 16 <- 15 - i) =
// 0x140.  ds_swizzle bitmask mode (offset bit 15 clear): source lane within the 32-lane group =
// ((lane & and) | or) ^ xor, with and = offset[4:0], or = offset[9:5], xor = offset[14:10].
template <int OFFSET>
__device__ __forceinline__ float swizzle(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), OFFSET));
}

// Maximum over the 32-lane half of the wave that the calling lane belongs to, in every lane, of
// non-negative floats given by their bit patterns (whose unsigned order is the float order).
__device__ __forceinline__ uint32_t half_max_bits(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));  // lane ^ 16
  return v;
}

// The sum of an int over each row of 16 lanes, in the row's last lane (DPP row shifts, in-row
// prefix sums; integer adds, so the order is immaterial).  Every lane of the wave must be active.
__device__ __forceinline__ int row16_isum_last(int s) {
  s += __builtin_amdgcn_update_dpp(0, s, 0x111, 0xf, 0xf, false);  // row_shr:1
  s += __builtin_amdgcn_update_dpp(0, s, 0x112, 0xf, 0xf, false);  // row_shr:2
  s += __builtin_amdgcn_update_dpp(0, s, 0x114, 0xf, 0xf, false);  // row_shr:4
  s += __builtin_amdgcn_update_dpp(0, s, 0x118, 0xf, 0xf, false);  // row_shr:8
  return s;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, not for its
// outstanding global loads (which __syncthreads would wait for).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace svl
