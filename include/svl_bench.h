/*
 * svl_bench.h -- measurement and numerics helpers exported by libsvl.so.  They have no
 * counterpart in the reference: they calibrate the HBM traffic counters the decode-step kernels
 * are profiled with, and expose the step's norm statistics to numerics tests.
 */
#ifndef SVL_BENCH_H
#define SVL_BENCH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dst[0..bytes) = src[0..bytes) on device `device` with one plain streaming copy kernel
 * (16-byte loads and stores), enqueued on `stream` (a hipStream_t, or NULL for the default
 * stream).  bytes must be a multiple of 16 and both pointers 16-byte aligned device memory. */
int svl_bench_copy(int device, const void* src, void* dst, size_t bytes, void* stream);

/* The norm statistics of `rows` rows of `k` f32 values (x: device memory, row-major) exactly as
 * the decode step's RMSNorm / LayerNorm prologues compute them -- candle-nn's CPU order, one f32
 * accumulator per row adding the elements in index order: out[2 r] = sum of x^2, out[2 r + 1] =
 * sum of x (LayerNorm; 0 for RMSNorm).  norm is SVL_NORM_RMS or SVL_NORM_LAYER (svl.h); k a
 * multiple of 4 in [4, 4096]; out device memory; enqueued on `stream`.  Exposes the summation
 * for numerics tests on chosen rows. */
int svl_bench_row_stats(int device, const float* x, int rows, int k, int norm, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif
