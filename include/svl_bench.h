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

/* A bare streaming read of src[0..bytes) on device `device` by `blocks` workgroups of `threads`
 * threads (64 .. 1024, a multiple of 64; blocks 1 .. 65536), four non-temporal 16-byte loads in
 * flight per thread; out[t] (device memory, blocks * threads words) receives a fold of the words
 * thread t read.  bytes a multiple of 16, src 16-byte aligned.  Launched back to back over buffers
 * larger than every cache, it gives the per-launch floor of moving a kernel's bytes. */
int svl_bench_read(int device, const void* src, size_t bytes, int blocks, int threads, uint32_t* out, void* stream);

/* The norm statistics of `rows` rows of `k` f32 values (x: device memory, row-major) exactly as
 * the decode step's RMSNorm / LayerNorm prologues compute them -- candle-nn's CPU order, one f32
 * accumulator per row adding the elements in index order: out[2 r] = sum of x^2, out[2 r + 1] =
 * sum of x (LayerNorm; 0 for RMSNorm).  norm is SVL_NORM_RMS or SVL_NORM_LAYER (svl.h); k a
 * multiple of 4 in [4, 4096]; out device memory; enqueued on `stream`.  Exposes the summation
 * for numerics tests on chosen rows. */
int svl_bench_row_stats(int device, const float* x, int rows, int k, int norm, float* out, void* stream);

/* The step kernels' element functions on n f32 values (x, y: device memory, enqueued on `stream`):
 * kind 0 exp (the reference's Cody-Waite + Taylor exp), 1 SiLU, 2 GELU-tanh, 3 erf GELU -- the
 * functions the FF epilogues, the attention softmax and the flow head evaluate.  Exposes them for
 * the known-answer sweeps of the numerics tests. */
int svl_bench_activation(int device, int kind, const float* x, size_t n, float* y, void* stream);

/* Launches phase `phase` (program order) of the state's decode-step program -- program 0 the
 * STT step, 1 the TTS backbone step -- `reps` times back to back on the state's stream, after one
 * untimed launch, and returns the mean time per launch from HIP events around the batch (which
 * includes the gap between back-to-back launches).  An attention phase launches as the state's
 * next step would (split over several units per head when its streams' visible keys call for
 * it).  info[6] receives the phase's kind, weight
 * format, linear rows and input width (GEMV phases), work units and attention heads per unit.
 * The phases recompute their outputs from the state's current contents; use a state whose
 * contents do not matter afterwards (a duplicate). */
typedef struct svl_model svl_model;
typedef struct svl_state svl_state;
int svl_bench_phase(const svl_model* model, svl_state* state, int program, int phase, int reps,
                    float* us_per_launch, int* info);

#ifdef __cplusplus
}
#endif

#endif
