/*
 * svl_bench.h -- measurement helpers exported by libsvl.so.  They have no counterpart in the
 * reference: they exist to calibrate the HBM traffic counters that the decode-step kernel is
 * profiled with.
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

#ifdef __cplusplus
}
#endif

#endif
