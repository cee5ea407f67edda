/*
 * rlk_stream_ceiling.h -- the streaming ceiling that the benchmark reports beside each
 * return-estimation kernel.  Not part of the rl_triton API: it has no counterpart in the
 * reference.  It is the copy-kernel ceiling of the same byte pattern: a kernel that
 * reads n_in float32 arrays and writes n_out, one 16-byte non-temporal access per array
 * per thread in 512-thread workgroups (the access pattern of the short-row scan kernel at
 * [4096, 128]), with no scan.  Output k is (k + 1) times the sum of the inputs, so no load
 * is dead.  Built into its own library, librlk_stream_ceiling.so.
 */
#ifndef RLK_STREAM_CEILING_H
#define RLK_STREAM_CEILING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* in: n_in (1..6) device pointers, out: n_out (1..2) device pointers, each array n
 * float32 elements, n a multiple of 4, every pointer 16-byte aligned.  Enqueued on
 * `stream` (a hipStream_t; NULL = the default stream).  Returns 0, -1 for an invalid
 * argument, -3 if the launch failed; n == 0 returns 0 without a launch. */
int rlk_stream_ceiling(const float* const* in, int n_in, float* const* out, int n_out,
                       int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif
