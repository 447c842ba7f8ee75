/*
 * Device-ceiling probes used by bench.py to price kernels whose bound is not
 * a published peak.  No counterpart in the reference.
 */
#ifndef GRAFT_DIAG_H
#define GRAFT_DIAG_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rate of fire-and-forget fp32 atomic-add requests (global_atomic_add_f32,
 * no return) to pseudo-random 64-byte lines of d_buf, each request carrying
 * dwords_per_line (1, 2, 4, 8 or 16) consecutive lanes of one line: the
 * ceiling of the hash-grid gradient scatter, whose cost per request does not
 * depend on how many dwords of the line it adds to.  Launches one workgroup
 * of 256 threads per CU, about 2^24 requests per launch, one warm-up launch
 * and 5 timed ones on `stream`, and blocks until they finish.  d_buf (at
 * least 64 KiB; its contents are overwritten) is used up to the largest
 * power-of-two number of lines it holds.  Writes line requests per second to
 * *requests_per_s.  Returns 0, or non-zero with tinymlp_last_error() set. */
int graft_diag_atomic_line_rate(float* d_buf, size_t bytes, int dwords_per_line, double* requests_per_s,
                                hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
