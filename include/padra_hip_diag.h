/* padra_hip_diag.h - diagnostics of libpadra_hip.so, outside the drop-in surface.
 *
 * padra_hip.h declares the entry points that replace the reference's kernels; a runtime
 * that drops the library in needs nothing else.  The functions below have no counterpart
 * in the reference: device self-checks of the identities two fast paths rely on, which a
 * deployment may run once at start-up, and the streaming copy that the benchmark times as
 * the practical HBM ceiling.  Same conventions and status codes as padra_hip.h.
 */
#ifndef PADRA_HIP_DIAG_H
#define PADRA_HIP_DIAG_H

#include "padra_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* padra_CheckFP8Paths: no counterpart in the reference.  Checks, over their whole domains,
 * the two identities padra_NormFP8's fast path relies on (the hardware E4M3 conversion, and
 * the reciprocal-plus-correction quotient) and writes the mismatch counts to counts[0..1]
 * (device memory, 2 x u64; both 0 when the fast path is exact).  About 4.4e9 evaluations,
 * a few milliseconds. */
int padra_CheckFP8Paths(void *stream, unsigned long long *counts);
/* padra_CheckQ8Path: no counterpart in the reference.  Checks the reciprocal form of the q8
 * KV code (kv_q8::Encode's RNE(x / scale), kv_q8.cuh:12-14) that the store kernels use on
 * heads whose scale is at least 2^-100: for every such BF16 maximum and every BF16
 * value up to it, both signs, the code equals the correctly rounded division's.  Writes the
 * mismatch count to counts[0] (device memory, u64; 0 when exact).  About 2.1e9
 * evaluations, a few milliseconds. */
int padra_CheckQ8Path(void *stream, unsigned long long *counts);
/* padra_StreamCopy: no counterpart in the reference.  Copies `bytes` (a multiple of 16;
 * 16-byte aligned pointers) with the best one-pass streaming kernel found for MI355X
 * (16-byte non-temporal loads, all before the stores); the bench times it at the chain's
 * byte count as the practical HBM ceiling. */
int padra_StreamCopy(void *stream, void *dst, const void *src, long long bytes);


#ifdef __cplusplus
}
#endif
#endif
