/*
 * nanoserve_probe.h -- measurement kernels of libnanoserve_amd.so: the memory-system ceiling and
 * the launch floor that the W4 GEMV timings are reported against (bench.py). Not part of the
 * W4 linear-layer contract; same conventions as nanoserve_w4.h (device pointers, `stream` a
 * hipStream_t as void*, asynchronous, no allocation, return 0 / -2 / hipError_t).
 */
#ifndef NANOSERVE_PROBE_H
#define NANOSERVE_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Counterpart of the reference's bandwidth-ceiling kernel (bench/bench_w4a16.cu:122-136, a
 * 16-byte copy kernel timed in the same run as the GEMVs), as a read-only stream because a
 * GEMV only reads its weights: reads floor(bytes / 1024) KiB blocks of p with the W4 GEMV's
 * access pattern (one 1 KiB block per wave instruction, 16 bytes per lane, non-temporal buffer
 * loads), `grid` workgroups of `waves` wavefronts, `depth` (1, 2 or 4) loads in flight per
 * wave. sink [1] uint32 is written only for an input no test produces (it keeps the loads).
 * Returns -2 for bytes < 1024 or >= 2^31 - 2^16, grid outside 1..65535, waves outside 1..16,
 * another depth, NULL or misaligned pointers (p 16-byte, sink 4-byte).
 */
int ns_probe_read(const void* p, size_t bytes, void* sink, int grid, int waves, int depth,
                  void* stream);

/*
 * No counterpart in the reference: launches an empty kernel of `grid` workgroups of `threads`
 * threads (the per-launch floor of a graph of kernels). Returns -2 for grid outside 1..65535 or
 * threads outside 1..1024.
 */
int ns_probe_empty(int grid, int threads, void* stream);

/*
 * The reference's benchmark times back-to-back launches on one stream from its C++ host loop
 * (bench/bench_w4a16.cu:42-78); this is that loop for bench.py: ns_w4_linear(X[i], Wq[i],
 * S[i], Y[i], M[i], N[i], K[i], G, stream) for i = 0 .. ncalls - 1, in order, with no host
 * work between the launches. Returns 0, -2 for NULL arrays or ncalls < 1, or the first
 * non-zero return of ns_w4_linear (the launches before it were issued).
 */
int ns_probe_linear_loop(const void* const* X, const void* const* Wq, const void* const* S,
                         void* const* Y, const int* M, const int* N, const int* K, int G,
                         int ncalls, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOSERVE_PROBE_H */
