// Measurement kernels: the memory-system ceiling and the launch floor against which the W4 GEMV
// is judged. The reference measures its bandwidth ceiling with a 16-byte copy kernel in the same
// run as its GEMV timings (bench/bench_w4a16.cu:122-136) and reports every GEMV as a percentage
// of it. A GEMV only reads its weights, so the ceiling here is a read-only stream with the GEMV's
// own access pattern (1 KiB per wave instruction, 16 bytes per lane, non-temporal buffer loads);
// the launch floor is an empty kernel, whose per-launch time in a graph is what every launch
// pays before it moves a byte.
#include <stdint.h>

#include "../../include/nanoserve_probe.h"
#include "../../include/nanoserve_w4.h"
#include "w4_common.h"

namespace ns {
namespace {

// Wave w of the grid reads 1 KiB blocks w, w + W, w + 2W, ... (W = waves in the grid), DEPTH
// loads in flight per wave: the wave issues DEPTH loads, then folds them into a checksum. Blocks
// past the end read through the buffer's range check (zeros, no memory traffic). The checksum is
// stored only if it equals a value no input produces here, so the loads cannot be removed.
template <int DEPTH>
__global__ __launch_bounds__(1024) void probe_read_kernel(const uint32_t* __restrict__ p,
                                                          uint32_t nblk, uint32_t* __restrict__ sink) {
  constexpr uint32_t kOOB = 0x7fffffc0u;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t waves = gridDim.x * (blockDim.x >> 6);
  const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p), (short)0, (int)(nblk * 1024u), 0x00020000);
  uint32_t acc = 0;
  for (uint32_t b0 = wave; b0 < nblk; b0 += waves * DEPTH) {
    u32x4_t v[DEPTH];
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
      const uint32_t b = b0 + (uint32_t)r * waves;
      v[r] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs, 16u * lane, b < nblk ? 1024u * b : kOOB, kStreamAux));
    }
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) acc ^= v[r][0] ^ v[r][1] ^ v[r][2] ^ v[r][3];
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ void probe_empty_kernel() {}

}  // namespace
}  // namespace ns

extern "C" {

int ns_probe_read(const void* p, size_t bytes, void* sink, int grid, int waves, int depth,
                  void* stream) {
  if (!p || !sink || bytes < 1024 || bytes >= 0x7fff0000ull) return -2;
  if (grid < 1 || grid > 65535 || waves < 1 || waves > 16) return -2;
  if ((reinterpret_cast<uintptr_t>(p) & 15) || (reinterpret_cast<uintptr_t>(sink) & 3)) return -2;
  const uint32_t nblk = static_cast<uint32_t>(bytes / 1024);
  const auto st = static_cast<hipStream_t>(stream);
  const auto src = static_cast<const uint32_t*>(p);
  const auto out = static_cast<uint32_t*>(sink);
  switch (depth) {
    case 1: hipLaunchKernelGGL(ns::probe_read_kernel<1>, dim3(grid), dim3(64 * waves), 0, st, src, nblk, out); break;
    case 2: hipLaunchKernelGGL(ns::probe_read_kernel<2>, dim3(grid), dim3(64 * waves), 0, st, src, nblk, out); break;
    case 4: hipLaunchKernelGGL(ns::probe_read_kernel<4>, dim3(grid), dim3(64 * waves), 0, st, src, nblk, out); break;
    default: return -2;
  }
  return static_cast<int>(hipGetLastError());
}

int ns_probe_empty(int grid, int threads, void* stream) {
  if (grid < 1 || grid > 65535 || threads < 1 || threads > 1024) return -2;
  hipLaunchKernelGGL(ns::probe_empty_kernel, dim3(grid), dim3(threads), 0,
                     static_cast<hipStream_t>(stream));
  return static_cast<int>(hipGetLastError());
}

int ns_probe_linear_loop(const void* const* X, const void* const* Wq, const void* const* S,
                         void* const* Y, const int* M, const int* N, const int* K, int G, int ncalls,
                         void* stream) {
  if (!X || !Wq || !S || !Y || !M || !N || !K || ncalls < 1) return -2;
  for (int i = 0; i < ncalls; ++i) {
    const int rc = ns_w4_linear(X[i], Wq[i], S[i], Y[i], M[i], N[i], K[i], G, stream);
    if (rc != 0) return rc;
  }
  return 0;
}

}  // extern "C"
