// bf16 GEMV for one token (M = 1), for the decode step's lm_head: y[n] = x . W[n], W [N][K]
// bf16 row-major, fp32 accumulation, bf16 (RNE) output -- the reference's
// F.linear(h, lm_head) (python/nanoserve/qwen.py:164), which it runs through cuBLAS. Optionally
// the final residual add + RMSNorm is fused into the activation load (the reference's
// `norm(x, d, final_norm)` of qwen.py:161-162 followed by the lm_head).
//
// HBM-bound (the lm_head of Qwen2.5-7B is 1.09 GB of bf16 per token). Organisation for
// gfx950:
//  * a wave owns whole rows: each row is read as consecutive 1 KiB wave loads (16 bytes per
//    lane), so HBM sees long sequential runs; the next row's loads are issued before the
//    current row is reduced, so a wave always has a row in flight;
//  * every wave holds the whole activation in registers (lane l keeps elements
//    512 b + 8 l .. +8 of each 512-element block b), so no LDS and no barriers: with the norm
//    fused, each wave computes the row's sum of squares itself (one wave reduction);
//  * products on v_dot2c_f32_bf16 (two bf16 products per instruction, fp32 accumulate), one
//    64-lane reduction per row.
#include <stdint.h>

#include "../../include/nanoserve_decode.h"
#include "w4_common.h"
#include "w4_kernels.h"

namespace ns {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Waves per workgroup. At the largest K (MAXKB 16) a wave holds three 64-register row buffers
// (current row, next row, activation); four-wave workgroups let it use the accumulation
// registers as well, so nothing spills to memory.
template <int MAXKB>
constexpr int lm_waves() { return MAXKB > 8 ? 4 : 8; }

// The vector elements are copied to scalars before the bit casts: this compiler, given
// __builtin_bit_cast of a vector element directly, emits the first element's register for all
// four products (checked in the generated code).
__device__ __forceinline__ float dot8(const u32x4_t& a, const u32x4_t& b, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ai = a[i], bi = b[i];
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, ai),
                                          __builtin_bit_cast(bf16x2_t, bi), acc, false);
  }
  return acc;
}

// MAXKB: 512-element blocks per row the registers are sized for; KB = ceil(K / 512) <= MAXKB.
template <int MAXKB, bool kNorm>
__global__ void __launch_bounds__(lm_waves<MAXKB>() * kWave)
    bf16_gemv_kernel(const uint16_t* __restrict__ X, const uint16_t* __restrict__ res,
                     const uint16_t* __restrict__ radd, const uint16_t* __restrict__ nw,
                     float eps, const uint16_t* __restrict__ W, uint16_t* __restrict__ Y, int N,
                     int K) {
  const int lane = threadIdx.x & (kWave - 1);
  const int KB = (K + 511) >> 9;
  constexpr int kLmWaves = lm_waves<MAXKB>();
  const long long wave0 = (long long)blockIdx.x * kLmWaves + (threadIdx.x >> 6);
  const long long nwaves = (long long)gridDim.x * kLmWaves;

  // the row loads of this wave's first row go out before anything else
  u32x4_t cur[MAXKB], nxt[MAXKB];
  long long row = wave0;
  auto load_row = [&](long long r, u32x4_t (&dst)[MAXKB]) {
    const uint16_t* base = W + r * K;
#pragma unroll
    for (int b = 0; b < MAXKB; ++b) {
      const int k = 512 * b + 8 * lane;
      // read once per token: non-temporal, as the W4 weight streams
      dst[b] = b < KB && k < K ? __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + k))
                               : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  if (row < N) load_row(row, cur);

  // the activation slice of this lane (zeros past K)
  u32x4_t xv[MAXKB];
  if constexpr (kNorm) {
    float v[MAXKB][8];
    float ss = 0.f;
#pragma unroll
    for (int b = 0; b < MAXKB; ++b) {
      const int k = 512 * b + 8 * lane;
      const bool in = b < KB && k < K;
      unpack8(in ? *reinterpret_cast<const u32x4_t*>(res + k) : u32x4_t{0u, 0u, 0u, 0u}, v[b]);
      if (radd) {
        float a[8];
        unpack8(in ? *reinterpret_cast<const u32x4_t*>(radd + k) : u32x4_t{0u, 0u, 0u, 0u}, a);
#pragma unroll
        for (int q = 0; q < 8; ++q) v[b][q] = round_bf16(v[b][q] + a[q]);
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) ss = fmaf(v[b][q], v[b][q], ss);
    }
    const float inv = rsqrtf(wave_sum(ss) / static_cast<float>(K) + eps);
#pragma unroll
    for (int b = 0; b < MAXKB; ++b) {
      const int k = 512 * b + 8 * lane;
      float g[8], o[8];
      unpack8(b < KB && k < K ? *reinterpret_cast<const u32x4_t*>(nw + k)
                              : u32x4_t{0u, 0u, 0u, 0u}, g);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = v[b][q] * inv * g[q];
      xv[b] = pack8(o);
    }
  } else {
#pragma unroll
    for (int b = 0; b < MAXKB; ++b) {
      const int k = 512 * b + 8 * lane;
      xv[b] = b < KB && k < K ? *reinterpret_cast<const u32x4_t*>(X + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
  }

  for (; row < N; row += nwaves) {
    const long long next = row + nwaves;
    if (next < N) load_row(next, nxt);
    float acc = 0.f;
#pragma unroll
    for (int b = 0; b < MAXKB; ++b)
      if (b < KB) acc = dot8(cur[b], xv[b], acc);
    acc = wave_sum(acc);
    if (lane == 0) Y[row] = static_cast<uint16_t>(f32_to_bf16_rne(acc));
#pragma unroll
    for (int b = 0; b < MAXKB; ++b) cur[b] = nxt[b];
  }
}

template <int MAXKB>
void launch_bf16(const uint16_t* X, const uint16_t* res, const uint16_t* radd,
                 const uint16_t* nw, float eps, const uint16_t* W, uint16_t* Y, int N, int K,
                 hipStream_t st) {
  constexpr int kLmWaves = lm_waves<MAXKB>();
  int cus = 0;
  if (cached_cu_count(&cus) != hipSuccess) cus = 256;  // the launch's own error is reported
  const long long blocks = (static_cast<long long>(N) + kLmWaves - 1) / kLmWaves;
  const long long cap = (MAXKB > 8 ? 1LL : 2LL) * cus;  // workgroups resident at once
  const int grid = static_cast<int>(blocks < cap ? blocks : cap);
  if (res)
    hipLaunchKernelGGL((bf16_gemv_kernel<MAXKB, true>), dim3(grid), dim3(kLmWaves * kWave), 0, st,
                       X, res, radd, nw, eps, W, Y, N, K);
  else
    hipLaunchKernelGGL((bf16_gemv_kernel<MAXKB, false>), dim3(grid), dim3(kLmWaves * kWave), 0,
                       st, X, res, radd, nw, eps, W, Y, N, K);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace
}  // namespace ns

extern "C" {

int ns_bf16_gemv(const void* X, const void* res, const void* r, const void* norm_w, float eps,
                 const void* W, void* Y, int N, int K, void* stream) {
  if (N <= 0 || K <= 0 || K % 8 || K > 8192) return -2;
  if (!W || !Y || (!res && !X) || (res && !norm_w)) return -2;
  if (!ns::aligned(W, 16) || !ns::aligned(Y, 2) || !ns::aligned(X, 16) || !ns::aligned(res, 16) ||
      !ns::aligned(r, 16) || !ns::aligned(norm_w, 16))
    return -2;
  const auto st = static_cast<hipStream_t>(stream);
  const auto x = static_cast<const uint16_t*>(X);
  const auto rs = static_cast<const uint16_t*>(res);
  const auto ra = static_cast<const uint16_t*>(r);
  const auto nw = static_cast<const uint16_t*>(norm_w);
  const auto w = static_cast<const uint16_t*>(W);
  const auto y = static_cast<uint16_t*>(Y);
  const int KB = (K + 511) / 512;
  if (KB <= 4)
    ns::launch_bf16<4>(x, rs, ra, nw, eps, w, y, N, K, st);
  else if (KB <= 8)
    ns::launch_bf16<8>(x, rs, ra, nw, eps, w, y, N, K, st);
  else
    ns::launch_bf16<16>(x, rs, ra, nw, eps, w, y, N, K, st);
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
