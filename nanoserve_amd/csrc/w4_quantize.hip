// W4 group quantizer: W [N][K] bf16 -> Wq [N][K/8] uint32 + S [N][K/G] bf16.
//
// Replaces quantize_w4_kernel / w4_quantize (kernels/quant/w4a16.cuh:272-301 in the reference),
// bit for bit: per (row, group) scale = bf16_rne(max|w| / 7) (1 for an all-zero group),
// q = clamp(rint_half_even(w / scale) + 8, 0, 15), packed low nibble first. The fp32 division
// is IEEE (correctly rounded), max is exact, so the result does not depend on evaluation order.
//
// One thread per packed output word (8 weights); the G / 8 threads of a group compute the
// group maximum together with cross-lane max when G / 8 is a power of two no larger than the
// wavefront, otherwise each thread scans its whole group.
#include "w4_common.h"
#include "w4_kernels.h"

namespace ns {

namespace {

__device__ __forceinline__ float abs_bf16(uint32_t h) { return bf16_bits_to_f32(h & 0x7fffu); }

template <bool kShuffle>
__global__ __launch_bounds__(256) void w4_quantize_kernel(const uint16_t* __restrict__ W,
                                                          uint32_t* __restrict__ Wq,
                                                          uint16_t* __restrict__ S, int N, int K,
                                                          int G) {
  const int KW = K >> 3, WPG = G >> 3, KG = K / G;
  const size_t total = (size_t)N * KW;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t base = (size_t)blockIdx.x * blockDim.x; base < total; base += stride) {
    const size_t idx = base + threadIdx.x;
    const bool live = idx < total;
    const size_t n = live ? idx / KW : 0;
    const int word = live ? (int)(idx - n * KW) : 0;
    const int g = word / WPG;
    const uint16_t* wrow = W + n * K;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wrow + (size_t)word * 8);
    float mx = 0.f;
    if (kShuffle) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        mx = fmaxf(mx, abs_bf16(v[i] & 0xffffu));
        mx = fmaxf(mx, abs_bf16(v[i] >> 16));
      }
      // Word-threads of one group are WPG consecutive lanes (WPG divides 64, groups never
      // straddle a row because K % G == 0), so an xor butterfly of width WPG is exact.
      for (int o = WPG >> 1; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    } else {
      const uint16_t* gp = wrow + (size_t)g * G;
      for (int i = 0; i < G; ++i) mx = fmaxf(mx, abs_bf16(gp[i]));
    }
    const uint32_t sb = f32_to_bf16_rne(mx > 0.f ? mx / 7.f : 1.f);
    const float sf = bf16_bits_to_f32(sb);
    uint32_t out = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t hbits = (i & 1) ? (v[i >> 1] >> 16) : (v[i >> 1] & 0xffffu);
      int q = (int)((uint32_t)f2i_rn(bf16_bits_to_f32(hbits) / sf) + 8u);
      q = q < 0 ? 0 : (q > 15 ? 15 : q);
      out |= (uint32_t)q << (4 * i);
    }
    if (live) {
      Wq[idx] = out;
      if (word % WPG == 0) S[n * KG + g] = (uint16_t)sb;
    }
  }
}

}  // namespace

hipError_t launch_quantize(const uint16_t* W, uint32_t* Wq, uint16_t* S, int N, int K, int G,
                           hipStream_t st) {
  const size_t words = (size_t)N * (K >> 3);
  const size_t blocks_needed = (words + 255) / 256;
  const int blocks = (int)(blocks_needed < 65536 ? blocks_needed : 65536);
  const int wpg = G >> 3;
  const bool pow2 = (wpg & (wpg - 1)) == 0 && wpg <= kWave;
  if (pow2)
    hipLaunchKernelGGL((w4_quantize_kernel<true>), dim3(blocks), dim3(256), 0, st, W, Wq, S, N, K,
                       G);
  else
    hipLaunchKernelGGL((w4_quantize_kernel<false>), dim3(blocks), dim3(256), 0, st, W, Wq, S, N,
                       K, G);
  return hipSuccess;
}

}  // namespace ns
