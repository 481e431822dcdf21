// Calibrated W4 quantization: GPTQ (Frantar et al., "GPTQ: Accurate Post-Training Quantization
// for Generative Pre-trained Transformers", 2022, Algorithm 1, one scale per row and 128-column
// group, columns in their natural order) writing the reference's on-disk format (Wq [N][K/8]
// uint32 low nibble first, S [N][K/128] bf16, w = (q - 8) * s), so that ns_w4_linear and every
// other consumer of the format reads its output unchanged. The reference quantizes by round to
// nearest only (kernels/quant/w4a16.cuh:272-297) and names calibrated methods as its next step
// (README.md:233-235).
//
// Arithmetic, fixed so that a sequential CPU restatement reproduces it bit for bit:
//  * column i of a row is quantized as the round-to-nearest quantizer does (q = clamp(
//    rint_half_even(w / s) + 8, 0, 15)), with the group's scale s = bf16_rne(max|w| / 7) (1 for
//    an all-zero group) taken from the row's group values as they stand when the group starts;
//  * its error e = (w - (q - 8) s) / U[i][i] (the product is exact: |q - 8| <= 8 and s has an
//    8-bit significand) goes onto every later column j of the row as w_j <- fma(-e, U[i][j], w_j),
//    U the upper Cholesky factor of the damped inverse Hessian, computed by the caller;
//  * so every w_j receives its updates from i = 0, 1, ..., j - 1 in that order, one fused
//    multiply-add each, whichever of the two kernels below applies them.
//
// Kernels, per 128-column group k0:
//  * w4_gptq_group_kernel: the sequential part. One thread per row keeps the row's 128 group
//    values in registers and the group's 128 x 128 block of U in LDS, stored with each row shifted
//    to its diagonal (ub[i][d] = U[k0+i][k0+i+d], zero past the block) so that the column being
//    quantized is always register 0 and the update is a fixed, fully unrolled shift-and-FMA:
//    no register is ever indexed at run time. All lanes read the same LDS word (a broadcast).
//    It writes the group's codes and scale and the scaled errors E [128][N].
//  * w4_gptq_update_kernel: the columns after the group, W[:, k0+128:] updated by the 128 errors
//    of each row: a rank-128 update, i.e. a GEMM (N x 128) x (128 x rest) on fp32 FMAs in the
//    order above (no MFMA: its internal summation order is not the sequential chain). 128 x 128
//    output tiles per workgroup, 8 x 8 per thread, E and U staged through LDS 32 rows at a time.
#include <stdint.h>

#include "../../include/nanoserve_w4.h"
#include "w4_common.h"

namespace ns {
namespace {

constexpr int kGq = 128;      // group size: columns per group launch
constexpr int kUpTile = 128;  // update kernel: rows and columns per workgroup tile
constexpr int kUpK = 32;      // update kernel: error rows staged per LDS pass

__global__ void __launch_bounds__(64)
    w4_gptq_group_kernel(const float* __restrict__ W, const float* __restrict__ U,
                         uint32_t* __restrict__ Wq, uint16_t* __restrict__ S,
                         float* __restrict__ E, int N, int K, int k0) {
  __shared__ float ub[kGq][kGq];
  for (int idx = threadIdx.x; idx < kGq * kGq; idx += blockDim.x) {
    const int i = idx / kGq, d = idx % kGq;
    ub[i][d] = i + d < kGq ? U[(size_t)(k0 + i) * K + k0 + i + d] : 0.f;
  }
  __syncthreads();
  const long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N) return;

  const float* wr = W + row * K + k0;
  float w[kGq];
#pragma unroll
  for (int i = 0; i < kGq; i += 4) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(wr + i);
    w[i] = v[0];
    w[i + 1] = v[1];
    w[i + 2] = v[2];
    w[i + 3] = v[3];
  }
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < kGq; ++i) mx = fmaxf(mx, fabsf(w[i]));
  const uint32_t sb = f32_to_bf16_rne(mx > 0.f ? mx / 7.f : 1.f);
  const float sf = bf16_bits_to_f32(sb);
  S[row * (K / kGq) + k0 / kGq] = static_cast<uint16_t>(sb);

  uint32_t* qr = Wq + row * (K >> 3) + (k0 >> 3);
  uint32_t word = 0u;
#pragma unroll 1
  for (int i = 0; i < kGq; ++i) {
    const float c = w[0];
    int q = (int)((uint32_t)f2i_rn(c / sf) + 8u);
    q = q < 0 ? 0 : (q > 15 ? 15 : q);
    const float e = fmaf(-static_cast<float>(q - 8), sf, c) / ub[i][0];
    E[(size_t)i * N + row] = e;
    word = (word >> 4) | (static_cast<uint32_t>(q) << 28);
    if ((i & 7) == 7) qr[i >> 3] = word;
#pragma unroll
    for (int d = 1; d < kGq; ++d) w[d - 1] = fmaf(-e, ub[i][d], w[d]);
    w[kGq - 1] = 0.f;
  }
}

// W[n][j] for j >= k0 + 128: acc = W[n][j], then acc = fma(-E[i][n], U[k0+i][j], acc) for
// i = 0 .. 127 in order. Thread t owns rows n0 + 8 (t / 16) + a and columns j0 + 8 (t % 16) + b.
__global__ void __launch_bounds__(256)
    w4_gptq_update_kernel(float* __restrict__ W, const float* __restrict__ U,
                          const float* __restrict__ E, int N, int K, int k0) {
  __shared__ float es[kUpK][kUpTile];
  __shared__ float us[kUpK][kUpTile];
  const int t = threadIdx.x;
  const int tn = t >> 4, tj = t & 15;
  const long long n0 = (long long)blockIdx.x * kUpTile;
  const int j0 = k0 + kGq + blockIdx.y * kUpTile;

  float acc[8][8];
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const long long n = n0 + 8 * tn + a;
    if (n < N) {
      const float* src = W + n * K + j0 + 8 * tj;
      const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(src);
      const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(src + 4);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        acc[a][b] = lo[b];
        acc[a][b + 4] = hi[b];
      }
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[a][b] = 0.f;
    }
  }

  for (int i0 = 0; i0 < kGq; i0 += kUpK) {
    __syncthreads();
    // stage E[i0 .. i0+31][n0 .. n0+127] and U[k0+i0 .. +31][j0 .. j0+127]: 4 x 4 floats a thread
#pragma unroll
    for (int s = 0; s < kUpK * kUpTile / (256 * 4); ++s) {
      const int idx = (s * 256 + t) * 4;
      const int r = idx / kUpTile, c = idx % kUpTile;
      f32x4_t ev = {0.f, 0.f, 0.f, 0.f};
      const float* ep = E + (size_t)(i0 + r) * N + n0 + c;
      if (n0 + c + 3 < N && (N & 3) == 0) {
        ev = *reinterpret_cast<const f32x4_t*>(ep);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) ev[q] = n0 + c + q < N ? ep[q] : 0.f;
      }
      *reinterpret_cast<f32x4_t*>(&es[r][c]) = ev;
      *reinterpret_cast<f32x4_t*>(&us[r][c]) =
          *reinterpret_cast<const f32x4_t*>(U + (size_t)(k0 + i0 + r) * K + j0 + c);
    }
    __syncthreads();
#pragma unroll 4
    for (int i = 0; i < kUpK; ++i) {
      const f32x4_t e0 = *reinterpret_cast<const f32x4_t*>(&es[i][8 * tn]);
      const f32x4_t e1 = *reinterpret_cast<const f32x4_t*>(&es[i][8 * tn + 4]);
      const f32x4_t u0 = *reinterpret_cast<const f32x4_t*>(&us[i][8 * tj]);
      const f32x4_t u1 = *reinterpret_cast<const f32x4_t*>(&us[i][8 * tj + 4]);
      const float ev[8] = {-e0[0], -e0[1], -e0[2], -e0[3], -e1[0], -e1[1], -e1[2], -e1[3]};
      const float uv[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[a][b] = fmaf(ev[a], uv[b], acc[a][b]);
    }
  }

#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const long long n = n0 + 8 * tn + a;
    if (n < N) {
      float* dst = W + n * K + j0 + 8 * tj;
      *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{acc[a][0], acc[a][1], acc[a][2], acc[a][3]};
      *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{acc[a][4], acc[a][5], acc[a][6], acc[a][7]};
    }
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace
}  // namespace ns

extern "C" {

size_t ns_w4_gptq_workspace(int N) {
  return N > 0 ? static_cast<size_t>(ns::kGq) * static_cast<size_t>(N) * sizeof(float) : 0;
}

int ns_w4_gptq(void* W, const void* U, void* Wq, void* S, void* work, size_t work_bytes, int N,
               int K, int G, void* stream) {
  if (G != ns::kGq || N <= 0 || K <= 0 || K % G) return -2;
  if (!W || !U || !Wq || !S || !work || work_bytes < ns_w4_gptq_workspace(N)) return -2;
  if (!ns::aligned(W, 16) || !ns::aligned(U, 16) || !ns::aligned(Wq, 16) || !ns::aligned(S, 2) ||
      !ns::aligned(work, 16))
    return -2;
  const auto st = static_cast<hipStream_t>(stream);
  auto w = static_cast<float*>(W);
  const auto u = static_cast<const float*>(U);
  auto e = static_cast<float*>(work);
  const unsigned grow = static_cast<unsigned>((N + 63) / 64);
  const unsigned gup = static_cast<unsigned>((N + ns::kUpTile - 1) / ns::kUpTile);
  for (int k0 = 0; k0 < K; k0 += G) {
    hipLaunchKernelGGL(ns::w4_gptq_group_kernel, dim3(grow), dim3(64), 0, st, w, u,
                       static_cast<uint32_t*>(Wq), static_cast<uint16_t*>(S), e, N, K, k0);
    const int rest = K - k0 - G;
    if (rest > 0)
      hipLaunchKernelGGL(ns::w4_gptq_update_kernel, dim3(gup, rest / ns::kUpTile), dim3(256), 0,
                         st, w, u, e, N, K, k0);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return static_cast<int>(err);
  }
  return 0;
}

}  // extern "C"
