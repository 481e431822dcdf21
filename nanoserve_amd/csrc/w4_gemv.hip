// W4A16 decode GEMV for M = 1..8 on gfx950 (CDNA4).
//
// Replaces w4a16_gemv_kernel / w4a16_gemv (kernels/quant/w4a16.cuh:34-115 in the reference):
//   Y[M][N] (bf16, RNE) = X[M][K] (bf16) . deq(Wq, S)^T, fp32 accumulation.
//
// Design (fast path, K % 128 == 0 and G % 128 == 0):
//  * A wavefront owns a 16-row tile of W (RT tiles) and a contiguous range of 128-k chunks;
//    the NW wavefronts of a workgroup split K (split-K inside the workgroup) and are reduced
//    through LDS at the end.
//  * Lane l = 16 h + r streams one 16-byte load of row r (words 4h..4h+3 of the chunk) per
//    chunk: the whole wave reads 1 KiB of packed weights per chunk per tile.
//  * The products run on the matrix cores: v_mfma_f32_16x16x32_bf16 with A = weights
//    (row i = output feature), B = X^T (column j = batch row, padded to 16). The weight operand
//    is the exact integer 128 + q in bf16 (0x4300 | q: one byte permute and one AND-OR per two
//    weights, no float arithmetic); a second MFMA with the constant -136 per chunk removes the
//    offset, so the chunk partial is sum_k x * (q - 8) exactly as the reference's integer
//    dequant, and the bf16 group scale is applied in fp32 after the chunk. No weight is ever
//    rounded: the dequant is exact, as in the reference GEMV (w4a16.cuh:28-32).
//  * Loads of W and X are issued in batches of UB chunks, so each wave has up to UB x RT KiB
//    of HBM reads in flight; several waves per SIMD overlap one another's batches.
//  * Scales for the workgroup's rows are staged once in LDS, transposed to [group][row] so a
//    lane reads its four rows' scales with one 8-byte LDS read.
//
// Generic path (any K % 32 == 0, G % 32 == 0, K % G == 0): one wavefront per output row,
// VALU fp32 FMAs with the exact fp32 dequant, cross-lane reduction.
#include "w4_common.h"
#include "w4_kernels.h"

namespace ns {

namespace {

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

template <int RT, int NW, int UB>
__global__ __launch_bounds__(NW * kWave) void w4_gemv_mfma_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int M, int N, int K, int G) {
  constexpr int ROWS = 16 * RT;
  extern __shared__ __align__(16) unsigned char smem[];
  const int KG = K / G;
  uint16_t* sl = reinterpret_cast<uint16_t*>(smem);  // [KG + 1][ROWS], group KG is all zero
  float* red = reinterpret_cast<float*>(smem + (((KG + 1) * ROWS * 2 + 15) & ~15));  // [NW][RT][4][64]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar chunk math
  const int n0 = blockIdx.x * ROWS;

  // Stage this tile's scales: rows n0..n0+ROWS-1 are one contiguous run of S.
  for (int e = tid; e < ROWS * KG; e += NW * kWave) {
    const int row = e / KG, g = e - row * KG;
    sl[g * ROWS + row] = (n0 + row < N) ? S[(size_t)n0 * KG + e] : (uint16_t)0;
  }
  for (int e = tid; e < ROWS; e += NW * kWave) sl[KG * ROWS + e] = 0;
  __syncthreads();

  const int r16 = lane & 15, h = lane >> 4;
  const int C = K >> 7;                          // 128-k chunks
  const int c0 = (C * wv) / NW, c1 = (C * (wv + 1)) / NW;
  const int cpg = G >> 7;                        // chunks per scale group

  const u32x4_t* wp[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = min(n0 + 16 * rt + r16, N - 1);  // rows past N are computed and dropped
    wp[rt] = reinterpret_cast<const u32x4_t*>(Wq + (size_t)row * (K >> 3)) + h;
  }
  // Batch columns j >= M of the MFMA are computed on a duplicate of row M-1 and never stored:
  // every lane loads valid memory, so no load needs a per-lane predicate.
  const u32x4_t* xp =
      reinterpret_cast<const u32x4_t*>(X + (size_t)min(r16, M - 1) * K) + 4 * h;

  f32x4_t acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};  // bf16 -136

  // Batches of UB chunks: all loads of a batch are issued back to back, then the chunks are
  // consumed in issue order, each waiting only for its own loads. The body has no branches:
  // chunk indices past the wave's range are clamped to its last chunk (valid memory) and read
  // the all-zero scale row, so they add nothing. Nothing is carried across batches.
  const int clast = c1 - 1;
  for (int cb = c0; cb < c1; cb += UB) {
    u32x4_t wb[UB][RT], xb[UB][4];
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int c = min(cb + u, clast);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) wb[u][rt] = wp[rt][4 * c];
#pragma unroll
      for (int s = 0; s < 4; ++s) xb[u][s] = xp[16 * c + s];
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any math
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int c = cb + u;
      const int g = c < c1 ? c / cpg : KG;
      // -136 * sum_k x over the chunk, shared by every row tile.
      f32x4_t corr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        corr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kNeg136), as_bf16x8(xb[u][s]),
                                                       corr, 0, 0, 0);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        f32x4_t t = corr;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          uint32_t d[4];
          unpack_word_128q(wb[u][rt][s], d);
          const u32x4_t a = {d[0], d[1], d[2], d[3]};
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(xb[u][s]), t, 0, 0, 0);
        }
        // t[r] = partial for row 16 rt + 4 h + r, batch row r16.
        const uint2 sv = *reinterpret_cast<const uint2*>(&sl[g * ROWS + 16 * rt + 4 * h]);
        acc[rt][0] = __builtin_fmaf(bf16_bits_to_f32(sv.x & 0xffffu), t[0], acc[rt][0]);
        acc[rt][1] = __builtin_fmaf(bf16_bits_to_f32(sv.x >> 16), t[1], acc[rt][1]);
        acc[rt][2] = __builtin_fmaf(bf16_bits_to_f32(sv.y & 0xffffu), t[2], acc[rt][2]);
        acc[rt][3] = __builtin_fmaf(bf16_bits_to_f32(sv.y >> 16), t[3], acc[rt][3]);
      }
    }
  }

  // Split-K reduction across the NW waves through LDS.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wv * RT + rt) * 4 + r) * kWave + lane] = acc[rt][r];
  __syncthreads();
  // Wave w finalises entries e = w, w + NW, ... of the RT*4 (tile, register) pairs.
  for (int e = wv; e < RT * 4; e += NW) {
    const int rt = e >> 2, r = e & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[((w * RT + rt) * 4 + r) * kWave + lane];
    const int n = n0 + 16 * rt + 4 * h + r;
    if (r16 < M && n < N) Y[(size_t)r16 * N + n] = (uint16_t)f32_to_bf16_rne(v);
  }
}

// Generic fallback: one wavefront per output row, exact fp32 dequant, fp32 FMA.
template <int MMAX>
__global__ __launch_bounds__(256) void w4_gemv_generic_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int M, int N, int K, int G) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int KW = K >> 3, KG = K / G;
  float acc[MMAX];
#pragma unroll
  for (int m = 0; m < MMAX; ++m) acc[m] = 0.f;
  for (int j = lane; j < KW; j += kWave) {
    const uint32_t q = Wq[(size_t)n * KW + j];
    const float s = bf16_bits_to_f32(S[(size_t)n * KG + (8 * j) / G]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float w = (float)((int)((q >> (4 * i)) & 0xFu) - 8) * s;
#pragma unroll
      for (int m = 0; m < MMAX; ++m)
        if (m < M) acc[m] = __builtin_fmaf(bf16_bits_to_f32(X[(size_t)m * K + 8 * j + i]), w, acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < MMAX; ++m) {
    float v = acc[m];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    if (lane == 0 && m < M) Y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v);
  }
}

template <int RT, int NW, int UB>
hipError_t launch_mfma(const GemvArgs& a, hipStream_t st) {
  const int KG = a.K / a.G;
  const size_t lds = (size_t)(((KG + 1) * 16 * RT * 2 + 15) & ~15) + (size_t)NW * RT * 4 * kWave * 4;
  const dim3 grid((a.N + 16 * RT - 1) / (16 * RT));
  hipLaunchKernelGGL((w4_gemv_mfma_kernel<RT, NW, UB>), grid, dim3(NW * kWave), lds, st, a.X,
                     a.Wq, a.S, a.Y, a.M, a.N, a.K, a.G);
  return hipSuccess;
}

}  // namespace

// Scale staging must fit comfortably in LDS next to the reduction buffer.
bool gemv_fast_path_ok(int M, int N, int K, int G) {
  (void)N;
  return M >= 1 && M <= 8 && K % 128 == 0 && G % 128 == 0 && (K / G + 1) * 32 * 2 <= 32768;
}

GemvPlan gemv_plan(int M, int N, int K, int G) {
  GemvPlan p{};
  p.fast = gemv_fast_path_ok(M, N, K, G);
  if (!p.fast) return p;
  const int C = K / 128;
  const int tiles1 = (N + 15) / 16;
  // Row tiles of 32 when there are plenty of rows (halves the X traffic per weight byte),
  // then split K over enough waves that the chip holds >= ~2048 waves, keeping >= 2 chunks
  // per wave.
  p.rt = tiles1 >= 2048 ? 2 : 1;
  const int tiles = (N + 16 * p.rt - 1) / (16 * p.rt);
  int nw = 1;
  while (nw < 8 && (long)tiles * nw < 2048 && C / (2 * nw) >= 2) nw *= 2;
  p.nw = nw;
  return p;
}

hipError_t launch_gemv(const GemvArgs& a, const GemvPlan& p, hipStream_t st) {
  if (!p.fast) {
    hipLaunchKernelGGL((w4_gemv_generic_kernel<8>), dim3((a.N + 3) / 4), dim3(256), 0, st, a.X,
                       a.Wq, a.S, a.Y, a.M, a.N, a.K, a.G);
    return hipSuccess;
  }
#define NS_GEMV_CASE(RT_, NW_)                                   \
  if (p.rt == RT_ && p.nw == NW_) return launch_mfma<RT_, NW_, 4>(a, st);
  NS_GEMV_CASE(1, 1)
  NS_GEMV_CASE(1, 2)
  NS_GEMV_CASE(1, 4)
  NS_GEMV_CASE(1, 8)
  NS_GEMV_CASE(2, 1)
  NS_GEMV_CASE(2, 2)
  NS_GEMV_CASE(2, 4)
  NS_GEMV_CASE(2, 8)
#undef NS_GEMV_CASE
  return hipErrorInvalidValue;
}

}  // namespace ns
