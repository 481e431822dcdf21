// W4A16 prefill GEMM on gfx950 bf16 matrix cores.
//
// Replaces w4a16_gemm_kernel / w4a16_gemm_cfg / w4a16_gemm (kernels/quant/w4a16.cuh:117-270 in
// the reference):  C[M][N] (bf16, RNE) = A[M][K] (bf16) . deq(Wq, S)^T, fp32 accumulation.
//
// Numerics follow the reference GEMM exactly at the point that matters: each weight is staged
// as bf16_rne((q - 8) * s) (w4a16.cuh:190-198) before the bf16 multiply. Here that value is
// computed as fma(q, s, -8 s) (exact, since (q - 8) s has at most 12 significant bits) and
// rounded by the hardware RNE convert.
//
// Design:
//  * v_mfma_f32_32x32x16_bf16 with A = activations (row i = m), B = weights (column j = n).
//    A B-fragment lane holds 8 consecutive k of one column, which is exactly one packed word,
//    so weights go HBM -> VGPR -> dequant -> MFMA with no LDS round trip. Each wavefront owns
//    distinct columns (waves tile N only), so every weight is dequantized once per workgroup.
//  * The activation tile (BM x 64 bf16) is double-buffered in LDS (row pitch padded by 16 B
//    so the 16-byte fragment reads are bank-conflict free) and shared by all wavefronts.
//  * Within a 64-k block, lane (n, kh) loads words 4kh..4kh+3 of its row with one 16-byte
//    load (k = 32 kh .. 32 kh + 31); k16-step s uses word 4 kh + s, and the A fragment is read
//    at the same permuted k offset (32 kh + 8 s), so both operands agree on k.
//  * Next block's A tile (global -> registers) and weights are issued before the current
//    block's MFMAs.
#include "w4_common.h"
#include "w4_kernels.h"

namespace ns {

namespace {

constexpr int BK = 64;
constexpr int APAD = 8;  // bf16 elements of row padding in the LDS activation tile

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// One packed word -> 8 staged weights bf16_rne((q - 8) * s), natural k order, as 4 bf16x2.
__device__ __forceinline__ u32x4_t dequant_word_bf16(uint32_t w, float s, float ns8) {
  const uint32_t t0 = w & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 in bytes 0..3
  const uint32_t t1 = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
  u32x4_t d;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = (float)((t0 >> (8 * j)) & 0xFFu);
    const float hi = (float)((t1 >> (8 * j)) & 0xFFu);
    d[j] = pack_bf16x2_rne(__builtin_fmaf(lo, s, ns8), __builtin_fmaf(hi, s, ns8));
  }
  return d;
}

template <int BM, int WN, int NWN>
__global__ __launch_bounds__(NWN * kWave) void w4_gemm_kernel(
    const uint16_t* __restrict__ A, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ C, int M, int N, int K, int G) {
  constexpr int THREADS = NWN * kWave;
  constexpr int MI = BM / 32, NJ = WN / 32, BN = WN * NWN;
  constexpr int LDA = BK + APAD;
  constexpr int A_CHUNKS = BM * BK / 8;          // 16-byte chunks per tile
  constexpr int A_PER_THREAD = A_CHUNKS / THREADS;
  static_assert(A_CHUNKS % THREADS == 0, "even activation-tile split");
  __shared__ __align__(16) uint16_t As[2][BM * LDA];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int KW = K >> 3, KG = K / G;
  const int KB = (K + BK - 1) / BK;

  // ---- activation tile loader (global -> registers -> LDS). Every load is issued for every
  // lane (addresses clamped into the tensor), so the number of loads in flight never depends
  // on the path; columns past K (only when K % 64 == 32) are zeroed when stored to LDS.
  const uint16_t* a_src[A_PER_THREAD];
  int a_dst[A_PER_THREAD], a_col[A_PER_THREAD];
#pragma unroll
  for (int p = 0; p < A_PER_THREAD; ++p) {
    const int v = tid + p * THREADS;
    const int row = v / (BK / 8), c8 = (v % (BK / 8)) * 8;
    const int gm = min(m0 + row, M - 1);  // rows past M are computed and dropped
    a_src[p] = A + (size_t)gm * K + c8;
    a_dst[p] = row * LDA + c8;
    a_col[p] = c8;
  }
  u32x4_t a_reg[A_PER_THREAD];
  auto load_a = [&](int kb) {
#pragma unroll
    for (int p = 0; p < A_PER_THREAD; ++p) {
      const int k0 = kb * BK + a_col[p] < K ? kb * BK : 0;
      a_reg[p] = *reinterpret_cast<const u32x4_t*>(a_src[p] + k0);
    }
  };
  auto store_a = [&](int stage, int kb) {
    if ((kb + 1) * BK > K) {  // tail block: zero the columns past K
#pragma unroll
      for (int p = 0; p < A_PER_THREAD; ++p)
        if (kb * BK + a_col[p] >= K) a_reg[p] = u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int p = 0; p < A_PER_THREAD; ++p)
      *reinterpret_cast<u32x4_t*>(&As[stage][a_dst[p]]) = a_reg[p];
  };

  // ---- weight loader: lane (n = lane % 32, kh = lane / 32), one 16-byte load per n-frag.
  // Words past the row end (K % 64 == 32 tail) are read from the row start instead; they meet
  // zero activations.
  const int ln = lane & 31, kh = lane >> 5;
  const u32x4_t* w_src[NJ];
  const uint16_t* s_src[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = min(n0 + wv * WN + 32 * j + ln, N - 1);  // columns past N are dropped
    w_src[j] = reinterpret_cast<const u32x4_t*>(Wq + (size_t)n * KW);
    s_src[j] = S + (size_t)n * KG;
  }
  struct WRegs {
    u32x4_t w[NJ];
    uint32_t s[NJ];  // bf16 bits of the group scale
  };
  auto load_w = [&](WRegs& r, int kb) {
    int word = kb * (BK / 8) + 4 * kh;  // first of this lane's 4 words
    word = word < KW ? word : 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      r.w[j] = w_src[j][word >> 2];
      r.s[j] = s_src[j][(word * 8) / G];
    }
  };

  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto compute = [&](int stage, const WRegs& r) {
    const uint16_t* as = As[stage];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t bfrag[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float sc = bf16_bits_to_f32(r.s[j]);
        bfrag[j] = dequant_word_bf16(r.w[j][s], sc, -8.f * sc);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const u32x4_t afrag =
            *reinterpret_cast<const u32x4_t*>(&as[(32 * i + ln) * LDA + 32 * kh + 8 * s]);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(afrag), as_bf16x8(bfrag[j]),
                                                              acc[i][j], 0, 0, 0);
      }
    }
  };

  // ---- main loop, unrolled by two K blocks: LDS stage and weight registers alternate, so no
  // in-flight register is ever copied. Weights are loaded two blocks ahead, activations one.
  const int klast = KB - 1;
  WRegs wb0, wb1;
  load_w(wb0, 0);
  load_w(wb1, min(1, klast));
  load_a(0);
  store_a(0, 0);
  __syncthreads();
  int kb = 0;
  for (; kb + 1 < KB; kb += 2) {
    load_a(kb + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(0, wb0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wb0, min(kb + 2, klast));
    store_a(1, kb + 1);
    __syncthreads();

    load_a(min(kb + 2, klast));
    __builtin_amdgcn_sched_barrier(0);
    compute(1, wb1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wb1, min(kb + 3, klast));
    store_a(0, min(kb + 2, klast));
    __syncthreads();
  }
  if (kb < KB) compute(0, wb0);  // odd KB: the last block is in stage 0 / wb0

  // ---- epilogue: D[i][j] of lane l, register r: j = l % 32, i = 8 (r / 4) + 4 (l / 32) + r % 4
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = n0 + wv * WN + 32 * j + ln;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < M && n < N) C[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(acc[i][j][r]);
      }
    }
}

struct TileCfg {
  int bm, bn;
  float eff;  // relative per-tile efficiency used by the planner
};
constexpr TileCfg kCfgs[] = {
    {256, 256, 1.00f},  // 0: BM 256, 4 waves x 64 cols
    {256, 128, 0.90f},  // 1: BM 256, 4 waves x 32 cols
    {128, 256, 0.85f},  // 2: BM 128, 4 waves x 64 cols
    {128, 128, 0.75f},  // 3: BM 128, 4 waves x 32 cols
};

}  // namespace

GemmPlan gemm_plan(int M, int N, int K, int G) {
  (void)K;
  (void)G;
  constexpr int kCUs = 256;
  int best = 0;
  double best_cost = 1e300;
  for (int c = 0; c < (int)(sizeof(kCfgs) / sizeof(kCfgs[0])); ++c) {
    const long tiles = (long)((M + kCfgs[c].bm - 1) / kCfgs[c].bm) * ((N + kCfgs[c].bn - 1) / kCfgs[c].bn);
    const long rounds = (tiles + kCUs - 1) / kCUs;
    const double cost = (double)rounds * kCfgs[c].bm * kCfgs[c].bn / kCfgs[c].eff;
    if (cost < best_cost) {
      best_cost = cost;
      best = c;
    }
  }
  return GemmPlan{best, kCfgs[best].bm, kCfgs[best].bn};
}

hipError_t launch_gemm(const GemmArgs& a, const GemmPlan& p, hipStream_t st) {
  const dim3 grid((a.N + p.bn - 1) / p.bn, (a.M + p.bm - 1) / p.bm);
  switch (p.cfg) {
    case 0:
      hipLaunchKernelGGL((w4_gemm_kernel<256, 64, 4>), grid, dim3(256), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, a.G);
      return hipSuccess;
    case 1:
      hipLaunchKernelGGL((w4_gemm_kernel<256, 32, 4>), grid, dim3(256), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, a.G);
      return hipSuccess;
    case 2:
      hipLaunchKernelGGL((w4_gemm_kernel<128, 64, 4>), grid, dim3(256), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, a.G);
      return hipSuccess;
    case 3:
      hipLaunchKernelGGL((w4_gemm_kernel<128, 32, 4>), grid, dim3(256), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, a.G);
      return hipSuccess;
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace ns
