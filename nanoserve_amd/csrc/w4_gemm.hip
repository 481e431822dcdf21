// W4A16 prefill GEMM on gfx950 bf16 matrix cores.
//
// Replaces w4a16_gemm_kernel / w4a16_gemm_cfg / w4a16_gemm (kernels/quant/w4a16.cuh:117-270 in
// the reference):  C[M][N] (bf16, RNE) = A[M][K] (bf16) . deq(Wq, S)^T, fp32 accumulation.
//
// Numerics follow the reference GEMM exactly at the point that matters: each weight is staged
// as bf16_rne((q - 8) * s) (w4a16.cuh:190-198) before the bf16 multiply. Here that value is
// computed as fma(1024 + q, s, -1032 s) on an fp16 (1024 + q) (exact, since (q - 8) s has at
// most 12 significant bits) and rounded by the hardware RNE convert.
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
// One v_and_or_b32 per two nibbles builds an fp16 pair (1024 + q_a, 1024 + q_b): the nibbles
// land in the low mantissa bits of two halves whose exponent field (0x6400) means 1024
// (vmask = 0x000F000F in a VGPR, w shifted by 0/4/8/12 bits). The fp32 fma takes the fp16
// operand widened in the instruction itself (v_fma_mix_f32), so a weight costs half a logic op
// and one fma: fma(1024 + q, s, -1032 s) = (q - 8) s, exact because s is a bf16 (1032 s and
// (1024 + q) s fit fp32's 24-bit significand) for |s| < 2^118; v_cvt_pk_bf16_f32 then rounds
// to nearest even. The quantizer's scales (absmax / 7 of bf16 weights) are far below that
// bound.
__device__ __forceinline__ uint32_t and_or_s(uint32_t a, uint32_t vmask, uint32_t sbits) {
  uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(vmask), "s"(sbits));
  return d;
}

__device__ __forceinline__ u32x4_t dequant_word_bf16(uint32_t w, uint32_t vmask, float s,
                                                     float ns1032) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  constexpr uint32_t kE1024 = 0x64006400u;  // fp16 1024.0 in both halves
  const h2_t h0 = __builtin_bit_cast(h2_t, and_or_s(w, vmask, kE1024));        // q0, q4
  const h2_t h1 = __builtin_bit_cast(h2_t, and_or_s(w >> 4, vmask, kE1024));   // q1, q5
  const h2_t h2 = __builtin_bit_cast(h2_t, and_or_s(w >> 8, vmask, kE1024));   // q2, q6
  const h2_t h3 = __builtin_bit_cast(h2_t, and_or_s(w >> 12, vmask, kE1024));  // q3, q7
  u32x4_t d;
  d[0] = pack_bf16x2_rne(__builtin_fmaf((float)h0[0], s, ns1032), __builtin_fmaf((float)h1[0], s, ns1032));
  d[1] = pack_bf16x2_rne(__builtin_fmaf((float)h2[0], s, ns1032), __builtin_fmaf((float)h3[0], s, ns1032));
  d[2] = pack_bf16x2_rne(__builtin_fmaf((float)h0[1], s, ns1032), __builtin_fmaf((float)h1[1], s, ns1032));
  d[3] = pack_bf16x2_rne(__builtin_fmaf((float)h2[1], s, ns1032), __builtin_fmaf((float)h3[1], s, ns1032));
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

  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));

  // One 64-k block: four k16 steps, software-pipelined: while the 16 MFMAs of step s run, the
  // A fragments of step s + 1 are read from LDS and its B fragments dequantized; the group
  // barriers interleave them (1 MFMA, a few VALU ops, an LDS read, ...).
  auto compute = [&](int stage, const WRegs& r) {
    const uint16_t* as = As[stage];
    float sc[NJ], nb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      sc[j] = bf16_bits_to_f32(r.s[j]);
      nb[j] = -1032.f * sc[j];
    }
    u32x4_t af[2][MI], bf[2][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
      af[0][i] = *reinterpret_cast<const u32x4_t*>(&as[(32 * i + ln) * LDA + 32 * kh]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) bf[0][j] = dequant_word_bf16(r.w[j][0], vmask, sc[j], nb[j]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s < 3) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
          af[nxt][i] = *reinterpret_cast<const u32x4_t*>(&as[(32 * i + ln) * LDA + 32 * kh + 8 * (s + 1)]);
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[nxt][j] = dequant_word_bf16(r.w[j][s + 1], vmask, sc[j], nb[j]);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(af[cur][i]), as_bf16x8(bf[cur][j]),
                                                              acc[i][j], 0, 0, 0);
      if (s < 3) {
        // MI * NJ MFMAs; NJ * 23 dequant VALU ops and MI LDS reads spread between them.
        constexpr int kMfma = MI * NJ;
        constexpr int kValu = (NJ * 23 + kMfma - 1) / kMfma;
#pragma unroll
        for (int k = 0; k < kMfma; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);  // VALU
          if (k < MI) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        }
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

// ---------------------------------------------------------------------------------------------
// v2 pipeline (K % 64 == 0, G a power of two >= 32): activations go global -> LDS directly with
// buffer loads into LDS (no staging registers), through a ring of ST stages; weights go to a
// ring of ST register slots. At block kb the loads for block kb + ST - 1 are issued, so ST - 1
// blocks of both are in flight while one is computed. Per block: one explicit wait for this
// wave's loads of the block, one barrier (all waves' LDS writes visible, and the stage about to
// be refilled is no longer read), then the loads for block kb + ST - 1, then the MFMAs.
//
// LDS activation layout: row-major rows of 64 bf16 (128 B, eight 16-byte chunks) with the chunk
// index XOR-swizzled by (row >> 1) & 7, so the 16-byte fragment reads of 16 consecutive rows hit
// 16 distinct bank groups. A 16-byte LDS load by lane L lands at base + 16 L, so each load
// instruction fills 8 rows: lane L fetches row L / 8, chunk (L % 8) ^ ((row >> 1) & 7).
// Rows past M and blocks past K read as zero through the buffer range check.

// Epilogue through LDS (the activation ring is free once the K loop is done). Each wave owns
// a BMW x WN sub-tile (rows m0 .., columns n0w ..): its 32x32 accumulators are rounded to
// bf16 and written to a wave-private LDS tile of row stride LS elements with 2-byte stores
// (LS = WN + 8, where it fits, keeps the two row halves of a store on different banks), then
// read back 16 bytes per lane and stored to Y as whole 16-byte row segments. Rows past M /
// columns past N are not stored.
template <int MI, int NJ, int LS>
__device__ __forceinline__ void store_tile_lds(const f32x16_t (&acc)[MI][NJ], uint16_t* lds, uint16_t* C,
                                               int M, int N, int m0, int n0w) {
  constexpr int WN = 32 * NJ, BMW = 32 * MI;
  const int lane = threadIdx.x & 63, ln = lane & 31, kh = lane >> 5;
  // registers r, r + 1 (r even) are rows m, m + 1 of one column: one hardware RNE convert
  // (v_cvt_pk_bf16_f32) rounds both
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const int row = 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        const uint32_t pk = pack_bf16x2_rne(acc[i][j][r], acc[i][j][r + 1]);
        lds[row * LS + 32 * j + ln] = (uint16_t)pk;
        lds[(row + 1) * LS + 32 * j + ln] = (uint16_t)(pk >> 16);
      }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's tile is in LDS
  constexpr int CPR = WN / 8;          // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;        // rows per 64-lane pass
  const int cr = lane / CPR, cc = lane % CPR;
  const bool full = m0 + BMW <= M && n0w + WN <= N;
#pragma unroll
  for (int p = 0; p < BMW / RPI; ++p) {
    const int row = p * RPI + cr;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&lds[row * LS + 8 * cc]);
    const int m = m0 + row, n = n0w + 8 * cc;
    if (full || (m < M && n + 8 <= N)) {
      *reinterpret_cast<u32x4_t*>(&C[(size_t)m * N + n]) = v;
    } else if (m < M) {
      for (int e = 0; e < 8; ++e)
        if (n + e < N) C[(size_t)m * N + n + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Direct epilogue (used when the tile does not fit the LDS ring): one bf16 store per value.
// D[i][j] of lane l, register r: j = l % 32, i = 8 (r / 4) + 4 (l / 32) + r % 4.
template <int MI, int NJ>
__device__ __forceinline__ void store_tile_direct(const f32x16_t (&acc)[MI][NJ], uint16_t* C, int M,
                                                  int N, int m0, int n0w) {
  const int lane = threadIdx.x & 63, ln = lane & 31, kh = lane >> 5;
  const bool full = m0 + 32 * MI <= M && n0w + 32 * NJ <= N;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = n0w + 32 * j + ln;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (full || (m < M && n < N)) C[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(acc[i][j][r]);
      }
    }
}

// SwiGLU epilogue (weights' rows are gate and up rows interleaved in blocks of 8: columns 16b ..
// 16b+7 of the product are gate rows 8b .., columns 16b+8 .. 16b+15 the matching up rows).
// Column pairs (n, n + 8) sit in lanes l and l ^ 8 of a 32x32 fragment (same row), so one
// shuffle pairs them; each product is rounded to bf16 first, as the separate GEMM and SwiGLU
// would store it, and Y [M][N/2] gets bf16(silu(g) * u) at column 8b + n % 8.
template <int MI, int NJ>
__device__ __forceinline__ void store_tile_swiglu(const f32x16_t (&acc)[MI][NJ], uint16_t* Y,
                                                  int M, int N, int m0, int n0w) {
  const int lane = threadIdx.x & 63, ln = lane & 31, kh = lane >> 5;
  const int Nh = N >> 1;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = n0w + 32 * j + ln;
      const int o = ((n >> 4) << 3) + (n & 7);
      const bool gate = (ln & 8) == 0 && n < N;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        const float g = round_bf16(acc[i][j][r]);
        const float u = lane_xor8(g);
        if (gate && m < M) Y[(size_t)m * Nh + o] = (uint16_t)f32_to_bf16_rne(silu_mul(g, u));
      }
    }
}

// One 16-byte buffer load per lane into LDS at dst + 16 * lane. (A plain device function: the
// builtin inside a lambda of a kernel template keeps the host pass from emitting the launch stub.)
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t voff,
                                           uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff,
                                           soff, 0, 0);
}

// Workgroup barrier for the LDS rings. The compiler models a buffer-to-LDS load as writing 16
// bytes at its LDS pointer, while the hardware writes 16 bytes per lane (1 KiB per wave); the
// empty asm with a memory clobber keeps LDS reads from being merged with, or moved above, the
// barrier that publishes those writes.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }

template <int N>
__device__ __forceinline__ void wait_vmcnt_c() {
  // s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0], expcnt, lgkmcnt, vmcnt[5:4])
  constexpr int imm = (N & 0xF) | (0x7 << 4) | (0xF << 8) | (((N >> 4) & 0x3) << 14);
  __builtin_amdgcn_s_waitcnt(imm);
}

// K-split handoff of the GEMMs: group g hands its accumulators (MI x NJ vectors of R floats) to
// group 0 in round g through pb (this wave's slice of the free LDS ring, lane-major: word r * 64
// + lane); group 0 adds them in group order. Every wave of the workgroup calls it (it holds
// barriers).
template <int KS, int MI, int NJ, typename V>
__device__ __forceinline__ void k_group_handoff(V (&acc)[MI][NJ], float* pb, int ks, int lane) {
  constexpr int R = sizeof(V) / sizeof(float);
#pragma unroll 1
  for (int g = 1; g < KS; ++g) {
    if (ks == g) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int r = 0; r < R; ++r) pb[((i * NJ + j) * R + r) * kWave + lane] = acc[i][j][r];
    }
    lds_barrier();
    if (ks == 0) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int r = 0; r < R; ++r) acc[i][j][r] += pb[((i * NJ + j) * R + r) * kWave + lane];
    }
    lds_barrier();
  }
}

// KS > 1 (tile grids too small to fill the chip, e.g. down at M = 512): KS groups of NWN waves
// split K inside the workgroup. Group ks computes 64-k blocks ks, ks + KS, ... into its own
// accumulators through its own part of the LDS ring (step t loads and computes block t KS + ks
// in every group); at the end groups 1 .. KS-1 hand their accumulators to group 0 through LDS,
// one group per round, and group 0 adds them in group order and stores the tile.
// 256-row tiles carry 128 accumulators per lane: the launch bound asks for two waves per SIMD
// (two four-wave workgroups per CU, or one eight-wave workgroup with KS = 2) so the compiler
// keeps them in VGPRs beside the operands.
template <int BM, int WN, int NWN, int ST, bool SW = false, int KS = 1, int WD = 1>
__global__ __launch_bounds__(NWN * KS * kWave, BM >= 256 && KS == 1 ? 2 : 1) void w4_gemm2_kernel(
    const uint16_t* __restrict__ A, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ C, int M, int N, int K, int lgG) {
  constexpr int MI = BM / 32, NJ = WN / 32, BN = WN * NWN;
  constexpr int STAGE = BM * BK;                 // bf16 elements per stage and K group
  constexpr int IPW = BM / (8 * NWN);            // 16-byte LDS-load instructions per wave per block
  static_assert(BM % (8 * NWN) == 0, "whole LDS-load instructions per wave");
  constexpr uint32_t kOOB = 0x7fffffc0u;
  constexpr int RING = ST * KS * STAGE;                          // bf16 elements
  constexpr int PART = KS > 1 ? NWN * kWave * MI * NJ * 16 * 2 : 0;  // one group's partials
  __shared__ __align__(16) uint16_t As[RING > PART ? RING : PART];
  constexpr int ELS = NWN * BM * (WN + 8) <= RING ? WN + 8 : WN;  // epilogue row stride
  constexpr bool kLdsEpilogue = NWN * BM * ELS <= RING;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wq % NWN, ks = wq / NWN;  // column slice and K group of this wave
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int KW = K >> 3, KG = K >> lgG;
  const int KB = K / BK;
  const int T = (KB + KS - 1) / KS;  // steps

  const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(A), (short)0, (int)((size_t)M * K * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wq), (short)0, (int)((size_t)N * KW * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(S), (short)0, (int)((size_t)N * KG * 2), 0x00020000);

  // activation loader: this lane's row / swizzled chunk inside each of the wave's instructions
  uint32_t a_voff[IPW];
#pragma unroll
  for (int t = 0; t < IPW; ++t) {
    const int row = 8 * (wv * IPW + t) + (lane >> 3);
    const int ch = (lane & 7) ^ ((row >> 1) & 7);
    a_voff[t] = ((uint32_t)(m0 + row) * (uint32_t)K + 8u * ch) * 2u;
  }
  auto issue_a = [&](int stage, int kb) {
    const uint32_t so = kb < KB ? 128u * kb : kOOB;
#pragma unroll
    for (int t = 0; t < IPW; ++t)
      lds_load16(ares, &As[(stage * KS + ks) * STAGE + 512 * (wv * IPW + t)], a_voff[t], so);
  };

  // weight loader: lane (n = lane % 32, kh = lane / 32), 16 bytes (words 4 kh .. 4 kh + 3 of the
  // block) per n-frag, plus the group scale of those 32 k.
  const int ln = lane & 31, kh = lane >> 5;
  uint32_t w_voff[NJ], s_voff[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t n = (uint32_t)(n0 + wv * WN + 32 * j + ln);
    w_voff[j] = n * (uint32_t)KW * 4u + 16u * kh;
    s_voff[j] = n * (uint32_t)KG * 2u;
  }
  struct WRegs {
    u32x4_t w[NJ];
    uint32_t s[NJ];
  };
  auto issue_w = [&](WRegs& r, int kb) {
    const bool live = kb < KB;
    const uint32_t so = live ? 32u * kb : kOOB;
    const uint32_t ss = live ? 2u * (uint32_t)((kb * BK + 32 * kh) >> lgG) : kOOB;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      r.w[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wres, w_voff[j], so, 0));
      r.s[j] = __builtin_amdgcn_raw_buffer_load_b16(sres, s_voff[j] + ss, 0, 0);
    }
  };

  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  // LDS offset (elements) of this lane's A fragment: row 32 i + ln, chunk 4 kh + s (swizzled)
  auto a_frag = [&](const uint16_t* as, int i, int s) {
    const int row = 32 * i + ln;
    const int ch = (4 * kh + s) ^ ((row >> 1) & 7);
    return *reinterpret_cast<const u32x4_t*>(&as[row * BK + 8 * ch]);
  };

  auto compute = [&](int stage, const WRegs& r) {
    const uint16_t* as = &As[(stage * KS + ks) * STAGE];
    float sc[NJ], nb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      sc[j] = bf16_bits_to_f32(r.s[j]);
      nb[j] = -1032.f * sc[j];
    }
    u32x4_t af[2][MI], bf[2][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) af[0][i] = a_frag(as, i, 0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) bf[0][j] = dequant_word_bf16(r.w[j][0], vmask, sc[j], nb[j]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s < 3) {
#pragma unroll
        for (int i = 0; i < MI; ++i) af[nxt][i] = a_frag(as, i, s + 1);
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[nxt][j] = dequant_word_bf16(r.w[j][s + 1], vmask, sc[j], nb[j]);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(af[cur][i]), as_bf16x8(bf[cur][j]),
                                                              acc[i][j], 0, 0, 0);
      if (s < 3) {
        constexpr int kMfma = MI * NJ;
        constexpr int kValu = (NJ * 23 + kMfma - 1) / kMfma;
#pragma unroll
        for (int k = 0; k < kMfma; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
          if (k < MI) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
    }
  };

  if constexpr (WD > 1) {
    // Weights and scales WD - 1 blocks further ahead than the activation tiles: a ring of
    // WR = ST + WD - 1 register slots. Per block the activation tile is issued first, then the
    // weights (scheduling barriers keep that order), so when block kb starts only the weight
    // loads of the block after the tile of kb, and the (ST - 2) blocks' loads between, may still
    // be in flight: the explicit wait counts exactly those, and the weights of block kb were
    // issued before its tile.
    constexpr int WR = ST + WD - 1;
    constexpr int UNR = ST * WR / gcd_c(ST, WR);  // the loop body sees every (stage, slot) pair
    WRegs wr[WR];
#pragma unroll
    for (int p = 0; p < WR - 1; ++p) {
      __builtin_amdgcn_sched_barrier(0);
      if (p < ST - 1) issue_a(p, p * KS + ks);
      __builtin_amdgcn_sched_barrier(0);
      issue_w(wr[p], p * KS + ks);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int t0 = 0; t0 < T; t0 += UNR) {
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int kb = (t0 + u) * KS + ks;
        wait_vmcnt_c<2 * NJ + (ST - 2) * (IPW + 2 * NJ)>();  // block kb's tile has landed
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue_a((u + ST - 1) % ST, kb + (ST - 1) * KS);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(wr[(u + WR - 1) % WR], kb + (WR - 1) * KS);
        __builtin_amdgcn_sched_barrier(0);
        if (kb < KB) compute(u % ST, wr[u % WR]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
  // Explicit waits count only the LDS-DMA activation loads (IPW per wave per block): those stay
  // in program order, while the compiler may move the weight and scale loads (whose register
  // uses it guards itself). Counting only later DMA loads can over-wait, never under-wait.
  WRegs wr[ST];
#pragma unroll
  for (int p = 0; p < ST - 1; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    issue_w(wr[p], p * KS + ks);
    issue_a(p, p * KS + ks);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int t0 = 0; t0 < T; t0 += ST) {
#pragma unroll
    for (int u = 0; u < ST; ++u) {
      const int kb = (t0 + u) * KS + ks;
      wait_vmcnt_c<IPW * (ST - 2)>();  // this wave's activation loads of block kb have landed
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue_w(wr[(u + ST - 1) % ST], kb + (ST - 1) * KS);
      issue_a((u + ST - 1) % ST, kb + (ST - 1) * KS);
      __builtin_amdgcn_sched_barrier(0);
      if (kb < KB) compute(u, wr[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  }

  wait_vmcnt_c<0>();  // the trailing out-of-range loads have landed before the LDS is reused
  lds_barrier();      // every wave is done reading the ring
  if constexpr (KS > 1) {
    k_group_handoff<KS>(acc, reinterpret_cast<float*>(As) + wv * (kWave * MI * NJ * 16), ks, lane);
    if (ks != 0) return;  // no barrier follows
  }
  if constexpr (SW)
    store_tile_swiglu<MI, NJ>(acc, C, M, N, m0, n0 + wv * WN);
  else if constexpr (kLdsEpilogue)
    store_tile_lds<MI, NJ, ELS>(acc, &As[wv * BM * ELS], C, M, N, m0, n0 + wv * WN);
  else
    store_tile_direct<MI, NJ>(acc, C, M, N, m0, n0 + wv * WN);
}

// Epilogue of the 16x16x32 GEMMs: a wave's BM x 32 accumulators (16-row fragments i, 16-column
// halves jj; registers r, r + 1 are rows m, m + 1 of one column) rounded to bf16 into its private
// LDS sub-tile lds (row stride 32), then stored as 16-byte row segments of C (element by element
// at the edges of C or when C's rows are not 16-byte aligned).
template <int BM>
__device__ __forceinline__ void store_tile_16x16(const f32x4_t (&acc)[BM / 16][2], uint16_t* lds,
                                                 uint16_t* C, int M, int N, int m0, int n0w, int lane) {
  const int fr = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int i = 0; i < BM / 16; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const int row = 16 * i + 4 * kg + r;
        const uint32_t pk = pack_bf16x2_rne(acc[i][jj][r], acc[i][jj][r + 1]);
        lds[row * 32 + 16 * jj + fr] = (uint16_t)pk;
        lds[(row + 1) * 32 + 16 * jj + fr] = (uint16_t)(pk >> 16);
      }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's sub-tile is in LDS
  const int cr = lane >> 2, cc = lane & 3;
  const bool full = m0 + BM <= M && n0w + 32 <= N && (N & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(C) & 15) == 0;
#pragma unroll
  for (int p = 0; p < BM / 16; ++p) {
    const int row = 16 * p + cr;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&lds[row * 32 + 8 * cc]);
    const int m = m0 + row, n = n0w + 8 * cc;
    if (full) {
      *reinterpret_cast<u32x4_t*>(&C[(size_t)m * N + n]) = v;
    } else if (m < M) {
      for (int e = 0; e < 8; ++e)
        if (n + e < N) C[(size_t)m * N + n + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// SwiGLU epilogue of the 16x16x32 GEMMs for gate/up weights interleaved in blocks of 8 rows
// (features 16b .. 16b+7 gate, 16b+8 .. 16b+15 the matching up rows): lane (j, kg) holds feature
// column j of its 16-column half, so a gate value (j < 8) finds its up value in lane j + 8 of the
// same row. Y[m][o] = bf16(silu(g) * u) with g, u rounded to bf16 first (the values the plain
// GEMM would store), o = 8 b + j; the wave's 16 outputs per row go through its private LDS
// sub-tile (row stride 16) and out as 16-byte segments (element by element at the edges of Y or
// when its rows are not 16-byte aligned).
template <int BM>
__device__ __forceinline__ void store_tile_16x16_swiglu(const f32x4_t (&acc)[BM / 16][2], uint16_t* lds,
                                                        uint16_t* Y, int M, int N, int m0, int n0w,
                                                        int lane) {
  const int fr = lane & 15, kg = lane >> 4, Nh = N >> 1;
#pragma unroll
  for (int i = 0; i < BM / 16; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float g = round_bf16(acc[i][jj][r]);
        const float u = lane_xor8(g);
        if (fr < 8)
          lds[(16 * i + 4 * kg + r) * 16 + 8 * jj + fr] = (uint16_t)f32_to_bf16_rne(silu_mul(g, u));
      }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's sub-tile is in LDS
  const int o0 = n0w >> 1;             // the wave's first output column
  const bool full = m0 + BM <= M && n0w + 32 <= N && (Nh & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
  const int cr = lane >> 1, cc = lane & 1;
#pragma unroll
  for (int p = 0; p < BM / 32; ++p) {
    const int row = 32 * p + cr;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&lds[row * 16 + 8 * cc]);
    const int m = m0 + row, o = o0 + 8 * cc;
    if (full) {
      *reinterpret_cast<u32x4_t*>(&Y[(size_t)m * Nh + o]) = v;
    } else if (m < M) {
      for (int e = 0; e < 8; ++e)
        if (2 * (o + e) < N) Y[(size_t)m * Nh + o + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Packed tile format (ns_w4_repack: tiles of 16 rows x 128 k, lane l's 16 bytes = row l % 16 at
// k = 32 s + 8 (l / 16) + e, word s, nibbles in the order e = 0 2 4 6 1 3 5 7) -> 8 staged weights
// bf16_rne((q - 8) * s) in natural k order: with that nibble order the pairs (e0, e1), (e2, e3),
// (e4, e5), (e6, e7) sit at bit offsets 0/16, 4/20, 8/24, 12/28, so each v_and_or_b32 of a
// shifted word yields one fp16 pair (1024 + q) already in k order; the rest is dequant_word_bf16.
__device__ __forceinline__ u32x4_t dequant_word_bf16_pk(uint32_t w, uint32_t vmask, float s,
                                                        float ns1032) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  constexpr uint32_t kE1024 = 0x64006400u;
  const h2_t h0 = __builtin_bit_cast(h2_t, and_or_s(w, vmask, kE1024));        // e0, e1
  const h2_t h1 = __builtin_bit_cast(h2_t, and_or_s(w >> 4, vmask, kE1024));   // e2, e3
  const h2_t h2 = __builtin_bit_cast(h2_t, and_or_s(w >> 8, vmask, kE1024));   // e4, e5
  const h2_t h3 = __builtin_bit_cast(h2_t, and_or_s(w >> 12, vmask, kE1024));  // e6, e7
  u32x4_t d;
  d[0] = pack_bf16x2_rne(__builtin_fmaf((float)h0[0], s, ns1032), __builtin_fmaf((float)h0[1], s, ns1032));
  d[1] = pack_bf16x2_rne(__builtin_fmaf((float)h1[0], s, ns1032), __builtin_fmaf((float)h1[1], s, ns1032));
  d[2] = pack_bf16x2_rne(__builtin_fmaf((float)h2[0], s, ns1032), __builtin_fmaf((float)h2[1], s, ns1032));
  d[3] = pack_bf16x2_rne(__builtin_fmaf((float)h3[0], s, ns1032), __builtin_fmaf((float)h3[1], s, ns1032));
  return d;
}

// One fp16 pair of dequant_word_bf16_pk on its own (pair D = nibbles 2D, 2D + 1 of the packed
// order, the word's output dword D): the GEMM spreads one word's dequant over several MFMAs.
template <int D>
__device__ __forceinline__ uint32_t dequant_pair_bf16_pk(uint32_t w, uint32_t vmask, float s,
                                                         float ns1032) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  constexpr uint32_t kE1024 = 0x64006400u;
  const h2_t h = __builtin_bit_cast(h2_t, and_or_s(D ? (w >> (4 * D)) : w, vmask, kE1024));
  return pack_bf16x2_rne(__builtin_fmaf((float)h[0], s, ns1032), __builtin_fmaf((float)h[1], s, ns1032));
}

// Prefill GEMM on the packed tile format (the pre-shuffled layout the reference's README:148-151
// proposes for its GEMM): C[M][N] (bf16, RNE) = A[M][K] . deq(Wp, Sp)^T with the reference GEMM's
// numerics (each weight staged as bf16_rne((q - 8) s), w4a16.cuh:190-198; fp32 accumulation).
//  * v_mfma_f32_16x16x32_bf16: a packed tile's lane (j, kg) run is, word by word, exactly the
//    B operand of lane (j, kg) for the tile's four 32-k steps, so one 16-byte load per lane per
//    tile-row and 128 k feeds four steps (the standard layout needs one per 64 k), and the
//    nibble order gives k-ordered fp16 pairs without a byte permute.
//  * BM x 32 NWN output tiles, NWN waves of BM rows x 32 columns (two tile-rows) per K group:
//    each staged weight word feeds BM / 16 MFMAs; 128 x 128 tiles (64 accumulators per lane)
//    run four four-wave workgroups per CU, or two eight-wave ones with K split over two groups.
//  * The activation tile (BM x 64 bf16 per stage, two stages per K group) comes in by
//    buffer-to-LDS loads with the standard GEMM's XOR swizzle (16-byte chunk c of row r at
//    c ^ (r / 2) % 8: the 16 rows of a fragment read hit distinct banks); 64-k block 2c + h uses
//    words 2h, 2h + 1 of the lane's run of tile column c. The weights of a group's tile column
//    WD steps ahead are issued at the step's first block into a register ring of WD + 1 slots.
//  * KS > 1 (tile grids that do not fill the chip, e.g. the 7B down projection): KS groups of
//    NWN waves split the tile columns (group g takes columns g, g + KS, ..., through its own
//    two stages); groups 1 .. KS-1 then hand their accumulators to group 0 through LDS, one
//    group per round, and group 0 adds them in group order.
//  * Epilogue (group 0): each wave rounds its BM x 32 sub-tile to bf16 into a private part of
//    the (then free) LDS ring and stores 16-byte row segments.
template <int BM, int NWN, int KS, int WD, bool SW = false>
__global__ __launch_bounds__(NWN * KS * kWave, KS > 1 ? 1 : 4)
void w4_gemm_pk_kernel(const uint16_t* __restrict__ A, const uint32_t* __restrict__ Wp,
                       const uint16_t* __restrict__ Sp, uint16_t* __restrict__ C, int M, int N, int K) {
  constexpr int NJ = 2, MI = BM / 16, BN = 32 * NWN, ST = 2;
  constexpr int STAGE = BM * BK;          // bf16 elements per activation stage
  constexpr int IPW = BM / (8 * NWN);     // 16-byte LDS-load instructions per wave per stage
  static_assert(BM % (8 * NWN) == 0, "whole LDS-load instructions per wave");
  constexpr int WR = WD + 1;              // weight ring slots (tile columns)
  constexpr uint32_t kOOB = 0x7fffffc0u;
  constexpr int RING = ST * KS * STAGE;                           // bf16 elements
  constexpr int PART = KS > 1 ? NWN * kWave * MI * NJ * 4 * 2 : 0;  // one group's partials
  constexpr int EPI = NWN * BM * 32;                              // epilogue sub-tiles
  constexpr int LDSN = RING > PART ? (RING > EPI ? RING : EPI) : (PART > EPI ? PART : EPI);
  __shared__ __align__(16) uint16_t As[LDSN];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wq % NWN, ks = wq / NWN;  // column slice and K group of this wave
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int CT = K >> 7;                  // tile columns
  const int T = (CT + KS - 1) / KS;       // steps (tile columns per group)
  const int NT = (N + 15) >> 4;           // tile rows

  const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(A), (short)0, (int)((size_t)M * K * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wp), (short)0, (int)((size_t)NT * CT * 1024), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Sp), (short)0, (int)((size_t)NT * CT * 32), 0x00020000);

  uint32_t a_voff[IPW];
#pragma unroll
  for (int t = 0; t < IPW; ++t) {
    const int row = 8 * (wv * IPW + t) + (lane >> 3);
    const int ch = (lane & 7) ^ ((row >> 1) & 7);
    a_voff[t] = ((uint32_t)(m0 + row) * (uint32_t)K + 8u * ch) * 2u;
  }
  // stage st of this group <- 64-k block kb (past K: zeros)
  auto issue_a = [&](int st, int kb) {
    const uint32_t so = kb < 2 * CT ? 128u * kb : kOOB;
#pragma unroll
    for (int t = 0; t < IPW; ++t)
      lds_load16(ares, &As[(st * KS + ks) * STAGE + 512 * (wv * IPW + t)], a_voff[t], so);
  };

  // weights: lane (j, kg)'s 16-byte run of tile (tile-row n0 / 16 + 2 wv + jj, column c) and
  // the scale of that tile's row j
  uint32_t w_voff[NJ], s_voff[NJ];
#pragma unroll
  for (int jj = 0; jj < NJ; ++jj) {
    const uint32_t tr = (uint32_t)((n0 >> 4) + NJ * wv + jj);
    w_voff[jj] = tr * (uint32_t)CT * 1024u + 16u * lane;
    s_voff[jj] = (tr * (uint32_t)CT * 16u + (uint32_t)(lane & 15)) * 2u;
  }
  struct WRegs {
    u32x4_t w[NJ];
    uint32_t s[NJ];
  };
  auto issue_w = [&](WRegs& r, int c) {
    const bool live = c < CT;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      r.w[jj] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                wres, w_voff[jj], live ? 1024u * c : kOOB, 0));
      r.s[jj] = __builtin_amdgcn_raw_buffer_load_b16(sres, s_voff[jj], live ? 32u * c : kOOB, 0);
    }
  };

  f32x4_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) acc[i][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  const int fr = lane & 15, kg = lane >> 4;
  // one 64-k stage: two 32-k steps; step s2 reads chunk 4 s2 + kg of rows 16 i + fr. The second
  // step's weights are dequantized one fp16 pair at a time between the first step's row blocks
  // of MFMAs (the same values, and the same MFMA order per accumulator: the same bits; on
  // MI355X 0.8-2.2 % faster on the config-4 shapes than dequantizing each step up front).
  auto compute = [&](int st, const WRegs& r, auto half_c) {
    constexpr int H = decltype(half_c)::value;
    const uint16_t* as = &As[(st * KS + ks) * STAGE];
    float sc[NJ], nb[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      sc[jj] = bf16_bits_to_f32(r.s[jj] & 0xffffu);
      nb[jj] = -1032.f * sc[jj];
    }
    u32x4_t b0[NJ], b1[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) b0[jj] = dequant_word_bf16_pk(r.w[jj][2 * H], vmask, sc[jj], nb[jj]);
    constexpr int PER = (4 * NJ + MI - 1) / MI;  // second-step pairs per row block
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int row = 16 * i + fr;
      const int ch = kg ^ ((row >> 1) & 7);
      const u32x4_t af = *reinterpret_cast<const u32x4_t*>(&as[row * BK + 8 * ch]);
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
        acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(b0[jj]), acc[i][jj], 0, 0, 0);
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int q = PER * i + p;  // pair q % 4 of word q / 4
        if (q < 4 * NJ) {
          const int jj = q >> 2;
          const uint32_t wd = r.w[jj][2 * H + 1];
          uint32_t v;
          switch (q & 3) {
            case 0: v = dequant_pair_bf16_pk<0>(wd, vmask, sc[jj], nb[jj]); break;
            case 1: v = dequant_pair_bf16_pk<1>(wd, vmask, sc[jj], nb[jj]); break;
            case 2: v = dequant_pair_bf16_pk<2>(wd, vmask, sc[jj], nb[jj]); break;
            default: v = dequant_pair_bf16_pk<3>(wd, vmask, sc[jj], nb[jj]); break;
          }
          b1[jj][q & 3] = v;
        }
      }
      __builtin_amdgcn_sched_barrier(0x0100);  // only LDS reads may move across
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int row = 16 * i + fr;
      const int ch = (4 + kg) ^ ((row >> 1) & 7);
      const u32x4_t af = *reinterpret_cast<const u32x4_t*>(&as[row * BK + 8 * ch]);
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
        acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(b1[jj]), acc[i][jj], 0, 0, 0);
    }
  };

  WRegs wr[WR];
  // step t covers this group's tile column c = ks + KS t: blocks 2c (half 0) and 2c + 1 (half
  // 1). The weights of the first WD steps go first, then the first activation stage (the
  // per-block wait below counts only the weight loads issued after a block's stage)
#pragma unroll
  for (int p = 0; p < WD; ++p) issue_w(wr[p], ks + KS * p);
  __builtin_amdgcn_sched_barrier(0);
  issue_a(0, 2 * ks);
  __builtin_amdgcn_sched_barrier(0);
  constexpr int UNR = 2 * WR;  // blocks per period: every (stage, slot, half) combination
  for (int b0 = 0; b0 < 2 * T; b0 += UNR) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int bi = b0 + u, t = bi >> 1;  // this group's block bi: step t, half u % 2
      const int c = ks + KS * t;
      // block bi's stage was issued in block bi - 1, followed by that block's weight loads when
      // bi - 1 starts a step
      if (u & 1)
        wait_vmcnt_c<2 * NJ>();
      else
        wait_vmcnt_c<0>();
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // the next block of this group: the second half of column c, or the first of c + KS
      issue_a((u + 1) % ST, (u & 1) ? 2 * (c + KS) : 2 * c + 1);
      __builtin_amdgcn_sched_barrier(0);
      if ((u & 1) == 0) issue_w(wr[(u / 2 + WD) % WR], c + KS * WD);
      __builtin_amdgcn_sched_barrier(0);
      if (c < CT) {
        if (u & 1)
          compute(u % ST, wr[(u / 2) % WR], std::integral_constant<int, 1>{});
        else
          compute(u % ST, wr[(u / 2) % WR], std::integral_constant<int, 0>{});
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  wait_vmcnt_c<0>();
  lds_barrier();  // every wave is done with the ring

  if constexpr (KS > 1) {
    k_group_handoff<KS>(acc, reinterpret_cast<float*>(As) + wv * (kWave * MI * NJ * 4), ks, lane);
    if (ks != 0) return;  // no barrier follows
  }
  if constexpr (SW)
    store_tile_16x16_swiglu<BM>(acc, &As[wv * (BM * 32)], C, M, N, m0, n0 + 32 * wv, lane);
  else
    store_tile_16x16<BM>(acc, &As[wv * (BM * 32)], C, M, N, m0, n0 + 32 * wv, lane);
}

inline int ilog2(int g) { return 31 - __builtin_clz((unsigned)g); }

struct TileCfg {
  int bm, bn;
  float eff;  // relative per-tile efficiency used by the planner
};
constexpr TileCfg kCfgs[] = {
    {256, 256, 1.00f},  // 0: v1, BM 256, 4 waves x 64 cols (not offered: spills)
    {256, 128, 0.90f},  // 1: v1, BM 256, 4 waves x 32 cols
    {128, 256, 0.85f},  // 2: v1, BM 128, 4 waves x 64 cols
    {128, 128, 0.75f},  // 3: v1, BM 128, 4 waves x 32 cols
    {128, 128, 1.00f},  // 4: v2, BM 128, 4 waves x 32 cols, 3 stages
    {128, 128, 1.00f},  // 5: v2, BM 128, K split over 2 wave groups of 4, 2 stages, two per CU
    {256, 128, 1.00f},  // 6: v2, BM 256, 4 waves x 32 cols, 2 stages, two workgroups per CU
    {256, 128, 1.00f},  // 7: v2, BM 256, K split over 2 wave groups of 4, 2 stages, one per CU
    {128, 64, 1.00f},   // 8: v2, BM 128, K split over 4 wave groups of 2, 2 stages, one per CU
    {64, 64, 1.00f},    // 9: v2, BM 64, K split over 4 wave groups of 2, 2 stages, two per CU
};

}  // namespace

// The v2 kernel addresses A, Wq and S through 32-bit buffer offsets (rows up to M + 256 included)
// and reads whole 64-k blocks whose 32-k halves sit inside one power-of-two group.
bool gemm_v2_ok(int M, int N, int K, int G) {
  if (K % 64 != 0 || G < 32 || (G & (G - 1)) != 0) return false;
  const uint64_t limit = 0x7fffffffull;
  return (uint64_t)(M + 256) * K * 2 < limit && (uint64_t)N * K / 2 < limit &&
         (uint64_t)N * (K / G) * 2 < limit;
}

GemmPlan gemm_plan(int M, int N, int K, int G) {
  int cus = 256;  // the device's CU count (a failed query leaves MI355X's; the launch reports it)
  if (cached_cu_count(&cus) != hipSuccess || cus <= 0) cus = 256;
  if (gemm_v2_ok(M, N, K, G)) {
    // Tile plans, measured on MI355X (A/B runs of the four config-4 shapes and the other shapes
    // quoted):
    //  * 128 x 128 tiles, three workgroups per CU: the default.
    //  * 256 x 128 tiles (each wave 256 x 32: one dequantized weight word feeds eight MFMAs, not
    //    four), two workgroups per CU, when there are at least four rounds of them: gate/up at
    //    M = 2048 590 -> 555 us; with fewer rounds (gate/up M = 512) 128 x 128 is faster.
    //  * 256 x 128 tiles with K split over two groups of four waves, one eight-wave workgroup per
    //    CU (two waves per SIMD on one tile, the K loop halved), when those tiles fill three
    //    quarters to all of the CUs once and K >= 8192: down 3584 x 18944 at M = 2048 320 -> 301
    //    and 303.6 -> 289.7 us on two boxes, 4096 x 14336 263 -> 244 us; with short K (3584 x
    //    3584: 68 -> 72) or 128 such tiles (half the CUs: 159 -> 206) 128 x 128 stays.
    //  * When 128 x 128 tiles fill at most one round of the CUs, K split inside the workgroup:
    //    128 x 64 tiles over four wave groups of two (each wave a 32-column slice), one eight-wave
    //    workgroup per CU, when they fill three quarters to all of the CUs (down at M = 512:
    //    121.8 -> 102.2 us, 4096 x 14336 at M = 512 98.8 -> 86.2); else, with more than half the
    //    CUs holding a 128 x 128 tile, those tiles over two groups of four waves, two eight-wave
    //    workgroups per CU (against the 64 x 64 plan below, us: 3584 x 18944 at M = 1024 219.1 ->
    //    161.5, M = 768 210.3 -> 148.6, 3328 x 11008 at M = 1024 132.4 -> 93.9, qkv 4608 x 3584 at
    //    M = 512 37.0 -> 32.6, 3584 x 3584 at M = 768 39.2 -> 32.7; at exactly one round, 4096 x
    //    14336 at M = 1024, 144.5 -> 135.2 against 128 x 128 unsplit; where the 128 x 64 plan
    //    applies it stays ahead: down at M = 512 95.3 against 146.4); else 64 x 64 tiles over
    //    four groups of two, two per CU (down at M = 256 113.6 -> 65.2 us, 3584 x 3584 24.7 ->
    //    17.8).
    const long tiles = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long tiles256 = (long)((M + 255) / 256) * ((N + 127) / 128);
    const bool ks256 = tiles256 <= cus && 4 * tiles256 >= 3 * cus && K >= 8192;
    int c = ks256 ? 7 : tiles256 >= 4 * cus ? 6 : 4;
    if (tiles <= cus) {
      const long t128x64 = (long)((M + 127) / 128) * ((N + 63) / 64);
      c = tiles < cus && 4 * t128x64 >= 3 * cus && t128x64 <= cus ? 8 : 2 * tiles > cus ? 5 : 9;
    }
    return GemmPlan{c, kCfgs[c].bm, kCfgs[c].bn};
  }
  // register-staged fallback (K % 64 == 32, or a group size that is not a power of two):
  // plans 1..3; plan 0 (256 x 256 tiles, 64-column waves) needs more than the 512 registers a
  // lane has at one wave per SIMD and spills, so it is not offered
  int best = 1;
  double best_cost = 1e300;
  for (int c = 1; c < 4; ++c) {
    const long tiles = (long)((M + kCfgs[c].bm - 1) / kCfgs[c].bm) * ((N + kCfgs[c].bn - 1) / kCfgs[c].bn);
    const long rounds = (tiles + cus - 1) / cus;
    const double cost = (double)rounds * kCfgs[c].bm * kCfgs[c].bn / kCfgs[c].eff;
    if (cost < best_cost) {
      best_cost = cost;
      best = c;
    }
  }
  return GemmPlan{best, kCfgs[best].bm, kCfgs[best].bn};
}

// Weight prefetch distance of the 128- and 256-row plans, in blocks beyond the activation tiles
// (WD): 3 measured best on MI355X (gate/up M = 2048 537-541 -> 520-523 us, M = 512 159-161 ->
// 153-157, down M = 2048 313 -> 308, against 1; 4 and 5 no better; same outputs bit for bit).
constexpr int kWeightAhead = 3;

// Tile plan of the packed-format GEMM (M > 16 through ns_w4_linear_packed). On MI355X (interleaved
// A/B runs, us; the standard GEMM in brackets where the shape is a config-4 one):
//  * 128 x 128 tiles, four workgroups per CU, when they make more than two rounds of the CUs
//    (gate/up 37888 x 3584 at M = 512 133.0 [152.2], at M = 2048 476.3 [530.8]; qkv 4608 x 3584
//    at M = 2048 77.4 against 81.3 split).
//  * The same tiles with K split over two wave groups (one eight-wave workgroup, two per CU)
//    when they make one to two rounds (down 3584 x 18944 at M = 2048: 266.2 [298.2], 300.5
//    unsplit, 284.4 for 256 x 128 tiles split the same way; at short K too: qkv at M = 512 31.8
//    against 39.4 unsplit, at M = 1024 49.6 against 54.1, 3584 x 3584 at M = 2048 57.0 against
//    62.7, gate/up at M = 128 50.3 against 54.4).
//  * 128 x 64 tiles with K split over four groups of two waves when 128 x 128 tiles would leave
//    CUs idle and the 128 x 64 ones fill three quarters to all of them (down at M = 512: 98.8
//    [102.3], 189.8 for 128 x 128 tiles; 3584 x 3584 at M = 512 24.1 against 31.4 split in two).
//  * 64 x 64 tiles with K split over four groups of two waves, two per CU, on smaller grids
//    (down at M = 256 57.7 against 89.3 for 128 x 64 tiles and 140.5 for the two-group split,
//    64.6 for the standard GEMM; 3584 x 3584 at M = 256 15.4 against 22.4; qkv at M = 128 15.1
//    against 22.4) and whenever M <= 64, where 128-row tiles would be half empty (gate/up at
//    M = 32 33.7 against 49.7 for the two-group split).
// Weights one tile column (128 k) ahead in every plan: two columns ahead ran 3-8 % slower
// (gate/up at M = 2048 489.6 against 473.0, M = 512 142.9 against 132.4), three 13 %.
int gemm_packed_plan(int M, int N, int K) {
  (void)K;
  int cus = 256;  // the device's CU count (a failed query leaves MI355X's; the launch reports it)
  if (cached_cu_count(&cus) != hipSuccess || cus <= 0) cus = 256;
  if (M <= 64) return 3;
  const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
  const long t128x64 = (long)((M + 127) / 128) * ((N + 63) / 64);
  if (t128 < cus && 4 * t128x64 >= 3 * cus && t128x64 <= cus) return 2;
  if (t128 > 2 * cus) return 0;
  return 2 * t128 > cus ? 1 : 3;
}

namespace {
template <bool SW>
hipError_t launch_gemm_packed_t(const uint16_t* A, const uint32_t* Wp, const uint16_t* Sp, uint16_t* C,
                                int M, int N, int K, int plan, hipStream_t st) {
  switch (plan) {
    case 0:  // 128 x 128 tiles
      hipLaunchKernelGGL((w4_gemm_pk_kernel<128, 4, 1, 1, SW>), dim3((N + 127) / 128, (M + 127) / 128),
                         dim3(256), 0, st, A, Wp, Sp, C, M, N, K);
      return hipSuccess;
    case 1:  // 128 x 128 tiles, K split over two groups of four waves
      hipLaunchKernelGGL((w4_gemm_pk_kernel<128, 4, 2, 1, SW>), dim3((N + 127) / 128, (M + 127) / 128),
                         dim3(512), 0, st, A, Wp, Sp, C, M, N, K);
      return hipSuccess;
    case 2:  // 128 x 64 tiles, K split over four groups of two waves
      hipLaunchKernelGGL((w4_gemm_pk_kernel<128, 2, 4, 1, SW>), dim3((N + 63) / 64, (M + 127) / 128),
                         dim3(512), 0, st, A, Wp, Sp, C, M, N, K);
      return hipSuccess;
    case 3:  // 64 x 64 tiles, K split over four groups of two waves
      hipLaunchKernelGGL((w4_gemm_pk_kernel<64, 2, 4, 1, SW>), dim3((N + 63) / 64, (M + 63) / 64),
                         dim3(512), 0, st, A, Wp, Sp, C, M, N, K);
      return hipSuccess;
    default:
      return hipErrorInvalidValue;
  }
}
}  // namespace

hipError_t launch_gemm_packed(const uint16_t* A, const uint32_t* Wp, const uint16_t* Sp, uint16_t* C,
                              int M, int N, int K, int plan, bool swiglu, hipStream_t st) {
  return swiglu ? launch_gemm_packed_t<true>(A, Wp, Sp, C, M, N, K, plan, st)
                : launch_gemm_packed_t<false>(A, Wp, Sp, C, M, N, K, plan, st);
}

hipError_t launch_gemm(const GemmArgs& a, const GemmPlan& p, hipStream_t st) {
  const dim3 grid((a.N + p.bn - 1) / p.bn, (a.M + p.bm - 1) / p.bm);
  switch (p.cfg) {
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
    case 4:
      hipLaunchKernelGGL((w4_gemm2_kernel<128, 32, 4, 3, false, 1, kWeightAhead>), grid, dim3(256), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 5:
      hipLaunchKernelGGL((w4_gemm2_kernel<128, 32, 4, 2, false, 2, kWeightAhead>), grid, dim3(512), 0, st, a.A,
                         a.Wq, a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 6:
      hipLaunchKernelGGL((w4_gemm2_kernel<256, 32, 4, 2, false, 1, kWeightAhead>), grid, dim3(256), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 7:
      hipLaunchKernelGGL((w4_gemm2_kernel<256, 32, 4, 2, false, 2, kWeightAhead>), grid, dim3(512), 0, st, a.A, a.Wq, a.S,
                         a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 8:
      hipLaunchKernelGGL((w4_gemm2_kernel<128, 32, 2, 2, false, 4, kWeightAhead>), grid, dim3(512), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 9:
      hipLaunchKernelGGL((w4_gemm2_kernel<64, 32, 2, 2, false, 4, kWeightAhead>), grid, dim3(512), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_swiglu(const GemmArgs& a, const GemmPlan& p, hipStream_t st) {
  const dim3 grid((a.N + p.bn - 1) / p.bn, (a.M + p.bm - 1) / p.bm);
  switch (p.cfg) {
    case 4:
      hipLaunchKernelGGL((w4_gemm2_kernel<128, 32, 4, 3, true, 1, kWeightAhead>), grid, dim3(256), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 5:
      hipLaunchKernelGGL((w4_gemm2_kernel<128, 32, 4, 2, true, 2, kWeightAhead>), grid, dim3(512), 0, st, a.A,
                         a.Wq, a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 6:
      hipLaunchKernelGGL((w4_gemm2_kernel<256, 32, 4, 2, true, 1, kWeightAhead>), grid, dim3(256), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 7:
      hipLaunchKernelGGL((w4_gemm2_kernel<256, 32, 4, 2, true, 2, kWeightAhead>), grid, dim3(512), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 8:
      hipLaunchKernelGGL((w4_gemm2_kernel<128, 32, 2, 2, true, 4, kWeightAhead>), grid, dim3(512), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    case 9:
      hipLaunchKernelGGL((w4_gemm2_kernel<64, 32, 2, 2, true, 4, kWeightAhead>), grid, dim3(512), 0, st, a.A, a.Wq,
                         a.S, a.C, a.M, a.N, a.K, ilog2(a.G));
      return hipSuccess;
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace ns
