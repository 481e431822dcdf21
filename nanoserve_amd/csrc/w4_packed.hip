// Pre-shuffled ("packed") W4 weights and the GEMV that reads them, for gfx950 (wave64).
//
// No counterpart in the reference's kernels: its README (149-151) names a Marlin-style
// pre-shuffled format as the next step for the W4 path. The interchange format (Wq [N][K/8]
// uint32, S [N][K/G] bf16, w = (q - 8) * s) stays what ns_w4_quantize / ns_w4_linear use;
// ns_w4_repack rewrites it once, offline, into tiles laid out for the MFMA operands:
//
//   tile (t, c) = rows 16t .. 16t+15 x k = 128c .. 128c+127 (G = 128: one scale per row), 1 KiB
//   of codes: lane l (0..63) of a wave owns bytes 16l .. 16l+15, four words s = 0..3, word s =
//   row 16t + l%16 at k = 128c + 32s + 8(l/16) + e, e = 0..7, nibbles in the order
//   e0 e2 e4 e6 e1 e3 e5 e7, so that (word >> 4i) & 0x000F000F holds elements 2i, 2i+1: one
//   shift and one AND-OR per pair give the B operand of v_mfma_f32_16x16x32_bf16 in natural k
//   order. Tiles are stored tile-row by tile-row (t major, c minor): a tile-row is one
//   contiguous (K/128) KiB run. Scales: 16 bf16 per tile (32 bytes), row order, same tile order.
//   Rows past N (N not a multiple of 16) are zero codes with zero scales.
//
// The GEMV (M = 1..16 activation rows): each wave owns a fixed set of k-groups c (c = wave,
// wave + NW, ...), holds the activation's slices for them in registers for the whole kernel
// (A operand: lane l = activation row l%16, k slice 8(l/16)..+7), and streams its tiles of
// every tile-row it visits: one 16-byte load per lane per tile is the tile's B operand. The
// accumulator of a tile starts at -136 * sum(x) over the group (an MFMA of x with a constant
// -136 operand, once per group), so 4 MFMAs on bf16(128 + q) give sum x (q - 8) exactly before
// the fp32 scale. The waves' partial sums of a tile-row are added through LDS, one barrier per
// tile-row; no LDS reads of the activation and no diagonal extraction in the inner loop.
#include <stdint.h>

#include <type_traits>

#include "../../include/nanoserve_w4.h"
#include "w4_common.h"
#include "w4_kernels.h"

namespace ns {
namespace {

constexpr uint32_t kPackOOB = 0x7fffffc0u;

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>), in order
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// One packed word -> eight bf16 (128 + q) in natural k order.
__device__ __forceinline__ u32x4_t unpack_packed(uint32_t w) {
  u32x4_t d;
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = ((w >> (4 * i)) & 0x000F000Fu) | 0x43004300u;
  return d;
}

// element e of a natural-order word -> nibble position in the packed word
__device__ __forceinline__ uint32_t pack_nibbles(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int p = (e & 1) ? 4 + (e >> 1) : (e >> 1);
    o |= ((w >> (4 * e)) & 0xFu) << (4 * p);
  }
  return o;
}

__global__ void __launch_bounds__(256)
    w4_repack_kernel(const uint32_t* __restrict__ Wq, const uint16_t* __restrict__ S,
                     uint32_t* __restrict__ Wp, uint16_t* __restrict__ Sp, int N, int K) {
  const int C = K >> 7, KW = K >> 3;
  const long long NT = (N + 15) >> 4;
  const long long words = NT * C * 256;
  for (long long idx = blockIdx.x * 256LL + threadIdx.x; idx < words;
       idx += (long long)gridDim.x * 256) {
    const long long tile = idx >> 8;
    const int wi = static_cast<int>(idx & 255), lane = wi >> 2, s4 = wi & 3;
    const long long t = tile / C;
    const int c = static_cast<int>(tile % C);
    const long long row = 16 * t + (lane & 15);
    const uint32_t w = row < N ? Wq[row * KW + 16 * c + 4 * s4 + (lane >> 4)] : 0u;
    Wp[idx] = pack_nibbles(w);
  }
  const long long scales = NT * C * 16;
  for (long long idx = blockIdx.x * 256LL + threadIdx.x; idx < scales;
       idx += (long long)gridDim.x * 256) {
    const long long tile = idx >> 4;
    const long long t = tile / C;
    const int c = static_cast<int>(tile % C);
    const long long row = 16 * t + (idx & 15);
    Sp[idx] = row < N ? S[row * C + c] : static_cast<uint16_t>(0);
  }
}

// NW waves per workgroup; GW: k-groups per wave the registers are sized for (C <= GW * NW).
template <int NW, int GW>
__global__ __launch_bounds__(NW * kWave) void w4_gemv_packed_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wp,
    const uint16_t* __restrict__ Sp, uint16_t* __restrict__ Y, int M, int N, int K) {
  __shared__ float part[2][NW][256];
  const int C = K >> 7;
  const int NT = (N + 15) >> 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int ng = wv < C ? (C - 1 - wv) / NW + 1 : 0;  // this wave's k-groups (uniform)

  // activation slices first (the weight loads issued after them do not hold them up)
  u32x4_t xf[GW][4];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    const int c = wv + NW * g;
    const bool ok = g < ng && j < M;
    const uint16_t* src = X + (size_t)j * K + 128 * c + 8 * kg;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      xf[g][s4] = ok ? *reinterpret_cast<const u32x4_t*>(src + 32 * s4) : u32x4_t{0u, 0u, 0u, 0u};
  }

  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wp), (short)0, (int)((size_t)NT * C * 1024), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Sp), (short)0, (int)((size_t)NT * C * 32), 0x00020000);
  u32x4_t wr[2][GW];
  uint32_t sr[2][GW];
  auto issue = [&](auto slot_c, int t) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const bool live = t < NT && g < ng;
      const uint32_t tile = (uint32_t)(t * C + wv + NW * g);
      wr[slot][g] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                    wres, 16u * lane, live ? 1024u * tile : kPackOOB, kStreamAux));
      sr[slot][g] = __builtin_amdgcn_raw_buffer_load_b16(sres, 2u * j, live ? 32u * tile : kPackOOB, kStreamAux);
    }
  };
  const int step = gridDim.x;
  int t = blockIdx.x;
  issue(std::integral_constant<int, 0>{}, t);

  // -136 * sum_k x[i][k] over each group: D layout (lane holds rows 4 kg + r)
  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  f32x4_t corr[GW];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xf[g][s4]),
                                                  __builtin_bit_cast(bf16x8_t, kNeg136), d, 0, 0, 0);
    corr[g] = d;
  }

  auto body = [&](auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    issue(std::integral_constant<int, slot ^ 1>{}, t + step);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      if (g < ng) {
        f32x4_t d = corr[g];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, xf[g][s4]),
              __builtin_bit_cast(bf16x8_t, unpack_packed(wr[slot][g][s4])), d, 0, 0, 0);
        const float sc = bf16_bits_to_f32(sr[slot][g] & 0xffffu);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc, d[r], acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) part[slot][wv][(4 * kg + r) * 16 + j] = acc[r];
    __syncthreads();
    for (int o = tid; o < 16 * M; o += NW * kWave) {
      const int i = o >> 4, jj = o & 15;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += part[slot][w][i * 16 + jj];
      const int n = 16 * t + jj;
      if (n < N) Y[(size_t)i * N + n] = static_cast<uint16_t>(f32_to_bf16_rne(v));
    }
    t += step;
  };
  while (t < NT) {
    body(std::integral_constant<int, 0>{});
    if (t >= NT) break;
    body(std::integral_constant<int, 1>{});
  }
}

// Long rows (K > 32 * 128): the activation's group slices do not fit in registers. Each wave
// still owns the k-groups c = wave, wave + NW, ... and issues all its tiles of a tile-row at once
// (a long row gives each wave up to GW of them: the memory-level parallelism a 16-row tile-row of
// a long row needs), but the activation passes through LDS in chunks: chunk g holds the k-groups
// NW g .. NW g + NW - 1 of all M rows, xl[c % NW][m][128], so each wave finds its g-th group there.
// Chunk g + 1 is loaded into registers while chunk g is used (two barriers per chunk); lanes of
// activation rows >= M use zeros. The -136 sum(x) correction of a group is the same MFMA against a
// constant -136 operand as in the register kernel, taken when the group's chunk is in LDS. Any
// M <= 16 and K <= 128 NW GW fit: the LDS holds one chunk (M NW 256 bytes).
template <int NW, int GW>
__global__ __launch_bounds__(NW * kWave) void w4_gemv_packed_lds_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wp,
    const uint16_t* __restrict__ Sp, uint16_t* __restrict__ Y, int M, int N, int K) {
  __shared__ float part[2][NW][256];
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT_ = NW * kWave;
  const int C = K >> 7;
  const int NT = (N + 15) >> 4;
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);  // [NW][M][128]: one chunk of k-groups
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int ng = wv < C ? (C - 1 - wv) / NW + 1 : 0;
  const int nch = (C + NW - 1) / NW;  // chunks (uniform)

  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wp), (short)0, (int)((size_t)NT * C * 1024), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Sp), (short)0, (int)((size_t)NT * C * 32), 0x00020000);
  // the activation through its own range-checked buffer: vectors past M K read as zeros
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(X), (short)0, (int)((size_t)M * K * 2), 0x00020000);
  // this wave's tile of chunk g into ring slot g % PD (PD tiles in flight per wave)
  constexpr int PD = 3;
  u32x4_t wr[PD];
  uint32_t sr[PD];
  auto issue = [&](int t, auto g_c) {
    constexpr int g = decltype(g_c)::value;
    const bool live = t < NT && g < ng;
    const uint32_t tile = (uint32_t)(t * C + wv + NW * g);
    wr[g % PD] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                 wres, 16u * lane, live ? 1024u * tile : kPackOOB, kStreamAux));
    sr[g % PD] = __builtin_amdgcn_raw_buffer_load_b16(sres, 2u * j, live ? 32u * tile : kPackOOB, kStreamAux);
  };
  // chunk g: vector e of the chunk (16 bytes) is row m = (e / 16) % M of k-group
  // NW g + e / (16 M), k = 8 (e % 16) of the group; at most 4 vectors per thread (M <= 16)
  const int cvec = M * NW * 16;
  // per vector slot i of this thread: its k-group within a chunk (cl, or C when the slot is
  // unused) and its byte offset in chunk 0; chunk g adds 256 NW g bytes
  int xcl[4];
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid + i * NT_;
    const int cl = e / (M * 16), m = (e >> 4) % M;
    xcl[i] = e < cvec ? cl : C;
    xoff[i] = 2u * (uint32_t)(m * K + 128 * cl + 8 * (e & 15));
  }
  auto load_chunk = [&](int g, u32x4_t (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = NW * g + xcl[i] < C;
      const uint32_t off = ok ? xoff[i] + 256u * (uint32_t)(NW * g) : kPackOOB;
      v[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 0, 0));
    }
  };
  auto store_chunk = [&](const u32x4_t (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + i * NT_;
      if (e < cvec) *reinterpret_cast<u32x4_t*>(&xl[8 * e]) = v[i];
    }
  };
  auto afrag = [&](int s4) {  // this wave's group of the chunk in LDS
    return j < M ? *reinterpret_cast<const u32x4_t*>(&xl[((size_t)wv * M + j) * 128 + 32 * s4 + 8 * kg])
                 : u32x4_t{0u, 0u, 0u, 0u};
  };
  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};

  for (int it = 0, t = blockIdx.x; t < NT; ++it, t += gridDim.x) {
    u32x4_t xv[4];
    load_chunk(0, xv);  // ahead of the weights: the first chunk is needed first
    issue(t, std::integral_constant<int, 0>{});
    issue(t, std::integral_constant<int, 1>{});
    issue(t, std::integral_constant<int, 2>{});
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    static_for<GW>([&](auto g_c) {
      constexpr int g = decltype(g_c)::value;
      if (g < nch) {  // uniform
        lds_sync();   // every wave is done with the previous chunk
        store_chunk(xv);
        lds_sync();
        if (g + 1 < nch) load_chunk(g + 1, xv);
        if (g < ng) {
          f32x4_t d = {0.f, 0.f, 0.f, 0.f};
          u32x4_t xf[4];
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) {
            xf[s4] = afrag(s4);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xf[s4]),
                                                        __builtin_bit_cast(bf16x8_t, kNeg136), d, 0, 0, 0);
          }
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, xf[s4]),
                __builtin_bit_cast(bf16x8_t, unpack_packed(wr[g % PD][s4])), d, 0, 0, 0);
          const float sc = bf16_bits_to_f32(sr[g % PD] & 0xffffu);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc, d[r], acc[r]);
        }
        if constexpr (g + PD < GW) issue(t, std::integral_constant<int, g + PD>{});
      }
    });
    float* pw = &part[it & 1][wv][0];
#pragma unroll
    for (int r = 0; r < 4; ++r) pw[(4 * kg + r) * 16 + j] = acc[r];
    __syncthreads();
    for (int o = tid; o < 16 * M; o += NT_) {
      const int i = o >> 4, jj = o & 15;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += part[it & 1][w][i * 16 + jj];
      const int n = 16 * t + jj;
      if (n < N) Y[(size_t)i * N + n] = static_cast<uint16_t>(f32_to_bf16_rne(v));
    }
  }
}

// dynamic LDS of the long-row kernel: one chunk of NW k-groups of the M activation rows
size_t packed_lds_bytes(int NW, int M) { return (size_t)NW * M * 256; }

template <int NW, int GW>
hipError_t launch_packed_lds(const uint16_t* X, const uint32_t* Wp, const uint16_t* Sp,
                             uint16_t* Y, int M, int N, int K, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&w4_gemv_packed_lds_kernel<NW, GW>);
  const hipError_t attr = cached_max_dynamic_lds(fn, 128 * 1024);
  if (attr != hipSuccess) return attr;
  int cus = 0;
  hipError_t e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int NT = (N + 15) / 16;
  const int grid = NT < cus ? NT : cus;
  hipLaunchKernelGGL((w4_gemv_packed_lds_kernel<NW, GW>), dim3(grid), dim3(NW * kWave),
                     packed_lds_bytes(NW, M), st, X, Wp, Sp, Y, M, N, K);
  return hipSuccess;
}

template <int NW, int GW>
hipError_t launch_packed(const uint16_t* X, const uint32_t* Wp, const uint16_t* Sp, uint16_t* Y,
                         int M, int N, int K, hipStream_t st) {
  int cus = 0;
  hipError_t e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  // measured on MI355X: two workgroups per CU with one k-group per wave, one with two
  const int NT = (N + 15) / 16;
  const int cap = (GW == 1 ? 2 : 1) * cus;
  const int grid = NT < cap ? NT : cap;
  hipLaunchKernelGGL((w4_gemv_packed_kernel<NW, GW>), dim3(grid), dim3(NW * kWave), 0, st, X, Wp,
                     Sp, Y, M, N, K);
  return hipSuccess;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

size_t packed_weight_bytes(int N, int K) { return (size_t)((N + 15) / 16) * (K / 128) * 1024; }
size_t packed_scale_bytes(int N, int K) { return (size_t)((N + 15) / 16) * (K / 128) * 32; }

}  // namespace ns

extern "C" {

int ns_w4_repack(const void* Wq, const void* S, void* Wp, void* Sp, int N, int K, int G,
                 void* stream) {
  if (N <= 0 || K <= 0 || G != 128 || K % 128) return -2;
  if (ns::packed_weight_bytes(N, K) >= (1ull << 31)) return -2;
  if (!Wq || !S || !Wp || !Sp || !ns::aligned(Wq, 4) || !ns::aligned(S, 2) ||
      !ns::aligned(Wp, 16) || !ns::aligned(Sp, 16))
    return -2;
  const size_t words = ns::packed_weight_bytes(N, K) / 4;
  const unsigned grid = static_cast<unsigned>(words / 256 < 4096 ? (words + 255) / 256 : 4096);
  hipLaunchKernelGGL(ns::w4_repack_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(Wq),
                     static_cast<const uint16_t*>(S), static_cast<uint32_t*>(Wp),
                     static_cast<uint16_t*>(Sp), N, K);
  return static_cast<int>(hipGetLastError());
}

int ns_w4_linear_packed(const void* X, const void* Wp, const void* Sp, void* Y, int M, int N,
                        int K, int G, void* stream) {
  // M = 1 is not taken: the standard format's M = 1 kernel (ns_w4_linear) streams the same
  // bytes faster (MI355X, Qwen2.5-7B layers: gate/up 13.8 against 15.2 us, q/k/v 4.7 against
  // 5.1), so the packed format serves batched decode, M = 2..16, where it is the faster one,
  // and prefill, M > 16
  // M > 16 (prefill) runs the GEMM on the packed tiles: its activation offsets (rows up to M +
  // 255 of the last tile) stay in 31 bits
  if (M < 2 || N <= 0 || K <= 0 || G != 128 || K % 128) return -2;
  if (M > 16 && (uint64_t)(M + 256) * (uint64_t)K * 2 >= (1ull << 31)) return -2;
  if (ns::packed_weight_bytes(N, K) >= (1ull << 31)) return -2;
  if (!X || !Wp || !Sp || !Y || !ns::aligned(X, 16) || !ns::aligned(Wp, 16) ||
      !ns::aligned(Sp, 16) || !ns::aligned(Y, 2))
    return -2;
  const int C = K / 128;
  const auto st = static_cast<hipStream_t>(stream);
  const auto x = static_cast<const uint16_t*>(X);
  const auto wp = static_cast<const uint32_t*>(Wp);
  const auto sp = static_cast<const uint16_t*>(Sp);
  const auto y = static_cast<uint16_t*>(Y);
  hipError_t e;
  if (M > 16)
    e = ns::launch_gemm_packed(x, wp, sp, y, M, N, K, ns::gemm_packed_plan(M, N, K), false, st);
  else if (C <= 16)
    e = ns::launch_packed<16, 1>(x, wp, sp, y, M, N, K, st);
  else if (C <= 32)
    e = ns::launch_packed<16, 2>(x, wp, sp, y, M, N, K, st);
  else if (C <= 160)
    e = ns::launch_packed_lds<16, 10>(x, wp, sp, y, M, N, K, st);
  else
    return -2;
  if (e != hipSuccess) return static_cast<int>(e);
  return static_cast<int>(hipGetLastError());
}

int ns_w4_linear_packed_swiglu(const void* X, const void* Wp, const void* Sp, void* Y, int M,
                               int N, int K, int G, void* stream) {
  // prefill only (M > 16): the GEMM on the packed tiles with the SwiGLU epilogue; the gate/up
  // rows come interleaved in blocks of 8, so N is a multiple of 16
  if (M <= 16 || N <= 0 || K <= 0 || G != 128 || K % 128 || N % 16) return -2;
  if ((uint64_t)(M + 256) * (uint64_t)K * 2 >= (1ull << 31)) return -2;
  if (ns::packed_weight_bytes(N, K) >= (1ull << 31)) return -2;
  if (!X || !Wp || !Sp || !Y || !ns::aligned(X, 16) || !ns::aligned(Wp, 16) ||
      !ns::aligned(Sp, 16) || !ns::aligned(Y, 2))
    return -2;
  const hipError_t e = ns::launch_gemm_packed(
      static_cast<const uint16_t*>(X), static_cast<const uint32_t*>(Wp),
      static_cast<const uint16_t*>(Sp), static_cast<uint16_t*>(Y), M, N, K,
      ns::gemm_packed_plan(M, N, K), true, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return static_cast<int>(e);
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
