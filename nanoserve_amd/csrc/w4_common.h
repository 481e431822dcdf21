// Shared device helpers for the W4A16 kernels (gfx950 / CDNA4, wave64).
//
// Weight format (kernels/quant/w4a16.cuh:5-9 in the reference):
//   Wq [N][K/8] uint32: word j of row n holds k = 8j..8j+7, k = 8j+i in bits 4i..4i+3
//   S  [N][K/G] bf16:   one scale per G consecutive k
//   w[n][k] = (q - 8) * S[n][k / G],  q in [0, 15]
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace ns {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

constexpr int kWave = 64;

// Cache policy of the GEMV weight and scale streams (the aux operand of buffer loads: bit 0 =
// sc0, bit 1 = nt). Each byte is read once per launch, so the loads are marked non-temporal:
// on MI355X this made every M = 1 and M = 8 GEMV layer 3-8 % faster than default-policy loads
// (same outputs); sc0 with nt measured on par with nt alone, slightly ahead on gate/up.
constexpr int kStreamAux = 3;

// Cache rows per split of the decode attention (decode_ops.hip); the attention-merging
// activation load of the decode GEMV (w4_gemv.hip) reads the same split layout.
constexpr int kAttnDecodeChunk = 128;

// Workgroup barrier for LDS traffic: this wave's LDS operations complete (lgkmcnt(0)), then
// s_barrier. Outstanding global loads and stores stay in flight; the release fence of
// __syncthreads() would make a wave that has stored to global memory wait for every vector
// memory operation it issued before (loads and stores share one in-order counter on gfx9).
// The empty asm statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // gfx9 encoding: vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h16) {
  return __uint_as_float(h16 << 16);
}

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet (the reference's
// __float2bfloat16 / __floats2bfloat162_rn semantics, kernels/fused/vec.cuh:14-19). Written as
// a select, not an early return: the compiler turns the early-return form into a divergent
// branch (exec-mask save and restore) around every conversion.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : r;
}

// Two fp32 -> packed bf16x2 (lo in bits 0..15), RNE. An fp32 -> bf16 vector truncation, which
// gfx950 lowers to its single v_cvt_pk_bf16_f32 (round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t f = {lo, hi};
  const bf16x2_t v = __builtin_convertvector(f, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

// One packed word (8 nibbles, k ascending) -> four bf16x2 dwords holding (128 + q) exactly:
// dword j = bf16(128 + q[2j]) | bf16(128 + q[2j+1]) << 16. bf16(128 + q) is 0x4300 | q for
// q in [0, 15] (exponent 2^7, q in the low mantissa bits), so no arithmetic is needed:
// one byte permute places nibble 2j (byte j of w) and nibble 2j+1 (byte j of w >> 4) in the
// low nibbles of the two halves, one AND-OR masks them and sets the exponent.
__device__ __forceinline__ void unpack_word_128q(uint32_t w, uint32_t (&d)[4]) {
  const uint32_t w4 = w >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // selector bytes: out0 <- w.byte j, out1 <- 0, out2 <- w4.byte j, out3 <- 0
    const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + j) << 16) | (uint32_t)j;
    const uint32_t t = __builtin_amdgcn_perm(w4, w, sel);
    d[j] = (t & 0x000F000Fu) | 0x43004300u;
  }
}

// Eight bf16 (one 16-byte vector, element 2i in the low half of word i) <-> fp32.
__device__ __forceinline__ void unpack8(const u32x4_t& u, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4_t pack8(const float (&f)[8]) {
  u32x4_t u;
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = pack_bf16x2_rne(f[2 * i], f[2 * i + 1]);
  return u;
}

// fp32 rounded to the nearest bf16 (ties to even), as an fp32: the hardware conversion
// (v_cvt_pk_bf16_f32, one instruction) and a shift, where the integer form takes six
// instructions. The same rounding as f32_to_bf16_rne for every non-NaN input.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(pack_bf16x2_rne(f, 0.f));
}

// The value of lane l ^ 32 and of lane l ^ 16, by the gfx950 lane-swap instructions (no LDS
// round trip, unlike a shuffle): v_permlane32_swap of a register with itself yields its lower
// half-wave in both halves of the first result and its upper half-wave in the second;
// v_permlane16_swap does the same for the even / odd 16-lane rows.
__device__ __forceinline__ float lane_xor32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (__lane_id() & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (__lane_id() & 16) ? r[0] : r[1]);
}
// The value of lane l ^ 8 (DPP row_ror:8 rotates each 16-lane row by 8).
__device__ __forceinline__ float lane_xor8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
}

// Sum over the 64 lanes, returned to every lane. DPP row shifts build each 16-lane row's sum in
// its last lane (inclusive scan, lanes shifted in from outside the row add 0), two row
// broadcasts (gfx9 row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3) carry it
// to lane 63, which is read back as a scalar: no LDS round trips, unlike lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
  auto dpp = [](float x, auto ctrl, auto rmask) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                 decltype(ctrl)::value,
                                                                 decltype(rmask)::value, 0xf, false));
  };
  using C111 = std::integral_constant<int, 0x111>;
  using C112 = std::integral_constant<int, 0x112>;
  using C114 = std::integral_constant<int, 0x114>;
  using C118 = std::integral_constant<int, 0x118>;
  using C142 = std::integral_constant<int, 0x142>;
  using C143 = std::integral_constant<int, 0x143>;
  using MF = std::integral_constant<int, 0xf>;
  using MA = std::integral_constant<int, 0xa>;
  using MC = std::integral_constant<int, 0xc>;
  v += dpp(v, C111{}, MF{});
  v += dpp(v, C112{}, MF{});
  v += dpp(v, C114{}, MF{});
  v += dpp(v, C118{}, MF{});
  v += dpp(v, C142{}, MA{});
  v += dpp(v, C143{}, MC{});
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// silu(g) * u, the reference's SwiGLU (kernels/fused/swiglu.cuh:8), in fp32.
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.f + __expf(-g)) * u; }

// Round half to even, then a saturating int32 conversion with NaN -> 0 (the semantics of the
// reference's __float2int_rn), written out so no out-of-range conversion is left undefined.
__device__ __forceinline__ int f2i_rn(float x) {
  if (!(x == x)) return 0;
  const float r = __builtin_rintf(x);
  if (r >= 2147483648.f) return 0x7fffffff;
  if (r < -2147483648.f) return (int)0x80000000u;
  return (int)r;
}

}  // namespace ns
