// W4A16 decode GEMV for M = 1..8 on gfx950 (CDNA4).
//
// Replaces w4a16_gemv_kernel / w4a16_gemv (kernels/quant/w4a16.cuh:34-115 in the reference):
//   Y[M][N] (bf16, RNE) = X[M][K] (bf16) . deq(Wq, S)^T, fp32 accumulation.
//
// Every fast-path kernel (K % 128 == 0, G % 128 == 0) shares one arithmetic: the weight operand
// of v_mfma_f32_16x16x32_bf16 is the exact integer 128 + q in bf16 (0x4300 | q: bit operations,
// no float arithmetic), the accumulator starts at -136 * sum_k x over the chunk (one MFMA
// against a constant), so a chunk's partial is sum_k x * (q - 8) exactly, and the bf16 group
// scale is applied in fp32 after the chunk. No weight is ever rounded: the dequant is exact, as
// in the reference GEMV (w4a16.cuh:28-32). The kernels differ in how HBM is streamed:
//  * w4_gemv_m1_kernel (M = 1, G = 128): the weights as one sequential stream of 1 KiB blocks
//    (16 row pieces of 128 k), the partial of each piece on the diagonal of one MFMA, workgroups
//    persistent over row groups (or one round of ceil(N / CUs) rows per CU for small layers),
//    with the neighbouring decode operators fused into its activation load and its output.
//  * w4_gemv_m8_kernel (M = 2..8, G = 128, K % 256 == 0 up to 20480): the same stream as
//    8 rows x 128 B per wave instruction, activation fragments held in registers; K of more
//    than 32 pairs (256 k each) runs in K slices whose fp32 partials w4_gemv_m8_merge_kernel sums.
//  * w4_gemv_lds_kernel / w4_gemv_xlds_kernel (the M = 2..8 shapes the previous kernel does
//    not take): weights or activations staged in LDS.
//  * w4_gemv_mfma_kernel (the remaining M = 2..8 shapes): 16-row tiles per wave, split K inside
//    the workgroup, loads issued in batches.
// The launchers (gemv_plan, launch_gemv and the fused decode entries, end of file) pick the
// kernel and its layout per shape from the device's CU count.
//
// Generic path (any K % 32 == 0, G % 32 == 0, K % G == 0): one wavefront per output row,
// VALU fp32 FMAs with the exact fp32 dequant, cross-lane reduction.
#include <type_traits>

#include "w4_common.h"
#include "w4_kernels.h"

namespace ns {

namespace {

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Bytes of the scale array (N x C bf16) that a buffer resource covers in the kernels loading
// scales 16 bytes at a time: rounded up to whole dwords. A dword load that reaches past the
// resource's range reads as zero as a whole, so with N * C odd the array's last scale, which
// shares a dword with the two bytes after the array, would read as zero. The launcher sends a
// scale array that is not 4-byte aligned to another kernel in that case, so the two extra bytes
// lie in the (4-byte aligned) dword that holds the last scale; they only ever land in the
// scale slot of a row past N, whose output is not stored.
__host__ __device__ inline int scale_span_bytes(int N, int C) {
  return (int)((((size_t)N * C * 2) + 3) & ~(size_t)3);
}

// Row-tiled kernel: a wavefront owns RT 16-row tiles of W and a contiguous range of 128-k
// chunks; the NW wavefronts of a workgroup split K and are reduced through LDS at the end.
// Lane l = 16 h + r loads 16 bytes of row r (words 4h..4h+3 of the chunk) per chunk, so the
// wave reads 1 KiB of packed weights per chunk per tile; MFMA A = weights (row i = output
// feature), B = X^T (column j = batch row, padded to 16). Loads of W and X are issued in
// batches of UB chunks (up to UB x RT KiB in flight per wave). The workgroup's scales are
// staged once in LDS, transposed to [group][row], so a lane reads its four rows' scales with
// one 8-byte LDS read.
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
      for (int rt = 0; rt < RT; ++rt) wb[u][rt] = __builtin_nontemporal_load(&wp[rt][4 * c]);
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

// Activations-in-LDS kernel, used whenever M x K bf16 fits in LDS (every M = 1 shape, and
// M = 8 up to K of about 7000). Same arithmetic as w4_gemv_mfma_kernel, organised to keep the
// VALU work per weight near one instruction:
//  * Weights come through buffer loads (one 16-byte load per lane per chunk and row tile):
//    the per-lane row offset is computed once, the chunk offset is a scalar, and rows past N
//    read as zero through the buffer's range check, so no address or clamp math per chunk.
//  * Nibbles are paired (i, i + 4): dword i = bf16(128 + q[i]) | bf16(128 + q[i+4]) << 16 is
//    one shift and one v_and_or_b32 (mask in a VGPR, exponent bits in an SGPR). X is staged in
//    LDS with the same pairing (k order 0,4,1,5,2,6,3,7 inside every 8), so both MFMA
//    operands agree on k.
//  * The -136 * sum_k x offsets are computed once per wave for all of its chunks, 16 / Mp
//    chunks per MFMA group (B column j = (batch row j % Mp, chunk j / Mp), A = -136), kept in
//    LDS, and enter each chunk's product as the MFMA accumulator's initial value.
//  * Scales are staged in LDS as fp32, transposed to [group][row]: a lane reads its four
//    rows' scales with one 16-byte LDS read.
//  * Weights stream through two fixed register sets of UB chunks (double buffering): one set
//    is in flight while the other is consumed, and a set is refilled only after its last use.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t vmask, uint32_t sbits) {
  uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(vmask), "s"(sbits));
  return d;
}

// Packed word (nibbles k = 0..7) -> four bf16x2 dwords (128 + q[i], 128 + q[i + 4]), i = 0..3.
__device__ __forceinline__ u32x4_t unpack_word_paired(uint32_t w, uint32_t vmask, uint32_t sbits) {
  u32x4_t d;
  d[0] = and_or(w, vmask, sbits);
  d[1] = and_or(w >> 4, vmask, sbits);
  d[2] = and_or(w >> 8, vmask, sbits);
  d[3] = and_or(w >> 12, vmask, sbits);
  return d;
}

// Eight bf16 in natural order (4 dwords) -> the same eight in pair order (0,4),(1,5),(2,6),(3,7).
__device__ __forceinline__ u32x4_t pair_order(const u32x4_t& v) {
  u32x4_t o;
  o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
  o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
  o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
  o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
  return o;
}

// Chunk bookkeeping of the LDS-activation kernel: every wave owns NCW chunks of each row tile,
// a multiple of the ring depth R, over a chunk range padded to CP = NW * NCW >= C. LDS tables
// are padded with zeros up to CP, so the loop has no per-chunk clamps, divisions or branches.
struct XldsGeom {
  int ncw, cp;
};
__host__ __device__ inline XldsGeom xlds_geom(int K, int nw, int r) {
  const int C = K >> 7;
  const int ncw = r * ((C + nw * r - 1) / (nw * r));
  return XldsGeom{ncw, nw * ncw};
}

// Persistent workgroups: X (pair order) and the per-chunk offsets are staged once per
// workgroup, then the workgroup walks row tiles t = blockIdx.x, + gridDim.x, ... Each wave
// owns a fixed slice of K (split-K inside the workgroup); its weight stream runs through the
// tiles without a break: the batch after a tile's last one is the next tile's first, and the
// next tile's scales are loaded during the current tile. One barrier per tile publishes the
// split-K partials; wave (i % NW) finishes tile i.
//
// Weights stream through a ring of R register slots (one chunk of RT row tiles each): a slot
// is consumed, then immediately refilled with the chunk R positions ahead in the wave's stream
// (continuing into the next tile), so R - 1 chunks are always in flight per wave.
//
// MFMA roles: A = X (row i = batch row m), B = W^T (column j = output row n), so the result
// D[m][n] sits in lane (n = lane % 16, m = 4 (lane / 16) + r): each lane needs one scale per
// chunk, its own row's. Those come from one buffer load per tile (the wave's NCW <= 8 SL
// consecutive groups of the lane's row) into a wave-private LDS slab. Loads for padded chunks
// and for tiles past the end use out-of-range buffer offsets: they return zero and touch no
// memory.
template <int RT, int NW, int R, int SL>
__global__ __launch_bounds__(NW * kWave) void w4_gemv_xlds_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int M, int N, int K, int G) {
  constexpr int ROWS = 16 * RT;
  constexpr uint32_t kOOB = 0x7fffffc0u;  // buffer offset past any range: reads return zero
  extern __shared__ __align__(16) unsigned char smem[];
  (void)G;  // this kernel requires G == 128: one scale per chunk
  const XldsGeom geo = xlds_geom(K, NW, R);
  const int KG = K >> 7, C = K >> 7, CP = geo.cp, XP = 128 * CP + 8, KV = K >> 3;
  const int NCW = geo.ncw;  // chunks per wave per tile, a multiple of R
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                  // [M][128 CP + 8], pair order
  size_t off = ((size_t)M * XP * 2 + 15) & ~(size_t)15;
  float* xs = reinterpret_cast<float*>(smem + off);                   // [CP][16]
  off += (size_t)CP * 16 * 4;
  uint32_t* slab = reinterpret_cast<uint32_t*>(smem + off);           // [NW][RT][16][4 SL] bf16x2
  off += (size_t)NW * RT * 16 * 4 * SL * 4;
  float* red = reinterpret_cast<float*>(smem + off);                  // [2][NW][RT][4][64]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, h = lane >> 4;
  const int c0 = wv * NCW;
  const int ntiles = (N + ROWS - 1) / ROWS;
  const int tstep = gridDim.x;

  // Weight rows through a buffer resource: rows >= N read as zero (range check).
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wq), (short)0, (int)((size_t)N * (K >> 1)), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(S), (short)0, scale_span_bytes(N, KG), 0x00020000);
  const uint32_t rowb = (uint32_t)(K >> 1);
  auto issue = [&](u32x4_t (&w)[RT], int tile, int cw) {
    const bool live = tile < ntiles;
    const uint32_t vb = (uint32_t)(min(tile, ntiles - 1) * ROWS + r16) * rowb + 16u * h;
    const int c = c0 + cw;
    const uint32_t so = (live && c < C) ? 64u * c : kOOB;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      w[rt] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              wres, vb + 16u * rt * rowb, so, kStreamAux));
  };
  // Scales of a tile: lane (r16, h == rt) loads groups c0 .. c0 + 8 SL - 1 of row 16 rt + r16.
  auto load_scales = [&](u32x4_t (&sv)[SL], int tile) {
    const int rt = min(h, RT - 1);
    const bool live = tile < ntiles;
    const uint32_t vb = ((uint32_t)(min(tile, ntiles - 1) * ROWS + 16 * rt + r16) * (uint32_t)KG + c0) * 2u;
#pragma unroll
    for (int j = 0; j < SL; ++j)
      sv[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              sres, vb, live ? 16u * j : kOOB, 0));
  };
  uint32_t* wslab = slab + wv * RT * 16 * 4 * SL;
  auto store_scales = [&](const u32x4_t (&sv)[SL]) {
    if (h < RT) {
#pragma unroll
      for (int j = 0; j < SL; ++j)
        *reinterpret_cast<u32x4_t*>(&wslab[(h * 16 + r16) * 4 * SL + 4 * j]) = sv[j];
    }
  };

  int tile = blockIdx.x;
  // The first R chunks are in flight while X is staged and the offsets are computed.
  u32x4_t ring[R][RT];
  u32x4_t sv[SL];
#pragma unroll
  for (int u = 0; u < R; ++u) issue(ring[u], tile, u);
  load_scales(sv, tile);
  __builtin_amdgcn_sched_barrier(0);

  const u32x4_t* x4 = reinterpret_cast<const u32x4_t*>(X);
  const int XV = 16 * CP;  // 8-element pieces per padded row
  for (int e = tid; e < M * XV; e += NW * kWave) {
    const int m = e / XV, v = e - m * XV;
    const u32x4_t val = v < KV ? pair_order(x4[m * KV + v]) : u32x4_t{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(&xl[m * XP + 8 * v]) = val;
  }
  store_scales(sv);
  __syncthreads();

  // xs[c][m] = -136 * sum_k x[m][k] over chunk c: one MFMA group covers 16 / mp chunks
  // (B column j = (batch row j % mp, chunk j / mp), A = -136); columns m >= M hold 0.
  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};  // bf16 -136
  {
    const int mp = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    const int per = 16 / mp;
    const int mj = min(r16 % mp, M - 1), cc = r16 / mp;
    for (int cg = c0; cg < c0 + NCW; cg += per) {
      const int c = min(cg + cc, CP - 1);
      const uint16_t* xr = &xl[mj * XP + 128 * c + 32 * h];
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(kNeg136), as_bf16x8(*reinterpret_cast<const u32x4_t*>(xr + 8 * s)), d, 0, 0, 0);
      if (h == 0) {
        const int m = r16 % mp;
        if (cg + cc < CP) {
          xs[(cg + cc) * 16 + m] = m < M ? d[0] : 0.f;
          if (m == mp - 1)
            for (int z = mp; z < 16; ++z) xs[(cg + cc) * 16 + z] = 0.f;
        }
      }
    }
  }
  __syncthreads();

  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  const uint32_t sbits = 0x43004300u;  // bf16 exponent of 128 in both halves
  const int mx = min(r16, M - 1);
  const uint16_t* xl_l = xl + mx * XP + 32 * h;
  const float* xs_l = xs + 4 * h;
  const uint16_t* sl_l = reinterpret_cast<const uint16_t*>(wslab) + r16 * 8 * SL;
  f32x4_t acc[RT];

  auto compute = [&](const u32x4_t (&w)[RT], int cw) {
    const int c = c0 + cw;
    const f32x4_t init = *reinterpret_cast<const f32x4_t*>(xs_l + c * 16);
    u32x4_t xb[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) xb[s] = *reinterpret_cast<const u32x4_t*>(xl_l + 128 * c + 8 * s);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      f32x4_t t = init;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(xb[s]), as_bf16x8(unpack_word_paired(w[rt][s], vmask, sbits)), t, 0, 0, 0);
      const float sc = bf16_bits_to_f32(sl_l[rt * 16 * 8 * SL + cw]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[rt][r] = __builtin_fmaf(sc, t[r], acc[rt][r]);
    }
  };

  for (int it = 0; tile < ntiles; ++it, tile += tstep) {
    const int tnext = tile + tstep;  // may be past the end: its loads are out of range
    load_scales(sv, tnext);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < NCW; j += R) {
      const bool last = j + R >= NCW;  // refills of this pass go to the next tile
#pragma unroll
      for (int u = 0; u < R; ++u) {
        compute(ring[u], j + u);
        __builtin_amdgcn_sched_barrier(0);
        issue(ring[u], last ? tnext : tile, last ? u : j + R + u);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float* rd = red + (it & 1) * NW * RT * 4 * kWave;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) rd[((wv * RT + rt) * 4 + r) * kWave + lane] = acc[rt][r];
    store_scales(sv);  // wave-private; its last reader was the compute above
    __syncthreads();
    if (wv == it % NW) {
      const int n0 = tile * ROWS;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = 0.f;
#pragma unroll
          for (int w = 0; w < NW; ++w) v += rd[((w * RT + rt) * 4 + r) * kWave + lane];
          const int m = 4 * h + r, n = n0 + 16 * rt + r16;
          if (m < M && n < N) Y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v);
        }
    }
  }
}

// M = 1 streaming kernel ("diagonal" MFMA). The packed weights are read as one contiguous
// stream: every wave instruction loads 1 KiB = 16 consecutive 64-byte pieces, and with
// G = 128 and K % 128 == 0 a piece is exactly one scale group (128 k) of one row. Lane
// l = 16 kg + j holds 16 bytes (words 4 kg .. 4 kg + 3) of piece j.
//  * MFMA roles: A row j = the X slice matching piece j (from LDS, per lane), B column j =
//    piece j. The diagonal D[j][j] = sum over the piece of x * (128 + q) is the piece's partial
//    dot product; off-diagonal entries are cross terms and are discarded. Per 2048 weights
//    this is the same four MFMAs as the row-tiled kernel, but HBM sees a purely sequential
//    stream.
//  * The accumulator starts at -136 * sum(x over the piece's k range) (per-chunk table xs in
//    LDS, filled while the activation is staged: 16-lane DPP sums, so one barrier covers both),
//    so D[j][j] = sum x * (q - 8) as in the reference dequant.
//  * The piece's scale is S[flat piece index] (S is [N][K / 128], i.e. one bf16 per piece in
//    the same order): 16 consecutive bf16 per block, one 2-byte buffer load per lane.
//  * Workgroups are persistent over GR-row groups; the ceil(GR C / 16) blocks of a group are
//    dealt to the NW waves round-robin. A group's pieces are contiguous in Wq, so its blocks
//    start at any 64-byte piece boundary, and when GR C is not a multiple of 16 the lanes of
//    the last block past the group's end write to the dummy slot (their loads read the next
//    group's pieces, or zeros past the buffer). Each diagonal lane writes scale * D[j][j] to an
//    LDS partial table (double-buffered by group parity); after the group's barrier the rows'
//    C partials are summed either by one wave per row, lane-wise then a wave sum (the "wide"
//    form: 16-wave plans, groups taller than 16 rows and the one-round layout), or by wave
//    (i % NW) for all rows, 16 lanes per row; the form fixes the addition order, so entry
//    points that must give the same bits use the same form.
// Template parameters: NW waves per workgroup; R ring slots; GR rows per group (0: one round,
// fz.rows rows per workgroup); XM the activation source (kXPlain: X; kXNorm / kXNormAdd:
// RMSNorm of the residual, with the add; kXAttn: the merge of the attention splits); YM the
// output (kYPlain, or kYSwiglu: silu(gate) * up of interleaved row pairs); XV 16-byte
// activation vectors per thread staged ahead of the weights; FC each lane's activation
// fragments held in registers for the whole kernel (16 NW a multiple of C); XF the
// activation loads of every wave issued before any weight load (one barrier between them).
//  * Blocks stream through a ring of R register slots (R - 1 blocks in flight per wave),
//    continuing across row groups; the ring's refill cursor (group, slot) advances
//    incrementally in scalar registers.
//  * Branch-free inner loop: the per-chunk offsets are stored four times (one 16-byte LDS read
//    initialises the whole MFMA accumulator), the diagonal value is picked with three selects,
//    and lanes off the diagonal (or on a padded slot) write to a private dummy slot.
template <int NW, int R, int GR, int XM, int YM, int XV, bool FC, bool XF>
__global__ __launch_bounds__(NW * kWave) void w4_gemv_m1_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int N, int K, M1Fuse fz) {
  constexpr uint32_t kOOB = 0x7fffffc0u;
  constexpr int XR = 136;
  extern __shared__ __align__(16) unsigned char smem[];
  const int C = K >> 7, KV = K >> 3;
  const int CP = (C + 15) & ~15;
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                      // [CP][136]
  f32x4_t* xs4 = reinterpret_cast<f32x4_t*>(smem + (size_t)CP * XR * 2); // [CP]
  float* part = reinterpret_cast<float*>(xs4 + CP);                      // [2][GR C] + 64 dummies

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int GRr = GR > 0 ? GR : fz.rows;  // rows per group (GR == 0: chosen at launch)
  const int ngroups = (N + GRr - 1) / GRr;
  const int gstep = gridDim.x;
  const int NP = GRr * C;          // pieces per group
  const int NBG = (NP + 15) >> 4;  // 1 KiB blocks per group (the last one may be partial)
  const int nbp = R * ((NBG + NW * R - 1) / (NW * R));

  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wq), (short)0, (int)((size_t)N * (K >> 1)), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(S), (short)0, (int)((size_t)N * C * 2), 0x00020000);
  const uint32_t vw = 64u * j + 16u * kg;
  const uint32_t vs = 2u * j;

  // refill cursor: (group gr, slot ir) in this wave's stream; slot i is block wv + NW i
  int gr = blockIdx.x, ir = 0;
  auto issue = [&](u32x4_t& w, uint32_t& sc) {
    const int b = wv + NW * ir;
    const bool live = gr < ngroups && b < NBG;
    const uint32_t p0 = (uint32_t)(gr * NP + 16 * b);  // first piece of the block
    w = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                        wres, vw, live ? 64u * p0 : kOOB, kStreamAux));
    sc = __builtin_amdgcn_raw_buffer_load_b16(sres, vs, live ? 2u * p0 : kOOB, kStreamAux);
    if (++ir == nbp) {
      ir = 0;
      gr += gstep;
    }
  };

  // The activation's loads go first: the counter the compiler waits on completes in issue
  // order, so loads issued after the weight ring would wait for the ring's HBM latency too.
  // Buffer loads past the end of a vector return zeros (the K -> 16 CP padding), branch-free.
  constexpr int NT = NW * kWave;
  auto vec_rsrc = [&](const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, K * 2, 0x00020000);
  };
  auto vec_load = [&](__amdgpu_buffer_rsrc_t r, int e) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, 16u * e, 0, 0));
  };
  u32x4_t xa[XV], xb[XV], xw[XV];
  // attention merge: this thread's 8 dims (head v / 16) of kAttnBatch splits per round (fewer
  // with more waves: registers). One-round layouts (GR == 0: one workgroup of 14 or 16 waves per
  // CU) with at least two threads per activation vector split each round's splits over two
  // halves of the threads (thread t < KV and thread t + KV, same dims), which combine through
  // LDS, so a round covers 2 kAttnBatch splits with one load each.
  constexpr int kAttnBatch = NW <= 8 ? 8 : 4;
  const int ahalves = GR == 0 && NT >= 2 * KV ? 2 : 1;  // uniform
  const int kAttnRound = kAttnBatch * ahalves;
  const int ahf = ahalves == 2 && tid >= KV ? 1 : 0;  // which half of each round
  const int av = tid - ahf * KV;                           // activation vector merged
  float2 aml[kAttnBatch];
  f32x4_t ao[kAttnBatch][2];
  int nsplit = 0;
  if constexpr (XM == kXPlain) {
    const auto rx = vec_rsrc(X);
#pragma unroll
    for (int i = 0; i < XV; ++i) xa[i] = vec_load(rx, tid + i * NT);
  } else if constexpr (XM == kXAttn) {
    static_assert(XV == 1, "one activation vector per thread");
    // The position (a scalar load) and this thread's partials of the first kAttnBatch splits
    // are all issued before any is used: the partial loads do not wait for the position (a
    // split past it is masked after its load), so the two round trips overlap. Splits past
    // the workspace read as zeros through the buffer range check.
    const int posv = __builtin_amdgcn_readfirstlane(*fz.pos);
    xa[0] = vec_load(vec_rsrc(X), tid);
    const int hq = av >> 4, d0 = 8 * (av & 15);
    const int smax = (fz.max_len + kAttnDecodeChunk - 1) / kAttnDecodeChunk;
    const auto ores = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(fz.opart), (short)0,
                                                        smax * fz.heads * 128 * 4, 0x00020000);
    const auto mres = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(fz.ml), (short)0,
                                                        smax * fz.heads * 2 * 4, 0x00020000);
    const bool tl = av < KV && tid < ahalves * KV;
#pragma unroll
    for (int sp0 = 0; sp0 < kAttnBatch; ++sp0) {
      const int sp = ahf * kAttnBatch + sp0;
      const uint32_t oo = tl ? 4u * (uint32_t)((sp * fz.heads + hq) * 128 + d0) : kOOB;
      const uint32_t mo = tl ? 4u * (uint32_t)((sp * fz.heads + hq) * 2) : kOOB;
      ao[sp0][0] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ores, oo, 0, 0));
      ao[sp0][1] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ores, oo + 16u, 0, 0));
      const auto m2 = __builtin_amdgcn_raw_buffer_load_b64(mres, mo, 0, 0);
      aml[sp0] = make_float2(__builtin_bit_cast(float, (uint32_t)m2[0]),
                             __builtin_bit_cast(float, (uint32_t)m2[1]));
    }
    const int n = min(posv + 1, fz.max_len);
    nsplit = n > 0 ? (n + kAttnDecodeChunk - 1) / kAttnDecodeChunk : 0;
#pragma unroll
    for (int sp0 = 0; sp0 < kAttnBatch; ++sp0) {
      const int sp = ahf * kAttnBatch + sp0;
      if (!(nsplit > 1 && sp < nsplit && tl)) {  // masked after the load (no branch around it)
        aml[sp0] = make_float2(-INFINITY, 0.f);
        ao[sp0][0] = ao[sp0][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
  } else {
    const auto rr = vec_rsrc(fz.res), rw = vec_rsrc(fz.nw);
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      xa[i] = vec_load(rr, tid + i * NT);
      xw[i] = vec_load(rw, tid + i * NT);
    }
    if constexpr (XM == kXNormAdd) {
      const auto ra = vec_rsrc(fz.radd);
#pragma unroll
      for (int i = 0; i < XV; ++i) xb[i] = vec_load(ra, tid + i * NT);
    }
  }

  u32x4_t ring[R];
  uint32_t rsc[R];
  // (one workgroup per CU) the vector memory pipeline returns loads in issue order, so the
  // activation, issued by every wave before this barrier, does not wait for weight blocks
  if constexpr (XF) __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int u = 0; u < R; ++u) issue(ring[u], rsc[u]);
  __builtin_amdgcn_sched_barrier(0);

  // Staging of activation vector e (8 bf16, natural order; all lanes of the wave call it): the
  // vector goes to xl in pair order, and the 16 lanes holding chunk e / 16 (16 consecutive lanes
  // of one wave, as e = tid + i * NW * 64) add their sums with four row shifts (DPP); the
  // chunk's last lane stores the MFMA accumulator initialiser -136 * sum_k x, four times.
  auto stage = [&](int e, const u32x4_t& v) {
    float f[8];
    unpack8(v, f);
    float sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    // row_shr:1, 2, 4, 8 (inclusive scan; lanes shifted in from outside the row add 0)
    sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x111, 0xf, 0xf, false));
    sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x112, 0xf, 0xf, false));
    sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x114, 0xf, 0xf, false));
    sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x118, 0xf, 0xf, false));
    if (e < 16 * CP) {
      *reinterpret_cast<u32x4_t*>(&xl[(e >> 4) * XR + 8 * (e & 15)]) = pair_order(v);
      if ((e & 15) == 15) {
        const float o = -136.f * sum;
        xs4[e >> 4] = f32x4_t{o, o, o, o};
      }
    }
  };
  if constexpr (XM == kXAttn) {
    // merge the splits as the attention's own merge does: rescale to the running max
    // (base-2 logits), sum, divide once
    u32x4_t xv = xa[0];
    if (nsplit > 1) {
      const int hq = av >> 4, d0 = 8 * (av & 15);
      float m = -INFINITY, l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < nsplit; s0 += kAttnRound) {
        if (s0 > 0) {  // later rounds (contexts beyond one round of splits)
#pragma unroll
          for (int sp = 0; sp < kAttnBatch; ++sp) {
            aml[sp] = make_float2(-INFINITY, 0.f);
            ao[sp][0] = ao[sp][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            const int spl = s0 + ahf * kAttnBatch + sp;
            if (spl < nsplit && av < KV && tid < ahalves * KV) {
              const size_t row = (size_t)spl * fz.heads + hq;
              aml[sp] = *reinterpret_cast<const float2*>(&fz.ml[row * 2]);
              const f32x4_t* src = reinterpret_cast<const f32x4_t*>(&fz.opart[row * 128 + d0]);
              ao[sp][0] = src[0];
              ao[sp][1] = src[1];
            }
          }
        }
#pragma unroll
        for (int sp = 0; sp < kAttnBatch; ++sp) {
          const float mn = fmaxf(m, aml[sp].x);
          if (mn == -INFINITY) continue;  // nothing yet (absent splits)
          const float fo = exp2f(m - mn), fs = exp2f(aml[sp].x - mn);
          l = l * fo + aml[sp].y * fs;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[q] = acc[q] * fo + ao[sp][0][q] * fs;
            acc[4 + q] = acc[4 + q] * fo + ao[sp][1][q] * fs;
          }
          m = mn;
        }
      }
      if (ahalves == 2) {
        // the second half's (max, sum, output) through LDS (after the partial table), combined
        // by the first half as one more split
        float* xch = part + 2 * NP + 64 + 12 * av;
        if (ahf == 1 && av < KV) {
          *reinterpret_cast<f32x4_t*>(xch) = f32x4_t{m, l, 0.f, 0.f};
          *reinterpret_cast<f32x4_t*>(xch + 4) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
          *reinterpret_cast<f32x4_t*>(xch + 8) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
        }
        __syncthreads();
        if (ahf == 0 && av < KV) {
          const f32x4_t ml1 = *reinterpret_cast<const f32x4_t*>(xch);
          const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(xch + 4);
          const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(xch + 8);
          const float mn = fmaxf(m, ml1[0]);  // finite: split 0 is in the first half
          const float fo = exp2f(m - mn), fs = exp2f(ml1[0] - mn);
          l = l * fo + ml1[1] * fs;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[q] = acc[q] * fo + a0[q] * fs;
            acc[4 + q] = acc[4 + q] * fo + a1[q] * fs;
          }
        }
      }
      const float il = 1.f / l;
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] *= il;
      xv = pack8(acc);
    }
    stage(tid, tid < KV ? xv : u32x4_t{0u, 0u, 0u, 0u});
  } else if constexpr (XM != kXPlain) {
    // x = rmsnorm(res + radd) * nw, as the fused RMSNorm kernel: residual rounded to bf16,
    // sum of squares over the row (wave sums, then the workgroup's in LDS), one bf16 rounding
    // of v * inv * w; one workgroup also stores the new residual stream.
    __shared__ float nred[NW];
    u32x4_t* o4 = blockIdx.x == 0 ? reinterpret_cast<u32x4_t*>(fz.res_out) : nullptr;
    float v[XV][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int e = tid + i * NT;
      unpack8(xa[i], v[i]);  // zeros past the row: they add nothing
      if constexpr (XM == kXNormAdd) {
        float b[8];
        unpack8(xb[i], b);
#pragma unroll
        for (int q = 0; q < 8; ++q) v[i][q] = round_bf16(v[i][q] + b[q]);
        if (o4 && e < KV) o4[e] = pack8(v[i]);
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) ss = fmaf(v[i][q], v[i][q], ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) nred[wv] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) tot += nred[i];
    const float inv = rsqrtf(tot / static_cast<float>(K) + fz.eps);
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      float g[8], o[8];
      unpack8(xw[i], g);  // zeros past the row: o is zero there
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = v[i][q] * inv * g[q];
      stage(tid + i * NT, pack8(o));
    }
  } else {
#pragma unroll
    for (int i = 0; i < XV; ++i) stage(tid + i * NT, xa[i]);  // zeros past the row
    // rows longer than XV vectors per thread (K > 8 XV NT): the rest, loaded here (the loop
    // bound is uniform across each wave: NT is a multiple of 64)
    const u32x4_t* x4 = reinterpret_cast<const u32x4_t*>(X);
    for (int e0 = XV * NT; e0 < 16 * CP; e0 += NT) {
      const int e = e0 + tid;
      stage(e, e < KV ? x4[e] : u32x4_t{0u, 0u, 0u, 0u});
    }
  }
  __syncthreads();

  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  const uint32_t sbits = 0x43004300u;
  const bool diag = kg == (j >> 2);
  const int dr = j & 3;
  const bool s1 = dr == 1, s2 = dr == 2, s3 = dr == 3;
  float* dummy = part + 2 * NP + lane;
  const int c_first = (16 * wv + j) % C;
  const int c_step = (16 * NW) % C;
  // FC (the launcher checks that 16 NW is a multiple of C, e.g. gate/up: C = 28, NW = 14):
  // every block a lane sees belongs to the same k-group, so its activation fragments and
  // offset are read from LDS once, not per block (the same values either way).
  f32x4_t t_fix{};
  u32x4_t x_fix[4];
  if constexpr (FC) {
    t_fix = xs4[c_first];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      x_fix[s4] = *reinterpret_cast<const u32x4_t*>(&xl[XR * c_first + 32 * kg + 8 * s4]);
  }
  int g = blockIdx.x;
  for (int it = 0; g < ngroups; ++it, g += gstep) {
    float* pt = part + (it & 1) * NP + j;
    int c = c_first;
    auto block = [&](auto fixed, int u, int b) {
      f32x4_t t;
      u32x4_t xf[4];
      if constexpr (decltype(fixed)::value) {
        t = t_fix;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) xf[s4] = x_fix[s4];
      } else {
        t = xs4[c];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          xf[s4] = *reinterpret_cast<const u32x4_t*>(&xl[XR * c + 32 * kg + 8 * s4]);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(xf[s4]), as_bf16x8(unpack_word_paired(ring[u][s4], vmask, sbits)), t, 0, 0, 0);
      float v = s1 ? t[1] : t[0];
      v = s2 ? t[2] : v;
      v = s3 ? t[3] : v;
      // (groups of a multiple of 16 rows always end on a block boundary)
      const bool in_group = GR > 0 && GR % 16 == 0 ? b < NBG : 16 * b + j < NP;
      float* dst = diag && in_group ? pt + 16 * b : dummy;
      *dst = __uint_as_float(rsc[u] << 16) * v;  // the 16-bit load zero-extends
      if constexpr (!decltype(fixed)::value) {
        c += c_step;
        c = c >= C ? c - C : c;
      }
    };
    auto pass = [&](auto fixed) {
      for (int i0 = 0; i0 < nbp; i0 += R) {
#pragma unroll
        for (int u = 0; u < R; ++u) {
          block(fixed, u, wv + NW * (i0 + u));
          __builtin_amdgcn_sched_barrier(0);
          issue(ring[u], rsc[u]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    pass(std::integral_constant<bool, FC>{});
    __syncthreads();
    // 16-wave workgroups serve the long rows (the planner picks NW = 16 for C >= 64, e.g. down,
    // C = 148), and the one-round layouts (GR == 0) have every wave free at the end: a wave per
    // row, its lanes taking the row's partials c = lane, lane + 64, ... (one lane-wise pass,
    // then a wave sum) instead of one wave walking C / 4 partials per lane for all the rows.
    // The order of additions per row depends only on which form runs, not on the group height,
    // so the attention-merging launcher, which swaps one layout for another, sets fz.wide to
    // keep the plain GEMV's bits.
    constexpr bool kWideCT = YM != kYSwiglu && (NW == 16 || GR > 16 || GR == 0);
    const bool wide = kWideCT || (XM == kXAttn && fz.wide != 0);
    if (wide) {
      for (int rw = wv; rw < GRr; rw += NW) {
        const float* pr = part + (it & 1) * NP + rw * C;
        float v = 0.f;
        for (int cc = lane; cc < C; cc += kWave) v += pr[cc];
        v = wave_sum(v);
        const int n = GRr * g + rw;
        if (lane == 0 && n < N) Y[n] = (uint16_t)f32_to_bf16_rne(v);
      }
    } else if (wv == it % NW) {
      const float* pr = part + (it & 1) * NP;
      float v = 0.f;
      if (j < GRr)
        for (int cc = kg; cc < C; cc += 4) v += pr[j * C + cc];
      v += lane_xor16(v);
      v += lane_xor32(v);
      if constexpr (YM == kYSwiglu) {
        // rows 16g..16g+7 are gate rows 8g.., rows 16g+8.. the matching up rows: the bf16
        // outputs of row j and row j + 8 give activation 8g + j
        static_assert(GR == 16, "SwiGLU output needs 16-row groups");
        const float y = round_bf16(v);
        const float up = lane_xor8(y);
        const int n = 8 * g + j;
        if (kg == 0 && j < 8 && 16 * g + j < N) Y[n] = (uint16_t)f32_to_bf16_rne(silu_mul(y, up));
      } else {
        const int n = GRr * g + j;
        if (kg == 0 && j < GRr && n < N) Y[n] = (uint16_t)f32_to_bf16_rne(v);
      }
    }
  }
}

// Dynamic LDS of w4_gemv_m1_kernel: the staged activation, the offsets, the double-buffered
// partial table with its dummy slots and, for the two-half attention merge, its exchange area.
size_t m1_bytes(int K, int gr, bool attn_halves = false) {
  const int C = K >> 7, CP = (C + 15) & ~15;
  return (size_t)CP * 136 * 2 + (size_t)CP * 16 + (size_t)(2 * gr * C + 64) * 4 +
         (attn_halves ? (size_t)(K >> 3) * 12 * 4 : 0);
}


// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8],
// vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  constexpr int imm = (N & 0xF) | (0x7 << 4) | (0x0 << 8) | (((N >> 4) & 0x3) << 14);
  __builtin_amdgcn_s_waitcnt(imm);
}

// 16 bytes per lane from a buffer into LDS at dst + 16 * lane (a plain device function: the
// builtin inside a lambda of a kernel template keeps the host pass from emitting the stub).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff,
                                           soff, 0, kStreamAux);
}

// LDS-staged GEMV for M = 1..8 and K <= 32 x 128 (whole rows of a 16-row group fit in LDS).
//  * HBM sees contiguous row segments: each 16-row group (16 rows x K/2 bytes) and its scales
//    (16 x K/128 bf16, contiguous in S) are copied straight into LDS by buffer-to-LDS loads
//    (up to 1 KiB of one row per wave instruction), into one of two stages; rows are padded
//    by 16 bytes so a fragment read of 16 rows hits 16 different bank groups.
//  * The MFMAs are row-tiled (v_mfma_f32_16x16x32_bf16, A = activations, B = weights of the
//    16 rows): wave w owns chunks (128 k) w, w + NW, ... of every group and keeps their
//    activation fragments (pair order) in registers for the whole kernel, together with the
//    accumulator initialiser -136 * sum_k x[m][k] per chunk, computed once by an MFMA with a
//    constant -136 operand (it lands directly in the accumulator layout).
//  * Weights as exact bf16 128 + q (paired-nibble unpack), fp32 scale per (row, chunk) after
//    each chunk: the same exact dequant as the other GEMV kernels.
//  * One barrier per group: after it, the next group's loads are issued into the other stage,
//    the group is computed, and each wave leaves its partial sums in a double-buffered LDS
//    area; wave (it % NW) reduces them after the following barrier and writes Y.
template <int MP, int NW, int CW, int ST, int DPW>
__global__ __launch_bounds__(NW * kWave) void w4_gemv_lds_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int M, int N, int K) {
  constexpr uint32_t kOOB = 0x7fffffc0u;
  extern __shared__ __align__(16) unsigned char smem[];
  const int C = K >> 7;
  const int RS = 64 * C + 16;                      // LDS row stride (bytes)
  const int STG = 16 * RS;                         // one stage of weights
  const int IPR = (C + 15) >> 4;                   // DMA instructions per row
  unsigned char* wst = smem;                                          // [ST][16][RS]
  uint16_t* sst = reinterpret_cast<uint16_t*>(smem + ST * STG);           // [ST][16 C]
  f32x4_t* red = reinterpret_cast<f32x4_t*>(sst + ST * 16 * C);           // [2][NW][64]
  unsigned char* dummy = reinterpret_cast<unsigned char*>(red + 2 * NW * 64);  // 1 KiB sink

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int ngroups = (N + 15) >> 4;
  const int gstep = gridDim.x;
  const uint32_t RB = (uint32_t)(K >> 1);          // bytes per weight row

  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wq), (short)0, (int)((size_t)N * RB), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(S), (short)0, scale_span_bytes(N, C), 0x00020000);

  // group g -> stage st: copy q (of 16 IPR + 1) is row q / IPR, bytes [1024 h, ...) with
  // h = q % IPR, or the group's 32 C scale bytes for q = 16 IPR. Wave w issues copies
  // w, w + NW, ... and pads to exactly DPW copies (extra ones read out of range into a sink),
  // so every wave has the same, compile-time number of copies per group in flight.
  auto issue_group = [&](int g, int st) {
    const bool live = g < ngroups;
#pragma unroll
    for (int t = 0; t < DPW; ++t) {
      const int q = wv + NW * t;
      if (q < 16 * IPR) {
        const int r = q / IPR, h = q - r * IPR;
        if (1024 * h + 16 * lane < 64 * C)
          dma16(wres, wst + st * STG + r * RS + 1024 * h,
                (uint32_t)(16 * g + r) * RB + 1024u * h + 16u * lane, live ? 0u : kOOB);
      } else if (q == 16 * IPR) {
        if (16 * lane < 32 * C)
          dma16(sres, sst + st * 16 * C, 32u * (uint32_t)C * (uint32_t)g + 16u * lane, live ? 0u : kOOB);
      } else {
        dma16(wres, dummy, 0u, kOOB);
      }
    }
  };

  int g = blockIdx.x;
#pragma unroll
  for (int p = 0; p < ST - 1; ++p) issue_group(g + p * gstep, p);

  // activation fragments of this wave's chunks: lane (i = l % 16, kg), step s: row m = i
  // (MP = 1: row 0 on every lane), k = 128 c + 32 kg + 8 s .. + 7 (the k of word 4 kg + s of
  // the weight lane (n, kg)), pair order
  u32x4_t xa[CW][4];
  f32x4_t xi[CW];
  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  const int mrow = MP == 1 ? 0 : j;
#pragma unroll
  for (int t = 0; t < CW; ++t) {
    const int c = wv + NW * t;
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (c < C && mrow < M)
        v = pair_order(*reinterpret_cast<const u32x4_t*>(&X[(size_t)mrow * K + 128 * c + 32 * kg + 8 * s4]));
      xa[t][s4] = v;
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(v), as_bf16x8(kNeg136), d, 0, 0, 0);
    }
    xi[t] = d;  // D[m][n] = -136 * sum_k x[m][k]: lane (n, kg) register r holds m = 4 kg + r
  }

  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  const uint32_t sbits = 0x43004300u;
  const uint32_t voffw = (uint32_t)(j * RS + 16 * kg);  // this lane's bytes of a row chunk
  int it = 0, st = 0;
  for (; g < ngroups; ++it, g += gstep, st = st == ST - 1 ? 0 : st + 1) {
    // this wave's copies of group g have landed (those of the ST - 2 later groups may still be
    // in flight; a wave's stores in between only make the wait longer), then everyone's
    wait_vmcnt_lgkm0<DPW * (ST - 2)>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (it > 0 && wv == (it - 1) % NW) {
      // reduce group g - gstep: output (m, n) = lane 16 (m / 4) + n, register m % 4
      const f32x4_t* rb = red + ((it - 1) & 1) * NW * 64;
      f32x4_t v = rb[lane];
      for (int w = 1; w < NW; ++w) {
        const f32x4_t u = rb[w * 64 + lane];
        v[0] += u[0]; v[1] += u[1]; v[2] += u[2]; v[3] += u[3];
      }
      const int n = 16 * (g - gstep) + j;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * kg + r;
        if (m < M && n < N && (MP > 1 || (kg == 0 && r == 0))) Y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v[r]);
      }
    }
    issue_group(g + (ST - 1) * gstep, st == 0 ? ST - 1 : st - 1);
    const unsigned char* ws = wst + st * STG;
    const uint16_t* ss = sst + st * 16 * C;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < CW; ++t) {
      const int c = wv + NW * t;
      if (c < C) {
        const u32x4_t wv4 = *reinterpret_cast<const u32x4_t*>(ws + voffw + 64 * c);
        f32x4_t d = xi[t];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              as_bf16x8(xa[t][s4]), as_bf16x8(unpack_word_paired(wv4[s4], vmask, sbits)), d, 0, 0, 0);
        const float sc = bf16_bits_to_f32(ss[j * C + c]);
        acc[0] += sc * d[0];
        if (MP > 1) {
          acc[1] += sc * d[1];
          acc[2] += sc * d[2];
          acc[3] += sc * d[3];
        }
      }
    }
    red[(it & 1) * NW * 64 + wv * 64 + lane] = acc;
  }
  // last group's reduction
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  if (it > 0 && wv == (it - 1) % NW) {
    const f32x4_t* rb = red + ((it - 1) & 1) * NW * 64;
    f32x4_t v = rb[lane];
    for (int w = 1; w < NW; ++w) {
      const f32x4_t u = rb[w * 64 + lane];
      v[0] += u[0]; v[1] += u[1]; v[2] += u[2]; v[3] += u[3];
    }
    const int n = 16 * (g - gstep) + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * kg + r;
      if (m < M && n < N && (MP > 1 || (kg == 0 && r == 0))) Y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v[r]);
    }
  }
}

size_t lds_bytes(int K, int nw, int st) {
  const int C = K >> 7;
  return (size_t)st * 16 * (64 * C + 16) + (size_t)st * 16 * C * 2 + (size_t)2 * nw * 64 * 16 + 1024;
}

// 4 x 4 transpose over the lane rows (row r = lanes 16 r .. 16 r + 15) and four registers: on
// entry register j of a lane in row r holds element (r, j) of the transposed layout's
// (j, r), i.e. afterwards register s of row r holds what register r of row s held. Two
// stages of gfx950 lane swaps per dword: v_permlane32_swap exchanges the upper half-wave of
// its first operand with the lower half-wave of its second (rows 2, 3 <-> 0, 1),
// v_permlane16_swap the odd rows of its first operand with the even rows of its second.
__device__ __forceinline__ void xpose_rows(u32x4_t (&r)[4]) {
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto v = __builtin_amdgcn_permlane32_swap(r[c][w], r[c + 2][w], false, false);
      r[c][w] = v[0];
      r[c + 2][w] = v[1];
    }
#pragma unroll
  for (int c = 0; c < 4; c += 2)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto v = __builtin_amdgcn_permlane16_swap(r[c][w], r[c + 1][w], false, false);
      r[c][w] = v[0];
      r[c + 1][w] = v[1];
    }
}

// M = 2..8 streaming kernel ("half-pair" MFMA). Generalises the M = 1 kernel's diagonal trick
// from 16 pieces of one row to 8 rows x 2 pieces: a wave instruction loads 8 rows x 128 bytes
// (row-contiguous 128-byte runs), i.e. one 256-k "pair" (two 128-k chunks) of 8 rows.
//  * MFMA roles (v_mfma_f32_16x16x32_bf16): B column j = (row j % 8 of the tile, half j / 8),
//    lane (j, kq) holding words 4 kq .. 4 kq + 3 of that half-pair (step s uses word s);
//    A row i = (activation row i % 8, half i / 8) with the matching activation k's. D[i][j] is
//    a chunk's partial sum when the halves agree; the other half of D is discarded (the MFMA
//    work is cheap next to the HBM stream). Rows m >= M of A are zero.
//  * Each wave owns fixed pairs p = w, w + NW, ... (CW of them) of every row, so its
//    activation fragments (pair order, 64 bytes per lane per pair) stay in registers for the
//    whole kernel; the -136 * sum_k x accumulator initialisers (one MFMA against a constant
//    operand per step) stay in registers too when a wave holds up to three pairs, else in a
//    wave-private LDS table (one 16-byte read per block).
//  * Weights as exact bf16 128 + q (paired-nibble unpack) and one fp32 scale per (row, chunk)
//    after the four MFMAs of a block: the same exact dequant as the other GEMV kernels.
//  * Workgroups are persistent over groups of GT 8-row tiles; a wave's CW x GT blocks of a
//    group stream through an R-slot register ring that continues into the next group. Each
//    wave leaves its per-tile partials (4 rows m x 1 row n per useful lane) in a double-
//    buffered LDS table; after the group's barrier GT waves sum them over waves and halves
//    and store Y.
template <int CW, int GT, int R>
__global__ __launch_bounds__(1024) void w4_gemv_m8_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int M, int N, int K, int ks,
    float* __restrict__ part) {
  constexpr uint32_t kOOB = 0x7fffffc0u;
  constexpr int NB = CW * GT;  // 1 KiB blocks per wave per group
  static_assert(NB % R == 0, "each ring slot serves fixed blocks of a group");
  extern __shared__ __align__(16) unsigned char smem[];
  const int NW = blockDim.x >> 6;
  f32x4_t* xil = reinterpret_cast<f32x4_t*>(smem);  // [NW][CW][64]
  // partials per tile and wave: only the 32 useful lanes' (compact table, for taller groups)
  // or all 64 lanes' (fewer registers: the compiler needs more for the compact stores)
  constexpr bool kCompact = GT > 2;
  constexpr int kSlots = kCompact ? 32 : kWave;
  f32x4_t* red = xil + NW * CW * kWave;              // [2][NW][GT][kSlots]

  const int P = K >> 8, C = K >> 7;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int ntiles = (N + 7) >> 3;
  const int ngroups = (ntiles + GT - 1) / GT;
  // K slices: workgroup b serves slice b % ks (pairs [pa, pb)) of groups b / ks, b / ks + gstep..
  const int slice = (int)blockIdx.x % ks, ph = (P + ks - 1) / ks;
  const int pa = slice * ph, pb = min(P, pa + ph);
  const int gstep = (int)gridDim.x / ks;
  const uint32_t RB = (uint32_t)(K >> 1);  // bytes per weight row

  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wq), (short)0, (int)((size_t)N * RB), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(S), (short)0, (int)((size_t)N * C * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(X), (short)0, (int)((size_t)M * K * 2), 0x00020000);

  // activations first (their wait must not include the weight ring's latency). Lane
  // (i = (m, h), kq) needs, for step s of pair t, the 16-byte piece 4 kq + s of
  // x[m][256 p + 128 h .. + 127]; it loads piece 4 s + kq instead (so the four lanes of a row
  // read 64 contiguous bytes per instruction, not four pieces 64 bytes apart) and a 4 x 4
  // transpose across the lane rows (xpose_rows) puts them in place. Rows m >= M and pairs
  // p >= P read zeros through the range check.
  const int xm = c16 & 7, xh = c16 >> 3;
  const uint32_t vx = ((uint32_t)xm * (uint32_t)K + 128u * xh) * 2u + 16u * kq;
  u32x4_t xa[CW][4];
#pragma unroll
  for (int t = 0; t < CW; ++t) {
    const int p = pa + wv + NW * t;
    const uint32_t so = p < pb ? 512u * (uint32_t)p : kOOB;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      xa[t][s] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xres, vx + 64u * s, so, 0));
  }

  // weight lane (j = (row nl, half hc), kq): row nl of the tile, bytes 64 hc + 16 kq of a pair
  const int nl = c16 & 7, hc = c16 >> 3;
  const uint32_t vw = (uint32_t)nl * RB + 64u * hc + 16u * kq;
  const uint32_t vs = ((uint32_t)nl * (uint32_t)C + hc) * 2u;
  auto issue = [&](u32x4_t& w, uint32_t& sc, int g, int i) {
    const int t = i / GT, u = i % GT;
    const int p = pa + wv + NW * t;
    const bool live = g < ngroups && p < pb;
    const uint32_t row0 = 8u * (uint32_t)(GT * g + u);
    w = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                        wres, vw, live ? row0 * RB + 128u * p : kOOB, kStreamAux));
    sc = __builtin_amdgcn_raw_buffer_load_b16(
        sres, vs, live ? (row0 * (uint32_t)C + 2u * p) * 2u : kOOB, kStreamAux);
  };
  u32x4_t ring[R];
  uint32_t rsc[R];
  int g = (int)blockIdx.x / ks;
  // With up to three pairs per wave, every wave issues its activation loads before any wave of
  // the workgroup issues weight loads (the CU returns loads in issue order, so a later wave's
  // activation would otherwise wait behind the earlier waves' weight blocks): on MI355X at M = 8
  // o 5.61 -> 5.20 us, qkv 7.06 -> 6.90, gate/up 17.60 -> 17.47. With four or five pairs (down,
  // 300 KB of activation per workgroup) the weights wait longer than the activation gains
  // (18.88 -> 19.27 us), so those keep the interleaved order (one interleaved run each).
  if constexpr (CW <= 3) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < R; ++i) issue(ring[i], rsc[i], g, i);
  __builtin_amdgcn_sched_barrier(0);

  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  const uint32_t sbits = 0x43004300u;
  // a useful lane (its half hc equals the half of its accumulator rows, kq / 2) stores its
  // four rows m = 4 (kq % 2) + r of output row nl at slot (8 hc + nl) * 2 + kq % 2
  const bool useful = (kq >> 1) == hc;
  const int slot = (8 * hc + nl) * 2 + (kq & 1);
  // With up to three pairs per wave, the first group (FIRST) transposes each pair's activation
  // fragments into place, converts them to pair order and computes its accumulator initialiser
  // -136 * sum_k x (one MFMA against a constant operand per step) just before the pair's first
  // block, so the first blocks do not wait for the activation loads of later pairs. (With four
  // or five pairs the register budget does not allow it: the compiler then spills, so those
  // convert everything before the first group.)
  constexpr bool kLazy = CW <= 3;
  // with the lazy conversion the initialisers also stay in registers (no LDS read per block)
  f32x4_t xir[kLazy ? CW : 1];
  auto group = [&](auto first, int it) {
    constexpr bool FIRST = decltype(first)::value;
    f32x4_t acc[GT];
#pragma unroll
    for (int u = 0; u < GT; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int t = i / GT, u = i % GT, sl = i % R;
      if constexpr (FIRST) {
        if (u == 0) {
          f32x4_t d0 = {0.f, 0.f, 0.f, 0.f};
          xpose_rows(xa[t]);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            xa[t][s] = pair_order(xa[t][s]);
            d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[t][s]), as_bf16x8(kNeg136), d0, 0, 0, 0);
          }
          if constexpr (kLazy)
            xir[t] = d0;
          else
            xil[(wv * CW + t) * kWave + lane] = d0;  // read back only by this wave
        }
      }
      f32x4_t d;
      if constexpr (kLazy)
        d = xir[t];
      else
        d = xil[(wv * CW + t) * kWave + lane];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(xa[t][s]), as_bf16x8(unpack_word_paired(ring[sl][s], vmask, sbits)), d, 0, 0, 0);
      const float sc = bf16_bits_to_f32(rsc[sl] & 0xffffu);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[u][r] = __builtin_fmaf(sc, d[r], acc[u][r]);
      __builtin_amdgcn_sched_barrier(0);
      // refill: block i + R of this group, or of the next one
      if (i + R < NB)
        issue(ring[sl], rsc[sl], g, i + R);
      else
        issue(ring[sl], rsc[sl], g + gstep, i + R - NB);
      __builtin_amdgcn_sched_barrier(0);
    }
    f32x4_t* rb = red + (size_t)(it & 1) * NW * GT * kSlots;
    if constexpr (kCompact) {
      if (useful) {
#pragma unroll
        for (int u = 0; u < GT; ++u) rb[(wv * GT + u) * kSlots + slot] = acc[u];
      }
    } else {
#pragma unroll
      for (int u = 0; u < GT; ++u) rb[(wv * GT + u) * kSlots + lane] = acc[u];
    }
    __syncthreads();
    // output (m = lane / 8, row nl = lane % 8) of tile u: half h of every wave sits at slot
    // (8 h + nl) * 2 + m / 4 (compact table) or lane (j = nl + 8 h, kq = 2 h + m / 4), register
    // m % 4
    for (int u = (wv - it % NW + NW) % NW; u < GT; u += NW) {  // every tile, also when NW < GT
      const int om = lane >> 3, on = lane & 7;
      const int q0 = kCompact ? 4 * (2 * on + (om >> 2)) + (om & 3)
                              : 4 * (on + 16 * (om >> 2)) + (om & 3);
      const int q1 = kCompact ? q0 + 4 * 16 : q0 + 4 * (8 + 32);
      float v = 0.f;
      for (int w = 0; w < NW; ++w) {
        const float* pw = reinterpret_cast<const float*>(rb + (w * GT + u) * kSlots);
        v += pw[q0] + pw[q1];
      }
      const int n = 8 * (GT * g + u) + on;
      if (om < M && n < N) {
        if (ks == 1)
          Y[(size_t)om * N + n] = (uint16_t)f32_to_bf16_rne(v);
        else
          part[((size_t)slice * M + om) * N + n] = v;
      }
    }
  };
  int it = 0;
  if constexpr (kLazy) {
    if (g < ngroups) {
      group(std::true_type{}, 0);
      it = 1;
      g += gstep;
    }
  } else {
#pragma unroll
    for (int t = 0; t < CW; ++t) {
      f32x4_t d0 = {0.f, 0.f, 0.f, 0.f};
      xpose_rows(xa[t]);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        xa[t][s] = pair_order(xa[t][s]);
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[t][s]), as_bf16x8(kNeg136), d0, 0, 0, 0);
      }
      xil[(wv * CW + t) * kWave + lane] = d0;
    }
  }
  for (; g < ngroups; ++it, g += gstep) group(std::false_type{}, it);
}

// Sums the ks K-slice partials ([ks][M][N] fp32) of the M = 2..8 kernel in slice order and
// rounds to bf16: a separate launch, so the slices' partials are visible without device-scope
// fences inside the streaming kernel (on gfx950 such a fence writes back and invalidates the
// XCD's L2; one per group made the down projection ten times slower).
__global__ __launch_bounds__(256) void w4_gemv_m8_merge_kernel(const float* __restrict__ part,
                                                               uint16_t* __restrict__ Y, int MN,
                                                               int ks) {
  const int i = (int)(blockIdx.x * 256 + threadIdx.x);
  if (i >= MN) return;
  float v = 0.f;
  for (int s = 0; s < ks; ++s) v += part[(size_t)s * MN + i];
  Y[i] = (uint16_t)f32_to_bf16_rne(v);
}

size_t m8_bytes(int nw, int cw, int gt) {
  return (size_t)nw * cw * kWave * 16 + (size_t)2 * nw * gt * (gt > 2 ? 32 : kWave) * 16;
}

// M = 2..8 with long rows (more than 32 pairs): the half-pair MFMA of w4_gemv_m8_kernel with the
// activation streamed through LDS instead of held in registers, in one launch and without a
// workspace.
//  * 16 waves per workgroup, persistent over groups of two 8-row tiles (16 rows). K runs in
//    chunks of 16 pairs (4096 k); wave w takes pair w of every chunk, for both tiles: two 1 KiB
//    blocks per chunk, sharing one set of activation fragments and one -136 * sum_k x
//    initialiser (four MFMAs against a constant operand).
//  * Each chunk's activation (8 rows x 16 pairs x 512 B = 64 KiB; rows m >= M and pairs past
//    K read as zeros) is loaded by the whole workgroup, four 16-byte pieces per thread, one
//    chunk ahead, and stored in pair order into one of two LDS buffers. Within a pair, the
//    16-byte unit of (piece e' = 4 kq + s of a half, row-half mh = 2 m + h) sits at
//    16 e' + ((mh + e') mod 16): the 16 lanes of a fragment read (fixed e', every mh) and
//    the 16 lanes of a staging store (fixed mh, every e') each cover all 64 banks once.
//  * The weight blocks stream through a four-slot register ring two chunks ahead (it
//    continues into the next group). One barrier per chunk publishes the next chunk's buffer;
//    each wave's per-tile partials go to a compact LDS table at a group's last chunk, and two
//    waves sum them over waves and halves after that chunk's barrier. A group's activation is
//    read once per workgroup from L2 (each workgroup serves about one group on the 7B down
//    projection), against once per wave and pair in registers before any weight block in
//    the register kernel.
__global__ __launch_bounds__(1024) void w4_gemv_m8c_kernel(
    const uint16_t* __restrict__ X, const uint32_t* __restrict__ Wq,
    const uint16_t* __restrict__ S, uint16_t* __restrict__ Y, int M, int N, int K) {
  constexpr uint32_t kOOB = 0x7fffffc0u;
  constexpr int NW = 16, PC = 16, GT = 2, R = 4;
  extern __shared__ __align__(16) unsigned char smem[];
  u32x4_t* xl = reinterpret_cast<u32x4_t*>(smem);                           // [2][PC][256]
  f32x4_t* red = reinterpret_cast<f32x4_t*>(smem + (size_t)2 * PC * 4096);  // [NW][GT][32]

  const int P = K >> 8, C = K >> 7;
  const int nch = (P + PC - 1) / PC;  // >= 3 (the planner sends K > 8192 only)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int ntiles = (N + 7) >> 3;
  const int ngroups = (ntiles + GT - 1) / GT;
  const int gstep = (int)gridDim.x;
  const uint32_t RB = (uint32_t)(K >> 1);

  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(Wq), (short)0, (int)((size_t)N * RB), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(S), (short)0, (int)((size_t)N * C * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(X), (short)0, (int)((size_t)M * K * 2), 0x00020000);

  // staging: piece q = tid + 1024 i of a chunk is 16-byte piece e = q % 32 of row m = (q / 32)
  // % 8 of pair pl = q / 256 (= wv / 4 + 4 i: uniform across the wave)
  const int se = tid & 31, sm = (tid >> 5) & 7;
  const uint32_t sxo = sm < M ? ((uint32_t)sm * (uint32_t)K + 8u * se) * 2u : kOOB;
  const int sunit = 16 * (se & 15) + (((2 * sm + (se >> 4)) + (se & 15)) & 15);
  u32x4_t xv[4];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = PC * c + (wv >> 2) + 4 * i;
      xv[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              xres, sxo, p < P ? 512u * (uint32_t)p : kOOB, 0));
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xl[(buf * PC + (wv >> 2) + 4 * i) * 256 + sunit] = pair_order(xv[i]);
  };

  // weight lane (j = (row nl, half hc), kq): row nl of the tile, bytes 64 hc + 16 kq of a pair
  const int nl = c16 & 7, hc = c16 >> 3;
  const uint32_t vw = (uint32_t)nl * RB + 64u * hc + 16u * kq;
  const uint32_t vs = ((uint32_t)nl * (uint32_t)C + hc) * 2u;
  // block (group g, chunk c, tile u): pair p = 16 c + wv of rows 8 (2 g + u) ..
  auto issue = [&](u32x4_t& w, uint32_t& sc, int g, int c, int u) {
    const int p = PC * c + wv;
    const bool live = g < ngroups && p < P;
    const uint32_t row0 = 8u * (uint32_t)(GT * g + u);
    w = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                        wres, vw, live ? row0 * RB + 128u * p : kOOB, kStreamAux));
    sc = __builtin_amdgcn_raw_buffer_load_b16(
        sres, vs, live ? (row0 * (uint32_t)C + 2u * p) * 2u : kOOB, kStreamAux);
  };

  // fragment reads: lane (i = (m, h), kq), step s: unit 16 e' + ((mh + e') mod 16), e' = 4 kq + s
  const int mh = 2 * (c16 & 7) + (c16 >> 3);
  const u32x4_t kNeg136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  uint32_t vmask;
  asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(vmask));
  const uint32_t sbits = 0x43004300u;
  const bool useful = (kq >> 1) == hc;
  const int slot = (8 * hc + nl) * 2 + (kq & 1);

  int g = (int)blockIdx.x;
  // the first chunk's activation ahead of the weight ring (loads complete in issue order)
  load_chunk(0);
  u32x4_t ring[R];
  uint32_t rsc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) issue(ring[i], rsc[i], g, i >> 1, i & 1);
  __builtin_amdgcn_sched_barrier(0);
  store_chunk(0);
  lds_sync();

  f32x4_t acc[GT];
  // chunk c of group g in LDS buffer PAR (ring slots 2 PAR, 2 PAR + 1)
  auto chunk = [&](auto par, int c) {
    constexpr int PAR = decltype(par)::value;
    const bool last = c + 1 == nch;
    // next chunk's activation (the next group's first chunk after a group's last)
    const bool more = !last || g + gstep < ngroups;
    if (more) load_chunk(last ? 0 : c + 1);
    u32x4_t xa[4];
    f32x4_t d0 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int e = 4 * kq + s;
      xa[s] = xl[(PAR * PC + wv) * 256 + 16 * e + ((mh + e) & 15)];
      d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[s]), as_bf16x8(kNeg136), d0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < GT; ++u) {
      constexpr int kSlot0 = 2 * PAR;
      f32x4_t d = d0;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(xa[s]), as_bf16x8(unpack_word_paired(ring[kSlot0 + u][s], vmask, sbits)), d, 0, 0, 0);
      const float sc = bf16_bits_to_f32(rsc[kSlot0 + u] & 0xffffu);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[u][r] = __builtin_fmaf(sc, d[r], acc[u][r]);
      __builtin_amdgcn_sched_barrier(0);
      // refill with the block two chunks ahead (into the next group past the last chunk)
      if (c + 2 < nch)
        issue(ring[kSlot0 + u], rsc[kSlot0 + u], g, c + 2, u);
      else
        issue(ring[kSlot0 + u], rsc[kSlot0 + u], g + gstep, c + 2 - nch, u);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (last && useful) {
#pragma unroll
      for (int u = 0; u < GT; ++u) red[(wv * GT + u) * 32 + slot] = acc[u];
    }
    if (more) store_chunk(1 - PAR);
    lds_sync();
  };

  int cc = 0;  // chunks done by this workgroup: its parity picks the buffer and ring slots
  for (; g < ngroups; g += gstep) {
#pragma unroll
    for (int u = 0; u < GT; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nch; ++c, ++cc) {
      if (cc & 1)
        chunk(std::integral_constant<int, 1>{}, c);
      else
        chunk(std::integral_constant<int, 0>{}, c);
    }
    // output (m = lane / 8, row nl = lane % 8) of tile u: half h of every wave sits at slot
    // (8 h + nl) * 2 + m / 4, register m % 4. The table is rewritten only at this
    // workgroup's next group's last chunk, nch >= 3 barriers later.
    if (wv < GT) {
      const int u = wv, om = lane >> 3, on = lane & 7;
      const int q0 = 4 * (2 * on + (om >> 2)) + (om & 3), q1 = q0 + 4 * 16;
      float v = 0.f;
      for (int w = 0; w < NW; ++w) {
        const float* pw = reinterpret_cast<const float*>(red + (w * GT + u) * 32);
        v += pw[q0] + pw[q1];
      }
      const int n = 8 * (GT * g + u) + on;
      if (om < M && n < N) Y[(size_t)om * N + n] = (uint16_t)f32_to_bf16_rne(v);
    }
  }
}

constexpr size_t kM8cBytes = (size_t)2 * 16 * 4096 + (size_t)16 * 2 * 32 * 16;

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

size_t xlds_bytes(int M, int K, int G, int rt, int nw, int r, int sl) {
  (void)G;
  const XldsGeom geo = xlds_geom(K, nw, r);
  const size_t a = ((size_t)M * (128 * geo.cp + 8) * 2 + 15) & ~(size_t)15;
  return a + (size_t)geo.cp * 16 * 4 + (size_t)nw * rt * 16 * 4 * sl * 4 +
         (size_t)2 * nw * rt * 4 * kWave * 4;
}

// Smallest scale-slab size (in 16-byte loads per lane) covering a wave's chunks; 0 if none.
int xlds_sl(int K, int G, int rt, int nw, int r) {
  if (G != 128 || rt > 4 || (K / G) % 2) return 0;  // dword-aligned scale loads need even K/G
  const XldsGeom geo = xlds_geom(K, nw, r);
  const int ncw = geo.ncw;
  return ncw <= 8 ? 1 : ncw <= 16 ? 2 : ncw <= 32 ? 4 : 0;
}

template <int RT, int NW, int R, int SL>
hipError_t launch_xlds(const GemvArgs& a, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&w4_gemv_xlds_kernel<RT, NW, R, SL>);
  // Opt in (once per instantiation and device) to LDS beyond 64 KiB (gfx950 has 160 KiB per CU).
  const hipError_t attr = cached_max_dynamic_lds(fn, 160 * 1024);
  if (attr != hipSuccess) return attr;
  const size_t lds = xlds_bytes(a.M, a.K, a.G, RT, NW, R, SL);
  int per_cu = 0;
  hipError_t e = cached_occupancy(fn, NW * kWave, lds, &per_cu);
  if (e != hipSuccess) return e;
  int cus = 0;
  e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int ntiles = (a.N + 16 * RT - 1) / (16 * RT);
  const int grid = max(1, min(ntiles, max(per_cu, 1) * cus));
  hipLaunchKernelGGL((w4_gemv_xlds_kernel<RT, NW, R, SL>), dim3(grid), dim3(NW * kWave), lds, st,
                     a.X, a.Wq, a.S, a.Y, a.M, a.N, a.K, a.G);
  return hipSuccess;
}

template <int NW, int R, int GR, int XM, int YM, int XV, bool FC, bool XF>
hipError_t launch_m1_fc(const GemvArgs& a, hipStream_t st, const M1Fuse& fz, int wpc) {
  const void* fn = reinterpret_cast<const void*>(&w4_gemv_m1_kernel<NW, R, GR, XM, YM, XV, FC, XF>);
  // the dynamic part stays under this limit: 96 KiB at 16-row groups (the M = 1 filter), at most
  // 127 KiB for one round of up to 32 long rows per CU; the rest of the CU's 160 KiB holds the
  // static LDS
  const hipError_t attr = cached_max_dynamic_lds(fn, 128 * 1024);
  if (attr != hipSuccess) return attr;
  const int rows = GR > 0 ? GR : fz.rows;
  if (rows <= 0) return hipErrorInvalidValue;
  const size_t lds = m1_bytes(a.K, rows, XM == kXAttn && GR == 0);
  int per_cu = 0;
  hipError_t e = cached_occupancy(fn, NW * kWave, lds, &per_cu);
  if (e != hipSuccess) return e;
  int cus = 0;
  e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  // wpc workgroups per CU (two unless the plan says otherwise): more resident waves only
  // lengthen the memory queues.
  const int ngroups = (a.N + rows - 1) / rows;
  const int grid = max(1, min(ngroups, min(max(per_cu, 1), wpc) * cus));
  hipLaunchKernelGGL((w4_gemv_m1_kernel<NW, R, GR, XM, YM, XV, FC, XF>), dim3(grid), dim3(NW * kWave), lds,
                     st, a.X, a.Wq, a.S, a.Y, a.N, a.K, fz);
  return hipSuccess;
}

// FC when 16 NW is a multiple of K / 128; the activation-first barrier (XF) when the layout asks
// for it, compiled only for the layouts that take it: one workgroup per CU, and the fused SwiGLU
// GEMV's two fourteen-wave workgroups per CU.
template <int NW, int R, int GR, int XM = kXPlain, int YM = kYPlain, int XV = kXVecs>
hipError_t launch_m1(const GemvArgs& a, hipStream_t st, const M1Fuse& fz = M1Fuse{}, int wpc = 2) {
  const bool fc = (16 * NW) % (a.K >> 7) == 0;
  if constexpr (GR == 0 || (NW == 16 && GR == 16) || (NW == 14 && GR == 16 && YM == kYSwiglu)) {
    if (fz.xfirst) {
      if (fc) return launch_m1_fc<NW, R, GR, XM, YM, XV, true, true>(a, st, fz, wpc);
      return launch_m1_fc<NW, R, GR, XM, YM, XV, false, true>(a, st, fz, wpc);
    }
  }
  if (fc) return launch_m1_fc<NW, R, GR, XM, YM, XV, true, false>(a, st, fz, wpc);
  return launch_m1_fc<NW, R, GR, XM, YM, XV, false, false>(a, st, fz, wpc);
}

// Workgroups per CU the M = 2..8 kernel can hold (occupancy), or a negative error.
template <int CW, int GT, int R>
int m8_per_cu(int nw, hipError_t* err) {
  const void* fn = reinterpret_cast<const void*>(&w4_gemv_m8_kernel<CW, GT, R>);
  const hipError_t attr = cached_max_dynamic_lds(fn, 160 * 1024);
  *err = attr;
  if (attr != hipSuccess) return 0;
  const size_t lds = m8_bytes(nw, CW, GT);
  if (lds > 160 * 1024 || nw < 1 || nw > 16) {
    *err = hipErrorInvalidValue;
    return 0;
  }
  int per_cu = 0;
  *err = cached_occupancy(fn, nw * kWave, lds, &per_cu);
  return max(per_cu, 1);
}

// K slices of the M = 2..8 kernel: ks workgroups share each group, each writing its fp32
// partials to the caller's workspace ([ks][M][N]); a merge launch sums them into Y.
struct M8Split {
  int ks = 1;
  float* part = nullptr;
};

template <int CW, int GT, int R>
hipError_t launch_m8(const GemvArgs& a, int nw, int cap, const M8Split& sp, hipStream_t st) {
  hipError_t e;
  const int per_cu = m8_per_cu<CW, GT, R>(nw, &e);
  if (e != hipSuccess) return e;
  const size_t lds = m8_bytes(nw, CW, GT);
  int cus = 0;
  e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int ngroups = ((a.N + 7) / 8 + GT - 1) / GT;
  // workgroups per slice: every slice serves every group, so the grid is a multiple of ks
  const int per_slice = max(1, min(ngroups, min(max(per_cu, 1), cap) * cus / sp.ks));
  hipLaunchKernelGGL((w4_gemv_m8_kernel<CW, GT, R>), dim3(per_slice * sp.ks), dim3(nw * kWave), lds,
                     st, a.X, a.Wq, a.S, a.Y, a.M, a.N, a.K, sp.ks, sp.part);
  if (sp.ks > 1) {
    const int mn = a.M * a.N;
    hipLaunchKernelGGL(w4_gemv_m8_merge_kernel, dim3((mn + 255) / 256), dim3(256), 0, st, sp.part,
                       a.Y, mn, sp.ks);
  }
  return hipSuccess;
}

// The chunked-activation M = 2..8 kernel: one workgroup per CU at most, each over 16-row
// groups.
hipError_t launch_m8c(const GemvArgs& a, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&w4_gemv_m8c_kernel);
  hipError_t e = cached_max_dynamic_lds(fn, (int)kM8cBytes);
  if (e != hipSuccess) return e;
  int cus = 0;
  e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int ngroups = ((a.N + 7) / 8 + 1) / 2;
  hipLaunchKernelGGL(w4_gemv_m8c_kernel, dim3(max(1, min(ngroups, cus))), dim3(1024), kM8cBytes, st,
                     a.X, a.Wq, a.S, a.Y, a.M, a.N, a.K);
  return hipSuccess;
}

// Tile-group height and workgroups per CU for the M = 2..8 kernel with one or two pairs per
// wave, from a per-CU byte count: every workgroup reads the whole activation (M K bf16, from
// L2) once and its groups' weights, and the busiest CU sets the time. Among the plans within 2 %
// of the cheapest, the one that keeps the most CUs busy wins (more of the chip streams weights),
// then the taller group (fewer group barriers), then fewer workgroups per CU. On MI355X at
// M = 8 this picks 16-row groups at one workgroup per CU for qkv (4608 x 3584: 256 workgroups
// against 144 with 32-row groups, 6.89 -> 6.63 us) and o (3584 x 3584), and 32-row groups for
// gate/up (37888 x 3584, one workgroup per CU), each the fastest of the candidates measured.
template <int CW>
hipError_t launch_m8_auto(const GemvArgs& a, int nw, const M8Split& sp, hipStream_t st) {
  int cus = 0;
  hipError_t e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int pc2 = m8_per_cu<CW, 2, 2>(nw, &e);
  if (e != hipSuccess) return e;
  const int pc4 = m8_per_cu<CW, 4, 4>(nw, &e);
  if (e != hipSuccess) return e;
  const double xb = 2.0 * a.M * a.K / sp.ks, rowb = 0.5 * a.K / sp.ks;
  const int ntiles = (a.N + 7) / 8;
  // Two refinements of the byte count, measured on MI355X (M = 8 / M = 4, us): with one pair
  // per wave and twelve or more waves, 32-row groups whenever they fill every CU (fewer group
  // barriers: 28672 x 4096 17.8 / 17.2 -> 16.6 / 16.0; the 7B gate/up already took them); with
  // six waves or fewer, two workgroups per CU at least (17920 x 1536 8.3 / 8.0 -> 6.5 / 6.1).
  if (CW == 1 && sp.ks == 1 && nw >= 12 && (ntiles + 3) / 4 >= cus && pc4 >= 1)
    return launch_m8<CW, 4, 4>(a, nw, 1, sp, st);
  const int min_cap = sp.ks == 1 && nw <= 6 ? 2 : 1;
  struct Cand {
    int gt, cap, wgs;
    double cost;
  } cand[4];
  int nc = 0;
  double best = 0;
  for (int gt = 4; gt >= 2; gt -= 2) {
    for (int cap = min(min_cap, gt == 4 ? pc4 : pc2); cap <= min(2, gt == 4 ? pc4 : pc2); ++cap) {
      const int groups = (ntiles + gt - 1) / gt;
      const int wgs = max(1, min(groups, cap * cus / sp.ks));
      const int gpw = (groups + wgs - 1) / wgs, wpc = (sp.ks * wgs + cus - 1) / cus;
      const double cost = wpc * (xb + gpw * gt * 8 * rowb);
      cand[nc++] = Cand{gt, cap, wgs, cost};
      if (best == 0 || cost < best) best = cost;
    }
  }
  int bgt = 2, bcap = 1, bwgs = 0;
  for (int i = 0; i < nc; ++i)  // candidates come tallest first, then fewer per CU
    if (cand[i].cost <= 1.02 * best && cand[i].wgs > bwgs) {
      bgt = cand[i].gt;
      bcap = cand[i].cap;
      bwgs = cand[i].wgs;
    }
  if (bgt == 4) return launch_m8<CW, 4, 4>(a, nw, bcap, sp, st);
  return launch_m8<CW, 2, 2>(a, nw, bcap, sp, st);
}

template <int MP, int NW, int CW, int ST, int DPW>
hipError_t launch_lds(const GemvArgs& a, hipStream_t st, int grid_cap) {
  const void* fn = reinterpret_cast<const void*>(&w4_gemv_lds_kernel<MP, NW, CW, ST, DPW>);
  const hipError_t attr = cached_max_dynamic_lds(fn, 160 * 1024);
  if (attr != hipSuccess) return attr;
  const size_t lds = lds_bytes(a.K, NW, ST);
  int cus = 0;
  hipError_t e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int ngroups = (a.N + 15) / 16;
  const int grid = max(1, min(ngroups, grid_cap * cus));
  hipLaunchKernelGGL((w4_gemv_lds_kernel<MP, NW, CW, ST, DPW>), dim3(grid), dim3(NW * kWave), lds, st, a.X,
                     a.Wq, a.S, a.Y, a.M, a.N, a.K);
  return hipSuccess;
}

// Launch layout of the M = 1 kernel. The plain and the fused entry points take the same layout
// for a shape, so they sum its partials in the same order and give the same bits.
struct M1Layout {
  int nw = 8;           // waves per workgroup
  int gr = 16;          // rows per group as a template argument (0: `rows`, chosen here)
  int rows = 0;
  int wpc = 2;          // workgroups per CU
  bool xfirst = false;  // activation loads ahead of the workgroup's weight loads
};

// Layouts by shape (C = K / 128 k-groups, so a 16-row group is C blocks of 1 KiB). A wave count
// NW "fits" C when C % NW == 0 (every wave streams the same number of a group's blocks) and
// 16 NW % C == 0 (FC: each lane meets one k-group, its activation fragments stay in registers).
// All layouts sum a row's partials in one of two fixed orders, and a shape's plain and fused
// entry points take the same layout, so they give the same bits. Measured on MI355X (256 CUs,
// interleaved A/B runs, us; 7B shapes first, then other model shapes the planner was checked on):
// * Long rows (C >= 64, e.g. down): one workgroup per CU, activation first. Sixteen waves over
//   16-row groups when those fill between half and all of the CUs once (the 7B down, 224
//   groups: 8.83, against 9.57 with 14 rows on every CU) or make two or more full rounds
//   (8192 x 8192, 512 groups: 8.36 against 9.44 in one round of 32 rows); otherwise one round
//   of ceil(N / CUs) rows per CU: sixteen waves when the groups would fill half the CUs or fewer
//   (1536 x 8960 6.06 -> 4.56 with 6 rows per CU, 2048 x 11008 6.22 -> 5.48), fourteen when
//   they make one to two rounds (5120 x 13824, 320 groups: 12.34 -> 9.28; sixteen waves 9.66)
//   or when fourteen gives FC (C = 112: 4096 x 14336 8.26 -> 8.06; C = 224: 8192 x 28672 22.6
//   either way).
// * Many groups (gate/up: at least 1024 16-row groups, C >= 14): 16-row groups, four seven-wave
//   workgroups per CU where seven waves fit C (the 7B gate/up, C = 28: 13.7 against 15.6 with
//   eight waves), two eight-wave ones where C % 8 == 0 (22016 x 2048 8.00 -> 6.83 and 28672 x
//   4096 13.55 -> 12.11 against one round per CU), else fourteen waves, two per CU.
// * Tiny layers (at most 10 blocks per CU in one round): 16-row groups of eight waves, two per
//   CU (2048 x 1536 4.17 -> 3.49, 2048 x 2048 4.19 -> 3.46 against one round per CU).
// * Layers of at most 32 blocks per CU in one round (qkv, o), or 80 with fewer than 512 16-row
//   groups: one workgroup per CU with ceil(N / CUs) rows, activation first; fourteen waves past
//   32 blocks or where 14 fits C up to 28 blocks, else sixteen (qkv 5.71 -> 4.68, o 4.68 -> 4.41
//   against 16-row groups at eight waves, two per CU; 5120 x 5120 6.92 -> 5.54 and 6144 x 4096
//   5.92 -> 5.47 likewise; with 1120 groups, 17920 x 1536, 16-row groups stay ahead: 5.99
//   against 6.52 in one round). One round as two workgroups per CU of half the rows each (eight
//   or seven waves, with or without the activation first) is slower: qkv 4.69 against
//   4.98-5.75, o 4.43 against 4.69-4.85; so are three-slot rings (qkv 5.32-5.39, o 4.88-5.30).
// * Otherwise eight waves per 16-row group (8-row groups when 16-row ones would give each CU
//   only one or two), two workgroups per CU.
hipError_t m1_layout(int N, int K, M1Layout* L) {
  int cus = 0;
  const hipError_t e = cached_cu_count(&cus);
  if (e != hipSuccess) return e;
  const int C = K >> 7, groups16 = (N + 15) / 16;
  const int rows1 = (N + cus - 1) / cus, blocks1 = (rows1 * C + 15) / 16;
  M1Layout l;
  if (C >= 64) {
    const bool fc14 = (16 * 14) % C == 0;
    l.nw = 16;
    l.wpc = 1;
    l.xfirst = true;
    if (groups16 <= 2 * cus && (fc14 || 2 * groups16 <= cus || (groups16 > cus && groups16 < 2 * cus))) {
      l.gr = 0;  // one round of ceil(N / CUs) rows per CU
      l.rows = rows1;
      if (fc14 || groups16 > cus) l.nw = 14;
    }
  } else if (groups16 >= 1024 && C >= 14) {
    l.nw = C % 7 == 0 && 112 % C == 0 ? 7 : C % 8 == 0 ? 8 : 14;
    l.wpc = l.nw == 7 ? 4 : 2;
  } else if (blocks1 <= 10) {
    l.nw = 8;
  } else if (blocks1 <= 32 || (blocks1 <= 80 && groups16 < 512)) {
    l.nw = blocks1 > 32 || (blocks1 <= 28 && 224 % C == 0) ? 14 : 16;
    l.gr = 0;
    l.rows = rows1;
    l.wpc = 1;
    l.xfirst = true;
  } else {
    l.gr = groups16 > 256 && groups16 < 512 && C % 2 == 0 ? 8 : 16;
  }
  *L = l;
  return hipSuccess;
}

}  // namespace

// Pairs per wave (cw) and waves (nw) of the M = 2..8 kernel for one of ks K slices: up to 16
// waves, each holding the fewest pairs that cover the slice (K < 256: one pair, no waves).
void m8_shape(int K, int ks, int* cw, int* nw) {
  const int ph = (K / 256 + ks - 1) / ks;
  *cw = max(1, (ph + 15) / 16);
  *nw = (ph + *cw - 1) / *cw;
}

// Register-X kernel limits: scale staging must fit comfortably in LDS next to the reduction.
bool gemv_fast_path_ok(int M, int N, int K, int G) {
  (void)N;
  return M >= 1 && M <= 8 && K % 128 == 0 && G % 128 == 0 && (K / G + 1) * 32 * 2 <= 32768;
}

GemvPlan gemv_plan(int M, int N, int K, int G) {
  GemvPlan p{};
  p.fast = gemv_fast_path_ok(M, N, K, G);
  if (!p.fast) return p;
  const int C = K / 128;
  // LDS-activation kernel when X fits and the weight bytes fit a 31-bit buffer offset.
  const bool small_buf = (size_t)N * (K / 2) + (size_t)16 * K < ((size_t)1 << 31);
  p.m1 = M == 1 && G == 128 && small_buf && m1_bytes(K, 16) <= 96 * 1024;
  if (p.m1) return p;  // waves, group height and grid come from m1_layout at launch
  // M = 2..8, K a multiple of 256 up to 20480: the half-pair streaming kernel, each wave
  // holding up to five pairs of activation fragments in registers.
  int cw = 0;
  m8_shape(K, 1, &cw, &p.nw);
  p.m8 = M >= 2 && G == 128 && K >= 256 && K % 256 == 0 && cw <= 5 && small_buf &&
         (size_t)M * K * 2 < ((size_t)1 << 31);
  if (p.m8) {
    p.rt = cw;
    // Past 32 pairs (three to five per wave, leaving registers for a two-block ring only, and a
    // workgroup per CU reading the whole activation for its one or two groups) K runs in the
    // fewest slices of at most two pairs per wave, each workgroup streaming ks times the rows
    // against 1 / ks of the activation, plus a merge launch. On MI355X at M = 8 (interleaved
    // A/B, us): 1536 x 8960 9.1 unsplit -> 7.9 in two slices (8.3 in three); 2048 x 11008
    // 11.4 -> 8.7 (9.9); 4096 x 14336 14.4 in two, 16.4 in three; 3584 x 18944 18.87 -> 16.81 in
    // three (17.70 in two); at 32 pairs and fewer every split was slower (3584 x 8192 9.2 ->
    // 9.5 / 10.3, 7168 x 5120 8.4 -> 10.3). M = 2 and 4 follow (2048 x 11008 at M = 2:
    // 8.6 -> 7.7).
    const int P = K / 256;
    p.ks = P > 32 ? (P + 31) / 32 : 1;
    return p;
  }
  // M = 2..8 with whole rows of a 16-row group in LDS (K <= 4096): weights staged in LDS.
  p.lds = M >= 2 && G == 128 && C <= 32 && small_buf;
  if (p.lds) {
    // waves and chunks per wave covering C (sixteen waves of two chunks past 28 chunks: three
    // chunks per wave spilled registers)
    p.nw = C <= 16 ? 8 : C <= 28 ? 14 : 16;
    p.rt = 2;
    return p;
  }
  p.rt = 1;
  p.nw = N >= 16384 ? 4 : 8;
  while (p.nw > 1 && C / p.nw < 2) p.nw /= 2;
  p.sl = xlds_sl(K, G, p.rt, p.nw, 4);
  p.xlds = small_buf && p.sl > 0 && xlds_bytes(M, K, G, p.rt, p.nw, 4, p.sl) <= 96 * 1024;
  if (!p.xlds) {
    const int tiles1 = (N + 15) / 16;
    p.rt = tiles1 >= 2048 ? 2 : 1;
    const int tiles = (N + 16 * p.rt - 1) / (16 * p.rt);
    int nw = 1;
    while (nw < 8 && (long)tiles * nw < 2048 && C / (2 * nw) >= 2) nw *= 2;
    p.nw = nw;
  }
  return p;
}

size_t gemv_split_bytes(int M, int N, int K, int G) {
  if (M < 2 || M > 8 || N <= 0 || K <= 0 || G <= 0 || K % 32 || G % 32 || K % G) return 0;
  const GemvPlan p = gemv_plan(M, N, K, G);
  return p.fast && p.m8 && p.ks > 1 ? (size_t)p.ks * M * N * sizeof(float) : 0;
}

hipError_t launch_gemv(const GemvArgs& a, const GemvPlan& p, hipStream_t st, float* ws,
                       size_t ws_bytes) {
  if (!p.fast) {
    hipLaunchKernelGGL((w4_gemv_generic_kernel<8>), dim3((a.N + 3) / 4), dim3(256), 0, st, a.X,
                       a.Wq, a.S, a.Y, a.M, a.N, a.K, a.G);
    return hipSuccess;
  }
  if (p.m1) {
    M1Layout L;
    const hipError_t e = m1_layout(a.N, a.K, &L);
    if (e != hipSuccess) return e;
    M1Fuse fz;
    fz.rows = L.rows;
    fz.xfirst = L.xfirst;
    if (L.gr == 0) {
      if (L.nw == 14) return launch_m1<14, 2, 0>(a, st, fz, L.wpc);
      return launch_m1<16, 2, 0>(a, st, fz, L.wpc);
    }
    if (L.nw == 16) return launch_m1<16, 2, 16>(a, st, fz, L.wpc);
    // seven-wave workgroups, four per CU, for gate/up: each lane keeps its activation
    // fragments in registers, and a group barrier waits for seven waves, not fourteen (gate/up
    // 14.7 -> 14.2 us on MI355X against fourteen-wave workgroups, two per CU; same outputs)
    if (L.nw == 7) return launch_m1<7, 2, 16>(a, st, fz, L.wpc);
    if (L.nw == 14) return launch_m1<14, 2, 16>(a, st, fz, L.wpc);
    // Eight-wave plans run with seven waves when seven fits K / 128 (C % 7 == 0 and 16 x 7 a
    // multiple of C): each lane then meets one k-group only and keeps its activation fragments
    // in registers (same outputs). Without C % 7 == 0 the seven waves stream unequal shares
    // (C = 16: 22016 x 2048 9.70 against 6.91 us with eight waves on MI355X). The fused decode
    // entries keep eight waves (their activation staging needs one vector per thread).
    const int C = a.K >> 7;
    const bool fc7 = C % 7 == 0 && 112 % C == 0;
    if (L.gr == 16) return fc7 ? launch_m1<7, 2, 16>(a, st, fz, L.wpc) : launch_m1<8, 2, 16>(a, st, fz, L.wpc);
    return fc7 ? launch_m1<7, 2, 8>(a, st, fz, L.wpc) : launch_m1<8, 2, 8>(a, st, fz, L.wpc);
  }
  if (p.m8) {
    // Long rows at M >= 6 with about one 16-row group per CU (the 7B down projection at
    // M = 8: 224 groups): the chunked-activation kernel, one launch, no workspace. On MI355X
    // (interleaved A/B, us, M = 8 / M = 4): 3584 x 18944 15.9 / 15.3 against 16.6 / 15.4 in K
    // slices and 18.6 / 15.8 unsplit; 4096 x 14336 13.5 / 12.9 against 14.6 / 13.2 and 15.2 /
    // 12.5. With two or more groups per workgroup (8192 x 11008: 18.6 against 16.9 unsplit)
    // or fewer groups than three quarters of the CUs (2048 x 11008: 10.2 against 8.7 split)
    // and at M = 2 (15.0 against 14.2 unsplit) it is slower, so those keep the other plans.
    if (p.ks > 1 && a.M >= 6) {
      int cus = 0;
      const hipError_t e = cached_cu_count(&cus);
      if (e != hipSuccess) return e;
      const int groups = ((a.N + 7) / 8 + 1) / 2;
      if (4 * groups >= 3 * cus && groups <= cus) return launch_m8c(a, st);
    }
    // the K split runs only in the caller's workspace (ns_w4_linear_ws); ns_w4_linear passes
    // none and runs every shape unsplit
    M8Split sp;
    if (p.ks > 1 && ws && (size_t)p.ks * a.M * a.N * sizeof(float) <= ws_bytes) {
      sp.ks = p.ks;
      sp.part = ws;
    }
    int cw = 0, nw = 0;
    m8_shape(a.K, sp.ks, &cw, &nw);
    switch (cw) {
      case 1: return launch_m8_auto<1>(a, nw, sp, st);
      case 2: return launch_m8_auto<2>(a, nw, sp, st);
      case 3: return launch_m8<3, 2, 2>(a, nw, 2, sp, st);
      case 4: return launch_m8<4, 2, 2>(a, nw, 2, sp, st);
      case 5: return launch_m8<5, 2, 2>(a, nw, 2, sp, st);
      default: return hipErrorInvalidValue;
    }
  }
  if ((p.lds || p.xlds) && ((size_t)a.N * (a.K >> 7)) % 2 != 0 &&
      (reinterpret_cast<uintptr_t>(a.S) & 3) != 0) {
    // the 16-byte scale loads of those kernels would need the two bytes after a scale array
    // that is not 4-byte aligned (scale_span_bytes): the kernel with 2-byte scale loads
    hipLaunchKernelGGL((w4_gemv_generic_kernel<8>), dim3((a.N + 3) / 4), dim3(256), 0, st, a.X,
                       a.Wq, a.S, a.Y, a.M, a.N, a.K, a.G);
    return hipSuccess;
  }
  if (p.lds) {
    // copies per wave per group: 16 rows x ceil(C / 16) row pieces + the scale slab
    if (p.nw == 8) return launch_lds<8, 8, 2, 3, 3>(a, st, 1);
    if (p.nw == 14) return launch_lds<8, 14, 2, 3, 3>(a, st, 1);
    if (p.nw == 16) return launch_lds<8, 16, 2, 3, 3>(a, st, 1);
    return hipErrorInvalidValue;
  }
  if (p.xlds) {
#define NS_XLDS_CASE(NW_, SL_) \
  if (p.rt == 1 && p.nw == NW_ && p.sl == SL_) return launch_xlds<1, NW_, 4, SL_>(a, st);
    NS_XLDS_CASE(1, 1) NS_XLDS_CASE(1, 2) NS_XLDS_CASE(1, 4)
    NS_XLDS_CASE(2, 1) NS_XLDS_CASE(2, 2) NS_XLDS_CASE(2, 4)
    NS_XLDS_CASE(4, 1) NS_XLDS_CASE(4, 2) NS_XLDS_CASE(4, 4)
    NS_XLDS_CASE(8, 1) NS_XLDS_CASE(8, 2) NS_XLDS_CASE(8, 4)
#undef NS_XLDS_CASE
    return hipErrorInvalidValue;
  }
#define NS_GEMV_CASE(RT_, NW_)                                   \
  if (p.rt == RT_ && p.nw == NW_) return launch_mfma<RT_, NW_, 2>(a, st);
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


namespace {

// The norm prologue keeps its vectors live across the row reduction, so it is compiled for
// as few vectors per thread as the row needs (registers decide how many workgroups fit a CU).
template <int NW, int GR, int YM, int XV>
hipError_t launch_m1_norm(const GemvArgs& a, const M1Fuse& fz, hipStream_t st, int wpc) {
  if (fz.radd) return launch_m1<NW, 2, GR, kXNormAdd, YM, XV>(a, st, fz, wpc);
  return launch_m1<NW, 2, GR, kXNorm, YM, XV>(a, st, fz, wpc);
}

template <int NW, int GR, int YM>
hipError_t launch_m1_x(const GemvArgs& a, const M1Fuse& fz, bool norm, hipStream_t st, int wpc) {
  if (!norm) return launch_m1<NW, 2, GR, kXPlain, YM>(a, st, fz, wpc);
  const int C = a.K >> 7, nvec = 16 * ((C + 15) & ~15);
  if (nvec <= NW * kWave) return launch_m1_norm<NW, GR, YM, 1>(a, fz, st, wpc);
  if (nvec <= 2 * NW * kWave) return launch_m1_norm<NW, GR, YM, 2>(a, fz, st, wpc);
  return launch_m1_norm<NW, GR, YM, 4>(a, fz, st, wpc);
}

template <int NW, int GR>
hipError_t launch_m1_fused(const GemvArgs& a, const M1Fuse& fz, bool norm, bool swiglu,
                           hipStream_t st, int wpc) {
  if (swiglu) return launch_m1_x<NW, GR, kYSwiglu>(a, fz, norm, st, wpc);
  return launch_m1_x<NW, GR, kYPlain>(a, fz, norm, st, wpc);
}

}  // namespace

hipError_t launch_gemv_attn(const GemvArgs& a, const GemvPlan& p, const M1Fuse& fz0,
                            hipStream_t st, int* reject) {
  *reject = 0;
  const int C = a.K >> 7, CP = (C + 15) & ~15;
  if (!p.m1) {
    *reject = 1;
    return hipSuccess;
  }
  M1Layout L;
  const hipError_t e = m1_layout(a.N, a.K, &L);
  if (e != hipSuccess) return e;
  // the plain plan's seven-wave workgroups: fourteen here (one activation vector per thread)
  const int nw = L.nw == 7 ? 14 : L.nw;
  if (L.nw == 7) L.wpc = 2;
  M1Fuse fz = fz0;
  fz.rows = L.rows;
  // no activation-first barrier here: each workgroup reads every split's partials (115 KB at
  // 28 heads and 8 splits), and the weight stream should not queue behind them
  fz.xfirst = 0;
  if (16 * CP > nw * kWave) {
    // The merge needs one activation vector per thread. Where the plain layout's workgroups have
    // fewer threads (50 to 63 heads: one round on fourteen waves, or eight-wave groups), the
    // merging GEMV runs sixteen-wave workgroups of 16-row groups, two per CU, up to 64 heads; it
    // reduces rows in the wide form, so it agrees with the plain GEMV to rounding, not in bits.
    if (16 * CP > 16 * kWave) {
      *reject = 1;
      return hipSuccess;
    }
    return launch_m1<16, 2, 16, kXAttn, kYPlain, 1>(a, st, fz, 2);
  }
  if (L.gr == 0) {
    // Where the plain layout is one round with up to 16 rows per CU (the o projection), the
    // attention-merging GEMV runs eight-wave workgroups of 16-row groups, two per CU: every
    // workgroup merges all the splits' partials (115 KB at 28 heads and 8 splits), and this
    // layout's weight stream overlaps that better (decode step 1.385 -> 1.364 ms per token on
    // MI355X against the one-round layout with eight waves of four blocks, one interleaved
    // run). Both sum each row's partials in the same order: the same bits as the plain GEMV.
    if (L.rows <= 16 && 16 * CP <= 8 * kWave) {
      fz.wide = 1;  // the one-round layout's reduction form
      return launch_m1<8, 2, 16, kXAttn, kYPlain, 1>(a, st, fz, 2);
    }
    if (nw == 14) return launch_m1<14, 2, 0, kXAttn, kYPlain, 1>(a, st, fz, L.wpc);
    return launch_m1<16, 2, 0, kXAttn, kYPlain, 1>(a, st, fz, L.wpc);
  }
  if (nw == 16 && L.gr == 16) return launch_m1<16, 2, 16, kXAttn, kYPlain, 1>(a, st, fz, L.wpc);
  if (nw == 14 && L.gr == 16) return launch_m1<14, 2, 16, kXAttn, kYPlain, 1>(a, st, fz, L.wpc);
  if (nw == 8 && L.gr == 16) return launch_m1<8, 2, 16, kXAttn, kYPlain, 1>(a, st, fz, L.wpc);
  if (nw == 8 && L.gr == 8) return launch_m1<8, 2, 8, kXAttn, kYPlain, 1>(a, st, fz, L.wpc);
  *reject = 1;
  return hipSuccess;
}

hipError_t launch_gemv_fused(const GemvArgs& a, const GemvPlan& p, const M1Fuse& fz0, bool norm,
                             bool swiglu, hipStream_t st, int* reject) {
  *reject = 0;
  const int C = a.K >> 7, CP = (C + 15) & ~15;
  if (!p.m1 || (swiglu && a.N % 16)) {
    *reject = 1;
    return hipSuccess;
  }
  M1Layout L;
  const hipError_t e = m1_layout(a.N, a.K, &L);
  if (e != hipSuccess) return e;
  // the SwiGLU pairing needs 16-row groups; the plain plan's seven-wave workgroups run with
  // fourteen waves, two per CU (the decode step measured 1.511 against 1.458 ms per token
  // with seven-wave fused GEMVs)
  if (swiglu && L.gr != 16) L = M1Layout{L.nw == 16 ? 16 : 8, 16, 0, 2, false};
  const int nw = L.nw == 7 ? 14 : L.nw;
  if (L.nw == 7) L.wpc = 2;
  if (norm && 16 * CP > kXVecs * nw * kWave) {
    *reject = 1;
    return hipSuccess;
  }
  M1Fuse fz = fz0;
  fz.rows = L.rows;
  // The fourteen-wave SwiGLU GEMV issues every wave's activation (and norm) loads before any
  // weight load: decode step 1.370 -> 1.349 ms per token on MI355X (one interleaved run, same
  // logits); the plain gate/up plan does not gain from it (seven waves, four per CU: 14.47 ->
  // 14.87 us; fourteen waves with it: 14.08 -> 14.51 us).
  fz.xfirst = L.xfirst || (swiglu && nw == 14);
  if (L.gr == 0) {
    if (nw == 14) return launch_m1_x<14, 0, kYPlain>(a, fz, norm, st, L.wpc);
    return launch_m1_x<16, 0, kYPlain>(a, fz, norm, st, L.wpc);
  }
  if (nw == 16 && L.gr == 16) return launch_m1_fused<16, 16>(a, fz, norm, swiglu, st, L.wpc);
  if (nw == 14 && L.gr == 16) return launch_m1_fused<14, 16>(a, fz, norm, swiglu, st, L.wpc);
  if (nw == 8 && L.gr == 16) return launch_m1_fused<8, 16>(a, fz, norm, swiglu, st, L.wpc);
  if (nw == 8 && L.gr == 8 && !swiglu) return launch_m1_x<8, 8, kYPlain>(a, fz, norm, st, L.wpc);
  *reject = 1;
  return hipSuccess;
}

}  // namespace ns
