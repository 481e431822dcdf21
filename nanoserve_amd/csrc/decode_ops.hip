// Operators around the W4 linear layers in one decoder step, for gfx950 (wave64):
//   * residual-add + RMSNorm, RoPE and SwiGLU with the reference's C entry points and
//     semantics (csrc/nanoserve_ops.cu:20-44, kernels/fused/{rmsnorm,rope,swiglu}.cuh);
//   * the one-token attention step of the reference's runner (python/nanoserve/qwen.py:
//     119-133, 147-151), which the reference does with PyTorch ops: bias + RoPE + KV-cache
//     append in one kernel, and grouped-query attention over the cache split across
//     workgroups (partial softmax per split, then a combine kernel).
// Contracts are in include/nanoserve_decode.h. All of these are memory- or latency-bound:
// 16-byte accesses where rows allow it, fp32 arithmetic, bf16 round-to-nearest-even stores.
#include <math.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "../../include/nanoserve_decode.h"
#include "w4_common.h"

namespace ns {
namespace {

constexpr int kBlock = 256;

// The prompt-pass operators behind the reference's ns_rmsnorm / ns_rope / ns_swiglu entry
// points, organised for wave64 with buffer loads: the buffer's range check returns zeros past
// the end of a row or vector and drops stores there, so no lane needs a tail branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bytes_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ void st16(__amdgpu_buffer_rsrc_t r, uint32_t off, const u32x4_t& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((__vector_size__(4 * sizeof(int)))) int, v), r, off, 0, 0);
}

// ------------------------------------------------------------------ residual add + RMSNorm
// One wave per row, four rows per workgroup. Lane l holds vectors l, l + 64, ... (VPL of them,
// 8 bf16 each) of its row for the whole kernel; the sum of squares is a DPP wave sum, so there
// is no LDS and no barrier. With r, the bf16 residual stream x + r is written back first.
constexpr int kRowsPerBlock = 4;
template <int VPL>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
    rms_rows_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ r,
                    const uint16_t* __restrict__ w, uint16_t* __restrict__ y, int T, int H,
                    float eps) {
  const int row = blockIdx.x * kRowsPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= T) return;  // the whole wave
  const uint32_t lane = threadIdx.x & 63, rb = 2u * (uint32_t)H;
  const size_t base = (size_t)row * H;
  const auto xr = bytes_rsrc(x + base, rb), wr = bytes_rsrc(w, rb), yr = bytes_rsrc(y + base, rb);
  u32x4_t xv[VPL], gv[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    xv[v] = ld16(xr, 16u * (lane + 64u * v));
    gv[v] = ld16(wr, 16u * (lane + 64u * v));
  }
  float f[VPL][8];
  float ss = 0.f;
  if (r) {
    const auto rr = bytes_rsrc(r + base, rb);
    u32x4_t rv[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) rv[v] = ld16(rr, 16u * (lane + 64u * v));
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      float a[8];
      unpack8(xv[v], f[v]);
      unpack8(rv[v], a);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[v][e] = round_bf16(f[v][e] + a[e]);
      st16(xr, 16u * (lane + 64u * v), pack8(f[v]));
    }
  } else {
#pragma unroll
    for (int v = 0; v < VPL; ++v) unpack8(xv[v], f[v]);
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(f[v][e], f[v][e], ss);
  const float inv = rsqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    float g[8];
    unpack8(gv[v], g);
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = f[v][e] * inv * g[e];
    st16(yr, 16u * (lane + 64u * v), pack8(g));
  }
}

// ------------------------------------------------------------------ RoPE
// One wave per (token, block of kHeadsPerWave heads): lane p owns rotation pairs p, p + 64, ...
// of every head of the block (elements p and p + D/2), so each pair's angle is computed once
// per wave and serves all the block's heads; a wave instruction moves 64 consecutive bf16 of a
// head half. All the block's loads are issued before the rotations.
constexpr int kHeadsPerWave = 8;
template <int PPL>
__global__ void __launch_bounds__(256)
    rope_heads_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                      const float* __restrict__ inv_freq, int T, int Hq, int Hk, int D, int pos0,
                      long long qs, long long ks) {
  const int H = Hq + Hk, nblk = (H + kHeadsPerWave - 1) / kHeadsPerWave;
  const long long wid = (long long)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wid >= (long long)T * nblk) return;  // the whole wave
  const long long t = wid / nblk;
  const int h0 = (int)(wid % nblk) * kHeadsPerWave;
  const int lane = threadIdx.x & 63, half = D >> 1;
  const float pos = static_cast<float>(pos0 + t);
  float cs[PPL], sn[PPL];
#pragma unroll
  for (int s = 0; s < PPL; ++s) {
    const int p = lane + 64 * s;
    cs[s] = 1.f;
    sn[s] = 0.f;
    if (p < half) sincosf(pos * inv_freq[p], &sn[s], &cs[s]);
  }
  uint16_t* hp[kHeadsPerWave];
  uint32_t lo[kHeadsPerWave][PPL], hi[kHeadsPerWave][PPL];
#pragma unroll
  for (int i = 0; i < kHeadsPerWave; ++i) {
    const int h = min(h0 + i, H - 1);  // heads past H repeat the last one and are not stored
    hp[i] = h < Hq ? q + t * qs + (long long)h * D : k + t * ks + (long long)(h - Hq) * D;
#pragma unroll
    for (int s = 0; s < PPL; ++s) {
      const int p = min(lane + 64 * s, half - 1);
      lo[i][s] = hp[i][p];
      hi[i][s] = hp[i][p + half];
    }
  }
#pragma unroll
  for (int i = 0; i < kHeadsPerWave; ++i) {
    if (h0 + i >= H) break;  // uniform over the wave
#pragma unroll
    for (int s = 0; s < PPL; ++s) {
      const int p = lane + 64 * s;
      if (p >= half) continue;
      const float a = bf16_bits_to_f32(lo[i][s]), b = bf16_bits_to_f32(hi[i][s]);
      hp[i][p] = (uint16_t)f32_to_bf16_rne(a * cs[s] - b * sn[s]);
      hp[i][p + half] = (uint16_t)f32_to_bf16_rne(b * cs[s] + a * sn[s]);
    }
  }
}

// ------------------------------------------------------------------ SwiGLU
// Workgroup b covers the 16-byte vectors [kSwigluSpan b, kSwigluSpan (b + 1)) of the flattened
// tensors, two per thread, through buffers clamped to the tensor's end (no tail branch, no
// grid-stride loop: the grid covers the tensor exactly).
constexpr int kSwigluVecs = 2;
constexpr int kSwigluSpan = 256 * kSwigluVecs;
__global__ void __launch_bounds__(256)
    swiglu_vec_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                      uint16_t* __restrict__ out, size_t n8) {
  const size_t v0 = (size_t)blockIdx.x * kSwigluSpan;
  const uint32_t bytes = (uint32_t)(16 * min((size_t)kSwigluSpan, n8 - v0));
  const auto gr = bytes_rsrc(gate + 8 * v0, bytes), ur = bytes_rsrc(up + 8 * v0, bytes),
             orr = bytes_rsrc(out + 8 * v0, bytes);
  u32x4_t g[kSwigluVecs], u[kSwigluVecs];
#pragma unroll
  for (int j = 0; j < kSwigluVecs; ++j) {
    const uint32_t off = 16u * (threadIdx.x + 256u * j);
    g[j] = ld16(gr, off);
    u[j] = ld16(ur, off);
  }
#pragma unroll
  for (int j = 0; j < kSwigluVecs; ++j) {
    float a[8], b[8];
    unpack8(g[j], a);
    unpack8(u[j], b);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = silu_mul(a[e], b[e]);
    st16(orr, 16u * (threadIdx.x + 256u * j), pack8(a));
  }
}

// ------------------------------------------------------------------ decode: bias + RoPE + cache
// Items 0 .. (Hq + Hk) * D/16 - 1 rotate one chunk pair of a q or k head; the rest copy one
// 16-byte chunk of a v head. Every element gets the bias first (bf16 add, as the reference's
// `q += bq`); k and v rows also go to the cache at row *pos.
__global__ void __launch_bounds__(kBlock)
    decode_qkv_kernel(uint16_t* __restrict__ qkv, const uint16_t* __restrict__ bias,
                      const float* __restrict__ inv_freq, const int* __restrict__ pos_p,
                      uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int Hq, int Hk, int D,
                      int max_len) {
  const int pos = *pos_p;
  const bool store = pos >= 0 && pos < max_len;
  const int half_chunks = D >> 4;
  const int rope_items = (Hq + Hk) * half_chunks;
  const int total = rope_items + Hk * (D >> 3);
  for (int idx = blockIdx.x * kBlock + threadIdx.x; idx < total; idx += gridDim.x * kBlock) {
    if (idx < rope_items) {
      const int c = idx % half_chunks, h = idx / half_chunks;
      const int off_lo = h * D + 8 * c, off_hi = off_lo + D / 2;
      u32x4_t* lo_p = reinterpret_cast<u32x4_t*>(qkv + off_lo);
      u32x4_t* hi_p = reinterpret_cast<u32x4_t*>(qkv + off_hi);
      float lo[8], hi[8];
      unpack8(*lo_p, lo);
      unpack8(*hi_p, hi);
      if (bias) {
        float blo[8], bhi[8];
        unpack8(*reinterpret_cast<const u32x4_t*>(bias + off_lo), blo);
        unpack8(*reinterpret_cast<const u32x4_t*>(bias + off_hi), bhi);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          lo[e] = round_bf16(lo[e] + blo[e]);
          hi[e] = round_bf16(hi[e] + bhi[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {  // pair (8c + e, 8c + e + D/2) at this position's angle
        float sn, cs;
        sincosf(static_cast<float>(pos) * inv_freq[8 * c + e], &sn, &cs);
        const float a = lo[e], b = hi[e];
        lo[e] = a * cs - b * sn;
        hi[e] = b * cs + a * sn;
      }
      const u32x4_t plo = pack8(lo), phi = pack8(hi);
      *lo_p = plo;
      *hi_p = phi;
      if (h >= Hq && store) {
        uint16_t* row = kc + ((size_t)(h - Hq) * max_len + pos) * D;
        *reinterpret_cast<u32x4_t*>(row + 8 * c) = plo;
        *reinterpret_cast<u32x4_t*>(row + D / 2 + 8 * c) = phi;
      }
    } else {
      const int j = idx - rope_items;
      const int vchunks = D >> 3;
      const int h = j / vchunks, c = j % vchunks;
      const int off = (Hq + Hk + h) * D + 8 * c;
      u32x4_t* p = reinterpret_cast<u32x4_t*>(qkv + off);
      u32x4_t v = *p;
      if (bias) {
        float a[8], b[8];
        unpack8(v, a);
        unpack8(*reinterpret_cast<const u32x4_t*>(bias + off), b);
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = a[e] + b[e];
        v = pack8(a);
        *p = v;
      }
      if (store)
        *reinterpret_cast<u32x4_t*>(vc + ((size_t)h * max_len + pos) * D + 8 * c) = v;
    }
  }
}

// ------------------------------------------------------------------ decode attention
// Workgroup (s, g, z) covers cache rows [s*kChunk, (s+1)*kChunk) of kv head g for all R = Hq/Hk
// query heads of the group. It computes the split's max m (base-2 logits), sum l of
// 2^(logit - m) and unnormalised output sum_p 2^(logit_p - m) v_p in fp32. A single split
// normalises and writes the output itself; otherwise the splits' partials go to the workspace
// and a second kernel (decode_attn_merge_kernel) merges them; the kernel boundary orders the
// partial stores before the merge's loads (an in-kernel merge by the last workgroup needs
// device-scope fences, measured slower than the second launch).
//
// kFused: q is the fused projection output qkv [(Hq + 2Hk) * D]; every workgroup applies the
// bias and RoPE to its group's q heads itself, and the workgroup whose split holds row *pos
// also builds that row's k (bias + RoPE) and v (bias), appends both to the cache and takes
// them from LDS (ns_decode_qkv followed by ns_decode_attention, in one launch).
//
// A kernel this small costs its memory round trips and its longest chain of dependent
// instructions, so: every global load (k and v rows, q, bias) is issued at the start; the
// scores of a wave's 16 rows x 16 query-head slots come from four v_mfma_f32_16x16x32_bf16
// (A = k rows, lane l: row l%16, dims 32s + 8(l/16)..+7; B = q heads, lane l: head l%16, same
// dims; D: lane l holds rows 4(l/16)+r of head l%16), so each lane owns one head and the
// per-head max and sum need two lane swaps instead of a 64-lane reduction per head; the values
// are a VALU loop, probabilities broadcast from LDS. Each split is served by two workgroups
// (blockIdx.z), each producing half of the value dimensions: both compute the same scores and
// softmax (the k rows are read twice, a small cost next to the value loop), lane l of a wave
// owns dimension 64 z + l of each of the wave's rows (a 2-byte load per row), so each
// workgroup's value loop and output reduction are half as long; workgroup z = 0 alone appends
// the token's row to the cache and writes the split's (max, sum).
constexpr int kAttnWaves = kAttnDecodeChunk / 16;  // waves per attention workgroup, 16 rows each
constexpr int kAttnBlock = kAttnWaves * kWave;
constexpr int kChunk = kAttnDecodeChunk;   // cache rows per split
static_assert(kChunk == 16 * kAttnWaves, "one 16-row score tile per wave");
constexpr int kHeadDim = 128;
constexpr int kMaxGroup = 8;  // query heads per kv head (score columns 0..7 of 16 used)

template <bool kFused>
__global__ void __launch_bounds__(kAttnBlock)
    decode_attn_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ bias,
                       const float* __restrict__ inv_freq, const float* __restrict__ rot_tab,
                       uint16_t* __restrict__ kc,
                       uint16_t* __restrict__ vc, const int* __restrict__ pos_p,
                       uint16_t* __restrict__ out, float* __restrict__ opart,
                       float* __restrict__ ml, int Hq, int Hk, int max_len, float qscale) {
  constexpr int D = kHeadDim;
  constexpr int RP = kMaxGroup;
  constexpr int NWV = kAttnWaves;
  constexpr int QS = D + 8;  // padded q row (bf16 elements)
  __shared__ __attribute__((aligned(16))) uint16_t qb[16][QS];
  __shared__ float red_m[NWV][16];
  __shared__ float red_l[NWV][16];
  __shared__ float ored[NWV][RP][D / 2];
  __shared__ float rot[2][D / 2];
  __shared__ __attribute__((aligned(16))) uint16_t knew[D];
  __shared__ __attribute__((aligned(16))) uint16_t vnew[D];

  const int split = blockIdx.x, g = blockIdx.y;
  const int dh = blockIdx.z;  // which half of the value dimensions this workgroup produces
  const int R = Hq / Hk;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int start = split * kChunk;

  // ---- every load is issued first, branch-free, in the order the work needs them: the
  // position (a scalar load), q / bias and (fused) the token's own k / v heads, then the cache
  // rows of this split, k (MFMA A fragments) and v (two dims per row). Buffer range checks
  // return zeros for rows past the cache and for lanes with nothing to load, so no load sits
  // behind a branch (a branch join would make the compiler wait for every load before it).
  constexpr uint32_t kOOB = 0x7fffffc0u;
  const int pos = __builtin_amdgcn_readfirstlane(*pos_p);
  const int r16 = lane & 15, grp = lane >> 4;
  const int krow = 16 * w + r16;  // this lane's k row within the chunk
  // fused: thread t < 8R: q head t/8, rotation chunk pair t%8; then 8 threads for the k
  // head's chunk pairs and 16 for the v head's chunks
  const int nq = 8 * R;
  const bool is_q = kFused && tid < nq;
  const bool ld_k = kFused && tid >= nq && tid < nq + 8;
  const bool ld_v = kFused && tid >= nq + 8 && tid < nq + 24;
  const int c = is_q ? tid % 8 : tid - nq;
  const int qrows = kFused ? Hq + 2 * Hk : Hq;
  const auto qres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(q), (short)0,
                                                      qrows * D * 2, 0x00020000);
  const auto bres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(bias), (short)0,
                                                      bias ? qrows * D * 2 : 0, 0x00020000);
  auto ld16 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  };
  // (fused) the rotation angles: with a table (rot_tab [2][D/2] = cos, sin of this position,
  // written once per decode step by ns_decode_embed), the cosines and sines of the 8 pairs a
  // q / k thread rotates are loaded with everything else; without one, threads 0 .. D/2 - 1
  // load their frequency and compute the angles once the position is known.
  const bool tab = kFused && rot_tab != nullptr;  // uniform
  float frq = 0.f;
  u32x4_t tc0{}, tc1{}, ts0{}, ts1{};
  if constexpr (kFused) {
    const auto fres = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(inv_freq), (short)0,
                                                        tab ? 0 : D / 2 * 4, 0x00020000);
    frq = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                        fres, tid < D / 2 ? 4u * tid : kOOB, 0, 0));
    const auto tres = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rot_tab), (short)0,
                                                        tab ? D * 4 : 0, 0x00020000);
    const int tci = tid < nq ? tid % 8 : tid - nq;  // pair chunk of a q or k thread
    const uint32_t to = tid < nq + 8 ? 32u * (uint32_t)tci : kOOB;
    tc0 = ld16(tres, to);
    tc1 = ld16(tres, to == kOOB ? kOOB : to + 16u);
    ts0 = ld16(tres, to == kOOB ? kOOB : to + 4u * (D / 2));
    ts1 = ld16(tres, to == kOOB ? kOOB : to + 4u * (D / 2) + 16u);
  }
  u32x4_t a0, a1, b0, b1;
  if constexpr (kFused) {
    // element offsets of the two halves this thread rotates (q / k) or its v chunk
    const int off = is_q ? (g * R + tid / 8) * D + 8 * c
                  : ld_k ? (Hq + g) * D + 8 * c : (Hq + Hk + g) * D + 8 * (tid - nq - 8);
    const bool any = is_q || ld_k || ld_v;
    const uint32_t o0 = any ? 2u * off : kOOB, o1 = (is_q || ld_k) ? 2u * (off + D / 2) : kOOB;
    a0 = ld16(qres, o0);
    a1 = ld16(qres, o1);
    b0 = ld16(bres, o0);
    b1 = ld16(bres, o1);
  } else {  // 16 dims per thread of head tid / 8: two 16-byte loads
    const int h = tid / 8, cc = tid % 8;
    const uint32_t o0 = tid < 8 * 16 && h < R ? 2u * ((g * R + h) * D + 16 * cc) : kOOB;
    a0 = ld16(qres, o0);
    a1 = ld16(qres, o0 == kOOB ? kOOB : o0 + 16u);
    b0 = b1 = u32x4_t{};
  }
  // Every wave's q / bias / angle loads are issued before any wave issues its cache rows: the
  // CU's vector memory path returns data in issue order, so otherwise the q of the later waves
  // waits behind the earlier waves' cache rows (and q is needed first).
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t head_bytes = (uint32_t)max_len * D * 2;
  const auto kres = __builtin_amdgcn_make_buffer_rsrc(kc + (size_t)g * max_len * D, (short)0,
                                                      (int)head_bytes, 0x00020000);
  const auto vres = __builtin_amdgcn_make_buffer_rsrc(vc + (size_t)g * max_len * D, (short)0,
                                                      (int)head_bytes, 0x00020000);
  u32x4_t ka[4];
  const uint32_t krow_off = (uint32_t)(start + krow) * D * 2 + 16u * grp;
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) ka[s4] = ld16(kres, krow_off + 64u * s4);
  // value rows in the MFMA B layout: lane l holds rows 4 (l / 16) + t (t < 4) of the wave's 16
  // at dims D/2 dh + 16 j + l % 16 (j < 4), one 2-byte load each: vv[4 j + t]
  const uint32_t vrow_off =
      (uint32_t)(start + 16 * w + 4 * grp) * D * 2 + 2u * (D / 2 * dh + r16);
  uint32_t vv[16];
#pragma unroll
  for (int jt = 0; jt < 16; ++jt)
    vv[jt] = __builtin_amdgcn_raw_buffer_load_b16(
        vres, vrow_off + (uint32_t)(jt & 3) * D * 2 + 32u * (uint32_t)(jt >> 2), 0, 0);

  // ---- the position
  const int n = min(pos + 1, max_len);
  if (n <= 0 || start >= n) {  // uniform over the workgroup
    // The loaded values are inputs of this (empty) statement, so the loads are needed on this
    // path too and stay ahead of the branch; otherwise the compiler drops them here and
    // branches first, which puts the position's round trip in front of every load.
    uint32_t used = a0[0] ^ a1[0] ^ b0[0] ^ b1[0] ^ __builtin_bit_cast(uint32_t, frq) ^ tc0[0] ^
                    tc1[0] ^ ts0[0] ^ ts1[0];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) used ^= ka[s4][0];
#pragma unroll
    for (int i = 0; i < 16; ++i) used ^= vv[i];
    asm volatile("" ::"v"(used));
    if (n <= 0 && split == 0 && dh == 0)  // no rows: zeros
      for (int i = tid; i < R * D; i += kAttnBlock) out[(size_t)g * R * D + i] = 0;
    return;
  }
  const int cnt = min(kChunk, n - start);
  const int nsplit = (n + kChunk - 1) / kChunk;
  // row `pos` (the token's own) is in this split when it is in the cache at all
  const bool has_new = kFused && pos < max_len && pos - start < kChunk;
  const bool k_is_new = has_new && start + krow == pos;
  // rows of this wave inside the position; the value loop skips the others (their loads read
  // whatever the cache holds), and does not touch vv before then, so the value rows are not
  // waited for until they are used
  const int rows = min(16, cnt - 16 * w);
  const bool is_k = has_new && ld_k;
  const bool is_v = has_new && ld_v;

  if constexpr (kFused) {
    if (!tab && tid < D / 2) {  // the D/2 rotation angles of this position, once per workgroup
      float sn, cs;
      sincosf(static_cast<float>(pos) * frq, &sn, &cs);
      rot[0][tid] = cs;
      rot[1][tid] = sn;
    }
    if (tid >= nq && tid < 8 * 16) {  // zero q slots of heads R .. 15
      const int h = tid / 8, cc = tid % 8;
      *reinterpret_cast<u32x4_t*>(&qb[h][16 * cc]) = u32x4_t{};
      *reinterpret_cast<u32x4_t*>(&qb[h][16 * cc + 8]) = u32x4_t{};
    }
    if (!tab) lds_sync();  // the angles in LDS (uniform branch; the q slots are read after
                                // the next barrier)
    if (is_q || is_k) {
      float lo[8], hi[8];
      unpack8(a0, lo);
      unpack8(a1, hi);
      if (bias) {
        float blo[8], bhi[8];
        unpack8(b0, blo);
        unpack8(b1, bhi);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          lo[e] = round_bf16(lo[e] + blo[e]);
          hi[e] = round_bf16(hi[e] + bhi[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t tcs = e < 4 ? tc0[e & 3] : tc1[e & 3], tsn = e < 4 ? ts0[e & 3] : ts1[e & 3];
        const float cs = tab ? __builtin_bit_cast(float, tcs) : rot[0][8 * c + e];
        const float sn = tab ? __builtin_bit_cast(float, tsn) : rot[1][8 * c + e];
        const float x1 = lo[e], x2 = hi[e];
        lo[e] = x1 * cs - x2 * sn;
        hi[e] = x2 * cs + x1 * sn;
      }
      const u32x4_t plo = pack8(lo), phi = pack8(hi);
      if (is_q) {
        const int h = tid / 8;
        *reinterpret_cast<u32x4_t*>(&qb[h][8 * c]) = plo;
        *reinterpret_cast<u32x4_t*>(&qb[h][D / 2 + 8 * c]) = phi;
      } else {
        *reinterpret_cast<u32x4_t*>(&knew[8 * c]) = plo;
        *reinterpret_cast<u32x4_t*>(&knew[D / 2 + 8 * c]) = phi;
        if (dh == 0) {  // one of the two workgroups of the split appends the row
          uint16_t* row = kc + ((size_t)g * max_len + pos) * D;
          *reinterpret_cast<u32x4_t*>(row + 8 * c) = plo;
          *reinterpret_cast<u32x4_t*>(row + D / 2 + 8 * c) = phi;
        }
      }
    } else if (is_v) {
      u32x4_t v = a0;
      if (bias) {
        float x[8], b[8];
        unpack8(a0, x);
        unpack8(b0, b);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] += b[e];
        v = pack8(x);
      }
      const int cv = tid - nq - 8;
      *reinterpret_cast<u32x4_t*>(&vnew[8 * cv]) = v;
      if (dh == 0) *reinterpret_cast<u32x4_t*>(vc + ((size_t)g * max_len + pos) * D + 8 * cv) = v;
    }
  } else {
    if (tid < 8 * 16) {
      const int h = tid / 8, cc = tid % 8;
      *reinterpret_cast<u32x4_t*>(&qb[h][16 * cc]) = a0;
      *reinterpret_cast<u32x4_t*>(&qb[h][16 * cc + 8]) = a1;
    }
  }
  lds_sync();
  // the token's own row comes from LDS; its value row is swapped in where the value operands
  // are built (a substitution here would make every value load complete first)
  int inew = -1;
  uint32_t vnw[4] = {0u, 0u, 0u, 0u};
  if (has_new) {
    if (k_is_new) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        ka[s4] = *reinterpret_cast<const u32x4_t*>(&knew[32 * s4 + 8 * grp]);
    }
    inew = pos - start - 16 * w - 4 * grp;  // its t in this lane's four rows, if there
#pragma unroll
    for (int j = 0; j < 4; ++j) vnw[j] = vnew[D / 2 * dh + 16 * j + r16];
  }

  // ---- scores: S[row][head] for the wave's 16 rows and 16 head slots
  f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    const u32x4_t qf = *reinterpret_cast<const u32x4_t*>(&qb[r16][32 * s4 + 8 * grp]);
    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[s4]),
                                                 __builtin_bit_cast(bf16x8_t, qf), sc, 0, 0, 0);
  }
  // lane: head h = r16, rows 16w + 4 grp + r (base-2 logits). Each wave normalises against its
  // own maximum; the waves are merged in the output reduction (flash-attention style), so the
  // softmax needs no workgroup barrier.
  const int h = r16;
  float sr[4];
  float m = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool ok = 16 * w + 4 * grp + r < cnt;
    sr[r] = ok ? sc[r] * qscale : -INFINITY;
    m = fmaxf(m, sr[r]);
  }
  m = fmaxf(m, lane_xor16(m));
  m = fmaxf(m, lane_xor32(m));
  const float mz = m == -INFINITY ? 0.f : m;  // a wave past the position: all p = 0
  // fp32 probabilities as two bf16 MFMA operands, p = hi + lo to within 2^-16 of p: the
  // products stay as exact as the fp32 loop they replace
  float l = 0.f;
  float ph[4], pl[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float p = exp2f(sr[r] - mz);  // 0 for masked rows
    l += p;
    ph[r] = round_bf16(p);
    pl[r] = p - ph[r];
  }
  l += lane_xor16(l);
  l += lane_xor32(l);
  if (grp == 0) {
    red_m[w][h] = m;
    red_l[w][h] = l;
  }

  // ---- values on the matrix cores: O[head][dim] = sum over the wave's 16 rows of P[head][row]
  // V[row][dim]. v_mfma_f32_16x16x16_bf16: A = P (lane l: head l % 16, rows 4 (l / 16) + t,
  // exactly the score layout), B = V (lane l: rows 4 (l / 16) + t, dim l % 16 of each 16-dim
  // block j), D: lane l holds heads 4 (l / 16) + r of dim l % 16. Rows past the position get a
  // zero value (their probability is 0 too; a zero also keeps stale cache words out).
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  const s16x4_t pah = __builtin_bit_cast(
      s16x4_t, make_uint2(pack_bf16x2_rne(ph[0], ph[1]), pack_bf16x2_rne(ph[2], ph[3])));
  const s16x4_t pal = __builtin_bit_cast(
      s16x4_t, make_uint2(pack_bf16x2_rne(pl[0], pl[1]), pack_bf16x2_rne(pl[2], pl[3])));
  f32x4_t ov[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t e[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t v = t == inew ? vnw[j] : vv[4 * j + t];
      e[t] = 4 * grp + t < rows ? v & 0xffffu : 0u;
    }
    const s16x4_t vb = __builtin_bit_cast(s16x4_t, make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16)));
    ov[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pah, vb, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    ov[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pal, vb, ov[j], 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * grp + r < RP) ored[w][4 * grp + r][16 * j + r16] = ov[j][r];
  lds_sync();

  // ---- merge of the waves: each wave's output and sum rescaled from its maximum to the
  // workgroup's (waves with no row in the position have maximum -inf and weight 0)
  const bool single = nsplit == 1;
  for (int i = tid; i < R * D / 2; i += kAttnBlock) {
    const int hh = i / (D / 2), d = D / 2 * dh + i % (D / 2);
    float mt = red_m[0][hh];
#pragma unroll
    for (int k = 1; k < NWV; ++k) mt = fmaxf(mt, red_m[k][hh]);
    float o = 0.f, lt = 0.f;
#pragma unroll
    for (int k = 0; k < NWV; ++k) {
      const float f = exp2f(red_m[k][hh] - mt);
      o = fmaf(f, ored[k][hh][d - D / 2 * dh], o);
      lt = fmaf(f, red_l[k][hh], lt);
    }
    if (single) {
      out[(size_t)(g * R + hh) * D + d] = static_cast<uint16_t>(f32_to_bf16_rne(o / lt));
    } else {
      opart[((size_t)split * Hq + g * R + hh) * D + d] = o;
      if (dh == 0 && d == 0)
        *reinterpret_cast<float2*>(&ml[((size_t)split * Hq + g * R + hh) * 2]) = make_float2(mt, lt);
    }
  }
}

// Second launch: the splits' partial results merged into the attention output. One workgroup
// per (query head, 64 dimensions), eight waves, lane = dimension: wave w merges splits w,
// w + 8, ... with a running maximum (loads issued 16 splits at a time), then wave 0 combines the
// eight waves' results, each rescaled from its own maximum to the overall one. The grid grows with
// the query heads, not the splits, so a long context (hundreds of splits) is merged by 56
// workgroups of short loops (the earlier form, one workgroup per kv head walking every split,
// took as long as the attention itself at 16384 cache rows).
constexpr int kMergeWaves = 8;
__global__ void __launch_bounds__(kMergeWaves * kWave)
    decode_attn_merge_kernel(const float* __restrict__ opart, const float* __restrict__ ml,
                             const int* __restrict__ pos_p, uint16_t* __restrict__ out, int Hq,
                             int max_len) {
  constexpr int D = kHeadDim;
  constexpr int SB = 16;  // splits per load batch of a wave
  __shared__ float red_m[kMergeWaves], red_l[kMergeWaves];
  __shared__ float red_o[kMergeWaves][kWave];
  const int n = min(*pos_p + 1, max_len);
  const int nsplit = n > 0 ? (n + kChunk - 1) / kChunk : 0;
  if (nsplit <= 1) return;  // written by the attention kernel itself
  const int h = blockIdx.x, lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int d = kWave * blockIdx.y + lane;
  float m_w = -INFINITY, l_w = 0.f, acc = 0.f;
  // every split below nsplit holds at least one cache row, so its maximum is finite and the
  // batch maximum below is too (split sb is always in the batch)
  for (int sb = w; sb < nsplit; sb += kMergeWaves * SB) {
    float mv[SB], lv[SB], ov[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int sp = sb + kMergeWaves * u;
      const bool valid = sp < nsplit;
      const size_t row = (size_t)(valid ? sp : sb) * Hq + h;
      const float2 m2 = *reinterpret_cast<const float2*>(&ml[row * 2]);
      mv[u] = valid ? m2.x : -INFINITY;
      lv[u] = valid ? m2.y : 0.f;
      ov[u] = valid ? opart[row * D + d] : 0.f;
    }
    float mb = m_w;
#pragma unroll
    for (int u = 0; u < SB; ++u) mb = fmaxf(mb, mv[u]);
    const float f_old = exp2f(m_w - mb);  // 0 for the first batch (m_w = -inf, mb finite)
    acc *= f_old;
    l_w *= f_old;
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const float f = exp2f(mv[u] - mb);  // 0 for splits past nsplit
      acc = fmaf(f, ov[u], acc);
      l_w = fmaf(f, lv[u], l_w);
    }
    m_w = mb;
  }
  if (lane == 0) {
    red_m[w] = m_w;
    red_l[w] = l_w;
  }
  red_o[w][lane] = acc;
  __syncthreads();
  if (w != 0) return;
  float mt = red_m[0];  // finite: wave 0 holds split 0
#pragma unroll
  for (int k = 1; k < kMergeWaves; ++k) mt = fmaxf(mt, red_m[k]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int k = 0; k < kMergeWaves; ++k) {
    const float f = exp2f(red_m[k] - mt);  // 0 for a wave without splits
    num = fmaf(f, red_o[k][lane], num);
    den = fmaf(f, red_l[k], den);
  }
  out[(size_t)h * D + d] = static_cast<uint16_t>(f32_to_bf16_rne(num / den));
}

// ------------------------------------------------------------------ decode-step start
// The token's embedding row is copied to x, 16 bytes per thread through buffers whose range
// checks turn a token id outside [0, vocab) into a zero row and drop stores past the row; and
// workgroup 0 computes the step's rotation table rot [2][D/2] = cos, sin of fp32(pos) *
// inv_freq[i], the values the attention kernel would otherwise compute in every workgroup of
// every layer (same expression, same compiler, so the same bits).
__global__ void __launch_bounds__(kBlock)
    decode_embed_kernel(const int* __restrict__ tok_p, const int* __restrict__ pos_p,
                        const uint16_t* __restrict__ embed, int vocab, int H,
                        const float* __restrict__ inv_freq, int half, uint16_t* __restrict__ x,
                        float* __restrict__ rot) {
  const int tok = __builtin_amdgcn_readfirstlane(*tok_p);
  const bool ok = tok >= 0 && tok < vocab;
  const uint32_t rb = 2u * (uint32_t)H;
  const auto er = bytes_rsrc(embed + (ok ? (size_t)tok * H : 0), ok ? rb : 0u);
  const auto xr = bytes_rsrc(x, rb);
  const uint32_t off = 16u * (blockIdx.x * kBlock + threadIdx.x);
  st16(xr, off, ld16(er, off));
  if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < half) {
    const int pos = __builtin_amdgcn_readfirstlane(*pos_p);
    float sn, cs;
    sincosf(static_cast<float>(pos) * inv_freq[threadIdx.x], &sn, &cs);
    rot[threadIdx.x] = cs;
    rot[half + threadIdx.x] = sn;
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int last_status() { return static_cast<int>(hipGetLastError()); }

unsigned grid_for(size_t items) {
  const size_t g = (items + kBlock - 1) / kBlock;
  return static_cast<unsigned>(g < 65536 ? (g ? g : 1) : 65536);
}

size_t attn_splits(int max_len) { return (static_cast<size_t>(max_len) + kChunk - 1) / kChunk; }

// Workspace: split outputs [splits][Hq][D] and split (max, sum) pairs [splits][Hq][2], fp32.
size_t attn_workspace(int Hq, int Hk, int D, int max_len) {
  if (Hq <= 0 || Hk <= 0 || D != kHeadDim || max_len <= 0) return 0;
  return attn_splits(max_len) * static_cast<size_t>(Hq) * (D + 2) * sizeof(float);
}

int attn_shape_check(int Hq, int Hk, int D, int max_len) {
  if (D != kHeadDim || Hq <= 0 || Hk <= 0 || Hq % Hk || Hq / Hk > 8 || max_len <= 0) return -2;
  if (attn_splits(max_len) > 65535) return -2;
  return 0;
}

int attn_check(int Hq, int Hk, int D, int max_len, size_t work_bytes, const void* work) {
  if (attn_shape_check(Hq, Hk, D, max_len)) return -2;
  if (!work || !aligned(work, 16) || work_bytes < attn_workspace(Hq, Hk, D, max_len)) return -2;
  return 0;
}

template <bool kFused>
int launch_attn(const void* q, const void* bias, const void* inv_freq, void* kc, void* vc,
                const int* pos, void* out, void* work, int Hq, int Hk, int max_len,
                hipStream_t st, bool merge = true, const float* rot = nullptr) {
  const size_t splits = attn_splits(max_len);
  float* opart = static_cast<float*>(work);
  float* ml = opart + splits * Hq * kHeadDim;
  const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(kHeadDim));  // log2(e)/sqrt(D)
  const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(Hk), 2u);
  hipLaunchKernelGGL(decode_attn_kernel<kFused>, grid, dim3(kAttnBlock), 0, st,
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(bias),
                     static_cast<const float*>(inv_freq), rot, static_cast<uint16_t*>(kc),
                     static_cast<uint16_t*>(vc), pos, static_cast<uint16_t*>(out), opart, ml, Hq,
                     Hk, max_len, qscale);
  if (merge && splits > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    hipLaunchKernelGGL(decode_attn_merge_kernel, dim3(Hq, kHeadDim / kWave), dim3(kMergeWaves * kWave),
                       0, st, opart, ml, pos, static_cast<uint16_t*>(out), Hq, max_len);
  }
  return last_status();
}

}  // namespace

// ------------------------------------------------------------------ allocation-free attention
// ns_decode_attention_noalloc keeps the per-split partials, which ns_decode_attention writes to
// its caller's workspace, in this file-scope device array instead: each GPU holds its own copy
// from the library's load until the process ends, and every call on that GPU shares it. Nothing
// in it has to start at zero: the attention kernel writes every partial slot that the merge
// kernel of the same call reads. On the host, `scratch` names a stand-in, not a device
// address, so host code never passes it to a kernel or a copy: it uses the address that
// hipGetSymbolAddress gives for the current device, taken once per device on the entry point's
// first call there, with that device current.
constexpr size_t kScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_addr[kMaxDevices];
std::mutex scratch_mu;

// The current device's copy of `scratch`: 0 and its address in *out, -2 for a device index past
// kMaxDevices, or the hipError_t of hipGetDevice / hipGetSymbolAddress.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return -2;
  void* p = scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

}  // namespace
}  // namespace ns

extern "C" {

int ns_rmsnorm(void* x, const void* r, const void* w, void* y, int T, int H, float eps,
               void* stream) {
  if (T < 0 || H <= 0 || H % 8 || H > 8192) return -1;
  if (!x || !w || !y) return -1;
  if (!ns::aligned(x, 16) || !ns::aligned(w, 16) || !ns::aligned(y, 16) || !ns::aligned(r, 16))
    return -1;
  if (T == 0) return 0;
  const auto st = static_cast<hipStream_t>(stream);
  const dim3 grid((T + ns::kRowsPerBlock - 1) / ns::kRowsPerBlock), block(64 * ns::kRowsPerBlock);
  auto xp = static_cast<uint16_t*>(x);
  auto rp = static_cast<const uint16_t*>(r);
  auto wp = static_cast<const uint16_t*>(w);
  auto yp = static_cast<uint16_t*>(y);
  const int vpl = (H / 8 + 63) / 64;  // 16-byte vectors per lane: 1 .. 16
  if (vpl <= 1)
    hipLaunchKernelGGL(ns::rms_rows_kernel<1>, grid, block, 0, st, xp, rp, wp, yp, T, H, eps);
  else if (vpl <= 2)
    hipLaunchKernelGGL(ns::rms_rows_kernel<2>, grid, block, 0, st, xp, rp, wp, yp, T, H, eps);
  else if (vpl <= 4)
    hipLaunchKernelGGL(ns::rms_rows_kernel<4>, grid, block, 0, st, xp, rp, wp, yp, T, H, eps);
  else if (vpl <= 8)
    hipLaunchKernelGGL(ns::rms_rows_kernel<8>, grid, block, 0, st, xp, rp, wp, yp, T, H, eps);
  else
    hipLaunchKernelGGL(ns::rms_rows_kernel<16>, grid, block, 0, st, xp, rp, wp, yp, T, H, eps);
  return ns::last_status();
}

int ns_rope(void* q, void* k, const void* inv_freq, int T, int Hq, int Hk, int D, int pos0,
            long long q_stride, long long k_stride, void* stream) {
  if (T < 0 || Hq < 0 || Hk < 0 || D <= 0 || D % 16 || D > 512) return -1;
  if (q_stride < 0) q_stride = static_cast<long long>(Hq) * D;
  if (k_stride < 0) k_stride = static_cast<long long>(Hk) * D;
  if (q_stride % 8 || k_stride % 8) return -1;
  if (!q || !k || !inv_freq || !ns::aligned(q, 16) || !ns::aligned(k, 16) ||
      !ns::aligned(inv_freq, 4))
    return -1;
  const long long waves = static_cast<long long>(T) *
                          ((Hq + Hk + ns::kHeadsPerWave - 1) / ns::kHeadsPerWave);
  if (waves == 0) return 0;
  if ((waves + 3) / 4 > 0x7fffffffLL) return -1;
  const dim3 grid(static_cast<unsigned>((waves + 3) / 4)), block(256);
  const auto st = static_cast<hipStream_t>(stream);
  auto qp = static_cast<uint16_t*>(q);
  auto kp = static_cast<uint16_t*>(k);
  auto fp = static_cast<const float*>(inv_freq);
  if (D <= 128)
    hipLaunchKernelGGL(ns::rope_heads_kernel<1>, grid, block, 0, st, qp, kp, fp, T, Hq, Hk, D,
                       pos0, q_stride, k_stride);
  else if (D <= 256)
    hipLaunchKernelGGL(ns::rope_heads_kernel<2>, grid, block, 0, st, qp, kp, fp, T, Hq, Hk, D,
                       pos0, q_stride, k_stride);
  else
    hipLaunchKernelGGL(ns::rope_heads_kernel<4>, grid, block, 0, st, qp, kp, fp, T, Hq, Hk, D,
                       pos0, q_stride, k_stride);
  return ns::last_status();
}

int ns_swiglu(const void* gate, const void* up, void* out, int T, int I, void* stream) {
  if (T < 0 || I < 0) return -1;
  const long long n = static_cast<long long>(T) * I;
  if (n % 8) return -1;  // the reference's own rejection (nanoserve_ops.cu:39)
  if (n == 0) return 0;
  if (!gate || !up || !out || !ns::aligned(gate, 16) || !ns::aligned(up, 16) ||
      !ns::aligned(out, 16))
    return -1;
  const size_t n8 = static_cast<size_t>(n / 8);
  const size_t blocks = (n8 + ns::kSwigluSpan - 1) / ns::kSwigluSpan;
  if (blocks > 0x7fffffffu) return -1;
  hipLaunchKernelGGL(ns::swiglu_vec_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate),
                     static_cast<const uint16_t*>(up), static_cast<uint16_t*>(out), n8);
  return ns::last_status();
}

int ns_decode_qkv(void* qkv, const void* bias, const void* inv_freq, const int* pos,
                  void* k_cache, void* v_cache, int Hq, int Hk, int D, int max_len,
                  void* stream) {
  if (Hq <= 0 || Hk <= 0 || D <= 0 || D % 16 || max_len <= 0) return -2;
  if (!qkv || !inv_freq || !pos || !k_cache || !v_cache) return -2;
  if (!ns::aligned(qkv, 16) || !ns::aligned(bias, 16) || !ns::aligned(inv_freq, 4) ||
      !ns::aligned(pos, 4) || !ns::aligned(k_cache, 16) || !ns::aligned(v_cache, 16))
    return -2;
  const size_t items = static_cast<size_t>(Hq + Hk) * (D / 16) + static_cast<size_t>(Hk) * (D / 8);
  hipLaunchKernelGGL(ns::decode_qkv_kernel, dim3(ns::grid_for(items)), dim3(ns::kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t*>(qkv),
                     static_cast<const uint16_t*>(bias), static_cast<const float*>(inv_freq), pos,
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), Hq, Hk, D,
                     max_len);
  return ns::last_status();
}

size_t ns_decode_attention_workspace(int Hq, int Hk, int D, int max_len) {
  return ns::attn_workspace(Hq, Hk, D, max_len);
}

int ns_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* pos,
                        void* out, void* work, size_t work_bytes, int Hq, int Hk, int D,
                        int max_len, void* stream) {
  const int rc = ns::attn_check(Hq, Hk, D, max_len, work_bytes, work);
  if (rc) return rc;
  if (!q || !k_cache || !v_cache || !pos || !out) return -2;
  if (!ns::aligned(q, 16) || !ns::aligned(k_cache, 16) || !ns::aligned(v_cache, 16) ||
      !ns::aligned(pos, 4) || !ns::aligned(out, 2))
    return -2;
  return ns::launch_attn<false>(q, nullptr, nullptr, const_cast<void*>(k_cache),
                                const_cast<void*>(v_cache), pos, out, work, Hq, Hk, max_len,
                                static_cast<hipStream_t>(stream));
}

int ns_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                const int* pos, void* out, int Hq, int Hk, int D, int max_len,
                                void* stream) {
  if (ns::attn_shape_check(Hq, Hk, D, max_len)) return -2;
  if (ns::attn_workspace(Hq, Hk, D, max_len) > ns::kScratchBytes) return -2;
  if (!q || !k_cache || !v_cache || !pos || !out) return -2;
  if (!ns::aligned(q, 16) || !ns::aligned(k_cache, 16) || !ns::aligned(v_cache, 16) ||
      !ns::aligned(pos, 4) || !ns::aligned(out, 2))
    return -2;
  void* work = nullptr;
  const int rc = ns::scratch_address(&work);
  if (rc) return rc;
  return ns::launch_attn<false>(q, nullptr, nullptr, const_cast<void*>(k_cache),
                                const_cast<void*>(v_cache), pos, out, work, Hq, Hk, max_len,
                                static_cast<hipStream_t>(stream));
}

int ns_decode_qkv_attention(const void* qkv, const void* bias, const void* inv_freq,
                            const int* pos, void* k_cache, void* v_cache, void* out, void* work,
                            size_t work_bytes, int Hq, int Hk, int D, int max_len, int merge,
                            const float* rot, void* stream) {
  const int rc = ns::attn_check(Hq, Hk, D, max_len, work_bytes, work);
  if (rc) return rc;
  if (!qkv || !inv_freq || !pos || !k_cache || !v_cache || !out) return -2;
  if (!ns::aligned(qkv, 16) || !ns::aligned(bias, 16) || !ns::aligned(inv_freq, 4) ||
      !ns::aligned(pos, 4) || !ns::aligned(k_cache, 16) || !ns::aligned(v_cache, 16) ||
      !ns::aligned(out, 2) || !ns::aligned(rot, 16))
    return -2;
  return ns::launch_attn<true>(qkv, bias, inv_freq, k_cache, v_cache, pos, out, work, Hq, Hk,
                               max_len, static_cast<hipStream_t>(stream), merge != 0, rot);
}

int ns_decode_embed(const int* tok, const int* pos, const void* embed, int vocab, int H,
                    const void* inv_freq, int D, void* x, float* rot, void* stream) {
  if (vocab <= 0 || H <= 0 || H % 8 || D <= 0 || D % 16 || D > 512) return -2;
  if (!tok || !pos || !embed || !inv_freq || !x || !rot) return -2;
  if (!ns::aligned(tok, 4) || !ns::aligned(pos, 4) || !ns::aligned(embed, 16) ||
      !ns::aligned(inv_freq, 4) || !ns::aligned(x, 16) || !ns::aligned(rot, 16))
    return -2;
  const unsigned grid = static_cast<unsigned>((H / 8 + ns::kBlock - 1) / ns::kBlock);
  hipLaunchKernelGGL(ns::decode_embed_kernel, dim3(grid), dim3(ns::kBlock), 0,
                     static_cast<hipStream_t>(stream), tok, pos,
                     static_cast<const uint16_t*>(embed), vocab, H,
                     static_cast<const float*>(inv_freq), D / 2, static_cast<uint16_t*>(x), rot);
  return ns::last_status();
}

}  // extern "C"
