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

#include "../../include/nanoserve_decode.h"
#include "w4_common.h"

namespace ns {
namespace {

constexpr int kBlock = 256;

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

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_rne(f));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// ------------------------------------------------------------------ residual add + RMSNorm
// One workgroup per row; each thread keeps up to MAXV 8-element vectors of the row in
// registers between the sum of squares and the scaling, so x and r are read once.
template <int MAXV>
__global__ void __launch_bounds__(kBlock)
    rmsnorm_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ r,
                   const uint16_t* __restrict__ w, uint16_t* __restrict__ y, int H, float eps) {
  __shared__ float part[kBlock / kWave];
  const size_t row = blockIdx.x;
  const int vecs = H >> 3;
  u32x4_t* xr = reinterpret_cast<u32x4_t*>(x + row * H);
  const u32x4_t* rr = r ? reinterpret_cast<const u32x4_t*>(r + row * H) : nullptr;
  const u32x4_t* wr = reinterpret_cast<const u32x4_t*>(w);
  u32x4_t* yr = reinterpret_cast<u32x4_t*>(y + row * H);

  float v[MAXV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int idx = threadIdx.x + i * kBlock;
    if (idx < vecs) {
      unpack8(xr[idx], v[i]);
      if (rr) {
        float b[8];
        unpack8(rr[idx], b);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = round_bf16(v[i][e] + b[e]);
        xr[idx] = pack8(v[i]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[i][e], v[i][e], ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kBlock / kWave; ++i) tot += part[i];
  const float inv = rsqrtf(tot / static_cast<float>(H) + eps);
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int idx = threadIdx.x + i * kBlock;
    if (idx < vecs) {
      float g[8], o[8];
      unpack8(wr[idx], g);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[i][e] * inv * g[e];
      yr[idx] = pack8(o);
    }
  }
}

// ------------------------------------------------------------------ RoPE
// Rotates one 16-byte chunk of the first half of a head and its partner in the second half.
__device__ __forceinline__ void rotate8(float (&lo)[8], float (&hi)[8], const float* inv_freq,
                                        int c, float pos) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float s, co;
    sincosf(pos * inv_freq[8 * c + e], &s, &co);
    const float x1 = lo[e], x2 = hi[e];
    lo[e] = x1 * co - x2 * s;
    hi[e] = x2 * co + x1 * s;
  }
}

__global__ void __launch_bounds__(kBlock)
    rope_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                const float* __restrict__ inv_freq, int T, int Hq, int Hk, int D, int pos0,
                long long qs, long long ks) {
  const int chunks = D >> 4;
  const size_t total = (size_t)T * (Hq + Hk) * chunks;
  for (size_t idx = blockIdx.x * (size_t)kBlock + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * kBlock) {
    const int c = static_cast<int>(idx % chunks);
    const size_t rest = idx / chunks;
    const int h = static_cast<int>(rest % (Hq + Hk));
    const long long t = static_cast<long long>(rest / (Hq + Hk));
    uint16_t* base = h < Hq ? q + t * qs + (long long)h * D : k + t * ks + (long long)(h - Hq) * D;
    u32x4_t* lo_p = reinterpret_cast<u32x4_t*>(base + 8 * c);
    u32x4_t* hi_p = reinterpret_cast<u32x4_t*>(base + D / 2 + 8 * c);
    float lo[8], hi[8];
    unpack8(*lo_p, lo);
    unpack8(*hi_p, hi);
    rotate8(lo, hi, inv_freq, c, static_cast<float>(pos0 + t));
    *lo_p = pack8(lo);
    *hi_p = pack8(hi);
  }
}

// ------------------------------------------------------------------ SwiGLU
__global__ void __launch_bounds__(kBlock)
    swiglu_kernel(const u32x4_t* __restrict__ gate, const u32x4_t* __restrict__ up,
                  u32x4_t* __restrict__ out, size_t n8) {
  for (size_t i = blockIdx.x * (size_t)kBlock + threadIdx.x; i < n8;
       i += (size_t)gridDim.x * kBlock) {
    float g[8], u[8];
    unpack8(gate[i], g);
    unpack8(up[i], u);
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = g[e] / (1.f + __expf(-g[e])) * u[e];
    out[i] = pack8(g);
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
      rotate8(lo, hi, inv_freq, c, static_cast<float>(pos));
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
// Split over cache rows: workgroup (s, g) covers rows [s*kChunk, (s+1)*kChunk) of kv head g
// for all R = Hq/Hk query heads of the group (padded to RP). It writes, per query head, the
// split's running max m (base-2 logits), sum l of 2^(logit - m) and the unnormalised output
// sum_p 2^(logit_p - m) v_p (fp32); the combine kernel merges the splits.
//
// Scores: wave w takes rows 16w .. 16w+15 of the chunk, four lanes per row, each lane 32 of
// the 128 dims (four 16-byte loads of its k row); the four partial dot products are summed
// with two lane swaps. Values: wave w takes the same 16 rows, each lane two dims of a row
// (one 4-byte load per row, the wave reads the 256-byte row whole); the four waves' partial
// outputs are summed through LDS.
constexpr int kChunk = 64;
constexpr int kHeadDim = 128;

template <int RP>
__global__ void __launch_bounds__(kBlock)
    decode_attn_partial_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                               const uint16_t* __restrict__ vc, const int* __restrict__ pos_p,
                               float* __restrict__ opart, float* __restrict__ ml, int Hq, int Hk,
                               int max_len, float qscale) {
  constexpr int D = kHeadDim;
  constexpr int NWV = kBlock / kWave;
  __shared__ float qs[RP][D];
  __shared__ float ps[kChunk][RP];
  __shared__ float red[NWV][RP];
  __shared__ float stat[2][RP];
  __shared__ float ored[NWV][RP][D];

  const int n = min(*pos_p + 1, max_len);
  const int split = blockIdx.x, g = blockIdx.y;
  const int start = split * kChunk;
  if (start >= n) return;  // uniform over the workgroup
  const int cnt = min(kChunk, n - start);
  const int R = Hq / Hk;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;

  for (int i = tid; i < RP * D; i += kBlock) {
    const int h = i / D, d = i % D;
    qs[h][d] = h < R ? bf16_bits_to_f32(q[(size_t)(g * R + h) * D + d]) * qscale : 0.f;
  }
  __syncthreads();

  // ---- scores (base-2 logits)
  const int quarter = lane & 3;
  const int pl = 16 * w + (lane >> 2);
  const bool valid = pl < cnt;
  float s[RP];
#pragma unroll
  for (int h = 0; h < RP; ++h) s[h] = 0.f;
  if (valid) {
    const u32x4_t* krow = reinterpret_cast<const u32x4_t*>(
        kc + ((size_t)g * max_len + start + pl) * D + 32 * quarter);
    u32x4_t kv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) kv[j] = krow[j];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float kf[8];
      unpack8(kv[j], kf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 32 * quarter + 8 * j + e;
#pragma unroll
        for (int h = 0; h < RP; ++h) s[h] = fmaf(kf[e], qs[h][d], s[h]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < RP; ++h) {
    s[h] += __shfl_xor(s[h], 1, kWave);
    s[h] += __shfl_xor(s[h], 2, kWave);
  }

  // ---- max over the chunk
#pragma unroll
  for (int h = 0; h < RP; ++h) {
    const float m = wave_max(valid ? s[h] : -INFINITY);
    if (lane == 0) red[w][h] = m;
  }
  __syncthreads();
  if (tid < RP) {
    float m = red[0][tid];
#pragma unroll
    for (int i = 1; i < NWV; ++i) m = fmaxf(m, red[i][tid]);
    stat[0][tid] = m;
  }
  __syncthreads();

  // ---- probabilities and their sum (each row counted once, by its quarter-0 lane)
#pragma unroll
  for (int h = 0; h < RP; ++h) {
    const float p = valid ? exp2f(s[h] - stat[0][h]) : 0.f;
    if (valid && quarter == 0) ps[pl][h] = p;
    const float l = wave_sum(quarter == 0 ? p : 0.f);
    if (lane == 0) red[w][h] = l;
  }
  __syncthreads();
  if (tid < RP) {
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < NWV; ++i) l += red[i][tid];
    stat[1][tid] = l;
  }

  // ---- values
  float acc[RP][2];
#pragma unroll
  for (int h = 0; h < RP; ++h) acc[h][0] = acc[h][1] = 0.f;
  const uint16_t* vbase = vc + ((size_t)g * max_len + start) * D + 2 * lane;
  const int rows = min(16, cnt - 16 * w);
  uint32_t vv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    vv[i] = i < rows ? *reinterpret_cast<const uint32_t*>(vbase + (size_t)(16 * w + i) * D) : 0u;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i < rows) {
      const float v0 = __uint_as_float(vv[i] << 16), v1 = __uint_as_float(vv[i] & 0xffff0000u);
#pragma unroll
      for (int h = 0; h < RP; ++h) {
        const float p = ps[16 * w + i][h];
        acc[h][0] = fmaf(p, v0, acc[h][0]);
        acc[h][1] = fmaf(p, v1, acc[h][1]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < RP; ++h) {
    ored[w][h][2 * lane] = acc[h][0];
    ored[w][h][2 * lane + 1] = acc[h][1];
  }
  __syncthreads();
  for (int i = tid; i < R * D; i += kBlock) {
    const int h = i / D, d = i % D;
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < NWV; ++k) o += ored[k][h][d];
    opart[((size_t)split * Hq + g * R + h) * D + d] = o;
  }
  if (tid < R) {
    ml[((size_t)split * Hq + g * R + tid) * 2] = stat[0][tid];
    ml[((size_t)split * Hq + g * R + tid) * 2 + 1] = stat[1][tid];
  }
}

// One workgroup per query head, one thread per dim: merge the splits' partial softmaxes.
__global__ void __launch_bounds__(kHeadDim)
    decode_attn_combine_kernel(const float* __restrict__ opart, const float* __restrict__ ml,
                               const int* __restrict__ pos_p, uint16_t* __restrict__ out, int Hq,
                               int max_len) {
  const int h = blockIdx.x, d = threadIdx.x;
  const int n = min(*pos_p + 1, max_len);
  const int splits = n > 0 ? (n + kChunk - 1) / kChunk : 0;
  float m = -INFINITY;
  for (int s = 0; s < splits; ++s) m = fmaxf(m, ml[((size_t)s * Hq + h) * 2]);
  float l = 0.f, o = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float f = exp2f(ml[((size_t)s * Hq + h) * 2] - m);
    l = fmaf(f, ml[((size_t)s * Hq + h) * 2 + 1], l);
    o = fmaf(f, opart[((size_t)s * Hq + h) * kHeadDim + d], o);
  }
  out[(size_t)h * kHeadDim + d] = static_cast<uint16_t>(f32_to_bf16_rne(splits ? o / l : 0.f));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int last_status() { return static_cast<int>(hipGetLastError()); }

unsigned grid_for(size_t items) {
  const size_t g = (items + kBlock - 1) / kBlock;
  return static_cast<unsigned>(g < 65536 ? (g ? g : 1) : 65536);
}

size_t attn_splits(int max_len) { return (static_cast<size_t>(max_len) + kChunk - 1) / kChunk; }

}  // namespace
}  // namespace ns

extern "C" {

int ns_rmsnorm(void* x, const void* r, const void* w, void* y, int T, int H, float eps,
               void* stream) {
  if (T < 0 || H <= 0 || H % 8 || H > 8 * ns::kBlock * 4) return -1;
  if (!x || !w || !y) return -1;
  if (!ns::aligned(x, 16) || !ns::aligned(w, 16) || !ns::aligned(y, 16) || !ns::aligned(r, 16))
    return -1;
  if (T == 0) return 0;
  hipLaunchKernelGGL(ns::rmsnorm_kernel<4>, dim3(T), dim3(ns::kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t*>(x),
                     static_cast<const uint16_t*>(r), static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(y), H, eps);
  return ns::last_status();
}

int ns_rope(void* q, void* k, const void* inv_freq, int T, int Hq, int Hk, int D, int pos0,
            long long q_stride, long long k_stride, void* stream) {
  if (T < 0 || Hq < 0 || Hk < 0 || D <= 0 || D % 16) return -1;
  if (q_stride < 0) q_stride = static_cast<long long>(Hq) * D;
  if (k_stride < 0) k_stride = static_cast<long long>(Hk) * D;
  if (q_stride % 8 || k_stride % 8) return -1;
  if (!q || !k || !inv_freq || !ns::aligned(q, 16) || !ns::aligned(k, 16) ||
      !ns::aligned(inv_freq, 4))
    return -1;
  const size_t total = static_cast<size_t>(T) * (Hq + Hk) * (D / 16);
  if (total == 0) return 0;
  hipLaunchKernelGGL(ns::rope_kernel, dim3(ns::grid_for(total)), dim3(ns::kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t*>(q),
                     static_cast<uint16_t*>(k), static_cast<const float*>(inv_freq), T, Hq, Hk,
                     D, pos0, q_stride, k_stride);
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
  hipLaunchKernelGGL(ns::swiglu_kernel, dim3(ns::grid_for(n8)), dim3(ns::kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const ns::u32x4_t*>(gate),
                     static_cast<const ns::u32x4_t*>(up), static_cast<ns::u32x4_t*>(out), n8);
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

size_t ns_decode_attention_workspace(int Hq, int D, int max_len) {
  if (Hq <= 0 || D != ns::kHeadDim || max_len <= 0) return 0;
  return ns::attn_splits(max_len) * static_cast<size_t>(Hq) * (D + 2) * sizeof(float);
}

int ns_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* pos,
                        void* out, void* work, size_t work_bytes, int Hq, int Hk, int D,
                        int max_len, void* stream) {
  if (D != ns::kHeadDim || Hq <= 0 || Hk <= 0 || Hq % Hk || Hq / Hk > 8 || max_len <= 0)
    return -2;
  const size_t splits = ns::attn_splits(max_len);
  if (splits > 65535) return -2;
  if (work_bytes < ns_decode_attention_workspace(Hq, D, max_len)) return -2;
  if (!q || !k_cache || !v_cache || !pos || !out || !work) return -2;
  if (!ns::aligned(q, 16) || !ns::aligned(k_cache, 16) || !ns::aligned(v_cache, 16) ||
      !ns::aligned(pos, 4) || !ns::aligned(out, 2) || !ns::aligned(work, 16))
    return -2;
  float* opart = static_cast<float*>(work);
  float* ml = opart + splits * Hq * D;
  const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(D));  // log2(e)/sqrt(D)
  const auto st = static_cast<hipStream_t>(stream);
  const auto qq = static_cast<const uint16_t*>(q);
  const auto kc = static_cast<const uint16_t*>(k_cache);
  const auto vc = static_cast<const uint16_t*>(v_cache);
  const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(Hk));
  const int R = Hq / Hk;
  if (R <= 4)
    hipLaunchKernelGGL(ns::decode_attn_partial_kernel<4>, grid, dim3(ns::kBlock), 0, st, qq, kc,
                       vc, pos, opart, ml, Hq, Hk, max_len, qscale);
  else
    hipLaunchKernelGGL(ns::decode_attn_partial_kernel<8>, grid, dim3(ns::kBlock), 0, st, qq, kc,
                       vc, pos, opart, ml, Hq, Hk, max_len, qscale);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return static_cast<int>(e);
  hipLaunchKernelGGL(ns::decode_attn_combine_kernel, dim3(Hq), dim3(ns::kHeadDim), 0, st, opart,
                     ml, pos, static_cast<uint16_t*>(out), Hq, max_len);
  return ns::last_status();
}

}  // extern "C"
