/*
 * CPU oracle for the W4A16 linear-layer path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker. The product path (nanoserve_amd) never calls it.
 *
 * Each function restates the reference algorithm in plain C, citing the reference
 * file:line it follows (paths relative to the Uttaprexa/nanoserve tree):
 *
 *   orc_bf16_rne        kernels/fused/vec.cuh:14-19 (__floats2bfloat162_rn: RNE)
 *   orc_hash_fill       bench/bench_w4a16.cu:32-40 (fill_kernel, integer hash -> bf16)
 *   orc_quantize        kernels/quant/w4a16.cuh:272-297 (quantize_w4_kernel)
 *   orc_dequant_f32     kernels/quant/w4a16.cuh:5-9, 28-32; bench/bench_w4a16.cu:156-162
 *   orc_dequant_bf16    kernels/quant/w4a16.cuh:190-198 (GEMM staging: RNE of the above)
 *   orc_linear_f64      bench/bench_w4a16.cu:163-173 (double accumulation)
 *   orc_linear_w4_f64   same, dequantizing on the fly (no N*K float buffer)
 *   orc_gptq            GPTQ (Frantar et al. 2022, Algorithm 1, natural column order) with the
 *                       quantization rule of kernels/quant/w4a16.cuh:272-297; the reference has
 *                       no calibrated quantizer (README.md:233-235 names it as next)
 *   orc_gemv_ref_order  kernels/quant/w4a16.cuh:21-24, 42-95 (<M,1,float>: per-lane FMA
 *                       order and xor-shuffle tree of the reference GEMV, fp32)
 *
 * Pinning (what fixes each function independently of this restatement) is listed in
 * tests/test_oracle.py; functions are compiled with -ffp-contract=off so every fp32
 * operation rounds exactly once, as written.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static inline float f32_of_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t bits_of_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quiet). vec.cuh:14-19 */
uint16_t orc_bf16_rne(float f) {
  uint32_t u = bits_of_f32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return f32_of_bits((uint32_t)h << 16); }

void orc_bf16_rne_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_rne(in[i]);
}

/* bench_w4a16.cu:32-40. Deterministic integer hash -> uniform in [-1, 1) * 1.732 * scale,
 * stored as bf16 (RNE). (h & 0xFFFFFF) / 2^24 * 2 - 1 is exact in fp32; the two multiplies
 * round once each, left to right. */
void orc_hash_fill(uint16_t* p, size_t n, uint32_t seed, float scale) {
  for (size_t i = 0; i < n; ++i) {
    uint32_t h = ((uint32_t)i * 2654435761u) ^ seed;
    h ^= h >> 15;
    h *= 2246822519u;
    h ^= h >> 13;
    h *= 3266489917u;
    h ^= h >> 16;
    const float u = (float)(h & 0xFFFFFFu) / 16777216.f * 2.f - 1.f;
    const float a = u * 1.732f;
    p[i] = orc_bf16_rne(a * scale);
  }
}

/* Round-half-even float -> int32 with the GPU's saturating conversion (NaN -> 0). */
static int32_t f2i_rn_sat(float x) {
  if (x != x) return 0;
  const float r = nearbyintf(x); /* default rounding mode: to nearest, ties to even */
  if (r >= 2147483648.f) return INT32_MAX;
  if (r < -2147483648.f) return INT32_MIN;
  return (int32_t)r;
}

/* w4a16.cuh:272-297. One (row, group) at a time: scale = bf16(max|w| / 7) (1 when the group
 * is all zero), q = clamp(rint(w / scale) + 8, 0, 15), packed low nibble first. The +8 wraps
 * like the device's 32-bit integer add. Returns 0, or -1 when K % G or G % 32 (the C-ABI's
 * own rejection, nanoserve_ops.cu:67). */
int orc_quantize(const uint16_t* W, uint32_t* Wq, uint16_t* S, int N, int K, int G) {
  if (G <= 0 || K % G || G % 32) return -1;
  const int KG = K / G;
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < KG; ++g) {
      const uint16_t* w = W + (size_t)n * K + (size_t)g * G;
      float mx = 0.f;
      for (int i = 0; i < G; ++i) mx = fmaxf(mx, fabsf(orc_bf16_to_f32(w[i])));
      const uint16_t sb = orc_bf16_rne(mx > 0.f ? mx / 7.f : 1.f);
      const float sf = orc_bf16_to_f32(sb);
      S[(size_t)n * KG + g] = sb;
      for (int j = 0; j < G / 8; ++j) {
        uint32_t word = 0;
        for (int i = 0; i < 8; ++i) {
          const float r = orc_bf16_to_f32(w[j * 8 + i]) / sf;
          int32_t q = (int32_t)((uint32_t)f2i_rn_sat(r) + 8u);
          q = q < 0 ? 0 : q;
          q = q > 15 ? 15 : q;
          word |= (uint32_t)q << (4 * i);
        }
        Wq[(size_t)n * (K / 8) + (size_t)g * (G / 8) + j] = word;
      }
    }
  return 0;
}

/* w4a16.cuh:5-9, 28-32 and bench_w4a16.cu:156-162: w[n,k] = (q - 8) * S[n, k / G] in fp32.
 * Exact: |q - 8| <= 8 and a bf16 scale has 8 significant bits. */
void orc_dequant_f32(const uint32_t* Wq, const uint16_t* S, float* Wd, int N, int K, int G) {
  const int KG = K / G;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      const uint32_t word = Wq[(size_t)n * (K / 8) + k / 8];
      const int q = (int)((word >> (4 * (k % 8))) & 0xFu);
      Wd[(size_t)n * K + k] = (float)(q - 8) * orc_bf16_to_f32(S[(size_t)n * KG + k / G]);
    }
}

/* w4a16.cuh:190-198 (dequant8 then pack8): the prefill GEMM stages each weight as
 * bf16_rne((q - 8) * s) before the bf16 matrix multiply. */
void orc_dequant_bf16(const uint32_t* Wq, const uint16_t* S, uint16_t* Wb, int N, int K, int G) {
  const int KG = K / G;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      const uint32_t word = Wq[(size_t)n * (K / 8) + k / 8];
      const int q = (int)((word >> (4 * (k % 8))) & 0xFu);
      const float w = (float)(q - 8) * orc_bf16_to_f32(S[(size_t)n * KG + k / G]);
      Wb[(size_t)n * K + k] = orc_bf16_rne(w);
    }
}

/* bench_w4a16.cu:163-173: Y[m,n] = sum_k X[m,k] * Wd[n,k], accumulated in double. */
void orc_linear_f64(const uint16_t* X, const float* Wd, double* Y, int M, int N, int K) {
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      const uint16_t* x = X + (size_t)m * K;
      const float* w = Wd + (size_t)n * K;
      for (int k = 0; k < K; ++k) acc += (double)orc_bf16_to_f32(x[k]) * (double)w[k];
      Y[(size_t)m * N + n] = acc;
    }
}

/* Same contraction as orc_linear_f64 with W dequantized on the fly from (Wq, S). When bf16_w
 * is nonzero the weight is first rounded to bf16 (the GEMM staging of orc_dequant_bf16). */
void orc_linear_w4_f64(const uint16_t* X, const uint32_t* Wq, const uint16_t* S, double* Y, int M,
                       int N, int K, int G, int bf16_w) {
  const int KG = K / G;
  for (int n = 0; n < N; ++n) {
    for (int m = 0; m < M; ++m) Y[(size_t)m * N + n] = 0.0;
    for (int k = 0; k < K; ++k) {
      const uint32_t word = Wq[(size_t)n * (K / 8) + k / 8];
      const int q = (int)((word >> (4 * (k % 8))) & 0xFu);
      float w = (float)(q - 8) * orc_bf16_to_f32(S[(size_t)n * KG + k / G]);
      if (bf16_w) w = orc_bf16_to_f32(orc_bf16_rne(w));
      for (int m = 0; m < M; ++m)
        Y[(size_t)m * N + n] += (double)orc_bf16_to_f32(X[(size_t)m * K + k]) * (double)w;
    }
  }
}

/* w4a16.cuh:42-95 with R = 1, fp32 output: one 32-lane warp per row n; lane handles the
 * 16-byte vectors v = lane, lane + 32, ...; for each vector, four 8-weight sub-steps j of
 * acc = fma(x, w, acc) (nvcc contracts `acc += a * b`); then the xor-shuffle reduction with
 * offsets 16, 8, 4, 2, 1 (w4a16.cuh:21-24), lane 0's value is stored. Reproduces the reference
 * GEMV's rounding sequence bit for bit. */
void orc_gemv_ref_order(const uint16_t* X, const uint32_t* Wq, const uint16_t* S, float* Y, int M,
                        int N, int K, int G) {
  const int nvec = K / 32, KG = K / G;
  for (int n = 0; n < N; ++n)
    for (int m = 0; m < M; ++m) {
      float lane_acc[32];
      for (int lane = 0; lane < 32; ++lane) {
        float acc = 0.f;
        for (int v = lane; v < nvec; v += 32) {
          const int k0 = v * 32;
          const float s = orc_bf16_to_f32(S[(size_t)n * KG + k0 / G]);
          for (int j = 0; j < 4; ++j) {
            const uint32_t q = Wq[(size_t)n * (K / 8) + (size_t)v * 4 + j];
            for (int i = 0; i < 8; ++i) {
              const float x = orc_bf16_to_f32(X[(size_t)m * K + k0 + 8 * j + i]);
              const float w = (float)((int)((q >> (4 * i)) & 0xFu) - 8) * s;
              acc = fmaf(x, w, acc);
            }
          }
        }
        lane_acc[lane] = acc;
      }
      for (int o = 16; o > 0; o >>= 1) {
        float nxt[32];
        for (int lane = 0; lane < 32; ++lane) nxt[lane] = lane_acc[lane] + lane_acc[lane ^ o];
        memcpy(lane_acc, nxt, sizeof nxt);
      }
      Y[(size_t)m * N + n] = lane_acc[0];
    }
}

/* GPTQ, unblocked and sequential, one row at a time (rows are independent). W [N][K] fp32 is
 * updated in place; U [K][K] fp32 is the upper Cholesky factor of the damped inverse Hessian.
 * For each group g, the scale comes from the row's group values as they stand when the group
 * starts, by the rule of orc_quantize: s = bf16_rne(max|w| / 7) (1 for an all-zero group).
 * Then for each column i of the group: q = clamp(rint(w_i / s) + 8, 0, 15) (saturating
 * conversion, NaN -> 0), e = fma(-(q - 8), s, w_i) / U[i][i] (the product is exact), and
 * w_j = fma(-e, U[i][j], w_j) for every j > i, in that order. Afterwards W[n][i] holds the value
 * column i had when it was quantized. Codes and scales in the format of orc_quantize. */
int orc_gptq(float* W, const float* U, uint32_t* Wq, uint16_t* S, int N, int K, int G) {
  if (G <= 0 || K % G || G % 8) return -1;
  const int KG = K / G;
  for (int n = 0; n < N; ++n) {
    float* w = W + (size_t)n * K;
    for (int g = 0; g < KG; ++g) {
      float mx = 0.f;
      for (int i = g * G; i < (g + 1) * G; ++i) mx = fmaxf(mx, fabsf(w[i]));
      const uint16_t sb = orc_bf16_rne(mx > 0.f ? mx / 7.f : 1.f);
      const float sf = orc_bf16_to_f32(sb);
      S[(size_t)n * KG + g] = sb;
      uint32_t word = 0;
      for (int i = g * G; i < (g + 1) * G; ++i) {
        int32_t q = (int32_t)((uint32_t)f2i_rn_sat(w[i] / sf) + 8u);
        q = q < 0 ? 0 : (q > 15 ? 15 : q);
        word |= (uint32_t)q << (4 * (i & 7));
        if ((i & 7) == 7) {
          Wq[(size_t)n * (K / 8) + i / 8] = word;
          word = 0;
        }
        const float e = fmaf(-(float)(q - 8), sf, w[i]) / U[(size_t)i * K + i];
        const float* ur = U + (size_t)i * K;
        for (int j = i + 1; j < K; ++j) w[j] = fmaf(-e, ur[j], w[j]);
      }
    }
  }
  return 0;
}
