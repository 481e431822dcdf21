/*
 * nanoserve_w4.h -- C ABI of the MI355X-native W4A16 linear-layer engine (libnanoserve_amd.so).
 *
 * Drop-in replacement for the two W4 entry points of the reference's C ABI
 * (Uttaprexa/nanoserve csrc/nanoserve_ops.cu), same symbol names, argument order, types and
 * return codes. All pointers are caller-allocated device memory; the library allocates
 * nothing, keeps no per-call state and never calls exit(). `stream` is a hipStream_t passed as
 * void* (torch.cuda.current_stream().cuda_stream on ROCm; NULL = default stream). Work is
 * asynchronous on that stream.
 *
 * Weight format (reference kernels/quant/w4a16.cuh:5-9):
 *   Wq [N][K/8] uint32 : word j of row n holds k = 8j..8j+7, k = 8j+i in bits 4i..4i+3
 *   S  [N][K/G] bf16   : one scale per G consecutive k;  w[n][k] = (q - 8) * S[n][k/G]
 *
 * Return codes: 0 on success; -1 / -2 as documented per function (arguments are validated
 * before any HIP call, so these never touch the GPU); otherwise the hipError_t reported by
 * hipGetLastError() after the launch, as the reference returns cudaGetLastError().
 */
#ifndef NANOSERVE_W4_H
#define NANOSERVE_W4_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Replaces ns_w4_quantize (reference csrc/nanoserve_ops.cu:65-71; kernel
 * kernels/quant/w4a16.cuh:272-301).
 * W [N][K] bf16 -> Wq [N][K/8] uint32 and S [N][K/G] bf16, bit-identical to the reference's
 * quantizer: scale = bf16_rne(max|w| / 7) (1 for an all-zero group),
 * q = clamp(rint_half_even(w / scale) + 8, 0, 15).
 * Returns -1 if K % G != 0 or G % 32 != 0 (as the reference), and also for G <= 0, negative
 * sizes, a NULL pointer or a W pointer that is not 16-byte aligned. N == 0 or K == 0 is a
 * no-op returning 0.
 */
int ns_w4_quantize(const void* W, void* Wq, void* S, int N, int K, int G, void* stream);

/*
 * Replaces ns_w4_linear (reference csrc/nanoserve_ops.cu:73-90).
 * Y [M][N] bf16 (RNE) = X [M][K] bf16 . deq(Wq, S)^T with fp32 accumulation.
 *   M in 1..8                                   -> decode GEMV (requires K % 32 == 0,
 *                                                  G % 32 == 0, K % G == 0)
 *   M % 128 == 0, N % 128 == 0, K % 32 == 0,
 *   G % 32 == 0, K % G == 0                     -> prefill GEMM (weights staged as
 *                                                  bf16_rne((q - 8) * s), as the reference)
 *   anything else                               -> -2
 * Differences from the reference, all on inputs it mishandles: M = 3, 5, 6, 7 run natively
 * (the reference returns -2; its Python wrapper pads them to 4 or 8); a GEMV shape that
 * violates K % 32, G % 32 or K % G returns -2 (the reference calls exit()); a GEMM shape with
 * K % G != 0 returns -2 (the reference reads past the scale row); M, N, K <= 0, NULL
 * pointers, X or Wq not 16-byte aligned, or S or Y not 2-byte aligned return -2.
 * Every shape runs as one pass over K: the call allocates nothing, keeps no state and gives
 * the same bits on every call (eager or inside graph capture). ns_w4_linear_ws below is the
 * same operation with the decode GEMV's K split.
 */
int ns_w4_linear(const void* X, const void* Wq, const void* S, void* Y, int M, int N, int K,
                 int G, void* stream);

/*
 * No counterpart in the reference (its C ABI has only ns_w4_linear, nanoserve_ops.cu:73-90).
 * Bytes of device workspace ns_w4_linear_ws uses for this shape: ks * M * N * 4 when the
 * M = 2..8 decode GEMV splits K into ks slices (K > 8192 at G = 128: ks = ceil(K / 8192)),
 * 0 for every other shape (and for shapes ns_w4_linear rejects).
 */
size_t ns_w4_linear_workspace(int M, int N, int K, int G);

/*
 * No counterpart in the reference. ns_w4_linear with a caller-provided workspace for the K
 * split of the M = 2..8 decode GEMV (long rows, e.g. K = 11008 or 18944): the slices write
 * fp32 partials [ks][M][N] to `work` and a second launch sums them in slice order and rounds
 * to bf16. Same arithmetic and tolerance as ns_w4_linear, deterministic, but another fp32
 * summation order (outputs may differ from ns_w4_linear's by one bf16 ulp). Shapes whose
 * ns_w4_linear_workspace is 0 run exactly as ns_w4_linear (work may then be NULL); so do the
 * shapes that both entry points run in one pass with the activation streamed through LDS
 * (M >= 6 with about one 16-row group per compute unit, e.g. the 7B down projection at M = 8
 * on MI355X), which leave the workspace unused.
 * Returns -2 when the shape needs a workspace and work is NULL, not 16-byte aligned or smaller
 * than ns_w4_linear_workspace(M, N, K, G); otherwise as ns_w4_linear. Calls that overlap in
 * time need workspaces of their own.
 */
int ns_w4_linear_ws(const void* X, const void* Wq, const void* S, void* Y, int M, int N, int K,
                    int G, void* work, size_t work_bytes, void* stream);

/*
 * No counterpart in the reference (its README:149-151 names a Marlin-style pre-shuffled weight
 * format as the next step). Rewrites (Wq, S) of ns_w4_quantize's format, G == 128, into the
 * packed tile format ns_w4_linear_packed reads: tiles of 16 rows x 128 k, tile (t, c) at
 * Wp + 1024 * (t * (K/128) + c) bytes and Sp + 32 * (t * (K/128) + c) bytes; within a tile the
 * 16-byte run of lane l holds row 16t + l%16, k = 128c + 32s + 8(l/16) + e in word s, nibbles
 * in the order e = 0 2 4 6 1 3 5 7; scales in row order. Sizes: Wp ceil(N/16) * (K/128) * 1024
 * bytes, Sp ceil(N/16) * (K/128) * 32 bytes; rows past N are zero. Returns -2 for G != 128,
 * K % 128 != 0, a packed size of 2 GiB or more, NULL or misaligned pointers (Wp, Sp 16-byte).
 */
int ns_w4_repack(const void* Wq, const void* S, void* Wp, void* Sp, int N, int K, int G,
                 void* stream);

/*
 * No counterpart in the reference. ns_w4_linear on packed weights (ns_w4_repack), for batched
 * decode and prefill: Y [M][N] bf16 (RNE) = X [M][K] bf16 . deq(W)^T with fp32 accumulation.
 * M = 2..16: the same exact dequantisation and products as ns_w4_linear's decode GEMV (fp32 sums
 * over k-groups in another order: outputs agree with ns_w4_linear's to one bf16 ulp, most bit for
 * bit); K up to 20480 (longer rows pass the activation through LDS in chunks). M > 16: the
 * prefill GEMM on the packed tiles, with the reference GEMM's numerics (each weight staged as
 * bf16_rne((q - 8) s) before the bf16 products, as ns_w4_linear's GEMM; another fp32 summation
 * order, so outputs agree with ns_w4_linear's to one bf16 ulp); (M + 256) K * 2 below 2^31.
 * M = 1 is not taken: there the standard format's kernel (ns_w4_linear) is the faster one.
 * Returns -2 for M < 2, G != 128, K % 128 != 0, K > 20480 at M <= 16, an M > 16 past the size
 * limit, a packed size of 2 GiB or more, NULL or misaligned pointers (X, Wp, Sp 16-byte aligned).
 */
int ns_w4_linear_packed(const void* X, const void* Wp, const void* Sp, void* Y, int M, int N,
                        int K, int G, void* stream);

/*
 * No counterpart in the reference's C ABI: ns_w4_linear_packed's prefill GEMM followed by
 * ns_swiglu (the reference MLP's swiglu(linear(h, "g"), linear(h, "u")), python/nanoserve/
 * qwen.py:159) in one launch, on packed weights whose rows are gate and up rows interleaved in
 * blocks of 8 as for ns_w4_linear_swiglu (N = 2 I, N % 16 == 0). Y [M][N/2] bf16 =
 * bf16(silu(g) * u), g and u the bf16 outputs ns_w4_linear_packed gives for the gate and up
 * rows, silu in fp32 as ns_swiglu. M > 16 only (batched decode keeps the GEMV and a separate
 * SwiGLU). Returns -2 for M <= 16 and otherwise as ns_w4_linear_packed's GEMM.
 */
int ns_w4_linear_packed_swiglu(const void* X, const void* Wp, const void* Sp, void* Y, int M,
                               int N, int K, int G, void* stream);

/*
 * No counterpart in the reference's C ABI: ns_w4_linear followed by ns_swiglu, the reference's
 * MLP activation (python/nanoserve/qwen.py:159, swiglu(linear(h, "g"), linear(h, "u"))), in
 * one launch. The rows of Wq / S are gate and up rows interleaved in blocks of 8 (rows 16b ..
 * 16b+7 = gate rows 8b .. 8b+7, rows 16b+8 .. 16b+15 = up rows 8b .. 8b+7; N = 2 I).
 * Y [M][N/2] bf16 = bf16(silu(g) * u), g and u the bf16 outputs ns_w4_linear would give for
 * the gate and up rows, silu in fp32 as ns_swiglu. M == 1: the decode GEMV (G == 128,
 * K % 128 == 0, as ns_w4_gemv_decode); M % 128 == 0: the prefill GEMM (N % 128 == 0, K % 64 == 0,
 * G a power of two >= 32, K % G == 0). Returns -2 for any other shape, N % 16 != 0, NULL or
 * misaligned pointers (X, Wq 16-byte aligned).
 */
int ns_w4_linear_swiglu(const void* X, const void* Wq, const void* S, void* Y, int M, int N,
                        int K, int G, void* stream);

/*
 * Bytes of fp32 workspace ns_w4_gptq needs for N rows (128 * N * 4); 0 for N <= 0.
 */
size_t ns_w4_gptq_workspace(int N);

/*
 * No counterpart in the reference's C ABI: the calibrated quantizer its README.md:233-235 names
 * as the next step after ns_w4_quantize (GPTQ, Frantar et al. 2022, columns in natural order,
 * one scale per row and 128-column group). Output format exactly as ns_w4_quantize's.
 *   W [N][K] fp32: the weights, overwritten (working memory; its contents afterwards are
 *   unspecified). U [K][K] fp32: the upper Cholesky factor of the damped inverse Hessian of the
 *   layer's calibration activations (U^T U = (2 X^T X / T + damping)^-1), computed by the caller;
 *   only its upper triangle is read. work: ns_w4_gptq_workspace(N) bytes of device memory.
 * Column i of each row is quantized with the round-to-nearest rule of ns_w4_quantize, the group
 * scale taken from the row's group values as they stand when the group starts; its error
 * e = (w_i - (q - 8) s) / U[i][i] updates each later column j as w_j <- fma(-e, U[i][j], w_j),
 * the updates of each w_j applied in increasing i. With U diagonal and bf16-valued W, (Wq, S)
 * equal ns_w4_quantize's.
 * Returns -2 for G != 128, K % 128 != 0, N <= 0, work_bytes too small, NULL or misaligned
 * pointers (W, U, Wq, work 16-byte aligned).
 */
int ns_w4_gptq(void* W, const void* U, void* Wq, void* S, void* work, size_t work_bytes, int N,
               int K, int G, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOSERVE_W4_H */
