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
 */
int ns_w4_linear(const void* X, const void* Wq, const void* S, void* Y, int M, int N, int K,
                 int G, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOSERVE_W4_H */
