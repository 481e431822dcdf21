/*
 * nanoserve_decode.h -- C ABI of the operators around the W4 linear layers in one decoder
 * step (libnanoserve_amd.so): the reference's fused residual-add + RMSNorm, RoPE and SwiGLU
 * entry points, and the one-token attention step that the reference's runner does with
 * PyTorch ops.
 *
 * Same conventions as nanoserve_w4.h: caller-allocated device memory, bf16 tensors passed as
 * void* (row-major, 16-byte aligned where a kernel reads 16-byte vectors), `stream` a
 * hipStream_t as void*, asynchronous, no allocation, no host synchronisation (every entry
 * point may be captured in a HIP graph). Return codes: 0 on success, -1 / -2 for rejected
 * arguments (checked before any HIP call), otherwise the hipError_t after the launch.
 */
#ifndef NANOSERVE_DECODE_H
#define NANOSERVE_DECODE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Replaces ns_rmsnorm (reference csrc/nanoserve_ops.cu:20-27; kernel
 * kernels/fused/rmsnorm.cuh:1-52).
 * x [T][H] residual stream; if r != NULL, x <- bf16_rne(x + r) in place (r [T][H]), else x
 * is only read. y [T][H] = bf16_rne(x * rsqrt(mean(x^2) + eps) * w), w [H], fp32 arithmetic.
 * Returns -1 for H % 8 != 0, H > 8192 (the reference's limit, where it calls exit()), T < 0,
 * NULL x / w / y, or a pointer that is not 16-byte aligned. T == 0 is a no-op.
 */
int ns_rmsnorm(void* x, const void* r, const void* w, void* y, int T, int H, float eps,
               void* stream);

/*
 * Replaces ns_rope (reference csrc/nanoserve_ops.cu:29-36; kernel kernels/fused/rope.cuh:1-46).
 * In place on q [T][Hq][D] and k [T][Hk][D], token strides q_stride / k_stride in elements
 * (negative: Hq*D / Hk*D). Token t is at position pos0 + t; for i < D/2, with
 * a = fp32(pos0 + t) * inv_freq[i] (inv_freq [D/2] fp32):
 *   x[i] <- x[i] cos a - x[i + D/2] sin a,   x[i + D/2] <- x[i + D/2] cos a + x[i] sin a.
 * Returns -1 for D % 16 != 0, D > 512, T < 0, Hq < 0, Hk < 0, strides not a multiple of 8,
 * NULL or pointers not 16-byte aligned (q, k) / 4-byte aligned (inv_freq).
 */
int ns_rope(void* q, void* k, const void* inv_freq, int T, int Hq, int Hk, int D, int pos0,
            long long q_stride, long long k_stride, void* stream);

/*
 * Replaces ns_swiglu (reference csrc/nanoserve_ops.cu:38-44; kernel kernels/fused/swiglu.cuh:
 * 35-52). out [T][I] = bf16_rne(silu(gate) * up), gate and up contiguous [T][I],
 * silu(g) = g / (1 + exp(-g)) in fp32. Returns -1 if T*I % 8 != 0 (as the reference), for
 * negative sizes, NULL or pointers that are not 16-byte aligned.
 */
int ns_swiglu(const void* gate, const void* up, void* out, int T, int I, void* stream);

/*
 * No counterpart in the reference's C ABI: the reference does this step with PyTorch ops
 * (python/nanoserve/qwen.py:147-151: bias add, rope, and the cache store of 119-122).
 * One decode token: qkv [(Hq + 2 Hk) * D] bf16 is the fused projection output (q heads, then
 * k heads, then v heads). In place: every element gets bf16_rne(qkv + bias) (bias NULL: no
 * add), then q and k heads are rotated as by ns_rope at position *pos. The rotated k heads and the v heads are
 * also written to k_cache / v_cache [Hk][max_len][D] at row *pos (one layer's slice of a
 * [layers][Hk][max_len][D] cache). pos is a device int32 so that a captured graph can be
 * replayed at any position; a position outside [0, max_len) writes no cache row.
 * Returns -2 for D % 16 != 0, Hq <= 0, Hk <= 0, max_len <= 0, NULL or misaligned pointers.
 */
int ns_decode_qkv(void* qkv, const void* bias, const void* inv_freq, const int* pos,
                  void* k_cache, void* v_cache, int Hq, int Hk, int D, int max_len,
                  void* stream);

/*
 * Bytes of device workspace that ns_decode_attention and ns_decode_qkv_attention need for
 * these sizes: per-split partial results (fp32) of the split over cache rows. Launches that
 * may overlap in time need workspaces of their own. 0 for invalid sizes.
 */
size_t ns_decode_attention_workspace(int Hq, int Hk, int D, int max_len);

/*
 * No counterpart in the reference's C ABI: the reference's decode attention is PyTorch SDPA
 * over the cache (python/nanoserve/qwen.py:124-133). One query token, grouped-query heads:
 * out [Hq][D] bf16 = softmax(q_h . K_g^T / sqrt(D)) V_g over cache rows 0 .. n-1,
 * n = min(*pos + 1, max_len), g = h / (Hq / Hk); q [Hq][D] bf16, k_cache / v_cache
 * [Hk][max_len][D] bf16, fp32 scores, softmax and accumulation (the cache rows are split
 * over workgroups; when there is more than one split a second kernel merges them). work:
 * ns_decode_attention_workspace(...) bytes of device memory, overwritten.
 * n <= 0 gives zeros. Returns -2 for D != 128, Hq % Hk != 0, Hq / Hk > 8, max_len <= 0,
 * work_bytes too small, NULL or misaligned pointers.
 */
int ns_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* pos,
                        void* out, void* work, size_t work_bytes, int Hq, int Hk, int D,
                        int max_len, void* stream);

/*
 * No counterpart in the reference: ns_decode_attention for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments without the workspace, same outputs bit for bit: the per-split partials go to
 * a 4 MiB scratch array that the library holds in each GPU's memory until the process ends. The
 * call allocates and frees nothing. Calls on one GPU share that GPU's scratch: calls that may
 * overlap in time on one GPU (other streams, other host threads) race and must not be issued.
 * Returns -2 where ns_decode_attention does and also when its workspace for these sizes,
 * ns_decode_attention_workspace(Hq, Hk, D, max_len), exceeds 4 MiB (4194304 bytes; at Hq = 28
 * that is max_len <= 36864); a hipError_t if the scratch address cannot be obtained.
 */
int ns_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                const int* pos, void* out, int Hq, int Hk, int D, int max_len,
                                void* stream);

/*
 * No counterpart in the reference's C ABI (its runner does these steps with PyTorch ops,
 * python/nanoserve/qwen.py:119-133, 147-151). ns_decode_qkv followed by ns_decode_attention in
 * one launch, without modifying qkv: the q heads get bias + RoPE at position *pos, the new k
 * (bias + RoPE) and v (bias) rows are appended to the cache at row *pos, and out [Hq][D] is the
 * attention of the rotated q over rows 0 .. min(*pos + 1, max_len) - 1. Same arguments,
 * workspace and return codes as those two. merge == 0 leaves the per-split partial results in
 * the workspace instead of merging them (out is then written only when the rows fit one
 * split): ns_w4_gemv_decode_attn merges them while it loads its activation. rot: NULL, or the
 * rotation table [2][D/2] fp32 (cos, then sin) of this position written by ns_decode_embed on
 * the same stream: the angles are then read from it instead of being computed in every
 * workgroup (same values, same outputs). 16-byte aligned.
 */
int ns_decode_qkv_attention(const void* qkv, const void* bias, const void* inv_freq,
                            const int* pos, void* k_cache, void* v_cache, void* out, void* work,
                            size_t work_bytes, int Hq, int Hk, int D, int max_len, int merge,
                            const float* rot, void* stream);

/*
 * No counterpart in the reference's C ABI (its runner gathers the embedding row with PyTorch,
 * python/nanoserve/qwen.py:141, and computes the rotation angles inside its RoPE): the start
 * of a decode step. x [H] bf16 = embed [vocab][H] row *tok (a token id outside [0, vocab) gives
 * a zero row), and rot [2][D/2] fp32 = cos, sin of fp32(*pos) * inv_freq[i] for i < D/2, the
 * table ns_decode_qkv_attention takes for every layer of the step. tok and pos are device int32
 * so a captured graph replays at any token and position. Returns -2 for vocab <= 0, H <= 0,
 * H % 8 != 0, D % 16 != 0, D > 512, NULL or misaligned pointers (embed, x, rot 16-byte aligned).
 */
int ns_decode_embed(const int* tok, const int* pos, const void* embed, int vocab, int H,
                    const void* inv_freq, int D, void* x, float* rot, void* stream);

/*
 * No counterpart in the reference's C ABI: the decode-step GEMV (M = 1) with its neighbouring
 * operators fused, for a one-token decoder step (the reference launches them one by one:
 * python/nanoserve/qwen.py:145-162 with kernels/fused/rmsnorm.cuh and swiglu.cuh).
 *   input:  res != NULL: the activation is rmsnorm(res + r) * norm_w, exactly as ns_rmsnorm
 *           computes it (r may be NULL: rmsnorm(res) * norm_w); if res_out and r are not NULL,
 *           res_out [K] receives the new residual stream bf16(res + r) (res_out must not alias
 *           res or r). res == NULL: X [K] bf16 is the activation.
 *   output: swiglu == 0: Y [N] bf16, as ns_w4_linear with M = 1.
 *           swiglu != 0: the rows of Wq / S are gate and up rows interleaved in blocks of 8
 *           (rows 16b .. 16b+7 = gate rows 8b .. 8b+7, rows 16b+8 .. 16b+15 = up rows
 *           8b .. 8b+7); Y [N/2] = bf16(silu(g) * u) of the bf16 outputs g, u of each row pair,
 *           as ns_swiglu over ns_w4_linear's output. Needs N % 16 == 0.
 * Weight format as ns_w4_linear with G == 128. Returns -2 for G != 128, K % 128 != 0, K > 16384
 * with res, N % 16 != 0 with swiglu, NULL or misaligned pointers (X, res, r, norm_w, res_out
 * and Wq 16-byte aligned), res_out aliasing res or r.
 */
int ns_w4_gemv_decode(const void* X, const void* res, const void* r, const void* norm_w,
                      float eps, void* res_out, const void* Wq, const void* S, void* Y, int N,
                      int K, int G, int swiglu, void* stream);

/*
 * No counterpart in the reference's C ABI: ns_w4_gemv_decode (plain activation, Y [N] =
 * x . deq(Wq, S)^T) whose activation x [K = Hq * 128] is the output of an
 * ns_decode_qkv_attention(..., merge = 0) launched before it on the same stream with the same
 * pos, max_len, Hq and workspace: when that attention used more than one split of the cache
 * rows, their partial results are merged here (fp32, as the attention's own merge); otherwise
 * attn_out [K] bf16, which the attention then wrote, is read. Returns -2 for K != Hq * 128,
 * G != 128, max_len <= 0, Hq > 64, NULL or misaligned pointers.
 */
int ns_w4_gemv_decode_attn(const void* attn_out, const void* work, const int* pos, int max_len,
                           int Hq, const void* Wq, const void* S, void* Y, int N, int K, int G,
                           void* stream);

/*
 * Replaces the reference's bf16 lm_head product for one token, F.linear(h, lm_head)
 * (python/nanoserve/qwen.py:164, cuBLAS there), with the final norm optionally fused
 * (qwen.py:161-162): Y [N] bf16 = a . W^T, W [N][K] bf16 row-major, fp32 accumulation, where
 * the activation a is X [K] bf16, or, if res != NULL, rmsnorm(res + r) * norm_w computed as
 * ns_rmsnorm does (r may be NULL; res is not written). Returns -2 for K % 8 != 0, K > 8192,
 * NULL or misaligned pointers (X, res, r, norm_w and W 16-byte aligned).
 */
int ns_bf16_gemv(const void* X, const void* res, const void* r, const void* norm_w, float eps,
                 const void* W, void* Y, int N, int K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOSERVE_DECODE_H */
