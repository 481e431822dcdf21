// C ABI of the W4A16 engine: the drop-in boundary for csrc/nanoserve_ops.cu:65-90 of the
// reference. Declarations and the full contract are in include/nanoserve_w4.h.
//
// Every argument check happens before the first HIP call, so the error paths run (and are
// tested) on a machine without a GPU; HIP itself initialises lazily on the first launch.
#include <stdint.h>

#include "../../include/nanoserve_decode.h"
#include "../../include/nanoserve_w4.h"
#include "w4_common.h"
#include "w4_kernels.h"

namespace {

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int last_status() { return static_cast<int>(hipGetLastError()); }

}  // namespace

extern "C" {

int ns_w4_quantize(const void* W, void* Wq, void* S, int N, int K, int G, void* stream) {
  if (G <= 0 || N < 0 || K < 0) return -1;
  if (K % G || G % 32) return -1;  // the reference's own rejection (nanoserve_ops.cu:67)
  if (N == 0 || K == 0) return 0;
  if (!W || !Wq || !S || !aligned(W, 16) || !aligned(Wq, 4) || !aligned(S, 2)) return -1;
  const hipError_t e =
      ns::launch_quantize(static_cast<const uint16_t*>(W), static_cast<uint32_t*>(Wq),
                          static_cast<uint16_t*>(S), N, K, G, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return static_cast<int>(e);
  return last_status();
}

}  // extern "C"

namespace {

// ns_w4_linear and ns_w4_linear_ws: the same checks and dispatch; `ws` (may be null) is the
// K-split GEMV's partials buffer.
int w4_linear(const void* X, const void* Wq, const void* S, void* Y, int M, int N, int K, int G,
              void* ws, size_t ws_bytes, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0) return -2;
  if (!X || !Wq || !S || !Y) return -2;
  if (!aligned(X, 16) || !aligned(Wq, 16) || !aligned(S, 2) || !aligned(Y, 2)) return -2;
  const bool fmt_ok = K % 32 == 0 && G % 32 == 0 && K % G == 0;
  const auto st = static_cast<hipStream_t>(stream);
  const auto x = static_cast<const uint16_t*>(X);
  const auto wq = static_cast<const uint32_t*>(Wq);
  const auto s = static_cast<const uint16_t*>(S);
  const auto y = static_cast<uint16_t*>(Y);
  hipError_t e;
  if (M <= 8) {
    if (!fmt_ok) return -2;
    const ns::GemvArgs a{x, wq, s, y, M, N, K, G};
    e = ns::launch_gemv(a, ns::gemv_plan(M, N, K, G), st, static_cast<float*>(ws), ws_bytes);
  } else if (M % 128 == 0 && N % 128 == 0 && fmt_ok) {
    const ns::GemmArgs a{x, wq, s, y, M, N, K, G};
    e = ns::launch_gemm(a, ns::gemm_plan(M, N, K, G), st);
  } else {
    return -2;
  }
  if (e != hipSuccess) return static_cast<int>(e);
  return last_status();
}

}  // namespace

extern "C" {

int ns_w4_linear(const void* X, const void* Wq, const void* S, void* Y, int M, int N, int K,
                 int G, void* stream) {
  return w4_linear(X, Wq, S, Y, M, N, K, G, nullptr, 0, stream);
}

size_t ns_w4_linear_workspace(int M, int N, int K, int G) {
  return ns::gemv_split_bytes(M, N, K, G);
}

int ns_w4_linear_ws(const void* X, const void* Wq, const void* S, void* Y, int M, int N, int K,
                    int G, void* work, size_t work_bytes, void* stream) {
  const size_t need = ns::gemv_split_bytes(M, N, K, G);
  if (need > 0 && (!work || work_bytes < need || !aligned(work, 16))) return -2;
  return w4_linear(X, Wq, S, Y, M, N, K, G, need > 0 ? work : nullptr, work_bytes, stream);
}

int ns_w4_linear_swiglu(const void* X, const void* Wq, const void* S, void* Y, int M, int N,
                        int K, int G, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0 || N % 16) return -2;
  if (!X || !Wq || !S || !Y) return -2;
  if (!aligned(X, 16) || !aligned(Wq, 16) || !aligned(S, 2) || !aligned(Y, 2)) return -2;
  if (M == 1) return ns_w4_gemv_decode(X, nullptr, nullptr, nullptr, 0.f, nullptr, Wq, S, Y, N, K,
                                       G, 1, stream);
  if (M % 128 || N % 128 || K % 32 || G % 32 || K % G || !ns::gemm_v2_ok(M, N, K, G)) return -2;
  const ns::GemmArgs a{static_cast<const uint16_t*>(X), static_cast<const uint32_t*>(Wq),
                       static_cast<const uint16_t*>(S), static_cast<uint16_t*>(Y), M, N, K, G};
  const hipError_t e = ns::launch_gemm_swiglu(a, ns::gemm_plan(M, N, K, G),
                                              static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return static_cast<int>(e);
  return last_status();
}

int ns_w4_gemv_decode(const void* X, const void* res, const void* r, const void* norm_w,
                      float eps, void* res_out, const void* Wq, const void* S, void* Y, int N,
                      int K, int G, int swiglu, void* stream) {
  if (N <= 0 || K <= 0 || G != 128 || K % 128 || (res && K > 16384)) return -2;
  if (!Wq || !S || !Y || (!res && !X) || (res && !norm_w)) return -2;
  if (!aligned(Wq, 16) || !aligned(S, 2) || !aligned(Y, 2) || !aligned(X, 16) ||
      !aligned(res, 16) || !aligned(r, 16) || !aligned(norm_w, 16) || !aligned(res_out, 16))
    return -2;
  if (res_out && (res_out == res || res_out == r)) return -2;
  const ns::GemvArgs a{static_cast<const uint16_t*>(X), static_cast<const uint32_t*>(Wq),
                       static_cast<const uint16_t*>(S), static_cast<uint16_t*>(Y), 1, N, K, G};
  ns::M1Fuse fz;
  fz.res = static_cast<const uint16_t*>(res);
  fz.radd = static_cast<const uint16_t*>(r);
  fz.nw = static_cast<const uint16_t*>(norm_w);
  fz.res_out = static_cast<uint16_t*>(res_out);
  fz.eps = eps;
  int reject = 0;
  const hipError_t e = ns::launch_gemv_fused(a, ns::gemv_plan(1, N, K, G), fz, res != nullptr,
                                             swiglu != 0, static_cast<hipStream_t>(stream),
                                             &reject);
  if (reject) return -2;
  if (e != hipSuccess) return static_cast<int>(e);
  return last_status();
}

int ns_w4_gemv_decode_attn(const void* attn_out, const void* work, const int* pos, int max_len,
                           int Hq, const void* Wq, const void* S, void* Y, int N, int K, int G,
                           void* stream) {
  if (N <= 0 || K <= 0 || G != 128 || Hq <= 0 || K != Hq * 128 || max_len <= 0) return -2;
  if (!attn_out || !work || !pos || !Wq || !S || !Y) return -2;
  if (!aligned(attn_out, 16) || !aligned(work, 16) || !aligned(pos, 4) || !aligned(Wq, 16) ||
      !aligned(S, 2) || !aligned(Y, 2))
    return -2;
  const ns::GemvArgs a{static_cast<const uint16_t*>(attn_out), static_cast<const uint32_t*>(Wq),
                       static_cast<const uint16_t*>(S), static_cast<uint16_t*>(Y), 1, N, K, G};
  const size_t splits = (static_cast<size_t>(max_len) + ns::kAttnDecodeChunk - 1) /
                        ns::kAttnDecodeChunk;
  ns::M1Fuse fz;
  fz.opart = static_cast<const float*>(work);
  fz.ml = fz.opart + splits * static_cast<size_t>(K);
  fz.pos = pos;
  fz.max_len = max_len;
  fz.heads = Hq;
  int reject = 0;
  const hipError_t e = ns::launch_gemv_attn(a, ns::gemv_plan(1, N, K, G), fz,
                                            static_cast<hipStream_t>(stream), &reject);
  if (reject) return -2;
  if (e != hipSuccess) return static_cast<int>(e);
  return last_status();
}

}  // extern "C"
