// Host-side interface between the C ABI (ns_w4_ops.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ns {

// Launch-time device facts, cached per device (launch_cache.hip): the current device's CU count
// and a kernel's occupancy (workgroups per CU) at a block size and dynamic LDS size.
hipError_t cached_cu_count(int* cus);
hipError_t cached_occupancy(const void* fn, int threads, size_t lds, int* per_cu);
// Opts kernel fn into `bytes` of dynamic LDS on the current device, once per (kernel, device).
hipError_t cached_max_dynamic_lds(const void* fn, int bytes);

// K-split M = 2..8 GEMV: the slices' fp32 partials [ks][M][N] live in a caller-provided
// workspace (ns_w4_linear_ws); without one the kernel runs unsplit.
size_t gemv_split_bytes(int M, int N, int K, int G);

struct GemvArgs {
  const uint16_t* X;
  const uint32_t* Wq;
  const uint16_t* S;
  uint16_t* Y;
  int M, N, K, G;
};

struct GemvPlan {
  bool fast;  // MFMA kernels (K % 128 == 0, G % 128 == 0); otherwise the generic kernel
  bool m1;    // M = 1 streaming kernel (w4_gemv_m1_kernel)
  bool xlds;  // activations staged in LDS (w4_gemv_xlds_kernel); otherwise in registers
  bool lds;   // weights staged in LDS per 16-row group (w4_gemv_lds_kernel, M = 2..8)
  bool m8;    // M = 2..8 half-pair streaming kernel (w4_gemv_m8_kernel); rt holds its pairs per wave
  int rt;     // 16-row tiles per wavefront
  int nw;     // wavefronts per workgroup splitting K
  int sl;     // scale slab loads per lane per tile (LDS-activation kernel)
  int ks;     // K slices of the M = 2..8 kernel (1: unsplit)
};

bool gemv_fast_path_ok(int M, int N, int K, int G);
GemvPlan gemv_plan(int M, int N, int K, int G);
// ws / ws_bytes: the K-split workspace (gemv_split_bytes); nullptr splits no shape (shapes the
// chunked-activation kernel serves run in one pass either way).
hipError_t launch_gemv(const GemvArgs& a, const GemvPlan& p, hipStream_t st,
                       float* ws = nullptr, size_t ws_bytes = 0);

// Neighbouring operators fused into the M = 1 GEMV (w4_gemv_m1_kernel):
//   XM == kXNorm:    the activation is rmsnorm(res) * nw;
//   XM == kXNormAdd: the activation is rmsnorm(res + radd) * nw; workgroup 0 stores
//                    bf16(res + radd) to res_out when it is given.
//   YM == kYSwiglu: rows interleaved gate/up in blocks of 8; Y[8g + j] = silu(g) * u.
//   XM == kXAttn:    the activation is the decode attention's output: the merge of its
//                    per-split partials (opart [splits][heads][128], ml [splits][heads][2])
//                    when it used more than one split, else X (bf16, written by it).
enum { kXPlain = 0, kXNorm = 1, kXNormAdd = 2, kXAttn = 3 };
enum { kYPlain = 0, kYSwiglu = 1 };
constexpr int kXVecs = 4;  // 16-byte activation vectors per thread loaded ahead of the weights
struct M1Fuse {
  const uint16_t* res = nullptr;
  const uint16_t* radd = nullptr;
  const uint16_t* nw = nullptr;
  uint16_t* res_out = nullptr;
  float eps = 0.f;
  const float* opart = nullptr;
  const float* ml = nullptr;
  const int* pos = nullptr;
  int max_len = 0;
  int heads = 0;
  // launch layout (set by the launcher, not by the fused operators):
  int rows = 0;    // rows per group when the kernel's GR template argument is 0
  int wide = 0;    // the group's rows are reduced a wave per row (the form the one-round
                   // layouts take), for a launcher that runs another layout in their place
  int xfirst = 0;  // (read by the launcher, which compiles it in) every wave issues its
                   // activation loads before any wave of the workgroup issues weight loads (one
                   // workgroup per CU: the activation then does not queue behind the weight
                   // stream in the CU's memory pipeline)
};
hipError_t launch_gemv_attn(const GemvArgs& a, const GemvPlan& p, const M1Fuse& fz,
                            hipStream_t st, int* reject);
// Decode GEMV with fusions; the plan must be an M = 1 plan (p.m1). -2 if the shape does not
// fit the fused kernel (checked on the host before any launch).
hipError_t launch_gemv_fused(const GemvArgs& a, const GemvPlan& p, const M1Fuse& fz, bool norm,
                             bool swiglu, hipStream_t st, int* reject);

struct GemmArgs {
  const uint16_t* A;   // X [M][K] bf16
  const uint32_t* Wq;  // [N][K/8]
  const uint16_t* S;   // [N][K/G] bf16
  uint16_t* C;         // Y [M][N] bf16
  int M, N, K, G;
};

struct GemmPlan {
  int cfg;  // index into the tile-configuration table of w4_gemm.hip
  int bm, bn;
};

GemmPlan gemm_plan(int M, int N, int K, int G);
hipError_t launch_gemm(const GemmArgs& a, const GemmPlan& p, hipStream_t st);
// GEMM on the packed tile format (ns_w4_repack's Wp, Sp), K % 128 == 0, any M >= 1; plan from
// gemm_packed_plan (0: 128 x 128 tiles, 1: the same with K split over two wave groups,
// 2: 128 x 64 tiles with K split over four, 3: 64 x 64 tiles with K split over four). swiglu:
// rows are gate/up interleaved in blocks of 8
// (N % 16 == 0) and C [M][N/2] receives bf16(silu(g) * u).
int gemm_packed_plan(int M, int N, int K);
hipError_t launch_gemm_packed(const uint16_t* A, const uint32_t* Wp, const uint16_t* Sp, uint16_t* C,
                              int M, int N, int K, int plan, bool swiglu, hipStream_t st);
// The GEMM with the SwiGLU epilogue (a.C is Y [M][N/2]); only the plans gemm_v2_ok admits.
bool gemm_v2_ok(int M, int N, int K, int G);
hipError_t launch_gemm_swiglu(const GemmArgs& a, const GemmPlan& p, hipStream_t st);

hipError_t launch_quantize(const uint16_t* W, uint32_t* Wq, uint16_t* S, int N, int K, int G,
                           hipStream_t st);

}  // namespace ns
