// Launch-time device facts, looked up once and then read from tables: the current device's CU
// count, each kernel's occupancy (workgroups per CU at a block size and dynamic LDS size) and
// its opt-in to more than 64 KiB of dynamic LDS.
// A decode step launches hundreds of kernels, so the launch path must not query HIP for these
// every time; all three are keyed by the current device (hipGetDevice), so a process that drives
// several GPUs gets each device's own figures. The same file keeps the K-split GEMV's
// per-(device, stream) workspace.
#include <atomic>
#include <mutex>
#include <tuple>
#include <vector>

#include "w4_kernels.h"

namespace ns {

namespace {

constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];

struct OccEntry {
  const void* fn;
  int threads;
  size_t lds;
  int dev;
  int per_cu;
};
std::mutex g_occ_mu;
std::vector<OccEntry> g_occ;  // a few dozen entries: one per (kernel, block, LDS size, device)

struct LdsEntry {
  const void* fn;
  int dev;
};
std::mutex g_lds_mu;
std::vector<LdsEntry> g_lds;  // one per (kernel, device) that asked for more than 64 KiB

}  // namespace

hipError_t current_device(int* dev) {
  const hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return e;
  return (*dev < 0 || *dev >= kMaxDevices) ? hipErrorInvalidDevice : hipSuccess;
}

hipError_t cached_cu_count(int* cus) {
  int dev = 0;
  hipError_t e = current_device(&dev);
  if (e != hipSuccess) return e;
  int v = g_cus[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (v <= 0) return hipErrorInvalidDevice;
    g_cus[dev].store(v, std::memory_order_relaxed);
  }
  *cus = v;
  return hipSuccess;
}

hipError_t cached_occupancy(const void* fn, int threads, size_t lds, int* per_cu) {
  int dev = 0;
  hipError_t e = current_device(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_occ_mu);
  for (const OccEntry& o : g_occ)
    if (o.fn == fn && o.threads == threads && o.lds == lds && o.dev == dev) {
      *per_cu = o.per_cu;
      return hipSuccess;
    }
  int v = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, fn, threads, lds);
  if (e != hipSuccess) return e;
  g_occ.push_back(OccEntry{fn, threads, lds, dev, v});
  *per_cu = v;
  return hipSuccess;
}

hipError_t cached_max_dynamic_lds(const void* fn, int bytes) {
  int dev = 0;
  hipError_t e = current_device(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_lds_mu);
  for (const LdsEntry& l : g_lds)
    if (l.fn == fn && l.dev == dev) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  // only a success is remembered: after a failure the next launch asks again
  if (e == hipSuccess) g_lds.push_back(LdsEntry{fn, dev});
  return e;
}

}  // namespace ns
