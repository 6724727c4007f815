// Per-device launch state shared by every launcher: the CU count of the
// current device and the dynamic-LDS opt-in of each kernel, both keyed by
// device and safe to use from several host threads at once (the reference
// calls the MoE from one executor thread per GPU,
// mstar/worker/worker.py:1164-1175).
#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>

#include "common.h"
#include "launch.h"

namespace mstar {

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  return dev;
}

std::mutex g_mu;
// (device, kernel) -> largest dynamic LDS size opted in
std::map<std::pair<int, const void*>, size_t> g_lds_optin;
// (device, kernel, threads, LDS bytes) -> resident workgroups per CU
std::map<std::tuple<int, const void*, int, size_t>, int> g_occupancy;
}  // namespace

int device_cu_count() {
  const int dev = current_device();
  if (dev < kMaxDevices) {
    const int c = g_cu_count[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < kMaxDevices) g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

int ensure_dynamic_lds(const void* kernel, size_t bytes, const char* what) {
  if (bytes <= 64 * 1024) return kOk;  // below the default limit: no opt-in needed
  const int dev = current_device();
  std::lock_guard<std::mutex> lock(g_mu);
  size_t& done = g_lds_optin[{dev, kernel}];
  if (bytes <= done) return kOk;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) {
    set_last_error("%s: cannot reserve %zu bytes of LDS", what, bytes);
    return kLaunchError;
  }
  done = bytes;
  return kOk;
}

int occupancy_per_cu(const void* kernel, int threads, size_t lds_bytes) {
  const int dev = current_device();
  std::lock_guard<std::mutex> lock(g_mu);
  auto key = std::make_tuple(dev, kernel, threads, lds_bytes);
  auto it = g_occupancy.find(key);
  if (it != g_occupancy.end()) return it->second;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds_bytes) != hipSuccess || occ <= 0)
    occ = 1;
  g_occupancy.emplace(key, occ);
  return occ;
}

}  // namespace mstar
