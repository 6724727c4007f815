// Per-device launch state shared by every launcher: the CU count of the
// current device, the dynamic-LDS opt-in of each kernel and its occupancy,
// all keyed by device and safe to use from several host threads at once (the
// reference calls the MoE from one executor thread per GPU,
// mstar/worker/worker.py:1164-1175).
//
// The hit path takes no lock: each device has a small open-addressed table
// of atomics per kind, filled once per (kernel, size); only a miss (the
// first launch of a kernel at a size on a device) takes the mutex, makes the
// HIP call and publishes the entry (value first, then key, release order).
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "common.h"
#include "launch.h"

namespace mstar {

namespace {
constexpr int kMaxDevices = 64;
constexpr int kSlots = 256;  // per device and kind; ~60 kernels x a few sizes

std::atomic<int> g_cu_count[kMaxDevices];

// One table entry: a 64-bit key (0 = empty) and its value.
struct Slot {
  std::atomic<uint64_t> key{0};
  std::atomic<uint64_t> val{0};
};
Slot g_lds[kMaxDevices][kSlots];  // key: kernel address; val: LDS bytes opted in
Slot g_occ[kMaxDevices][kSlots];  // key: hash of (kernel, threads, LDS); val: packed key check + occupancy
std::mutex g_mu;                  // serialises misses

// The calling thread's device, or -1 with the error message set.
int current_device() {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0) {
    set_last_error("hipGetDevice failed: %s", hipGetErrorString(e));
    return -1;
  }
  if (dev >= kMaxDevices) {
    set_last_error("device %d is beyond the %d devices this library tracks", dev, kMaxDevices);
    return -1;
  }
  return dev;
}

uint64_t mix(uint64_t x) {  // splitmix64 finaliser
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// Index of `key` in `tab`, or of the first empty slot on its probe path;
// -1 if the table is full.
int probe(Slot* tab, uint64_t key) {
  const uint64_t h = mix(key);
  for (int i = 0; i < kSlots; ++i) {
    const int s = (int)((h + (uint64_t)i) % kSlots);
    const uint64_t k = tab[s].key.load(std::memory_order_acquire);
    if (k == key || k == 0) return s;
  }
  return -1;
}
}  // namespace

int device_cu_count() {
  const int dev = current_device();
  if (dev < 0) return 0;
  const int c = g_cu_count[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  int n = 0;
  const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess || n <= 0) {
    set_last_error("cannot read the CU count of device %d: %s", dev, hipGetErrorString(e));
    return 0;
  }
  g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

int ensure_dynamic_lds(const void* kernel, size_t bytes, const char* what) {
  if (bytes <= 64 * 1024) return kOk;  // below the default limit: no opt-in needed
  const int dev = current_device();
  if (dev < 0) return kLaunchError;
  Slot* tab = g_lds[dev];
  const uint64_t key = (uint64_t)(uintptr_t)kernel;
  int s = probe(tab, key);
  if (s >= 0 && tab[s].key.load(std::memory_order_acquire) == key &&
      tab[s].val.load(std::memory_order_acquire) >= bytes)
    return kOk;
  std::lock_guard<std::mutex> lock(g_mu);
  s = probe(tab, key);
  const bool have = s >= 0 && tab[s].key.load(std::memory_order_relaxed) == key;
  if (have && tab[s].val.load(std::memory_order_relaxed) >= bytes) return kOk;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) {
    set_last_error("%s: cannot reserve %zu bytes of LDS", what, bytes);
    return kLaunchError;
  }
  if (s >= 0) {  // a full table only means the next launch asks HIP again
    tab[s].val.store(bytes, std::memory_order_release);
    if (!have) tab[s].key.store(key, std::memory_order_release);
  }
  return kOk;
}

int occupancy_per_cu(const void* kernel, int threads, size_t lds_bytes) {
  const int dev = current_device();
  if (dev < 0) return 0;
  Slot* tab = g_occ[dev];
  // The key hashes all three; the value repeats (threads, LDS) so that a
  // hash collision cannot return another configuration's occupancy.
  const uint64_t tag = ((uint64_t)(uint32_t)threads << 32) | (uint64_t)(uint32_t)lds_bytes;
  const uint64_t key = mix((uint64_t)(uintptr_t)kernel ^ mix(tag)) | 1;
  auto unpack = [&](uint64_t v) -> int { return (int)(v & 0xffff); };
  auto check_of = [&](uint64_t v) -> uint64_t { return v >> 16; };
  const uint64_t want = mix(tag ^ (uint64_t)(uintptr_t)kernel) >> 16;
  int s = probe(tab, key);
  if (s >= 0 && tab[s].key.load(std::memory_order_acquire) == key) {
    const uint64_t v = tab[s].val.load(std::memory_order_acquire);
    if (check_of(v) == want) return unpack(v);
  }
  std::lock_guard<std::mutex> lock(g_mu);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds_bytes) != hipSuccess || occ <= 0)
    occ = 1;
  s = probe(tab, key);
  if (s >= 0 && tab[s].key.load(std::memory_order_relaxed) != key) {
    tab[s].val.store((want << 16) | (uint64_t)(occ & 0xffff), std::memory_order_release);
    tab[s].key.store(key, std::memory_order_release);
  }
  return occ;
}

}  // namespace mstar
