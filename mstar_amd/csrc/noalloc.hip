// mstar_moe_layer_noalloc: the routed layer of mstar_moe_layer with its
// workspace taken from a fixed device array instead of the caller, for
// callers that cannot allocate (code under stream capture, serving loops
// that forbid hipMalloc).  No counterpart in the reference.
//
// The array lives in this library's code object: one copy per device,
// resident until the process ends.  Host code never passes the array's name
// to a kernel (on the host that name is only a stand-in); its device address
// is looked up once per device with hipGetSymbolAddress, with that device
// current, and that address is what the layer receives.
//
// Every call on a device shares that device's array and overwrites it, so
// calls that overlap in time on one device (two streams, two threads) race.
// Nothing in the layer's workspace has to start at zero: every routing
// histogram, slot list and intermediate buffer is written in full by the
// launch that reads it next, so the array is never cleared.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "common.h"
#include "launch.h"
#include "../../include/mstar_moe.h"

namespace mstar {
namespace {

constexpr size_t kScratchBytes = MSTAR_MOE_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this device's `scratch` (looked up on the first call on
// the device, with it current); nullptr with the message set on failure.
void* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_last_error("moe_layer_noalloc: no current device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    set_last_error("moe_layer_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                   hipGetErrorString(e));
    return nullptr;
  }
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace
}  // namespace mstar

using namespace mstar;

extern "C" int mstar_moe_layer_noalloc(const void* hidden, int act_dtype, int64_t num_tokens,
                                       int64_t hidden_size, const void* router_logits,
                                       int logits_dtype, int renormalize, const void* w1,
                                       const void* w2, int num_experts, int64_t inter, int quant,
                                       const void* w1_scale, const void* w2_scale, int top_k,
                                       int activation, void* out, float* topk_weights_out,
                                       int64_t* topk_ids_out, void* stream) {
  size_t need = 0;
  int st = mstar_moe_layer_workspace_size(num_tokens, hidden_size, num_experts, inter, top_k, quant,
                                          act_dtype, &need);
  if (st != kOk) return st;
  if (need > kScratchBytes) {
    set_last_error("moe_layer_noalloc: these sizes need %zu bytes of workspace, more than the "
                   "%zu-byte device array (num_tokens=%lld); call mstar_moe_layer with a "
                   "workspace instead",
                   need, kScratchBytes, (long long)num_tokens);
    return kWorkspaceTooSmall;
  }
  void* ws = scratch_ptr();
  if (!ws) return kLaunchError;
  // The two-launch decode form: the one-launch kernel's sync words would sit
  // in the shared array, where overlapping calls would reset each other's.
  return moe_layer_impl(hidden, act_dtype, num_tokens, hidden_size, router_logits, logits_dtype,
                        renormalize, w1, w2, num_experts, inter, quant, w1_scale, w2_scale, top_k,
                        activation, out, topk_weights_out, topk_ids_out, ws, kScratchBytes, stream,
                        false);
}
