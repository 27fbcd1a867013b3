// fwn_attn_fwd_launch_noalloc: the forward launcher with the library's own static scratch in place
// of a caller-provided workspace, for callers that cannot allocate device memory at all.
//
// The scratch is a file-scope __device__ array, so every GPU that loads the library holds one copy
// of FWN_SCRATCH_BYTES until the process ends. Its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and kept; the array's name is only a host-side
// handle and is never passed to a kernel. Calls on one device share its array: split work items
// write their partial results there and the combine pass reads them back in stream order, so calls
// whose kernels can overlap on one device (different streams, or different threads) race. Nothing
// in the scratch needs to start at zero: every slot the combine pass reads is written first by the
// same call.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "fwn_attn.h"
#include "fwn_internal.h"

namespace fwn {
namespace {

static __device__ __align__(256) unsigned char scratch[FWN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch (looked up on the first call on that device).
int scratch_address(void** out) {
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
    return fail(FWN_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(FWN_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess || !p)
        return fail(FWN_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FWN_OK;
}

}  // namespace
}  // namespace fwn

extern "C" int fwn_attn_fwd_launch_noalloc(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                                           const fwn_tiles* tiles, void* o, float* lse, void* stream) {
  uint64_t need = 0;
  if (int rc = fwn_attn_workspace_size(desc, tiles, &need)) return rc;  // validates desc and tiles
  if (desc->precision != FWN_PREC_NATIVE)
    return fwn::fail(FWN_ERR_UNSUPPORTED, "the scratch forward takes FWN_PREC_NATIVE only (bf16x3 splits k and v "
                                          "into a workspace: use fwn_attn_fwd_launch)");
  if (need > FWN_SCRATCH_BYTES)
    return fwn::fail(FWN_ERR_INVALID_ARG,
                     "the split schedule needs %llu bytes of scratch; the static scratch holds %llu "
                     "(use longer work items, or fwn_attn_fwd_launch with a workspace)",
                     (unsigned long long)need, (unsigned long long)FWN_SCRATCH_BYTES);
  void* ptr = nullptr;
  if (need > 0) {
    if (int rc = fwn::scratch_address(&ptr)) return rc;
  }
  return fwn_attn_fwd_launch(desc, q, k, v, tiles, o, lse, ptr, need > 0 ? FWN_SCRATCH_BYTES : 0, stream);
}
