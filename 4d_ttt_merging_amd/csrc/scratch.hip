// Static device scratch of vgo_mass_bias_attn_fwd_static.
//
// The array sits in a translation unit of its own, with no kernels: HIP loads a
// code object on a device when one of its kernels or variables is first used
// there (deferred loading), so the array takes device memory only in processes
// that call the allocation-free entry, not in every process that launches the
// attention kernels.  Once looked up, every GPU the library runs on holds its
// copy until the process ends.
//
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address); it uses the per-device address that
// static_scratch() looks up with hipGetSymbolAddress.
#include <mutex>

#include "vgo_common.h"

namespace {

__device__ __align__(256) unsigned char scratch[VGO_ATTN_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace vgo {

int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(VGO_ELAUNCH, "mass_bias_attention(static): no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(VGO_ELAUNCH, std::string("mass_bias_attention(static): hipGetSymbolAddress: ") +
                                   hipGetErrorString(err));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return VGO_OK;
}

}  // namespace vgo
