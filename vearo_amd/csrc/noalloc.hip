// noalloc.hip -- the device-resident scratch behind the allocation-free entry
// points (vh_layernorm_bwd_noalloc).
//
// `scratch` is a file-scope device array: each GPU the library runs on holds
// its own copy, at its own address, until the process ends. In host code the
// array's name is only a host-side stand-in, never a device address, so
// vh_init takes each device's address once with hipGetSymbolAddress (with that
// device current) and every host use goes through that pointer.
//
// Every call on a GPU shares that GPU's array and finds the previous call's
// contents in it; calls that overlap on one GPU race. The kernels that use it
// overwrite everything they read back, so nothing needs clearing.
#include <hip/hip_runtime.h>

#include <string>

#include "rt_internal.h"

static __device__ __align__(256) unsigned char scratch[VH_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

namespace vh_rt {

int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return fail(VH_ERR_UNSUPPORTED, "device-resident scratch: device " + std::to_string(device) +
                                        " is past the " + std::to_string(kMaxDevices) + "-device table");
  if (g_scratch_ptr[device]) return VH_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return fail(VH_ERR_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
  g_scratch_ptr[device] = p;
  return VH_OK;
}

void* noalloc_scratch(int device) {
  return (device >= 0 && device < kMaxDevices) ? g_scratch_ptr[device] : nullptr;
}

}  // namespace vh_rt
