// rt_internal.h -- runtime helpers shared by libvearo_hip.so's translation
// units. Hidden: not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <string>

namespace vh_rt {
#define VH_RT_HIDDEN __attribute__((visibility("hidden")))
// Records msg as this thread's vh_last_error() text and returns code.
VH_RT_HIDDEN int fail(int code, const std::string& msg);
// VH_OK once vh_init has run, else VH_ERR_NOT_INIT.
VH_RT_HIDDEN int require_init();
// The stream a `void* stream` argument names (NULL: the runtime's own).
VH_RT_HIDDEN hipStream_t stream_of(void* s);
}  // namespace vh_rt
