// rt_internal.h -- runtime helpers shared by libvearo_hip.so's translation
// units. Hidden: not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/vearo_hip.h"

namespace vh_rt {
#define VH_RT_HIDDEN __attribute__((visibility("hidden")))
// Records msg as this thread's vh_last_error() text and returns code.
VH_RT_HIDDEN int fail(int code, const std::string& msg);
// VH_OK once vh_init has run, else VH_ERR_NOT_INIT.
VH_RT_HIDDEN int require_init();
// The stream a `void* stream` argument names (NULL: the runtime's own).
VH_RT_HIDDEN hipStream_t stream_of(void* s);
// An unbatched dense product (no addend, or a bias over the output columns;
// accumulation allowed) through hipBLASLt; *taken is false when it does not
// take the layout or has no algorithm, and the caller runs its own kernel.
// akc / bkc: A / B have their unit stride along k.
VH_RT_HIDDEN int blaslt_gemm(const vh_gemm_desc* d, bool akc, bool bkc, void* stream, bool* taken);
// Releases hipBLASLt's handle, workspace and cached plans (vh_shutdown).
VH_RT_HIDDEN void blaslt_shutdown();
// Takes the current device's address of the device-resident scratch
// (noalloc.hip) once per device; vh_init calls it with `device` current.
VH_RT_HIDDEN int noalloc_setup(int device);
// That address (VH_NOALLOC_SCRATCH_BYTES bytes), or NULL before setup.
VH_RT_HIDDEN void* noalloc_scratch(int device);
}  // namespace vh_rt
