/*
 * vx_ops_internal.h -- what the library ops (ops.cpp) need from the dispatch
 * core (hip_dispatch.cpp): the caller stream, device checks, and the
 * per-launch hook that honours VX_HIP_SYNC.
 */
#ifndef VX_AMD_OPS_INTERNAL_H
#define VX_AMD_OPS_INTERNAL_H

#include <hip/hip_runtime.h>

namespace vxops {
hipStream_t stream();
bool device_present();
bool on_device(const void *p);
void launched(const char *what);
bool chatty();
/* Whether the caller stream is capturing a hipGraph now. */
bool capturing();
} // namespace vxops

#endif /* VX_AMD_OPS_INTERNAL_H */
