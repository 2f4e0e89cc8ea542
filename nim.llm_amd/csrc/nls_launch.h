// nls_launch.h -- launchers of the sampler's two main kernels, each
// instantiated in its own translation unit (nls_stream_*.hip, nls_generic.hip)
// so that the library's build runs them in parallel.
#pragma once
#include <hip/hip_runtime.h>

#include "nls_internal.h"

namespace nls {

// stream_kernel for NT-thread workgroups and 16-byte (VEC) or 4-byte loads,
// picking the wave or block path and the refresh width from the plan.
template <int NT, bool VEC>
hipError_t launch_stream_variant(const StreamArgs& a, const LaunchPlan& p, hipStream_t s);
template <int NT, bool VEC>
hipError_t set_stream_attributes();

hipError_t launch_k64(const StreamArgs& a, const LaunchPlan& p, hipStream_t s);
hipError_t set_k64_attributes();

hipError_t launch_generic(const GenericArgs& ga, const LaunchPlan& lp, hipStream_t s);

hipError_t launch_floor(const FloorArgs& fa, const LaunchPlan& lp, bool vec4, hipStream_t s);
hipError_t set_floor_attributes();
hipError_t set_generic_attributes();

}  // namespace nls
