// nls_stream_inst.h -- the definitions behind nls_launch.h's stream_kernel
// launchers; included by the nls_stream_*.hip units, each of which
// instantiates one (workgroup size, load width) pair.
#pragma once
#include "nls_device.h"
#include "nls_launch.h"

namespace nls {

template <int NT, bool VEC, int Q, bool WAVE>
static hipError_t launch_stream_t(const StreamArgs& a, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((stream_kernel<NT, VEC, Q, WAVE>), dim3(a.B * a.S), dim3(NT), lds, s, a);
  return hipGetLastError();
}

template <int NT, bool VEC, int Q, bool WAVE>
static hipError_t set_attr_one() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&stream_kernel<NT, VEC, Q, WAVE>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_dynamic_lds());
}

// 512-thread workgroups serve only the block path (k > 64)
template <int NT, bool VEC>
hipError_t launch_stream_variant(const StreamArgs& a, const LaunchPlan& p, hipStream_t s) {
  if constexpr (NT != 512) {
    if (p.wave) return launch_stream_t<NT, VEC, 1, true>(a, p.lds, s);
  }
  switch (p.q) {
    case 1: return launch_stream_t<NT, VEC, 1, false>(a, p.lds, s);
    case 2: return launch_stream_t<NT, VEC, 2, false>(a, p.lds, s);
    case 4: return launch_stream_t<NT, VEC, 4, false>(a, p.lds, s);
    default: return launch_stream_t<NT, VEC, 8, false>(a, p.lds, s);
  }
}

template <int NT, bool VEC>
hipError_t set_stream_attributes() {
  hipError_t e;
  if constexpr (NT != 512) {
    if ((e = set_attr_one<NT, VEC, 1, true>()) != hipSuccess) return e;
  }
  if ((e = set_attr_one<NT, VEC, 1, false>()) != hipSuccess) return e;
  if ((e = set_attr_one<NT, VEC, 2, false>()) != hipSuccess) return e;
  if ((e = set_attr_one<NT, VEC, 4, false>()) != hipSuccess) return e;
  return set_attr_one<NT, VEC, 8, false>();
}

}  // namespace nls

#ifdef NLS_PHASE_STAMPS
// this unit's copy of the phase stamps (the phases build only)
#define NLS_STREAM_STAMP_READER(NT, VEC)                                                            \
  extern "C" int nls_stream_stamps_##NT##_##VEC(uint64_t* out) {                                    \
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_phase_stamp),                               \
                               sizeof(uint64_t) * nls::kStampRows * 16) == hipSuccess ? 0 : 3;      \
  }
#else
#define NLS_STREAM_STAMP_READER(NT, VEC)
#endif

#define NLS_INSTANTIATE_STREAM(NT, VEC)                                                             \
  namespace nls {                                                                                  \
  template hipError_t launch_stream_variant<NT, VEC>(const StreamArgs&, const LaunchPlan&, hipStream_t); \
  template hipError_t set_stream_attributes<NT, VEC>();                                            \
  }                                                                                                \
  NLS_STREAM_STAMP_READER(NT, VEC)
