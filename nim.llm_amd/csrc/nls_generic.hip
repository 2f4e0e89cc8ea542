// generic_kernel (full-sort rows and rows the streaming kernel hands on; see
// nls_device.h) and its launcher.
#include "nls_device.h"
#include "nls_launch.h"

namespace nls {

hipError_t launch_generic(const GenericArgs& ga, const LaunchPlan& lp, hipStream_t s) {
  if (ga.claim)
    hipLaunchKernelGGL((generic_kernel<kGenericThreads, true>), dim3(lp.gen_blocks), dim3(kGenericThreads),
                       ga.grouped ? lp.gen_lds : 0, s, ga);
  else
    hipLaunchKernelGGL((generic_kernel<kGenericThreads, false>), dim3(lp.gen_blocks), dim3(kGenericThreads),
                       ga.grouped ? lp.gen_lds : 0, s, ga);
  return hipGetLastError();
}

hipError_t set_generic_attributes() {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&generic_kernel<kGenericThreads, true>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)group_lds_bytes(kGrpMaxV));
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&generic_kernel<kGenericThreads, false>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)group_lds_bytes(kGrpMaxV));
}

}  // namespace nls

#ifdef NLS_PHASE_STAMPS
// The grouped path's phase stamps of this unit: [4096 x 16] uint64 (host).
extern "C" int nls_generic_stamps(uint64_t* out) {
  const size_t bytes = sizeof(uint64_t) * nls::kStampRows * 16;
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_gen_stamp), bytes) == hipSuccess ? 0 : 3;
}
#endif
