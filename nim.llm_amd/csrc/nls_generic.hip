// generic_kernel (full-sort rows and rows the streaming kernel hands on; see
// nls_device.h) and its launcher.
#include "nls_device.h"
#include "nls_launch.h"

namespace nls {

hipError_t launch_generic(const GenericArgs& ga, const LaunchPlan& lp, hipStream_t s) {
  hipLaunchKernelGGL(generic_kernel<kGenericThreads>, dim3(lp.gen_blocks), dim3(kGenericThreads),
                     ga.grouped ? lp.gen_lds : 0, s, ga);
  return hipGetLastError();
}

hipError_t set_generic_attributes() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&generic_kernel<kGenericThreads>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)group_lds_bytes(kGrpMaxV));
}

}  // namespace nls
