// generic_kernel (full-sort rows and rows the streaming kernel hands on; see
// nls_device.h) and its launcher.
#include <algorithm>

#include "nls_device.h"
#include "nls_launch.h"

namespace nls {

hipError_t launch_generic(const GenericArgs& ga, const LaunchPlan& lp, hipStream_t s) {
  const size_t lds = ga.grouped ? lp.gen_lds : 0;
  if (ga.fb_list) {
    // grouped rows first; the rows they leave (fallback list) after them
    if (ga.claim)
      hipLaunchKernelGGL((generic_grouped_kernel<kGenericThreads, true>), dim3(lp.gen_blocks),
                         dim3(kGenericThreads), lds, s, ga);
    else
      hipLaunchKernelGGL((generic_grouped_kernel<kGenericThreads, false>), dim3(lp.gen_blocks),
                         dim3(kGenericThreads), lds, s, ga);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ga.walk_split) {
      // the stored rows' walks, one wave each, and their member searches
      hipLaunchKernelGGL((walk_member_kernel<kGenericThreads>), dim3(std::max(1, lp.walk_blocks)),
                         dim3(kGenericThreads), lp.walk_lds, s, ga);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    GenericArgs fb = ga;
    fb.generic_list = ga.fb_list;
    fb.generic_count = ga.fb_count;
    fb.next_count = ga.fb_next;
    fb.claim = nullptr;
    fb.next_claim = nullptr;
    fb.fixed_list = nullptr;
    fb.n_fixed = 0;
    fb.fb_in = 1;
    hipLaunchKernelGGL((generic_kernel<kGenericThreads, false>), dim3(lp.gen_blocks), dim3(kGenericThreads), lds,
                       s, fb);
  } else if (ga.claim) {
    hipLaunchKernelGGL((generic_kernel<kGenericThreads, true>), dim3(lp.gen_blocks), dim3(kGenericThreads), lds,
                       s, ga);
  } else {
    hipLaunchKernelGGL((generic_kernel<kGenericThreads, false>), dim3(lp.gen_blocks), dim3(kGenericThreads), lds,
                       s, ga);
  }
  return hipGetLastError();
}

hipError_t set_generic_attributes() {
  const int lds = (int)group_lds_bytes(kGrpMaxV);
  const void* fns[5] = {reinterpret_cast<const void*>(&generic_kernel<kGenericThreads, true>),
                        reinterpret_cast<const void*>(&generic_kernel<kGenericThreads, false>),
                        reinterpret_cast<const void*>(&generic_grouped_kernel<kGenericThreads, true>),
                        reinterpret_cast<const void*>(&generic_grouped_kernel<kGenericThreads, false>),
                        reinterpret_cast<const void*>(&walk_member_kernel<kGenericThreads>)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace nls

#ifdef NLS_PHASE_STAMPS
// The grouped path's phase stamps of this unit: [4096 x 16] uint64 (host).
extern "C" int nls_generic_stamps(uint64_t* out) {
  const size_t bytes = sizeof(uint64_t) * nls::kStampRows * 16;
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(nls::nls_gen_stamp), bytes) == hipSuccess ? 0 : 3;
}
#endif
