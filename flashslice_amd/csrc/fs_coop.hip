// Dispatch of the block-cooperative G-blocked kernels (fs_coop_kernels.h):
// bf16 dots on 16-bit point tensors.
#include "fs_coop_kernels.h"

namespace fs {

template <typename T>
static hipError_t coop_dispatch(int kind, const Args& a, hipStream_t st) {
  const dim3 grid(a.P, a.B * a.H), blk(kCoopThreads);
  switch (kind) {
    case CK_SLICE_FWD:
      if (a.stats_in) hipLaunchKernelGGL((k_coop_slice_fwd<T, true>), grid, blk, 0, st, a);
      else hipLaunchKernelGGL((k_coop_slice_fwd<T, false>), grid, blk, 0, st, a);
      break;
    case CK_SLICE_BWD: hipLaunchKernelGGL((k_coop_bwd<T, true>), grid, blk, 0, st, a); break;
    case CK_DESLICE_BWD: hipLaunchKernelGGL((k_coop_bwd<T, false>), grid, blk, 0, st, a); break;
    case CK_DESLICE_FWD:
      if (a.stats_in) hipLaunchKernelGGL((k_coop_deslice_fwd<T, true>), grid, blk, 0, st, a);
      else hipLaunchKernelGGL((k_coop_deslice_fwd<T, false>), grid, blk, 0, st, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool coop_ok(int G, int D, int DV) { return coop_serves(G, D, DV); }

hipError_t launch_coop(int kind, const Args& a, int dtype, hipStream_t st) {
  if (!coop_serves(a.G, a.D, a.DV)) return hipErrorNotSupported;
  if (dtype == DT_BF16) return coop_dispatch<__bf16>(kind, a, st);
  if (dtype == DT_F16) return coop_dispatch<_Float16>(kind, a, st);
  return hipErrorNotSupported;
}

}  // namespace fs
