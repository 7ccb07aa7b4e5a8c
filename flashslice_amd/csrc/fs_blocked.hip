// Dispatch of the G-blocked family: maps the point dtype and the dot level to
// the explicitly instantiated launch templates of fs_blocked_kernels.h (one
// generated translation unit per instance).
#include "fs_blocked_kernels.h"

namespace fs {

int blocked_width_blocks(int D, int DV) {
  const int nb = ((D > DV ? D : DV) + 31) / 32;
  return nb <= 1 ? 1 : nb <= 2 ? 2 : nb <= 4 ? 4 : nb <= 8 ? 8 : 0;
}

template <int K>
static hipError_t blocked_dispatch(const Args& a, int dtype, int mode, hipStream_t st) {
  if (dtype == DT_F32) return blocked_launch<K, float, 0>(a, st);
  if (dtype == DT_BF16) {
    if (mode == 1) return blocked_launch<K, __bf16, 1>(a, st);
    if (mode == 2) return blocked_launch<K, __bf16, 2>(a, st);
    return blocked_launch<K, __bf16, 0>(a, st);
  }
  if (mode == 1) return blocked_launch<K, _Float16, 1>(a, st);
  if (mode == 2) return blocked_launch<K, _Float16, 2>(a, st);
  return blocked_launch<K, _Float16, 0>(a, st);
}

hipError_t launch_gp_prep(const Args& a, int mode, hipStream_t st) {
  const dim3 grid((a.G + 31) / 32, a.B * a.H, 6), blk(256);
  if (mode == 1)
    hipLaunchKernelGGL(k_gp_prep<1>, grid, blk, 0, st, a);
  else if (mode == 2)
    hipLaunchKernelGGL(k_gp_prep<2>, grid, blk, 0, st, a);
  else
    hipLaunchKernelGGL(k_gp_prep<0>, grid, blk, 0, st, a);
  return hipGetLastError();
}

hipError_t launch_blocked(int kind, const Args& a, int dtype, int mode, hipStream_t st) {
  switch (kind) {
    case BK_STATS: return blocked_dispatch<BK_STATS>(a, dtype, mode, st);
    case BK_DESLICE_N: return blocked_dispatch<BK_DESLICE_N>(a, dtype, mode, st);
    case BK_DESLICE_ONLINE: return blocked_dispatch<BK_DESLICE_ONLINE>(a, dtype, mode, st);
    case BK_SLICE_G: return blocked_dispatch<BK_SLICE_G>(a, dtype, mode, st);
    case BK_SLICE_BWD_N: return blocked_dispatch<BK_SLICE_BWD_N>(a, dtype, mode, st);
    case BK_SLICE_BWD_G: return blocked_dispatch<BK_SLICE_BWD_G>(a, dtype, mode, st);
    case BK_DESLICE_BWD_N: return blocked_dispatch<BK_DESLICE_BWD_N>(a, dtype, mode, st);
    case BK_DESLICE_BWD_G: return blocked_dispatch<BK_DESLICE_BWD_G>(a, dtype, mode, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fs
