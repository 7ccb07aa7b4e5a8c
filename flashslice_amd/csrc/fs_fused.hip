// Dispatch of the whole-G ("fused") family: maps the point dtype and the
// dot level to the explicitly instantiated launch templates of
// fs_fused_kernels.h (one generated translation unit per instance).
#include "fs_fused_kernels.h"

namespace fs {

bool fused_fits(int D, int DV, int G) {
  const int g = blocks_of(G), d = blocks_of(D), v = blocks_of(DV);
#define X(G_, D_, V_) if (g == G_ && d == D_ && v == V_) return true;
  FS_COMBOS(X)
#undef X
  return false;
}

template <int K>
static hipError_t fused_dispatch(const Args& a, int dtype, int mode, hipStream_t st) {
  if (dtype == DT_F32) return fused_launch<K, float, 0>(a, st);
  if (dtype == DT_BF16) {
    if (mode == 1) return fused_launch<K, __bf16, 1>(a, st);
    if (mode == 2) return fused_launch<K, __bf16, 2>(a, st);
    return fused_launch<K, __bf16, 0>(a, st);
  }
  if (mode == 1) return fused_launch<K, _Float16, 1>(a, st);
  if (mode == 2) return fused_launch<K, _Float16, 2>(a, st);
  return fused_launch<K, _Float16, 0>(a, st);
}

hipError_t launch_fused_slice_fwd(const Args& a, int dtype, int mode, hipStream_t st) {
  return fused_dispatch<FK_SLICE_FWD>(a, dtype, mode, st);
}
hipError_t launch_fused_deslice_fwd(const Args& a, int dtype, int mode, hipStream_t st) {
  return fused_dispatch<FK_DESLICE_FWD>(a, dtype, mode, st);
}
hipError_t launch_fused_slice_bwd(const Args& a, int dtype, int mode, hipStream_t st) {
  return fused_dispatch<FK_SLICE_BWD>(a, dtype, mode, st);
}
hipError_t launch_fused_deslice_bwd(const Args& a, int dtype, int mode, hipStream_t st) {
  return fused_dispatch<FK_DESLICE_BWD>(a, dtype, mode, st);
}
hipError_t launch_fused_tied_bwd(const Args& a, int dtype, int mode, hipStream_t st) {
  return fused_dispatch<FK_TIED_BWD>(a, dtype, mode, st);
}

}  // namespace fs
