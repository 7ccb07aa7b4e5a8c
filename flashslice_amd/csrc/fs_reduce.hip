// Deterministic second level of every cross-tile reduction.
//
// The point-streaming kernels leave one partial per wave (a static
// tile -> wave assignment). This kernel sums them in a fixed order -- over
// b, then h, then the wave's partition p, sequentially, accumulating in
// fp64 -- and folds the batch / head axes the parameter is shared along, so
// repeated runs are bitwise identical (no atomics). It replaces the
// reference's torch ``.sum`` calls over per-program partials
// (slice_ops.py:481-500, 819, 843, 884-885; blocked.py:1367, 1402-1403,
// 1467-1469).
#include "fs_internal.h"

namespace fs {

__global__ __launch_bounds__(256) void k_reduce_parts(const float* __restrict__ part,
                                                      int64_t wstride, int64_t off, int E, int B,
                                                      int H, int P, int Bo, int Ho,
                                                      float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)Bo * Ho * E;
  if (idx >= total) return;
  const int e = (int)(idx % E);
  const int oh = (int)((idx / E) % Ho);
  const int ob = (int)(idx / ((int64_t)E * Ho));
  const int b0 = Bo > 1 ? ob : 0, b1 = Bo > 1 ? ob + 1 : B;
  const int h0 = Ho > 1 ? oh : 0, h1 = Ho > 1 ? oh + 1 : H;
  double acc = 0.0;
  for (int b = b0; b < b1; ++b)
    for (int h = h0; h < h1; ++h) {
      const float* src = part + ((int64_t)(b * H + h) * P) * wstride + off + e;
      int p = 0;
      for (; p + 4 <= P; p += 4) {
        const float v0 = src[(int64_t)(p + 0) * wstride];
        const float v1 = src[(int64_t)(p + 1) * wstride];
        const float v2 = src[(int64_t)(p + 2) * wstride];
        const float v3 = src[(int64_t)(p + 3) * wstride];
        acc += (double)v0;
        acc += (double)v1;
        acc += (double)v2;
        acc += (double)v3;
      }
      for (; p < P; ++p) acc += (double)src[(int64_t)p * wstride];
    }
  out[idx] = (float)acc;
}

hipError_t launch_reduce_parts(const float* part, int64_t wave_stride, int64_t off, int E, int B,
                               int H, int P, int Bo, int Ho, float* out, hipStream_t st) {
  const int64_t total = (int64_t)Bo * Ho * E;
  if (total <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipLaunchKernelGGL(k_reduce_parts, dim3(blocks), dim3(256), 0, st, part, wave_stride, off, E, B,
                     H, P, Bo, Ho, out);
  return hipGetLastError();
}

hipError_t launch_reduce_scalar(const float* part, int64_t wave_stride, int64_t off, int B, int H,
                                int P, float* out, hipStream_t st) {
  return launch_reduce_parts(part, wave_stride, off, 1, B, H, P, 1, H, out, st);
}

}  // namespace fs
