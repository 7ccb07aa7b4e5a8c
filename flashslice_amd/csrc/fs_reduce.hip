// Deterministic second level of every cross-tile reduction.
//
// The point-streaming kernels leave one partial per wave (a static
// tile -> wave assignment). One launch per op sums them into every output
// of the op (z_num and s; dW, db and dtau; ...), folding the batch / head
// axes a parameter is shared along. Each block owns 32 consecutive output
// elements of one segment; its 8 thread groups each sum a fixed,
// interleaved subset of the contributing partials in fp64, and the 8 group
// sums are added in a fixed order -- so repeated runs are bitwise identical
// (no atomics). Reads are coalesced (32 consecutive floats per partial).
//
// Replaces the reference's torch ``.sum`` over per-program partials
// (slice_ops.py:481-500, 819, 843, 884-885; blocked.py:1367, 1402-1403,
// 1467-1469).
#include "fs_internal.h"

namespace fs {

__global__ __launch_bounds__(256) void k_reduce_segments(int B, int H, ReduceSegments segs) {
  __shared__ double red[8][33];
  // locate this block's segment
  int blk = blockIdx.x, s = 0;
  for (; s < segs.n; ++s) {
    const int nb = ((segs.seg[s].E + 31) / 32) * segs.seg[s].Bo * segs.seg[s].Ho;
    if (blk < nb) break;
    blk -= nb;
  }
  if (s >= segs.n) return;
  const ReduceSegment& sg = segs.seg[s];
  const float* __restrict__ part = sg.part;
  const int64_t wstride = sg.wstride;
  const int P = sg.P;
  const int eblocks = (sg.E + 31) / 32;
  const int eb = blk % eblocks;
  const int oh = (blk / eblocks) % sg.Ho;
  const int ob = blk / (eblocks * sg.Ho);
  const int el = threadIdx.x & 31, grp = threadIdx.x >> 5;
  const int e = eb * 32 + el;
  const int nbs = sg.Bo > 1 ? 1 : B, nhs = sg.Ho > 1 ? 1 : H;
  const int b0 = sg.Bo > 1 ? ob : 0, h0 = sg.Ho > 1 ? oh : 0;
  const int C = nbs * nhs * P;  // contributors, ordered (b, h, p)
  double acc0 = 0.0, acc1 = 0.0;
  if (e < sg.E) {
    int c = grp;
    for (; c + 8 < C; c += 16) {
      const int c1 = c + 8;
      const int p0 = c % P, bh0 = c / P, p1 = c1 % P, bh1 = c1 / P;
      const int b_0 = b0 + bh0 / nhs, h_0 = h0 + bh0 % nhs;
      const int b_1 = b0 + bh1 / nhs, h_1 = h0 + bh1 % nhs;
      acc0 += (double)part[((int64_t)(b_0 * H + h_0) * P + p0) * wstride + sg.off + e];
      acc1 += (double)part[((int64_t)(b_1 * H + h_1) * P + p1) * wstride + sg.off + e];
    }
    if (c < C) {
      const int p0 = c % P, bh0 = c / P;
      const int b_0 = b0 + bh0 / nhs, h_0 = h0 + bh0 % nhs;
      acc0 += (double)part[((int64_t)(b_0 * H + h_0) * P + p0) * wstride + sg.off + e];
    }
  }
  red[grp][el] = acc0 + acc1;
  __syncthreads();
  if (grp == 0 && e < sg.E) {
    double t = 0.0;
#pragma unroll
    for (int g = 0; g < 8; ++g) t += red[g][el];
    sg.out[((int64_t)ob * sg.Ho + oh) * sg.E + e] = (float)t;
  }
}

hipError_t launch_reduce(int B, int H, const ReduceSegments& segs, hipStream_t st) {
  int64_t blocks = 0;
  for (int s = 0; s < segs.n; ++s)
    blocks += (int64_t)((segs.seg[s].E + 31) / 32) * segs.seg[s].Bo * segs.seg[s].Ho;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_reduce_segments, dim3((unsigned)blocks), dim3(256), 0, st, B, H, segs);
  return hipGetLastError();
}

}  // namespace fs
