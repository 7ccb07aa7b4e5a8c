// Deterministic second level of every cross-tile reduction.
//
// The point-streaming kernels leave one partial per wave (G-blocked family)
// or per block of four waves (whole-G family), from a static tile -> wave
// assignment. One launch per op sums them into every output
// of the op (z_num and s; dW, db and dtau; ...), folding the batch / head
// axes a parameter is shared along. Each block owns 32 consecutive output
// elements of one segment; its 8 thread groups each sum a fixed,
// interleaved subset of the contributing partials in fp64 (four
// accumulators, four loads in flight), and the group sums are added in a
// fixed order -- so repeated runs are bitwise identical (no atomics). Reads
// are coalesced (32 consecutive floats per partial).
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
  auto load = [&](int cc) -> double {
    const int pp = cc % P, bhc = cc / P;
    const int bb = b0 + bhc / nhs, hh = h0 + bhc % nhs;
    return (double)part[((int64_t)(bb * H + hh) * P + pp) * wstride + sg.off + e];
  };
  // group grp sums contributors grp, grp + 8, ... into four accumulators
  // (contributor grp + 8 j goes to accumulator j % 4); sixteen loads are
  // issued before their adds (the sum is latency-bound: a few dozen
  // contributors per thread), the adds keep that order
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  if (e < sg.E) {
    int c = grp, j = 0;
    for (; c + 8 * 15 < C; c += 8 * 16, j += 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = (float)load(c + 8 * u);
#pragma unroll
      for (int u = 0; u < 16; ++u) acc[u & 3] += (double)v[u];
    }
    for (; c + 24 < C; c += 32, j += 4) {
      const double v0 = load(c), v1 = load(c + 8), v2 = load(c + 16), v3 = load(c + 24);
      acc[0] += v0;
      acc[1] += v1;
      acc[2] += v2;
      acc[3] += v3;
    }
    for (; c < C; c += 8, ++j) acc[j & 3] += load(c);
  }
  red[grp][el] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
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
