// LayerNorm over the last axis of a row-major (rows, C) fp32 tensor, for
// the point streams of the layer around the slice/deslice path (the
// Transolver blocks normalise every point's C = 256 features before the
// physics-attention and the MLP; at N = 2e6 each LayerNorm reads and writes
// 2 GB). Not part of the reference's kernels: its model uses
// torch.nn.LayerNorm, whose kernels ran at ~1.9 TB/s here.
//
// Forward: one wave per row at a time (rows strided over the grid's waves),
// the row held in registers as float4 words (C / 4 words over 64 lanes),
// mean and variance in two passes over the registers (a butterfly over the
// wave: every lane ends with the same bits), y = (x - mean) rstd gamma + beta;
// mean and rstd saved per row for the backward.
// Backward: dx = rstd (g - mean(g) - xhat mean(g xhat)) with g = dy gamma,
// xhat = (x - mean) rstd; dgamma = sum_rows dy xhat and dbeta = sum_rows dy
// accumulate lane-locally (each lane owns its columns) over the wave's rows,
// are summed over the block's four waves in a fixed order and written as one
// partial per block, which the fixed-order reduction (fs_reduce.hip) sums.
// The row-to-wave assignment is a function of the shape only: bitwise
// reproducible.
#include "fs_internal.h"

namespace fs {

namespace {

constexpr int kLnWaves = 4;
constexpr int kLnMaxC = 2048;  // columns: 8 float4 words per lane

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float sum4(const float4& a) { return (a.x + a.y) + (a.z + a.w); }

// NV: float4 words per lane (C <= 256 NV)
template <int NV>
__global__ __launch_bounds__(256) void k_ln_fwd(const float* __restrict__ x,
                                                const float* __restrict__ gamma,
                                                const float* __restrict__ beta,
                                                float* __restrict__ y, float* __restrict__ mean,
                                                float* __restrict__ rstd, int64_t rows, int C,
                                                float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (int64_t)blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * kLnWaves;
  const int c4 = C >> 2;
  const float inv_c = 1.f / (float)C;
  float4 gm[NV], bt[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int q = lane + 64 * v;
    gm[v] = q < c4 ? reinterpret_cast<const float4*>(gamma)[q] : make_float4(0, 0, 0, 0);
    bt[v] = q < c4 ? reinterpret_cast<const float4*>(beta)[q] : make_float4(0, 0, 0, 0);
  }
  for (int64_t r = w0; r < rows; r += nw) {
    const float4* xr = reinterpret_cast<const float4*>(x + r * C);
    float4 xv[NV];
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int q = lane + 64 * v;
      xv[v] = q < c4 ? xr[q] : make_float4(0, 0, 0, 0);
      s += sum4(xv[v]);
    }
    const float mu = wave_sum64(s) * inv_c;
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (lane + 64 * v < c4) {
        const float4 d = make_float4(xv[v].x - mu, xv[v].y - mu, xv[v].z - mu, xv[v].w - mu);
        ss += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
      }
    }
    const float rs = 1.f / sqrtf(wave_sum64(ss) * inv_c + eps);
    float4* yr = reinterpret_cast<float4*>(y + r * C);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int q = lane + 64 * v;
      if (q < c4) {
        float4 o;
        o.x = fmaf((xv[v].x - mu) * rs, gm[v].x, bt[v].x);
        o.y = fmaf((xv[v].y - mu) * rs, gm[v].y, bt[v].y);
        o.z = fmaf((xv[v].z - mu) * rs, gm[v].z, bt[v].z);
        o.w = fmaf((xv[v].w - mu) * rs, gm[v].w, bt[v].w);
        yr[q] = o;
      }
    }
    if (lane == 0) {
      mean[r] = mu;
      rstd[r] = rs;
    }
  }
}

template <int NV>
__global__ __launch_bounds__(256) void k_ln_bwd(const float* __restrict__ dy,
                                                const float* __restrict__ x,
                                                const float* __restrict__ gamma,
                                                const float* __restrict__ mean,
                                                const float* __restrict__ rstd,
                                                float* __restrict__ dx, float* __restrict__ part,
                                                int64_t rows, int C) {
  __shared__ float buf[2 * kLnMaxC];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t w0 = (int64_t)blockIdx.x * kLnWaves + wid;
  const int64_t nw = (int64_t)gridDim.x * kLnWaves;
  const int c4 = C >> 2;
  const float inv_c = 1.f / (float)C;
  float4 gm[NV], dg[NV], db[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int q = lane + 64 * v;
    gm[v] = q < c4 ? reinterpret_cast<const float4*>(gamma)[q] : make_float4(0, 0, 0, 0);
    dg[v] = make_float4(0, 0, 0, 0);
    db[v] = make_float4(0, 0, 0, 0);
  }
  for (int64_t r = w0; r < rows; r += nw) {
    const float mu = mean[r], rs = rstd[r];
    const float4* xr = reinterpret_cast<const float4*>(x + r * C);
    const float4* gr = reinterpret_cast<const float4*>(dy + r * C);
    float4 xh[NV], g[NV];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int q = lane + 64 * v;
      const float4 xv = q < c4 ? xr[q] : make_float4(0, 0, 0, 0);
      const float4 dv = q < c4 ? gr[q] : make_float4(0, 0, 0, 0);
      xh[v] = make_float4((xv.x - mu) * rs, (xv.y - mu) * rs, (xv.z - mu) * rs,
                          (xv.w - mu) * rs);
      if (q >= c4) xh[v] = make_float4(0, 0, 0, 0);
      g[v] = make_float4(dv.x * gm[v].x, dv.y * gm[v].y, dv.z * gm[v].z, dv.w * gm[v].w);
      s1 += sum4(g[v]);
      s2 += (g[v].x * xh[v].x + g[v].y * xh[v].y) + (g[v].z * xh[v].z + g[v].w * xh[v].w);
      dg[v].x = fmaf(dv.x, xh[v].x, dg[v].x);
      dg[v].y = fmaf(dv.y, xh[v].y, dg[v].y);
      dg[v].z = fmaf(dv.z, xh[v].z, dg[v].z);
      dg[v].w = fmaf(dv.w, xh[v].w, dg[v].w);
      db[v].x += dv.x;
      db[v].y += dv.y;
      db[v].z += dv.z;
      db[v].w += dv.w;
    }
    const float m1 = wave_sum64(s1) * inv_c, m2 = wave_sum64(s2) * inv_c;
    float4* dr = reinterpret_cast<float4*>(dx + r * C);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int q = lane + 64 * v;
      if (q < c4) {
        float4 o;
        o.x = rs * (g[v].x - m1 - xh[v].x * m2);
        o.y = rs * (g[v].y - m1 - xh[v].y * m2);
        o.z = rs * (g[v].z - m1 - xh[v].z * m2);
        o.w = rs * (g[v].w - m1 - xh[v].w * m2);
        dr[q] = o;
      }
    }
  }
  // the block's four waves in a fixed order, then one partial [dgamma | dbeta]
  for (int w = 0; w < kLnWaves; ++w) {
    if (wid == w) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int q = lane + 64 * v;
        if (q < c4) {
          float* pg = buf + 4 * q;
          float* pb = buf + C + 4 * q;
          const float a[4] = {dg[v].x, dg[v].y, dg[v].z, dg[v].w};
          const float b[4] = {db[v].x, db[v].y, db[v].z, db[v].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pg[e] = w == 0 ? a[e] : pg[e] + a[e];
            pb[e] = w == 0 ? b[e] : pb[e] + b[e];
          }
        }
      }
    }
    __syncthreads();
  }
  float* dst = part + (int64_t)blockIdx.x * 2 * C;
  for (int i = threadIdx.x; i < 2 * C; i += 256) dst[i] = buf[i];
}

}  // namespace

int64_t ln_blocks(int64_t rows) {
  // about 16 rows per wave, at most 2048 blocks (8 per CU)
  const int64_t want = (rows + 16 * kLnWaves - 1) / (16 * kLnWaves);
  return want < 1 ? 1 : want > 2048 ? 2048 : want;
}

#define FS_LN_NV(C) ((C) <= 256 ? 1 : (C) <= 512 ? 2 : (C) <= 1024 ? 4 : 8)

hipError_t ln_fwd_launch(const float* x, const float* gamma, const float* beta, float* y,
                         float* mean, float* rstd, int64_t rows, int C, float eps,
                         hipStream_t st) {
  const dim3 grid((unsigned)ln_blocks(rows)), block(256);
  switch (FS_LN_NV(C)) {
    case 1: hipLaunchKernelGGL(k_ln_fwd<1>, grid, block, 0, st, x, gamma, beta, y, mean, rstd, rows, C, eps); break;
    case 2: hipLaunchKernelGGL(k_ln_fwd<2>, grid, block, 0, st, x, gamma, beta, y, mean, rstd, rows, C, eps); break;
    case 4: hipLaunchKernelGGL(k_ln_fwd<4>, grid, block, 0, st, x, gamma, beta, y, mean, rstd, rows, C, eps); break;
    default: hipLaunchKernelGGL(k_ln_fwd<8>, grid, block, 0, st, x, gamma, beta, y, mean, rstd, rows, C, eps); break;
  }
  return hipGetLastError();
}

hipError_t ln_bwd_launch(const float* dy, const float* x, const float* gamma, const float* mean,
                         const float* rstd, float* dx, float* dgamma, float* dbeta, float* part,
                         int64_t rows, int C, hipStream_t st) {
  const int64_t nb = ln_blocks(rows);
  const dim3 grid((unsigned)nb), block(256);
  switch (FS_LN_NV(C)) {
    case 1: hipLaunchKernelGGL(k_ln_bwd<1>, grid, block, 0, st, dy, x, gamma, mean, rstd, dx, part, rows, C); break;
    case 2: hipLaunchKernelGGL(k_ln_bwd<2>, grid, block, 0, st, dy, x, gamma, mean, rstd, dx, part, rows, C); break;
    case 4: hipLaunchKernelGGL(k_ln_bwd<4>, grid, block, 0, st, dy, x, gamma, mean, rstd, dx, part, rows, C); break;
    default: hipLaunchKernelGGL(k_ln_bwd<8>, grid, block, 0, st, dy, x, gamma, mean, rstd, dx, part, rows, C); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  ReduceSegments segs{};
  segs.seg[0] = ReduceSegment{part, 2 * (int64_t)C, 0, (int)nb, C, 1, 1, dgamma};
  segs.seg[1] = ReduceSegment{part, 2 * (int64_t)C, C, (int)nb, C, 1, 1, dbeta};
  segs.n = 2;
  return launch_reduce(1, 1, segs, st);
}

}  // namespace fs
