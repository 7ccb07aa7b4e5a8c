// Whole-G ("fused") slice/deslice kernel templates for gfx950.
//
// One wave owns one (b, h) and a strided sequence of 32-point tiles
// (tile t = pid, pid + P, ...; a static assignment, so per-wave partial sums
// are deterministic). The whole slot axis G (padded to NGB blocks of 32) is
// held in registers, so the softmax over G is exact in one pass and the
// N x H x G weight tensor never exists outside registers. Every dot runs on
// MFMA: v_mfma_f32_32x32x2_f32 for the ieee/tf32/tf32x3 levels and
// v_mfma_f32_32x32x16_bf16 for the bf16 levels (see fs_device.h for the
// fragment convention). Slot-indexed sums (z_num, s, dtokens, dW, db, dtau)
// are accumulated per wave and written as per-wave partials that
// fs_reduce.hip sums in a fixed order.
//
// Reference kernels these replace: _slice_fwd_kernel (slice_ops.py:554-599),
// _deslice_fwd_kernel (:602-640), _slice_bwd_kernel (:643-710),
// _deslice_bwd_kernel (:713-776).
#pragma once
#include "fs_device.h"
#include "fs_internal.h"

namespace fs {

// DK: 0 = every dot fp32 MFMA; 1 = value dots bf16 (reference level 2,
// "bf16v"); 2 = every dot bf16 (level 3).
template <int DK> struct Modes {
  static constexpr int L = (DK == 2) ? MMA_BF16 : MMA_F32;
  static constexpr int V = (DK >= 1) ? MMA_BF16 : MMA_F32;
};

// Per-wave constants of the logits: W as the A operand [g-outer, d-inner],
// and bias * log2(e) / tau per output slot (-inf on padded slots).
template <int NGB, int NDB>
__device__ __forceinline__ void load_logit_consts(float (&wA)[NGB][NDB][16], float (&bc)[NGB][16],
                                                  const float* Wp, const float* Bp, float cst,
                                                  int G, int D, int c, int h) {
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_mat_rowouter(wA[gb][db], Wp, 32 * gb, G, 32 * db, D, c, h);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int g = 32 * gb + kmap(r, h);
      bc[gb][r] = g < G ? Bp[g] * cst : -INFINITY;
    }
  }
}

// Scaled logits t2 = (x . W + b) * log2(e) / tau of one tile, as
// [point-outer, slot-inner] fragments.
template <int ML, int NGB, int NDB>
__device__ __forceinline__ void logits_tile(float (&t2)[NGB][16], const float (&wA)[NGB][NDB][16],
                                            const float (&xf)[NDB][16], const float (&bc)[NGB][16],
                                            float cst) {
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    f32x16 s = zero16();
#pragma unroll
    for (int db = 0; db < NDB; ++db) s = mma32<ML>(wA[gb][db], xf[db], s);
#pragma unroll
    for (int r = 0; r < 16; ++r) t2[gb][r] = fmaf(s[r], cst, bc[gb][r]);
  }
}

// Softmax over the G slots of each point (lane pair c, c + 32 holds one
// point). Returns w (zero for points beyond N) and the row max m2 (log2
// units). The row sum is formed in a fixed order (lane-local, then the
// partner), so both lanes of a pair hold the same value.
template <int NGB>
__device__ __forceinline__ void softmax_tile(float (&w)[NGB][16], float& m2, float& lsum,
                                             const float (&t2)[NGB][16], bool pv) {
  float m = -INFINITY;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, t2[gb][r]);
  m = fmaxf(m, xor32(m));
  float l = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(t2[gb][r] - m);
      w[gb][r] = e;
      l += e;
    }
  l += xor32(l);
  const float inv = 1.f / l;  // correctly rounded (no fast-math)
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) w[gb][r] = pv ? w[gb][r] * inv : 0.f;
  m2 = m;
  lsum = l;
}

// Softmax statistics of one point in the reference layout (B, H, 2, N):
// the row max of the natural-unit logits and the sum of exponentials
// (reference blocked.py:1329-1335). Written by lane h = 0 of each pair.
__device__ __forceinline__ void store_stats(float* stats, int bh, int N, int p, bool pv, int h,
                                            float m2, float l) {
  if (stats && pv && h == 0) {
    float* base = stats + (int64_t)bh * 2 * N;
    base[p] = m2 * kLn2;
    base[N + p] = l;
  }
}

// The softmax Jacobian of one tile given omega = dL/dw: Lb = w (omega -
// delta), delta = sum_g w omega, both from the same rounded products.
// Overwrites om with ab = Lb / tau and returns the row term
// sum_g Lb (t2 - m2) of the temperature gradient (natural units up to a
// factor ln 2; zero on lanes h = 1 and on points beyond N).
template <int NGB>
__device__ __forceinline__ float jacobian_tile(float (&om)[NGB][16], const float (&w)[NGB][16],
                                               const float (&t2)[NGB][16], float m2,
                                               float inv_tau, bool pv, int h) {
  float d = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) d += w[gb][r] * om[gb][r];
  d += xor32(d);
  float rt = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float lb = w[gb][r] * (om[gb][r] - d);
      rt += (w[gb][r] > 0.f) ? lb * (t2[gb][r] - m2) : 0.f;
      om[gb][r] = lb * inv_tau;
    }
  rt += xor32(rt);
  return (pv && h == 0) ? rt : 0.f;
}

#define FS_PROLOGUE                                                     \
  __shared__ float smem[kWavesPerBlock * kLdsTile];                     \
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;           \
  const int c = lane & 31, h = lane >> 5;                               \
  const int bh = blockIdx.y * kWavesPerBlock + wid;                     \
  if (bh >= a.B * a.H) return;                                          \
  const int b = bh / a.H, hd = bh - b * a.H;                           \
  float* lds = smem + wid * kLdsTile;                                   \
  const float* Wp = a.W + b * a.swb + hd * a.swh;                       \
  const float* Bp = a.bias + b * a.sbb + hd * a.sbh;                    \
  const float tauf = a.tau[hd];                                         \
  const float cst = (float)(1.4426950408889634 / (double)tauf);        \
  const float inv_tau = 1.f / tauf;                                     \
  (void)inv_tau; (void)lds;

// ------------------------------------------------------------------ slice fwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, 2) void k_fused_slice_fwd(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  FS_PROLOGUE
  const int G = a.G, D = a.D, DV = a.DV, N = a.N;
  float wA[NGB][NDB][16], bc[NGB][16];
  load_logit_consts<NGB, NDB>(wA, bc, Wp, Bp, cst, G, D, c, h);
  f32x16 zacc[NGB][NVB];
  float sacc[NGB];
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    sacc[gb] = 0.f;
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) zacc[gb][vb] = zero16();
  }
  const T* xb = (const T*)a.x + b * a.sxb + hd * a.sxh;
  const T* fb = (const T*)a.f + b * a.sfb + hd * a.sfh;
  // the next tile's operands are loaded while the current one is computed
  float xn[NDB][16], fn[NVB][16];
  auto load_tile = [&](int t) {
    const int p0 = t * kTile, p = p0 + c;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_rows<T>(xn[db], xb + (int64_t)p * a.sxn, p < N, 32 * db, D, a.vec_x, h);
    // fx as [v-outer, point-inner]: a coalesced row read per register
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int pj = p0 + kmap(j, h), v = 32 * vb + c;
        fn[vb][j] = (pj < N && v < DV) ? to_f<T>(fb[(int64_t)pj * a.sfn + v]) : 0.f;
      }
  };
  if ((int)blockIdx.x < a.ntiles) load_tile(blockIdx.x);
  for (int t = blockIdx.x; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16], fT[NVB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) xf[db][j] = xn[db][j];
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
      for (int j = 0; j < 16; ++j) fT[vb][j] = fn[vb][j];
    if (t + a.P < a.ntiles) load_tile(t + a.P);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    store_stats(a.stats_out, bh, N, p, pv, h, m2, lsum);
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      float wT[16];
      transpose32(wT, w[gb], lds, c, h);
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) zacc[gb][vb] = mma32<MV>(fT[vb], wT, zacc[gb][vb]);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s += wT[j];
      sacc[gb] += s;
    }
  }
  float* pw = a.part + ((int64_t)bh * a.P + blockIdx.x) * part_floats_slice_fwd(G, DV);
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    const int g = 32 * gb + c;
    const float s = sacc[gb] + xor32(sacc[gb]);
    if (g < G) {
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = 32 * vb + kmap(r, h);
          if (v < DV) pw[(int64_t)g * DV + v] = zacc[gb][vb][r];
        }
      if (h == 0) pw[(int64_t)G * DV + g] = s;
    }
  }
}

// ---------------------------------------------------------------- deslice fwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, 2) void k_fused_deslice_fwd(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  FS_PROLOGUE
  const int G = a.G, D = a.D, DV = a.DV, N = a.N;
  float wA[NGB][NDB][16], bc[NGB][16];
  load_logit_consts<NGB, NDB>(wA, bc, Wp, Bp, cst, G, D, c, h);
  const float* Tp = a.tok + (int64_t)bh * G * DV;
  float tC[NVB][NGB][16];  // tokens as [v-outer, g-inner]
#pragma unroll
  for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb)
      load_frag_mat_colouter(tC[vb][gb], Tp, 32 * gb, G, 32 * vb, DV, c, h);
  const T* xb = (const T*)a.x + b * a.sxb + hd * a.sxh;
  T* ob = (T*)a.o1 + b * a.s1b + hd * a.s1h;
  float xn[NDB][16];
  auto load_tile = [&](int t) {
    const int p = t * kTile + c;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_rows<T>(xn[db], xb + (int64_t)p * a.sxn, p < N, 32 * db, D, a.vec_x, h);
  };
  if ((int)blockIdx.x < a.ntiles) load_tile(blockIdx.x);
  for (int t = blockIdx.x; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) xf[db][j] = xn[db][j];
    if (t + a.P < a.ntiles) load_tile(t + a.P);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    store_stats(a.stats_out, bh, N, p, pv, h, m2, lsum);
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) o = mma32<MV>(tC[vb][gb], w[gb], o);
      store_frag_rows<T>(ob + (int64_t)p * a.s1n, o, pv, 32 * vb, DV, a.vec_1, h);
    }
  }
}

// ------------------------------------------------------------------ slice bwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, 2) void k_fused_slice_bwd(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  FS_PROLOGUE
  const int G = a.G, D = a.D, DV = a.DV, N = a.N;
  float wA[NGB][NDB][16], bc[NGB][16];
  load_logit_consts<NGB, NDB>(wA, bc, Wp, Bp, cst, G, D, c, h);
  const float* Zp = a.tok + (int64_t)bh * G * DV;
  const float* Sp = a.ds + (int64_t)bh * G;
  float wC[NDB][NGB][16];   // W as [d-outer, g-inner]
  float zR[NGB][NVB][16];   // dz_num as [g-outer, v-inner]
  float zC[NVB][NGB][16];   // dz_num as [v-outer, g-inner]
  float dsv[NGB][16];       // d s per output slot
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_mat_colouter(wC[db][gb], Wp, 32 * gb, G, 32 * db, D, c, h);
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) {
      load_frag_mat_rowouter(zR[gb][vb], Zp, 32 * gb, G, 32 * vb, DV, c, h);
      load_frag_mat_colouter(zC[vb][gb], Zp, 32 * gb, G, 32 * vb, DV, c, h);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int g = 32 * gb + kmap(r, h);
      dsv[gb][r] = g < G ? Sp[g] : 0.f;
    }
  }
  f32x16 dW[NGB][NDB];
  float dbacc[NGB], dtacc = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    dbacc[gb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) dW[gb][db] = zero16();
  }
  const T* xb = (const T*)a.x + b * a.sxb + hd * a.sxh;
  const T* fb = (const T*)a.f + b * a.sfb + hd * a.sfh;
  T* dxb = (T*)a.o1 + b * a.s1b + hd * a.s1h;
  T* dfb = (T*)a.o2 + b * a.s2b + hd * a.s2h;
  float xn[NDB][16], fnx[NVB][16];
  auto load_tile = [&](int t) {
    const int p = t * kTile + c;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_rows<T>(xn[db], xb + (int64_t)p * a.sxn, p < N, 32 * db, D, a.vec_x, h);
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
      load_frag_rows<T>(fnx[vb], fb + (int64_t)p * a.sfn, p < N, 32 * vb, DV, a.vec_f, h);
  };
  if ((int)blockIdx.x < a.ntiles) load_tile(blockIdx.x);
  for (int t = blockIdx.x; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16], ff[NVB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) xf[db][j] = xn[db][j];
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
      for (int j = 0; j < 16; ++j) ff[vb][j] = fnx[vb][j];
    if (t + a.P < a.ntiles) load_tile(t + a.P);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    // dfx = w dz_num
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) o = mma32<MV>(zC[vb][gb], w[gb], o);
      store_frag_rows<T>(dfb + (int64_t)p * a.s2n, o, pv, 32 * vb, DV, a.vec_2, h);
    }
    // omega = fx . dz_num + ds
    float om[NGB][16];
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      f32x16 o = zero16();
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) o = mma32<MV>(zR[gb][vb], ff[vb], o);
#pragma unroll
      for (int r = 0; r < 16; ++r) om[gb][r] = o[r] + dsv[gb][r];
    }
    dtacc += jacobian_tile<NGB>(om, w, t2, m2, inv_tau, pv, h);
    // dx = ab W
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) o = mma32<MV>(wC[db][gb], om[gb], o);
      store_frag_rows<T>(dxb + (int64_t)p * a.s1n, o, pv, 32 * db, D, a.vec_1, h);
    }
    // dW += ab^T x, db += sum_n ab
    float xT[NDB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db) transpose32(xT[db], xf[db], lds, c, h);
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      float aT[16];
      transpose32(aT, om[gb], lds, c, h);
#pragma unroll
      for (int db = 0; db < NDB; ++db) dW[gb][db] = mma32<MV>(xT[db], aT, dW[gb][db]);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s += aT[j];
      dbacc[gb] += s;
    }
  }
  float* pw = a.part + ((int64_t)bh * a.P + blockIdx.x) * part_floats_slice_bwd(G, D);
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    const int g = 32 * gb + c;
    const float s = dbacc[gb] + xor32(dbacc[gb]);
    if (g < G) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = 32 * db + kmap(r, h);
          if (d < D) pw[(int64_t)g * D + d] = dW[gb][db][r];
        }
      if (h == 0) pw[(int64_t)G * D + g] = s;
    }
  }
  const float dt = half_wave_sum(dtacc);
  if (lane == 0) pw[(int64_t)G * D + G] = -kLn2 * inv_tau * dt;
}

// ---------------------------------------------------------------- deslice bwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, 2) void k_fused_deslice_bwd(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  FS_PROLOGUE
  const int G = a.G, D = a.D, DV = a.DV, N = a.N;
  float wA[NGB][NDB][16], bc[NGB][16];
  load_logit_consts<NGB, NDB>(wA, bc, Wp, Bp, cst, G, D, c, h);
  const float* Tp = a.tok + (int64_t)bh * G * DV;
  float wC[NDB][NGB][16];   // W as [d-outer, g-inner]
  float tR[NGB][NVB][16];   // tokens as [g-outer, v-inner]
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_mat_colouter(wC[db][gb], Wp, 32 * gb, G, 32 * db, D, c, h);
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
      load_frag_mat_rowouter(tR[gb][vb], Tp, 32 * gb, G, 32 * vb, DV, c, h);
  }
  f32x16 dT[NGB][NVB], dW[NGB][NDB];
  float dbacc[NGB], dtacc = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    dbacc[gb] = 0.f;
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) dT[gb][vb] = zero16();
#pragma unroll
    for (int db = 0; db < NDB; ++db) dW[gb][db] = zero16();
  }
  const T* xb = (const T*)a.x + b * a.sxb + hd * a.sxh;
  const T* ob = (const T*)a.f + b * a.sfb + hd * a.sfh;
  T* dxb = (T*)a.o1 + b * a.s1b + hd * a.s1h;
  float xn[NDB][16], fnx[NVB][16];
  auto load_tile = [&](int t) {
    const int p = t * kTile + c;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      load_frag_rows<T>(xn[db], xb + (int64_t)p * a.sxn, p < N, 32 * db, D, a.vec_x, h);
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
      load_frag_rows<T>(fnx[vb], ob + (int64_t)p * a.sfn, p < N, 32 * vb, DV, a.vec_f, h);
  };
  if ((int)blockIdx.x < a.ntiles) load_tile(blockIdx.x);
  for (int t = blockIdx.x; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16], of[NVB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) xf[db][j] = xn[db][j];
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
      for (int j = 0; j < 16; ++j) of[vb][j] = fnx[vb][j];
    if (t + a.P < a.ntiles) load_tile(t + a.P);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    // dtokens += w^T d_out
    float oT[NVB][16];
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) transpose32(oT[vb], of[vb], lds, c, h);
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      float wT[16];
      transpose32(wT, w[gb], lds, c, h);
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) dT[gb][vb] = mma32<MV>(oT[vb], wT, dT[gb][vb]);
    }
    // omega = d_out . tokens
    float om[NGB][16];
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      f32x16 o = zero16();
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) o = mma32<MV>(tR[gb][vb], of[vb], o);
      from16(om[gb], o);
    }
    dtacc += jacobian_tile<NGB>(om, w, t2, m2, inv_tau, pv, h);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) o = mma32<MV>(wC[db][gb], om[gb], o);
      store_frag_rows<T>(dxb + (int64_t)p * a.s1n, o, pv, 32 * db, D, a.vec_1, h);
    }
    float xT[NDB][16];
#pragma unroll
    for (int db = 0; db < NDB; ++db) transpose32(xT[db], xf[db], lds, c, h);
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      float aT[16];
      transpose32(aT, om[gb], lds, c, h);
#pragma unroll
      for (int db = 0; db < NDB; ++db) dW[gb][db] = mma32<MV>(xT[db], aT, dW[gb][db]);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s += aT[j];
      dbacc[gb] += s;
    }
  }
  float* pw = a.part + ((int64_t)bh * a.P + blockIdx.x) * part_floats_deslice_bwd(G, D, DV);
  const int64_t offW = (int64_t)G * DV, offB = offW + (int64_t)G * D;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    const int g = 32 * gb + c;
    const float s = dbacc[gb] + xor32(dbacc[gb]);
    if (g < G) {
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = 32 * vb + kmap(r, h);
          if (v < DV) pw[(int64_t)g * DV + v] = dT[gb][vb][r];
        }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = 32 * db + kmap(r, h);
          if (d < D) pw[offW + (int64_t)g * D + d] = dW[gb][db][r];
        }
      if (h == 0) pw[offB + g] = s;
    }
  }
  const float dt = half_wave_sum(dtacc);
  if (lane == 0) pw[offB + G] = -kLn2 * inv_tau * dt;
}

// ------------------------------------------------------------ launch templates
// (NGB, NDB, NVB): slot, logits-width and value-width blocks of 32 held in
// registers; the fused family serves shapes whose slot-indexed accumulators
// fit (NGB * NDB <= 4 and NGB * NVB <= 4).
#define FS_COMBOS(X) \
  X(1, 1, 1) X(1, 1, 2) X(1, 1, 4) X(1, 2, 1) X(1, 2, 2) X(1, 2, 4) X(1, 4, 1) X(1, 4, 2) \
  X(1, 4, 4) X(2, 1, 1) X(2, 1, 2) X(2, 2, 1) X(2, 2, 2) X(4, 1, 1)

enum FusedKind { FK_SLICE_FWD = 0, FK_DESLICE_FWD = 1, FK_SLICE_BWD = 2, FK_DESLICE_BWD = 3 };

__host__ inline int blocks_of(int n) {
  const int k = (n + 31) / 32;
  return k <= 1 ? 1 : k <= 2 ? 2 : k <= 4 ? 4 : 8;
}

// Launch the fused kernel of kind K for point dtype T and dot kind DK.
// Explicitly instantiated in the generated translation units (build.py),
// one per (K, T, DK), so they compile in parallel.
template <int K, typename T, int DK>
hipError_t fused_launch(const Args& a, hipStream_t st) {
  const int g = blocks_of(a.G), d = blocks_of(a.D), v = blocks_of(a.DV);
  const dim3 grid(a.P, (a.B * a.H + kWavesPerBlock - 1) / kWavesPerBlock), block(256);
#define FS_TRY(G_, D_, V_)                                                                    \
  if (g == G_ && d == D_ && v == V_) {                                                        \
    if constexpr (K == FK_SLICE_FWD)                                                          \
      hipLaunchKernelGGL((k_fused_slice_fwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);      \
    else if constexpr (K == FK_DESLICE_FWD)                                                   \
      hipLaunchKernelGGL((k_fused_deslice_fwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);    \
    else if constexpr (K == FK_SLICE_BWD)                                                     \
      hipLaunchKernelGGL((k_fused_slice_bwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);      \
    else                                                                                      \
      hipLaunchKernelGGL((k_fused_deslice_bwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);    \
    return hipGetLastError();                                                                 \
  }
  FS_COMBOS(FS_TRY)
#undef FS_TRY
  return hipErrorNotSupported;
}

#define FS_FUSED_INSTANCES(X)                                                        \
  X(0, float, 0) X(0, __bf16, 0) X(0, __bf16, 1) X(0, __bf16, 2) X(0, _Float16, 0)   \
  X(0, _Float16, 1) X(0, _Float16, 2)                                                \
  X(1, float, 0) X(1, __bf16, 0) X(1, __bf16, 1) X(1, __bf16, 2) X(1, _Float16, 0)   \
  X(1, _Float16, 1) X(1, _Float16, 2)                                                \
  X(2, float, 0) X(2, __bf16, 0) X(2, __bf16, 1) X(2, __bf16, 2) X(2, _Float16, 0)   \
  X(2, _Float16, 1) X(2, _Float16, 2)                                                \
  X(3, float, 0) X(3, __bf16, 0) X(3, __bf16, 1) X(3, __bf16, 2) X(3, _Float16, 0)   \
  X(3, _Float16, 1) X(3, _Float16, 2)

#define FS_DECLARE_EXTERN(K_, T_, DK_) \
  extern template hipError_t fused_launch<K_, T_, DK_>(const Args&, hipStream_t);
FS_FUSED_INSTANCES(FS_DECLARE_EXTERN)
#undef FS_DECLARE_EXTERN

}  // namespace fs
