// G-blocked slice/deslice kernel templates for gfx950: any slot count G,
// head widths D, DV up to 256.
//
// When the slot axis does not fit in registers, the softmax over G is
// carried by per-point statistics (m, l) -- the row max of the logits and
// the sum of exponentials against it, (B, H, 2, N) fp32 -- and the work is
// split two ways (the structure of reference blocked.py:1-66):
//   * point-owned kernels ("_n") own a 32-point tile and loop over G in
//     blocks of 32 slots: the statistics pass, the deslice forward (from
//     saved statistics, or online -- FlashAttention's rescaled accumulator --
//     emitting them), and the two point-indexed backward passes (dfx, the
//     Jacobian row term delta, dx and the per-row temperature term);
//   * slot-owned kernels ("_g") own one 32-slot block (grid z) and stream
//     points: z_num / s partials, and the dW / db / dtokens partials of the
//     backward, which need delta from the point-owned pass.
// Every dot runs on MFMA with the fragment convention of fs_device.h; the
// slot-block operands (W, tokens, dz_num rows) are read from global memory
// (they are small and stay in L2). Per-wave partials are reduced in a fixed
// order by fs_reduce.hip, so results are bitwise reproducible.
//
// Reference kernels these replace: _stats_kernel / _stats_twopass_kernel
// (blocked.py:292-400), _slice_fwd_g_kernel (:403-462), _deslice_fwd_n_kernel
// (:465-510), _deslice_fwd_online_kernel (:513-573), _slice_bwd_n_kernel
// (:576-673), _slice_bwd_g_kernel (:676-741), _deslice_bwd_n_kernel
// (:744-815), _deslice_bwd_g_kernel (:818-888).
#pragma once
#include "fs_gp_kernels.h"
#include "fs_tile.h"

namespace fs {

// A 32 x C block of a small fp32 matrix M (rows g, row stride C) as NB
// fragments: [g-outer, col-inner] or [col-outer, g-inner]; blocks k >= nc
// and entries outside (G, C) are zero.
template <int NB>
__device__ __forceinline__ void blk_rowouter(float (&f)[NB][16], const float* M, int g0, int G,
                                             int C, int nc, int c, int h) {
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    if (k < nc) {
      load_frag_mat_rowouter(f[k], M, g0, G, 32 * k, C, c, h);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) f[k][j] = 0.f;
    }
  }
}
template <int NB>
__device__ __forceinline__ void blk_colouter(float (&f)[NB][16], const float* M, int g0, int G,
                                             int C, int nc, int c, int h) {
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    if (k < nc) {
      load_frag_mat_colouter(f[k], M, g0, G, 32 * k, C, c, h);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) f[k][j] = 0.f;
    }
  }
}

// bias * log2(e) / tau of the 32 output slots of a block (kNoSlot beyond G)
__device__ __forceinline__ void blk_bias(float (&bc)[16], const float* Bp, int g0, int G,
                                         float cst, int h) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int g = g0 + kmap(r, h);
    bc[r] = g < G ? Bp[g] * cst : kNoSlot;
  }
}

// per output slot of a block: a small fp32 vector (zero beyond G)
__device__ __forceinline__ void blk_vec(float (&v)[16], const float* V, int g0, int G, int h) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int g = g0 + kmap(r, h);
    v[r] = g < G ? V[g] : 0.f;
  }
}

// scaled logits of one slot block: t2 = (x . W_blk + b) log2(e) / tau
template <int ML, int NB>
__device__ __forceinline__ void blk_logits(float (&t2)[16], const float (&wA)[NB][16],
                                           const float (&xf)[NB][16], const float (&bc)[16],
                                           float cst, int nd) {
  f32x16 s = zero16();
#pragma unroll
  for (int k = 0; k < NB; ++k)
    if (k < nd) s = mma32<ML>(wA[k], xf[k], s);
#pragma unroll
  for (int r = 0; r < 16; ++r) t2[r] = fmaf(s[r], cst, bc[r]);
}

// point rows of a tile: NB fragments, blocks beyond nc zero
template <typename T, int NB>
__device__ __forceinline__ void load_rows_nb(float (&f)[NB][16], const T* base, int64_t sn, int p,
                                             int N, int C, int nc, bool fast, bool vec, int h) {
  const T* row = base + (int64_t)(fast ? (p < N ? p : N - 1) : p) * sn;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    if (k < nc) {
      if (fast)
        load_frag_rows_fast<T>(f[k], row, 32 * k, h);
      else
        load_frag_rows<T>(f[k], row, p < N, 32 * k, C, vec, h);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) f[k][j] = 0.f;
    }
  }
}

// saved statistics of point p (clamped to N - 1: finite for padded points,
// whose results are masked): m in log2 units and l
// (`sm`: this sample and head's max row, Rows::stats_off; its sum row NS
// floats further)
__device__ __forceinline__ void load_stats(float& m2, float& l, const float* sm, int64_t NS,
                                           int N, int p) {
  const int q = p < N ? p : N - 1;
  m2 = sm[q] * kLog2e;
  l = sm[NS + q];
}

// a per-point fp32 value of this sample and head's row `row` (Rows::pt_off;
// clamped like load_stats)
__device__ __forceinline__ float load_delta(const float* row, int N, int p) {
  return row[p < N ? p : N - 1];
}

#define BK_PROLOGUE                                                          \
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;                \
  const int c = lane & 31, h = lane >> 5;                                    \
  const int bh = blockIdx.y;                                                 \
  const int b = bh / a.H, hd = bh - b * a.H;                                \
  const int pid = blockIdx.x * kWavesPerBlock + wid;                         \
  const int G = a.G, D = a.D, DV = a.DV, nd = a.nd, nv = a.nv;               \
  /* this sample's rows (row splits of a ragged batch) and per-point buffers */ \
  const Rows R_ = rows_of(a, b, hd);                                         \
  const int64_t row0_ = R_.row0;                                             \
  const int N = R_.N, ntiles_ = R_.ntiles;                                   \
  const float* Wp = a.W + b * a.swb + hd * a.swh;                            \
  const float* Bp = a.bias + b * a.sbb + hd * a.sbh;                         \
  const float tauf = a.tau[hd];                                              \
  const float cst = (float)(1.4426950408889634 / (double)tauf);             \
  const float inv_tau = 1.f / tauf;                                          \
  const bool fast = a.fast != 0;                                             \
  const int ngt = (G + 31) / 32;                                             \
  (void)inv_tau; (void)DV; (void)nv; (void)ngt; (void)fast; (void)row0_;

// ------------------------------------------------------------------ stats (n)
template <typename T, int DK, int NB>
__global__ __launch_bounds__(256, 2) void k_blk_stats(Args a) {
  constexpr int ML = Modes<DK>::L;
  BK_PROLOGUE
  const T* xb = (const T*)a.x + b * a.sxb + row0_ * a.sxn + hd * a.sxh;
  for (int t = pid; t < ntiles_; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NB][16];
    load_rows_nb<T, NB>(xf, xb, a.sxn, p, N, D, nd, fast, a.vec_x, h);
    float m = -INFINITY, l = 0.f;
    if (a.two_pass) {
      // max over every slot block, then the sum against the final max
      for (int gb = 0; gb < ngt; ++gb) {
        float wA[NB][16], bc[16], t2[16];
        blk_rowouter<NB>(wA, Wp, 32 * gb, G, D, nd, c, h);
        blk_bias(bc, Bp, 32 * gb, G, cst, h);
        blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, t2[r]);
      }
      // the sum against the max exactly as consumers read it back
      m = fmaxf(m, xor32(m));
      const float mc = stats_max_roundtrip(m);
      for (int gb = 0; gb < ngt; ++gb) {
        float wA[NB][16], bc[16], t2[16];
        blk_rowouter<NB>(wA, Wp, 32 * gb, G, D, nd, c, h);
        blk_bias(bc, Bp, 32 * gb, G, cst, h);
        blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
#pragma unroll
        for (int r = 0; r < 16; ++r) l += __builtin_amdgcn_exp2f(t2[r] - mc);
      }
      l += xor32(l);
    } else {
      // online over slot blocks on this lane's 16 slots of each block, then
      // one combine with the partner lane (commutative: both lanes agree)
      for (int gb = 0; gb < ngt; ++gb) {
        float wA[NB][16], bc[16], t2[16];
        blk_rowouter<NB>(wA, Wp, 32 * gb, G, D, nd, c, h);
        blk_bias(bc, Bp, 32 * gb, G, cst, h);
        blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
        float mb = m;
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = fmaxf(mb, t2[r]);
        float sb = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) sb += __builtin_amdgcn_exp2f(t2[r] - mb);
        l = l * __builtin_amdgcn_exp2f(m - mb) + sb;
        m = mb;
      }
      const float mo = xor32(m), lo = xor32(l);
      const float mm = fmaxf(m, mo);
      l = l * __builtin_amdgcn_exp2f(m - mm) + lo * __builtin_amdgcn_exp2f(mo - mm);
      m = mm;
    }
    store_stats(a.stats_out ? a.stats_out + R_.stats_off() : nullptr, R_.NS, p, pv, h, m, l,
                a.two_pass != 0);
  }
}

// ---------------------------------------------------------------- deslice (n)
// ONLINE: no statistics in hand -- rescale the accumulator and the row sum
// whenever the row max moves, and emit (m, l) (reference blocked.py:513-573).
// Otherwise normalise with the saved statistics (blocked.py:465-510).
template <typename T, int DK, int NB, bool ONLINE>
__global__ __launch_bounds__(256, 2) void k_blk_deslice(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  __shared__ float smem_rows[kWavesPerBlock * 32];
  BK_PROLOGUE
  float* lds_x = smem_rows + wid * 32;
  const T* xb = (const T*)a.x + b * a.sxb + row0_ * a.sxn + hd * a.sxh;
  T* ob = (T*)a.o1 + b * a.s1b + row0_ * a.s1n + hd * a.s1h;
  const float* Tp = a.tok + (int64_t)bh * G * DV;
  for (int t = pid; t < ntiles_; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NB][16];
    load_rows_nb<T, NB>(xf, xb, a.sxn, p, N, D, nd, fast, a.vec_x, h);
    // with saved statistics the row is normalised by the sum of the very
    // exponentials it accumulates (formed here, lane-local then the partner),
    // so each row of weights sums to one to one summation's precision
    float m2 = -INFINITY, l = 0.f, lown = 0.f;
    if (!ONLINE) load_stats(m2, l, a.stats_in + R_.stats_off(), R_.NS, N, p);
    f32x16 acc[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) acc[k] = zero16();
    for (int gb = 0; gb < ngt; ++gb) {
      float wA[NB][16], bc[16], t2[16];
      blk_rowouter<NB>(wA, Wp, 32 * gb, G, D, nd, c, h);
      blk_bias(bc, Bp, 32 * gb, G, cst, h);
      blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
      float e[16];
      if (ONLINE) {
        float mb = m2;
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = fmaxf(mb, t2[r]);
        mb = fmaxf(mb, xor32(mb));
        const float alpha = __builtin_amdgcn_exp2f(m2 - mb);
        float sb = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          e[r] = __builtin_amdgcn_exp2f(t2[r] - mb);
          sb += e[r];
        }
        sb += xor32(sb);
        l = l * alpha + sb;
        m2 = mb;
        // acc is [v-outer, point-inner]: rescale register r by its point's alpha
        float alpha_r[16];
        gather_rows(alpha_r, alpha, lds_x, c, h);
#pragma unroll
        for (int k = 0; k < NB; ++k)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[k][r] *= alpha_r[r];
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          e[r] = __builtin_amdgcn_exp2f(t2[r] - m2);
          lown += e[r];
        }
      }
      float tc[NB][16];
      blk_colouter<NB>(tc, Tp, 32 * gb, G, DV, nv, c, h);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nv) acc[k] = mma32<MV>(e, tc[k], acc[k]);
    }
    if (!ONLINE) l = lown + xor32(lown);
    // acc is [v-outer, point-inner]: point kmap(r, h)'s row sum lives on the
    // lanes holding that point, so gather it by register from the pair
    const float inv_l = 1.f / l;
    float inv_r[16];
    gather_rows(inv_r, inv_l, lds_x, c, h);
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nv) {
        f32x16 o = acc[k];
#pragma unroll
        for (int r = 0; r < 16; ++r) o[r] *= inv_r[r];
        store_cols<T>(ob, a.s1n, o, t * kTile, N, 32 * k, DV, c, h);
      }
    if (ONLINE)
      store_stats(a.stats_out ? a.stats_out + R_.stats_off() : nullptr, R_.NS, p, pv, h, m2, l);
  }
}

// ------------------------------------------------------------------ slice (g)
template <typename T, int DK, int NB>
__global__ __launch_bounds__(256, 2) void k_blk_slice_g(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  __shared__ float smem[kWavesPerBlock * kLdsTile];
  BK_PROLOGUE
  float* lds = smem + wid * kLdsTile;
  const int g0 = 32 * blockIdx.z;
  float wA[NB][16], bc[16];
  blk_rowouter<NB>(wA, Wp, g0, G, D, nd, c, h);
  blk_bias(bc, Bp, g0, G, cst, h);
  f32x16 zacc[NB];
  float sacc = 0.f;
#pragma unroll
  for (int k = 0; k < NB; ++k) zacc[k] = zero16();
  const T* xb = (const T*)a.x + b * a.sxb + row0_ * a.sxn + hd * a.sxh;
  const T* fb = (const T*)a.f + b * a.sfb + row0_ * a.sfn + hd * a.sfh;
  for (int t = pid, it = 0; t < ntiles_; t += a.P, ++it) {
    const int p0 = t * kTile, p = p0 + c;
    const bool pv = p < N;
    float xf[NB][16];
    load_rows_nb<T, NB>(xf, xb, a.sxn, p, N, D, nd, fast, a.vec_x, h);
    float fT[NB][16];  // fx as [v-outer, point-inner]
#pragma unroll
    for (int k = 0; k < NB; ++k)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int pj = p0 + kmap(j, h), v = 32 * k + c;
        fT[k][j] = (k < nv && pj < N && v < DV) ? to_f<T>(fb[(int64_t)pj * a.sfn + v]) : 0.f;
      }
    float m2, l;
    load_stats(m2, l, a.stats_in + R_.stats_off(), R_.NS, N, p);
    float t2[16], w[16];
    blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
    const float sg = tile_sign(it);  // the weights carry the tile's sign (acc_add)
    const float inv_l = pv ? sg / l : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) w[r] = __builtin_amdgcn_exp2f(t2[r] - m2) * inv_l;
    float wT[16];
    transpose32(wT, w, lds, c, h);
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nv) mma32_acc<MV>(zacc[k], fT[k], wT, sg);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += wT[j];
    sacc = fmaf(s, sg, sacc);
  }
  float* pw = a.part + ((int64_t)bh * a.P + pid) * part_floats_slice_fwd(G, DV);
  const int g = g0 + c;
  const float s = sacc + xor32(sacc);
  if (g < G) {
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nv)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = 32 * k + kmap(r, h);
          if (v < DV) pw[(int64_t)g * DV + v] = zacc[k][r];
        }
    if (h == 0) pw[(int64_t)G * DV + g] = s;
  }
}

// ---------------------------------------------------- slice / deslice bwd (n)
// Point-owned backward (reference blocked.py:576-673, :744-815). Pass 1 over
// the slot blocks: the Jacobian numerator sum_g e omega (and, for the slice,
// dfx = e dz_num), divided by l once. Pass 2: dl = e (omega - delta) / l (the
// difference first, as in the G-blocked kernels), dx += dl W, and the row term
// sum_g dl (t2 - m2) of the temperature gradient, formed row by row over
// all of G before anything is added across rows.
// SLICE: omega = fx . dz_num + ds, also writes dfx; else omega = d_out . T.
template <typename T, int DK, int NB, bool SLICE>
__global__ __launch_bounds__(256, 2) void k_blk_bwd_n(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  __shared__ float smem_rows[kWavesPerBlock * 32];
  BK_PROLOGUE
  float* lds_x = smem_rows + wid * 32;
  const T* xb = (const T*)a.x + b * a.sxb + row0_ * a.sxn + hd * a.sxh;
  const T* fb = (const T*)a.f + b * a.sfb + row0_ * a.sfn + hd * a.sfh;
  T* dxb = (T*)a.o1 + b * a.s1b + row0_ * a.s1n + hd * a.s1h;
  T* dfb = SLICE ? (T*)a.o2 + b * a.s2b + row0_ * a.s2n + hd * a.s2h : nullptr;
  const float* Zp = a.tok + (int64_t)bh * G * DV;  // dz_num (slice) or tokens (deslice)
  const float* Sp = SLICE ? a.ds + (int64_t)bh * G : nullptr;
  float dtacc = 0.f;
  for (int t = pid; t < ntiles_; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NB][16], ff[NB][16];
    load_rows_nb<T, NB>(xf, xb, a.sxn, p, N, D, nd, fast, a.vec_x, h);
    load_rows_nb<T, NB>(ff, fb, a.sfn, p, N, DV, nv, fast, a.vec_f, h);
    float m2, lsaved;
    load_stats(m2, lsaved, a.stats_in + R_.stats_off(), R_.NS, N, p);
    (void)lsaved;
    // pass 1: the row sum l is formed here from the same exponentials, so
    // sum_g dl vanishes to one summation's precision whatever rounding the
    // saved sum carries; it is handed to the slot-owned pass
    f32x16 dfacc[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) dfacc[k] = zero16();
    float sdw = 0.f, lown = 0.f;
    for (int gb = 0; gb < ngt; ++gb) {
      float wA[NB][16], bc[16], t2[16], e[16];
      blk_rowouter<NB>(wA, Wp, 32 * gb, G, D, nd, c, h);
      blk_bias(bc, Bp, 32 * gb, G, cst, h);
      blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
      float lb = 0.f;  // per slot block, then across blocks
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        e[r] = __builtin_amdgcn_exp2f(t2[r] - m2);
        lb += e[r];
      }
      lown += lb;
      if (SLICE) {
        float zc[NB][16];
        blk_colouter<NB>(zc, Zp, 32 * gb, G, DV, nv, c, h);
#pragma unroll
        for (int k = 0; k < NB; ++k)
          if (k < nv) dfacc[k] = mma32<MV>(e, zc[k], dfacc[k]);
      }
      float zr[NB][16];
      blk_rowouter<NB>(zr, Zp, 32 * gb, G, DV, nv, c, h);
      f32x16 o = zero16();
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nv) o = mma32<MV>(zr[k], ff[k], o);
      float dsv[16];
      if (SLICE) blk_vec(dsv, Sp, 32 * gb, G, h);
      float sb = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) sb = fmaf(e[r], SLICE ? o[r] + dsv[r] : o[r], sb);
      sdw += sb;
    }
    sdw += xor32(sdw);
    const float l = lown + xor32(lown);
    const float inv_l = 1.f / l;
    const float delta = sdw * inv_l;
    if (pv && h == 0) {
      a.delta[R_.pt_off() + p] = delta;
      a.lsum[R_.pt_off() + p] = l;
    }
    if (SLICE) {
      // dfx is [v-outer, point-inner]: scale register r by its point's 1/l
      float inv_r[16];
      gather_rows(inv_r, inv_l, lds_x, c, h);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nv) {
          f32x16 o = dfacc[k];
#pragma unroll
          for (int r = 0; r < 16; ++r) o[r] *= inv_r[r];
          store_cols<T>(dfb, a.s2n, o, t * kTile, N, 32 * k, DV, c, h);
        }
    }
    // pass 2
    f32x16 dxacc[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) dxacc[k] = zero16();
    float rt = 0.f;
    for (int gb = 0; gb < ngt; ++gb) {
      float wA[NB][16], bc[16], t2[16];
      blk_rowouter<NB>(wA, Wp, 32 * gb, G, D, nd, c, h);
      blk_bias(bc, Bp, 32 * gb, G, cst, h);
      blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
      float zr[NB][16];
      blk_rowouter<NB>(zr, Zp, 32 * gb, G, DV, nv, c, h);
      f32x16 o = zero16();
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nv) o = mma32<MV>(zr[k], ff[k], o);
      float dsv[16];
      if (SLICE) blk_vec(dsv, Sp, 32 * gb, G, h);
      float dl[16], rb = 0.f;  // row term per slot block, then across blocks
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = __builtin_amdgcn_exp2f(t2[r] - m2);
        const float om = SLICE ? o[r] + dsv[r] : o[r];
        dl[r] = e * (om - delta) * inv_l;
        rb = fmaf(dl[r], t2[r] - m2, rb);
      }
      rt += rb;
      float wc[NB][16];
      blk_colouter<NB>(wc, Wp, 32 * gb, G, D, nd, c, h);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nd) dxacc[k] = mma32<MV>(dl, wc[k], dxacc[k]);
    }
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nd) {
        f32x16 o = dxacc[k];
#pragma unroll
        for (int r = 0; r < 16; ++r) o[r] *= inv_tau;
        store_cols<T>(dxb, a.s1n, o, t * kTile, N, 32 * k, D, c, h);
      }
    rt += xor32(rt);
    dtacc += (pv && h == 0) ? rt : 0.f;
  }
  const float dt = half_wave_sum(dtacc);
  if (lane == 0) a.part2[(int64_t)bh * a.P + pid] = -kLn2 * inv_tau * dt;
}

// --------------------------------------------------- slice / deslice bwd (g)
// Slot-owned backward (reference blocked.py:676-741, :818-888): one 32-slot
// block, streaming points with the saved statistics and delta.
// SLICE: dW, db partials (omega = fx . dz_num + ds); else also dtokens
// (omega = d_out . T).
template <typename T, int DK, int NB, bool SLICE>
__global__ __launch_bounds__(256, 2) void k_blk_bwd_g(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  __shared__ float smem[kWavesPerBlock * kLdsTile];
  BK_PROLOGUE
  float* lds = smem + wid * kLdsTile;
  const int g0 = 32 * blockIdx.z;
  const float* Zp = a.tok + (int64_t)bh * G * DV;
  float wA[NB][16], bc[16], zr[NB][16], dsv[16];
  blk_rowouter<NB>(wA, Wp, g0, G, D, nd, c, h);
  blk_bias(bc, Bp, g0, G, cst, h);
  blk_rowouter<NB>(zr, Zp, g0, G, DV, nv, c, h);
  if (SLICE)
    blk_vec(dsv, a.ds + (int64_t)bh * G, g0, G, h);
  else
#pragma unroll
    for (int r = 0; r < 16; ++r) dsv[r] = 0.f;
  f32x16 dW[NB], dT[NB];
  float dbacc = 0.f;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    dW[k] = zero16();
    dT[k] = zero16();
  }
  const T* xb = (const T*)a.x + b * a.sxb + row0_ * a.sxn + hd * a.sxh;
  const T* fb = (const T*)a.f + b * a.sfb + row0_ * a.sfn + hd * a.sfh;
  for (int t = pid, it = 0; t < ntiles_; t += a.P, ++it) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NB][16], ff[NB][16];
    load_rows_nb<T, NB>(xf, xb, a.sxn, p, N, D, nd, fast, a.vec_x, h);
    load_rows_nb<T, NB>(ff, fb, a.sfn, p, N, DV, nv, fast, a.vec_f, h);
    float m2, l;
    load_stats(m2, l, a.stats_in + R_.stats_off(), R_.NS, N, p);
    l = load_delta(a.lsum + R_.pt_off(), N, p);  // the row sum the point-owned pass formed
    const float delta = load_delta(a.delta + R_.pt_off(), N, p);
    float t2[16], w[16];
    blk_logits<ML, NB>(t2, wA, xf, bc, cst, nd);
    // the weights -- and through them Lb -- carry the tile's sign (acc_add)
    const float sg = tile_sign(it);
    const float inv_l = pv ? sg / l : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) w[r] = __builtin_amdgcn_exp2f(t2[r] - m2) * inv_l;
    if (!SLICE) {
      // dtokens += w^T d_out
      float wT[16];
      transpose32(wT, w, lds, c, h);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nv) {
          float oT[16];
          transpose32(oT, ff[k], lds, c, h);
          mma32_acc<MV>(dT[k], oT, wT, sg);
        }
    }
    f32x16 o = zero16();
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nv) o = mma32<MV>(zr[k], ff[k], o);
    float ab[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ab[r] = w[r] * (o[r] + dsv[r] - delta) * inv_tau;
    float aT[16];
    transpose32(aT, ab, lds, c, h);
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nd) {
        float xT[16];
        transpose32(xT, xf[k], lds, c, h);
        mma32_acc<MV>(dW[k], xT, aT, sg);
      }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += aT[j];
    dbacc = fmaf(s, sg, dbacc);
  }
  const int g = g0 + c;
  const float s = dbacc + xor32(dbacc);
  if (g < G) {
    if (SLICE) {
      float* pw = a.part + ((int64_t)bh * a.P + pid) * part_floats_slice_bwd(G, D);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k < nd)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * k + kmap(r, h);
            if (d < D) pw[(int64_t)g * D + d] = dW[k][r];
          }
      if (h == 0) pw[(int64_t)G * D + g] = s;
    } else {
      float* pw = a.part + ((int64_t)bh * a.P + pid) * part_floats_deslice_bwd(G, D, DV);
      const int64_t offW = (int64_t)G * DV, offB = offW + (int64_t)G * D;
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        if (k < nv)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = 32 * k + kmap(r, h);
            if (v < DV) pw[(int64_t)g * DV + v] = dT[k][r];
          }
        if (k < nd)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * k + kmap(r, h);
            if (d < D) pw[offW + (int64_t)g * D + d] = dW[k][r];
          }
      }
      if (h == 0) pw[offB + g] = s;
    }
  }
}

// ---------------------------------------------------------------- launching
// NB: 32-wide blocks held per point row for D and DV together. One or two
// (D, DV <= 64) go to the prepared-fragment kernels of fs_gp_kernels.h; the
// kernels of this file serve four and eight.
template <int K, typename T, int DK>
hipError_t blocked_launch(const Args& a, hipStream_t st) {
  const int nb = a.nd > a.nv ? a.nd : a.nv;
  const int NBc = nb <= 1 ? 1 : nb <= 2 ? 2 : nb <= 4 ? 4 : 8;
  const int bh = a.B * a.H;
  const dim3 gn(a.P / kWavesPerBlock, bh), gg(a.P / kWavesPerBlock, bh, (a.G + 31) / 32);
  const dim3 blk(256);
  if (gp_serves(a.D, a.DV)) {
    // prepared-fragment kernels (fs_gp_kernels.h); slot-owned grids run the
    // slot blocks fastest
    const dim3 gq((a.G + 31) / 32, a.P / kWavesPerBlock, bh);
#define GP_TRY(NB_)                                                                            \
    if (NBc == NB_) {                                                                          \
      if constexpr (K == BK_STATS)                                                             \
        hipLaunchKernelGGL((k_gp_stats<T, DK, NB_>), gn, blk, 0, st, a);                       \
      else if constexpr (K == BK_DESLICE_N)                                                    \
        hipLaunchKernelGGL((k_gp_deslice<T, DK, NB_, false>), gn, blk, 0, st, a);              \
      else if constexpr (K == BK_DESLICE_ONLINE)                                               \
        hipLaunchKernelGGL((k_gp_deslice<T, DK, NB_, true>), gn, blk, 0, st, a);               \
      else if constexpr (K == BK_SLICE_G)                                                      \
        hipLaunchKernelGGL((k_gp_slice_g<T, DK, NB_>), gq, blk, 0, st, a);                     \
      else if constexpr (K == BK_SLICE_BWD_N)                                                  \
        hipLaunchKernelGGL((k_gp_bwd_n<T, DK, NB_, true>), gn, blk, 0, st, a);                 \
      else if constexpr (K == BK_SLICE_BWD_G)                                                  \
        hipLaunchKernelGGL((k_gp_bwd_g<T, DK, NB_, true>), gq, blk, 0, st, a);                 \
      else if constexpr (K == BK_DESLICE_BWD_N)                                                \
        hipLaunchKernelGGL((k_gp_bwd_n<T, DK, NB_, false>), gn, blk, 0, st, a);                \
      else                                                                                     \
        hipLaunchKernelGGL((k_gp_bwd_g<T, DK, NB_, false>), gq, blk, 0, st, a);                \
      return hipGetLastError();                                                                \
    }
    GP_TRY(1) GP_TRY(2)
#undef GP_TRY
    return hipErrorNotSupported;
  }
#define BK_TRY(NB_)                                                                            \
  if (NBc == NB_) {                                                                            \
    if constexpr (K == BK_STATS)                                                               \
      hipLaunchKernelGGL((k_blk_stats<T, DK, NB_>), gn, blk, 0, st, a);                        \
    else if constexpr (K == BK_DESLICE_N)                                                      \
      hipLaunchKernelGGL((k_blk_deslice<T, DK, NB_, false>), gn, blk, 0, st, a);               \
    else if constexpr (K == BK_DESLICE_ONLINE)                                                 \
      hipLaunchKernelGGL((k_blk_deslice<T, DK, NB_, true>), gn, blk, 0, st, a);                \
    else if constexpr (K == BK_SLICE_G)                                                        \
      hipLaunchKernelGGL((k_blk_slice_g<T, DK, NB_>), gg, blk, 0, st, a);                      \
    else if constexpr (K == BK_SLICE_BWD_N)                                                    \
      hipLaunchKernelGGL((k_blk_bwd_n<T, DK, NB_, true>), gn, blk, 0, st, a);                  \
    else if constexpr (K == BK_SLICE_BWD_G)                                                    \
      hipLaunchKernelGGL((k_blk_bwd_g<T, DK, NB_, true>), gg, blk, 0, st, a);                  \
    else if constexpr (K == BK_DESLICE_BWD_N)                                                  \
      hipLaunchKernelGGL((k_blk_bwd_n<T, DK, NB_, false>), gn, blk, 0, st, a);                 \
    else                                                                                       \
      hipLaunchKernelGGL((k_blk_bwd_g<T, DK, NB_, false>), gg, blk, 0, st, a);                 \
    return hipGetLastError();                                                                  \
  }
  BK_TRY(4) BK_TRY(8)
#undef BK_TRY
  return hipErrorNotSupported;
}

#define FS_BLOCKED_INSTANCES(X)                                                            \
  X(0, float, 0) X(1, float, 0) X(2, float, 0) X(3, float, 0) X(4, float, 0)               \
  X(5, float, 0) X(6, float, 0) X(7, float, 0)                                             \
  X(0, __bf16, 0) X(1, __bf16, 0) X(2, __bf16, 0) X(3, __bf16, 0) X(4, __bf16, 0)          \
  X(5, __bf16, 0) X(6, __bf16, 0) X(7, __bf16, 0)                                          \
  X(0, __bf16, 1) X(1, __bf16, 1) X(2, __bf16, 1) X(3, __bf16, 1) X(4, __bf16, 1)          \
  X(5, __bf16, 1) X(6, __bf16, 1) X(7, __bf16, 1)                                          \
  X(0, __bf16, 2) X(1, __bf16, 2) X(2, __bf16, 2) X(3, __bf16, 2) X(4, __bf16, 2)          \
  X(5, __bf16, 2) X(6, __bf16, 2) X(7, __bf16, 2)                                          \
  X(0, _Float16, 0) X(1, _Float16, 0) X(2, _Float16, 0) X(3, _Float16, 0) X(4, _Float16, 0) \
  X(5, _Float16, 0) X(6, _Float16, 0) X(7, _Float16, 0)                                    \
  X(0, _Float16, 1) X(1, _Float16, 1) X(2, _Float16, 1) X(3, _Float16, 1) X(4, _Float16, 1) \
  X(5, _Float16, 1) X(6, _Float16, 1) X(7, _Float16, 1)                                    \
  X(0, _Float16, 2) X(1, _Float16, 2) X(2, _Float16, 2) X(3, _Float16, 2) X(4, _Float16, 2) \
  X(5, _Float16, 2) X(6, _Float16, 2) X(7, _Float16, 2)

#define FS_DECLARE_BLK_EXTERN(K_, T_, DK_) \
  extern template hipError_t blocked_launch<K_, T_, DK_>(const Args&, hipStream_t);
FS_BLOCKED_INSTANCES(FS_DECLARE_BLK_EXTERN)
#undef FS_DECLARE_BLK_EXTERN

}  // namespace fs
