// G-blocked slice/deslice kernels on prepared operand fragments (gfx950),
// any slot count G, head widths D, DV <= 64.
//
// The same split as fs_blocked_kernels.h (reference blocked.py:1-66):
// point-owned kernels ("_n") own 32-point tiles and loop over G in slot
// blocks of 32, slot-owned kernels ("_g") own one slot block and stream the
// points; per-point softmax statistics (m, l) carry the normalisation
// between them. What differs is how the small operands reach the MFMAs and
// how the dots run:
//   * k_gp_prep turns W, W / tau, the tokens (or dz_num) and the per-slot
//     bias and d s into MFMA-ready fragments once per call (exact bf16x6
//     split for the fp32-accurate levels, fs_mma.h), laid out so that one
//     wave reads one 1 KB word per instruction;
//   * the point-owned kernels stage each slot block's fragments into LDS
//     with direct-to-LDS buffer loads, double-buffered: the four waves of a
//     block (one head) prefetch slot block s + 1 while computing slot block
//     s, one barrier per slot block;
//   * the slot-owned kernels stage their one slot block once and stream the
//     points like the whole-G kernels (ping-pong registers, buffer I/O);
//     the grid runs the slot blocks fastest, so the blocks in flight share
//     point tiles in L2.
// Every dot runs on the bf16 matrix cores (MMA_X6 for ieee / tf32 / tf32x3,
// bf16 for the bf16 levels). Per-wave partials are reduced in a fixed order
// by fs_reduce.hip: results are bitwise reproducible.
//
// Reference kernels these replace: _stats_kernel / _stats_twopass_kernel
// (blocked.py:292-400), _slice_fwd_g_kernel (:403-462), _deslice_fwd_n_kernel
// (:465-510), _deslice_fwd_online_kernel (:513-573), _slice_bwd_n_kernel
// (:576-673), _slice_bwd_g_kernel (:676-741), _deslice_bwd_n_kernel
// (:744-815), _deslice_bwd_g_kernel (:818-888).
#pragma once
#include <type_traits>

#include "fs_mma.h"
#include "fs_tile.h"

namespace fs {

// Waves per SIMD the kernels are compiled for: two for one 32-column block,
// one (512 registers) for two. With one block, the slot-owned slice forward,
// the point-owned backward and the slot-owned slice backward are compiled for
// three (168 registers, a few values spilled): measured at C3 (G = 256),
// 1-7 % faster each; the slot-owned deslice backward spills too much there
// (288 bytes per lane, 29 % slower) and keeps two.
constexpr int gp_waves(int nb) { return nb == 1 ? 2 : 1; }

// Column blocks k < NB are guarded by the call's block counts nd / nv; block 0
// always exists (D, DV >= 1), and saying so (k == 0 || k < nd) lets the MFMA
// chains start without materialising a zero accumulator for the skipped case.
template <int DK> struct GModes {
  static constexpr int L = (DK == 2) ? MMA_BF16 : MMA_X6;
  static constexpr int V = (DK >= 1) ? MMA_BF16 : MMA_X6;
};

typedef __attribute__((address_space(3))) void* LdsPtr;

// ------------------------------------------------------------------- prep
// Grid (ngb, B * H, 6 kinds); wave w builds items k = w, w + 4, ... of its
// (kind, bh, slot block). fp32 sources: W (.., G, D) through its strides,
// V = a.tok (B, H, G, DV) contiguous, bias, tau, d s (B, H, G).
template <int DK>
__global__ __launch_bounds__(256) void k_gp_prep(Args a) {
  constexpr int ML = GModes<DK>::L, MV = GModes<DK>::V;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, c = lane & 31, h = lane >> 5;
  const int gb = blockIdx.x, bh = blockIdx.y, kind = blockIdx.z, ngb = gridDim.x;
  const int b = bh / a.H, hd = bh - b * a.H;
  const int G = a.G, D = a.D, DV = a.DV, nd = a.nd, nv = a.nv;
  const float* Wp = a.W + b * a.swb + hd * a.swh;
  const float* Vp = a.tok ? a.tok + (int64_t)bh * G * DV : nullptr;
  const float tauf = a.tau[hd];
  const float inv_tau = 1.f / tauf;
  const float cst = (float)(1.4426950408889634 / (double)tauf);
  u32x4* fr = reinterpret_cast<u32x4*>(a.frags);
  auto put = [&](int knd, int nk, int k, int fw, const u32x4* words, int nw) {
    u32x4* dst = fr + a.foff[knd] + ((int64_t)(bh * ngb + gb) * nk + k) * fw;
    for (int w = 0; w < nw; ++w) dst[w * 64 + lane] = words[w];
  };
  // fragment element j of lane (c, h): row-outer -> M[32 gb + c][32 k +
  // kmap(j, h)], col-outer -> M[32 gb + kmap(j, h)][32 k + c]
  auto build = [&](const float* M, int C, int k, bool rowouter, float scale, float (&f)[16]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int g = 32 * gb + (rowouter ? c : kmap(j, h));
      const int col = 32 * k + (rowouter ? kmap(j, h) : c);
      f[j] = (g < G && col < C) ? M[(int64_t)g * C + col] * scale : 0.f;
    }
  };
  if (kind == GP_WR) {
    for (int k = wid; k < nd; k += kWavesPerBlock) {
      float f[16];
      build(Wp, D, k, true, 1.f, f);
      Frag<ML> q;
      prep<ML>(q, f);
      put(GP_WR, nd, k, frag_words<ML>(), q.q, Frag<ML>::W);
    }
  } else if (kind == GP_WC) {
    for (int k = wid; k < nd; k += kWavesPerBlock) {
      float f[16];
      build(Wp, D, k, false, inv_tau, f);
      Frag<MV> q;
      prep<MV>(q, f);
      put(GP_WC, nd, k, frag_words<MV>(), q.q, Frag<MV>::W);
    }
  } else if (kind == GP_VR || kind == GP_VC) {
    if (!Vp) return;
    for (int k = wid; k < nv; k += kWavesPerBlock) {
      float f[16];
      build(Vp, DV, k, kind == GP_VR, 1.f, f);
      Frag<MV> q;
      prep<MV>(q, f);
      put(kind, nv, k, frag_words<MV>(), q.q, Frag<MV>::W);
    }
  } else if (wid == 0) {
    // per-slot vectors: word q of lane (c, h) holds slots 32 gb + 8 q + 4 h + 0..3
    const float* Bp = a.bias + b * a.sbb + hd * a.sbh;
    const float* Sp = a.ds ? a.ds + (int64_t)bh * G : nullptr;
    u32x4 words[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int g = 32 * gb + 8 * q + 4 * h + i;
        const float v = kind == GP_BC ? (g < G ? Bp[g] * cst : kNoSlot)
                                      : ((Sp && g < G) ? Sp[g] : 0.f);
        words[q][i] = __float_as_uint(v);
      }
    put(kind, 1, 0, kGpVecFw, words, 4);
  }
}

// ------------------------------------------------------------ common pieces
// Stage n 1 KB words (64 lanes x 16 bytes) from global `src` into LDS `dst`
// with direct-to-LDS buffer loads, dealt round-robin to the block's waves.
__device__ __forceinline__ void gp_stage(u32x4* dst, const u32x4* src, int n, int wid, int lane) {
  const Rsrc r = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(src), (short)0, n * 1024,
                                                   kRsrcWord3);
  for (int i = wid; i < n; i += kWavesPerBlock)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)(dst + i * 64), 16,
                                             (uint32_t)(i * 1024 + lane * 16), 0, 0, 0);
}
// a per-slot vector item from LDS: lane half h's 16 values
__device__ __forceinline__ void gp_vec(float (&v)[16], const u32x4* item, int lane) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4 w = item[q * 64 + lane];
    v[4 * q + 0] = __uint_as_float(w[0]);
    v[4 * q + 1] = __uint_as_float(w[1]);
    v[4 * q + 2] = __uint_as_float(w[2]);
    v[4 * q + 3] = __uint_as_float(w[3]);
  }
}

#define GP_PROLOGUE                                                               \
  const int lane = threadIdx.x & 63;                                              \
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);               \
  const int c = lane & 31, h = lane >> 5;                                         \
  const int G = a.G, D = a.D, DV = a.DV, nd = a.nd, nv = a.nv;                    \
  const int ngb = (G + 31) / 32;                                                  \
  (void)D; (void)DV; (void)nd; (void)nv;

#define GP_HEAD(BH)                                                               \
  const int bh = (BH);                                                            \
  const int b = bh / a.H, hd = bh - b * a.H;                                      \
  const float tauf = a.tau[hd];                                                   \
  const float cst = (float)(1.4426950408889634 / (double)tauf);                  \
  const float inv_tau = 1.f / tauf;                                               \
  const bool fast = a.fast != 0;                                                  \
  const u32x4* fr = reinterpret_cast<const u32x4*>(a.frags);                     \
  /* this sample's rows (row splits of a ragged batch) and per-point buffers */ \
  const Rows R_ = rows_of(a, b, hd);                                              \
  const int64_t row0_ = R_.row0;                                                  \
  const int N = R_.N, ntiles_ = R_.ntiles;                                        \
  (void)inv_tau; (void)fast; (void)b; (void)row0_; (void)ntiles_;

// point slice of one (b, h): byte base, row stride, row width, lane row
#define GP_SLICE(NAME, PTR, SB, SN, SH, C)                                                \
  const char* NAME##_b =                                                                  \
      (const char*)(PTR) + (b * (SB) + row0_ * (SN) + hd * (SH)) * (int64_t)sizeof(T);    \
  const int64_t NAME##_sn = (SN) * (int64_t)sizeof(T);                                    \
  const int64_t NAME##_w = (int64_t)(C) * (int64_t)sizeof(T);                             \
  const uint32_t NAME##_row = (uint32_t)(c * NAME##_sn);

// the item of a kind for slot block gb of this head
#define GP_ITEM(KIND, NK, GB, FW) (fr + a.foff[KIND] + ((int64_t)(bh * ngb + (GB)) * (NK)) * (FW))

// point rows of one tile in either load form (nk of the NB blocks used)
template <typename T, int NB>
__device__ __forceinline__ void gp_rows(float (&f)[NB][16], Rsrc r, uint32_t row, bool fast,
                                        int C, int h) {
  if (fast)
    ld_rows<T, NB, true>(f, r, row + 4 * h * (uint32_t)sizeof(T), C, h);
  else
    ld_rows<T, NB, false>(f, r, row, C, h);
}

// logits of one slot block from staged W fragments: t2 = (x . W + b) log2(e) / tau
template <int ML, int NB>
__device__ __forceinline__ void gp_logits(float (&t2)[16], const u32x4* sw, const u32x4* sbc,
                                          const Frag<ML> (&xq)[NB], int nd, float cst, int lane) {
  f32x16 s = zero16();
#pragma unroll
  for (int k = 0; k < NB; ++k)
    if (k == 0 || k < nd) {
      Frag<ML> wq;
      lds_get<ML>(wq, sw + k * frag_words<ML>(), lane);
      s = mma<ML>(wq, xq[k], s);
    }
  float bc[16];
  gp_vec(bc, sbc, lane);
#pragma unroll
  for (int r = 0; r < 16; ++r) t2[r] = fmaf(s[r], cst, bc[r]);
}

// ------------------------------------------------------------ stats (n)
// Per tile: x prepared once, then every slot block's logits; online max / sum
// per lane (or two passes: max, then the sum against the max as consumers
// read it back), combined with the partner lane.
template <typename T, int DK, int NB>
__global__ __launch_bounds__(256, gp_waves(NB)) void k_gp_stats(Args a) {
  constexpr int ML = GModes<DK>::L;
  constexpr int FWL = frag_words<ML>();
  constexpr int SETW = NB * FWL + kGpVecFw;
  __shared__ __attribute__((aligned(16))) u32x4 sbuf[2][SETW];
  GP_PROLOGUE
  GP_HEAD(blockIdx.y)
  GP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  const float* sm = a.stats_out ? a.stats_out + R_.stats_off() : nullptr;
  const float* sl = sm ? sm + R_.NS : nullptr;
  const int passes = a.two_pass ? 2 : 1, nstage = passes * ngb;
  auto stage = [&](int buf, int s) {
    const int gb = s % ngb;
    gp_stage(sbuf[buf], GP_ITEM(GP_WR, nd, gb, FWL), nd * Frag<ML>::W, wid, lane);
    gp_stage(sbuf[buf] + NB * FWL, GP_ITEM(GP_BC, 1, gb, kGpVecFw), 4, wid, lane);
  };
  int g = 0;
  stage(0, 0);
  // with the logits' operands split (the fp32-accurate levels) a tile's
  // rows are loaded one tile ahead, right after the previous tile's were
  // split (the slot blocks' staging waits absorb the load; config 3, G =
  // 256: statistics and deslice 5 % faster); with bf16 dots the registers
  // that takes would cost a wave per SIMD, and the rows are loaded at the
  // tile's start
  constexpr bool PF = ML == MMA_X6;
  const int64_t pstep = (int64_t)kWavesPerBlock * gridDim.x * kTile;
  float xf[NB][16];
  if constexpr (PF)
    gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, (int64_t)(kWavesPerBlock * blockIdx.x + wid) * kTile, N),
                   x_row, fast, D, h);
  __syncthreads();
  for (int it = 0;; ++it) {
    const int tb = kWavesPerBlock * (blockIdx.x + it * gridDim.x);
    if (tb >= ntiles_) break;
    const int64_t p0 = (int64_t)(tb + wid) * kTile;
    const bool more = tb + kWavesPerBlock * (int)gridDim.x < ntiles_;
    if constexpr (!PF) gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, p0, N), x_row, fast, D, h);
    Frag<ML> xq[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) prep<ML>(xq[k], xf[k]);
    if constexpr (PF) gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, p0 + pstep, N), x_row, fast, D, h);
    float m = -INFINITY, l = 0.f, mc = 0.f;
    for (int s = 0; s < nstage; ++s, ++g) {
      if (s + 1 < nstage || more) stage((g + 1) & 1, (s + 1) % nstage);
      const u32x4* sw = sbuf[g & 1];
      float t2[16];
      gp_logits<ML, NB>(t2, sw, sw + NB * FWL, xq, nd, cst, lane);
      if (a.two_pass) {
        if (s < ngb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) m = fmaxf(m, t2[r]);
          if (s == ngb - 1) {
            m = pair_max(m);
            mc = stats_max_roundtrip(m);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) l += __builtin_amdgcn_exp2f(t2[r] - mc);
        }
      } else {
        float mb = m;
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = fmaxf(mb, t2[r]);
        float sb = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) sb += __builtin_amdgcn_exp2f(t2[r] - mb);
        l = l * __builtin_amdgcn_exp2f(m - mb) + sb;
        m = mb;
      }
      __syncthreads();
    }
    if (a.two_pass) {
      l = pair_sum(l);
    } else {
      float mlo, mhi, llo, lhi;
      halves(m, mlo, mhi);
      halves(l, llo, lhi);
      const float mm = fmaxf(mlo, mhi);
      l = llo * __builtin_amdgcn_exp2f(mlo - mm) + lhi * __builtin_amdgcn_exp2f(mhi - mm);
      m = mm;
    }
    store_stats_tile(sm, sl, p0, N, c, h, m, l, a.two_pass != 0);
  }
}

// ---------------------------------------------------------------- deslice (n)
// ONLINE: rescale the accumulator and the row sum whenever the row max moves,
// and emit (m, l) (reference blocked.py:513-573). Otherwise normalise with
// the saved row max and the sum of the very exponentials accumulated here
// (blocked.py:465-510).
template <typename T, int DK, int NB, bool ONLINE>
__global__ __launch_bounds__(256, gp_waves(NB)) void k_gp_deslice(Args a) {
  constexpr int ML = GModes<DK>::L, MV = GModes<DK>::V;
  constexpr int FWL = frag_words<ML>(), FWV = frag_words<MV>();
  constexpr int SETW = NB * FWL + NB * FWV + kGpVecFw;
  __shared__ __attribute__((aligned(16))) u32x4 sbuf[2][SETW];
  __shared__ float srows[kWavesPerBlock * 32];
  GP_PROLOGUE
  GP_HEAD(blockIdx.y)
  float* lds_x = srows + wid * 32;
  GP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  GP_SLICE(o, a.o1, a.s1b, a.s1n, a.s1h, DV)
  (void)o_row;
  uint32_t vco[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) vco[k] = col_off<T>(k, DV, o_sn, c, h);
  const float* sin_m = ONLINE ? nullptr : a.stats_in + R_.stats_off();
  // the statistics are optional output of the online pass (null: not kept)
  const float* sout_m = (ONLINE && a.stats_out) ? a.stats_out + R_.stats_off() : nullptr;
  const float* sout_l = sout_m ? sout_m + R_.NS : nullptr;
  auto stage = [&](int buf, int gb) {
    gp_stage(sbuf[buf], GP_ITEM(GP_WR, nd, gb, FWL), nd * Frag<ML>::W, wid, lane);
    gp_stage(sbuf[buf] + NB * FWL, GP_ITEM(GP_VC, nv, gb, FWV), nv * Frag<MV>::W, wid, lane);
    gp_stage(sbuf[buf] + NB * FWL + NB * FWV, GP_ITEM(GP_BC, 1, gb, kGpVecFw), 4, wid, lane);
  };
  int g = 0;
  stage(0, 0);
  // a tile's rows (and saved row max) one tile ahead where the logits'
  // operands are split, as in the statistics pass
  constexpr bool PF = ML == MMA_X6;
  const int64_t pstep = (int64_t)kWavesPerBlock * gridDim.x * kTile;
  float xf[NB][16], mn = 0.f;
  if constexpr (PF) {
    const int64_t pf = (int64_t)(kWavesPerBlock * blockIdx.x + wid) * kTile;
    gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, pf, N), x_row, fast, D, h);
    if (!ONLINE) mn = ld_pt(pts_rsrc(sin_m, pf, N), c);
  }
  __syncthreads();
  for (int it = 0;; ++it) {
    const int tb = kWavesPerBlock * (blockIdx.x + it * gridDim.x);
    if (tb >= ntiles_) break;
    const int64_t p0 = (int64_t)(tb + wid) * kTile;
    const bool pv = p0 + c < N;
    const bool more = tb + kWavesPerBlock * (int)gridDim.x < ntiles_;
    if constexpr (!PF) {
      gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, p0, N), x_row, fast, D, h);
      if (!ONLINE) mn = ld_pt(pts_rsrc(sin_m, p0, N), c);
    }
    Frag<ML> xq[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) prep<ML>(xq[k], xf[k]);
    float m2 = -INFINITY, l = 0.f, lown = 0.f;
    if (!ONLINE) m2 = mn * kLog2e;
    if constexpr (PF) {
      gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, p0 + pstep, N), x_row, fast, D, h);
      if (!ONLINE) mn = ld_pt(pts_rsrc(sin_m, p0 + pstep, N), c);
    }
    f32x16 acc[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) acc[k] = zero16();
    for (int s = 0; s < ngb; ++s, ++g) {
      if (s + 1 < ngb || more) stage((g + 1) & 1, (s + 1) % ngb);
      const u32x4* sw = sbuf[g & 1];
      float t2[16], e[16];
      gp_logits<ML, NB>(t2, sw, sw + NB * FWL + NB * FWV, xq, nd, cst, lane);
      if (ONLINE) {
        float mb = m2;
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = fmaxf(mb, t2[r]);
        mb = pair_max(mb);
        const float alpha = __builtin_amdgcn_exp2f(m2 - mb);
        float sb = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          e[r] = __builtin_amdgcn_exp2f(t2[r] - mb);
          sb += e[r];
        }
        sb = pair_sum(sb);
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
      Frag<MV> eq;
      prep<MV>(eq, e);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nv) {
          Frag<MV> tq;
          lds_get<MV>(tq, sw + NB * FWL + k * FWV, lane);
          acc[k] = mma<MV>(eq, tq, acc[k]);
        }
      __syncthreads();
    }
    if (!ONLINE) l = pair_sum(lown);
    const float inv_l = pv ? 1.f / l : 0.f;
    float inv_r[16];
    gather_rows(inv_r, inv_l, lds_x, c, h);
    const Rsrc ro = rows_rsrc(o_b, o_sn, o_w, p0, N);
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k == 0 || k < nv) {
        f32x16 o = acc[k];
#pragma unroll
        for (int r = 0; r < 16; ++r) o[r] *= inv_r[r];
        st_cols<T>(ro, vco[k], (uint32_t)o_sn, o);
      }
    if (ONLINE) store_stats_tile(sout_m, sout_l, p0, N, c, h, m2, l);
  }
}

// ------------------------------------------------------------------ slice (g)
// One slot block per block (blockIdx.x, fastest), point partition
// blockIdx.y, head blockIdx.z: z_num, s partials of its 32 slots. Compiled
// for three waves per SIMD with one column block (168 registers and a few
// spilled values; measured 2 % faster at C3 than two waves with 192).
template <typename T, int DK, int NB>
__global__ __launch_bounds__(256, NB == 1 ? 3 : 1) void k_gp_slice_g(Args a) {
  constexpr int ML = GModes<DK>::L, MV = GModes<DK>::V;
  constexpr int FWL = frag_words<ML>();
  __shared__ __attribute__((aligned(16))) u32x4 sq[NB * FWL + kGpVecFw];
  __shared__ float stile[kWavesPerBlock * kLdsTile];
  GP_PROLOGUE
  GP_HEAD(blockIdx.z)
  const int gb = blockIdx.x;
  const int P = a.P, pid = blockIdx.y * kWavesPerBlock + wid;
  float* lds = stile + wid * kLdsTile;
  gp_stage(sq, GP_ITEM(GP_WR, nd, gb, FWL), nd * Frag<ML>::W, wid, lane);
  gp_stage(sq + NB * FWL, GP_ITEM(GP_BC, 1, gb, kGpVecFw), 4, wid, lane);
  __syncthreads();
  f32x16 zacc[NB];
  float sacc = 0.f;
#pragma unroll
  for (int k = 0; k < NB; ++k) zacc[k] = zero16();
  GP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  GP_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  (void)f_row;
  uint32_t vcf[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) vcf[k] = col_off<T>(k, DV, f_sn, c, h);
  const float* sm = a.stats_in + R_.stats_off();
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    // a tile's statistics (m, l) travel with its rows in the register set,
    // loaded two tiles ahead: a load issued and waited for in the tile's own
    // body would be the youngest outstanding, and waiting for it would wait
    // for the prefetched tiles too (config 3's slice forward: 3.44 -> 3.26
    // ms at G = 256, 12.7 -> 11.9 at G = 1024, 7.5 -> 7.3 with bf16 dots)
    float xA[NB][16], xB[NB][16], fA[NB][16], fB[NB][16], sA[2], sB[2];
    auto load = [&](float (&xn)[NB][16], float (&fn)[NB][16], float (&sn)[2], int t) {
      const int64_t p0 = (int64_t)t * kTile;
      ld_rows<T, NB, FAST>(xn, rows_rsrc(x_b, x_sn, x_w, p0, N), vrx, D, h);
      const Rsrc rf = rows_rsrc(f_b, f_sn, f_w, p0, N);
#pragma unroll
      for (int k = 0; k < NB; ++k) ld_cols<T>(fn[k], rf, vcf[k], (uint32_t)f_sn);
      sn[0] = ld_pt(pts_rsrc(sm, p0, N), c);
      sn[1] = ld_pt(pts_rsrc(sm + R_.NS, p0, N), c);
    };
    auto body = [&](const float (&xf)[NB][16], const float (&fT)[NB][16], const float (&sv)[2],
                    int t, auto par) {
      const int64_t p0 = (int64_t)t * kTile;
      const bool pv = p0 + c < N;
      const float m2 = sv[0] * kLog2e;
      const float l = sv[1];
      Frag<ML> xq[NB];
#pragma unroll
      for (int k = 0; k < NB; ++k) prep<ML>(xq[k], xf[k]);
      float t2[16], w[16];
      gp_logits<ML, NB>(t2, sq, sq + NB * FWL, xq, nd, cst, lane);
      // the weights carry the tile's sign (acc_add)
      constexpr float sg = decltype(par)::sign;
      const float inv_l = pv ? sg / l : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) w[r] = __builtin_amdgcn_exp2f(t2[r] - m2) * inv_l;
      float wT[16];
      transpose32(wT, w, lds, c, h);
      Frag<MV> wq;
      prep<MV>(wq, wT);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nv) {
          Frag<MV> fq;
          prep<MV>(fq, fT[k]);
          mma_acc<MV>(zacc[k], fq, wq, sg);
        }
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s += wT[j];
      sacc = fmaf(s, sg, sacc);
    };
    FS_TILE_LOOP(load, body, false, FS_ARGS3(xA, fA, sA), FS_ARGS3(xB, fB, sB))
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  float* pw = a.part + ((int64_t)bh * P + pid) * part_floats_slice_fwd(G, DV);
  const int gg = 32 * gb + c;
  const float s = pair_sum(sacc);
  if (gg < G) {
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k == 0 || k < nv)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = 32 * k + kmap(r, h);
          if (v < DV) pw[(int64_t)gg * DV + v] = zacc[k][r];
        }
    if (h == 0) pw[(int64_t)G * DV + gg] = s;
  }
}

// ---------------------------------------------------- slice / deslice bwd (n)
// Point-owned backward (reference blocked.py:576-673, :744-815). Pass 1 over
// the slot blocks: the Jacobian numerator sum_g e omega (and, for the slice,
// dfx = e dz_num), divided by the row sum l formed from the same
// exponentials. Pass 2: dl = e (omega - delta) / l (the difference first:
// with a near-uniform softmax omega sits close to delta, and e omega - e delta
// would cancel most of two rounded products), dx += dl (W / tau), and the row
// term sum_g dl (t2 - m2) of the temperature gradient. delta and l go to the
// slot-owned pass.
// SLICE: omega = fx . dz_num + ds, also writes dfx; else omega = d_out . T.
template <typename T, int DK, int NB, bool SLICE>
__global__ __launch_bounds__(256, NB == 1 ? 3 : gp_waves(NB)) void k_gp_bwd_n(Args a) {
  constexpr int ML = GModes<DK>::L, MV = GModes<DK>::V;
  constexpr int FWL = frag_words<ML>(), FWV = frag_words<MV>();
  // stage layout: W (logits) | V rows (omega) | V cols (dfx, pass 1) or W / tau (dx, pass 2)
  // | bias vector | ds vector
  constexpr int O_VR = NB * FWL, O_X = O_VR + NB * FWV, O_BC = O_X + NB * FWV;
  constexpr int O_DS = O_BC + kGpVecFw, SETW = O_DS + kGpVecFw;
  __shared__ __attribute__((aligned(16))) u32x4 sbuf[2][SETW];
  __shared__ float srows[kWavesPerBlock * 32];
  GP_PROLOGUE
  GP_HEAD(blockIdx.y)
  const int pid = blockIdx.x * kWavesPerBlock + wid;
  float* lds_x = srows + wid * 32;
  GP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  GP_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  GP_SLICE(dx, a.o1, a.s1b, a.s1n, a.s1h, D)
  GP_SLICE(df, a.o2, a.s2b, a.s2n, a.s2h, DV)
  (void)dx_row; (void)df_row;
  uint32_t vcx[NB], vcf[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    vcx[k] = col_off<T>(k, D, dx_sn, c, h);
    vcf[k] = col_off<T>(k, DV, df_sn, c, h);
  }
  const float* sm = a.stats_in + R_.stats_off();
  const float* sdel = a.delta + R_.pt_off();
  const float* slsum = a.lsum + R_.pt_off();
  const int nstage = 2 * ngb;
  auto stage = [&](int buf, int s) {
    const int gb = s % ngb, pass = s / ngb;
    gp_stage(sbuf[buf], GP_ITEM(GP_WR, nd, gb, FWL), nd * Frag<ML>::W, wid, lane);
    gp_stage(sbuf[buf] + O_VR, GP_ITEM(GP_VR, nv, gb, FWV), nv * Frag<MV>::W, wid, lane);
    if (pass == 0) {
      if (SLICE) gp_stage(sbuf[buf] + O_X, GP_ITEM(GP_VC, nv, gb, FWV), nv * Frag<MV>::W, wid, lane);
    } else {
      gp_stage(sbuf[buf] + O_X, GP_ITEM(GP_WC, nd, gb, FWV), nd * Frag<MV>::W, wid, lane);
    }
    gp_stage(sbuf[buf] + O_BC, GP_ITEM(GP_BC, 1, gb, kGpVecFw), 4, wid, lane);
    if (SLICE) gp_stage(sbuf[buf] + O_DS, GP_ITEM(GP_DS, 1, gb, kGpVecFw), 4, wid, lane);
  };
  float dtacc = 0.f;
  int g = 0;
  stage(0, 0);
  __syncthreads();
  for (int it = 0;; ++it) {
    const int tb = kWavesPerBlock * (blockIdx.x + it * gridDim.x);
    if (tb >= ntiles_) break;
    const int64_t p0 = (int64_t)(tb + wid) * kTile;
    const bool pv = p0 + c < N;
    const bool more = tb + kWavesPerBlock * (int)gridDim.x < ntiles_;
    float xf[NB][16], ff[NB][16];
    gp_rows<T, NB>(xf, rows_rsrc(x_b, x_sn, x_w, p0, N), x_row, fast, D, h);
    gp_rows<T, NB>(ff, rows_rsrc(f_b, f_sn, f_w, p0, N), f_row, fast, DV, h);
    const float m2 = ld_pt(pts_rsrc(sm, p0, N), c) * kLog2e;
    Frag<ML> xq[NB];
    Frag<MV> fq[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      prep<ML>(xq[k], xf[k]);
      prep<MV>(fq[k], ff[k]);
    }
    f32x16 acc[NB];  // pass 1: dfx numerator; pass 2: dx
#pragma unroll
    for (int k = 0; k < NB; ++k) acc[k] = zero16();
    float sdw = 0.f, lown = 0.f, delta = 0.f, inv_l = 0.f, rt = 0.f;
    // one slot block: prefetch the next stage's fragments, logits, exponentials
    // and omega of this one
    auto stage_in = [&](int s, const u32x4*& sw, float (&t2)[16], float (&e)[16],
                        float (&om)[16]) {
      if (s + 1 < nstage || more) stage((g + 1) & 1, (s + 1) % nstage);
      sw = sbuf[g & 1];
      gp_logits<ML, NB>(t2, sw, sw + O_BC, xq, nd, cst, lane);
#pragma unroll
      for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(t2[r] - m2);
      f32x16 o = zero16();
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nv) {
          Frag<MV> vq;
          lds_get<MV>(vq, sw + O_VR + k * FWV, lane);
          o = mma<MV>(vq, fq[k], o);
        }
      float dsv[16];
      if (SLICE) gp_vec(dsv, sw + O_DS, lane);
#pragma unroll
      for (int r = 0; r < 16; ++r) om[r] = SLICE ? o[r] + dsv[r] : o[r];
    };
    // pass 1 over the slot blocks: row sum, delta numerator (and dfx)
    for (int s = 0; s < ngb; ++s, ++g) {
      const u32x4* sw;
      float t2[16], e[16], om[16];
      stage_in(s, sw, t2, e, om);
      float lb = 0.f, sb = 0.f;  // per slot block, then across blocks
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        lb += e[r];
        sb = fmaf(e[r], om[r], sb);
      }
      lown += lb;
      sdw += sb;
      if (SLICE) {
        Frag<MV> eq;
        prep<MV>(eq, e);
#pragma unroll
        for (int k = 0; k < NB; ++k)
          if (k == 0 || k < nv) {
            Frag<MV> zq;
            lds_get<MV>(zq, sw + O_X + k * FWV, lane);
            acc[k] = mma<MV>(eq, zq, acc[k]);
          }
      }
      __syncthreads();
    }
    {
      const float l = pair_sum(lown);
      inv_l = 1.f / l;
      delta = pair_sum(sdw) * inv_l;
      st_pt(pts_rsrc(sdel, p0, N), c, h, delta);
      st_pt(pts_rsrc(slsum, p0, N), c, h, l);
      if (SLICE) {
        float inv_r[16];
        gather_rows(inv_r, pv ? inv_l : 0.f, lds_x, c, h);
        const Rsrc rdf = rows_rsrc(df_b, df_sn, df_w, p0, N);
#pragma unroll
        for (int k = 0; k < NB; ++k)
          if (k == 0 || k < nv) {
            f32x16 o = acc[k];
#pragma unroll
            for (int r = 0; r < 16; ++r) o[r] *= inv_r[r];
            st_cols<T>(rdf, vcf[k], (uint32_t)df_sn, o);
          }
      }
#pragma unroll
      for (int k = 0; k < NB; ++k) acc[k] = zero16();
    }
    // pass 2: dl = e (omega - delta) / l, dx += dl (W / tau), the row term
    // of dtau
    for (int s = ngb; s < nstage; ++s, ++g) {
      const u32x4* sw;
      float t2[16], e[16], om[16];
      stage_in(s, sw, t2, e, om);
      // the row term summed per slot block, then across blocks: dtau is a
      // strongly cancelling sum, and one chain over all of G (128 terms at
      // G = 256) lost ~15x eager's accuracy on it
      float dl[16], rb = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dl[r] = e[r] * (om[r] - delta) * inv_l;
        rb = fmaf(dl[r], t2[r] - m2, rb);
      }
      rt += rb;
      Frag<MV> dq;
      prep<MV>(dq, dl);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nd) {
          Frag<MV> wq;
          lds_get<MV>(wq, sw + O_X + k * FWV, lane);
          acc[k] = mma<MV>(dq, wq, acc[k]);
        }
      __syncthreads();
    }
    const Rsrc rdx = rows_rsrc(dx_b, dx_sn, dx_w, p0, N);
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k == 0 || k < nd) st_cols<T>(rdx, vcx[k], (uint32_t)dx_sn, acc[k]);
    rt = pair_sum(rt);
    dtacc += (pv && h == 0) ? rt : 0.f;
  }
  const float dt = half_wave_sum(dtacc);
  if (lane == 0) a.part2[(int64_t)bh * a.P + pid] = -kLn2 * inv_tau * dt;
}

// --------------------------------------------------- slice / deslice bwd (g)
// Slot-owned backward (reference blocked.py:676-741, :818-888): one 32-slot
// block, streaming points with the saved statistics, delta and row sums.
// SLICE: dW, db partials (omega = fx . dz_num + ds); else also dtokens
// (omega = d_out . T).
template <typename T, int DK, int NB, bool SLICE>
__global__ __launch_bounds__(256, NB == 1 && SLICE ? 3 : gp_waves(NB)) void k_gp_bwd_g(Args a) {
  constexpr int ML = GModes<DK>::L, MV = GModes<DK>::V;
  constexpr int FWL = frag_words<ML>(), FWV = frag_words<MV>();
  constexpr int O_VR = NB * FWL, O_BC = O_VR + NB * FWV, O_DS = O_BC + kGpVecFw;
  __shared__ __attribute__((aligned(16))) u32x4 sq[O_DS + kGpVecFw];
  // TR (one column block, bf16 value dots): the transposed operands are the
  // bf16 operands already formed, read back transposed (tr_put / tr_get)
  // through one region per wave -- d_out's (formed for omega), w's, Lb's,
  // then x's (formed for the logits and held in registers meanwhile) -- and
  // db is Lb^T's row sum on the matrix cores; no fp32 transposes. Measured at
  // C3 (G = 256): deslice bwd 4.12 -> 3.82 ms with bf16 dots; with the bf16x6
  // split the same form (4 splits instead of 6) needs 242 registers and runs
  // two waves per SIMD instead of four, and was no faster.
  constexpr bool TR = NB == 1 && MV == MMA_BF16;
  constexpr int WF = TR ? tr_bytes<ML>() / 4 : kLdsTile;
  __shared__ __attribute__((aligned(16))) float stile[kWavesPerBlock * WF];
  GP_PROLOGUE
  GP_HEAD(blockIdx.z)
  const int gb = blockIdx.x;
  const int P = a.P, pid = blockIdx.y * kWavesPerBlock + wid;
  float* lds = stile + wid * WF;
  char* trS = reinterpret_cast<char*>(lds);
  (void)trS;
  gp_stage(sq, GP_ITEM(GP_WR, nd, gb, FWL), nd * Frag<ML>::W, wid, lane);
  gp_stage(sq + O_VR, GP_ITEM(GP_VR, nv, gb, FWV), nv * Frag<MV>::W, wid, lane);
  gp_stage(sq + O_BC, GP_ITEM(GP_BC, 1, gb, kGpVecFw), 4, wid, lane);
  if (SLICE) gp_stage(sq + O_DS, GP_ITEM(GP_DS, 1, gb, kGpVecFw), 4, wid, lane);
  __syncthreads();
  f32x16 dW[NB], dT[NB];
  float dbacc = 0.f;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    dW[k] = zero16();
    dT[k] = zero16();
  }
  GP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  GP_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  const float* sm = a.stats_in + R_.stats_off();
  const float* sdel = a.delta + R_.pt_off();
  const float* slsum = a.lsum + R_.pt_off();
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    const uint32_t vrf = FAST ? f_row + 4 * h * (uint32_t)sizeof(T) : f_row;
    // with the value operands split (the fp32-accurate levels), a tile's
    // per-point values (m, l, delta) travel with its rows in the register
    // set, loaded two tiles ahead as in the slot-owned slice (config 3,
    // slice backward: 8.33 -> 8.01 ms at G = 256, 30.5 -> 29.8 at G = 1024);
    // with bf16 dots they are loaded in the tile's own body (prefetched,
    // the G = 1024 slice backward took 5 % longer)
    constexpr bool PF = GModes<DK>::V == MMA_X6;
    float xA[NB][16], xB[NB][16], fA[NB][16], fB[NB][16], sA[3], sB[3];
    auto load = [&](float (&xn)[NB][16], float (&fn)[NB][16], float (&sn)[3], int t) {
      const int64_t p0 = (int64_t)t * kTile;
      ld_rows<T, NB, FAST>(xn, rows_rsrc(x_b, x_sn, x_w, p0, N), vrx, D, h);
      ld_rows<T, NB, FAST>(fn, rows_rsrc(f_b, f_sn, f_w, p0, N), vrf, DV, h);
      if constexpr (PF) {
        sn[0] = ld_pt(pts_rsrc(sm, p0, N), c);
        sn[1] = ld_pt(pts_rsrc(slsum, p0, N), c);
        sn[2] = ld_pt(pts_rsrc(sdel, p0, N), c);
      }
    };
    auto body = [&](const float (&xf)[NB][16], const float (&ff)[NB][16], const float (&sv)[3],
                    int t, auto par) {
      const int64_t p0 = (int64_t)t * kTile;
      const bool pv = p0 + c < N;
      const float m2 = (PF ? sv[0] : ld_pt(pts_rsrc(sm, p0, N), c)) * kLog2e;
      const float l = PF ? sv[1] : ld_pt(pts_rsrc(slsum, p0, N), c);
      const float delta = PF ? sv[2] : ld_pt(pts_rsrc(sdel, p0, N), c);
      Frag<ML> xq[NB];
#pragma unroll
      for (int k = 0; k < NB; ++k) prep<ML>(xq[k], xf[k]);
      float t2[16], w[16];
      gp_logits<ML, NB>(t2, sq, sq + O_BC, xq, nd, cst, lane);
      // the weights -- and through them Lb -- carry the tile's sign (acc_add)
      constexpr float sg = decltype(par)::sign;
      const float inv_l = pv ? sg / l : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) w[r] = __builtin_amdgcn_exp2f(t2[r] - m2) * inv_l;
      if constexpr (TR) {
        Frag<MV> fq;  // d_out (or fx) rows, split once: omega and d_out^T
        prep<MV>(fq, ff[0]);
        if (!SLICE) {
          // dtokens += w^T d_out
          Frag<MV> oTq, wq, wTq;
          tr_put<MV>(trS, fq, c, h, 0u);
          tr_get<MV>(oTq, trS, lane);
          prep<MV>(wq, w);
          tr_put<MV>(trS, wq, c, h, 0u);
          tr_get<MV>(wTq, trS, lane);
          mma_acc<MV>(dT[0], oTq, wTq, sg);
        }
        Frag<MV> vq;
        lds_get<MV>(vq, sq + O_VR, lane);
        const f32x16 o = mma<MV>(vq, fq, zero16());
        float dsv[16];
        if (SLICE) gp_vec(dsv, sq + O_DS, lane);
        float ab[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) ab[r] = w[r] * ((SLICE ? o[r] + dsv[r] : o[r]) - delta);
        // dW += x^T Lb, db += sum_n Lb from the pieces read back transposed
        Frag<MV> aq, aTq, xTq;
        prep<MV>(aq, ab);
        tr_put<MV>(trS, aq, c, h, 0u);
        tr_get<MV>(aTq, trS, lane);
        tr_put<ML>(trS, xq[0], c, h, 0u);
        tr_get<MV>(xTq, trS, lane);
        mma_acc<MV>(dW[0], xTq, aTq, sg);
        dbacc = fmaf(row_sums<MV>(aTq)[0], sg, dbacc);
        return;
      }
      if (!SLICE) {
        // dtokens += w^T d_out
        float wT[16];
        transpose32(wT, w, lds, c, h);
        Frag<MV> wq;
        prep<MV>(wq, wT);
#pragma unroll
        for (int k = 0; k < NB; ++k)
          if (k == 0 || k < nv) {
            float oT[16];
            transpose32(oT, ff[k], lds, c, h);
            Frag<MV> oq;
            prep<MV>(oq, oT);
            mma_acc<MV>(dT[k], oq, wq, sg);
          }
      }
      f32x16 o = zero16();
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nv) {
          Frag<MV> vq, fq;
          lds_get<MV>(vq, sq + O_VR + k * FWV, lane);
          prep<MV>(fq, ff[k]);
          o = mma<MV>(vq, fq, o);
        }
      float dsv[16];
      if (SLICE) gp_vec(dsv, sq + O_DS, lane);
      float ab[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) ab[r] = w[r] * ((SLICE ? o[r] + dsv[r] : o[r]) - delta);
      float aT[16];
      transpose32(aT, ab, lds, c, h);
      Frag<MV> aq;
      prep<MV>(aq, aT);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nd) {
          float xT[16];
          transpose32(xT, xf[k], lds, c, h);
          Frag<MV> xtq;
          prep<MV>(xtq, xT);
          mma_acc<MV>(dW[k], xtq, aq, sg);
        }
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s += aT[j];
      dbacc = fmaf(s, sg, dbacc);
    };
    FS_TILE_LOOP(load, body, false, FS_ARGS3(xA, fA, sA), FS_ARGS3(xB, fB, sB))
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  const int gg = 32 * gb + c;
  // TR: row_sums gave both lane halves the whole tile's sum
  const float s = (TR ? dbacc : pair_sum(dbacc)) * inv_tau;
  if (gg < G) {
    if (SLICE) {
      float* pw = a.part + ((int64_t)bh * P + pid) * part_floats_slice_bwd(G, D);
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (k == 0 || k < nd)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * k + kmap(r, h);
            if (d < D) pw[(int64_t)gg * D + d] = dW[k][r] * inv_tau;
          }
      if (h == 0) pw[(int64_t)G * D + gg] = s;
    } else {
      float* pw = a.part + ((int64_t)bh * P + pid) * part_floats_deslice_bwd(G, D, DV);
      const int64_t offW = (int64_t)G * DV, offB = offW + (int64_t)G * D;
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        if (k == 0 || k < nv)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = 32 * k + kmap(r, h);
            if (v < DV) pw[(int64_t)gg * DV + v] = dT[k][r];
          }
        if (k == 0 || k < nd)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * k + kmap(r, h);
            if (d < D) pw[offW + (int64_t)gg * D + d] = dW[k][r] * inv_tau;
          }
      }
      if (h == 0) pw[offB + gg] = s;
    }
  }
}

}  // namespace fs
