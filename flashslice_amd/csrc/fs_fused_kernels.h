// Whole-G ("fused") slice/deslice kernel templates for gfx950.
//
// A block is four waves working on the same (b, h): the block stages that
// head's slice projection W (G x D) and its tokens / dz_num (G x DV) in LDS
// once, and each wave owns one point partition pid = 4 * blockIdx.x + wave,
// i.e. the strided tile sequence t = pid, pid + P, ... (a static
// assignment, so per-wave partial sums are deterministic). The whole slot
// axis G (padded to NGB blocks of 32) is held in registers, so the softmax
// over G is exact in one pass and the N x H x G weight tensor never exists
// outside registers. Every dot runs on MFMA: v_mfma_f32_32x32x2_f32 for the
// ieee/tf32/tf32x3 levels and v_mfma_f32_32x32x16_bf16 for the bf16 levels
// (fragment convention: fs_device.h). Slot-indexed sums (z_num, s,
// dtokens, dW, db, dtau) are accumulated per wave and written as per-wave
// partials that fs_reduce.hip sums in a fixed order. The next tile's point
// rows are loaded while the current tile is computed.
//
// Reference kernels these replace: _slice_fwd_kernel (slice_ops.py:554-599),
// _deslice_fwd_kernel (:602-640), _slice_bwd_kernel (:643-710),
// _deslice_bwd_kernel (:713-776).
#pragma once
#include "fs_tile.h"

namespace fs {

// LDS of one block: W [32 NGB][SW], tokens / dz_num [32 NGB][SV] (row
// strides padded so fragment reads are conflict-free), one transpose tile
// per wave.
template <int NGB, int NDB, int NVB> struct Smem {
  static constexpr int GP = 32 * NGB;
  static constexpr int SW = 32 * NDB + 4, SV = 32 * NVB + 4;
  static constexpr int W_OFF = 0, V_OFF = GP * SW, T_OFF = V_OFF + GP * SV;
  static constexpr int TOTAL = T_OFF + kWavesPerBlock * kLdsTile;
};

// Stage a small (G x C) fp32 matrix, zero-padded to (rows x cols), into LDS
// with row stride S; all 256 threads of the block take part.
__device__ __forceinline__ void stage_matrix(float* dst, int S, const float* src, int R, int C,
                                             int rows, int cols) {
  for (int i = threadIdx.x; i < rows * cols; i += 256) {
    const int r = i / cols, col = i - r * cols;
    dst[r * S + col] = (r < R && col < C) ? src[(int64_t)r * C + col] : 0.f;
  }
}

// Block prologue shared by the four kernels: head constants, LDS carve-up,
// and the logits operands (W as the A operand [g-outer, d-inner] in
// registers, bias * log2(e) / tau per output slot, -inf on padded slots).
#define FS_PROLOGUE(NGB, NDB, NVB)                                                  \
  using SM = Smem<NGB, NDB, NVB>;                                                   \
  __shared__ float smem[SM::TOTAL];                                                 \
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;                       \
  const int c = lane & 31, h = lane >> 5;                                           \
  const int bh = blockIdx.y;                                                        \
  const int b = bh / a.H, hd = bh - b * a.H;                                       \
  const int pid = blockIdx.x * kWavesPerBlock + wid;                                \
  const int G = a.G, D = a.D, DV = a.DV, N = a.N;                                   \
  float* sW = smem + SM::W_OFF;                                                     \
  float* sV = smem + SM::V_OFF;                                                     \
  float* lds = smem + SM::T_OFF + wid * kLdsTile;                                   \
  const float* Wp = a.W + b * a.swb + hd * a.swh;                                   \
  const float* Bp = a.bias + b * a.sbb + hd * a.sbh;                                \
  const float tauf = a.tau[hd];                                                     \
  const float cst = (float)(1.4426950408889634 / (double)tauf);                    \
  const float inv_tau = 1.f / tauf;                                                 \
  const bool fast = a.fast != 0;                                                    \
  (void)inv_tau; (void)sV; (void)lds; (void)DV;                                     \
  stage_matrix(sW, SM::SW, Wp, G, D, SM::GP, 32 * NDB);                             \
  if (a.tok) stage_matrix(sV, SM::SV, a.tok + (int64_t)bh * G * DV, G, DV, SM::GP, 32 * NVB); \
  __syncthreads();                                                                  \
  float wA[NGB][NDB][16], bc[NGB][16];                                              \
  _Pragma("unroll") for (int gb = 0; gb < NGB; ++gb) {                              \
    _Pragma("unroll") for (int db = 0; db < NDB; ++db)                              \
      lds_frag_rowouter(wA[gb][db], sW, SM::SW, 32 * gb, 32 * db, c, h);            \
    _Pragma("unroll") for (int r = 0; r < 16; ++r) {                                \
      const int g = 32 * gb + kmap(r, h);                                           \
      bc[gb][r] = g < G ? Bp[g] * cst : kNoSlot;                                  \
    }                                                                               \
  }

// ------------------------------------------------------------------ slice fwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, 2) void k_fused_slice_fwd(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  FS_PROLOGUE(NGB, NDB, NVB)
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
    const int p0 = t * kTile;
    load_rows<T, NDB>(xn, xb, a.sxn, p0 + c, N, D, fast, a.vec_x, h);
    // fx as [v-outer, point-inner]: one coalesced row read per register
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int pj = p0 + kmap(j, h), v = 32 * vb + c;
        if (fast)
          fn[vb][j] = to_f<T>(fb[(int64_t)(pj < N ? pj : N - 1) * a.sfn + v]);
        else
          fn[vb][j] = (pj < N && v < DV) ? to_f<T>(fb[(int64_t)pj * a.sfn + v]) : 0.f;
      }
  };
  if (pid < a.ntiles) load_tile(pid);
  for (int t = pid; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16], fT[NVB][16];
    copy_frags<T, NDB>(xf, xn);
    copy_frags<T, NVB>(fT, fn);
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
  float* pw = a.part + ((int64_t)bh * a.P + pid) * part_floats_slice_fwd(G, DV);
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
  FS_PROLOGUE(NGB, NDB, NVB)
  float tC[NVB][NGB][16];  // tokens as [v-outer, g-inner]
#pragma unroll
  for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb)
      lds_frag_colouter(tC[vb][gb], sV, SM::SV, 32 * gb, 32 * vb, c, h);
  const T* xb = (const T*)a.x + b * a.sxb + hd * a.sxh;
  T* ob = (T*)a.o1 + b * a.s1b + hd * a.s1h;
  float xn[NDB][16];
  if (pid < a.ntiles) load_rows<T, NDB>(xn, xb, a.sxn, pid * kTile + c, N, D, fast, a.vec_x, h);
  for (int t = pid; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16];
    copy_frags<T, NDB>(xf, xn);
    if (t + a.P < a.ntiles)
      load_rows<T, NDB>(xn, xb, a.sxn, (t + a.P) * kTile + c, N, D, fast, a.vec_x, h);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    store_stats(a.stats_out, bh, N, p, pv, h, m2, lsum);
    // out as [v-outer, point-inner]: whole-row stores
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) o = mma32<MV>(w[gb], tC[vb][gb], o);
      store_cols<T>(ob, a.s1n, o, t * kTile, N, 32 * vb, DV, c, h);
    }
  }
}

// ------------------------------------------------------------------ slice bwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, 2) void k_fused_slice_bwd(Args a) {
  constexpr int ML = Modes<DK>::L, MV = Modes<DK>::V;
  FS_PROLOGUE(NGB, NDB, NVB)
  // sW holds W, sV holds dz_num; dz_num is read per tile as [g-outer,
  // v-inner] (omega) and [v-outer, g-inner] (dfx), W as [d-outer, g-inner].
  const float* Sp = a.ds + (int64_t)bh * G;
  float dsv[NGB][16];  // d s per output slot
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int g = 32 * gb + kmap(r, h);
      dsv[gb][r] = g < G ? Sp[g] : 0.f;
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
    load_rows<T, NDB>(xn, xb, a.sxn, p, N, D, fast, a.vec_x, h);
    load_rows<T, NVB>(fnx, fb, a.sfn, p, N, DV, fast, a.vec_f, h);
  };
  if (pid < a.ntiles) load_tile(pid);
  for (int t = pid; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16], ff[NVB][16];
    copy_frags<T, NDB>(xf, xn);
    copy_frags<T, NVB>(ff, fnx);
    if (t + a.P < a.ntiles) load_tile(t + a.P);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    // dfx = w dz_num
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) {
        float zc[16];
        lds_frag_colouter(zc, sV, SM::SV, 32 * gb, 32 * vb, c, h);
        o = mma32<MV>(w[gb], zc, o);
      }
      store_cols<T>(dfb, a.s2n, o, t * kTile, N, 32 * vb, DV, c, h);
    }
    // omega = fx . dz_num + ds
    float om[NGB][16];
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      f32x16 o = zero16();
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) {
        float zr[16];
        lds_frag_rowouter(zr, sV, SM::SV, 32 * gb, 32 * vb, c, h);
        o = mma32<MV>(zr, ff[vb], o);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) om[gb][r] = o[r] + dsv[gb][r];
    }
    dtacc += jacobian_tile<NGB>(om, w, t2, m2, inv_tau, pv, h);
    // dx = ab W
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) {
        float wc[16];
        lds_frag_colouter(wc, sW, SM::SW, 32 * gb, 32 * db, c, h);
        o = mma32<MV>(om[gb], wc, o);
      }
      store_cols<T>(dxb, a.s1n, o, t * kTile, N, 32 * db, D, c, h);
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
  float* pw = a.part + ((int64_t)bh * a.P + pid) * part_floats_slice_bwd(G, D);
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
  FS_PROLOGUE(NGB, NDB, NVB)
  // sW holds W (read as [d-outer, g-inner] for dx), sV the tokens (read as
  // [g-outer, v-inner] for omega).
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
    load_rows<T, NDB>(xn, xb, a.sxn, p, N, D, fast, a.vec_x, h);
    load_rows<T, NVB>(fnx, ob, a.sfn, p, N, DV, fast, a.vec_f, h);
  };
  if (pid < a.ntiles) load_tile(pid);
  for (int t = pid; t < a.ntiles; t += a.P) {
    const int p = t * kTile + c;
    const bool pv = p < N;
    float xf[NDB][16], of[NVB][16];
    copy_frags<T, NDB>(xf, xn);
    copy_frags<T, NVB>(of, fnx);
    if (t + a.P < a.ntiles) load_tile(t + a.P);
    float t2[NGB][16], w[NGB][16], m2, lsum;
    logits_tile<ML, NGB, NDB>(t2, wA, xf, bc, cst);
    softmax_tile<NGB>(w, m2, lsum, t2, pv);
    // dtokens += w^T d_out (rows of d_out beyond N meet zero weights)
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
      for (int vb = 0; vb < NVB; ++vb) {
        float tr[16];
        lds_frag_rowouter(tr, sV, SM::SV, 32 * gb, 32 * vb, c, h);
        o = mma32<MV>(tr, of[vb], o);
      }
      from16(om[gb], o);
    }
    dtacc += jacobian_tile<NGB>(om, w, t2, m2, inv_tau, pv, h);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      f32x16 o = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) {
        float wc[16];
        lds_frag_colouter(wc, sW, SM::SW, 32 * gb, 32 * db, c, h);
        o = mma32<MV>(om[gb], wc, o);
      }
      store_cols<T>(dxb, a.s1n, o, t * kTile, N, 32 * db, D, c, h);
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
  float* pw = a.part + ((int64_t)bh * a.P + pid) * part_floats_deslice_bwd(G, D, DV);
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
// one per (K, T, DK), so they compile in parallel. Grid: (P / 4, B * H).
template <int K, typename T, int DK>
hipError_t fused_launch(const Args& a, hipStream_t st) {
  const int g = blocks_of(a.G), d = blocks_of(a.D), v = blocks_of(a.DV);
  const dim3 grid(a.P / kWavesPerBlock, a.B * a.H), block(256);
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
