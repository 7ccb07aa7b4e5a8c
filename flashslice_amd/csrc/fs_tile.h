// Per-tile building blocks shared by the whole-G and the G-blocked kernels:
// logits on MFMA, the softmax over slots of a point pair, the softmax
// Jacobian, and row loads/stores of (B, N, H, C) point tensors.
#pragma once
#include "fs_device.h"
#include "fs_internal.h"
#include "fs_io.h"

namespace fs {

// Logits of slots that do not exist (g >= G): finite and far below any real
// logit, so exp2 gives exactly 0 and 0 * (t2 - m2) stays 0.
constexpr float kNoSlot = -1e30f;

// DK: 0 = every dot fp32 MFMA; 1 = value dots bf16 (reference level 2,
// "bf16v"); 2 = every dot bf16 (level 3).
template <int DK> struct Modes {
  static constexpr int L = (DK == 2) ? MMA_BF16 : MMA_F32;
  static constexpr int V = (DK >= 1) ? MMA_BF16 : MMA_F32;
};

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
// point). Shifts t2 in place to t2 - m2 (the exponent of each weight, which
// the backward's temperature term reuses) and returns w (zero for points
// beyond N), the row max m2 (log2 units) and the row sum. The row sum is
// formed in a fixed order (lane-local, then the partner), so both lanes of a
// pair hold the same value.
template <int NGB>
__device__ __forceinline__ void softmax_tile(float (&w)[NGB][16], float& m2, float& lsum,
                                             float (&t2)[NGB][16], bool pv) {
  float m = -INFINITY;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, t2[gb][r]);
  m = pair_max(m);
  float l = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      t2[gb][r] -= m;
      const float e = __builtin_amdgcn_exp2f(t2[gb][r]);
      w[gb][r] = e;
      l += e;
    }
  l = pair_sum(l);
  const float inv = pv ? 1.f / l : 0.f;  // correctly rounded (no fast-math)
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) w[gb][r] *= inv;
  m2 = m;
  lsum = l;
}

// The row max as consumers of saved statistics reconstruct it: stored in
// natural units (m = m2 ln 2) and read back as m * log2(e). A row sum that is
// to normalise weights formed against that value must be taken against it
// too, or every weight of the row carries the same relative error
// 2^(m2 - m2') and the row stops summing to one.
__device__ __forceinline__ float stats_max_roundtrip(float m2) { return (m2 * kLn2) * kLog2e; }

// Softmax statistics of one point in the reference layout (B, H, 2, N):
// the row max of the natural-unit logits and the sum of exponentials
// against the max consumers will read back (reference blocked.py:1329-1335).
// `sm` is this sample and head's max row (Rows::stats_off), its sum row NS
// floats further. `l` is the sum against `m2`; it is rescaled once to the
// round-tripped max. Written by lane h = 0 of each pair.
// `l_roundtrip`: l is already the sum against stats_max_roundtrip(m2).
__device__ __forceinline__ void store_stats(float* sm, int64_t NS, int p, bool pv, int h,
                                            float m2, float l, bool l_roundtrip = false) {
  if (sm && pv && h == 0) {
    sm[p] = m2 * kLn2;
    sm[NS + p] = l_roundtrip ? l : l * __builtin_amdgcn_exp2f(m2 - stats_max_roundtrip(m2));
  }
}

// The softmax Jacobian of one tile given omega = dL/dw: Lb = w (omega -
// delta), delta = sum_g w omega, both from the same rounded products.
// Overwrites om with Lb (the callers apply 1 / tau: to the W operand of dx
// and to the dW, db partials) and returns the row term sum_g Lb (t2 - m2)
// of the temperature gradient (natural units up to a factor ln 2; zero on
// lanes h = 1 and on points beyond N). `t2s` holds t2 - m2 (softmax_tile's
// shifted logits). Shifting the logits by the row max is exact in real
// arithmetic (sum_g Lb = 0) and keeps the terms small.
template <int NGB>
__device__ __forceinline__ float jacobian_tile(float (&om)[NGB][16], const float (&w)[NGB][16],
                                               const float (&t2s)[NGB][16], bool pv, int h) {
  float d = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb)
#pragma unroll
    for (int r = 0; r < 16; ++r) d += w[gb][r] * om[gb][r];
  d = pair_sum(d);
  float rt = 0.f;  // per slot block, then across blocks (a cancelling sum)
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    float rb = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float lb = w[gb][r] * (om[gb][r] - d);
      rb = fmaf(lb, t2s[gb][r], rb);
      om[gb][r] = lb;
    }
    rt += rb;
  }
  rt = pair_sum(rt);
  return (pv && h == 0) ? rt : 0.f;
}

// store_stats for the tile loops that address points through buffer
// resources: `sm` / `sl` are the max and sum rows of this (b, h) (null: no
// statistics); points beyond N and lanes h = 1 store nothing.
__device__ __forceinline__ void store_stats_at(Rsrc rm, Rsrc rl, int c, int h, float m2, float l,
                                               bool l_roundtrip = false) {
  st_pt(rm, c, h, m2 * kLn2);
  st_pt(rl, c, h, l_roundtrip ? l : l * __builtin_amdgcn_exp2f(m2 - stats_max_roundtrip(m2)));
}
__device__ __forceinline__ void store_stats_tile(const float* sm, const float* sl, int64_t p0,
                                                 int N, int c, int h, float m2, float l,
                                                 bool l_roundtrip = false) {
  store_stats_at(pts_rsrc(sm, p0, N), pts_rsrc(sl, p0, N), c, h, m2, l, l_roundtrip);
}

// A 32-point tile's [point-outer, column-inner] fragments of one (B, N, H, C)
// tensor: the fast form on full aligned rows (row clamped to N - 1), the
// masked form otherwise.
template <typename T, int NB>
__device__ __forceinline__ void load_rows(float (&f)[NB][16], const T* base, int64_t sn, int p,
                                          int N, int C, bool fast, bool vec, int h) {
  if (fast) {
    const T* row = base + (int64_t)(p < N ? p : N - 1) * sn;
#pragma unroll
    for (int k = 0; k < NB; ++k) load_frag_rows_fast<T>(f[k], row, 32 * k, h);
  } else {
    const T* row = base + (int64_t)p * sn;
#pragma unroll
    for (int k = 0; k < NB; ++k) load_frag_rows<T>(f[k], row, p < N, 32 * k, C, vec, h);
  }
}

template <typename T>
__device__ __forceinline__ void store_rows(T* row, const f32x16& v, bool pv, int c0, int C,
                                           bool fast, bool vec, int h) {
  if (fast) {
    if (!pv) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      typename Vec4<T>::type o;
      o[0] = from_f<T>(v[4 * q + 0]);
      o[1] = from_f<T>(v[4 * q + 1]);
      o[2] = from_f<T>(v[4 * q + 2]);
      o[3] = from_f<T>(v[4 * q + 3]);
      *reinterpret_cast<typename Vec4<T>::type*>(row + c0 + 8 * q + 4 * h) = o;
    }
  } else {
    store_frag_rows<T>(row, v, pv, c0, C, vec, h);
  }
}

// A per-point value held by the lane pair of each point (c, both h) as the
// 16 values of a [column-outer, point-inner] fragment: o[r] = value of point
// kmap(r, h). Through a 32-float wave-private LDS slot.
__device__ __forceinline__ void gather_rows(float (&o)[16], float v, float* lds, int c, int h) {
  __builtin_amdgcn_wave_barrier();
  if (h == 0) lds[c] = v;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 t = *reinterpret_cast<const float4*>(lds + 8 * q + 4 * h);
    o[4 * q + 0] = t.x;
    o[4 * q + 1] = t.y;
    o[4 * q + 2] = t.z;
    o[4 * q + 3] = t.w;
  }
  __builtin_amdgcn_wave_barrier();
}

// Store a [column-outer, point-inner] fragment of a (B, N, H, C) tensor:
// lane (c, h) writes column c0 + c of points p0 + kmap(r, h), so every store
// instruction writes two whole contiguous 32-column row segments (128 B in
// fp32) -- the write pattern HBM streams at full rate. `base` points at
// element (b, 0, head, 0). Points >= N and columns >= C are skipped.
template <typename T>
__device__ __forceinline__ void store_cols(T* base, int64_t sn, const f32x16& v, int p0, int N,
                                           int c0, int C, int c, int h) {
  const int col = c0 + c;
  if (col >= C) return;
  T* colp = base + col;
  const int pb = p0 + 4 * h;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int p = pb + 8 * (r >> 2) + (r & 3);
    if (p < N) colp[(int64_t)p * sn] = from_f<T>(v[r]);
  }
}

template <typename T, int NB>
__device__ __forceinline__ void copy_frags(float (&dst)[NB][16], const float (&src)[NB][16]) {
#pragma unroll
  for (int k = 0; k < NB; ++k)
#pragma unroll
    for (int j = 0; j < 16; ++j) dst[k][j] = src[k][j];
}

// First point of the wave's tile t (of the sequence pid, pid + P, ... below
// ntiles). With rev set the sequence covers the tiles last-first (tile t
// holds the points of tile ntiles - 1 - t), and the whole-G prologue maps
// the blocks to (b, h) pairs last-first as well: a grid that takes several
// dispatch rounds streams its pairs in blockIdx.y order, so that a kernel
// which follows one that swept in order starts on the pairs and points its
// predecessor touched last, part of which the 256 MB last-level cache still
// holds. An index at or past ntiles (a prefetch past the wave's last tile)
// stays past the end.
__device__ __forceinline__ int64_t tile_p0(int t, int ntiles, int rev) {
  return (int64_t)(rev && t < ntiles ? ntiles - 1 - t : t) * kTile;
}

// Issue priority of a wave from its remaining tiles (after tile t of the
// sequence pid, pid + P, ... below ntiles): the quarter of its work still
// ahead of it, 3 (all of it) down to 0. Waves of one SIMD that share a
// priority level issue oldest first, which on MI355X let the waves resident
// together finish the same number of tiles up to 1.6x apart (per-block
// timestamps), leaving a tail in which a fraction of the resident waves
// streams alone; with the level falling as a wave gets ahead, the waves that
// lag are served first and the resident waves finish close together
// (FS_TILE_LOOP with BAL; measured faster for the whole-G kernels at C2,
// neutral to slower for the G-blocked kernels, which do without it).
__device__ __forceinline__ void balance_prio(int t, int pid, int ntiles, int P) {
  const int left = (ntiles - 1 - t) / P, total = (ntiles - 1 - pid) / P + 1;
  const int l4 = 4 * left;
  if (l4 >= 3 * total) __builtin_amdgcn_s_setprio(3);
  else if (l4 >= 2 * total) __builtin_amdgcn_s_setprio(2);
  else if (l4 >= total) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// The tile loop of the point-streaming kernels (wave pid owns tiles pid,
// pid + a.P, ...): two register sets of point
// rows alternate, each reloaded (two tiles ahead) right after the tile it
// held is computed, so no registers are copied between iterations. The first
// pass is peeled so that the loop is entered with the same memory operations
// outstanding as on every back edge: the compiler then waits only for the
// rows a tile needs, never for the stores still in flight. A load beyond the
// last tile reads an empty range (zeros, no memory traffic). The caller's
// scope defines ntiles_, the tiles of its (b, h).
#define FS_TILE_LOOP(LOAD, BODY, BAL, A_ARGS, B_ARGS)                                     \
  {                                                                                       \
    LOAD(A_ARGS, pid);                                                                    \
    LOAD(B_ARGS, pid + a.P);                                                              \
    FS_TILE_LOOP_BODY_(LOAD, BODY, BAL, (A_ARGS), (B_ARGS))                               \
  }
// The same loop entered with the first two loads (tiles pid and pid + a.P
// into A and B) already issued.
#define FS_TILE_LOOP_LOADED(LOAD, BODY, BAL, A_ARGS, B_ARGS)                              \
  FS_TILE_LOOP_BODY_(LOAD, BODY, BAL, (A_ARGS), (B_ARGS))
// (A and B come parenthesised: a register set may be a comma-separated
// list, FS_ARGS2)
#define FS_UNPAREN_(...) __VA_ARGS__
#define FS_TILE_LOOP_BODY_(LOAD, BODY, BAL, A_P, B_P)                                     \
  {                                                                                       \
    int t_ = pid;                                                                         \
    if (t_ < ntiles_) {                                                                   \
      BODY(FS_UNPAREN_ A_P, t_, TileEven());                                              \
      LOAD(FS_UNPAREN_ A_P, t_ + 2 * a.P);                                                \
      if constexpr (BAL) balance_prio(t_, pid, ntiles_, a.P);                             \
      t_ += a.P;                                                                          \
      while (t_ < ntiles_) {                                                              \
        BODY(FS_UNPAREN_ B_P, t_, TileOdd());                                             \
        LOAD(FS_UNPAREN_ B_P, t_ + 2 * a.P);                                              \
        if constexpr (BAL) balance_prio(t_, pid, ntiles_, a.P);                           \
        t_ += a.P;                                                                        \
        if (t_ >= ntiles_) break;                                                         \
        BODY(FS_UNPAREN_ A_P, t_, TileEven());                                            \
        LOAD(FS_UNPAREN_ A_P, t_ + 2 * a.P);                                              \
        if constexpr (BAL) balance_prio(t_, pid, ntiles_, a.P);                           \
        t_ += a.P;                                                                        \
      }                                                                                   \
    }                                                                                     \
  }
#define FS_ARGS2(X, Y) X, Y
#define FS_ARGS3(X, Y, Z) X, Y, Z

}  // namespace fs
