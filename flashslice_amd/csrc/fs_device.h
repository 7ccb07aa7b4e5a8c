// Device-side building blocks of the FlashSlice HIP kernels (gfx950 / CDNA4).
//
// Fragment convention (one wave64, one 32 x 32 tile):
//   A "fragment" is 16 floats per lane. Lane l = c + 32 h (c = l % 32,
//   h = l / 32) holds element j of the 32 x 32 tile Y[outer = c][inner =
//   kmap(j, h)], kmap(j, h) = 8 (j / 4) + 4 h + (j % 4).
//   This is exactly the accumulator layout of v_mfma_f32_32x32x2_f32 /
//   v_mfma_f32_32x32x16_bf16: output register r of lane l holds
//   C[row = kmap(r, h)][col = c]. So a product C = A B (C[i][j] = sum_k
//   A[i][k] B[k][j]) takes A as the fragment [i-outer, k-inner] and B as
//   [j-outer, k-inner] and yields [j-outer, i-inner] -- the output of one
//   product is directly the operand of the next whenever its row index is
//   the next contraction index (the K permutation kmap is the same on both
//   sides, so any bijection is a valid contraction order).
//
// Everything the kernels compute per point (logits, softmax weights, the
// Jacobian) lives in [point-outer, slot-inner] fragments: the softmax over
// G is a register-local reduction plus one exchange with lane l ^ 32.
// Slot-indexed sums over points (z_num, dtokens, dW) need the transposed
// fragments, formed through a per-wave LDS tile (transpose32).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fs {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

constexpr int kLdsStride = 36;         // floats per LDS transpose row (conflict-free)
constexpr int kLdsTile = 32 * kLdsStride;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// dot modes (reference slice_ops.py:338-343): 0 ieee, 1 tf32, 2 bf16v,
// 3 bf16, 4 tf32x3. On gfx950 (no xf32 MFMA) levels 0/1/4 all run the
// exact fp32 MFMA; 2 runs the value dots in bf16; 3 runs every dot in bf16.
enum MmaMode { MMA_F32 = 0, MMA_BF16 = 1, MMA_X6 = 2 };

__device__ __forceinline__ int kmap(int j, int h) { return 8 * (j >> 2) + 4 * h + (j & 3); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// C += A B over one 32-wide contraction block (see the fragment convention).
template <int MODE>
__device__ __forceinline__ f32x16 mma32(const float (&a)[16], const float (&b)[16], f32x16 c) {
  if constexpr (MODE == MMA_F32) {
#pragma unroll
    for (int j = 0; j < 16; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], c, 0, 0, 0);
  } else {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 av, bv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        av[e] = (__bf16)a[8 * s + e];
        bv[e] = (__bf16)b[8 * s + e];
      }
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
    }
  }
  return c;
}


// A value the wave holds in every lane alike, moved to scalar registers (the
// compiler cannot always prove it uniform, e.g. after a load through a
// vector register).
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Accumulators that run over a wave's whole stream of point tiles (z_num,
// dtokens, dW) are kept free of the bf16 MFMA's rounding bias. On MI355X the
// MFMA sums its products with a small downward bias when they span many
// binades (softmax weights do): measured at about -0.03 x 2^-24 x the largest
// product per MFMA, the same with an operand negated. Chained over hundreds
// of tiles, and through an accumulator whose magnitude keeps growing, that
// bias shifted every slot's z_num by the same few 1e-6 (relative) at
// N = 1e6. Hence:
//   * each tile's block is summed by the MFMAs from zero and added to acc in
//     fp32 (round to nearest even), so the bias is relative to one tile's
//     sum, not to the running total;
//   * every other tile negates one MFMA operand and subtracts its block
//     (`sgn` = -1): the bias then enters with alternating signs and cancels
//     while the values add up unchanged (t * -1 is exact; fma(t, -1, acc) is
//     the correctly rounded acc - t).
// `tile_sign` gives the sign for a wave's i-th tile; the ping-pong tile loop
// (FS_TILE_LOOP) hands its bodies the parity as a type (TileEven / TileOdd)
// instead, so that the sign folds into the code (negation as a source
// modifier, fma(t, -1, acc) as a subtraction).
__device__ __forceinline__ float tile_sign(int i) { return (i & 1) ? -1.f : 1.f; }
struct TileEven {
  static constexpr float sign = 1.f;
};
struct TileOdd {
  static constexpr float sign = -1.f;
};
__device__ __forceinline__ void acc_add(f32x16& acc, const f32x16& t, float sgn) {
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = fmaf(t[i], sgn, acc[i]);
}
template <int MODE>
__device__ __forceinline__ void mma32_acc(f32x16& acc, const float (&a)[16], const float (&b)[16],
                                          float sgn) {
  acc_add(acc, mma32<MODE>(a, b, zero16()), sgn);
}

// Scheduling hints for the machine scheduler (no instructions are emitted).
// A tile's steps form short dependent chains (a split on the VALU, then an
// MFMA chain on its pieces); left to itself the scheduler issues each MFMA
// chain back to back, so one wave keeps only one of the two pipes busy.
// sched_fence() closes a scheduling region; sched_mfma_valu<N, K>() asks for
// the region's next N MFMAs to be issued one at a time, each followed by K
// VALU instructions of the independent work placed in the same region.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }
template <int N, int K> __device__ __forceinline__ void sched_mfma_valu() {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, K, 0);
  }
}

// ---------------------------------------------------------------- dtype I/O
template <typename T> __device__ __forceinline__ float to_f(T v);
template <> __device__ __forceinline__ float to_f<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f<__bf16>(__bf16 v) { return (float)v; }
template <> __device__ __forceinline__ float to_f<_Float16>(_Float16 v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f(float v);
template <> __device__ __forceinline__ float from_f<float>(float v) { return v; }
template <> __device__ __forceinline__ __bf16 from_f<__bf16>(float v) { return (__bf16)v; }
template <> __device__ __forceinline__ _Float16 from_f<_Float16>(float v) { return (_Float16)v; }

template <typename T> struct Vec4;
template <> struct Vec4<float> { typedef float __attribute__((ext_vector_type(4))) type; };
template <> struct Vec4<__bf16> { typedef __bf16 __attribute__((ext_vector_type(4))) type; };
template <> struct Vec4<_Float16> { typedef _Float16 __attribute__((ext_vector_type(4))) type; };

// Load the [point-outer, column-inner] fragment of a 32-point tile of a
// (B, N, H, C) tensor: lane (c, h) reads row p = p0 + c, columns
// c0 + kmap(j, h). `row` points at element (b, p0 + c, h_head, 0) (only
// dereferenced when p < N). Columns >= C and rows >= N read as zero.
// `vec`: rows are 4-element aligned and C % 4 == 0, so each group of four
// columns is one vector load.
template <typename T>
__device__ __forceinline__ void load_frag_rows(float (&f)[16], const T* row, bool pvalid, int c0,
                                               int C, bool vec, int h) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = c0 + 8 * q + 4 * h;
    if (pvalid && vec && col + 3 < C) {
      typename Vec4<T>::type v = *reinterpret_cast<const typename Vec4<T>::type*>(row + col);
      f[4 * q + 0] = to_f<T>(v[0]);
      f[4 * q + 1] = to_f<T>(v[1]);
      f[4 * q + 2] = to_f<T>(v[2]);
      f[4 * q + 3] = to_f<T>(v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        f[4 * q + i] = (pvalid && col + i < C) ? to_f<T>(row[col + i]) : 0.f;
    }
  }
}

// The branch-free form of load_frag_rows for full tiles of aligned rows
// whose width is a multiple of 32: four vector loads of the (clamped,
// always valid) row. Points beyond N read row N - 1; callers zero their
// weights.
template <typename T>
__device__ __forceinline__ void load_frag_rows_fast(float (&f)[16], const T* row, int c0, int h) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    typename Vec4<T>::type v =
        *reinterpret_cast<const typename Vec4<T>::type*>(row + c0 + 8 * q + 4 * h);
    f[4 * q + 0] = to_f<T>(v[0]);
    f[4 * q + 1] = to_f<T>(v[1]);
    f[4 * q + 2] = to_f<T>(v[2]);
    f[4 * q + 3] = to_f<T>(v[3]);
  }
}

// Store a [point-outer, column-inner] fragment: row p (lane c), columns
// c0 + kmap(r, h), masked to p < N and column < C.
template <typename T>
__device__ __forceinline__ void store_frag_rows(T* row, const f32x16& v, bool pvalid, int c0,
                                                int C, bool vec, int h) {
  if (!pvalid) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = c0 + 8 * q + 4 * h;
    if (vec && col + 3 < C) {
      typename Vec4<T>::type o;
      o[0] = from_f<T>(v[4 * q + 0]);
      o[1] = from_f<T>(v[4 * q + 1]);
      o[2] = from_f<T>(v[4 * q + 2]);
      o[3] = from_f<T>(v[4 * q + 3]);
      *reinterpret_cast<typename Vec4<T>::type*>(row + col) = o;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (col + i < C) row[col + i] = from_f<T>(v[4 * q + i]);
    }
  }
}

// Fragment of a small contiguous fp32 matrix M (R rows x C cols, row
// stride C) read as [row-outer, col-inner]: lane (c, h) gets
// M[r0 + c][c0 + kmap(j, h)], zero outside.
__device__ __forceinline__ void load_frag_mat_rowouter(float (&f)[16], const float* M, int r0,
                                                       int R, int c0, int C, int c, int h) {
  const int r = r0 + c;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int col = c0 + kmap(j, h);
    f[j] = (r < R && col < C) ? M[(int64_t)r * C + col] : 0.f;
  }
}

// The transposed read of the same matrix: [col-outer, row-inner]: lane
// (c, h) gets M[r0 + kmap(j, h)][c0 + c].
__device__ __forceinline__ void load_frag_mat_colouter(float (&f)[16], const float* M, int r0,
                                                       int R, int c0, int C, int c, int h) {
  const int col = c0 + c;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int r = r0 + kmap(j, h);
    f[j] = (r < R && col < C) ? M[(int64_t)r * C + col] : 0.f;
  }
}

// Fragments of a matrix staged in LDS with row stride S (floats, S % 4 == 0
// and S / 4 odd so that 8 consecutive rows fall in distinct bank groups):
// [row-outer, col-inner] (four 16-byte reads) and [col-outer, row-inner]
// (sixteen 4-byte reads), both bank-conflict-free.
__device__ __forceinline__ void lds_frag_rowouter(float (&f)[16], const float* M, int S, int r0,
                                                  int c0, int c, int h) {
  const float* row = M + (r0 + c) * S + c0 + 4 * h;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 v = *reinterpret_cast<const float4*>(row + 8 * q);
    f[4 * q + 0] = v.x;
    f[4 * q + 1] = v.y;
    f[4 * q + 2] = v.z;
    f[4 * q + 3] = v.w;
  }
}
__device__ __forceinline__ void lds_frag_colouter(float (&f)[16], const float* M, int S, int r0,
                                                  int c0, int c, int h) {
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = M[(r0 + kmap(j, h)) * S + c0 + c];
}

// A per-slot vector v[0..31] in LDS as lane half h's 16 values v[kmap(j, h)]
// (four 16-byte reads; the 32 lanes of a half read the same words).
__device__ __forceinline__ void lds_frag_vec(float (&f)[16], const float* v, int h) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 t = *reinterpret_cast<const float4*>(v + 8 * q + 4 * h);
    f[4 * q + 0] = t.x;
    f[4 * q + 1] = t.y;
    f[4 * q + 2] = t.z;
    f[4 * q + 3] = t.w;
  }
}

// [a-outer, b-inner] -> [b-outer, a-inner] through a wave-private LDS tile
// of 32 x 36 floats. Writes are four 16-byte stores per lane, reads sixteen
// 4-byte loads; both conflict-free. LDS instructions of one wave complete in
// issue order, so no barrier is needed between the phases; the wave barriers
// only keep the compiler from moving LDS accesses across them.
__device__ __forceinline__ void transpose32(float (&y)[16], const float (&x)[16], float* lds, int c,
                                            int h) {
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float4 v = make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
    *reinterpret_cast<float4*>(lds + c * kLdsStride + 8 * q + 4 * h) = v;
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < 16; ++j) y[j] = lds[kmap(j, h) * kLdsStride + c];
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ f32x16 as16(const float (&x)[16]) {
  f32x16 v;
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = x[i];
  return v;
}
__device__ __forceinline__ void from16(float (&x)[16], const f32x16& v) {
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = v[i];
}

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Fixed-order sum over the 32 lanes that share h (butterfly; every lane ends
// with the total of its half). Deterministic: the tree shape is fixed.
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

}  // namespace fs
