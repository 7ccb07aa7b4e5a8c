// Point-tensor I/O through buffer resources (gfx950 raw buffer loads/stores).
//
// A kernel addresses one (b, h) slice of a (B, N, H, C) tensor per 32-point
// tile through a buffer resource whose base is the tile's first row and whose
// range ends at row N. Out-of-range loads return zero and out-of-range stores
// are dropped by the hardware, so the tail tile, tiles beyond the last one
// (the prefetch of a wave's final iteration) and masked columns (offset
// kOff) need no branches: every load and store of the tile loops is issued
// unconditionally, which lets the compiler wait for exactly the loads an
// instruction needs instead of draining every outstanding store.
//
// Offsets inside a tile are 32-bit byte offsets in the VGPR operand (the
// scalar offset operand stays 0; only the vector and immediate offsets are
// range checked). The host checks 32 * row stride < 2^31 bytes, so every
// in-tile offset and every kOff + in-tile offset stays below 2^32.
#pragma once
#include "fs_device.h"

namespace fs {

typedef __amdgpu_buffer_rsrc_t Rsrc;

// Word 3 of a raw buffer resource on gfx9-class GPUs: 32-bit data format
// (any nonzero format enables untyped buffer_load/store_dword*).
constexpr int kRsrcWord3 = 0x00020000;
// An offset beyond every resource built here (ranges are clamped below 2^31).
constexpr uint32_t kOff = 0x80000000u;
// Cache policy of the point streams: the default one. (Non-temporal loads
// and stores -- each byte is touched once per kernel -- measured 20 %
// slower on MI355X: the stores' 128-byte row segments are combined in L2.)
constexpr int kStream = 0;

// Rows [p0, N) of a slice with row stride snb bytes whose rows are rowb
// bytes wide (the range ends with row N - 1, so rows >= N fall outside it
// whenever snb >= rowb; with snb < rowb -- broadcast or overlapping input
// rows -- every row is still inside it). Empty when p0 >= N.
__device__ __forceinline__ Rsrc rows_rsrc(const void* base, int64_t snb, int64_t rowb, int64_t p0,
                                          int64_t N) {
  int64_t rem = p0 < N ? (N - 1 - p0) * snb + rowb : 0;
  rem = rem > 0x7fffffff ? 0x7fffffff : rem;
  const char* p = (const char*)base + (p0 < N ? p0 : 0) * snb;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), (short)0, (int)rem, kRsrcWord3);
}

// rows_rsrc formed with selects instead of a branch (the compiler branches
// over the 64-bit multiply of the form above): one multiply of the start row
// clamped to N. Used inside the tile bodies whose steps are interleaved by
// scheduling hints, where a branch would end the scheduling region; the
// branching form costs fewer registers where that matters more.
__device__ __forceinline__ Rsrc rows_rsrc_sel(const void* base, int64_t snb, int64_t rowb,
                                              int64_t p0, int64_t N) {
  const bool in = p0 < N;
  const int64_t off = (in ? p0 : N) * snb;
  int64_t rem = (N - 1) * snb + rowb - off;
  rem = !in ? 0 : rem > 0x7fffffff ? 0x7fffffff : rem;
  const char* p = (const char*)base + (in ? off : 0);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), (short)0, (int)rem, kRsrcWord3);
}

// The tiles a wave visits in a fixed sequence (first, first + P, ...) of one
// stream: a cursor holds the current tile's first row and the rows from it
// to N, and forms the tile's resource with 32-bit arithmetic (the range
// covers at most the tile's 32 rows, below 2^31 bytes by the host's check of
// 32 x row stride) instead of the 64-bit multiply of rows_rsrc per tile. The
// resources equal rows_rsrc's wherever the tile's accesses fall.
struct TileCursor {
  const char* p;  // the current tile's first row
  int64_t step;   // bytes from one tile of the sequence to the next
  int left;       // rows from the current tile's first row to N (<= 0: none)
  int pstep;      // rows from one tile of the sequence to the next
  int snb, rowb;  // row stride and row width in bytes
  __device__ __forceinline__ Rsrc rsrc() const {
    const int rows = left < 32 ? left : 32;
    const int rem = rows > 0 ? (rows - 1) * snb + rowb : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), (short)0, rem, kRsrcWord3);
  }
  __device__ __forceinline__ void next() {
    p += step;
    left -= pstep;
  }
};
// A cursor at tile t0 of a slice (byte base of row 0, row stride snb, row
// width rowb bytes) that advances by P tiles of 32 rows.
__device__ __forceinline__ TileCursor tile_cursor(const void* base, int64_t snb, int64_t rowb,
                                                  int t0, int P, int N) {
  TileCursor k;
  k.p = (const char*)base + (int64_t)t0 * 32 * snb;
  k.step = (int64_t)P * 32 * snb;
  k.left = N - 32 * t0;
  k.pstep = 32 * P;
  k.snb = (int)snb;
  k.rowb = (int)rowb;
  return k;
}

// Typed single-element and four-element accesses (fp32 compute values).
template <typename T> struct Buf;
template <> struct Buf<float> {
  static __device__ __forceinline__ float ld1(Rsrc r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kStream));
  }
  static __device__ __forceinline__ void ld4(float* o, Rsrc r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kStream);
    o[0] = __uint_as_float(v[0]);
    o[1] = __uint_as_float(v[1]);
    o[2] = __uint_as_float(v[2]);
    o[3] = __uint_as_float(v[3]);
  }
  static __device__ __forceinline__ void st1(Rsrc r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kStream);
  }
};
template <> struct Buf<__bf16> {
  static __device__ __forceinline__ float bits2f(uint32_t b16) { return __uint_as_float(b16 << 16); }
  static __device__ __forceinline__ float ld1(Rsrc r, uint32_t off) {
    return bits2f(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kStream));
  }
  static __device__ __forceinline__ void ld4(float* o, Rsrc r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kStream);
    o[0] = __uint_as_float(v[0] << 16);
    o[1] = __uint_as_float(v[0] & 0xffff0000u);
    o[2] = __uint_as_float(v[1] << 16);
    o[3] = __uint_as_float(v[1] & 0xffff0000u);
  }
  static __device__ __forceinline__ void st1(Rsrc r, uint32_t off, float v) {
    const __bf16 b = (__bf16)v;
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, b), r, off, 0, kStream);
  }
  // four consecutive elements, one 8-byte store (off 8-byte aligned)
  static __device__ __forceinline__ void st4(Rsrc r, uint32_t off, float v0, float v1, float v2,
                                             float v3) {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    const b4 b = {(__bf16)v0, (__bf16)v1, (__bf16)v2, (__bf16)v3};
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, b), r, off, 0, kStream);
  }
};
template <> struct Buf<_Float16> {
  static __device__ __forceinline__ float h2f(uint32_t b16) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)b16);
  }
  static __device__ __forceinline__ float ld1(Rsrc r, uint32_t off) {
    return h2f(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kStream));
  }
  static __device__ __forceinline__ void ld4(float* o, Rsrc r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kStream);
    o[0] = h2f(v[0] & 0xffffu);
    o[1] = h2f(v[0] >> 16);
    o[2] = h2f(v[1] & 0xffffu);
    o[3] = h2f(v[1] >> 16);
  }
  static __device__ __forceinline__ void st1(Rsrc r, uint32_t off, float v) {
    const _Float16 b = (_Float16)v;
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, b), r, off, 0, kStream);
  }
  static __device__ __forceinline__ void st4(Rsrc r, uint32_t off, float v0, float v1, float v2,
                                             float v3) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 b = {(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3};
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, b), r, off, 0, kStream);
  }
};

// Row offset (in rows, inside a tile) of register j of a [column-outer,
// point-inner] fragment on lane half h = 0; lane half 1 adds 4.
__device__ __forceinline__ constexpr int tile_row(int j) { return 8 * (j >> 2) + (j & 3); }

// [point-outer, column-inner] fragments (lane (c, h): row c, columns
// 32 k + kmap(j, h)) of NB column blocks.
// FAST: rows 16-byte aligned (8-byte for 16-bit types) and C a multiple of
// 32: four vector loads per block from `vr` = c * snb + 4 h * sizeof(T).
// Otherwise one load per element, columns >= C masked to zero; `rowb` = c * snb.
template <typename T, int NB, bool FAST>
__device__ __forceinline__ void ld_rows(float (&f)[NB][16], Rsrc r, uint32_t vr, int C, int h) {
  constexpr uint32_t e = sizeof(T);
#pragma unroll
  for (int k = 0; k < NB; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (FAST) {
        Buf<T>::ld4(&f[k][4 * q], r, vr + (uint32_t)(32 * k + 8 * q) * e);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int col = 32 * k + 8 * q + 4 * h + i;
          f[k][4 * q + i] = Buf<T>::ld1(r, col < C ? vr + (uint32_t)col * e : kOff);
        }
      }
    }
}

// Lane offset of the [column-outer, point-inner] pattern for column block k:
// column 32 k + c of row 4 h, or kOff where the column is >= C.
template <typename T>
__device__ __forceinline__ uint32_t col_off(int k, int C, int64_t snb, int c, int h) {
  const int col = 32 * k + c;
  return col < C ? (uint32_t)(4 * h * snb) + (uint32_t)col * (uint32_t)sizeof(T) : kOff;
}

// [column-outer, point-inner] fragment: lane (c, h) reads column (from vc)
// of rows 4 h + tile_row(j). Each load instruction reads two whole row
// segments of 32 columns.
template <typename T>
__device__ __forceinline__ void ld_cols(float (&f)[16], Rsrc r, uint32_t vc, uint32_t snb) {
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = Buf<T>::ld1(r, vc + (uint32_t)tile_row(j) * snb);
}
// ld_cols whose sixteen row offsets are formed at the call (one add each)
// rather than hoisted out of the tile loop by the compiler as sixteen
// loop-invariant registers per call site: for the wide kernels, where those
// registers would be spilled.
template <typename T>
__device__ __forceinline__ void ld_cols_here(float (&f)[16], Rsrc r, uint32_t vc, uint32_t snb) {
  asm volatile("" : "+v"(vc));
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = Buf<T>::ld1(r, vc + (uint32_t)tile_row(j) * snb);
}

// This lane's index in its wave, formed anew at each use: the asm is
// volatile, so the compiler neither hoists it out of a loop nor shares it
// between uses. Offsets derived from it are rematerialised at their use
// instead of being held across a tile loop, which a kernel at its register
// limit would spill (each reload from scratch waits for every load in flight,
// the next tile's prefetch included).
__device__ __forceinline__ int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Store a [column-outer, point-inner] fragment (the transposed twin of
// ld_cols): every store instruction writes two whole 32-column row segments.
template <typename T>
__device__ __forceinline__ void st_cols(Rsrc r, uint32_t vc, uint32_t snb, const f32x16& v) {
#pragma unroll
  for (int j = 0; j < 16; ++j) Buf<T>::st1(r, vc + (uint32_t)tile_row(j) * snb, v[j]);
}

// The pair reductions of a wave whose lanes c and c + 32 hold the two
// halves of one point's slots: v_permlane32_swap exchanges the wave's halves
// in one VALU instruction, and both lanes combine (lower, upper) in the same
// order, so they hold bitwise equal results.
__device__ __forceinline__ void halves(float v, float& lo, float& hi) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  lo = __uint_as_float(p[0]);
  hi = __uint_as_float(p[1]);
}
__device__ __forceinline__ float pair_max(float v) {
  float lo, hi;
  halves(v, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float pair_sum(float v) {
  float lo, hi;
  halves(v, lo, hi);
  return lo + hi;
}

// Per-point scalars of one tile (stats rows, delta, row sums): a resource
// over floats [p0, N) of a length-N row; lane h = 0 of each pair writes.
__device__ __forceinline__ Rsrc pts_rsrc(const float* row, int64_t p0, int64_t N) {
  return rows_rsrc(row, 4, 4, p0, row ? N : 0);
}
__device__ __forceinline__ void st_pt(Rsrc r, int c, int h, float v) {
  Buf<float>::st1(r, h == 0 ? (uint32_t)c * 4u : kOff, v);
}
__device__ __forceinline__ float ld_pt(Rsrc r, int c) { return Buf<float>::ld1(r, (uint32_t)c * 4u); }

}  // namespace fs
