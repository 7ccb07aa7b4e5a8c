// MFMA operand fragments prepared once and reused (gfx950).
//
// A Frag<M> is a 32 x 32 fragment (fragment convention of fs_device.h) in
// the register form the MFMA of mode M consumes:
//   MMA_BF16: one bf16 piece, v_mfma_f32_32x32x16_bf16 (2 per contraction
//             block of 32);
//   MMA_X6:   fp32 split exactly into three bf16 pieces v = v0 + v1 + v2
//             (v0 = v rounded to bf16, v1 = (v - v0) rounded, v2 = the
//             rest, which has at most 8 significant bits), and a product
//             a b taken as the six piece products a_i b_j with i + j <= 2
//             (12 bf16 MFMAs per contraction block). The dropped terms are
//             below 2^-23 |a b|; the products are exact and accumulate in
//             fp32, so the result is as accurate as an fp32 FMA dot (the
//             tests gate it against float64) while running on the bf16
//             matrix cores, which -- unlike v_mfma_f32_32x32x2_f32 -- execute
//             alongside the VALU.
//   MMA_F32:  sixteen fp32 values, v_mfma_f32_32x32x2_f32.
// Register j of a fragment holds contraction index kmap(j, h); MFMA s of a
// bf16 pair takes registers 8 s .. 8 s + 7 of both operands (lane half h
// supplies k slots 8 h .. 8 h + 7), the same index set on both sides.
#pragma once
#include "fs_device.h"

namespace fs {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int M> struct Frag;
template <> struct Frag<MMA_F32> {
  static constexpr int W = 4;  // 16-byte words per lane
  u32x4 q[4];
};
template <> struct Frag<MMA_BF16> {
  static constexpr int W = 2;
  u32x4 q[2];
};
template <> struct Frag<MMA_X6> {
  static constexpr int W = 6;  // q[2 * piece + s]
  u32x4 q[6];
};

template <int M> __device__ __forceinline__ void prep(Frag<M>& o, const float (&v)[16]);

template <> __device__ __forceinline__ void prep<MMA_F32>(Frag<MMA_F32>& o, const float (&v)[16]) {
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int e = 0; e < 4; ++e) o.q[w][e] = __float_as_uint(v[4 * w + e]);
}

template <> __device__ __forceinline__ void prep<MMA_BF16>(Frag<MMA_BF16>& o, const float (&v)[16]) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = (__bf16)v[8 * s + e];
    o.q[s] = __builtin_bit_cast(u32x4, b);
  }
}

// The exact split, per pair of values (a, b): p0 = bf16(a, b) rounded to
// nearest, r = (a, b) - p0, p1 = bf16(r), s = r - p1, p2 = bf16(s). Each
// residual is exact in fp32 and the last one has at most 8 significant
// bits, so a = p0 + p1 + p2 exactly. The residuals come from
// v_dot2c_f32_bf16 (a - p0.lo as the dot of p0 with (-1, 0) accumulated
// onto a), one VALU instruction each: 3.5 instructions per value.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
// The pair (-1, 0) is materialised in an SGPR: as an immediate the
// compiler encodes it as the inline constant -1.0, which the hardware reads
// as the 32-bit float (bf16 pair (0, -1)).
__device__ __forceinline__ bf16x2 neg_one_lo() {
  uint32_t r;
  asm("s_mov_b32 %0, 0xbf80" : "=s"(r));
  return __builtin_bit_cast(bf16x2, r);
}
__device__ __forceinline__ float minus_lo(uint32_t p, float a) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), neg_one_lo(), a, false);
}
__device__ __forceinline__ float minus_hi(uint32_t p, float b) {
  const bf16x2 m = {(__bf16)0.0f, (__bf16)-1.0f};  // bits 0xbf800000
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), m, b, false);
}

template <> __device__ __forceinline__ void prep<MMA_X6>(Frag<MMA_X6>& o, const float (&v)[16]) {
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float va = v[8 * s + 2 * e], vb = v[8 * s + 2 * e + 1];
      const uint32_t p0 = pk_bf16(va, vb);
      const float ra = minus_lo(p0, va), rb = minus_hi(p0, vb);
      const uint32_t p1 = pk_bf16(ra, rb);
      const float sa = minus_lo(p1, ra), sb = minus_hi(p1, rb);
      o.q[s][e] = p0;
      o.q[2 + s][e] = p1;
      o.q[4 + s][e] = pk_bf16(sa, sb);
    }
}

__device__ __forceinline__ f32x16 mfma_bf16(const u32x4& a, const u32x4& b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// C += A B over one contraction block of 32 (A [i-outer, k-inner], B
// [j-outer, k-inner], C [j-outer, i-inner]).
template <int M>
__device__ __forceinline__ f32x16 mma(const Frag<M>& a, const Frag<M>& b, f32x16 c);

template <>
__device__ __forceinline__ f32x16 mma<MMA_F32>(const Frag<MMA_F32>& a, const Frag<MMA_F32>& b,
                                               f32x16 c) {
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.q[w][e]),
                                               __uint_as_float(b.q[w][e]), c, 0, 0, 0);
  return c;
}

template <>
__device__ __forceinline__ f32x16 mma<MMA_BF16>(const Frag<MMA_BF16>& a, const Frag<MMA_BF16>& b,
                                                f32x16 c) {
  c = mfma_bf16(a.q[0], b.q[0], c);
  return mfma_bf16(a.q[1], b.q[1], c);
}

// The six piece products, smallest first.
template <>
__device__ __forceinline__ f32x16 mma<MMA_X6>(const Frag<MMA_X6>& a, const Frag<MMA_X6>& b,
                                              f32x16 c) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    c = mfma_bf16(a.q[4 + s], b.q[s], c);
    c = mfma_bf16(a.q[2 + s], b.q[2 + s], c);
    c = mfma_bf16(a.q[s], b.q[4 + s], c);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    c = mfma_bf16(a.q[2 + s], b.q[s], c);
    c = mfma_bf16(a.q[s], b.q[2 + s], c);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) c = mfma_bf16(a.q[s], b.q[s], c);
  return c;
}

// acc += sgn (A B) over one contraction block for an accumulator that runs
// over many point tiles (summed from zero, then added in fp32; the caller
// has negated one operand when sgn = -1: acc_add).
template <int M>
__device__ __forceinline__ void mma_acc(f32x16& acc, const Frag<M>& a, const Frag<M>& b,
                                        float sgn) {
  acc_add(acc, mma<M>(a, b, zero16()), sgn);
}

// ------------------------------------------------ transposing split fragments
// A fragment's bf16 pieces can be transposed through LDS without splitting
// the transposed values again: the wave writes them as rows (tr_put) and
// reads them back with ds_read_b64_tr_b16 (tr_get), gfx950's transposing LDS
// load. Its lane layout, measured on the part: in each group of 16 lanes,
// element i of lane q is element q % 4 of the 8 bytes that lane 4 i + q / 4
// of the group addressed. So if lane (group g, index L) of the reading wave
// addresses row 16 s + 4 (g / 2) + L / 4 (+ 8), columns 16 (g % 2) + 4 (L % 4)
// .. + 3, lane (c, h) receives column c of rows 16 s + 4 h + i (+ 8): the
// transposed fragment in the MFMA operand layout (fragment convention of
// fs_device.h).
// Region of one fragment: [piece][32 rows][32 columns] bf16, rows of 64
// bytes; the eight 8-byte column segments of a row are XOR-swizzled by
// (row / 2) % 8. Measured on MI355X, 8-byte LDS writes are served 16 lanes
// at a time against 32 banks of 4 bytes, 8-byte reads (plain and
// transposing) 32 lanes at a time against 64 banks. A row write's 16 lanes
// are 16 consecutive rows at one segment: rows of equal parity share their
// banks modulo 32 and the swizzle gives the 8 of each parity 8 different
// segments (a (row / 4) % 8 swizzle leaves pairs of them colliding: 30 %
// slower writes). A transposing read's 32 lanes cover 4 whole rows,
// conflict-free under any swizzle within rows.
constexpr int kTrRowB = 64, kTrPieceB = 32 * kTrRowB;
template <int M> constexpr int tr_pieces() { return M == MMA_X6 ? 3 : 1; }
template <int M> constexpr int tr_bytes() { return tr_pieces<M>() * kTrPieceB; }
__device__ __forceinline__ int tr_off(int row, int col) {
  return row * kTrRowB + ((col ^ (4 * ((row >> 1) & 7))) << 1);
}
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4* LdsI16x4;

// Write fragment f ([outer = c][inner = kmap(j, h)]) of lane (c, h) as rows;
// `neg` (0 or 0x80008000) flips the sign of every piece written.
template <int M>
__device__ __forceinline__ void tr_put(char* region, const Frag<M>& f, int c, int h, uint32_t neg) {
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int pi = 0; pi < tr_pieces<M>(); ++pi)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 w = f.q[2 * pi + s];
      char* base = region + pi * kTrPieceB;
      *reinterpret_cast<uint2*>(base + tr_off(c, 16 * s + 4 * h)) = make_uint2(w[0] ^ neg, w[1] ^ neg);
      *reinterpret_cast<uint2*>(base + tr_off(c, 16 * s + 8 + 4 * h)) =
          make_uint2(w[2] ^ neg, w[3] ^ neg);
    }
  __builtin_amdgcn_wave_barrier();
}

// Read the transposed fragment ([outer = column][inner = kmap(j, h) over
// rows]) of what tr_put wrote (pieces of mode M, M's own piece count: an
// MMA_BF16 read of MMA_X6 pieces takes piece 0, the bf16 rounding).
template <int M>
__device__ __forceinline__ void tr_get(Frag<M>& f, const char* region, int lane) {
  const int L = lane & 15, g = lane >> 4;
  const int r0 = 4 * (g >> 1) + (L >> 2), col = 16 * (g & 1) + 4 * (L & 3);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int pi = 0; pi < tr_pieces<M>(); ++pi)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const char* base = region + pi * kTrPieceB;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (LdsI16x4)(const_cast<char*>(base) + tr_off(16 * s + r0, col)));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (LdsI16x4)(const_cast<char*>(base) + tr_off(16 * s + 8 + r0, col)));
      const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
      f.q[2 * pi + s] = u32x4{l2.x, l2.y, h2.x, h2.y};
    }
  __builtin_amdgcn_wave_barrier();
}

// Row sums of a fragment B ([outer = c][inner = k]): sum_k B[c][k] in every
// register of lane (c, h) (a ones operand times B on the bf16 matrix cores,
// the result's lanes indexing B's outer axis; the pieces of an MMA_X6
// fragment are exact, smallest first).
template <int M> __device__ __forceinline__ f32x16 row_sums(const Frag<M>& b) {
  const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  f32x16 t = zero16();
#pragma unroll
  for (int pi = tr_pieces<M>() - 1; pi >= 0; --pi)
#pragma unroll
    for (int s = 0; s < 2; ++s) t = mfma_bf16(ones, b.q[2 * pi + s], t);
  return t;
}

// Ready fragments in LDS: word w of lane l at slot[w * 64 + l] (16-byte
// words; a wave reads or writes 1 KB of consecutive words per instruction,
// conflict-free).
template <int M> __device__ __forceinline__ void lds_put(u32x4* slot, const Frag<M>& f, int lane) {
#pragma unroll
  for (int w = 0; w < Frag<M>::W; ++w) slot[w * 64 + lane] = f.q[w];
}
template <int M> __device__ __forceinline__ void lds_get(Frag<M>& f, const u32x4* slot, int lane) {
#pragma unroll
  for (int w = 0; w < Frag<M>::W; ++w) f.q[w] = slot[w * 64 + lane];
}
template <int M> constexpr int frag_words() { return Frag<M>::W * 64; }  // u32x4 per fragment

}  // namespace fs
