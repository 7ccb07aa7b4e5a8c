// MFMA operand fragments prepared once and reused (gfx950).
//
// A Frag<M> is a 32 x 32 fragment (fragment convention of fs_device.h) in
// the register form the MFMA of mode M consumes:
//   MMA_BF16: one bf16 piece, v_mfma_f32_32x32x16_bf16 (2 per contraction
//             block of 32);
//   MMA_X6:   fp32 split exactly into three bf16 pieces v = v0 + v1 + v2
//             (v0 = v truncated to bf16, v1 = (v - v0) truncated, v2 = the
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

// bf16 bits of the high halves of a (low half of the result) and b.
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

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

template <> __device__ __forceinline__ void prep<MMA_X6>(Frag<MMA_X6>& o, const float (&v)[16]) {
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float va = v[8 * s + 2 * e], vb = v[8 * s + 2 * e + 1];
      const uint32_t ua = __float_as_uint(va), ub = __float_as_uint(vb);
      o.q[s][e] = hi_pair(ua, ub);
      const float ra = va - __uint_as_float(ua & 0xffff0000u);
      const float rb = vb - __uint_as_float(ub & 0xffff0000u);
      const uint32_t qa = __float_as_uint(ra), qb = __float_as_uint(rb);
      o.q[2 + s][e] = hi_pair(qa, qb);
      const float sa = ra - __uint_as_float(qa & 0xffff0000u);
      const float sb = rb - __uint_as_float(qb & 0xffff0000u);
      o.q[4 + s][e] = hi_pair(__float_as_uint(sa), __float_as_uint(sb));
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
