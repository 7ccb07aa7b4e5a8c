// Internal launch interface between the C-ABI (fs_abi.cpp) and the kernel
// translation units. Not part of the public C-ABI (include/flashslice_hip.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fs {

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

// One launch's operands. Point tensors (B, N, H, C) are read and written
// through element strides along b, n, h with unit stride along the last
// dim. Small tensors are fp32 and contiguous; weight and bias carry the
// element strides along b and h that are zero where the tensor is shared
// (reference slice_ops.py:461-478).
struct Args {
  const void* x;  int64_t sxb, sxn, sxh;   // x_mid (B, N, H, D)
  const void* f;  int64_t sfb, sfn, sfh;   // fx_mid or d_out (B, N, H, DV)
  void* o1;       int64_t s1b, s1n, s1h;   // out (deslice fwd) or dx (bwd)
  void* o2;       int64_t s2b, s2n, s2h;   // dfx (slice bwd)
  const void* g;  int64_t sgb, sgn, sgh;   // d_out of the tied backward (B, N, H, DV)
  const float* W;    int64_t swb, swh;     // (.., G, D)
  const float* bias; int64_t sbb, sbh;     // (.., G)
  const float* tau;                        // (H,)
  const float* tok;                        // (B, H, G, DV): tokens or dz_num
  const float* tok2;                       // (B, H, G, DV): tokens of the tied backward
  const float* ds;                         // (B, H, G): d s (slice bwd)
  const float* stats_in;                   // (B, H, 2, N) or null
  float* stats_out;                        // (B, H, 2, N) or null
  float* delta;                            // (B, H, N) softmax-Jacobian row terms (blocked bwd)
  float* lsum;                             // (B, H, N) row sums formed by the point-owned bwd pass
  float* part;                             // per-wave partials (workspace)
  float* part2;                            // per-wave dtau partials of point-owned kernels
  const int64_t* rows;                     // row splits (B + 1) of a ragged batch, or null
                                           // (point strides along b are then 0; rows_of)
  int64_t rows_total;                      // rows of the ragged batch's point tensors
  int B, N, H, D, DV, G;
  int P;                                   // point partitions per (b, h), a multiple of 4
  int no_dtok;                             // tied bwd: dtokens not asked for (not formed)
  int rev;                                 // whole-G kernels: tiles visited last-first (tile_p0)
  int ntiles;                              // ceil(N / 32)
  int vec_x, vec_f, vec_1, vec_2;          // 4-element alignment of rows
  int fast;                                // all rows aligned, D and DV multiples of 32
  int nd, nv;                              // 32-wide blocks of D and DV (blocked family)
  int two_pass;                            // statistics: max pass, then sum pass
  // G-blocked family, widths up to 64: operand fragments and per-slot
  // vectors prepared once per call (k_gp_prep) at u32x4 offsets foff[kind]
  // of `frags` (gp_layout)
  void* frags;
  int64_t foff[6];
};

// The row range of sample b and where its per-point buffers start. Without
// row splits: the sample's N points from row 0 of its slice of every point
// tensor, and per-point buffers -- statistics (planes, 2, NS), delta and
// row sums (planes, NS) -- in plane b * H + h of NS = N rows. With row
// splits (a ragged batch): rows rows[b] .. rows[b + 1] - 1 of the
// concatenated point tensors (clamped to their rows_total rows and to N rows
// per sample, so malformed splits cannot address outside the tensors), and
// per-point buffers in plane h of NS = rows_total rows, indexed by row: the
// statistics of a ragged batch are (1, H, 2, rows_total).
struct Rows {
  int64_t row0, plane, NS;
  int N, ntiles;
  __device__ int64_t stats_off() const { return plane * 2 * NS + row0; }
  __device__ int64_t pt_off() const { return plane * NS + row0; }
};
__device__ __forceinline__ int64_t clamp_rows(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}
__device__ __forceinline__ Rows rows_of(const Args& a, int b, int hd) {
  Rows r;
  if (!a.rows) {
    r.row0 = 0;
    r.plane = (int64_t)b * a.H + hd;
    r.NS = a.N;
    r.N = a.N;
    r.ntiles = a.ntiles;
    return r;
  }
  r.row0 = clamp_rows(a.rows[b], 0, a.rows_total);
  const int64_t r1 = clamp_rows(a.rows[b + 1], r.row0, a.rows_total);
  r.N = (int)(r1 - r.row0 < (int64_t)a.N ? r1 - r.row0 : (int64_t)a.N);
  r.ntiles = (r.N + 31) / 32;
  r.plane = hd;
  r.NS = a.rows_total;
  return r;
}

// Kinds of prepared fragments (G-blocked family): W [g-outer, d-inner] in the
// logits mode; W / tau [d-outer, g-inner], V [g-outer, v-inner] and V
// [v-outer, g-inner] (V = tokens or dz_num) in the value mode; and two
// per-slot vectors in lane-ready form (4 u32x4 per lane: lane half h's 16
// values of slots kmap(j, h)): bias * log2(e) / tau (-1e30 beyond G) and d s
// (0 beyond G). Item k of slot block gb of head bh is at foff[kind] +
// ((bh * ngb + gb) * nk + k) * FW (nk = blocks of D or DV, or 1 for the
// vectors; FW = u32x4 per item).
enum GpKind { GP_WR = 0, GP_WC = 1, GP_VR = 2, GP_VC = 3, GP_BC = 4, GP_DS = 5 };
struct GpLayout {
  int64_t off[6];
  int64_t total_u32x4;
};
// u32x4 per 32 x 32 fragment in the dot kind's logits / value mode
__host__ __device__ inline int gp_fw(int dk, bool logits) {
  const bool x6 = logits ? dk != 2 : dk == 0;
  return (x6 ? 6 : 2) * 64;
}
constexpr int kGpVecFw = 4 * 64;  // u32x4 per per-slot vector item
__host__ __device__ inline GpLayout gp_layout(int B, int H, int G, int D, int DV, int dk) {
  GpLayout l;
  const int64_t bhg = (int64_t)B * H * ((G + 31) / 32);
  const int64_t nd = (D + 31) / 32, nv = (DV + 31) / 32;
  l.off[GP_WR] = 0;
  l.off[GP_WC] = l.off[GP_WR] + bhg * nd * gp_fw(dk, true);
  l.off[GP_VR] = l.off[GP_WC] + bhg * nd * gp_fw(dk, false);
  l.off[GP_VC] = l.off[GP_VR] + bhg * nv * gp_fw(dk, false);
  l.off[GP_BC] = l.off[GP_VC] + bhg * nv * gp_fw(dk, false);
  l.off[GP_DS] = l.off[GP_BC] + bhg * kGpVecFw;
  l.total_u32x4 = l.off[GP_DS] + bhg * kGpVecFw;
  return l;
}
// the prepared-fragment kernels serve D, DV <= 64 (older kernels above)
__host__ __device__ inline bool gp_serves(int D, int DV) { return D <= 64 && DV <= 64; }

// Partial-buffer layout of one wave (floats), fused family:
//   slice fwd:   z [G][DV], s [G]
//   slice bwd:   dW [G][D], db [G], dtau [1]
//   deslice bwd: dtok [G][DV], dW [G][D], db [G], dtau [1]
__host__ __device__ inline int64_t part_floats_slice_fwd(int G, int DV) { return (int64_t)G * DV + G; }
__host__ __device__ inline int64_t part_floats_slice_bwd(int G, int D) { return (int64_t)G * D + G + 1; }
__host__ __device__ inline int64_t part_floats_deslice_bwd(int G, int D, int DV) {
  return (int64_t)G * DV + (int64_t)G * D + G + 1;
}

constexpr int kWavesPerBlock = 4;
constexpr int kTile = 32;               // points per wave tile

// fused (whole G in registers) family; returns hipSuccess or an error
hipError_t launch_fused_slice_fwd(const Args& a, int dtype, int mode, hipStream_t st);
hipError_t launch_fused_deslice_fwd(const Args& a, int dtype, int mode, hipStream_t st);
hipError_t launch_fused_slice_bwd(const Args& a, int dtype, int mode, hipStream_t st);
hipError_t launch_fused_deslice_bwd(const Args& a, int dtype, int mode, hipStream_t st);
// backward of a deslice -> slice coupling in one pass; partials in the
// deslice-bwd layout (dtokens, dW, db, dtau)
hipError_t launch_fused_tied_bwd(const Args& a, int dtype, int mode, hipStream_t st);
bool fused_fits(int D, int DV, int G);

// G-blocked family (any G; fs_blocked.hip). Point-owned kernels ("_n") run
// on grid (P / 4, B * H); slot-owned kernels ("_g") on (P / 4, B * H,
// ceil(G / 32)) and write the same per-wave partial layout as the fused
// family (every wave its own 32 slot rows).
enum BlockedKind {
  BK_STATS = 0,          // (m, l) per point, online or two-pass
  BK_DESLICE_N = 1,      // out from saved statistics
  BK_DESLICE_ONLINE = 2, // out and the statistics in one online pass
  BK_SLICE_G = 3,        // z_num, s partials from saved statistics
  BK_SLICE_BWD_N = 4,    // dfx, delta, dx, dtau partials
  BK_SLICE_BWD_G = 5,    // dW, db partials
  BK_DESLICE_BWD_N = 6,  // delta, dx, dtau partials
  BK_DESLICE_BWD_G = 7   // dtokens, dW, db partials
};
hipError_t launch_blocked(int kind, const Args& a, int dtype, int mode, hipStream_t st);
// builds a.frags / a.fvec for the G-blocked kernels of one call (gp_serves)
hipError_t launch_gp_prep(const Args& a, int mode, hipStream_t st);
int blocked_width_blocks(int D, int DV);  // 1, 2, 4 or 8 (0 if D or DV > 256)

// Block-cooperative kernels of the G-blocked family (fs_coop.hip): bf16 dots
// on 16-bit point tensors, 128 < G <= 256, D, DV <= 32 (coop_serves). A block
// of eight waves takes one point tile at a time, wave w slots 32 w ..; grid
// (P, B * H) with a.P = the blocks per (b, h); one partial per block in the
// whole-G layout (part_floats_*). The backward kernels need statistics.
enum CoopKind { CK_SLICE_FWD = 0, CK_SLICE_BWD = 1, CK_DESLICE_BWD = 2, CK_DESLICE_FWD = 3 };
hipError_t launch_coop(int kind, const Args& a, int dtype, hipStream_t st);

// Waves per SIMD the whole-G slice forward is compiled for, by its blocks of
// 32 slots / logits width / value width (the host sizes its grid to fill
// them): three at one block (168 registers, a few values spilled; 5 % faster
// at C2 with 1536 blocks); two for a wide shape whose slot accumulators and
// split pieces fit 256 registers (one block of x, at most two slot blocks,
// z_num blocks NGB x NVB <= 4); else one.
__host__ __device__ constexpr int slice_fwd_waves(int ngb, int ndb, int nvb) {
  return ngb * ndb * nvb == 1 ? 3 : (ndb == 1 && ngb <= 2 && ngb * nvb <= 4 ? 2 : 1);
}
bool coop_ok(int G, int D, int DV);

// Deterministic reduction of per-wave partials (fs_reduce.hip). One output
// segment: out[ob][oh][e] = sum over the contributing waves (b -> ob =
// Bo > 1 ? b : 0, h -> oh = Ho > 1 ? h : 0, every partition p < P) of
// part[((b * H + h) * P + p) * wstride + off + e], e < E.
struct ReduceSegment {
  const float* part;
  int64_t wstride, off;
  int P, E, Bo, Ho;
  float* out;
};
struct ReduceSegments {
  ReduceSegment seg[4];
  int n;
};
hipError_t launch_reduce(int B, int H, const ReduceSegments& segs, hipStream_t st);

// LayerNorm of (rows, C) fp32 rows (fs_layernorm.hip); C % 4 == 0, C <= 2048.
int64_t ln_blocks(int64_t rows);
hipError_t ln_fwd_launch(const float* x, const float* gamma, const float* beta, float* y,
                         float* mean, float* rstd, int64_t rows, int C, float eps,
                         hipStream_t st);
hipError_t ln_bwd_launch(const float* dy, const float* x, const float* gamma, const float* mean,
                         const float* rstd, float* dx, float* dgamma, float* dbeta, float* part,
                         int64_t rows, int C, hipStream_t st);

}  // namespace fs
