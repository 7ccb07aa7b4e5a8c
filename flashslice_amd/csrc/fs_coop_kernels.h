// Block-cooperative kernels of the G-blocked family: bf16 dots (dot kind 2),
// 128 < G <= 256, D and DV <= 32 (config 3's G = 256 in bf16).
//
// The G-blocked kernels split a pass into a point-owned and a slot-owned
// kernel and carry the normalisation between them through per-point
// buffers: every (point, slot) weight is recomputed in each of them (nine
// exponentials per step at config 3) and every point tile is read once per
// 32-slot block. Here a block of eight waves takes one point tile at a time
// and wave w owns slots 32 w .. 32 w + 31, so the whole slot axis of the tile
// is in the block's registers at once. What a point needs from every slot is
// combined across the waves through LDS -- the softmax max and sum (slice
// forward without statistics), delta = sum_g w omega (backward), and the
// per-point outputs dx and dfx, each wave's partial over its own slots summed
// in a fixed wave order -- and what a slot needs from every point stays in its
// wave (z_num, s, dW, db, dtokens). Each op is one pass with one exponential
// per (point, slot), and each point tile is read from HBM once.
//
// Each point tile is loaded once per block: 256 threads load it (16 bytes
// each; two tiles ahead in the forward kernels, one in the backward) and
// store it in LDS as bf16 rows in the transposable layout of tr_put, three
// buffers deep; the waves read
// their MFMA operands from there, plain ([point, column]) or transposed
// (ds_read_b64_tr_b16), with no fp32 round trip. Per tile, a slice forward
// waits at one block barrier (the next tile and, without statistics, the
// waves' (max, sum) pairs), a backward at two (the next tile and delta; the
// dx / dfx exchange). The tile loop is identical in every wave of a block,
// so the barriers are uniform.
#pragma once
#include <type_traits>
#include "fs_device.h"
#include "fs_internal.h"
#include "fs_io.h"
#include "fs_mma.h"
#include "fs_tile.h"

namespace fs {

constexpr int kCoopWaves = 8;
// the exponent shift of points beyond N: every weight exp2(t2 - shift) is 0
// and every product with the shifted logit stays finite
constexpr float kFarShift = 3.0e38f;
constexpr int kCoopThreads = 64 * kCoopWaves;
constexpr int kCoopStride = 36;                  // staging row stride (floats), conflict-free
constexpr int kCoopTr = kTrPieceB / 4;           // the wave's transpose region (floats)
// per wave, during the prologue: the fp32 staging of its 32 rows of W and of
// tokens / dz_num (the backward) or of W (the slice forward)
constexpr int kCoopWReg = 2 * 32 * kCoopStride;
// The backward's tile loop reuses the waves' staging regions: eight
// transpose regions, then the block's [point][slot] bf16 buffers of Lb and
// w (32 rows of 256 slots, each row padded by 16 bytes: the 16 lanes that
// read one 16-byte chunk of 16 rows hit 16 different chunks of the banks)
constexpr int kPsRowB = 256 * 2 + 16;
constexpr int kPsBufB = 32 * kPsRowB;
static_assert(kCoopWaves * kTrPieceB + 2 * kPsBufB <= kCoopWaves * kCoopWReg * 4,
              "coop backward buffers exceed the staging regions");
// the deslice forward's two weight buffers in the forward's staging regions
static_assert(2 * kPsBufB <= kCoopWaves * (kCoopTr + 17 * 64) * 4,
              "coop deslice buffers exceed the staging regions");
constexpr int kCoopPts = 4 * kCoopWaves * 32;    // per-point exchange: 2 buffers x 2 rows per wave
constexpr int kCoopVec = 2 * 32 * kCoopWaves;    // per-slot vectors: bias * cst, d s
constexpr int kCoopTileB = kTrPieceB;            // one staged 32 x 32 bf16 tile (bytes)
constexpr int kCoopTiles = 3 * 2 * kCoopTileB / 4;  // 3 buffers x (x, fx / d_out) (floats)
// the slice forward's wave region: the staging of W, then the transpose
// region and the point-sum buffer of coop_point_sum (no exchange fragments):
// 68 KB per block, so two blocks share a CU
constexpr int kCoopWRegFwd = kCoopTr + 17 * 64;
static_assert(32 * kCoopStride <= kCoopWRegFwd, "coop forward staging exceeds its region");

// the shapes these kernels serve (the host picks them for dot kind 2)
__host__ __device__ inline bool coop_serves(int G, int D, int DV) {
  return G > 128 && G <= 32 * kCoopWaves && D <= 32 && DV <= 32;
}

// Stage a (R x C) fp32 matrix (row stride C), zero-padded to 32 x 32, into
// LDS with row stride kCoopStride; the 64 lanes of one wave.
__device__ __forceinline__ void coop_stage(float* dst, const float* src, int R, int C, int lane) {
  for (int i = lane; i < 32 * 32; i += 64) {
    const int r = i >> 5, col = i & 31;
    dst[r * kCoopStride + col] = (r < R && col < C) ? src[(int64_t)r * C + col] : 0.f;
  }
}

// Sum over the 32 point lanes of each lane half of a per-lane [point, slot]
// accumulator (16 registers): slot kmap(j, h) of the wave's 32. Through the
// wave's LDS region; lane t < 32 returns slot t's sum (fixed order).
__device__ __forceinline__ float coop_point_sum(const float (&v)[16], float* reg, int lane) {
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < 16; ++j) reg[lane * 17 + j] = v[j];
  __builtin_amdgcn_wave_barrier();
  float s = 0.f;
  if (lane < 32) {
    const int hs = (lane >> 2) & 1, j = ((lane >> 3) << 2) | (lane & 3);
    for (int p = 0; p < 32; ++p) s += reg[(p + 32 * hs) * 17 + j];
  }
  __builtin_amdgcn_wave_barrier();
  return s;
}

#define COOP_PROLOGUE(WREG)                                                             \
  constexpr int kWReg_ = (WREG);                                                        \
  __shared__ __attribute__((aligned(16))) float smem[kCoopWaves * kWReg_ + kCoopPts +    \
                                                     kCoopVec + kCoopTiles];            \
  constexpr int M = MMA_BF16;                                                           \
  const int lane = threadIdx.x & 63;                                                    \
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);                     \
  const int c = lane & 31, h = lane >> 5;                                               \
  const int bh = blockIdx.y;                                                            \
  const int b = bh / a.H, hd = bh - b * a.H;                                            \
  const Rows R_ = rows_of(a, b, hd);                                                    \
  const int64_t row0_ = uniform64(R_.row0);                                             \
  const int N = __builtin_amdgcn_readfirstlane(R_.N);                                   \
  const int ntiles_ = __builtin_amdgcn_readfirstlane(R_.ntiles);                        \
  const int G = a.G, D = a.D, DV = a.DV;                                                \
  const int g0 = 32 * wid;                                                              \
  const int pid = blockIdx.x;                                                           \
  float* wreg = smem + wid * kWReg_;                                                    \
  char* trS = reinterpret_cast<char*>(wreg);                                            \
  float* xpt = smem + kCoopWaves * kWReg_;                                              \
  float* sBC = xpt + kCoopPts;                                                          \
  float* sDS = sBC + 32 * kCoopWaves;                                                   \
  char* tiles_ = reinterpret_cast<char*>(sDS + 32 * kCoopWaves);                        \
  const float tauf = a.tau[hd];                                                         \
  const float cst = (float)(1.4426950408889634 / (double)tauf);                        \
  const float inv_tau = 1.f / tauf;                                                     \
  const bool fast = a.fast != 0;                                                        \
  const float* Wp = a.W + b * a.swb + hd * a.swh;                                       \
  const float* Bp = a.bias + b * a.sbb + hd * a.sbh;                                    \
  const int Rw = G - g0 < 32 ? G - g0 : 32;                                             \
  coop_stage(wreg, Wp + (int64_t)g0 * D, Rw, D, lane);                                  \
  if (a.tok && kWReg_ >= 2 * 32 * kCoopStride)                                          \
    coop_stage(wreg + 32 * kCoopStride, a.tok + ((int64_t)bh * G + g0) * DV, Rw, DV, lane); \
  if (lane < 32) {                                                                      \
    const int g = g0 + lane;                                                            \
    sBC[g0 + lane] = g < G ? Bp[g] * cst : kNoSlot;                                     \
    sDS[g0 + lane] = (a.ds && g < G) ? a.ds[(int64_t)bh * G + g] : 0.f;                \
  }                                                                                     \
  __syncthreads();                                                                      \
  Frag<M> qL; /* W [g, d]: the logits operand */                                       \
  {                                                                                     \
    float f_[16];                                                                       \
    lds_frag_rowouter(f_, wreg, kCoopStride, 0, 0, c, h);                               \
    prep<M>(qL, f_);                                                                    \
  }                                                                                     \
  (void)inv_tau; (void)fast; (void)DV; (void)row0_;

// Point slices of one (b, h) (as FS_SLICE): byte base from the sample's
// first row, byte row stride, row width, this lane's row c.
#define COOP_SLICE(NAME, PTR, SB, SN, SH, C)                                                \
  const char* NAME##_b =                                                                  \
      (const char*)(PTR) + (b * (SB) + row0_ * (SN) + hd * (SH)) * (int64_t)sizeof(T);    \
  const int64_t NAME##_sn = (SN) * (int64_t)sizeof(T);                                    \
  const int64_t NAME##_w = (int64_t)(C) * (int64_t)sizeof(T);                             \
  const uint32_t NAME##_row = (uint32_t)(c * NAME##_sn);

// scaled logits t2 = (x . W + b) log2(e) / tau of the wave's 32 slots
#define COOP_LOGITS(T2, XQ)                                                             \
  {                                                                                     \
    const f32x16 s_ = mma<M>(qL, XQ, zero16());                                         \
    float bc_[16];                                                                      \
    lds_frag_vec(bc_, sBC + g0, h);                                                     \
    _Pragma("unroll") for (int r = 0; r < 16; ++r) T2[r] = fmaf(s_[r], cst, bc_[r]);    \
  }

// ---------------------------------------------------------- staged tiles
// Thread i < 128's share of one tile of a (B, N, H, C) 16-bit point slice:
// row i / 4, columns 8 (i % 4) .. + 7 (16 bytes). Rows beyond the slice's
// range and columns beyond C read as zero.
template <typename T, bool FAST>
__device__ __forceinline__ void coop_tile_load(uint32_t (&v)[4], Rsrc r, int64_t snb, int C,
                                               int i) {
  const int row = i >> 2, col0 = 8 * (i & 3);
  const uint32_t off = (uint32_t)(row * snb) + (uint32_t)col0 * 2u;
  if constexpr (FAST) {
    const auto q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kStream);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = q[e];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(r, col0 + 2 * e < C ? off + 4u * e : kOff,
                                                               0, kStream);
      const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(
          r, col0 + 2 * e + 1 < C ? off + 4u * e + 2u : kOff, 0, kStream);
      v[e] = (lo & 0xffffu) | (hi << 16);
    }
  }
}
__device__ __forceinline__ void coop_tile_store(char* region, const uint32_t (&v)[4], int i) {
  const int row = i >> 2, col0 = 8 * (i & 3);
  *reinterpret_cast<uint2*>(region + tr_off(row, col0)) = make_uint2(v[0], v[1]);
  *reinterpret_cast<uint2*>(region + tr_off(row, col0 + 4)) = make_uint2(v[2], v[3]);
}
// The [row, column] fragment of a staged tile (the inverse of tr_put): lane
// (c, h) row c, columns kmap(j, h).
__device__ __forceinline__ void tile_rows(Frag<MMA_BF16>& f, const char* region, int c, int h) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const uint2 lo = *reinterpret_cast<const uint2*>(region + tr_off(c, 16 * s + 4 * h));
    const uint2 hi = *reinterpret_cast<const uint2*>(region + tr_off(c, 16 * s + 8 + 4 * h));
    f.q[s] = u32x4{lo.x, lo.y, hi.x, hi.y};
  }
}

// Staging of the block's point tiles: threads 0..127 take x, 128..255 the
// second stream (fx or d_out; TWO = false: none), each 16 bytes of a tile
// into a ring of DEPTH register sets, tiles t, t + P, ... in order; a tile
// is published from its set into one of three rotating LDS buffers (so the
// tile stored for the next step never overwrites one a slower wave may still
// read), and the set is refilled with the tile DEPTH steps later. Set
// indices are compile-time (the tile loop is unrolled over the ring). Waves
// that stage nothing issue the same loads on an empty range (zeros, no
// memory traffic): every wave then has the same loads outstanding, and the
// compiler waits at a publish for that one tile, not for all of them.
#define COOP_STAGING(FAST, TWO, DEPTH)                                                  \
  /* waves 0, 1 load x, waves 2, 3 the second stream: conditions on the   */           \
  /* (scalar) wave index, so each load sees one uniform buffer resource   */           \
  const int li_ = ((wid & 1) << 6) | lane;                                              \
  const bool ldx_ = wid < 2, ldf_ = (TWO) && wid >= 2 && wid < 4;                       \
  uint32_t stg_[DEPTH][4];                                                              \
  _Pragma("unroll") for (int s_ = 0; s_ < (DEPTH); ++s_)                                \
    _Pragma("unroll") for (int e_ = 0; e_ < 4; ++e_) stg_[s_][e_] = 0u;                 \
  /* the block's tiles in order: pid, pid + P, ... (one cursor per wave) */             \
  TileCursor gk_ = ldx_ ? tile_cursor(x_b, x_sn, x_w, pid, a.P, N)                      \
                        : tile_cursor(f_b, f_sn, f_w, pid, a.P, N);                     \
  const int64_t gsn_ = ldx_ ? x_sn : f_sn;                                              \
  const int gC_ = ldx_ ? D : DV;                                                        \
  auto gload = [&](auto s_c) {                                                          \
    constexpr int s = decltype(s_c)::value;                                             \
    const Rsrc r_ = (ldx_ || ldf_) ? gk_.rsrc()                                         \
                                   : __builtin_amdgcn_make_buffer_rsrc(                 \
                                         const_cast<char*>(x_b), (short)0, 0, kRsrcWord3); \
    coop_tile_load<T, FAST>(stg_[s], r_, gsn_, gC_, li_);                               \
    gk_.next();                                                                         \
  };                                                                                    \
  auto tile_at = [&](int buf, int stream) -> char* {                                    \
    return tiles_ + (2 * buf + stream) * kCoopTileB;                                    \
  };                                                                                    \
  auto lstore = [&](int buf, auto s_c) {                                                \
    constexpr int s = decltype(s_c)::value;                                             \
    if (ldx_ || ldf_) coop_tile_store(tile_at(buf, ldx_ ? 0 : 1), stg_[s], li_);        \
  };
template <int V> using IC = std::integral_constant<int, V>;
// Tiles in flight per block: two for the forward kernels (at config 3's
// G = 256 with bf16 dots the slice forward 0.952 -> 0.918 ms, the deslice
// forward 0.652 -> 0.609 ms against one); one for the backward, which two
// did not speed up (1.66 ms either way: it is bound by its two barriers and
// its LDS traffic per tile).
constexpr int kCoopDepthFwd = 2, kCoopDepthBwd = 1;

// The tile loop of a block-cooperative kernel: the first DEPTH tiles
// staged and the first one published (PRE: what else the first tile needs
// before the first barrier), then BODY(t, LDS buffer, parity, ring set to
// publish and refill) per tile, unrolled over the ring and the parity.
#define COOP_TILE_LOOP(DEPTH, BODY, PRE)                                                \
  {                                                                                     \
    int t = pid, cur = 0;                                                               \
    constexpr int DP = (DEPTH);                                                         \
    static_assert(DP == 1 || DP == 2 || DP == 4, "staging depth 1, 2 or 4");           \
    gload(IC<0>());                                                                     \
    if constexpr (DP > 1) gload(IC<1 % DP>());                                          \
    if constexpr (DP > 2) {                                                             \
      gload(IC<2 % DP>());                                                              \
      gload(IC<3 % DP>());                                                              \
    }                                                                                   \
    lstore(0, IC<0>());                                                                 \
    gload(IC<0>()); /* tile DP */                                                       \
    PRE;                                                                                \
    __syncthreads();                                                                    \
    auto adv_ = [&]() {                                                                 \
      t += a.P;                                                                         \
      cur = cur == 2 ? 0 : cur + 1;                                                     \
      return t < ntiles_;                                                               \
    };                                                                                  \
    while (t < ntiles_) {                                                               \
      BODY(t, cur, TileEven(), IC<1 % DP>());                                           \
      if (!adv_()) break;                                                               \
      BODY(t, cur, TileOdd(), IC<2 % DP>());                                            \
      if (!adv_()) break;                                                               \
      if constexpr (DP > 2) {                                                           \
        BODY(t, cur, TileEven(), IC<3 % DP>());                                         \
        if (!adv_()) break;                                                             \
        BODY(t, cur, TileOdd(), IC<4 % DP>());                                          \
        if (!adv_()) break;                                                             \
      }                                                                                 \
    }                                                                                   \
  }

// ------------------------------------------------------------------ slice fwd
// z_num, s of the wave's slots. Exponentials against the wave's own row max;
// with saved statistics each weight is rescaled to the row's max and sum,
// else the waves' (max, sum) pairs are combined after the tile's barrier
// (buffers alternate by tile parity, so a wave may write the next tile's
// pair while another still reads this one's) and written to stats_out when
// asked for.
template <typename T, bool SM_>
__global__ __launch_bounds__(kCoopThreads, 4) void k_coop_slice_fwd(Args a) {
  COOP_PROLOGUE(kCoopWRegFwd)
  __syncthreads();  // the staging area becomes the transpose region
  f32x16 zacc = zero16();
  float sacc[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
  COOP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  COOP_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  (void)x_row; (void)f_row;
  const float* sm = a.stats_in ? a.stats_in + R_.stats_off() : nullptr;
  const float* st_m = a.stats_out ? a.stats_out + R_.stats_off() : nullptr;
  const float* st_l = st_m ? st_m + R_.NS : nullptr;
  auto run = [&](auto fast_c, auto sm_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    constexpr bool SM = decltype(sm_c)::value;  // saved statistics read
    COOP_STAGING(FAST, true, kCoopDepthFwd)
    // per-point statistics of the block's tiles, in order: saved ones read
    // one tile ahead (smv / slv by tile parity; a load waited for in its own
    // tile would expose a whole memory latency per tile), or formed ones
    // written by wave 0
    TileCursor km = tile_cursor(sm ? sm : st_m, 4, 4, pid, a.P, (sm || st_m) ? N : 0);
    TileCursor kl = tile_cursor(sm ? sm + R_.NS : st_l, 4, 4, pid, a.P, (sm || st_m) ? N : 0);
    float smv[2] = {0.f, 0.f}, slv[2] = {1.f, 1.f};
    auto sload = [&](int q) {
      smv[q] = ld_pt(km.rsrc(), c);
      slv[q] = ld_pt(kl.rsrc(), c);
      km.next();
      kl.next();
    };
    auto body = [&](int t, int cur, auto par, auto slot) {
      const bool pv = t * kTile + c < N;
      constexpr float sg = decltype(par)::sign;
      Frag<M> xq;
      tile_rows(xq, tile_at(cur, 0), c, h);
      float t2[16];
      COOP_LOGITS(t2, xq)
      float w[16];
      float m = 0.f;
      float* xb = xpt + (sg < 0.f ? 2 * kCoopWaves * 32 : 0);
      if constexpr (SM) {
        // w = exp2(t2 - m2) / l = exp2(t2 - sh), sh = m2 + log2 l (the
        // saved l >= 1); points beyond N get sh = kFarShift, hence w = 0
        constexpr int q = sg < 0.f ? 1 : 0;
        const float sh = pv ? fmaf(smv[q], kLog2e, __builtin_amdgcn_logf(slv[q])) : kFarShift;
        sload(q ^ 1);  // t + P
#pragma unroll
        for (int r = 0; r < 16; ++r) w[r] = __builtin_amdgcn_exp2f(t2[r] - sh);
      } else {
        m = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, t2[r]);
        m = pair_max(m);
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          w[r] = __builtin_amdgcn_exp2f(t2[r] - m);
          ls += w[r];
        }
        ls = pair_sum(ls);
        if (h == 0) {
          xb[wid * 32 + c] = m;
          xb[kCoopWaves * 32 + wid * 32 + c] = ls;
        }
      }
      lstore(cur == 2 ? 0 : cur + 1, slot);  // publish the next tile
      __syncthreads();
      gload(slot);  // tile t + (1 + depth) P into the set just published
      if constexpr (!SM) {
        float m2 = xb[c];
#pragma unroll
        for (int w_ = 1; w_ < kCoopWaves; ++w_) m2 = fmaxf(m2, xb[w_ * 32 + c]);
        float l = 0.f;
#pragma unroll
        for (int w_ = 0; w_ < kCoopWaves; ++w_)
          l += xb[kCoopWaves * 32 + w_ * 32 + c] * __builtin_amdgcn_exp2f(xb[w_ * 32 + c] - m2);
        if (wid == 0 && st_m) store_stats_at(km.rsrc(), kl.rsrc(), c, h, m2, l);
        km.next();
        kl.next();
        // w = exp2(t2 - m) exp2(m - m2) / l
        const float inv = pv ? __builtin_amdgcn_exp2f(m - m2) * __builtin_amdgcn_rcpf(l) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) w[r] *= inv;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] += w[r];
      // z_num += w^T fx: w read back transposed, fx^T straight from the
      // staged tile, chained through the accumulator (the sign alternation
      // of the fp32-accurate kernels, acc_add, is below bf16's resolution)
      Frag<M> wq, wTq, fT;
      prep<M>(wq, w);
      tr_put<M>(trS, wq, c, h, 0u);
      tr_get<M>(wTq, trS, lane);
      tr_get<M>(fT, tile_at(cur, 1), lane);
      zacc = mma<M>(fT, wTq, zacc);
    };
    COOP_TILE_LOOP(kCoopDepthFwd, body, if constexpr (SM) sload(0))
  };
  // saved statistics read (a.stats_in non-null): a compile-time case of
  // the kernel, so that each case gets its own register allocation
  using SMc = std::integral_constant<bool, SM_>;
  if (fast) run(std::true_type(), SMc()); else run(std::false_type(), SMc());
  // the block's partial: the wave's slots of z_num (rows g0 + c) and s
  const int64_t E = part_floats_slice_fwd(G, DV);
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  const float s = coop_point_sum(sacc, wreg + kCoopTr, lane);
  const int g = g0 + c;
  if (g < G) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = kmap(r, h);
      if (v < DV) pw[(int64_t)g * DV + v] = zacc[r];
    }
    if (h == 0) pw[(int64_t)G * DV + g] = s;
  }
}

// ---------------------------------------------------------------- deslice fwd
// A [point][slot] bf16 buffer of the block (rows of kPsRowB bytes): lane
// (c, h) of wave wid writes its fragment f ([point c][slot 32 wid + kmap(j,
// h)]) as four 8-byte pieces, slots 32 wid + 8 q + 4 h .. + 3.
__device__ __forceinline__ void ps_put(char* buf, const Frag<MMA_BF16>& f, int wid, int c, int h) {
  char* row = buf + c * kPsRowB + 8 * h + 64 * wid;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      *reinterpret_cast<uint2*>(row + 16 * (2 * s + hh)) =
          make_uint2(f.q[s][2 * hh], f.q[s][2 * hh + 1]);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One 16-point x 16-column block of a contraction over all of a tile's slots
// with v_mfma_f32_16x16x32_bf16 (operand lanes l supply contraction indices
// 8 (l / 16) .. + 7, the same on both operands; output lane l holds column
// l % 16 and rows 4 (l / 16) .. + 3): A = the wave's register operand ([16
// columns][slots 32 ks + 8 kg + e]), B = rows of a [point][slot] buffer read
// 16 bytes at a time. Lane (l16, kg) gets the block's point op = 16 ph + l16,
// columns 4 kg .. + 3 (of the block's 16).
__device__ __forceinline__ f32x4 ps_contract(const bf16x8 (&A)[kCoopWaves], const char* buf, int op,
                                             int kg) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const char* brow = buf + op * kPsRowB + 16 * kg;
#pragma unroll
  for (int ks = 0; ks < kCoopWaves; ++ks) {
    const bf16x8 bv = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(brow + 64 * ks));
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[ks], bv, acc, 0, 0, 0);
  }
  return acc;
}

// A wave's register operand for ps_contract: columns 16 dh .. + 15 of a
// (G x C) fp32 matrix src (row stride C), times sc, as [column][slot].
__device__ __forceinline__ void ps_operand(bf16x8 (&A)[kCoopWaves], const float* src, int G, int C,
                                           int dh, float sc, bool on, int lane) {
  const int kg = lane >> 4, col = 16 * dh + (lane & 15);
#pragma unroll
  for (int ks = 0; ks < kCoopWaves; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int g = 32 * ks + 8 * kg + e;
      A[ks][e] = (__bf16)((on && g < G && col < C) ? src[(int64_t)g * C + col] * sc : 0.f);
    }
}

// out = w tokens: every wave forms the weights of its 32 slots and writes
// them into the block's [point][slot] buffer (two, alternating by tile
// parity); after the tile's barrier waves 0..3 each contract one 16 x 16
// block of out over all slots (ps_contract) and store it, four consecutive
// columns of one point per lane. With saved statistics w = exp2(t2 - (m2 +
// log2 l)) and one barrier per tile; without, the waves' (max, sum) pairs
// are combined after a first barrier (as in the slice forward) and written
// to stats_out when asked for. Compiled for four waves per SIMD (128
// registers; its 68 KB of LDS fits two blocks per CU, which the two staged
// tiles would otherwise cost at 129).
template <typename T, bool SM_>
__global__ __launch_bounds__(kCoopThreads, 4) void k_coop_deslice_fwd(Args a) {
  COOP_PROLOGUE(kCoopWRegFwd)
  const int ph = (wid >> 1) & 1, dh = wid & 1;
  const bool out_ = wid < 4;
  const int kg = lane >> 4, l16 = lane & 15;
  bf16x8 Ao[kCoopWaves];  // tokens [v][g]
  ps_operand(Ao, a.tok + (int64_t)bh * G * DV, G, DV, dh, 1.f, out_, lane);
  __syncthreads();  // the staging area becomes the weight buffers
  char* wbuf = reinterpret_cast<char*>(smem);
  COOP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  COOP_SLICE(f, a.x, a.sxb, a.sxn, a.sxh, D)  // no second stream (never loaded)
  COOP_SLICE(o, a.o1, a.s1b, a.s1n, a.s1h, DV)
  (void)x_row; (void)f_row; (void)o_row;
  const float* sm = a.stats_in ? a.stats_in + R_.stats_off() : nullptr;
  const float* st_m = a.stats_out ? a.stats_out + R_.stats_off() : nullptr;
  const int op = 16 * ph + l16, oc = 16 * dh + 4 * kg;
  auto run = [&](auto fast_c, auto sm_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    constexpr bool SM = decltype(sm_c)::value;  // saved statistics read
    COOP_STAGING(FAST, false, kCoopDepthFwd)
    // statistics (saved ones, read one tile ahead; or computed ones,
    // written by wave 0) and out, the block's tiles in order
    const float* srow = sm ? sm : st_m;
    TileCursor km = tile_cursor(srow, 4, 4, pid, a.P, srow ? N : 0);
    TileCursor kl = tile_cursor(srow ? srow + R_.NS : nullptr, 4, 4, pid, a.P, srow ? N : 0);
    TileCursor ko = tile_cursor(o_b, o_sn, o_w, pid, a.P, N);
    const uint32_t ooff = (uint32_t)(op * o_sn) + (uint32_t)(oc * (int)sizeof(T));
    float smv[2] = {0.f, 0.f}, slv[2] = {0.f, 0.f};
    auto sload = [&](int q) {
      smv[q] = ld_pt(km.rsrc(), c);
      slv[q] = ld_pt(kl.rsrc(), c);
      km.next();
      kl.next();
    };
    auto body = [&](int t, int cur, auto par, auto slot) {
      const bool pv = t * kTile + c < N;
      constexpr float sg = decltype(par)::sign;
      constexpr int q = sg < 0.f ? 1 : 0;
      char* wb = wbuf + q * kPsBufB;
      Frag<M> xq;
      tile_rows(xq, tile_at(cur, 0), c, h);
      float t2[16], w[16];
      COOP_LOGITS(t2, xq)
      if constexpr (SM) {
        const float sh = pv ? fmaf(smv[q], kLog2e, __builtin_amdgcn_logf(slv[q])) : kFarShift;
        sload(q ^ 1);  // t + P
#pragma unroll
        for (int r = 0; r < 16; ++r) w[r] = __builtin_amdgcn_exp2f(t2[r] - sh);
        lstore(cur == 2 ? 0 : cur + 1, slot);  // publish the next tile
      } else {
        float m = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, t2[r]);
        m = pair_max(m);
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          w[r] = __builtin_amdgcn_exp2f(t2[r] - m);
          ls += w[r];
        }
        ls = pair_sum(ls);
        float* xb = xpt + q * 2 * kCoopWaves * 32;
        if (h == 0) {
          xb[wid * 32 + c] = m;
          xb[kCoopWaves * 32 + wid * 32 + c] = ls;
        }
        lstore(cur == 2 ? 0 : cur + 1, slot);  // publish the next tile
        __syncthreads();
        float m2 = xb[c];
#pragma unroll
        for (int wv = 1; wv < kCoopWaves; ++wv) m2 = fmaxf(m2, xb[wv * 32 + c]);
        float l = 0.f;
#pragma unroll
        for (int wv = 0; wv < kCoopWaves; ++wv)
          l += xb[kCoopWaves * 32 + wv * 32 + c] * __builtin_amdgcn_exp2f(xb[wv * 32 + c] - m2);
        if (wid == 0 && st_m) store_stats_at(km.rsrc(), kl.rsrc(), c, h, m2, l);
        km.next();
        kl.next();
        const float inv = pv ? __builtin_amdgcn_exp2f(m - m2) * __builtin_amdgcn_rcpf(l) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) w[r] *= inv;
      }
      Frag<M> wq;
      prep<M>(wq, w);
      ps_put(wb, wq, wid, c, h);
      __syncthreads();
      gload(slot);  // tile t + (1 + depth) P into the set just published
      const Rsrc ro = ko.rsrc();
      ko.next();
      if (out_) {
        const f32x4 acc = ps_contract(Ao, wb, op, kg);
        if (FAST) {
          Buf<T>::st4(ro, ooff, acc[0], acc[1], acc[2], acc[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            Buf<T>::st1(ro, oc + r < DV ? ooff + (uint32_t)(r * (int)sizeof(T)) : kOff, acc[r]);
        }
      }
    };
    COOP_TILE_LOOP(kCoopDepthFwd, body, if constexpr (SM) sload(0))
  };
  // saved statistics read (a.stats_in non-null): a compile-time case of
  // the kernel, so that each case gets its own register allocation
  using SMc = std::integral_constant<bool, SM_>;
  if (fast) run(std::true_type(), SMc()); else run(std::false_type(), SMc());
}

// ---------------------------------------------------------------- backward
// One pass of the slice (SLICE) or deslice backward from saved statistics:
// omega = fx . dz_num + d s (slice) or d_out . tokens (deslice); delta and
// Lb = w (omega - delta) per point; dx = Lb W / tau and (slice) dfx =
// w dz_num; dW, db, (deslice) dtokens and the dtau row terms of the wave's
// slots.
//
// dx and dfx contract over all G slots, which the eight waves hold 32 each:
// every wave writes its Lb (and w) into the block's [point][slot] buffers,
// and after the tile's second barrier four waves per output each compute a
// 16-point x 16-column block of it over all slots (ps_contract; A = (W /
// tau) [d][g] or dz_num [v][g], held in registers for the whole pass). The
// sum over slots is the MFMA's own, in a fixed order, and each lane stores
// four consecutive columns of one point.
template <typename T, bool SLICE>
__global__ __launch_bounds__(kCoopThreads, 1) void k_coop_bwd(Args a) {
  COOP_PROLOGUE(kCoopWReg)
  Frag<M> qVr;  // V [g, v] (omega)
  {
    float f_[16];
    lds_frag_rowouter(f_, wreg + 32 * kCoopStride, kCoopStride, 0, 0, c, h);
    prep<M>(qVr, f_);
  }
  f32x16 dsC = zero16();  // d s of the wave's slots, per register (slice)
  if (SLICE) {
    float dsv[16];
    lds_frag_vec(dsv, sDS + g0, h);
#pragma unroll
    for (int r = 0; r < 16; ++r) dsC[r] = dsv[r];
  }
  // this wave's output block: stream os (0 dx, 1 dfx), points 16 ph ..,
  // columns 16 dh ..; its A operand over the 8 slot steps of 32 (slots
  // 32 ks + 8 kg + e of lane group kg = lane / 16)
  const int os = SLICE ? wid >> 2 : 0, ph = (wid >> 1) & 1, dh = wid & 1;
  const bool out_ = SLICE || wid < 4;
  const int kg = lane >> 4, l16 = lane & 15;
  bf16x8 Ao[kCoopWaves];
  ps_operand(Ao, os == 0 ? Wp : a.tok + (int64_t)bh * G * DV, G, os == 0 ? D : DV, dh,
             os == 0 ? inv_tau : 1.f, out_, lane);
  __syncthreads();  // the staging regions become the transpose regions and buffers
  char* trB = reinterpret_cast<char*>(smem) + wid * kTrPieceB;
  char* lbuf = reinterpret_cast<char*>(smem) + kCoopWaves * kTrPieceB;
  char* wbuf = lbuf + kPsBufB;
  const char* obuf = os == 0 ? lbuf : wbuf;  // B operand of this wave's output
  f32x16 dW = zero16(), dT = zero16();
  float dbacc[16], dtacc = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) dbacc[r] = 0.f;
  COOP_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  COOP_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  COOP_SLICE(dx, a.o1, a.s1b, a.s1n, a.s1h, D)
  COOP_SLICE(df, a.o2, a.s2b, a.s2n, a.s2h, DV)
  (void)x_row; (void)f_row; (void)dx_row; (void)df_row;
  const float* sm = a.stats_in + R_.stats_off();
  const float* sl = sm + R_.NS;
  // the output block's lane: point 16 ph + l16, columns oc .. oc + 3
  const int op = 16 * ph + l16, oc = 16 * dh + 4 * kg;
  const int oC = os == 0 ? D : DV;
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    COOP_STAGING(FAST, true, kCoopDepthBwd)
    // the statistics of a wave's tiles, loaded one tile ahead (a load waited
    // for in the same tile would expose a whole memory latency per tile);
    // [parity]: the even / odd bodies of the unrolled loop
    float smv[2], slv[2];
    TileCursor km = tile_cursor(sm, 4, 4, pid, a.P, N), kl = tile_cursor(sl, 4, 4, pid, a.P, N);
    auto sload = [&](int q) {
      smv[q] = ld_pt(km.rsrc(), c);
      slv[q] = ld_pt(kl.rsrc(), c);
      km.next();
      kl.next();
    };
    TileCursor ko = os == 0 ? tile_cursor(dx_b, dx_sn, dx_w, pid, a.P, N)
                            : tile_cursor(df_b, df_sn, df_w, pid, a.P, N);
    const int64_t osn = os == 0 ? dx_sn : df_sn;
    const uint32_t ooff = (uint32_t)(op * osn) + (uint32_t)(oc * (int)sizeof(T));
    auto body = [&](int t, int cur, auto par, auto slot) {
      const bool pv = t * kTile + c < N;
      constexpr int q = decltype(par)::sign < 0.f ? 1 : 0;
      Frag<M> xq, fq;
      tile_rows(xq, tile_at(cur, 0), c, h);
      tile_rows(fq, tile_at(cur, 1), c, h);
      float t2[16];
      COOP_LOGITS(t2, xq)
      // w = exp2(t2 - m2) / l = exp2(t2 - sh) with sh = m2 + log2 l (the
      // saved l >= 1); points beyond N get sh = kFarShift, hence w = 0. The
      // row term below uses t2 - sh: shifting a point's logits by a constant
      // leaves sum_g Lb t2 unchanged, since sum_g Lb = 0.
      const float sh = pv ? fmaf(smv[q], kLog2e, __builtin_amdgcn_logf(slv[q])) : kFarShift;
      sload(q ^ 1);  // t + P
      float w[16], om[16];
      {
        // omega = V x (+ d s, the slice backward's per-slot term, as the
        // accumulator's initial value)
        const f32x16 o = mma<M>(qVr, fq, dsC);
        float d = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          t2[r] -= sh;
          w[r] = __builtin_amdgcn_exp2f(t2[r]);
          om[r] = o[r];
          d += w[r] * om[r];
        }
        d = pair_sum(d);
        if (h == 0) xpt[wid * 32 + c] = d;
      }
      Frag<M> wq;
      prep<M>(wq, w);
      if (!SLICE) {
        // dtokens += w^T d_out: d_out^T straight from the staged tile, w
        // read back transposed
        Frag<M> oTq, wTq;
        tr_get<M>(oTq, tile_at(cur, 1), lane);
        tr_put<M>(trB, wq, c, h, 0u);
        tr_get<M>(wTq, trB, lane);
        dT = mma<M>(oTq, wTq, dT);
      }
      lstore(cur == 2 ? 0 : cur + 1, slot);  // publish the next tile
      __syncthreads();
      gload(slot);  // tile t + (1 + depth) P into the set just published
      float delta = 0.f;
#pragma unroll
      for (int wv = 0; wv < kCoopWaves; ++wv) delta += xpt[wv * 32 + c];
      float rt = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float lb = w[r] * (om[r] - delta);
        rt = fmaf(lb, t2[r], rt);
        dbacc[r] += lb;
        om[r] = lb;
      }
      rt = pair_sum(rt);
      dtacc += (pv && h == 0) ? rt : 0.f;
      Frag<M> lq;
      prep<M>(lq, om);
      // Lb (and w) into the block's buffers for the dx (dfx) contraction
      ps_put(lbuf, lq, wid, c, h);
      if (SLICE) ps_put(wbuf, wq, wid, c, h);
      // dW += x^T Lb: x^T straight from the staged tile, Lb read back
      // transposed
      {
        Frag<M> xTq, lTq;
        tr_put<M>(trB, lq, c, h, 0u);
        tr_get<M>(lTq, trB, lane);
        tr_get<M>(xTq, tile_at(cur, 0), lane);
        dW = mma<M>(xTq, lTq, dW);
      }
      __syncthreads();
      // this wave's 16 x 16 block of dx (dfx) over all slots
      const Rsrc ro = ko.rsrc();
      ko.next();
      if (out_) {
        const f32x4 acc = ps_contract(Ao, obuf, op, kg);
        if (FAST) {
          Buf<T>::st4(ro, ooff, acc[0], acc[1], acc[2], acc[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            Buf<T>::st1(ro, oc + r < oC ? ooff + (uint32_t)(r * (int)sizeof(T)) : kOff, acc[r]);
        }
      }
    };
    COOP_TILE_LOOP(kCoopDepthBwd, body, sload(0))
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  // the block's partial: dW, db (and dtokens) of the wave's slots; dtau of
  // the block (the waves' row terms summed in a fixed order)
  const float dtw = half_wave_sum(dtacc);
  __syncthreads();
  if (lane == 0) xpt[wid] = dtw;
  const float db = coop_point_sum(dbacc, wreg + kCoopTr, lane) * inv_tau;
  __syncthreads();
  const int g = g0 + c;
  const int64_t E = SLICE ? part_floats_slice_bwd(G, D) : part_floats_deslice_bwd(G, D, DV);
  const int64_t offW = SLICE ? 0 : (int64_t)G * DV, offB = offW + (int64_t)G * D;
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  if (g < G) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = kmap(r, h);
      if (d < D) pw[offW + (int64_t)g * D + d] = dW[r] * inv_tau;
      if (!SLICE && d < DV) pw[(int64_t)g * DV + d] = dT[r];
    }
    if (h == 0) pw[offB + g] = db;
  }
  if (wid == 0 && lane == 0) {
    float dt = 0.f;
    for (int wv = 0; wv < kCoopWaves; ++wv) dt += xpt[wv];
    pw[offB + G] = -kLn2 * inv_tau * dt;
  }
}

}  // namespace fs
