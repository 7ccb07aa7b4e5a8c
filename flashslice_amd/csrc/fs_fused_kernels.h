// Whole-G ("fused") slice/deslice kernel templates for gfx950.
//
// A block is four waves working on the same (b, h): the block stages that
// head's slice projection W (G x D) and its tokens / dz_num (G x DV) in LDS
// once -- as the MFMA-ready operand fragments every tile reuses -- and each
// wave owns one point partition pid = 4 * blockIdx.x + wave, i.e. the
// strided tile sequence t = pid, pid + P, ... (a static assignment, so
// per-wave partial sums are deterministic). The whole slot axis G (padded to
// NGB blocks of 32) is held in registers, so the softmax over G is exact in
// one pass and the N x H x G weight tensor never exists outside registers.
// Every dot runs on the bf16 matrix cores (fs_mma.h): the ieee / tf32 /
// tf32x3 levels as the exact three-piece split (MMA_X6, fp32-accurate), the
// bf16 levels as plain bf16 MFMAs. Slot-indexed sums (z_num, s, dtokens, dW,
// db, dtau) are accumulated per wave, summed over the block's four waves in
// a fixed order, and written as per-block partials that fs_reduce.hip sums
// in a fixed order. The next tile's point rows are loaded
// while the current tile is computed.
//
// Reference kernels these replace: _slice_fwd_kernel (slice_ops.py:554-599),
// _deslice_fwd_kernel (:602-640), _slice_bwd_kernel (:643-710),
// _deslice_bwd_kernel (:713-776).
#pragma once
#include <type_traits>

#include "fs_mma.h"
#include "fs_tile.h"

namespace fs {

// MFMA modes of the whole-G kernels per dot kind DK: 0 = every dot fp32
// accurate (MMA_X6); 1 = value dots bf16, logits fp32 accurate (reference
// level 2, "bf16v"); 2 = every dot bf16 (level 3).
template <int DK> struct FModes {
  static constexpr int L = (DK == 2) ? MMA_BF16 : MMA_X6;
  static constexpr int V = (DK >= 1) ? MMA_BF16 : MMA_X6;
};

// LDS of one block (floats): region 0 holds first the fp32 staging of W
// [32 NGB][SW] and tokens / dz_num [32 NGB][SV] (row strides padded so
// fragment reads are conflict-free) and, once the ready fragments are
// built, the four per-wave regions of WF floats (a transpose tile, or the
// regions of split fragments transposed through LDS); then NQL ready
// fragments of the logits mode and NQV of the value mode; then two per-slot
// vectors (the scaled bias, and d s in the slice backward).
template <int NGB, int NDB, int NVB, int ML, int MV, int NQL, int NQV, int WF> struct FLds {
  static constexpr int GP = 32 * NGB;
  static constexpr int SW = 32 * NDB + 4, SV = 32 * NVB + 4;
  static constexpr int STAGE = GP * SW + GP * SV, TILES = kWavesPerBlock * WF;
  static constexpr int R0 = ((STAGE > TILES ? STAGE : TILES) + 3) / 4 * 4;
  static constexpr int QL_OFF = R0;
  static constexpr int QV_OFF = QL_OFF + NQL * frag_words<ML>() * 4;
  static constexpr int VEC_OFF = QV_OFF + NQV * frag_words<MV>() * 4;  // bias * cst, ds
  static constexpr int TOTAL = VEC_OFF + 2 * GP;
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

// Build n ready fragments of mode M into LDS (wave w builds i = w, w + 4,
// ...); src(i, f) fills the fp32 fragment i from the staged matrices.
template <int M, typename Src>
__device__ __forceinline__ void build_frags(u32x4* dst, int n, int wid, int lane, Src&& src) {
  for (int i = wid; i < n; i += kWavesPerBlock) {
    float f[16];
    src(i, f);
    Frag<M> q;
    prep<M>(q, f);
    lds_put<M>(dst + i * frag_words<M>(), q, lane);
  }
}

// Sum the four waves' partials of a block in a fixed order (wave 0, 1, 2,
// 3) through the LDS buffer `buf` (region 0: the loops' transpose tiles,
// free once every wave has left its loop) and write the block's partial
// (E floats) to `dst`. `put(buf, first)` stores (first wave) or adds this
// wave's values; every element is owned by exactly one lane of each wave.
template <typename Put>
__device__ __forceinline__ void block_partial(float* buf, int E, int wid, float* dst, Put&& put) {
  __syncthreads();
  for (int w = 0; w < kWavesPerBlock; ++w) {
    if (wid == w) put(buf, w == 0);
    __syncthreads();
  }
  for (int i = threadIdx.x; i < E; i += 256) dst[i] = buf[i];
  __syncthreads();
}
__device__ __forceinline__ void acc_put(float& t, float v, bool first) { t = first ? v : t + v; }


// Block prologue shared by the whole-G kernels: head constants and the LDS
// carve-up (FS_PROLOGUE_DECL), then the fp32 staging of W and tokens /
// dz_num and the logits operand W [g-outer, d-inner] as ready fragments
// qL[gb * NDB + db] (bias * log2(e) / tau per output slot in LDS, -1e30 on
// padded slots; FS_PROLOGUE_STAGE). The kernel builds its value-mode
// fragments next and then calls FS_PROLOGUE_END. A kernel may issue its
// first point loads between the two halves, so that they are in flight
// while the block stages W (the slice forward: 1 % at C2).
#define FS_PROLOGUE_DECL(NGB, NDB, NVB, NQV, WF)                                    \
  constexpr int ML = FModes<DK>::L, MV = FModes<DK>::V;                             \
  using SM = FLds<NGB, NDB, NVB, ML, MV, NGB * NDB, NQV, (WF)>;                    \
  __shared__ __attribute__((aligned(16))) float smem[SM::TOTAL];                    \
  const int lane = threadIdx.x & 63;                                                \
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);                 \
  const int c = lane & 31, h = lane >> 5;                                           \
  /* rev: (b, h) pairs last-first too (tile_p0) */                                  \
  const int bh = a.rev ? (int)gridDim.y - 1 - (int)blockIdx.y : (int)blockIdx.y;   \
  const int b = bh / a.H, hd = bh - b * a.H;                                       \
  const int pid = blockIdx.x * kWavesPerBlock + wid;                                \
  /* this sample's rows (row splits of a ragged batch) and per-point buffers */   \
  const Rows R_ = rows_of(a, b, hd);                                                \
  const int64_t row0_ = R_.row0;                                                    \
  const int G = a.G, D = a.D, DV = a.DV;                                            \
  const int N = R_.N;                                                               \
  const int ntiles_ = R_.ntiles;                                                    \
  const int rev_ = a.rev;                                                           \
  float* sW = smem;                                                                 \
  float* sV = smem + SM::GP * SM::SW;                                               \
  float* lds = smem + wid * (WF);                                                   \
  u32x4* qL = reinterpret_cast<u32x4*>(smem + SM::QL_OFF);                          \
  u32x4* qV = reinterpret_cast<u32x4*>(smem + SM::QV_OFF);                          \
  float* sBC = smem + SM::VEC_OFF;                                                  \
  float* sDS = sBC + SM::GP;                                                        \
  constexpr int FWL = frag_words<ML>(), FWV = frag_words<MV>();                     \
  const float* Wp = a.W + b * a.swb + hd * a.swh;                                   \
  const float* Bp = a.bias + b * a.sbb + hd * a.sbh;                                \
  const float tauf = a.tau[hd];                                                     \
  const float cst = (float)(1.4426950408889634 / (double)tauf);                    \
  const float inv_tau = 1.f / tauf;                                                 \
  const bool fast = a.fast != 0;                                                    \
  (void)inv_tau; (void)sV; (void)qV; (void)FWV; (void)DV; (void)sDS;

#define FS_PROLOGUE_STAGE(NGB, NDB, NVB)                                            \
  stage_matrix(sW, SM::SW, Wp, G, D, SM::GP, 32 * NDB);                             \
  for (int i = threadIdx.x; i < SM::GP; i += 256) sBC[i] = i < G ? Bp[i] * cst : kNoSlot; \
  if (a.tok) stage_matrix(sV, SM::SV, a.tok + (int64_t)bh * G * DV, G, DV, SM::GP, 32 * NVB); \
  __syncthreads();                                                                  \
  build_frags<ML>(qL, NGB * NDB, wid, lane, [&](int i, float(&f)[16]) {             \
    lds_frag_rowouter(f, sW, SM::SW, 32 * (i / NDB), 32 * (i % NDB), c, h);         \
  });

#define FS_PROLOGUE(NGB, NDB, NVB, NQV, WF) \
  FS_PROLOGUE_DECL(NGB, NDB, NVB, NQV, WF) FS_PROLOGUE_STAGE(NGB, NDB, NVB)

// The staged fp32 matrices are dead once every ready fragment is built: the
// transpose tiles reuse their space.
#define FS_PROLOGUE_END __syncthreads();

// Scaled logits t2 = (x . W + b) * log2(e) / tau of one tile from the
// prepared x fragments, as [point-outer, slot-inner] fragments.
#define FS_LOGITS(T2, XQ)                                                           \
  _Pragma("unroll") for (int gb = 0; gb < NGB; ++gb) {                              \
    f32x16 s_ = zero16();                                                           \
    _Pragma("unroll") for (int db = 0; db < NDB; ++db) {                            \
      Frag<ML> wq_;                                                                 \
      lds_get<ML>(wq_, qL + (gb * NDB + db) * FWL, lane);                           \
      s_ = mma<ML>(wq_, XQ[db], s_);                                                \
    }                                                                               \
    float bc_[16];                                                                  \
    lds_frag_vec(bc_, sBC + 32 * gb, h);                                            \
    _Pragma("unroll") for (int r = 0; r < 16; ++r) T2[gb][r] = fmaf(s_[r], cst, bc_[r]); \
  }

// Point slices of one (b, h): byte base, byte row stride and row width in
// bytes of a (B, N, H, C) tensor with element strides (sb, sn, sh) -- of a
// (1, rows, H, C) tensor from row row0_ on with row splits (sb = 0) -- and
// the byte offset of this lane's row c inside a tile.
#define FS_SLICE(NAME, PTR, SB, SN, SH, C)                                                \
  const char* NAME##_b =                                                                  \
      (const char*)(PTR) + (b * (SB) + row0_ * (SN) + hd * (SH)) * (int64_t)sizeof(T);    \
  const int64_t NAME##_sn = (SN) * (int64_t)sizeof(T);                                    \
  const int64_t NAME##_w = (int64_t)(C) * (int64_t)sizeof(T);                             \
  const uint32_t NAME##_row = (uint32_t)(c * NAME##_sn);


// Waves per SIMD a whole-G kernel is compiled for: two (256 registers per
// lane) for one block of 32 on every axis, one (512, the accumulators in
// AGPRs) for the wider shapes, whose slot accumulators and operand fragments
// spill at 256. The slice forward at one block is compiled for three (168
// registers, a few values spilled; 5 % faster at C2 with 1536 blocks).
constexpr int fused_waves(int ngb, int ndb, int nvb) { return ngb * ndb * nvb == 1 ? 2 : 1; }


// ------------------------------------------------------------------ slice fwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, slice_fwd_waves(NGB, NDB, NVB)) void k_fused_slice_fwd(Args a) {
  FS_PROLOGUE_DECL(NGB, NDB, NVB, 0, kLdsTile)
  f32x16 zacc[NGB][NVB];
  float sacc[NGB];
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    sacc[gb] = 0.f;
#pragma unroll
    for (int vb = 0; vb < NVB; ++vb) zacc[gb][vb] = zero16();
  }
  FS_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  FS_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  (void)f_row;
  uint32_t vcf[NVB];  // fx is read as [v-outer, point-inner]: whole-row loads
#pragma unroll
  for (int vb = 0; vb < NVB; ++vb) vcf[vb] = col_off<T>(vb, DV, f_sn, c, h);
  const float* st_m = a.stats_out ? a.stats_out + R_.stats_off() : nullptr;
  const float* st_l = st_m ? st_m + R_.NS : nullptr;
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    float xA[NDB][16], xB[NDB][16], fA[NVB][16], fB[NVB][16];
    auto load = [&](float (&xn)[NDB][16], float (&fn)[NVB][16], int t) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      ld_rows<T, NDB, FAST>(xn, rows_rsrc(x_b, x_sn, x_w, p0, N), vrx, D, h);
      const Rsrc rf = rows_rsrc(f_b, f_sn, f_w, p0, N);
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) {
        // with per-element x loads (unaligned rows, or a width not a multiple
        // of 32) the sixteen hoisted fx row offsets would be spilled, and each
        // reload from scratch would wait for every load in flight
        if constexpr (FAST) ld_cols<T>(fn[vb], rf, vcf[vb], (uint32_t)f_sn);
        else ld_cols_here<T>(fn[vb], rf, vcf[vb], (uint32_t)f_sn);
      }
    };
    // the wave's first two tiles are in flight while the block stages W
    load(xA, fA, pid);
    load(xB, fB, pid + a.P);
    FS_PROLOGUE_STAGE(NGB, NDB, NVB)
    FS_PROLOGUE_END
    auto body = [&](const float (&xf)[NDB][16], const float (&fT)[NVB][16], int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      constexpr float sg = decltype(par)::sign;
      float t2[NGB][16], w[NGB][16], m2, lsum;
      Frag<MV> fq[NVB];  // fx carries the tile's sign (acc_add)
      {
        Frag<ML> xq[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db) prep<ML>(xq[db], xf[db]);
        // one block on every axis: the logits on the matrix cores while fx
        // is split (sched_mfma_valu)
        constexpr bool IL = NGB * NDB * NVB == 1;
        if constexpr (IL) sched_fence();
        FS_LOGITS(t2, xq)
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) {
          float fs[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) fs[j] = fT[vb][j] * sg;
          prep<MV>(fq[vb], fs);
        }
        if constexpr (IL) {
          sched_mfma_valu<12, 5>();
          sched_fence();
        }
      }
      softmax_tile<NGB>(w, m2, lsum, t2, pv);
      store_stats_tile(st_m, st_l, p0, N, c, h, m2, lsum);
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) {
        float wT[16];
        transpose32(wT, w[gb], lds, c, h);
        Frag<MV> wq;
        prep<MV>(wq, wT);
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) mma_acc<MV>(zacc[gb][vb], fq[vb], wq, sg);
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) s += wT[j];
        sacc[gb] += s;
      }
    };
    FS_TILE_LOOP_LOADED(load, body, true, FS_ARGS2(xA, fA), FS_ARGS2(xB, fB))
  };
  // The wider shapes: one buffer per point stream, each reloaded for the
  // wave's next tile right after its last use (x after the logits, each
  // value block of fx right after its split), and w's split pieces held for
  // all slot blocks while fx's are held for one value block: 254 registers
  // without spills at C4's shape, two waves per SIMD.
  auto run_wide = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    float xb[NDB][16], fb[NVB][16];
    auto load_x = [&](int t) {
      ld_rows<T, NDB, FAST>(xb, rows_rsrc(x_b, x_sn, x_w, tile_p0(t, ntiles_, rev_), N), vrx, D, h);
    };
    auto load_f = [&](int t) {
      const Rsrc rf = rows_rsrc(f_b, f_sn, f_w, tile_p0(t, ntiles_, rev_), N);
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) ld_cols_here<T>(fb[vb], rf, vcf[vb], (uint32_t)f_sn);
    };
    // one value block of fx, reloaded for the wave's next tile right after
    // its split (at C4's shape 0.826 -> 0.803 ms against reloading both
    // blocks after the last product, and no scratch in the tile loop)
    auto load_f1 = [&](int t, int vb) {
      const Rsrc rf = rows_rsrc_sel(f_b, f_sn, f_w, tile_p0(t, ntiles_, rev_), N);
      ld_cols_here<T>(fb[vb], rf, vcf[vb], (uint32_t)f_sn);
    };
    auto body = [&](int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      constexpr float sg = decltype(par)::sign;
      float t2[NGB][16], w[NGB][16], m2, lsum;
      {
        Frag<ML> xq[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db) prep<ML>(xq[db], xb[db]);
        FS_LOGITS(t2, xq)
      }
      load_x(t + a.P);
      softmax_tile<NGB>(w, m2, lsum, t2, pv);
      store_stats_tile(st_m, st_l, p0, N, c, h, m2, lsum);
      // w^T of every slot block as MFMA pieces, then one value block of fx
      // at a time: the split pieces held are w's for all slot blocks and fx's
      // for one value block (instead of fx's for all of them next to w in
      // fp32), which fits two waves per SIMD at config 4's shape
      Frag<MV> wq[NGB];
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) {
        float wT[16];
        transpose32(wT, w[gb], lds, c, h);
        prep<MV>(wq[gb], wT);
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) s += wT[j];
        sacc[gb] += s;
      }
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) {
        Frag<MV> fq;  // fx carries the tile's sign (acc_add)
        {
          float fs[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) fs[j] = fb[vb][j] * sg;
          prep<MV>(fq, fs);
        }
        load_f1(t + a.P, vb);
#pragma unroll
        for (int gb = 0; gb < NGB; ++gb) mma_acc<MV>(zacc[gb][vb], fq, wq[gb], sg);
        // one value block's products (each a fresh 16-register accumulator,
        // acc_add) at a time
        sched_fence();
      }
    };
    int t = pid;
    load_x(t);
    load_f(t);
    while (t < ntiles_) {
      body(t, TileEven());
      t += a.P;
      if (t >= ntiles_) break;
      body(t, TileOdd());
      t += a.P;
    }
  };
  if constexpr (NGB * NDB * NVB > 1) {
    FS_PROLOGUE_STAGE(NGB, NDB, NVB)
    FS_PROLOGUE_END
    if (fast) run_wide(std::true_type()); else run_wide(std::false_type());
  } else {
    if (fast) run(std::true_type()); else run(std::false_type());
  }
  float ssum[NGB];
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) ssum[gb] = pair_sum(sacc[gb]);
  const int64_t E = part_floats_slice_fwd(G, DV);
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  block_partial(smem, (int)E, wid, pw, [&](float* buf, bool first) {
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      const int g = 32 * gb + c;
      if (g < G) {
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = 32 * vb + kmap(r, h);
            if (v < DV) acc_put(buf[g * DV + v], zacc[gb][vb][r], first);
          }
        if (h == 0) acc_put(buf[G * DV + g], ssum[gb], first);
      }
    }
  });
}

// ---------------------------------------------------------------- deslice fwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, fused_waves(NGB, NDB, NVB)) void k_fused_deslice_fwd(Args a) {
  FS_PROLOGUE(NGB, NDB, NVB, NVB * NGB, kLdsTile)
  // tokens as [v-outer, g-inner]: qV[vb * NGB + gb]
  build_frags<MV>(qV, NVB * NGB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_colouter(f, sV, SM::SV, 32 * (i % NGB), 32 * (i / NGB), c, h);
  });
  FS_PROLOGUE_END
  FS_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  FS_SLICE(o, a.o1, a.s1b, a.s1n, a.s1h, DV)
  (void)o_row;
  uint32_t vco[NVB];  // out is written as [v-outer, point-inner]: whole-row stores
#pragma unroll
  for (int vb = 0; vb < NVB; ++vb) vco[vb] = col_off<T>(vb, DV, o_sn, c, h);
  const float* st_m = a.stats_out ? a.stats_out + R_.stats_off() : nullptr;
  const float* st_l = st_m ? st_m + R_.NS : nullptr;
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    float xA[NDB][16], xB[NDB][16];
    auto load = [&](float (&xn)[NDB][16], int t) {
      ld_rows<T, NDB, FAST>(xn, rows_rsrc(x_b, x_sn, x_w, tile_p0(t, ntiles_, rev_), N), vrx, D, h);
    };
    auto body = [&](const float (&xf)[NDB][16], int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      float t2[NGB][16], w[NGB][16], m2, lsum;
      {
        Frag<ML> xq[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db) prep<ML>(xq[db], xf[db]);
        FS_LOGITS(t2, xq)
      }
      softmax_tile<NGB>(w, m2, lsum, t2, pv);
      store_stats_tile(st_m, st_l, p0, N, c, h, m2, lsum);
      f32x16 o[NVB];
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) o[vb] = zero16();
#pragma unroll
      for (int gb = 0; gb < NGB; ++gb) {
        Frag<MV> wq;
        prep<MV>(wq, w[gb]);
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) {
          Frag<MV> tq;
          lds_get<MV>(tq, qV + (vb * NGB + gb) * FWV, lane);
          o[vb] = mma<MV>(wq, tq, o[vb]);
        }
      }
      const Rsrc ro = rows_rsrc(o_b, o_sn, o_w, p0, N);
#pragma unroll
      for (int vb = 0; vb < NVB; ++vb) st_cols<T>(ro, vco[vb], (uint32_t)o_sn, o[vb]);
    };
    FS_TILE_LOOP(load, body, true, xA, xB)
  };
  if (fast) run(std::true_type()); else run(std::false_type());
}

// Store offsets (col_off) of NB column blocks of a point output, indexed
// like an array at each store: held in registers, formed before the tile
// loop, at one block of 32 on every axis; formed anew at each store from the
// lane index (lane_here) where RM is set, for the wider shapes, whose
// registers are full: held there, they were spilled, and each reload from
// scratch waits for every load in flight, the next tile's prefetch included.
template <typename T, bool RM, int NB>
struct StoreOffs {
  uint32_t held[NB];
  int C;
  int64_t snb;
  __device__ __forceinline__ StoreOffs(int C_, int64_t snb_, int c, int h) : C(C_), snb(snb_) {
    if constexpr (!RM) {
#pragma unroll
      for (int k = 0; k < NB; ++k) held[k] = col_off<T>(k, C, snb, c, h);
    }
  }
  __device__ __forceinline__ uint32_t operator[](int k) const {
    if constexpr (RM) {
      const int l = lane_here();
      return col_off<T>(k, C, snb, l & 31, l >> 5);
    } else {
      return held[k];
    }
  }
};

// dx = Lb (W / tau) and dW += Lb^T x, db += sum_n Lb (scaled by 1 / tau
// when the partials are written) for the two backward kernels: `om` holds
// Lb ([point-outer, slot-inner]); qWc the ready fragments of W / tau as
// [d-outer, g-inner] (index db * NGB + gb); x^T carries the tile's sign SG
// (acc_add).
#define FS_DX_DW(OM, QWC, SG)                                                       \
  {                                                                                 \
    f32x16 o_[NDB];                                                                 \
    _Pragma("unroll") for (int db = 0; db < NDB; ++db) o_[db] = zero16();           \
    _Pragma("unroll") for (int gb = 0; gb < NGB; ++gb) {                            \
      Frag<MV> aq_;                                                                 \
      prep<MV>(aq_, OM[gb]);                                                        \
      _Pragma("unroll") for (int db = 0; db < NDB; ++db) {                          \
        Frag<MV> wq_;                                                               \
        lds_get<MV>(wq_, QWC + (db * NGB + gb) * FWV, lane);                        \
        o_[db] = mma<MV>(aq_, wq_, o_[db]);                                         \
      }                                                                             \
    }                                                                               \
    const Rsrc rdx_ = rows_rsrc(dx_b, dx_sn, dx_w, p0, N);                          \
    _Pragma("unroll") for (int db = 0; db < NDB; ++db)                              \
      st_cols<T>(rdx_, vcx[db], (uint32_t)dx_sn, o_[db]);                           \
  }                                                                                 \
  {                                                                                 \
    Frag<MV> xTq_[NDB];                                                             \
    _Pragma("unroll") for (int db = 0; db < NDB; ++db) {                            \
      float xT_[16];                                                                \
      transpose32(xT_, xf[db], lds, c, h);                                          \
      _Pragma("unroll") for (int j = 0; j < 16; ++j) xT_[j] *= (SG);                \
      prep<MV>(xTq_[db], xT_);                                                      \
    }                                                                               \
    _Pragma("unroll") for (int gb = 0; gb < NGB; ++gb) {                            \
      float aT_[16];                                                                \
      transpose32(aT_, OM[gb], lds, c, h);                                          \
      Frag<MV> aTq_;                                                                \
      prep<MV>(aTq_, aT_);                                                          \
      _Pragma("unroll") for (int db = 0; db < NDB; ++db)                            \
        mma_acc<MV>(dW[gb][db], xTq_[db], aTq_, (SG));                              \
      float s_ = 0.f;                                                               \
      _Pragma("unroll") for (int j = 0; j < 16; ++j) s_ += aT_[j];                  \
      dbacc[gb] += s_;                                                              \
    }                                                                               \
  }

// FS_DX_DW for one block of 32 on every axis, from split pieces (TR): Lb is
// split once, as dx's operand; its pieces, written back with the tile's sign
// SG and read transposed, give dW's operand and db (their row sums on the
// matrix cores, the whole tile's sum in both lane halves); x^T comes from the
// pieces the logits' split left in trX.
#define FS_DX_DW_TR(OM, QWC, SG)                                                    \
  {                                                                                 \
    Frag<MV> aq_;                                                                   \
    prep<MV>(aq_, OM[0]);                                                           \
    {                                                                               \
      Frag<MV> wc_;                                                                 \
      lds_get<MV>(wc_, QWC, lane);                                                  \
      const f32x16 o_ = mma<MV>(aq_, wc_, zero16());                                \
      st_cols<T>(rows_rsrc_sel(dx_b, dx_sn, dx_w, p0, N), vcx[0], (uint32_t)dx_sn, o_);  \
    }                                                                               \
    tr_put<MV>(trS, aq_, c, h, (SG) < 0.f ? 0x80008000u : 0u);                      \
    Frag<MV> aTq_, xTq_;                                                            \
    tr_get<MV>(aTq_, trS, lane);                                                    \
    tr_get<MV>(xTq_, trX, lane);                                                    \
    mma_acc<MV>(dW[0][0], xTq_, aTq_, (SG));                                        \
    dbacc[0] = fmaf(row_sums<MV>(aTq_)[0], (SG), dbacc[0]);                         \
  }

// Per-wave LDS of the TR form: x's pieces and one more split fragment.
template <int DK> constexpr int tr_wave_floats() {
  return (tr_bytes<FModes<DK>::L>() + tr_bytes<FModes<DK>::V>()) / 4;
}

// ------------------------------------------------------------------ slice bwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, fused_waves(NGB, NDB, NVB)) void k_fused_slice_bwd(Args a) {
  // TR ((1,1,1), C2): x^T and Lb^T from split pieces read back transposed and
  // db on the matrix cores (FS_DX_DW_TR): 4 bf16x6 splits per tile instead of 6
  constexpr bool TR = NGB == 1 && NDB == 1 && NVB == 1;
  FS_PROLOGUE(NGB, NDB, NVB, 2 * NGB * NVB + NDB * NGB, TR ? tr_wave_floats<DK>() : kLdsTile)
  char* trX = reinterpret_cast<char*>(lds);
  char* trS = trX + tr_bytes<ML>();
  (void)trS;
  // dz_num as [g-outer, v-inner] (omega, qZr[gb * NVB + vb]) and [v-outer,
  // g-inner] (dfx, qZc[vb * NGB + gb]); W as [d-outer, g-inner] (dx).
  u32x4* qZr = qV;
  u32x4* qZc = qV + NGB * NVB * FWV;
  u32x4* qWc = qV + 2 * NGB * NVB * FWV;
  build_frags<MV>(qZr, NGB * NVB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_rowouter(f, sV, SM::SV, 32 * (i / NVB), 32 * (i % NVB), c, h);
  });
  build_frags<MV>(qZc, NVB * NGB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_colouter(f, sV, SM::SV, 32 * (i % NGB), 32 * (i / NGB), c, h);
  });
  build_frags<MV>(qWc, NDB * NGB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_colouter(f, sW, SM::SW, 32 * (i % NGB), 32 * (i / NGB), c, h);
#pragma unroll
    for (int j = 0; j < 16; ++j) f[j] *= inv_tau;
  });
  for (int i = threadIdx.x; i < SM::GP; i += 256) sDS[i] = i < G ? a.ds[(int64_t)bh * G + i] : 0.f;
  FS_PROLOGUE_END
  f32x16 dW[NGB][NDB];
  float dbacc[NGB], dtacc = 0.f;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    dbacc[gb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) dW[gb][db] = zero16();
  }
  FS_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  FS_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  FS_SLICE(dx, a.o1, a.s1b, a.s1n, a.s1h, D)
  FS_SLICE(df, a.o2, a.s2b, a.s2n, a.s2h, DV)
  (void)dx_row; (void)df_row;
  constexpr bool RM = NGB * NDB * NVB > 1;
  const StoreOffs<T, RM, NDB> vcx(D, dx_sn, c, h);
  const StoreOffs<T, RM, NVB> vcf(DV, df_sn, c, h);
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    const uint32_t vrf = FAST ? f_row + 4 * h * (uint32_t)sizeof(T) : f_row;
    // x is double-buffered; fx is dead once omega is formed, so its one
    // buffer is reloaded for the wave's next tile right there
    float xA[NDB][16], xB[NDB][16], ff[NVB][16];
    auto load = [&](float (&xn)[NDB][16], int t) {
      ld_rows<T, NDB, FAST>(xn, rows_rsrc_sel(x_b, x_sn, x_w, tile_p0(t, ntiles_, rev_), N), vrx, D, h);
    };
    auto load_f = [&](int t) {
      ld_rows<T, NVB, FAST>(ff, rows_rsrc_sel(f_b, f_sn, f_w, tile_p0(t, ntiles_, rev_), N), vrf, DV, h);
    };
    auto body = [&](const float (&xf)[NDB][16], int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      constexpr float sg = decltype(par)::sign;
      float t2[NGB][16], w[NGB][16], m2, lsum;
      float om[NGB][16];
      if constexpr (TR) {
        // Three regions pair an MFMA chain with independent VALU work: the
        // logits with fx's split, omega with the softmax, dfx with the
        // Jacobian (sched_mfma_valu).
        Frag<ML> xq[1];
        prep<ML>(xq[0], xf[0]);
        tr_put<ML>(trX, xq[0], c, h, 0u);
        sched_fence();
        FS_LOGITS(t2, xq)
        Frag<MV> fq;
        prep<MV>(fq, ff[0]);
        sched_mfma_valu<12, 5>();
        sched_fence();
        // omega = fx . dz_num + ds; fx is dead once split, so its buffer is
        // reloaded for the next tile a whole tile ahead
        load_f(t + a.P);
        sched_fence();
        f32x16 o;
        {
          Frag<MV> zq;
          lds_get<MV>(zq, qZr, lane);
          o = mma<MV>(zq, fq, zero16());
        }
        softmax_tile<NGB>(w, m2, lsum, t2, pv);
        sched_mfma_valu<12, 7>();
        sched_fence();
        {
          float dsv[16];  // d s per output slot
          lds_frag_vec(dsv, sDS, h);
#pragma unroll
          for (int r = 0; r < 16; ++r) om[0][r] = o[r] + dsv[r];
        }
        // dfx = w dz_num
        Frag<MV> wq;
        prep<MV>(wq, w[0]);
        sched_fence();
        {
          Frag<MV> zq;
          lds_get<MV>(zq, qZc, lane);
          const f32x16 df = mma<MV>(wq, zq, zero16());
          st_cols<T>(rows_rsrc_sel(df_b, df_sn, df_w, p0, N), vcf[0], (uint32_t)df_sn, df);
        }
        dtacc += jacobian_tile<NGB>(om, w, t2, pv, h);
        sched_mfma_valu<12, 6>();
        sched_fence();
        FS_DX_DW_TR(om, qWc, sg)
      } else {
        {
          Frag<ML> xq[NDB];
#pragma unroll
          for (int db = 0; db < NDB; ++db) prep<ML>(xq[db], xf[db]);
          FS_LOGITS(t2, xq)
        }
        // omega = fx . dz_num + ds (needs no weights: formed first, so that
        // fx's buffer is reloaded for the next tile a whole tile ahead)
        {
          Frag<MV> fq[NVB];
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) prep<MV>(fq[vb], ff[vb]);
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            f32x16 o = zero16();
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb) {
              Frag<MV> zq;
              lds_get<MV>(zq, qZr + (gb * NVB + vb) * FWV, lane);
              o = mma<MV>(zq, fq[vb], o);
            }
            float dsv[16];  // d s per output slot
            lds_frag_vec(dsv, sDS + 32 * gb, h);
#pragma unroll
            for (int r = 0; r < 16; ++r) om[gb][r] = o[r] + dsv[r];
          }
        }
        load_f(t + a.P);
        softmax_tile<NGB>(w, m2, lsum, t2, pv);
        // dfx = w dz_num
        {
          f32x16 o[NVB];
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) o[vb] = zero16();
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            Frag<MV> wq;
            prep<MV>(wq, w[gb]);
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb) {
              Frag<MV> zq;
              lds_get<MV>(zq, qZc + (vb * NGB + gb) * FWV, lane);
              o[vb] = mma<MV>(wq, zq, o[vb]);
            }
          }
          // no dfx wanted (a.o2 null): an empty range drops every store
          const Rsrc rdf = rows_rsrc_sel(df_b, df_sn, df_w, p0, a.o2 ? N : 0);
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) st_cols<T>(rdf, vcf[vb], (uint32_t)df_sn, o[vb]);
        }
        dtacc += jacobian_tile<NGB>(om, w, t2, pv, h);
        FS_DX_DW(om, qWc, sg)
      }
    };
    load_f(pid);
    FS_TILE_LOOP(load, body, true, xA, xB)
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  float dbs[NGB];  // TR: row_sums gave both lane halves the whole tile's sum
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) dbs[gb] = (TR ? dbacc[gb] : pair_sum(dbacc[gb])) * inv_tau;
  const float dt = -kLn2 * inv_tau * half_wave_sum(dtacc);
  const int64_t E = part_floats_slice_bwd(G, D);
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  block_partial(smem, (int)E, wid, pw, [&](float* buf, bool first) {
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      const int g = 32 * gb + c;
      if (g < G) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * db + kmap(r, h);
            if (d < D) acc_put(buf[g * D + d], dW[gb][db][r] * inv_tau, first);
          }
        if (h == 0) acc_put(buf[G * D + g], dbs[gb], first);
      }
    }
    if (lane == 0) acc_put(buf[G * D + G], dt, first);
  });
}

// ---------------------------------------------------------------- deslice bwd
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, fused_waves(NGB, NDB, NVB)) void k_fused_deslice_bwd(Args a) {
  // TR ((1,1,1), C2): the transposed operands (d_out^T, w^T, x^T, Lb^T) are
  // the pieces already split for omega, the logits and dx, read back
  // transposed (tr_put / tr_get), and db is their row sum on the matrix
  // cores: 4 bf16x6 splits per tile instead of 7, no fp32 transposes. Each
  // wave's LDS region holds x's pieces and one region that carries d_out's,
  // then w's, then Lb's.
  constexpr bool TR = NGB == 1 && NDB == 1 && NVB == 1;
  FS_PROLOGUE(NGB, NDB, NVB, NGB * NVB + NDB * NGB, TR ? tr_wave_floats<DK>() : kLdsTile)
  char* trX = reinterpret_cast<char*>(lds);
  char* trS = trX + tr_bytes<ML>();
  (void)trS;
  // tokens as [g-outer, v-inner] (omega, qTr[gb * NVB + vb]); W as [d-outer,
  // g-inner] (dx).
  u32x4* qTr = qV;
  u32x4* qWc = qV + NGB * NVB * FWV;
  build_frags<MV>(qTr, NGB * NVB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_rowouter(f, sV, SM::SV, 32 * (i / NVB), 32 * (i % NVB), c, h);
  });
  build_frags<MV>(qWc, NDB * NGB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_colouter(f, sW, SM::SW, 32 * (i % NGB), 32 * (i / NGB), c, h);
#pragma unroll
    for (int j = 0; j < 16; ++j) f[j] *= inv_tau;
  });
  FS_PROLOGUE_END
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
  FS_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  FS_SLICE(g, a.f, a.sfb, a.sfn, a.sfh, DV)
  FS_SLICE(dx, a.o1, a.s1b, a.s1n, a.s1h, D)
  (void)dx_row;
  const StoreOffs<T, (NGB * NDB * NVB > 1), NDB> vcx(D, dx_sn, c, h);
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    const uint32_t vrg = FAST ? g_row + 4 * h * (uint32_t)sizeof(T) : g_row;
    // x is double-buffered; d_out is dead once omega is formed, so its one
    // buffer is reloaded for the wave's next tile right there
    float xA[NDB][16], xB[NDB][16], of[NVB][16];
    auto load = [&](float (&xn)[NDB][16], int t) {
      ld_rows<T, NDB, FAST>(xn, rows_rsrc_sel(x_b, x_sn, x_w, tile_p0(t, ntiles_, rev_), N), vrx, D, h);
    };
    auto load_g = [&](int t) {
      ld_rows<T, NVB, FAST>(of, rows_rsrc_sel(g_b, g_sn, g_w, tile_p0(t, ntiles_, rev_), N), vrg, DV, h);
    };
    auto body = [&](const float (&xf)[NDB][16], int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      constexpr float sg = decltype(par)::sign;
      float t2[NGB][16], w[NGB][16], m2, lsum;
      float om[NGB][16];
      if constexpr (TR) {
        // Three regions pair an MFMA chain with independent VALU work: the
        // logits with d_out's split, omega with the softmax, dtokens with
        // the Jacobian (sched_mfma_valu).
        Frag<ML> xq[1];
        prep<ML>(xq[0], xf[0]);
        tr_put<ML>(trX, xq[0], c, h, 0u);
        sched_fence();
        FS_LOGITS(t2, xq)
        Frag<MV> oq;
        prep<MV>(oq, of[0]);
        tr_put<MV>(trS, oq, c, h, 0u);
        sched_mfma_valu<12, 5>();
        sched_fence();
        f32x16 o;
        {
          Frag<MV> tq;
          lds_get<MV>(tq, qTr, lane);
          o = mma<MV>(tq, oq, zero16());
        }
        // d_out is dead once split: its buffer is reloaded for the wave's
        // next tile a whole tile ahead
        load_g(t + a.P);
        softmax_tile<NGB>(w, m2, lsum, t2, pv);
        sched_mfma_valu<12, 7>();
        sched_fence();
        from16(om[0], o);
        // dtokens += w^T d_out: d_out^T from its pieces; w (carrying the
        // tile's sign, acc_add) split and read back transposed
        Frag<MV> oTq, wq, wTq;
        tr_get<MV>(oTq, trS, lane);
        float ws[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) ws[j] = w[0][j] * sg;
        prep<MV>(wq, ws);
        tr_put<MV>(trS, wq, c, h, 0u);
        tr_get<MV>(wTq, trS, lane);
        sched_fence();
        mma_acc<MV>(dT[0][0], oTq, wTq, sg);
        dtacc += jacobian_tile<NGB>(om, w, t2, pv, h);
        sched_mfma_valu<12, 6>();
        sched_fence();
        FS_DX_DW_TR(om, qWc, sg)
      } else {
        {
          Frag<ML> xq[NDB];
#pragma unroll
          for (int db = 0; db < NDB; ++db) prep<ML>(xq[db], xf[db]);
          FS_LOGITS(t2, xq)
        }
        // everything d_out feeds is prepared before the softmax (omega, and
        // d_out transposed for dtokens), so that its buffer is reloaded for
        // the next tile a whole tile ahead
        {
          Frag<MV> oq[NVB];
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) prep<MV>(oq[vb], of[vb]);
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            f32x16 o = zero16();
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb) {
              Frag<MV> tq;
              lds_get<MV>(tq, qTr + (gb * NVB + vb) * FWV, lane);
              o = mma<MV>(tq, oq[vb], o);
            }
            from16(om[gb], o);
          }
        }
        {
          // d_out^T, carrying the tile's sign (acc_add); split into MFMA pieces
          // here when several slot blocks share it, else next to its one use
          // (16 registers across the softmax instead of the split's 24)
          float oT[NVB][16];
          Frag<MV> oTq[NVB];
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) {
            transpose32(oT[vb], of[vb], lds, c, h);
#pragma unroll
            for (int j = 0; j < 16; ++j) oT[vb][j] *= sg;
            if constexpr (NGB > 1) prep<MV>(oTq[vb], oT[vb]);
          }
          load_g(t + a.P);
          softmax_tile<NGB>(w, m2, lsum, t2, pv);
          // dtokens += w^T d_out (rows of d_out beyond N read as zero)
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            float wT[16];
            transpose32(wT, w[gb], lds, c, h);
            Frag<MV> wTq;
            prep<MV>(wTq, wT);
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb) {
              if constexpr (NGB == 1) prep<MV>(oTq[vb], oT[vb]);
              mma_acc<MV>(dT[gb][vb], oTq[vb], wTq, sg);
            }
          }
          dtacc += jacobian_tile<NGB>(om, w, t2, pv, h);
          FS_DX_DW(om, qWc, sg)
        }
      }
    };
    load_g(pid);
    FS_TILE_LOOP(load, body, true, xA, xB)
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  float dbs[NGB];  // TR: row_sums gave both lane halves the whole tile's sum
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) dbs[gb] = (TR ? dbacc[gb] : pair_sum(dbacc[gb])) * inv_tau;
  const float dt = -kLn2 * inv_tau * half_wave_sum(dtacc);
  const int64_t offW = (int64_t)G * DV, E = part_floats_deslice_bwd(G, D, DV);
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  // two passes through the LDS buffer: dtokens, then dW, db, dtau
  block_partial(smem, (int)offW, wid, pw, [&](float* buf, bool first) {
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      const int g = 32 * gb + c;
      if (g < G) {
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = 32 * vb + kmap(r, h);
            if (v < DV) acc_put(buf[g * DV + v], dT[gb][vb][r], first);
          }
      }
    }
  });
  block_partial(smem, (int)(E - offW), wid, pw + offW, [&](float* buf, bool first) {
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      const int g = 32 * gb + c;
      if (g < G) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * db + kmap(r, h);
            if (d < D) acc_put(buf[g * D + d], dW[gb][db][r] * inv_tau, first);
          }
        if (h == 0) acc_put(buf[G * D + g], dbs[gb], first);
      }
    }
    if (lane == 0) acc_put(buf[G * D + G], dt, first);
  });
}

// ------------------------------------------------------------------- tied bwd
// Backward of a deslice -> slice coupling on one x_mid, W, b, tau (out =
// deslice(tokens), (z_num, s) = slice(fx); fx not computed from out), both
// ops' gradients from one recompute of w per tile:
//   dfx = w dz_num,  dtokens += w^T d_out,
//   omega = fx . dz_num + ds + d_out . tokens  (the two Jacobian inputs:
//   Lb = w (omega - sum_g w omega) is linear in omega, so one Jacobian, one
//   dx = Lb W / tau, one dW += Lb^T x, db, dtau serve both ops).
// Point traffic: reads x, fx, d_out, writes dx, dfx (5 passes) against the
// two backward kernels' 4 + 3 and autograd's sum of their two dx (3 more).
// Value fragments in LDS: dz_num [g, v] (omega) and [v, g] (dfx), tokens
// [g, v] (omega), W / tau [d, g] (dx). Partials in the deslice-bwd layout.
// Two waves per SIMD for one block of 32 on every axis (256 registers; the
// aligned-row tile path does not spill: 1.283 -> 1.137 ms at C2's shape with
// 1024 blocks), one for the wider shapes (the slot accumulators of both ops).
template <typename T, int DK, int NGB, int NDB, int NVB>
__global__ __launch_bounds__(256, (NGB * NDB * NVB == 1) ? 2 : 1) void k_fused_tied_bwd(Args a) {
  FS_PROLOGUE(NGB, NDB, NVB, 3 * NGB * NVB + NDB * NGB, kLdsTile)
  static_assert(SM::TOTAL * 4 <= 160 * 1024, "tied backward LDS exceeds 160 KB");
  u32x4* qZr = qV;
  u32x4* qZc = qV + NGB * NVB * FWV;
  u32x4* qTr = qV + 2 * NGB * NVB * FWV;
  u32x4* qWc = qV + 3 * NGB * NVB * FWV;
  build_frags<MV>(qZr, NGB * NVB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_rowouter(f, sV, SM::SV, 32 * (i / NVB), 32 * (i % NVB), c, h);
  });
  build_frags<MV>(qZc, NVB * NGB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_colouter(f, sV, SM::SV, 32 * (i % NGB), 32 * (i / NGB), c, h);
  });
  build_frags<MV>(qWc, NDB * NGB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_colouter(f, sW, SM::SW, 32 * (i % NGB), 32 * (i / NGB), c, h);
#pragma unroll
    for (int j = 0; j < 16; ++j) f[j] *= inv_tau;
  });
  for (int i = threadIdx.x; i < SM::GP; i += 256) sDS[i] = i < G ? a.ds[(int64_t)bh * G + i] : 0.f;
  // the staging area now takes the tokens (dz_num's fragments are built)
  __syncthreads();
  stage_matrix(sV, SM::SV, a.tok2 + (int64_t)bh * G * DV, G, DV, SM::GP, 32 * NVB);
  __syncthreads();
  build_frags<MV>(qTr, NGB * NVB, wid, lane, [&](int i, float(&f)[16]) {
    lds_frag_rowouter(f, sV, SM::SV, 32 * (i / NVB), 32 * (i % NVB), c, h);
  });
  FS_PROLOGUE_END
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
  FS_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  FS_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  FS_SLICE(g, a.g, a.sgb, a.sgn, a.sgh, DV)
  FS_SLICE(dx, a.o1, a.s1b, a.s1n, a.s1h, D)
  FS_SLICE(df, a.o2, a.s2b, a.s2n, a.s2h, DV)
  (void)dx_row; (void)df_row;
  constexpr bool RM = NGB * NDB * NVB > 1;
  const StoreOffs<T, RM, NDB> vcx(D, dx_sn, c, h);
  const StoreOffs<T, RM, NVB> vcf(DV, df_sn, c, h);
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    const uint32_t vrf = FAST ? f_row + 4 * h * (uint32_t)sizeof(T) : f_row;
    const uint32_t vrg = FAST ? g_row + 4 * h * (uint32_t)sizeof(T) : g_row;
    // x is double-buffered; fx and d_out have one buffer each, reloaded
    // once omega and d_out's transpose have consumed them
    float xA[NDB][16], xB[NDB][16], ff[NVB][16], of[NVB][16];
    auto load = [&](float (&xn)[NDB][16], int t) {
      ld_rows<T, NDB, FAST>(xn, rows_rsrc_sel(x_b, x_sn, x_w, tile_p0(t, ntiles_, rev_), N), vrx, D, h);
    };
    auto load_f = [&](int t) {
      ld_rows<T, NVB, FAST>(ff, rows_rsrc_sel(f_b, f_sn, f_w, tile_p0(t, ntiles_, rev_), N), vrf, DV, h);
    };
    auto load_g = [&](int t) {
      ld_rows<T, NVB, FAST>(of, rows_rsrc_sel(g_b, g_sn, g_w, tile_p0(t, ntiles_, rev_), N), vrg, DV, h);
    };
    auto body = [&](const float (&xf)[NDB][16], int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      constexpr float sg = decltype(par)::sign;
      float t2[NGB][16], w[NGB][16], m2, lsum;
      float om[NGB][16];
      {
        Frag<ML> xq[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db) prep<ML>(xq[db], xf[db]);
        FS_LOGITS(t2, xq)
      }
      // omega = fx . dz_num + d_out . tokens + ds, one accumulator per slot
      // block; one value block's split pieces live at a time
      {
        f32x16 o[NGB];
#pragma unroll
        for (int gb = 0; gb < NGB; ++gb) o[gb] = zero16();
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) {
          Frag<MV> fq;
          prep<MV>(fq, ff[vb]);
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            Frag<MV> zq;
            lds_get<MV>(zq, qZr + (gb * NVB + vb) * FWV, lane);
            o[gb] = mma<MV>(zq, fq, o[gb]);
          }
        }
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) {
          Frag<MV> oq;
          prep<MV>(oq, of[vb]);
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            Frag<MV> tq;
            lds_get<MV>(tq, qTr + (gb * NVB + vb) * FWV, lane);
            o[gb] = mma<MV>(tq, oq, o[gb]);
          }
        }
#pragma unroll
        for (int gb = 0; gb < NGB; ++gb) {
          float dsv[16];  // d s per output slot
          lds_frag_vec(dsv, sDS + 32 * gb, h);
#pragma unroll
          for (int r = 0; r < 16; ++r) om[gb][r] = o[gb][r] + dsv[r];
        }
      }
      {
        // d_out^T carrying the tile's sign (acc_add), split here when several
        // slot blocks share it, else next to its one use
        float oT[NVB][16];
        Frag<MV> oTq[NVB];
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb) {
          transpose32(oT[vb], of[vb], lds, c, h);
#pragma unroll
          for (int j = 0; j < 16; ++j) oT[vb][j] *= sg;
          if constexpr (NGB > 1) prep<MV>(oTq[vb], oT[vb]);
        }
        softmax_tile<NGB>(w, m2, lsum, t2, pv);
        // dtokens += w^T d_out (rows of d_out beyond N read as zero), first:
        // d_out's transposed pieces die before dfx's accumulators are live
#pragma unroll
        for (int gb = 0; gb < NGB; ++gb) {
          float wT[16];
          transpose32(wT, w[gb], lds, c, h);
          Frag<MV> wTq;
          prep<MV>(wTq, wT);
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) {
            if constexpr (NGB == 1) prep<MV>(oTq[vb], oT[vb]);
            mma_acc<MV>(dT[gb][vb], oTq[vb], wTq, sg);
          }
        }
        // dfx = w dz_num (rows beyond N are not stored)
        {
          f32x16 o[NVB];
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) o[vb] = zero16();
#pragma unroll
          for (int gb = 0; gb < NGB; ++gb) {
            Frag<MV> wq;
            prep<MV>(wq, w[gb]);
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb) {
              Frag<MV> zq;
              lds_get<MV>(zq, qZc + (vb * NGB + gb) * FWV, lane);
              o[vb] = mma<MV>(wq, zq, o[vb]);
            }
          }
          // no dfx wanted (a.o2 null): an empty range drops every store
          const Rsrc rdf = rows_rsrc_sel(df_b, df_sn, df_w, p0, a.o2 ? N : 0);
#pragma unroll
          for (int vb = 0; vb < NVB; ++vb) st_cols<T>(rdf, vcf[vb], (uint32_t)df_sn, o[vb]);
        }
        dtacc += jacobian_tile<NGB>(om, w, t2, pv, h);
        // fx and d_out are reloaded for the wave's next tile only now: from
        // omega to here (the register peak) their buffers are dead, and dx,
        // dW and the next tile's logits still cover the loads' latency
        load_f(t + a.P);
        load_g(t + a.P);
        FS_DX_DW(om, qWc, sg)
      }
    };
    load_f(pid);
    load_g(pid);
    FS_TILE_LOOP(load, body, true, xA, xB)
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  float dbs[NGB];
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) dbs[gb] = pair_sum(dbacc[gb]) * inv_tau;
  const float dt = -kLn2 * inv_tau * half_wave_sum(dtacc);
  const int64_t offW = (int64_t)G * DV, E = part_floats_deslice_bwd(G, D, DV);
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  block_partial(smem, (int)offW, wid, pw, [&](float* buf, bool first) {
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      const int g = 32 * gb + c;
      if (g < G) {
#pragma unroll
        for (int vb = 0; vb < NVB; ++vb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = 32 * vb + kmap(r, h);
            if (v < DV) acc_put(buf[g * DV + v], dT[gb][vb][r], first);
          }
      }
    }
  });
  block_partial(smem, (int)(E - offW), wid, pw + offW, [&](float* buf, bool first) {
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      const int g = 32 * gb + c;
      if (g < G) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * db + kmap(r, h);
            if (d < D) acc_put(buf[g * D + d], dW[gb][db][r] * inv_tau, first);
          }
        if (h == 0) acc_put(buf[G * D + g], dbs[gb], first);
      }
    }
    if (lane == 0) acc_put(buf[G * D + G], dt, first);
  });
}

// ------------------------------------------- tied bwd without dtokens, TR
// The tied backward of a slice -> deslice coupling (slice-first: dtokens has
// been formed before this pass, by the slice forward kernel on d_out, and
// is not asked for) at one block of 32 on every axis (C2's shape): the
// slice backward's tile body (TR form of k_fused_slice_bwd: x^T and Lb^T
// from split pieces read back transposed, db on the matrix cores) with the
// deslice's Jacobian input added to omega: omega = fx . dz_num + d_out .
// tokens + ds. Per tile: 5 bf16x6 splits (x, fx, d_out, w, Lb) and 78 bf16
// MFMAs, against k_fused_tied_bwd's general body, which also forms d_out^T
// and w^T for dtokens (two more splits, 12 more MFMAs) and splits x and Lb
// again for their transposes. Partials in the deslice-bwd layout, the
// dtokens part left unwritten.
template <typename T, int DK>
__global__ __launch_bounds__(256, 2) void k_fused_tied_nodt(Args a) {
  constexpr int NGB = 1, NDB = 1, NVB = 1;
  FS_PROLOGUE(NGB, NDB, NVB, 4, tr_wave_floats<DK>())
  char* trX = reinterpret_cast<char*>(lds);
  char* trS = trX + tr_bytes<ML>();
  // dz_num as [g-outer, v-inner] (omega) and [v-outer, g-inner] (dfx),
  // tokens as [g-outer, v-inner] (omega), W / tau as [d-outer, g-inner] (dx)
  u32x4* qZr = qV;
  u32x4* qZc = qV + FWV;
  u32x4* qTr = qV + 2 * FWV;
  u32x4* qWc = qV + 3 * FWV;
  build_frags<MV>(qZr, 1, wid, lane, [&](int, float(&f)[16]) {
    lds_frag_rowouter(f, sV, SM::SV, 0, 0, c, h);
  });
  if (wid == 1) {
    float f[16];
    lds_frag_colouter(f, sV, SM::SV, 0, 0, c, h);
    Frag<MV> q;
    prep<MV>(q, f);
    lds_put<MV>(qZc, q, lane);
  } else if (wid == 2) {
    float f[16];
    lds_frag_colouter(f, sW, SM::SW, 0, 0, c, h);
#pragma unroll
    for (int j = 0; j < 16; ++j) f[j] *= inv_tau;
    Frag<MV> q;
    prep<MV>(q, f);
    lds_put<MV>(qWc, q, lane);
  }
  for (int i = threadIdx.x; i < SM::GP; i += 256) sDS[i] = i < G ? a.ds[(int64_t)bh * G + i] : 0.f;
  // the staging area now takes the tokens (dz_num's fragments are built)
  __syncthreads();
  stage_matrix(sV, SM::SV, a.tok2 + (int64_t)bh * G * DV, G, DV, SM::GP, 32);
  __syncthreads();
  if (wid == 3) {
    float f[16];
    lds_frag_rowouter(f, sV, SM::SV, 0, 0, c, h);
    Frag<MV> q;
    prep<MV>(q, f);
    lds_put<MV>(qTr, q, lane);
  }
  FS_PROLOGUE_END
  f32x16 dW[1][1];
  dW[0][0] = zero16();
  float dbacc[1] = {0.f}, dtacc = 0.f;
  FS_SLICE(x, a.x, a.sxb, a.sxn, a.sxh, D)
  FS_SLICE(f, a.f, a.sfb, a.sfn, a.sfh, DV)
  FS_SLICE(g, a.g, a.sgb, a.sgn, a.sgh, DV)
  FS_SLICE(dx, a.o1, a.s1b, a.s1n, a.s1h, D)
  FS_SLICE(df, a.o2, a.s2b, a.s2n, a.s2h, DV)
  (void)dx_row; (void)df_row;
  uint32_t vcx[1], vcf[1];
  vcx[0] = col_off<T>(0, D, dx_sn, c, h);
  vcf[0] = col_off<T>(0, DV, df_sn, c, h);
  auto run = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const uint32_t vrx = FAST ? x_row + 4 * h * (uint32_t)sizeof(T) : x_row;
    const uint32_t vrf = FAST ? f_row + 4 * h * (uint32_t)sizeof(T) : f_row;
    const uint32_t vrg = FAST ? g_row + 4 * h * (uint32_t)sizeof(T) : g_row;
    // x is double-buffered; fx and d_out have one buffer each, reloaded for
    // the wave's next tile as soon as each is split
    float xA[1][16], xB[1][16], ff[1][16], of[1][16];
    auto load = [&](float (&xn)[1][16], int t) {
      ld_rows<T, 1, FAST>(xn, rows_rsrc_sel(x_b, x_sn, x_w, tile_p0(t, ntiles_, rev_), N), vrx, D, h);
    };
    auto load_f = [&](int t) {
      ld_rows<T, 1, FAST>(ff, rows_rsrc_sel(f_b, f_sn, f_w, tile_p0(t, ntiles_, rev_), N), vrf, DV, h);
    };
    auto load_g = [&](int t) {
      ld_rows<T, 1, FAST>(of, rows_rsrc_sel(g_b, g_sn, g_w, tile_p0(t, ntiles_, rev_), N), vrg, DV, h);
    };
    auto body = [&](const float (&xf)[1][16], int t, auto par) {
      const int64_t p0 = tile_p0(t, ntiles_, rev_);
      const bool pv = p0 + c < N;
      constexpr float sg = decltype(par)::sign;
      float t2[1][16], w[1][16], m2, lsum;
      float om[1][16];
      // Four regions pair an MFMA chain with independent VALU work: the
      // logits with fx's split, fx . dz_num with d_out's split, d_out .
      // tokens with the softmax, dfx with the Jacobian (sched_mfma_valu).
      Frag<ML> xq[1];
      prep<ML>(xq[0], xf[0]);
      tr_put<ML>(trX, xq[0], c, h, 0u);
      sched_fence();
      FS_LOGITS(t2, xq)
      Frag<MV> fq;
      prep<MV>(fq, ff[0]);
      sched_mfma_valu<12, 5>();
      sched_fence();
      load_f(t + a.P);
      sched_fence();
      f32x16 o;
      {
        Frag<MV> zq;
        lds_get<MV>(zq, qZr, lane);
        o = mma<MV>(zq, fq, zero16());
      }
      Frag<MV> gq;
      prep<MV>(gq, of[0]);
      sched_mfma_valu<12, 5>();
      sched_fence();
      load_g(t + a.P);
      sched_fence();
      {
        Frag<MV> tq;
        lds_get<MV>(tq, qTr, lane);
        o = mma<MV>(tq, gq, o);
      }
      softmax_tile<NGB>(w, m2, lsum, t2, pv);
      sched_mfma_valu<12, 7>();
      sched_fence();
      {
        float dsv[16];  // d s per output slot
        lds_frag_vec(dsv, sDS, h);
#pragma unroll
        for (int r = 0; r < 16; ++r) om[0][r] = o[r] + dsv[r];
      }
      // dfx = w dz_num (no dfx wanted, a.o2 null: an empty range drops the stores)
      Frag<MV> wq;
      prep<MV>(wq, w[0]);
      sched_fence();
      {
        Frag<MV> zq;
        lds_get<MV>(zq, qZc, lane);
        const f32x16 df = mma<MV>(wq, zq, zero16());
        st_cols<T>(rows_rsrc_sel(df_b, df_sn, df_w, p0, a.o2 ? N : 0), vcf[0], (uint32_t)df_sn,
                   df);
      }
      dtacc += jacobian_tile<NGB>(om, w, t2, pv, h);
      sched_mfma_valu<12, 6>();
      sched_fence();
      FS_DX_DW_TR(om, qWc, sg)
    };
    load_f(pid);
    load_g(pid);
    FS_TILE_LOOP(load, body, true, xA, xB)
  };
  if (fast) run(std::true_type()); else run(std::false_type());
  const float dbs = dbacc[0] * inv_tau;  // row_sums gave both lane halves the whole tile's sum
  const float dt = -kLn2 * inv_tau * half_wave_sum(dtacc);
  const int64_t offW = (int64_t)G * DV, E = part_floats_deslice_bwd(G, D, DV);
  float* pw = a.part + ((int64_t)bh * gridDim.x + blockIdx.x) * E;
  block_partial(smem, (int)(E - offW), wid, pw + offW, [&](float* buf, bool first) {
    if (c < G) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = kmap(r, h);
        if (d < D) acc_put(buf[c * D + d], dW[0][0][r] * inv_tau, first);
      }
      if (h == 0) acc_put(buf[G * D + c], dbs, first);
    }
    if (lane == 0) acc_put(buf[G * D + G], dt, first);
  });
}

// ------------------------------------------------------------ launch templates
// (NGB, NDB, NVB): slot, logits-width and value-width blocks of 32 held in
// registers; the fused family serves shapes whose slot-indexed accumulators
// fit (NGB * NDB <= 4 and NGB * NVB <= 4).
#define FS_COMBOS(X) \
  X(1, 1, 1) X(1, 1, 2) X(1, 1, 4) X(1, 2, 1) X(1, 2, 2) X(1, 2, 4) X(1, 4, 1) X(1, 4, 2) \
  X(1, 4, 4) X(2, 1, 1) X(2, 1, 2) X(2, 2, 1) X(2, 2, 2) X(4, 1, 1)

enum FusedKind {
  FK_SLICE_FWD = 0,
  FK_DESLICE_FWD = 1,
  FK_SLICE_BWD = 2,
  FK_DESLICE_BWD = 3,
  FK_TIED_BWD = 4
};

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
  if constexpr (K == FK_TIED_BWD) {
    if (a.no_dtok && g == 1 && d == 1 && v == 1) {
      hipLaunchKernelGGL((k_fused_tied_nodt<T, DK>), grid, block, 0, st, a);
      return hipGetLastError();
    }
  }
#define FS_TRY(G_, D_, V_)                                                                    \
  if (g == G_ && d == D_ && v == V_) {                                                        \
    if constexpr (K == FK_SLICE_FWD)                                                          \
      hipLaunchKernelGGL((k_fused_slice_fwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);      \
    else if constexpr (K == FK_DESLICE_FWD)                                                   \
      hipLaunchKernelGGL((k_fused_deslice_fwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);    \
    else if constexpr (K == FK_SLICE_BWD)                                                     \
      hipLaunchKernelGGL((k_fused_slice_bwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);      \
    else if constexpr (K == FK_TIED_BWD)                                                      \
      hipLaunchKernelGGL((k_fused_tied_bwd<T, DK, G_, D_, V_>), grid, block, 0, st, a);       \
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
  X(3, _Float16, 1) X(3, _Float16, 2)                                                \
  X(4, float, 0) X(4, __bf16, 0) X(4, __bf16, 1) X(4, __bf16, 2) X(4, _Float16, 0)   \
  X(4, _Float16, 1) X(4, _Float16, 2)

#define FS_DECLARE_EXTERN(K_, T_, DK_) \
  extern template hipError_t fused_launch<K_, T_, DK_>(const Args&, hipStream_t);
FS_FUSED_INSTANCES(FS_DECLARE_EXTERN)
#undef FS_DECLARE_EXTERN

}  // namespace fs
