// C-ABI of the FlashSlice HIP kernels (declared in include/flashslice_hip.h).
//
// Validates every argument before any launch, picks the kernel family
// (whole-G when the slot axis fits in registers, else G-blocked), derives the
// launch geometry from the shape alone (never from the device, so the
// per-wave partial layout -- and therefore every sum's order -- is the same
// on every run and every GPU), carves the caller's workspace, launches the
// point-streaming kernels and then the fixed-order reduction of their
// partials. Nothing here allocates, frees or synchronises.
#include <initializer_list>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/flashslice_hip.h"
#include "fs_internal.h"

namespace {

thread_local std::string g_err;

int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int32_t hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return FS_OK;
  if (e == hipErrorNotSupported)
    return fail(FS_ERR_UNSUPPORTED, "%s: no kernel instantiation serves this shape", what);
  return fail(FS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ------------------------------------------------------------------ geometry
// Point-owned grids: blocks of 4 waves on one (b, h), grid (P / 4, B * H);
// the number of blocks targets the waves each kernel keeps resident per SIMD
// on a 256-CU MI355X. Slot-owned grids add ceil(G / 32) along z.
struct Geo {
  int ntiles, P;
};

Geo geo_n(const fs_slice_params* p, int64_t target_blocks) {
  Geo g;
  g.ntiles = (int)((p->N + fs::kTile - 1) / fs::kTile);
  const int64_t bh = p->B * p->H;
  int64_t bx = (target_blocks + bh - 1) / bh;
  const int64_t need = (g.ntiles + fs::kWavesPerBlock - 1) / fs::kWavesPerBlock;
  if (bx > need) bx = need;
  if (bx < 1) bx = 1;
  g.P = (int)(bx * fs::kWavesPerBlock);
  return g;
}

// partials per (b, h) of a whole-G launch: one per block of four waves
int pb(const Geo& g) { return g.P / fs::kWavesPerBlock; }

// Blocks per launch of the G-blocked kernels by kind, measured on MI355X at
// C3 (N = 1e6, H = 8, D = DV = 32, G = 256 and 1024). The point-owned kernels
// run best with several times more blocks than stay resident (the statistics
// pass and the deslice most: 0.90 -> 0.68 ms for the deslice at G = 256 with
// bf16 dots). The slot-owned ones want more with the bf16x6 split (their
// 4096-block grids 6 % faster at G = 1024) and the fewest with bf16 dots
// (dk 2: 512; 4096 was 15 % slower).
enum GpGrid { GPG_STATS, GPG_DESLICE, GPG_BWD_N, GPG_SLOT };
int64_t gp_blocks(GpGrid k, int dk) {
  switch (k) {
    case GPG_STATS: return 2048;
    case GPG_DESLICE: return 4096;
    case GPG_BWD_N: return 2048;
    default: return dk == 2 ? 512 : 4096;
  }
}

constexpr int64_t kRaggedBlocksPerBH = 8;
Geo geo_gp(const fs_slice_params* p, GpGrid k, int dk) {
  int64_t t = gp_blocks(k, dk);
  // a ragged batch: at least a few blocks per (sample, head), as the whole-G
  // launches below
  const int64_t rt = kRaggedBlocksPerBH * p->B * p->H;
  if (p->row_splits && rt > t) t = rt;
  return geo_n(p, t);
}

// slot-owned grids: the target is shared among the ceil(G / 32) slot blocks;
// dk -1 sizes for the largest of the dot kinds (workspace planning)
Geo geo_g(const fs_slice_params* p, int dk) {
  const int64_t nsg = (p->G + 31) / 32;
  const int64_t t = dk < 0 ? gp_blocks(GPG_SLOT, 0) : gp_blocks(GPG_SLOT, dk);
  return geo_n(p, (t + nsg - 1) / nsg);
}

// The block-cooperative G-blocked kernels (fs_coop_kernels.h): bf16 dots
// (dot kind 2) on 16-bit point tensors at 128 < G <= 256, D, DV <= 32. One
// 8-wave block per CU (86 KB of LDS, two waves per SIMD), so the grid targets
// one block per CU; P = blocks per (b, h), at most the G-blocked slot-owned
// grid's partitions, whose partial buffer it reuses (one partial per block).
// The slice forward (128 registers, 68 KB of LDS) fits two blocks per CU.
constexpr int64_t kCoopBlocksBwd = 256, kCoopBlocksFwd = 512;
bool coop_on(const fs_slice_params* p, int mode) {
  return mode == 2 && fs::coop_ok((int)p->G, (int)p->D, (int)p->DV);
}
Geo geo_coop(const fs_slice_params* p, int64_t target) {
  Geo g;
  g.ntiles = (int)((p->N + fs::kTile - 1) / fs::kTile);
  const int64_t bh = p->B * p->H;
  int64_t P = (target + bh - 1) / bh;
  if (P > g.ntiles) P = g.ntiles;
  if (P < 1) P = 1;
  const int64_t cap = geo_g(p, -1).P;
  g.P = (int)(P < cap ? P : cap);
  return g;
}

// Blocks per launch of the whole-G kernels (measured on MI355X at C2: N = 1e6,
// H = 8, D = DV = G = 32, and at C4: G = 64, DV = 64): at C2's shape the
// kernels run best with several times more blocks than stay resident, so
// that the hardware keeps refilling CUs as blocks finish -- except the
// deslice backward, whose blocks each stream long runs of tiles; the wider
// shapes' one-wave-per-SIMD kernels run best in one dispatch round.
// A ragged batch (row splits) sizes its grid by the longest sample, so every
// (sample, head) gets the same blocks: at least 8 each, so that the longest
// samples' tiles are spread over enough waves to keep the tail short
// (measured on 64 meshes of N ~ U[2000, 40000]: 4.31 ms per step with the
// plain targets, 4.20 / 3.67 / 3.75 ms with 4 / 8 / 16 blocks per pair).
int64_t fused_target(int32_t op, const fs_slice_params* p) {
  const bool one = p->G <= 32 && p->D <= 32 && p->DV <= 32;
  int64_t t;
  switch (op) {
    // wider shapes: one block per CU, one dispatch round (C4: 2.056 -> 2.000
    // ms against 512 blocks, bf16 points and dots 0.962 -> 0.916; 384: 2.59)
    case FS_OP_DESLICE_BWD: t = one ? 512 : 256; break;
    // wider shapes: one wave per SIMD, one 125 KB block per CU at C4, one
    // dispatch round (measured at C4 against 512 / 1024 / 2048 blocks: 1 / 3 /
    // 9 % faster); one block of 32 on every axis: two waves per SIMD, 1536
    // blocks (C2's shape, the transposed-piece kernel without dtokens:
    // 1.180 / 1.119 / 1.070 / 1.057 / 1.084 ms at 512 / 768 / 1024 / 1536 /
    // 2048)
    case FS_OP_TIED_BWD: t = one ? 1536 : 256; break;
    // wider shapes: one dispatch round of the kernel's waves per SIMD (one
    // wave, 256 blocks; C4 at one wave: 0.973 ms against 0.995 at 512)
    case FS_OP_SLICE_FWD: {
      auto b32 = [](int64_t n) { return n <= 32 ? 1 : n <= 64 ? 2 : n <= 128 ? 4 : 8; };
      t = one ? 1536 : 256 * fs::slice_fwd_waves(b32(p->G), b32(p->D), b32(p->DV));
      break;
    }
    // wider shapes: one wave per SIMD and one 100 KB block per CU at C4, one
    // dispatch round (measured at C4: 1.99 ms against 2.13 at 1536 blocks,
    // 2.03 at 512)
    case FS_OP_SLICE_BWD: t = one ? 1536 : 256; break;
    // wider shapes: two waves per SIMD (C4: 0.680 ms at 1024 blocks against
    // 0.690 / 0.684 / 0.696 at 1536 / 512 / 2048)
    case FS_OP_DESLICE_FWD: t = one ? 2048 : 1024; break;
    default: t = 1536;
  }
  const int64_t rt = kRaggedBlocksPerBH * p->B * p->H;
  if (p->row_splits && rt > t) t = rt;
  return t;
}

// Sweep direction of the whole-G kernels (Args::rev, tile_p0): the slice
// forward and the deslice backward visit the (b, h) pairs and their tiles in
// order, the deslice forward, the slice backward and the merged backward
// last-first. In both orders a training step runs them in -- slice forward,
// deslice forward, dtokens pass (the slice forward's kernel), merged
// backward; or slice forward, deslice forward, deslice backward, slice
// backward -- each kernel then starts on the points its predecessor touched
// last, part of which the 256 MB last-level cache still holds. Measured on
// C2's coupling step (three runs, two boxes): 2.298 / 2.338 / 2.326 ms
// against 2.301 / 2.342 / 2.373 with every pass in order; the slice forward
// and the dtokens pass gain 2-3 %, the reversed deslice forward loses ~2 %
// (reversing the tiles alone, not the pairs, changed nothing).
int sweep_rev(int32_t op) {
  return op == FS_OP_DESLICE_FWD || op == FS_OP_SLICE_BWD || op == FS_OP_TIED_BWD;
}

// ------------------------------------------------------------------ checks
int32_t check_params(const fs_slice_params* p, const char* who) {
  if (!p) return fail(FS_ERR_INVALID, "%s: params is NULL", who);
  if (p->B < 1 || p->N < 1 || p->H < 1)
    return fail(FS_ERR_INVALID, "%s: B, N, H must be >= 1 (got %lld, %lld, %lld)", who,
                (long long)p->B, (long long)p->N, (long long)p->H);
  if (p->D < 1 || p->D > 256 || p->DV < 1 || p->DV > 256)
    return fail(FS_ERR_INVALID, "%s: D and DV must be in [1, 256] (got %lld, %lld)", who,
                (long long)p->D, (long long)p->DV);
  if (p->G < 1) return fail(FS_ERR_INVALID, "%s: G must be >= 1 (got %lld)", who, (long long)p->G);
  if (p->G > (1 << 20))
    return fail(FS_ERR_INVALID, "%s: G = %lld exceeds 2^20", who, (long long)p->G);
  if (p->N > (int64_t)0x7fffffff - 64)
    return fail(FS_ERR_INVALID, "%s: N = %lld exceeds 2^31 - 64", who, (long long)p->N);
  if (p->B * p->H > 65535)
    return fail(FS_ERR_INVALID, "%s: B * H = %lld exceeds 65535", who, (long long)(p->B * p->H));
  if (!p->weight || !p->bias || !p->tau)
    return fail(FS_ERR_INVALID, "%s: weight, bias and tau must be non-NULL", who);
  if (p->dot < 0 || p->dot > 4)
    return fail(FS_ERR_INVALID, "%s: dot level %d is not in [0, 4]", who, p->dot);
  if (p->family < 0 || p->family > 2)
    return fail(FS_ERR_INVALID, "%s: family %d is not 0, 1 or 2", who, p->family);
  if (p->row_splits && (p->total_rows < 1 || p->total_rows > (int64_t)0x7fffffff - 64))
    return fail(FS_ERR_INVALID, "%s: total_rows = %lld must be in [1, 2^31 - 64] with row splits",
                who, (long long)p->total_rows);
  return FS_OK;
}

int32_t check_points(const fs_points* t, const char* name, int64_t width, const char* who) {
  if (!t || !t->data) return fail(FS_ERR_INVALID, "%s: %s is NULL", who, name);
  if (t->dtype < 0 || t->dtype > 2)
    return fail(FS_ERR_INVALID, "%s: %s has unknown dtype %d", who, name, t->dtype);
  if (t->width != width)
    return fail(FS_ERR_INVALID, "%s: %s has width %d, expected %lld", who, name, t->width,
                (long long)width);
  // the kernels address a 32-point tile with 32-bit byte offsets from the
  // tile's first row (fs_io.h)
  const int64_t esz = t->dtype == fs::DT_F32 ? 4 : 2;
  if (t->stride_b < 0 || t->stride_n < 0 || t->stride_h < 0)
    return fail(FS_ERR_INVALID, "%s: %s has a negative stride", who, name);
  if (t->stride_n * esz * fs::kTile >= (int64_t(1) << 30) ||
      (int64_t)width * esz >= (int64_t(1) << 20))
    return fail(FS_ERR_UNSUPPORTED, "%s: %s row stride %lld elements is too large", who, name,
                (long long)t->stride_n);
  return FS_OK;
}
// Outputs: rows must not overlap (a tile's stores of points >= N then fall
// outside the range the kernels write through).
int32_t check_out_points(const fs_points* t, const char* name, int64_t width, const char* who) {
  const int32_t rc = check_points(t, name, width, who);
  if (rc) return rc;
  if (t->stride_n < width)
    return fail(FS_ERR_INVALID, "%s: %s rows overlap (stride along N %lld < width %lld)", who,
                name, (long long)t->stride_n, (long long)width);
  return FS_OK;
}

// D and DV multiples of 32: every column group of a fragment is in range
bool full_widths(const fs_slice_params* p) { return p->D % 32 == 0 && p->DV % 32 == 0; }

int vec_ok(const fs_points* t) {
  const int64_t esz = t->dtype == fs::DT_F32 ? 4 : 2;
  const uintptr_t addr = (uintptr_t)t->data;
  return (addr % (4 * esz) == 0) && (t->stride_b % 4 == 0) && (t->stride_n % 4 == 0) &&
         (t->stride_h % 4 == 0);
}

// the dot level as the kernels' DK: 0 all fp32, 1 bf16 value dots, 2 all bf16
int mode_of(int dot, int dtype) {
  if (dtype == fs::DT_F32) return 0;
  if (dot == 2) return 1;
  if (dot == 3) return 2;
  return 0;
}

// 1 = whole-G, 2 = G-blocked; the whole-G family only when asked for
// nothing else (family 0 or 1) and the shape fits
int family_of(const fs_slice_params* p) {
  if (p->family == 2) return 2;
  return fs::fused_fits((int)p->D, (int)p->DV, (int)p->G) ? 1 : 2;
}

fs::Args base_args(const fs_slice_params* p, const Geo& g) {
  fs::Args a;
  std::memset(&a, 0, sizeof(a));
  a.W = p->weight;
  a.swb = p->w_stride_b;
  a.swh = p->w_stride_h;
  a.bias = p->bias;
  a.sbb = p->b_stride_b;
  a.sbh = p->b_stride_h;
  a.tau = p->tau;
  a.B = (int)p->B;
  a.N = (int)p->N;
  a.H = (int)p->H;
  a.D = (int)p->D;
  a.DV = (int)p->DV;
  a.G = (int)p->G;
  a.P = g.P;
  a.ntiles = g.ntiles;
  a.nd = (int)((p->D + 31) / 32);
  a.nv = (int)((p->DV + 31) / 32);
  a.rows = p->row_splits;
  a.rows_total = p->row_splits ? p->total_rows : 0;
  return a;
}



// A point tensor's pointer and strides; a ragged batch addresses sample b
// from its first row (row splits), so its stride along b is not used.
void set_in(const fs_slice_params* p, const fs_points* t, const void** d, int64_t* sb,
            int64_t* sn, int64_t* sh) {
  *d = t->data;
  *sb = p->row_splits ? 0 : t->stride_b;
  *sn = t->stride_n;
  *sh = t->stride_h;
}
void set_out(const fs_slice_params* p, const fs_points* t, void** d, int64_t* sb, int64_t* sn,
             int64_t* sh) {
  *d = t->data;
  *sb = p->row_splits ? 0 : t->stride_b;
  *sn = t->stride_n;
  *sh = t->stride_h;
}

int64_t wave_floats(int32_t op, const fs_slice_params* p) {
  const int G = (int)p->G, D = (int)p->D, DV = (int)p->DV;
  switch (op) {
    case FS_OP_SLICE_FWD: return fs::part_floats_slice_fwd(G, DV);
    case FS_OP_SLICE_BWD: return fs::part_floats_slice_bwd(G, D);
    case FS_OP_DESLICE_BWD: return fs::part_floats_deslice_bwd(G, D, DV);
    case FS_OP_TIED_BWD: return fs::part_floats_deslice_bwd(G, D, DV);
    default: return 0;
  }
}

// ------------------------------------------------------------------ workspace
// The workspace of one op, carved in 256-byte aligned pieces.
struct Workspace {
  float* stats = nullptr;  // (B, H, 2, N) when the caller hands none in
  float* delta = nullptr;  // (B, H, N)
  float* lsum = nullptr;   // (B, H, N)
  float* part2 = nullptr;  // (B H, P_n)
  float* part = nullptr;   // (B H, P, wave_floats)
  float* frags = nullptr;  // prepared operand fragments (G-blocked, widths <= 64)
  size_t bytes = 0;
};

// G-blocked calls served by the prepared-fragment kernels
bool gp_on(const fs_slice_params* p) { return fs::gp_serves((int)p->D, (int)p->DV); }

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Rows of one per-point buffer (delta, row sums; the statistics hold two
// such): B * H planes of N points, or for a ragged batch H planes of its
// total_rows rows (fs::rows_of).
int64_t pt_rows(const fs_slice_params* p) {
  return p->row_splits ? p->H * p->total_rows : p->B * p->H * p->N;
}

Workspace plan_ws(int32_t op, const fs_slice_params* p, char* base) {
  Workspace w;
  size_t off = 0;
  auto take = [&](size_t nfloats) -> float* {
    float* ptr = base ? (float*)(base + off) : nullptr;
    off += align256(nfloats * sizeof(float));
    return ptr;
  };
  const int64_t bh = p->B * p->H;
  // the tied backward runs on the whole-G family only (else unsupported)
  if (op == FS_OP_TIED_BWD && family_of(p) != 1) return w;
  // the fragment buffer: sized for the largest (fp32-accurate) fragments,
  // whatever the call's dtype
  const bool blocked = op == FS_OP_STATS || family_of(p) == 2;
  if (blocked && gp_on(p))
    w.frags = take((size_t)fs::gp_layout((int)p->B, (int)p->H, (int)p->G, (int)p->D, (int)p->DV,
                                         0).total_u32x4 * 4);
  if (op == FS_OP_DESLICE_FWD || op == FS_OP_STATS) {
    w.bytes = off;
    return w;
  }
  if (family_of(p) == 1) {
    // whole-G kernels leave one partial per block (its four waves summed)
    const Geo g = geo_n(p, fused_target(op, p));
    w.part = take((size_t)(bh * pb(g) * wave_floats(op, p)));
  } else {
    const Geo gn = geo_gp(p, GPG_BWD_N, 0), gg = geo_g(p, -1);
    w.stats = take((size_t)(pt_rows(p) * 2));
    if (op != FS_OP_SLICE_FWD) {
      w.delta = take((size_t)pt_rows(p));
      w.lsum = take((size_t)pt_rows(p));
      w.part2 = take((size_t)(bh * gn.P));
    }
    w.part = take((size_t)(bh * gg.P * wave_floats(op, p)));
  }
  w.bytes = off;
  return w;
}

int32_t check_ws(size_t need, size_t have, void* ws, const char* who) {
  if (need == 0) return FS_OK;
  if (!ws || have < need)
    return fail(FS_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, need, have);
  return FS_OK;
}

int Bo_of(int64_t stride_b, int64_t B) { return stride_b != 0 ? (int)B : 1; }
int Ho_of(int64_t stride_h, int64_t H) { return stride_h != 0 ? (int)H : 1; }

fs::ReduceSegment seg(const float* part, int64_t wstride, int64_t off, int P, int E, int Bo,
                      int Ho, float* out) {
  fs::ReduceSegment s;
  s.part = part;
  s.wstride = wstride;
  s.off = off;
  s.P = P;
  s.E = E;
  s.Bo = Bo;
  s.Ho = Ho;
  s.out = out;
  return s;
}

// Prepared operand fragments of one G-blocked call (k_gp_prep) into the
// workspace, from a's W, bias, tau and (when set) tokens / dz_num and ds.
int32_t gp_prepare(fs::Args& a, const fs_slice_params* p, const Workspace& ws, int mode,
                   hipStream_t st, const char* who) {
  if (!gp_on(p)) return FS_OK;
  const fs::GpLayout l =
      fs::gp_layout((int)p->B, (int)p->H, (int)p->G, (int)p->D, (int)p->DV, mode);
  a.frags = ws.frags;
  for (int k = 0; k < 6; ++k) a.foff[k] = l.off[k];
  return hip_check(fs::launch_gp_prep(a, mode, st), who);
}

// statistics of the logits into `stats` with the point-owned stats kernel;
// `prepared`: a call's Args whose fragments are already built
int32_t run_stats(const fs_points* x, const fs_slice_params* p, float* stats, int two_pass,
                  const fs::Args& prepared, hipStream_t st, const char* who) {
  const Geo g = geo_gp(p, GPG_STATS, 0);
  fs::Args a = base_args(p, g);
  set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  a.vec_x = vec_ok(x);
  a.fast = a.vec_x && full_widths(p);
  a.stats_out = stats;
  a.two_pass = two_pass;
  a.frags = prepared.frags;
  for (int k = 0; k < 6; ++k) a.foff[k] = prepared.foff[k];
  return hip_check(fs::launch_blocked(fs::BK_STATS, a, x->dtype, mode_of(p->dot, x->dtype), st),
                   who);
}

}  // namespace

extern "C" {

const char* fs_last_error(void) { return g_err.c_str(); }

const char* fs_version(void) { return "flashslice_amd 0.1.0 (gfx950)"; }

int32_t fs_family(const fs_slice_params* p) {
  if (!p) return 0;
  return family_of(p);
}

size_t fs_workspace_bytes(int32_t op, const fs_slice_params* p) {
  if (check_params(p, "fs_workspace_bytes") != FS_OK) return 0;
  return plan_ws(op, p, nullptr).bytes;
}

int32_t fs_compute_stats(const fs_points* x, const fs_slice_params* p, float* stats,
                         int32_t two_pass, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_compute_stats";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (rc) return rc;
  if (!stats) return fail(FS_ERR_INVALID, "%s: stats is NULL", who);
  const Workspace ws = plan_ws(FS_OP_STATS, p, (char*)workspace);
  rc = check_ws(ws.bytes, workspace_bytes, workspace, who);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  fs::Args a = base_args(p, geo_gp(p, GPG_STATS, 0));
  rc = gp_prepare(a, p, ws, mode_of(p->dot, x->dtype), st, who);
  if (rc) return rc;
  return run_stats(x, p, stats, two_pass ? 1 : 0, a, st, who);
}

}  // extern "C"

// Scratch of fs_slice_fwd_static: one copy per GPU the library runs on, held
// until the process ends; every call on a GPU shares it. Nothing in it needs
// to start at zero: the slice forward writes every partial (and statistic)
// it later reads, as with a fresh, uninitialised workspace.
constexpr size_t kScratchBytes = FS_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// The slice forward on a given workspace: fs_slice_fwd (caller's buffer) and
// fs_slice_fwd_static (the library's scratch array) share it.
int32_t slice_fwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                  const float* stats_in, float* stats_out, float* z_num, float* s,
                  void* workspace, size_t workspace_bytes, void* stream, const char* who) {
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(fx, "fx_mid", p->DV, who);
  if (rc) return rc;
  if (fx->dtype != x->dtype) return fail(FS_ERR_INVALID, "%s: x_mid and fx_mid dtypes differ", who);
  if (!z_num || !s) return fail(FS_ERR_INVALID, "%s: z_num and s must be non-NULL", who);
  const Workspace ws = plan_ws(FS_OP_SLICE_FWD, p, (char*)workspace);
  rc = check_ws(ws.bytes, workspace_bytes, workspace, who);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int mode = mode_of(p->dot, x->dtype);
  const int64_t wf = wave_floats(FS_OP_SLICE_FWD, p);
  const int G = (int)p->G, DV = (int)p->DV;
  Geo g;
  if (family_of(p) == 1) {
    // the whole-G kernels form the statistics exactly in their one pass, so
    // handed-in statistics (of these very logits) are not needed
    g = geo_n(p, fused_target(FS_OP_SLICE_FWD, p));
    fs::Args a = base_args(p, g);
    a.rev = sweep_rev(FS_OP_SLICE_FWD);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(fx);
    a.fast = a.vec_x && a.vec_f && full_widths(p);
    a.part = ws.part;
    a.stats_out = stats_out;
    rc = hip_check(fs::launch_fused_slice_fwd(a, x->dtype, mode, st), who);
  } else if (coop_on(p, mode)) {
    // one pass: the statistics from stats_in, or formed in the pass
    g = geo_coop(p, kCoopBlocksFwd);
    fs::Args a = base_args(p, g);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(fx);
    a.fast = a.vec_x && a.vec_f && full_widths(p);
    a.part = ws.part;
    a.stats_in = stats_in;
    a.stats_out = stats_in ? nullptr : stats_out;
    rc = hip_check(fs::launch_coop(fs::CK_SLICE_FWD, a, x->dtype, st), who);
  } else {
    g = geo_g(p, mode);
    fs::Args a = base_args(p, g);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(fx);
    a.fast = a.vec_x && a.vec_f && full_widths(p);
    a.part = ws.part;
    rc = gp_prepare(a, p, ws, mode, st, who);
    if (rc) return rc;
    const float* stats = stats_in;
    if (!stats) {
      float* dst = stats_out ? stats_out : ws.stats;
      rc = run_stats(x, p, dst, 0, a, st, who);
      if (rc) return rc;
      stats = dst;
    }
    a.stats_in = stats;
    rc = hip_check(fs::launch_blocked(fs::BK_SLICE_G, a, x->dtype, mode, st), who);
  }
  if (rc) return rc;
  // partials: one per block (whole-G, cooperative) or per wave (G-blocked)
  const int np = family_of(p) == 1 ? pb(g) : g.P;
  fs::ReduceSegments rs{};
  rs.seg[0] = seg(ws.part, wf, 0, np, G * DV, (int)p->B, (int)p->H, z_num);
  rs.seg[1] = seg(ws.part, wf, (int64_t)G * DV, np, G, (int)p->B, (int)p->H, s);
  rs.n = 2;
  return hip_check(fs::launch_reduce((int)p->B, (int)p->H, rs, st), who);
}

// Device address of `scratch` per device, looked up once per device with
// that device current (hipGetSymbolAddress: in host code the array's name
// is not a device address).
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

int32_t scratch_of_current_device(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FS_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FS_ERR_UNSUPPORTED, "%s: device %d is beyond the %d this library serves", who, dev,
                kMaxDevices);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr)
        return fail(FS_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                    hipGetErrorString(e));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return FS_OK;
}

}  // namespace

extern "C" {

int32_t fs_slice_fwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                     const float* stats_in, float* stats_out, float* z_num, float* s,
                     void* workspace, size_t workspace_bytes, void* stream) {
  return slice_fwd(x, fx, p, stats_in, stats_out, z_num, s, workspace, workspace_bytes, stream,
                   "fs_slice_fwd");
}

int32_t fs_slice_fwd_static(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                            const float* stats_in, float* stats_out, float* z_num, float* s,
                            void* stream) {
  const char* who = "fs_slice_fwd_static";
  int32_t rc = check_params(p, who);
  if (rc) return rc;
  const size_t need = plan_ws(FS_OP_SLICE_FWD, p, nullptr).bytes;
  if (need > kScratchBytes)
    return fail(FS_ERR_WORKSPACE,
                "%s: this shape needs %zu bytes of scratch, the library's static buffer holds "
                "%zu; call fs_slice_fwd with a workspace", who, need, kScratchBytes);
  void* ptr = nullptr;
  if (need > 0) {
    rc = scratch_of_current_device(&ptr, who);
    if (rc) return rc;
  }
  return slice_fwd(x, fx, p, stats_in, stats_out, z_num, s, ptr, kScratchBytes, stream, who);
}

int32_t fs_deslice_fwd(const fs_points* x, const fs_slice_params* p, const float* tokens,
                       const float* stats_in, float* stats_out, const fs_points* out,
                       void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_deslice_fwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_out_points(out, "out", p->DV, who);
  if (rc) return rc;
  if (out->dtype != x->dtype) return fail(FS_ERR_INVALID, "%s: out and x_mid dtypes differ", who);
  if (!tokens) return fail(FS_ERR_INVALID, "%s: tokens is NULL", who);
  const Workspace ws = plan_ws(FS_OP_DESLICE_FWD, p, (char*)workspace);
  rc = check_ws(ws.bytes, workspace_bytes, workspace, who);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int mode = mode_of(p->dot, x->dtype);
  if (family_of(p) == 1) {
    const Geo g = geo_n(p, fused_target(FS_OP_DESLICE_FWD, p));
    fs::Args a = base_args(p, g);
    a.rev = sweep_rev(FS_OP_DESLICE_FWD);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_out(p, out, &a.o1, &a.s1b, &a.s1n, &a.s1h);
    a.vec_x = vec_ok(x);
    a.vec_1 = vec_ok(out);
    a.fast = a.vec_x && a.vec_1 && full_widths(p);
    a.tok = tokens;
    a.stats_out = stats_out;
    return hip_check(fs::launch_fused_deslice_fwd(a, x->dtype, mode, st), who);
  }
  if (coop_on(p, mode)) {
    // one pass: the weights of a tile's 256 slots through LDS, out over all
    // of them on the matrix cores (statistics read or formed in the pass)
    fs::Args a = base_args(p, geo_coop(p, kCoopBlocksFwd));
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_out(p, out, &a.o1, &a.s1b, &a.s1n, &a.s1h);
    a.vec_x = vec_ok(x);
    a.vec_1 = vec_ok(out);
    a.fast = a.vec_x && a.vec_1 && full_widths(p);
    a.tok = tokens;
    a.stats_in = stats_in;
    a.stats_out = stats_in ? nullptr : stats_out;
    return hip_check(fs::launch_coop(fs::CK_DESLICE_FWD, a, x->dtype, st), who);
  }
  const Geo g = geo_gp(p, GPG_DESLICE, mode);
  fs::Args a = base_args(p, g);
  set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  set_out(p, out, &a.o1, &a.s1b, &a.s1n, &a.s1h);
  a.vec_x = vec_ok(x);
  a.vec_1 = vec_ok(out);
  a.fast = a.vec_x && a.vec_1 && full_widths(p);
  a.tok = tokens;
  rc = gp_prepare(a, p, ws, mode, st, who);
  if (rc) return rc;
  if (stats_in) {
    a.stats_in = stats_in;
    return hip_check(fs::launch_blocked(fs::BK_DESLICE_N, a, x->dtype, mode, st), who);
  }
  a.stats_out = stats_out;  // may be NULL: then the statistics are not kept
  return hip_check(fs::launch_blocked(fs::BK_DESLICE_ONLINE, a, x->dtype, mode, st), who);
}

int32_t fs_slice_bwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                     const float* stats_in, const float* dz_num, const float* ds,
                     const fs_points* dx, const fs_points* dfx, float* dweight, float* dbias,
                     float* dtau, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_slice_bwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(fx, "fx_mid", p->DV, who);
  if (!rc) rc = check_out_points(dx, "dx", p->D, who);
  if (!rc) rc = check_out_points(dfx, "dfx", p->DV, who);
  if (rc) return rc;
  if (fx->dtype != x->dtype || dx->dtype != x->dtype || dfx->dtype != x->dtype)
    return fail(FS_ERR_INVALID, "%s: point tensors must share one dtype", who);
  if (!dz_num || !ds || !dweight || !dbias || !dtau)
    return fail(FS_ERR_INVALID, "%s: dz_num, ds, dweight, dbias, dtau must be non-NULL", who);
  const Workspace ws = plan_ws(FS_OP_SLICE_BWD, p, (char*)workspace);
  rc = check_ws(ws.bytes, workspace_bytes, workspace, who);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int mode = mode_of(p->dot, x->dtype);
  const int64_t wf = wave_floats(FS_OP_SLICE_BWD, p);
  const int G = (int)p->G, D = (int)p->D;
  const int Bw = Bo_of(p->w_stride_b, p->B), Hw = Ho_of(p->w_stride_h, p->H);
  const int Bb = Bo_of(p->b_stride_b, p->B), Hb = Ho_of(p->b_stride_h, p->H);
  fs::ReduceSegments rs{};
  if (family_of(p) == 1) {
    const Geo g = geo_n(p, fused_target(FS_OP_SLICE_BWD, p));
    fs::Args a = base_args(p, g);
    a.rev = sweep_rev(FS_OP_SLICE_BWD);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
    set_out(p, dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
    set_out(p, dfx, &a.o2, &a.s2b, &a.s2n, &a.s2h);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(fx);
    a.vec_1 = vec_ok(dx);
    a.vec_2 = vec_ok(dfx);
    a.fast = a.vec_x && a.vec_f && a.vec_1 && a.vec_2 && full_widths(p);
    a.tok = dz_num;
    a.ds = ds;
    a.part = ws.part;
    rc = hip_check(fs::launch_fused_slice_bwd(a, x->dtype, mode, st), who);
    if (rc) return rc;
    rs.seg[0] = seg(ws.part, wf, 0, pb(g), G * D, Bw, Hw, dweight);
    rs.seg[1] = seg(ws.part, wf, (int64_t)G * D, pb(g), G, Bb, Hb, dbias);
    rs.seg[2] = seg(ws.part, wf, (int64_t)G * D + G, pb(g), 1, 1, (int)p->H, dtau);
  } else {
    const Geo gn = geo_gp(p, GPG_BWD_N, mode), gg = geo_g(p, mode);
    fs::Args a = base_args(p, gn);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
    set_out(p, dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
    set_out(p, dfx, &a.o2, &a.s2b, &a.s2n, &a.s2h);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(fx);
    a.vec_1 = vec_ok(dx);
    a.vec_2 = vec_ok(dfx);
    a.fast = a.vec_x && a.vec_f && a.vec_1 && a.vec_2 && full_widths(p);
    a.tok = dz_num;
    a.ds = ds;
    const bool coop = coop_on(p, mode);
    const float* stats = stats_in;
    if (!coop || !stats) {
      rc = gp_prepare(a, p, ws, mode, st, who);
      if (rc) return rc;
    }
    if (!stats) {
      rc = run_stats(x, p, ws.stats, 0, a, st, who);
      if (rc) return rc;
      stats = ws.stats;
    }
    a.stats_in = stats;
    if (coop) {
      // one pass from the statistics: dfx, dx, and dW, db, dtau per block
      const Geo gc = geo_coop(p, kCoopBlocksBwd);
      a.P = gc.P;
      a.part = ws.part;
      rc = hip_check(fs::launch_coop(fs::CK_SLICE_BWD, a, x->dtype, st), who);
      if (rc) return rc;
      rs.seg[0] = seg(ws.part, wf, 0, gc.P, G * D, Bw, Hw, dweight);
      rs.seg[1] = seg(ws.part, wf, (int64_t)G * D, gc.P, G, Bb, Hb, dbias);
      rs.seg[2] = seg(ws.part, wf, (int64_t)G * D + G, gc.P, 1, 1, (int)p->H, dtau);
      rs.n = 3;
      return hip_check(fs::launch_reduce((int)p->B, (int)p->H, rs, st), who);
    }
    a.delta = ws.delta;
    a.lsum = ws.lsum;
    a.part2 = ws.part2;
    rc = hip_check(fs::launch_blocked(fs::BK_SLICE_BWD_N, a, x->dtype, mode, st), who);
    if (rc) return rc;
    a.P = gg.P;
    a.part = ws.part;
    rc = hip_check(fs::launch_blocked(fs::BK_SLICE_BWD_G, a, x->dtype, mode, st), who);
    if (rc) return rc;
    rs.seg[0] = seg(ws.part, wf, 0, gg.P, G * D, Bw, Hw, dweight);
    rs.seg[1] = seg(ws.part, wf, (int64_t)G * D, gg.P, G, Bb, Hb, dbias);
    rs.seg[2] = seg(ws.part2, 1, 0, gn.P, 1, 1, (int)p->H, dtau);
  }
  rs.n = 3;
  return hip_check(fs::launch_reduce((int)p->B, (int)p->H, rs, st), who);
}

int32_t fs_deslice_bwd(const fs_points* x, const fs_slice_params* p, const float* tokens,
                       const float* stats_in, const fs_points* d_out, const fs_points* dx,
                       float* dtokens, float* dweight, float* dbias, float* dtau,
                       void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_deslice_bwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(d_out, "d_out", p->DV, who);
  if (!rc) rc = check_out_points(dx, "dx", p->D, who);
  if (rc) return rc;
  if (d_out->dtype != x->dtype || dx->dtype != x->dtype)
    return fail(FS_ERR_INVALID, "%s: point tensors must share one dtype", who);
  if (!tokens || !dtokens || !dweight || !dbias || !dtau)
    return fail(FS_ERR_INVALID, "%s: tokens, dtokens, dweight, dbias, dtau must be non-NULL",
                who);
  const Workspace ws = plan_ws(FS_OP_DESLICE_BWD, p, (char*)workspace);
  rc = check_ws(ws.bytes, workspace_bytes, workspace, who);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int mode = mode_of(p->dot, x->dtype);
  const int64_t wf = wave_floats(FS_OP_DESLICE_BWD, p);
  const int G = (int)p->G, D = (int)p->D, DV = (int)p->DV;
  const int64_t offW = (int64_t)G * DV, offB = offW + (int64_t)G * D;
  const int Bw = Bo_of(p->w_stride_b, p->B), Hw = Ho_of(p->w_stride_h, p->H);
  const int Bb = Bo_of(p->b_stride_b, p->B), Hb = Ho_of(p->b_stride_h, p->H);
  fs::ReduceSegments rs{};
  if (family_of(p) == 1) {
    const Geo g = geo_n(p, fused_target(FS_OP_DESLICE_BWD, p));
    fs::Args a = base_args(p, g);
    a.rev = sweep_rev(FS_OP_DESLICE_BWD);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, d_out, &a.f, &a.sfb, &a.sfn, &a.sfh);
    set_out(p, dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(d_out);
    a.vec_1 = vec_ok(dx);
    a.fast = a.vec_x && a.vec_f && a.vec_1 && full_widths(p);
    a.tok = tokens;
    a.part = ws.part;
    rc = hip_check(fs::launch_fused_deslice_bwd(a, x->dtype, mode, st), who);
    if (rc) return rc;
    rs.seg[0] = seg(ws.part, wf, 0, pb(g), G * DV, (int)p->B, (int)p->H, dtokens);
    rs.seg[1] = seg(ws.part, wf, offW, pb(g), G * D, Bw, Hw, dweight);
    rs.seg[2] = seg(ws.part, wf, offB, pb(g), G, Bb, Hb, dbias);
    rs.seg[3] = seg(ws.part, wf, offB + G, pb(g), 1, 1, (int)p->H, dtau);
  } else {
    const float* stats = stats_in;
    const Geo gn = geo_gp(p, GPG_BWD_N, mode), gg = geo_g(p, mode);
    fs::Args a = base_args(p, gn);
    set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
    set_in(p, d_out, &a.f, &a.sfb, &a.sfn, &a.sfh);
    set_out(p, dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
    a.vec_x = vec_ok(x);
    a.vec_f = vec_ok(d_out);
    a.vec_1 = vec_ok(dx);
    a.fast = a.vec_x && a.vec_f && a.vec_1 && full_widths(p);
    a.tok = tokens;
    const bool coop = coop_on(p, mode);
    if (!coop || !stats) {
      rc = gp_prepare(a, p, ws, mode, st, who);
      if (rc) return rc;
    }
    if (!stats) {
      rc = run_stats(x, p, ws.stats, 0, a, st, who);
      if (rc) return rc;
      stats = ws.stats;
    }
    a.stats_in = stats;
    if (coop) {
      // one pass from the statistics: dx, and dtokens, dW, db, dtau per block
      const Geo gc = geo_coop(p, kCoopBlocksBwd);
      a.P = gc.P;
      a.part = ws.part;
      rc = hip_check(fs::launch_coop(fs::CK_DESLICE_BWD, a, x->dtype, st), who);
      if (rc) return rc;
      rs.seg[0] = seg(ws.part, wf, 0, gc.P, G * DV, (int)p->B, (int)p->H, dtokens);
      rs.seg[1] = seg(ws.part, wf, offW, gc.P, G * D, Bw, Hw, dweight);
      rs.seg[2] = seg(ws.part, wf, offB, gc.P, G, Bb, Hb, dbias);
      rs.seg[3] = seg(ws.part, wf, offB + G, gc.P, 1, 1, (int)p->H, dtau);
      rs.n = 4;
      return hip_check(fs::launch_reduce((int)p->B, (int)p->H, rs, st), who);
    }
    a.delta = ws.delta;
    a.lsum = ws.lsum;
    a.part2 = ws.part2;
    rc = hip_check(fs::launch_blocked(fs::BK_DESLICE_BWD_N, a, x->dtype, mode, st), who);
    if (rc) return rc;
    a.P = gg.P;
    a.part = ws.part;
    rc = hip_check(fs::launch_blocked(fs::BK_DESLICE_BWD_G, a, x->dtype, mode, st), who);
    if (rc) return rc;
    rs.seg[0] = seg(ws.part, wf, 0, gg.P, G * DV, (int)p->B, (int)p->H, dtokens);
    rs.seg[1] = seg(ws.part, wf, offW, gg.P, G * D, Bw, Hw, dweight);
    rs.seg[2] = seg(ws.part, wf, offB, gg.P, G, Bb, Hb, dbias);
    rs.seg[3] = seg(ws.part2, 1, 0, gn.P, 1, 1, (int)p->H, dtau);
  }
  rs.n = 4;
  return hip_check(fs::launch_reduce((int)p->B, (int)p->H, rs, st), who);
}

int32_t fs_tied_bwd(const fs_points* x, const fs_points* fx, const fs_points* d_out,
                    const fs_slice_params* p, const float* tokens, const float* dz_num,
                    const float* ds, const fs_points* dx, const fs_points* dfx,
                    float* dtokens, float* dweight, float* dbias, float* dtau,
                    void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_tied_bwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(fx, "fx_mid", p->DV, who);
  if (!rc) rc = check_points(d_out, "d_out", p->DV, who);
  if (!rc) rc = check_out_points(dx, "dx", p->D, who);
  // dfx may be NULL (or have a NULL data pointer): not written
  const bool want_dfx = dfx && dfx->data;
  if (!rc && want_dfx) rc = check_out_points(dfx, "dfx", p->DV, who);
  if (rc) return rc;
  if (fx->dtype != x->dtype || d_out->dtype != x->dtype || dx->dtype != x->dtype ||
      (want_dfx && dfx->dtype != x->dtype))
    return fail(FS_ERR_INVALID, "%s: point tensors must share one dtype", who);
  if (!tokens || !dz_num || !ds || !dweight || !dbias || !dtau)
    return fail(FS_ERR_INVALID,
                "%s: tokens, dz_num, ds, dweight, dbias, dtau must be non-NULL", who);
  if (family_of(p) != 1)
    return fail(FS_ERR_UNSUPPORTED,
                "%s: served by the whole-G kernels only (G <= 128 and D, DV small enough); "
                "run fs_deslice_bwd and fs_slice_bwd", who);
  const Workspace ws = plan_ws(FS_OP_TIED_BWD, p, (char*)workspace);
  rc = check_ws(ws.bytes, workspace_bytes, workspace, who);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int mode = mode_of(p->dot, x->dtype);
  const int64_t wf = wave_floats(FS_OP_TIED_BWD, p);
  const int G = (int)p->G, D = (int)p->D, DV = (int)p->DV;
  const int64_t offW = (int64_t)G * DV, offB = offW + (int64_t)G * D;
  const int Bw = Bo_of(p->w_stride_b, p->B), Hw = Ho_of(p->w_stride_h, p->H);
  const int Bb = Bo_of(p->b_stride_b, p->B), Hb = Ho_of(p->b_stride_h, p->H);
  const Geo g = geo_n(p, fused_target(FS_OP_TIED_BWD, p));
  fs::Args a = base_args(p, g);
  a.rev = sweep_rev(FS_OP_TIED_BWD);
  set_in(p, x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  set_in(p, fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
  set_in(p, d_out, &a.g, &a.sgb, &a.sgn, &a.sgh);
  set_out(p, dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
  if (want_dfx) set_out(p, dfx, &a.o2, &a.s2b, &a.s2n, &a.s2h);
  a.vec_x = vec_ok(x);
  a.vec_f = vec_ok(fx) && vec_ok(d_out);
  a.vec_1 = vec_ok(dx);
  a.vec_2 = want_dfx ? vec_ok(dfx) : 1;
  a.fast = a.vec_x && a.vec_f && a.vec_1 && a.vec_2 && full_widths(p);
  a.tok = dz_num;
  a.tok2 = tokens;
  a.ds = ds;
  a.part = ws.part;
  a.no_dtok = dtokens == nullptr;
  rc = hip_check(fs::launch_fused_tied_bwd(a, x->dtype, mode, st), who);
  if (rc) return rc;
  fs::ReduceSegments rs{};
  rs.n = 0;
  // dtokens may be NULL: not reduced
  if (dtokens) rs.seg[rs.n++] = seg(ws.part, wf, 0, pb(g), G * DV, (int)p->B, (int)p->H, dtokens);
  rs.seg[rs.n++] = seg(ws.part, wf, offW, pb(g), G * D, Bw, Hw, dweight);
  rs.seg[rs.n++] = seg(ws.part, wf, offB, pb(g), G, Bb, Hb, dbias);
  rs.seg[rs.n++] = seg(ws.part, wf, offB + G, pb(g), 1, 1, (int)p->H, dtau);
  return hip_check(fs::launch_reduce((int)p->B, (int)p->H, rs, st), who);
}

// ------------------------------------------------------------- LayerNorm
// The layer's normalisation of (rows, cols) fp32 rows (fs_layernorm.hip).
static int32_t ln_check(const char* who, int64_t rows, int32_t cols,
                        std::initializer_list<const void*> ptrs) {
  if (rows < 1) return fail(FS_ERR_INVALID, "%s: rows must be >= 1 (got %lld)", who, (long long)rows);
  if (cols < 4 || cols > 2048 || cols % 4)
    return fail(FS_ERR_INVALID, "%s: cols must be a multiple of 4 in [4, 2048] (got %d)", who,
                (int)cols);
  for (const void* q : ptrs) {
    if (!q) return fail(FS_ERR_INVALID, "%s: a tensor pointer is NULL", who);
    if (reinterpret_cast<uintptr_t>(q) % 16)
      return fail(FS_ERR_INVALID, "%s: tensors must be 16-byte aligned", who);
  }
  return FS_OK;
}

size_t fs_layernorm_workspace_bytes(int64_t rows, int32_t cols) {
  if (rows < 1 || cols < 4 || cols > 2048 || cols % 4) return 0;
  return (size_t)fs::ln_blocks(rows) * 2 * (size_t)cols * sizeof(float);
}

int32_t fs_layernorm_fwd(const float* x, const float* gamma, const float* beta, float* y,
                         float* mean, float* rstd, int64_t rows, int32_t cols, float eps,
                         void* stream) {
  const char* who = "fs_layernorm_fwd";
  int32_t rc = ln_check(who, rows, cols, {x, gamma, beta, y});
  if (rc) return rc;
  if (!mean || !rstd) return fail(FS_ERR_INVALID, "%s: mean / rstd is NULL", who);
  return hip_check(fs::ln_fwd_launch(x, gamma, beta, y, mean, rstd, rows, cols, eps,
                                     (hipStream_t)stream), who);
}

int32_t fs_layernorm_bwd(const float* dy, const float* x, const float* gamma, const float* mean,
                         const float* rstd, float* dx, float* dgamma, float* dbeta,
                         void* workspace, size_t workspace_bytes, int64_t rows, int32_t cols,
                         void* stream) {
  const char* who = "fs_layernorm_bwd";
  int32_t rc = ln_check(who, rows, cols, {dy, x, gamma, dx, workspace});
  if (rc) return rc;
  if (!mean || !rstd || !dgamma || !dbeta)
    return fail(FS_ERR_INVALID, "%s: mean / rstd / dgamma / dbeta is NULL", who);
  if (workspace_bytes < fs_layernorm_workspace_bytes(rows, cols))
    return fail(FS_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", who, workspace_bytes,
                fs_layernorm_workspace_bytes(rows, cols));
  return hip_check(fs::ln_bwd_launch(dy, x, gamma, mean, rstd, dx, dgamma, dbeta,
                                     static_cast<float*>(workspace), rows, cols,
                                     (hipStream_t)stream), who);
}

}  // extern "C"
