// C-ABI of the FlashSlice HIP kernels (declared in include/flashslice_hip.h).
//
// Validates every argument before any launch, picks the kernel family,
// derives the launch geometry from the shape alone (never from the device,
// so the per-wave partial layout -- and therefore every sum's order -- is
// the same on every run and every GPU), launches the point-streaming
// kernel and then the fixed-order reductions of its partials.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
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

// Blocks of the point-streaming grid: kTargetBlocks in total (two 4-wave
// blocks per CU on a 256-CU MI355X), split over ceil(B*H / 4) block rows.
constexpr int kTargetBlocks = 512;

struct Geo {
  int ntiles, P;
};

Geo geometry(const fs_slice_params* p) {
  Geo g;
  g.ntiles = (int)((p->N + fs::kTile - 1) / fs::kTile);
  const int64_t rows = (p->B * p->H + fs::kWavesPerBlock - 1) / fs::kWavesPerBlock;
  int64_t P = (kTargetBlocks + rows - 1) / rows;
  if (P > g.ntiles) P = g.ntiles;
  if (P < 1) P = 1;
  g.P = (int)P;
  return g;
}

int32_t check_params(const fs_slice_params* p, const char* who) {
  if (!p) return fail(FS_ERR_INVALID, "%s: params is NULL", who);
  if (p->B < 1 || p->N < 1 || p->H < 1)
    return fail(FS_ERR_INVALID, "%s: B, N, H must be >= 1 (got %lld, %lld, %lld)", who,
                (long long)p->B, (long long)p->N, (long long)p->H);
  if (p->D < 1 || p->D > 256 || p->DV < 1 || p->DV > 256)
    return fail(FS_ERR_INVALID, "%s: D and DV must be in [1, 256] (got %lld, %lld)", who,
                (long long)p->D, (long long)p->DV);
  if (p->G < 1) return fail(FS_ERR_INVALID, "%s: G must be >= 1 (got %lld)", who, (long long)p->G);
  if (p->N > (int64_t)0x7fffffff - 64)
    return fail(FS_ERR_INVALID, "%s: N = %lld exceeds 2^31 - 64", who, (long long)p->N);
  if (!p->weight || !p->bias || !p->tau)
    return fail(FS_ERR_INVALID, "%s: weight, bias and tau must be non-NULL", who);
  if (p->dot < 0 || p->dot > 4)
    return fail(FS_ERR_INVALID, "%s: dot level %d is not in [0, 4]", who, p->dot);
  return FS_OK;
}

int32_t check_points(const fs_points* t, const char* name, int64_t width, const char* who) {
  if (!t || !t->data) return fail(FS_ERR_INVALID, "%s: %s is NULL", who, name);
  if (t->dtype < 0 || t->dtype > 2)
    return fail(FS_ERR_INVALID, "%s: %s has unknown dtype %d", who, name, t->dtype);
  if (t->width != width)
    return fail(FS_ERR_INVALID, "%s: %s has width %d, expected %lld", who, name, t->width,
                (long long)width);
  return FS_OK;
}

int vec_ok(const fs_points* t) {
  const int64_t esz = t->dtype == fs::DT_F32 ? 4 : 2;
  const uintptr_t addr = (uintptr_t)t->data;
  return (addr % (4 * esz) == 0) && (t->stride_b % 4 == 0) && (t->stride_n % 4 == 0) &&
         (t->stride_h % 4 == 0);
}

// the dot level as the fused kernels' DK: 0 all fp32, 1 bf16 value dots, 2 all bf16
int mode_of(int dot, int dtype) {
  if (dtype == fs::DT_F32) return 0;
  if (dot == 2) return 1;
  if (dot == 3) return 2;
  return 0;
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
  return a;
}

void set_in(const fs_points* t, const void** d, int64_t* sb, int64_t* sn, int64_t* sh) {
  *d = t->data;
  *sb = t->stride_b;
  *sn = t->stride_n;
  *sh = t->stride_h;
}
void set_out(const fs_points* t, void** d, int64_t* sb, int64_t* sn, int64_t* sh) {
  *d = t->data;
  *sb = t->stride_b;
  *sn = t->stride_n;
  *sh = t->stride_h;
}

int64_t wave_floats(int32_t op, const fs_slice_params* p) {
  const int G = (int)p->G, D = (int)p->D, DV = (int)p->DV;
  switch (op) {
    case FS_OP_SLICE_FWD: return fs::part_floats_slice_fwd(G, DV);
    case FS_OP_SLICE_BWD: return fs::part_floats_slice_bwd(G, D);
    case FS_OP_DESLICE_BWD: return fs::part_floats_deslice_bwd(G, D, DV);
    default: return 0;
  }
}

size_t fused_ws(int32_t op, const fs_slice_params* p) {
  const Geo g = geometry(p);
  return (size_t)(p->B * p->H * g.P * wave_floats(op, p)) * sizeof(float);
}

int32_t check_ws(size_t need, size_t have, void* ws, const char* who) {
  if (need == 0) return FS_OK;
  if (!ws || have < need)
    return fail(FS_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, need, have);
  return FS_OK;
}

bool fused_family(const fs_slice_params* p) { return fs::fused_fits((int)p->D, (int)p->DV, (int)p->G); }

int32_t unsupported_blocked(const char* who, const fs_slice_params* p) {
  return fail(FS_ERR_UNSUPPORTED,
              "%s: D=%lld DV=%lld G=%lld needs the G-blocked kernels, not in this build", who,
              (long long)p->D, (long long)p->DV, (long long)p->G);
}

int Bo_of(int64_t stride_b, int64_t B) { return stride_b != 0 ? (int)B : 1; }
int Ho_of(int64_t stride_h, int64_t H) { return stride_h != 0 ? (int)H : 1; }

}  // namespace

extern "C" {

const char* fs_last_error(void) { return g_err.c_str(); }

const char* fs_version(void) { return "flashslice_amd 0.1.0 (gfx950)"; }

int32_t fs_family(const fs_slice_params* p) {
  if (!p) return 0;
  return fused_family(p) ? 1 : 2;
}

size_t fs_workspace_bytes(int32_t op, const fs_slice_params* p) {
  if (check_params(p, "fs_workspace_bytes") != FS_OK) return 0;
  if (op == FS_OP_DESLICE_FWD || op == FS_OP_STATS) return 0;
  return fused_ws(op, p);
}

int32_t fs_compute_stats(const fs_points* x, const fs_slice_params* p, float* stats,
                         int32_t two_pass, void* workspace, size_t workspace_bytes, void* stream) {
  (void)x; (void)stats; (void)two_pass; (void)workspace; (void)workspace_bytes; (void)stream;
  int32_t rc = check_params(p, "fs_compute_stats");
  if (rc) return rc;
  return unsupported_blocked("fs_compute_stats", p);
}

int32_t fs_slice_fwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                     const float* stats_in, float* stats_out, float* z_num, float* s,
                     void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_slice_fwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(fx, "fx_mid", p->DV, who);
  if (rc) return rc;
  if (fx->dtype != x->dtype) return fail(FS_ERR_INVALID, "%s: x_mid and fx_mid dtypes differ", who);
  if (!z_num || !s) return fail(FS_ERR_INVALID, "%s: z_num and s must be non-NULL", who);
  // the whole-G kernels recompute the statistics exactly in their one pass,
  // so handed-in statistics (of these very logits) are not needed there
  (void)stats_in;
  if (!fused_family(p)) return unsupported_blocked(who, p);
  rc = check_ws(fused_ws(FS_OP_SLICE_FWD, p), workspace_bytes, workspace, who);
  if (rc) return rc;
  const Geo g = geometry(p);
  fs::Args a = base_args(p, g);
  set_in(x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  set_in(fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
  a.vec_x = vec_ok(x);
  a.vec_f = vec_ok(fx);
  a.part = (float*)workspace;
  a.stats_out = stats_out;
  hipStream_t st = (hipStream_t)stream;
  rc = hip_check(fs::launch_fused_slice_fwd(a, x->dtype, mode_of(p->dot, x->dtype), st), who);
  if (rc) return rc;
  const int G = a.G, DV = a.DV;
  fs::ReduceSegments rs{};
  rs.seg[0] = {z_num, 0, G * DV, a.B, a.H, 1.f};
  rs.seg[1] = {s, (int64_t)G * DV, G, a.B, a.H, 1.f};
  rs.n = 2;
  return hip_check(
      fs::launch_reduce(a.part, wave_floats(FS_OP_SLICE_FWD, p), a.B, a.H, a.P, rs, st), who);
}

int32_t fs_deslice_fwd(const fs_points* x, const fs_slice_params* p, const float* tokens,
                       const float* stats_in, float* stats_out, const fs_points* out,
                       void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace; (void)workspace_bytes;
  const char* who = "fs_deslice_fwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(out, "out", p->DV, who);
  if (rc) return rc;
  if (out->dtype != x->dtype) return fail(FS_ERR_INVALID, "%s: out and x_mid dtypes differ", who);
  if (!tokens) return fail(FS_ERR_INVALID, "%s: tokens is NULL", who);
  (void)stats_in;
  if (!fused_family(p)) return unsupported_blocked(who, p);
  const Geo g = geometry(p);
  fs::Args a = base_args(p, g);
  set_in(x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  set_out(out, &a.o1, &a.s1b, &a.s1n, &a.s1h);
  a.stats_out = stats_out;
  a.vec_x = vec_ok(x);
  a.vec_1 = vec_ok(out);
  a.tok = tokens;
  return hip_check(
      fs::launch_fused_deslice_fwd(a, x->dtype, mode_of(p->dot, x->dtype), (hipStream_t)stream),
      who);
}

int32_t fs_slice_bwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                     const float* stats_in, const float* dz_num, const float* ds,
                     const fs_points* dx, const fs_points* dfx, float* dweight, float* dbias,
                     float* dtau, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_slice_bwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(fx, "fx_mid", p->DV, who);
  if (!rc) rc = check_points(dx, "dx", p->D, who);
  if (!rc) rc = check_points(dfx, "dfx", p->DV, who);
  if (rc) return rc;
  if (fx->dtype != x->dtype || dx->dtype != x->dtype || dfx->dtype != x->dtype)
    return fail(FS_ERR_INVALID, "%s: point tensors must share one dtype", who);
  if (!dz_num || !ds || !dweight || !dbias || !dtau)
    return fail(FS_ERR_INVALID, "%s: dz_num, ds, dweight, dbias, dtau must be non-NULL", who);
  (void)stats_in;
  if (!fused_family(p)) return unsupported_blocked(who, p);
  rc = check_ws(fused_ws(FS_OP_SLICE_BWD, p), workspace_bytes, workspace, who);
  if (rc) return rc;
  const Geo g = geometry(p);
  fs::Args a = base_args(p, g);
  set_in(x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  set_in(fx, &a.f, &a.sfb, &a.sfn, &a.sfh);
  set_out(dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
  set_out(dfx, &a.o2, &a.s2b, &a.s2n, &a.s2h);
  a.vec_x = vec_ok(x);
  a.vec_f = vec_ok(fx);
  a.vec_1 = vec_ok(dx);
  a.vec_2 = vec_ok(dfx);
  a.tok = dz_num;
  a.ds = ds;
  a.part = (float*)workspace;
  hipStream_t st = (hipStream_t)stream;
  rc = hip_check(fs::launch_fused_slice_bwd(a, x->dtype, mode_of(p->dot, x->dtype), st), who);
  if (rc) return rc;
  const int G = a.G, D = a.D;
  fs::ReduceSegments rs{};
  rs.seg[0] = {dweight, 0, G * D, Bo_of(p->w_stride_b, p->B), Ho_of(p->w_stride_h, p->H), 1.f};
  rs.seg[1] = {dbias, (int64_t)G * D, G, Bo_of(p->b_stride_b, p->B), Ho_of(p->b_stride_h, p->H),
               1.f};
  rs.seg[2] = {dtau, (int64_t)G * D + G, 1, 1, a.H, 1.f};
  rs.n = 3;
  return hip_check(
      fs::launch_reduce(a.part, wave_floats(FS_OP_SLICE_BWD, p), a.B, a.H, a.P, rs, st), who);
}

int32_t fs_deslice_bwd(const fs_points* x, const fs_slice_params* p, const float* tokens,
                       const float* stats_in, const fs_points* d_out, const fs_points* dx,
                       float* dtokens, float* dweight, float* dbias, float* dtau,
                       void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "fs_deslice_bwd";
  int32_t rc = check_params(p, who);
  if (!rc) rc = check_points(x, "x_mid", p->D, who);
  if (!rc) rc = check_points(d_out, "d_out", p->DV, who);
  if (!rc) rc = check_points(dx, "dx", p->D, who);
  if (rc) return rc;
  if (d_out->dtype != x->dtype || dx->dtype != x->dtype)
    return fail(FS_ERR_INVALID, "%s: point tensors must share one dtype", who);
  if (!tokens || !dtokens || !dweight || !dbias || !dtau)
    return fail(FS_ERR_INVALID, "%s: tokens, dtokens, dweight, dbias, dtau must be non-NULL",
                who);
  (void)stats_in;
  if (!fused_family(p)) return unsupported_blocked(who, p);
  rc = check_ws(fused_ws(FS_OP_DESLICE_BWD, p), workspace_bytes, workspace, who);
  if (rc) return rc;
  const Geo g = geometry(p);
  fs::Args a = base_args(p, g);
  set_in(x, &a.x, &a.sxb, &a.sxn, &a.sxh);
  set_in(d_out, &a.f, &a.sfb, &a.sfn, &a.sfh);
  set_out(dx, &a.o1, &a.s1b, &a.s1n, &a.s1h);
  a.vec_x = vec_ok(x);
  a.vec_f = vec_ok(d_out);
  a.vec_1 = vec_ok(dx);
  a.tok = tokens;
  a.part = (float*)workspace;
  hipStream_t st = (hipStream_t)stream;
  rc = hip_check(fs::launch_fused_deslice_bwd(a, x->dtype, mode_of(p->dot, x->dtype), st), who);
  if (rc) return rc;
  const int G = a.G, D = a.D, DV = a.DV;
  const int64_t offW = (int64_t)G * DV, offB = offW + (int64_t)G * D;
  fs::ReduceSegments rs{};
  rs.seg[0] = {dtokens, 0, G * DV, a.B, a.H, 1.f};
  rs.seg[1] = {dweight, offW, G * D, Bo_of(p->w_stride_b, p->B), Ho_of(p->w_stride_h, p->H), 1.f};
  rs.seg[2] = {dbias, offB, G, Bo_of(p->b_stride_b, p->B), Ho_of(p->b_stride_h, p->H), 1.f};
  rs.seg[3] = {dtau, offB + G, 1, 1, a.H, 1.f};
  rs.n = 4;
  return hip_check(
      fs::launch_reduce(a.part, wave_floats(FS_OP_DESLICE_BWD, p), a.B, a.H, a.P, rs, st), who);
}

}  // extern "C"
