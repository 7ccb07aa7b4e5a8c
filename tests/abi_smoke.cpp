// Torch-free check of the C ABI (include/flashslice_hip.h): what a C or C++
// caller of the library does, with nothing but the HIP runtime. A
// slice -> deslice coupling runs forward through fs_slice_fwd and
// fs_deslice_fwd and the slice backward through fs_slice_bwd, on hipMalloc'd
// buffers and workspaces sized by fs_workspace_bytes, on a stream of its own;
// every output is compared with double-precision loops over the same inputs
// (the softmax over slots of (x . W + b) / tau per point and head, its sums
// over points, and the softmax Jacobian for the backward). Prints one line
// per output with its relative error and exits 0 when all are below 1e-5
// (1 on a mismatch, 2 on a library or HIP error).
//
// Built by flashslice_amd/build.py into tests/_bin/fs_abi_smoke (host code
// only, linked against libflashslice_hip.so); run by tests/test_abi_gpu.py.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../include/flashslice_hip.h"

namespace {

constexpr int B = 2, N = 300, H = 3, D = 32, DV = 32, G = 32;

#define CHECK_HIP(e)                                                              \
  do {                                                                            \
    hipError_t err_ = (e);                                                        \
    if (err_ != hipSuccess) {                                                     \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(err_), __LINE__); \
      std::exit(2);                                                               \
    }                                                                             \
  } while (0)
#define CHECK_FS(e)                                                              \
  do {                                                                           \
    int32_t rc_ = (e);                                                           \
    if (rc_ != FS_OK) {                                                          \
      std::printf("library error %d: %s (line %d)\n", rc_, fs_last_error(), __LINE__); \
      std::exit(2);                                                              \
    }                                                                            \
  } while (0)

uint64_t g_state = 0x9E3779B97F4A7C15ull;
float uniform() {  // xorshift64*, in [-1, 1)
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  const uint64_t r = g_state * 0x2545F4914F6CDD1Dull;
  return (float)((double)(r >> 11) / 9007199254740992.0 * 2.0 - 1.0);
}

float* to_device(const std::vector<float>& h) {
  float* d = nullptr;
  CHECK_HIP(hipMalloc(&d, h.size() * sizeof(float)));
  CHECK_HIP(hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
  return d;
}
std::vector<float> to_host(const float* d, size_t n) {
  std::vector<float> h(n);
  CHECK_HIP(hipMemcpy(h.data(), d, n * sizeof(float), hipMemcpyDeviceToHost));
  return h;
}
void* workspace(int32_t op, const fs_slice_params* p, size_t* bytes) {
  *bytes = fs_workspace_bytes(op, p);
  void* w = nullptr;
  if (*bytes) CHECK_HIP(hipMalloc(&w, *bytes));
  return w;
}
fs_points points(float* data, int width) {
  fs_points t;
  t.data = data;
  t.stride_b = (int64_t)N * H * width;
  t.stride_n = (int64_t)H * width;
  t.stride_h = width;
  t.dtype = FS_F32;
  t.width = width;
  return t;
}
double relerr(const std::vector<float>& a, const std::vector<double>& r) {
  double num = 0, den = 0;
  for (size_t i = 0; i < r.size(); ++i) {
    num += (a[i] - r[i]) * (a[i] - r[i]);
    den += r[i] * r[i];
  }
  return std::sqrt(num / (den > 0 ? den : 1));
}

}  // namespace

int main() {
  const size_t nx = (size_t)B * N * H * D, nf = (size_t)B * N * H * DV;
  std::vector<float> x(nx), fx(nf), W((size_t)H * G * D), bias((size_t)H * G), tau(H);
  std::vector<float> dz((size_t)B * H * G * DV), ds((size_t)B * H * G);
  for (auto& v : x) v = 1.7f * uniform();
  for (auto& v : fx) v = 1.7f * uniform();
  for (auto& v : W) v = 0.3f * uniform();
  for (auto& v : bias) v = 0.1f * uniform();
  for (int h = 0; h < H; ++h) tau[h] = 0.65f + 0.35f * uniform();
  for (auto& v : dz) v = uniform();
  for (auto& v : ds) v = uniform();

  // ---- the reference in double precision
  auto X = [&](int b, int n, int h, int d) { return (double)x[(((size_t)b * N + n) * H + h) * D + d]; };
  auto F = [&](int b, int n, int h, int v) { return (double)fx[(((size_t)b * N + n) * H + h) * DV + v]; };
  std::vector<double> L((size_t)B * N * H * G), w(L.size());
  for (int b = 0; b < B; ++b)
    for (int n = 0; n < N; ++n)
      for (int h = 0; h < H; ++h) {
        double mx = -1e300;
        for (int g = 0; g < G; ++g) {
          double a = bias[h * G + g];
          for (int d = 0; d < D; ++d) a += X(b, n, h, d) * W[((size_t)h * G + g) * D + d];
          const double l = a / tau[h];
          L[(((size_t)b * N + n) * H + h) * G + g] = l;
          mx = l > mx ? l : mx;
        }
        double sum = 0;
        for (int g = 0; g < G; ++g) sum += std::exp(L[(((size_t)b * N + n) * H + h) * G + g] - mx);
        for (int g = 0; g < G; ++g) {
          const size_t i = (((size_t)b * N + n) * H + h) * G + g;
          w[i] = std::exp(L[i] - mx) / sum;
        }
      }
  auto Wt = [&](int b, int n, int h, int g) { return w[(((size_t)b * N + n) * H + h) * G + g]; };
  std::vector<double> z((size_t)B * H * G * DV, 0.0), s((size_t)B * H * G, 0.0);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h)
      for (int g = 0; g < G; ++g)
        for (int n = 0; n < N; ++n) {
          s[((size_t)b * H + h) * G + g] += Wt(b, n, h, g);
          for (int v = 0; v < DV; ++v) z[(((size_t)b * H + h) * G + g) * DV + v] += Wt(b, n, h, g) * F(b, n, h, v);
        }
  std::vector<float> tok(z.size());
  for (size_t i = 0; i < z.size(); ++i) tok[i] = (float)(z[i] / (s[i / DV] + 1e-5));
  std::vector<double> out(nf, 0.0), dfx(nf, 0.0), dx(nx, 0.0), dW(W.size(), 0.0), db(bias.size(), 0.0),
      dtau(H, 0.0);
  for (int b = 0; b < B; ++b)
    for (int n = 0; n < N; ++n)
      for (int h = 0; h < H; ++h) {
        double om[G], delta = 0;
        for (int g = 0; g < G; ++g) {
          const double wg = Wt(b, n, h, g);
          double o = ds[((size_t)b * H + h) * G + g];
          for (int v = 0; v < DV; ++v) {
            const size_t iv = (((size_t)b * H + h) * G + g) * DV + v;
            out[(((size_t)b * N + n) * H + h) * DV + v] += wg * tok[iv];
            dfx[(((size_t)b * N + n) * H + h) * DV + v] += wg * dz[iv];
            o += F(b, n, h, v) * dz[iv];
          }
          om[g] = o;
          delta += wg * o;
        }
        for (int g = 0; g < G; ++g) {
          const double lb = Wt(b, n, h, g) * (om[g] - delta) / tau[h];  // d loss / d (x . W + b)
          db[h * G + g] += lb;
          dtau[h] -= lb * L[(((size_t)b * N + n) * H + h) * G + g];
          for (int d = 0; d < D; ++d) {
            dx[(((size_t)b * N + n) * H + h) * D + d] += lb * W[((size_t)h * G + g) * D + d];
            dW[((size_t)h * G + g) * D + d] += lb * X(b, n, h, d);
          }
        }
      }

  // ---- the library, on a stream of its own
  hipStream_t st;
  CHECK_HIP(hipStreamCreate(&st));
  float *dx_in = to_device(x), *dfx_in = to_device(fx), *dW_in = to_device(W), *db_in = to_device(bias),
        *dtau_in = to_device(tau), *dtok = to_device(tok), *ddz = to_device(dz), *dds = to_device(ds);
  float *d_z, *d_s, *d_out, *d_dx, *d_dfx, *d_dW, *d_db, *d_dtau;
  CHECK_HIP(hipMalloc(&d_z, z.size() * 4));
  CHECK_HIP(hipMalloc(&d_s, s.size() * 4));
  CHECK_HIP(hipMalloc(&d_out, nf * 4));
  CHECK_HIP(hipMalloc(&d_dx, nx * 4));
  CHECK_HIP(hipMalloc(&d_dfx, nf * 4));
  CHECK_HIP(hipMalloc(&d_dW, W.size() * 4));
  CHECK_HIP(hipMalloc(&d_db, bias.size() * 4));
  CHECK_HIP(hipMalloc(&d_dtau, H * 4));
  fs_slice_params p = {};
  p.B = B; p.N = N; p.H = H; p.D = D; p.DV = DV; p.G = G;
  p.weight = dW_in; p.w_stride_b = 0; p.w_stride_h = (int64_t)G * D;
  p.bias = db_in; p.b_stride_b = 0; p.b_stride_h = G;
  p.tau = dtau_in; p.dot = 0; p.family = 0; p.row_splits = nullptr;
  const fs_points px = points(dx_in, D), pf = points(dfx_in, DV), po = points(d_out, DV),
                   pdx = points(d_dx, D), pdf = points(d_dfx, DV);
  size_t n1, n2, n3;
  void* w1 = workspace(FS_OP_SLICE_FWD, &p, &n1);
  void* w2 = workspace(FS_OP_DESLICE_FWD, &p, &n2);
  void* w3 = workspace(FS_OP_SLICE_BWD, &p, &n3);
  std::printf("family %d, workspace bytes %zu %zu %zu\n", fs_family(&p), n1, n2, n3);
  CHECK_FS(fs_slice_fwd(&px, &pf, &p, nullptr, nullptr, d_z, d_s, w1, n1, st));
  CHECK_FS(fs_deslice_fwd(&px, &p, dtok, nullptr, nullptr, &po, w2, n2, st));
  CHECK_FS(fs_slice_bwd(&px, &pf, &p, nullptr, ddz, dds, &pdx, &pdf, d_dW, d_db, d_dtau, w3, n3, st));
  CHECK_HIP(hipStreamSynchronize(st));

  struct Row { const char* name; double err; };
  const Row rows[] = {
      {"z_num", relerr(to_host(d_z, z.size()), z)},   {"s", relerr(to_host(d_s, s.size()), s)},
      {"out", relerr(to_host(d_out, nf), out)},       {"dx", relerr(to_host(d_dx, nx), dx)},
      {"dfx", relerr(to_host(d_dfx, nf), dfx)},       {"dW", relerr(to_host(d_dW, W.size()), dW)},
      {"db", relerr(to_host(d_db, bias.size()), db)}, {"dtau", relerr(to_host(d_dtau, H), dtau)},
  };
  bool ok = true;
  for (const Row& r : rows) {
    std::printf("%-6s relerr %.3e\n", r.name, r.err);
    ok = ok && r.err < 1e-5;
  }
  for (void* q : {(void*)dx_in, (void*)dfx_in, (void*)dW_in, (void*)db_in, (void*)dtau_in, (void*)dtok,
                  (void*)ddz, (void*)dds, (void*)d_z, (void*)d_s, (void*)d_out, (void*)d_dx, (void*)d_dfx,
                  (void*)d_dW, (void*)d_db, (void*)d_dtau, w1, w2, w3})
    if (q) CHECK_HIP(hipFree(q));
  CHECK_HIP(hipStreamDestroy(st));
  std::printf(ok ? "OK\n" : "MISMATCH\n");
  return ok ? 0 : 1;
}
