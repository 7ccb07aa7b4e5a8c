/*
 * flashslice_hip.h -- C ABI of the MI355X (gfx950) FlashSlice kernels.
 *
 * The drop-in boundary of this build is the reference's custom-operator
 * layer: the eight torch.library ops in namespace "flashslice"
 * (reference flashslice/kernels/slice_ops.py:787-801 and
 * flashslice/kernels/blocked.py:1477-1494), whose implementations are
 * registered for the CUDA dispatch key (slice_ops.py:888-891,
 * blocked.py:1496-1499). The Python package flashslice_amd keeps those op
 * names, schemas, fake implementations and autograd formulas, and its
 * CUDA-key implementations call the entry points below through ctypes.
 *
 * Conventions
 *  - No entry point allocates, frees, or synchronises. Every output and the
 *    workspace are caller-owned device buffers. Launches are asynchronous on
 *    `stream` (a hipStream_t passed as void*; NULL = the null stream).
 *  - Return value: FS_OK (0) or an FS_ERR_* code; fs_last_error() gives the
 *    text for the calling thread. Shape and layout errors are detected
 *    before any launch.
 *  - Point tensors (B, N, H, C) are passed as fs_points with element strides
 *    along b, n, h and a unit stride along C. Supported dtypes: fp32, bf16,
 *    fp16; every point tensor of one call must share one dtype.
 *  - The slice projection (weight (.., G, D), bias (.., G), tau (H,)) and the
 *    small per-slot tensors (tokens, dz_num, ds, stats) are fp32 and
 *    contiguous. Parameter gradients are written in the parameter's own
 *    shape (Bw, Hw, G, D) / (Bb, Hb, G), Bw = B if w_stride_b != 0 else 1,
 *    Hw = H if w_stride_h != 0 else 1 (likewise for the bias).
 *  - Results are bitwise reproducible: cross-tile sums use fixed per-wave
 *    partials reduced in a fixed order, never atomics.
 */
#ifndef FLASHSLICE_HIP_H
#define FLASHSLICE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fs_status {
  FS_OK = 0,
  FS_ERR_INVALID = 1,     /* bad shape, stride, dtype or pointer */
  FS_ERR_UNSUPPORTED = 2, /* a valid request no kernel in this build serves */
  FS_ERR_WORKSPACE = 3,   /* workspace smaller than fs_workspace_bytes() */
  FS_ERR_HIP = 4          /* a HIP launch error (text in fs_last_error) */
};

enum fs_dtype { FS_F32 = 0, FS_BF16 = 1, FS_F16 = 2 };

enum fs_op {
  FS_OP_SLICE_FWD = 0,
  FS_OP_DESLICE_FWD = 1,
  FS_OP_SLICE_BWD = 2,
  FS_OP_DESLICE_BWD = 3,
  FS_OP_STATS = 4,
  FS_OP_TIED_BWD = 5
};

/* A (B, N, H, width) tensor of points: x_mid, fx_mid, d_out, out, dx, dfx. */
typedef struct fs_points {
  void* data;
  int64_t stride_b, stride_n, stride_h; /* in elements */
  int32_t dtype;                        /* enum fs_dtype */
  int32_t width;                        /* D or DV */
} fs_points;

/* Shape, slice projection and dot level of one call. */
typedef struct fs_slice_params {
  int64_t B, N, H, D, DV, G;
  const float* weight;                  /* (.., G, D) fp32 contiguous */
  int64_t w_stride_b, w_stride_h;       /* 0 where shared */
  const float* bias;                    /* (.., G) fp32 contiguous */
  int64_t b_stride_b, b_stride_h;       /* 0 where shared */
  const float* tau;                     /* (H,) fp32 */
  int32_t dot;                          /* 0 ieee, 1 tf32, 2 bf16v, 3 bf16, 4 tf32x3 */
  int32_t family;                       /* 0 auto, 1 whole-G where it fits, 2 G-blocked */
  /* Ragged batch (NULL = none): B samples of different lengths concatenated
   * along the point axis; sample b is rows row_splits[b] .. row_splits[b+1]-1
   * of every point tensor, whose stride_b is then ignored. Device memory,
   * B + 1 non-decreasing int64 with row_splits[0] = 0 and no sample longer
   * than N (N sizes the launch; it is not read from the device). Served by
   * both kernel families; the statistics of a ragged batch (stats_in,
   * stats_out, fs_compute_stats) are (1, H, 2, total_rows) fp32, indexed by
   * row. Slot sums and parameter gradients stay per sample (B, H, ...).
   * No counterpart in the reference, whose ROADMAP.md:66-68 plans it.
   * The library never reads the splits on the host (that would synchronise):
   * the kernels clamp every split to [0, total_rows] and every sample to N
   * rows, so malformed splits give wrong sums but no access outside the
   * point tensors' total_rows rows. */
  const int64_t* row_splits;
  /* Rows of every point tensor of a ragged batch (>= 1 with row_splits;
   * ignored without). */
  int64_t total_rows;
} fs_slice_params;

/* Bytes of workspace an op needs for this shape (op: enum fs_op). */
size_t fs_workspace_bytes(int32_t op, const fs_slice_params* p);

/* Replaces blocked.compute_stats / _stats_kernel (reference
 * flashslice/kernels/blocked.py:1329-1343, :292-400): stats (B, H, 2, N) fp32,
 * [..., 0, n] = max_g L, [..., 1, n] = sum_g exp(L - max). two_pass selects the
 * max-then-sum form (reference set_stats_mode("two-pass"), blocked.py:101-120). */
int32_t fs_compute_stats(const fs_points* x, const fs_slice_params* p, float* stats,
                         int32_t two_pass, void* workspace, size_t workspace_bytes,
                         void* stream);

/* Replaces flashslice::flash_slice (_slice_impl, slice_ops.py:804-819) and
 * flashslice::slice_blk (_slice_blk_impl, blocked.py:1346-1368):
 * z_num (B, H, G, DV) fp32, s (B, H, G) fp32. stats_in (nullable) are
 * statistics of these very logits; stats_out (nullable) receives them. */
int32_t fs_slice_fwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                     const float* stats_in, float* stats_out, float* z_num, float* s,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the static scratch array fs_slice_fwd_static uses (32 MiB). */
#define FS_SCRATCH_BYTES ((size_t)32 << 20)

/* fs_slice_fwd without a workspace argument: it allocates nothing (no
 * hipMalloc, hipFree or allocating library call), for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. No counterpart in the reference. The partials (and
 * the statistics the G-blocked kernels form when none are handed in) live in
 * a file-scope device array of FS_SCRATCH_BYTES, one per GPU the library
 * runs on, held until the process ends; its address is looked up once per
 * device on the first call there. Shapes whose workspace
 * (fs_workspace_bytes(FS_OP_SLICE_FWD, p)) exceeds it return
 * FS_ERR_WORKSPACE before any launch. Results are bitwise equal to
 * fs_slice_fwd's. Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, or two threads without ordering) race. */
int32_t fs_slice_fwd_static(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                            const float* stats_in, float* stats_out, float* z_num, float* s,
                            void* stream);

/* Replaces flashslice::flash_deslice (_deslice_impl, slice_ops.py:846-859)
 * and flashslice::deslice_blk (_deslice_blk_impl, blocked.py:1406-1433):
 * out (B, N, H, DV) in the point dtype from tokens (B, H, G, DV) fp32. */
int32_t fs_deslice_fwd(const fs_points* x, const fs_slice_params* p, const float* tokens,
                       const float* stats_in, float* stats_out, const fs_points* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Replaces flashslice::flash_slice_bwd (_slice_bwd_impl, slice_ops.py:822-843)
 * and flashslice::slice_blk_bwd (_slice_blk_bwd_impl, blocked.py:1371-1403):
 * dx (like x), dfx (like fx), dweight, dbias (parameter shapes, fp32),
 * dtau (H,) fp32, from dz_num (B, H, G, DV) and ds (B, H, G) fp32. */
int32_t fs_slice_bwd(const fs_points* x, const fs_points* fx, const fs_slice_params* p,
                     const float* stats_in, const float* dz_num, const float* ds,
                     const fs_points* dx, const fs_points* dfx, float* dweight, float* dbias,
                     float* dtau, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces flashslice::flash_deslice_bwd (_deslice_bwd_impl,
 * slice_ops.py:862-885) and flashslice::deslice_blk_bwd (_deslice_blk_bwd_impl,
 * blocked.py:1436-1469): dx, dtokens (B, H, G, DV) fp32, dweight, dbias, dtau
 * from d_out (B, N, H, DV). */
int32_t fs_deslice_bwd(const fs_points* x, const fs_slice_params* p, const float* tokens,
                       const float* stats_in, const fs_points* d_out, const fs_points* dx,
                       float* dtokens, float* dweight, float* dbias, float* dtau,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Backward of a deslice -> slice coupling on one x_mid, weight, bias, tau
 * (out = deslice(tokens), (z_num, s) = slice(fx_mid), fx_mid not computed
 * from out) in one pass over the points: both ops' gradients from one
 * recompute of the softmax weights, one softmax Jacobian and one dx. Writes
 * dx (like x), dfx (like fx), dtokens (B, H, G, DV) fp32 and the summed
 * dweight, dbias, dtau of both ops. It replaces the pair fs_deslice_bwd +
 * fs_slice_bwd and autograd's sum of their two dx, i.e. the reference's
 * _deslice_bwd_impl and _slice_bwd_impl (slice_ops.py:822-885) run back to
 * back on the same saved inputs; it is the "tied backward fusion" of the
 * reference's ROADMAP.md:58-65, which the reference does not implement.
 * Served by the whole-G family only (fs_family() == 1); other shapes return
 * FS_ERR_UNSUPPORTED and the caller runs the two backward ops.
 * dfx (or its data pointer) and dtokens may be NULL: that output is not
 * written. A deslice -> MLP -> slice chain has formed dfx before the MLP's
 * backward, and a slice -> deslice chain has formed dtokens before the token
 * mixing's backward; the rest of both ops' backward is this one pass. */
int32_t fs_tied_bwd(const fs_points* x, const fs_points* fx, const fs_points* d_out,
                    const fs_slice_params* p, const float* tokens, const float* dz_num,
                    const float* ds, const fs_points* dx, const fs_points* dfx,
                    float* dtokens, float* dweight, float* dbias, float* dtau,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Which kernel family serves this call: 1 = whole-G (the slot axis held in
 * registers, one pass per op; chosen where the shape fits, G <= 128 and
 * D, DV small enough), 2 = G-blocked (any G: per-point softmax statistics,
 * point-owned and slot-owned kernels). p->family = 2 forces G-blocked. */
int32_t fs_family(const fs_slice_params* p);

/* Text of the last error on the calling thread ("" if none). */
const char* fs_last_error(void);

/* Library version string. */
const char* fs_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASHSLICE_HIP_H */
