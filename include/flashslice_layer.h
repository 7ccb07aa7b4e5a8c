/*
 * flashslice_layer.h -- C ABI of the kernels for the layer around the
 * slice/deslice path (same library as flashslice_hip.h, whose conventions
 * apply: caller-owned memory, asynchronous launches on `stream`, FS_OK or an
 * FS_ERR_* code with text from fs_last_error(), bitwise-reproducible sums).
 *
 * No counterpart in the reference's kernels: its model normalises with
 * torch.nn.LayerNorm (reference flashslice/models/transolver.py:51-63).
 * These entry points serve flashslice_amd.layers (PointLayerNorm), which
 * keeps nn.LayerNorm's parameters and state dict.
 */
#ifndef FLASHSLICE_LAYER_H
#define FLASHSLICE_LAYER_H

#include <stddef.h>
#include <stdint.h>

#include "flashslice_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* LayerNorm over the last axis of contiguous (rows, cols) fp32 rows:
 * y = (x - mean) * rstd * gamma + beta, rstd = 1 / sqrt(var + eps) (biased
 * variance), mean and rstd (rows,) saved for the backward. cols is a
 * multiple of 4 in [4, 2048]; x, y, gamma, beta 16-byte aligned. */
int32_t fs_layernorm_fwd(const float* x, const float* gamma, const float* beta, float* y,
                         float* mean, float* rstd, int64_t rows, int32_t cols, float eps,
                         void* stream);

/* Bytes of workspace fs_layernorm_bwd needs (0 for an unsupported shape). */
size_t fs_layernorm_workspace_bytes(int64_t rows, int32_t cols);

/* dx = rstd (g - mean(g) - xhat mean(g xhat)), g = dy gamma,
 * xhat = (x - mean) rstd; dgamma = sum_rows dy xhat, dbeta = sum_rows dy
 * (cols,). mean and rstd as fs_layernorm_fwd wrote them. */
int32_t fs_layernorm_bwd(const float* dy, const float* x, const float* gamma, const float* mean,
                         const float* rstd, float* dx, float* dgamma, float* dbeta,
                         void* workspace, size_t workspace_bytes, int64_t rows, int32_t cols,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHSLICE_LAYER_H */
