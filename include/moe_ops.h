/* moe_ops.h -- C ABI of the matvec inputs' producers (add + RMSNorm, SwiGLU, both quantizing their output) and
 * of the mixture-of-experts glue around the expert matvecs (libpurhie_qmv.so, gfx950).
 *
 * Drop-in for those parts of the reference's src/gpu_ops.h: same names, argument meaning and error
 * convention (hipError_t; hipErrorInvalidValue for bad arguments). All launches are asynchronous on `stream`;
 * every buffer is device memory owned by the caller. */
#ifndef PURHIE_MOE_OPS_H
#define PURHIE_MOE_OPS_H

#include <hip/hip_runtime.h>

#include "qmatvec.h"

#ifdef __cplusplus
extern "C" {
#endif

/* replaces src/gpu_ops.h:20-25 (kernels src/gpu_ops.hip:17-100): for each of T rows of n values, x_out = x_in +
 * add (add NULL: x_out is not written and x_in is normalized), then y = x_out / sqrt(mean(x_out^2) + eps) * w
 * (w NULL: no gamma); x_out must not alias x_in when add is set. With q8, the T rows of y are also quantized
 * into it as one flattened [T * n] vector in the same launch (n % 256 == 0, T * n <= q8->max_k). A row's
 * result does not depend on T. */
hipError_t gpu_add_rmsnorm(const float *x_in, const float *add, float *x_out, const float *w, float *y, int n, int T,
                           float eps, const qmatvec_q8 *q8, hipStream_t stream);

/* replaces src/gpu_ops.h:29 (kernel src/gpu_ops.hip:103-113): out = SiLU(g) * u = g / (1 + exp(-g)) * u for
 * n values, quantized into q8 in the same launch when q8 is not NULL (n % 32 == 0, n <= q8->max_k; the Q8_K
 * side is complete only for whole 256-value blocks). With q8 set, out may be NULL: only the quantized form is
 * written (no counterpart in the reference, whose out is always written). */
hipError_t gpu_swiglu(const float *g, const float *u, float *out, int n, const qmatvec_q8 *q8, hipStream_t stream);

/* replaces src/gpu_ops.h:36-37 (kernels src/gpu_ops.hip:149-241): for T tokens, logits [T][n_expert] ->
 * softmax -> the n_used largest probabilities in descending order (equal values: the lower expert) into
 * ids [T][ids_stride] and their weights p / max(sum, 6.103515625e-5) into wts [T][n_used]; with w_shexp [n],
 * sg [T] = sigmoid(x[t] . w_shexp) (x [T][n]). ids_stride 0 means n_used; a larger stride sets the entry
 * after the selection to -1 (the shared expert's slot). n_expert <= 1024, n_used <= 64. */
hipError_t gpu_moe_router(const float *logits, const float *x, const float *w_shexp, int *ids, float *wts, float *sg,
                          int n_expert, int n_used, int n, int T, hipStream_t stream, int ids_stride);

/* replaces src/gpu_ops.h:40-41 (kernel src/gpu_ops.hip:245-264): out [T][n] = sum_j wts[t][j] * down[t][j]
 * in slot order (+ sg[t] * shared[t] with shared; + shared[t] when sg is NULL); down [T][n_used][n]. wts NULL:
 * weights 1. Every product and sum is rounded on its own (no fused multiply-add). */
hipError_t gpu_moe_combine(const float *down, const float *wts, const float *shared, const float *sg, float *out,
                           int n_used, int n, int T, hipStream_t stream);

/* replaces src/gpu_ops.h:44-46: as gpu_moe_combine, each expert's output first multiplied by
 * exp_scale[ids[t][j]] when exp_scale is not NULL. */
hipError_t gpu_moe_combine_scaled(const float *down, const float *wts, const float *shared, const float *sg,
                                  const int *ids, const float *exp_scale, float *out, int n_used, int n, int T,
                                  hipStream_t stream);

/* replaces src/gpu_ops.h:72-75: the most tiles gpu_moe_group can write for T tokens of n_used slots */
static inline int gpu_moe_max_tiles(int T, int n_used, int n_expert, int tile) {
    const int n = T * n_used, bound = n_expert + n / tile;
    return n < bound ? n : bound;
}

/* replaces src/gpu_ops.h:76-77 (kernel src/gpu_ops.hip:273-330): group the entries (token t, slot j) of
 * ids [T][n_used] by expert for the expert-tiled GEMM (qmatvec_launch_q8_id_batch): entry p of the sorted
 * order has tok_rows[p] = t and pair_rows[p] = t * n_used + j; each expert's run is cut into tiles of up to
 * `tile` entries (tile_e, tile_start, tile_n; *n_tiles of them, in expert order). Counts and tiles are
 * deterministic, the order inside an expert's run is not. n_expert <= 1024; ids outside [0, n_expert) are
 * left out. */
hipError_t gpu_moe_group(const int *ids, int T, int n_used, int n_expert, int tile, int *tok_rows, int *pair_rows,
                         int *n_tiles, int *tile_e, int *tile_start, int *tile_n, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
