/* moe_layer.h -- one MoE FFN (router, the routed experts and the shared expert) as one call of
 * libpurhie_qmv.so (gfx950). No counterpart in the reference's library ABI: it is the engine's moe_core /
 * moe_core_one / shared_as_slot (src/qwen_model.cpp:1093-1166) over the kernels of qmatvec.h and moe_ops.h,
 * with the same dispatch rules:
 *   - one token with a shared expert of the routed experts' width, types and row sizes: the shared expert rides
 *     as slot n_used (id -1) of the experts' launches (gate / up, SwiGLU, down in 3 launches instead of 6; the
 *     same arithmetic per row, the shared output added last by the combine);
 *   - 8 tokens or more: the (token, slot) entries grouped by expert for the expert-tiled GEMMs, at the largest
 *     tile all three expert matrices take (qmatvec_id_batch_tile), but at most 64 entries where the experts' mean
 *     entry count m (T n_used / n_expert) is at most 56 or fills fewer 64-entry than 128-entry slots;
 *   - otherwise the expert-indexed matvecs, token by token in the decode order (gate / up as one pair launch,
 *     down with x_per_slot; for a Q8_0-activation down type the SwiGLU and its quantization run inside the down
 *     launch, qmatvec_launch_q8_id_swiglu, with the same bits);
 *   - the shared expert's gate / up and down as plain launches, its output weighted by sigmoid(x . shexp_gate)
 *     (or 1 without one) and added after the routed experts.
 * The router logits come from the int8 path when the router's type has an int8 kernel at n_embd, else from
 * the float-activation path (F32 / F16 / BF16 routers). */
#ifndef PURHIE_MOE_LAYER_H
#define PURHIE_MOE_LAYER_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qmatvec.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct purhie_moe_weights {
    int n_embd, n_ff_exp, n_ff_shexp, n_expert, n_expert_used;
    /* the routed experts: gate / up [n_expert * n_ff_exp] rows of n_embd (one type), down [n_expert * n_embd]
     * rows of n_ff_exp */
    int type_gate_up, type_down;
    const void *gate_exps, *up_exps, *down_exps;
    size_t rb_gate_up, rb_down;
    /* the router: [n_expert] rows of n_embd */
    int type_router;
    const void *router;
    size_t rb_router;
    /* the shared expert (gate_shexp NULL: none): gate / up [n_ff_shexp] rows of n_embd, down [n_embd] rows of
     * n_ff_shexp; shexp_gate [n_embd] fp32 (NULL: weight 1) */
    int type_shexp_gate_up, type_shexp_down;
    const void *gate_shexp, *up_shexp, *down_shexp;
    size_t rb_shexp_gate_up, rb_shexp_down;
    const float *shexp_gate;
} purhie_moe_weights;

/* Device workspace bytes purhie_moe_ffn needs for T tokens (0: the layer cannot run: a type without an int8
 * kernel at its K, n_expert > 1024, n_expert_used > 63, or a size out of range). */
size_t purhie_moe_workspace_bytes(const purhie_moe_weights *w, int T);

/* 1 if a call with T tokens takes the one-token shared-expert-as-slot form */
int purhie_moe_shared_as_slot(const purhie_moe_weights *w, int T);

/* out [T][n_embd] = the MoE FFN of the T rows of xn [T][n_embd] (fp32), given xn also quantized as one
 * flattened [T * n_embd] vector in q8_xn (qmatvec_quantize, or a producer's fused quantization). ws: device
 * memory of at least purhie_moe_workspace_bytes(w, T) bytes, 256-byte aligned. Every launch goes on stream;
 * nothing is allocated. Returns hipErrorInvalidValue for bad arguments, else the first launch error. */
hipError_t purhie_moe_ffn(const purhie_moe_weights *w, const float *xn, const qmatvec_q8 *q8_xn, int T, float *out,
                          void *ws, size_t ws_bytes, hipStream_t stream);

/* Bytes of the static workspace purhie_moe_ffn_noalloc uses on each GPU (32 MiB). */
#define PURHIE_MOE_SCRATCH_BYTES ((size_t)32 << 20)

/* purhie_moe_ffn with the library's own workspace instead of the caller's. No counterpart in the reference: for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is a static device array of PURHIE_MOE_SCRATCH_BYTES on each GPU, held from the library's load
 * until the process ends; its address is looked up once per device, on the first call with that device current.
 * Returns hipErrorInvalidValue when purhie_moe_workspace_bytes(w, T) exceeds PURHIE_MOE_SCRATCH_BYTES (at n_embd
 * 2048, 128 experts of n_ff_exp 768, top 8, no shared expert: above 256 tokens) or for any argument
 * purhie_moe_ffn rejects. Every call on one GPU shares that GPU's array and leaves its contents behind (each call
 * writes every region before reading it): calls that overlap on one GPU (other streams, other threads) race.
 * Nothing is allocated. */
hipError_t purhie_moe_ffn_noalloc(const purhie_moe_weights *w, const float *xn, const qmatvec_q8 *q8_xn, int T,
                                  float *out, hipStream_t stream);

/* No counterpart in the reference: a test hook for the layer's stage-by-stage parity tests. Where purhie_moe_ffn(w,
 * T) puts its intermediate results in the caller's workspace, as byte offsets from ws (-1: not in this form):
 * the routed ids [T][ns] (ns = n_expert_used, or + 1 with the shared expert as slot n_expert_used), their weights
 * [T][n_expert_used] and the shared expert's gate [T]; the experts' gate and up outputs [T * ns][n_ff_exp] (written
 * where gu_written is 1; the grouped ROCmFP4 / FAST / NVFP4 form folds SwiGLU into its gate / up GEMM instead and
 * writes the quantized activation only); the quantized SwiGLU activation [T * ns][n_ff_exp] (a qmatvec_q8 of qx_k
 * values, qmatvec_q8_bind layout; written where act_written is 1); the down outputs [T * ns][n_embd] (row t * ns +
 * slot); the shared expert's output [T][n_embd] and its quantized activation (a qmatvec_q8 of qs_k values) outside
 * the slot form. Returns 0, or -1 when the layer cannot run (purhie_moe_workspace_bytes answers 0). */
typedef struct {
    long long ids, wts, sg, g, u, qx, down, shout, qs;
    int ns, qx_k, qs_k, slot, grouped, gu_written, act_written;
} purhie_moe_regions;
int purhie_moe_debug_regions(const purhie_moe_weights *w, int T, purhie_moe_regions *r);

#ifdef __cplusplus
}
#endif

#endif /* PURHIE_MOE_LAYER_H */
