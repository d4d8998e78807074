/* qmatvec.h -- y = W x for GGUF weight blocks on MI355X (gfx950), the drop-in for the reference's
 * src/qmatvec.h (aardbeiplantje/PURHIE). Same symbols, argument meaning, buffer layout and error
 * convention; the kernels are this library's own wave64 HIP code (libpurhie_qmv.so), linked in, so
 * no code object is loaded by path.
 *
 * Weights are HBM-resident: W is a device pointer to N rows of row_bytes = qt_row_size(type, K) bytes
 * in the unchanged GGUF block layout. All launches are asynchronous on `stream` (0 = the null stream)
 * with no internal synchronisation. Errors: hipErrorInvalidDeviceFunction (no kernel for this type /
 * shape), hipErrorInvalidValue (bad shape, alignment, capacity); launch errors pass through.
 *
 * Types with int8 kernels: Q8_0 (8), Q4_K (12), Q5_K (13), Q6_K (14), IQ4_XS (23), MXFP4 (39), NVFP4 (40),
 * Q4_0_ROCMFP4 (100), Q4_0_ROCMFP4_FAST (101). No launch allocates device memory.
 */
#ifndef PURHIE_QMATVEC_H
#define PURHIE_QMATVEC_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces src/qmatvec.h:17-18. The reference loads a code object from co_path; here the kernels are
 * part of the library and co_path is ignored. Returns 0 (a HIP device is present) or -1. Idempotent. */
int qmatvec_init(const char *co_path);
void qmatvec_free(void);

/* replaces src/qmatvec.h:24-26: NVFP4-style output scale registry (the outputs of launches on the
 * matrix at W, bytes long, are multiplied by s[0], or by s[e] for expert e of n stacked experts of bytes / n
 * each). s must stay readable by both the CPU and the GPU (pinned or managed memory) while it is registered:
 * dense launches read their factor on the host at launch time, expert-indexed launches and expert-tiled GEMMs
 * over n > 1 experts hand s to the kernel, which reads s[e] on the device. owner groups registrations for
 * qmatvec_drop_out_scales. Where registered ranges overlap, the earliest registration holding W applies.
 * Returns 0 or -1. */
int qmatvec_set_out_scale(const void *owner, const void *W, size_t bytes, const float *s, int n);
void qmatvec_drop_out_scales(const void *owner);

/* replaces src/qmatvec.h:29: 1 if a float-activation matvec exists for the type: F32, F16, BF16, and the quantized
 * types Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, MXFP4, NVFP4, ROCmFP4 and ROCmFP4_FAST (fp32 activations against the
 * exactly decoded weights; the int8 path below is the fast one) */
int qmatvec_supported(int type);

/* Float activations (replace src/qmatvec.h:33-75). F16 / BF16 weights multiply the activations rounded to the
 * weight type (nearest even), so every product is exact; F32, _bf16f and the quantized types multiply the fp32
 * activations as they are. Same arguments, checks and error codes as the reference's.
 *   qmatvec_launch_bf16f    BF16 weights (row_bytes = 2 K), fp32 activations not rounded, T rows
 *   qmatvec_launch          one row of x; a type qmatvec_supported takes, row_bytes = qt_row_size(type, K), K a
 *                           whole number of blocks; a registered output scale multiplies the quantized types' rows
 *   qmatvec_launch_batch    T rows; F16 / BF16 batches qmatvec_half_supported takes go to the MFMA GEMM (which
 *                           rounds x while staging it: nothing allocated), the rest to the decode kernels (a
 *                           token's row the same bits as qmatvec_launch gives it)
 *   qmatvec_launch_batch_h  the same with the caller's scratch xh (16-byte aligned, xh_bytes >= 2 T K) for the copy
 *   qmatvec_half_supported  F16 / BF16, GEMMs on, T >= 32 (any T in prefill mode), N >= 64, K % 8 == 0,
 *                           K < 2^22, row_bytes >= 2 K, a multiple of 16 and below 2^23, W 16-byte aligned
 *   qmatvec_round_half      x -> xh rounded to the type (n % 8 == 0, both 16-byte aligned)
 *   qmatvec_launch_batch_hx the GEMM on xh (T rows of K values) */
hipError_t qmatvec_launch_bf16f(const void *W, size_t row_bytes, const float *x, float *y, int N, int K, int T,
                                hipStream_t stream);
hipError_t qmatvec_launch(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                          hipStream_t stream);
hipError_t qmatvec_launch_batch(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                                int T, hipStream_t stream);
hipError_t qmatvec_launch_batch_h(int type, const void *W, size_t row_bytes, const float *x, uint16_t *xh,
                                  size_t xh_bytes, float *y, int N, int K, int T, hipStream_t stream);
int qmatvec_half_supported(int type, const void *W, size_t row_bytes, int N, int K, int T);
hipError_t qmatvec_round_half(int type, const float *x, uint16_t *xh, long long n, hipStream_t stream);
hipError_t qmatvec_launch_batch_hx(int type, const void *W, size_t row_bytes, const uint16_t *xh, float *y, int N,
                                   int K, int T, hipStream_t stream);

/* The split-Q8_0 copy of a float matrix, for the opt-in Q8_0 LM head (replace src/qmatvec.h:68-75): ggml's Q8_0
 * quantization per 32 values (d = amax / 127 stored as fp16, q = roundf(x / d) with the fp32 d) into values qs [N][K]
 * (16-byte aligned) and scales d [N][K / 32]; F32 / F16 / BF16 rows, K % 256 == 0. qmatvec_launch_q8_0s: y = qs x
 * with x given by the Q8_0 part of q, as ggml's Q8_0 x Q8_0 dot (K % 256 == 0, K <= q->max_k). */
int qmatvec_q8_0s_source_supported(int type, int K);
hipError_t qmatvec_quantize_rows_q8_0(int type, const void *W, size_t row_bytes, int N, int K, int8_t *qs, uint16_t *d,
                                      hipStream_t stream);

/* replaces src/qmatvec.h:49-54 (mode flags). Prefill mode routes every batch size to the GEMM
 * kernels (so a row's sums do not depend on how the prompt was cut into batches). */
void qmatvec_set_prefill(int on);
int qmatvec_prefill(void);
void qmatvec_set_prefill_fp32(int on);

/* ---------------------------------------------------------------- int8 path
 * The activation is quantized once (qmatvec_quantize) into both of ggml's CPU formats, Q8_0 (32-value
 * blocks, ROCmFP4 / Q8_0 weights) and Q8_K (256-value blocks, K-quants), bit-identical to the
 * reference's src/q8_device.h:54-104. Layout of qmatvec_q8 (src/qmatvec.h:82-93, src/qmatvec.cpp:395-419). */
typedef struct qmatvec_q8 {
    int8_t *q0;    /* Q8_0 values [K] */
    float *d0;     /* Q8_0 scales [K / 32], fp16-rounded */
    int8_t *qK;    /* Q8_K values [K] */
    float *dK;     /* Q8_K scales [K / 256] */
    int32_t *bsK;  /* Q8_K sums of every 16 values [K / 16] */
    int32_t *s0;   /* per 32 values: fp16(d * sum of the block's q) as float bits */
    int max_k;
    uint16_t *xh;  /* optional 16-bit copy (unused by this library's int8 kernels) */
    int xh_bf16;
} qmatvec_q8;

typedef struct qmatvec_q8_out {
    int8_t *q0;
    float *d0;
    int8_t *qK;
    float *dK;
    int32_t *bsK;
    int32_t *s0;
    uint16_t *xh;
    int xh_bf16;
} qmatvec_q8_out;

static inline qmatvec_q8_out qmatvec_q8_outputs(const qmatvec_q8 *q) {
    qmatvec_q8_out o = {0, 0, 0, 0, 0, 0, 0, 0};
    if (q) {
        o.q0 = q->q0;
        o.d0 = q->d0;
        o.qK = q->qK;
        o.dK = q->dK;
        o.bsK = q->bsK;
        o.s0 = q->s0;
        o.xh = q->xh;
        o.xh_bf16 = q->xh_bf16;
    }
    return o;
}

/* replaces src/qmatvec.h:118-119: bytes for vectors of up to max_k values (max_k % 256 == 0), and
 * binding a qmatvec_q8 to such device memory (16-byte aligned) */
size_t qmatvec_q8_bytes(int max_k);
void qmatvec_q8_bind(qmatvec_q8 *q, void *mem, int max_k);

/* replaces src/qmatvec.h:123: 1 if an int8 kernel handles the type at this K (Q8_0 / ROCmFP4: K % 64,
 * FAST: K % 128, K-quants: K % 256) */
int qmatvec_q8_supported(int type, int K);

/* replaces src/qmatvec.h:127: x[K] (device) -> q, both formats. K % 32 == 0, K <= q->max_k. */
hipError_t qmatvec_quantize(const float *x, int K, const qmatvec_q8 *q, hipStream_t stream);

/* replaces src/qmatvec.h:130-131: y = W x with x given by its quantized form */
hipError_t qmatvec_launch_q8(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N, int K,
                             hipStream_t stream);

/* replaces src/qmatvec.h:134-135: y = W x (N rows), y2 = W2 x (N2 rows) in one launch */
hipError_t qmatvec_launch_q8_pair(int type, const void *W, int N, float *y, const void *W2, int N2, float *y2,
                                  size_t row_bytes, const qmatvec_q8 *q, int K, hipStream_t stream);

/* replaces src/qmatvec.h:144-152: n (1..4) matvecs of one type and K on the same input in one launch;
 * the _t form takes T (1..4) tokens (input rows t of q, output rows ys[i] + t * Ns[i]), reading the
 * weights once, each token's result equal to its single-token launch bit for bit */
int qmatvec_q8_few_supported(int type, int K, int T);
hipError_t qmatvec_launch_q8_multi_t(int type, int n, const void *const *Ws, const int *Ns, float *const *ys,
                                     size_t row_bytes, const qmatvec_q8 *q, int K, int T, hipStream_t stream);
hipError_t qmatvec_launch_q8_multi(int type, int n, const void *const *Ws, const int *Ns, float *const *ys,
                                   size_t row_bytes, const qmatvec_q8 *q, int K, hipStream_t stream);

/* replaces src/qmatvec.h:157-158: Y[t] = W X[t] for T tokens, q the T rows quantized as one [T * K]
 * vector, row t of the result at y + t * ldy */
hipError_t qmatvec_launch_q8_batch(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y,
                                   long long ldy, int N, int K, int T, hipStream_t stream);

/* replaces src/qmatvec.h:167-179: MoE expert-indexed matvecs. W stacks every expert's N rows. For
 * token t and slot j < n_used, expert e = ids[t * n_used + j] multiplies input row t (x_per_slot = 0)
 * or t * n_used + j (x_per_slot = 1) into row t * n_used + j of y; an id of -1 selects Wx (W2x). */
hipError_t qmatvec_launch_q8_id(int type, const void *W, size_t row_bytes, const int32_t *ids, int n_used,
                                int x_per_slot, const qmatvec_q8 *q, float *y, int N, int K, int T, hipStream_t stream);
hipError_t qmatvec_launch_q8_id_pair(int type, const void *W, const void *W2, size_t row_bytes, const int32_t *ids,
                                     int n_used, int x_per_slot, const qmatvec_q8 *q, float *y, float *y2, int N, int K,
                                     int T, hipStream_t stream);
hipError_t qmatvec_launch_q8_id_x(int type, const void *W, const void *W2, const void *Wx, const void *W2x,
                                  size_t row_bytes, const int32_t *ids, int n_used, int x_per_slot,
                                  const qmatvec_q8 *q, float *y, float *y2, int N, int K, int T, hipStream_t stream);

/* No counterpart in the reference (it launches gpu_moe_router, then qmatvec_launch_q8_id_pair): the expert gate /
 * up pair of a decode step with the routing folded in. logits [T][n_expert]: every workgroup routes its token as
 * gpu_moe_router does (softmax, the n_used largest in descending order, weights divided by their sum; no shared
 * gate), ids [T][n_used] and wts [T][n_used] receive the same values as that launch's, and y / y2 the pair
 * launch's with x_per_slot = 0: bit-identical to the two launches, one launch fewer. Shapes the one-unit-per-lane
 * kernel does not take, n_expert > 256 or the per-wave decode path run the two launches. */
hipError_t qmatvec_launch_q8_id_pair_routed(int type, const void *W, const void *W2, size_t row_bytes,
                                            const float *logits, int n_expert, int32_t *ids, float *wts, int n_used,
                                            const qmatvec_q8 *q, float *y, float *y2, int N, int K, int T,
                                            hipStream_t stream);

/* No counterpart in the reference (it launches gpu_swiglu, then qmatvec_launch_q8_id with x_per_slot = 1): the
 * expert down matvec of a decode step with the SwiGLU launch folded in. Entry (t, slot) reads row t * n_used +
 * slot of g and u (K floats each), quantizes SwiGLU(g, u) = g / (1 + exp(-g)) * u to Q8_0 in the kernel and
 * multiplies it by expert ids[t * n_used + slot] (Wx for -1) into row t * n_used + slot of y: bit-identical to
 * the two launches, one launch fewer. For the Q8_0-activation types (Q8_0, ROCmFP4, FAST, MXFP4, NVFP4), K % 256
 * == 0, K <= 16384; _supported says whether a launch takes it. */
int qmatvec_q8_id_swiglu_supported(int type, int K);
hipError_t qmatvec_launch_q8_id_swiglu(int type, const void *W, const void *Wx, size_t row_bytes, const int32_t *ids,
                                       int n_used, const float *g, const float *u, float *y, int N, int K, int T,
                                       hipStream_t stream);

/* replaces src/qmatvec.h:189-195: MoE prefill over gpu_moe_group's expert tiles (tile k: expert
 * tile_e[k], entries tile_start[k] .. + tile_n[k] - 1 of in_rows / out_rows). qmatvec_id_batch_tile is the largest
 * tile a launch takes: 64 for the FP4 family, Q8_0 and MXFP4, 128 for the K-quants (any smaller tile works, with
 * the same bits). */
int qmatvec_id_batch_tile(int type, int N, int K);
int qmatvec_q8_id_batch_supported(int type, int K);
hipError_t qmatvec_launch_q8_id_batch(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N,
                                      int K, int max_tiles, int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                      const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                      const int32_t *out_rows, hipStream_t stream);

/* No counterpart in the reference (its engine calls qmatvec_launch_q8_id_batch for the experts' gate, then their
 * up projection, src/qwen_model.cpp:1060-1071): both over the same expert tiles in one launch, W into y and W2
 * into y2 (the same type, shape and row_bytes). Each output is bit-identical to the single launch's; one launch
 * instead of two lets the two matrices' workgroups share the chip. */
hipError_t qmatvec_launch_q8_id_batch_pair(int type, const void *W, const void *W2, size_t row_bytes,
                                           const qmatvec_q8 *q, float *y, float *y2, int N, int K, int max_tiles,
                                           int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                           const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                           const int32_t *out_rows, hipStream_t stream);

/* No counterpart in the reference (its engine runs the experts' gate and up GEMMs, then gpu_swiglu with the
 * down projection's quantization, src/qwen_model.cpp:1150-1156): the pair above with SwiGLU(gate, up) =
 * g / (1 + exp(-g)) u and its Q8_0 quantization in the GEMM's epilogue. Entry j's row out_rows[j] of h gets the
 * bits gpu_swiglu's quantizer writes there: q0, d0, and s0 where h binds it (the Q8_K side is not written, so the
 * consumer reads Q8_0). The gate and up outputs are not stored. For the types whose GEMM folds the activation scale
 * into its operands (ROCmFP4, ROCmFP4_FAST, NVFP4) with N a multiple of 128; _supported says whether a launch
 * takes the shape (else hipErrorInvalidDeviceFunction, before anything runs). */
int qmatvec_q8_id_batch_swiglu_supported(int type, int N, int K);
hipError_t qmatvec_launch_q8_id_batch_swiglu(int type, const void *W, const void *W2, size_t row_bytes,
                                             const qmatvec_q8 *q, const qmatvec_q8 *h, int N, int K, int max_tiles,
                                             int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                             const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                             const int32_t *out_rows, hipStream_t stream);

hipError_t qmatvec_launch_q8_0s(const int8_t *qs, const uint16_t *d, const qmatvec_q8 *q, float *y, int N, int K,
                                hipStream_t stream);
/* replace src/qmatvec.h:145-147: one token, y = W x with x = SiLU(lo * scale) for lo [n], zero-padded to K and
 * quantized to Q8_0 inside the kernel: the bits gpu_swiglu(lo * scale, 1, .., q8) followed by qmatvec_launch_q8
 * give (no output scale). ROCmFP4_FAST, K % 128 == 0, K <= 1024, n <= K, W and row_bytes 4-byte aligned. */
int qmatvec_q8_lr_supported(int type, int K);
hipError_t qmatvec_launch_q8_lr(int type, const void *W, size_t row_bytes, const float *lo, int n, int K, float scale,
                                float *y, int N, hipStream_t stream);

/* Float-activation MoE entries (replace src/qmatvec.h:179-180,195-199), for the types qmatvec_supported takes.
 * qmatvec_launch_id: token t, slot j < n_used: expert e = ids[t n_used + j] (rows e N .. e N + N - 1 of W) times
 * input row t (x_per_slot 0) or t n_used + j into output row t n_used + j; an id below 0 writes nothing.
 * qmatvec_launch_id_batch_f: the same over the grouping's expert tiles of up to `tile` <= 16 entries (in_rows:
 * input rows, out_rows: output rows); each entry gets the bits qmatvec_launch_id gives it, and a quantized type's
 * entry the bits qmatvec_launch gives that expert's rows. Registered output scales (per stacked expert) apply. */
hipError_t qmatvec_launch_id(int type, const void *W, size_t row_bytes, const int32_t *ids, int n_used, int x_per_slot,
                             const float *x, float *y, int N, int K, int T, hipStream_t stream);
int qmatvec_id_batch_f_supported(int type);
hipError_t qmatvec_launch_id_batch_f(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                                     int max_tiles, int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                     const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                     const int32_t *out_rows, hipStream_t stream);

/* No counterpart in the reference: test hooks for the parity tests (no effect on the results).
 * qmatvec_debug_capture(out, n_ints): capture mode on (out: device memory the caller zeroed) or off (out null).
 *   While on, each int8 launch runs its kernel's capture instantiation -- the same decode and integer dot code,
 *   which also adds every integer sum it forms into out (integer atomics, so sums a kernel splits over lanes
 *   arrive whole). Layouts (G = qmatvec_debug_capture_unit(type, 0), U = qmatvec_debug_capture_unit(type, 1)):
 *     decode, dense (launch_q8 / _pair / _multi / _multi_t, and _batch below the GEMM threshold): the dot of scale
 *       group g of launch row r (the rows of Ws[0], then Ws[1], ...) for token t at out[(t * Nrows + r) * (K / G) + g];
 *     decode, expert-indexed (_id / _id_pair / _id_x / _id_swiglu): matrix m's row r for output row o (t * n_used +
 *       slot) at out[((m * T * n_used + o) * N + r) * (K / G) + g]; the expert-tiled launch in decode order: output
 *       row o = out_rows[..] and m = 0;
 *     GEMM (_batch at the GEMM threshold, _id_batch): the exact integer the epilogue scales (K-quants: a 256-value
 *       super-block's sum of sub-block scale times dot) of token t (dense) or output row o (expert tiles) and row r
 *       at out[(t * N + r) * (K / U) + unit]; U = 0: that GEMM has no integer sums and writes nothing.
 *   A launch whose capture would not fit n_ints returns hipErrorInvalidValue (tiles mode: the caller sizes out for
 *   the largest output row). G is the values one weight scale covers (16 for ROCmFP4, NVFP4, Q6_K; else 32), the
 *   dots are of the raw levels (Q4_K 0..15, Q5_K 0..31, Q6_K 0..63, IQ4_XS the table levels).
 * qmatvec_debug_decode_path(mode): 1 = the tile kernels where they take the shape (the default; PURHIE_MV_TILE=0 in
 *   the environment at load makes it 0), 0 = the per-wave kernels only, other values only query; returns the
 *   previous mode. */
hipError_t qmatvec_debug_capture(int32_t *out, size_t n_ints);
int qmatvec_debug_capture_unit(int type, int gemm);
int qmatvec_debug_decode_path(int mode);

/* No counterpart in the reference: a measured alternative, not used by any launch above. The ROCmFP4 prefill GEMM
 * (dense, prefill semantics of qmatvec_launch_q8_batch: y [T][ldy] = W x for the Q8_0 activation q) on gfx950's
 * f8f6f4 matrix core, exact: the codebook levels and the activation's two 4-bit planes as E4M3 operands, every
 * 16-value group's integer dot from its own pair of instructions, and the reference's float epilogue per group.
 * K % 64 == 0; hipErrorInvalidValue otherwise. The benchmark times it beside the split GEMM. */
hipError_t qmatvec_debug_gemm_f8f6f4(const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int ldy, int N,
                                     int K, int T, hipStream_t stream);

/* No counterpart in the reference: a test hook, an independent scalar kernel. The integer dot of every weight
 * scale group (Q8_0 / FAST / MXFP4 / Q4_K / Q5_K / IQ4_XS: 32 values, ROCmFP4 / NVFP4 / Q6_K: 16) of every row
 * against the quantized activation, computed by the same device decoders as the matvec kernels: out[N][K / group].
 * Q4_K / Q5_K / Q6_K dot the raw levels (0..15 / 0..31 / 0..63), IQ4_XS the table levels (-127..113). */
hipError_t qmatvec_debug_block_dots(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, int32_t *out,
                                    int N, int K, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PURHIE_QMATVEC_H */
