/* oracle.h -- CPU restatement of the reference's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker of the HIP product (purhie_amd/), never a
 * part of it: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * Each function restates one reference function (file:line in the reference tree, cited at the
 * definition in oracle.c) in plain C with the reference's float expression order, compiled with
 * -ffp-contract=off so that no multiply-add is fused where the reference does not fuse one.
 *
 * Pinning (how each part is checked, see tests/test_oracle_*.py):
 *   fp16 <-> fp32                     numpy's IEEE conversions, exhaustively over all 2^16 halves and
 *                                     2^24 sampled floats, plus the reference's qz_fp32_to_fp16 (_ref)
 *   decoders (Q8_0 Q4_K Q6_K FP4 FAST) the reference's qt_to_float (_ref) bit for bit on random bytes,
 *                                     and closed forms of single-level blocks
 *   encoders                          the reference's qz_quantize (_ref) byte for byte, the committed
 *                                     golden fixtures, and the reference's own KATs (t/95-quantize.t)
 *   Q8_0 activation quantizer         the reference's cpu_q8_0_quantize (_ref) bit for bit; brute force
 *   Q8_K activation quantizer         closed form (q8_device.h:5-15 / matvec_verify.cpp q8_roundtrip),
 *                                     tie cases; "parity pinned by closed form only" (no CPU quantizer
 *                                     for Q8_K exists in the reference's C++)
 *   integer block dots                brute force: sum of dequantized weight x dequantized activation,
 *                                     recomputed in exact integer arithmetic from qt_to_float (_ref)
 *   expert matvec / FFN               the reference's cpu_matvec_* / cpu_expert_ffn (_ref)
 *   MoE router / group / combine      closed forms (softmax, stable top-k, prefix sums)
 */
#ifndef PURHIE_ORACLE_H
#define PURHIE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids of the path */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_IQ4_XS = 23, ORC_BF16 = 30,
       ORC_MXFP4 = 39, ORC_NVFP4 = 40, ORC_FP4 = 100, ORC_FAST = 101 };

/* ---- scalars */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
float orc_ue4m3_half(uint8_t e);      /* quant_types.cpp scale decoder (GGUF types 100/101) */
float orc_ue4m3_fp4common(uint8_t e); /* fp4_common.h decoder (gemm_act_fp4 only) */
float orc_e8m0_half(uint8_t e);       /* MXFP4's E8M0 scale at half scale */
void orc_f32_to_f16_n(const float *x, uint16_t *h, int64_t n);
void orc_f16_to_f32_n(const uint16_t *h, float *x, int64_t n);

/* ---- formats */
int orc_block_size(int type);           /* values per block, 0 if unsupported */
int orc_type_size(int type);            /* bytes per block */
size_t orc_row_size(int type, int64_t k);
int orc_to_float(int type, const void *src, float *dst, int64_t n);

/* ---- float activations over F32 / F16 / BF16 weights (src/matvec_q.hip:700-1075, 3391-3547)
 * orc_act_round: the activation as the kernels multiply it: rounded to the weight type when round is set
 * (F16: nearest even; BF16: (u + 0x7fff + lsb) >> 16 on the bits, no NaN case), else as it is (F32 always).
 * orc_matvec_float: ref[n] = sum_k w[n][k] act(x[k]) and mag[n] = sum_k |w act(x)| in double (the products of
 * 16-bit weights and rounded activations are exact); T tokens of K values in x, outputs [T][N]. */
float orc_act_round(int type, int round, float x);
void orc_act_round_n(int type, int round, const float *x, float *y, int64_t n);
int orc_matvec_float(int type, int round, const void *W, size_t rb, int N, int K, int T, const float *x, double *ref,
                     double *mag);

/* ---- encoders: nrows rows of k floats -> rows of orc_row_size bytes; n_threads <= 0: all cores */
int orc_quantize(int type, const float *x, void *dst, int64_t nrows, int64_t k, int n_threads);

/* ---- activation quantizers (one row of k values)
 * Q8_0: q0[k], d0[k/32] (fp16-rounded, as float), s0[k/32] (float bits of fp16(d * sum q))
 * Q8_K: qK[k], dK[k/256], bsK[k/16]; k % 256 == 0 */
void orc_quantize_q8_0(const float *x, int64_t k, int8_t *q0, float *d0, int32_t *s0);
void orc_quantize_q8_k(const float *x, int64_t k, int8_t *qK, float *dK, int32_t *bsK);

/* ---- integer per-group dot sums of one matrix against one quantized activation row.
 * Group = the weight type's scale group: Q8_0 32, FP4 16 (two per block), FAST 32, Q4_K 32 (sub-block),
 * Q6_K 16. Q4_K / Q6_K dot the raw levels (0..15 / 0..63) before any offset. out[N][K / group]. */
int orc_group_size(int type);
int orc_block_dots(int type, const void *W, size_t row_bytes, int N, int K, const int8_t *qx, int32_t *out);
/* the exact integer of each K-quant super-block before its float scales (see oracle.c) */
int orc_unit_isum(int t, const void *W, size_t rb, int N, int K, const int8_t *qK, const int32_t *bsK, int32_t *out);

/* ---- matvec y[N] = W x_q with the activation's quantized form (q0/d0 for Q8_0-activation types,
 * qK/dK/bsK for K-quants). The float order is the reference CPU path's (sequential over blocks,
 * per-block terms as the int8 kernels form them). mag[n] (optional) = sum over blocks of the absolute
 * values of the block terms; ref[n] (optional) = double sum of dequantized w x dequantized x. */
int orc_matvec(int type, const void *W, size_t row_bytes, int N, int K, const int8_t *q, const float *d,
               const int32_t *bs, float *y, double *ref, double *mag, int n_threads);

/* ---- the reference's CPU expert path (expert_cpu.cpp), scalar order */
void orc_cpu_q8_0_quantize(const float *x, int K, int8_t *q, float *d);
void orc_cpu_matvec_fp4fast_q8(const void *W, size_t row_bytes, int N, int K, const int8_t *q, const float *d,
                               float *y);
void orc_cpu_matvec_q8_q8(const void *W, size_t row_bytes, int N, int K, const int8_t *q, const float *d, float *y);
void orc_cpu_expert_ffn(const void *gate, const void *up, size_t row_bytes_gu, const void *down,
                        size_t row_bytes_d, int FE, int E, const int8_t *q, const float *d, float limit, float *out);

/* ---- MoE */
void orc_moe_router(const float *logits, int T, int n_expert, int n_used, int32_t *ids, float *wts);
int orc_moe_group(const int32_t *ids, int T, int n_used, int n_expert, int tile, int32_t *tok_rows,
                  int32_t *pair_rows, int32_t *tile_e, int32_t *tile_start, int32_t *tile_n);
void orc_moe_combine(const float *down, const float *wts, const float *shared, const float *sg, const int32_t *ids,
                     const float *es, float *out, int n_used, int n, int T);
float orc_shared_gate(const float *x, const float *w, int n);
void orc_swiglu(const float *g, const float *u, float *out, int64_t n);

/* ---- legacy gemm_act_fp4: C[M][N] = A_fp16[M][K] x deq(W)[N][K]^T, separate-plane layout */
void orc_gemm_act_fp4(const uint16_t *A, const uint8_t *W, const uint8_t *W_scales, float *C, int M, int N, int K);

#ifdef __cplusplus
}
#endif
#endif
