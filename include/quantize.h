/* quantize.h -- the weight encoders of libpurhie_qmv.so (gfx950), the drop-in for the reference's
 * src/quantize.h (aardbeiplantje/PURHIE) for the path's types: rows of any type quant_types.h decodes are
 * encoded as F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, MXFP4, NVFP4, Q4_0_ROCMFP4 or Q4_0_ROCMFP4_FAST,
 * bit-identical to the reference's CPU encoders (ggml's _ref quantizers and ROCmFPX's exhaustive UE4M3 scale
 * search). The encoding runs on the GPU; the host entry points copy the rows there and back. */
#ifndef PURHIE_QUANTIZE_H
#define PURHIE_QUANTIZE_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces src/quantize.h:21: 1 when rows can be encoded as dst_type */
int qz_supported(int dst_type);

/* replaces src/quantize.h:26-27: nrows rows of ncols values, src (src_type, host memory, rows back to back)
 * -> dst (dst_type, host memory, qt_row_size(dst_type, ncols) bytes a row). src_type == dst_type copies.
 * n_threads is accepted for the reference's signature (the work runs on the GPU). Returns 0, or -1 with a
 * message in err. */
int qz_quantize(int dst_type, void *dst, int src_type, const void *src, int64_t nrows, int64_t ncols, int n_threads,
                char *err, size_t err_len);

/* replaces src/quantize.h:30-31: the same with an importance matrix, which only the reference's IQ types use:
 * none of the types here (it is ignored) */
int qz_quantize_im(int dst_type, void *dst, int src_type, const void *src, int64_t nrows, int64_t ncols,
                   const float *imatrix, int n_threads, char *err, size_t err_len);

/* replaces src/quantize.h:33-38: FP8 e4m3fn rows (host memory) with a float32 scale per block_rows x block_cols
 * block (scale row r / block_rows of scale_cols values for source row r; src and scale start at a row that starts
 * a block): value = fp8 * scale, one rounding, then encoded as dst_type. The scale rows the call's rows use must
 * all be present. Returns 0, or -1 with a message in err. */
int qz_quantize_fp8_blocks(int dst_type, void *dst, const uint8_t *src, const float *scale, int64_t nrows, int64_t ncols,
                           int block_rows, int block_cols, int64_t scale_cols, int n_threads, char *err, size_t err_len);
float qz_fp8_e4m3_to_fp32(uint8_t v);

/* replace src/quantize.h:41-45: one row (host memory) at a time, and the scalar conversions */
void qz_row_q8_0(const float *x, void *y, int64_t n);
void qz_row_rocmfp4(const float *x, void *y, int64_t n);
void qz_row_rocmfp4_fast(const float *x, void *y, int64_t n);
uint16_t qz_fp32_to_fp16(float f);
uint16_t qz_fp32_to_bf16(float f);

/* No counterpart in the reference (a loader that keeps the weights in HBM): nrows rows of ncols fp32 values
 * in device memory -> dst_type rows in device memory, asynchronously on `stream`. hipErrorInvalidValue for a
 * type qz_supported rejects or ncols not a whole number of blocks. */
hipError_t qz_quantize_device(int dst_type, void *dst, const float *src, int64_t nrows, int64_t ncols,
                              hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
