// quantize.cpp -- the C ABI of the weight encoders (include/quantize.h): host rows go to the GPU in chunks,
// are decoded there when they are not fp32 (qt_to_float_device) and encoded by encode.hip's kernels, and come
// back. The reference's qz_quantize (src/quantize.cpp:1188-1224) runs the same encoders on CPU threads.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "kernels.h"
#include "quant_types.h"
#include "quantize.h"

namespace pq {
int encode_block_values(int type);
hipError_t launch_encode(int type, const float *x, uint8_t *y, long long nrows, long long ncols, long long row_bytes,
                         hipStream_t stream);
uint16_t host_f32_to_f16(float f);
uint16_t host_f32_to_bf16(float f);
float host_fp8_e4m3fn(uint8_t v);
hipError_t launch_fp8_blocks(const uint8_t *src, const float *scale, float *out, long long nrows, long long ncols,
                             long long r0, int block_rows, int block_cols, long long scale_cols, hipStream_t stream);
}  // namespace pq

using namespace pq;

namespace {

int fail(char *err, size_t err_len, const char *what, long long a = 0, long long b = 0) {
    if (err && err_len) snprintf(err, err_len, what, a, b);
    return -1;
}

}  // namespace

extern "C" {

int qz_supported(int t) { return encode_block_values(t) != 0; }

hipError_t qz_quantize_device(int dst_type, void *dst, const float *src, int64_t nrows, int64_t ncols,
                              hipStream_t stream) {
    const int vals = encode_block_values(dst_type);
    if (!vals || nrows < 0 || ncols <= 0 || ncols % vals || (!dst && nrows) || (!src && nrows))
        return hipErrorInvalidValue;
    return launch_encode(dst_type, src, (uint8_t *)dst, nrows, ncols, (long long)qt_row_size(dst_type, ncols), stream);
}

int qz_quantize_im(int dst_type, void *dst, int src_type, const void *src, int64_t nrows, int64_t ncols,
                   const float *imatrix, int n_threads, char *err, size_t err_len) {
    (void)imatrix;  // (only the reference's IQ types use one)
    (void)n_threads;
    const size_t src_row = qt_row_size(src_type, ncols);
    if (nrows < 0 || ncols <= 0 || !dst || !src)
        return fail(err, err_len, "quantize: bad arguments (%lld rows of %lld)", (long long)nrows, (long long)ncols);
    if (!src_row) return fail(err, err_len, "quantize: cannot decode type %lld rows of %lld", src_type, (long long)ncols);
    if (src_type == dst_type) {
        memcpy(dst, src, src_row * (size_t)nrows);
        return 0;
    }
    const size_t dst_row = qt_row_size(dst_type, ncols);
    if (!qz_supported(dst_type) || !dst_row || ncols % encode_block_values(dst_type))
        return fail(err, err_len, "quantize: cannot encode type %lld rows of %lld", dst_type, (long long)ncols);
    if (nrows == 0) return 0;
    // rows in chunks of about 16M values through device staging buffers
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(nrows, (int64_t)(16 << 20) / ncols));
    void *dsrc = nullptr, *dfl = nullptr, *ddst = nullptr;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreate(&s);
    if (e == hipSuccess) e = hipMalloc(&dsrc, src_row * (size_t)chunk);
    if (e == hipSuccess && src_type != QT_F32) e = hipMalloc(&dfl, (size_t)ncols * 4 * (size_t)chunk);
    if (e == hipSuccess) e = hipMalloc(&ddst, dst_row * (size_t)chunk);
    for (int64_t r0 = 0; e == hipSuccess && r0 < nrows; r0 += chunk) {
        const int64_t n = std::min(chunk, nrows - r0);
        e = hipMemcpyAsync(dsrc, (const uint8_t *)src + (size_t)r0 * src_row, src_row * (size_t)n,
                           hipMemcpyHostToDevice, s);
        const float *f = (const float *)dsrc;
        if (e == hipSuccess && src_type != QT_F32) {
            e = qt_to_float_device(src_type, dsrc, (float *)dfl, n * ncols, s);
            f = (const float *)dfl;
        }
        if (e == hipSuccess) e = qz_quantize_device(dst_type, ddst, f, n, ncols, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync((uint8_t *)dst + (size_t)r0 * dst_row, ddst, dst_row * (size_t)n, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    if (dsrc) (void)hipFree(dsrc);
    if (dfl) (void)hipFree(dfl);
    if (ddst) (void)hipFree(ddst);
    if (s) (void)hipStreamDestroy(s);
    if (e != hipSuccess) return fail(err, err_len, "quantize: HIP error %lld", (long long)e);
    return 0;
}

int qz_quantize(int dst_type, void *dst, int src_type, const void *src, int64_t nrows, int64_t ncols, int n_threads,
                char *err, size_t err_len) {
    return qz_quantize_im(dst_type, dst, src_type, src, nrows, ncols, nullptr, n_threads, err, err_len);
}

void qz_row_q8_0(const float *x, void *y, int64_t n) { (void)qz_quantize(QT_Q8_0, y, QT_F32, x, 1, n, 0, nullptr, 0); }

void qz_row_rocmfp4(const float *x, void *y, int64_t n) {
    (void)qz_quantize(QT_Q4_0_ROCMFP4, y, QT_F32, x, 1, n, 0, nullptr, 0);
}

void qz_row_rocmfp4_fast(const float *x, void *y, int64_t n) {
    (void)qz_quantize(QT_Q4_0_ROCMFP4_FAST, y, QT_F32, x, 1, n, 0, nullptr, 0);
}

float qz_fp8_e4m3_to_fp32(uint8_t v) { return host_fp8_e4m3fn(v); }

int qz_quantize_fp8_blocks(int dst_type, void *dst, const uint8_t *src, const float *scale, int64_t nrows, int64_t ncols,
                           int block_rows, int block_cols, int64_t scale_cols, int n_threads, char *err,
                           size_t err_len) {
    (void)n_threads;
    if (nrows < 0 || ncols <= 0 || !dst || !src || !scale || block_rows <= 0 || block_cols <= 0 ||
        scale_cols < (ncols + block_cols - 1) / block_cols)
        return fail(err, err_len, "quantize fp8: bad arguments (%lld rows of %lld)", (long long)nrows, (long long)ncols);
    const size_t dst_row = qt_row_size(dst_type, ncols);
    if (!qz_supported(dst_type) || !dst_row || ncols % encode_block_values(dst_type))
        return fail(err, err_len, "quantize fp8: cannot encode type %lld rows of %lld", dst_type, (long long)ncols);
    if (nrows == 0) return 0;
    // the scale rows the source rows use (they start a block), then the rows in chunks of about 16M values:
    // FP8 bytes -> device, value * block scale (fp32) -> the encoders -> host
    const size_t nsc = (size_t)((nrows + block_rows - 1) / block_rows) * (size_t)scale_cols;
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(nrows, (int64_t)(16 << 20) / ncols));
    void *dsc = nullptr, *dsrc = nullptr, *dfl = nullptr, *ddst = nullptr;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreate(&s);
    if (e == hipSuccess) e = hipMalloc(&dsc, nsc * 4);
    if (e == hipSuccess) e = hipMalloc(&dsrc, (size_t)ncols * (size_t)chunk);
    if (e == hipSuccess) e = hipMalloc(&dfl, (size_t)ncols * 4 * (size_t)chunk);
    if (e == hipSuccess) e = hipMalloc(&ddst, dst_row * (size_t)chunk);
    if (e == hipSuccess) e = hipMemcpyAsync(dsc, scale, nsc * 4, hipMemcpyHostToDevice, s);
    for (int64_t r0 = 0; e == hipSuccess && r0 < nrows; r0 += chunk) {
        const int64_t n = std::min(chunk, nrows - r0);
        e = hipMemcpyAsync(dsrc, src + (size_t)r0 * (size_t)ncols, (size_t)ncols * (size_t)n, hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = launch_fp8_blocks((const uint8_t *)dsrc, (const float *)dsc, (float *)dfl, n, ncols, r0, block_rows,
                                  block_cols, scale_cols, s);
        if (e == hipSuccess) e = qz_quantize_device(dst_type, ddst, (const float *)dfl, n, ncols, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync((uint8_t *)dst + (size_t)r0 * dst_row, ddst, dst_row * (size_t)n, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    for (void *p : {dsc, dsrc, dfl, ddst})
        if (p) (void)hipFree(p);
    if (s) (void)hipStreamDestroy(s);
    if (e != hipSuccess) return fail(err, err_len, "quantize fp8: HIP error %lld", (long long)e);
    return 0;
}

uint16_t qz_fp32_to_fp16(float f) { return host_f32_to_f16(f); }
uint16_t qz_fp32_to_bf16(float f) { return host_f32_to_bf16(f); }

}  // extern "C"
