/* quant_types.h -- GGUF weight block formats, the drop-in for the reference's src/quant_types.h
 * (aardbeiplantje/PURHIE). Same type ids, traits table fields, row sizes and return conventions.
 *
 * Block maps of the path's types (little-endian, unchanged on-disk GGUF layout):
 *   Q8_0  (8)    34 B / 32:  fp16 d @0, int8 qs[32] @2                        value = q * d
 *   Q4_K  (12)  144 B / 256: fp16 d @0, fp16 dmin @2, scales[12] @4, qs[128] @16   value = d*sc_j*q - dmin*m_j
 *   Q6_K  (14)  210 B / 256: ql[128] @0, qh[64] @128, int8 sc[16] @192, fp16 d @208  value = d*sc_g*(q - 32)
 *   Q4_0_ROCMFP4      (100) 18 B / 32: qs[16] @0, e0 @16, e1 @17 (UE4M3, one per 16 values)
 *   Q4_0_ROCMFP4_FAST (101) 17 B / 32: qs[16] @0, e @16
 *     FP4 value j < 16 = CB[low nibble of byte j] * s, j >= 16 = CB[high nibble of byte j - 16] * s,
 *     CB = {0,1,2,3,4,6,8,10,-0,-1,-2,-3,-4,-6,-8,-10}, s = ue4m3_half(e) (bytes >= 0x7F decode to 0).
 *
 * Decoding (qt_to_float) runs on the GPU: qt_to_float_device launches it on device buffers; the
 * reference-compatible qt_to_float takes host or device pointers and returns when done.
 */
#ifndef PURHIE_QUANT_TYPES_H
#define PURHIE_QUANT_TYPES_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces src/quant_types.h:19-48 (the ids of the path's types and the float types) */
enum qt_type {
    QT_F32 = 0,
    QT_F16 = 1,
    QT_Q8_0 = 8,
    QT_Q4_K = 12,
    QT_Q5_K = 13,
    QT_Q6_K = 14,
    QT_IQ4_XS = 23,
    QT_BF16 = 30,
    QT_MXFP4 = 39,
    QT_NVFP4 = 40,
    QT_Q4_0_ROCMFP4 = 100,
    QT_Q4_0_ROCMFP4_FAST = 101,
};

typedef void (*qt_to_float_fn)(const void *src, float *dst, int64_t n);

/* replaces src/quant_types.h:52-59 */
typedef struct {
    int type;
    const char *name;
    int blck_size;
    int type_size;
    qt_to_float_fn to_float; /* host or device pointers; synchronous */
    int verified;            /* 1 = bit-exact against the reference's decoder (tests/test_gpu_formats.py) */
} qt_traits;

/* replaces src/quant_types.h:62-76 */
const qt_traits *qt_get_traits(int type);
size_t qt_row_size(int type, int64_t ne0);
int qt_to_float(int type, const void *src, float *dst, int64_t n);
int qt_vec_dot_q8k(int type);
float qt_fp16_to_fp32(uint16_t h);
float qt_bf16_to_fp32(uint16_t h);

/* No counterpart in the reference (its decoders are CPU-only): decode n values of device memory src
 * into device memory dst on stream, asynchronously. Returns hipErrorInvalidValue for an unsupported
 * type or n not a multiple of the block size. */
hipError_t qt_to_float_device(int type, const void *src, float *dst, int64_t n, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PURHIE_QUANT_TYPES_H */
