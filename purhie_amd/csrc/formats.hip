// formats.hip -- GGUF block decoders on the GPU and the quant_types C ABI (include/quant_types.h).
//
// The decoders follow the reference's src/quant_types.cpp:182-382 value for value (the float products
// in the same order: Q4_K d * sc then * q minus dmin * m; Q6_K (d * sc) * (q - 32); FP4 CB * s), one
// thread per 32 values (Q8_0 / FP4 / FAST) or per 32-value sub-block of a super-block (K-quants).
#include "../../include/quant_types.h"
#include "device.h"

#include <string.h>

namespace pq {

__device__ __forceinline__ float rd16(const uint8_t *p) { return h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

__global__ void k_dequant(int type, const uint8_t *__restrict__ src, float *__restrict__ y, long long ngroups) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ngroups) return;
    float *o = y + g * 32;
    switch (type) {
    case TY_Q8_0: {
        const uint8_t *b = src + g * 34;
        const float d = rd16(b);
        for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)b[2 + j] * d;
        break;
    }
    case TY_FP4: {
        const uint8_t *b = src + g * 18;
        const float d0 = ue4m3_half(b[16]), d1 = ue4m3_half(b[17]);
        for (int j = 0; j < 16; ++j) {
            o[j] = (float)(int8_t)(fp4x4(b[j] & 0xfu) & 0xffu) * d0;
            o[j + 16] = (float)(int8_t)(fp4x4(b[j] >> 4) & 0xffu) * d1;
        }
        break;
    }
    case TY_FAST: {
        const uint8_t *b = src + g * 17;
        const float d = ue4m3_half(b[16]);
        for (int j = 0; j < 16; ++j) {
            o[j] = (float)(int8_t)(fp4x4(b[j] & 0xfu) & 0xffu) * d;
            o[j + 16] = (float)(int8_t)(fp4x4(b[j] >> 4) & 0xffu) * d;
        }
        break;
    }
    case TY_Q4_K: {
        const uint8_t *b = src + (g >> 3) * 144;
        const int j = (int)(g & 7);
        const uint32_t sc3[3] = {*(const uint32_t *)(b + 4), *(const uint32_t *)(b + 8), *(const uint32_t *)(b + 12)};
        int sc, mn;
        k4_scale_min(sc3, j, sc, mn);
        const float d1 = rd16(b) * (float)sc, m1 = rd16(b + 2) * (float)mn;
        const uint8_t *q = b + 16 + 32 * (j >> 1);
        for (int l = 0; l < 32; ++l) o[l] = d1 * (float)((j & 1) ? (q[l] >> 4) : (q[l] & 0xf)) - m1;
        break;
    }
    case TY_Q5_K: {  // Q4_K's nibble plus bit 2 (j / 2) + (j & 1) of qh byte l as bit 4 (src/quant_types.cpp:290-314)
        const uint8_t *b = src + (g >> 3) * 176;
        const int j = (int)(g & 7);
        const uint32_t sc3[3] = {*(const uint32_t *)(b + 4), *(const uint32_t *)(b + 8), *(const uint32_t *)(b + 12)};
        int sc, mn;
        k4_scale_min(sc3, j, sc, mn);
        const float d1 = rd16(b) * (float)sc, m1 = rd16(b + 2) * (float)mn;
        const uint8_t *q = b + 48 + 32 * (j >> 1);
        for (int l = 0; l < 32; ++l) {
            const int lv = ((j & 1) ? (q[l] >> 4) : (q[l] & 0xf)) | (((b[16 + l] >> j) & 1) << 4);
            o[l] = d1 * (float)lv - m1;
        }
        break;
    }
    case TY_IQ4_XS: {  // (d * (ls - 32)) * level (src/quant_types.cpp:111-125)
        const uint8_t *b = src + (g >> 3) * 136;
        const int j = (int)(g & 7);
        const uint32_t sh = (uint32_t)b[2] | ((uint32_t)b[3] << 8), sl = *(const uint32_t *)(b + 4);
        const float dl = rd16(b) * (float)iq4xs_scale(sh, sl, j);
        const uint8_t *q = b + 8 + 16 * j;
        for (int i = 0; i < 16; ++i) {
            o[i] = dl * (float)(int8_t)(iq4nl4(q[i] & 0xfu) & 0xff);
            o[i + 16] = dl * (float)(int8_t)(iq4nl4(q[i] >> 4) & 0xff);
        }
        break;
    }
    case TY_MXFP4: {  // E8M0 scale, then FAST's value bytes (src/quant_types.cpp:397-407)
        const uint8_t *b = src + g * 17;
        const float d = e8m0_half(b[0]);
        for (int j = 0; j < 16; ++j) {
            o[j] = (float)fp4_level<12>(b[1 + j] & 0xfu) * d;
            o[j + 16] = (float)fp4_level<12>(b[1 + j] >> 4) * d;
        }
        break;
    }
    case TY_NVFP4: {  // half (g & 1) of a 64-value block: sub-blocks 2h, 2h + 1 (src/quant_types.cpp:409-422)
        const uint8_t *b = src + (g >> 1) * 36;
        const int s0 = 2 * (int)(g & 1);
        for (int s = s0; s < s0 + 2; ++s) {
            const float d = nv_scale(b[s]);
            const uint8_t *q = b + 4 + 8 * s;
            float *os = o + 16 * (s - s0);
            for (int j = 0; j < 8; ++j) {
                os[j] = (float)fp4_level<12>(q[j] & 0xfu) * d;
                os[j + 8] = (float)fp4_level<12>(q[j] >> 4) * d;
            }
        }
        break;
    }
    case TY_Q6_K: {
        const uint8_t *b = src + (g >> 3) * 210;
        const int part = (int)(g & 7);  // values 32 part .. 32 part + 31
        const float d = rd16(b + 208);
        const int8_t *scs = (const int8_t *)(b + 192);
        for (int l2 = 0; l2 < 32; ++l2) {
            const int v = 32 * part + l2, h = v >> 7, jj = (v >> 5) & 3, l = v & 31;
            const uint8_t ql = b[64 * h + l + 32 * (jj & 1)], qh = b[128 + 32 * h + l];
            const int lv = ((jj >= 2) ? (ql >> 4) : (ql & 0xf)) | (((qh >> (2 * jj)) & 3) << 4);
            o[l2] = d * (float)scs[v >> 4] * (float)(lv - 32);
        }
        break;
    }
    case QT_F16: {
        const uint8_t *b = src + g * 64;
        for (int j = 0; j < 32; ++j) o[j] = rd16(b + 2 * j);
        break;
    }
    case QT_BF16: {
        const uint8_t *b = src + g * 64;
        for (int j = 0; j < 32; ++j) o[j] = __uint_as_float(((uint32_t)b[2 * j] | ((uint32_t)b[2 * j + 1] << 8)) << 16);
        break;
    }
    case QT_F32: {
        const float *b = (const float *)(src + g * 128);
        for (int j = 0; j < 32; ++j) o[j] = b[j];
        break;
    }
    }
}

}  // namespace pq

using namespace pq;

namespace {

void to_float_sync_q8_0(const void *s, float *d, int64_t n) { (void)qt_to_float(TY_Q8_0, s, d, n); }
void to_float_sync_q4_k(const void *s, float *d, int64_t n) { (void)qt_to_float(TY_Q4_K, s, d, n); }
void to_float_sync_q5_k(const void *s, float *d, int64_t n) { (void)qt_to_float(TY_Q5_K, s, d, n); }
void to_float_sync_q6_k(const void *s, float *d, int64_t n) { (void)qt_to_float(TY_Q6_K, s, d, n); }
void to_float_sync_iq4_xs(const void *s, float *d, int64_t n) { (void)qt_to_float(TY_IQ4_XS, s, d, n); }
void to_float_sync_fp4(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_Q4_0_ROCMFP4, s, d, n); }
void to_float_sync_fast(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_Q4_0_ROCMFP4_FAST, s, d, n); }
void to_float_sync_mxfp4(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_MXFP4, s, d, n); }
void to_float_sync_nvfp4(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_NVFP4, s, d, n); }
void to_float_sync_f32(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_F32, s, d, n); }
void to_float_sync_f16(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_F16, s, d, n); }
void to_float_sync_bf16(const void *s, float *d, int64_t n) { (void)qt_to_float(QT_BF16, s, d, n); }

// replaces the table of src/quant_types.cpp:586-615 for the path's types
const qt_traits k_traits[] = {
    {QT_F32, "f32", 1, 4, to_float_sync_f32, 1},
    {QT_F16, "f16", 1, 2, to_float_sync_f16, 1},
    {TY_Q8_0, "q8_0", 32, 34, to_float_sync_q8_0, 1},
    {TY_Q4_K, "q4_K", 256, 144, to_float_sync_q4_k, 1},
    {TY_Q5_K, "q5_K", 256, 176, to_float_sync_q5_k, 1},
    {TY_Q6_K, "q6_K", 256, 210, to_float_sync_q6_k, 1},
    {TY_IQ4_XS, "iq4_xs", 256, 136, to_float_sync_iq4_xs, 1},
    {QT_BF16, "bf16", 1, 2, to_float_sync_bf16, 1},
    {QT_MXFP4, "mxfp4", 32, 17, to_float_sync_mxfp4, 1},
    {QT_NVFP4, "nvfp4", 64, 36, to_float_sync_nvfp4, 1},
    {QT_Q4_0_ROCMFP4, "q4_0_rocmfp4", 32, 18, to_float_sync_fp4, 1},
    {QT_Q4_0_ROCMFP4_FAST, "q4_0_rocmfp4_fast", 32, 17, to_float_sync_fast, 1},
};

bool is_device_ptr(const void *p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

}  // namespace

extern "C" {

const qt_traits *qt_get_traits(int type) {
    for (const qt_traits &t : k_traits)
        if (t.type == type) return &t;
    return nullptr;
}

size_t qt_row_size(int type, int64_t ne0) {
    const qt_traits *t = qt_get_traits(type);
    if (!t || ne0 <= 0 || ne0 % t->blck_size != 0) return 0;
    return (size_t)(ne0 / t->blck_size) * (size_t)t->type_size;
}

int qt_vec_dot_q8k(int type) { return type == TY_Q4_K || type == TY_Q5_K || type == TY_Q6_K || type == TY_IQ4_XS; }

float qt_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float v = (float)m * 0x1p-24f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float qt_bf16_to_fp32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

hipError_t qt_to_float_device(int type, const void *src, float *dst, int64_t n, hipStream_t stream) {
    const qt_traits *t = qt_get_traits(type);
    if (!t || n < 0 || n % t->blck_size != 0 || n % 32 != 0) return hipErrorInvalidValue;
    const long long ng = n / 32;
    if (ng == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, stream, type,
                       (const uint8_t *)src, dst, ng);
    return hipGetLastError();
}

int qt_to_float(int type, const void *src, float *dst, int64_t n) {
    const qt_traits *t = qt_get_traits(type);
    if (!t || n % t->blck_size != 0 || n % 32 != 0) return -1;
    if (n == 0) return 0;
    const size_t in_bytes = (size_t)(n / t->blck_size) * (size_t)t->type_size, out_bytes = (size_t)n * 4;
    const bool dsrc = is_device_ptr(src), ddst = is_device_ptr(dst);
    void *s = (void *)src;
    float *d = dst;
    if (!dsrc && hipMalloc(&s, in_bytes) != hipSuccess) return -1;
    if (!ddst && hipMalloc((void **)&d, out_bytes) != hipSuccess) {
        if (!dsrc) (void)hipFree(s);
        return -1;
    }
    hipError_t e = hipSuccess;
    if (!dsrc) e = hipMemcpy(s, src, in_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = qt_to_float_device(type, s, d, n, 0);
    if (e == hipSuccess && !ddst) e = hipMemcpy(dst, d, out_bytes, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (!dsrc) (void)hipFree(s);
    if (!ddst) (void)hipFree(d);
    return e == hipSuccess ? 0 : -1;
}

}  // extern "C"
