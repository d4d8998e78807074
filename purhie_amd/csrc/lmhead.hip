// lmhead.hip -- the split-Q8_0 copy of a float matrix and its matvec (the reference's opt-in Q8_0 LM head:
// quantize_rows_q8_0 and matvec_q8_0s, src/matvec_q.hip:3550-3602, behind qmatvec_quantize_rows_q8_0 and
// qmatvec_launch_q8_0s, src/qmatvec.cpp:369-390).
//
// Quantization: per 32 values d = amax / 127 (stored as fp16), q = roundf(x (1 / d)) with the fp32 d, as ggml's
// quantize_row_q8_0_ref (and the reference's CPU Q8_0 encoder), into a split layout: values qs [N][K], scales
// d [N][K / 32]. A half-wave holds a 32-value block; the block maximum by DPP within the half.
//
// Matvec: y[n] = sum_b isum_b (d_w[b] d_x[b]) for the Q8_0 activation (q0, d0), isum_b the exact int32 block dot
// (v_dot4). HBM-bound: K + K / 16 bytes a row. A wave per row (four a workgroup); lane l takes the blocks l, l + 64,
// ..., four in flight; its float partial accumulates in block order, the wave's partials meet in a fixed butterfly.
#include "device.h"
#include "kernels.h"

namespace pq {

namespace {

constexpr int QS_THREADS = 256;
constexpr int QS_WAVES = 4;
constexpr int QS_U = 4;  // blocks a lane has in flight

// row n of W (F32 0, F16 1, BF16 30) -> qs, d
template <int TYPE>
__global__ void __launch_bounds__(QS_THREADS) k_quant_rows_q8_0(const uint8_t *__restrict__ W, long long rb, int K,
                                                                int8_t *__restrict__ qs, uint16_t *__restrict__ d) {
    const int n = blockIdx.x;
    const uint8_t *wr = W + (long long)n * rb;
    for (int k = threadIdx.x; k < K; k += QS_THREADS) {  // (K % 256 == 0: every lane of a half-wave active)
        float x;
        if constexpr (TYPE == 0) x = ((const float *)wr)[k];
        else if constexpr (TYPE == 1) x = h2f(((const uint16_t *)wr)[k]);
        else x = __uint_as_float((uint32_t)((const uint16_t *)wr)[k] << 16);
        const float am = group_max(fabsf(x), 32);
        const float dd = am / 127.0f, id = dd != 0.0f ? 1.0f / dd : 0.0f;
        qs[(long long)n * K + k] = (int8_t)(int)roundf(x * id);
        if ((threadIdx.x & 31) == 0) d[(long long)n * (K / 32) + k / 32] = __half_as_ushort(__float2half(dd));
    }
}

__global__ void __launch_bounds__(64 * QS_WAVES) k_mv_q8_0s(const int8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                                            const int8_t *__restrict__ q8, const float *__restrict__ d8,
                                                            float *__restrict__ y, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * QS_WAVES + (threadIdx.x >> 6);
    if (row >= N) return;  // (whole waves)
    const int nb = K / 32;
    const uint8_t *wr = (const uint8_t *)(qs + (long long)row * K);
    const uint16_t *dr = d + (long long)row * nb;
    float acc = 0.0f;
    for (int b0 = lane; b0 < nb; b0 += 64 * QS_U) {
        u32x4 w[QS_U][2];
        float dw[QS_U];
#pragma unroll
        for (int u = 0; u < QS_U; ++u) {
            const int b = b0 + 64 * u < nb ? b0 + 64 * u : b0;  // (a block past the row repeats b0, not used)
            w[u][0] = ld128_nt(wr + 32LL * b);
            w[u][1] = ld128_nt(wr + 32LL * b + 16);
            dw[u] = h2f(dr[b]);
        }
#pragma unroll
        for (int u = 0; u < QS_U; ++u) {
            const int b = b0 + 64 * u;
            if (b >= nb) break;
            const int4 x0 = ((const int4 *)q8)[2 * b], x1 = ((const int4 *)q8)[2 * b + 1];
            int s = 0;
            s = dot4((int)w[u][0].x, x0.x, s);
            s = dot4((int)w[u][0].y, x0.y, s);
            s = dot4((int)w[u][0].z, x0.z, s);
            s = dot4((int)w[u][0].w, x0.w, s);
            s = dot4((int)w[u][1].x, x1.x, s);
            s = dot4((int)w[u][1].y, x1.y, s);
            s = dot4((int)w[u][1].z, x1.z, s);
            s = dot4((int)w[u][1].w, x1.w, s);
            acc += (float)s * (dw[u] * d8[b]);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) y[row] = acc;
}

}  // namespace

hipError_t launch_quant_rows_q8_0(int type, const uint8_t *W, long long rb, int N, int K, int8_t *qs, uint16_t *d,
                                  hipStream_t stream) {
    if (N <= 0) return hipSuccess;
    switch (type) {
    case 0: hipLaunchKernelGGL((k_quant_rows_q8_0<0>), dim3((unsigned)N), dim3(QS_THREADS), 0, stream, W, rb, K, qs, d); break;
    case 1: hipLaunchKernelGGL((k_quant_rows_q8_0<1>), dim3((unsigned)N), dim3(QS_THREADS), 0, stream, W, rb, K, qs, d); break;
    case 30: hipLaunchKernelGGL((k_quant_rows_q8_0<30>), dim3((unsigned)N), dim3(QS_THREADS), 0, stream, W, rb, K, qs, d); break;
    default: return hipErrorInvalidDeviceFunction;
    }
    return hipGetLastError();
}

hipError_t launch_mv_q8_0s(const int8_t *qs, const uint16_t *d, const int8_t *q8, const float *d8, float *y, int N,
                           int K, hipStream_t stream) {
    if (N <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_mv_q8_0s, dim3((unsigned)((N + QS_WAVES - 1) / QS_WAVES)), dim3(64 * QS_WAVES), 0, stream, qs,
                       d, q8, d8, y, N, K);
    return hipGetLastError();
}

}  // namespace pq
