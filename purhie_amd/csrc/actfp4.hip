// actfp4.hip -- the legacy activation x FP4 GEMM, the reference's gemm_act_fp4 (src/gemm_act_fp4.hip:27-157):
// C[m][n] = sum_k A[m][k] Wdeq[n][k], A fp16 [M][K] row-major, W N lines of K 4-bit codes (value k in byte k / 2,
// low nibble first, Codebook10 with the sign in bit 3), C fp32 [M][N]. Weights are dequantized as the reference
// does, to fp16: with UE4M3 scales (one byte per 16 values, fp4_common.h's decoder, src/fp4_common.h:58-69),
// Wdeq = fp16(CB[nib] * scale); with float scales (W_scales_f: a scale and a min per 32 values, the Q4_1 layout),
// Wdeq = fp16(CB[nib] * scale + min).
//
// gfx950 form: one wave per 32 x 32 tile of C, 2 x 2 v_mfma_f32_16x16x32_f16 per 32 K-values, accumulated in
// fp32 throughout (the reference's wave32 WMMA rounds each 16-value strip's partial sum to fp16 before adding
// it up; here no partial sum is rounded to fp16). The A and weight fragments are read straight from memory:
// lane l holds A row (l & 15) and weight line (l & 15), K values 8 (l >> 4) .. + 7 of the step; values past
// M, N or K are zero.
#include <hip/hip_fp16.h>

#include "device.h"
#include "gemm_act_fp4.h"

namespace pq {

typedef _Float16 hv8 __attribute__((ext_vector_type(8)));
typedef float fv4 __attribute__((ext_vector_type(4)));

// fp4_common.h's UE4M3 decoder: exponent field = bits 3..6 (bit 7 too: (x >> 3) & 15), subnormal man / 512,
// normal (1 + man / 8) 2^(exp - 8), then halved
__device__ inline float ue4m3_common(uint32_t x) {
    const uint32_t e = (x >> 3) & 15u, m = x & 7u;
    const float raw = e == 0 ? (float)m * (1.0f / 512.0f) : __uint_as_float(((e + 119u) << 23) | (m << 20));
    return raw * 0.5f;
}

__device__ inline float codebook(uint32_t nib) {
    const float mags[8] = {0.0f, 1.0f, 2.0f, 3.0f, 4.0f, 6.0f, 8.0f, 10.0f};
    const float v = mags[nib & 7u];
    return (nib & 8u) ? -v : v;
}

}  // namespace pq

using namespace pq;

extern "C" __global__ void __launch_bounds__(64) gemm_act_fp4(const __half *A, const unsigned char *W,
                                                              const unsigned char *W_scales, const float *W_scales_f,
                                                              float *C, int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int m0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
    const int r = lane & 15, kq = 8 * (lane >> 4);
    const long long wrow = (long long)K / 2;
    fv4 acc[2][2] = {};
    for (int k0 = 0; k0 < K; k0 += 32) {
        const int kk = k0 + kq;  // this lane's 8 K positions: kk .. kk + 7 (K % 16 == 0: all or none past K)
        const bool kin = kk < K;
        hv8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = m0 + 16 * i + r;
            if (kin && m < M) {
                const uint4 v = *(const uint4 *)((const _Float16 *)A + (long long)m * K + kk);
                a[i] = __builtin_bit_cast(hv8, v);
            } else {
                a[i] = hv8{};
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + 16 * j + r;
            hv8 v = {};
            if (kin && n < N) {
                const uint32_t q = *(const uint32_t *)(W + n * wrow + kk / 2);
                if (!W_scales_f) {
                    const float s = ue4m3_common(W_scales[(long long)n * (K / 16) + kk / 16]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = (_Float16)(codebook((q >> (4 * e)) & 15u) * s);
                } else {
                    const float *f = W_scales_f + ((long long)n * (K / 32) + kk / 32) * 2;
                    const float s = f[0], mn = f[1];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = (_Float16)__builtin_fmaf(codebook((q >> (4 * e)) & 15u), s, mn);
                }
            }
            b[j] = v;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    // lane holds C rows 4 (lane / 16) .. + 3 of each 16 x 16 tile, column lane % 16
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + 16 * j + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + 16 * i + 4 * (lane >> 4) + e;
                if (m < M && n < N) C[(long long)m * N + n] = acc[i][j][e];
            }
        }
}

extern "C" hipError_t gemm_act_fp4_launch(const void *A, const unsigned char *W, const unsigned char *W_scales,
                                          const float *W_scales_f, float *C, int M, int N, int K, hipStream_t stream) {
    if (!A || !W || !C || M < 0 || N < 0 || K <= 0 || K % 16 || (!W_scales_f && !W_scales) ||
        (W_scales_f && K % 32) || ((uintptr_t)A & 15) || ((uintptr_t)W & 3))
        return hipErrorInvalidValue;
    if (M == 0 || N == 0) return hipSuccess;
    const dim3 grid((unsigned)((M + 31) / 32), (unsigned)((N + 31) / 32));
    hipLaunchKernelGGL(gemm_act_fp4, grid, dim3(64), 0, stream, (const __half *)A, W, W_scales, W_scales_f, C, M, N,
                       K);
    return hipGetLastError();
}
