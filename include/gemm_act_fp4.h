/* gemm_act_fp4.h -- the legacy activation x FP4 GEMM of libpurhie_qmv.so (gfx950), the drop-in for the
 * reference's gemm_act_fp4 (src/gemm_act_fp4.hip:27-157), which its callers (tests/actfp4_verify.cpp:110-121,
 * tests/attn_verify.cpp:279) launch from a wave32 code object with grid (M / 16, N / 16) x 32 threads.
 *
 * C[M][N] (fp32) = A[M][K] (fp16, row-major) x Wdeq^T, W: N lines of K 4-bit Codebook10 codes (value k in byte
 * k / 2 of its line, low nibble first, sign in bit 3). W_scales_f NULL: W_scales holds one UE4M3 byte per 16
 * values of a line (fp4_common.h's decoder) and Wdeq = fp16(CB * scale); otherwise W_scales_f holds a scale and
 * a min float per 32 values (Q4_1 layout) and Wdeq = fp16(CB * scale + min). Accumulated in fp32. */
#ifndef PURHIE_GEMM_ACT_FP4_H
#define PURHIE_GEMM_ACT_FP4_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces the reference's launch of the gemm_act_fp4 kernel (src/gemm_act_fp4.hip:27-29; the kernel of that
 * name is exported too, with this library's own geometry: grid ((M + 31) / 32, (N + 31) / 32) x 64 threads).
 * K % 16 == 0 (K % 32 with W_scales_f); A 16-byte and W 4-byte aligned; device pointers; async on stream. */
hipError_t gemm_act_fp4_launch(const void *A, const unsigned char *W, const unsigned char *W_scales,
                               const float *W_scales_f, float *C, int M, int N, int K, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
