// fmat.hip -- float activations over 16- and 32-bit weights (F16, BF16, F32): the decode matvec, and the MFMA
// GEMM of F16 / BF16 prefill batches (reference src/matvec_q.hip:700-1075, 3391-3547).
//
// Numerics are the reference's: F16 and BF16 weights take the activations rounded to the weight type (round to
// nearest even; F16 / BF16 is its own vec_dot_type in ggml), so every product is exact in fp32 and the kernels
// differ only in the order they sum in. BF16 weights with raw fp32 activations (qmatvec_launch_bf16f) and F32
// weights multiply in fp32.
//
// Decode (k_mv_float): one weight row per wave, four waves per workgroup; lane l takes the 8-value chunks l,
// l + 64, ... of the row (16-byte weight loads, four in flight before the arithmetic: 2.54 -> 2.85 TB/s on the
// BF16 decode set), for up to 4 tokens at once; then the wave's sum. HBM-bound: 2 (F16 / BF16) or 4 (F32)
// bytes per weight.
//
// GEMM (k_gemm_float): workgroup tile 128 weight rows x 128 tokens, four waves of 64 x 64; per 64-value stage the
// rows' 16-bit weights and the tokens' activations, rounded to 16 bits beforehand (k_round_half), go into LDS as
// they are; v_mfma_f32_16x16x32_f16 / _bf16 accumulate in fp32. The next stage's global loads are in flight during
// the MFMAs. Workgroups are numbered so that the token tiles of one weight-row tile run on the same XCD (its L2
// then fetches the weight tile once).
#include "device.h"
#include "kernels.h"

namespace pq {

namespace {

constexpr int QT_F32_ = 0, QT_F16_ = 1, QT_BF16_ = 30;

typedef _Float16 fh8 __attribute__((ext_vector_type(8)));
typedef __bf16 fb8 __attribute__((ext_vector_type(8)));
typedef float ff4 __attribute__((ext_vector_type(4)));

// fp32 -> the 16-bit type's bits, round to nearest even (BF16: on the bits, as the reference's bf16_round)
__device__ __forceinline__ uint32_t f16_bits(float v) { return __half_as_ushort(__float2half(v)); }
__device__ __forceinline__ uint32_t bf16_bits(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <int TYPE>
__device__ __forceinline__ uint32_t bits16(float v) {
    return TYPE == QT_F16_ ? f16_bits(v) : bf16_bits(v);
}

// 16-bit value (low half of w) -> float
template <int TYPE>
__device__ __forceinline__ float val16(uint32_t w) {
    return TYPE == QT_F16_ ? h2f(w & 0xffffu) : __uint_as_float(w << 16);
}

// the activation as the product sees it: rounded to the weight type (ROUND), else as it is
template <int TYPE, bool ROUND>
__device__ __forceinline__ float act(float v) {
    if constexpr (TYPE == QT_F32_ || !ROUND) return v;
    else return val16<TYPE>(bits16<TYPE>(v));
}

// ---------------------------------------------------------------- decode

constexpr int FMV_WAVES = 4;  // waves per workgroup
constexpr int FMV_RW = 1;     // weight rows per wave (4, each activation chunk rounded once for them, was slower:
                              // 7.1 -> 15.1 us on 4096 x 4096 F16, too few waves in flight)
constexpr int FMV_NT = 4;     // tokens per launch row (grid.y covers the rest)
constexpr int FMV_U = 4;      // 16-byte weight chunks a lane has in flight

// eight weights of a chunk as floats
template <int TYPE>
__device__ __forceinline__ void load8(const uint8_t *p, float (&w)[8]) {
    if constexpr (TYPE == QT_F32_) {
        const float4 a = ((const float4 *)p)[0], b = ((const float4 *)p)[1];
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
        const uint4 u = *(const uint4 *)p;
        const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w[2 * k] = val16<TYPE>(d[k]);
            w[2 * k + 1] = val16<TYPE>(d[k] >> 16);
        }
    }
}

template <int TYPE>
__device__ __forceinline__ float load1(const uint8_t *wr, int k) {
    if constexpr (TYPE == QT_F32_) return ((const float *)wr)[k];
    else return val16<TYPE>(((const uint16_t *)wr)[k]);
}

// rows row0 .. row0 + FMV_RW - 1 (those below N) of wave w = blockIdx.x * FMV_WAVES + threadIdx.x / 64
template <int TYPE, bool ROUND>
__global__ void __launch_bounds__(64 * FMV_WAVES) k_mv_float(const uint8_t *__restrict__ W, long long rb,
                                                               const float *__restrict__ x, float *__restrict__ y,
                                                               int N, int K, int T, int vec) {
    constexpr int EB = TYPE == QT_F32_ ? 4 : 2;
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * FMV_WAVES + (threadIdx.x >> 6)) * FMV_RW;
    if (row0 >= N) return;
    const int nr = min(FMV_RW, N - row0);
    const int t0 = blockIdx.y * FMV_NT, nt = min(FMV_NT, T - t0);
    const uint8_t *wr = W + (long long)row0 * rb;
    const float *xt = x + (long long)t0 * K;
    float acc[FMV_RW][FMV_NT];
#pragma unroll
    for (int r = 0; r < FMV_RW; ++r)
#pragma unroll
        for (int t = 0; t < FMV_NT; ++t) acc[r][t] = 0.0f;
    if (vec) {  // 16-byte aligned rows and activations, K % 8 == 0 (uniform)
        const int n8 = K / 8;
        // FMV_U chunks of each row in flight per lane: their weight loads are all issued before the arithmetic
        for (int i0 = lane; i0 < n8; i0 += 64 * FMV_U) {
            float w[FMV_RW][FMV_U][8];
#pragma unroll
            for (int r = 0; r < FMV_RW; ++r)
#pragma unroll
                for (int u = 0; u < FMV_U; ++u)
                    if (r < nr && i0 + 64 * u < n8) load8<TYPE>(wr + r * rb + (long long)EB * 8 * (i0 + 64 * u), w[r][u]);
#pragma unroll
            for (int u = 0; u < FMV_U; ++u) {
                const int i = i0 + 64 * u;
                if (i >= n8) break;
#pragma unroll
                for (int t = 0; t < FMV_NT; ++t)
                    if (t < nt) {
                        const float4 *xv = (const float4 *)(xt + (long long)t * K) + 2 * i;
                        const float4 a = xv[0], b = xv[1];
                        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                        for (int r = 0; r < FMV_RW; ++r)
                            if (r < nr) {
                                float s = acc[r][t];
#pragma unroll
                                for (int k = 0; k < 8; ++k) s = __builtin_fmaf(w[r][u][k], act<TYPE, ROUND>(xs[k]), s);
                                acc[r][t] = s;
                            }
                    }
            }
        }
    } else {
        for (int k = lane; k < K; k += 64) {
            float xa[FMV_NT];
#pragma unroll
            for (int t = 0; t < FMV_NT; ++t) xa[t] = t < nt ? act<TYPE, ROUND>(xt[(long long)t * K + k]) : 0.0f;
#pragma unroll
            for (int r = 0; r < FMV_RW; ++r)
                if (r < nr) {
                    const float w = load1<TYPE>(wr + r * rb, k);
#pragma unroll
                    for (int t = 0; t < FMV_NT; ++t)
                        if (t < nt) acc[r][t] = __builtin_fmaf(w, xa[t], acc[r][t]);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < FMV_RW; ++r)
#pragma unroll
        for (int t = 0; t < FMV_NT; ++t) {
            float a = acc[r][t];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
            if (lane == 0 && t < nt && r < nr) y[(long long)(t0 + t) * N + row0 + r] = a;
        }
}

// ---------------------------------------------------------------- GEMM

constexpr int GF_N = 128, GF_T = 128, GF_K = 64;
constexpr int GF_ROW = GF_K + 8;  // 16-bit values per LDS row (16 bytes of padding: conflict-free b128 reads)

template <int TYPE>
__device__ __forceinline__ ff4 mfma16(const uint4 a, const uint4 b, ff4 c) {
    if constexpr (TYPE == QT_F16_)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(fh8, a), __builtin_bit_cast(fh8, b), c, 0, 0,
                                                      0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(fb8, a), __builtin_bit_cast(fb8, b), c, 0, 0,
                                                       0);
}

// the activations: xh, 16-bit values of the weight type, or (XF) the fp32 x, rounded to them while staging. Wave w
// computes weight rows 64 (w & 1) .. + 63 x tokens 64 (w >> 1) .. + 63 (4 x 4 MFMA tiles). (A 256 x 128 tile with
// 128 x 64 waves reads fewer LDS bytes per MFMA but was slower: half the workgroups, and one weight row per thread
// coalesces badly; measured 99 -> 154 us on 4096 x 4096 x 2048.)
template <int TYPE, bool XF>
__global__ void __launch_bounds__(256, 2) k_gemm_float(const uint8_t *__restrict__ W, long long rb,
                                                       const void *__restrict__ xv, float *__restrict__ y, int N,
                                                       int K, int T) {
    __shared__ __attribute__((aligned(16))) uint16_t sW[GF_N * GF_ROW];
    __shared__ __attribute__((aligned(16))) uint16_t sX[GF_T * GF_ROW];

    // tile order: the grid's workgroups go round-robin over the 8 XCDs; renumber them so that XCD c runs a
    // contiguous range of tiles, in which the token tiles of a row tile are adjacent
    const int ntt = (T + GF_T - 1) / GF_T, nwg = gridDim.x;
    int b = blockIdx.x;
    if (nwg % 8 == 0) b = (b % 8) * (nwg / 8) + b / 8;
    const int t0 = (b % ntt) * GF_T, n0 = (b / ntt) * GF_N;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = (wave & 1) * 64, wt = (wave >> 1) * 64;

    // staging: thread t copies values 32 (t & 1) .. + 31 of the stage for weight row t / 2 and token t / 2
    const int sr = tid >> 1, sp = 32 * (tid & 1);
    const bool wok = n0 + sr < N, xok = t0 + sr < T;
    const uint8_t *wsrc = W + (long long)(wok ? n0 + sr : 0) * rb + 2 * sp;
    const long long xoff = (long long)(xok ? t0 + sr : 0) * K + sp;
    const uint16_t *hsrc = (const uint16_t *)xv + xoff;
    const float *fsrc = (const float *)xv + xoff;

    uint4 gw[4], gx[4];
    float4 fx[XF ? 8 : 1];
    auto issue = [&](int k0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bool in = k0 + sp + 8 * c < K;
            gw[c] = wok && in ? *(const uint4 *)(wsrc + 2 * (long long)(k0 + 8 * c)) : make_uint4(0, 0, 0, 0);
            if constexpr (XF) {
                const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                fx[2 * c] = xok && in ? *(const float4 *)(fsrc + k0 + 8 * c) : z;
                fx[2 * c + 1] = xok && in ? *(const float4 *)(fsrc + k0 + 8 * c + 4) : z;
            } else {
                gx[c] = xok && in ? *(const uint4 *)(hsrc + k0 + 8 * c) : make_uint4(0, 0, 0, 0);
            }
        }
    };

    ff4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = ff4{0.0f, 0.0f, 0.0f, 0.0f};

    issue(0);
    for (int k0 = 0; k0 < K; k0 += GF_K) {
        __syncthreads();  // the previous stage's LDS reads are done
        uint4 *dw = (uint4 *)(sW + sr * GF_ROW + sp);
        uint4 *dx = (uint4 *)(sX + sr * GF_ROW + sp);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            dw[c] = gw[c];
            if constexpr (XF) {
                const float4 a = fx[2 * c], b = fx[2 * c + 1];
                dx[c] = make_uint4(bits16<TYPE>(a.x) | bits16<TYPE>(a.y) << 16,
                                   bits16<TYPE>(a.z) | bits16<TYPE>(a.w) << 16,
                                   bits16<TYPE>(b.x) | bits16<TYPE>(b.y) << 16,
                                   bits16<TYPE>(b.z) | bits16<TYPE>(b.w) << 16);
            } else {
                dx[c] = gx[c];
            }
        }
        __syncthreads();
        if (k0 + GF_K < K) issue(k0 + GF_K);  // next stage's loads in flight during the MFMAs

#pragma unroll
        for (int s = 0; s < GF_K / 32; ++s) {
            const int kk = 32 * s + 8 * (lane >> 4);
            uint4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[i] = *(const uint4 *)(sW + (wn + 16 * i + (lane & 15)) * GF_ROW + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *(const uint4 *)(sX + (wt + 16 * j + (lane & 15)) * GF_ROW + kk);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<TYPE>(fa[i], fb[j], acc[i][j]);
        }
    }

    // lane holds weight rows 4 (lane / 16) .. + 3 of each 16 x 16 tile for token column lane % 16
    const bool v4 = ((N & 3) | ((uintptr_t)y & 15)) == 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = t0 + wt + 16 * j + (lane & 15);
        if (t >= T) continue;
        float *yr = y + (long long)t * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + wn + 16 * i + 4 * (lane >> 4);
            if (v4 && n + 3 < N) {
                *(float4 *)(yr + n) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) yr[n + r] = acc[i][j][r];
            }
        }
    }
}

// x -> its 16-bit rounding, 8 values per thread
template <int TYPE>
__global__ void __launch_bounds__(256) k_round_half(const float4 *__restrict__ x, uint4 *__restrict__ xh, long long n8) {
    const long long j = (long long)blockIdx.x * 256 + threadIdx.x;
    if (j >= n8) return;
    const float4 a = x[2 * j], b = x[2 * j + 1];
    xh[j] = make_uint4(bits16<TYPE>(a.x) | bits16<TYPE>(a.y) << 16, bits16<TYPE>(a.z) | bits16<TYPE>(a.w) << 16,
                       bits16<TYPE>(b.x) | bits16<TYPE>(b.y) << 16, bits16<TYPE>(b.z) | bits16<TYPE>(b.w) << 16);
}

template <int TYPE, bool ROUND>
hipError_t mv_float_t(const uint8_t *W, long long rb, const float *x, float *y, int N, int K, int T, hipStream_t s) {
    const int vec = ((((uintptr_t)W | (uintptr_t)rb | (uintptr_t)x) & 15) == 0 && K % 8 == 0) ? 1 : 0;
    constexpr int RPW = FMV_WAVES * FMV_RW;  // rows per workgroup
    const dim3 grid((unsigned)((N + RPW - 1) / RPW), (unsigned)((T + FMV_NT - 1) / FMV_NT));
    hipLaunchKernelGGL((k_mv_float<TYPE, ROUND>), grid, dim3(64 * FMV_WAVES), 0, s, W, rb, x, y, N, K, T, vec);
    return hipGetLastError();
}

template <int TYPE, bool XF>
hipError_t gemm_float_t(const uint8_t *W, long long rb, const void *x, float *y, int N, int K, int T, hipStream_t s) {
    const long long n = (long long)((N + GF_N - 1) / GF_N) * ((T + GF_T - 1) / GF_T);
    if (n > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm_float<TYPE, XF>), dim3((unsigned)n), dim3(256), 0, s, W, rb, x, y, N, K, T);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_mv_float(int type, bool round, const uint8_t *W, long long rb, const float *x, float *y, int N, int K,
                           int T, hipStream_t stream) {
    switch (type) {
    case QT_F32_: return mv_float_t<QT_F32_, false>(W, rb, x, y, N, K, T, stream);
    case QT_F16_: return mv_float_t<QT_F16_, true>(W, rb, x, y, N, K, T, stream);
    case QT_BF16_:
        return round ? mv_float_t<QT_BF16_, true>(W, rb, x, y, N, K, T, stream)
                     : mv_float_t<QT_BF16_, false>(W, rb, x, y, N, K, T, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

hipError_t launch_gemm_float(int type, const uint8_t *W, long long rb, const uint16_t *xh, float *y, int N, int K,
                             int T, hipStream_t stream) {
    switch (type) {
    case QT_F16_: return gemm_float_t<QT_F16_, false>(W, rb, xh, y, N, K, T, stream);
    case QT_BF16_: return gemm_float_t<QT_BF16_, false>(W, rb, xh, y, N, K, T, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

hipError_t launch_gemm_float_x(int type, const uint8_t *W, long long rb, const float *x, float *y, int N, int K,
                               int T, hipStream_t stream) {
    switch (type) {
    case QT_F16_: return gemm_float_t<QT_F16_, true>(W, rb, x, y, N, K, T, stream);
    case QT_BF16_: return gemm_float_t<QT_BF16_, true>(W, rb, x, y, N, K, T, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

hipError_t launch_round_half(int type, const float *x, uint16_t *xh, long long n, hipStream_t stream) {
    const long long n8 = n / 8;
    if (n8 == 0) return hipSuccess;
    const dim3 grid((unsigned)((n8 + 255) / 256));
    if (type == QT_F16_)
        hipLaunchKernelGGL(k_round_half<QT_F16_>, grid, dim3(256), 0, stream, (const float4 *)x, (uint4 *)xh, n8);
    else if (type == QT_BF16_)
        hipLaunchKernelGGL(k_round_half<QT_BF16_>, grid, dim3(256), 0, stream, (const float4 *)x, (uint4 *)xh, n8);
    else
        return hipErrorInvalidDeviceFunction;
    return hipGetLastError();
}

}  // namespace pq
