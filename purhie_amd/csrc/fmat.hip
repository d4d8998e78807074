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
// GEMM (k_gemm_float): workgroup tile 128 or 256 weight rows x 128 tokens, waves of 64 x 64; per stage the rows'
// 16-bit weights and the tokens' activations, rounded to 16 bits beforehand (k_round_half), go into LDS as they are;
// v_mfma_f32_16x16x32_f16 / _bf16 accumulate in fp32. Two LDS buffers with one barrier a stage, and each stage's
// global loads (raw buffer loads, zeros past K) issued two stages ahead. Workgroups are numbered XCD by XCD, in
// groups of token tiles that advance together over the row tiles (the XCD's L2 then holds their activations while
// the weights stream).
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

// rows row0 .. row0 + FMV_RW - 1 (those below N) of wave w = blockIdx.x * FMV_WAVES + threadIdx.x / 64.
// stage (vec only): the workgroup's nt tokens, as the products see them (act), go to LDS first, so the 4 waves read
// them there instead of each loading them from global memory (the activation was as many bytes as a row's weights:
// the loads, not the arithmetic, bound the kernel). The weight chunks a lane has in flight are loaded whether or not
// they are past the row's end (a past chunk reloads the last one and adds nothing): the loads have no branch around
// them, so the waits count them exactly. Every lane adds its chunks in the same order in every form: the same bits.
template <int TYPE, bool ROUND>
__global__ void __launch_bounds__(64 * FMV_WAVES) k_mv_float(const uint8_t *__restrict__ W, long long rb,
                                                               const float *__restrict__ x, float *__restrict__ y,
                                                               int N, int K, int T, int vec, int stage) {
    constexpr int EB = TYPE == QT_F32_ ? 4 : 2;
    extern __shared__ __attribute__((aligned(16))) float sx[];
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * FMV_WAVES + (threadIdx.x >> 6)) * FMV_RW;
    const int t0 = blockIdx.y * FMV_NT, nt = min(FMV_NT, T - t0);
    const float *xt = x + (long long)t0 * K;
    if (stage) {  // (uniform; every wave of the workgroup, before any returns)
        const int n4 = nt * K / 4;
        for (int j = threadIdx.x; j < n4; j += 64 * FMV_WAVES) {
            const float4 v = ((const float4 *)xt)[j];
            ((float4 *)sx)[j] = make_float4(act<TYPE, ROUND>(v.x), act<TYPE, ROUND>(v.y), act<TYPE, ROUND>(v.z),
                                            act<TYPE, ROUND>(v.w));
        }
        __syncthreads();
    }
    if (row0 >= N) return;
    const int nr = min(FMV_RW, N - row0);
    const uint8_t *wr = W + (long long)row0 * rb;
    float acc[FMV_RW][FMV_NT];
#pragma unroll
    for (int r = 0; r < FMV_RW; ++r)
#pragma unroll
        for (int t = 0; t < FMV_NT; ++t) acc[r][t] = 0.0f;
    if (vec) {  // 16-byte aligned rows and activations, K % 8 == 0 (uniform)
        const int n8 = K / 8;
        // FMV_U chunks of each row in flight per lane: their weight loads are all issued before the arithmetic
        for (int c0 = 0; c0 < n8; c0 += 64 * FMV_U) {
            float w[FMV_RW][FMV_U][8];
#pragma unroll
            for (int r = 0; r < FMV_RW; ++r)
#pragma unroll
                for (int u = 0; u < FMV_U; ++u) {
                    const int i = c0 + lane + 64 * u;
                    load8<TYPE>(wr + (r < nr ? r : 0) * rb + (long long)EB * 8 * (i < n8 ? i : n8 - 1), w[r][u]);
                }
#pragma unroll
            for (int u = 0; u < FMV_U; ++u) {
                const int i = c0 + lane + 64 * u;
                if (i >= n8) break;
#pragma unroll
                for (int t = 0; t < FMV_NT; ++t)
                    if (t < nt) {
                        float xs[8];
                        if (stage) {
                            const float4 a = ((const float4 *)(sx + t * K))[2 * i], b = ((const float4 *)(sx + t * K))[2 * i + 1];
                            xs[0] = a.x; xs[1] = a.y; xs[2] = a.z; xs[3] = a.w; xs[4] = b.x; xs[5] = b.y; xs[6] = b.z; xs[7] = b.w;
                        } else {
                            const float4 *xv = (const float4 *)(xt + (long long)t * K) + 2 * i;
                            const float4 a = xv[0], b = xv[1];
                            xs[0] = act<TYPE, ROUND>(a.x); xs[1] = act<TYPE, ROUND>(a.y);
                            xs[2] = act<TYPE, ROUND>(a.z); xs[3] = act<TYPE, ROUND>(a.w);
                            xs[4] = act<TYPE, ROUND>(b.x); xs[5] = act<TYPE, ROUND>(b.y);
                            xs[6] = act<TYPE, ROUND>(b.z); xs[7] = act<TYPE, ROUND>(b.w);
                        }
#pragma unroll
                        for (int r = 0; r < FMV_RW; ++r)
                            if (r < nr) {
                                float s = acc[r][t];
#pragma unroll
                                for (int k = 0; k < 8; ++k) s = __builtin_fmaf(w[r][u][k], xs[k], s);
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

constexpr int GF_T = 128;    // tokens of a workgroup tile (its weight rows: 128 or 256)
constexpr int GF_GROUP = 4;  // token tiles advancing together over the row tiles on an XCD (xcd_tile)
constexpr int GF_PD = 2;     // prefetch distance (stages)

template <int TYPE>
__device__ __forceinline__ ff4 mfma16(const uint4 a, const uint4 b, ff4 c) {
    if constexpr (TYPE == QT_F16_)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(fh8, a), __builtin_bit_cast(fh8, b), c, 0, 0,
                                                      0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(fb8, a), __builtin_bit_cast(fb8, b), c, 0, 0,
                                                       0);
}

// LDS place (bytes) of 16-byte chunk ch (values 8 ch .. 8 ch + 7) of row r of a stage of KS values: chunk ch of the
// 16 rows of group r / 16 lie side by side, so a fragment read (lane: row 16 i + lane % 16, chunk 4 h + lane / 16)
// and a staging store (the same map) each touch one contiguous KiB, with no bank conflict
template <int KS>
__device__ __forceinline__ int gf_at(int r, int ch) { return (r >> 4) * (32 * KS) + (ch << 8) + ((r & 15) << 4); }

template <int V>
using GfC = std::integral_constant<int, V>;

// raw buffer resource over bytes [p, p + n) (n < 2^31); a load at an offset past n returns zeros
constexpr uint32_t GF_OOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gf_rsrc(const void *p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint4 gf_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// One stage's global loads of a thread: LW weight chunks and LX token chunks (chunk c: row group c / CPR of the
// thread's, chunk 4 (c % CPR) + lane / 16 of the stage, CPR = KS / 32); XF: the fp32 activation chunks, two float4
// each
template <bool XF, int LW, int LX>
struct GfPre {
    uint4 w[LW], x[LX];
};
template <int LW, int LX>
struct GfPre<true, LW, LX> {
    uint4 w[LW];
    float4 f[2 * LX];
};

// the activations: xh, 16-bit values of the weight type, or (XF) the fp32 x, rounded to them while staging.
// Workgroup: ROWS weight rows x 128 tokens, ROWS / 32 waves; wave w computes rows 64 (w % (ROWS / 64)) .. + 63 x
// tokens 64 (w / (ROWS / 64)) .. + 63 (4 x 4 MFMA tiles). K runs in stages of KS values, double-buffered in LDS with
// one barrier a stage; every stage's global loads are issued PD stages before its LDS store, into one of PD register
// sets, and a stage past the end loads the last one again, so the steady loop has no conditions. The tiles of each
// 32 values are summed in K order, as in every form of this kernel: the outputs do not depend on the tile, the stage
// size or the pipeline.
template <int TYPE, bool XF, int ROWS, int KS, int PD, int OCC>
__global__ void __launch_bounds__(2 * ROWS, OCC) k_gemm_float(const uint8_t *__restrict__ W, long long rb,
                                                              const void *__restrict__ xv, float *__restrict__ y,
                                                              int N, int K, int T) {
    static_assert(PD == 2 || PD == 4, "prefetch distance");
    static_assert(KS == 32 || KS == 64, "stage size");
    static_assert(ROWS == 128 || ROWS == 256, "row tile");
    constexpr int NW = ROWS / 32;           // waves
    constexpr int XG = 8 / NW;              // 16-token row groups a wave stages
    constexpr int CPR = KS / 32, LW = 2 * CPR, LX = XG * CPR;
    __shared__ __attribute__((aligned(16))) uint8_t sW0[ROWS * KS * 2], sW1[ROWS * KS * 2];
    __shared__ __attribute__((aligned(16))) uint8_t sX0[GF_T * KS * 2], sX1[GF_T * KS * 2];

    int tt, rt;
    xcd_tile(tt, rt, GF_GROUP);  // grid (token tiles, row tiles), renumbered XCD by XCD
    const int t0 = tt * GF_T, n0 = rt * ROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = (wave % (ROWS / 64)) * 64, wt = (wave / (ROWS / 64)) * 64;
    const int nst = (K + KS - 1) / KS;

    // staging: weight rows 32 wave + lane % 16 (+ 16), token rows 16 XG wave + lane % 16 (+ 16), chunks sc (and
    // sc + 4), through raw buffer loads over the workgroup's row tile of W and token tile of x (rows past the end
    // repeat the last one; their outputs are not stored). A chunk past K (K % 8 == 0: a chunk is in or out whole)
    // reads at offset GF_OOB, past the buffer's range: zeros, with no branch, so the loads stay in one basic block
    // and their waits count exactly.
    constexpr uint32_t XB = XF ? 4 : 2;  // activation bytes per value
    const int sr = 32 * wave + (lane & 15), xr = 16 * XG * wave + (lane & 15), sc = lane >> 4;
    const int nr = N - n0 < ROWS ? N - n0 : ROWS, tr = T - t0 < GF_T ? T - t0 : GF_T;
    const __amdgpu_buffer_rsrc_t rw = gf_rsrc(W + (long long)n0 * rb, (uint32_t)(nr * rb));
    const __amdgpu_buffer_rsrc_t rx =
        gf_rsrc((const uint8_t *)xv + (long long)t0 * K * XB, (uint32_t)tr * (uint32_t)K * XB);
    uint32_t wb[2], xb[XG];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int n = sr + 16 * h;
        wb[h] = (uint32_t)((n < nr ? n : nr - 1) * rb) + 16u * sc;
    }
#pragma unroll
    for (int g = 0; g < XG; ++g) {
        const int t = xr + 16 * g;
        xb[g] = (uint32_t)(t < tr ? t : tr - 1) * (uint32_t)K * XB + 8u * XB * sc;
    }

    GfPre<XF, LW, LX> P[PD];
    auto issue = [&](GfPre<XF, LW, LX> &p, int s) {
        const int k0 = KS * (s < nst ? s : nst - 1);
#pragma unroll
        for (int c = 0; c < LW; ++c) {
            const int q = c % CPR;
            const bool in = k0 + 8 * (sc + 4 * q) < K;
            p.w[c] = gf_load(rw, in ? wb[c / CPR] + 2u * k0 + 64u * q : GF_OOB);
        }
#pragma unroll
        for (int c = 0; c < LX; ++c) {
            const int q = c % CPR;
            const bool in = k0 + 8 * (sc + 4 * q) < K;
            const uint32_t ox = xb[c / CPR] + XB * k0 + 32u * XB * q;
            if constexpr (XF) {
                p.f[2 * c] = __builtin_bit_cast(float4, gf_load(rx, in ? ox : GF_OOB));
                p.f[2 * c + 1] = __builtin_bit_cast(float4, gf_load(rx, in ? ox + 16u : GF_OOB));
            } else {
                p.x[c] = gf_load(rx, in ? ox : GF_OOB);
            }
        }
    };
    auto commit = [&](auto cc, const GfPre<XF, LW, LX> &p) {
        constexpr int c0 = decltype(cc)::value;
        uint8_t *sw = c0 ? sW1 : sW0, *sx = c0 ? sX1 : sX0;
#pragma unroll
        for (int c = 0; c < LW; ++c)
            *(uint4 *)(sw + gf_at<KS>(sr + 16 * (c / CPR), sc + 4 * (c % CPR))) = p.w[c];
#pragma unroll
        for (int c = 0; c < LX; ++c) {
            uint4 *d = (uint4 *)(sx + gf_at<KS>(xr + 16 * (c / CPR), sc + 4 * (c % CPR)));
            if constexpr (XF) {
                const float4 a = p.f[2 * c], b = p.f[2 * c + 1];
                *d = make_uint4(bits16<TYPE>(a.x) | bits16<TYPE>(a.y) << 16, bits16<TYPE>(a.z) | bits16<TYPE>(a.w) << 16,
                                bits16<TYPE>(b.x) | bits16<TYPE>(b.y) << 16, bits16<TYPE>(b.z) | bits16<TYPE>(b.w) << 16);
            } else {
                *d = p.x[c];
            }
        }
    };

    ff4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = ff4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](auto cc) {
        constexpr int c0 = decltype(cc)::value;
        const uint8_t *sw = c0 ? sW1 : sW0, *sx = c0 ? sX1 : sX0;
#pragma unroll
        for (int h = 0; h < CPR; ++h) {
            const int ch = 4 * h + (lane >> 4);
            uint4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[i] = *(const uint4 *)(sw + gf_at<KS>(wn + 16 * i + (lane & 15), ch));
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *(const uint4 *)(sx + gf_at<KS>(wt + 16 * j + (lane & 15), ch));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<TYPE>(fa[i], fb[j], acc[i][j]);
        }
    };

    // step s (s = s0 + u, s0 a multiple of PD): stage s is in LDS buffer s & 1 and its register set s % PD is free
    // (committed by step s - 1). Commit stage s + 1 (set (s + 1) % PD) into buffer 1 - (s & 1), whose stage s - 1
    // every wave finished before the previous barrier; issue stage s + PD into set s % PD; compute stage s.
    auto step = [&](auto uu, int s0) {
        constexpr int u = decltype(uu)::value, c = u & 1;
        commit(GfC<1 - c>{}, P[(u + 1) % PD]);
        issue(P[u % PD], s0 + u + PD);
        __builtin_amdgcn_sched_barrier(0);
        compute(GfC<c>{});
        __syncthreads();
    };

#pragma unroll
    for (int i = 0; i < PD; ++i) issue(P[i], i);
    commit(GfC<0>{}, P[0]);
    __syncthreads();
    int s = 0;
    for (; s + PD <= nst; s += PD) {
        step(GfC<0>{}, s);
        step(GfC<1>{}, s);
        if constexpr (PD == 4) {
            step(GfC<2>{}, s);
            step(GfC<3>{}, s);
        }
    }
    if (s < nst) step(GfC<0>{}, s);
    if constexpr (PD == 4) {
        if (s + 1 < nst) step(GfC<1>{}, s);
        if (s + 2 < nst) step(GfC<2>{}, s);
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
    // one token of 16-bit weights: its activation in LDS when it takes at most 48 KiB (K <= 12288; three such
    // workgroups a CU). Measured (one box, A/B): BF16 9728 x 2560 13.5 -> 10.6 us, 2560 x 9728 16.4 -> 12.5 us,
    // 151936 x 2560 160 -> 129 us, F16 4096 x 4096 7.0 -> 6.0 us; F32 (twice the weight bytes per value) 12.7 ->
    // 13.1 us and four tokens (four LDS reads per weight chunk) 23.5 -> 37.5 us, so those read x from global memory
    const long long lds = (long long)K * 4;
    const int stage = vec && T == 1 && TYPE != QT_F32_ && lds <= 49152 ? 1 : 0;
    hipLaunchKernelGGL((k_mv_float<TYPE, ROUND>), grid, dim3(64 * FMV_WAVES), stage ? (size_t)lds : 0, s, W, rb, x, y, N,
                       K, T, vec, stage);
    return hipGetLastError();
}

// Row tile: 256 rows (8 waves, stages of 32 values) read 384 rows of operands per 2 x 256 x 128 x K flop, against
// 512 for two 128-row tiles (4 waves, stages of 64 values); the kernel's loads, not its MFMAs, bound it (a timing
// copy without the steady loop's global loads ran twice as fast), so the launch lasts about as long as its busiest
// CU takes to read its tiles' rows: ceil(tiles / CUs) (ROWS + 128). The row tile that makes this smaller is taken
// (128 on a tie: twice the workgroups). Measured on BF16 9728 x 2560 x 2427: 234 -> 178 us; 4096 x 4096 x 2048:
// 122 -> 94.5 us; 9728 x 2560 x 256 stays on 128 rows (43 against 62 us).
template <int TYPE, bool XF>
hipError_t gemm_float_t(const uint8_t *W, long long rb, const void *x, float *y, int N, int K, int T, hipStream_t s) {
    const long long ntt = (T + GF_T - 1) / GF_T, ncu = device_cus();
    const long long n128 = (N + 127) / 128 * ntt, n256 = (N + 255) / 256 * ntt;
    const bool big = (n256 + ncu - 1) / ncu * 384 < (n128 + ncu - 1) / ncu * 256;
    const int rows = big ? 256 : 128;
    const long long nrt = (N + rows - 1) / rows;
    // (the raw buffers of a workgroup's row tile and token tile stay below 2^31 bytes)
    if (nrt > 65535 || nrt * ntt > 0x7fffffffLL || rows * rb >= (1LL << 31) || (long long)GF_T * K * 4 >= (1LL << 31))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)ntt, (unsigned)nrt);
    if (big)
        hipLaunchKernelGGL((k_gemm_float<TYPE, XF, 256, 32, GF_PD, 2>), grid, dim3(512), 0, s, W, rb, x, y, N, K, T);
    else
        hipLaunchKernelGGL((k_gemm_float<TYPE, XF, 128, 64, GF_PD, 2>), grid, dim3(256), 0, s, W, rb, x, y, N, K, T);
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
