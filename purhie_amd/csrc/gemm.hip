// gemm.hip -- the prefill GEMM Y[t][n] = sum_k W[n][k] X[t][k] for GGUF weights on gfx950 MFMA, and its
// MoE form over moe_group's expert tiles. Replaces the reference's matmul_wmma_<type> / matmul_q8_<type> /
// matmul_wmma_id_<type> (src/matvec_q.hip:2174-3348), whose per-32-block int32 tile sums are followed by a
// float epilogue per block.
//
// MI355X-first design (fp16 MFMA on exactly decoded operands):
//   * int8 MFMA would need a float fix-up per 16 / 32 K-values of every output (ROCmFP4 has a UE4M3 scale
//     per 16 weights, Q8_0 activations one per 32): at 32 multiply-adds per output per block the matrix
//     core outruns the vector ALU by 2-6x. Instead the ROCmFP4 weight value CB[nibble] * ue4m3(e) is exact
//     in fp16 (|CB * (8 + m)| <= 150 fits 11 bits), so the weight scale rides inside the MFMA operand and
//     v_mfma_f32_16x16x32_f16 over one 32-value block yields the reference's block term
//     c0 * e0 + c1 * e1 with exact products; one FMA per output per block applies the activation scale:
//     acc += d_x * C_block (the reference's d_x * (c0 e0 + c1 e1)).
//   * the token operand is the Q8_0 int8 activation, exact in fp16, converted once per call by a pre-pass
//     (k_act_f16) into the GEMM's K order; the weights are decoded in-kernel into LDS once per tile
//     through a 256-entry half2 table (a byte's two nibbles -> two fp16 codebook values) and a packed
//     fp16 multiply by the two half-block scales. Within a 32-block the K order is permuted so that a
//     byte's low / high nibble (values j, j + 16) land side by side; the pre-pass permutes the token
//     operand identically, so every MFMA sums the same pairs.
//   * workgroup tile 128 weight rows x 128 tokens, 4 waves of 64 x 64 (4 x 4 MFMA tiles), K stages of 128
//     (4 blocks) with the next stage's global loads in flight (registers) while the current one runs.
#include "device.h"
#include "kernels.h"

namespace pq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int GB_N = 128;           // weight rows per workgroup
constexpr int GB_T = 128;           // tokens per workgroup
constexpr int GB_K = 128;           // K per stage
constexpr int G_THREADS = 256;
constexpr int LDS_ROW = GB_K + 8;   // halves per LDS row (16 bytes of padding: conflict-free b128 reads)

// ---------------------------------------------------------------- token pre-pass
// One thread per 32-value block of one token row: int8 q -> fp16 (exact), in the weight type's K order
// (perm: position 2j <- value j, 2j + 1 <- value j + 16), plus the block scales; rows >= T (up to Tpad,
// plus one extra all-zero row used by MoE tiles) are zero.
__global__ void k_act_f16(const int8_t *__restrict__ q, const float *__restrict__ d, int T, int K, int Tpad,
                          int perm, _Float16 *__restrict__ xh, float *__restrict__ dxp) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nb = K / 32;
    if (i >= (long long)(Tpad + 1) * nb) return;
    const int t = (int)(i / nb), b = (int)(i % nb);
    _Float16 *o = xh + (long long)t * K + 32 * b;
    if (t >= T) {
        for (int j = 0; j < 32; ++j) o[j] = (_Float16)0.0f;
        dxp[i] = 0.0f;
        return;
    }
    const int8_t *s = q + (long long)t * K + 32 * b;
    for (int j = 0; j < 16; ++j) {
        const _Float16 lo = (_Float16)(float)s[j], hi = (_Float16)(float)s[j + 16];
        if (perm) {
            o[2 * j] = lo;
            o[2 * j + 1] = hi;
        } else {
            o[j] = lo;
            o[j + 16] = hi;
        }
    }
    dxp[i] = d[(long long)t * nb + b];
}

// ---------------------------------------------------------------- weight stage decoders
// Each fills rows of the LDS weight tile [GB_N][LDS_ROW] (fp16, the type's K order) for K values
// k0 .. k0 + 127, and for Q8_0 the per-row block scales sdw[4][GB_N].

// 256-entry table: byte -> half2(CB[low nibble], CB[high nibble]) (TOP: the codebook's top level)
template <int TOP = 10>
__device__ __forceinline__ void init_fp4_lut(uint32_t *lut) {
    const int b = threadIdx.x;  // blockDim == 256
    const int lo = fp4_level<TOP>(b & 15), hi = fp4_level<TOP>(b >> 4);
    h2 v;
    v.x = (_Float16)(float)lo;
    v.y = (_Float16)(float)hi;
    lut[b] = __builtin_bit_cast(uint32_t, v);
}

// one 32-value FP4 block: 16 value bytes (4 dwords) and the two half-block scales -> 16 half2 in LDS (the scales
// are fp16 values: UE4M3 at half scale lies in [2^-10, 240], and a level times it is exact; 1 for the E8M0 types,
// whose scale is applied per block outside the product)
__device__ __forceinline__ void fp4_block_to_lds(const uint32_t qs[4], float e0, float e1, const uint32_t *lut,
                                                 _Float16 *dst) {
    h2 sc;
    sc.x = (_Float16)e0;  // exact: a UE4M3 half-scale value is an fp16 value
    sc.y = (_Float16)e1;
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const h2 c = __builtin_bit_cast(h2, lut[(qs[k] >> (8 * j)) & 0xffu]);
            o[4 * k + j] = __builtin_bit_cast(uint32_t, c * sc);  // v_pk_mul_f16: exact products
        }
    uint4 *d4 = (uint4 *)dst;
#pragma unroll
    for (int m = 0; m < 4; ++m) d4[m] = make_uint4(o[4 * m], o[4 * m + 1], o[4 * m + 2], o[4 * m + 3]);
}

// int8 -> fp16 for 4 bytes: (b ^ 0x80) placed as the low byte of 0x64xx is 1024 + 128 + b, minus 1152
__device__ __forceinline__ void i8x4_to_h4(uint32_t w, uint32_t &h01, uint32_t &h23) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0u, u, 0x0c010c00u) | 0x64006400u;
    const uint32_t b = __builtin_amdgcn_perm(0u, u, 0x0c030c02u) | 0x64006400u;
    h2 bias;
    bias.x = (_Float16)1152.0f;
    bias.y = (_Float16)1152.0f;
    h01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) - bias);
    h23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, b) - bias);
}

template <int TYPE>
struct GStage;

// ROCmFP4: thread t decodes row t / 2, blocks 2 (t & 1) and 2 (t & 1) + 1 of the stage (36 bytes, 4-aligned)
template <>
struct GStage<TY_FP4> {
    static constexpr bool PERM = true, ROW_SCALE = false, LUT = true;
    static constexpr int TOP = 10;
    struct Raw {
        uint32_t w[9];
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int k0, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1), p = threadIdx.x & 1;
        if (row >= N) {
#pragma unroll
            for (int k = 0; k < 9; ++k) r.w[k] = 0;
            return;
        }
        const uint8_t *b = W + (long long)row * rb + (long long)(k0 / 32 + 2 * p) * 18;
#pragma unroll
        for (int k = 0; k < 9; ++k) r.w[k] = ld32(b + 4 * k);
    }
    __device__ static void store(const Raw &r, const uint32_t *lut, _Float16 *sW, float *) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        _Float16 *dst = sW + row * LDS_ROW + 64 * p;
        const uint32_t qa[4] = {r.w[0], r.w[1], r.w[2], r.w[3]};
        uint32_t qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qb[k] = align_bytes(r.w[5 + k], r.w[4 + k], 2);
        fp4_block_to_lds(qa, ue4m3_half(r.w[4]), ue4m3_half(r.w[4] >> 8), lut, dst);
        fp4_block_to_lds(qb, ue4m3_half(r.w[8] >> 16), ue4m3_half(r.w[8] >> 24), lut, dst + 32);
    }
};

// ROCmFP4_FAST: thread t decodes row t / 2, blocks 2 (t & 1), 2 (t & 1) + 1 (34 bytes at a 2-aligned offset,
// realigned by v_alignbyte)
template <>
struct GStage<TY_FAST> {
    static constexpr bool PERM = true, ROW_SCALE = false, LUT = true;
    static constexpr int TOP = 10;
    // The pair starts 0 or 2 bytes past a dword boundary (row bytes are a multiple of 4): nine aligned dwords
    // from the boundary below cover its 34 bytes. A pair at offset 0 is never a row's last (that one starts
    // at row_bytes - 34, 2 past a boundary), so the two spare bytes it reads are still inside the row.
    struct Raw {
        uint32_t w[9];
        uint32_t off;
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int k0, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1), p = threadIdx.x & 1;
        if (row >= N) {
#pragma unroll
            for (int k = 0; k < 9; ++k) r.w[k] = 0;
            r.off = 0;
            return;
        }
        const uint8_t *b = W + (long long)row * rb + (long long)(k0 / 32 + 2 * p) * 17;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *a = b - r.off;
#pragma unroll
        for (int k = 0; k < 9; ++k) r.w[k] = ld32(a + 4 * k);
    }
    __device__ static void store(const Raw &r, const uint32_t *lut, _Float16 *sW, float *) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        _Float16 *dst = sW + row * LDS_ROW + 64 * p;
        uint32_t w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = align_bytes(k < 8 ? r.w[k + 1] : 0u, r.w[k], r.off);
        // block 0: bytes 0..15 values, 16 scale; block 1: bytes 17..32 values, 33 scale
        const uint32_t qa[4] = {w[0], w[1], w[2], w[3]};
        uint32_t qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qb[k] = align_bytes(w[5 + k], w[4 + k], 1);
        const float ea = ue4m3_half(w[4]), eb = ue4m3_half(w[8] >> 8);
        fp4_block_to_lds(qa, ea, ea, lut, dst);
        fp4_block_to_lds(qb, eb, eb, lut, dst + 32);
    }
};

// Q8_0: thread t decodes row t / 2, blocks 2 (t & 1), 2 (t & 1) + 1 (68 bytes, 4-aligned): the int8 values
// (exact in fp16) in natural order, and the two fp16 block scales into sdw[block][row]
template <>
struct GStage<TY_Q8_0> {
    static constexpr bool PERM = false, ROW_SCALE = true, LUT = false;
    static constexpr int TOP = 10;
    struct Raw {
        uint32_t w[17];
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int k0, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1), p = threadIdx.x & 1;
        if (row >= N) {
#pragma unroll
            for (int k = 0; k < 17; ++k) r.w[k] = 0;
            return;
        }
        const uint8_t *b = W + (long long)row * rb + (long long)(k0 / 32 + 2 * p) * 34;
#pragma unroll
        for (int k = 0; k < 17; ++k) r.w[k] = ld32(b + 4 * k);
    }
    __device__ static void store(const Raw &r, const uint32_t *, _Float16 *sW, float *sdw) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        uint4 *d4 = (uint4 *)(sW + row * LDS_ROW + 64 * p);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            uint32_t v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = blk == 0 ? align_bytes(r.w[k + 1], r.w[k], 2) : r.w[9 + k];
            uint32_t h[16];
#pragma unroll
            for (int k = 0; k < 8; ++k) i8x4_to_h4(v[k], h[2 * k], h[2 * k + 1]);
#pragma unroll
            for (int m = 0; m < 4; ++m) d4[4 * blk + m] = make_uint4(h[4 * m], h[4 * m + 1], h[4 * m + 2], h[4 * m + 3]);
        }
        sdw[(2 * p) * GB_N + row] = h2f(r.w[0] & 0xffffu);
        sdw[(2 * p + 1) * GB_N + row] = h2f(r.w[8] >> 16);
    }
};

// MXFP4: FAST's pair of 17-byte blocks with the E8M0 scale first (byte 0 of a block, values bytes 1..16). An
// E8M0 scale (2^-128 .. 2^127) is no fp16 value, so the levels go into LDS unscaled (exact) and the scales
// into sdw as Q8_0's do: each block's exact integer dot then takes (e dx) outside the MFMA, the reference's
// per-block form (src/matvec_q.hip:1461-1472).
template <>
struct GStage<TY_MXFP4> {
    static constexpr bool PERM = true, ROW_SCALE = true, LUT = true;
    static constexpr int TOP = 12;
    using Raw = GStage<TY_FAST>::Raw;
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int k0, Raw &r) {
        GStage<TY_FAST>::load(W, rb, N, n0, k0, r);
    }
    __device__ static void store(const Raw &r, const uint32_t *lut, _Float16 *sW, float *sdw) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        _Float16 *dst = sW + row * LDS_ROW + 64 * p;
        uint32_t w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = align_bytes(k < 8 ? r.w[k + 1] : 0u, r.w[k], r.off);
        // block 0: byte 0 scale, bytes 1..16 values; block 1: byte 17 scale, bytes 18..33 values
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            qa[k] = align_bytes(w[k + 1], w[k], 1);
            qb[k] = align_bytes(w[k + 5], w[k + 4], 2);
        }
        fp4_block_to_lds(qa, 1.0f, 1.0f, lut, dst);
        fp4_block_to_lds(qb, 1.0f, 1.0f, lut, dst + 32);
        sdw[(2 * p) * GB_N + row] = e8m0_half(w[0]);
        sdw[(2 * p + 1) * GB_N + row] = e8m0_half(w[4] >> 8);
    }
};

template <int TYPE>
__global__ void __launch_bounds__(G_THREADS, 2) k_gemm(GemmArgs a) {
    using S = GStage<TYPE>;
    __shared__ __attribute__((aligned(16))) _Float16 sW[GB_N * LDS_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 sX[GB_T * LDS_ROW];
    __shared__ float sdx[4 * GB_T];   // [block][token]
    __shared__ float sdw[4 * GB_N];   // [block][row] (Q8_0 weights)
    __shared__ uint32_t lut[256];

    // tile coordinates
    int n0, e = 0;
    TokMap tm;
    const int32_t *orow = nullptr;
    if (a.n_tiles) {  // MoE: grid (row tiles, tiles)
        const int k = blockIdx.y;
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        const int st = a.tile_start[k];
        tm = {a.in_rows + st, 0, a.tile_n[k], a.zero_row};
        orow = a.out_rows + st;
        n0 = blockIdx.x * GB_N;
    } else {          // dense: grid (token tiles, row tiles); a row tile's token tiles are adjacent
        tm = {nullptr, (int)blockIdx.x * GB_T, GB_T, a.zero_row};
        n0 = blockIdx.y * GB_N;
    }
    const uint8_t *W = a.W + (long long)e * a.N * a.row_bytes;
    if (S::LUT) init_fp4_lut<S::TOP>(lut);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = (wave & 1) * 64, wt = (wave >> 1) * 64;  // the wave's 64 x 64 sub-tile
    const int nb = a.K / 32;

    // token operand staging: thread t copies 64 halves (128 bytes) of token row t / 2
    const int xr = tid >> 1, xp = tid & 1;
    const _Float16 *xsrc = a.xh + (long long)tm.row(xr) * a.K + 64 * xp;
    const float *dsrc = a.dx + (long long)tm.row(tid & 127) * nb;

    typename S::Raw raw;
    uint4 xv0, xv1, xv2, xv3, xv4, xv5, xv6, xv7;
    float2 dv;
    // global loads of stage k0: the weight bytes, 64 token halves, and the scales of blocks k0/32 + 2 (tid >> 7)
    // and + 1 for token tid & 127
#define GEMM_ISSUE(k0)                                                  \
    do {                                                                \
        S::load(W, a.row_bytes, a.N, n0, (k0), raw);                    \
        const uint4 *s4 = (const uint4 *)(xsrc + (k0));                 \
        xv0 = s4[0];                                                    \
        xv1 = s4[1];                                                    \
        xv2 = s4[2];                                                    \
        xv3 = s4[3];                                                    \
        xv4 = s4[4];                                                    \
        xv5 = s4[5];                                                    \
        xv6 = s4[6];                                                    \
        xv7 = s4[7];                                                    \
        dv = *(const float2 *)(dsrc + (k0) / 32 + 2 * (tid >> 7));      \
    } while (0)

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    GEMM_ISSUE(0);
    for (int k0 = 0; k0 < a.K; k0 += GB_K) {
        __syncthreads();  // the previous stage's LDS reads are done (and the table is written)
        S::store(raw, lut, sW, sdw);
        uint4 *xd = (uint4 *)(sX + xr * LDS_ROW + 64 * xp);
        xd[0] = xv0;
        xd[1] = xv1;
        xd[2] = xv2;
        xd[3] = xv3;
        xd[4] = xv4;
        xd[5] = xv5;
        xd[6] = xv6;
        xd[7] = xv7;
        sdx[(2 * (tid >> 7)) * GB_T + (tid & 127)] = dv.x;
        sdx[(2 * (tid >> 7) + 1) * GB_T + (tid & 127)] = dv.y;
        __syncthreads();
        if (k0 + GB_K < a.K) GEMM_ISSUE(k0 + GB_K);  // next stage's global loads in flight during the MFMAs

#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int kk = b * 32 + 8 * (lane >> 4);
            h8 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[i] = *(const h8 *)(sW + (wn + 16 * i + (lane & 15)) * LDS_ROW + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *(const h8 *)(sX + (wt + 16 * j + (lane & 15)) * LDS_ROW + kk);
            float dxj[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dxj[j] = sdx[b * GB_T + wt + 16 * j + (lane & 15)];
            float dwi[4][4];
            if (S::ROW_SCALE) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 v = *(const float4 *)(sdw + b * GB_N + wn + 16 * i + 4 * (lane >> 4));
                    dwi[i][0] = v.x;
                    dwi[i][1] = v.y;
                    dwi[i][2] = v.z;
                    dwi[i][3] = v.w;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], f4{0.0f, 0.0f, 0.0f, 0.0f}, 0,
                                                                         0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float s = S::ROW_SCALE ? dwi[i][r] * dxj[j] : dxj[j];
                        acc[i][j][r] = __builtin_fmaf(s, c[r], acc[i][j][r]);
                    }
                }
        }
    }

    // store: lane holds rows 4 (lane / 16) .. + 3 of each 16 x 16 tile, token column lane % 16
    const float sc = a.es ? a.es[e] : a.osc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int tt = wt + 16 * j + (lane & 15);
        long long yrow;
        if (orow) {
            if (tt >= tm.n) continue;
            yrow = (long long)orow[tt] * a.N;
        } else {
            const int t = tm.base + tt;
            if (t >= a.T) continue;
            yrow = (long long)t * a.ldy;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + wn + 16 * i + 4 * (lane >> 4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (n + r < a.N) a.y[yrow + n + r] = acc[i][j][r] * sc;
        }
    }
}

// ---------------------------------------------------------------- host launchers

int gemm_supported(int type) {
    return type == TY_FP4 || type == TY_FAST || type == TY_Q8_0 || type == TY_Q4_K || type == TY_Q5_K || type == TY_Q6_K ||
           type == TY_IQ4_XS || type == TY_MXFP4 || type == TY_NVFP4;
}

int gemm_k_multiple() { return GB_K; }

int gemm_token_tile() { return GB_T; }

hipError_t launch_act_f16(int type, const int8_t *q, const float *d, int T, int K, int Tpad, _Float16 *xh, float *dxp,
                          hipStream_t stream) {
    const long long n = (long long)(Tpad + 1) * (K / 32);
    const int perm = type == TY_FP4 || type == TY_FAST || type == TY_MXFP4;
    hipLaunchKernelGGL(k_act_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, q, d, T, K, Tpad, perm, xh,
                       dxp);
    return hipGetLastError();
}

hipError_t launch_gemm(int type, const GemmArgs &a, dim3 grid, hipStream_t stream) {
    switch (type) {
    case TY_FP4: hipLaunchKernelGGL(k_gemm<TY_FP4>, grid, dim3(G_THREADS), 0, stream, a); break;
    case TY_FAST: hipLaunchKernelGGL(k_gemm<TY_FAST>, grid, dim3(G_THREADS), 0, stream, a); break;
    case TY_Q8_0: hipLaunchKernelGGL(k_gemm<TY_Q8_0>, grid, dim3(G_THREADS), 0, stream, a); break;
    case TY_MXFP4: hipLaunchKernelGGL(k_gemm<TY_MXFP4>, grid, dim3(G_THREADS), 0, stream, a); break;
    default: return hipErrorInvalidDeviceFunction;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- split-activation GEMM (ROCmFP4, FAST)
// The activation value X = q dx (int8 q times its fp16-rounded block scale: at most 19 significant bits) enters
// the MFMAs as two fp16 planes, hi = fp16(X 2^s) and lo = fp16(X 2^s - hi), with a per-token power of two 2^s
// that puts the row's largest |X| just under 2^14. hi + lo carries X to 2^-22 relative (the lo rounding),
// products with the weight value CB * scale (exact in fp16) are exact in fp32, so the MFMAs chain straight
// through K with no per-block epilogue: y = (sum_k W'[n][k] (hi + lo)[t][k]) 2^-s. The matrix core does twice
// the multiplies of the per-block form. The planes are made in registers from the int8 values and the block's
// scale ds = fp16(dx 2^s) (exact: an fp16 value times a power of two, inside the fp16 range): hi = q * ds and
// lo = fma(q, ds, -hi), packed fp16 operations with one rounding each, which are the two roundings above.

// one workgroup per token row (rows >= T, up to Tpad + 1, are zero): the int8 values in the GEMM's K order (perm:
// position 2j <- value j, 2j + 1 <- value j + 16 of each 32-block), the block scales dx 2^s as fp16 and ts[t] = 2^-s
__global__ void __launch_bounds__(256) k_act_split(const int8_t *__restrict__ q, const float *__restrict__ d, int T,
                                                   int K, int perm, int8_t *__restrict__ xq,
                                                   _Float16 *__restrict__ xs, float *__restrict__ ts) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x, nb = K / 32;
    int8_t *oq = xq + (long long)t * K;
    _Float16 *os = xs + (long long)t * nb;
    if (t >= T) {  // (uniform)
        for (int k = tid; k < K; k += 256) oq[k] = 0;
        for (int b = tid; b < nb; b += 256) os[b] = (_Float16)0.0f;
        if (tid == 0) ts[t] = 0.0f;
        return;
    }
    const float *dt = d + (long long)t * nb;
    float m = 0.0f;
    for (int b = tid; b < nb; b += 256) m = fmaxf(m, dt[b]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // 127 m = f 2^e with f in [0.5, 1): |X| 2^s < 2^14 for s = 14 - e (clamped so that 2^s and 2^-s stay normal)
    int e = 0;
    if (m > 0.0f) (void)frexpf(127.0f * m, &e);
    int sh = 14 - e;
    sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
    const float up = ldexpf(1.0f, sh);
    if (tid == 0) ts[t] = ldexpf(1.0f, -sh);
    const int8_t *qt = q + (long long)t * K;
    for (int i = tid; i < K; i += 256) {
        const int b = i >> 5, j = i & 31;
        oq[perm ? 32 * b + (j < 16 ? 2 * j : 2 * (j - 16) + 1) : i] = qt[i];
    }
    for (int b = tid; b < nb; b += 256) os[b] = (_Float16)(dt[b] * up);
}

constexpr int GS_K = 64;                  // K per stage (two 32-blocks)
constexpr int GS_ROW = GS_K + 8;          // halves per LDS row (16 bytes of padding: conflict-free b128 reads)
constexpr int GS_N = 256;                 // weight rows per workgroup (one per thread when staging)
constexpr int GS_T = 128;                 // tokens per workgroup
constexpr int GS_T_MOE = 64;              // tokens per workgroup over MoE expert tiles and short prompts

// the stage's two weight blocks of row n0 + t (thread t), decoded into the 64 halves of its LDS row
template <int TYPE>
struct SplitStage {
    static constexpr int TOP = 10;
    static constexpr int BB = TYPE == TY_FP4 ? 18 : 17;  // block bytes
    struct Raw {
        uint32_t w[9];
        uint32_t off;
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int k0, Raw &r) {
        const int row = n0 + threadIdx.x;
        const int rr = row < N ? row : N - 1;  // (rows past the end repeat the last; their outputs are not stored)
        // nine dwords from the 4-aligned address at or below the pair (it starts 0 or 2 bytes past one: 2 BB k0 / 64
        // is even for ROCmFP4, and 34 m leaves 0 or 2 for FAST); each holds at least one byte of the pair
        const uint8_t *b = W + (long long)rr * rb + (long long)(k0 / 32) * BB;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *a = b - r.off;
#pragma unroll
        for (int k = 0; k < 9; ++k) r.w[k] = ld32(a + 4 * k);
    }
    __device__ static void store(const Raw &r, const uint32_t *lut, _Float16 *sW) {
        uint32_t w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = align_bytes(k < 8 ? r.w[k + 1] : 0u, r.w[k], r.off);
        _Float16 *dst = sW + threadIdx.x * GS_ROW;
        // block 0 at byte 0, block 1 at byte BB (values then scale bytes)
        const uint32_t qa[4] = {w[0], w[1], w[2], w[3]};
        uint32_t qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qb[k] = align_bytes(w[k + 5], w[k + 4], BB - 16);
        if (TYPE == TY_FP4) {
            fp4_block_to_lds(qa, ue4m3_half(w[4]), ue4m3_half(w[4] >> 8), lut, dst);
            fp4_block_to_lds(qb, ue4m3_half(w[8] >> 16), ue4m3_half(w[8] >> 24), lut, dst + 32);
        } else {
            const float ea = ue4m3_half(w[4]), eb = ue4m3_half(w[8] >> 8);
            fp4_block_to_lds(qa, ea, ea, lut, dst);
            fp4_block_to_lds(qb, eb, eb, lut, dst + 32);
        }
    }
};

// NVFP4: the stage is one 36-byte block (4-aligned). Its sub-blocks (0, 1) and (2, 3) are regrouped into the
// ROCmFP4 byte order of two 32-value blocks (byte i: value i low, value 16 + i high), which the permuted token
// rows expect, with the four UE4M3 scales as the half-block scales.
template <>
struct SplitStage<TY_NVFP4> {
    static constexpr int TOP = 12;
    struct Raw {
        uint32_t w[9];
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int k0, Raw &r) {
        const int row = n0 + threadIdx.x;
        const int rr = row < N ? row : N - 1;
        const uint8_t *b = W + (long long)rr * rb + (long long)(k0 / 64) * 36;
#pragma unroll
        for (int k = 0; k < 9; ++k) r.w[k] = ld32(b + 4 * k);
    }
    __device__ static void store(const Raw &r, const uint32_t *lut, _Float16 *sW) {
        _Float16 *dst = sW + threadIdx.x * GS_ROW;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t q[4];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t lo = r.w[1 + 4 * h + k], hi = r.w[3 + 4 * h + k];  // sub-blocks 2h, 2h + 1
                q[k] = (lo & 0x0f0f0f0fu) | ((hi & 0x0f0f0f0fu) << 4);
                q[2 + k] = ((lo >> 4) & 0x0f0f0f0fu) | (hi & 0xf0f0f0f0u);
            }
            fp4_block_to_lds(q, nv_scale(r.w[0] >> (16 * h)), nv_scale(r.w[0] >> (16 * h + 8)), lut, dst + 32 * h);
        }
    }
};

constexpr int GS_GROUP = 4;

__device__ inline void dense_tile(int &tt, int &rt) { xcd_tile(tt, rt, GS_GROUP); }

// workgroup tile 256 weight rows x TT tokens (128; 64 for MoE expert tiles, whose runs average a few dozen
// entries, and for prompts of at most 64 tokens); wave w computes rows 128 (w & 1) .. + 127 x tokens TT / 2 (w >> 1) .. (8 x TT / 32 MFMA tiles): per
// 32-block a wave reads 8 weight and 2 x TT / 32 token fragments for 16 TT / 32 MFMAs
template <int TYPE, int TT>
__global__ void __launch_bounds__(G_THREADS, 2) k_gemm_split(GemmArgs a) {
    using S = SplitStage<TYPE>;
    constexpr int NJ = TT / 32;          // token tiles per wave
    constexpr int TPR = G_THREADS / TT;  // staging threads per token row
    constexpr int BPT = GS_K / TPR;      // int8 values a staging thread copies (32 or 16: one 16-byte piece or two)
    constexpr int QROW = GS_K + 16;      // bytes per LDS token row (16 of padding: conflict-free 8-byte reads)
    __shared__ __attribute__((aligned(16))) _Float16 sW[GS_N * GS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sQ[TT * QROW];
    __shared__ uint16_t sD[TT * 2];  // the stage's two block scales of each token row (fp16 bits)
    __shared__ uint32_t lut[256];

    int n0, e = 0;
    TokMap tm;
    const int32_t *orow = nullptr;
    if (a.n_tiles) {  // MoE: grid (row tiles, tiles)
        const int k = blockIdx.y;
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        const int st = a.tile_start[k];
        tm = {a.in_rows + st, 0, a.tile_n[k], a.zero_row};
        orow = a.out_rows + st;
        n0 = blockIdx.x * GS_N;
    } else {          // dense: grid (token tiles, row tiles)
        int tt, rt;
        dense_tile(tt, rt);
        tm = {nullptr, tt * TT, TT, a.zero_row};
        n0 = rt * GS_N;
    }
    const uint8_t *W = a.W + (long long)e * a.N * a.row_bytes;
    init_fp4_lut<S::TOP>(lut);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = (wave & 1) * 128, wt = (wave >> 1) * (TT / 2);

    // token staging: thread t copies BPT int8 values of token row t / TPR, and the scale of their block (the
    // thread whose values start a block)
    const int xr = tid / TPR, xp = tid % TPR, xb = BPT * xp / 32;
    const bool xlead = BPT * xp % 32 == 0;
    const int8_t *qsrc = a.xq + (long long)tm.row(xr) * a.K + BPT * xp;
    const uint16_t *ssrc = (const uint16_t *)a.xs + (long long)tm.row(xr) * (a.K / 32) + xb;

    typename S::Raw raw;
    uint4 qv0, qv1;  // (qv1: BPT = 32 only)
    uint32_t sv;
#define GSPLIT_ISSUE(k0)                                                \
    do {                                                                \
        S::load(W, a.row_bytes, a.N, n0, (k0), raw);                    \
        const uint4 *q4 = (const uint4 *)(qsrc + (k0));                 \
        qv0 = q4[0];                                                    \
        if (BPT == 32) qv1 = q4[1];                                     \
        sv = ssrc[(k0) / 32];                                           \
    } while (0)

    f4 acc[8][NJ];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    GSPLIT_ISSUE(0);
    for (int k0 = 0; k0 < a.K; k0 += GS_K) {
        __syncthreads();  // the previous stage's LDS reads are done (and the table is written)
        S::store(raw, lut, sW);
        uint4 *qd = (uint4 *)(sQ + xr * QROW + BPT * xp);
        qd[0] = qv0;
        if (BPT == 32) qd[1] = qv1;
        if (xlead) sD[xr * 2 + xb] = (uint16_t)sv;
        __syncthreads();
        if (k0 + GS_K < a.K) GSPLIT_ISSUE(k0 + GS_K);  // next stage's global loads in flight during the MFMAs

        __builtin_amdgcn_s_setprio(1);  // the MFMA phase ahead of the other workgroup's staging on this SIMD
#pragma unroll
        for (int b = 0; b < GS_K / 32; ++b) {
            const int kk = b * 32 + 8 * (lane >> 4);
            h8 fa[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) fa[i] = *(const h8 *)(sW + (wn + 16 * i + (lane & 15)) * GS_ROW + kk);
            uint2 qq[NJ];
            uint32_t ds[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int row = wt + 16 * j + (lane & 15);
                qq[j] = *(const uint2 *)(sQ + row * QROW + kk);
                ds[j] = sD[row * 2 + b];
            }
            // per token tile: its hi and lo fragments from 8 int8 values and the block scale, then its 16 MFMAs (the
            // next tile's conversion overlaps them); each accumulator takes the block's hi product, then its lo one
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const h2 dd = __builtin_bit_cast(h2, ds[j] | (ds[j] << 16));
                uint32_t qh[4], hv[4], lv[4];
                i8x4_to_h4(qq[j].x, qh[0], qh[1]);
                i8x4_to_h4(qq[j].y, qh[2], qh[3]);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const h2 x = __builtin_bit_cast(h2, qh[c]);
                    const h2 h = x * dd;
                    hv[c] = __builtin_bit_cast(uint32_t, h);
                    lv[c] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(x, dd, -h));
                }
                const h8 fh = __builtin_bit_cast(h8, make_uint4(hv[0], hv[1], hv[2], hv[3]));
                const h8 fl = __builtin_bit_cast(h8, make_uint4(lv[0], lv[1], lv[2], lv[3]));
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fh, acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fl, acc[i][j], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
    }
#undef GSPLIT_ISSUE

    // store: lane holds rows 4 (lane / 16) .. + 3 of each 16 x 16 tile, token column lane % 16
    const float sc = a.es ? a.es[e] : a.osc;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int tt = wt + 16 * j + (lane & 15);
        long long yrow;
        if (orow) {
            if (tt >= tm.n) continue;
            yrow = (long long)orow[tt] * a.N;
        } else {
            const int t = tm.base + tt;
            if (t >= a.T) continue;
            yrow = (long long)t * a.ldy;
        }
        const float s = sc * a.ts[tm.row(tt)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = n0 + wn + 16 * i + 4 * (lane >> 4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (n + r < a.N) a.y[yrow + n + r] = acc[i][j][r] * s;
        }
    }
}

bool gemm_split(int type) { return type == TY_FP4 || type == TY_FAST || type == TY_NVFP4; }

int gemm_split_k_multiple() { return GS_K; }

int gemm_id_token_tile(int type) { return gemm_split(type) ? GS_T_MOE : GB_T; }

int gemm_dense_token_tile(int type, int T) { return gemm_split(type) && T <= GS_T_MOE ? GS_T_MOE : GB_T; }

int gemm_rows_per_wg(int type) { return gemm_split(type) ? GS_N : gemm_kquant(type) ? GEMM_KQ_ROWS : GB_N; }

hipError_t launch_act_split(int type, const int8_t *q, const float *d, int T, int K, int rows, int8_t *xq,
                            _Float16 *xs, float *ts, hipStream_t stream) {
    hipLaunchKernelGGL(k_act_split, dim3((unsigned)rows), dim3(256), 0, stream, q, d, T, K,
                       (type == TY_FP4 || type == TY_FAST || type == TY_NVFP4) ? 1 : 0, xq, xs, ts);
    return hipGetLastError();
}

hipError_t launch_gemm_split(int type, const GemmArgs &a, dim3 grid, hipStream_t stream) {
    switch (type) {
    case TY_FP4:
        if (a.n_tiles || a.tt == GS_T_MOE) hipLaunchKernelGGL((k_gemm_split<TY_FP4, GS_T_MOE>), grid, dim3(G_THREADS), 0, stream, a);
        else hipLaunchKernelGGL((k_gemm_split<TY_FP4, GS_T>), grid, dim3(G_THREADS), 0, stream, a);
        break;
    case TY_FAST:
        if (a.n_tiles || a.tt == GS_T_MOE) hipLaunchKernelGGL((k_gemm_split<TY_FAST, GS_T_MOE>), grid, dim3(G_THREADS), 0, stream, a);
        else hipLaunchKernelGGL((k_gemm_split<TY_FAST, GS_T>), grid, dim3(G_THREADS), 0, stream, a);
        break;
    case TY_NVFP4:
        if (a.n_tiles || a.tt == GS_T_MOE) hipLaunchKernelGGL((k_gemm_split<TY_NVFP4, GS_T_MOE>), grid, dim3(G_THREADS), 0, stream, a);
        else hipLaunchKernelGGL((k_gemm_split<TY_NVFP4, GS_T>), grid, dim3(G_THREADS), 0, stream, a);
        break;
    default: return hipErrorInvalidDeviceFunction;
    }
    return hipGetLastError();
}

}  // namespace pq
