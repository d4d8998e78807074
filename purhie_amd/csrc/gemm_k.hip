// gemm_k.hip -- the prefill GEMM Y[t][n] = sum_k W[n][k] X[t][k] for the K-quant formats (Q4_K, Q5_K, Q6_K) and
// IQ4_XS on
// gfx950 MFMA, dense and over MoE expert tiles. Replaces the reference's K-quant WMMA GEMM (matmul_wmma_q4_K /
// _q6_K and their _id forms: wmma_q8k, WStageK, src/matvec_q.hip:2975-3348), which reads Q8_K activations
// and applies d_x (d_w isum - dmin msum) to exact integer tile sums.
//
// MI355X-first design (fp16 MFMA on exact integer operands, one float epilogue per 256-value super-block):
//   * the Q8_K activation value qK (int8) is exact in fp16. The Q4_K weight's integer part sc_j q (6-bit
//     sub-block scale times 4-bit value, <= 945) is exact in fp16; Q6_K's sc_g (q - 32) (int8 scale times
//     6-bit value, |.| <= 4096) is written as two exact planes, its even part and its low bit. The
//     v_mfma_f32_16x16x32_f16 chain over a super-block's 8 blocks therefore sums exact integer products:
//     isum = sum_j sc_j sum_i q_i qK_i of the reference (exact in fp32 while below 2^24).
//   * the Q4_K min term msum = sum_j m_j sum_{i in j} qK_i runs as one v_mfma_f32_16x16x16_f16 per
//     super-block: the 16 group sums bsK of the activation (|.| <= 2032, exact in fp16) against the weight's
//     m_{g/2} (exact).
//   * per super-block and output, y += dK (d isum - dmin msum) (Q4_K) or y += dK d isum (Q6_K): three vector
//     operations per output per 256 K, against 8 (Q4_K) or 16 (Q6_K) MFMAs per 16 x 16 tile.
//   * workgroup tile 128 weight rows x 128 tokens, 4 waves of 64 x 64 (the super-block sums and the running
//     outputs both stay in registers), K stages of 64 (a quarter super-block) with the next stage's global
//     loads in flight during the MFMAs. The weights are decoded from their GGUF blocks into LDS once per tile.
#include "device.h"
#include "kernels.h"

namespace pq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int GK_N = GEMM_KQ_ROWS;  // weight rows per workgroup
constexpr int GK_T = 128;           // tokens per workgroup
constexpr int GK_S = 64;            // K per stage
constexpr int GK_ROW = GK_S + 8;    // halves per LDS row of a stage (16 bytes of padding: conflict-free b128 reads)
constexpr int GK_G = 24;            // halves per LDS row of a super-block's 16 group values (48 bytes)
constexpr int GK_THREADS = 256;

// ---------------------------------------------------------------- token pre-pass
// One workgroup per token row r (rows >= T are zero): xh[r][k] = qK as fp16, xb[r][g] = bsK as fp16 (the sums of 16
// int8 values, exact), xd[r][s] = dK.
__global__ void __launch_bounds__(256) k_act_q8k(const int8_t *__restrict__ q, const float *__restrict__ dK,
                                                 const int32_t *__restrict__ bs, int T, int K,
                                                 _Float16 *__restrict__ xh, _Float16 *__restrict__ xb,
                                                 float *__restrict__ xd) {
    const int r = blockIdx.x, tid = threadIdx.x;
    const bool live = r < T;
    const int8_t *qr = q + (long long)r * K;
    _Float16 *oh = xh + (long long)r * K;
    for (int k = 4 * tid; k < K; k += 1024) {
        const uint32_t w = live ? *(const uint32_t *)(qr + k) : 0u;
        h4 v;
        v.x = (_Float16)(float)(int8_t)(w & 0xffu);
        v.y = (_Float16)(float)(int8_t)((w >> 8) & 0xffu);
        v.z = (_Float16)(float)(int8_t)((w >> 16) & 0xffu);
        v.w = (_Float16)(float)(int8_t)(w >> 24);
        *(h4 *)(oh + k) = v;
    }
    const int ng = K / 16, ns = K / 256;
    for (int g = tid; g < ng; g += 256)
        xb[(long long)r * ng + g] = live ? (_Float16)(float)bs[(long long)r * ng + g] : (_Float16)0.0f;
    for (int s = tid; s < ns; s += 256) xd[(long long)r * ns + s] = live ? dK[(long long)r * ns + s] : 0.0f;
}

// ---------------------------------------------------------------- weight stages
// Stage c (0..3) of super-block s holds K values 256 s + 64 c .. + 63. Thread t decodes 32 of them for row
// n0 + t / 2 (rows past N repeat the last; their outputs are not stored): into LDS row t / 2 of each plane at
// 32 (t & 1), in natural K order. It also writes the row's super-block factors into sD and (Q4_K) the
// sub-block's min into the group table sG (groups 2j and 2j + 1 of sub-block j).

// 4 values (bytes 0..15 of v, one per byte) times sc (<= 63) -> 4 halves: two values per dword as
// (b0 + b1 2^16) sc | 0x6400 6400 = fp16 (1024 + b sc) pairs, minus 1024 (exact: b sc < 1024)
__device__ __forceinline__ void scaled_nibbles(uint32_t v, uint32_t sc, uint32_t &h01, uint32_t &h23) {
    const uint32_t a = (__builtin_amdgcn_perm(0u, v, 0x0c010c00u) * sc) | 0x64006400u;
    const uint32_t b = (__builtin_amdgcn_perm(0u, v, 0x0c030c02u) * sc) | 0x64006400u;
    h2 bias;
    bias.x = (_Float16)1024.0f;
    bias.y = (_Float16)1024.0f;
    h01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) - bias);
    h23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, b) - bias);
}

template <int TYPE>
struct KStage;

// Q4_K (144-byte super-block: d, dmin, 12 scale bytes, qs[128]; chunk c = qs bytes 32 c .. + 31, low nibbles
// sub-block 2c, high nibbles 2c + 1): thread t takes sub-block 2c + (t & 1). The block is 16-byte aligned (W
// 16-aligned, 144-byte units), so the header and the chunk are three 16-byte loads.
template <>
struct KStage<TY_Q4_K> {
    static constexpr int PLANES = 1, BB = 144;
    struct Raw {
        uint4 h, q0, q1;
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int s, int c, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1);
        const int rr = row < N ? row : N - 1;
        const uint8_t *b = W + (long long)rr * rb + (long long)s * BB;
        r.h = *(const uint4 *)b;
        r.q0 = *(const uint4 *)(b + 16 + 32 * c);
        r.q1 = *(const uint4 *)(b + 32 + 32 * c);
    }
    __device__ static void store(const Raw &r, int c, _Float16 *sW, _Float16 *sG, float2 *sD) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        const uint32_t s3[3] = {r.h.y, r.h.z, r.h.w};
        int sc0, mn0, sc1, mn1;
        k4_scale_min(s3, 2 * c, sc0, mn0);
        k4_scale_min(s3, 2 * c + 1, sc1, mn1);
        const uint32_t sc = (uint32_t)(p ? sc1 : sc0);
        const _Float16 mn = (_Float16)(float)(p ? mn1 : mn0);
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        uint32_t o[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) scaled_nibbles((q[k] >> (4 * p)) & 0x0f0f0f0fu, sc, o[2 * k], o[2 * k + 1]);
        uint4 *d4 = (uint4 *)(sW + row * GK_ROW + 32 * p);
#pragma unroll
        for (int m = 0; m < 4; ++m) d4[m] = make_uint4(o[4 * m], o[4 * m + 1], o[4 * m + 2], o[4 * m + 3]);
        h2 mm;
        mm.x = mn;
        mm.y = mn;
        *(h2 *)(sG + row * GK_G + 4 * c + 2 * p) = mm;
        if (p == 0) sD[row] = make_float2(h2f(r.h.x & 0xffffu), h2f(r.h.x >> 16));
    }
};

// Q5_K (176-byte super-block, 16-byte aligned: Q4_K's header, qh[32] @16, qs[128] @48): as Q4_K, with bit j of qh
// byte l as bit 4 of sub-block j's value l. sc q reaches 63 * 31 = 1953, past the 1024-value window of
// scaled_nibbles, so the low nibble and the high bit go through it apart (sc q_lo <= 945, sc 16 <= 1008) and are
// added in fp16 (exact: integers below 2048).
template <>
struct KStage<TY_Q5_K> {
    static constexpr int PLANES = 1, BB = 176;
    struct Raw {
        uint4 h, h0, h1, q0, q1;
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int s, int c, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1);
        const int rr = row < N ? row : N - 1;
        const uint8_t *b = W + (long long)rr * rb + (long long)s * BB;
        r.h = *(const uint4 *)b;
        r.h0 = *(const uint4 *)(b + 16);
        r.h1 = *(const uint4 *)(b + 32);
        r.q0 = *(const uint4 *)(b + 48 + 32 * c);
        r.q1 = *(const uint4 *)(b + 64 + 32 * c);
    }
    __device__ static void store(const Raw &r, int c, _Float16 *sW, _Float16 *sG, float2 *sD) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1, j = 2 * c + p;
        const uint32_t s3[3] = {r.h.y, r.h.z, r.h.w};
        int sc0, mn0, sc1, mn1;
        k4_scale_min(s3, 2 * c, sc0, mn0);
        k4_scale_min(s3, 2 * c + 1, sc1, mn1);
        const uint32_t sc = (uint32_t)(p ? sc1 : sc0);
        const _Float16 mn = (_Float16)(float)(p ? mn1 : mn0);
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
        uint32_t o[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t a01, a23, b01, b23;
            scaled_nibbles((q[k] >> (4 * p)) & 0x0f0f0f0fu, sc, a01, a23);
            scaled_nibbles(((qh[k] >> j) & 0x01010101u) << 4, sc, b01, b23);
            o[2 * k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a01) + __builtin_bit_cast(h2, b01));
            o[2 * k + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a23) + __builtin_bit_cast(h2, b23));
        }
        uint4 *d4 = (uint4 *)(sW + row * GK_ROW + 32 * p);
#pragma unroll
        for (int m = 0; m < 4; ++m) d4[m] = make_uint4(o[4 * m], o[4 * m + 1], o[4 * m + 2], o[4 * m + 3]);
        h2 mm;
        mm.x = mn;
        mm.y = mn;
        *(h2 *)(sG + row * GK_G + 4 * c + 2 * p) = mm;
        if (p == 0) sD[row] = make_float2(h2f(r.h.x & 0xffffu), h2f(r.h.x >> 16));
    }
};

// IQ4_XS (136-byte super-block, 8-byte aligned: d, scales_h, scales_l, qs[128] @8): thread parity p takes
// sub-block j = 2 c + p, whose 16 qs bytes hold values 32 j + i (low nibbles) and 32 j + 16 + i (high). The
// integer weight (ls - 32) * level reaches 32 * 127 = 4064, past fp16's exact integers: written as Q6_K's two
// planes, the even part and the low bit.
template <>
struct KStage<TY_IQ4_XS> {
    static constexpr int PLANES = 2, BB = 136;
    struct Raw {
        uint2 h, q0, q1;
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int s, int c, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1), p = threadIdx.x & 1;
        const int rr = row < N ? row : N - 1;
        const uint8_t *b = W + (long long)rr * rb + (long long)s * BB;
        r.h = *(const uint2 *)b;
        r.q0 = *(const uint2 *)(b + 8 + 16 * (2 * c + p));
        r.q1 = *(const uint2 *)(b + 16 + 16 * (2 * c + p));
    }
    __device__ static void store(const Raw &r, int c, _Float16 *sW, _Float16 *, float2 *sD) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        const int ls = iq4xs_scale(r.h.x >> 16, r.h.y, 2 * c + p);
        const uint32_t q[4] = {r.q0.x, r.q0.y, r.q1.x, r.q1.y};
        uint32_t hi[16], lo[16];
#pragma unroll
        for (int half = 0; half < 2; ++half) {  // low nibbles: values 0..15; high nibbles: 16..31
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t v = (uint32_t)iq4nl4((q[k] >> (4 * half)) & 0x0f0f0f0fu);
                _Float16 vh[4], vl[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int P = ls * (int)(int8_t)((v >> (8 * e)) & 0xffu);
                    vh[e] = (_Float16)(float)(P & ~1);  // even, |.| <= 4064: exact
                    vl[e] = (_Float16)(float)(P & 1);
                }
                hi[8 * half + 2 * k] = __builtin_bit_cast(uint32_t, h2{vh[0], vh[1]});
                hi[8 * half + 2 * k + 1] = __builtin_bit_cast(uint32_t, h2{vh[2], vh[3]});
                lo[8 * half + 2 * k] = __builtin_bit_cast(uint32_t, h2{vl[0], vl[1]});
                lo[8 * half + 2 * k + 1] = __builtin_bit_cast(uint32_t, h2{vl[2], vl[3]});
            }
        }
        uint4 *dh = (uint4 *)(sW + row * GK_ROW + 32 * p), *dl = (uint4 *)(sW + (GK_N + row) * GK_ROW + 32 * p);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            dh[m] = make_uint4(hi[4 * m], hi[4 * m + 1], hi[4 * m + 2], hi[4 * m + 3]);
            dl[m] = make_uint4(lo[4 * m], lo[4 * m + 1], lo[4 * m + 2], lo[4 * m + 3]);
        }
        if (p == 0) sD[row] = make_float2(h2f(r.h.x & 0xffffu), 0.0f);
    }
};

// Q6_K (210-byte super-block, 2-byte aligned: ql[128], qh[64] @128, sc[16] @192, d @208). Values 128 h + 32 i + l
// (h = 0, 1; i = 0..3; l < 32): ql byte 64 h + 32 (i & 1) + l, nibble i >> 1; qh byte 128 + 32 h + l, bits 2 i;
// scale sc[(128 h + 32 i + l) / 16]. Stage c is h = c >> 1, i = 2 (c & 1) + p for thread parity p. The runs of
// 32 ql and qh bytes are read as 9 dwords from the 4-aligned address at or below them: they start 0 or 2 bytes
// past one, so the 36 bytes read reach at most 2 bytes before a run (which then is not at the matrix start, W
// being 4-aligned) and 4 past it (still inside the block). The two scale bytes and d are 16-bit loads.
template <>
struct KStage<TY_Q6_K> {
    static constexpr int PLANES = 2, BB = 210;
    struct Raw {
        uint32_t l[9], h[9];
        uint32_t sc, d, off;
    };
    __device__ static void load(const uint8_t *W, long long rb, int N, int n0, int s, int c, Raw &r) {
        const int row = n0 + (threadIdx.x >> 1), p = threadIdx.x & 1;
        const int rr = row < N ? row : N - 1;
        const uint8_t *b = W + (long long)rr * rb + (long long)s * BB;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *bl = b - r.off + 64 * (c >> 1) + 32 * p, *bh = b - r.off + 128 + 32 * (c >> 1);
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            r.l[k] = ld32(bl + 4 * k);
            r.h[k] = ld32(bh + 4 * k);
        }
        r.sc = *(const uint16_t *)(b + 192 + 4 * c + 2 * p);
        r.d = *(const uint16_t *)(b + 208);
    }
    __device__ static void store(const Raw &r, int c, _Float16 *sW, _Float16 *, float2 *sD) {
        const int row = threadIdx.x >> 1, p = threadIdx.x & 1;
        const int u = c & 1;
        const int sc0 = (int)(int8_t)(r.sc & 0xffu), sc1 = (int)(int8_t)(r.sc >> 8);  // groups 4c + 2p, + 1
        uint32_t hi[16], lo[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t l = align_bytes(r.l[k + 1], r.l[k], r.off), h = align_bytes(r.h[k + 1], r.h[k], r.off);
            const uint32_t q = ((l >> (4 * u)) & 0x0f0f0f0fu) | (((h >> (4 * u + 2 * p)) & 0x03030303u) << 4);
            const int sc = k < 4 ? sc0 : sc1;
            _Float16 vh[4], vl[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int P = sc * ((int)((q >> (8 * e)) & 0xffu) - 32);
                vh[e] = (_Float16)(float)(P & ~1);  // even, |.| <= 4096: exact
                vl[e] = (_Float16)(float)(P & 1);
            }
            hi[2 * k] = __builtin_bit_cast(uint32_t, h2{vh[0], vh[1]});
            hi[2 * k + 1] = __builtin_bit_cast(uint32_t, h2{vh[2], vh[3]});
            lo[2 * k] = __builtin_bit_cast(uint32_t, h2{vl[0], vl[1]});
            lo[2 * k + 1] = __builtin_bit_cast(uint32_t, h2{vl[2], vl[3]});
        }
        uint4 *dh = (uint4 *)(sW + row * GK_ROW + 32 * p), *dl = (uint4 *)(sW + (GK_N + row) * GK_ROW + 32 * p);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            dh[m] = make_uint4(hi[4 * m], hi[4 * m + 1], hi[4 * m + 2], hi[4 * m + 3]);
            dl[m] = make_uint4(lo[4 * m], lo[4 * m + 1], lo[4 * m + 2], lo[4 * m + 3]);
        }
        if (p == 0) sD[row] = make_float2(h2f(r.d), 0.0f);
    }
};

// ---------------------------------------------------------------- the GEMM
// wave w computes rows 64 (w & 1) .. + 63 x tokens 64 (w >> 1) .. + 63 (4 x 4 MFMA tiles)
template <int TYPE, bool CAP = false>
__global__ void __launch_bounds__(GK_THREADS, 2) k_gemm_kq(GemmArgs a) {
    using S = KStage<TYPE>;
    constexpr bool MINS = TYPE == TY_Q4_K || TYPE == TY_Q5_K;
    constexpr int PL = S::PLANES;
    __shared__ __attribute__((aligned(16))) _Float16 sW[PL * GK_N * GK_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 sX[GK_T * GK_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 sG[MINS ? GK_N * GK_G : 8];  // weight mins per group
    __shared__ __attribute__((aligned(16))) _Float16 sB[MINS ? GK_T * GK_G : 8];  // token group sums
    __shared__ float2 sD[GK_N];                                                   // (d, dmin) per row
    __shared__ float sK[GK_T];                                                    // dK per token

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
        n0 = blockIdx.x * GK_N;
    } else {          // dense: grid (token tiles, row tiles); a row tile's token tiles are adjacent
        tm = {nullptr, (int)blockIdx.x * GK_T, GK_T, a.zero_row};
        n0 = blockIdx.y * GK_N;
    }
    const uint8_t *W = a.W + (long long)e * a.N * a.row_bytes;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = (wave & 1) * 64, wt = (wave >> 1) * 64;
    const int nsb = a.K / 256;

    // token staging: thread t copies 32 halves of token row t / 2 per stage, and per super-block 8 of its 16
    // group sums and its dK
    const int xr = tid >> 1, xp = tid & 1;
    const long long trow = tm.row(xr);
    const _Float16 *xsrc = a.xh + trow * a.K + 32 * xp;
    const _Float16 *bsrc = a.xb + trow * (a.K / 16) + 8 * xp;
    const float *ksrc = a.dx + trow * nsb;

    typename S::Raw raw;
    uint4 xv0, xv1, xv2, xv3, bv = make_uint4(0u, 0u, 0u, 0u);
    float kv;
#define GK_ISSUE(s, c)                                                  \
    do {                                                                \
        S::load(W, a.row_bytes, a.N, n0, (s), (c), raw);                \
        const uint4 *x4 = (const uint4 *)(xsrc + 256 * (s) + 64 * (c)); \
        xv0 = x4[0];                                                    \
        xv1 = x4[1];                                                    \
        xv2 = x4[2];                                                    \
        xv3 = x4[3];                                                    \
        if constexpr (MINS) bv = *(const uint4 *)(bsrc + 16 * (s));     \
        kv = ksrc[(s)];                                                 \
    } while (0)

    f4 acc[4][4], isum[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            isum[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }

    GK_ISSUE(0, 0);
    for (int s = 0; s < nsb; ++s) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            __syncthreads();  // the previous stage's (and super-block epilogue's) LDS reads are done
            S::store(raw, c, sW, sG, sD);
            uint4 *xd = (uint4 *)(sX + xr * GK_ROW + 32 * xp);
            xd[0] = xv0;
            xd[1] = xv1;
            xd[2] = xv2;
            xd[3] = xv3;
            if constexpr (MINS) *(uint4 *)(sB + xr * GK_G + 8 * xp) = bv;
            if (xp == 0) sK[xr] = kv;
            __syncthreads();
            // next stage's global loads in flight during the MFMAs
            if (c < 3) GK_ISSUE(s, c + 1);
            else if (s + 1 < nsb) GK_ISSUE(s + 1, 0);

#pragma unroll
            for (int b = 0; b < GK_S / 32; ++b) {
                const int kk = b * 32 + 8 * (lane >> 4);
                h8 fb[4], fa[PL][4];
#pragma unroll
                for (int j = 0; j < 4; ++j) fb[j] = *(const h8 *)(sX + (wt + 16 * j + (lane & 15)) * GK_ROW + kk);
#pragma unroll
                for (int pl = 0; pl < PL; ++pl)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        fa[pl][i] = *(const h8 *)(sW + (pl * GK_N + wn + 16 * i + (lane & 15)) * GK_ROW + kk);
#pragma unroll
                for (int pl = 0; pl < PL; ++pl)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            isum[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[pl][i], fb[j], isum[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);  // (keeps the next block's fragment reads from being hoisted here)
            }
        }
        if constexpr (CAP) {  // capture mode: the exact integer isum of each (token, row) for this super-block
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int tt = wt + 16 * j + (lane & 15);
                long long t;
                if (orow) t = tt < tm.n ? orow[tt] : -1;
                else t = tm.base + tt < a.T ? tm.base + tt : -1;
                if (t < 0) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n0 + wn + 16 * i + 4 * (lane >> 4) + r;
                        if (n < a.N) a.cap[(t * a.N + n) * nsb + s] = (int32_t)isum[i][j][r];
                    }
            }
        }
        // super-block epilogue: y += dK (d isum - dmin msum), the sums restart at zero
        float dk[4];
        h4 fs[4], fm[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dk[j] = sK[wt + 16 * j + (lane & 15)];
            if constexpr (MINS) fs[j] = *(const h4 *)(sB + (wt + 16 * j + (lane & 15)) * GK_G + 4 * (lane >> 4));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (MINS) fm[i] = *(const h4 *)(sG + (wn + 16 * i + (lane & 15)) * GK_G + 4 * (lane >> 4));
            float2 dd[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) dd[r] = sD[wn + 16 * i + 4 * (lane >> 4) + r];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f4 ms = f4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (MINS) ms = __builtin_amdgcn_mfma_f32_16x16x16f16(fm[i], fs[j], ms, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = dd[r].x * isum[i][j][r];
                    if constexpr (MINS) v = __builtin_fmaf(-dd[r].y, ms[r], v);
                    acc[i][j][r] = __builtin_fmaf(dk[j], v, acc[i][j][r]);
                    isum[i][j][r] = 0.0f;
                }
            }
        }
    }
#undef GK_ISSUE

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

// values per captured integer: the int8 K-quant GEMM's super-block isum, the per-block GEMM's block dot (Q8_0,
// MXFP4); the split GEMM (ROCmFP4, FAST, NVFP4) forms no integer sums
int gemm_cap_unit(int type) { return gemm_kquant(type) ? 256 : type == TY_Q8_0 || type == TY_MXFP4 ? 32 : 0; }

bool gemm_kquant(int type) { return type == TY_Q4_K || type == TY_Q5_K || type == TY_Q6_K || type == TY_IQ4_XS; }

hipError_t launch_act_q8k(const int8_t *q, const float *dK, const int32_t *bs, int T, int K, int rows, _Float16 *xh,
                          _Float16 *xb, float *xd, hipStream_t stream) {
    hipLaunchKernelGGL(k_act_q8k, dim3((unsigned)rows), dim3(256), 0, stream, q, dK, bs, T, K, xh, xb, xd);
    return hipGetLastError();
}

template <int TYPE>
static void launch_kq(const GemmArgs &a, dim3 grid, hipStream_t stream) {
    if (a.cap) hipLaunchKernelGGL((k_gemm_kq<TYPE, true>), grid, dim3(GK_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((k_gemm_kq<TYPE>), grid, dim3(GK_THREADS), 0, stream, a);
}

hipError_t launch_gemm_kquant(int type, const GemmArgs &a, dim3 grid, hipStream_t stream) {
    switch (type) {
    case TY_Q4_K: launch_kq<TY_Q4_K>(a, grid, stream); break;
    case TY_Q5_K: launch_kq<TY_Q5_K>(a, grid, stream); break;
    case TY_IQ4_XS: launch_kq<TY_IQ4_XS>(a, grid, stream); break;
    case TY_Q6_K: launch_kq<TY_Q6_K>(a, grid, stream); break;
    default: return hipErrorInvalidDeviceFunction;
    }
    return hipGetLastError();
}

}  // namespace pq
