// fquant.hip -- fp32 activations over quantized weights (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, MXFP4, NVFP4, ROCmFP4,
// ROCmFP4_FAST), and over F32 / F16 / BF16 weights for the expert-indexed forms: the reference's float path
// (matvec_<type>, matmul_f_<type>, matvec_id_<type>, matmul_f_id_<type>: src/matvec_q.hip:640-717, 1076-1237,
// behind qmatvec_launch, qmatvec_launch_batch, qmatvec_launch_id and qmatvec_launch_id_batch_f,
// src/qmatvec.cpp:274-286, 318-367, 601-671). The engine takes it where an input is not quantized.
//
// One kernel, k_mv_fq: a wave per weight row, four rows a workgroup; lane l takes the 32-value groups l, l + 64, ...
// of the row (a Q8_0 / FP4 / FAST / MXFP4 block, half an NVFP4 block, a K-quant sub-block), decodes the group to
// fp32 value for value as the reference's decoders do (src/quant_types.cpp:182-422: the weight is exactly the
// float the CPU dequantizer gives), and for each token accumulates s = fma(w_k, x_k, s) over the group's 32 values
// in order, then acc += s; the wave's 64 sums meet in a fixed butterfly. The weights are read once for all the tokens
// of a launch row. Three row maps share that arithmetic, so a (row, token) gets the same bits whichever form computes
// it: dense (up to FQ_NT tokens a launch row, grid.y over the rest: a batch equals its tokens one by one), expert-
// indexed (grid (rows, slot, token): expert ids[t n_used + slot], input row t or t n_used + slot), and expert
// tiles (grid (rows, tile): up to FQ_TILE entries of one expert, rows in_rows / out_rows: each entry equals the
// expert-indexed launch's result). The registered output scale multiplies the sum (per expert for stacked experts).
//
// The int8 path (activations quantized once, v_dot4 / MFMA) is the fast one; this path is VALU-bound (a decode
// and an fp32 fma per weight), for inputs that stay fp32.
#include "device.h"
#include "kernels.h"

namespace pq {

namespace {

constexpr int FQ_WAVES = 4;   // weight rows (waves) per workgroup
constexpr int FQ_NT = 4;      // tokens per launch row, dense
constexpr int FQ_TILE = 16;   // entries per expert tile (the reference's matmul_f_id tile)
#ifndef FQ_MAXWG_V
#define FQ_MAXWG_V 1024
#endif
constexpr int FQ_MAXWG = FQ_MAXWG_V;  // workgroups along the rows at most (4 a CU)
// A token's activations in LDS: 32 values of group g at g FQ_XS floats (36: the 16-byte reads of 16 lanes on
// consecutive groups fall in distinct banks). Read from global memory instead, each lane's own 128 bytes made every
// 16-byte load instruction touch 64 cache lines.
constexpr int FQ_XS = 36;
constexpr int FQ_LDS = 65536;
// groups a lane has in flight: 4 (F32: 2, its groups hold 128 bytes); 1 over expert tiles, whose 16 entries' rows
// and sums fill the registers
template <int TYPE, int MODE>
constexpr int fq_u() { return MODE == 2 ? 1 : TYPE == 0 ? 2 : 4; }
constexpr int QT_F32_ = 0, QT_F16_ = 1, QT_BF16_ = 30;

// NB bytes from p (any alignment) as realigned dwords: word k holds bytes 4k .. 4k + 3. The dwords are read from
// the 4-aligned address at or below p, up to the one holding the last byte (never past it).
template <int NB>
struct Bytes {
    static constexpr int NW = (NB + 3) / 4;
    uint32_t r[NW];
    __device__ __forceinline__ void load(const uint8_t *p) {
        const uint32_t off = (uint32_t)((uintptr_t)p & 3u);
        const uint8_t *al = p - off;
        uint32_t w[NW + 1];
#pragma unroll
        for (int k = 0; k < NW; ++k) w[k] = ld32(al + 4 * k);
        w[NW] = (int)((off + NB - 1) >> 2) == NW ? ld32(al + 4 * NW) : 0u;
#pragma unroll
        for (int k = 0; k < NW; ++k) r[k] = align_bytes(w[k + 1], w[k], off);
    }
    __device__ __forceinline__ uint32_t byte(int i) const { return (r[i >> 2] >> (8 * (i & 3))) & 0xffu; }
    __device__ __forceinline__ float half(int i) const { return h2f(byte(i) | (byte(i + 1) << 8)); }
};

// the four signed bytes of v as floats times d
__device__ __forceinline__ void i8x4(uint32_t v, float d, float *o) {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = (float)(int8_t)((v >> (8 * k)) & 0xffu) * d;
}

// Group g (values 32 g .. 32 g + 31) of a weight row: Grp<TYPE>::load reads its bytes (dword loads only, so that
// a lane can have several groups in flight), dec makes the 32 floats, value for value as the reference's decoders;
// values at or past K (float types only) are 0.
template <int TYPE>
struct Grp;

template <>
struct Grp<TY_Q8_0> {  // d, then 32 int8 values
    Bytes<34> b;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) { b.load(row + 34LL * g); }
    __device__ __forceinline__ void dec(int, float (&w)[32]) const {
        const float d = b.half(0);
#pragma unroll
        for (int j = 0; j < 32; ++j) w[j] = (float)(int8_t)b.byte(2 + j) * d;
    }
};

template <int TYPE>
struct GrpFp4 {  // ROCmFP4 / FAST: CB[code] scale; code byte i holds values i (low nibble) and i + 16
    static constexpr int BB = TYPE == TY_FP4 ? 18 : 17;
    Bytes<BB> b;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) { b.load(row + (long long)BB * g); }
    __device__ __forceinline__ void dec(int, float (&w)[32]) const {
        const float d0 = ue4m3_half(b.byte(16)), d1 = TYPE == TY_FP4 ? ue4m3_half(b.byte(17)) : d0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            i8x4((uint32_t)fp4x4_lo<10>(b.r[k]), d0, w + 4 * k);
            i8x4((uint32_t)fp4x4_hi<10>(b.r[k]), d1, w + 16 + 4 * k);
        }
    }
};
template <>
struct Grp<TY_FP4> : GrpFp4<TY_FP4> {};
template <>
struct Grp<TY_FAST> : GrpFp4<TY_FAST> {};

template <>
struct Grp<TY_MXFP4> {  // E8M0 scale, then FAST's value bytes
    Bytes<17> b;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) { b.load(row + 17LL * g); }
    __device__ __forceinline__ void dec(int, float (&w)[32]) const {
        const float d = e8m0_half(b.byte(0));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t v = align_bytes(b.r[k + 1], b.r[k], 1);  // bytes 1 + 4k .. 4 + 4k
            i8x4((uint32_t)fp4x4_lo<12>(v), d, w + 4 * k);
            i8x4((uint32_t)fp4x4_hi<12>(v), d, w + 16 + 4 * k);
        }
    }
};

template <>
struct Grp<TY_NVFP4> {  // half g & 1 of 36-byte block g / 2: sub-blocks 2 (g & 1) and 2 (g & 1) + 1
    Bytes<4> s;
    Bytes<16> q;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) {
        const uint8_t *blk = row + 36LL * (g >> 1);
        s.load(blk);
        q.load(blk + 4 + 16 * (g & 1));
    }
    __device__ __forceinline__ void dec(int g, float (&w)[32]) const {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float d = nv_scale(s.byte(2 * (g & 1) + h));
#pragma unroll
            for (int k = 0; k < 2; ++k) {  // byte i of a sub-block: values i (low nibble) and i + 8
                i8x4((uint32_t)fp4x4_lo<12>(q.r[2 * h + k]), d, w + 16 * h + 4 * k);
                i8x4((uint32_t)fp4x4_hi<12>(q.r[2 * h + k]), d, w + 16 * h + 8 + 4 * k);
            }
        }
    }
};

template <int TYPE>
struct GrpK45 {  // Q4_K / Q5_K sub-block g & 7: d sc q - dmin m (src/quant_types.cpp:182-208,290-314)
    static constexpr bool Q5 = TYPE == TY_Q5_K;
    static constexpr int BB = Q5 ? 176 : 144, QS = Q5 ? 48 : 16;
    Bytes<16> hd;
    Bytes<32> q;
    Bytes<Q5 ? 32 : 4> qh;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) {
        const uint8_t *blk = row + (long long)BB * (g >> 3);
        hd.load(blk);
        q.load(blk + QS + 32 * ((g & 7) >> 1));
        if constexpr (Q5) qh.load(blk + 16);
    }
    __device__ __forceinline__ void dec(int g, float (&w)[32]) const {
        const int j = g & 7;
        int sc, mn;
        k4_scale_min(hd.r + 1, j, sc, mn);
        const float d1 = hd.half(0) * (float)sc, m1 = hd.half(2) * (float)mn;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t lv = (j & 1) ? (q.r[k] >> 4) & 0x0f0f0f0fu : q.r[k] & 0x0f0f0f0fu;
            if constexpr (Q5) lv |= ((qh.r[k] >> j) & 0x01010101u) << 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[4 * k + i] = d1 * (float)((lv >> (8 * i)) & 0xffu) - m1;
        }
    }
};
template <>
struct Grp<TY_Q4_K> : GrpK45<TY_Q4_K> {};
template <>
struct Grp<TY_Q5_K> : GrpK45<TY_Q5_K> {};

template <>
struct Grp<TY_Q6_K> {  // values 32 (g & 7) .. of a 210-byte super-block: (d sc) (q - 32) (src/quant_types.cpp:262-288)
    Bytes<32> ql, qh;
    Bytes<2> sc, dd;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) {
        const uint8_t *blk = row + 210LL * (g >> 3);
        const int part = g & 7, h = part >> 2, jj = part & 3;
        ql.load(blk + 64 * h + 32 * (jj & 1));
        qh.load(blk + 128 + 32 * h);
        sc.load(blk + 192 + 2 * part);
        dd.load(blk + 208);
    }
    __device__ __forceinline__ void dec(int g, float (&w)[32]) const {
        const int jj = g & 3;
        const float d = dd.half(0);
        const float s0 = d * (float)(int8_t)sc.byte(0), s1 = d * (float)(int8_t)sc.byte(1);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t lo = (jj >= 2) ? (ql.r[k] >> 4) & 0x0f0f0f0fu : ql.r[k] & 0x0f0f0f0fu;
            const uint32_t lv = lo | (((qh.r[k] >> (2 * jj)) & 0x03030303u) << 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) w[4 * k + i] = (k < 4 ? s0 : s1) * (float)((int)((lv >> (8 * i)) & 0xffu) - 32);
        }
    }
};

template <>
struct Grp<TY_IQ4_XS> {  // sub-block g & 7: (d (ls - 32)) level (src/quant_types.cpp:111-125)
    Bytes<8> hd;
    Bytes<16> q;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int) {
        const uint8_t *blk = row + 136LL * (g >> 3);
        hd.load(blk);
        q.load(blk + 8 + 16 * (g & 7));
    }
    __device__ __forceinline__ void dec(int g, float (&w)[32]) const {
        const float dl = hd.half(0) * (float)iq4xs_scale(hd.r[0] >> 16, hd.r[1], g & 7);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            i8x4((uint32_t)iq4nl4_lo(q.r[k]), dl, w + 4 * k);
            i8x4((uint32_t)iq4nl4_hi(q.r[k]), dl, w + 16 + 4 * k);
        }
    }
};

template <int TYPE>
struct GrpFloat {  // F32 / F16 / BF16: 32 consecutive values (fewer in a last, partial group)
    static constexpr int EB = TYPE == QT_F32_ ? 4 : 2;
    uint32_t v[8 * EB];
    int n;
    __device__ __forceinline__ void load(const uint8_t *row, int g, int K) {
        const uint8_t *b = row + (long long)EB * 32 * g;
        n = K - 32 * g;
        if (n >= 32 && ((uintptr_t)b & 15) == 0) {
#pragma unroll
            for (int k = 0; k < 2 * EB; ++k) {
                const uint4 u = ((const uint4 *)b)[k];
                v[4 * k] = u.x;
                v[4 * k + 1] = u.y;
                v[4 * k + 2] = u.z;
                v[4 * k + 3] = u.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const uint32_t e = j < n ? (EB == 4 ? ((const uint32_t *)b)[j] : ((const uint16_t *)b)[j]) : 0u;
                if constexpr (EB == 4) v[j] = e;
                else if (j & 1) v[j >> 1] |= e << 16;
                else v[j >> 1] = e;
            }
        }
    }
    __device__ __forceinline__ void dec(int, float (&w)[32]) const {
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            float f;
            if constexpr (TYPE == QT_F32_) f = __uint_as_float(v[j]);
            else {
                const uint32_t e = (v[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                f = TYPE == QT_F16_ ? h2f(e) : __uint_as_float(e << 16);
            }
            w[j] = j < n ? f : 0.0f;
        }
    }
};
template <>
struct Grp<QT_F32_> : GrpFloat<QT_F32_> {};
template <>
struct Grp<QT_F16_> : GrpFloat<QT_F16_> {};
template <>
struct Grp<QT_BF16_> : GrpFloat<QT_BF16_> {};

enum { FQ_DENSE = 0, FQ_ID = 1, FQ_TILES = 2 };

struct FqArgs {
    const uint8_t *W;
    long long rb;
    const float *x;
    float *y;
    int N, K, T;
    int vec;  // x rows 16-byte aligned and K % 32 == 0 (uniform)
    int ns;   // tokens whose activations go to LDS at a time (0: read from global memory)
    // expert-indexed: ids [T][n_used], input row t or t n_used + slot
    const int32_t *ids;
    int n_used, x_per_slot;
    // expert tiles
    const int32_t *n_tiles, *tile_e, *tile_start, *tile_n, *in_rows, *out_rows;
    // output scale: es[e] per expert when es is set, else s
    const float *es;
    float s;
};

// the 32-value group's dot with the token's activation values (32 g ..), fma in order from 0
__device__ __forceinline__ float grp_dot(const float (&w)[32], const float *xg, int n, bool vec) {
    float s = 0.0f;
    if (vec) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = ((const float4 *)xg)[q];
            s = __builtin_fmaf(w[4 * q], v.x, s);
            s = __builtin_fmaf(w[4 * q + 1], v.y, s);
            s = __builtin_fmaf(w[4 * q + 2], v.z, s);
            s = __builtin_fmaf(w[4 * q + 3], v.w, s);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) s = __builtin_fmaf(w[j], j < n ? xg[j] : 0.0f, s);
    }
    return s;
}

// the same dot with the token's group in LDS (FQ_XS floats a group, 16-byte aligned)
__device__ __forceinline__ float grp_dot_lds(const float (&w)[32], const float *xg) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 v = ((const float4 *)xg)[q];
        s = __builtin_fmaf(w[4 * q], v.x, s);
        s = __builtin_fmaf(w[4 * q + 1], v.y, s);
        s = __builtin_fmaf(w[4 * q + 2], v.z, s);
        s = __builtin_fmaf(w[4 * q + 3], v.w, s);
    }
    return s;
}

template <int TYPE, int MODE, int NT>
__global__ void __launch_bounds__(64 * FQ_WAVES) k_mv_fq(FqArgs a) {
    const int lane = threadIdx.x & 63;
    // rows wave0, wave0 + stride, ... (a grid of at most FQ_MAXWG workgroups: waves that live for several rows keep
    // the SIMDs full where one short wave per row left them mostly empty, the wave launch being the bound)
    const int K = a.K;
    const int stride = gridDim.x * FQ_WAVES;
    const float *xr[NT];
    long long yb[NT];  // output row offsets (plus the weight row)
    int nt = 1;
    float sc = a.s;
    long long ebase = 0;  // the expert's first weight row
    int t0 = 0, st = 0;   // dense: the first token; tiles: the first entry
    long long xrow1 = 0;  // expert-indexed: the input row
    if constexpr (MODE == FQ_DENSE) {
        t0 = blockIdx.y * NT;
        nt = min(NT, a.T - t0);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int t = t0 + (j < nt ? j : 0);
            xr[j] = a.x + (long long)t * K;
            yb[j] = (long long)t * a.N;
        }
    } else if constexpr (MODE == FQ_ID) {
        const int slot = blockIdx.y, t = blockIdx.z, e = a.ids[t * a.n_used + slot];
        if (e < 0) return;  // (no expert: nothing is written)
        ebase = (long long)e * a.N;
        xrow1 = a.x_per_slot ? (long long)t * a.n_used + slot : (long long)t;
        xr[0] = a.x + xrow1 * K;
        yb[0] = ((long long)t * a.n_used + slot) * a.N;
        if (a.es) sc = a.es[e];
    } else {
        const int k = blockIdx.y;
        if (k >= *a.n_tiles) return;
        const int e = a.tile_e[k];
        st = a.tile_start[k];
        nt = min(NT, a.tile_n[k]);
        ebase = (long long)e * a.N;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int i = st + (j < nt ? j : 0);
            xr[j] = a.x + (long long)a.in_rows[i] * K;
            yb[j] = (long long)a.out_rows[i] * a.N;
        }
        if (a.es) sc = a.es[e];
    }
    const int ng = (K + 31) / 32;
    const bool vec = a.vec != 0;
    constexpr int FQ_U = fq_u<TYPE, MODE>();
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [ns][ng][FQ_XS]: ns tokens' activations
    const int ns = a.ns, tid = threadIdx.x;
    // stage the activations of tokens s0 .. s0 + sn - 1 into LDS: 16-byte chunk q of group g of token s0 + j,
    // consecutive threads on consecutive chunks
    auto stage = [&](int s0, int sn) {
        for (int i = tid; i < sn * ng * 8; i += 64 * FQ_WAVES) {
            const int j = i / (ng * 8), r = i - j * ng * 8, g = r >> 3, q = r & 7;
            const int tj = s0 + j;  // (< nt)
            const long long xrow = MODE == FQ_DENSE ? (long long)(t0 + tj) : MODE == FQ_ID ? xrow1 : a.in_rows[st + tj];
            const float *src = a.x + xrow * K + 32LL * g + 4 * q;
            float4 v;
            if (vec) v = *(const float4 *)src;
            else {
                const int k0 = 32 * g + 4 * q;
                v.x = k0 < K ? src[0] : 0.0f;
                v.y = k0 + 1 < K ? src[1] : 0.0f;
                v.z = k0 + 2 < K ? src[2] : 0.0f;
                v.w = k0 + 3 < K ? src[3] : 0.0f;
            }
            *(float4 *)(xs + ((long long)j * ng + g) * FQ_XS + 4 * q) = v;
        }
    };
    // every token in LDS at once: staged before the row loop
    const bool once = ns >= nt;
    if (ns && once) {
        stage(0, nt);
        __syncthreads();
    }
    // rows of the workgroup's waves: row0 + wave for row0 = FQ_WAVES blockIdx.x, + stride, ... (the loop and the
    // barriers inside are the whole workgroup's; a wave past N joins them without computing)
    for (int row0 = blockIdx.x * FQ_WAVES; row0 < a.N; row0 += stride) {
        const int row = row0 + (threadIdx.x >> 6);
        const bool live = row < a.N;
        const uint8_t *wr = a.W + (ebase + (live ? row : row0)) * a.rb;
        float acc[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = 0.0f;
        // the lane's groups g = lane + 64 i, FQ_U at a time: all their bytes requested before the first is decoded
        // (a group past the row re-reads group g0, which exists), for tokens s0 .. s0 + sn - 1: their activations
        // from LDS (ns > 0), else from global memory
        auto groups = [&](int s0, int sn) {
            for (int g0 = lane; g0 < ng; g0 += 64 * FQ_U) {
                Grp<TYPE> raw[FQ_U];
#pragma unroll
                for (int u = 0; u < FQ_U; ++u) {
                    const int g = g0 + 64 * u;
                    raw[u].load(wr, g < ng ? g : g0, K);
                }
#pragma unroll
                for (int u = 0; u < FQ_U; ++u) {
                    const int g = g0 + 64 * u;
                    if (g >= ng) break;
                    float w[32];
                    raw[u].dec(g, w);
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        if (j >= nt || j < s0 || j >= s0 + sn) continue;
                        acc[j] += ns ? grp_dot_lds(w, xs + ((long long)(j - s0) * ng + g) * FQ_XS)
                                     : grp_dot(w, xr[j] + 32LL * g, K - 32 * g, vec);
                    }
                }
            }
        };
        if (!ns || once) {
            if (live) groups(0, NT);
        } else {  // a few tokens at a time, staged again for each row group
            for (int s0 = 0; s0 < nt; s0 += ns) {
                const int sn = min(ns, nt - s0);
                __syncthreads();  // (the previous tokens' readers are done)
                stage(s0, sn);
                __syncthreads();
                if (live) groups(s0, sn);
            }
        }
        if (!live) continue;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            float v = acc[j];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0 && j < nt) a.y[yb[j] + row] = v * sc;
        }
    }
}

template <int TYPE>
hipError_t launch_t(int mode, FqArgs a, hipStream_t stream) {
    const unsigned gx = (unsigned)min((a.N + FQ_WAVES - 1) / FQ_WAVES, FQ_MAXWG);
    const dim3 blk(64 * FQ_WAVES);
    // tokens a workgroup stages at once: as many of its NT as fit FQ_LDS bytes (none: the global reads)
    const long long per = (long long)((a.K + 31) / 32) * FQ_XS * 4;
    const int nt = mode == FQ_DENSE ? min(a.T, FQ_NT) : mode == FQ_ID ? 1 : FQ_TILE;
    a.ns = (int)min((long long)nt, FQ_LDS / per);
    const size_t lds = (size_t)a.ns * per;
    switch (mode) {
    case FQ_DENSE:
        hipLaunchKernelGGL((k_mv_fq<TYPE, FQ_DENSE, FQ_NT>), dim3(gx, (unsigned)((a.T + FQ_NT - 1) / FQ_NT)), blk, lds,
                           stream, a);
        break;
    case FQ_ID:
        hipLaunchKernelGGL((k_mv_fq<TYPE, FQ_ID, 1>), dim3(gx, (unsigned)a.n_used, (unsigned)a.T), blk, lds, stream, a);
        break;
    default:
        hipLaunchKernelGGL((k_mv_fq<TYPE, FQ_TILES, FQ_TILE>), dim3(gx, (unsigned)a.T), blk, lds, stream, a);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_any(int type, int mode, const FqArgs &a, hipStream_t stream) {
    switch (type) {
    case TY_Q8_0: return launch_t<TY_Q8_0>(mode, a, stream);
    case TY_Q4_K: return launch_t<TY_Q4_K>(mode, a, stream);
    case TY_Q5_K: return launch_t<TY_Q5_K>(mode, a, stream);
    case TY_Q6_K: return launch_t<TY_Q6_K>(mode, a, stream);
    case TY_IQ4_XS: return launch_t<TY_IQ4_XS>(mode, a, stream);
    case TY_MXFP4: return launch_t<TY_MXFP4>(mode, a, stream);
    case TY_NVFP4: return launch_t<TY_NVFP4>(mode, a, stream);
    case TY_FP4: return launch_t<TY_FP4>(mode, a, stream);
    case TY_FAST: return launch_t<TY_FAST>(mode, a, stream);
    case QT_F32_: return launch_t<QT_F32_>(mode, a, stream);
    case QT_F16_: return launch_t<QT_F16_>(mode, a, stream);
    case QT_BF16_: return launch_t<QT_BF16_>(mode, a, stream);
    default: return hipErrorInvalidDeviceFunction;
    }
}

bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

bool fq_type(int type, bool with_float) {
    switch (type) {
    case TY_Q8_0: case TY_Q4_K: case TY_Q5_K: case TY_Q6_K: case TY_IQ4_XS: case TY_MXFP4: case TY_NVFP4: case TY_FP4:
    case TY_FAST: return true;
    case QT_F32_: case QT_F16_: case QT_BF16_: return with_float;
    default: return false;
    }
}

int fq_tile() { return FQ_TILE; }

hipError_t launch_fq_dense(int type, const uint8_t *W, long long rb, const float *x, float *y, int N, int K, int T,
                           float s, hipStream_t stream) {
    FqArgs a = {};
    a.W = W;
    a.rb = rb;
    a.x = x;
    a.y = y;
    a.N = N;
    a.K = K;
    a.T = T;
    a.vec = K % 32 == 0 && al16(x);
    a.s = s;
    return launch_any(type, FQ_DENSE, a, stream);
}

hipError_t launch_fq_id(int type, const uint8_t *W, long long rb, const int32_t *ids, int n_used, int x_per_slot,
                        const float *x, float *y, int N, int K, int T, const float *es, float s, hipStream_t stream) {
    FqArgs a = {};
    a.W = W;
    a.rb = rb;
    a.x = x;
    a.y = y;
    a.N = N;
    a.K = K;
    a.T = T;
    a.vec = K % 32 == 0 && al16(x);
    a.ids = ids;
    a.n_used = n_used;
    a.x_per_slot = x_per_slot;
    a.es = es;
    a.s = s;
    return launch_any(type, FQ_ID, a, stream);
}

hipError_t launch_fq_tiles(int type, const uint8_t *W, long long rb, const float *x, float *y, int N, int K,
                           int max_tiles, const int32_t *n_tiles, const int32_t *tile_e, const int32_t *tile_start,
                           const int32_t *tile_n, const int32_t *in_rows, const int32_t *out_rows, const float *es,
                           float s, hipStream_t stream) {
    FqArgs a = {};
    a.W = W;
    a.rb = rb;
    a.x = x;
    a.y = y;
    a.N = N;
    a.K = K;
    a.T = max_tiles;
    a.vec = K % 32 == 0 && al16(x);
    a.n_tiles = n_tiles;
    a.tile_e = tile_e;
    a.tile_start = tile_start;
    a.tile_n = tile_n;
    a.in_rows = in_rows;
    a.out_rows = out_rows;
    a.es = es;
    a.s = s;
    return launch_any(type, FQ_TILES, a, stream);
}

}  // namespace pq
