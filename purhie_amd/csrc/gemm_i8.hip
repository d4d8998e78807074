// gemm_i8.hip -- the K-quant prefill GEMM Y[t][n] = sum_k W[n][k] X[t][k] on gfx950's int8 matrix cores
// (v_mfma_i32_32x32x32_i8), dense and over MoE expert tiles, for Q4_K, Q5_K, Q6_K and IQ4_XS. Replaces the
// reference's K-quant WMMA GEMM (matmul_wmma_q4_K / _q6_K and their _id forms: wmma_q8k / WStageK,
// src/matvec_q.hip:2975-3348), which forms int32 sub-block dots, isum += sc * dot, and one float epilogue
// d_x (d_w isum - dmin msum) per 256-value super-block.
//
// MI355X-first design:
//   * the weight's integer part per value -- Q4_K / Q5_K sc_j q (<= 945 / 1953), Q6_K sc_g (q - 32) (|.| <= 4096),
//     IQ4_XS ls_j level (|.| <= 4064) -- is split exactly into two int8 planes: P = 128 hi + lo (lo in 0..127), or
//     for Q4_K P = 8 (sh q) + (sl q) with sc = 8 sh + sl. Two int8 MFMA chains over the super-block then give
//     H = sum hi x and L = sum lo x, and isum = 128 H + L (Q4_K: 8 H + L) is the
//     reference's exact integer with no per-sub-block vector work: the sub-block and group scales ride inside
//     the operands, so the matrix core, not the vector ALU, bounds the loop;
//   * Q4_K / Q5_K's min term msum = sum_j m_j sum32_j is one v_mfma_f32_32x32x8_f16 per 32 x 32 tile and
//     super-block on the activation's 32-value sums (|.| <= 4064, exact in fp16) against the 6-bit mins;
//   * per output and super-block: y += dK (d isum - dmin msum);
//   * the Q8_K activation is read where qmatvec_quantize (or a producer) left it: int8 values, dK, 16-value
//     sums. No pre-pass and no workspace;
//   * tokens are the MFMA's rows and weight rows its columns, so a lane's 16 outputs share one weight row:
//     d and dmin are per-lane values. Workgroup tile 128 tokens x 64 weight rows (4 waves of 64 x 32), two
//     workgroups per CU: they are not synchronised with each other, so one's MFMAs run while the other stages
//     or finishes a super-block. K stages of 64 double-buffered in LDS with one barrier a stage; each stage's
//     global loads are issued two stages ahead (two register sets). The dense grid is renumbered XCD by XCD
//     (xcd_tile). MoE expert tiles: 64 tokens x 64 rows (4 waves of 32 x 32).
#include <atomic>
#include <type_traits>

#include "device.h"
#include "kernels.h"

namespace pq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef short s2 __attribute__((ext_vector_type(2)));

constexpr int I8_ROW = 80;     // LDS bytes per row of a stage (64 + 16: conflict-free 16-byte fragment reads)
constexpr int I8_N = 64;       // weight rows per workgroup
constexpr int I8_THREADS = 256;
constexpr int I8_GROUP = 4;    // token tiles that advance together over the row tiles on an XCD (xcd_tile)

// ---------------------------------------------------------------- the two int8 planes of four values
// The four unsigned bytes of w, each minus `bias`, as 16-bit lanes (v = byte - bias), times s (both exact in 16
// bits: |v s| < 2^15); P = v s is split as hi = (P >> 7) - hcorr (arithmetic shift) and lo = P & 127, and the four
// hi and four lo bytes are packed. Every 16-bit step is a packed 16-bit operation (no borrow crosses lanes).
__device__ __forceinline__ void planes4(uint32_t w, short bias, short s, short hcorr, uint32_t &hi, uint32_t &lo) {
    const s2 v01 = __builtin_bit_cast(s2, __builtin_amdgcn_perm(0u, w, 0x0c010c00u)) - s2{bias, bias};
    const s2 v23 = __builtin_bit_cast(s2, __builtin_amdgcn_perm(0u, w, 0x0c030c02u)) - s2{bias, bias};
    const s2 p01 = v01 * s2{s, s}, p23 = v23 * s2{s, s};
    lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, p23), __builtin_bit_cast(uint32_t, p01), 0x06040200u) &
         0x7f7f7f7fu;
    const s2 h01 = (p01 >> (short)7) - s2{hcorr, hcorr}, h23 = (p23 >> (short)7) - s2{hcorr, hcorr};
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h23), __builtin_bit_cast(uint32_t, h01), 0x06040200u);
}

// IQ4_XS indices (one per byte, 0..15) -> their levels + 128 (kvalues_iq4nl + 128: 1 .. 241, unsigned bytes)
__device__ __forceinline__ uint32_t iq4nl4_u(uint32_t n) {
    const uint32_t sel = n & 0x07070707u, upper = (n & 0x08080808u) >> 1;
    const uint32_t a = __builtin_amdgcn_perm(0x766a5d4fu, 0x3f2d1801u, sel);  // indices 0..7
    const uint32_t b = __builtin_amdgcn_perm(0xf1d9c5b5u, 0xa6998d81u, sel);  // indices 8..15
    return __builtin_amdgcn_perm(b, a, 0x03020100u | upper);
}

// ---------------------------------------------------------------- weight stages
// Stage c (0..3) of super-block s holds K values 256 s + 64 c .. + 63 of weight rows n0 .. n0 + 63 in LDS as
// two planes [row][80 bytes] (hi, lo), in natural K order. Thread t stages row t / 4, quarter p = t & 3; at c == 0
// it also writes the row's super-block factors (d, dmin) and, for Q4_K / Q5_K, its 8 mins (fp16).
struct WDst {
    int8_t *hi, *lo;     // the stage's planes, row 0
    float2 *dd;          // the super-block's (d, dmin) per row
    _Float16 *mn;        // its mins, 8 per row
};

template <int TYPE>
struct I8Stage;

// four bytes (each <= 15) times s (<= 7) in place: the products stay below 128, so a packed 16-bit multiply of
// (b0 + 256 b1, b2 + 256 b3) by s carries nothing across bytes
__device__ __forceinline__ uint32_t bytes_times(uint32_t w, short s) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(s2, w) * s2{s, s});
}

// Q4_K / Q5_K: chunk c of qs (32 bytes; Q5_K: also qh, 32 bytes): low nibbles sub-block 2 c (stage K 0..31), high
// nibbles 2 c + 1 (32..63). Quarter p takes values 8 p .. + 7 of both sub-blocks (qs bytes 8 p .. + 7 of the chunk).
// Q4_K splits the 6-bit scale instead of the product: sc = 8 sh + sl (sh, sl <= 7), planes sh q and sl q (<= 105),
// isum = 8 H + L (two packed multiplies per four values). Q5_K's 5-bit levels (sc q <= 1953) take the product
// split, P = 128 hi + lo.
template <bool Q5>
struct I8StageK {
    static constexpr int BB = Q5 ? 176 : 144, QS = Q5 ? 48 : 16;
    static constexpr bool MINS = true;
    static constexpr int SHIFT = Q5 ? 7 : 3;  // isum = (H << SHIFT) + L
    // the super-block's 16 header bytes (d, dmin, the 12 scale bytes), loaded once for its four stages (hdr) and
    // kept apart from the stage's loads: loaded again at every stage they were two fifths of a stage's bytes
    static constexpr bool HDR = true;
    __device__ static uint4 hdr(const uint8_t *row, int s) { return *(const uint4 *)(row + s * BB); }
    struct Raw {
        uint4 h;    // (set from the kept header at the commit)
        uint2 q;
        uint2 qh;  // (Q5_K only)
    };
    __device__ static void load(const uint8_t *row, int s, int c, Raw &r) {
        const int p = threadIdx.x & 3;
        const uint8_t *b = row + s * BB;
        r.q = *(const uint2 *)(b + QS + 32 * c + 8 * p);
        if constexpr (Q5) r.qh = *(const uint2 *)(b + 16 + 8 * p);
        else r.qh = make_uint2(0u, 0u);
    }
    __device__ static void store(const Raw &r, int c, const WDst &o) {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        // the 8 six-bit scales and mins as bytes of two dwords each (sub-blocks 0..3, 4..7), from the scale dwords
        // y, z, w (bytes 4..15 of the block): scale j < 4 = y byte j & 63, j >= 4 = (w byte & 15) | (y byte >> 6)
        // << 4; min j < 4 = z byte j & 63, j >= 4 = (w byte >> 4) | (z byte >> 6) << 4
        const uint32_t y = r.h.y, z = r.h.z, w = r.h.w;
        const uint32_t scw = c < 2 ? y & 0x3f3f3f3fu : (w & 0x0f0f0f0fu) | ((y >> 2) & 0x30303030u);
        const int sa = (int)((scw >> (16 * (c & 1))) & 0xffu), sb = (int)((scw >> (16 * (c & 1) + 8)) & 0xffu);
        const uint32_t q[2] = {r.q.x, r.q.y};
        uint32_t qh[2] = {0u, 0u};
        if constexpr (Q5) {
            qh[0] = r.qh.x;
            qh[1] = r.qh.y;
        }
        uint32_t ha[2], la[2], hb[2], lb[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            uint32_t l4 = q[k] & 0x0f0f0f0fu, h4 = (q[k] >> 4) & 0x0f0f0f0fu;
            if (Q5) {
                l4 |= ((qh[k] >> (2 * c)) & 0x01010101u) << 4;
                h4 |= ((qh[k] >> (2 * c + 1)) & 0x01010101u) << 4;
            }
            if (Q5) {
                planes4(l4, 0, (short)sa, 0, ha[k], la[k]);
                planes4(h4, 0, (short)sb, 0, hb[k], lb[k]);
            } else {
                ha[k] = bytes_times(l4, (short)(sa >> 3));
                la[k] = bytes_times(l4, (short)(sa & 7));
                hb[k] = bytes_times(h4, (short)(sb >> 3));
                lb[k] = bytes_times(h4, (short)(sb & 7));
            }
        }
        int8_t *dh = o.hi + row * I8_ROW + 8 * p, *dl = o.lo + row * I8_ROW + 8 * p;
        *(uint2 *)dh = make_uint2(ha[0], ha[1]);
        *(uint2 *)dl = make_uint2(la[0], la[1]);
        *(uint2 *)(dh + 32) = make_uint2(hb[0], hb[1]);
        *(uint2 *)(dl + 32) = make_uint2(lb[0], lb[1]);
        if (c == 0) {
            if (p == 0) o.dd[row] = make_float2(h2f(r.h.x & 0xffffu), h2f(r.h.x >> 16));
            if (p < 2) {
                const uint32_t mw = p == 0 ? z & 0x3f3f3f3fu : ((w >> 4) & 0x0f0f0f0fu) | ((z >> 2) & 0x30303030u);
                h4 m;
#pragma unroll
                for (int i = 0; i < 4; ++i) m[i] = (_Float16)(float)((mw >> (8 * i)) & 0xffu);
                *(h4 *)(o.mn + row * 8 + 4 * p) = m;
            }
        }
    }
};
template <>
struct I8Stage<TY_Q4_K> : I8StageK<false> {};
template <>
struct I8Stage<TY_Q5_K> : I8StageK<true> {};

// Q6_K (210 bytes, 2-aligned): stage c is half h = c / 2 of the super-block, values 128 h + 64 (c & 1) + 0..63:
// K 0..31 from ql[64 h + l] and K 32..63 from ql[64 h + 32 + l] (low nibbles for even c, high for odd), each with
// two bits of qh[32 h + l] (bits 0-1 / 2-3 for even c, 4-5 / 6-7 for odd); group scale sc[4 c + 2 (K >= 32) + (l >=
// 16)]. Quarter p takes l = 8 p .. + 7; the dwords are read from the 4-aligned address at or below the bytes.
template <>
struct I8Stage<TY_Q6_K> {
    static constexpr int BB = 210;
    static constexpr bool MINS = false, HDR = false;
    static constexpr int SHIFT = 7;
    struct Raw {
        uint32_t a[3], b[3], h[3];
        uint32_t sc, d, off;
    };
    __device__ static void load(const uint8_t *row, int s, int c, Raw &r) {
        const int p = threadIdx.x & 3, h = c >> 1;
        const uint8_t *b = row + s * BB;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *ba = b - r.off;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            r.a[k] = ld32(ba + 64 * h + 8 * p + 4 * k);
            r.b[k] = ld32(ba + 64 * h + 32 + 8 * p + 4 * k);
            r.h[k] = ld32(ba + 128 + 32 * h + 8 * p + 4 * k);
        }
        // the scales of groups 4 c .. 4 c + 3 and d, read as 2-byte halves (the block is 2-aligned)
        r.sc = (uint32_t)*(const uint16_t *)(b + 192 + 4 * c) | (uint32_t)*(const uint16_t *)(b + 194 + 4 * c) << 16;
        r.d = *(const uint16_t *)(b + 208);
    }
    __device__ static void store(const Raw &r, int c, const WDst &o) {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        const int sh = (c & 1) ? 4 : 0, g = p >> 1;
        const int sca = (int)(int8_t)((r.sc >> (8 * g)) & 0xffu), scb = (int)(int8_t)((r.sc >> (8 * (2 + g))) & 0xffu);
        uint32_t ha[2], la[2], hb[2], lb[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t A = align_bytes(r.a[k + 1], r.a[k], r.off), B = align_bytes(r.b[k + 1], r.b[k], r.off);
            const uint32_t H = align_bytes(r.h[k + 1], r.h[k], r.off);
            const uint32_t qa = ((A >> sh) & 0x0f0f0f0fu) | (((H >> sh) & 0x03030303u) << 4);
            const uint32_t qb = ((B >> sh) & 0x0f0f0f0fu) | (((H >> (sh + 2)) & 0x03030303u) << 4);
            planes4(qa, 32, (short)sca, 0, ha[k], la[k]);  // sc (q - 32)
            planes4(qb, 32, (short)scb, 0, hb[k], lb[k]);
        }
        int8_t *dh = o.hi + row * I8_ROW + 8 * p, *dl = o.lo + row * I8_ROW + 8 * p;
        *(uint2 *)dh = make_uint2(ha[0], ha[1]);
        *(uint2 *)dl = make_uint2(la[0], la[1]);
        *(uint2 *)(dh + 32) = make_uint2(hb[0], hb[1]);
        *(uint2 *)(dl + 32) = make_uint2(lb[0], lb[1]);
        if (c == 0 && p == 0) o.dd[row] = make_float2(h2f(r.d), 0.0f);
    }
};

// IQ4_XS (136 bytes, 8-aligned): stage c holds sub-blocks 2 c (K 0..31) and 2 c + 1 (K 32..63); quarter p takes
// sub-block j = 2 c + (p >> 1), qs bytes 16 j + 8 (p & 1) .. + 7: low nibbles K 32 (p >> 1) + 8 (p & 1) + 0..7,
// high nibbles 16 further on. P = ls level = ls (u - 128) with u = level + 128: lo of ls u, hi of ls u minus ls.
template <>
struct I8Stage<TY_IQ4_XS> {
    static constexpr int BB = 136;
    static constexpr bool MINS = false, HDR = false;
    static constexpr int SHIFT = 7;
    struct Raw {
        uint2 h, q;
    };
    __device__ static void load(const uint8_t *row, int s, int c, Raw &r) {
        const int p = threadIdx.x & 3;
        const uint8_t *b = row + s * BB;
        r.h = *(const uint2 *)b;
        r.q = *(const uint2 *)(b + 8 + 16 * (2 * c + (p >> 1)) + 8 * (p & 1));
    }
    __device__ static void store(const Raw &r, int c, const WDst &o) {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        const int ls = iq4xs_scale(r.h.x >> 16, r.h.y, 2 * c + (p >> 1));
        const uint32_t q[2] = {r.q.x, r.q.y};
        uint32_t hl[2], ll[2], hh[2], lh[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            // level = u - 128: P = ls level = ls u - 128 ls, so lo is that of ls u and hi is (ls u >> 7) - ls
            planes4(iq4nl4_u(q[k] & 0x0f0f0f0fu), 0, (short)ls, (short)ls, hl[k], ll[k]);
            planes4(iq4nl4_u((q[k] >> 4) & 0x0f0f0f0fu), 0, (short)ls, (short)ls, hh[k], lh[k]);
        }
        const int k0 = 32 * (p >> 1) + 8 * (p & 1);
        int8_t *dh = o.hi + row * I8_ROW + k0, *dl = o.lo + row * I8_ROW + k0;
        *(uint2 *)dh = make_uint2(hl[0], hl[1]);
        *(uint2 *)dl = make_uint2(ll[0], ll[1]);
        *(uint2 *)(dh + 16) = make_uint2(hh[0], hh[1]);
        *(uint2 *)(dl + 16) = make_uint2(lh[0], lh[1]);
        if (c == 0 && p == 0) o.dd[row] = make_float2(h2f(r.h.x & 0xffffu), 0.0f);
    }
};

// ---------------------------------------------------------------- the GEMM
// a stage type's super-block header, loaded once for its four stages (HDR), and its store with that header
template <class S>
__device__ __forceinline__ uint4 stage_hdr(const uint8_t *row, int s) {
    if constexpr (S::HDR) return S::hdr(row, s);
    else return make_uint4(0u, 0u, 0u, 0u);
}
template <class S>
__device__ __forceinline__ void stage_store(const typename S::Raw &raw, uint4 h, int c, const WDst &o) {
    if constexpr (S::HDR) {
        typename S::Raw r = raw;
        r.h = h;
        S::store(r, c, o);
    } else {
        S::store(raw, c, o);
    }
}

// WI x 1 tiles of 32 x 32 per wave (tokens x rows); 4 waves, WT along the tokens and 4 / WT along the rows:
// BT = 32 WI WT tokens and I8_N = 32 (4 / WT) weight rows a workgroup.
template <int WI, int WT>
struct I8Geo {
    static_assert(32 * (4 / WT) == I8_N, "4 waves cover the workgroup's rows");
    static constexpr int BT = 32 * WI * WT;               // tokens per workgroup
    static constexpr int XB = BT * I8_ROW;                // token stage bytes
    static constexpr int WB = I8_N * I8_ROW;              // one weight plane's stage bytes
    static constexpr int OFF_W = 2 * XB;
    static constexpr int OFF_BS = OFF_W + 4 * WB;         // [2][BT][8] fp16
    static constexpr int OFF_MN = OFF_BS + 2 * BT * 16;   // [2][I8_N][8] fp16
    static constexpr int OFF_DD = OFF_MN + 2 * I8_N * 16; // [2][I8_N] float2
    static constexpr int OFF_DK = OFF_DD + 2 * I8_N * 8;  // [2][BT] float
    static constexpr int BYTES = OFF_DK + 2 * BT * 4;
};

template <int V>
using IC = std::integral_constant<int, V>;

// the first or the second of two objects, chosen at compile time
template <int B, class T>
__device__ __forceinline__ T &pick2(T &a, T &b) {
    if constexpr (B) return b;
    else return a;
}

template <int TYPE, int WI, int WT, bool MOE, bool CAP>
__global__ void __launch_bounds__(I8_THREADS, 2) k_gemm_i8kq(GemmArgs a) {
    using S = I8Stage<TYPE>;
    using G = I8Geo<WI, WT>;
    constexpr int BT = G::BT;
    constexpr bool MINS = S::MINS;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    int n0, e = 0;
    TokMap tm;
    const int32_t *orow = nullptr;
    if constexpr (MOE) {  // grid (row tiles, tiles)
        const int k = blockIdx.y;
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        const int st = a.tile_start[k];
        tm = {a.in_rows + st, 0, a.tile_n[k]};
        orow = a.out_rows + st;
        n0 = moe_row_tile(a) * I8_N;
    } else {              // grid (token tiles, row tiles), renumbered XCD by XCD
        int tt, rt;
        xcd_tile(tt, rt, I8_GROUP);
        tm = {nullptr, tt * BT, BT};
        n0 = rt * I8_N;
    }
    const int K = a.K, nsb = K / 256;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wt0 = (wave % WT) * 32 * WI, wn0 = (wave / WT) * 32;  // the wave's token and row offsets

    // token rows of this tile: real rows for j < n (dense: < T), else a repeat of a valid row (outputs not stored)
    auto trow = [&](int j) -> long long {
        if constexpr (MOE) return tm.rows[j < tm.n ? j : 0];
        const int t = tm.base + j;
        return t < a.T ? t : a.T - 1;
    };
    // Every pointer a thread stages from, computed once. Weights: row n0 + tid / 4 (rows past the end repeat the
    // last; their outputs are not stored). Tokens: 16 bytes (chunk tid & 3) of token rows tid / 4 + 64 i (BT / 64
    // rows). Super-block data: token tid / 2 (tid < 2 BT): 8 of its 16 group sums (half tid & 1) and dK.
    const int wr = n0 + (tid >> 2);
    const uint8_t *wrow = a.W + ((long long)e * a.N + (wr < a.N ? wr : a.N - 1)) * a.row_bytes;
    constexpr int XR = BT / 64;
    static_assert(BT % 64 == 0, "whole rounds of token staging");
    constexpr bool xon = true;
    const int8_t *xsrc[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) xsrc[i] = a.xq + trow((tid >> 2) + 64 * i) * K + 16 * (tid & 3);
    const bool son = tid < 2 * BT;
    const long long srow = trow(son ? tid >> 1 : 0);
    const int32_t *bsrc = a.xsum + srow * (K / 16) + 8 * (tid & 1);
    const float *ksrc = a.dx + srow * nsb;

    // the global loads of one stage, held in registers until committed to LDS; two sets: stage st's loads are
    // issued two stages ahead, into set st & 1
    struct Pre {
        typename S::Raw raw;
        uint4 xv[XR];
        int4 bv[2];
        float kv;
    };
    Pre P0, P1;
    // (HDR) the header of the super-block being committed (Hc) and of the next one (Hn: loaded with its stage 0,
    // which its commit reads; Hc takes it when that super-block's steps begin)
    uint4 Hc = make_uint4(0u, 0u, 0u, 0u), Hn = Hc;
    auto issue = [&](auto cc, Pre &p, int s) {
        constexpr int c = decltype(cc)::value;
        if constexpr (c == 0) Hn = stage_hdr<S>(wrow, s);
        S::load(wrow, s, c, p.raw);
#pragma unroll
        for (int i = 0; i < XR; ++i) p.xv[i] = *(const uint4 *)(xsrc[i] + 256 * s + 64 * c);
        if constexpr (c == 0) {
            if constexpr (MINS) {
#pragma unroll
                for (int i = 0; i < 2; ++i) p.bv[i] = *(const int4 *)(bsrc + 16 * s + 4 * i);
            }
            p.kv = ksrc[s];
        }
    };
    auto commit = [&](auto cc, const Pre &p, int s) {
        constexpr int c = decltype(cc)::value, buf = c & 1;
        const int sb = s & 1;
        int8_t *sx = (int8_t *)smem + buf * G::XB;
        if (xon) {
#pragma unroll
            for (int i = 0; i < XR; ++i) *(uint4 *)(sx + ((tid >> 2) + 64 * i) * I8_ROW + 16 * (tid & 3)) = p.xv[i];
        }
        WDst o;
        o.hi = (int8_t *)smem + G::OFF_W + (2 * buf) * G::WB;
        o.lo = o.hi + G::WB;
        o.dd = (float2 *)(smem + G::OFF_DD) + sb * I8_N;
        o.mn = (_Float16 *)(smem + G::OFF_MN) + sb * I8_N * 8;
        stage_store<S>(p.raw, c == 0 ? Hn : Hc, c, o);
        if constexpr (c == 0) {
            if (son) {
                if constexpr (MINS) {  // the 32-value sums of sub-blocks 4 (tid & 1) .. + 3
                    h4 v4;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        v4[j] = (_Float16)(float)(p.bv[j >> 1][2 * (j & 1)] + p.bv[j >> 1][2 * (j & 1) + 1]);
                    *(h4 *)((_Float16 *)(smem + G::OFF_BS) + (sb * BT + (tid >> 1)) * 8 + 4 * (tid & 1)) = v4;
                }
                if ((tid & 1) == 0) ((float *)(smem + G::OFF_DK))[sb * BT + (tid >> 1)] = p.kv;
            }
        }
    };

    v16f acc[WI];
    v16i H[WI], L[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    const int fr = lane & 31, fh = 16 * (lane >> 5);  // fragment row and K half of this lane

    // stage c of super-block s: its two 32-value sub-blocks' MFMAs (the first of a super-block start from zero)
    auto compute = [&](auto cc) {
        constexpr int c = decltype(cc)::value;
        const int8_t *sx = (const int8_t *)smem + (c & 1) * G::XB;
        const int8_t *swh = (const int8_t *)smem + G::OFF_W + (2 * (c & 1)) * G::WB, *swl = swh + G::WB;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int kk = 32 * b + fh;
            v4i fa[WI];
#pragma unroll
            for (int i = 0; i < WI; ++i) fa[i] = *(const v4i *)(sx + (wt0 + 32 * i + fr) * I8_ROW + kk);
            const v4i fbh = *(const v4i *)(swh + (wn0 + fr) * I8_ROW + kk);
            const v4i fbl = *(const v4i *)(swl + (wn0 + fr) * I8_ROW + kk);
#pragma unroll
            for (int i = 0; i < WI; ++i) {
                if (c == 0 && b == 0) {
                    const v16i z = {};
                    H[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fbh, z, 0, 0, 0);
                    L[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fbl, z, 0, 0, 0);
                } else {
                    H[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fbh, H[i], 0, 0, 0);
                    L[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fbl, L[i], 0, 0, 0);
                }
            }
        }
    };

    // super-block epilogue: y += dK (d isum - dmin msum), isum = 2^SHIFT H + L. Lane: weight row wn0 + fr; tokens
    // wt0 + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4 for its 16 values r.
    auto epilogue = [&](int s) {
        const int sb = s & 1;
        const float2 *dd = (const float2 *)(smem + G::OFF_DD) + sb * I8_N;
        const float *dk = (const float *)(smem + G::OFF_DK) + sb * BT;
        const _Float16 *bs = (const _Float16 *)(smem + G::OFF_BS) + sb * BT * 8;
        const _Float16 *mn = (const _Float16 *)(smem + G::OFF_MN) + sb * I8_N * 8;
        const int row = wn0 + fr;
        const float2 dw = dd[row];
        h4 fm;
        if constexpr (MINS) fm = *(const h4 *)(mn + row * 8 + 4 * (lane >> 5));
#pragma unroll
        for (int i = 0; i < WI; ++i) {
            v16f ms = {};
            if constexpr (MINS) {
                const h4 fs = *(const h4 *)(bs + (wt0 + 32 * i + fr) * 8 + 4 * (lane >> 5));
                ms = __builtin_amdgcn_mfma_f32_32x32x8f16(fs, fm, ms, 0, 0, 0);
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int t0 = wt0 + 32 * i + 8 * g + 4 * (lane >> 5);
                const float4 k4 = *(const float4 *)(dk + t0);
                const float kr[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 4 * g + q;
                    const int isum = (H[i][r] << S::SHIFT) + L[i][r];
                    if constexpr (CAP) {
                        const int tt = t0 + q;
                        long long t = -1;
                        if constexpr (MOE) t = tt < tm.n ? orow[tt] : -1;
                        else t = tm.base + tt < a.T ? tm.base + tt : -1;
                        if (t >= 0 && n0 + row < a.N) a.cap[(t * a.N + n0 + row) * nsb + s] = isum;
                    }
                    float v = dw.x * (float)isum;
                    if constexpr (MINS) v = __builtin_fmaf(-dw.y, ms[r], v);
                    acc[i][r] = __builtin_fmaf(kr[q], v, acc[i][r]);
                }
            }
        }
    };

    // stages st = 4 s + c; step c issues stage st + 2 (into set st & 1, whose stage st went to LDS in the previous
    // step), computes stage st (and the super-block's epilogue after its last stage), and commits stage st + 1 (set
    // (st + 1) & 1) before the barrier. UNC (Q6_K, IQ4_XS): past the last super-block the issues load its stages
    // again and the last step commits one of them into buffers nothing reads afterwards, so the loop body has no
    // branch and the waits count the loads exactly, and the loads are kept ahead of the MFMAs (sched_barrier):
    // Q6_K 9728 x 2560 / 2560 x 9728 x 2427 218 / 230 -> 210 / 205 us, IQ4_XS 204 -> 200 us. Q4_K and Q5_K keep the
    // branches (the same form measured 197 -> 204 and 216 -> 222 us on 9728 x 2560). One box, interleaved.
    constexpr bool UNC = TYPE == TY_Q6_K || TYPE == TY_IQ4_XS;
    auto step = [&](auto cc, int s) {
        constexpr int c = decltype(cc)::value;
        Pre &pi = pick2<c & 1>(P0, P1);
        Pre &pc = pick2<(c + 1) & 1>(P0, P1);
        if constexpr (c < 2) issue(IC<c + 2>{}, pi, s);
        else if (UNC || s + 1 < nsb) issue(IC<c - 2>{}, pi, s + 1 < nsb ? s + 1 : nsb - 1);
        if constexpr (UNC) __builtin_amdgcn_sched_barrier(0);
        compute(cc);
        if constexpr (c == 3) epilogue(s);
        if constexpr (c < 3) commit(IC<c + 1>{}, pc, s);
        else if (UNC || s + 1 < nsb) commit(IC<0>{}, pc, s + 1);
        __syncthreads();
    };

    issue(IC<0>{}, P0, 0);
    issue(IC<1>{}, P1, 0);
    commit(IC<0>{}, P0, 0);
    __syncthreads();
    for (int s = 0; s < nsb; ++s) {
        Hc = Hn;  // (HDR only; otherwise dead)
        step(IC<0>{}, s);
        step(IC<1>{}, s);
        step(IC<2>{}, s);
        step(IC<3>{}, s);
    }

    // store: lane's weight row n0 + wn0 + fr, tokens as above
    const float sc = a.es ? a.es[e] : a.osc;
    const int n = n0 + wn0 + fr;
    if (n < a.N) {
#pragma unroll
        for (int i = 0; i < WI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tt = wt0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                long long yrow;
                if constexpr (MOE) {
                    if (tt >= tm.n) continue;
                    yrow = (long long)orow[tt] * a.N;
                } else {
                    const int t = tm.base + tt;
                    if (t >= a.T) continue;
                    yrow = (long long)t * a.ldy;
                }
                a.y[yrow + n] = acc[i][r] * sc;
            }
    }
}

// ---------------------------------------------------------------- per-block GEMM (Q8_0, MXFP4)
// The reference's per-block form (src/matvec_q.hip:2566-2973, WStageQ8_0): one int8 MFMA per 32-value block gives
// the exact int32 block dot of each (token, row), and y += (e_w d_x) dot. The weight scale is per row and block (a
// per-lane value), d_x per token and block. Weights: Q8_0's int8 values as they are, MXFP4's E2M1 levels doubled
// (int8 -12..12; the E8M0 decoder's scale is already halved). Stage = two blocks (64 K); geometry, staging and the
// two-stage-ahead loads as the K-quant GEMM above; the Q8_0 activation (q0, d0) is read in place.
struct BDst {
    int8_t *w;   // the stage's values, row 0 (one plane)
    float *ew;   // the stage's weight scales [2 blocks][I8_N]
};

template <int TYPE>
struct I8Blk;

// Q8_0 (34-byte blocks, 2-aligned): quarter p takes block p >> 1, values 16 (p & 1) .. + 15 (bytes 2 + 16 (p & 1)
// of the block), read as five dwords from the 4-aligned address at or below them
template <>
struct I8Blk<TY_Q8_0> {
    static constexpr int BPB = 34;  // bytes per block
    struct Raw {
        uint32_t v[5];
        uint32_t off, e;
    };
    __device__ static void load(const uint8_t *row, int blk0, Raw &r) {
        const int p = threadIdx.x & 3;
        const uint8_t *b = row + (blk0 + (p >> 1)) * BPB;
        const uint8_t *v = b + 2 + 16 * (p & 1);
        r.off = (uint32_t)((uintptr_t)v & 3u);
        const uint8_t *va = v - r.off;
#pragma unroll
        for (int k = 0; k < 5; ++k) r.v[k] = ld32(va + 4 * k);
        r.e = *(const uint16_t *)b;
    }
    __device__ static void store(const Raw &r, const BDst &o) {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = align_bytes(r.v[k + 1], r.v[k], r.off);
        *(uint4 *)(o.w + row * I8_ROW + 16 * p) = make_uint4(q[0], q[1], q[2], q[3]);
        if ((p & 1) == 0) o.ew[(p >> 1) * I8_N + row] = h2f(r.e);
    }
};

// MXFP4 (17-byte blocks: E8M0 scale, then 16 value bytes: value j < 16 the low nibble of byte 1 + j, j >= 16 the
// high nibble of byte 1 + j - 16): quarter p takes block p >> 1, values 16 (p & 1) .. + 15
template <>
struct I8Blk<TY_MXFP4> {
    static constexpr int BPB = 17;
    struct Raw {
        uint32_t v[5];
        uint32_t off, e;
    };
    __device__ static void load(const uint8_t *row, int blk0, Raw &r) {
        const int p = threadIdx.x & 3;
        const uint8_t *b = row + (blk0 + (p >> 1)) * BPB;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *ba = b - r.off;
#pragma unroll
        for (int k = 0; k < 5; ++k) r.v[k] = ld32(ba + 4 * k);
        r.e = 0;
    }
    __device__ static void store(const Raw &r, const BDst &o) {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        uint32_t w[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) w[k] = align_bytes(k < 4 ? r.v[k + 1] : 0u, r.v[k], r.off);
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t b = align_bytes(w[k + 1], w[k], 1);  // value bytes 4 k .. 4 k + 3
            q[k] = (p & 1) ? (uint32_t)fp4x4_hi<12>(b) : (uint32_t)fp4x4_lo<12>(b);
        }
        *(uint4 *)(o.w + row * I8_ROW + 16 * p) = make_uint4(q[0], q[1], q[2], q[3]);
        if ((p & 1) == 0) o.ew[(p >> 1) * I8_N + row] = e8m0_half(w[0]);
    }
};

template <int TYPE, int WI, int WT, bool MOE, bool CAP>
__global__ void __launch_bounds__(I8_THREADS, 2) k_gemm_i8blk(GemmArgs a) {
    using S = I8Blk<TYPE>;
    constexpr int BT = 32 * WI * WT;
    static_assert(32 * (4 / WT) == I8_N, "4 waves cover the workgroup's rows");
    constexpr int XB = BT * I8_ROW, WB = I8_N * I8_ROW;
    constexpr int OFF_W = 2 * XB, OFF_EW = OFF_W + 2 * WB, OFF_DX = OFF_EW + 2 * 2 * I8_N * 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    int n0, e = 0;
    TokMap tm;
    const int32_t *orow = nullptr;
    if constexpr (MOE) {
        const int k = blockIdx.y;
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        const int st = a.tile_start[k];
        tm = {a.in_rows + st, 0, a.tile_n[k]};
        orow = a.out_rows + st;
        n0 = moe_row_tile(a) * I8_N;
    } else {
        int tt, rt;
        xcd_tile(tt, rt, I8_GROUP);
        tm = {nullptr, tt * BT, BT};
        n0 = rt * I8_N;
    }
    const int K = a.K, nst = K / 64, nb = K / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wt0 = (wave % WT) * 32 * WI, wn0 = (wave / WT) * 32;
    auto trow = [&](int j) -> long long {
        if constexpr (MOE) return tm.rows[j < tm.n ? j : 0];
        const int t = tm.base + j;
        return t < a.T ? t : a.T - 1;
    };
    const int wr = n0 + (tid >> 2);
    const uint8_t *wrow = a.W + ((long long)e * a.N + (wr < a.N ? wr : a.N - 1)) * a.row_bytes;
    constexpr int XR = BT / 64;
    const int8_t *xsrc[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) xsrc[i] = a.xq + trow((tid >> 2) + 64 * i) * K + 16 * (tid & 3);
    // token scales: thread t < 2 BT stages block t / BT of the stage for token t % BT (the other threads load the
    // same value as thread t % (2 BT) and store nothing: no branch around the load)
    const bool don = tid < 2 * BT;
    const float *dsrc = a.dx + trow(tid % BT) * nb + ((tid % (2 * BT)) / BT);

    struct Pre {
        typename S::Raw raw;
        uint4 xv[XR];
        float dv;
    };
    Pre P0, P1;
    auto issue = [&](Pre &p, int st) {
        S::load(wrow, 2 * st, p.raw);
#pragma unroll
        for (int i = 0; i < XR; ++i) p.xv[i] = *(const uint4 *)(xsrc[i] + 64 * st);
        p.dv = dsrc[2 * st];
    };
    auto commit = [&](auto cc, const Pre &p) {
        constexpr int buf = decltype(cc)::value;
        int8_t *sx = (int8_t *)smem + buf * XB;
#pragma unroll
        for (int i = 0; i < XR; ++i) *(uint4 *)(sx + ((tid >> 2) + 64 * i) * I8_ROW + 16 * (tid & 3)) = p.xv[i];
        BDst o;
        o.w = (int8_t *)smem + OFF_W + buf * WB;
        o.ew = (float *)(smem + OFF_EW) + buf * 2 * I8_N;
        S::store(p.raw, o);
        if (don) ((float *)(smem + OFF_DX))[buf * 2 * BT + tid] = p.dv;  // [buf][block][token]
    };

    v16f acc[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    const int fr = lane & 31, fh = 16 * (lane >> 5);

    // stage st (blocks 2 st, 2 st + 1): per block and tile a fresh MFMA, then y += (e_w d_x) dot
    auto compute = [&](auto cc, int st) {
        constexpr int buf = decltype(cc)::value;
        const int8_t *sx = (const int8_t *)smem + buf * XB, *sw = (const int8_t *)smem + OFF_W + buf * WB;
        const float *ew = (const float *)(smem + OFF_EW) + buf * 2 * I8_N;
        const float *dx = (const float *)(smem + OFF_DX) + buf * 2 * BT;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int kk = 32 * b + fh;
            const v4i fb = *(const v4i *)(sw + (wn0 + fr) * I8_ROW + kk);
            const float e_w = ew[b * I8_N + wn0 + fr];
#pragma unroll
            for (int i = 0; i < WI; ++i) {
                const v4i fa = *(const v4i *)(sx + (wt0 + 32 * i + fr) * I8_ROW + kk);
                const v16i z = {};
                const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, z, 0, 0, 0);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int t0 = wt0 + 32 * i + 8 * g + 4 * (lane >> 5);
                    const float4 x4 = *(const float4 *)(dx + b * BT + t0);
                    const float xr[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int r = 4 * g + q;
                        if constexpr (CAP) {
                            const int tt = t0 + q, n = n0 + wn0 + fr;
                            long long t = -1;
                            if constexpr (MOE) t = tt < tm.n ? orow[tt] : -1;
                            else t = tm.base + tt < a.T ? tm.base + tt : -1;
                            if (t >= 0 && n < a.N) a.cap[(t * a.N + n) * nb + 2 * st + b] = d[r];
                        }
                        acc[i][r] = __builtin_fmaf(e_w * xr[q], (float)d[r], acc[i][r]);
                    }
                }
            }
        }
    };

    // stage st: issue st + 2 (set st & 1), compute st, commit st + 1 (set (st + 1) & 1), barrier. A stage past the
    // end loads the last one again, committed into the idle buffer and never read: a step has no branch around its
    // loads, so the waits count them exactly. (The odd last step stays inside the loop: peeled after it, the
    // compiler's schedule held 256 registers and spilled.)
    auto step = [&](auto cc, int st) {
        constexpr int c = decltype(cc)::value;
        Pre &pi = pick2<c>(P0, P1);
        Pre &pc = pick2<1 - c>(P0, P1);
        issue(pi, st + 2 < nst ? st + 2 : nst - 1);
        compute(cc, st);
        commit(IC<1 - c>{}, pc);
        __syncthreads();
    };

    issue(P0, 0);
    issue(P1, nst > 1 ? 1 : 0);
    commit(IC<0>{}, P0);
    __syncthreads();
    for (int st = 0; st < nst; st += 2) {
        step(IC<0>{}, st);
        if (st + 1 < nst) step(IC<1>{}, st + 1);
    }

    const float sc = a.es ? a.es[e] : a.osc;
    const int n = n0 + wn0 + fr;
    if (n < a.N) {
#pragma unroll
        for (int i = 0; i < WI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tt = wt0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                long long yrow;
                if constexpr (MOE) {
                    if (tt >= tm.n) continue;
                    yrow = (long long)orow[tt] * a.N;
                } else {
                    const int t = tm.base + tt;
                    if (t >= a.T) continue;
                    yrow = (long long)t * a.ldy;
                }
                a.y[yrow + n] = acc[i][r] * sc;
            }
    }
}

// ---------------------------------------------------------------- host side

bool gemm_i8kq_supported(int type) {
    return type == TY_Q4_K || type == TY_Q5_K || type == TY_Q6_K || type == TY_IQ4_XS || type == TY_Q8_0 ||
           type == TY_MXFP4;
}

int gemm_supported(int type) { return gemm_i8kq_supported(type) || gemm_split(type); }

int gemm_cap_unit(int type) {
    if (type == TY_Q4_K || type == TY_Q5_K || type == TY_Q6_K || type == TY_IQ4_XS) return 256;
    return type == TY_Q8_0 || type == TY_MXFP4 ? 32 : 0;
}

int gemm_i8kq_token_tile(bool moe) { return moe ? I8Geo<1, 2>::BT : I8Geo<2, 2>::BT; }

// the largest expert tile: the K-quants' planes cost vector work per tile (each tile builds its expert's planes), so
// their tiles go up to the dense 128 tokens (the launch takes the 64-token form for tiles of at most 64); Q8_0 and
// MXFP4 stage their weights as they are and keep 64
int gemm_i8_moe_tile(int type) {
    return type == TY_Q8_0 || type == TY_MXFP4 ? I8Geo<1, 2>::BT : I8Geo<2, 2>::BT;
}

int gemm_i8kq_rows() { return I8_N; }

template <int TYPE, int WI, int WT, bool MOE, bool CAP>
static hipError_t launch_i8kq_t(const GemmArgs &a, dim3 grid, hipStream_t stream) {
    using G = I8Geo<WI, WT>;
    auto k = k_gemm_i8kq<TYPE, WI, WT, MOE, CAP>;
    // the tile's LDS is above the default 64 KiB: the attribute is set once per instantiation and device (a
    // second setting, from a racing thread, is harmless)
    static std::atomic<unsigned long long> set_on{0};
    int dev = 0;
    if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    const unsigned long long bit = dev < 64 ? 1ull << dev : 0ull;  // (past 64 devices: set at every launch)
    if (!bit || !(set_on.load(std::memory_order_acquire) & bit)) {
        const hipError_t e = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, G::BYTES);
        if (e != hipSuccess) return e;
        set_on.fetch_or(bit, std::memory_order_release);
    }
    hipLaunchKernelGGL(k, grid, dim3(I8_THREADS), G::BYTES, stream, a);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_i8kq_type(const GemmArgs &a, dim3 grid, hipStream_t stream) {
    if (a.n_tiles && a.tt > I8Geo<1, 2>::BT)  // expert tiles of up to 128 entries
        return a.cap ? launch_i8kq_t<TYPE, 2, 2, true, true>(a, grid, stream)
                     : launch_i8kq_t<TYPE, 2, 2, true, false>(a, grid, stream);
    if (a.n_tiles)
        return a.cap ? launch_i8kq_t<TYPE, 1, 2, true, true>(a, grid, stream)
                     : launch_i8kq_t<TYPE, 1, 2, true, false>(a, grid, stream);
    return a.cap ? launch_i8kq_t<TYPE, 2, 2, false, true>(a, grid, stream)
                 : launch_i8kq_t<TYPE, 2, 2, false, false>(a, grid, stream);
}

template <int TYPE, int WI, int WT, bool MOE, bool CAP>
static hipError_t launch_i8blk_t(const GemmArgs &a, dim3 grid, hipStream_t stream) {
    constexpr int BT = 32 * WI * WT;
    constexpr int BYTES = 2 * BT * I8_ROW + 2 * I8_N * I8_ROW + 2 * 2 * I8_N * 4 + 2 * 2 * BT * 4;
    hipLaunchKernelGGL((k_gemm_i8blk<TYPE, WI, WT, MOE, CAP>), grid, dim3(I8_THREADS), BYTES, stream, a);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_i8blk_type(const GemmArgs &a, dim3 grid, hipStream_t stream) {
    if (a.n_tiles)
        return a.cap ? launch_i8blk_t<TYPE, 1, 2, true, true>(a, grid, stream)
                     : launch_i8blk_t<TYPE, 1, 2, true, false>(a, grid, stream);
    return a.cap ? launch_i8blk_t<TYPE, 2, 2, false, true>(a, grid, stream)
                 : launch_i8blk_t<TYPE, 2, 2, false, false>(a, grid, stream);
}

// grid: dense (token tiles of gemm_i8kq_token_tile(false), row tiles of I8_N); MoE (row tiles, tiles)
hipError_t launch_gemm_i8kq(int type, const GemmArgs &a, dim3 grid, hipStream_t stream) {
    switch (type) {
    case TY_Q4_K: return launch_i8kq_type<TY_Q4_K>(a, grid, stream);
    case TY_Q5_K: return launch_i8kq_type<TY_Q5_K>(a, grid, stream);
    case TY_Q6_K: return launch_i8kq_type<TY_Q6_K>(a, grid, stream);
    case TY_IQ4_XS: return launch_i8kq_type<TY_IQ4_XS>(a, grid, stream);
    case TY_Q8_0: return launch_i8blk_type<TY_Q8_0>(a, grid, stream);
    case TY_MXFP4: return launch_i8blk_type<TY_MXFP4>(a, grid, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

}  // namespace pq
