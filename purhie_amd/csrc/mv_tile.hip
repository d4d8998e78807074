// mv_tile.hip -- the decode matvec y = W x_q with one whole quantization unit per lane (gfx950, wave64).
//
// Replaces the reference's matvec_q8_<type> / matvec_q8t_<type> / matvec_q8_id_<type> (src/matvec_q.hip:
// 1403-1965) for the shapes it covers (K a whole number of units, at most 256 units a row); the per-wave
// kernels of matvec.hip take the rest. The unit a lane owns (values of one row):
//   Q4_K / Q5_K: one 144 / 176-byte super-block (256)    Q6_K: one 210-byte super-block (256)
//   IQ4_XS: one 136-byte super-block (256)
//   ROCmFP4: eight 18-byte blocks (256)     ROCmFP4_FAST: eight 17-byte blocks (256)
//   Q8_0: four 34-byte blocks (128)
// so a scale decode serves a whole block and the integer work per byte is small.
//
// A workgroup (4 waves) owns a tile of whole rows of one matrix: its units, row-major, are one contiguous
// byte range, and wave w owns units 64 w .. 64 w + 63 -- again contiguous. Per workgroup:
//   1. the activation of the NT tokens (Q8_0 or Q8_K values, scales, group sums) is loaded first: the
//      vector-memory counter retires in issue order, so waiting for it does not wait for the weights;
//   2. each wave loads its byte range with consecutive lanes on consecutive 16-byte chunks (non-temporal;
//      a wave instruction covers 1 KiB of 8 cache lines, where one unit per lane would touch 64);
//   3. the activation goes to LDS (values padded by 16 bytes per 256, so that the unit columns sit in
//      different banks); barrier; each wave writes its chunks to its own LDS region and every lane reads
//      its unit back (LDS is in order within a wave: no barrier);
//   4. each lane forms its unit's exact per-block integer dots (v_dot4_i32_i8 on codes decoded by masks or
//      v_perm_b32 tables) and one float partial per token in the reference's per-block form;
//   5. partials go to LDS (the wave's region); barrier; a few threads per row add its partials in a fixed
//      order set by K.
// The grid holds every tile of the launch (no persistent loop): all weight loads of a launch are in flight
// from the start and each wave computes as its data arrives. A row's result is a sum of per-unit partials
// in an order set by K alone: it does not depend on the other matrices of the launch or on how many
// tokens share it.
#include <algorithm>

#include "device.h"
#include "kernels.h"
#include "moe_dev.h"

namespace pq {

constexpr int TL_THREADS = 256;  // the largest workgroup (64 and 128 threads: smaller tiles, more of them)
constexpr int TL_PAD = 272;      // LDS bytes per 256 activation values

// the dword at byte offset off (compile-time after unrolling) of the unit's dwords
template <int N>
__device__ __forceinline__ uint32_t dwb(const uint32_t (&w)[N], int off) {
    const int i = off >> 2, s = off & 3;
    if (s == 0) return w[i];
    return align_bytes(i + 1 < N ? w[i + 1] : 0u, w[i], (uint32_t)s);
}

// byte at offset off of the unit
template <int N>
__device__ __forceinline__ uint32_t byteb(const uint32_t (&w)[N], int off) {
    return (w[off >> 2] >> (8 * (off & 3))) & 0xffu;
}

// the activation as staged in LDS, at the lane's unit (token t: values x + t * xt, scales d + t * nd,
// group sums s + t * ns)
struct Lx {
    const int8_t *x;
    const float *d;
    const int32_t *s;
    const float *lut;  // scale byte -> its value (Tu<TYPE>::scale)
    int xt, nd, ns;
};

__device__ __forceinline__ int dot8(const int *v, const int4 a, const int4 b) {
    int s = dot4(v[0], a.x, 0);
    s = dot4(v[1], a.y, s);
    s = dot4(v[2], a.z, s);
    s = dot4(v[3], a.w, s);
    s = dot4(v[4], b.x, s);
    s = dot4(v[5], b.y, s);
    s = dot4(v[6], b.z, s);
    return dot4(v[7], b.w, s);
}

__device__ __forceinline__ int dot4x(const int *v, const int4 a) {
    int s = dot4(v[0], a.x, 0);
    s = dot4(v[1], a.y, s);
    s = dot4(v[2], a.z, s);
    return dot4(v[3], a.w, s);
}

// a unit's dwords from LDS: 16-byte aligned (b128 reads) or 8-byte aligned (b64 reads)
template <int N>
__device__ __forceinline__ void read16(const uint8_t *p, uint32_t (&w)[N], uint32_t &aux) {
    static_assert(N % 4 == 0, "whole 16-byte reads");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
        const uint4 v = ((const uint4 *)p)[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
    aux = 0;
}
template <int N>
__device__ __forceinline__ void read8(const uint8_t *p, uint32_t (&w)[N], uint32_t &aux) {
    static_assert(N % 2 == 0, "whole 8-byte reads");
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const uint2 v = ((const uint2 *)p)[i];
        w[2 * i] = v.x;
        w[2 * i + 1] = v.y;
    }
    aux = 0;
}

template <int TYPE>
struct Tu;

// Q4_K super-block: d, dmin (dword 0), 12 scale bytes (dwords 1..3), qs (dwords 4..35). Chunk c of qs
// (32 bytes) holds values 64 c + 0..31 in its low nibbles (sub-block 2 c) and 64 c + 32..63 in its high
// nibbles (sub-block 2 c + 1). The 6-bit scales and mins of the 8 sub-blocks are unpacked four at a time
// (reference src/quant_types.cpp:193-201): scale j < 4 = y byte j & 63, j >= 4 = (w byte & 15) | (y byte
// >> 6) << 4; min j < 4 = z byte j & 63, j >= 4 = (w byte >> 4) | (z byte >> 6) << 4 (y, z, w = dwords
// 1..3). Per super-block: d dx isum - dmin dx msum, isum = sum_j sc_j dot_j, msum = sum_j m_j sum32_j
// (reference src/matvec_q.hip:1752-1789). Q5_K (176 bytes) puts qh (32 bytes) between the scales and qs: the
// level's bit 4 is bit 2 c (low nibble) or 2 c + 1 (high nibble) of qh byte l (reference src/matvec_q.hip:
// 1752-1789 with Q5, 1928-1930).
template <bool Q5>
struct TuKq {
    static constexpr int VALS = 256, BYTES = Q5 ? 176 : 144, NDW = BYTES / 4, ACT = 256, SUMS = 32, LEAD = 0;
    static constexpr int QS = Q5 ? 12 : 4;  // first dword of qs
    static constexpr bool LUT = false;
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read16(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
        const uint32_t y = w[1], z = w[2], v = w[3];
        const uint32_t sc[2] = {y & 0x3f3f3f3fu, (v & 0x0f0f0f0fu) | ((y >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {z & 0x3f3f3f3fu, ((v >> 4) & 0x0f0f0f0fu) | ((z >> 2) & 0x30303030u)};
        int isum[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) isum[t] = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            int lo[8], hi[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t q = w[QS + 8 * c + k];
                uint32_t l4 = q & 0x0f0f0f0fu, h4 = (q >> 4) & 0x0f0f0f0fu;
                if (Q5) {
                    const uint32_t qh = w[4 + k];
                    l4 |= ((qh >> (2 * c)) & 0x01010101u) << 4;
                    h4 |= ((qh >> (2 * c + 1)) & 0x01010101u) << 4;
                }
                lo[k] = (int)l4;
                hi[k] = (int)h4;
            }
            const int sa = (int)((sc[c >> 1] >> (16 * (c & 1))) & 0xffu);
            const int sb = (int)((sc[c >> 1] >> (16 * (c & 1) + 8)) & 0xffu);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.x + t * x.xt + 64 * c);
                const int slo = dot8(lo, xv[0], xv[1]);
                const int shi = dot8(hi, xv[2], xv[3]);
                cap.put(t, 2 * c, slo);
                cap.put(t, 2 * c + 1, shi);
                isum[t] += __mul24(sa, slo) + __mul24(sb, shi);
            }
        }
        const float dw = h2f(w[0] & 0xffffu), dm = h2f(w[0] >> 16);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 s0 = *(const int4 *)(x.s + t * x.ns), s1 = *(const int4 *)(x.s + t * x.ns + 4);
            int msum = __mul24((int)(mn[0] & 0xffu), s0.x);
            msum += __mul24((int)((mn[0] >> 8) & 0xffu), s0.y);
            msum += __mul24((int)((mn[0] >> 16) & 0xffu), s0.z);
            msum += __mul24((int)(mn[0] >> 24), s0.w);
            msum += __mul24((int)(mn[1] & 0xffu), s1.x);
            msum += __mul24((int)((mn[1] >> 8) & 0xffu), s1.y);
            msum += __mul24((int)((mn[1] >> 16) & 0xffu), s1.z);
            msum += __mul24((int)(mn[1] >> 24), s1.w);
            const float dx = x.d[t * x.nd];
            acc[t] = __builtin_fmaf(dw * dx, (float)isum[t], -(dm * dx) * (float)msum);
        }
    }
};
template <>
struct Tu<TY_Q4_K> : TuKq<false> {};
template <>
struct Tu<TY_Q5_K> : TuKq<true> {};

// Q6_K super-block (210 bytes, 2-aligned): ql (bytes 0..127), qh (128..191), 16 int8 scales (192..207),
// d (208..209). Read as 53 dwords from the 4-aligned address at or below it and realigned. For half h,
// l in 0..31: values 128 h + l + {0, 32, 64, 96} are ql[64 h + l] & 15, ql[64 h + 32 + l] & 15,
// ql[64 h + l] >> 4, ql[64 h + 32 + l] >> 4, each with 2 bits of qh[32 h + l] (bits 0-1, 2-3, 4-5, 6-7) as
// bits 4-5; the 16-value group g has scale sc[g]. The -32 offset goes through the Q8_K 16-value sums:
// isum = sum_g sc_g (dot_g - 32 sum16_g) (reference src/matvec_q.hip:1716-1750).
template <>
struct Tu<TY_Q6_K> {
    static constexpr int VALS = 256, BYTES = 210, NDW = 53, ACT = 256, SUMS = 16, LEAD = 15;
    static constexpr bool LUT = false;
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) {
        const uint32_t *a = (const uint32_t *)((uintptr_t)p & ~(uintptr_t)3);
#pragma unroll
        for (int i = 0; i < NDW; ++i) w[i] = a[i];
        aux = (uint32_t)((uintptr_t)p & 3u);
    }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t off, const Lx &x, float (&acc)[NT],
                                   const Cap &cap) {
        uint32_t v[NDW];
#pragma unroll
        for (int i = 0; i < NDW; ++i) v[i] = align_bytes(i + 1 < NDW ? w[i + 1] : 0u, w[i], off);
        int isum[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) isum[t] = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int lc = 0; lc < 2; ++lc) {
                int q[4][4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t A = v[16 * h + 4 * lc + i], B = v[16 * h + 8 + 4 * lc + i];
                    const uint32_t H = v[32 + 8 * h + 4 * lc + i];
                    q[0][i] = (int)((A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u));
                    q[1][i] = (int)((B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u));
                    q[2][i] = (int)(((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u));
                    q[3][i] = (int)(((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u));
                }
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int g = 8 * h + 2 * m + lc;
                    const int sc = (int)(int8_t)((v[48 + (g >> 2)] >> (8 * (g & 3))) & 0xffu);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const int4 xa = *(const int4 *)(x.x + t * x.xt + 128 * h + 32 * m + 16 * lc);
                        const int dg = dot4x(q[m], xa);
                        cap.put(t, g, dg);
                        isum[t] += __mul24(sc, dg - 32 * x.s[t * x.ns + g]);
                    }
                }
            }
        }
        const float dw = h2f(v[52] & 0xffffu);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = (dw * x.d[t * x.nd]) * (float)isum[t];
    }
};

// Q8_0: four 34-byte blocks (fp16 scale, 32 int8 values); per block (e dx) sum
// (reference src/matvec_q.hip:1566-1573 q8_0_q8_block, 1576 mv_q8_0).
template <>
struct Tu<TY_Q8_0> {
    static constexpr int VALS = 128, BYTES = 136, NDW = 34, ACT = 32, SUMS = 0, LEAD = 8;
    static constexpr bool LUT = false;
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read8(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int off = 34 * b;
            int qs[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) qs[k] = (int)dwb(w, off + 2 + 4 * k);
            const float e = h2f((off & 3) ? (w[off >> 2] >> 16) : (w[off >> 2] & 0xffffu));
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.x + t * x.xt + 32 * b);
                const int s = dot8(qs, xv[0], xv[1]);
                cap.put(t, b, s);
                acc[t] = __builtin_fmaf(e * x.d[t * x.nd + b], (float)s, acc[t]);
            }
        }
    }
};

// ROCmFP4 (type 100): eight 18-byte blocks (16 value bytes: value j in the low nibble of byte j, j + 16 in
// the high nibble; UE4M3 half-block scales at bytes 16, 17). Per block (e0 dx) s0 + (e1 dx) s1
// (reference src/matvec_q.hip:1310-1327 P4ROCmFP4::block, 1428 mv_p4).
template <>
struct Tu<TY_FP4> {
    static constexpr int VALS = 256, BYTES = 144, NDW = 36, ACT = 32, SUMS = 0, LEAD = 0;
    static constexpr bool LUT = true;
    __device__ static float scale(uint32_t e) { return ue4m3_half(e); }
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read16(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const int off = 18 * b;
            int lo[4], hi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = dwb(w, off + 4 * k);
                lo[k] = fp4x4_lo(q);
                hi[k] = fp4x4_hi(q);
            }
            const float e0 = x.lut[byteb(w, off + 16)], e1 = x.lut[byteb(w, off + 17)];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.x + t * x.xt + 32 * b);
                const int s0 = dot4x(lo, xv[0]), s1 = dot4x(hi, xv[1]);
                cap.put(t, 2 * b, s0);
                cap.put(t, 2 * b + 1, s1);
                const float dx = x.d[t * x.nd + b];
                acc[t] += __builtin_fmaf(e1 * dx, (float)s1, e0 * dx * (float)s0);
            }
        }
    }
};

// IQ4_XS (type 23): one 136-byte super-block (8-aligned): d (fp16) and scales_h (dword 0), scales_l (dword 1),
// qs (dwords 2..33; sub-block j's 16 bytes hold values 32 j + i in the low nibbles, 32 j + 16 + i in the high),
// a nibble indexing kvalues_iq4nl. Per super-block (d dx) * isum, isum = sum_j (ls_j - 32) dot_j (reference
// src/matvec_q.hip:1788-1810 forms one float term per sub-block).
template <>
struct Tu<TY_IQ4_XS> {
    static constexpr int VALS = 256, BYTES = 136, NDW = 34, ACT = 256, SUMS = 0, LEAD = 8;
    static constexpr bool LUT = false;
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read8(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
        const uint32_t sh = w[0] >> 16, sl = w[1];
        int isum[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) isum[t] = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int lo[4], hi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = w[2 + 4 * j + k];
                lo[k] = iq4nl4_lo(q);
                hi[k] = iq4nl4_hi(q);
            }
            const int ls = iq4xs_scale(sh, sl, j);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.x + t * x.xt + 32 * j);
                const int dj = dot4x(lo, xv[0]) + dot4x(hi, xv[1]);
                cap.put(t, j, dj);
                isum[t] += ls * dj;
            }
        }
        const float dw = h2f(w[0] & 0xffffu);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = (dw * x.d[t * x.nd]) * (float)isum[t];
    }
};

// ROCmFP4_FAST (type 101): eight 17-byte blocks (16 value bytes, one UE4M3 scale at byte 16); per block
// (e dx) (s0 + s1) (reference src/matvec_q.hip:1492-1502, 1505 mv_fast).
template <>
struct Tu<TY_FAST> {
    static constexpr int VALS = 256, BYTES = 136, NDW = 34, ACT = 32, SUMS = 0, LEAD = 8;
    static constexpr bool LUT = true;
    __device__ static float scale(uint32_t e) { return ue4m3_half(e); }
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read8(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int off = 17 * j;
            int lo[4], hi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = dwb(w, off + 4 * k);
                lo[k] = fp4x4_lo(q);
                hi[k] = fp4x4_hi(q);
            }
            const float e = x.lut[byteb(w, off + 16)];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.x + t * x.xt + 32 * j);
                const int s = dot4x(lo, xv[0]) + dot4x(hi, xv[1]);
                cap.put(t, j, s);
                acc[t] = __builtin_fmaf(e * x.d[t * x.nd + j], (float)s, acc[t]);
            }
        }
    }
};

// MXFP4 (type 39): eight 17-byte blocks (an E8M0 scale byte, then FAST's 16 value bytes), E2M1 levels; per
// block (e dx) (s0 + s1) (reference src/matvec_q.hip:1461-1472 PFMXFP4, 1492-1502).
template <>
struct Tu<TY_MXFP4> {
    static constexpr int VALS = 256, BYTES = 136, NDW = 34, ACT = 32, SUMS = 0, LEAD = 8;
    static constexpr bool LUT = true;
    __device__ static float scale(uint32_t e) { return e8m0_half(e); }
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read8(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int off = 17 * j;
            int lo[4], hi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = dwb(w, off + 1 + 4 * k);
                lo[k] = fp4x4_lo<12>(q);
                hi[k] = fp4x4_hi<12>(q);
            }
            const float e = x.lut[byteb(w, off)];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.x + t * x.xt + 32 * j);
                const int s = dot4x(lo, xv[0]) + dot4x(hi, xv[1]);
                cap.put(t, j, s);
                acc[t] = __builtin_fmaf(e * x.d[t * x.nd + j], (float)s, acc[t]);
            }
        }
    }
};

// NVFP4 (type 40): four 36-byte blocks of 64 values (four scale bytes, then four 8-byte sub-blocks of 16: value
// i in the low nibble of byte i % 8, i >= 8 in the high nibble), E2M1 levels. Activation block 2 m + h takes
// sub-blocks 2 h (values 0..15) and 2 h + 1 (16..31) of block m: (dx e0) s0 + (dx e1) s1 (reference
// src/matvec_q.hip:1357-1372 P4NVFP4::block).
template <>
struct Tu<TY_NVFP4> {
    static constexpr int VALS = 256, BYTES = 144, NDW = 36, ACT = 32, SUMS = 0, LEAD = 0;
    static constexpr bool LUT = true;
    __device__ static float scale(uint32_t e) { return nv_scale(e); }
    __device__ static void read(const uint8_t *p, uint32_t (&w)[NDW], uint32_t &aux) { read16(p, w, aux); }
    template <int NT, class Cap>
    __device__ static void compute(const uint32_t (&w)[NDW], uint32_t, const Lx &x, float (&acc)[NT], const Cap &cap) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t a0 = w[9 * m + 1 + 4 * h], a1 = w[9 * m + 2 + 4 * h];
                const uint32_t b0 = w[9 * m + 3 + 4 * h], b1 = w[9 * m + 4 + 4 * h];
                const int la[4] = {fp4x4_lo<12>(a0), fp4x4_lo<12>(a1), fp4x4_hi<12>(a0), fp4x4_hi<12>(a1)};
                const int lb[4] = {fp4x4_lo<12>(b0), fp4x4_lo<12>(b1), fp4x4_hi<12>(b0), fp4x4_hi<12>(b1)};
                const float e0 = x.lut[byteb(w, 36 * m + 2 * h)], e1 = x.lut[byteb(w, 36 * m + 2 * h + 1)];
                const int b = 2 * m + h;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const int4 *xv = (const int4 *)(x.x + t * x.xt + 32 * b);
                    const int s0 = dot4x(la, xv[0]), s1 = dot4x(lb, xv[1]);
                    cap.put(t, 2 * b, s0);
                    cap.put(t, 2 * b + 1, s1);
                    const float dx = x.d[t * x.nd + b];
                    acc[t] += __builtin_fmaf(e1 * dx, (float)s1, e0 * dx * (float)s0);
                }
            }
        }
    }
};

// ---------------------------------------------------------------- LDS layout of a tile

template <int TYPE>
struct TileLds {
    static constexpr int REGION = (64 * Tu<TYPE>::BYTES + Tu<TYPE>::LEAD + 15) & ~15;  // a wave's weight bytes
    static constexpr int CH = (REGION / 16 + 63) / 64;                                  // its 16-byte chunks a lane
    static_assert(REGION >= 4 * 64 * 4, "a region also holds its wave's partials of up to 4 tokens");
    int xt, nd, ns;                                                                     // per token
    int off_d, off_s, off_lut, off_w, bytes;
    __host__ __device__ TileLds(int K, int NT, int thr) {
        using P = Tu<TYPE>;
        xt = (K + 255) / 256 * TL_PAD;
        nd = K / P::ACT;
        ns = P::SUMS ? K / P::SUMS : 0;
        off_d = NT * xt;
        off_s = off_d + ((NT * nd * 4 + 15) & ~15);
        off_lut = off_s + ((NT * ns * 4 + 15) & ~15);
        off_w = off_lut + (P::LUT ? 1024 : 0);
        bytes = off_w + (thr / 64) * REGION;
    }
};

// ---------------------------------------------------------------- the tile kernel body

constexpr int TL_QN = 4, TL_DN = 2, TL_SN = 4;  // activation loads a thread holds across the weight issue

// Stage the activation of NT tokens (global: values q + t K, scales d + t nd, Q8_K 16-value sums bs + t K / 16)
// into LDS. Each thread's first TL_QN value chunks, TL_DN scales and TL_SN group sums are loaded by issue() (before
// the weights), anything beyond by commit(); nothing in issue() waits for a load. The K-quants' group sums: one
// token (FORM) forms them from the staged values, exact integers equal to the sums in memory, which are then not
// read (half the bytes a tile loads: config 2's step 13.47 -> 13.24 us); several tokens, whose tiles are bound by
// their arithmetic rather than their loads, load them (measured 1.5% faster at T = 4). Q6_K's 16-value group is
// one chunk, Q4_K's 32-value group a chunk and its even / odd neighbour, which thread tid ^ 1 holds; loaded,
// Q4_K's 32-value sums are the two 16-value sums added when written.
template <int TYPE, int NT, int THR, bool SMALL = false>
struct Stager {
    // SMALL (the host's choice when every value chunk and scale has a thread of its own): one load of each a
    // thread, where the general form issues TL_QN and TL_DN clamped loads whatever K needs (config 2's pair launch:
    // 1024 value requests for 160 chunks)
    static constexpr int QN = SMALL ? 1 : TL_QN, DN = SMALL ? 1 : TL_DN;
    static constexpr bool PAIR = Tu<TYPE>::SUMS == 32;
    static constexpr bool FORM = Tu<TYPE>::SUMS != 0 && NT == 1;  // sums formed here (else loaded, if any)
    static constexpr bool LOAD = Tu<TYPE>::SUMS != 0 && !FORM;
    int4 qv[QN];
    float dv[DN];
    int2 sv[TL_SN];
    int nq, ndt, nst;

    __device__ __forceinline__ void issue(const TileLds<TYPE> &L, const int8_t *q, const float *d, const int32_t *bs,
                                          int K) {
        nq = NT * K / 16;
        ndt = NT * L.nd;
        nst = NT * L.ns;
        const int tid = threadIdx.x;
        // (unconditional loads, clamped to the last element: with a load skipped on some path the compiler
        // can no longer count the loads in flight and waits for all of them, the weights included)
#pragma unroll
        for (int i = 0; i < QN; ++i) {
            const int c = tid + i * THR;
            qv[i] = *(const int4 *)(q + 16 * (long long)(c < nq ? c : nq - 1));
        }
#pragma unroll
        for (int i = 0; i < DN; ++i) {
            const int e = tid + i * THR;
            dv[i] = d[e < ndt ? e : ndt - 1];
        }
        if constexpr (LOAD) {
#pragma unroll
            for (int i = 0; i < TL_SN; ++i) {
                const int e = tid + i * THR;
                sv[i] = load_s(bs, e < nst ? e : nst - 1);
            }
        }
    }
    __device__ static __forceinline__ int2 load_s(const int32_t *bs, int e) {
        if (PAIR) return *(const int2 *)(bs + 2 * (long long)e);
        return make_int2(bs[e], 0);
    }
    __device__ static __forceinline__ void put_s(const TileLds<TYPE> &L, uint8_t *smem, int e, int2 v) {
        ((int32_t *)(smem + L.off_s))[e] = PAIR ? v.x + v.y : v.x;
    }
    // chunk c's 16 values into LDS (c < nq: active) and, with FORM, its group sum. With FORM every lane calls it
    // (the pair's shuffle); c and c ^ 1 are both below nq or both not (nq is even)
    __device__ __forceinline__ void put(const TileLds<TYPE> &L, uint8_t *smem, int K, int c, int4 v) const {
        const bool active = c < nq;
        if constexpr (FORM) {
            int s = dot4(v.x, 0x01010101, 0);
            s = dot4(v.y, 0x01010101, s);
            s = dot4(v.z, 0x01010101, s);
            s = dot4(v.w, 0x01010101, s);
            if (PAIR) s += dpp_i<DPP_PAIR>(s);
            if (active && (!PAIR || (c & 1) == 0)) ((int32_t *)(smem + L.off_s))[PAIR ? c >> 1 : c] = s;
        }
        if (active) {
            // chunk c is chunk cc = c - t K / 16 of token t. One token, or K a multiple of 256: the tokens' padded
            // blocks are contiguous (t xt = t (K / 256) TL_PAD), so the place follows from c alone, with no division
            int off;
            if (NT == 1 || K % 256 == 0) {
                off = (c >> 4) * TL_PAD + (c & 15) * 16;
            } else {
                const int per = K / 16, t = c / per, cc = c - t * per;
                off = t * L.xt + (cc >> 4) * TL_PAD + (cc & 15) * 16;
            }
            *(int4 *)(smem + off) = v;
        }
    }
    __device__ __forceinline__ void commit(const TileLds<TYPE> &L, uint8_t *smem, const int8_t *q, const float *d,
                                           const int32_t *bs, int K) {
        const int tid = threadIdx.x;
        float *ld = (float *)(smem + L.off_d);
#pragma unroll
        for (int i = 0; i < QN; ++i)
            if (i * THR < nq) put(L, smem, K, tid + i * THR, qv[i]);  // (uniform)
#pragma unroll
        for (int i = 0; i < DN; ++i) {
            const int e = tid + i * THR;
            if (e < ndt) ld[e] = dv[i];
        }
        if constexpr (LOAD) {
#pragma unroll
            for (int i = 0; i < TL_SN; ++i) {
                const int e = tid + i * THR;
                if (e < nst) put_s(L, smem, e, sv[i]);
            }
        }
        // the rest (a thread and its tid ^ 1 partner leave the first loop together)
        for (int c = tid + QN * THR; c < nq; c += THR) put(L, smem, K, c, *(const int4 *)(q + 16 * (long long)c));
        for (int e = tid + DN * THR; e < ndt; e += THR) ld[e] = d[e];
        if constexpr (LOAD)
            for (int e = tid + TL_SN * THR; e < nst; e += THR) put_s(L, smem, e, load_s(bs, e));
        if constexpr (Tu<TYPE>::LUT)
            for (int e = tid; e < 256; e += THR) ((float *)(smem + L.off_lut))[e] = Tu<TYPE>::scale((uint32_t)e);
    }
};

// The activation of one token as SwiGLU(g, u) = g / (1 + exp(-g)) * u, quantized to Q8_0 straight into the tile's
// LDS (values and block scales where the stager puts them): the arithmetic of gpu_swiglu and of the quantizer's
// Q8_0 step (q8dev.h), so the tile sees the bits the two launches give. Half a wave holds a 32-value block (K % 32
// == 0: a half-wave is all in or all out). issue() loads the first SW_R values of each thread before the weights
// are issued (as the stager's first loads), commit() the rest, then computes and writes.
constexpr int SW_R = 4;
// A null u: the low-rank input instead, g[i] lsc for i < ln and 0 up to K, times u = 1 (SiLU(g lsc)).
template <int TYPE, int THR>
struct SwStager {
    float gv[SW_R], uv[SW_R];
    float lsc = 1.0f;
    int ln = 0;
    __device__ __forceinline__ float lr_a(const float *g, int i) const { return i < ln ? g[i] * lsc : 0.0f; }
    __device__ __forceinline__ void issue(const float *g, const float *u, int K) {
#pragma unroll
        for (int j = 0; j < SW_R; ++j) {
            const int i = j * THR + (int)threadIdx.x, c = i < K ? i : K - 1;  // (clamped, unconditional loads)
            if (u) {
                gv[j] = g[c];
                uv[j] = u[c];
            } else {
                gv[j] = lr_a(g, c);
                uv[j] = 1.0f;
            }
        }
    }
    __device__ __forceinline__ void put(const TileLds<TYPE> &L, uint8_t *smem, int i, bool active, float a,
                                        float b) {
        float v = 0.0f;
        if (active) v = a / (1.0f + expf(-a)) * b;
        const float am = group_max(fabsf(v), 32);
        const float id0 = am != 0.0f ? 127.0f / am : 0.0f;
        if (active) {
            smem[(i >> 8) * TL_PAD + (i & 255)] = (uint8_t)(int8_t)(int)rintf(v * id0);
            if ((threadIdx.x & 31) == 0) ((float *)(smem + L.off_d))[i >> 5] = __half2float(__float2half(am / 127.0f));
        }
    }
    __device__ __forceinline__ void commit(const TileLds<TYPE> &L, uint8_t *smem, const float *g, const float *u,
                                           int K) {
#pragma unroll
        for (int j = 0; j < SW_R; ++j) {
            const int i = j * THR + (int)threadIdx.x;
            if (j * THR < K) put(L, smem, i, i < K, gv[j], uv[j]);  // (uniform)
        }
        for (int base = SW_R * THR; base < K; base += THR) {
            const int i = base + (int)threadIdx.x;
            if (u) put(L, smem, i, i < K, i < K ? g[i] : 0.0f, i < K ? u[i] : 0.0f);
            else put(L, smem, i, i < K, i < K ? lr_a(g, i) : 0.0f, 1.0f);
        }
        if constexpr (Tu<TYPE>::LUT)
            for (int e = threadIdx.x; e < 256; e += THR)
                ((float *)(smem + L.off_lut))[e] = Tu<TYPE>::scale((uint32_t)e);
    }
};

// One tile: rows [row0, row0 + nr) of one matrix (contiguous, nb units each, nr * nb <= THR). SW: the activation
// is SwiGLU(sg, su) quantized here (NT 1, a Q8_0-activation type), else q / d / bs staged as they are. CAP
// (capture mode): every unit's integer group dots are added into cap (row r's groups at cap + r * K / G, token t
// cap_ts further on; r counted as row0 is). NP < NT (tokens whose activation does not fit the tile's LDS at once):
// the activation is staged NP tokens at a time into the same LDS while each lane keeps its unit's weights in
// registers, so the weights are still read once; every token's arithmetic is the single-token one.
// PRE: the caller has issued the stager's loads (*pre) already (the routed expert launch, before routing).
template <int TYPE, int NT, int THR, class Rows, bool SW = false, bool CAP = false, int NP = NT, bool SMALL = false,
          bool PRE = false>
__device__ __forceinline__ void tile_body(uint8_t *smem, const Rows &rows, int row0, int nr, int K, int nb, int lg,
                                          const int8_t *q, const float *d, const int32_t *bs,
                                          const float *sg = nullptr, const float *su = nullptr,
                                          int32_t *cap = nullptr, long long cap_ts = 0,
                                          const Stager<TYPE, NP, THR, SMALL> *pre = nullptr, float lr_scale = 1.0f,
                                          int lr_n = 0) {
    using P = Tu<TYPE>;
    using TL = TileLds<TYPE>;
    static_assert(!SW || (NT == 1 && P::ACT == 32 && P::SUMS == 0), "SwiGLU staging: one token, Q8_0 activation");
    static_assert(NT % NP == 0 && (!SW || NP == NT), "staging passes of NP tokens");
    static_assert(!PRE || !SW, "a pre-issued stager stages q / d / bs");
    const TL L(K, NP, THR);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    Stager<TYPE, NP, THR, SMALL> st;
    SwStager<TYPE, THR> sws;
    sws.lsc = lr_scale;
    sws.ln = lr_n;
    if constexpr (PRE) st = *pre;
    else if constexpr (SW) sws.issue(sg, su, K);
    else st.issue(L, q, d, bs, K);

    // this wave's units [64 wave, 64 wave + wu) of the tile: bytes [g, g + wu BYTES), loaded as the 16-byte
    // chunks from the aligned address a at or below g (each chunk holds at least one byte of the range)
    // (a wave past the tile's units loads the tile's first chunk; loads past a wave's last chunk repeat it)
    const int nu = nr * nb, u0 = 64 * wave;
    const int wu = nu - u0 < 0 ? 0 : nu - u0 > 64 ? 64 : nu - u0;
    const uint8_t *g = rows.w(row0) + (long long)(wu ? u0 : 0) * P::BYTES;
    const int lead = (int)((uintptr_t)g & 15u);
    const uint8_t *ga = g - lead;  // (pointer arithmetic keeps the global address space: no flat loads)
    const int nch = wu ? (lead + wu * P::BYTES + 15) >> 4 : 1;
    u32x4 c[TL::CH];
#pragma unroll
    for (int i = 0; i < TL::CH; ++i) {
        const int ci = lane + 64 * i;
        c[i] = ld128_nt(ga + 16 * (ci < nch ? ci : nch - 1));
    }

    if constexpr (SW) sws.commit(L, smem, sg, su, K);
    else st.commit(L, smem, q, d, bs, K);
    __syncthreads();
    uint8_t *region = smem + L.off_w + wave * TL::REGION;
#pragma unroll
    for (int i = 0; i < TL::CH; ++i) {
        const int ci = lane + 64 * i;
        if (ci < nch) *(u32x4 *)(region + 16 * ci) = c[i];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // this lane's unit (an idle lane reads unit 0 of its wave region and its partial is never used)
    const int u = tid < nu ? tid : u0;
    const int k = u % nb;
    uint32_t w[P::NDW], aux;
    P::read(region + lead + (u - u0) * P::BYTES, w, aux);
    const int v0 = k * P::VALS;
    Lx x;
    x.x = (const int8_t *)smem + (v0 >> 8) * TL_PAD + (v0 & 255);
    x.d = (const float *)(smem + L.off_d) + v0 / P::ACT;
    x.s = (const int32_t *)(smem + L.off_s) + (P::SUMS ? v0 / P::SUMS : 0);
    x.lut = (const float *)(smem + L.off_lut);
    x.xt = L.xt;
    x.nd = L.nd;
    x.ns = L.ns;
    float acc[NT];
#pragma unroll
    for (int pass = 0; pass < NT / NP; ++pass) {
        if (pass > 0) {  // (uniform) the next NP tokens' activation, once every wave has read the previous pass's
            __syncthreads();
            const int8_t *qp = q + (long long)pass * NP * K;
            const float *dp = d + (long long)pass * NP * L.nd;
            const int32_t *bp = bs ? bs + (long long)pass * NP * (K / 16) : nullptr;
            Stager<TYPE, NP, THR> sp;
            sp.issue(L, qp, dp, bp, K);
            sp.commit(L, smem, qp, dp, bp, K);
            __syncthreads();
        }
        float ap[NP];
        if constexpr (CAP) {
            constexpr int G = cap_group(TYPE);
            const DotCap dc{tid < nu ? cap + (long long)(row0 + u / nb) * (K / G) + (long long)k * (P::VALS / G) +
                                           (long long)pass * NP * cap_ts
                                     : nullptr,
                            cap_ts};
            P::template compute<NP>(w, aux, x, ap, dc);
        } else {
            P::template compute<NP>(w, aux, x, ap, NoCap{});
        }
#pragma unroll
        for (int t = 0; t < NP; ++t) acc[pass * NP + t] = ap[t];
    }

    // partials into the wave's own region (its units were read above; LDS is in order within a wave)
    float *part = (float *)region;
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t * 64 + lane] = acc[t];
    __syncthreads();
    // row r's sum: G = 2^lg threads per row each add every G-th partial, then a butterfly over the G
    // (a fixed order, set by K alone)
    // (every token in one pass over the partials, each token's sum in the same order)
    const int G = 1 << lg, r = tid >> lg, i = tid & (G - 1);
    const int rr = r < nr ? r : 0;
    float sum[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) sum[t] = 0.0f;
    for (int kk = i; kk < nb; kk += G) {
        const int uu = rr * nb + kk;
        const float *pp = (const float *)(smem + L.off_w + (uu >> 6) * TL::REGION) + (uu & 63);
#pragma unroll
        for (int t = 0; t < NT; ++t) sum[t] += pp[t * 64];
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) sum[t] = group_sum(sum[t], G);
    if (i == 0 && r < nr) rows.template store_all<NT>(row0 + r, sum);
}

// ---------------------------------------------------------------- kernels

// tiles of R rows, per matrix: matrix m owns tiles [tp[m - 1], tp[m]) of the grid; 2^lg threads add a row
struct TileArgs {
    int R, nb, lg, tp[4];
};

// R = thr / nb rows a tile. The threads per row's sum, 2^lg, depend on nb alone (the count a 256-thread tile
// allows), so a row's sum has the same order whatever the workgroup size: floor(thr / nb) 2^lg <= thr still
// holds for thr = 64 and 128, as floor(256 / nb) >= (256 / thr) floor(thr / nb).
static TileArgs tile_args(int nb, int thr) {
    TileArgs ta = {};
    ta.nb = nb;
    ta.R = thr / nb;
    const int R256 = TL_THREADS / nb;
    ta.lg = 0;
    while (ta.lg < 6 && (R256 << (ta.lg + 1)) <= TL_THREADS) ++ta.lg;
    return ta;
}

template <int TYPE, int NT, int THR, bool CAP = false, int NP = NT, bool SMALL = false, bool LR = false>
__global__ void __launch_bounds__(THR) k_mv_tile(MvArgs a, TileArgs ta) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const DenseRows rows{a};
    const int bx = (int)blockIdx.x;
    const int m = (bx >= ta.tp[0]) + (bx >= ta.tp[1]) + (bx >= ta.tp[2]);
    const int first = DenseRows::pick(m, 0, ta.tp[0], ta.tp[1], ta.tp[2]);
    const int row0 = rows.base(m) + (bx - first) * ta.R;
    const int end = DenseRows::pick(m, a.bound[0], a.bound[1], a.bound[2], a.bound[3]);
    const int nr = end - row0 < ta.R ? end - row0 : ta.R;
    if constexpr (LR)  // (the low-rank input: SiLU(lo scale) quantized in the stager)
        tile_body<TYPE, 1, THR, DenseRows, true, false, 1, false, false>(smem, rows, row0, nr, a.K, ta.nb, ta.lg,
                                                                          nullptr, nullptr, nullptr, a.lr_lo, nullptr,
                                                                          nullptr, 0, nullptr, a.lr_scale, a.lr_n);
    else
        tile_body<TYPE, NT, THR, DenseRows, false, CAP, NP, SMALL>(smem, rows, row0, nr, a.K, ta.nb, ta.lg, a.q, a.d,
                                                            a.bs, nullptr, nullptr, a.cap,
                                                            (long long)a.Nt * (a.K / cap_group(TYPE)));
}

// MoE: grid (tiles, n_used * nmat, T); slot j of token t uses expert ids[t * n_used + j] (-1: Wx). Tiles mode:
// grid (tiles, tile, max_tiles) over moe_group's expert tiles, one entry per block.
// SMALL: the stager's one-load form (a thread for every value chunk and scale). ROUTE: the activation's loads are
// issued before the routing (its rows do not depend on the experts), so their latency runs beside it.
template <int TYPE, int THR, bool SW = false, bool CAP = false, bool ROUTE = false, bool SMALL = false>
__global__ void __launch_bounds__(THR) k_mv_tile_id(MvIdArgs a, TileArgs ta) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    IdEntry en;
    Stager<TYPE, 1, THR, SMALL> pre;
    if constexpr (ROUTE) {  // the token's experts from its logits (every workgroup; the first one stores them)
        static_assert(THR == 256, "the router's reductions take 256 threads");
        static_assert(!SW, "the routed launch is the gate / up pair");
        // the router's LDS is the start of the tile's (activation, then weights), which the tile writes only after
        // the barrier below: no LDS of its own on top of the tile's (config 5's 1024-tile expert pair: 3 tiles a CU
        // with it, all 4 without)
        RouterLds<1> &rs = *reinterpret_cast<RouterLds<1> *>(smem);
        const int t = blockIdx.z, slot = (int)blockIdx.y % a.n_used;
        const bool first = blockIdx.x == 0 && blockIdx.y == 0;
        {
            const long long ir = a.x_per_slot ? (long long)t * a.n_used + slot : t;
            pre.issue(TileLds<TYPE>(a.K, 1, THR), a.q + ir * a.K, a.d + ir * (a.K / Tu<TYPE>::ACT),
                      a.bs ? a.bs + ir * (a.K / 16) : nullptr, a.K);
        }
        route_token(a.route_logits + (long long)t * a.route_ne, nullptr, nullptr,
                    first ? a.route_ids + (long long)t * a.n_used : nullptr,
                    first ? a.route_wts + (long long)t * a.n_used : nullptr, nullptr, a.route_ne, a.n_used, 0, a.n_used,
                    rs);
        en.m = (int)blockIdx.y >= a.n_used ? 1 : 0;
        en.e = rs.selid[slot];
        en.out_row = (long long)t * a.n_used + slot;
        en.in_row = a.x_per_slot ? en.out_row : t;
        __syncthreads();  // (every thread's reads of the router's LDS are done)
    } else if (!id_entry(a, en)) {
        return;  // (uniform: before any barrier)
    }
    const int m = en.m, e = en.e;
    const long long in_row = en.in_row;
    const int K = a.K;
    const IdRows rows{e >= 0 ? a.W[m] + (long long)e * a.N * a.row_bytes : a.Wx[m], a.row_bytes,
                      a.y[m] + en.out_row * a.N, e < 0 ? a.sx[m] : a.es[m] ? a.es[m][e] : a.s[m]};
    const int row0 = (int)blockIdx.x * ta.R;
    const int nr = a.N - row0 < ta.R ? a.N - row0 : ta.R;
    int32_t *cap = nullptr;
    if constexpr (CAP) cap = a.cap + ((long long)m * a.cap_rows + en.out_row) * a.N * (K / cap_group(TYPE));
    if constexpr (SW)
        tile_body<TYPE, 1, THR, IdRows, true, CAP>(smem, rows, row0, nr, K, ta.nb, ta.lg, nullptr, nullptr, nullptr,
                                                   a.sw_g + in_row * K, a.sw_u + in_row * K, cap, 0);
    else
        tile_body<TYPE, 1, THR, IdRows, false, CAP, 1, SMALL, ROUTE>(
            smem, rows, row0, nr, K, ta.nb, ta.lg, a.q + in_row * K, a.d + in_row * (K / Tu<TYPE>::ACT),
            a.bs ? a.bs + in_row * (K / 16) : nullptr, nullptr, nullptr, cap, 0, &pre);
}

// ---------------------------------------------------------------- host side

static bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// The tile kernels take a shape when K is a whole number of units (at most 256 a row), the tile's LDS fits
// in 64 KiB, and the operands are aligned for the wide reads: weight matrices 16 bytes with rows a multiple
// of 16 (Q4_K, ROCmFP4) or 8 (Q8_0, ROCmFP4_FAST) bytes (Q6_K: any even row), activation values 16 bytes,
// scales 4, Q4_K's paired group sums 8.
// Tokens a tile stages at a time: all NT when their activation fits the tile's 64 KiB of LDS, else the largest
// divisor of NT that does (passes over the same weights), 0 when none does
template <int TYPE>
static int tile_pass(int K, int NT) {
    for (int np = NT; np >= 1; --np)
        if (NT % np == 0 && TileLds<TYPE>(K, np, TL_THREADS).bytes <= 65536) return np;
    return 0;
}

template <int TYPE>
static bool tile_takes(int K, int NT, const uint8_t *const *W, int nW, long long row_bytes, const void *q,
                       const void *d, const void *bs) {
    using P = Tu<TYPE>;
    if (K <= 0 || K % P::VALS || K / P::VALS > TL_THREADS) return false;
    if (tile_pass<TYPE>(K, NT) == 0) return false;
    for (int i = 0; i < nW; ++i)
        if (!aligned(W[i], 16)) return false;
    if (row_bytes % (P::LEAD == 0 ? 16 : P::LEAD == 8 ? 8 : 2)) return false;
    if (!aligned(q, 16) || !aligned(d, 4)) return false;
    if (P::SUMS && (!bs || !aligned(bs, P::SUMS == 32 ? 8 : 4))) return false;
    return true;
}

// Workgroup size: 256 threads, halved (down to 64, while a tile still holds a whole row) as long as the launch
// would have fewer workgroups than the chip has CUs: a small matrix then spreads over more CUs in smaller tiles.
// (Measured: config 1's 3072 x 1024 Q8_0 matvec gains 12%; launches of 400+ workgroups lose with smaller tiles.)
// PURHIE_MV_THREADS (read once, mv_tune) fixes it.
constexpr long long TL_MIN_WG = 256;

static int tile_threads(int nb, long long rows) {
    if (const int t = mv_tune().threads; t && nb <= t) return t;
    auto wgs = [&](int t) {
        const long long R = t / nb;
        return (rows + R - 1) / R;
    };
    int thr = TL_THREADS;
    while (thr > 64 && nb <= thr / 2 && wgs(thr) < TL_MIN_WG) thr /= 2;
    return thr;
}

// CUs of the current device (read once per device)
int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = __atomic_load_n(&cus[dev], __ATOMIC_RELAXED);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        __atomic_store_n(&cus[dev], n, __ATOMIC_RELAXED);
    }
    return n;
}

// Rows a tile takes: at most Rmax, and fewer where that lightens the most loaded CU. Every tile of a launch is
// meant to be resident at once, so the launch lasts about as long as the CU with the most tiles; its rows,
// ceil(tiles / CUs) R, are what is minimised, over tile counts that stay resident (LDS: resident tiles a CU <=
// 160 KiB / lds). Config 2's pair launch: 25 rows a tile, 780 tiles, 4 on some CUs = 100 rows; 19 rows, 1024 tiles
// = 76 rows. The matrices have n[0..nm) rows, each launched `copies` times (expert slots, tokens). A row's sum does
// not depend on R. *load: that figure for the rows returned, doubled when its tiles cannot all be resident.
// (Smaller tiles, whose per-workgroup costs weigh more, keep thr / nb: config 1's 64-thread tiles measured slower
// balanced.)
static int tile_rows_balanced(int Rmax, const int *n, int nm, long long copies, int lds, long long *load = nullptr) {
    const int ncu = device_cus(), resident = lds > 0 ? 163840 / lds : 8;
    auto load_of = [&](int R, bool &fits) {
        long long wgs = 0;
        for (int i = 0; i < nm; ++i) wgs += n[i] > 0 ? (n[i] + R - 1) / R : 0;
        wgs *= copies;
        const long long per_cu = (wgs + ncu - 1) / ncu;
        fits = per_cu <= resident;
        return per_cu * R * (fits ? 1 : 2);
    };
    bool fits = true;
    int best = Rmax;
    long long best_load = load_of(Rmax, fits);
    if (mv_tune().balance)
        for (int R = Rmax - 1; R >= 1 && 2 * R >= Rmax; --R) {
            const long long l = load_of(R, fits);
            if (fits && l < best_load) {
                best_load = l;
                best = R;
            }
        }
    if (load) *load = best_load;
    return best;
}

// Three-wave tiles: beside the 256-thread tile, a 192-thread one of at most 192 / nb rows (its own balanced
// count) is considered, and taken when its most loaded CU carries no more rows. A four-wave tile of 190 units
// has a fourth wave that stages, computes on a repeated unit and joins the barriers for nothing, and takes a
// fourth weight region of LDS: config 2's pair launch at 4 tokens (48 KiB tiles, 3 resident a CU) had 780 tiles
// of 25 rows, 1024 tiles of 19 rows at 192 threads (39 KiB, 4 a CU) are all resident at once. Rows and every
// sum are the same (a row's order depends on K alone); PURHIE_MV_TRIM=0 keeps 256.
constexpr int TL_TRIM = 192;
static bool tile_trims(const TileArgs &ta) { return ta.R >= 1 && (ta.R << ta.lg) <= TL_TRIM; }

template <int TYPE, int NT, int THR, int NP>
static hipError_t tile_dense_launch(const MvArgs &a, const TileArgs &ta, int tiles, hipStream_t stream) {
    const size_t lds = (size_t)TileLds<TYPE>(a.K, NP, THR).bytes;
    if constexpr (NT == 1 && TYPE == TY_FAST) {
        if (a.lr_lo) {
            hipLaunchKernelGGL((k_mv_tile<TYPE, 1, THR, false, 1, false, true>), dim3((unsigned)tiles), dim3(THR), lds,
                               stream, a, ta);
            return hipGetLastError();
        }
    }
    if (a.lr_lo) return hipErrorNotSupported;
    if constexpr (NT == 1) {
        if (a.K / 16 <= THR && a.K / Tu<TYPE>::ACT <= THR) {  // a thread for every value chunk and scale
            if (a.cap)
                hipLaunchKernelGGL((k_mv_tile<TYPE, 1, THR, true, 1, true>), dim3((unsigned)tiles), dim3(THR), lds,
                                   stream, a, ta);
            else hipLaunchKernelGGL((k_mv_tile<TYPE, 1, THR, false, 1, true>), dim3((unsigned)tiles), dim3(THR), lds,
                                    stream, a, ta);
            return hipGetLastError();
        }
    }
    if (a.cap)
        hipLaunchKernelGGL((k_mv_tile<TYPE, NT, THR, true, NP>), dim3((unsigned)tiles), dim3(THR), lds, stream, a, ta);
    else hipLaunchKernelGGL((k_mv_tile<TYPE, NT, THR, false, NP>), dim3((unsigned)tiles), dim3(THR), lds, stream, a, ta);
    return hipGetLastError();
}

template <int TYPE, int NT, int THR, int NP = NT>
static hipError_t tile_dense_thr(const MvArgs &a, hipStream_t stream) {
    TileArgs ta = tile_args(a.K / Tu<TYPE>::VALS, THR);
    bool trim = false;
    if constexpr (THR == 256) {
        int n[4];
        for (int i = 0, lo = 0; i < 4; ++i) {
            n[i] = a.bound[i] - lo;
            lo = a.bound[i] > lo ? a.bound[i] : lo;
        }
        long long load = 0;
        ta.R = tile_rows_balanced(ta.R, n, 4, 1, TileLds<TYPE>(a.K, NP, THR).bytes, &load);
        if (NP == NT && mv_tune().trim) {
            TileArgs tb = tile_args(ta.nb, TL_TRIM);
            long long lb = 0;
            if (tb.R >= 1) tb.R = tile_rows_balanced(tb.R, n, 4, 1, TileLds<TYPE>(a.K, NP, TL_TRIM).bytes, &lb);
            if (tile_trims(tb) && lb <= load) {
                ta = tb;
                trim = true;
            }
        }
    }
    int tiles = 0, lo = 0;
    for (int i = 0; i < 4; ++i) {
        const int n = a.bound[i] - lo;
        tiles += n > 0 ? (n + ta.R - 1) / ta.R : 0;
        ta.tp[i] = tiles;
        lo = a.bound[i] > lo ? a.bound[i] : lo;
    }
    if constexpr (THR == 256 && NP == NT)
        if (trim) return tile_dense_launch<TYPE, NT, TL_TRIM, NP>(a, ta, tiles, stream);
    return tile_dense_launch<TYPE, NT, THR, NP>(a, ta, tiles, stream);
}

template <int TYPE, int NT>
static hipError_t tile_dense(const MvArgs &a, hipStream_t stream) {
    int nW = 1;
    while (nW < 4 && a.bound[nW - 1] < a.Nt) ++nW;
    if (!tile_takes<TYPE>(a.K, NT, a.W, nW, a.row_bytes, a.q, a.d, a.bs)) return hipErrorNotSupported;
    // staging passes (a large K at several tokens): whole 256-thread tiles, whose rows are many
    if constexpr (NT > 1) {
        const int np = tile_pass<TYPE>(a.K, NT);
        if (np == 1) return tile_dense_thr<TYPE, NT, 256, 1>(a, stream);
        if constexpr (NT == 4)
            if (np == 2) return tile_dense_thr<TYPE, NT, 256, 2>(a, stream);
    }
    switch (tile_threads(a.K / Tu<TYPE>::VALS, a.Nt)) {
    case 64: return tile_dense_thr<TYPE, NT, 64>(a, stream);
    case 128: return tile_dense_thr<TYPE, NT, 128>(a, stream);
    default: return tile_dense_thr<TYPE, NT, 256>(a, stream);
    }
}

template <int TYPE>
static hipError_t tile_dense_t(const MvArgs &a, hipStream_t stream) {
    switch (a.T) {
    case 1: return tile_dense<TYPE, 1>(a, stream);
    case 2: return tile_dense<TYPE, 2>(a, stream);
    case 3: return tile_dense<TYPE, 3>(a, stream);
    case 4: return tile_dense<TYPE, 4>(a, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_tile_lr(int type, const MvArgs &a, hipStream_t stream) {
    if (type != TY_FAST || a.T != 1 || !a.lr_lo) return hipErrorNotSupported;
    return tile_dense<TY_FAST, 1>(a, stream);
}

hipError_t launch_matvec_tile(int type, const MvArgs &a, hipStream_t stream) {
    switch (type) {
    case TY_Q8_0: return tile_dense_t<TY_Q8_0>(a, stream);
    case TY_FP4: return tile_dense_t<TY_FP4>(a, stream);
    case TY_FAST: return tile_dense_t<TY_FAST>(a, stream);
    case TY_MXFP4: return tile_dense_t<TY_MXFP4>(a, stream);
    case TY_NVFP4: return tile_dense_t<TY_NVFP4>(a, stream);
    case TY_Q4_K: return tile_dense_t<TY_Q4_K>(a, stream);
    case TY_Q5_K: return tile_dense_t<TY_Q5_K>(a, stream);
    case TY_IQ4_XS: return tile_dense_t<TY_IQ4_XS>(a, stream);
    case TY_Q6_K: return tile_dense_t<TY_Q6_K>(a, stream);
    }
    return hipErrorNotSupported;
}

// (expert-indexed launches keep four-wave tiles: three-wave ones measured slower there, config 4's decode token
// 23.2 -> 23.7 us)
template <int TYPE, int THR>
static hipError_t tile_id_launch(const MvIdArgs &a, const TileArgs &ta, hipStream_t stream);

template <int TYPE, int THR>
static hipError_t tile_id_thr(const MvIdArgs &a, hipStream_t stream) {
    TileArgs ta = tile_args(a.K / Tu<TYPE>::VALS, THR);
    if (THR == 256 && !a.n_tiles) ta.R = tile_rows_balanced(ta.R, &a.N, 1, (long long)a.n_used * a.nmat * a.T,
                                                             TileLds<TYPE>(a.K, 1, THR).bytes);
    return tile_id_launch<TYPE, THR>(a, ta, stream);
}

template <int TYPE, int THR>
static hipError_t tile_id_launch(const MvIdArgs &a, const TileArgs &ta, hipStream_t stream) {
    const unsigned gx = (unsigned)((a.N + ta.R - 1) / ta.R);
    const dim3 grid = a.n_tiles ? dim3(gx, (unsigned)a.tile, (unsigned)a.max_tiles)
                                : dim3(gx, (unsigned)(a.n_used * a.nmat), (unsigned)a.T);
    const size_t lds = (size_t)TileLds<TYPE>(a.K, 1, THR).bytes;
    if constexpr (Tu<TYPE>::ACT == 32 && Tu<TYPE>::SUMS == 0) {
        if (a.sw_g) {
            if (a.cap) hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, true, true>), grid, dim3(THR), lds, stream, a, ta);
            else hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, true>), grid, dim3(THR), lds, stream, a, ta);
            return hipGetLastError();
        }
    } else if (a.sw_g) {
        return hipErrorInvalidDeviceFunction;
    }
    const bool small = a.K / 16 <= THR && a.K / Tu<TYPE>::ACT <= THR;  // a thread for every value chunk and scale
    if (a.route_logits) {
        if constexpr (THR == 256) {
            // (the router's LDS lies within the tile's, which is at least its size; past 64 KiB the caller falls back
            // to the router and the pair as two launches)
            const size_t lr = std::max(lds, sizeof(RouterLds<1>));
            if (a.cap || a.n_tiles || lr > 65536) return hipErrorNotSupported;
            if (small)
                hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, false, false, true, true>), grid, dim3(THR), lr, stream, a,
                                   ta);
            else hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, false, false, true>), grid, dim3(THR), lr, stream, a, ta);
            return hipGetLastError();
        }
        return hipErrorNotSupported;
    }
    if (small) {
        if (a.cap)
            hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, false, true, false, true>), grid, dim3(THR), lds, stream, a, ta);
        else hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, false, false, false, true>), grid, dim3(THR), lds, stream, a,
                                ta);
        return hipGetLastError();
    }
    if (a.cap) hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR, false, true>), grid, dim3(THR), lds, stream, a, ta);
    else hipLaunchKernelGGL((k_mv_tile_id<TYPE, THR>), grid, dim3(THR), lds, stream, a, ta);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t tile_id(const MvIdArgs &a, hipStream_t stream) {
    // (null Wx entries pass the alignment check; a row of activation is K values, K / ACT scales and K / 16
    // sums on from the previous one, which keeps every row as aligned as the first when K % VALS == 0)
    const uint8_t *W[4] = {a.W[0], a.Wx[0], a.nmat > 1 ? a.W[1] : nullptr, a.nmat > 1 ? a.Wx[1] : nullptr};
    // (SwiGLU staging reads its floats one by one: no activation pointer to check, null passes)
    if (!tile_takes<TYPE>(a.K, 1, W, 4, a.row_bytes, a.sw_g ? nullptr : a.q, a.sw_g ? nullptr : a.d, a.bs))
        return hipErrorNotSupported;
    // (expert-indexed launches keep whole 256-thread tiles: every workgroup first reads its entry's expert id and
    // stages its activation, and smaller tiles measured slower, e.g. config 4's expert down matvec 7.5 vs 6.0 us)
    switch (tile_threads(a.K / Tu<TYPE>::VALS, 1ll << 40)) {
    case 64: return tile_id_thr<TYPE, 64>(a, stream);
    case 128: return tile_id_thr<TYPE, 128>(a, stream);
    default: return tile_id_thr<TYPE, 256>(a, stream);
    }
}

hipError_t launch_matvec_id_tile(int type, const MvIdArgs &a, hipStream_t stream) {
    switch (type) {
    case TY_Q8_0: return tile_id<TY_Q8_0>(a, stream);
    case TY_FP4: return tile_id<TY_FP4>(a, stream);
    case TY_FAST: return tile_id<TY_FAST>(a, stream);
    case TY_MXFP4: return tile_id<TY_MXFP4>(a, stream);
    case TY_NVFP4: return tile_id<TY_NVFP4>(a, stream);
    case TY_Q4_K: return tile_id<TY_Q4_K>(a, stream);
    case TY_Q5_K: return tile_id<TY_Q5_K>(a, stream);
    case TY_IQ4_XS: return tile_id<TY_IQ4_XS>(a, stream);
    case TY_Q6_K: return tile_id<TY_Q6_K>(a, stream);
    }
    return hipErrorNotSupported;
}

}  // namespace pq
