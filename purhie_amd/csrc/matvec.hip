// matvec.hip -- the HBM-bound decode matvec y = W x_q for GGUF weight blocks on gfx950 (wave64).
//
// Replaces the reference's matvec_q8_<type> / matvec_q8t_<type> / matvec_q8_id_<type>
// (src/matvec_q.hip:1403-1965). Structure, MI355X-first:
//   * a workgroup of 4 waves; L lanes (8..64, a power of two, a compile-time constant) per row, 64 / L
//     rows per wave; L is picked per shape so that a lane has about 6 "tasks" (a pair of Q8_0 / ROCmFP4
//     blocks, a quad of FAST blocks, or one 16-byte quarter of a K-quant super-block);
//   * every lane issues all its tasks' weight loads (wide, non-temporal: the weights stream past the
//     caches once) before any arithmetic, from one base pointer with compile-time offsets;
//   * the quantized activation (Q8_0 or Q8_K form, up to 4 tokens) is read through the L1 / L2 caches,
//     where it stays for every row of the launch; no barrier, every wave independent;
//   * integer dots with v_dot4_i32_i8 on codes decoded by v_perm_b32 byte tables, 24-bit integer
//     scale products, and per task a float term in the reference's per-block form
//     (scale_w * scale_x) * int_sum, summed per lane in task order, then a butterfly over the row's lanes.
// Per-block integer sums are exact, and the same as the reference's; the float order differs from the
// reference CPU path's sequential sum (checked to 1e-5 of sum |w x| by the parity tests). A token's
// result does not depend on how many tokens share the launch (the same code per token).
#include "device.h"
#include "kernels.h"

namespace pq {

constexpr int MV_THREADS = 256;
constexpr int MV_U = 8;  // tasks a lane keeps in flight

// quantized activation of NT tokens, already offset to the lane's first task
template <int NT>
struct Act {
    const int8_t *q[NT];
    const float *d[NT];
    const int32_t *bs[NT];
};

__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }

// ---------------------------------------------------------------- per-type task policies
// For a lane with index gl among its row's L lanes: wbase / xoff / doff / boff locate its first task in the
// row's weights and in the activation (values, scales, group sums); consecutive tasks of the lane are
// W_STEP / X_STEP / D_STEP / B_STEP further on (compile-time, given L).

template <int TYPE>
struct Mv;

// Q8_0: a task is a pair of 34-byte blocks (68 bytes, 4-aligned: K % 64 == 0). Block 0's fp16 scale is
// the low half of dword 0 and its values bytes 2..33; block 1's scale the high half of dword 8 and its
// values dwords 9..16.
template <>
struct Mv<TY_Q8_0> {
    static constexpr int ACT_BLK = 32;
    static constexpr bool KQ = false;
    __host__ __device__ static int tasks(int K) { return K / 64; }
    static constexpr int LDIV = 1, W_UNIT = 68, X_UNIT = 64, D_UNIT = 2, B_UNIT = 0;
    static constexpr int U = 3;  // tasks in flight per buffer (17 dwords each)
    struct Lane {
        __device__ Lane(int) {}
    };
    __device__ static long long wbase(int gl) { return 68LL * gl; }
    __device__ static int xoff(int gl) { return 64 * gl; }
    __device__ static int doff(int gl) { return 2 * gl; }
    __device__ static int boff(int) { return 0; }
    struct Raw {
        uint32_t w[17];
    };
    __device__ static void load(const uint8_t *p, Raw &r) {
#pragma unroll
        for (int k = 0; k < 17; ++k) r.w[k] = ld32_nt(p + 4 * k);
    }
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &, const Act<NT> &x, int xo, int dof, int, float acc[NT],
                                   bool v, const Cap &cap) {
        uint32_t qa[8], qb[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            qa[k] = align_bytes(r.w[k + 1], r.w[k], 2);
            qb[k] = r.w[9 + k];
        }
        const float e0 = h2f(r.w[0] & 0xffffu), e1 = h2f(r.w[8] >> 16);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 *xv = (const int4 *)(x.q[t] + xo);
            const int4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
            int s0 = dot4((int)qa[0], x0.x, 0);
            s0 = dot4((int)qa[1], x0.y, s0);
            s0 = dot4((int)qa[2], x0.z, s0);
            s0 = dot4((int)qa[3], x0.w, s0);
            s0 = dot4((int)qa[4], x1.x, s0);
            s0 = dot4((int)qa[5], x1.y, s0);
            s0 = dot4((int)qa[6], x1.z, s0);
            s0 = dot4((int)qa[7], x1.w, s0);
            int s1 = dot4((int)qb[0], x2.x, 0);
            s1 = dot4((int)qb[1], x2.y, s1);
            s1 = dot4((int)qb[2], x2.z, s1);
            s1 = dot4((int)qb[3], x2.w, s1);
            s1 = dot4((int)qb[4], x3.x, s1);
            s1 = dot4((int)qb[5], x3.y, s1);
            s1 = dot4((int)qb[6], x3.z, s1);
            s1 = dot4((int)qb[7], x3.w, s1);
            if (v) {
                cap.put(t, xo / 32, s0);
                cap.put(t, xo / 32 + 1, s1);
            }
            const float2 dx = *(const float2 *)(x.d[t] + dof);
            acc[t] = __builtin_fmaf(v ? e0 * dx.x : 0.0f, (float)s0, acc[t]);
            acc[t] = __builtin_fmaf(v ? e1 * dx.y : 0.0f, (float)s1, acc[t]);
        }
    }
};

// one 32-value FP4 block (16 value bytes as 4 dwords: value j in the low nibble of byte j, j + 16 in its
// high nibble) against its Q8_0 activation block: the two half-block integer sums (TOP: the codebook's top)
template <int TOP = 10>
__device__ __forceinline__ void fp4_block_dots(const uint32_t qs[4], const int4 xa, const int4 xb, int &s0, int &s1) {
    s0 = dot4(fp4x4_lo<TOP>(qs[0]), xa.x, 0);
    s0 = dot4(fp4x4_lo<TOP>(qs[1]), xa.y, s0);
    s0 = dot4(fp4x4_lo<TOP>(qs[2]), xa.z, s0);
    s0 = dot4(fp4x4_lo<TOP>(qs[3]), xa.w, s0);
    s1 = dot4(fp4x4_hi<TOP>(qs[0]), xb.x, 0);
    s1 = dot4(fp4x4_hi<TOP>(qs[1]), xb.y, s1);
    s1 = dot4(fp4x4_hi<TOP>(qs[2]), xb.z, s1);
    s1 = dot4(fp4x4_hi<TOP>(qs[3]), xb.w, s1);
}

// one 16-value NVFP4 sub-block (2 dwords: value i in the low nibble of byte i, i + 8 in the high nibble) against
// its 16 activation values
__device__ __forceinline__ int nv_sub_dot(uint32_t a0, uint32_t a1, const int4 x) {
    int s = dot4(fp4x4_lo<12>(a0), x.x, 0);
    s = dot4(fp4x4_lo<12>(a1), x.y, s);
    s = dot4(fp4x4_hi<12>(a0), x.z, s);
    return dot4(fp4x4_hi<12>(a1), x.w, s);
}

// ROCmFP4 (type 100): a task is a pair of 18-byte blocks (36 bytes, 4-aligned: K % 64 == 0): block 0's
// values dwords 0..3 and its two UE4M3 half-block scales bytes 16, 17; block 1's values bytes 18..33 and
// scales bytes 34, 35. Per block the reference's term (e0 dx) s0 + (e1 dx) s1.
template <>
struct Mv<TY_FP4> {
    static constexpr int ACT_BLK = 32;
    static constexpr bool KQ = false;
    __host__ __device__ static int tasks(int K) { return K / 64; }
    static constexpr int LDIV = 1, W_UNIT = 36, X_UNIT = 64, D_UNIT = 2, B_UNIT = 0;
    static constexpr int U = 5;  // 9 dwords each
    struct Lane {
        __device__ Lane(int) {}
    };
    __device__ static long long wbase(int gl) { return 36LL * gl; }
    __device__ static int xoff(int gl) { return 64 * gl; }
    __device__ static int doff(int gl) { return 2 * gl; }
    __device__ static int boff(int) { return 0; }
    struct Raw {
        uint32_t w[9];
    };
    __device__ static void load(const uint8_t *p, Raw &r) {
#pragma unroll
        for (int k = 0; k < 9; ++k) r.w[k] = ld32_nt(p + 4 * k);
    }
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &, const Act<NT> &x, int xo, int dof, int, float acc[NT],
                                   bool v, const Cap &cap) {
        const uint32_t qa[4] = {r.w[0], r.w[1], r.w[2], r.w[3]};
        uint32_t qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qb[k] = align_bytes(r.w[5 + k], r.w[4 + k], 2);
        const float ea0 = ue4m3_half(r.w[4]), ea1 = ue4m3_half(r.w[4] >> 8);
        const float eb0 = ue4m3_half(r.w[8] >> 16), eb1 = ue4m3_half(r.w[8] >> 24);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 *xv = (const int4 *)(x.q[t] + xo);
            int a0, a1, b0, b1;
            fp4_block_dots(qa, xv[0], xv[1], a0, a1);
            fp4_block_dots(qb, xv[2], xv[3], b0, b1);
            if (v) {
                cap.put(t, xo / 16, a0);
                cap.put(t, xo / 16 + 1, a1);
                cap.put(t, xo / 16 + 2, b0);
                cap.put(t, xo / 16 + 3, b1);
            }
            const float2 dl = *(const float2 *)(x.d[t] + dof);
            const float2 dx = v ? dl : make_float2(0.0f, 0.0f);  // (UE4M3 scales are finite: 0 x e = 0)
            const float ta = __builtin_fmaf(ea1 * dx.x, (float)a1, ea0 * dx.x * (float)a0);
            const float tb = __builtin_fmaf(eb1 * dx.y, (float)b1, eb0 * dx.y * (float)b0);
            acc[t] += ta;
            acc[t] += tb;
        }
    }
};

// ROCmFP4_FAST (type 101): a task is a quad of 17-byte blocks (68 bytes, 4-aligned: K % 128 == 0); block
// j's 16 value bytes start at byte 17 j, its UE4M3 scale at 17 j + 16 (extracted with v_alignbyte).
// Per block the reference's term (e dx) (s0 + s1).
template <>
struct Mv<TY_FAST> {
    static constexpr int ACT_BLK = 32;
    static constexpr bool KQ = false;
    __host__ __device__ static int tasks(int K) { return K / 128; }
    static constexpr int LDIV = 1, W_UNIT = 68, X_UNIT = 128, D_UNIT = 4, B_UNIT = 0;
    static constexpr int U = 3;  // 17 dwords each
    struct Lane {
        __device__ Lane(int) {}
    };
    __device__ static long long wbase(int gl) { return 68LL * gl; }
    __device__ static int xoff(int gl) { return 128 * gl; }
    __device__ static int doff(int gl) { return 4 * gl; }
    __device__ static int boff(int) { return 0; }
    struct Raw {
        uint32_t w[17];
    };
    __device__ static void load(const uint8_t *p, Raw &r) {
#pragma unroll
        for (int k = 0; k < 17; ++k) r.w[k] = ld32_nt(p + 4 * k);
    }
    __device__ static __forceinline__ uint32_t dw(const uint32_t *w, int off) {  // off compile-time
        return (off & 3) == 0 ? w[off >> 2] : align_bytes(w[(off >> 2) + 1], w[off >> 2], off & 3);
    }
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &, const Act<NT> &x, int xo, int dof, int, float acc[NT],
                                   bool v, const Cap &cap) {
        uint32_t w[18];
#pragma unroll
        for (int k = 0; k < 17; ++k) w[k] = r.w[k];
        w[17] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t qs[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) qs[k] = dw(w, 17 * j + 4 * k);
            const float e = ue4m3_half(dw(w, 17 * j + 16));
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.q[t] + xo + 32 * j);
                int s0, s1;
                fp4_block_dots(qs, xv[0], xv[1], s0, s1);
                if (v) cap.put(t, xo / 32 + j, s0 + s1);
                acc[t] = __builtin_fmaf(v ? e * x.d[t][dof + j] : 0.0f, (float)(s0 + s1), acc[t]);
            }
        }
    }
};

// MXFP4 (type 39): a task is a quad of 17-byte blocks (68 bytes, 4-aligned: K % 128 == 0); block j's E8M0
// scale at byte 17 j, its 16 value bytes from 17 j + 1. Per block the reference's term (e dx) (s0 + s1).
template <>
struct Mv<TY_MXFP4> : Mv<TY_FAST> {
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &, const Act<NT> &x, int xo, int dof, int, float acc[NT],
                                   bool v, const Cap &cap) {
        uint32_t w[18];
#pragma unroll
        for (int k = 0; k < 17; ++k) w[k] = r.w[k];
        w[17] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t qs[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) qs[k] = dw(w, 17 * j + 1 + 4 * k);
            const float e = e8m0_half(dw(w, 17 * j));
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int4 *xv = (const int4 *)(x.q[t] + xo + 32 * j);
                int s0, s1;
                fp4_block_dots<12>(qs, xv[0], xv[1], s0, s1);
                if (v) cap.put(t, xo / 32 + j, s0 + s1);
                acc[t] = __builtin_fmaf(v ? e * x.d[t][dof + j] : 0.0f, (float)(s0 + s1), acc[t]);
            }
        }
    }
};

// NVFP4 (type 40): a task is one 36-byte block (64 values, 4-aligned): its four scale bytes (dword 0) and four
// 8-byte sub-blocks (dwords 1..8). Activation blocks 2 g and 2 g + 1 take sub-blocks (0, 1) and (2, 3):
// (dx e0) s0 + (dx e1) s1 each.
template <>
struct Mv<TY_NVFP4> : Mv<TY_FP4> {
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &, const Act<NT> &x, int xo, int dof, int, float acc[NT],
                                   bool v, const Cap &cap) {
        float e[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) e[s] = nv_scale(r.w[0] >> (8 * s));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 *xv = (const int4 *)(x.q[t] + xo);
            const float2 dl = *(const float2 *)(x.d[t] + dof);
            const float2 dx = v ? dl : make_float2(0.0f, 0.0f);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int s0 = nv_sub_dot(r.w[1 + 4 * h], r.w[2 + 4 * h], xv[2 * h]);
                const int s1 = nv_sub_dot(r.w[3 + 4 * h], r.w[4 + 4 * h], xv[2 * h + 1]);
                if (v) {
                    cap.put(t, xo / 16 + 2 * h, s0);
                    cap.put(t, xo / 16 + 2 * h + 1, s1);
                }
                const float d = h ? dx.y : dx.x;
                acc[t] += __builtin_fmaf(e[2 * h + 1] * d, (float)s1, e[2 * h] * d * (float)s0);
            }
        }
    }
};

// Q4_K: a task is one of the 8 sixteen-byte quarter-chunks s of a 144-byte super-block (16-aligned):
// qs bytes 16 s .. 16 s + 15, i.e. chunk c = s / 2, values 64 c + l + 0..15 (low nibbles, sub-block 2c)
// and 64 c + 32 + l + 0..15 (high nibbles, sub-block 2c + 1), l = 16 (s & 1); plus the block header
// (d, dmin, the 12 scale bytes). The lane with quarter s also applies sub-block s's min through the Q8_K
// group sums 2 s, 2 s + 1 (reference src/matvec_q.hip:1752-1789). A lane's quarter s is fixed (L % 8 == 0).
// Q5_K (176 bytes, 16-aligned) has qh (bytes 16..47) before qs (48..175): the lane also loads qh bytes
// 16 (s & 1) .. + 15, whose bit 2 c (low nibbles) and 2 c + 1 (high nibbles) are the levels' bit 4.
template <bool Q5>
struct MvKq {
    static constexpr int ACT_BLK = 256;
    static constexpr bool KQ = true;
    __host__ __device__ static int tasks(int K) { return K / 256 * 8; }
    static constexpr int LDIV = 8, W_UNIT = Q5 ? 176 : 144, X_UNIT = 256, D_UNIT = 1, B_UNIT = 16;
    static constexpr int U = 6;  // 8 dwords each
    // 6-bit scales of sub-blocks 2c, 2c + 1 and the min of sub-block s from the scale dwords y, z, w
    // (bytes 4..15 of the block), gathered with v_perm_b32 using the lane's selectors:
    //   scales: (perm(w, y, p) & pmask) | ((perm(w, y, q) >> 6) & 0x0303) << 4
    //   min:    ((perm(w, z, m) >> msh) & mmask) | ((perm(w, z, n) >> 6) & 3) << 4
    struct Lane {
        uint32_t p, pmask, q, m, msh, mmask, n, hsh;
        __device__ Lane(int gl) {
            const int s = gl & 7, c = s >> 1;
            hsh = (uint32_t)(2 * c);
            if (c < 2) {  // sub-blocks 2c, 2c + 1 < 4: scale = byte j & 63 (y)
                p = (uint32_t)(2 * c) | (uint32_t)(2 * c + 1) << 8 | 0x0c0c0000u;
                pmask = 0x3f3fu;
                q = 0x0c0c0c0cu;
            } else {  // j = 4 + i: scale = (w byte i & 15) | (y byte i >> 6) << 4
                const int i = 2 * c - 4;
                p = (uint32_t)(4 + i) | (uint32_t)(5 + i) << 8 | 0x0c0c0000u;
                pmask = 0x0f0fu;
                q = (uint32_t)i | (uint32_t)(i + 1) << 8 | 0x0c0c0000u;
            }
            if (s < 4) {  // min = z byte s & 63
                m = (uint32_t)s | 0x0c0c0c00u;
                msh = 0;
                mmask = 63;
                n = 0x0c0c0c0cu;
            } else {  // min = (w byte i >> 4) | (z byte i >> 6) << 4
                const int i = s - 4;
                m = (uint32_t)(4 + i) | 0x0c0c0c00u;
                msh = 4;
                mmask = 15;
                n = (uint32_t)i | 0x0c0c0c00u;
            }
        }
    };
    __device__ static long long wbase(int gl) { return (long long)W_UNIT * (gl >> 3); }
    __device__ static int xoff(int gl) {
        const int s = gl & 7;
        return 256 * (gl >> 3) + 64 * (s >> 1) + 16 * (s & 1);
    }
    __device__ static int doff(int gl) { return gl >> 3; }
    __device__ static int boff(int gl) { return 16 * (gl >> 3) + 2 * (gl & 7); }
    struct Raw {
        u32x4 h, qs, qh;
    };
    // the task's block header and its quarter s of qs (and of qh); p = the block header of the lane's current task
    __device__ static void load(const uint8_t *p, Raw &r, int s) {
        r.h = ld128_nt(p);
        r.qs = ld128_nt(p + (Q5 ? 48 : 16) + 16 * s);
        if (Q5) r.qh = ld128_nt(p + 16 + 16 * (s & 1));
    }
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &o, const Act<NT> &x, int xo, int dof, int bo,
                                   float acc[NT], bool v, const Cap &cap) {
        const uint32_t sc2 = (__builtin_amdgcn_perm(r.h.w, r.h.y, o.p) & o.pmask) |
                             (((__builtin_amdgcn_perm(r.h.w, r.h.y, o.q) >> 6) & 0x0303u) << 4);
        const int sc_lo = (int)(sc2 & 0xffu), sc_hi = (int)(sc2 >> 8);
        const int mn = (int)(((__builtin_amdgcn_perm(r.h.w, r.h.z, o.m) >> o.msh) & o.mmask) |
                             (((__builtin_amdgcn_perm(r.h.w, r.h.z, o.n) >> 6) & 3u) << 4));
        const float dw = h2f(r.h.x & 0xffffu), dm = h2f(r.h.x >> 16);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        int lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t l4 = q[k] & 0x0f0f0f0fu, h4 = (q[k] >> 4) & 0x0f0f0f0fu;
            if (Q5) {
                const uint32_t qh = k == 0 ? r.qh.x : k == 1 ? r.qh.y : k == 2 ? r.qh.z : r.qh.w;
                l4 |= ((qh >> o.hsh) & 0x01010101u) << 4;
                h4 |= ((qh >> (o.hsh + 1)) & 0x01010101u) << 4;
            }
            lo[k] = (int)l4;
            hi[k] = (int)h4;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int8_t *xb = x.q[t] + xo;
            const int4 xl = *(const int4 *)xb, xh = *(const int4 *)(xb + 32);
            int slo = dot4(lo[0], xl.x, 0);
            slo = dot4(lo[1], xl.y, slo);
            slo = dot4(lo[2], xl.z, slo);
            slo = dot4(lo[3], xl.w, slo);
            int shi = dot4(hi[0], xh.x, 0);
            shi = dot4(hi[1], xh.y, shi);
            shi = dot4(hi[2], xh.z, shi);
            shi = dot4(hi[3], xh.w, shi);
            if (v) {  // (16 values of sub-block 2c and of 2c + 1: the other lane of the chunk adds the rest)
                cap.put(t, xo / 32, slo);
                cap.put(t, xo / 32 + 1, shi);
            }
            const int2 b2 = *(const int2 *)(x.bs[t] + bo);
            const int isum = mul24(sc_lo, slo) + mul24(sc_hi, shi);
            const int msum = mul24(mn, b2.x + b2.y);
            const float dx = x.d[t][dof];
            acc[t] = __builtin_fmaf(v ? dw * dx : 0.0f, (float)isum, acc[t]);
            acc[t] = __builtin_fmaf(v ? -(dm * dx) : 0.0f, (float)msum, acc[t]);
        }
    }
};
template <>
struct Mv<TY_Q4_K> : MvKq<false> {};

// IQ4_XS: a task is one of the 8 sub-blocks s of a 136-byte super-block (8-aligned): its 16 qs bytes (8 + 16 s,
// low nibbles values 32 s + 0..15, high 32 s + 16..31, levels kvalues_iq4nl) and the header (d, scales_h,
// scales_l); per task d dx ((ls_s - 32) dot) (reference src/matvec_q.hip:1788-1810).
template <>
struct Mv<TY_IQ4_XS> {
    static constexpr int ACT_BLK = 256;
    static constexpr bool KQ = true;
    __host__ __device__ static int tasks(int K) { return K / 256 * 8; }
    static constexpr int LDIV = 8, W_UNIT = 136, X_UNIT = 256, D_UNIT = 1, B_UNIT = 0;
    static constexpr int U = 6;  // 6 dwords each
    struct Lane {
        int s;
        __device__ Lane(int gl) : s(gl & 7) {}
    };
    __device__ static long long wbase(int gl) { return 136LL * (gl >> 3); }
    __device__ static int xoff(int gl) { return 256 * (gl >> 3) + 32 * (gl & 7); }
    __device__ static int doff(int gl) { return gl >> 3; }
    __device__ static int boff(int) { return 0; }
    struct Raw {
        uint32_t h0, h1, q[4];
    };
    __device__ static void load(const uint8_t *p, Raw &r, int s) {
        r.h0 = ld32_nt(p);
        r.h1 = ld32_nt(p + 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) r.q[k] = ld32_nt(p + 8 + 16 * s + 4 * k);
    }
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &o, const Act<NT> &x, int xo, int dof, int, float acc[NT],
                                   bool v, const Cap &cap) {
        int lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            lo[k] = iq4nl4_lo(r.q[k]);
            hi[k] = iq4nl4_hi(r.q[k]);
        }
        const int ls = iq4xs_scale(r.h0 >> 16, r.h1, o.s);
        const float dw = h2f(r.h0 & 0xffffu);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int8_t *xb = x.q[t] + xo;
            const int4 xl = *(const int4 *)xb, xh = *(const int4 *)(xb + 16);
            int s = dot4(lo[0], xl.x, 0);
            s = dot4(lo[1], xl.y, s);
            s = dot4(lo[2], xl.z, s);
            s = dot4(lo[3], xl.w, s);
            s = dot4(hi[0], xh.x, s);
            s = dot4(hi[1], xh.y, s);
            s = dot4(hi[2], xh.z, s);
            s = dot4(hi[3], xh.w, s);
            if (v) cap.put(t, xo / 32, s);
            acc[t] = __builtin_fmaf(v ? dw * x.d[t][dof] : 0.0f, (float)(ls * s), acc[t]);
        }
    }
};
template <>
struct Mv<TY_Q5_K> : MvKq<true> {};

// Q6_K: a task is one of the 8 quarters s of a 210-byte super-block (2-aligned): half h = s / 4, ql bytes
// 64 h + r .. + 15 (r = 16 (s & 3)) and qh bytes 128 + 32 h + (r & 31) .. + 15, loaded as realigned
// dwords; the low nibbles (with 2 bits of qh) are values v_lo = 128 h + 32 [r >= 32] + (r & 31) + 0..15,
// the high nibbles v_lo + 64 + 0..15. The -32 offset of every level goes through the Q8_K group sums
// (groups 2 s, 2 s + 1 on lane s), as the reference's src/matvec_q.hip:1716-1750.
template <>
struct Mv<TY_Q6_K> {
    static constexpr int ACT_BLK = 256;
    static constexpr bool KQ = true;
    __host__ __device__ static int tasks(int K) { return K / 256 * 8; }
    static constexpr int LDIV = 8, W_UNIT = 210, X_UNIT = 256, D_UNIT = 1, B_UNIT = 16;
    static constexpr int U = 4;  // 14 dwords each
    struct Lane {
        int s, qlo, qho, sh, g_lo;
        __device__ Lane(int gl) {
            s = gl & 7;
            const int h = s >> 2, rr = (s & 3) * 16, l = rr & 31, second = rr >= 32;
            qlo = 64 * h + rr;
            qho = 128 + 32 * h + l;
            sh = second ? 2 : 0;
            g_lo = 8 * h + (l >> 4) + (second ? 2 : 0);
        }
    };
    __device__ static long long wbase(int gl) { return 210LL * (gl >> 3); }
    __device__ static int xoff(int gl) {
        const int s = gl & 7, h = s >> 2, rr = (s & 3) * 16;
        return 256 * (gl >> 3) + 128 * h + (rr >= 32 ? 32 : 0) + (rr & 31);
    }
    __device__ static int doff(int gl) { return gl >> 3; }
    __device__ static int boff(int gl) { return 16 * (gl >> 3) + 2 * (gl & 7); }
    struct Raw {
        uint32_t ql[5], qh[5];
        uint32_t off;
        int sc_lo, sc_hi;
        uint32_t scp, d;
    };
    __device__ static void load(const uint8_t *b, Raw &r, const Lane &o) {
        const uint32_t off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *a1 = b + o.qlo - off, *a2 = b + o.qho - off;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            r.ql[k] = ld32_nt(a1 + 4 * k);
            r.qh[k] = ld32_nt(a2 + 4 * k);
        }
        r.off = off;
        r.sc_lo = (int)((const int8_t *)b)[192 + o.g_lo];
        r.sc_hi = (int)((const int8_t *)b)[192 + o.g_lo + 4];
        r.scp = *(const uint16_t *)(b + 192 + 2 * o.s);
        r.d = *(const uint16_t *)(b + 208);
    }
    template <int NT, class Cap>
    __device__ static void compute(const Raw &r, const Lane &o, const Act<NT> &x, int xo, int dof, int bo,
                                   float acc[NT], bool v, const Cap &cap) {
        int vlo[4], vhi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t ql = align_bytes(r.ql[k + 1], r.ql[k], r.off);
            const uint32_t qh = align_bytes(r.qh[k + 1], r.qh[k], r.off);
            vlo[k] = (int)((ql & 0x0f0f0f0fu) | (((qh >> o.sh) & 0x03030303u) << 4));
            vhi[k] = (int)(((ql >> 4) & 0x0f0f0f0fu) | (((qh >> (o.sh + 4)) & 0x03030303u) << 4));
        }
        const int sca = (int)(int8_t)(r.scp & 0xffu), scb = (int)(int8_t)(r.scp >> 8);
        const float dw = h2f(r.d);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int8_t *xb = x.q[t] + xo;
            const int4 xl = *(const int4 *)xb, xh = *(const int4 *)(xb + 64);
            int slo = dot4(vlo[0], xl.x, 0);
            slo = dot4(vlo[1], xl.y, slo);
            slo = dot4(vlo[2], xl.z, slo);
            slo = dot4(vlo[3], xl.w, slo);
            int shi = dot4(vhi[0], xh.x, 0);
            shi = dot4(vhi[1], xh.y, shi);
            shi = dot4(vhi[2], xh.z, shi);
            shi = dot4(vhi[3], xh.w, shi);
            if (v) {
                cap.put(t, xo / 16, slo);
                cap.put(t, xo / 16 + 4, shi);
            }
            const int2 b2 = *(const int2 *)(x.bs[t] + bo);
            int isum = mul24(r.sc_lo, slo) + mul24(r.sc_hi, shi);
            isum -= 32 * (mul24(sca, b2.x) + mul24(scb, b2.y));
            acc[t] = __builtin_fmaf(v ? dw * x.d[t][dof] : 0.0f, (float)isum, acc[t]);
        }
    }
};

// ---------------------------------------------------------------- the lane loop shared by the kernels

template <int TYPE>
__device__ __forceinline__ void load_task(const uint8_t *p, typename Mv<TYPE>::Raw &r, const typename Mv<TYPE>::Lane &o,
                                          int gl) {
    if constexpr (TYPE == TY_Q4_K || TYPE == TY_Q5_K || TYPE == TY_IQ4_XS) Mv<TYPE>::load(p, r, gl & 7);
    else if constexpr (TYPE == TY_Q6_K) Mv<TYPE>::load(p, r, o);
    else Mv<TYPE>::load(p, r);
}

// the row's partial sum of this lane: tasks gl, gl + L, ... of the row at wr, MV_U at a time, every load of
// a batch issued before its arithmetic
template <int TYPE, int NT, int L, class Cap>
__device__ __forceinline__ void row_sum(const uint8_t *wr, int K, int gl, const Act<NT> &x0, float acc[NT],
                                        const Cap &cap) {
    using P = Mv<TYPE>;
    constexpr int SL = L / P::LDIV;  // units of the lane's task stride
    constexpr int WS = P::W_UNIT * SL, XS = P::X_UNIT * SL, DS = P::D_UNIT * SL, BS = P::B_UNIT * SL;
    const int ntask = P::tasks(K);
    const int nu = (ntask - gl + L - 1) / L;  // tasks of this lane
    const typename P::Lane o(gl);
    const uint8_t *wp = wr + P::wbase(gl);
    int xo = P::xoff(gl), dof = P::doff(gl), bo = P::boff(gl);
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    for (int u0 = 0; u0 < nu; u0 += MV_U) {
        typename P::Raw raw[MV_U];
#pragma unroll
        for (int u = 0; u < MV_U; ++u)
            if (u0 + u < nu) load_task<TYPE>(wp + u * WS, raw[u], o, gl);
#pragma unroll
        for (int u = 0; u < MV_U; ++u)
            if (u0 + u < nu)
                P::template compute<NT>(raw[u], o, x0, xo + u * XS, dof + u * DS, bo + u * BS, acc, true, cap);
        wp += MV_U * WS;
        xo += MV_U * XS;
        dof += MV_U * DS;
        bo += MV_U * BS;
    }
}

template <int TYPE>
__host__ __device__ constexpr int act_blk() {
    return Mv<TYPE>::ACT_BLK;
}

template <int TYPE, int NT>
__device__ __forceinline__ void act_view(const int8_t *q, const float *d, const int32_t *bs, int K, Act<NT> &x) {
    const int nblk = K / act_blk<TYPE>();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        x.q[t] = q + t * K;
        x.d[t] = d + t * nblk;
        x.bs[t] = bs + t * (K / 16);
    }
}

// ---------------------------------------------------------------- long rows (more than MV_U tasks a lane)
// one row group per wave, the activation read through the caches

template <int TYPE, int NT, int L, bool CAP = false>
__global__ void __launch_bounds__(MV_THREADS) k_matvec(MvArgs a) {
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int row = (blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    if (row >= a.Nt) return;  // (a whole lane group: rows of 64 / L lanes)
    const int mat = (row >= a.bound[0]) + (row >= a.bound[1]) + (row >= a.bound[2]);
    const int base = mat == 0 ? 0 : a.bound[mat - 1];
    const uint8_t *wr = a.W[mat] + (long long)(row - base) * a.row_bytes;
    Act<NT> x;
    act_view<TYPE, NT>(a.q, a.d, a.bs, a.K, x);
    float acc[NT];
    if constexpr (CAP) {
        const int ng = a.K / cap_group(TYPE);
        row_sum<TYPE, NT, L>(wr, a.K, gl, x, acc, DotCap{a.cap + (long long)row * ng, (long long)a.Nt * ng});
    } else {
        row_sum<TYPE, NT, L>(wr, a.K, gl, x, acc, NoCap{});
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v = group_sum(acc[t], L);
        if (gl == 0) a.y[mat][(long long)t * a.ystride[mat] + (row - base)] = v * a.osc[mat];
    }
}

// The low-rank input (the reference's matvec_q8_lr, src/matvec_q.hip:2107-2135): every workgroup makes the Q8_0
// activation of SiLU(lo[i] scale) (i < n, 0 up to K) in LDS with the tile stager's arithmetic (that of gpu_swiglu
// with u = 1 and of its quantizer), then the rows as k_matvec computes them from it.
template <int TYPE, int L>
__global__ void __launch_bounds__(MV_THREADS) k_matvec_lr(MvArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t xs[LR_MAXK];
    __shared__ float xd[LR_MAXK / 32];
    for (int base = 0; base < a.K; base += MV_THREADS) {  // (a half-wave holds a 32-value block, all in or out)
        const int i = base + (int)threadIdx.x;
        const bool active = i < a.K;
        const float g = active && i < a.lr_n ? a.lr_lo[i] * a.lr_scale : 0.0f, u = 1.0f;
        float v = 0.0f;
        if (active) v = g / (1.0f + expf(-g)) * u;
        const float am = group_max(fabsf(v), 32);
        const float id0 = am != 0.0f ? 127.0f / am : 0.0f;
        if (active) {
            xs[i] = (int8_t)(int)rintf(v * id0);
            if ((threadIdx.x & 31) == 0) xd[i >> 5] = __half2float(__float2half(am / 127.0f));
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int row = (blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    if (row >= a.Nt) return;
    Act<1> x;
    x.q[0] = xs;
    x.d[0] = xd;
    x.bs[0] = nullptr;
    float acc[1];
    row_sum<TYPE, 1, L>(a.W[0] + (long long)row * a.row_bytes, a.K, gl, x, acc, NoCap{});
    const float v = group_sum(acc[0], L);
    if (gl == 0) a.y[0][row] = v * a.osc[0];
}

// ---------------------------------------------------------------- MoE expert-indexed kernel
// grid (row groups, n_used * nmat, T): slot j of token t uses expert ids[t * n_used + j] (-1: Wx)

template <int TYPE, int L, bool CAP = false>
__global__ void __launch_bounds__(MV_THREADS) k_matvec_id(MvIdArgs a) {
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int row = (blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    IdEntry en;
    if (row >= a.N || !id_entry(a, en)) return;
    const int m = en.m, e = en.e;
    const long long in_row = en.in_row;
    const int K = a.K;
    const int kb = K / act_blk<TYPE>();
    const uint8_t *wr = e >= 0 ? a.W[m] + ((long long)e * a.N + row) * a.row_bytes : a.Wx[m] + (long long)row * a.row_bytes;
    Act<1> x;
    act_view<TYPE, 1>(a.q + in_row * K, a.d + in_row * kb, a.bs ? a.bs + in_row * (K / 16) : nullptr, K, x);
    float acc[1];
    if constexpr (CAP) {
        const int ng = K / cap_group(TYPE);
        row_sum<TYPE, 1, L>(wr, K, gl, x, acc,
                            DotCap{a.cap + (((long long)m * a.cap_rows + en.out_row) * a.N + row) * ng, 0});
    } else {
        row_sum<TYPE, 1, L>(wr, K, gl, x, acc, NoCap{});
    }
    const float v = group_sum(acc[0], L);
    const float sc = e < 0 ? a.sx[m] : a.es[m] ? a.es[m][e] : a.s[m];
    if (gl == 0) a.y[m][en.out_row * a.N + row] = v * sc;
}

// ---------------------------------------------------------------- per-group integer dots (test hook)
// One thread per (row, group); the same code decoder (fp4x4) as the kernels above.

__device__ __forceinline__ int cb_value(uint32_t nib) { return (int)(int8_t)(fp4x4(nib) & 0xffu); }

template <int TYPE>
__global__ void k_block_dots(const uint8_t *W, long long rb, const int8_t *q, int32_t *out, int N, int K) {
    constexpr int G = (TYPE == TY_FP4 || TYPE == TY_Q6_K || TYPE == TY_NVFP4) ? 16 : 32;
    const int ng = K / G;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * ng) return;
    const int n = (int)(i / ng), g = (int)(i % ng);
    const uint8_t *row = W + (long long)n * rb;
    const int8_t *xg = q + (long long)g * G;
    int s = 0;
    if (TYPE == TY_Q8_0) {
        const uint8_t *b = row + 34 * g;
        for (int j = 0; j < 32; ++j) s += (int)(int8_t)b[2 + j] * xg[j];
    } else if (TYPE == TY_FP4 || TYPE == TY_FAST) {
        const int bpb = TYPE == TY_FP4 ? 18 : 17;
        const int blk = TYPE == TY_FP4 ? g >> 1 : g;
        const uint8_t *b = row + bpb * blk;
        for (int j = 0; j < G; ++j) {
            const int v = (TYPE == TY_FP4 ? (g & 1) * 16 : 0) + j;  // value index within the block
            const uint32_t nib = v < 16 ? (b[v] & 0xfu) : (b[v - 16] >> 4);
            s += cb_value(nib) * xg[j];
        }
    } else if (TYPE == TY_MXFP4) {
        const uint8_t *b = row + 17 * g + 1;
        for (int j = 0; j < 16; ++j)
            s += fp4_level<12>(b[j] & 0xfu) * xg[j] + fp4_level<12>(b[j] >> 4) * xg[16 + j];
    } else if (TYPE == TY_NVFP4) {
        const uint8_t *b = row + 36 * (g >> 2) + 4 + 8 * (g & 3);
        for (int j = 0; j < 8; ++j) s += fp4_level<12>(b[j] & 0xfu) * xg[j] + fp4_level<12>(b[j] >> 4) * xg[8 + j];
    } else if (TYPE == TY_IQ4_XS) {
        const uint8_t *b = row + 136 * (g >> 3) + 8 + 16 * (g & 7);
        for (int i2 = 0; i2 < 16; ++i2) {
            s += (int)(int8_t)(iq4nl4(b[i2] & 0xfu) & 0xff) * xg[i2];
            s += (int)(int8_t)(iq4nl4(b[i2] >> 4) & 0xff) * xg[16 + i2];
        }
    } else if (TYPE == TY_Q4_K || TYPE == TY_Q5_K) {
        const bool q5 = TYPE == TY_Q5_K;
        const uint8_t *b = row + (q5 ? 176 : 144) * (g >> 3);
        const int j = g & 7;  // sub-block: chunk j / 2, high nibbles for odd j (Q5_K: bit j of qh byte i2 as bit 4)
        for (int i2 = 0; i2 < 32; ++i2) {
            const uint8_t v = b[(q5 ? 48 : 16) + 32 * (j >> 1) + i2];
            const int hb = q5 ? ((b[16 + i2] >> j) & 1) << 4 : 0;
            s += ((int)((j & 1) ? (v >> 4) : (v & 0xf)) | hb) * xg[i2];
        }
    } else {  // Q6_K group of 16
        const uint8_t *b = row + 210 * (g >> 4);
        for (int i2 = 0; i2 < 16; ++i2) {
            const int v = 16 * (g & 15) + i2, h = v >> 7, jj = (v >> 5) & 3, l = v & 31;
            const uint8_t ql = b[64 * h + l + 32 * (jj & 1)], qh = b[128 + 32 * h + l];
            const int lv = ((jj >= 2) ? (ql >> 4) : (ql & 0xf)) | (((qh >> (2 * jj)) & 3) << 4);
            s += lv * xg[i2];
        }
    }
    out[i] = s;
}

// ---------------------------------------------------------------- host launchers

int matvec_lanes(int type, int K, long long rows) {
    int nt = 0, U = 1;
    switch (type) {
    case TY_Q8_0: nt = Mv<TY_Q8_0>::tasks(K); U = Mv<TY_Q8_0>::U; break;
    case TY_FP4: nt = Mv<TY_FP4>::tasks(K); U = Mv<TY_FP4>::U; break;
    case TY_FAST: case TY_MXFP4: nt = Mv<TY_FAST>::tasks(K); U = Mv<TY_FAST>::U; break;
    case TY_NVFP4: nt = Mv<TY_FP4>::tasks(K); U = Mv<TY_FP4>::U; break;
    case TY_Q4_K: nt = Mv<TY_Q4_K>::tasks(K); U = Mv<TY_Q4_K>::U; break;
    case TY_Q5_K: nt = Mv<TY_Q5_K>::tasks(K); U = Mv<TY_Q5_K>::U; break;
    case TY_IQ4_XS: nt = Mv<TY_IQ4_XS>::tasks(K); U = Mv<TY_IQ4_XS>::U; break;
    case TY_Q6_K: nt = Mv<TY_Q6_K>::tasks(K); U = Mv<TY_Q6_K>::U; break;
    default: return 0;
    }
    // the fewest lanes (>= 8: the K-quants' 8 quarters of a super-block) that keep a lane's tasks of a row
    // within the type's U, so the streaming kernels hold a whole row group in registers
    int L = 8;
    while (L < 64 && (nt + L - 1) / L > U) L <<= 1;
    (void)rows;
    if (mv_tune().lanes) L = mv_tune().lanes;
    return L;
}

namespace {
MvTune tune_from_env() {
    MvTune t{1, 0, 0, 1, 1};
    if (const char *e = getenv("PURHIE_MV_TILE")) t.tile = e[0] == '0' ? 0 : 1;
    if (const char *e = getenv("PURHIE_MV_BALANCE")) t.balance = e[0] == '0' ? 0 : 1;
    if (const char *e = getenv("PURHIE_MV_TRIM")) t.trim = e[0] == '0' ? 0 : 1;
    if (const char *e = getenv("PURHIE_MV_THREADS")) {
        const int v = atoi(e);
        t.threads = v == 64 || v == 128 || v == 256 ? v : 0;
    }
    if (const char *e = getenv("PURHIE_MV_LANES")) {
        const int v = atoi(e);
        t.lanes = v >= 8 && v <= 64 && (v & (v - 1)) == 0 ? v : 0;
    }
    return t;
}
MvTune g_tune = tune_from_env();  // (static initialisation: before any launch)
}  // namespace

const MvTune &mv_tune() { return g_tune; }
void mv_tune_set_tile(int on) { __atomic_store_n(&g_tune.tile, on ? 1 : 0, __ATOMIC_RELAXED); }

// the tile kernels where they take the shape, unless PURHIE_MV_TILE=0 or the test hook switched them off
static bool tile_enabled() { return __atomic_load_n(&g_tune.tile, __ATOMIC_RELAXED) != 0; }

bool mv_tile_on() { return tile_enabled(); }

template <int TYPE, int NT, int L>
static hipError_t launch_tl(const MvArgs &a, hipStream_t stream) {
    const int rows_per_wg = (MV_THREADS / 64) * (64 / L);
    const unsigned grid = (unsigned)((a.Nt + rows_per_wg - 1) / rows_per_wg);
    if (a.cap) hipLaunchKernelGGL((k_matvec<TYPE, NT, L, true>), dim3(grid), dim3(MV_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((k_matvec<TYPE, NT, L>), dim3(grid), dim3(MV_THREADS), 0, stream, a);
    return hipGetLastError();
}

template <int TYPE, int NT>
static hipError_t launch_t(const MvArgs &a, hipStream_t stream) {
    switch (a.L) {
    case 8: return launch_tl<TYPE, NT, 8>(a, stream);
    case 16: return launch_tl<TYPE, NT, 16>(a, stream);
    case 32: return launch_tl<TYPE, NT, 32>(a, stream);
    case 64: return launch_tl<TYPE, NT, 64>(a, stream);
    }
    return hipErrorInvalidValue;
}

template <int TYPE>
static hipError_t launch_nt(const MvArgs &a, hipStream_t stream) {
    switch (a.T) {
    case 1: return launch_t<TYPE, 1>(a, stream);
    case 2: return launch_t<TYPE, 2>(a, stream);
    case 3: return launch_t<TYPE, 3>(a, stream);
    case 4: return launch_t<TYPE, 4>(a, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_matvec(int type, const MvArgs &a, hipStream_t stream) {
    if (tile_enabled()) {
        const hipError_t e = launch_matvec_tile(type, a, stream);
        if (e != hipErrorNotSupported) return e;
    }
    switch (type) {
    case TY_Q8_0: return launch_nt<TY_Q8_0>(a, stream);
    case TY_FP4: return launch_nt<TY_FP4>(a, stream);
    case TY_FAST: return launch_nt<TY_FAST>(a, stream);
    case TY_MXFP4: return launch_nt<TY_MXFP4>(a, stream);
    case TY_NVFP4: return launch_nt<TY_NVFP4>(a, stream);
    case TY_Q4_K: return launch_nt<TY_Q4_K>(a, stream);
    case TY_Q5_K: return launch_nt<TY_Q5_K>(a, stream);
    case TY_IQ4_XS: return launch_nt<TY_IQ4_XS>(a, stream);
    case TY_Q6_K: return launch_nt<TY_Q6_K>(a, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

template <int L>
static hipError_t launch_lr_l(const MvArgs &a, hipStream_t stream) {
    const int rows_per_wg = (MV_THREADS / 64) * (64 / L);
    hipLaunchKernelGGL((k_matvec_lr<TY_FAST, L>), dim3((unsigned)((a.Nt + rows_per_wg - 1) / rows_per_wg)),
                       dim3(MV_THREADS), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_matvec_lr(int type, const MvArgs &a, hipStream_t stream) {
    if (type != TY_FAST || a.T != 1 || !a.lr_lo || a.K > LR_MAXK || a.K % 128) return hipErrorInvalidValue;
    if (tile_enabled()) {
        const hipError_t e = launch_matvec_tile_lr(type, a, stream);
        if (e != hipErrorNotSupported) return e;
    }
    switch (a.L) {
    case 8: return launch_lr_l<8>(a, stream);
    case 16: return launch_lr_l<16>(a, stream);
    case 32: return launch_lr_l<32>(a, stream);
    case 64: return launch_lr_l<64>(a, stream);
    }
    return hipErrorInvalidValue;
}

template <int TYPE, int L>
static hipError_t launch_id_tl(const MvIdArgs &a, hipStream_t stream) {
    const int rows_per_wg = (MV_THREADS / 64) * (64 / L);
    const unsigned gx = (unsigned)((a.N + rows_per_wg - 1) / rows_per_wg);
    const dim3 grid = a.n_tiles ? dim3(gx, (unsigned)a.tile, (unsigned)a.max_tiles)
                                : dim3(gx, (unsigned)(a.n_used * a.nmat), (unsigned)a.T);
    if (a.cap) hipLaunchKernelGGL((k_matvec_id<TYPE, L, true>), grid, dim3(MV_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((k_matvec_id<TYPE, L>), grid, dim3(MV_THREADS), 0, stream, a);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_id_t(const MvIdArgs &a, hipStream_t stream) {
    switch (a.L) {
    case 8: return launch_id_tl<TYPE, 8>(a, stream);
    case 16: return launch_id_tl<TYPE, 16>(a, stream);
    case 32: return launch_id_tl<TYPE, 32>(a, stream);
    case 64: return launch_id_tl<TYPE, 64>(a, stream);
    }
    return hipErrorInvalidValue;
}

// the SwiGLU-fused input exists in the tile kernel of the Q8_0-activation types only
bool matvec_id_swiglu_supported(int type, int K) {
    return tile_enabled() && (type == TY_Q8_0 || type == TY_FP4 || type == TY_FAST || type == TY_MXFP4 ||
                              type == TY_NVFP4) && K % 256 == 0 && K <= 16384;
}

hipError_t launch_matvec_id(int type, const MvIdArgs &a, hipStream_t stream) {
    if (a.sw_g) {  // (no per-wave form)
        const hipError_t e = launch_matvec_id_tile(type, a, stream);
        return e == hipErrorNotSupported ? hipErrorInvalidDeviceFunction : e;
    }
    if (tile_enabled()) {
        const hipError_t e = launch_matvec_id_tile(type, a, stream);
        if (e != hipErrorNotSupported) return e;
    }
    switch (type) {
    case TY_Q8_0: return launch_id_t<TY_Q8_0>(a, stream);
    case TY_FP4: return launch_id_t<TY_FP4>(a, stream);
    case TY_FAST: return launch_id_t<TY_FAST>(a, stream);
    case TY_MXFP4: return launch_id_t<TY_MXFP4>(a, stream);
    case TY_NVFP4: return launch_id_t<TY_NVFP4>(a, stream);
    case TY_Q4_K: return launch_id_t<TY_Q4_K>(a, stream);
    case TY_Q5_K: return launch_id_t<TY_Q5_K>(a, stream);
    case TY_IQ4_XS: return launch_id_t<TY_IQ4_XS>(a, stream);
    case TY_Q6_K: return launch_id_t<TY_Q6_K>(a, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

hipError_t launch_block_dots(int type, const uint8_t *W, long long rb, const int8_t *q, int32_t *out, int N, int K,
                             hipStream_t stream) {
    const int G = (type == TY_FP4 || type == TY_Q6_K || type == TY_NVFP4) ? 16 : 32;
    const long long n = (long long)N * (K / G);
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (type) {
    case TY_Q8_0: hipLaunchKernelGGL(k_block_dots<TY_Q8_0>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_FP4: hipLaunchKernelGGL(k_block_dots<TY_FP4>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_FAST: hipLaunchKernelGGL(k_block_dots<TY_FAST>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_MXFP4:
        hipLaunchKernelGGL(k_block_dots<TY_MXFP4>, grid, dim3(256), 0, stream, W, rb, q, out, N, K);
        break;
    case TY_NVFP4:
        hipLaunchKernelGGL(k_block_dots<TY_NVFP4>, grid, dim3(256), 0, stream, W, rb, q, out, N, K);
        break;
    case TY_Q4_K: hipLaunchKernelGGL(k_block_dots<TY_Q4_K>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_Q5_K: hipLaunchKernelGGL(k_block_dots<TY_Q5_K>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_IQ4_XS:
        hipLaunchKernelGGL(k_block_dots<TY_IQ4_XS>, grid, dim3(256), 0, stream, W, rb, q, out, N, K);
        break;
    case TY_Q6_K: hipLaunchKernelGGL(k_block_dots<TY_Q6_K>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    default: return hipErrorInvalidDeviceFunction;
    }
    return hipGetLastError();
}

}  // namespace pq
