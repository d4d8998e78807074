// matvec.hip -- the HBM-bound decode matvec y = W x_q for GGUF weight blocks on gfx950 (wave64).
//
// Replaces the reference's matvec_q8_<type> / matvec_q8t_<type> / matvec_q8_id_<type>
// (src/matvec_q.hip:1403-1965). Structure, MI355X-first:
//   * a workgroup of 4 waves; L lanes (8..64, a power of two) per row, 64 / L rows per wave;
//   * each lane streams a fixed number of "tasks" (a pair of Q8_0 / ROCmFP4 blocks, a quad of FAST
//     blocks, or one 16-byte quarter-chunk of a K-quant super-block) with wide global loads, U tasks in
//     flight before any arithmetic;
//   * the quantized activation (Q8_0 or Q8_K form, up to 4 tokens) is staged once per workgroup in LDS
//     while the first weight loads are in flight, and read back with 128-bit LDS reads;
//   * integer dots with v_dot4_i32_i8 on codes decoded by v_perm_b32 byte tables;
//   * per task a float term in the reference's per-block form (scale_w * scale_x) * int_sum, summed
//     per lane in task order, then a butterfly over the row's L lanes.
// Per-block integer sums are exact, and the same as the reference's; the float order differs from the
// reference CPU path's sequential sum (checked to 1e-5 of sum |w x| by the parity tests). A token's
// result does not depend on how many tokens share the launch (the same code per token).
#include "device.h"
#include "kernels.h"

namespace pq {

constexpr int MV_THREADS = 256;
constexpr int MV_U = 8;  // tasks a lane keeps in flight

// ---------------------------------------------------------------- activation view (LDS)
template <int NT>
struct Act {
    const int8_t *q[NT];
    const float *d[NT];
    const int32_t *bs[NT];
};

// ---------------------------------------------------------------- per-type task policies

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
    struct Raw {
        uint32_t w[17];
    };
    __device__ static void load(const uint8_t *wr, int task, Raw &r) {
        const uint8_t *p = wr + (long long)task * 68;
#pragma unroll
        for (int k = 0; k < 17; ++k) r.w[k] = ld32_nt(p + 4 * k);
    }
    template <int NT>
    __device__ static void compute(const Raw &r, int task, int, const Act<NT> &x, float acc[NT]) {
        uint32_t qa[8], qb[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            qa[k] = align_bytes(r.w[k + 1], r.w[k], 2);
            qb[k] = r.w[9 + k];
        }
        const float e0 = h2f(r.w[0] & 0xffffu), e1 = h2f(r.w[8] >> 16);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 *xv = (const int4 *)(x.q[t] + task * 64);
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
            const float2 dx = *(const float2 *)(x.d[t] + 2 * task);
            acc[t] = __builtin_fmaf(e0 * dx.x, (float)s0, acc[t]);
            acc[t] = __builtin_fmaf(e1 * dx.y, (float)s1, acc[t]);
        }
    }
};

// one 32-value FP4 block (16 value bytes as 4 dwords: value j in the low nibble of byte j, j + 16 in its
// high nibble) against its Q8_0 activation block: the two half-block integer sums
__device__ __forceinline__ void fp4_block_dots(const uint32_t qs[4], const int4 xa, const int4 xb, int &s0, int &s1) {
    s0 = dot4(fp4x4_lo(qs[0]), xa.x, 0);
    s0 = dot4(fp4x4_lo(qs[1]), xa.y, s0);
    s0 = dot4(fp4x4_lo(qs[2]), xa.z, s0);
    s0 = dot4(fp4x4_lo(qs[3]), xa.w, s0);
    s1 = dot4(fp4x4_hi(qs[0]), xb.x, 0);
    s1 = dot4(fp4x4_hi(qs[1]), xb.y, s1);
    s1 = dot4(fp4x4_hi(qs[2]), xb.z, s1);
    s1 = dot4(fp4x4_hi(qs[3]), xb.w, s1);
}

// ROCmFP4 (type 100): a task is a pair of 18-byte blocks (36 bytes, 4-aligned: K % 64 == 0): block 0's
// values dwords 0..3 and its two UE4M3 half-block scales bytes 16, 17; block 1's values bytes 18..33 and
// scales bytes 34, 35. Per block the reference's term (e0 dx) s0 + (e1 dx) s1.
template <>
struct Mv<TY_FP4> {
    static constexpr int ACT_BLK = 32;
    static constexpr bool KQ = false;
    __host__ __device__ static int tasks(int K) { return K / 64; }
    struct Raw {
        uint32_t w[9];
    };
    __device__ static void load(const uint8_t *wr, int task, Raw &r) {
        const uint8_t *p = wr + (long long)task * 36;
#pragma unroll
        for (int k = 0; k < 9; ++k) r.w[k] = ld32_nt(p + 4 * k);
    }
    template <int NT>
    __device__ static void compute(const Raw &r, int task, int, const Act<NT> &x, float acc[NT]) {
        const uint32_t qa[4] = {r.w[0], r.w[1], r.w[2], r.w[3]};
        uint32_t qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qb[k] = align_bytes(r.w[5 + k], r.w[4 + k], 2);
        const float ea0 = ue4m3_half(r.w[4]), ea1 = ue4m3_half(r.w[4] >> 8);
        const float eb0 = ue4m3_half(r.w[8] >> 16), eb1 = ue4m3_half(r.w[8] >> 24);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 *xv = (const int4 *)(x.q[t] + task * 64);
            int a0, a1, b0, b1;
            fp4_block_dots(qa, xv[0], xv[1], a0, a1);
            fp4_block_dots(qb, xv[2], xv[3], b0, b1);
            const float2 dx = *(const float2 *)(x.d[t] + 2 * task);
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
    struct Raw {
        uint32_t w[17];
    };
    __device__ static void load(const uint8_t *wr, int task, Raw &r) {
        const uint8_t *p = wr + (long long)task * 68;
#pragma unroll
        for (int k = 0; k < 17; ++k) r.w[k] = ld32_nt(p + 4 * k);
    }
    __device__ static __forceinline__ uint32_t dw(const uint32_t *w, int off) {  // off compile-time
        return (off & 3) == 0 ? w[off >> 2] : align_bytes(w[(off >> 2) + 1], w[off >> 2], off & 3);
    }
    template <int NT>
    __device__ static void compute(const Raw &r, int task, int, const Act<NT> &x, float acc[NT]) {
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
                const int4 *xv = (const int4 *)(x.q[t] + task * 128 + 32 * j);
                int s0, s1;
                fp4_block_dots(qs, xv[0], xv[1], s0, s1);
                acc[t] = __builtin_fmaf(e * x.d[t][4 * task + j], (float)(s0 + s1), acc[t]);
            }
        }
    }
};

// Q4_K: a task is one of the 8 sixteen-byte quarter-chunks s of a 144-byte super-block (16-aligned):
// qs bytes 16 s .. 16 s + 15, i.e. chunk c = s / 2, values 64 c + l + 0..15 (low nibbles, sub-block 2c)
// and 64 c + 32 + l + 0..15 (high nibbles, sub-block 2c + 1), l = 16 (s & 1); plus the block header
// (d, dmin, the 12 scale bytes). The lane with quarter s also applies sub-block s's min through the Q8_K
// group sums 2 s, 2 s + 1 (reference src/matvec_q.hip:1752-1789).
template <>
struct Mv<TY_Q4_K> {
    static constexpr int ACT_BLK = 256;
    static constexpr bool KQ = true;
    __host__ __device__ static int tasks(int K) { return K / 256 * 8; }
    struct Raw {
        u32x4 h, qs;
    };
    __device__ static void load(const uint8_t *wr, int task, Raw &r) {
        const uint8_t *p = wr + (long long)(task >> 3) * 144;
        r.h = ld128_nt(p);
        r.qs = ld128_nt(p + 16 + 16 * (task & 7));
    }
    // 6-bit scales of sub-blocks 2c, 2c + 1 and the min of sub-block s from the scale dwords y, z, w
    // (bytes 4..15 of the block), gathered with v_perm_b32 using lane-constant selectors.
    struct Sel {
        uint32_t p, pmask, q;   // scales: (perm(w, y, p) & pmask) | ((perm(w, y, q) >> 6) & 0x0303) << 4
        uint32_t m, msh, mmask, n;  // min: ((perm(w, z, m) >> msh) & mmask) | ((perm(w, z, n) >> 6) & 3) << 4
    };
    __device__ static Sel selectors(int s) {
        const int c = s >> 1;
        Sel o;
        if (c < 2) {  // sub-blocks 2c, 2c + 1 < 4: scale = byte j & 63 (y)
            o.p = (uint32_t)(2 * c) | (uint32_t)(2 * c + 1) << 8 | 0x0c0c0000u;
            o.pmask = 0x3f3fu;
            o.q = 0x0c0c0c0cu;
        } else {  // j = 4 + i: scale = (w byte i & 15) | (y byte i >> 6) << 4
            const int i = 2 * c - 4;
            o.p = (uint32_t)(4 + i) | (uint32_t)(5 + i) << 8 | 0x0c0c0000u;
            o.pmask = 0x0f0fu;
            o.q = (uint32_t)i | (uint32_t)(i + 1) << 8 | 0x0c0c0000u;
        }
        if (s < 4) {  // min = z byte s & 63
            o.m = (uint32_t)s | 0x0c0c0c00u;
            o.msh = 0;
            o.mmask = 63;
            o.n = 0x0c0c0c0cu;
        } else {  // min = (w byte i >> 4) | (z byte i >> 6) << 4
            const int i = s - 4;
            o.m = (uint32_t)(4 + i) | 0x0c0c0c00u;
            o.msh = 4;
            o.mmask = 15;
            o.n = (uint32_t)i | 0x0c0c0c00u;
        }
        return o;
    }
    template <int NT>
    __device__ static void compute(const Raw &r, int task, int s, const Act<NT> &x, float acc[NT]) {
        const Sel o = selectors(s);
        const uint32_t sc2 = (__builtin_amdgcn_perm(r.h.w, r.h.y, o.p) & o.pmask) |
                             (((__builtin_amdgcn_perm(r.h.w, r.h.y, o.q) >> 6) & 0x0303u) << 4);
        const int sc_lo = (int)(sc2 & 0xffu), sc_hi = (int)(sc2 >> 8);
        const int mn = (int)(((__builtin_amdgcn_perm(r.h.w, r.h.z, o.m) >> o.msh) & o.mmask) |
                             (((__builtin_amdgcn_perm(r.h.w, r.h.z, o.n) >> 6) & 3u) << 4));
        const float dw = h2f(r.h.x & 0xffffu), dm = h2f(r.h.x >> 16);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        const int sb = task >> 3, c = s >> 1, l = (s & 1) * 16;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int8_t *xb = x.q[t] + sb * 256 + 64 * c + l;
            const int4 xl = *(const int4 *)xb, xh = *(const int4 *)(xb + 32);
            int slo = dot4((int)(q[0] & 0x0f0f0f0fu), xl.x, 0);
            slo = dot4((int)(q[1] & 0x0f0f0f0fu), xl.y, slo);
            slo = dot4((int)(q[2] & 0x0f0f0f0fu), xl.z, slo);
            slo = dot4((int)(q[3] & 0x0f0f0f0fu), xl.w, slo);
            int shi = dot4((int)((q[0] >> 4) & 0x0f0f0f0fu), xh.x, 0);
            shi = dot4((int)((q[1] >> 4) & 0x0f0f0f0fu), xh.y, shi);
            shi = dot4((int)((q[2] >> 4) & 0x0f0f0f0fu), xh.z, shi);
            shi = dot4((int)((q[3] >> 4) & 0x0f0f0f0fu), xh.w, shi);
            const int2 b2 = *(const int2 *)(x.bs[t] + sb * 16 + 2 * s);
            const int isum = sc_lo * slo + sc_hi * shi;
            const int msum = mn * (b2.x + b2.y);
            const float dx = x.d[t][sb];
            acc[t] = __builtin_fmaf(dw * dx, (float)isum, acc[t]);
            acc[t] = __builtin_fmaf(-(dm * dx), (float)msum, acc[t]);
        }
    }
};

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
    struct Raw {
        uint32_t ql[5], qh[5];
        uint32_t off;
        int sc_lo, sc_hi;
        uint32_t scp, d;
    };
    __device__ static void load(const uint8_t *wr, int task, Raw &r) {
        const int s = task & 7, h = s >> 2, rr = (s & 3) * 16, l = rr & 31, second = rr >= 32;
        const uint8_t *b = wr + (long long)(task >> 3) * 210;
        const uint32_t off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *a1 = b + 64 * h + rr - off, *a2 = b + 128 + 32 * h + l - off;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            r.ql[k] = ld32_nt(a1 + 4 * k);
            r.qh[k] = ld32_nt(a2 + 4 * k);
        }
        r.off = off;
        const int g_lo = 8 * h + (l >> 4) + (second ? 2 : 0);
        r.sc_lo = (int)((const int8_t *)b)[192 + g_lo];
        r.sc_hi = (int)((const int8_t *)b)[192 + g_lo + 4];
        r.scp = *(const uint16_t *)(b + 192 + 2 * s);
        r.d = *(const uint16_t *)(b + 208);
    }
    template <int NT>
    __device__ static void compute(const Raw &r, int task, int s, const Act<NT> &x, float acc[NT]) {
        const int h = s >> 2, rr = (s & 3) * 16, l = rr & 31, second = rr >= 32;
        const int sh = second ? 2 : 0;
        const int v_lo = 128 * h + (second ? 32 : 0) + l;
        uint32_t vlo[4], vhi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t ql = align_bytes(r.ql[k + 1], r.ql[k], r.off);
            const uint32_t qh = align_bytes(r.qh[k + 1], r.qh[k], r.off);
            vlo[k] = (ql & 0x0f0f0f0fu) | (((qh >> sh) & 0x03030303u) << 4);
            vhi[k] = ((ql >> 4) & 0x0f0f0f0fu) | (((qh >> (sh + 4)) & 0x03030303u) << 4);
        }
        const int sca = (int)(int8_t)(r.scp & 0xffu), scb = (int)(int8_t)(r.scp >> 8);
        const float dw = h2f(r.d);
        const int sb = task >> 3;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int8_t *xb = x.q[t] + sb * 256 + v_lo;
            const int4 xl = *(const int4 *)xb, xh = *(const int4 *)(xb + 64);
            int slo = dot4((int)vlo[0], xl.x, 0);
            slo = dot4((int)vlo[1], xl.y, slo);
            slo = dot4((int)vlo[2], xl.z, slo);
            slo = dot4((int)vlo[3], xl.w, slo);
            int shi = dot4((int)vhi[0], xh.x, 0);
            shi = dot4((int)vhi[1], xh.y, shi);
            shi = dot4((int)vhi[2], xh.z, shi);
            shi = dot4((int)vhi[3], xh.w, shi);
            const int2 b2 = *(const int2 *)(x.bs[t] + sb * 16 + 2 * s);
            int isum = r.sc_lo * slo + r.sc_hi * shi;
            isum -= 32 * (sca * b2.x + scb * b2.y);
            acc[t] = __builtin_fmaf(dw * x.d[t][sb], (float)isum, acc[t]);
        }
    }
};

// Staging of NT tokens' activations into LDS: values (NT K bytes), scales (NT K / blk floats), group
// sums (K-quants, NT K / 16 ints); the sources are contiguous (token t at + t K, ...).
struct StageCtx {
    const int8_t *q;
    const float *d;
    const int32_t *bs;
    int8_t *sq;
    float *sd;
    int32_t *sbs;
    int nq, nd, nbs;  // bytes, floats, ints
};

__device__ __forceinline__ void stage_act(const StageCtx &c) {
    for (int i = threadIdx.x * 16; i < c.nq; i += MV_THREADS * 16) *(int4 *)(c.sq + i) = *(const int4 *)(c.q + i);
    for (int i = threadIdx.x; i < c.nd; i += MV_THREADS) c.sd[i] = c.d[i];
    for (int i = threadIdx.x; i < c.nbs; i += MV_THREADS) c.sbs[i] = c.bs[i];
    __syncthreads();
}

// ---------------------------------------------------------------- the row loop shared by the kernels

template <int TYPE, int NT, bool STAGE>
__device__ __forceinline__ void row_sum(const uint8_t *wr, int K, int gl, int L, const Act<NT> &x, float acc[NT],
                                        bool valid, const StageCtx &stage) {
    using P = Mv<TYPE>;
    const int ntask = P::tasks(K);
    const int s = gl & 7;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    typename P::Raw raw[MV_U];
    int task = gl;
    // first batch in flight before the activation is staged (STAGE) or read through the caches
#pragma unroll
    for (int u = 0; u < MV_U; ++u)
        if (valid && task + u * L < ntask) P::load(wr, task + u * L, raw[u]);
    if (STAGE) stage_act(stage);
    if (!valid) return;
    for (;;) {
#pragma unroll
        for (int u = 0; u < MV_U; ++u)
            if (task + u * L < ntask) P::template compute<NT>(raw[u], task + u * L, s, x, acc);
        task += MV_U * L;
        if (task >= ntask) break;
#pragma unroll
        for (int u = 0; u < MV_U; ++u)
            if (task + u * L < ntask) P::load(wr, task + u * L, raw[u]);
    }
}

template <int TYPE>
__host__ __device__ constexpr int act_blk() {
    return Mv<TYPE>::ACT_BLK;
}

// LDS bytes for NT tokens of K values
template <int TYPE>
__host__ __device__ inline int lds_bytes(int K, int NT) {
    return NT * K + NT * (K / act_blk<TYPE>()) * 4 + (Mv<TYPE>::KQ ? NT * (K / 16) * 4 : 0);
}

template <int TYPE, int NT>
__device__ __forceinline__ void setup_lds(uint8_t *smem, const int8_t *q, const float *d, const int32_t *bs, int K,
                                          StageCtx &c, Act<NT> &x) {
    const int nblk = K / act_blk<TYPE>();
    c.q = q;
    c.d = d;
    c.bs = bs;
    c.sq = (int8_t *)smem;
    c.sd = (float *)(smem + NT * K);
    c.sbs = (int32_t *)(c.sd + NT * nblk);
    c.nq = NT * K;
    c.nd = NT * nblk;
    c.nbs = Mv<TYPE>::KQ ? NT * (K / 16) : 0;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        x.q[t] = c.sq + t * K;
        x.d[t] = c.sd + t * nblk;
        x.bs[t] = c.sbs + t * (K / 16);
    }
}

// ---------------------------------------------------------------- dense decode kernel

template <int TYPE, int NT>
__device__ __forceinline__ void global_act(const int8_t *q, const float *d, const int32_t *bs, int K, Act<NT> &x) {
    const int nblk = K / act_blk<TYPE>();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        x.q[t] = q + t * K;
        x.d[t] = d + t * nblk;
        x.bs[t] = bs + t * (K / 16);
    }
}

// STAGE: the activation staged in LDS once per workgroup behind a barrier; otherwise read through the
// L1 / L2 caches (the weights stream past them with non-temporal loads), every wave independent.
template <int TYPE, int NT, bool STAGE>
__global__ void __launch_bounds__(MV_THREADS) k_matvec(MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    StageCtx c;
    Act<NT> x;
    if (STAGE) setup_lds<TYPE, NT>(smem, a.q, a.d, a.bs, a.K, c, x);
    else global_act<TYPE, NT>(a.q, a.d, a.bs, a.K, x);
    const int L = a.L;
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int row = (blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    const bool valid = row < a.Nt;
    const int mat = valid ? (row >= a.bound[0]) + (row >= a.bound[1]) + (row >= a.bound[2]) : 0;
    const int base = mat == 0 ? 0 : a.bound[mat - 1];
    const uint8_t *wr = a.W[mat] + (long long)(row - base) * a.row_bytes;
    float acc[NT];
    row_sum<TYPE, NT, STAGE>(wr, a.K, gl, L, x, acc, valid, c);
    if (!valid) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v = group_sum(acc[t], L);
        if (gl == 0) a.y[mat][(long long)t * a.ystride[mat] + (row - base)] = v * a.osc[mat];
    }
}

// ---------------------------------------------------------------- MoE expert-indexed kernel

template <int TYPE, bool STAGE>
__global__ void __launch_bounds__(MV_THREADS) k_matvec_id(MvIdArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int m = (int)blockIdx.y >= a.n_used ? 1 : 0;
    const int slot = (int)blockIdx.y - m * a.n_used, t = blockIdx.z;
    const int e = a.ids[t * a.n_used + slot];
    const long long in_row = a.x_per_slot ? (long long)t * a.n_used + slot : t;
    const int K = a.K;
    const int kb = K / act_blk<TYPE>();
    StageCtx c;
    Act<1> x;
    const int32_t *bsr = a.bs ? a.bs + in_row * (K / 16) : nullptr;
    if (STAGE) setup_lds<TYPE, 1>(smem, a.q + in_row * K, a.d + in_row * kb, bsr, K, c, x);
    else global_act<TYPE, 1>(a.q + in_row * K, a.d + in_row * kb, bsr, K, x);
    const int L = a.L;
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int row = (blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    const bool valid = row < a.N;
    const uint8_t *wr = e >= 0 ? a.W[m] + ((long long)e * a.N + row) * a.row_bytes : a.Wx[m] + (long long)row * a.row_bytes;
    float acc[1];
    row_sum<TYPE, 1, STAGE>(wr, K, gl, L, x, acc, valid, c);
    if (!valid) return;
    const float v = group_sum(acc[0], L);
    const float sc = e < 0 ? a.sx[m] : a.es[m] ? a.es[m][e] : a.s[m];
    if (gl == 0) a.y[m][((long long)t * a.n_used + slot) * a.N + row] = v * sc;
}

// ---------------------------------------------------------------- per-group integer dots (test hook)
// One thread per (row, group); the same code decoders as the kernels above.

__device__ __forceinline__ int cb_value(uint32_t nib) { return (int)(int8_t)(fp4x4(nib) & 0xffu); }

template <int TYPE>
__global__ void k_block_dots(const uint8_t *W, long long rb, const int8_t *q, int32_t *out, int N, int K) {
    constexpr int G = (TYPE == TY_FP4 || TYPE == TY_Q6_K) ? 16 : 32;
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
    } else if (TYPE == TY_Q4_K) {
        const uint8_t *b = row + 144 * (g >> 3);
        const int j = g & 7;  // sub-block: chunk j / 2, high nibbles for odd j
        for (int i2 = 0; i2 < 32; ++i2) {
            const uint8_t v = b[16 + 32 * (j >> 1) + i2];
            s += (int)((j & 1) ? (v >> 4) : (v & 0xf)) * xg[i2];
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

// PURHIE_MV_STAGE=1: stage the activation in LDS (the A/B alternative of the cached reads)
static bool stage_activations() {
    static const bool v = getenv("PURHIE_MV_STAGE") && atoi(getenv("PURHIE_MV_STAGE")) != 0;
    return v;
}

static int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

template <int TYPE>
static int tasks_of(int K) {
    return Mv<TYPE>::tasks(K);
}

int matvec_lanes(int type, int K, long long rows) {
    int nt = 0;
    switch (type) {
    case TY_Q8_0: nt = tasks_of<TY_Q8_0>(K); break;
    case TY_FP4: nt = tasks_of<TY_FP4>(K); break;
    case TY_FAST: nt = tasks_of<TY_FAST>(K); break;
    case TY_Q4_K: nt = tasks_of<TY_Q4_K>(K); break;
    case TY_Q6_K: nt = tasks_of<TY_Q6_K>(K); break;
    default: return 0;
    }
    // about 6 tasks per lane (all of a lane's loads in flight at once, MV_U = 8), at least 8 lanes (the
    // K-quants' 8 quarters of a super-block)
    int L = pow2_at_least((nt + 5) / 6);
    if (L < 8) L = 8;
    if (L > 64) L = 64;
    // few rows in the launch: more lanes per row, to keep enough waves in flight
    while (L < 64 && rows * L / 64 < 2048 && nt > L) L <<= 1;
    if (const char *e = getenv("PURHIE_MV_LANES")) {
        const int v = atoi(e);
        if (v >= 8 && v <= 64 && (v & (v - 1)) == 0) L = v;
    }
    return L;
}

template <int TYPE, int NT>
static hipError_t launch_t(const MvArgs &a, hipStream_t stream) {
    const int rows_per_wg = (MV_THREADS / 64) * (64 / a.L);
    const unsigned grid = (unsigned)((a.Nt + rows_per_wg - 1) / rows_per_wg);
    const size_t lds = (size_t)lds_bytes<TYPE>(a.K, NT);
    if (stage_activations() && lds <= 65536)
        hipLaunchKernelGGL((k_matvec<TYPE, NT, true>), dim3(grid), dim3(MV_THREADS), lds, stream, a);
    else
        hipLaunchKernelGGL((k_matvec<TYPE, NT, false>), dim3(grid), dim3(MV_THREADS), 0, stream, a);
    return hipGetLastError();
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
    switch (type) {
    case TY_Q8_0: return launch_nt<TY_Q8_0>(a, stream);
    case TY_FP4: return launch_nt<TY_FP4>(a, stream);
    case TY_FAST: return launch_nt<TY_FAST>(a, stream);
    case TY_Q4_K: return launch_nt<TY_Q4_K>(a, stream);
    case TY_Q6_K: return launch_nt<TY_Q6_K>(a, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

template <int TYPE>
static hipError_t launch_id_t(const MvIdArgs &a, hipStream_t stream) {
    const int rows_per_wg = (MV_THREADS / 64) * (64 / a.L);
    const dim3 grid((unsigned)((a.N + rows_per_wg - 1) / rows_per_wg), (unsigned)(a.n_used * a.nmat), (unsigned)a.T);
    const size_t lds = (size_t)lds_bytes<TYPE>(a.K, 1);
    if (stage_activations() && lds <= 65536)
        hipLaunchKernelGGL((k_matvec_id<TYPE, true>), grid, dim3(MV_THREADS), lds, stream, a);
    else
        hipLaunchKernelGGL((k_matvec_id<TYPE, false>), grid, dim3(MV_THREADS), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_matvec_id(int type, const MvIdArgs &a, hipStream_t stream) {
    switch (type) {
    case TY_Q8_0: return launch_id_t<TY_Q8_0>(a, stream);
    case TY_FP4: return launch_id_t<TY_FP4>(a, stream);
    case TY_FAST: return launch_id_t<TY_FAST>(a, stream);
    case TY_Q4_K: return launch_id_t<TY_Q4_K>(a, stream);
    case TY_Q6_K: return launch_id_t<TY_Q6_K>(a, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

hipError_t launch_block_dots(int type, const uint8_t *W, long long rb, const int8_t *q, int32_t *out, int N, int K,
                             hipStream_t stream) {
    const int G = (type == TY_FP4 || type == TY_Q6_K) ? 16 : 32;
    const long long n = (long long)N * (K / G);
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (type) {
    case TY_Q8_0: hipLaunchKernelGGL(k_block_dots<TY_Q8_0>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_FP4: hipLaunchKernelGGL(k_block_dots<TY_FP4>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_FAST: hipLaunchKernelGGL(k_block_dots<TY_FAST>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_Q4_K: hipLaunchKernelGGL(k_block_dots<TY_Q4_K>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    case TY_Q6_K: hipLaunchKernelGGL(k_block_dots<TY_Q6_K>, grid, dim3(256), 0, stream, W, rb, q, out, N, K); break;
    default: return hipErrorInvalidDeviceFunction;
    }
    return hipGetLastError();
}

}  // namespace pq
