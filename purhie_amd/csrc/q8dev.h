// q8dev.h -- the activation quantizer's per-value step, shared by the standalone quantizer (q8act.hip) and
// the producer kernels that quantize their own output (moe.hip's swiglu), as the reference's q8_block_value
// (src/q8_device.h:54-104).
//
// A 256-thread workgroup (4 waves) holds one 256-value block, one value per thread, and writes both of
// ggml's activation formats, bit-identical to the reference:
//   Q8_0: per 32 values am = max|x|, q = rint(x * (127 / am)) (ties to even), d = fp16(am / 127),
//         s0 = fp16((am / 127) * sum q) kept as float bits (the Q8_1 block sum);
//   Q8_K: per 256 values v = the signed value of largest |x| (lowest index on ties), iscale = -127 / v,
//         q = min(127, rint(iscale * x)), d = 1 / iscale (0 for an all-zero block), sums of every 16 q.
// A 32-value Q8_0 block is half a wave: its reductions stay inside it.
#pragma once

#include "device.h"
#include "kernels.h"

namespace pq {

struct Q8Shared {
    float a[4], v[4];
    int i[4];
};

// value v of thread t of block b (i = 256 b + t; inactive threads past the end hold 0); every thread of the
// workgroup calls it (a barrier inside when o.qK is set)
__device__ __forceinline__ void q8_quantize_value(float v, bool active, int b, Q8Shared &sh, const Q8Ptrs &o) {
    const int t = threadIdx.x, i = b * 256 + t;
    const int lane = t & 63, w = t >> 6;
    const float a = fabsf(v);

    // Q8_0 over the 32 values of this half-wave
    const float am = group_max(a, 32);
    const float id0 = am != 0.0f ? 127.0f / am : 0.0f;
    const int q0 = active ? (int)rintf(v * id0) : 0;
    const int s0 = group_isum(q0, 32);
    if (active) {
        o.q0[i] = (int8_t)q0;
        if ((lane & 31) == 0) {
            const float d = am / 127.0f;
            o.d0[i >> 5] = __half2float(__float2half(d));
            if (o.s0) {
                // fp16(d * s) rounds the product to fp32 first, as the reference. The register barrier keeps the
                // backend from folding multiply and conversion into one v_fma_mix rounding, which differs on the
                // fp16 ties the fp32 rounding makes or breaks (seen at 1 block in ~2700).
                float p = d * (float)s0;
                __asm__ volatile("" : "+v"(p));
                o.s0[i >> 5] = __float_as_int(__half2float(__float2half(p)));
            }
        }
    }
    if (!o.qK) return;  // (uniform)

    // Q8_K over the 256 values: largest |x|, the lowest index on ties
    // (largest |x| with the lowest index is a total order: any order of the pairwise steps picks the same value;
    // the steps are group_sum's, DPP within rows and scalar reads across them)
    float ba = a, bv = v;
    int bi = t;
    auto take = [&](float oa, float ov, int oi) {
        if (oa > ba || (oa == ba && oi < bi)) {
            ba = oa;
            bi = oi;
            bv = ov;
        }
    };
    take(dpp_f<DPP_PAIR>(ba), dpp_f<DPP_PAIR>(bv), dpp_i<DPP_PAIR>(bi));
    take(dpp_f<DPP_QHALF>(ba), dpp_f<DPP_QHALF>(bv), dpp_i<DPP_QHALF>(bi));
    take(dpp_f<DPP_HALF_MIRROR>(ba), dpp_f<DPP_HALF_MIRROR>(bv), dpp_i<DPP_HALF_MIRROR>(bi));
    take(dpp_f<DPP_MIRROR>(ba), dpp_f<DPP_MIRROR>(bv), dpp_i<DPP_MIRROR>(bi));
    {
        const float ra[4] = {readlane_f(ba, 0), readlane_f(ba, 16), readlane_f(ba, 32), readlane_f(ba, 48)};
        const float rv[4] = {readlane_f(bv, 0), readlane_f(bv, 16), readlane_f(bv, 32), readlane_f(bv, 48)};
        const int ri[4] = {__builtin_amdgcn_readlane(bi, 0), __builtin_amdgcn_readlane(bi, 16),
                           __builtin_amdgcn_readlane(bi, 32), __builtin_amdgcn_readlane(bi, 48)};
        ba = ra[0];
        bv = rv[0];
        bi = ri[0];
#pragma unroll
        for (int k = 1; k < 4; ++k) take(ra[k], rv[k], ri[k]);
    }
    if (lane == 0) {
        sh.a[w] = ba;
        sh.v[w] = bv;
        sh.i[w] = bi;
    }
    __syncthreads();
    float fa = sh.a[0], fv = sh.v[0];
    int fi = sh.i[0];
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (sh.a[k] > fa || (sh.a[k] == fa && sh.i[k] < fi)) {
            fa = sh.a[k];
            fi = sh.i[k];
            fv = sh.v[k];
        }
    int q = 0;
    float iscale = 0.0f;
    if (fa != 0.0f) {
        iscale = -127.0f / fv;
        q = min(127, (int)rintf(iscale * v));
    }
    const int s16 = group_isum(q, 16);
    if (active) {
        o.qK[i] = (int8_t)q;
        if (t == 0) o.dK[b] = fa != 0.0f ? 1.0f / iscale : 0.0f;
        if ((lane & 15) == 0) o.bsK[i >> 4] = s16;
    }
}

// The same two formats with a wave per 256-value block b: lane l holds values 4l .. 4l + 3 of it (v, the first at
// index i = 256 b + 4 l; active: inside n, which is a multiple of 32, so a lane's four values are in or out
// together). A Q8_0 block is 8 lanes and the Q8_K block the wave, so the maxima and sums stay in the wave (no LDS,
// no barrier); q0 / qK are written a dword a lane (4-byte aligned). The arithmetic is q8_quantize_value's, value for
// value: maxima and integer sums are exact in any order, and the Q8_K pick (largest |x|, lowest index) is a total
// order, so both write the same bits.
__device__ __forceinline__ void q8_quantize4(const float (&v)[4], bool active, int b, long long i, int lane,
                                             const Q8Ptrs &o) {
    // Q8_0 over 32 values: 8 lanes
    float a[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = fabsf(v[r]);
    const float am = group_max(fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])), 8);
    const float id0 = am != 0.0f ? 127.0f / am : 0.0f;
    int q[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = active ? (int)rintf(v[r] * id0) : 0;
    const int s0 = group_isum((q[0] + q[1]) + (q[2] + q[3]), 8);
    auto pack = [](const int *x) {
        return (uint32_t)(x[0] & 0xff) | (uint32_t)(x[1] & 0xff) << 8 | (uint32_t)(x[2] & 0xff) << 16 |
               (uint32_t)(x[3] & 0xff) << 24;
    };
    if (active) {
        *(uint32_t *)(o.q0 + i) = pack(q);
        if ((lane & 7) == 0) {
            const float d = am / 127.0f;
            o.d0[i >> 5] = __half2float(__float2half(d));
            if (o.s0) {
                float p = d * (float)s0;
                __asm__ volatile("" : "+v"(p));  // (fp16 of the fp32 product: no fused conversion)
                o.s0[i >> 5] = __float_as_int(__half2float(__float2half(p)));
            }
        }
    }
    if (!o.qK) return;

    // Q8_K over the wave's 256 values: the lane's own pick (strict: the lowest index), then the wave's
    float ba = a[0], bv = v[0];
    int bi = 4 * lane;
#pragma unroll
    for (int r = 1; r < 4; ++r)
        if (a[r] > ba) {
            ba = a[r];
            bv = v[r];
            bi = 4 * lane + r;
        }
    auto take = [&](float oa, float ov, int oi) {
        if (oa > ba || (oa == ba && oi < bi)) {
            ba = oa;
            bi = oi;
            bv = ov;
        }
    };
    take(dpp_f<DPP_PAIR>(ba), dpp_f<DPP_PAIR>(bv), dpp_i<DPP_PAIR>(bi));
    take(dpp_f<DPP_QHALF>(ba), dpp_f<DPP_QHALF>(bv), dpp_i<DPP_QHALF>(bi));
    take(dpp_f<DPP_HALF_MIRROR>(ba), dpp_f<DPP_HALF_MIRROR>(bv), dpp_i<DPP_HALF_MIRROR>(bi));
    take(dpp_f<DPP_MIRROR>(ba), dpp_f<DPP_MIRROR>(bv), dpp_i<DPP_MIRROR>(bi));
    const float ra[4] = {readlane_f(ba, 0), readlane_f(ba, 16), readlane_f(ba, 32), readlane_f(ba, 48)};
    const float rv[4] = {readlane_f(bv, 0), readlane_f(bv, 16), readlane_f(bv, 32), readlane_f(bv, 48)};
    const int ri[4] = {__builtin_amdgcn_readlane(bi, 0), __builtin_amdgcn_readlane(bi, 16),
                       __builtin_amdgcn_readlane(bi, 32), __builtin_amdgcn_readlane(bi, 48)};
    ba = ra[0];
    bv = rv[0];
    bi = ri[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) take(ra[r], rv[r], ri[r]);
    float iscale = 0.0f;
    if (ba != 0.0f) iscale = -127.0f / bv;
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = ba != 0.0f ? min(127, (int)rintf(iscale * v[r])) : 0;
    const int s16 = group_isum((q[0] + q[1]) + (q[2] + q[3]), 4);
    if (active) {
        *(uint32_t *)(o.qK + i) = pack(q);
        if (lane == 0) o.dK[b] = ba != 0.0f ? 1.0f / iscale : 0.0f;
        if ((lane & 3) == 0) o.bsK[i >> 4] = s16;
    }
}

}  // namespace pq
