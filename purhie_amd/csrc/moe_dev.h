// moe_dev.h -- device code of the MoE router, shared by its own kernel (moe.hip) and by the expert matvec launch
// that routes in-kernel (mv_tile.hip)
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#include "device.h"

namespace pq {

constexpr int MOE_MAX_EXPERTS = 1024;
constexpr int MOE_MAX_USED = 64;

// sum / max over the 256 threads of a workgroup (4 waves), the result in every thread
__device__ __forceinline__ float wg_sum(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float wg_max(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// the router's LDS for up to 256 PER experts (wkey, part: the forms for at most 128 and at most 256)
template <int PER>
struct RouterLds {
    unsigned long long key[256 * PER];
    unsigned long long wkey[4][128];
    int part[4][128];
    float red[4];
    float selw[MOE_MAX_USED];
    int selid[MOE_MAX_USED];
    float wsum;
};

// 64-bit key of a probability p of expert e: high word p's bits plus one (probabilities are >= 0, so their bits
// order as the values; a NaN gets 0 and ranks below every number), low word ~e (equal probabilities: the lower
// expert ahead). Keys are distinct, so ranks by them are too.
__device__ __forceinline__ unsigned long long route_key(float p, int e) {
    const uint32_t hi = p == p ? __float_as_uint(p) + 1u : 0u;
    return ((unsigned long long)hi << 32) | (uint32_t)~e;
}

// At most 128 experts: every wave reads all the logits (experts lane and lane + 64), so the softmax's max and sum
// are wave reductions without a barrier, in one order set by n_expert alone (all four waves compute the same
// bits). Each wave keeps its own copy of the keys in LDS (in order within the wave: no barrier) and counts, for
// both its experts, the keys ahead of them among experts [32 w, 32 w + 32); the four counts meet behind one
// barrier. Two barriers in all where the general form takes seven, and wave reductions by DPP: the expert pair
// launch with the routing inside (config 4's decode token) 10.2 -> 8.8 us, the router kernel 4.1 -> 2.5 us. Results
// as route_token's.
template <int PER>
__device__ __forceinline__ void route_token_128(const float *__restrict__ l, const float *__restrict__ x,
                                                const float *__restrict__ w_sh, int *__restrict__ ids,
                                                float *__restrict__ wts, float *__restrict__ sg, int n_expert,
                                                int n_used, int n, int ids_stride, RouterLds<PER> &s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool h0 = lane < n_expert, h1 = lane + 64 < n_expert;
    const float v0 = h0 ? l[lane] : -INFINITY, v1 = h1 ? l[lane + 64] : -INFINITY;
    float dsum = 0.0f;
    if (w_sh) {  // (uniform)
        for (int i = tid; i < n; i += 256) dsum = fmaf(x[i], w_sh[i], dsum);
    }
    const float mx = group_max(fmaxf(v0, v1), 64);
    const float e0 = h0 ? expf(v0 - mx) : 0.0f, e1 = h1 ? expf(v1 - mx) : 0.0f;
    const float sum = group_sum(e0 + e1, 64);
    const float inv = 1.0f / sum;
    const float p0 = e0 * inv, p1 = e1 * inv;
    const unsigned long long k0 = route_key(p0, lane), k1 = route_key(p1, lane + 64);
    // (a missing expert's key is 0, below every real key, so it never counts ahead: the 32 comparisons of a wave
    // need no bound and unroll, their 16 LDS reads in flight together)
    unsigned long long *wk = s.wkey[wave];
    wk[lane] = h0 ? k0 : 0ull;
    wk[lane + 64] = h1 ? k1 : 0ull;
    __builtin_amdgcn_wave_barrier();
    int r0 = 0, r1 = 0;
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
        const ulonglong2 u = *(const ulonglong2 *)(wk + 32 * wave + j);
        r0 += (u.x > k0) + (u.y > k0);
        r1 += (u.x > k1) + (u.y > k1);
    }
    s.part[wave][lane] = r0;
    s.part[wave][lane + 64] = r1;
    __syncthreads();
    if (tid < n_expert) {
        const int r = (s.part[0][tid] + s.part[1][tid]) + (s.part[2][tid] + s.part[3][tid]);
        if (r < n_used) {
            if (ids) ids[r] = tid;
            s.selid[r] = tid;
            s.selw[r] = tid < 64 ? p0 : p1;  // (thread tid holds expert tid as its lane's first or second)
        }
    }
    if (ids && tid == n_used && ids_stride > n_used) ids[n_used] = -1;  // the shared slot
    if (w_sh) {  // (uniform) the shared expert's gate
        dsum = wg_sum(dsum, s.red);
        if (tid == 0) *sg = 1.0f / (1.0f + expf(-dsum));
    }
    __syncthreads();
    if (wts) {  // (uniform) the sum in slot order, as the reference's loop (every thread the same), 8 reads at once
        float ws = 0.0f;
        for (int b = 0; b < n_used; b += 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = s.selw[b + i < n_used ? b + i : 0];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (b + i < n_used) ws += v[i];
        }
        ws = fmaxf(ws, 6.103515625e-5f);
        if (tid < n_used) wts[tid] = s.selw[tid] / ws;
    }
}

// 129 to 256 experts: the 128-expert form with four experts a lane (lane + 64 j). Every wave computes the softmax
// with wave reductions and all the keys; wave w writes the keys of its slice, experts 64 w .. 64 w + 63 (its lanes'
// j = w keys), to its own LDS row and counts, for each of its lanes' four keys, the slice keys ahead of it (32
// 16-byte reads and 256 comparisons a lane); the four waves' counts (at most 64 each, bytes) meet behind one
// barrier. The general form's ranks took each thread 128 LDS reads and 256 comparisons against all the keys, behind
// seven barriers: config 5's decode token (the router inside its expert gate / up launch) 47.0 -> 34.8 us (rounds
// of a wave-wide argmax instead, one per expert used, measured 36.3). Results as route_token's.
template <int PER>
__device__ __forceinline__ void route_token_256(const float *__restrict__ l, const float *__restrict__ x,
                                                const float *__restrict__ w_sh, int *__restrict__ ids,
                                                float *__restrict__ wts, float *__restrict__ sg, int n_expert,
                                                int n_used, int n, int ids_stride, RouterLds<PER> &s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = lane + 64 * j < n_expert ? l[lane + 64 * j] : -INFINITY;
    float dsum = 0.0f;
    if (w_sh) {  // (uniform)
        for (int i = tid; i < n; i += 256) dsum = fmaf(x[i], w_sh[i], dsum);
    }
    const float mx = group_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), 64);
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = lane + 64 * j < n_expert ? expf(v[j] - mx) : 0.0f;
    const float inv = 1.0f / group_sum((p[0] + p[1]) + (p[2] + p[3]), 64);
    unsigned long long k[4];  // (a missing expert's key is 0: below every real key, it never counts ahead)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p[j] *= inv;
        k[j] = lane + 64 * j < n_expert ? route_key(p[j], lane + 64 * j) : 0ull;
    }
    auto mine = [&](auto a) { return wave == 0 ? a[0] : wave == 1 ? a[1] : wave == 2 ? a[2] : a[3]; };
    unsigned long long *wk = s.wkey[wave];
    wk[lane] = mine(k);
    __builtin_amdgcn_wave_barrier();
    int r[4] = {0, 0, 0, 0};
    // (16 keys, 8 reads, at a time: the whole slice's 32 reads in flight took 60 more registers in every kernel
    // that inlines the router)
#pragma unroll 1
    for (int j0 = 0; j0 < 64; j0 += 16) {
#pragma unroll
        for (int j = j0; j < j0 + 16; j += 2) {
            const ulonglong2 u = *(const ulonglong2 *)(wk + j);
#pragma unroll
            for (int q = 0; q < 4; ++q) r[q] += (u.x > k[q]) + (u.y > k[q]);
        }
    }
    uint8_t *part = (uint8_t *)s.part;  // [4][256] bytes within the 128-expert form's ints
#pragma unroll
    for (int q = 0; q < 4; ++q) part[256 * wave + lane + 64 * q] = (uint8_t)r[q];
    __syncthreads();
    if (tid < n_expert) {  // thread tid holds expert tid as its lane's key j = wave
        const int rk = ((int)part[tid] + (int)part[256 + tid]) + ((int)part[512 + tid] + (int)part[768 + tid]);
        if (rk < n_used) {
            if (ids) ids[rk] = tid;
            s.selid[rk] = tid;
            s.selw[rk] = mine(p);
        }
    }
    if (ids && tid == n_used && ids_stride > n_used) ids[n_used] = -1;  // the shared slot
    if (w_sh) {  // (uniform) the shared expert's gate
        dsum = wg_sum(dsum, s.red);
        if (tid == 0) *sg = 1.0f / (1.0f + expf(-dsum));
    }
    __syncthreads();
    if (wts) {  // (uniform) the sum in slot order, as the reference's loop (every thread the same), 8 reads at once
        float ws = 0.0f;
        for (int b = 0; b < n_used; b += 8) {
            float w8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) w8[i] = s.selw[b + i < n_used ? b + i : 0];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (b + i < n_used) ws += w8[i];
        }
        ws = fmaxf(ws, 6.103515625e-5f);
        if (tid < n_used) wts[tid] = s.selw[tid] / ws;
    }
}

// One token's routing by a 256-thread workgroup (every thread calls it; it has barriers): softmax of the n_expert
// logits l (exp(l - max) / sum), the n_used largest probabilities in descending order (equal values: the lower
// expert) by each expert's rank among 64-bit (probability, ~index) keys, their weights divided by max(sum, 2^-14),
// and the shared-expert gate sigmoid(x . w_sh) (w_sh set). Expert e is thread e % 256's e / 256-th value, so the
// reductions' order, and every bit of the result, depend on n_expert alone. Results: ids (ids[n_used] = -1 when
// ids_stride > n_used), wts and sg where those are set, and s.selid / s.selw for every thread on return.
template <int PER>
__device__ __forceinline__ void route_token(const float *__restrict__ l, const float *__restrict__ x,
                                            const float *__restrict__ w_sh, int *__restrict__ ids,
                                            float *__restrict__ wts, float *__restrict__ sg, int n_expert, int n_used,
                                            int n, int ids_stride, RouterLds<PER> &s) {
    if (n_expert <= 128) {  // (uniform)
        route_token_128(l, x, w_sh, ids, wts, sg, n_expert, n_used, n, ids_stride, s);
        return;
    }
    if (n_expert <= 256) {  // (uniform)
        route_token_256(l, x, w_sh, ids, wts, sg, n_expert, n_used, n, ids_stride, s);
        return;
    }
    const int tid = threadIdx.x;
    // the logits once into registers, and the shared expert's dot product, before any wait
    float lv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid + 256 * j;
        lv[j] = e < n_expert ? l[e] : -INFINITY;
    }
    float dsum = 0.0f;
    if (w_sh) {  // (uniform)
        for (int i = tid; i < n; i += 256) dsum = fmaf(x[i], w_sh[i], dsum);
    }

    float mx = lv[0];
#pragma unroll
    for (int j = 1; j < PER; ++j) mx = fmaxf(mx, lv[j]);
    mx = wg_max(mx, s.red);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid + 256 * j;
        lv[j] = e < n_expert ? expf(lv[j] - mx) : 0.0f;
        sum += lv[j];
    }
    sum = wg_sum(sum, s.red);
    const float inv = 1.0f / sum;

    // top n_used by rank: expert e's rank is the number of experts ahead of it, those with a larger probability
    // or an equal one at a lower index (the order of the reference's rounds of argmax). One 64-bit key per
    // expert orders both at once: high word the probability's bits plus one (probabilities are >= 0, so their
    // bits order as the values; a NaN gets 0 and ranks below every number), low word ~e. Keys are distinct, so
    // the ranks are too.
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid + 256 * j;
        if (e < n_expert) {
            const float p = lv[j] * inv;
            lv[j] = p;
            s.key[e] = route_key(p, e);
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid + 256 * j;
        if (256 * j < n_expert) {  // (uniform)
            if (e < n_expert) {
                const unsigned long long k = s.key[e];
                int r = 0;
                int f = 0;
                for (; f + 2 <= n_expert; f += 2) {
                    const ulonglong2 u = *(const ulonglong2 *)(s.key + f);
                    r += (u.x > k) + (u.y > k);
                }
                if (f < n_expert) r += s.key[f] > k;
                if (r < n_used) {
                    if (ids) ids[r] = e;
                    s.selid[r] = e;
                    s.selw[r] = lv[j];
                }
            }
        }
    }
    if (ids && tid == n_used && ids_stride > n_used) ids[n_used] = -1;  // the shared slot
    if (w_sh) {  // (uniform) the shared expert's gate
        dsum = wg_sum(dsum, s.red);
        if (tid == 0) *sg = 1.0f / (1.0f + expf(-dsum));
    }
    __syncthreads();
    if (tid == 0) {  // the sum in slot order, as the reference's loop
        float ws = 0.0f;
        for (int r = 0; r < n_used; ++r) ws += s.selw[r];
        s.wsum = fmaxf(ws, 6.103515625e-5f);
    }
    __syncthreads();
    if (wts && tid < n_used) wts[tid] = s.selw[tid] / s.wsum;
}

}  // namespace pq
