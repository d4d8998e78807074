// moe_dev.h -- device code of the MoE router, shared by its own kernel (moe.hip) and by the expert matvec launch
// that routes in-kernel (mv_tile.hip)
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

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

// the router's LDS for up to 256 PER experts
template <int PER>
struct RouterLds {
    unsigned long long key[256 * PER];
    float red[4];
    float selw[MOE_MAX_USED];
    int selid[MOE_MAX_USED];
    float wsum;
};

// One token's routing by a 256-thread workgroup (every thread calls it; it has barriers): softmax of the n_expert
// logits l (exp(l - max) / sum), the n_used largest probabilities in descending order (equal values: the lower
// expert) by each expert's rank among 64-bit (probability, ~index) keys, their weights divided by max(sum, 2^-14),
// and the shared-expert gate sigmoid(x . w_sh) (w_sh set). Expert e is thread e % 256's e / 256-th value, so the
// reductions' order, and every bit of the result, depend on n_expert alone. Results: ids (ids[n_used] = -1 when
// ids_stride > n_used), wts and sg where those are set, and s.selid / s.selw / s.wsum for every thread on return.
template <int PER>
__device__ __forceinline__ void route_token(const float *__restrict__ l, const float *__restrict__ x,
                                            const float *__restrict__ w_sh, int *__restrict__ ids,
                                            float *__restrict__ wts, float *__restrict__ sg, int n_expert, int n_used,
                                            int n, int ids_stride, RouterLds<PER> &s) {
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
            const uint32_t hi = p == p ? __float_as_uint(p) + 1u : 0u;
            s.key[e] = ((unsigned long long)hi << 32) | (uint32_t)~e;
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
