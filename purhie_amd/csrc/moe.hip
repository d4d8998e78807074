// moe.hip -- the mixture-of-experts glue around the expert matvecs (gfx950, wave64): router, grouping,
// combine and SwiGLU with the activation quantizer fused in. The reference's gpu_ops.hip:103-330
// (swiglu, moe_router + router_select, moe_combine, moe_group); the C ABI is include/moe_ops.h.
//
//   k_add_rmsnorm  x_out = x_in + add, y = RMSNorm(x_out) * w, and y quantized in the same launch (the producer of
//                  most matvec inputs; k_add_rmsnorm_rows for many rows, the same bits).
//   k_swiglu4      out = SiLU(g) * u (g / (1 + exp(-g)) * u), and, with a qmatvec_q8, quantized in the same
//                  launch: a wave per 256-value block, four values a lane; k_swiglu, a 256-thread workgroup per
//                  block (q8dev.h), takes unaligned buffers and n % 32 != 0. Both write the same bits.
//   k_moe_router   a workgroup per token: softmax of the router logits (exp(l - max) / sum), the n_used
//                  largest probabilities in descending order (equal values: the lower expert) by each expert's
//                  rank among 64-bit (probability, ~index) keys, their weights divided by max(sum, 2^-14), and
//                  the shared-expert gate sigmoid(x . w_shexp).
//   k_moe_combine  out = sum_j w_j down_j in slot order (+ sg shared), rounded after every product and sum
//                  (no contraction) as the reference's CPU add chain.
//   k_moe_group    one 1024-thread workgroup: entries (token, slot) counted per expert in LDS, two exclusive
//                  scans (entry and tile offsets), then each entry placed by an LDS atomic. Counts and tiles
//                  are deterministic; the order of the entries inside an expert's run is not, and nothing
//                  depends on it (every entry's value is computed alone).
#include "q8dev.h"
#include "moe_dev.h"
#include "moe_ops.h"

namespace pq {

// bpw 256-value blocks per workgroup (8 for large n: one block per workgroup spends its time starting workgroups),
// one value per thread each, the next block's inputs loaded before the current one is quantized
__global__ void __launch_bounds__(256) k_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                                                float *__restrict__ out, int n, Q8Ptrs o, int quantize, int bpw) {
    __shared__ Q8Shared sh;
    const int b0 = blockIdx.x * bpw, t = threadIdx.x;
    const int nb = (n + 255) / 256, bn = nb - b0 < bpw ? nb - b0 : bpw;
    float ga = 0.0f, ua = 0.0f;
    if (b0 * 256 + t < n) {
        ga = g[b0 * 256 + t];
        ua = u[b0 * 256 + t];
    }
    for (int k = 0; k < bn; ++k) {  // (uniform)
        const int i = (b0 + k) * 256 + t;
        const bool active = i < n;
        const float a = ga, ub = ua;
        if (k + 1 < bn && i + 256 < n) {
            ga = g[i + 256];
            ua = u[i + 256];
        }
        float v = 0.0f;
        if (active) {
            v = a / (1.0f + expf(-a)) * ub;
            if (out) out[i] = v;  // (uniform: null when only the quantized form is wanted)
        }
        if (quantize) {  // (uniform)
            if (k) __syncthreads();  // the previous block's reads of sh are done
            q8_quantize_value(v, active, b0 + k, sh, o);
        }
    }
}

// The same values and bits with a wave per 256-value block (n % 32 == 0, 16-byte aligned g / u / out, 4-byte
// aligned q0 / qK): lane l holds values 4l .. 4l + 3 of the block (one 16-byte load of g and of u, one store), and
// q8_quantize4 quantizes them within the wave. BW blocks a wave, their loads issued before the first is computed.
template <int BW>
__global__ void __launch_bounds__(256) k_swiglu4(const float4 *__restrict__ g, const float4 *__restrict__ u,
                                                 float4 *__restrict__ out, int n, Q8Ptrs o, int quantize) {
    const int lane = threadIdx.x & 63;
    const int b0 = ((blockIdx.x * blockDim.x + threadIdx.x) >> 6) * BW, nb = (n + 255) / 256;
    float4 ga[BW], ua[BW];
    // every lane loads (past the end: the last four values again, never used), so the loads have no branch around
    // them and the waits count them exactly
    const long long last4 = n / 4 - 1;
#pragma unroll
    for (int k = 0; k < BW; ++k) {
        const long long i4 = (long long)(b0 + k) * 64 + lane;
        ga[k] = g[i4 < last4 ? i4 : last4];
        ua[k] = u[i4 < last4 ? i4 : last4];
    }
#pragma unroll
    for (int k = 0; k < BW; ++k) {
        const int b = b0 + k;
        if (b >= nb) break;  // (uniform)
        const long long i4 = (long long)b * 64 + lane;
        const bool active = 4 * i4 < n;  // (n % 32 == 0: a lane's four values together)
        const float gv[4] = {ga[k].x, ga[k].y, ga[k].z, ga[k].w}, uv[4] = {ua[k].x, ua[k].y, ua[k].z, ua[k].w};
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = active ? gv[r] / (1.0f + expf(-gv[r])) * uv[r] : 0.0f;
        if (active && out) out[i4] = make_float4(v[0], v[1], v[2], v[3]);  // (out null: only the quantized form)
        if (quantize) q8_quantize4(v, active, b, 4 * i4, lane, o);
    }
}

// ---------------------------------------------------------------- add + RMSNorm, the matvec inputs' producer
// x_out = x_in + add (add set), y = x_out / sqrt(mean(x_out^2) + eps) * w, and y quantized for the int8 matvecs
// in the same launch (src/gpu_ops.hip:17-100). The sum of squares has one order in both kernels: thread t adds
// the squares of values t, t + 256, ... in turn, a wave64 butterfly adds the 64 threads of a wave, and the four
// wave sums are added as (w0 + w1) + (w2 + w3); a row's result is therefore the same whatever T is.
__device__ __forceinline__ float norm_total(float ss, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// one token's row in blocks: grid (ceil(n / 256), T); every workgroup sums its row's squares itself (a row is a
// few KB, its re-reads hit the cache) and normalizes and quantizes its own 256 values, so the whole GPU works on
// one token
__global__ void __launch_bounds__(256) k_add_rmsnorm(const float *__restrict__ x_in, const float *__restrict__ add,
                                                     float *__restrict__ x_out, const float *__restrict__ w,
                                                     float *__restrict__ y, int n, float eps, Q8Ptrs o, int quantize) {
    __shared__ float red[4];
    __shared__ Q8Shared sh;
    const long long row = (long long)blockIdx.y * n;
    const float *xi = x_in + row, *ad = add ? add + row : nullptr;
    const int t = threadIdx.x, i = blockIdx.x * 256 + t;
    float ss = 0.0f;
    for (int k = t; k < n; k += 256) {
        const float v = ad ? xi[k] + ad[k] : xi[k];
        ss += v * v;
    }
    const float inv = 1.0f / sqrtf(norm_total(ss, red) / (float)n + eps);
    const bool active = i < n;
    float v = 0.0f;
    if (active) {
        v = ad ? xi[i] + ad[i] : xi[i];
        if (ad) x_out[row + i] = v;
        v = v * inv * (w ? w[i] : 1.0f);
        y[row + i] = v;
    }
    if (quantize) q8_quantize_value(v, active, (int)blockIdx.y * (n / 256) + (int)blockIdx.x, sh, o);  // (uniform)
}

// many rows (prefill): one workgroup per row, read once; thread t holds values t + 256 j (n <= 256 NORM_ROWS_V)
constexpr int NORM_ROWS_V = 32;
__global__ void __launch_bounds__(256) k_add_rmsnorm_rows(const float *__restrict__ x_in,
                                                          const float *__restrict__ add, float *__restrict__ x_out,
                                                          const float *__restrict__ w, float *__restrict__ y, int n,
                                                          float eps, Q8Ptrs o, int quantize) {
    __shared__ float red[4];
    __shared__ Q8Shared sh;
    const long long row = (long long)blockIdx.x * n;
    const float *xi = x_in + row, *ad = add ? add + row : nullptr;
    const int t = threadIdx.x, nb = (n + 255) / 256;
    float x[NORM_ROWS_V];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NORM_ROWS_V; ++j) {
        const int k = t + 256 * j;
        x[j] = 0.0f;
        if (j < nb && k < n) {
            x[j] = ad ? xi[k] + ad[k] : xi[k];
            ss += x[j] * x[j];
        }
    }
    const float inv = 1.0f / sqrtf(norm_total(ss, red) / (float)n + eps);
#pragma unroll
    for (int j = 0; j < NORM_ROWS_V; ++j) {
        if (j < nb) {  // (uniform)
            const int k = t + 256 * j;
            const bool active = k < n;
            float v = 0.0f;
            if (active) {
                if (ad) x_out[row + k] = x[j];
                v = x[j] * inv * (w ? w[k] : 1.0f);
                y[row + k] = v;
            }
            if (quantize) {  // (uniform; n % 256 == 0 when quantizing)
                if (j) __syncthreads();  // the previous block's reads of sh are done
                q8_quantize_value(v, active, (int)blockIdx.x * nb + j, sh, o);
            }
        }
    }
}

__global__ void __launch_bounds__(256) k_moe_router(const float *__restrict__ logits, const float *__restrict__ x,
                                                    const float *__restrict__ w_sh, int *__restrict__ ids,
                                                    float *__restrict__ wts, float *__restrict__ sg, int n_expert,
                                                    int n_used, int n, int ids_stride) {
    __shared__ RouterLds<MOE_MAX_EXPERTS / 256> s;
    const int t = blockIdx.x;
    route_token(logits + (long long)t * n_expert, w_sh ? x + (long long)t * n : nullptr, w_sh,
                ids + (long long)t * ids_stride, wts + (long long)t * n_used, w_sh ? sg + t : nullptr, n_expert, n_used,
                n, ids_stride, s);
}

// Up to CB slots' values of an output are loaded together before the add chain (slots past n_used load slot
// n_used - 1 again, unused), the rest one after another.
constexpr int CB = 8;

__global__ void __launch_bounds__(256) k_moe_combine(const float *__restrict__ down, const float *__restrict__ wts,
                                                     const float *__restrict__ shared, const float *__restrict__ sg,
                                                     const int *__restrict__ ids, const float *__restrict__ es,
                                                     float *__restrict__ out, int n_used, int n) {
#pragma clang fp contract(off)  // (every product and sum rounds on its own, as the reference's add chain)
    const int t = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float *d = down + (long long)t * n_used * n + i;
    float dv[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) dv[j] = d[(long long)(j < n_used ? j : n_used - 1) * n];
    const float s = shared ? shared[(long long)t * n + i] : 0.0f;
    auto dj = [&](int j) { return j < CB ? dv[j] : d[(long long)j * n]; };
    float acc;
    if (!wts) {  // (uniform) weight 1
        acc = dv[0];
#pragma unroll
        for (int j = 1; j < CB; ++j)
            if (j < n_used) acc = acc + dv[j];
        for (int j = CB; j < n_used; ++j) acc = acc + d[(long long)j * n];
    } else {
        const float *w = wts + (long long)t * n_used;
        const int *e = ids + (long long)t * n_used;
        acc = es ? (dv[0] * es[e[0]]) * w[0] : w[0] * dv[0];
#pragma unroll
        for (int j = 1; j < CB; ++j)
            if (j < n_used) acc = acc + (es ? (dv[j] * es[e[j]]) * w[j] : w[j] * dv[j]);
        for (int j = CB; j < n_used; ++j) {
            const float v = dj(j);
            acc = acc + (es ? (v * es[e[j]]) * w[j] : w[j] * v);
        }
    }
    if (shared) acc = acc + (sg ? s * sg[t] : s);
    out[(long long)t * n + i] = acc;
}

// inclusive scans of a and b over the 1024 threads (16 waves); wsum: 2 x 16 LDS ints
__device__ __forceinline__ void scan1024(int &a, int &b, int (*wsum)[16]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int ua = __shfl_up(a, d, 64), ub = __shfl_up(b, d, 64);
        if (lane >= d) {
            a += ua;
            b += ub;
        }
    }
    if (lane == 63) {
        wsum[0][w] = a;
        wsum[1][w] = b;
    }
    __syncthreads();
    int ba = 0, bb = 0;
    for (int k = 0; k < w; ++k) {
        ba += wsum[0][k];
        bb += wsum[1][k];
    }
    a += ba;
    b += bb;
}

__global__ void __launch_bounds__(1024) k_moe_group(const int *__restrict__ ids, int T, int n_used, int n_expert,
                                                    int tile, int *__restrict__ tok_rows, int *__restrict__ pair_rows,
                                                    int *__restrict__ n_tiles, int *__restrict__ tile_e,
                                                    int *__restrict__ tile_start, int *__restrict__ tile_n) {
    __shared__ int cnt[MOE_MAX_EXPERTS], slot[MOE_MAX_EXPERTS];
    __shared__ int wsum[2][16];
    const int tid = threadIdx.x, n = T * n_used;
    // (each pass reads GR ids a thread at a time, their loads in flight together: a loop of one load and its wait
    // per entry made the 19416 entries of a 2427-token prompt ~19 memory round trips a pass)
    constexpr int GR = 8;
    cnt[tid] = 0;
    __syncthreads();
    for (int i0 = tid; i0 < n; i0 += GR * 1024) {
        int e[GR];
#pragma unroll
        for (int k = 0; k < GR; ++k) e[k] = i0 + 1024 * k < n ? ids[i0 + 1024 * k] : -1;
#pragma unroll
        for (int k = 0; k < GR; ++k)
            if (e[k] >= 0 && e[k] < n_expert) atomicAdd(&cnt[e[k]], 1);
    }
    __syncthreads();
    const int c = tid < n_expert ? cnt[tid] : 0, nt = (c + tile - 1) / tile;
    int a = c, b = nt;
    scan1024(a, b, wsum);
    const int eo = a - c, to = b - nt;  // exclusive: expert tid's first entry and first tile
    slot[tid] = eo;
    if (tid < n_expert) {
        for (int k = 0; k < nt; ++k) {
            tile_e[to + k] = tid;
            tile_start[to + k] = eo + k * tile;
            tile_n[to + k] = min(tile, c - k * tile);
        }
        if (tid == n_expert - 1) *n_tiles = to + nt;
    }
    __syncthreads();
    for (int i0 = tid; i0 < n; i0 += GR * 1024) {
        int e[GR];
#pragma unroll
        for (int k = 0; k < GR; ++k) e[k] = i0 + 1024 * k < n ? ids[i0 + 1024 * k] : -1;
#pragma unroll
        for (int k = 0; k < GR; ++k) {
            const int i = i0 + 1024 * k;
            if (e[k] < 0 || e[k] >= n_expert) continue;
            const int p = atomicAdd(&slot[e[k]], 1);
            tok_rows[p] = i / n_used;
            pair_rows[p] = i;
        }
    }
}

}  // namespace pq

using namespace pq;

extern "C" {

hipError_t gpu_swiglu(const float *g, const float *u, float *out, int n, const qmatvec_q8 *q8, hipStream_t stream) {
    if (!g || !u || (!out && !q8) || n < 0) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    Q8Ptrs o{};
    if (q8) {
        if (n % 32 != 0 || n > q8->max_k) return hipErrorInvalidValue;
        o = Q8Ptrs{q8->q0, q8->d0, q8->qK, q8->dK, q8->bsK, q8->s0};
    }
    const int nb = (n + 255) / 256;
    auto al = [](const void *p, uintptr_t m) { return ((uintptr_t)p & m) == 0; };
    if (n % 32 == 0 && al(g, 15) && al(u, 15) && al(out, 15) && (!q8 || (al(o.q0, 3) && (!o.qK || al(o.qK, 3))))) {
        // a wave per block; many blocks: two a wave, 256-thread workgroups (four a wave measured 39.3 against 35.4
        // us over config 4's 2427-token prompt, one 38.8)
        if (nb >= 4096)
            hipLaunchKernelGGL(k_swiglu4<2>, dim3((unsigned)((nb + 7) / 8)), dim3(256), 0, stream, (const float4 *)g,
                               (const float4 *)u, (float4 *)out, n, o, q8 ? 1 : 0);
        else
            hipLaunchKernelGGL(k_swiglu4<1>, dim3((unsigned)nb), dim3(64), 0, stream, (const float4 *)g,
                               (const float4 *)u, (float4 *)out, n, o, q8 ? 1 : 0);
        return hipGetLastError();
    }
    const int bpw = nb >= 4096 ? 8 : 1;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((nb + bpw - 1) / bpw)), dim3(256), 0, stream, g, u, out, n, o,
                       q8 ? 1 : 0, bpw);
    return hipGetLastError();
}

hipError_t gpu_add_rmsnorm(const float *x_in, const float *add, float *x_out, const float *w, float *y, int n, int T,
                           float eps, const qmatvec_q8 *q8, hipStream_t stream) {
    if (!x_in || !y || n <= 0 || T < 0 || (add && (!x_out || x_out == x_in))) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    Q8Ptrs o{};
    if (q8) {
        if (n % 256 != 0 || (long long)T * n > q8->max_k) return hipErrorInvalidValue;
        o = Q8Ptrs{q8->q0, q8->d0, q8->qK, q8->dK, q8->bsK, q8->s0};
    }
    // one token (or a few): its row in blocks over the whole GPU; many rows of at most 8192 values: a workgroup each
    if (T >= 8 && n <= 256 * NORM_ROWS_V)
        hipLaunchKernelGGL(k_add_rmsnorm_rows, dim3((unsigned)T), dim3(256), 0, stream, x_in, add, x_out, w, y, n, eps, o,
                           q8 ? 1 : 0);
    else
        hipLaunchKernelGGL(k_add_rmsnorm, dim3((unsigned)((n + 255) / 256), (unsigned)T), dim3(256), 0, stream, x_in,
                           add, x_out, w, y, n, eps, o, q8 ? 1 : 0);
    return hipGetLastError();
}

hipError_t gpu_moe_router(const float *logits, const float *x, const float *w_shexp, int *ids, float *wts, float *sg,
                          int n_expert, int n_used, int n, int T, hipStream_t stream, int ids_stride) {
    if (ids_stride == 0) ids_stride = n_used;
    if (!logits || !ids || !wts || n_expert < 1 || n_expert > MOE_MAX_EXPERTS || n_used < 1 ||
        n_used > MOE_MAX_USED || n_used > n_expert || T < 0 || ids_stride < n_used || (w_shexp && (!x || !sg || n <= 0)))
        return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    hipLaunchKernelGGL(k_moe_router, dim3((unsigned)T), dim3(256), 0, stream, logits, x, w_shexp, ids, wts, sg, n_expert,
                       n_used, n, ids_stride);
    return hipGetLastError();
}

hipError_t gpu_moe_combine_scaled(const float *down, const float *wts, const float *shared, const float *sg,
                                  const int *ids, const float *exp_scale, float *out, int n_used, int n, int T,
                                  hipStream_t stream) {
    if (!down || !out || n_used < 1 || n < 0 || T < 0 || (exp_scale && (!ids || !wts))) return hipErrorInvalidValue;
    if (n == 0 || T == 0) return hipSuccess;
    // a few tokens: 64-thread workgroups, so one token's outputs spread over 32 CUs instead of 8 (config 4's decode
    // token: 19.8 -> 18.8 us; 128 threads measured as 256)
    const int thr = T <= 4 ? 64 : 256;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n + thr - 1) / thr), (unsigned)T), dim3(thr), 0, stream, down,
                       wts, shared, sg, ids, exp_scale, out, n_used, n);
    return hipGetLastError();
}

hipError_t gpu_moe_combine(const float *down, const float *wts, const float *shared, const float *sg, float *out,
                           int n_used, int n, int T, hipStream_t stream) {
    return gpu_moe_combine_scaled(down, wts, shared, sg, nullptr, nullptr, out, n_used, n, T, stream);
}

hipError_t gpu_moe_group(const int *ids, int T, int n_used, int n_expert, int tile, int *tok_rows, int *pair_rows,
                         int *n_tiles, int *tile_e, int *tile_start, int *tile_n, hipStream_t stream) {
    if (!ids || !tok_rows || !pair_rows || !n_tiles || !tile_e || !tile_start || !tile_n || T < 0 || n_used < 1 ||
        n_expert < 1 || n_expert > MOE_MAX_EXPERTS || tile < 1)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), 0, stream, ids, T, n_used, n_expert, tile, tok_rows, pair_rows,
                       n_tiles, tile_e, tile_start, tile_n);
    return hipGetLastError();
}

}  // extern "C"
