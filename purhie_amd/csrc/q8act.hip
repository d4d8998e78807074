// q8act.hip -- activation quantizer for the int8 path (wave64), the equivalent of the reference's
// quantize_q8 / q8_block_value (src/matvec_q.hip:1281-1286, src/q8_device.h:54-104).
//
// One 256-thread workgroup (4 waves) per 256-value block, one value per thread, into both of ggml's
// activation formats, bit-identical to the reference:
//   Q8_0: per 32 values am = max|x|, q = rint(x * (127 / am)) (ties to even), d = fp16(am / 127),
//         s0 = fp16((am / 127) * sum q) kept as float bits (the Q8_1 block sum);
//   Q8_K: per 256 values v = the signed value of largest |x| (lowest index on ties), iscale = -127 / v,
//         q = min(127, rint(iscale * x)), d = 1 / iscale (0 for an all-zero block), sums of every 16 q.
// A 32-value Q8_0 block is half a wave: the xor reductions use offsets 16..1, which stay inside it.
#include "device.h"
#include "kernels.h"

namespace pq {

__global__ void __launch_bounds__(256) k_quantize_q8(const float *__restrict__ x, int n, Q8Ptrs o) {
    __shared__ float s_a[4];
    __shared__ float s_v[4];
    __shared__ int s_i[4];
    const int t = threadIdx.x, b = blockIdx.x, i = b * 256 + t;
    const int lane = t & 63, w = t >> 6;
    const bool active = i < n;
    const float v = active ? x[i] : 0.0f;
    const float a = fabsf(v);

    // Q8_0 over the 32 values of this half-wave
    float am = a;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 64));
    const float id0 = am != 0.0f ? 127.0f / am : 0.0f;
    const int q0 = active ? (int)rintf(v * id0) : 0;
    int s0 = q0;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) s0 += __shfl_xor(s0, off, 64);
    if (active) {
        o.q0[i] = (int8_t)q0;
        if ((lane & 31) == 0) {
            const float d = am / 127.0f;
            o.d0[i >> 5] = __half2float(__float2half(d));
            if (o.s0) o.s0[i >> 5] = __float_as_int(__half2float(__float2half(d * (float)s0)));
        }
    }
    if (!o.qK) return;  // (uniform)

    // Q8_K over the 256 values: largest |x|, the lowest index on ties
    float ba = a, bv = v;
    int bi = t;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(ba, off, 64), ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (oa > ba || (oa == ba && oi < bi)) {
            ba = oa;
            bi = oi;
            bv = ov;
        }
    }
    if (lane == 0) {
        s_a[w] = ba;
        s_v[w] = bv;
        s_i[w] = bi;
    }
    __syncthreads();
    float fa = s_a[0], fv = s_v[0];
    int fi = s_i[0];
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (s_a[k] > fa || (s_a[k] == fa && s_i[k] < fi)) {
            fa = s_a[k];
            fi = s_i[k];
            fv = s_v[k];
        }
    int q = 0;
    float iscale = 0.0f;
    if (fa != 0.0f) {
        iscale = -127.0f / fv;
        q = min(127, (int)rintf(iscale * v));
    }
    int s16 = q;
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) s16 += __shfl_xor(s16, off, 64);
    if (active) {
        o.qK[i] = (int8_t)q;
        if (t == 0) o.dK[b] = fa != 0.0f ? 1.0f / iscale : 0.0f;
        if ((lane & 15) == 0) o.bsK[i >> 4] = s16;
    }
}

hipError_t launch_quantize_q8(const float *x, int n, const Q8Ptrs &o, hipStream_t stream) {
    hipLaunchKernelGGL(k_quantize_q8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, n, o);
    return hipGetLastError();
}

}  // namespace pq
