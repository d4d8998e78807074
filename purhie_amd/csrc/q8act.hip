// q8act.hip -- the standalone activation quantizer for the int8 path (wave64), the reference's quantize_q8
// (src/matvec_q.hip:1281-1286). k_quantize_q8_4: a wave per 256-value block, four values a lane (one 16-byte load),
// quantized within the wave (q8dev.h q8_quantize4), four blocks a wave for long inputs with their loads issued
// first; k_quantize_q8, a 256-thread workgroup per block, takes x that is not 16-byte aligned. The same bits.
#include "q8dev.h"

namespace pq {

__global__ void __launch_bounds__(256) k_quantize_q8(const float *__restrict__ x, int n, Q8Ptrs o) {
    __shared__ Q8Shared sh;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const bool active = i < n;
    q8_quantize_value(active ? x[i] : 0.0f, active, blockIdx.x, sh, o);
}

template <int BW>
__global__ void __launch_bounds__(256) k_quantize_q8_4(const float4 *__restrict__ x, int n, Q8Ptrs o) {
    const int lane = threadIdx.x & 63;
    const int b0 = ((blockIdx.x * blockDim.x + threadIdx.x) >> 6) * BW, nb = (n + 255) / 256;
    float4 xa[BW];
#pragma unroll
    for (int k = 0; k < BW; ++k) {
        const long long i4 = (long long)(b0 + k) * 64 + lane;
        xa[k] = b0 + k < nb && 4 * i4 < n ? x[i4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < BW; ++k) {
        const int b = b0 + k;
        if (b >= nb) break;  // (uniform)
        const long long i4 = (long long)b * 64 + lane;
        const float v[4] = {xa[k].x, xa[k].y, xa[k].z, xa[k].w};
        q8_quantize4(v, 4 * i4 < n, b, 4 * i4, lane, o);  // (n % 32 == 0: a lane's four values together)
    }
}

hipError_t launch_quantize_q8(const float *x, int n, const Q8Ptrs &o, hipStream_t stream) {
    const int nb = (n + 255) / 256;
    auto al = [](const void *p, uintptr_t m) { return ((uintptr_t)p & m) == 0; };
    if (n % 32 == 0 && al(x, 15) && al(o.q0, 3) && (!o.qK || al(o.qK, 3))) {
        if (nb >= 4096)
            hipLaunchKernelGGL(k_quantize_q8_4<4>, dim3((unsigned)((nb + 15) / 16)), dim3(256), 0, stream,
                               (const float4 *)x, n, o);
        else
            hipLaunchKernelGGL(k_quantize_q8_4<1>, dim3((unsigned)nb), dim3(64), 0, stream, (const float4 *)x, n, o);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_quantize_q8, dim3((unsigned)nb), dim3(256), 0, stream, x, n, o);
    return hipGetLastError();
}

}  // namespace pq
