// q8act.hip -- the standalone activation quantizer for the int8 path (wave64), the reference's quantize_q8
// (src/matvec_q.hip:1281-1286): one 256-thread workgroup per 256-value block (q8dev.h).
#include "q8dev.h"

namespace pq {

__global__ void __launch_bounds__(256) k_quantize_q8(const float *__restrict__ x, int n, Q8Ptrs o) {
    __shared__ Q8Shared sh;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const bool active = i < n;
    q8_quantize_value(active ? x[i] : 0.0f, active, blockIdx.x, sh, o);
}

hipError_t launch_quantize_q8(const float *x, int n, const Q8Ptrs &o, hipStream_t stream) {
    hipLaunchKernelGGL(k_quantize_q8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, n, o);
    return hipGetLastError();
}

}  // namespace pq
