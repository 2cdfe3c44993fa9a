// Device probe of the sampler's division (div_rn in elem.h) against IEEE float division, for the numerics tests.
// Test infrastructure: built next to this file by __graft_entry__.build(), loaded only by tests/.
#include <hip/hip_runtime.h>

#include "elem.h"

namespace {

__global__ void probe_kernel(const float* x, const float* d, int64_t n, float* out_rn, float* out_ieee) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float xv = x[i], dv = d[i];
    out_rn[i] = mis::div_rn(xv, dv, 1.0 / (double)dv);
    out_ieee[i] = xv / dv;
}

}  // namespace

extern "C" int divprobe_run(const float* x, const float* d, int64_t n, float* out_rn, float* out_ieee, void* stream) {
    if (n <= 0) return 0;
    const int threads = 256;
    const int64_t grid = (n + threads - 1) / threads;
    hipLaunchKernelGGL(probe_kernel, dim3((unsigned)grid), dim3(threads), 0, (hipStream_t)stream, x, d, n, out_rn,
                       out_ieee);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
