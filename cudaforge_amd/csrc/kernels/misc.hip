// misc.hip — small device kernels of the operator layer.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

// CausalMask: mask[i][j] = 0 for j <= i, -inf above the diagonal
// (src/operator/nn/causal_mask.c:17-21).
__global__ void causal_mask_kernel(float* __restrict__ mask, int64_t S) {
    const int64_t n = S * S;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / S, j = idx - i * S;
        mask[idx] = j <= i ? 0.0f : -INFINITY;
    }
}

// v[i] = value (set) or v[i] += value: the device-held decode lengths a graph advances
// once per step (a kernel, not a memset, so recordings replay it reliably).
__global__ void i32_update_kernel(int32_t* __restrict__ v, int32_t n, int32_t value, int32_t add) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) v[i] = add ? v[i] + value : value;
}

}  // namespace

extern "C" int cf_launch_i32_update(int32_t* v, int32_t n, int32_t value, int32_t add, void* stream) {
    if (!v || n <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(i32_update_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, v, n,
                       value, add);
    return (int)hipGetLastError();
}

extern "C" int cf_launch_causal_mask(float* mask, int64_t S, void* stream) {
    if (!mask || S <= 0) return (int)hipErrorInvalidValue;
    const int64_t n = S * S;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(causal_mask_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, mask, S);
    return (int)hipGetLastError();
}
