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

}  // namespace

extern "C" int cf_launch_causal_mask(float* mask, int64_t S, void* stream) {
    if (!mask || S <= 0) return (int)hipErrorInvalidValue;
    const int64_t n = S * S;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(causal_mask_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, mask, S);
    return (int)hipGetLastError();
}
