// misc.hip — small device kernels of the operator layer.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "cdna4.h"

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

// Byte copy by the compute units, 16 bytes per lane where both ends allow: for small
// transfers between pinned host memory (mapped, device-accessible) and device memory
// that sit between kernels on one stream, where a DMA-engine copy would add the
// engines' hand-over latency on both sides.
__global__ void copy_bytes_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, size_t n, int vec) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const size_t n16 = n / 16;
        for (size_t k = i; k < n16; k += stride) ((uint4*)dst)[k] = ((const uint4*)src)[k];
        for (size_t k = n16 * 16 + i; k < n; k += stride) dst[k] = src[k];
    } else {
        for (size_t k = i; k < n; k += stride) dst[k] = src[k];
    }
}

// Synthetic benchmark inputs: N(mean, stddev) by splitmix64 and Box-Muller, the
// generator the CPU baseline's inputs come from, evaluated by counter so that every pair
// is independent.  The sequence seeded with s has state s + k * 0x9E3779B97F4A7C15 after
// k steps; pair i takes outputs 2i+1 and 2i+2 as uniforms u1, u2 in (0, 1] (top 53 bits
// plus one, times 2^-53), and elements 2i, 2i+1 are mean + stddev * r * (cos, sin)(2 pi u2)
// with r = sqrt(-2 ln u1), in double, rounded to float and then (fp16) to half, both by
// round-to-nearest-even.
__device__ __forceinline__ double splitmix_unit(uint64_t seed, uint64_t k) {
    uint64_t z = seed + k * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return ((double)(z >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

template <typename T>
__global__ void fill_normal_kernel(T* __restrict__ out, size_t n, uint64_t seed, float mean, float stddev) {
    const size_t pairs = (n + 1) / 2;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs; i += (size_t)gridDim.x * blockDim.x) {
        const double u1 = splitmix_unit(seed, 2 * i + 1), u2 = splitmix_unit(seed, 2 * i + 2);
        const double r = sqrt(-2.0 * log(u1)), a = 6.283185307179586 * u2;
        out[2 * i] = (T)(float)(mean + stddev * r * cos(a));
        if (2 * i + 1 < n) out[2 * i + 1] = (T)(float)(mean + stddev * r * sin(a));
    }
}

}  // namespace

extern "C" int cf_launch_fill_normal(void* out, size_t n, int elem, uint64_t seed, float mean, float stddev,
                                     void* stream) {
    if (n == 0) return 0;
    if (!out || (elem != CF_ELEM_F16 && elem != CF_ELEM_F32)) return (int)hipErrorInvalidValue;
    size_t blocks = ((n + 1) / 2 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (elem == CF_ELEM_F16)
        hipLaunchKernelGGL(fill_normal_kernel<_Float16>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (_Float16*)out, n, seed, mean, stddev);
    else
        hipLaunchKernelGGL(fill_normal_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (float*)out, n, seed, mean, stddev);
    return (int)hipGetLastError();
}

// The kernels' launch-time divisor (cdna4::FastDiv), run on the host for checking:
// n / d through the same multiplier and shift the kernels use.
extern "C" int32_t cf_fastdiv_quotient(int32_t n, int32_t d) {
    return cdna4::fastdiv(n, cdna4::fastdiv_make(d));
}

extern "C" int cf_launch_copy_bytes(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    if (!dst || !src) return (int)hipErrorInvalidValue;
    const int vec = (((uintptr_t)dst | (uintptr_t)src) % 16) == 0;
    size_t blocks = (bytes / (vec ? 16 : 1) + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (uint8_t*)dst,
                       (const uint8_t*)src, bytes, vec);
    return (int)hipGetLastError();
}

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
