// layer_ops.hip — the operators next to attention in an FP16 transformer layer that
// keep it on the device: LayerNorm (layernorm.c:85-122, norm_f16_cuda.cu:47-108), the
// Cast conversions (cast_cuda.cu:6-64) and the transpose the MatMul op needs for its
// transposed operands (matmul_cuda.cu:320-352).  All HBM-bound, so: one wave per
// LayerNorm row with 8-byte vector accesses and the row kept in registers, grid-stride
// elementwise loops, and an LDS-tiled transpose.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "cdna4.h"

namespace {

using cdna4::wave_sum;   // DPP and row swaps: no LDS round trip per reduction step

template <typename T> struct Vec4;
template <> struct Vec4<float> { typedef float type __attribute__((ext_vector_type(4))); };
template <> struct Vec4<_Float16> { typedef _Float16 type __attribute__((ext_vector_type(4))); };

// LayerNorm, one wave per row; each lane holds VPL groups of 4 consecutive elements
// (lane l, group j: elements 4*(64*j + l) .. +3), D == 256*VPL... or fewer groups when
// the row is shorter (masked).  Requires D % 4 == 0 and 8/16-byte aligned rows.
template <typename T, int VPL>
__global__ __launch_bounds__(256) void layernorm_vec(cf_layernorm_args_t a) {
    typedef typename Vec4<T>::type V;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.N) return;
    const int D = a.D, ng = D >> 2;
    const V* x = (const V*)((const T*)a.x + row * D);
    float v[VPL][4];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const int gi = 64 * j + lane;
        if (gi < ng) {
            const V q = x[gi];
#pragma unroll
            for (int e = 0; e < 4; e++) { v[j][e] = (float)q[e]; s += v[j][e]; }
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) v[j][e] = 0.0f;
        }
    }
    const float mean = wave_sum(s) / (float)D;
    float q2 = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++)
        if (64 * j + lane < ng) {
#pragma unroll
            for (int e = 0; e < 4; e++) { const float dv = v[j][e] - mean; q2 += dv * dv; }
        }
    const float inv_std = 1.0f / sqrtf(wave_sum(q2) / (float)D + a.eps);
    const V* g = (const V*)a.gamma;
    const V* b = (const V*)a.beta;
    V* y = (V*)((T*)a.y + row * D);
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const int gi = 64 * j + lane;
        if (gi < ng) {
            const V gv = g[gi], bv = b[gi];
            V o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = (T)((v[j][e] - mean) * inv_std * (float)gv[e] + (float)bv[e]);
            y[gi] = o;
        }
    }
}

// Any D: one wave per row, three passes over the row (it stays in L1/L2).
template <typename T>
__global__ __launch_bounds__(256) void layernorm_any(cf_layernorm_args_t a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.N) return;
    const int D = a.D;
    const T* x = (const T*)a.x + row * D;
    float s = 0.0f;
    for (int i = lane; i < D; i += 64) s += (float)x[i];
    const float mean = wave_sum(s) / (float)D;
    float q2 = 0.0f;
    for (int i = lane; i < D; i += 64) { const float dv = (float)x[i] - mean; q2 += dv * dv; }
    const float inv_std = 1.0f / sqrtf(wave_sum(q2) / (float)D + a.eps);
    const T* g = (const T*)a.gamma;
    const T* b = (const T*)a.beta;
    T* y = (T*)a.y + row * D;
    for (int i = lane; i < D; i += 64) y[i] = (T)(((float)x[i] - mean) * inv_std * (float)g[i] + (float)b[i]);
}

template <typename T>
hipError_t launch_layernorm(const cf_layernorm_args_t& a, hipStream_t s) {
    const unsigned blocks = (unsigned)((a.N + 3) / 4);
    const uintptr_t al = (uintptr_t)a.x | (uintptr_t)a.y | (uintptr_t)a.gamma | (uintptr_t)a.beta;
    const bool vec = a.D % 4 == 0 && al % (4 * sizeof(T)) == 0;
    const int groups = (a.D / 4 + 63) / 64;
    if (vec && groups <= 1) hipLaunchKernelGGL((layernorm_vec<T, 1>), dim3(blocks), dim3(256), 0, s, a);
    else if (vec && groups <= 2) hipLaunchKernelGGL((layernorm_vec<T, 2>), dim3(blocks), dim3(256), 0, s, a);
    else if (vec && groups <= 4) hipLaunchKernelGGL((layernorm_vec<T, 4>), dim3(blocks), dim3(256), 0, s, a);
    else if (vec && groups <= 8) hipLaunchKernelGGL((layernorm_vec<T, 8>), dim3(blocks), dim3(256), 0, s, a);
    else if (vec && groups <= 16) hipLaunchKernelGGL((layernorm_vec<T, 16>), dim3(blocks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((layernorm_any<T>), dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

// Cast: grid-stride elementwise.
template <typename I, typename O>
__global__ __launch_bounds__(256) void cast_kernel(const I* __restrict__ in, O* __restrict__ out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = (O)in[i];
}

// Transpose through a 64 x 65 LDS tile (the pad keeps column reads conflict-free).
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                        int64_t rows, int64_t cols, int64_t in_stride,
                                                        int64_t out_stride) {
    __shared__ T tile[64][65];
    const int64_t b = blockIdx.z;
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const T* src = in + b * in_stride;
    T* dst = out + b * out_stride;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4)
        if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = src[(r0 + r) * cols + c0 + tx];
    __syncthreads();
    for (int c = ty; c < 64; c += 4)
        if (c0 + c < cols && r0 + tx < rows) dst[(c0 + c) * rows + r0 + tx] = tile[tx][c];
}

unsigned grid_1d(int64_t n) {
    const int64_t blocks = (n + 255) / 256;
    return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace

extern "C" int cf_launch_layernorm(const cf_layernorm_args_t* a, void* stream) {
    if (!a || !a->x || !a->gamma || !a->beta || !a->y || a->N < 0 || a->D <= 0) return (int)hipErrorInvalidValue;
    if (a->N == 0) return 0;
    if ((a->N + 3) / 4 > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    return (int)(a->elem == CF_ELEM_F16 ? launch_layernorm<_Float16>(*a, s) : launch_layernorm<float>(*a, s));
}

extern "C" int cf_launch_cast(const void* in, void* out, int64_t n, int32_t kind, void* stream) {
    if (!in || !out || n < 0) return (int)hipErrorInvalidValue;
    if (n == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    const dim3 g(grid_1d(n)), b(256);
    switch (kind) {
        case CF_CAST_I64_F32: hipLaunchKernelGGL((cast_kernel<int64_t, float>), g, b, 0, s, (const int64_t*)in, (float*)out, n); break;
        case CF_CAST_F32_I64: hipLaunchKernelGGL((cast_kernel<float, int64_t>), g, b, 0, s, (const float*)in, (int64_t*)out, n); break;
        case CF_CAST_F32_F16: hipLaunchKernelGGL((cast_kernel<float, _Float16>), g, b, 0, s, (const float*)in, (_Float16*)out, n); break;
        case CF_CAST_F16_F32: hipLaunchKernelGGL((cast_kernel<_Float16, float>), g, b, 0, s, (const _Float16*)in, (float*)out, n); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

extern "C" int cf_launch_transpose(const void* in, void* out, int64_t rows, int64_t cols, int64_t batch,
                                   int64_t in_stride, int64_t out_stride, int32_t elem_bytes, void* stream) {
    if (!in || !out || rows < 0 || cols < 0 || batch < 1 || (elem_bytes != 2 && elem_bytes != 4))
        return (int)hipErrorInvalidValue;
    if (rows == 0 || cols == 0) return 0;
    const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
    if (gx > 0x7fffffffLL || gy > 65535 || batch > 65535) return (int)hipErrorInvalidValue;
    const dim3 g((unsigned)gx, (unsigned)gy, (unsigned)batch), b(256);
    hipStream_t s = (hipStream_t)stream;
    if (elem_bytes == 2)
        hipLaunchKernelGGL(transpose_kernel<uint16_t>, g, b, 0, s, (const uint16_t*)in, (uint16_t*)out, rows, cols,
                           in_stride, out_stride);
    else
        hipLaunchKernelGGL(transpose_kernel<uint32_t>, g, b, 0, s, (const uint32_t*)in, (uint32_t*)out, rows, cols, in_stride,
                           out_stride);
    return (int)hipGetLastError();
}
