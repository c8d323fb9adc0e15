// rope.hip — rotary position encoding (the reference's RoPE op, rope.c:17-66 and
// rope_cuda.cu:9-59) and its decode form, which rotates the new token's Q and K in place
// between the projection and the attention of MHA_Decode.
//
// One thread per rotated pair.  The angles come from a host-computed (cos, sin) table
// (the reference formula with glibc powf/cosf/sinf) rather than device math: angle =
// pos / base^(2i/d) reaches thousands of radians, where one ulp of a different powf moves
// cos and sin by ~1e-4, beyond the FP32 parity bound.  The rotation itself is fp32 with
// contraction off (x0*c - x1*s rounded per operation, as the CPU computes it).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float ld(const float* p) { return *p; }
__device__ __forceinline__ float ld(const _Float16* p) { return (float)*p; }
__device__ __forceinline__ void st(float* p, float v) { *p = v; }
__device__ __forceinline__ void st(_Float16* p, float v) { *p = (_Float16)v; }

template <typename T>
__device__ __forceinline__ void rotate(const T* in, T* out, float2 cs) {
#pragma clang fp contract(off)
    const float x0 = ld(in), x1 = ld(in + 1);
    const float a = x0 * cs.x, b = x1 * cs.y;
    const float c = x0 * cs.y, e = x1 * cs.x;
    st(out, a - b);
    st(out + 1, c + e);
}

// (rows, H, d): pair index -> (row = position, head, i).  I is the index type: 32-bit
// when the pair count fits (integer division is far cheaper), else 64-bit.
template <typename T, typename I>
__global__ __launch_bounds__(kThreads) void rope_rows(cf_rope_args_t a) {
    const I half = (I)(a.d >> 1), H = (I)a.H;
    const I total = (I)a.rows * H * half;
    for (I idx = (I)blockIdx.x * kThreads + threadIdx.x; idx < total; idx += (I)gridDim.x * kThreads) {
        const I i = idx % half;
        const I rh = idx / half;                    // row * H + h
        const I pos = rh / H;
        const size_t off = (size_t)rh * a.d + 2 * i;
        rotate((const T*)a.in + off, (T*)a.out + off, ((const float2*)a.table)[(size_t)pos * half + i]);
    }
}

// Decode: pair index -> (b, head among H_q + H_kv, i); Q heads first, then K heads.
template <typename T>
__global__ __launch_bounds__(kThreads) void rope_decode(cf_rope_decode_args_t a) {
    const int half = a.d >> 1, heads = a.H_q + a.H_kv;
    const int total = a.B * heads * half;           // < 2^31: checked by the launcher
    for (int idx = blockIdx.x * kThreads + threadIdx.x; idx < total; idx += gridDim.x * kThreads) {
        const int i = idx % half;
        const int bh = idx / half;
        const int h = bh % heads, b = bh / heads;
        const int64_t pos = a.lens ? (int64_t)a.lens[b] : a.pos_uniform;
        if (pos < 0 || pos >= a.max_seq) continue;
        T* p = h < a.H_q ? (T*)a.q + ((size_t)b * a.H_q + h) * a.d
                         : (T*)a.k_cache + (((size_t)b * a.max_seq + pos) * a.H_kv + (h - a.H_q)) * a.d;
        rotate(p + 2 * i, p + 2 * i, ((const float2*)a.table)[pos * half + i]);
    }
}

unsigned grid_for(int64_t total) {
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace

extern "C" int cf_launch_rope(const cf_rope_args_t* a, void* stream) {
    if (!a || !a->in || !a->out || !a->table || a->rows < 0 || a->H <= 0 || a->d <= 0 || (a->d & 1))
        return (int)hipErrorInvalidValue;
    const int64_t total = a->rows * a->H * (a->d / 2);
    if (total == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    const dim3 g(grid_for(total)), b(kThreads);
    const bool narrow = total < (1LL << 31) - 65536LL * kThreads;
    if (a->elem == CF_ELEM_F16) {
        if (narrow) hipLaunchKernelGGL((rope_rows<_Float16, int32_t>), g, b, 0, s, *a);
        else hipLaunchKernelGGL((rope_rows<_Float16, int64_t>), g, b, 0, s, *a);
    } else {
        if (narrow) hipLaunchKernelGGL((rope_rows<float, int32_t>), g, b, 0, s, *a);
        else hipLaunchKernelGGL((rope_rows<float, int64_t>), g, b, 0, s, *a);
    }
    return (int)hipGetLastError();
}

extern "C" int cf_launch_rope_decode(const cf_rope_decode_args_t* a, void* stream) {
    if (!a || !a->q || !a->k_cache || !a->table || a->B <= 0 || a->H_q <= 0 || a->H_kv <= 0 || a->d <= 0 ||
        (a->d & 1) || a->max_seq <= 0)
        return (int)hipErrorInvalidValue;
    const int64_t total = (int64_t)a->B * (a->H_q + a->H_kv) * (a->d / 2);
    if (total >= (1LL << 31) - 65536LL * kThreads) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(rope_decode<_Float16>, dim3(grid_for(total)), dim3(kThreads), 0, s, *a);
    else
        hipLaunchKernelGGL(rope_decode<float>, dim3(grid_for(total)), dim3(kThreads), 0, s, *a);
    return (int)hipGetLastError();
}
