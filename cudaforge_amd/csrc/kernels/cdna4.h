// cdna4.h — small device helpers shared by the gfx950 kernels: vector types, direct
// global->LDS loads with explicit completion waits, and the LDS transposing read.
#ifndef CF_CDNA4_H_
#define CF_CDNA4_H_

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace cdna4 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 lds_h4_t;
#define CF_LDS __attribute__((address_space(3)))
// Global memory, for pointers the compiler cannot trace back to a kernel argument (it
// would otherwise emit flat loads, which also count against lgkmcnt).
#define CF_GLOBAL __attribute__((address_space(1)))

// Quotient of 0 <= n < 2^31 by a divisor d >= 1 fixed at launch, without the ~25
// instructions of a runtime division: q = (n * mul) >> shift in 64 bits, with
// shift = 31 + ceil(log2 d) and mul = ceil(2^shift / d) < 2^32, computed once on the host.
// Exact: mul * d = 2^shift + e with 0 <= e < d, so n * mul / 2^shift = n / d + n e / (d 2^shift),
// and n e < n d < 2^31 * 2^ceil(log2 d) = 2^shift keeps the second term below 1/d.
// Wave-uniform operands compile to scalar multiplies.
struct FastDiv {
    uint32_t mul;
    uint32_t shift;
};
__host__ inline FastDiv fastdiv_make(int d) {
    uint32_t l = 0;
    while ((1u << l) < (uint32_t)d) l++;
    const uint32_t shift = 31 + l;
    return FastDiv{(uint32_t)(((1ull << shift) + (uint64_t)d - 1) / (uint64_t)d), shift};
}
__host__ __device__ __forceinline__ int fastdiv(int n, FastDiv f) {
    return (int)(((uint64_t)(uint32_t)n * f.mul) >> f.shift);
}

// s_waitcnt vmcnt(N), expcnt/lgkmcnt left at their maxima (gfx9 encoding).  The empty
// asm after it keeps the compiler from hoisting LDS reads above the wait.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    asm volatile("" ::: "memory");
}

// Wait until at most `ahead` (clamped to 0..N_AHEAD) ring stages of NL loads each are
// still in flight.
template <int NL, int N_AHEAD>
__device__ __forceinline__ void wait_ahead(int ahead) {
    if (ahead >= N_AHEAD) wait_vm<N_AHEAD * NL>();
    else if constexpr (N_AHEAD > 0) wait_ahead<NL, N_AHEAD - 1>(ahead);
}

// Ring loops with the stage index as a compile-time constant: calls
// step(i, std::integral_constant<int, i % NS>{}) for i = 0 .. n-1, unrolled NS times, so
// that LDS addresses inside a stage become a per-lane register plus an immediate offset.
template <typename F, int... S>
__device__ __forceinline__ void stage_group(int i0, int n, F& step, std::integer_sequence<int, S...>) {
    ((i0 + S < n ? step(i0 + S, std::integral_constant<int, S>{}) : void()), ...);
}

template <int NS, typename F>
__device__ __forceinline__ void for_each_stage(int n, F&& step) {
    for (int i0 = 0; i0 < n; i0 += NS) stage_group(i0, n, step, std::make_integer_sequence<int, NS>{});
}

// s_waitcnt lgkmcnt(0): every LDS read issued so far has returned its data, so a DMA
// may refill the stage it read.
__device__ __forceinline__ void wait_lds_reads() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
    asm volatile("" ::: "memory");
}

// 16 bytes per lane from global memory into LDS at lds_base + 16*lane (M0 = lds_base).
// Issued as inline asm so the compiler does not treat the LDS ring as pending DMA
// writes (it would then wait for every load before each LDS read); completion is
// tracked with explicit vmcnt waits instead.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "s"(lds_base) : "memory", "m0");
}
// Same, addressing global memory as a uniform 64-bit base (SGPR pair) plus a per-lane
// 32-bit byte offset: no per-lane 64-bit address arithmetic.
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void* sbase, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Reductions across lane i and lane i^16 / i^32 with the gfx950 row-swap permutes (VALU,
// no LDS round trip).  v_permlane16_swap a, b swaps the odd 16-lane rows of a with the
// even rows of b (v_permlane32_swap: the upper half of a with the lower half of b), so
// with a = b = x every lane ends with {own value, partner value} in a and b; max and +
// are commutative, so both partners get the same bits.  Issued as inline asm (with the
// two wait states a VALU write needs before the permute reads it): the compiler's own
// folding of these builtins treats the two results of swap(x, x) as equal, which they
// are not across lanes.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void swap_xor16(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_xor32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
#pragma clang diagnostic pop
__device__ __forceinline__ float max_xor16(float x) { float a = x, b = x; swap_xor16(a, b); return fmaxf(a, b); }
__device__ __forceinline__ float max_xor32(float x) { float a = x, b = x; swap_xor32(a, b); return fmaxf(a, b); }
__device__ __forceinline__ float add_xor16(float x) { float a = x, b = x; swap_xor16(a, b); return a + b; }
__device__ __forceinline__ float add_xor32(float x) { float a = x, b = x; swap_xor32(a, b); return a + b; }

// DPP moves inside 16-lane rows (gfx9 dpp_ctrl encodings), VALU operands with no LDS
// round trip (a ds_bpermute or ds_swizzle exchange waits on the LDS pipe): quad_perm
// [1,0,3,2] reads lane ^ 1, quad_perm [2,3,0,1] lane ^ 2, row_half_mirror lane ^ 7 within
// 8 lanes, row_mirror lane ^ 15 within 16, row_shr:n lane - n within the row (bound_ctrl:
// 0 where that leaves the row), row_ror:n lane - n mod 16 within the row.
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140, kDppShr = 0x110,
             kDppRor = 0x120 };
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) { return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, true); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) { return __int_as_float(dpp_i<CTRL>(__float_as_int(x))); }

// The wave's maximum and sum in every lane.  After the two quad steps every lane of a
// quad holds the quad's value, so the half-row mirror pairs quads and the row mirror
// pairs 8-lane halves; the row swaps finish across rows.  Each step combines two equal
// pairs of operands (a + b on one lane, b + a on its partner), so all lanes get the
// same bits.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_f<kDppXor1>(x));
    x = fmaxf(x, dpp_f<kDppXor2>(x));
    x = fmaxf(x, dpp_f<kDppHalfMirror>(x));
    x = fmaxf(x, dpp_f<kDppMirror>(x));
    return max_xor32(max_xor16(x));
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_f<kDppXor1>(x);
    x += dpp_f<kDppXor2>(x);
    x += dpp_f<kDppHalfMirror>(x);
    x += dpp_f<kDppMirror>(x);
    return add_xor32(add_xor16(x));
}

// Sum over each 16-lane row, in every lane of it (the first four steps of wave_sum).
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp_f<kDppXor1>(x);
    x += dpp_f<kDppXor2>(x);
    x += dpp_f<kDppHalfMirror>(x);
    return x + dpp_f<kDppMirror>(x);
}

// Sum over the lanes with the same lane % S (S = 1, 2, 4, 8, 16 or 32): rotations inside
// each 16-lane row by S, 2S, .. 8, then the row swaps.  Lanes of one class can end with
// different roundings (each adds its own pairs first); callers read one lane per class.
template <int S>
__device__ __forceinline__ float sum_stride(float x) {
    static_assert(S == 1 || S == 2 || S == 4 || S == 8 || S == 16 || S == 32, "stride");
    if constexpr (S == 1) return wave_sum(x);
    if constexpr (S <= 2) x += dpp_f<kDppRor + 2>(x);
    if constexpr (S <= 4) x += dpp_f<kDppRor + 4>(x);
    if constexpr (S <= 8) x += dpp_f<kDppRor + 8>(x);
    if constexpr (S <= 16) x = add_xor16(x);
    return add_xor32(x);
}

// Exclusive prefix sum of v over lanes 0 .. lane - 1: an inclusive scan inside each
// 16-lane row (row_shr 1, 2, 4, 8), then every row adds the totals of the rows before it
// (read from lanes 15, 31, 47).
__device__ __forceinline__ int wave_excl_sum(int v, int lane) {
    int x = v;
    x += dpp_i<kDppShr + 1>(x);
    x += dpp_i<kDppShr + 2>(x);
    x += dpp_i<kDppShr + 4>(x);
    x += dpp_i<kDppShr + 8>(x);
    const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
    const int r2 = __builtin_amdgcn_readlane(x, 47);
    const int row = lane >> 4;
    x += (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
    return x - v;
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const CF_LDS void*)p;
}

// Workgroup barrier without the vmcnt(0) wait __syncthreads implies (a ring keeps DMA
// loads in flight across it); the empty asm statements stop the compiler from moving
// LDS accesses across the barrier.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ds_read_b64_tr_b16: in each 16-lane group, lane i receives element i%4 of the 4-half
// chunks addressed by lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4.  With lane j addressing
// X[kb + j/4][nb + 4(j%4)] of a row-major fp16 tile, lane i gets X[kb..kb+3][nb + i].
__device__ __forceinline__ h4_t ds_read_tr4(const _Float16* p) {
    return __builtin_bit_cast(h4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((CF_LDS lds_h4_t*)p));
}

__device__ __forceinline__ h8_t cat8(h4_t lo, h4_t hi) {
    return h8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Compute units of the current device (cached per device; 256 on MI355X).
inline int cu_count() {
    static int dev_cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (dev_cus[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        dev_cus[dev] = n;
    }
    return dev_cus[dev];
}

}  // namespace cdna4

#endif  // CF_CDNA4_H_
