// gemm.hip — prefill projections of MHA_Fused on the matrix cores (gfx950).
//
// C = A·W + bias (+ residual) with A (M, K) row-major and W (K, N) row-major, the
// layout of the reference's "x·W" projections (mha_fused.c:68-88 and :152-171).
// The epilogue either writes C row-major or scatters the Q | K | V column segments into
// head-major buffers for the attention kernel: q (B,H_q,S,d), k (B,H_kv,S,d) and V
// transposed, vt (B,H_kv,d,S), so attention reads keys contiguously for P·V.
//
// fp16: 128x128x64 workgroup tile, 4 waves as 2x2, each wave 64x64 = 4x4 tiles of
//       v_mfma_f32_16x16x32_f16.  Both tiles are staged in LDS in their natural global
//       layout (A as [m][k], W as [k][n]) through a two-stage ring: the next k-tile's
//       16-byte global loads are in flight while the current one is multiplied, and
//       there is one barrier per k-tile.  The MFMA B operand needs 8 consecutive k of
//       one column per lane; it comes from W[k][n] with two ds_read_b64_tr_b16
//       (gfx950 LDS transpose reads): in each 16-lane group, lane j addresses
//       W[kb + j/4][nb + 4(j%4)] and lane i receives W[kb..kb+3][nb + i].
// fp32: 128x128x16 tile with v_mfma_f32_16x16x4_f32, both tiles staged k-major so each
//       operand is one conflict-free ds_read_b32 (the FP32 operator's parity path).
// Tile edges are zero-filled on load and masked on store.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 lds_h4_t;
#define CF_LDS __attribute__((address_space(3)))

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128;

struct Tiling {
    int n_tiles_m;
    int seg_start[4];   // first column tile of each segment
    int a_vec;          // A rows may be read with vector loads (alignment and K)
    int w_vec[3];       // W rows of segment s may be read with vector loads
};

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

__device__ __forceinline__ int find_seg(const cf_gemm_args_t& a, const Tiling& t, int tile_n) {
    int seg = 0;
    if (a.nseg > 1 && tile_n >= t.seg_start[1]) seg = 1;
    if (a.nseg > 2 && tile_n >= t.seg_start[2]) seg = 2;
    return seg;
}

// Destination offsets split as row part + column part:
//   row-major:          m*N + n
//   q, k (B,H,S,d):     (b*H*S + s)*d      + (n/d)*S*d + n%d
//   vt   (B,H,d,S):     b*H*d*S + s        + n*S
__device__ __forceinline__ size_t row_part(const cf_gemm_args_t& a, int seg, int m) {
    if (a.out_kind == CF_GEMM_OUT_ROWMAJOR) return (size_t)m * a.n[0];
    const int b = m / a.S, s = m - b * a.S;
    const int H = seg == 0 ? a.H_q : a.H_kv;
    if (seg < 2) return ((size_t)b * H * a.S + s) * a.d;
    return (size_t)b * H * a.d * a.S + s;
}

__device__ __forceinline__ size_t col_part(const cf_gemm_args_t& a, int seg, int n) {
    if (a.out_kind == CF_GEMM_OUT_ROWMAJOR) return (size_t)n;
    if (seg < 2) {
        const int h = n / a.d;
        return (size_t)h * a.S * a.d + (n - h * a.d);
    }
    return (size_t)n * a.S;
}

// Store the accumulators of a wave tile: acc[i][j][e] is C[m0 + 16i + 4*lq + e][n0 + 16j + lr].
template <typename T>
__device__ __forceinline__ void store_tile(const cf_gemm_args_t& a, int seg, int N, int m0, int n0,
                                           int lr, int lq, const f4_t (&acc)[4][4]) {
    const T* __restrict__ bias = (const T*)a.bias[seg];
    const T* __restrict__ res = a.out_kind == CF_GEMM_OUT_ROWMAJOR ? (const T*)a.residual : nullptr;
    T* __restrict__ out = (T*)a.out[seg];
    size_t cp[4];
    float bv[4];
    bool nok[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + 16 * j + lr;
        nok[j] = n < N;
        cp[j] = nok[j] ? col_part(a, seg, n) : 0;
        bv[j] = (bias && nok[j]) ? to_f(bias[n]) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = m0 + 16 * i + 4 * lq + e;
            if (m >= a.M) continue;
            const size_t rp = row_part(a, seg, m);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (!nok[j]) continue;
                float v = acc[i][j][e] + bv[j];
                if (res) v += to_f(res[rp + cp[j]]);
                out[rp + cp[j]] = from_f<T>(v);
            }
        }
}

// ------------------------------------------------------------------------- fp16 ---
constexpr int BK16 = 64;
constexpr int LDA16 = BK16 + 8;   // halves per A row in LDS
constexpr int LDW16 = BN + 8;     // halves per W row in LDS
constexpr int A_STAGE = BM * LDA16;
constexpr int W_STAGE = BK16 * LDW16;

__global__ __launch_bounds__(kThreads, 2)
void gemm_f16(cf_gemm_args_t a, Tiling t) {
    __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (A_STAGE + W_STAGE)];

    const int tile_m = blockIdx.x % t.n_tiles_m;
    const int tile_n = blockIdx.x / t.n_tiles_m;
    const int seg = find_seg(a, t, tile_n);
    const int N = a.n[seg];
    const int m0 = tile_m * BM;
    const int n0 = (tile_n - t.seg_start[seg]) * BN;
    const _Float16* __restrict__ A = (const _Float16*)a.a;
    const _Float16* __restrict__ W = (const _Float16*)a.w[seg];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
    const int lr = lane & 15, lq = lane >> 4;
    const bool a_vec = t.a_vec != 0;
    const bool w_vec = t.w_vec[seg] != 0;

    // Global -> register staging: A chunk c = tid + 256*i is row c>>3, k (c&7)*8;
    // W chunk c is row (k) c>>4, column (c&15)*8.
    h8_t ra[4], rw[4];
    auto load_tiles = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int ch = tid + i * kThreads;
            const int gm = m0 + (ch >> 3), gk = k0 + (ch & 7) * 8;
            h8_t v{};
            if (gm < a.M) {
                const _Float16* src = A + (size_t)gm * a.K + gk;
                if (a_vec && gk + 8 <= a.K) v = *(const h8_t*)src;
                else {
#pragma unroll
                    for (int e = 0; e < 8; e++) if (gk + e < a.K) v[e] = src[e];
                }
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int ch = tid + i * kThreads;
            const int gk = k0 + (ch >> 4), gn = n0 + (ch & 15) * 8;
            h8_t v{};
            if (gk < a.K) {
                const _Float16* src = W + (size_t)gk * N + gn;
                if (w_vec && gn + 8 <= N) v = *(const h8_t*)src;
                else {
#pragma unroll
                    for (int e = 0; e < 8; e++) if (gn + e < N) v[e] = src[e];
                }
            }
            rw[i] = v;
        }
    };
    auto store_tiles = [&](int stage) {
        _Float16* As = smem + stage * (A_STAGE + W_STAGE);
        _Float16* Ws = As + A_STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int ch = tid + i * kThreads;
            *(h8_t*)&As[(ch >> 3) * LDA16 + (ch & 7) * 8] = ra[i];
            *(h8_t*)&Ws[(ch >> 4) * LDW16 + (ch & 15) * 8] = rw[i];
        }
    };

    f4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int nk = (a.K + BK16 - 1) / BK16;
    load_tiles(0);
    store_tiles(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int stage = kt & 1;
        if (kt + 1 < nk) load_tiles((kt + 1) * BK16);
        const _Float16* As = smem + stage * (A_STAGE + W_STAGE);
        const _Float16* Ws = As + A_STAGE;
#pragma unroll
        for (int kk = 0; kk < BK16; kk += 32) {
            h8_t af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = *(const h8_t*)&As[(wm + 16 * i + lr) * LDA16 + kk + 8 * lq];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const _Float16* p = &Ws[(kk + 8 * lq + (lr >> 2)) * LDW16 + wn + 16 * j + 4 * (lr & 3)];
                const lds_h4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((CF_LDS lds_h4_t*)p);
                const lds_h4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((CF_LDS lds_h4_t*)(p + 4 * LDW16));
                const h4_t l4 = __builtin_bit_cast(h4_t, lo), h4 = __builtin_bit_cast(h4_t, hi);
                bf[j] = h8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_tiles(stage ^ 1);
        __syncthreads();
    }
    store_tile<_Float16>(a, seg, N, m0 + wm, n0 + wn, lr, lq, acc);
}

// ------------------------------------------------------------------------- fp32 ---
constexpr int BK32 = 16;
constexpr int LDM32 = BM + 4;     // floats per k-major LDS row

__global__ __launch_bounds__(kThreads)
void gemm_f32(cf_gemm_args_t a, Tiling t) {
    __shared__ float As[BK32 * LDM32];   // [k][m]
    __shared__ float Bs[BK32 * LDM32];   // [k][n]

    const int tile_m = blockIdx.x % t.n_tiles_m;
    const int tile_n = blockIdx.x / t.n_tiles_m;
    const int seg = find_seg(a, t, tile_n);
    const int N = a.n[seg];
    const int m0 = tile_m * BM;
    const int n0 = (tile_n - t.seg_start[seg]) * BN;
    const float* __restrict__ A = (const float*)a.a;
    const float* __restrict__ W = (const float*)a.w[seg];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
    const int lr = lane & 15, lq = lane >> 4;
    const bool a_vec = t.a_vec != 0;
    const bool w_vec = t.w_vec[seg] != 0;

    f4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < a.K; k0 += BK32) {
        // A: 128 rows x 16 k = 512 chunks of 4; 2 per thread; stored transposed [k][m].
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const int ch = tid + it * kThreads;
            const int r = ch >> 2, kc = (ch & 3) * 4;
            const int gm = m0 + r, gk = k0 + kc;
            f4_t v{};
            if (gm < a.M) {
                const float* src = A + (size_t)gm * a.K + gk;
                if (a_vec && gk + 4 <= a.K) v = *(const f4_t*)src;
                else {
#pragma unroll
                    for (int e = 0; e < 4; e++) if (gk + e < a.K) v[e] = src[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) As[(kc + e) * LDM32 + r] = v[e];
        }
        // W: 16 k x 128 n = 512 chunks of 4; 2 per thread; stored [k][n].
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const int ch = tid + it * kThreads;
            const int kr = ch >> 5, nc = (ch & 31) * 4;
            const int gk = k0 + kr, gn = n0 + nc;
            f4_t v{};
            if (gk < a.K) {
                const float* src = W + (size_t)gk * N + gn;
                if (w_vec && gn + 4 <= N) v = *(const f4_t*)src;
                else {
#pragma unroll
                    for (int e = 0; e < 4; e++) if (gn + e < N) v[e] = src[e];
                }
            }
            *(f4_t*)&Bs[kr * LDM32 + nc] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK32; kk += 4) {
            float af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = As[(kk + lq) * LDM32 + wm + 16 * i + lr];
#pragma unroll
            for (int j = 0; j < 4; j++) bf[j] = Bs[(kk + lq) * LDM32 + wn + 16 * j + lr];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    store_tile<float>(a, seg, N, m0 + wm, n0 + wn, lr, lq, acc);
}

}  // namespace

extern "C" int cf_launch_gemm(const cf_gemm_args_t* a, void* stream) {
    if (a->nseg < 1 || a->nseg > 3 || a->M <= 0 || a->K <= 0) return (int)hipErrorInvalidValue;
    Tiling t{};
    t.n_tiles_m = (a->M + BM - 1) / BM;
    int acc = 0;
    for (int s = 0; s < a->nseg; s++) {
        t.seg_start[s] = acc;
        acc += (a->n[s] + BN - 1) / BN;
    }
    for (int s = a->nseg; s < 4; s++) t.seg_start[s] = acc;
    // fp16 reads 8 halves at a time from A and W; fp32 reads 4 floats.
    const int vec = a->elem == CF_ELEM_F16 ? 8 : 4;
    t.a_vec = (a->K % vec == 0) && ((uintptr_t)a->a % 16 == 0);
    for (int s = 0; s < a->nseg; s++)
        t.w_vec[s] = (a->n[s] % vec == 0) && ((uintptr_t)a->w[s] % 16 == 0);
    const long long blocks = (long long)acc * t.n_tiles_m;
    if (blocks <= 0 || blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    dim3 grid((unsigned)blocks);
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(gemm_f16, grid, dim3(kThreads), 0, (hipStream_t)stream, *a, t);
    else
        hipLaunchKernelGGL(gemm_f32, grid, dim3(kThreads), 0, (hipStream_t)stream, *a, t);
    return (int)hipGetLastError();
}
