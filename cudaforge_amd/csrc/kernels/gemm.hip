// gemm.hip — prefill projections of MHA_Fused on the matrix cores (gfx950).
//
// C = A·W + bias (+ residual) with A (M, K) row-major and W (K, N) row-major, the
// layout of the reference's "x·W" projections (mha_fused.c:68-88 and :152-171).
// The epilogue either writes C row-major or scatters the Q | K | V column segments into
// head-major buffers for the attention kernel: q (B,H_q,S,d), k (B,H_kv,S,d) and V
// transposed, vt (B,H_kv,d,S), so attention reads keys contiguously for P·V.
//
// fp16: 128x128x64 workgroup tile, 4 waves as 2x2, each wave 64x64 = 4x4 tiles of
//       v_mfma_f32_16x16x32_f16.  The W tile is transposed to [n][k] while it is
//       staged in LDS (8x4 register blocks -> 16-byte LDS rows), so every MFMA operand
//       is one ds_read_b128.
// fp32: same tiling with v_mfma_f32_16x16x4_f32, both tiles staged k-major so each
//       operand is one conflict-free ds_read_b32.
// Tile edges are zero-filled on load and masked on store.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

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

// Store one accumulator element of output column n (segment-local), row m.
template <typename T>
__device__ __forceinline__ void store_out(const cf_gemm_args_t& a, int seg, int m, int n, float v) {
    const T* bias = (const T*)a.bias[seg];
    if (bias) v += to_f(bias[n]);
    if (a.out_kind == CF_GEMM_OUT_ROWMAJOR) {
        const size_t idx = (size_t)m * a.n[0] + n;
        if (a.residual) v += to_f(((const T*)a.residual)[idx]);
        ((T*)a.out[0])[idx] = from_f<T>(v);
        return;
    }
    const int b = m / a.S, s = m - b * a.S;
    const int h = n / a.d, i = n - h * a.d;
    const int H = seg == 0 ? a.H_q : a.H_kv;
    size_t idx;
    if (seg < 2) idx = (((size_t)b * H + h) * a.S + s) * a.d + i;
    else idx = (((size_t)b * H + h) * a.d + i) * a.S + s;
    ((T*)a.out[seg])[idx] = from_f<T>(v);
}

__device__ __forceinline__ int find_seg(const cf_gemm_args_t& a, const Tiling& t, int tile_n) {
    int seg = 0;
    if (a.nseg > 1 && tile_n >= t.seg_start[1]) seg = 1;
    if (a.nseg > 2 && tile_n >= t.seg_start[2]) seg = 2;
    return seg;
}

// ------------------------------------------------------------------------- fp16 ---
constexpr int BK16 = 64;
constexpr int LDA16 = BK16 + 8;   // halves per LDS row (pad keeps 16-byte rows off one bank set)

__global__ __launch_bounds__(kThreads)
void gemm_f16(cf_gemm_args_t a, Tiling t) {
    __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDA16];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDA16];

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

    f4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < a.K; k0 += BK16) {
        // A tile: 128 rows x 64 halves = 1024 chunks of 8; 4 per thread.
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int ch = tid + it * kThreads;
            const int r = ch >> 3, kc = (ch & 7) * 8;
            const int gm = m0 + r, gk = k0 + kc;
            h8_t v{};
            if (gm < a.M) {
                const _Float16* src = A + (size_t)gm * a.K + gk;
                if (a_vec && gk + 8 <= a.K) v = *(const h8_t*)src;
                else {
#pragma unroll
                    for (int e = 0; e < 8; e++) if (gk + e < a.K) v[e] = src[e];
                }
            }
            *(h8_t*)&As[r * LDA16 + kc] = v;
        }
        // W tile: 64 k x 128 n.  Thread owns an 8(k) x 4(n) block, 256 blocks.
        {
            const int kb = (tid & 7) * 8;       // k offset of the block
            const int nb = (tid >> 3) * 4;      // n offset of the block
            h4_t rows[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int gk = k0 + kb + j, gn = n0 + nb;
                h4_t v{};
                if (gk < a.K) {
                    const _Float16* src = W + (size_t)gk * N + gn;
                    if (w_vec && gn + 4 <= N) v = *(const h4_t*)src;
                    else {
#pragma unroll
                        for (int e = 0; e < 4; e++) if (gn + e < N) v[e] = src[e];
                    }
                }
                rows[j] = v;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                h8_t col;
#pragma unroll
                for (int j = 0; j < 8; j++) col[j] = rows[j][c];
                *(h8_t*)&Bs[(nb + c) * LDA16 + kb] = col;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK16; kk += 32) {
            h8_t af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = *(const h8_t*)&As[(wm + 16 * i + lr) * LDA16 + kk + 8 * lq];
#pragma unroll
            for (int j = 0; j < 4; j++) bf[j] = *(const h8_t*)&Bs[(wn + 16 * j + lr) * LDA16 + kk + 8 * lq];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // acc[i][j][e]: row = wm + 16i + 4*lq + e, col = wn + 16j + lr  (A rows = m, B rows = n)
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm + 16 * i + 4 * lq + e;
                const int n = n0 + wn + 16 * j + lr;
                if (m < a.M && n < N) store_out<_Float16>(a, seg, m, n, acc[i][j][e]);
            }
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
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm + 16 * i + 4 * lq + e;
                const int n = n0 + wn + 16 * j + lr;
                if (m < a.M && n < N) store_out<float>(a, seg, m, n, acc[i][j][e]);
            }
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
    // fp16 A is read 8 halves at a time and W 4 at a time; fp32 reads 4 floats.
    const int avec = a->elem == CF_ELEM_F16 ? 8 : 4;
    t.a_vec = (a->K % avec == 0) && ((uintptr_t)a->a % 16 == 0);
    for (int s = 0; s < a->nseg; s++)
        t.w_vec[s] = (a->n[s] % 4 == 0) && ((uintptr_t)a->w[s] % 16 == 0);
    const long long blocks = (long long)acc * t.n_tiles_m;
    if (blocks <= 0 || blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    dim3 grid((unsigned)blocks);
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(gemm_f16, grid, dim3(kThreads), 0, (hipStream_t)stream, *a, t);
    else
        hipLaunchKernelGGL(gemm_f32, grid, dim3(kThreads), 0, (hipStream_t)stream, *a, t);
    return (int)hipGetLastError();
}
