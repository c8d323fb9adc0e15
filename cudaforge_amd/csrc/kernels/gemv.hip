// gemv.hip — skinny GEMM (M <= 16 rows per tile) on MFMA for the decode projections.
//
// Decode's Q/K/V and output projections (mha_decode.c:54-86 and :117-121) are
// Y = X·W + b with X = one token per sequence (M = B rows) and W (K, N) row-major.
// They are bound by reading W once, so the kernel streams W with 16-byte loads and
// keeps the multiply on the matrix cores, where the batch rows ride along for free:
//
//   MFMA rows  <- output columns n   (A operand = W^T, transposed in registers)
//   MFMA cols  <- batch rows m       (B operand = X, k-contiguous rows of X)
//   MFMA k     <- reduction index k
//
// fp16: v_mfma_f32_16x16x32_f16.  A lane loads an 8(k) x 8(n) block of W (eight
//       16-byte row segments), and the 8 columns become 8 A operands of 8 k values.
// fp32: v_mfma_f32_16x16x4_f32.  A lane loads 1(k) x 4(n) twice per k step.
// A workgroup (4 waves) owns a 128-column tile and one of `k_split` K chunks; waves
// interleave k steps and reduce through LDS.  With k_split = 1 the workgroup adds the
// bias and scatters the result; otherwise it writes an fp32 partial per K chunk and a
// second launch (gemv_reduce) sums the partials, adds the bias and scatters.  The kernel
// boundary orders the partials: no fences or atomics (each XCD has its own L2).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kColTile = 128;
constexpr int kMTile = 16;
constexpr int kAcc = 8;                      // MFMA tiles per lane (8 x 16 columns)
constexpr int kTileVals = kMTile * kColTile; // 2048 outputs per tile

template <typename T> struct Cfg;
template <> struct Cfg<_Float16> { static constexpr int KSTEP = 32; static constexpr int VEC = 8; };
template <> struct Cfg<float>    { static constexpr int KSTEP = 4;  static constexpr int VEC = 4; };

struct Tiles {
    int start[CF_GEMV_MAX_SEGS + 1];  // first column tile of each segment; start[nseg] = total
    int k_chunk;
    int vec_ok;
};

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

template <typename T, typename V>
__device__ __forceinline__ V load_row(const T* __restrict__ p, int col, int ncols, bool vec_ok) {
    constexpr int VEC = Cfg<T>::VEC;
    if (vec_ok && col + VEC <= ncols) return *(const V*)(p + col);
    V v{};
#pragma unroll
    for (int e = 0; e < VEC; e++)
        if (col + e < ncols) v[e] = p[col + e];
    return v;
}

// Column offset (within the tile) of accumulator c, element i, for lane l.
template <typename T> __device__ __forceinline__ int tile_col(int c, int i, int l);
template <> __device__ __forceinline__ int tile_col<_Float16>(int c, int i, int l) {
    return 8 * (4 * (l >> 4) + i) + c;
}
template <> __device__ __forceinline__ int tile_col<float>(int c, int i, int l) {
    return 64 * (c >> 2) + 4 * (4 * (l >> 4) + i) + (c & 3);
}

template <typename T>
__device__ __forceinline__ void kstep(const cf_gemv_args_t& a, const T* __restrict__ W, int N, int nb,
                                      int m, int k0, int kend, bool vec_ok, f4_t (&acc)[kAcc]);

template <>
__device__ __forceinline__ void kstep<_Float16>(const cf_gemv_args_t& a, const _Float16* __restrict__ W,
                                                int N, int nb, int m, int k0, int kend, bool vec_ok,
                                                f4_t (&acc)[kAcc]) {
    const int l = threadIdx.x & 63, q = l >> 4, r = l & 15;
    const int kq = k0 + 8 * q;
    // B operand: X[m][kq .. kq+7]
    h8_t xb{};
    if (m < a.M) {
        const _Float16* xr = (const _Float16*)a.x + (size_t)m * a.K;
        if (vec_ok && kq + 8 <= kend) xb = *(const h8_t*)(xr + kq);
        else {
#pragma unroll
            for (int e = 0; e < 8; e++) if (kq + e < kend) xb[e] = xr[kq + e];
        }
    }
    // A operands: rows kq..kq+7 of W, columns nb + 8r .. +7, transposed.
    h8_t rows[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (kq + j < kend) rows[j] = load_row<_Float16, h8_t>(W + (size_t)(kq + j) * N, nb + 8 * r, N, vec_ok);
        else rows[j] = h8_t{};
    }
#pragma unroll
    for (int c = 0; c < 8; c++) {
        h8_t av;
#pragma unroll
        for (int j = 0; j < 8; j++) av[j] = rows[j][c];
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xb, acc[c], 0, 0, 0);
    }
}

template <>
__device__ __forceinline__ void kstep<float>(const cf_gemv_args_t& a, const float* __restrict__ W,
                                             int N, int nb, int m, int k0, int kend, bool vec_ok,
                                             f4_t (&acc)[kAcc]) {
    const int l = threadIdx.x & 63, q = l >> 4, r = l & 15;
    const int kr = k0 + q;
    float xb = 0.0f;
    f4_t v0{}, v1{};
    if (kr < kend) {
        if (m < a.M) xb = ((const float*)a.x)[(size_t)m * a.K + kr];
        const float* wr = W + (size_t)kr * N;
        v0 = load_row<float, f4_t>(wr, nb + 4 * r, N, vec_ok);
        v1 = load_row<float, f4_t>(wr, nb + 64 + 4 * r, N, vec_ok);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0[c], xb, acc[c], 0, 0, 0);
        acc[4 + c] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1[c], xb, acc[4 + c], 0, 0, 0);
    }
}

// Store one finished output element (bias added) of segment `seg`, segment-local column n.
template <typename T>
__device__ __forceinline__ void store_out(const cf_gemv_args_t& a, const cf_gemv_seg_t& sg, int m, int n, float v) {
    const T* __restrict__ bias = (const T*)sg.bias;
    if (bias) v += to_f(bias[n]);
    const int64_t pos = a.pos_lens ? (int64_t)a.pos_lens[m] : a.pos_uniform;
    if (a.pos_limit == 0 || (pos >= 0 && pos < a.pos_limit))
        ((T*)sg.out)[(size_t)m * sg.ld_m + (size_t)pos * sg.ld_pos + n] = from_f<T>(v);
}

__device__ __forceinline__ int seg_of(const cf_gemv_args_t& a, const Tiles& t, int tile) {
    int seg = 0;
#pragma unroll
    for (int s = 1; s < CF_GEMV_MAX_SEGS; s++)
        if (s < a.nseg && tile >= t.start[s]) seg = s;
    return seg;
}

// Split-K partial kernel.  With one K chunk it applies the epilogue itself; otherwise
// it writes fp32 partials [k_split][Mp][ncols] (ncols = 128 * column tiles) for
// gemv_reduce.
template <typename T>
__global__ __launch_bounds__(kThreads)
void gemv_kernel(cf_gemv_args_t a, Tiles t) {
    constexpr int KSTEP = Cfg<T>::KSTEP;
    __shared__ float red[kWaves * kTileVals];  // 32 KB

    const int tile = blockIdx.x, ks = blockIdx.y, mt = blockIdx.z;
    const int seg = seg_of(a, t, tile);
    const cf_gemv_seg_t& sg = a.seg[seg];
    const int N = (int)sg.n;
    const int nb = (tile - t.start[seg]) * kColTile;
    const T* __restrict__ W = (const T*)sg.w;
    const bool vec_ok = t.vec_ok != 0;

    const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
    const int m = mt * kMTile + (l & 15);
    const int kbeg = ks * t.k_chunk;
    const int kend = min(a.K, kbeg + t.k_chunk);

    f4_t acc[kAcc];
#pragma unroll
    for (int c = 0; c < kAcc; c++) acc[c] = f4_t{0.f, 0.f, 0.f, 0.f};
    for (int k0 = kbeg + wave * KSTEP; k0 < kend; k0 += kWaves * KSTEP)
        kstep<T>(a, W, N, nb, m, k0, kend, vec_ok, acc);

    // Cross-wave reduction: value (c, i) of lane l lives at red[w][(c*4 + i)*64 + l].
#pragma unroll
    for (int c = 0; c < kAcc; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[wave * kTileVals + (c * 4 + i) * 64 + l] = acc[c][i];
    __syncthreads();
    const int ncols = t.start[a.nseg] * kColTile;
    const int Mp = gridDim.z * kMTile;
#pragma unroll
    for (int j = 0; j < kTileVals / kThreads; j++) {
        const int idx = tid + j * kThreads;
        float s = red[idx];
#pragma unroll
        for (int w = 1; w < kWaves; w++) s += red[w * kTileVals + idx];
        const int li = idx & 63, ci = idx >> 6;
        const int lc = tile_col<T>(ci >> 2, ci & 3, li);
        const int mm = mt * kMTile + (li & 15);
        if (a.k_split > 1) {
            a.partials[((size_t)ks * Mp + mm) * ncols + (size_t)tile * kColTile + lc] = s;
        } else if (nb + lc < N && mm < a.M) {
            store_out<T>(a, sg, mm, nb + lc, s);
        }
    }
}

// Sums the K-chunk partials of every output element and applies the epilogue.
template <typename T>
__global__ __launch_bounds__(256)
void gemv_reduce(cf_gemv_args_t a, Tiles t) {
    const int ncols = t.start[a.nseg] * kColTile;
    const int Mp = (a.M + kMTile - 1) / kMTile * kMTile;
    const size_t total = (size_t)a.M * ncols;
    const size_t plane = (size_t)Mp * ncols;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
        const int m = (int)(idx / ncols), col = (int)(idx - (size_t)m * ncols);
        const int tile = col / kColTile;
        const int seg = seg_of(a, t, tile);
        const int n = (tile - t.start[seg]) * kColTile + (col - tile * kColTile);
        if (n >= a.seg[seg].n) continue;
        const float* p = a.partials + (size_t)m * ncols + col;
        // Eight independent loads in flight per round trip.
        float s0 = 0.0f, s1 = 0.0f;
        int kk = 0;
        for (; kk + 8 <= a.k_split; kk += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = p[(size_t)(kk + j) * plane];
#pragma unroll
            for (int j = 0; j < 8; j += 2) { s0 += v[j]; s1 += v[j + 1]; }
        }
        for (; kk < a.k_split; kk++) s0 += p[(size_t)kk * plane];
        store_out<T>(a, a.seg[seg], m, n, s0 + s1);
    }
}

Tiles make_tiles(const cf_gemv_args_t* a) {
    Tiles t{};
    int acc = 0;
    for (int s = 0; s < a->nseg; s++) {
        t.start[s] = acc;
        acc += (int)((a->seg[s].n + kColTile - 1) / kColTile);
    }
    for (int s = a->nseg; s <= CF_GEMV_MAX_SEGS; s++) t.start[s] = acc;
    const int kstep = a->elem == CF_ELEM_F16 ? Cfg<_Float16>::KSTEP : Cfg<float>::KSTEP;
    const int vec = a->elem == CF_ELEM_F16 ? 8 : 4;
    const int ks = a->k_split > 0 ? a->k_split : 1;
    int chunk = (a->K + ks - 1) / ks;
    chunk = (chunk + kstep - 1) / kstep * kstep;
    t.k_chunk = chunk;
    int ok = (a->K % vec == 0) && (((uintptr_t)a->x) % 16 == 0);
    for (int s = 0; s < a->nseg; s++)
        ok = ok && (a->seg[s].n % vec == 0) && (((uintptr_t)a->seg[s].w) % 16 == 0);
    t.vec_ok = ok;
    return t;
}

}  // namespace

extern "C" int32_t cf_gemv_col_tile(int32_t elem) { (void)elem; return kColTile; }
extern "C" int32_t cf_gemv_k_step(int32_t elem) {
    return elem == CF_ELEM_F16 ? Cfg<_Float16>::KSTEP : Cfg<float>::KSTEP;
}

extern "C" size_t cf_gemv_partials_floats(const cf_gemv_args_t* a) {
    if (a->k_split <= 1) return 0;
    const Tiles t = make_tiles(a);
    const size_t Mp = (size_t)((a->M + kMTile - 1) / kMTile) * kMTile;
    return (size_t)a->k_split * Mp * (size_t)t.start[a->nseg] * kColTile;
}

extern "C" int cf_launch_gemv(const cf_gemv_args_t* a, void* stream) {
    const Tiles t = make_tiles(a);
    // Every K chunk must be non-empty (each writes its full partial plane).
    const int ks = a->k_split > 0 ? a->k_split : 1;
    if ((ks - 1) * t.k_chunk >= a->K) return (int)hipErrorInvalidValue;
    cf_gemv_args_t args = *a;
    args.k_split = ks;
    hipStream_t s = (hipStream_t)stream;
    const int m_tiles = (a->M + kMTile - 1) / kMTile;
    dim3 grid((unsigned)t.start[a->nseg], (unsigned)ks, (unsigned)m_tiles);
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(gemv_kernel<_Float16>, grid, dim3(kThreads), 0, s, args, t);
    else
        hipLaunchKernelGGL(gemv_kernel<float>, grid, dim3(kThreads), 0, s, args, t);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ks == 1) return (int)e;
    const size_t total = (size_t)a->M * t.start[a->nseg] * kColTile;
    size_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(gemv_reduce<_Float16>, dim3((unsigned)blocks), dim3(256), 0, s, args, t);
    else
        hipLaunchKernelGGL(gemv_reduce<float>, dim3((unsigned)blocks), dim3(256), 0, s, args, t);
    return (int)hipGetLastError();
}
