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
// Two kernels:
// * gemv_f16_dma (fp16, K % 32 == 0, every segment width % 64 == 0, 16-byte aligned):
//   one wave per 64/128/256 columns and K chunk, W and X streamed by DMA into an LDS
//   ring and multiplied as Y = X . W on MFMA (see the kernel); the K split is planned
//   here from the CU count.
// * gemv_kernel (any shape, fp16 or fp32), with the roles swapped:
//   MFMA rows  <- output columns n   (A operand = W^T, transposed in registers)
//   MFMA cols  <- batch rows m       (B operand = X, k-contiguous rows of X)
//   MFMA k     <- reduction index k
//   fp16: v_mfma_f32_16x16x32_f16.  A lane loads an 8(k) x 8(n) block of W (eight
//         16-byte row segments), and the 8 columns become 8 A operands of 8 k values.
//   fp32: v_mfma_f32_16x16x4_f32.  A lane loads 1(k) x 4(n) twice per k step.
//   A workgroup (4 waves) owns a 128-column tile and one of `k_split` K chunks; waves
//   interleave k steps and reduce through LDS.
// With one K chunk the workgroup adds the bias and scatters the result; otherwise it
// writes an fp32 partial per K chunk and a second launch (gemv_reduce4) sums the
// partials, adds the bias, optionally rotates RoPE pairs (decode's Q and K_new) and
// scatters.  The kernel boundary orders the partials: no fences or atomics (each XCD
// has its own L2).  The launch's last kernel can also advance the caller's device-held
// decode lengths (cf_gemv_args_t.advance), since nothing after it in the step reads them.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kernels.h"
#include "cdna4.h"

namespace {

using namespace cdna4;

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
    int bn;                           // columns per tile
    int ks;                           // K chunks (workgroups along K)
    int dma;                          // fp16 DMA path: its tile width (64/128/256), else 0
    int small;                        // one-pass kernel for small projections (gemv_small)
    // The K-chunk sum's divisors, set by the launcher: column tiles, lanes per row
    // (bn / 4), and the RoPE head size (2 without RoPE).
    FastDiv div_tiles, div_lpr, div_rd;
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

// The launch's last kernel advances the caller's device lengths (its first workgroup).
__device__ __forceinline__ void advance_lengths(const cf_gemv_args_t& a) {
    if (a.advance && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
        for (int i = threadIdx.x; i < a.advance_n; i += blockDim.x) a.advance[i] += 1;
}

// Rows are stored unless their position is out of [0, pos_limit); the limit applies only
// to segments indexed by position (ld_pos != 0, the cache rows K_new and V_new), so the Q
// segment is always written and the attention has a defined query even for a length the
// cache cannot take.
__device__ __forceinline__ bool pos_ok(const cf_gemv_args_t& a, const cf_gemv_seg_t& sg, int64_t pos) {
    return sg.ld_pos == 0 || a.pos_limit == 0 || (pos >= 0 && pos < a.pos_limit);
}

// Store one finished output element of segment `seg`, segment-local column n.
template <typename T>
__device__ __forceinline__ void store_val(const cf_gemv_args_t& a, const cf_gemv_seg_t& sg, int m, int n, float v) {
    const int64_t pos = a.pos_lens ? (int64_t)a.pos_lens[m] : a.pos_uniform;
    if (pos_ok(a, sg, pos))
        ((T*)sg.out)[(size_t)m * sg.ld_m + (size_t)(sg.ld_pos ? pos : 0) * sg.ld_pos + n] = from_f<T>(v);
}

// ... with the segment's bias added first.
template <typename T>
__device__ __forceinline__ void store_out(const cf_gemv_args_t& a, const cf_gemv_seg_t& sg, int m, int n, float v) {
    const T* __restrict__ bias = (const T*)sg.bias;
    if (bias) v += to_f(bias[n]);
    store_val<T>(a, sg, m, n, v);
}

// One RoPE pair, rotated as the rope operator does it (fp32, no contraction).
__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float2 cs) {
#pragma clang fp contract(off)
    const float a = x0 * cs.x, b = x1 * cs.y;
    const float c = x0 * cs.y, e = x1 * cs.x;
    x0 = a - b;
    x1 = c + e;
}

__device__ __forceinline__ int seg_of(const cf_gemv_args_t& a, const Tiles& t, int tile) {
    int seg = 0;
#pragma unroll
    for (int s = 1; s < CF_GEMV_MAX_SEGS; s++)
        if (s < a.nseg && tile >= t.start[s]) seg = s;
    return seg;
}

// Split-K partial kernel.  With one K chunk it applies the epilogue itself; otherwise
// it writes fp32 partials [k_split][M][ncols] (ncols = 128 * column tiles) for
// gemv_reduce4.
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
    if (a.k_split == 1) advance_lengths(a);
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
            if (mm < a.M) a.partials[((size_t)ks * a.M + mm) * ncols + (size_t)tile * kColTile + lc] = s;
        } else if (nb + lc < N && mm < a.M) {
            store_out<T>(a, sg, mm, nb + lc, s);
        }
    }
}

// ---- fp16 DMA path: one wave per workgroup owns BN = 64, 128 or 256 columns and one K
// chunk of an M tile of 16 rows.  Per 32-row k step, W (32 x BN) and X (16 x 32) go
// from HBM straight into an NS-deep LDS ring (global_load_lds_dwordx4 with a uniform
// base and per-lane offsets fixed for the whole loop, so the issue is scalar work), and
// the wave runs BN/16 MFMAs  Y(16 rows x 16 cols) += X(16 x 32) . W(32 x 16): the X
// fragment is one ds_read_b128, each W fragment two ds_read_b64_tr_b16 (8 consecutive k
// of one column).  LDS rows are XOR-swizzled in 16-byte chunks so both read patterns
// are bank-conflict free.  Wider tiles read longer contiguous row segments of W.
constexpr int kDK = 32;

template <int BN> struct Dma;
template <> struct Dma<64>  { static constexpr int NS = 6; static constexpr int PER_CU = 4; };
template <> struct Dma<128> { static constexpr int NS = 5; static constexpr int PER_CU = 3; };
template <> struct Dma<256> { static constexpr int NS = 4; static constexpr int PER_CU = 2; };

template <int BN>
__device__ __forceinline__ int wswz(int row) {
    if constexpr (BN == 64) return (((row >> 1) & 1) << 1) | (((row >> 3) & 1) << 2);
    else return ((row & 3) << 1) | (((row >> 3) & 1) << 3);
}
__device__ __forceinline__ int xswz(int row) { return (row >> 2) & 3; }

template <int BN>
__global__ __launch_bounds__(64)
void gemv_f16_dma(cf_gemv_args_t a, Tiles t) {
    constexpr int NS = Dma<BN>::NS;
    constexpr int CPR = BN / 8;                  // 16-byte chunks per W row
    constexpr int RPI = 64 / CPR;                // W rows per DMA instruction
    constexpr int NI = kDK / RPI;                // W DMA instructions per stage
    constexpr int NL = NI + 1;                   // ... plus one for X
    constexpr int NT = BN / 16;                  // MFMA column tiles
    constexpr int STAGE = kDK * BN + kMTile * kDK;   // halves per stage: W then X
    static_assert((NS - 1) * NL < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) _Float16 ring[NS * STAGE];

    const int tile = blockIdx.x, ks = blockIdx.y, mt = blockIdx.z;
    const int seg = seg_of(a, t, tile);
    const cf_gemv_seg_t& sg = a.seg[seg];
    const int N = (int)sg.n;
    const int n0 = (tile - t.start[seg]) * BN;
    const int kbeg = ks * t.k_chunk;
    const int nst = (min(a.K, kbeg + t.k_chunk) - kbeg) / kDK;     // K % 32 == 0 on this path
    const int lane = threadIdx.x, lr = lane & 15, lq = lane >> 4;
    const _Float16* __restrict__ W = (const _Float16*)sg.w;
    const _Float16* __restrict__ X = (const _Float16*)a.x;

    // DMA: W instruction u fills k rows RPI*u .. (lane L: row RPI*u + L/CPR, physical
    // chunk L%CPR = logical chunk (L%CPR) ^ wswz(row)); the X instruction fills the 16
    // rows of the M tile (lane L: row L/4, clamped to the last real row, chunk
    // (L%4) ^ xswz(row)).
    uint32_t woff[NI];
#pragma unroll
    for (int u = 0; u < NI; u++) {
        const int row = RPI * u + lane / CPR;
        woff[u] = (uint32_t)row * (uint32_t)N * 2u + 16u * (uint32_t)((lane % CPR) ^ wswz<BN>(row));
    }
    const int xr = lane >> 2;
    const uint32_t xoff = (uint32_t)min(mt * kMTile + xr, a.M - 1) * (uint32_t)a.K * 2u +
                          16u * (uint32_t)((lane & 3) ^ xswz(xr));
    const uint32_t base = lds_offset(ring);
    auto issue = [&](int st, int stage) {           // stage == st % NS
        const int k0 = kbeg + st * kDK;
        const uint32_t sb = base + (uint32_t)(stage * STAGE) * 2u;
        const _Float16* wb = W + (size_t)k0 * N + n0;
#pragma unroll
        for (int u = 0; u < NI; u++) lds_dma16_s(woff[u], wb, sb + u * 1024u);
        lds_dma16_s(xoff, X + k0, sb + (uint32_t)(kDK * BN) * 2u);
    };

    // Per-lane LDS read offsets (halves) inside a stage.
    const int x_rd = kDK * BN + lr * kDK + 8 * (lq ^ xswz(lr));
    int w_rd[NT][2];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = 8 * lq + 4 * h + (lr >> 2);
            const int col = 16 * j + 4 * (lr & 3);
            w_rd[j][h] = row * BN + 8 * ((col >> 3) ^ wswz<BN>(row)) + (col & 7);
        }

    f4_t acc[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) acc[j] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < NS - 1; st++)
        if (st < nst) issue(st, st);
    for_each_stage<NS>(nst, [&](int st, auto stage_c) {
        constexpr int stage = decltype(stage_c)::value;
        // Refill the previous step's stage before waiting for this one, so all NS stages
        // are in flight during the wait.  Its LDS reads have returned (their values fed
        // its MFMAs): one wave needs no barrier.
        if (st + NS - 1 < nst) {
            wait_lds_reads();
            issue(st + NS - 1, (stage + NS - 1) % NS);
        }
        wait_ahead<NL, NS - 1>(min(NS - 1, nst - 1 - st));
        const _Float16* sp = ring + stage * STAGE;
        const h8_t xa = *(const h8_t*)(sp + x_rd);
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const h8_t wb = cat8(ds_read_tr4(sp + w_rd[j][0]), ds_read_tr4(sp + w_rd[j][1]));
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wb, acc[j], 0, 0, 0);
        }
    });

    // Lane (lr, lq) holds Y[m = 16mt + 4lq + i][n0 + 16j + lr].
    if (t.ks == 1) {
        advance_lengths(a);
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = mt * kMTile + 4 * lq + i;
                if (m < a.M) store_out<_Float16>(a, sg, m, n0 + 16 * j + lr, acc[j][i]);
            }
    } else {
        // Partials of real rows only; a full M tile stores without per-lane tests.
        const int ncols = t.start[a.nseg] * BN;
        float* dst = a.partials + ((size_t)ks * a.M + mt * kMTile + 4 * lq) * ncols + (size_t)tile * BN + lr;
        if (mt * kMTile + kMTile <= a.M) {
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) dst[(size_t)i * ncols + 16 * j] = acc[j][i];
        } else {
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (mt * kMTile + 4 * lq + i < a.M) dst[(size_t)i * ncols + 16 * j] = acc[j][i];
        }
    }
}

int g_dma_bn = 0;   // tuning override of the DMA path's tile width (0 = automatic)
int g_dma_ks = 0;   // tuning override of the DMA path's K split (0 = automatic)

// Tile width of the DMA path, or 0 if it does not apply: 128 columns (measured best at
// the decode shapes; 64 and 256 ran 5-15 % slower), else the widest that divides every
// segment.
int dma_bn(const cf_gemv_args_t* a) {
    if (a->elem != CF_ELEM_F16 || a->K % kDK != 0 || ((uintptr_t)a->x) % 16 != 0) return 0;
    int bn = 128;
    for (int s = 0; s < a->nseg; s++) {
        if (((uintptr_t)a->seg[s].w) % 16 != 0) return 0;
        while (bn >= 64 && a->seg[s].n % bn != 0) bn /= 2;
    }
    if (bn < 64) return 0;
    if (g_dma_bn >= 64 && g_dma_bn <= bn) bn = g_dma_bn;
    return bn;
}

// Partial reduce.  A wave owns rows of one column tile (t.bn = 64, 128 or 256 columns):
// bn / 4 lanes per row, each with 4 adjacent columns, so the tile, its segment and the
// segment's pointers are uniform per wave (scalar loads of the argument block).  Every
// load that does not need the partials is issued around them: the row's position and
// the bias before, the RoPE angles (which need the position) right after, so the whole
// reduction is about one round trip to memory.  A thread issues all of its K-chunk
// loads (16-byte) before summing: KS >= k_split loads, unconditional, the chunk index
// clamped to the last chunk and the surplus left out of the sum (a load under a branch
// was waited for right there).  One-wave workgroups spread the partials over the CUs
// (16 rows x 6144 columns is 384 of them).
constexpr int kReduceThreads = 64;
constexpr int kMaxKSplit = 32;    // K chunks the reduce keeps in flight
template <typename T, int KS>
__global__ __launch_bounds__(kReduceThreads)
void gemv_reduce4(cf_gemv_args_t a, Tiles t) {
    static_assert(KS <= kMaxKSplit, "K chunks");
    const int ntiles = t.start[a.nseg], bn = t.bn;
    const int lpr = bn / 4, rpw = fastdiv(kReduceThreads, t.div_lpr);   // lanes per row, rows per wave
    const int ncols = ntiles * bn;
    const size_t plane = (size_t)a.M * ncols;
    advance_lengths(a);
    const int rb = fastdiv((int)blockIdx.x, t.div_tiles), tile = (int)blockIdx.x - rb * ntiles;
    const int tq = fastdiv((int)threadIdx.x, t.div_lpr);
    const int m = rb * rpw + tq;
    if (m >= a.M) return;
    const int lc = 4 * ((int)threadIdx.x - tq * lpr);
    const int seg = seg_of(a, t, tile);
    const cf_gemv_seg_t& sg = a.seg[seg];
    const int n = (tile - t.start[seg]) * bn + lc;        // segment-local column
    // Optional operands are read through a stand-in (the partials, always valid) and the
    // value selected afterwards: a load under a branch makes the compiler wait for it at
    // the branch's end, one round trip each.
    const float* const dummy = a.partials;
    const int32_t* const pl = a.pos_lens ? a.pos_lens : (const int32_t*)dummy;
    const int32_t pl_m = pl[m];
    const T* __restrict__ bias = (const T*)sg.bias;
    const T* const bp = bias ? bias : (const T*)dummy;
    float bv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) bv[e] = to_f(bp[min(n + e, (int)sg.n - 1)]);
    const float* p = a.partials + (size_t)m * ncols + (size_t)tile * bn + lc;
    const int nk = min(KS, a.k_split);                    // the launcher picks KS >= k_split
    f4_t v[KS];
#pragma unroll
    for (int k = 0; k < KS; k++) v[k] = *(const f4_t*)(p + (size_t)min(k, nk - 1) * plane);
    const int64_t pos = a.pos_lens ? (int64_t)pl_m : a.pos_uniform;
    const bool rotate = a.rope_table && ((a.rope_segs >> seg) & 1) && pos >= 0 && pos < a.rope_rows;
    // n is a multiple of 4 and rope_d is even, so (n, n+1) and (n+2, n+3) are pairs.
    const int rd = a.rope_table ? a.rope_d : 2;
    const float2* tb = a.rope_table ? (const float2*)a.rope_table + (rotate ? pos : 0) * (rd >> 1)
                                    : (const float2*)dummy;
    const float2 c0 = tb[(n - fastdiv(n, t.div_rd) * rd) >> 1], c1 = tb[(n + 2 - fastdiv(n + 2, t.div_rd) * rd) >> 1];
    const float2 cs[2] = {rotate ? c0 : float2{1.f, 0.f}, rotate ? c1 : float2{1.f, 0.f}};
    f4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KS; k += 2) {
        if (k < nk) s0 += v[k];
        if (k + 1 < nk) s1 += v[k + 1];
    }
    s0 += s1;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = n + e < sg.n && bias ? s0[e] + bv[e] : s0[e];
    if (rotate)
#pragma unroll
        for (int e = 0; e < 4; e += 2)
            if (n + e + 1 < sg.n) rotate_pair(o[e], o[e + 1], cs[e >> 1]);
    if (!pos_ok(a, sg, pos)) return;
    T* out = (T*)sg.out + (size_t)m * sg.ld_m + (size_t)(sg.ld_pos ? pos : 0) * sg.ld_pos + n;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (n + e < sg.n) out[e] = from_f<T>(o[e]);
}

// ---- small projections (a few batch rows, weights of a few MB, e.g. GPT-2-small
// decode at batch 1): one pass over all of K, so no partials and no second launch; at
// that size the fixed cost of the extra launch is most of the time.  A workgroup owns
// kSmallCols = 16 columns and its 4 waves a quarter of K each.  A lane loads 16 bytes of
// a W row (VEC columns; LPR lanes per row, RPI = 64 / LPR rows per wave instruction),
// NB rows in flight, and multiplies them with X staged in LDS (fp32).  The first batch
// of W loads is issued before X is staged, so both arrive in one round trip.  Lanes of
// one column group then sum over their rows with shuffles, the waves through LDS, and
// M * 4 threads add the bias, rotate RoPE pairs and store 4 columns each.
constexpr int kSmallCols = 16;
constexpr int kSmallMaxM = 4;
constexpr int kSmallMaxX = 4096;                  // M * K floats of X staged in LDS
constexpr long long kSmallMaxBytes = 8ll << 20;   // weight bytes up to which the path is taken
template <typename T>
__global__ __launch_bounds__(kThreads)
void gemv_small(cf_gemv_args_t a, Tiles t) {
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int LPR = kSmallCols / VEC;         // lanes per W row
    constexpr int RPI = 64 / LPR;                 // rows per wave instruction
    constexpr int NB = sizeof(T) == 4 ? 16 : 8;   // row loads in flight per lane
    using V = std::conditional_t<sizeof(T) == 4, f4_t, h8_t>;
    __shared__ float xs[kSmallMaxX];
    __shared__ float wsum[kWaves][kSmallMaxM][kSmallCols];
    const int tile = blockIdx.x;
    const int seg = seg_of(a, t, tile);
    const cf_gemv_seg_t& sg = a.seg[seg];
    const int N = (int)sg.n;
    const int nb = (tile - t.start[seg]) * kSmallCols;
    const T* __restrict__ W = (const T*)sg.w + nb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane / LPR, c = lane % LPR;
    const int M = a.M, K = a.K;
    const int kq = (K + kWaves * RPI - 1) / (kWaves * RPI) * RPI;   // rows per wave
    const int k_lo = wave * kq, k_hi = min(K, k_lo + kq);
    // The storing threads' position, bias and RoPE angles are loaded with the first W
    // batch and X, not after the sums, where they would cost another round trip.  Each
    // load is unconditional (an optional operand is read through a stand-in, W, and the
    // value selected afterwards; non-storing threads read row M - 1): a load under a
    // branch is waited for at the branch's end.  The position goes first, so the RoPE
    // angles that need it wait only for it.
    const int store_m = tid / (kSmallCols / 4), n = nb + 4 * (tid % (kSmallCols / 4));
    const bool storer = tid < M * (kSmallCols / 4);
    const T* const stand_in = (const T*)sg.w;
    const int32_t* const pl = a.pos_lens ? a.pos_lens : (const int32_t*)stand_in;
    const int32_t pl_m = pl[min(store_m, M - 1)];
    V w[NB];
    auto load_batch = [&](int r0) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int k = min(r0 + j * RPI + lr, K - 1);
            w[j] = *(const V*)(W + (size_t)k * N + c * VEC);
        }
    };
    if (k_lo < k_hi) load_batch(k_lo);
    const T* __restrict__ bias = (const T*)sg.bias;
    const T* const bp = bias ? bias : stand_in;
    float bv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) bv[e] = to_f(bp[n + e]);   // n + 3 < N: segments are whole tiles
    // Every X load is issued before the first LDS store, so they share the W loads'
    // round trip.
    constexpr int XPT = kSmallMaxX / kThreads;
    const T* __restrict__ xg = (const T*)a.x;
    const int nx = M * K;
    T xv[XPT];
#pragma unroll
    for (int j = 0; j < XPT; j++) xv[j] = xg[min(tid + j * kThreads, nx - 1)];
    const int64_t pos = a.pos_lens ? (int64_t)pl_m : a.pos_uniform;
    const bool rotate = a.rope_table && ((a.rope_segs >> seg) & 1) && pos >= 0 && pos < a.rope_rows;
    // n is a multiple of 4 and rope_d is even, so (n, n+1) and (n+2, n+3) are pairs.
    const int rd = a.rope_table ? a.rope_d : 2;
    const float2* tb = a.rope_table ? (const float2*)a.rope_table + (rotate ? pos : 0) * (rd >> 1)
                                    : (const float2*)stand_in;
    const float2 c0 = tb[(n - fastdiv(n, t.div_rd) * rd) >> 1], c1 = tb[(n + 2 - fastdiv(n + 2, t.div_rd) * rd) >> 1];
    const float2 rot[2] = {rotate ? c0 : float2{1.f, 0.f}, rotate ? c1 : float2{1.f, 0.f}};
#pragma unroll
    for (int j = 0; j < XPT; j++)
        if (tid + j * kThreads < nx) xs[tid + j * kThreads] = to_f(xv[j]);
    __syncthreads();
    float acc[kSmallMaxM][VEC];
#pragma unroll
    for (int m = 0; m < kSmallMaxM; m++)
#pragma unroll
        for (int v = 0; v < VEC; v++) acc[m][v] = 0.0f;
    for (int r0 = k_lo; r0 < k_hi; r0 += NB * RPI) {
        if (r0 != k_lo) load_batch(r0);
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int k = r0 + j * RPI + lr;
            if (k < k_hi) {
#pragma unroll
                for (int m = 0; m < kSmallMaxM; m++) {
                    if (m >= M) break;
                    const float xv = xs[m * K + k];
#pragma unroll
                    for (int v = 0; v < VEC; v++) acc[m][v] = __builtin_fmaf(to_f(w[j][v]), xv, acc[m][v]);
                }
            }
        }
    }
    // Sum over the rows of the wave (lanes with the same column group c = lane % LPR):
    // inside each 16-lane row by DPP rotations of LPR, 2 LPR, .. 8 lanes, then across rows
    // with the row swaps (no LDS round trip); lanes lr == 0 store the wave's 16 column
    // sums per batch row.
    static_assert(LPR == 2 || LPR == 4, "column groups");
#pragma unroll
    for (int m = 0; m < kSmallMaxM; m++) {
        if (m >= M) break;
#pragma unroll
        for (int v = 0; v < VEC; v++) {
            float x = acc[m][v];
            if constexpr (LPR == 2) x += dpp_f<kDppRor + 2>(x);
            x += dpp_f<kDppRor + 4>(x);
            x += dpp_f<kDppRor + 8>(x);
            x = add_xor32(add_xor16(x));
            if (lr == 0) wsum[wave][m][c * VEC + v] = x;
        }
    }
    __syncthreads();
    advance_lengths(a);
    if (!storer) return;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float x = 0.0f;
#pragma unroll
        for (int q = 0; q < kWaves; q++) x += wsum[q][store_m][n - nb + e];
        v[e] = bias ? x + bv[e] : x;
    }
    if (rotate) {
        rotate_pair(v[0], v[1], rot[0]);
        rotate_pair(v[2], v[3], rot[1]);
    }
    if (pos_ok(a, sg, pos)) {
        T* out = (T*)sg.out + (size_t)store_m * sg.ld_m + (size_t)(sg.ld_pos ? pos : 0) * sg.ld_pos + n;
#pragma unroll
        for (int e = 0; e < 4; e++) out[e] = from_f<T>(v[e]);
    }
}

int g_small = 1;    // 0: never take gemv_small; 1: for small weights; 2: wherever it applies

int small_ok(const cf_gemv_args_t* a) {
    if (g_small == 0 || a->M > kSmallMaxM || (long long)a->M * a->K > kSmallMaxX) return 0;
    if (((uintptr_t)a->x) % 4 != 0) return 0;
    const long long esz = a->elem == CF_ELEM_F16 ? 2 : 4;
    long long bytes = 0;
    for (int s = 0; s < a->nseg; s++) {
        if (a->seg[s].n % kSmallCols != 0 || ((uintptr_t)a->seg[s].w) % 16 != 0) return 0;
        bytes += (long long)a->K * a->seg[s].n * esz;
    }
    return g_small == 2 || bytes <= kSmallMaxBytes;
}

Tiles make_tiles(const cf_gemv_args_t* a) {
    Tiles t{};
    if (small_ok(a)) {
        t.small = 1;
        t.bn = kSmallCols;
        int acc = 0;
        for (int s = 0; s < a->nseg; s++) {
            t.start[s] = acc;
            acc += (int)(a->seg[s].n / kSmallCols);
        }
        for (int s = a->nseg; s <= CF_GEMV_MAX_SEGS; s++) t.start[s] = acc;
        t.ks = 1;
        t.k_chunk = a->K;
        t.vec_ok = 1;
        return t;
    }
    const int bn = dma_bn(a);
    t.dma = bn;
    t.bn = bn ? bn : kColTile;
    int acc = 0;
    for (int s = 0; s < a->nseg; s++) {
        t.start[s] = acc;
        acc += (int)((a->seg[s].n + t.bn - 1) / t.bn);
    }
    for (int s = a->nseg; s <= CF_GEMV_MAX_SEGS; s++) t.start[s] = acc;
    const int kstep = bn ? kDK : (a->elem == CF_ELEM_F16 ? Cfg<_Float16>::KSTEP : Cfg<float>::KSTEP);
    int ks;
    if (bn) {
        // Enough one-wave workgroups per CU for the ring depth of this tile width: the
        // largest split whose workgroups give every CU the same count in one round
        // (config 2's output projection: 16 chunks, 512 workgroups, measured 1 us faster
        // on the op than 22 chunks, 704 workgroups, 2 or 3 per CU), else as many as
        // fill the ring slots.
        const int per_cu = bn == 64 ? Dma<64>::PER_CU : bn == 128 ? Dma<128>::PER_CU : Dma<256>::PER_CU;
        const int m_tiles = (a->M + kMTile - 1) / kMTile;
        const int units = acc * m_tiles;
        const int cus = cu_count();
        const int kmax = min(kMaxKSplit, a->K / kDK);
        ks = 0;
        for (int s = kmax; s >= 1 && !ks; s--) {
            const int chunk = ((a->K + s - 1) / s + kDK - 1) / kDK * kDK;
            const long long wgs = (long long)units * ((a->K + chunk - 1) / chunk);
            if (wgs <= (long long)per_cu * cus && wgs % cus == 0) ks = (a->K + chunk - 1) / chunk;
        }
        if (!ks) ks = min((per_cu * cus + units - 1) / units, a->K / kDK);
        if (g_dma_ks > 0) ks = g_dma_ks;
        if (ks < 1) ks = 1;
    } else {
        ks = a->k_split > 0 ? a->k_split : 1;
    }
    if (ks > kMaxKSplit) ks = kMaxKSplit;
    int chunk = (a->K + ks - 1) / ks;
    chunk = (chunk + kstep - 1) / kstep * kstep;
    t.k_chunk = chunk;
    t.ks = (a->K + chunk - 1) / chunk;   // every chunk non-empty
    const int vec = a->elem == CF_ELEM_F16 ? 8 : 4;
    int ok = (a->K % vec == 0) && (((uintptr_t)a->x) % 16 == 0);
    for (int s = 0; s < a->nseg; s++)
        ok = ok && (a->seg[s].n % vec == 0) && (((uintptr_t)a->seg[s].w) % 16 == 0);
    t.vec_ok = ok;
    return t;
}

}  // namespace

extern "C" int32_t cf_gemv_col_tile(int32_t elem) { (void)elem; return kColTile; }
extern "C" void cf_gemv_set_dma_tile(int32_t bn) { g_dma_bn = bn; }
extern "C" void cf_gemv_set_dma_ksplit(int32_t ks) { g_dma_ks = ks; }
extern "C" void cf_gemv_set_small(int32_t mode) { g_small = mode >= 0 && mode <= 2 ? mode : 1; }
extern "C" int32_t cf_gemv_fuses_rope(const cf_gemv_args_t* a) {
    const Tiles t = make_tiles(a);
    return t.small || t.ks > 1 ? 1 : 0;
}
extern "C" int32_t cf_gemv_k_step(int32_t elem) {
    return elem == CF_ELEM_F16 ? Cfg<_Float16>::KSTEP : Cfg<float>::KSTEP;
}

extern "C" size_t cf_gemv_partials_floats(const cf_gemv_args_t* a) {
    const Tiles t = make_tiles(a);
    if (t.ks <= 1) return 0;
    return (size_t)t.ks * (size_t)a->M * (size_t)t.start[a->nseg] * t.bn;
}

extern "C" int cf_launch_gemv(const cf_gemv_args_t* a, void* stream) {
    const Tiles t = make_tiles(a);
    if (a->M <= 0 || a->K <= 0 || t.start[a->nseg] <= 0) return (int)hipErrorInvalidValue;
    // RoPE is applied in the K-chunk sum or the one-pass small kernel only.
    if (a->rope_table && ((t.ks == 1 && !t.small) || a->rope_d <= 0 || (a->rope_d & 1)))
        return (int)hipErrorInvalidValue;
    cf_gemv_args_t args = *a;
    args.k_split = t.ks;
    hipStream_t s = (hipStream_t)stream;
    if (t.small) {
        Tiles ts = t;
        ts.div_rd = fastdiv_make(a->rope_table ? (int)a->rope_d : 2);
        if (a->elem == CF_ELEM_F16)
            hipLaunchKernelGGL(gemv_small<_Float16>, dim3((unsigned)t.start[a->nseg]), dim3(kThreads), 0, s, args, ts);
        else
            hipLaunchKernelGGL(gemv_small<float>, dim3((unsigned)t.start[a->nseg]), dim3(kThreads), 0, s, args, ts);
        return (int)hipGetLastError();
    }
    const int m_tiles = (a->M + kMTile - 1) / kMTile;
    dim3 grid((unsigned)t.start[a->nseg], (unsigned)t.ks, (unsigned)m_tiles);
    if (t.dma == 256)
        hipLaunchKernelGGL(gemv_f16_dma<256>, grid, dim3(64), 0, s, args, t);
    else if (t.dma == 128)
        hipLaunchKernelGGL(gemv_f16_dma<128>, grid, dim3(64), 0, s, args, t);
    else if (t.dma == 64)
        hipLaunchKernelGGL(gemv_f16_dma<64>, grid, dim3(64), 0, s, args, t);
    else if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(gemv_kernel<_Float16>, grid, dim3(kThreads), 0, s, args, t);
    else
        hipLaunchKernelGGL(gemv_kernel<float>, grid, dim3(kThreads), 0, s, args, t);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || t.ks == 1) return (int)e;
    // A wave per (column tile, kReduceThreads / (bn / 4) rows).
    const int rpw = kReduceThreads / (t.bn / 4);
    const dim3 rgrid((unsigned)(t.start[a->nseg] * ((a->M + rpw - 1) / rpw)));
    Tiles tr = t;
    tr.div_tiles = fastdiv_make(t.start[a->nseg]);
    tr.div_lpr = fastdiv_make(t.bn / 4);
    tr.div_rd = fastdiv_make(a->rope_table ? (int)a->rope_d : 2);
    auto reduce = [&](auto ks_c) {
        constexpr int KS = decltype(ks_c)::value;
        if (a->elem == CF_ELEM_F16)
            hipLaunchKernelGGL((gemv_reduce4<_Float16, KS>), rgrid, dim3(kReduceThreads), 0, s, args, tr);
        else
            hipLaunchKernelGGL((gemv_reduce4<float, KS>), rgrid, dim3(kReduceThreads), 0, s, args, tr);
    };
    if (t.ks <= 4) reduce(std::integral_constant<int, 4>{});
    else if (t.ks <= 8) reduce(std::integral_constant<int, 8>{});
    else if (t.ks <= 16) reduce(std::integral_constant<int, 16>{});
    else reduce(std::integral_constant<int, kMaxKSplit>{});
    return (int)hipGetLastError();
}
