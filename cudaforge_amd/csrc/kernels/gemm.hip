// gemm.hip — prefill projections of MHA_Fused on the matrix cores (gfx950).
//
// C = A·W + bias (+ residual) with A (M, K) row-major and W (K, N) row-major, the
// layout of the reference's "x·W" projections (mha_fused.c:68-88 and :152-171).
// The epilogue either writes C row-major or scatters the Q | K | V column segments into
// head-major buffers for the attention kernel: q (B,H_q,S,d), k (B,H_kv,S,d) and V
// transposed, vt (B,H_kv,d,S), so attention reads keys contiguously for P·V.
//
// fp16: 128x128 workgroup tile, 4 waves as 2x2, each wave 64x64 = 4x4 tiles of
//       v_mfma_f32_16x16x32_f16.  Both operands are staged in LDS in their natural
//       global layout (A as [m][k], W as [k][n]).  The MFMA B operand needs 8 consecutive
//       k of one column per lane; it comes from W[k][n] with two ds_read_b64_tr_b16
//       (gfx950 LDS transpose reads): in each 16-lane group, lane j addresses
//       W[kb + j/4][nb + 4(j%4)] and lane i receives W[kb..kb+3][nb + i].
//       Full tiles use an LDS ring filled by global_load_lds_dwordx4 (no VGPR staging):
//       3 stages of 32 k, i.e. three workgroups per CU, when there are more tiles than
//       two per CU, else 2 stages of 64 k; it stores straight from the accumulators,
//       16 bytes per lane after a permlane swap between neighbouring tiles.  Edge shapes
//       use a 2-stage register-staged kernel whose output tile goes through LDS (fp16 in
//       one pass without a residual, fp32 in two with one) so stores are 16 bytes along
//       the destination's contiguous direction.
// fp32: 128x128x16 tile with v_mfma_f32_16x16x4_f32, both tiles staged k-major so each
//       operand is one conflict-free ds_read_b32 (the FP32 operator's parity path).
// Tile edges are zero-filled on load and masked on store.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include <climits>

#include "kernels.h"
#include "cdna4.h"

namespace {

using namespace cdna4;

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128;

struct Tiling {
    int n_tiles_m;
    int seg_start[4];   // first column tile of each segment
    int a_vec;          // A rows may be read with vector loads (alignment and K)
    int w_vec[3];       // W rows of segment s may be read with vector loads
    int epi_vec;        // fp16 epilogue may use 8-element stores (alignment and shape)
    int group_m;        // tile rows per group of the XCD-aware tile order
    int n_tiles_n;      // column tiles (set_order)
    // Divisors of the tile order, fixed per launch (set_order): group_m * n_tiles_n,
    // group_m, and the last group's height n_tiles_m - (groups - 1) * group_m.
    FastDiv div_group, div_gm, div_gm_last;
};

// Fills the tile order's divisors; every launch of a kernel that calls tile_of_block
// sets them first (as runtime divisions they were ~75 scalar instructions of every
// workgroup's prologue).
inline void set_order(Tiling& t, int tiles_n) {
    t.n_tiles_n = tiles_n;
    const int gm = t.group_m > 0 ? t.group_m : 1;
    const int groups = (t.n_tiles_m + gm - 1) / gm;
    t.div_group = fastdiv_make(gm * tiles_n > 0 ? gm * tiles_n : 1);
    t.div_gm = fastdiv_make(gm);
    const int last = t.n_tiles_m - (groups - 1) * gm;
    t.div_gm_last = fastdiv_make(last > 0 ? last : 1);
}

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

// XCD-aware tile order.  Workgroup ids are dealt round-robin to MI355X's 8 XCDs, each
// with its own L2, so workgroup b runs on XCD b % 8.  XCD x receives a contiguous range
// of the tile order, and inside it tiles go column-major over groups of kGroupM tile
// rows: the workgroups an XCD runs together share A row tiles and W column tiles in
// that XCD's L2 instead of fetching them from MALL/HBM once per workgroup.
constexpr int kXcds = 8;
constexpr int kGroupM = 4;

__device__ __forceinline__ void tile_of_block(int blk, const Tiling& tl, int& tm, int& tn) {
    const int tiles_m = tl.n_tiles_m, tiles_n = tl.n_tiles_n, group_m = tl.group_m;
    const int T = tiles_m * tiles_n;
    const int x = blk % kXcds, j = blk / kXcds;
    const int base = T / kXcds, rem = T % kXcds;
    const int t = x * base + min(x, rem) + j;      // position in the tile order
    const int per_group = group_m * tiles_n;
    const int g = fastdiv(t, tl.div_group);
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int r = t - g * per_group;
    const int q = gm == group_m ? fastdiv(r, tl.div_gm) : fastdiv(r, tl.div_gm_last);
    tm = first_m + (r - q * gm);
    tn = q;
}

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
template <typename T, int NJ = 4>
__device__ __forceinline__ void store_tile(const cf_gemm_args_t& a, int seg, int N, int m0, int n0,
                                           int lr, int lq, const f4_t (&acc)[4][NJ]) {
    const T* __restrict__ bias = (const T*)a.bias[seg];
    const T* __restrict__ res = a.out_kind == CF_GEMM_OUT_ROWMAJOR ? (const T*)a.residual : nullptr;
    T* __restrict__ out = (T*)a.out[seg];
    size_t cp[NJ];
    float bv[NJ];
    bool nok[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
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
            for (int j = 0; j < NJ; j++) {
                if (!nok[j]) continue;
                float v = acc[i][j][e] + bv[j];
                if (res) v += to_f(res[rp + cp[j]]);
                out[rp + cp[j]] = from_f<T>(v);
            }
        }
}

// ------------------------------------------------------------------------- fp16 ---
// Epilogue shared by both fp16 kernels: the C tile goes through LDS in fp32, 64 rows at a
// time, so bias and residual are added before the single rounding to fp16, and stores
// are 16 bytes along the destination's contiguous direction (n for row-major / q / k,
// s for v^T).  `Cs` must hold 64 x (BN + 4) floats and be free (after a barrier).
constexpr int LDCF = BN + 4;
__device__ __forceinline__ void epilogue_f16(const cf_gemm_args_t& a, int seg, int N, int m0, int n0, int wm,
                                             int wn, int lr, int lq, int tid, const f4_t (&acc)[4][4],
                                             float* Cs) {
    const _Float16* __restrict__ bias = (const _Float16*)a.bias[seg];
    _Float16* __restrict__ out = (_Float16*)a.out[seg];
    const _Float16* __restrict__ res = a.out_kind == CF_GEMM_OUT_ROWMAJOR ? (const _Float16*)a.residual : nullptr;
    const bool along_n = a.out_kind == CF_GEMM_OUT_ROWMAJOR || seg < 2;
    for (int half = 0; half < 2; half++) {
        if (wm == 64 * half) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int nl = wn + 16 * j + lr;
                const float bv = (bias && n0 + nl < N) ? (float)bias[n0 + nl] : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) Cs[(16 * i + 4 * lq + e) * LDCF + nl] = acc[i][j][e] + bv;
            }
        }
        __syncthreads();
        const int mh = m0 + 64 * half;
#pragma unroll
        for (int it = 0; it < (64 * BN / 8) / kThreads; it++) {
            const int ch = tid + it * kThreads;
            h8_t v;
            if (along_n) {
                const int r = ch >> 4, c8 = (ch & 15) * 8;
                const int m = mh + r, n = n0 + c8;
                if (m >= a.M || n >= N) continue;
                const size_t off = row_part(a, seg, m) + col_part(a, seg, n);
                const f4_t lo = *(const f4_t*)&Cs[r * LDCF + c8], hi = *(const f4_t*)&Cs[r * LDCF + c8 + 4];
                float f[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                if (res) {
                    const h8_t rv = *(const h8_t*)(res + off);
#pragma unroll
                    for (int e = 0; e < 8; e++) f[e] += (float)rv[e];
                }
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (_Float16)f[e];
                *(h8_t*)(out + off) = v;
            } else {
                const int col = ch & (BN - 1), r8 = (ch / BN) * 8;
                const int m = mh + r8, n = n0 + col;
                if (m >= a.M || n >= N) continue;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (_Float16)Cs[(r8 + e) * LDCF + col];
                *(h8_t*)(out + row_part(a, seg, m) + col_part(a, seg, n)) = v;
            }
        }
        __syncthreads();
    }
}

// MFMA B operand (8 consecutive k of one column) from a W tile stored [k][n] in LDS:
// two ds_read_b64_tr_b16.  p points at W[kb + lr/4][nb + 4*(lr%4)] of the caller's
// lane; the second read is 4 rows further.
__device__ __forceinline__ h8_t b_frag_tr(const _Float16* p, const _Float16* p4) {
    const lds_h4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((CF_LDS lds_h4_t*)p);
    const lds_h4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((CF_LDS lds_h4_t*)p4);
    const h4_t l4 = __builtin_bit_cast(h4_t, lo), h4 = __builtin_bit_cast(h4_t, hi);
    return h8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
}

// ---- general kernel: any shape; registers stage the next k-tile (zero-filled edges).
constexpr int BK16 = 64;
constexpr int LDA16 = BK16 + 8;   // halves per A row in LDS
constexpr int LDW16 = BN + 8;     // halves per W row in LDS
constexpr int A_STAGE = BM * LDA16;
constexpr int W_STAGE = BK16 * LDW16;

__global__ __launch_bounds__(kThreads, 2)
void gemm_f16(cf_gemm_args_t a, Tiling t) {
    __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (A_STAGE + W_STAGE)];

    int tile_m, tile_n;
    tile_of_block(blockIdx.x, t, tile_m, tile_n);
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

    // A chunk c = tid + 256*i is row c>>3, k (c&7)*8; W chunk c is row (k) c>>4, column (c&15)*8.
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
                bf[j] = b_frag_tr(p, p + 4 * LDW16);
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
    if (t.epi_vec) epilogue_f16(a, seg, N, m0, n0, wm, wn, lr, lq, tid, acc, (float*)smem);
    else store_tile<_Float16>(a, seg, N, m0 + wm, n0 + wn, lr, lq, acc);
}

// Epilogues of the pipelined kernel, straight from the accumulators (no LDS pass).
// Full tiles only, with the alignment the launcher's epi_vec check implies (16 bytes).
// Each lane first holds four consecutive outputs of one 16x16 MFMA tile; a row swap
// with the lane 16 apart (v_permlane16_swap) between two neighbouring tiles gives each
// lane eight consecutive outputs, so the stores are 16 bytes (measured: 16-row x 32-byte
// 8-byte stores take ~1.7x as long as 16-row x 64-byte 16-byte ones for this output).
// After swap(a = tile B, b = tile A), even lane rows (lq = 0, 2) hold tile B's four
// values then the partner's next four, odd rows the partner's tile-A four then their own.
__device__ __forceinline__ uint2 pack4(float x0, float x1, float x2, float x3) {
    return __builtin_bit_cast(uint2, h4_t{(_Float16)x0, (_Float16)x1, (_Float16)x2, (_Float16)x3});
}

__device__ __forceinline__ void pair_swap(uint2& tb, uint2& ta) {
    float a0 = __builtin_bit_cast(float, tb.x), b0 = __builtin_bit_cast(float, ta.x);
    float a1 = __builtin_bit_cast(float, tb.y), b1 = __builtin_bit_cast(float, ta.y);
    swap_xor16(a0, b0);
    swap_xor16(a1, b1);
    tb = uint2{__builtin_bit_cast(uint32_t, a0), __builtin_bit_cast(uint32_t, a1)};
    ta = uint2{__builtin_bit_cast(uint32_t, b0), __builtin_bit_cast(uint32_t, b1)};
}

// Columns-contiguous destinations (row-major C, head-major q and k): the main loop
// accumulates C^T (MFMA operands swapped), so acc[i][j][e] = C[m][n + e] with
// m = m0 + wm + 16i + lr and n = n0 + wn + 16j + 4lq.  Tiles j = 2p, 2p+1 pair up; the
// lane then stores C[m][n0 + wn + 32p + 16 * (lq even) + 8 * (lq / 2) .. +7].  Bias, then
// the residual, are added in fp32 before the single rounding to fp16.
template <int NJ>
__device__ __forceinline__ void store_ct_f16(const cf_gemm_args_t& a, int seg, int m0, int n0, int wm, int wn,
                                             int lr, int lq, const f4_t (&acc)[4][NJ]) {
    const _Float16* __restrict__ bias = (const _Float16*)a.bias[seg];
    const _Float16* __restrict__ res = a.out_kind == CF_GEMM_OUT_ROWMAJOR ? (const _Float16*)a.residual : nullptr;
    _Float16* __restrict__ out = (_Float16*)a.out[seg];
    const bool odd = lq & 1;
    float bv[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int n = n0 + wn + 16 * j + 4 * lq;
#pragma unroll
        for (int e = 0; e < 4; e++) bv[j][e] = bias ? (float)bias[n + e] : 0.0f;
    }
    size_t cp[NJ / 2], cs = 0;
#pragma unroll
    for (int p = 0; p < NJ / 2; p++) cp[p] = col_part(a, seg, n0 + wn + 32 * p + (odd ? 0 : 16) + 8 * (lq >> 1));
    if constexpr (NJ % 2) cs = col_part(a, seg, n0 + wn + 16 * (NJ - 1) + 4 * lq);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + wm + 16 * i + lr;
        const size_t rp = row_part(a, seg, m);
        uint2 t[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            float f[4];
#pragma unroll
            for (int e = 0; e < 4; e++) f[e] = acc[i][j][e] + bv[j][e];
            if (res) {
                const h4_t r = *(const h4_t*)(res + rp + col_part(a, seg, n0 + wn + 16 * j + 4 * lq));
#pragma unroll
                for (int e = 0; e < 4; e++) f[e] += (float)r[e];
            }
            t[j] = pack4(f[0], f[1], f[2], f[3]);
        }
#pragma unroll
        for (int p = 0; p < NJ / 2; p++) {
            pair_swap(t[2 * p + 1], t[2 * p]);
            *(uint4*)(out + rp + cp[p]) = uint4{t[2 * p + 1].x, t[2 * p + 1].y, t[2 * p].x, t[2 * p].y};
        }
        // An odd last block has no partner: its four columns go out as 8 bytes.
        if constexpr (NJ % 2) *(uint2*)(out + rp + cs) = t[NJ - 1];
    }
}

// Rows-contiguous destination (v^T, (B, H_kv, d, S)): the main loop accumulates C, so
// acc[i][j][e] = C[m + e][n] with m = m0 + wm + 16i + 4lq and n = n0 + wn + 16j + lr: four
// consecutive positions s of one (head, dim) row of v^T.  Tiles i = 2p, 2p+1 pair up the
// same way, and the lane stores positions m0 + wm + 32p + 16 * (lq even) + 8 * (lq / 2) .. +7.
template <int NJ>
__device__ __forceinline__ void store_cn_f16(const cf_gemm_args_t& a, int seg, int m0, int n0, int wm, int wn,
                                             int lr, int lq, const f4_t (&acc)[4][NJ]) {
    const _Float16* __restrict__ bias = (const _Float16*)a.bias[seg];
    _Float16* __restrict__ out = (_Float16*)a.out[seg];
    const bool odd = lq & 1;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int n = n0 + wn + 16 * j + lr;
        const size_t cp = col_part(a, seg, n);
        const float bv = bias ? (float)bias[n] : 0.0f;
#pragma unroll
        for (int p = 0; p < 2; p++) {
            uint2 ta = pack4(acc[2 * p][j][0] + bv, acc[2 * p][j][1] + bv, acc[2 * p][j][2] + bv, acc[2 * p][j][3] + bv);
            uint2 tb = pack4(acc[2 * p + 1][j][0] + bv, acc[2 * p + 1][j][1] + bv, acc[2 * p + 1][j][2] + bv,
                             acc[2 * p + 1][j][3] + bv);
            pair_swap(tb, ta);
            const int m = m0 + wm + 32 * p + (odd ? 0 : 16) + 8 * (lq >> 1);
            *(uint4*)(out + row_part(a, seg, m) + cp) = uint4{tb.x, tb.y, ta.x, ta.y};
        }
    }
}

// ---- pipelined kernel: full tiles only (M % 128, N % BNT, K % BK == 0, aligned).
// STAGES LDS stages of BK k, filled by global_load_lds_dwordx4 (global -> LDS without
// VGPRs): STAGES-1 k-tiles are in flight while one is multiplied.  A lane-contiguous
// 1 KB of LDS per load instruction fixes the LDS layout, so the global side is
// permuted instead: the 16-byte chunk c of row r is stored at chunk c ^ swz(r), which
// makes the MFMA A reads (16 rows x one chunk) and the W transpose reads (4 rows x 32 B
// per 16-lane group) hit distinct banks.
// BNT = 128, 96 or 192 output columns per tile (waves 2 x 2, each 64 rows x BNT/2
// columns); the launcher takes 96 only where 128 leaves CUs idle, and 192 where it
// brings three tiles per CU down to two (fewer bytes loaded per flop on the busiest CU).
// BK = 32 or 64 k per stage.  An A row of a stage is BK * 2 bytes of one 128-byte line:
// at BK = 32 each load instruction reads half lines of 16 rows, and direct-to-LDS loads
// of half lines measured ~68 GB/s per CU from L2 against ~118 GB/s for whole lines (three
// workgroups per CU, 3-deep rings of 16 KB).  BK = 64 reads whole lines at twice the LDS
// per stage: 2 stages of 32 KB, two workgroups per CU.
constexpr int BKA = 32;

// A rows are BK * 2 bytes: 4 chunks (BK 32) or 8 (BK 64).  (row >> 1) & (chunks - 1) is
// the permutation under which the fragment reads (ds_read_b128, 16 rows x one chunk)
// measure conflict-free on gfx950 (SQ_LDS_BANK_CONFLICT) at BK 32; (row >> 2) & 3 and
// row & 3 both measure two-way conflicts.  At BK 64 the 16 rows of a read cover all
// (row & 1, chunk) pairs, i.e. the 16 distinct 16-byte bank slots of a 256-byte row.
template <int BK>
__device__ __forceinline__ int swz_a(int row) { return (row >> 1) & (BK / 8 - 1); }
// W rows are BNT * 2 bytes: 16 chunks (BNT = 128), 12 (96) or 24 (192).  The 96- and
// 192-column permutations flip chunk bits 1-2 only, so they stay inside the row's
// chunks.  At 96, rows 8 apart (read by the same half-wave) then sit 32 bytes apart in
// the banks.  A transpose read takes 32 bytes from each of 16 rows, 8r + 4h + 0..3 for
// r < 4, and the LDS serves it 32 lanes (8 rows, r = 0, 1 or r = 2, 3) at a time, so
// each half-wave's 8 rows must cover the 8 32-byte slots of the 256-byte bank window
// once.  At 192 a row is 384 bytes, so odd rows start half a window after even ones,
// and the even (and odd) rows x, x+2, x+8, x+10 of a half-wave take the four slots of
// their half through row bits 1 and 3.  (An earlier ((row >> 1) ^ (row >> 3)) & 3
// covered each slot twice per full wave but only half the slots per half-wave:
// SQ_LDS_BANK_CONFLICT counted 37 % of the LDS cycles of config 3's QKV product.)
// All three depend on row bits 0..4 only, so the rows of the second 32-k half of a
// BK = 64 stage (row + 32) are permuted like the first.
template <int BNT>
__device__ __forceinline__ int swz_w(int row) {
    if constexpr (BNT == 128) return ((row & 3) << 1) ^ (((row >> 3) & 1) << 3);
    else if constexpr (BNT == 192) return (((row >> 1) & 1) | ((row >> 2) & 2)) << 1;
    else return ((row >> 3) & 1) << 1;
}

// KSPLIT = 2: two groups of 4 waves split the k-loop of one tile, each with its own ring
// (dynamic LDS), and the second group's accumulators are added to the first's through
// LDS before the epilogue.  For grids of at most one tile per CU, where one 4-wave
// workgroup per CU leaves each SIMD a single wave to hide load and LDS latency.
template <int STAGES, int BNT, int BK, int KSPLIT = 1>
__global__ __launch_bounds__(kThreads * KSPLIT, 2 / KSPLIT)
void gemm_f16_async(cf_gemm_args_t a, Tiling t) {
    constexpr int A_ST = BM * BK;                   // halves per stage: A [128][BK]
    constexpr int W_ST = BK * BNT;                  // halves per stage: W [BK][BNT]
    constexpr int ST = A_ST + W_ST;
    constexpr int NJ = BNT / 32;                    // 16-column MFMA blocks per wave
    constexpr int KS = BK / 32;                     // MFMA k-steps per stage
    constexpr int A_CPR = BK / 8;                   // 16-byte chunks per A row
    constexpr int A_RPI = 64 / A_CPR;               // A rows per 1 KB load instruction
    constexpr int A_PW = BM * BK * 2 / 1024 / 4;    // A load instructions per wave per stage
    constexpr int W_INSTR = W_ST * 2 / 1024;        // W load instructions per stage
    constexpr int W_PW = (W_INSTR + 3) / 4;         // ... per wave, at most
    constexpr int CPR = BNT / 8;                    // 16-byte chunks per W row
    static_assert(BK == 32 || BK == 64, "stages are 32 or 64 k deep");
    static_assert(STAGES >= 2 && STAGES <= 4, "2 to 4 stages");
    static_assert(KSPLIT == 1 || KSPLIT == 2, "one or two k groups");
    __shared__ __attribute__((aligned(16))) _Float16 smem_s[KSPLIT == 1 ? STAGES * ST : 8];
    extern __shared__ __attribute__((aligned(16))) _Float16 smem_dyn[];
    const int kg = KSPLIT == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));   // k group
    _Float16* const smem = (KSPLIT == 1 ? smem_s : smem_dyn) + kg * STAGES * ST;

    int tile_m, tile_n;
    tile_of_block(blockIdx.x, t, tile_m, tile_n);
    const int seg = find_seg(a, t, tile_n);
    const int N = a.n[seg];
    const int K = a.K;
    const int m0 = tile_m * BM;
    const int n0 = (tile_n - t.seg_start[seg]) * BNT;
    // Group kg multiplies k in [kg * K / KSPLIT, (kg + 1) * K / KSPLIT) (the launcher
    // keeps K / BK a multiple of KSPLIT, so both groups run the same steps and barriers).
    const int k_begin = kg * (K / KSPLIT);
    const _Float16* __restrict__ A = (const _Float16*)a.a + k_begin;
    const _Float16* __restrict__ W = (const _Float16*)a.w[seg] + (size_t)k_begin * N;

    const int tid = threadIdx.x & (kThreads - 1), lane = tid & 63, wave = tid >> 6;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * (BNT / 2);
    const int lr = lane & 15, lq = lane >> 4;

    // Wave w fills A instructions u = A_PW*w .. A_PW*w + A_PW-1 (rows A_RPI*u ..; lane L
    // owns physical chunk L % A_CPR) and W instructions u = w, w + 4, ... (< W_INSTR) of
    // every stage; W instruction u covers the stage's chunks 64u .. 64u+63 in row-major
    // order.  Loads are a uniform base (the k-step's first column of A, first row of W)
    // plus per-lane byte offsets fixed for the whole loop (the launcher keeps M*K*2 and
    // K*N*2 below 2^32), so issuing them is scalar work.
    int nw = 0;                                     // W instructions of this wave
#pragma unroll
    for (int v = 0; v < W_PW; v++) nw += (wave + 4 * v < W_INSTR) ? 1 : 0;
    uint32_t a_off[A_PW], w_off[W_PW];
#pragma unroll
    for (int v = 0; v < A_PW; v++) {
        const int u = A_PW * wave + v;
        const int ra = A_RPI * u + lane / A_CPR, ca = (lane % A_CPR) ^ swz_a<BK>(ra);
        a_off[v] = ((uint32_t)(m0 + ra) * (uint32_t)K + 8u * (uint32_t)ca) * 2u;
    }
#pragma unroll
    for (int v = 0; v < W_PW; v++) {
        const int q = 64 * (wave + 4 * v) + lane;  // W chunk index in the stage
        const int rw = q / CPR, cw = (q % CPR) ^ swz_w<BNT>(rw);
        w_off[v] = ((uint32_t)rw * (uint32_t)N + (uint32_t)(n0 + 8 * cw)) * 2u;
    }
    const uint32_t wave_lds = __builtin_amdgcn_readfirstlane(lds_offset(smem) + (uint32_t)(A_PW * wave) * 1024u);
    const uint32_t wave_lds_w = __builtin_amdgcn_readfirstlane(lds_offset(smem) + (uint32_t)(A_ST * 2 + wave * 1024));
    auto issue = [&](int k0, auto stage_c) {
        constexpr int stage = decltype(stage_c)::value;
        const _Float16* ab = A + k0;
        const _Float16* wb = W + (size_t)k0 * N;
#pragma unroll
        for (int v = 0; v < A_PW; v++)
            lds_dma16_s(a_off[v], ab, wave_lds + (uint32_t)(stage * ST * 2 + v * 1024));
#pragma unroll
        for (int v = 0; v < W_PW; v++)
            if (v < nw) lds_dma16_s(w_off[v], wb, wave_lds_w + (uint32_t)(stage * ST * 2 + 4 * v * 1024));
    };

    f4_t acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    // Per-lane LDS read offsets inside a stage, for its k-step s (32 k each).
    int a_rd[KS][4], w_rd[NJ][2];
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = wm + 16 * i + lr;
            a_rd[s][i] = row * BK + 8 * ((4 * s + lq) ^ swz_a<BK>(row));
        }
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = 8 * lq + 4 * h + (lr >> 2);
            const int col = wn + 16 * j + 4 * (lr & 3);
            w_rd[j][h] = row * BNT + 8 * ((col >> 3) ^ swz_w<BNT>(row)) + (col & 7);
        }

    const int nk = K / BK / KSPLIT;
    if (0 < nk) issue(0, std::integral_constant<int, 0>{});
    if constexpr (STAGES > 2)
        if (1 < nk) issue(BK, std::integral_constant<int, 1>{});
    if constexpr (STAGES > 3)
        if (2 < nk) issue(2 * BK, std::integral_constant<int, 2>{});
    // CT: accumulate C^T (operands swapped) for destinations contiguous along n.
    auto main_loop = [&](auto ct_c) {
        constexpr bool CT = decltype(ct_c)::value;
        for_each_stage<STAGES>(nk, [&](int kt, auto stage_c) {
            constexpr int stage = decltype(stage_c)::value;        // kt % STAGES
            // Tiles issued after kt that may still be in flight: min(STAGES-2, nk-1-kt),
            // A_PW + nw load instructions each.
            if (nw == W_PW) wait_ahead<A_PW + W_PW, STAGES - 2>(nk - 1 - kt);
            else wait_ahead<A_PW + W_PW - 1, STAGES - 2>(nk - 1 - kt);
            ring_barrier();
            if (kt + STAGES - 1 < nk)
                issue((kt + STAGES - 1) * BK, std::integral_constant<int, (stage + STAGES - 1) % STAGES>{});
            const _Float16* As = smem + stage * ST;
            const _Float16* Ws = As + A_ST;
#pragma unroll
            for (int s = 0; s < KS; s++) {
                h8_t af[4], bf[NJ];
#pragma unroll
                for (int i = 0; i < 4; i++) af[i] = *(const h8_t*)&As[a_rd[s][i]];
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    bf[j] = b_frag_tr(Ws + 32 * s * BNT + w_rd[j][0], Ws + 32 * s * BNT + w_rd[j][1]);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[i][j] = CT ? __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], af[i], acc[i][j], 0, 0, 0)
                                       : __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        });
    };
    // Every DMA load was waited for in the last step, and the epilogue does not touch LDS.
    // With two k groups, group 1 hands its accumulators to group 0 through the (then
    // idle) rings: [wave][i][j][lane] as f4, 16 KB x NJ in all.
    auto reduce_groups = [&]() {
        if constexpr (KSPLIT == 2) {
            static_assert(4 * 4 * NJ * 64 * 16 <= 2 * STAGES * ST * 2, "the rings hold the partial tile");
            f4_t* red = (f4_t*)smem_dyn;
            ring_barrier();                                // every wave is done with both rings
            if (kg == 1) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++) red[((wave * 4 + i) * NJ + j) * 64 + lane] = acc[i][j];
                wait_lds_reads();                          // lgkmcnt(0): the writes are done
            }
            ring_barrier();
            if (kg == 0) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++) acc[i][j] += red[((wave * 4 + i) * NJ + j) * 64 + lane];
            }
        }
    };
    if (a.out_kind == CF_GEMM_OUT_ROWMAJOR || seg < 2) {
        main_loop(std::true_type{});
        reduce_groups();
        if (kg == 0) store_ct_f16<NJ>(a, seg, m0, n0, wm, wn, lr, lq, acc);
    } else {
        main_loop(std::false_type{});
        reduce_groups();
        if (kg == 0) store_cn_f16<NJ>(a, seg, m0, n0, wm, wn, lr, lq, acc);
    }
}

// ------------------------------------------------------------------------- fp32 ---
// 128 x BNT tiles (BNT = 128, or 96 where 128-column tiles leave CUs idle), k-tiles of
// 16 double-buffered in LDS: the next k-tile is loaded into registers while the current
// one is multiplied, then stored to the other buffer, one barrier per k-tile.  Both
// operands are stored k-major so each MFMA operand is one conflict-free ds_read_b32.
constexpr int BK32 = 16;
constexpr int LDM32 = BM + 4;     // floats per k-major LDS row of A

template <int BNT>
__global__ __launch_bounds__(kThreads, 2)
void gemm_f32(cf_gemm_args_t a, Tiling t) {
    constexpr int NJ = BNT / 32;                  // 16-column MFMA blocks per wave
    constexpr int LDN = BNT + 4;                  // floats per k-major LDS row of W
    constexpr int WCH = BK32 * BNT / 4;           // float4 chunks of a W k-tile
    constexpr int WPT = (WCH + kThreads - 1) / kThreads;
    __shared__ float As[2][BK32 * LDM32];   // [k][m]
    __shared__ float Bs[2][BK32 * LDN];     // [k][n]

    int tile_m, tile_n;
    tile_of_block(blockIdx.x, t, tile_m, tile_n);
    const int seg = find_seg(a, t, tile_n);
    const int N = a.n[seg];
    const int m0 = tile_m * BM;
    const int n0 = (tile_n - t.seg_start[seg]) * BNT;
    const float* __restrict__ A = (const float*)a.a;
    const float* __restrict__ W = (const float*)a.w[seg];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * (BNT / 2);
    const int lr = lane & 15, lq = lane >> 4;
    const bool a_vec = t.a_vec != 0;
    const bool w_vec = t.w_vec[seg] != 0;

    f4_t acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    // A: 128 rows x 16 k = 512 chunks of 4 (2 per thread); W: 16 k x BNT n (WPT per thread).
    f4_t ra[2], rw[WPT];
    auto load = [&](int k0) {
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
            ra[it] = v;
        }
#pragma unroll
        for (int it = 0; it < WPT; it++) {
            const int ch = tid + it * kThreads;
            const int kr = ch / (BNT / 4), nc = (ch % (BNT / 4)) * 4;
            const int gk = k0 + kr, gn = n0 + nc;
            f4_t v{};
            if (ch < WCH && gk < a.K) {
                const float* src = W + (size_t)gk * N + gn;
                if (w_vec && gn + 4 <= N) v = *(const f4_t*)src;
                else {
#pragma unroll
                    for (int e = 0; e < 4; e++) if (gn + e < N) v[e] = src[e];
                }
            }
            rw[it] = v;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const int ch = tid + it * kThreads;
            const int r = ch >> 2, kc = (ch & 3) * 4;
#pragma unroll
            for (int e = 0; e < 4; e++) As[buf][(kc + e) * LDM32 + r] = ra[it][e];
        }
#pragma unroll
        for (int it = 0; it < WPT; it++) {
            const int ch = tid + it * kThreads;
            if (ch < WCH) *(f4_t*)&Bs[buf][(ch / (BNT / 4)) * LDN + (ch % (BNT / 4)) * 4] = rw[it];
        }
    };

    const int nk = (a.K + BK32 - 1) / BK32;
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * BK32);
#pragma unroll
        for (int kk = 0; kk < BK32; kk += 4) {
            float af[4], bf[NJ];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = As[buf][(kk + lq) * LDM32 + wm + 16 * i + lr];
#pragma unroll
            for (int j = 0; j < NJ; j++) bf[j] = Bs[buf][(kk + lq) * LDN + wn + 16 * j + lr];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }
    store_tile<float, NJ>(a, seg, N, m0 + wm, n0 + wn, lr, lq, acc);
}

// ------------------------------------------------------ fp16, wave-specialised ---
// BM x BN tiles (BM = 256 or 128) of 8 waves: waves 4-7 only issue the direct-to-LDS
// loads, waves 0-3 only read LDS and run MFMAs, and one barrier per 64-k stage orders the
// two.  A wave that both issues a stage's DMA instructions and multiplies stalls at the
// issue (measured ~650 clocks of every stage) and its MFMAs never overlap the loads: a
// loop of MFMAs and DMA took the sum of the two alone.  Stages are 64 k deep so every A
// DMA instruction reads 8 rows x 128 B, whole cache lines: per CU the load path moves ~50
// B/clk for whole lines and ~15 B/clk for the 16 rows x 64 B that one MFMA fragment's
// rows are.  A rows in LDS are 128 B with chunk c of row r at c ^ ((r >> 1) & 7), so the
// A fragment reads (ds_read_b128, 16 rows x one chunk) are conflict-free; W rows (BN
// columns of one k) are padded by one 16-byte chunk, which the transposing B reads
// (ds_read_b64_tr_b16) measure at the ds_read_b64 rate.  A compute wave owns 64 rows x
// BN / NWN columns (NWN = 256 / BM waves along N).
//
// Columns are the concatenation of the segments (Q | K | V for the projection), and a
// tile may straddle a segment boundary: every 8-column chunk belongs to one segment (the
// launcher checks n[s] % 8), so loads and stores are routed per chunk.  The epilogue
// stages the tile in the (then idle) LDS, bias added in fp32 and, without a residual,
// rounded once to fp16; with a residual the fp32 sum is staged and the residual added
// before the single rounding, as in the other kernels.  All 8 waves then store 16-byte
// chunks: along n for row-major C and head-major q / k, along s (8 rows of one column,
// read down the staged column) for v^T.
constexpr int WS_BK = 64;

template <int BM, int BN>
struct WsShape {
    static constexpr int NWN = 256 / BM;           // compute waves along N
    static constexpr int WN = BN / NWN;            // columns per compute wave
    static constexpr int NJ = WN / 16;             // 16-column MFMA blocks per compute wave
    static constexpr int A_ST = BM * WS_BK;        // halves per stage of A
    static constexpr int WCPR = BN / 8 + 1;        // 16-byte chunks per padded W row
    static constexpr int LDW = WCPR * 8;           // halves per W row in LDS
    static constexpr int W_CH = WS_BK * WCPR;      // chunks per W stage
    static constexpr int W_INSTR = (W_CH + 63) / 64;
    static constexpr int W_ST = W_INSTR * 512;     // halves per stage of W (whole DMA instructions)
    static constexpr int ST = A_ST + W_ST;
    static constexpr int A_PW = A_ST * 2 / 1024 / 4;   // A DMA instructions per loader wave
    static constexpr int W_PW = (W_INSTR + 3) / 4;     // W DMA instructions per loader wave, at most
    static_assert(WN % 16 == 0 && BN % 8 == 0, "tile width");
};

template <int BM, int BN, int S>
constexpr unsigned ws_lds_bytes() { return (unsigned)S * WsShape<BM, BN>::ST * 2u; }

// What the epilogue reads of the launch arguments, loaded into registers at kernel start:
// reading them from the argument block after the main loop cost ~1 us per group of fields
// (config-3 QKV product, 22.8 -> 19 us without those late reads).
struct WsEpi {
    CF_GLOBAL _Float16* out0;
    CF_GLOBAL _Float16* out1;
    CF_GLOBAL _Float16* out2;
    const CF_GLOBAL _Float16* bias0;
    const CF_GLOBAL _Float16* bias1;
    const CF_GLOBAL _Float16* bias2;
    const CF_GLOBAL _Float16* res;
    int S, Hq, Hkv, d, n0w;
    // Per-segment pointers as the first one plus a selected distance: a select among the
    // pointers themselves is turned into an indexed load of the struct, which then lives
    // in scratch memory.
    __device__ CF_GLOBAL _Float16* out(int s) const {
        return out0 + (s == 1 ? out1 - out0 : (ptrdiff_t)0) + (s == 2 ? out2 - out0 : (ptrdiff_t)0);
    }
    __device__ const CF_GLOBAL _Float16* bias(int s) const {
        return bias0 + (s == 1 ? bias1 - bias0 : (ptrdiff_t)0) + (s == 2 ? bias2 - bias0 : (ptrdiff_t)0);
    }
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ WsEpi ws_epi(const cf_gemm_args_t& a) {
    WsEpi e;
    e.out0 = (CF_GLOBAL _Float16*)a.out[0];
    e.out1 = (CF_GLOBAL _Float16*)a.out[1];
    e.out2 = (CF_GLOBAL _Float16*)a.out[2];
    e.bias0 = (const CF_GLOBAL _Float16*)a.bias[0];
    e.bias1 = (const CF_GLOBAL _Float16*)a.bias[1];
    e.bias2 = (const CF_GLOBAL _Float16*)a.bias[2];
    e.res = (const CF_GLOBAL _Float16*)a.residual;
    e.S = a.S;
    e.Hq = a.H_q;
    e.Hkv = a.H_kv;
    e.d = a.d;
    e.n0w = a.out_kind == CF_GEMM_OUT_ROWCAT ? a.n[0] + a.n[1] + a.n[2] : a.n[0];
    // Empty asm that "modifies" every field: the loads happen here, not where first used.
    asm volatile("" : "+s"(e.out0), "+s"(e.out1), "+s"(e.out2), "+s"(e.bias0), "+s"(e.bias1), "+s"(e.bias2),
                 "+s"(e.res));
    asm volatile("" : "+s"(e.S), "+s"(e.Hq), "+s"(e.Hkv), "+s"(e.d), "+s"(e.n0w));
    return e;
}
#pragma clang diagnostic pop

// Destination offsets of gemm_f16_ws's Q|K|V scatter (row_part + col_part) without an
// integer division per chunk: the tile's first row is split into (batch, position) once
// per thread and a row r rows further carries over at most a few sequence ends; a
// power-of-two head size splits columns with a shift (the split by division measured
// ~1 us of the config-3 QKV product).
struct WsRows {
    int m0, b0, s0;       // the tile's first row and its (batch, position)
    int dsh;              // log2(d) when d is a power of two, else -1
};
__device__ __forceinline__ WsRows ws_rows(const WsEpi& e, int m0) {
    WsRows w;
    w.m0 = m0;
    w.b0 = m0 / e.S;
    w.s0 = m0 - w.b0 * e.S;
    w.dsh = (e.d & (e.d - 1)) == 0 ? __builtin_ctz(e.d) : -1;
    return w;
}
__device__ __forceinline__ size_t ws_qkv_off(const WsEpi& e, const WsRows& w, int seg, int m, int n) {
    int s = w.s0 + (m - w.m0), b = w.b0;
    while (s >= e.S) {
        s -= e.S;
        ++b;
    }
    const int H = seg == 0 ? e.Hq : e.Hkv;
    if (seg == 2) return (size_t)b * H * e.d * e.S + s + (size_t)n * e.S;
    const int h = w.dsh >= 0 ? n >> w.dsh : n / e.d;
    return ((size_t)b * H * e.S + s) * e.d + (size_t)h * e.S * e.d + (n - h * e.d);
}

// Segment of concatenated column gc (a multiple of 8) and its column inside it.
__device__ __forceinline__ int ws_seg_n(int nseg, const int (&start)[4], int gc, int& col) {
    const int s = (nseg > 1 && gc >= start[1]) ? ((nseg > 2 && gc >= start[2]) ? 2 : 1) : 0;
    col = gc - start[s];
    return s;
}
__device__ __forceinline__ int ws_seg(const cf_gemm_args_t& a, const int (&start)[4], int gc, int& col) {
    return ws_seg_n(a.nseg, start, gc, col);
}

// Epilogue kinds of gemm_f16_ws, a template parameter so that each launch carries only its
// own staging and store code (a run-time switch between them measured ~1 us per switch
// on the config-3 QKV product).
enum { WS_EPI_ROWMAJOR = 0, WS_EPI_RESIDUAL = 1, WS_EPI_QKV = 2 };

template <int BM, int BN, int EPI>
__device__ __forceinline__ void ws_store(const WsEpi& e, const int (&start)[4], int nseg, int m0, int n0, int tid,
                                         const _Float16* smem, bool vt_tile);

template <int BM, int BN, int S, int EPI>
__global__ __launch_bounds__(512, 1)
void gemm_f16_ws(cf_gemm_args_t a, Tiling t) {
    using SH = WsShape<BM, BN>;
    constexpr int NJ = SH::NJ, A_ST = SH::A_ST, LDW = SH::LDW, ST = SH::ST, A_PW = SH::A_PW, W_PW = SH::W_PW;
    constexpr int WCPR = SH::WCPR, W_CH = SH::W_CH, W_INSTR = SH::W_INSTR;
    extern __shared__ __attribute__((aligned(16))) _Float16 smem_ws[];
    _Float16* const smem = smem_ws;

    const WsEpi epi = ws_epi(a);
    // Column space: segment s covers [start[s], start[s] + n[s]).
    int start[4];
    start[0] = 0;
    start[1] = a.n[0];
    start[2] = a.n[0] + (a.nseg > 1 ? a.n[1] : 0);
    start[3] = start[2] + (a.nseg > 2 ? a.n[2] : 0);
    int tile_m, tile_n;
    tile_of_block(blockIdx.x, t, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int K = a.K, nk = K / WS_BK;
    // Every column of the tile goes to v^T: accumulate C and stage it column-major.
    const bool vt_tile = EPI == WS_EPI_QKV && a.nseg == 3 && n0 >= start[2];
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lq = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cw = wave & 3;

    if (wave >= 4) {
        // Loader waves.  A: instruction u of a stage covers rows 8u .. 8u+7 (lane L: row
        // 8u + L/8, stored chunk L%8 holding k-chunk (L%8) ^ swz(row)), a uniform base (the
        // stage's first k) plus per-lane 32-bit offsets.  W: instruction u covers padded
        // chunks 64u .. 64u+63 of the stage; a lane keeps its chunk's 64-bit address and
        // steps it by 64 rows of its segment per stage (pad chunks re-read the row's last).
        const _Float16* __restrict__ A = (const _Float16*)a.a;
        uint32_t a_off[A_PW];
#pragma unroll
        for (int v = 0; v < A_PW; v++) {
            const int row = 8 * (A_PW * cw + v) + (lane >> 3), pc = lane & 7;
            a_off[v] = ((uint32_t)(m0 + row) * (uint32_t)K + 8u * (uint32_t)(pc ^ ((row >> 1) & 7))) * 2u;
        }
        const _Float16* w_ptr[W_PW];
        uint32_t w_step[W_PW];
        int nw = 0;
        // A chunk's segment, base, width and first column.  A tile inside one segment
        // takes them wave-uniform; a tile over two segments picks one of two uniform sets
        // per chunk by one compare against the boundary; only a tile over three (segments
        // narrower than a tile) makes the three-way choice per chunk, whose selects and
        // 64-bit arithmetic, done for every tile, had delayed every product's first W
        // loads.  Pointers are selected, never indexed per lane: a per-lane index into the
        // argument block would move it to scratch memory.
        const _Float16* const wb0 = (const _Float16*)a.w[0];
        const _Float16* const wb1 = a.nseg > 1 ? (const _Float16*)a.w[1] : wb0;
        const _Float16* const wb2 = a.nseg > 2 ? (const _Float16*)a.w[2] : wb1;
        const int ns0 = a.n[0], ns1 = a.nseg > 1 ? a.n[1] : ns0, ns2 = a.nseg > 2 ? a.n[2] : ns1;
        const int st1 = a.nseg > 1 ? start[1] : INT_MAX, st2 = a.nseg > 2 ? start[2] : INT_MAX;
        const int last = n0 + BN - 8;
        const int s_lo = n0 >= st2 ? 2 : n0 >= st1 ? 1 : 0, s_hi = last >= st2 ? 2 : last >= st1 ? 1 : 0;
        if (s_hi == s_lo) {
            // One segment (every tile of a one-segment product, most of a Q|K|V one):
            // wave-uniform base, width and start.
            const _Float16* const wb = s_lo == 2 ? wb2 : s_lo == 1 ? wb1 : wb0;
            const int ns = s_lo == 2 ? ns2 : s_lo == 1 ? ns1 : ns0;
            const int st = s_lo == 2 ? st2 : s_lo == 1 ? st1 : 0;
#pragma unroll
            for (int v = 0; v < W_PW; v++) {
                const int u = cw + 4 * v;
                nw += u < W_INSTR ? 1 : 0;
                const int q = min(64 * u + lane, W_CH - 1);
                const int r = q / WCPR, c = min(q - r * WCPR, BN / 8 - 1);
                w_ptr[v] = wb + ((size_t)r * ns + (n0 + 8 * c - st));
                w_step[v] = (uint32_t)(WS_BK * ns);
            }
        } else if (s_hi - s_lo == 1) {
            const _Float16* const wlo = s_lo == 2 ? wb2 : s_lo == 1 ? wb1 : wb0;
            const _Float16* const whi = s_hi == 2 ? wb2 : s_hi == 1 ? wb1 : wb0;
            const int nlo = s_lo == 2 ? ns2 : s_lo == 1 ? ns1 : ns0, nhi = s_hi == 2 ? ns2 : s_hi == 1 ? ns1 : ns0;
            const int slo = s_lo == 2 ? st2 : s_lo == 1 ? st1 : 0;
            const int shi = s_hi == s_lo ? INT_MAX : s_hi == 2 ? st2 : st1;   // the boundary, if any
#pragma unroll
            for (int v = 0; v < W_PW; v++) {
                const int u = cw + 4 * v;
                nw += u < W_INSTR ? 1 : 0;
                const int q = min(64 * u + lane, W_CH - 1);
                const int r = q / WCPR, c = min(q - r * WCPR, BN / 8 - 1);
                const int gc = n0 + 8 * c;
                const bool hi = gc >= shi;
                const int ns = hi ? nhi : nlo;
                w_ptr[v] = (hi ? whi : wlo) + ((size_t)r * ns + (gc - (hi ? shi : slo)));
                w_step[v] = (uint32_t)(WS_BK * ns);
            }
        } else {
#pragma unroll
            for (int v = 0; v < W_PW; v++) {
                const int u = cw + 4 * v;
                nw += u < W_INSTR ? 1 : 0;
                const int q = min(64 * u + lane, W_CH - 1);
                const int r = q / WCPR, c = min(q - r * WCPR, BN / 8 - 1);
                const int gc = n0 + 8 * c;
                const bool in1 = gc >= st1, in2 = gc >= st2;     // start[2] >= start[1]: in2 implies in1
                const int ns = in2 ? ns2 : in1 ? ns1 : ns0;
                w_ptr[v] = (in2 ? wb2 : in1 ? wb1 : wb0) + ((size_t)r * ns + (gc - (in2 ? st2 : in1 ? st1 : 0)));
                w_step[v] = (uint32_t)(WS_BK * ns);
            }
        }
        const uint32_t lds0 = lds_offset(smem);
        const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(A_PW * cw) * 1024u);
        const uint32_t w_lds = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)A_ST * 2u + (uint32_t)cw * 1024u);
        auto issue = [&](int kt, int stage) {
            const _Float16* ab = A + kt * WS_BK;
            const uint32_t so = (uint32_t)stage * ST * 2u;
#pragma unroll
            for (int v = 0; v < A_PW; v++) lds_dma16_s(a_off[v], ab, a_lds + so + v * 1024u);
#pragma unroll
            for (int v = 0; v < W_PW; v++)
                if (v < nw) {
                    lds_dma16(w_ptr[v], w_lds + so + 4u * v * 1024u);
                    w_ptr[v] += w_step[v];
                }
        };
        for (int s = 0; s < S - 1 && s < nk; s++) issue(s, s);
        if (nw == W_PW) wait_ahead<A_PW + W_PW, S - 2>(min(S - 2, nk - 1));
        else wait_ahead<A_PW + W_PW - 1, S - 2>(min(S - 2, nk - 1));
        ring_barrier();
        for_each_stage<S>(nk, [&](int kt, auto stage_c) {
            constexpr int stage = decltype(stage_c)::value;
            // Stage (kt - 1) % S was read in step kt - 1, finished before this barrier.
            if (kt + S - 1 < nk) issue(kt + S - 1, (stage + S - 1) % S);
            // Stage kt + 1 is complete at the next barrier; later ones may stay in flight.
            if (kt + 1 < nk) {
                const int after = min(S - 2, nk - 2 - kt);
                if (nw == W_PW) wait_ahead<A_PW + W_PW, S - 2>(after);
                else wait_ahead<A_PW + W_PW - 1, S - 2>(after);
            }
            ring_barrier();
        });
    } else {
        // Compute waves: rows wm .. wm+63, columns wn .. wn + BN/NWN - 1 of the tile.
        const int wm = 64 * (cw % (4 / SH::NWN)), wn = SH::WN * (cw / (4 / SH::NWN));
        int a_rd[2][4], w_rd[2];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = wm + 16 * i + lr;
                a_rd[h][i] = row * WS_BK + 8 * ((4 * h + lq) ^ ((row >> 1) & 7));
            }
#pragma unroll
        for (int e = 0; e < 2; e++) w_rd[e] = A_ST + (8 * lq + 4 * e + (lr >> 2)) * LDW + wn + 4 * (lr & 3);
        // CT: accumulate C^T (operands swapped), acc[i][j][e] = C[wm + 16i + lr][wn + 16j + 4lq + e],
        // for destinations contiguous along n; otherwise C, acc[i][j][e] = C[wm + 16i + 4lq + e]
        // [wn + 16j + lr], for tiles whose every column goes to v^T (contiguous along s).
        auto run = [&](auto ct_c) {
            constexpr bool CT = decltype(ct_c)::value;
            // The epilogue's bias values (CT: four columns of one segment per lane and j;
            // v^T tiles: column n's value), loaded before the main loop so that their round
            // trip is not paid after it (config-3 QKV product: ~1 us), except for the
            // scatter epilogue, whose widest tile would then spill registers.
            h4_t b4[NJ];
            _Float16 bc[NJ];
            auto load_bias = [&]() {
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    if constexpr (CT) {
                        int col;
                        const int sg = ws_seg(a, start, n0 + wn + 16 * j + 4 * lq, col);
                        const CF_GLOBAL _Float16* bias = epi.bias(sg);
                        b4[j] = bias ? *(const CF_GLOBAL h4_t*)(bias + col) : h4_t{0, 0, 0, 0};
                    } else {
                        bc[j] = epi.bias2 ? epi.bias2[n0 + wn + 16 * j + lr - start[2]] : (_Float16)0;
                    }
                }
            };
            if constexpr (EPI != WS_EPI_QKV) load_bias();
            f4_t acc[4][NJ];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
            ring_barrier();
            for_each_stage<S>(nk, [&](int kt, auto stage_c) {
                constexpr int stage = decltype(stage_c)::value;
                const _Float16* st = smem + stage * ST;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    h8_t af[4], bf[NJ];
#pragma unroll
                    for (int i = 0; i < 4; i++) af[i] = *(const h8_t*)(st + a_rd[h][i]);
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        bf[j] = b_frag_tr(st + 32 * h * LDW + w_rd[0] + 16 * j, st + 32 * h * LDW + w_rd[1] + 16 * j);
#pragma unroll
                    for (int j = 0; j < NJ; j++)
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            acc[i][j] = CT ? __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], af[i], acc[i][j], 0, 0, 0)
                                           : __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
                ring_barrier();
            });
            if constexpr (EPI == WS_EPI_QKV) load_bias();
            if constexpr (CT) {
                // Stage [BM][BN]: bias added in fp32; fp16 (one rounding) without a residual,
                // fp32 with one.  A lane's four columns lie in one segment (n[s] % 8 == 0).
                constexpr bool f32s = EPI == WS_EPI_RESIDUAL;
#pragma unroll
                for (int j = 0; j < NJ; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = wm + 16 * i + lr, c = wn + 16 * j + 4 * lq;
                        const float v0 = acc[i][j][0] + (float)b4[j][0], v1 = acc[i][j][1] + (float)b4[j][1];
                        const float v2 = acc[i][j][2] + (float)b4[j][2], v3 = acc[i][j][3] + (float)b4[j][3];
                        if constexpr (f32s) *(f4_t*)((float*)smem + r * (BN + 4) + c) = f4_t{v0, v1, v2, v3};
                        else *(uint2*)(smem + r * (BN + 8) + c) = pack4(v0, v1, v2, v3);
                    }
            } else {
                // A v^T tile: stage [BM][BN] (column-major), bias of column n added in fp32.
#pragma unroll
                for (int j = 0; j < NJ; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float bv = (float)bc[j];
                        *(uint2*)(smem + (wn + 16 * j + lr) * (BM + 8) + wm + 16 * i + 4 * lq) =
                            pack4(acc[i][j][0] + bv, acc[i][j][1] + bv, acc[i][j][2] + bv, acc[i][j][3] + bv);
                    }
            }
        };
        if constexpr (EPI == WS_EPI_QKV) {
            if (vt_tile) run(std::false_type{});
            else run(std::true_type{});
        } else {
            run(std::true_type{});
        }
    }
    ring_barrier();   // every loader is past its last stage and the tile is staged
    ws_store<BM, BN, EPI>(epi, start, a.nseg, m0, n0, tid, smem, vt_tile);
}

// Store phase of gemm_f16_ws (all 512 threads): the staged tile goes out as 16-byte chunks,
// 8 columns of one row (row-major C, head-major q and k; consecutive threads along the
// row) or, for v^T columns, 8 rows of one column read down the staged column.  Each pass
// has a fixed trip count, and all of a thread's LDS reads are issued before its stores.
template <int BM, int BN, int EPI>
__device__ __forceinline__ void ws_store(const WsEpi& e, const int (&start)[4], int nseg, int m0, int n0, int tid,
                                         const _Float16* smem, bool vt_tile) {
    constexpr int CPR = BN / 8, NCH = BM * CPR, IT = (NCH + 511) / 512;
    constexpr bool qkv = EPI == WS_EPI_QKV;
    const WsRows wr = ws_rows(e, m0);
    if constexpr (EPI == WS_EPI_ROWMAJOR) {
        // Row-major C: consecutive threads along a row.
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int id = tid + 512 * it;
            if (id < NCH) {
                const int r = id / CPR, c8 = id - r * CPR;
                *(CF_GLOBAL h8_t*)(e.out0 + (size_t)(m0 + r) * e.n0w + n0 + 8 * c8) = *(const h8_t*)(smem + r * (BN + 8) + 8 * c8);
            }
        }
        return;
    }
    if (qkv && vt_tile) {
        // Staged [BN][BM + 8]: chunks of 8 consecutive rows (positions s) of one column.
        constexpr int RPC = BM / 8, NV = BN * RPC, ITV = (NV + 511) / 512;
        h8_t v[ITV];
        size_t off[ITV];
#pragma unroll
        for (int it = 0; it < ITV; it++) {
            const int id = min(tid + 512 * it, NV - 1), c = id / RPC, r8 = 8 * (id - c * RPC);
            v[it] = *(const h8_t*)(smem + c * (BM + 8) + r8);
            off[it] = ws_qkv_off(e, wr, 2, m0 + r8, n0 + c - start[2]);
        }
#pragma unroll
        for (int it = 0; it < ITV; it++)
            if (tid + 512 * it < NV) *(CF_GLOBAL h8_t*)(e.out2 + off[it]) = v[it];
        return;
    }
    if constexpr (EPI == WS_EPI_RESIDUAL) {
        const CF_GLOBAL _Float16* __restrict__ res = e.res;
        f4_t lo[IT], hi[IT];
        h8_t rv[IT];
        size_t off[IT];
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int id = min(tid + 512 * it, NCH - 1), r = id / CPR, c8 = id - r * CPR;
            const float* sp = (const float*)smem + r * (BN + 4) + 8 * c8;
            off[it] = (size_t)(m0 + r) * e.n0w + n0 + 8 * c8;
            lo[it] = *(const f4_t*)sp;
            hi[it] = *(const f4_t*)(sp + 4);
            rv[it] = *(const CF_GLOBAL h8_t*)(res + off[it]);
        }
#pragma unroll
        for (int it = 0; it < IT; it++) {
            if (tid + 512 * it >= NCH) continue;
            const float f[8] = {lo[it][0], lo[it][1], lo[it][2], lo[it][3], hi[it][0], hi[it][1], hi[it][2], hi[it][3]};
            h8_t v;
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = (_Float16)(f[e] + (float)rv[it][e]);
            *(CF_GLOBAL h8_t*)(e.out0 + off[it]) = v;
        }
        return;
    }
    {
        h8_t v[IT];
        size_t off[IT];
        int sg[IT];
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int id = min(tid + 512 * it, NCH - 1), r = id / CPR, c8 = id - r * CPR;
            int col;
            sg[it] = ws_seg_n(nseg, start, n0 + 8 * c8, col);
            off[it] = ws_qkv_off(e, wr, sg[it], m0 + r, col);
            v[it] = *(const h8_t*)(smem + r * (BN + 8) + 8 * c8);
        }
#pragma unroll
        for (int it = 0; it < IT; it++) {
            if (tid + 512 * it >= NCH || (qkv && sg[it] == 2)) continue;   // v^T: below
            *(CF_GLOBAL h8_t*)(e.out(sg[it]) + off[it]) = v[it];
        }
    }
    if (qkv && n0 + BN > start[2]) {
        // The tile's columns in the V segment, [max(n0, start[2]), n0 + BN): chunks of 8 rows.
        const int c_lo = max(n0, start[2]) - n0, ncol = BN - c_lo, nv = ncol * (BM / 8);
        constexpr int ITV = (BN * (BM / 8) + 511) / 512;
        h8_t v[ITV];
        size_t off[ITV];
#pragma unroll
        for (int it = 0; it < ITV; it++) {
            const int id = min(tid + 512 * it, nv - 1);
            const int c = c_lo + id % ncol, r8 = 8 * (id / ncol);
#pragma unroll
            for (int e = 0; e < 8; e++) v[it][e] = smem[(r8 + e) * (BN + 8) + c];
            off[it] = ws_qkv_off(e, wr, 2, m0 + r8, n0 + c - start[2]);
        }
#pragma unroll
        for (int it = 0; it < ITV; it++)
            if (tid + 512 * it < nv) *(h8_t*)(e.out2 + off[it]) = v[it];
    }
}

// Per-tile cost model of the wave-specialised kernel, in CU clocks: the larger of its DMA
// (~32 B/clk per CU with whole A lines) and its MFMA work at ~60 % of the CU's 4096
// FLOP/clk (one compute wave per SIMD), times the rounds of tiles over the CUs.
inline double ws_cost(long long M, long long Ntot, long long K, int bm, int bn, int cus) {
    const long long tiles = (M / bm) * (Ntot / bn);
    const double dma = (double)(bm + bn) * (double)K * 2.0 / 32.0;
    const double mfma = 2.0 * bm * bn * (double)K / 2500.0;
    const long long rounds = (tiles + cus - 1) / cus;
    return (double)rounds * (dma > mfma ? dma : mfma);
}

int g_gemm_stages = 0;   // tuning override of the direct-to-LDS kernel's ring depth (3, 4; 0 = automatic)
int g_gemm_bn = 0;       // tuning override of its tile width (96, 128; 0 = automatic)

int g_gemm_bk = 0;       // tuning override of its stage depth in k (32, 64; 0 = automatic)

template <int STAGES, int BK>
void launch_async(int bn, dim3 grid, hipStream_t s, const cf_gemm_args_t& a, const Tiling& t) {
    if (bn == 96) hipLaunchKernelGGL((gemm_f16_async<STAGES, 96, BK>), grid, dim3(kThreads), 0, s, a, t);
    else hipLaunchKernelGGL((gemm_f16_async<STAGES, 128, BK>), grid, dim3(kThreads), 0, s, a, t);
}

// Two k groups (8 waves) per tile: 2 stages of 64 k per group, 112 KB (96 columns) or
// 128 KB (128 columns) of dynamic LDS, one workgroup per CU.
int g_gemm_ksplit = 0;   // tuning/test override: 1 = one k group, 2 = two where K allows, 0 = automatic

// The dynamic-LDS limit is raised once per device (a bit per device id below 64, every
// launch above); a failure is returned to the caller rather than left to the launch.
template <int BNT>
hipError_t launch_ksplit2(dim3 grid, hipStream_t s, const cf_gemm_args_t& a, const Tiling& t) {
    constexpr unsigned lds = 2u * 2u * (128u * 64u + 64u * BNT) * 2u;
    static std::atomic<uint64_t> raised{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev >= 64 || !((raised.load(std::memory_order_acquire) >> dev) & 1u)) {
        e = hipFuncSetAttribute((const void*)gemm_f16_async<2, BNT, 64, 2>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (dev < 64) raised.fetch_or(1ull << dev, std::memory_order_release);
    }
    hipLaunchKernelGGL((gemm_f16_async<2, BNT, 64, 2>), grid, dim3(2 * kThreads), lds, s, a, t);
    return hipSuccess;
}

// 192-column tiles: 3 stages of 32 k (60 KB of LDS; two workgroups per CU).
void launch_async_192(dim3 grid, hipStream_t s, const cf_gemm_args_t& a, const Tiling& t) {
    hipLaunchKernelGGL((gemm_f16_async<3, 192, 32>), grid, dim3(kThreads), 0, s, a, t);
}

int g_gemm_ws = 0;        // 0: wave-specialised kernel where it applies; 1: never
int g_gemm_ws_bm = 0;     // tuning/test override of its tile (both 0 = cost model)
int g_gemm_ws_bn = 0;

// The wave-specialised kernel's dynamic LDS above 64 KB is enabled once per device and
// instantiation (a bit per device id below 64, every launch above).
template <int BM, int BN, int S, int EPI>
hipError_t launch_ws_epi(dim3 grid, hipStream_t st, const cf_gemm_args_t& a, const Tiling& t) {
    constexpr unsigned lds = ws_lds_bytes<BM, BN, S>();
    static std::atomic<uint64_t> raised{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev >= 64 || !((raised.load(std::memory_order_acquire) >> dev) & 1u)) {
        e = hipFuncSetAttribute((const void*)gemm_f16_ws<BM, BN, S, EPI>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds);
        if (e != hipSuccess) return e;
        if (dev < 64) raised.fetch_or(1ull << dev, std::memory_order_release);
    }
    hipLaunchKernelGGL((gemm_f16_ws<BM, BN, S, EPI>), grid, dim3(512), lds, st, a, t);
    return hipSuccess;
}

template <int BM, int BN, int S>
hipError_t launch_ws(dim3 grid, hipStream_t st, const cf_gemm_args_t& a, const Tiling& t) {
    if (a.out_kind == CF_GEMM_OUT_QKV) return launch_ws_epi<BM, BN, S, WS_EPI_QKV>(grid, st, a, t);
    if (a.residual) return launch_ws_epi<BM, BN, S, WS_EPI_RESIDUAL>(grid, st, a, t);
    return launch_ws_epi<BM, BN, S, WS_EPI_ROWMAJOR>(grid, st, a, t);
}

struct WsCandidate {
    int bm, bn;
    unsigned lds;
    hipError_t (*launch)(dim3, hipStream_t, const cf_gemm_args_t&, const Tiling&);
};
// 256-row tiles hold 192 columns on 2 stages (LDS), narrower ones on 3; 128-row tiles on 3.
const WsCandidate kWsShapes[] = {
    {256, 192, ws_lds_bytes<256, 192, 2>(), launch_ws<256, 192, 2>},
    {256, 144, ws_lds_bytes<256, 144, 3>(), launch_ws<256, 144, 3>},
    {256, 128, ws_lds_bytes<256, 128, 3>(), launch_ws<256, 128, 3>},
    {256, 96, ws_lds_bytes<256, 96, 3>(), launch_ws<256, 96, 3>},
    {256, 64, ws_lds_bytes<256, 64, 3>(), launch_ws<256, 64, 3>},
    {256, 48, ws_lds_bytes<256, 48, 3>(), launch_ws<256, 48, 3>},
    {128, 192, ws_lds_bytes<128, 192, 3>(), launch_ws<128, 192, 3>},
    {128, 128, ws_lds_bytes<128, 128, 3>(), launch_ws<128, 128, 3>},
    {128, 96, ws_lds_bytes<128, 96, 3>(), launch_ws<128, 96, 3>},
    {128, 64, ws_lds_bytes<128, 64, 3>(), launch_ws<128, 64, 3>},
};

// The wave-specialised shape for this product, or nullptr where the kernel does not apply
// (fp16 only; 16-byte aligned rows and stores; M a multiple of the tile height; K a
// multiple of 64; every segment width a multiple of 8; 32-bit A offsets).
const WsCandidate* ws_pick(const cf_gemm_args_t* a, const Tiling& t) {
    if (g_gemm_ws == 1 || a->elem != CF_ELEM_F16 || !t.epi_vec || !t.a_vec) return nullptr;
    // Row-major outputs only by default: with the Q|K|V scatter the kernel measured no
    // faster than the pipelined one (BERT-base 4096 x 2304 x 768: 23.8 vs 23.2 us with
    // biases; the same product stored row-major takes 19.2 us), while the output
    // projections gain (4096 x 768 x 768: 8.4 vs 9.9 us; 4096 x 1024 x 1024: 12.1 vs
    // 13.3 us).  A tile override (cf_gemm_set_ws_shape) still routes the scatter here.
    if (a->out_kind == CF_GEMM_OUT_QKV && g_gemm_ws_bm == 0) return nullptr;
    if (a->out_kind == CF_GEMM_OUT_ROWCAT && a->residual) return nullptr;
    if (a->K % WS_BK != 0 || (long long)a->M * a->K * 2 >= (1LL << 32)) return nullptr;
    long long ntot = 0;
    for (int s = 0; s < a->nseg; s++) {
        if (!t.w_vec[s] || a->n[s] % 8 != 0 || (uintptr_t)a->bias[s] % 16 != 0) return nullptr;
        ntot += a->n[s];
    }
    const bool res32 = a->residual != nullptr && a->out_kind == CF_GEMM_OUT_ROWMAJOR;
    const WsCandidate* best = nullptr;
    double best_cost = 0.0;
    for (const WsCandidate& c : kWsShapes) {
        if (a->M % c.bm != 0 || ntot % c.bn != 0) continue;
        // The staged tile (fp32 with a residual, else fp16) fits in the rings.
        const unsigned staged = res32 ? (unsigned)c.bm * (c.bn + 4) * 4u : (unsigned)c.bm * (c.bn + 8) * 2u;
        const unsigned staged_vt = (unsigned)c.bn * (c.bm + 8) * 2u;     // v^T tiles, column-major
        if (staged > c.lds || staged_vt > c.lds) continue;
        if (c.bm == g_gemm_ws_bm && c.bn == g_gemm_ws_bn) return &c;   // an override that fits
        const double cost = ws_cost(a->M, ntot, a->K, c.bm, c.bn, cu_count());
        if (!best || cost < best_cost) {
            best = &c;
            best_cost = cost;
        }
    }
    return best;
}

}  // namespace

extern "C" void cf_gemm_set_stages(int32_t stages) { g_gemm_stages = stages; }

extern "C" void cf_gemm_set_bk(int32_t bk) { g_gemm_bk = bk == 32 || bk == 64 ? bk : 0; }

extern "C" void cf_gemm_set_ksplit(int32_t ks) { g_gemm_ksplit = ks == 1 || ks == 2 ? ks : 0; }

extern "C" void cf_gemm_set_bn(int32_t bn) { g_gemm_bn = bn == 96 || bn == 128 || bn == 192 ? bn : 0; }

extern "C" void cf_gemm_set_ws(int32_t mode) { g_gemm_ws = mode == 1 ? 1 : 0; }

// The checks cf_launch_gemm runs before taking the wave-specialised kernel, for a
// row-concatenated output (which only that kernel writes).
extern "C" int32_t cf_gemm_rowcat_ok(const cf_gemm_args_t* a) {
    if (a->out_kind != CF_GEMM_OUT_ROWCAT || a->nseg < 1 || a->nseg > 3 || a->M <= 0 || a->K <= 0) return 0;
    Tiling t{};
    t.a_vec = (a->K % 8 == 0) && ((uintptr_t)a->a % 16 == 0);
    for (int s = 0; s < a->nseg; s++) t.w_vec[s] = (a->n[s] % 8 == 0) && ((uintptr_t)a->w[s] % 16 == 0);
    t.epi_vec = (uintptr_t)a->out[0] % 16 == 0;
    return ws_pick(a, t) ? 1 : 0;
}

extern "C" void cf_gemm_set_ws_shape(int32_t bm, int32_t bn) {
    g_gemm_ws_bm = bm > 0 ? bm : 0;
    g_gemm_ws_bn = bn > 0 ? bn : 0;
}

int g_gemm_group_m = 0;  // tuning override of the tile-order group height (0 = kGroupM)

extern "C" void cf_gemm_set_group_m(int32_t group_m) { g_gemm_group_m = group_m > 0 ? group_m : 0; }

extern "C" int cf_launch_gemm(const cf_gemm_args_t* a, void* stream) {
    if (a->nseg < 1 || a->nseg > 3 || a->M <= 0 || a->K <= 0) return (int)hipErrorInvalidValue;
    Tiling t{};
    // fp16 reads 8 halves at a time from A and W; fp32 reads 4 floats.
    const int vec = a->elem == CF_ELEM_F16 ? 8 : 4;
    t.a_vec = (a->K % vec == 0) && ((uintptr_t)a->a % 16 == 0);
    for (int s = 0; s < a->nseg; s++)
        t.w_vec[s] = (a->n[s] % vec == 0) && ((uintptr_t)a->w[s] % 16 == 0);
    // 8-element stores stay inside one destination row: N % 8 (row-major), d % 8 and
    // S % 8 (head-major q/k and transposed v), with 16-byte aligned buffers.
    uintptr_t ptrs = (uintptr_t)a->out[0] | (uintptr_t)a->residual;
    for (int s = 1; s < a->nseg; s++) ptrs |= (uintptr_t)a->out[s];
    int ev = (ptrs % 16 == 0);
    if (a->out_kind == CF_GEMM_OUT_ROWMAJOR) ev = ev && a->n[0] % 8 == 0;
    else if (a->out_kind == CF_GEMM_OUT_QKV) ev = ev && a->d % 8 == 0 && a->S % 8 == 0;
    t.epi_vec = ev;
    t.group_m = g_gemm_group_m > 0 ? g_gemm_group_m : kGroupM;
    if (a->out_kind == CF_GEMM_OUT_ROWCAT && !ws_pick(a, t)) return (int)hipErrorInvalidValue;
    // The wave-specialised kernel where it applies (its tile chosen by the cost model).
    if (const WsCandidate* c = ws_pick(a, t)) {
        long long ntot = 0;
        for (int s = 0; s < a->nseg; s++) ntot += a->n[s];
        t.n_tiles_m = a->M / c->bm;
        const long long blocks = (long long)t.n_tiles_m * (ntot / c->bn);
        if (blocks <= 0 || blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
        set_order(t, (int)(ntot / c->bn));
        const hipError_t e = c->launch(dim3((unsigned)blocks), (hipStream_t)stream, *a, t);
        if (e != hipSuccess) return (int)e;
        return (int)hipGetLastError();
    }
    // Full tiles with aligned rows take the pipelined direct-to-LDS kernel.  Its tile is
    // 128 columns wide unless that leaves CUs idle and 96 columns fills more of them
    // (BERT-base's 4096 x 768 output projection: 192 tiles of 128 x 128 on 256 CUs, 256 of
    // 128 x 96).  Narrower tiles load more from L2 per flop, so with more tiles than CUs
    // the balance they buy measured slower (the 4096 x 2304 QKV product: 27.4 us at 96
    // columns, three tiles per CU, vs 26.6 us at 128, 2.25 per CU).  192 columns are
    // taken where 128-column tiles need three workgroups on some CU and 192-column tiles
    // at most two: the busiest CU does the same MFMA work on 17 % fewer loaded bytes
    // (that QKV product: 576 -> 384 tiles, 23.0 -> 20.3 us).
    const long long tiles_m = (a->M + BM - 1) / BM;
    bool full = a->elem == CF_ELEM_F16 && t.epi_vec && a->M % BM == 0 && a->K % BKA == 0 && t.a_vec &&
                (long long)a->M * a->K * 2 < (1LL << 32);
    for (int s = 0; s < a->nseg; s++) full = full && (long long)a->K * a->n[s] * 2 < (1LL << 32);
    for (int s = 0; s < a->nseg; s++) full = full && t.w_vec[s];
    auto fits = [&](int bn) {
        for (int s = 0; s < a->nseg; s++)
            if (a->n[s] % bn) return false;
        return true;
    };
    auto tiles = [&](int bn) {
        long long tn = 0;
        for (int s = 0; s < a->nseg; s++) tn += a->n[s] / bn;
        return tiles_m * tn;
    };
    int bn = BN;
    // fp32: 96-column tiles where 128 leaves CUs idle and 96 fills more of them.
    if (a->elem == CF_ELEM_F32 && fits(96) && (!fits(128) || (tiles(128) < cu_count() && tiles(96) > tiles(128))))
        bn = 96;
    if (full) {
        const bool f128 = fits(128), f96 = fits(96), f192 = fits(192);
        if (!f128 && !f96 && !f192) full = false;
        else if (g_gemm_bn && fits(g_gemm_bn)) bn = g_gemm_bn;
        else if (f128 && f192 && tiles(128) > 2LL * cu_count() && tiles(192) <= 2LL * cu_count()) bn = 192;
        else if (f96 && (!f128 || (tiles(128) < cu_count() && tiles(96) > tiles(128)))) bn = 96;
        else if (!f128) bn = 192;
    }
    t.n_tiles_m = (int)tiles_m;
    int acc = 0;
    for (int s = 0; s < a->nseg; s++) {
        t.seg_start[s] = acc;
        acc += (int)((a->n[s] + bn - 1) / bn);
    }
    for (int s = a->nseg; s < 4; s++) t.seg_start[s] = acc;
    const long long blocks = (long long)acc * t.n_tiles_m;
    if (blocks <= 0 || blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    set_order(t, acc);
    dim3 grid((unsigned)blocks);
    hipStream_t st = (hipStream_t)stream;
    if (full) {
        // Up to two tiles per CU: two workgroups per CU, each with 64 KB of ring, as 2
        // stages of 64 k (whole 128-byte A lines; 10.2 vs 11.0 us on BERT-base's output
        // projection) rather than 4 of 32.  More tiles: three workgroups per CU on
        // 3 stages of 32 k, since 160 KB of LDS holds no third 64 KB ring.
        const bool two_per_cu = blocks <= 2LL * cu_count();
        int bk = two_per_cu && a->K % 64 == 0 ? 64 : 32;
        if (g_gemm_bk == 32 || (g_gemm_bk == 64 && a->K % 64 == 0)) bk = g_gemm_bk;
        int stages = two_per_cu ? 4 : 3;
        if (g_gemm_stages == 3 || g_gemm_stages == 4) stages = g_gemm_stages;
        // At most one tile per CU: two k groups of 4 waves per tile (K a multiple of 128).
        bool ks2 = blocks <= (long long)cu_count() && bn != 192 && a->K % 128 == 0;
        if (g_gemm_ksplit == 1) ks2 = false;
        if (g_gemm_ksplit == 2) ks2 = bn != 192 && a->K % 128 == 0;
        hipError_t e = hipSuccess;
        if (bn == 192) launch_async_192(grid, st, *a, t);
        else if (ks2 && bn == 96) e = launch_ksplit2<96>(grid, st, *a, t);
        else if (ks2) e = launch_ksplit2<128>(grid, st, *a, t);
        else if (bk == 64) launch_async<2, 64>(bn, grid, st, *a, t);
        else if (stages == 3) launch_async<3, 32>(bn, grid, st, *a, t);
        else launch_async<4, 32>(bn, grid, st, *a, t);
        if (e != hipSuccess) return (int)e;
    } else if (a->elem == CF_ELEM_F16) {
        hipLaunchKernelGGL(gemm_f16, grid, dim3(kThreads), 0, st, *a, t);
    } else if (bn == 96) {
        hipLaunchKernelGGL(gemm_f32<96>, grid, dim3(kThreads), 0, st, *a, t);
    } else {
        hipLaunchKernelGGL(gemm_f32<128>, grid, dim3(kThreads), 0, st, *a, t);
    }
    return (int)hipGetLastError();
}
