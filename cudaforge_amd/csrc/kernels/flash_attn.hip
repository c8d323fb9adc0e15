// flash_attn.hip — prefill multi-head attention with an online softmax (gfx950).
//
// Computes, per (b, query head h), softmax(Q·K^T·scale)·V over keys 0..S-1 (or
// 0..i for causal query i, the rule of mha_fused_cuda.cu:336 / causal_mask.c:19),
// reading the projections the GEMM epilogue laid out head-major:
//   q (B,H_q,S,d), k (B,H_kv,S,d), vt (B,H_kv,d,S)  ->  o (B,S,H_q,d).
// kv head = h / (H_q/H_kv) (mha_decode.c:77).  The reference CPU semantics it must match
// are mha_fused.c:98-131 (two-pass softmax); the online form changes only rounding.
//
// fp16 path (d = 64 or 128): a workgroup owns 128 queries, 32 per wave (two 16-query
// column blocks, so every K and V^T fragment read from LDS feeds two MFMAs).  Key blocks
// of 64 are staged in LDS (K as [key][dim], V^T as [dim][key]) through a two-stage ring
// whose next block is loaded into registers while the current one is used (for d = 64
// and S % 8 == 0, flash_f16_dma64 streams the blocks by DMA instead, see there).  Each wave
// computes S^T = K·Q^T with v_mfma_f32_16x16x32_f16, so a lane holds 16 scores of ONE
// query per column block: the row max and row sum are lane-local plus a 4-lane exchange.
// The probabilities are converted to fp16 in registers and fed back as the B operand of
// O^T += V^T·P^T; the key order inside each 32-key MFMA step is permuted so that the
// registers a lane already holds are exactly its B operand (the V^T reads follow the
// same permutation).  No score or probability goes through LDS.  Masks are evaluated
// only on blocks that cross the sequence end or the causal diagonal.  Causal workgroups
// of this kernel and of the DMA kernel below are issued heaviest-first (the DMA kernel
// can also pair each causal query block with its mirror, equal work per workgroup).
//
// fp32 path (d = 64 or 128): the same structure on v_mfma_f32_16x16x4_f32, see flash_f32.
// Generic path (other head sizes): one thread per query, online softmax in fp32 with Q
// and the accumulator in LDS.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "cdna4.h"

namespace {

using namespace cdna4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQB = 128;     // queries per workgroup (32 per wave)
constexpr int kKB = 64;      // keys per block
constexpr int kThreads = 256;

template <int D>
__global__ __launch_bounds__(kThreads, 2)
void flash_f16(cf_flash_args_t a) {
    constexpr int LDK = D + 8;        // halves per K row in LDS
    constexpr int LDV = kKB + 8;      // halves per V^T row in LDS
    constexpr int KT = D / 32;        // 32-dim steps of S^T
    constexpr int UT = D / 16;        // 16-dim tiles of O^T
    constexpr int K_ST = kKB * LDK, V_ST = D * LDV;
    constexpr int KCH = kKB * D / 8 / kThreads;   // 16-byte K chunks per thread per block
    constexpr int VCH = D * kKB / 8 / kThreads;   // 16-byte V^T chunks per thread per block
    __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (K_ST + V_ST)];

    // XCD-aware order: workgroup id w runs on XCD w % 8.  Ids are laid out as
    // ((group * nqb + qb) * 8 + r) with head-batch index hb = group * 8 + r, so every
    // query block of one (b, h) lands on the same XCD and shares its K/V in that L2.
    const int nqb = (a.S + kQB - 1) / kQB;
    const int HB = a.B * a.H_q;
    const int w = blockIdx.x, r8 = w & 7, rest = w >> 3;
    const int qi = rest % nqb, grp = rest / nqb;
    const int hb = grp * 8 + r8;
    if (hb >= HB) return;                          // padding of the last group of 8
    const int qb = a.causal ? (nqb - 1 - qi) : qi;
    const int h = hb % a.H_q, b = hb / a.H_q;
    const int S = a.S;
    const int kvh = h / (a.H_q / a.H_kv);
    const int q0 = qb * kQB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int qw = q0 + 32 * wave;                 // first query of this wave

    const _Float16* __restrict__ qp = (const _Float16*)a.q + (((size_t)b * a.H_q + h) * S) * D;
    const _Float16* __restrict__ kp = (const _Float16*)a.k + (((size_t)b * a.H_kv + kvh) * S) * D;
    const _Float16* __restrict__ vp = (const _Float16*)a.vt + (((size_t)b * a.H_kv + kvh) * D) * (size_t)S;

    int query[2];
    h8_t qf[2][KT];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        query[j] = qw + 16 * j + lr;
#pragma unroll
        for (int kt = 0; kt < KT; kt++)
            qf[j][kt] = query[j] < S ? *(const h8_t*)(qp + (size_t)query[j] * D + 32 * kt + 8 * lq) : h8_t{};
    }

    const float c = a.scale * kLog2e;
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
    f4_t acc[2][UT];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int u = 0; u < UT; u++) acc[j][u] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int k_end = a.causal ? min(S, q0 + kQB) : S;
    const bool v_vec = (S % 8) == 0;
    h8_t rk[KCH], rv[VCH];
    auto load_block = [&](int k0) {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int ch = tid + i * kThreads;
            const int r = ch / (D / 8), cc = (ch % (D / 8)) * 8;
            rk[i] = k0 + r < S ? *(const h8_t*)(kp + (size_t)(k0 + r) * D + cc) : h8_t{};
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            const int ch = tid + i * kThreads;
            const int dm = ch / (kKB / 8), kc = (ch % (kKB / 8)) * 8;
            const _Float16* src = vp + (size_t)dm * S + k0 + kc;
            h8_t v{};
            if (v_vec && k0 + kc + 8 <= S) v = *(const h8_t*)src;
            else {
#pragma unroll
                for (int e = 0; e < 8; e++) if (k0 + kc + e < S) v[e] = src[e];
            }
            rv[i] = v;
        }
    };
    auto store_block = [&](int stage) {
        _Float16* Ks = smem + stage * (K_ST + V_ST);
        _Float16* Vs = Ks + K_ST;
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int ch = tid + i * kThreads;
            *(h8_t*)&Ks[(ch / (D / 8)) * LDK + (ch % (D / 8)) * 8] = rk[i];
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            const int ch = tid + i * kThreads;
            *(h8_t*)&Vs[(ch / (kKB / 8)) * LDV + (ch % (kKB / 8)) * 8] = rv[i];
        }
    };

    const int nblk = (k_end + kKB - 1) / kKB;
    load_block(0);
    store_block(0);
    __syncthreads();
    for (int bi = 0; bi < nblk; bi++) {
        const int k0 = bi * kKB;
        if (bi + 1 < nblk) load_block(k0 + kKB);
        const _Float16* Ks = smem + (bi & 1) * (K_ST + V_ST);
        const _Float16* Vs = Ks + K_ST;

        // S^T tiles: st[j][t][i] = score(key k0 + 16t + 4*lq + i, query[j]).
        f4_t st[2][4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            st[0][t] = f4_t{0.f, 0.f, 0.f, 0.f};
            st[1][t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < KT; kt++) {
                const h8_t kf = *(const h8_t*)&Ks[(16 * t + lr) * LDK + 32 * kt + 8 * lq];
                st[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[0][kt], st[0][t], 0, 0, 0);
                st[1][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[1][kt], st[1][t], 0, 0, 0);
            }
        }
        const bool edge = (k0 + kKB > S) || (a.causal && k0 + kKB - 1 > qw);
        h8_t pf[2][2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if (edge) {
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = k0 + 16 * t + 4 * lq + i;
                        if (key >= S || (a.causal && key > query[j])) st[j][t][i] = -INFINITY;
                    }
            }
            float mloc = fmaxf(fmaxf(st[j][0][0], st[j][0][1]), fmaxf(st[j][0][2], st[j][0][3]));
#pragma unroll
            for (int t = 1; t < 4; t++)
                mloc = fmaxf(mloc, fmaxf(fmaxf(st[j][t][0], st[j][t][1]), fmaxf(st[j][t][2], st[j][t][3])));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
            // Scores are raw dot products; the scale folds into the exponent: p = 2^(s*c - m*c).
            const float m_new = fmaxf(m_run[j], mloc * c);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run[j] - m_use);
            m_run[j] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[j][t][i], c, -m_use));
                    psum += p;
                    pf[j][t >> 1][(t & 1) * 4 + i] = (_Float16)p;
                }
            l_run[j] = l_run[j] * alpha + psum;
#pragma unroll
            for (int u = 0; u < UT; u++) acc[j][u] *= alpha;
        }
        // O^T[16u + 4*lq + i][query] += V^T · P^T; in 32-key step s, k-slot e of lane group
        // lq is key 32s + 16*(e/4) + 4*lq + (e%4).
#pragma unroll
        for (int u = 0; u < UT; u++)
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const _Float16* vr = &Vs[(16 * u + lr) * LDV + 32 * s + 4 * lq];
                const h4_t lo = *(const h4_t*)vr;
                const h4_t hi = *(const h4_t*)(vr + 16);
                const h8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                acc[0][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[0][s], acc[0][u], 0, 0, 0);
                acc[1][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[1][s], acc[1][u], 0, 0, 0);
            }
        if (bi + 1 < nblk) store_block((bi + 1) & 1);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        float l_tot = l_run[j] + __shfl_xor(l_run[j], 16);
        l_tot += __shfl_xor(l_tot, 32);
        if (query[j] < S) {
            const float inv = 1.0f / l_tot;
            _Float16* op = (_Float16*)a.o + (((size_t)b * S + query[j]) * a.H_q + h) * D;
#pragma unroll
            for (int u = 0; u < UT; u++) {
                const h4_t ov = {(_Float16)(acc[j][u][0] * inv), (_Float16)(acc[j][u][1] * inv),
                                 (_Float16)(acc[j][u][2] * inv), (_Float16)(acc[j][u][3] * inv)};
                *(h4_t*)(op + 16 * u + 4 * lq) = ov;
            }
        }
    }
}

// ---- d = 64, S % 8 == 0: the same computation with K and V^T blocks streamed by DMA
// (global_load_lds_dwordx4) into a kFlashStages-deep LDS ring instead of through
// registers, so kFlashStages - 1 key blocks are in flight while one is used and no
// wave waits on a block's loads before storing them.  K rows (128 B) and V^T rows (64
// keys, 128 B) are XOR-swizzled in 16-byte chunks so the K fragment reads (16 rows, one
// chunk: chunk ^ (row / 2) % 8) and the V^T fragment reads (16 rows, 8 bytes: chunk ^
// (row / 2 ^ row / 16) % 8) are bank-conflict free.  The V^T term in row / 16 makes the
// reads of row blocks u and u+1 differ by more than a constant, so the compiler keeps
// them as separate ds_read_b64 instead of pairing them into ds_read2st64_b64, which
// measured four times the LDS cycles (SQ_LDS_BANK_CONFLICT) on gfx950.  Rows and chunks
// past the sequence end are clamped to the last valid ones (S % 8 == 0 keeps every 8-key
// chunk whole) and get p = 0.  The row max is reduced with the gfx950 row swaps, and the
// running max only moves when a block exceeds it by more than kLazy (log2 units), so the
// accumulators are rarely rescaled.
// The kernel is bound by its VALU work per score (the exponential and its neighbours),
// so everything else is kept off the VALU: the loop is unrolled by ring stage (LDS
// addresses become immediates), full blocks are loaded as a uniform base plus per-lane
// offsets fixed for the whole loop, and the row sum of p comes out of the matrix core:
// one more MFMA per 32 keys with an all-ones A operand gives every lane the full sum
// over the block's keys for its query, from the same fp16 p that weights V.
constexpr int kFlashStages = 3;
constexpr float kLazy = 8.0f;

__device__ __forceinline__ int fswz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int vswz(int row) { return ((row >> 1) ^ (row >> 4)) & 7; }

// V rows [key][dim] (the row-concatenated input), read transposed by ds_read_b64_tr_b16:
// rows of one 32-lane half of a read (keys kb .. kb+7) land in distinct banks.
__device__ __forceinline__ int trswz(int row) { return 2 * ((row >> 1) & 3); }

// RC: Q, K and V come from the row-concatenated (B*S, qkv_ld) matrix (K and V rows as
// they are; V read transposed from LDS), else from q / k / vt laid out head-major.
// Waves per SIMD the build must allow: three 16-query workgroups per CU; the 32-query
// build (taken with at least two workgroups per CU) at three would spill registers.
template <int NJ, bool RC = false>
__global__ __launch_bounds__(kThreads, NJ == 1 ? 3 : 2)
void flash_f16_dma64(cf_flash_args_t a, int pairs, FastDiv div_slot, FastDiv div_hq, FastDiv div_g) {
    constexpr int D = 64;
    constexpr int QW = 16 * NJ;                   // queries per wave
    constexpr int QB = 4 * QW;                    // queries per workgroup
    constexpr int KT = D / 32;                    // 32-dim steps of S^T
    constexpr int UT = D / 16;                    // 16-dim tiles of O^T
    constexpr int TILE = kKB * D;                 // halves per block per tensor (8 KB)
    constexpr int NS = kFlashStages;
    static_assert(NS == 3, "the prologue issues two blocks");
    __shared__ __attribute__((aligned(16))) _Float16 ring[NS * 2 * TILE];

    // Causal (pairs == 0, the default): one query block per workgroup, every head's
    // heaviest blocks first (slot-major order), so later, lighter blocks fill the CUs
    // that finish early.  With pairs, workgroup slot qi runs query block nqb-1-qi and
    // then its mirror qi, so every workgroup does nqb+1 key blocks (one block per slot
    // when the two meet).
    const int nqb = (a.S + QB - 1) / QB;
    const int HB = a.B * a.H_q;
    const int paired = a.causal && pairs;
    const int nslot = paired ? (nqb + 1) / 2 : nqb;
    // The launcher's divisors (FastDiv): div_slot by ngrp (causal, one block per
    // workgroup) or nslot, div_hq by H_q, div_g by H_q / H_kv.
    const int w = blockIdx.x, r8 = w & 7, rest = w >> 3;
    const int ngrp = (HB + 7) / 8;
    const int rq = fastdiv(rest, div_slot), rr = rest - rq * (a.causal && !pairs ? ngrp : nslot);
    const int qi = a.causal && !pairs ? rq : rr;
    const int grp = a.causal && !pairs ? rr : rq;
    const int hb = grp * 8 + r8;
    if (hb >= HB) return;                          // padding of the last group of 8
    const int b = fastdiv(hb, div_hq), h = hb - b * a.H_q;
    const int S = a.S;
    const int kvh = fastdiv(h, div_g);
  auto run = [&](int qb) {
    const int q0 = qb * QB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int qw = q0 + QW * wave;                 // first query of this wave

    // Row strides (halves) of Q and K (and of V when RC).
    const size_t ld = RC ? (size_t)a.qkv_ld : (size_t)D;
    const _Float16* __restrict__ rc0 = (const _Float16*)a.q + (size_t)b * S * ld;
    const _Float16* __restrict__ qp =
        RC ? rc0 + (size_t)h * D : (const _Float16*)a.q + (((size_t)b * a.H_q + h) * S) * D;
    const _Float16* __restrict__ kp =
        RC ? rc0 + (size_t)(a.H_q + kvh) * D : (const _Float16*)a.k + (((size_t)b * a.H_kv + kvh) * S) * D;
    const _Float16* __restrict__ vp =
        RC ? rc0 + (size_t)(a.H_q + a.H_kv + kvh) * D
           : (const _Float16*)a.vt + (((size_t)b * a.H_kv + kvh) * D) * (size_t)S;

    int query[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) query[j] = qw + 16 * j + lr;

    // DMA: each wave fills K rows 16w .. 16w+15 and V^T rows 16w .. 16w+15 of a stage,
    // 8 rows per instruction; lane L writes physical chunk L % 8 of row 8u + L / 8.  A
    // full block is a uniform base (its first key) plus these per-lane byte offsets
    // (V^T rows are S keys apart: the launcher keeps 64 * S * 2 bytes below 2^32).
    const uint32_t ring_base = lds_offset(ring);
    const uint32_t wave_lds = __builtin_amdgcn_readfirstlane(ring_base + (uint32_t)(16 * wave) * 128u);
    const int drow0 = 16 * wave + (lane >> 3), dch = lane & 7;
    uint32_t koff[2], voff[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int row = drow0 + 8 * u;
        koff[u] = ((uint32_t)row * (uint32_t)ld + 8u * (uint32_t)(dch ^ fswz(row))) * 2u;
        voff[u] = RC ? ((uint32_t)row * (uint32_t)ld + 8u * (uint32_t)(dch ^ trswz(row))) * 2u
                     : ((uint32_t)row * (uint32_t)S + 8u * (uint32_t)(dch ^ vswz(row))) * 2u;
    }
    auto issue = [&](int blk, auto stage_c) {
        constexpr int stage = decltype(stage_c)::value;
        const int k0 = blk * kKB;
        const uint32_t kb = wave_lds + (uint32_t)(stage * 2 * TILE) * 2u;
        const uint32_t vb = kb + (uint32_t)TILE * 2u;
        if (k0 + kKB <= S) {
            const _Float16* kblk = kp + (size_t)k0 * ld;
            const _Float16* vblk = RC ? vp + (size_t)k0 * ld : vp + k0;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                lds_dma16_s(koff[u], kblk, kb + (uint32_t)(8 * u) * 128u);
                lds_dma16_s(voff[u], vblk, vb + (uint32_t)(8 * u) * 128u);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int row = drow0 + 8 * u;
                const int kc = dch ^ fswz(row);
                lds_dma16(kp + (size_t)min(k0 + row, S - 1) * ld + 8 * kc, kb + (uint32_t)(8 * u) * 128u);
                if constexpr (RC) {
                    lds_dma16(vp + (size_t)min(k0 + row, S - 1) * ld + 8 * (dch ^ trswz(row)),
                              vb + (uint32_t)(8 * u) * 128u);
                } else {
                    const int vcol = min(k0 + 8 * (dch ^ vswz(row)), S - 8);
                    lds_dma16(vp + (size_t)row * S + vcol, vb + (uint32_t)(8 * u) * 128u);
                }
            }
        }
    };
    // Per-lane LDS read offsets (halves) inside a stage.
    int k_rd[4][KT];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int kt = 0; kt < KT; kt++) {
            const int row = 16 * t + lr;
            k_rd[t][kt] = row * D + 8 * ((4 * kt + lq) ^ fswz(row));
        }
    int v_rd[UT][2][2];
#pragma unroll
    for (int u = 0; u < UT; u++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                if constexpr (RC) {
                    // V[key][dim]: lane (lr, lq) addresses key 32s + 16hh + 4lq + lr/4, dims
                    // 16u + 4(lr%4) .. +3, and receives dim 16u + lr of those 4 keys.
                    const int row = 32 * s2 + 16 * hh + 4 * lq + (lr >> 2);
                    const int col = 16 * u + 4 * (lr & 3);
                    v_rd[u][s2][hh] = TILE + row * D + 8 * ((col >> 3) ^ trswz(row)) + (col & 7);
                } else {
                    const int row = 16 * u + lr;
                    const int ch = 4 * s2 + 2 * hh + (lq >> 1);      // keys 32s + 16hh + 4lq
                    v_rd[u][s2][hh] = TILE + row * kKB + 8 * (ch ^ vswz(row)) + 4 * (lq & 1);
                }
            }

    const float c = a.scale * kLog2e;
    h8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
    // Held in VGPRs for the whole loop: kept as a scalar constant, it was moved into
    // VGPRs before the row-sum MFMAs of every block (two VALU moves per block).
    asm volatile("" : "+v"(ones));
    float m_run[NJ];
    f4_t acc[NJ][UT], lsum[NJ];                    // lsum: every element is the query's sum of p
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        m_run[j] = -INFINITY;
        lsum[j] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int u = 0; u < UT; u++) acc[j][u] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int k_end = a.causal ? min(S, q0 + QB) : S;
    const int nblk = (k_end + kKB - 1) / kKB;
    // The workgroup's Q rows (QB x 128 B, swizzled like K) go by DMA into ring stage
    // NS-1, which the first blocks leave free, ahead of blocks 0 and 1: the Q and K/V
    // latencies overlap.  Wave w loads rows 8u .. 8u+7 for u = QB/32 * w + v.
    constexpr int QI = QB / 32;                   // Q DMA instructions per wave
    {
        const uint32_t qb_lds = ring_base + (uint32_t)((NS - 1) * 2 * TILE) * 2u;
#pragma unroll
        for (int v = 0; v < QI; v++) {
            const int u = QI * wave + v, row = 8 * u + (lane >> 3);
            lds_dma16(qp + (size_t)min(q0 + row, S - 1) * ld + 8 * (dch ^ fswz(row)),
                      __builtin_amdgcn_readfirstlane(qb_lds + (uint32_t)u * 1024u));
        }
    }
    if (0 < nblk) issue(0, std::integral_constant<int, 0>{});
    if (1 < nblk) issue(1, std::integral_constant<int, 1>{});
    // Q landed when at most the blocks' loads (4 per block) are outstanding.
    if (nblk >= 2) wait_vm<8>();
    else wait_vm<4>();
    ring_barrier();
    // B operand Q^T: lane (lr, lq) holds Q[query][32kt + 8lq .. +7].
    h8_t qf[NJ][KT];
    {
        const _Float16* qs = ring + (NS - 1) * 2 * TILE;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int row = QW * wave + 16 * j + lr;
#pragma unroll
            for (int kt = 0; kt < KT; kt++) qf[j][kt] = *(const h8_t*)(qs + row * D + 8 * ((4 * kt + lq) ^ fswz(row)));
        }
    }
    wait_lds_reads();                              // stage NS-1 is refilled after the next barrier
    auto step = [&](int bi, auto stage_c) {
        constexpr int stage = decltype(stage_c)::value;
        // Blocks issued after this one that may still be in flight (4 loads each).
        wait_ahead<4, NS - 2>(nblk - 1 - bi);
        ring_barrier();                            // every wave's part of block bi landed;
                                                   // block bi-1's stage is free again
        if (bi + NS - 1 < nblk) issue(bi + NS - 1, std::integral_constant<int, (stage + NS - 1) % NS>{});
        const int k0 = bi * kKB;
        const _Float16* st = ring + stage * 2 * TILE;

        // S^T tiles: sc[j][t][i] = score(key k0 + 16t + 4*lq + i, query[j]).
        f4_t sc[NJ][4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int j = 0; j < NJ; j++) sc[j][t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < KT; kt++) {
                const h8_t kf = *(const h8_t*)(st + k_rd[t][kt]);
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    sc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[j][kt], sc[j][t], 0, 0, 0);
            }
        }
        const bool edge = (k0 + kKB > S) || (a.causal && k0 + kKB - 1 > qw);
        h8_t pf[NJ][2];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (edge) {
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = k0 + 16 * t + 4 * lq + i;
                        if (key >= S || (a.causal && key > query[j])) sc[j][t][i] = -INFINITY;
                    }
            }
            // A chain of three-input maxima (v_max3_f32): 8 instructions for the 16 scores.
            float mloc = fmaxf(fmaxf(sc[j][0][0], sc[j][0][1]), sc[j][0][2]);
#pragma unroll
            for (int e = 3; e < 15; e += 2)
                mloc = fmaxf(fmaxf(mloc, sc[j][e >> 2][e & 3]), sc[j][(e + 1) >> 2][(e + 1) & 3]);
            mloc = fmaxf(mloc, sc[j][3][3]);
            mloc = max_xor32(max_xor16(mloc)) * c;     // -inf if the whole row is masked
            if (__builtin_amdgcn_ballot_w64(mloc > m_run[j] + kLazy)) {
                const float m_new = mloc > m_run[j] + kLazy ? mloc : m_run[j];
                const float alpha = __builtin_amdgcn_exp2f(m_run[j] - m_new);   // 0 on the first move
                m_run[j] = m_new;
                lsum[j] *= alpha;
#pragma unroll
                for (int u = 0; u < UT; u++) acc[j][u] *= alpha;
            }
            // Rows with nothing visible yet keep m = -inf: use 0 so p = 2^-inf = 0.
            const float m_use = m_run[j] == -INFINITY ? 0.0f : m_run[j];
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    pf[j][t >> 1][(t & 1) * 4 + i] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][t][i], c, -m_use));
        }
        // O^T[16u + 4*lq + i][query] += V^T . P^T; in 32-key step s, k-slot e of lane group
        // lq is key 32s + 16*(e/4) + 4*lq + (e%4).
#pragma unroll
        for (int u = 0; u < UT; u++)
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                const h4_t lo = RC ? ds_read_tr4(st + v_rd[u][s2][0]) : *(const h4_t*)(st + v_rd[u][s2][0]);
                const h4_t hi = RC ? ds_read_tr4(st + v_rd[u][s2][1]) : *(const h4_t*)(st + v_rd[u][s2][1]);
                const h8_t vf = cat8(lo, hi);
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[j][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[j][s2], acc[j][u], 0, 0, 0);
            }
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++)
                lsum[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[j][s2], lsum[j], 0, 0, 0);
    };
    for_each_stage<NS>(nblk, step);

    // Lane (lr, lq) holds O[query][16u + 4lq .. +3].  A row swap with the lane 16 apart
    // between dim blocks u = 2p and 2p+1 gives each lane eight consecutive dims (even lane
    // rows: block 2p+1 from 4lq; odd rows: block 2p from 4(lq-1)), stored as 16 bytes.  The
    // swaps run on every lane; only the store is predicated.
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float inv = 1.0f / lsum[j][0];
        _Float16* op = (_Float16*)a.o + (((size_t)b * S + min(query[j], S - 1)) * a.H_q + h) * D;
#pragma unroll
        for (int p = 0; p < UT / 2; p++) {
            const f4_t& x = acc[j][2 * p];
            const f4_t& y = acc[j][2 * p + 1];
            float ta[2], tb[2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                ta[k] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h2_t{(_Float16)(x[2 * k] * inv),
                                                                                   (_Float16)(x[2 * k + 1] * inv)}));
                tb[k] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h2_t{(_Float16)(y[2 * k] * inv),
                                                                                   (_Float16)(y[2 * k + 1] * inv)}));
                swap_xor16(tb[k], ta[k]);
            }
            if (query[j] < S)
                *(uint4*)(op + 32 * p + ((lq & 1) ? 0 : 16) + 8 * (lq >> 1)) =
                    uint4{__builtin_bit_cast(uint32_t, tb[0]), __builtin_bit_cast(uint32_t, tb[1]),
                          __builtin_bit_cast(uint32_t, ta[0]), __builtin_bit_cast(uint32_t, ta[1])};
        }
    }
  };
    if (!a.causal) {
        run(qi);
        return;
    }
    const int heavy = nqb - 1 - qi;
    if (!pairs) {
        run(heavy);
        return;
    }
    run(heavy);
    if (qi < heavy) {
        wait_vm<0>();                              // the first block's output stores
        ring_barrier();                            // every wave is done with the ring
        run(qi);
    }
}

// ---- fp32 (the FP32 operator's attention), d = 64 or 128: true fp32 on the matrix
// cores, v_mfma_f32_16x16x4_f32 (the reference FP32 path's bound is 1e-4, which fp16 or
// reduced-precision operands would not meet).  A workgroup owns 4 waves x 16*NJ queries;
// 64-key blocks of K ([key][dim]) and V^T ([dim][key]) go through a two-stage LDS ring,
// the next block loaded into registers while the current one is used.
// S^T = K.Q^T per 16-key tile: in MFMA step s, k-slot j (lane group l/16) stands for
// dim (D/4)*j + s, so a lane's K operand for all D/4 steps is one contiguous run of its
// key row (ds_read_b128), and Q^T stays in registers in the same order.  The result
// gives lane l scores of keys 4*(l/16) + e (e = 0..3) of query l%16; in P.V step kk the
// lane's own score e = kk is its B operand, which makes k-slot j stand for key
// 4j + kk, so the V^T operand of all four steps is one ds_read_b128 of its dim row.
// Online softmax in fp32 (exp2 of the scaled score minus the running max).
constexpr int kQB32 = 64;         // queries per workgroup per 16-query column block
template <int D, int NJ>
__global__ __launch_bounds__(kThreads, D == 64 ? 2 : 1)   // d = 128: 134 KB of LDS, one per CU
void flash_f32(cf_flash_args_t a) {
    constexpr int LDK = D + 4;        // floats per K row in LDS
    constexpr int LDV = kKB + 4;      // floats per V^T row in LDS
    constexpr int NS = D / 4;         // MFMA steps of S^T per 16-key tile
    constexpr int UT = D / 16;        // 16-dim tiles of O^T
    constexpr int K_ST = kKB * LDK, V_ST = D * LDV;
    constexpr int KCH = kKB * D / 4 / kThreads;   // float4 K chunks per thread per block
    constexpr int VCH = D * kKB / 4 / kThreads;   // float4 V^T chunks per thread per block
    constexpr int QB = kQB32 * NJ;                // queries per workgroup
    __shared__ __attribute__((aligned(16))) float smem[2 * (K_ST + V_ST)];

    const int nqb = (a.S + QB - 1) / QB;
    const int qi = blockIdx.x;
    const int qb = a.causal ? (nqb - 1 - qi) : qi;     // causal: heaviest blocks first
    const int h = blockIdx.y, b = blockIdx.z;
    const int S = a.S;
    const int kvh = h / (a.H_q / a.H_kv);
    const int q0 = qb * QB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int qw = q0 + 16 * NJ * wave;            // first query of this wave

    const float* __restrict__ qp = (const float*)a.q + (((size_t)b * a.H_q + h) * S) * D;
    const float* __restrict__ kp = (const float*)a.k + (((size_t)b * a.H_kv + kvh) * S) * D;
    const float* __restrict__ vp = (const float*)a.vt + (((size_t)b * a.H_kv + kvh) * D) * (size_t)S;

    int query[NJ];
    float qf[NJ][NS];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        query[j] = qw + 16 * j + lr;
#pragma unroll
        for (int v = 0; v < NS / 4; v++) {
            const f4_t x = query[j] < S ? *(const f4_t*)(qp + (size_t)query[j] * D + NS * lq + 4 * v) : f4_t{};
#pragma unroll
            for (int e = 0; e < 4; e++) qf[j][4 * v + e] = x[e];
        }
    }

    const float c = a.scale * kLog2e;
    float m_run[NJ], l_run[NJ];
    f4_t acc[NJ][UT];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        m_run[j] = -INFINITY;
        l_run[j] = 0.0f;
#pragma unroll
        for (int u = 0; u < UT; u++) acc[j][u] = f4_t{0.f, 0.f, 0.f, 0.f};
    }

    const int k_end = a.causal ? min(S, q0 + QB) : S;
    const bool v_vec = (S % 4) == 0;
    f4_t rk[KCH], rv[VCH];
    auto load_block = [&](int k0) {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int ch = tid + i * kThreads;
            const int r = ch / (D / 4), cc = (ch % (D / 4)) * 4;
            rk[i] = k0 + r < S ? *(const f4_t*)(kp + (size_t)(k0 + r) * D + cc) : f4_t{};
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            const int ch = tid + i * kThreads;
            const int dm = ch / (kKB / 4), kc = (ch % (kKB / 4)) * 4;
            const float* src = vp + (size_t)dm * S + k0 + kc;
            f4_t v{};
            if (v_vec && k0 + kc + 4 <= S) v = *(const f4_t*)src;
            else {
#pragma unroll
                for (int e = 0; e < 4; e++) if (k0 + kc + e < S) v[e] = src[e];
            }
            rv[i] = v;
        }
    };
    auto store_block = [&](int stage) {
        float* Ks = smem + stage * (K_ST + V_ST);
        float* Vs = Ks + K_ST;
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int ch = tid + i * kThreads;
            *(f4_t*)&Ks[(ch / (D / 4)) * LDK + (ch % (D / 4)) * 4] = rk[i];
        }
#pragma unroll
        for (int i = 0; i < VCH; i++) {
            const int ch = tid + i * kThreads;
            *(f4_t*)&Vs[(ch / (kKB / 4)) * LDV + (ch % (kKB / 4)) * 4] = rv[i];
        }
    };

    const int nblk = (k_end + kKB - 1) / kKB;
    load_block(0);
    store_block(0);
    __syncthreads();
    for (int bi = 0; bi < nblk; bi++) {
        const int k0 = bi * kKB;
        if (bi + 1 < nblk) load_block(k0 + kKB);
        const float* Ks = smem + (bi & 1) * (K_ST + V_ST);
        const float* Vs = Ks + K_ST;

        // st[j][t][e] = score(key k0 + 16t + 4*lq + e, query[j]).
        f4_t st[NJ][4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int j = 0; j < NJ; j++) st[j][t] = f4_t{0.f, 0.f, 0.f, 0.f};
            const float* kr = &Ks[(16 * t + lr) * LDK + NS * lq];
#pragma unroll
            for (int v = 0; v < NS / 4; v++) {
                const f4_t kf = *(const f4_t*)(kr + 4 * v);
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        st[j][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[e], qf[j][4 * v + e], st[j][t], 0, 0, 0);
            }
        }
        const bool edge = (k0 + kKB > S) || (a.causal && k0 + kKB - 1 > qw);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (edge) {
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int key = k0 + 16 * t + 4 * lq + e;
                        if (key >= S || (a.causal && key > query[j])) st[j][t][e] = -INFINITY;
                    }
            }
            float mloc = st[j][0][0];
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int e = 0; e < 4; e++) mloc = fmaxf(mloc, st[j][t][e]);
            mloc = max_xor16(mloc);
            mloc = max_xor32(mloc);
            // Raw dot products; the scale folds into the exponent: p = 2^(s*c - m).
            const float m_new = fmaxf(m_run[j], mloc * c);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = exp2f(m_run[j] - m_use);
            m_run[j] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float pv = exp2f(__builtin_fmaf(st[j][t][e], c, -m_use));
                    st[j][t][e] = pv;
                    psum += pv;
                }
            l_run[j] = l_run[j] * alpha + psum;
#pragma unroll
            for (int u = 0; u < UT; u++) acc[j][u] *= alpha;
        }
        // O^T[16u + 4*lq + e][query] += V^T . P^T; step kk of key tile t: k-slot lq is
        // key k0 + 16t + 4*lq + kk.
#pragma unroll
        for (int u = 0; u < UT; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const f4_t vf = *(const f4_t*)&Vs[(16 * u + lr) * LDV + 16 * t + 4 * lq];
#pragma unroll
                for (int kk = 0; kk < 4; kk++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[j][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[kk], st[j][t][kk], acc[j][u], 0, 0, 0);
            }
        if (bi + 1 < nblk) store_block((bi + 1) & 1);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float l_tot = add_xor32(add_xor16(l_run[j]));
        if (query[j] < S) {
            const float inv = 1.0f / l_tot;
            float* op = (float*)a.o + (((size_t)b * S + query[j]) * a.H_q + h) * D;
#pragma unroll
            for (int u = 0; u < UT; u++) *(f4_t*)(op + 16 * u + 4 * lq) = acc[j][u] * inv;
        }
    }
}

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

// Threads (queries) per workgroup of the generic kernel: 64, or 32 when d > 64 so the
// two [threads][d+1] float arrays stay within 64 KB of LDS.
inline int gen_threads(int d) { return d > 64 ? 32 : 64; }

template <typename T>
__global__ __launch_bounds__(64)
void flash_generic(cf_flash_args_t a) {
    extern __shared__ float smem[];
    const int D = a.d, LD = a.d + 1;
    const int nt = blockDim.x;
    float* qs = smem;                     // [nt][D+1]
    float* os = smem + nt * LD;           // [nt][D+1]
    const int nqb = gridDim.x;
    const int qb = a.causal ? (nqb - 1 - (int)blockIdx.x) : (int)blockIdx.x;
    const int h = blockIdx.y, b = blockIdx.z, S = a.S;
    const int kvh = h / (a.H_q / a.H_kv);
    const int t = threadIdx.x;
    const int query = qb * nt + t;
    const T* __restrict__ qp = (const T*)a.q + (((size_t)b * a.H_q + h) * S) * D;
    const T* __restrict__ kp = (const T*)a.k + (((size_t)b * a.H_kv + kvh) * S) * D;
    const T* __restrict__ vp = (const T*)a.vt + (((size_t)b * a.H_kv + kvh) * D) * (size_t)S;
    float* qrow = qs + t * LD;
    float* orow = os + t * LD;
    const float c = a.scale * kLog2e;
    for (int i = 0; i < D; i++) {
        qrow[i] = query < S ? to_f(qp[(size_t)query * D + i]) : 0.0f;
        orow[i] = 0.0f;
    }
    float m_run = -INFINITY, l_run = 0.0f;
    const int k_end = a.causal ? min(S, query + 1) : S;
    for (int j = 0; j < k_end; j++) {
        const T* kr = kp + (size_t)j * D;
        float s = 0.0f;
        for (int i = 0; i < D; i++) s = __builtin_fmaf(qrow[i], to_f(kr[i]), s);
        const float x = s * c;
        const float m_new = fmaxf(m_run, x);
        const float alpha = exp2f(m_run - m_new);
        const float p = exp2f(x - m_new);
        l_run = l_run * alpha + p;
        for (int i = 0; i < D; i++) orow[i] = __builtin_fmaf(p, to_f(vp[(size_t)i * S + j]), orow[i] * alpha);
        m_run = m_new;
    }
    if (query < S) {
        T* op = (T*)a.o + (((size_t)b * S + query) * a.H_q + h) * D;
        const float inv = 1.0f / l_run;
        for (int i = 0; i < D; i++) op[i] = from_f<T>(orow[i] * inv);
    }
}

// Tuning/test switch for fp16 d = 64: 0 register-staged kernel, 1 DMA kernel with 32
// queries per wave, 2 DMA kernel with 16 per wave, 3 (default) DMA kernel, chosen by size.
int g_flash_mode = 3;
int g_flash_pairs = 0;   // causal DMA kernel: 1 pairs each query block with its mirror; 0 (default)
                         // one block per workgroup, heaviest first

}  // namespace

extern "C" void cf_flash_set_mode(int32_t mode) { g_flash_mode = mode >= 0 && mode <= 3 ? mode : 3; }
extern "C" void cf_flash_set_causal_pairs(int32_t on) { g_flash_pairs = on > 0 ? 1 : 0; }

extern "C" int32_t cf_flash_rowcat_ok(const cf_flash_args_t* a) {
    return a->elem == CF_ELEM_F16 && a->d == 64 && a->S > 0 && a->S % 8 == 0 && a->S <= (1 << 24) &&
           a->H_kv > 0 && a->H_q % a->H_kv == 0 && a->scale > 0.0f &&
           a->qkv_ld == (a->H_q + 2 * a->H_kv) * 64 && ((uintptr_t)a->q | (uintptr_t)a->o) % 16 == 0;
}

extern "C" int cf_launch_flash_attn(const cf_flash_args_t* a, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (a->S <= 0 || a->d <= 0 || a->H_kv <= 0 || a->H_q % a->H_kv != 0) return (int)hipErrorInvalidValue;
    if (a->qkv_ld != 0 && !cf_flash_rowcat_ok(a)) return (int)hipErrorInvalidValue;
    const bool aligned = a->qkv_ld ? true : ((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->vt | (uintptr_t)a->o) % 16 == 0;
    // The fast kernel takes the row max of raw scores and scales it, valid for scale > 0.
    if (a->elem == CF_ELEM_F16 && aligned && (a->d == 64 || a->d == 128) && a->scale > 0.0f) {
        const long long nqb = (a->S + kQB - 1) / kQB;
        const long long groups = ((long long)a->B * a->H_q + 7) / 8;
        if (groups * nqb * 8 > 0x7fffffffLL) return (int)hipErrorInvalidValue;
        dim3 grid((unsigned)(groups * nqb * 8));
        // The DMA kernel addresses V^T rows with 32-bit byte offsets: 64 * S * 2 < 2^32.
        if (a->d == 64 && a->S % 8 == 0 && a->S <= (1 << 24) && (g_flash_mode != 0 || a->qkv_ld)) {
            // 16 queries per wave (64 per workgroup) doubles the workgroups, and with
            // them the waves per SIMD that hide each block's latency chain; 32 per wave
            // halves the LDS traffic per query (every wave reads the whole K/V^T block),
            // better once there are two 128-query workgroups per CU.
            // Causal: one query block per workgroup, the heaviest blocks of every head
            // first, so the CUs that finish early take the light ones.  Pairing each block
            // with its mirror (equal work per workgroup, half as many) measured slower at
            // 16-query waves: S = 512, 96 heads 12.3 against 9.35 us; S = 1024, 64 heads
            // 18.5 against 17.3 us; S = 2048, 32 heads 30.6 against 26.7 us.  The query
            // width is still chosen as if paired (32-query waves only with two paired
            // workgroups per CU), which keeps config 5 on 16-query waves.
            auto nblocks = [&](int nj) { return (a->S + 64LL * nj - 1) / (64LL * nj); };
            auto pair_slots = [&](int nj) { return a->causal ? (nblocks(nj) + 1) / 2 : nblocks(nj); };
            const int nj = g_flash_mode == 1 ? 2 : g_flash_mode == 2 ? 1
                         : (groups * pair_slots(2) * 8 < 2LL * cu_count() ? 1 : 2);
            const int pairs = a->causal && g_flash_pairs ? 1 : 0;
            const long long nslot = pairs ? pair_slots(nj) : nblocks(nj);
            dim3 grid2((unsigned)(groups * nslot * 8));
            // The kernel's grid decomposition divides by these (measured: ~0.45 us of
            // config 5's attention as runtime divisions in every workgroup's prologue).
            const FastDiv dslot = fastdiv_make((int)(a->causal && !pairs ? groups : nslot));
            const FastDiv dhq = fastdiv_make(a->H_q), dg = fastdiv_make(a->H_q / a->H_kv);
            if (a->qkv_ld) {
                if (nj == 1) hipLaunchKernelGGL((flash_f16_dma64<1, true>), grid2, dim3(kThreads), 0, s, *a, pairs, dslot, dhq, dg);
                else hipLaunchKernelGGL((flash_f16_dma64<2, true>), grid2, dim3(kThreads), 0, s, *a, pairs, dslot, dhq, dg);
            } else if (nj == 1) hipLaunchKernelGGL(flash_f16_dma64<1>, grid2, dim3(kThreads), 0, s, *a, pairs, dslot, dhq, dg);
            else hipLaunchKernelGGL(flash_f16_dma64<2>, grid2, dim3(kThreads), 0, s, *a, pairs, dslot, dhq, dg);
        } else if (a->d == 64) hipLaunchKernelGGL(flash_f16<64>, grid, dim3(kThreads), 0, s, *a);
        else hipLaunchKernelGGL(flash_f16<128>, grid, dim3(kThreads), 0, s, *a);
        return (int)hipGetLastError();
    }
    if (a->elem == CF_ELEM_F32 && aligned && (a->d == 64 || a->d == 128) && a->scale > 0.0f) {
        // 32 queries per wave where that still gives two workgroups per CU, else 16.
        const long long bh = (long long)a->B * a->H_q;
        const int nj = bh * ((a->S + 2 * kQB32 - 1) / (2 * kQB32)) >= 2LL * cu_count() ? 2 : 1;
        dim3 grid((unsigned)((a->S + nj * kQB32 - 1) / (nj * kQB32)), (unsigned)a->H_q, (unsigned)a->B);
        if (a->d == 64) {
            if (nj == 2) hipLaunchKernelGGL((flash_f32<64, 2>), grid, dim3(kThreads), 0, s, *a);
            else hipLaunchKernelGGL((flash_f32<64, 1>), grid, dim3(kThreads), 0, s, *a);
        } else {
            if (nj == 2) hipLaunchKernelGGL((flash_f32<128, 2>), grid, dim3(kThreads), 0, s, *a);
            else hipLaunchKernelGGL((flash_f32<128, 1>), grid, dim3(kThreads), 0, s, *a);
        }
        return (int)hipGetLastError();
    }
    if (a->d > 240) return (int)hipErrorInvalidValue;
    const int nt = gen_threads(a->d);
    dim3 grid((unsigned)((a->S + nt - 1) / nt), (unsigned)a->H_q, (unsigned)a->B);
    const size_t lds = (size_t)2 * nt * (a->d + 1) * sizeof(float);
    if (a->elem == CF_ELEM_F16) hipLaunchKernelGGL(flash_generic<_Float16>, grid, dim3(nt), lds, s, *a);
    else hipLaunchKernelGGL(flash_generic<float>, grid, dim3(nt), lds, s, *a);
    return (int)hipGetLastError();
}
