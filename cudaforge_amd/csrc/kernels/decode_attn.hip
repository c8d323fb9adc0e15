// decode_attn.hip — split-KV single-token attention over a KV cache for gfx950.
//
// Replaces the reference's one-block-per-batch-row decode kernel
// (src/operator/nn/mha_decode_cuda.cu:11-157).  Two launches:
//
// 1. split kernel, grid = (split, kv head, batch row).  A workgroup streams one `chunk`
//    of positions of one (b, kv head) and serves the whole GQA group of G query heads
//    (kv head = h / G, mha_decode.c:77) from a single read of every K and V row, and
//    writes a partial (m, l = sum p, acc = sum p*v) in the log2 domain.
//    fp16 (d = 64/128, G = 1/2/4/8): one wave per workgroup, single pass with an online
//      softmax over 32-position blocks that arrive by DMA in an LDS ring; both products
//      on the matrix cores (see split_f16).
//    fp32 (d = 64/128): four waves, two passes over LDS-resident scores (pass 1 streams
//      K and stores s = q.k * scale*log2(e), pass 2 streams V with p = 2^(s - m)); lanes
//      own 4 dims of a row and dot products are reduced across the row's lanes.
//    Other head or group sizes: a generic kernel, one query head per workgroup.
// 2. merge kernel: the log-sum-exp combine
//      O = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s
//    (the reference's split/merge formula, mha_fused_cuda.cu:847-863 and :895-931,
//    restated per (b, head) with the head index it lacked); one workgroup per output
//    row (merge_rows), or one thread per element when d % 4 != 0.  A sequence that fits
//    in one split is finished by the split kernel and skipped here.
// No fences or atomics: the kernel boundary orders the partials, which matters on
// MI355X where each XCD has its own L2.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "cdna4.h"

namespace {

using namespace cdna4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyMax = 8.0f;           // fp16 split kernel: max headroom of p (log2 units)
constexpr int kChunkMax = 4096;            // positions per split of the fp32 / generic kernels
                                           // (their scores live in LDS: chunk * G floats)
constexpr int kChunkMaxF16 = 1 << 20;      // fp16 split kernel: LDS use is independent of the chunk
constexpr int kF16Quantum = 32;            // fp16 split kernel: positions per block
constexpr int kDecodeStages = 3;           // fp16 split kernel: default LDS ring depth (16 KB per stage at d = 128;
                                           // 3 stages = 3 workgroups per CU, best measured with HBM-resident KV)
constexpr int kLdsPerCu = 160 * 1024;      // LDS of one gfx950 CU
constexpr int kF32Threads = 256;
constexpr int kF32Unroll = 4;
constexpr int kGenericThreads = 128;
constexpr int kMergeThreads = 256;
constexpr int kMergeWaveSplits = 16;       // merge_wave holds every split in registers

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

__device__ __forceinline__ int attended(const cf_decode_attn_args_t& a, int b) {
    const int cl = a.seq_lens ? a.seq_lens[b] : a.cache_len;
    return min(max(cl + 1, 1), a.max_seq);
}

// Partial record of one split: [m (Gx)] [l (Gx)] [pad to 4 floats] [acc (Gx*D)], so
// every record and its acc block start 16-byte aligned when D % 4 == 0.
__host__ __device__ constexpr int part_hdr(int Gx) { return (2 * Gx + 3) & ~3; }
__host__ __device__ constexpr int part_stride(int Gx, int D) { return part_hdr(Gx) + Gx * D; }

__device__ __forceinline__ float* partial_at(const cf_decode_attn_args_t& a, int unit, int split, int Gx, int D) {
    return a.partials + ((size_t)unit * a.n_split + split) * (size_t)part_stride(Gx, D);
}

// Balanced ragged split (a.balanced, grouped fp16 kernel): every workgroup takes one
// contiguous range of one sequence, and the ranges are about equal across the batch.
// With W = sum of the attended lengths T_b and L = ceil(W / (n_split - B)), sequence b
// gets ns_b = ceil(T_b / L) workgroups of C_b = ceil(T_b / ns_b) positions (ns_b then
// recounted as ceil(T_b / C_b), so no range is empty): sum ns_b <= W / L + B <= n_split,
// and no workgroup holds more than L positions.  (Ranges that straddled two sequences
// paid a second ring fill and drain, and those workgroups set the kernel's end.)
// Sequence b's workgroups are first_b .. first_b + ns_b - 1; workgroup w writes record
// (w, kv head) at w * H_kv + kv head, so b's records are contiguous from first_b.
// Every lane of the calling wave gets the geometry (B <= 64: lane b holds sequence b's
// figures), from one load per lane, a wave sum and a wave prefix sum.
struct BalancedGeom {
    int W;             // total attended positions
    int used;          // workgroups with a range (sum of ns_b)
    int T, ns, C;      // lane b: T_b, its workgroups, positions per workgroup
    int first;         // lane b: its first workgroup (= its first record piece)
};
__device__ __forceinline__ BalancedGeom balanced_geom(const cf_decode_attn_args_t& a) {
    const int lane = threadIdx.x & 63;
    BalancedGeom g;
    g.T = lane < a.B ? attended(a, lane) : 0;
    const int P = wave_excl_sum(g.T, lane);
    g.W = __builtin_amdgcn_readlane(P + g.T, 63);
    const int avail = max(a.n_split - a.B, 1);           // the launcher keeps n_split >= 2B
    const int L = max((g.W + avail - 1) / avail, 1);
    int ns = (g.T + L - 1) / L;
    g.C = ns > 0 ? (g.T + ns - 1) / ns : 0;
    g.ns = g.C > 0 ? (g.T + g.C - 1) / g.C : 0;
    g.first = wave_excl_sum(g.ns, lane);
    g.used = __builtin_amdgcn_readlane(g.first + g.ns, 63);
    return g;
}

// The range of workgroup w (< geo.used) in the balanced split: its sequence b and
// positions [t0, t1) of it, and the number of workgroups b has.
struct BalancedRange { int b, t0, t1, ns; };
__device__ __forceinline__ BalancedRange balanced_range(const cf_decode_attn_args_t& a, const BalancedGeom& geo, int w) {
    const int lane = threadIdx.x & 63;
    // b = the last sequence whose first workgroup is at or before w (sequences have ns >= 1).
    const unsigned long long m = __ballot(lane < a.B && geo.first <= w);
    const int b = 63 - __builtin_clzll(m);
    const int first = __builtin_amdgcn_readlane(geo.first, b), C = __builtin_amdgcn_readlane(geo.C, b);
    const int T = __builtin_amdgcn_readlane(geo.T, b), t0 = (w - first) * C;
    return {b, t0, min(t0 + C, T), __builtin_amdgcn_readlane(geo.ns, b)};
}

// The splits of (b, unit): their count and where split s's record is (first + s * step
// records of `stride` floats).
struct SplitRecords { int n; const float* first; size_t step; };
// The merge launches' divisors (FastDiv): the row's group size Gx, the units per batch
// row, and the split length.
struct MergeDivs { FastDiv gx, ub, chunk; };
__device__ __forceinline__ SplitRecords split_records(const cf_decode_attn_args_t& a, int b, int unit,
                                                      int units_per_b, int stride, const MergeDivs& md) {
    if (!a.balanced) {
        const int T_b = attended(a, b);
        return {fastdiv(T_b + a.chunk - 1, md.chunk), a.partials + (size_t)unit * a.n_split * stride, (size_t)stride};
    }
    const BalancedGeom geo = balanced_geom(a);
    const int ns = __builtin_amdgcn_readlane(geo.ns, b), first = __builtin_amdgcn_readlane(geo.first, b);
    return {ns, a.partials + ((size_t)first * a.H_kv + (unit - b * units_per_b)) * stride, (size_t)a.H_kv * stride};
}

// ------------------------------------------------------------------ fp16 split ---
// One wave streams `chunk` positions of one (b, kv head) for its whole GQA group, in
// blocks of 32 positions.  K and V rows go straight from HBM into an NS-stage LDS ring
// (global_load_lds_dwordx4, no VGPR staging), so NS-1 blocks (16 KB each at d = 128) are
// in flight while one is computed.  Per block, on the matrix cores:
//   scores  S^T (16 positions x 16 heads) = K (16 x 32 dims) . Q^T, two row blocks:
//           lane (lr, lq) gets positions 4lq..4lq+3 and 16+4lq..16+4lq+3 of head lr;
//   values  O^T (16 dims x 16 heads) += V^T (16 dims x 32 positions) . P^T, one MFMA per
//           16 dims.  The k index of that MFMA runs over the block's positions in the
//           order the score lanes already hold them, so P^T is the lane's own 8
//           probabilities converted to fp16; V^T comes from the LDS ring with
//           ds_read_b64_tr_b16 (4 positions of one dim per read) in the same order.
// Online softmax per block: m <- max(m, block max), alpha = 2^(m_old - m) rescales the
// lane's accumulator columns (each lane's column is its own head), p = 2^(s - m).
// LDS rows are XOR-swizzled in 16-byte chunks (kswz for the K fragment reads, vswz for
// the transposing V reads) so both read patterns are bank-conflict free.
template <int D>
__device__ __forceinline__ int kswz(int row) { return (row / (128 / D)) % (D / 8); }
template <int D>
__device__ __forceinline__ int vswz(int row) { return 2 * ((row / (128 / D)) % (D / 16)); }

// WIDE: one workgroup per (split, b) with one wave per KV head (H_kv <= 8 waves), each
// wave streaming its head's 16-position blocks through its own 2-stage ring.  The waves
// of a workgroup read the same cache rows at about the same time, so the DRAM sees whole
// rows (all KV heads) instead of one head's slice at a time: a streaming probe with the
// config-2 layout reads 6.1 TB/s this way against 5.5-5.9 TB/s with one workgroup per
// (split, KV head).  With 16 positions per block, P.V runs on v_mfma_f32_16x16x16_f16,
// whose B operand is exactly the four probabilities a score lane holds.
// Positions [t0, t1) of (b, kv head kvh) through one wave's ring: the partial goes to
// `part`, or, when part is null (the range is the whole sequence), O itself.
template <int D, int G, int NS, bool WIDE>
__device__ __forceinline__ void split_range(const cf_decode_attn_args_t& a, _Float16* ring, int b, int kvh,
                                            int t0, int t1, float* part) {
    constexpr int KT = D / 32;          // 32-dim MFMA steps per 16 positions
    constexpr int BP = WIDE ? 16 : 32;  // positions per block
    constexpr int NH = BP / 16;         // 16-position row blocks per block
    constexpr int CPR = D / 8;          // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;       // rows per DMA instruction (1 KB)
    constexpr int NI = BP / RPI;        // DMA instructions per block per tensor
    constexpr int NL = 2 * NI;          // ... for K and V
    constexpr int TILE = BP * D;        // halves per block per tensor
    constexpr int NT = D / 16;          // output tiles of 16 dims
    constexpr int HDR = part_hdr(G);
    static_assert((NS - 1) * NL < 64, "vmcnt range");
    constexpr int QH = (G * D * 2 + 1023) / 1024 * 512;   // halves of the Q area (whole DMA KBs)
    const int nblk = (t1 - t0 + BP - 1) / BP;
    const int lane = threadIdx.x & 63, lr = lane & 15, lq = lane >> 4;
    wait_lds_reads();                                     // a previous range's reads of the ring

    const size_t row_stride = (size_t)a.H_kv * D;
    const size_t unit_off = ((size_t)b * a.max_seq * a.H_kv + kvh) * D;
    const _Float16* __restrict__ kg = (const _Float16*)a.k + unit_off;
    const _Float16* __restrict__ vg = (const _Float16*)a.v + unit_off;
    const int h0 = kvh * G;

    const float qk_scale = a.scale * kLog2e;

    // DMA: instruction u of a block fills rows RPI*u .. +RPI-1; lane L writes physical
    // chunk L % CPR of row RPI*u + L / CPR, which holds logical chunk (L % CPR) ^ swz(row).
    // A full block is addressed as a uniform base (its first row) plus per-lane 32-bit
    // offsets fixed for the whole loop; in the last, partial block rows past t1 are
    // clamped to row t1 - 1 (always valid) and those positions get p = 0.
    const uint32_t ring_base = lds_offset(ring);
    const int drow = lane / CPR, dchunk = lane % CPR;
    const uint32_t row_bytes = (uint32_t)row_stride * 2u;
    uint32_t koff[NI], voff[NI];
#pragma unroll
    for (int u = 0; u < NI; u++) {
        const int row = RPI * u + drow;
        koff[u] = (uint32_t)row * row_bytes + 16u * (uint32_t)(dchunk ^ kswz<D>(row));
        voff[u] = (uint32_t)row * row_bytes + 16u * (uint32_t)(dchunk ^ vswz<D>(row));
    }
    auto issue = [&](int blk, int stage) {           // stage == blk % NS
        const int p0 = t0 + blk * BP;
        const uint32_t kbase = ring_base + (uint32_t)(stage * 2 * TILE) * 2u;
        const uint32_t vbase = kbase + (uint32_t)TILE * 2u;
        if (p0 + BP <= t1) {
            const _Float16* kblk = kg + (size_t)p0 * row_stride;
            const _Float16* vblk = vg + (size_t)p0 * row_stride;
#pragma unroll
            for (int u = 0; u < NI; u++) {
                lds_dma16_s(koff[u], kblk, kbase + u * 1024u);
                lds_dma16_s(voff[u], vblk, vbase + u * 1024u);
            }
        } else {
#pragma unroll
            for (int u = 0; u < NI; u++) {
                const int row = RPI * u + drow;
                const size_t g_row = (size_t)min(p0 + row, t1 - 1) * row_stride;
                lds_dma16(kg + g_row + 8 * (dchunk ^ kswz<D>(row)), kbase + u * 1024u);
                lds_dma16(vg + g_row + 8 * (dchunk ^ vswz<D>(row)), vbase + u * 1024u);
            }
        }
    };

    // Per-lane LDS read offsets (halves) inside a stage.
    int k_rd[NH][KT];
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int kt = 0; kt < KT; kt++) {
            const int row = 16 * h + lr;
            k_rd[h][kt] = row * D + 8 * ((4 * kt + lq) ^ kswz<D>(row));
        }
    int v_rd[NT][NH];
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            const int row = 16 * hh + 4 * lq + (lr >> 2);
            const int col = 16 * n + 4 * (lr & 3);                  // halves
            v_rd[n][hh] = TILE + row * D + 8 * ((col >> 3) ^ vswz<D>(row)) + (col & 7);
        }

    f4_t acc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = f4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;      // head lr; lanes lr < G are meaningful

    // Q (G rows of D halves, contiguous) also arrives by DMA, ahead of the first block,
    // so the kernel issues no compiler-visible global loads whose waits would drain the
    // ring; lanes past the G*D*2 bytes re-read the last 16 bytes of Q (never used).
    {
        const _Float16* qg = (const _Float16*)a.q + ((size_t)b * a.H_q + h0) * D;
        const uint32_t qbase = ring_base + (uint32_t)(NS * 2 * TILE) * 2u;
#pragma unroll
        for (int u = 0; u < QH / 512; u++)
            lds_dma16(qg + min(8 * (64 * u + lane), G * D - 8), __builtin_amdgcn_readfirstlane(qbase + u * 1024u));
    }
#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < nblk) issue(s, s);
    // B operand Q^T: lane (lr, lq) holds Q[head lr][32kt + 8lq .. +7]; heads >= G are 0.
    h8_t qf[KT];

    // One block; its ring stage is a compile-time constant (for_each_stage).
    auto step = [&](int blk, auto stage_c) {
        constexpr int stage = decltype(stage_c)::value;
        // Refill the stage of the previous block before waiting for this one, so all NS
        // stages are in flight during the wait.  That block's LDS reads have returned
        // (their values fed its MFMAs): a single wave needs no barrier.
        if (blk + NS - 1 < nblk) {
            wait_lds_reads();
            issue(blk + NS - 1, (stage + NS - 1) % NS);
        }
        // Blocks issued after this one that may still be in flight.
        wait_ahead<NL, NS - 1>(min(NS - 1, nblk - 1 - blk));
        if (stage == 0 && blk == 0) {                // Q landed with block 0
            const _Float16* qs = ring + NS * 2 * TILE + min(lr, G - 1) * D + 8 * lq;
#pragma unroll
            for (int kt = 0; kt < KT; kt++) qf[kt] = lr < G ? *(const h8_t*)(qs + 32 * kt) : h8_t{};
        }

        const _Float16* st = ring + stage * 2 * TILE;
        f4_t s[NH];
#pragma unroll
        for (int h = 0; h < NH; h++) {
            s[h] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < KT; kt++)
                s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const h8_t*)(st + k_rd[h][kt]), qf[kt], s[h], 0, 0, 0);
        }
        // Raw scores; positions past t1 (last block only) -> -inf.  scale > 0, so the
        // max of the raw scores times scale*log2(e) is the max of the scaled ones.
        const int p0 = t0 + blk * BP;
        float x[4 * NH];
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) x[4 * h + j] = s[h][j];
        if (p0 + BP > t1) {
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (p0 + 16 * h + 4 * lq + j >= t1) x[4 * h + j] = -INFINITY;
        }
        float mb = x[0];
#pragma unroll
        for (int i = 1; i < 4 * NH; i++) mb = fmaxf(mb, x[i]);
        mb = max_xor32(max_xor16(mb)) * qk_scale;                   // finite: p0 < t1
        // The running max moves only when a block exceeds it by more than kLazyMax (log2
        // units): until then p = 2^(s - m) <= 2^kLazyMax, exact enough in fp16 and far
        // from its range limit, and the accumulators need no rescaling.  The first block
        // always moves it (m = -inf).  The rescale runs only if some head moved (a
        // wave-uniform branch), so the accumulators normally stay in the matrix unit.
        const bool grow = mb > m_run + kLazyMax;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float m_new = grow ? mb : m_run;                    // finite: p0 < t1
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // 0 on the first block
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int n = 0; n < NT; n++) acc[n] *= alpha;
        }
        float ps = 0.0f;
        _Float16 pv[4 * NH];
#pragma unroll
        for (int i = 0; i < 4 * NH; i++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], qk_scale, -m_run));
            ps += p;
            pv[i] = (_Float16)p;
        }
        l_run += ps;
        if constexpr (NH == 2) {
            const h8_t pf = {pv[0], pv[1], pv[2], pv[3], pv[4], pv[5], pv[6], pv[7]};
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const h8_t vf = cat8(ds_read_tr4(st + v_rd[n][0]), ds_read_tr4(st + v_rd[n][1]));
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, acc[n], 0, 0, 0);
            }
        } else {
            const h4_t pf = {pv[0], pv[1], pv[2], pv[3]};
#pragma unroll
            for (int n = 0; n < NT; n++)
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ds_read_tr4(st + v_rd[n][0]), pf, acc[n], 0, 0, 0);
        }
    };
    for_each_stage<NS>(nblk, step);

    // l: the lanes of one head hold partial sums over their positions.
    l_run = add_xor32(add_xor16(l_run));
    if (lr >= G) return;
    // Lane (lr, lq) holds O^T rows d = 16n + 4lq + i of head h0 + lr.
    if (!part) {
        const float inv = 1.0f / l_run;
        _Float16* out = (_Float16*)a.o + ((size_t)b * a.H_q + h0 + lr) * D + 4 * lq;
#pragma unroll
        for (int n = 0; n < NT; n++) {
            h4_t o;
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = (_Float16)(acc[n][i] * inv);
            *(h4_t*)(out + 16 * n) = o;
        }
        return;
    }
#pragma unroll
    for (int n = 0; n < NT; n++) *(f4_t*)(part + HDR + lr * D + 16 * n + 4 * lq) = acc[n];
    if (lq == 0) {
        part[lr] = m_run;
        part[G + lr] = l_run;
    }
}

// K in registers (grouped kernel): the score MFMA's A operand is 16 contiguous bytes of
// one K row per lane (row lr, dims 32kt + 8lq .. +7), so K goes straight from HBM into
// VGPRs with ordinary loads and only V, which the value MFMA needs transposed, takes the
// LDS ring.  That frees the ring for V alone: NSV stages of 16 positions, NV = NSV - 1
// blocks of V in flight, and K runs NK = P - 1 blocks ahead in P rotating register sets.
// Per block a wave issues KT K loads (compiler-visible) then NI V DMAs (inline asm).
// Waits: vmcnt counts both kinds, but a DMA into LDS and a load into VGPRs issued after
// it do not complete in issue order relative to each other (measured: counting the K
// loads issued after V[j] as complete let the value MFMA read a stage before its DMA had
// landed), while each kind completes in order within itself.  So the wait for V[j]
// allows only the V DMAs issued after it to be outstanding, vmcnt(NI * ahead), whatever
// the K loads are doing; that also leaves at most NI * NV <= KT * NK of the K loads issued
// after K[j] outstanding, so K[j] has landed too.  The compiler's own wait before K[j]'s
// first use counts only K loads and is then already met.
// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled.
template <typename F, int... S>
__device__ __forceinline__ void static_for_seq(F& f, std::integer_sequence<int, S...>) {
    (f(std::integral_constant<int, S>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

template <int D>
struct KvRing {
    static constexpr int KT = D / 32;        // 32-dim MFMA steps (K loads per block per lane)
    static constexpr int CPR = D / 8;        // 16-byte chunks per row
    static constexpr int RPI = 64 / CPR;     // rows per V DMA instruction (1 KB)
    static constexpr int NI = 16 / RPI;      // V DMA instructions per 16-position block
    static constexpr int TILE = 16 * D;      // halves of one V stage
    static constexpr int NT = D / 16;        // output tiles of 16 dims
};

template <int D, int G, int NSV, int P>
__device__ __forceinline__ void split_range_kv(const cf_decode_attn_args_t& a, _Float16* ring, int b, int kvh,
                                               int t0, int t1, float* part) {
    using R = KvRing<D>;
    constexpr int KT = R::KT, CPR = R::CPR, RPI = R::RPI, NI = R::NI, TILE = R::TILE, NT = R::NT;
    constexpr int NV = NSV - 1, NK = P - 1;
    constexpr int HDR = part_hdr(G);
    static_assert(NI * NV <= KT * NK, "the V wait also covers K[j]");
    static_assert(NI * NV < 64, "vmcnt range");
    const int nblk = (t1 - t0 + 15) / 16;
    const int lane = threadIdx.x & 63, lr = lane & 15, lq = lane >> 4;
    wait_lds_reads();                                     // a previous range's reads of the ring

    const uint32_t row_stride = (uint32_t)a.H_kv * D;     // halves
    const size_t unit_off = ((size_t)b * a.max_seq * a.H_kv + kvh) * D;
    const _Float16* __restrict__ kg = (const _Float16*)a.k + unit_off;
    const _Float16* __restrict__ vg = (const _Float16*)a.v + unit_off;
    const int h0 = kvh * G;
    const float qk_scale = a.scale * kLog2e;

    // Q^T (B operand): lane (lr, lq) holds Q[head lr][32kt + 8lq .. +7]; heads >= G are 0.
    h8_t qf[KT];
    {
        const _Float16* qs = (const _Float16*)a.q + ((size_t)b * a.H_q + h0 + min(lr, G - 1)) * D + 8 * lq;
#pragma unroll
        for (int kt = 0; kt < KT; kt++) qf[kt] = *(const h8_t*)(qs + 32 * kt);
#pragma unroll
        for (int kt = 0; kt < KT; kt++)
            if (lr >= G) qf[kt] = h8_t{};
    }

    // K rows as a uniform base plus a 32-bit per-lane byte offset (the saddr form of
    // global_load_dwordx4: no per-lane 64-bit addresses held across the loop).
    h8_t kf[P][KT];
    const char* kgb = (const char*)kg;
    auto load_k = [&](int blk, auto set_c) {
        constexpr int set = decltype(set_c)::value;
        const uint32_t row = (uint32_t)min(t0 + 16 * blk + lr, t1 - 1);
        const uint32_t off = row * row_stride * 2u + 16u * (uint32_t)lq;
#pragma unroll
        for (int kt = 0; kt < KT; kt++) kf[set][kt] = *(const h8_t*)(kgb + off + 64u * kt);
    };

    const uint32_t ring_base = lds_offset(ring);
    const int drow = lane / CPR, dchunk = lane % CPR;
    uint32_t voff[NI];
#pragma unroll
    for (int u = 0; u < NI; u++) {
        const int row = RPI * u + drow;
        voff[u] = (uint32_t)row * row_stride * 2u + 16u * (uint32_t)(dchunk ^ vswz<D>(row));
    }
    auto issue_v = [&](int blk, int stage) {
        const int p0 = t0 + 16 * blk;
        const uint32_t vbase = ring_base + (uint32_t)(stage * TILE) * 2u;
        if (p0 + 16 <= t1) {
            const _Float16* vblk = vg + (size_t)p0 * row_stride;
#pragma unroll
            for (int u = 0; u < NI; u++) lds_dma16_s(voff[u], vblk, vbase + u * 1024u);
        } else {
#pragma unroll
            for (int u = 0; u < NI; u++) {
                const int row = RPI * u + drow;
                const size_t g_row = (size_t)min(p0 + row, t1 - 1) * row_stride;
                lds_dma16(vg + g_row + 8 * (dchunk ^ vswz<D>(row)), vbase + u * 1024u);
            }
        }
    };
    int v_rd[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int row = 4 * lq + (lr >> 2);
        const int col = 16 * n + 4 * (lr & 3);
        v_rd[n] = row * D + 8 * ((col >> 3) ^ vswz<D>(row)) + (col & 7);
    }

    f4_t acc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = f4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;

    // Prologue: the issue order of steps -NK .. -1 (K of blocks 0 .. NK-1, V of 0 .. NV-1).
    static_for<NK>([&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        load_k(S, s_c);
        if (S >= NK - NV && S - (NK - NV) < nblk) issue_v(S - (NK - NV), S - (NK - NV));
    });

    // The V stage is a runtime index (blk % NSV, kept in an SGPR), so the K register
    // rotation P need not be a multiple of NSV.
    int stage = 0;
    auto step = [&](int blk, auto set_c) {
        constexpr int set = decltype(set_c)::value;           // == blk % P
        load_k(blk + NK, std::integral_constant<int, (set + NK) % P>{});
        if (blk + NV < nblk) {
            wait_lds_reads();                                  // block blk - 1's reads of that stage
            issue_v(blk + NV, stage == 0 ? NV : stage - 1);    // (blk + NV) % NSV
        }
        wait_ahead<NI, NV>(min(NV, nblk - 1 - blk));

        f4_t s = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < KT; kt++) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[set][kt], qf[kt], s, 0, 0, 0);
        const int p0 = t0 + 16 * blk;
        float x[4] = {s[0], s[1], s[2], s[3]};
        if (p0 + 16 > t1) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (p0 + 4 * lq + j >= t1) x[j] = -INFINITY;
        }
        float mb = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        mb = max_xor32(max_xor16(mb)) * qk_scale;
        const bool grow = mb > m_run + kLazyMax;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float m_new = grow ? mb : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int n = 0; n < NT; n++) acc[n] *= alpha;
        }
        float ps = 0.0f;
        _Float16 pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], qk_scale, -m_run));
            ps += p;
            pv[i] = (_Float16)p;
        }
        l_run += ps;
        const h4_t pf = {pv[0], pv[1], pv[2], pv[3]};
        const _Float16* st = ring + stage * TILE;
#pragma unroll
        for (int n = 0; n < NT; n++)
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ds_read_tr4(st + v_rd[n]), pf, acc[n], 0, 0, 0);
        stage = stage == NSV - 1 ? 0 : stage + 1;
    };
    // Whole groups of P blocks unconditionally (the same loads on every path, so the
    // compiler's waits hold across the back edge), then the last nblk % P blocks.
    int i0 = 0;
    for (; i0 + P <= nblk; i0 += P) static_for<P>([&](auto s_c) { step(i0 + decltype(s_c)::value, s_c); });
    static_for<P - 1>([&](auto s_c) {
        if (i0 + decltype(s_c)::value < nblk) step(i0 + decltype(s_c)::value, s_c);
    });

    l_run = add_xor32(add_xor16(l_run));
    if (lr >= G) return;
    if (!part) {
        const float inv = 1.0f / l_run;
        _Float16* out = (_Float16*)a.o + ((size_t)b * a.H_q + h0 + lr) * D + 4 * lq;
#pragma unroll
        for (int n = 0; n < NT; n++) {
            h4_t o;
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = (_Float16)(acc[n][i] * inv);
            *(h4_t*)(out + 16 * n) = o;
        }
        return;
    }
#pragma unroll
    for (int n = 0; n < NT; n++) *(f4_t*)(part + HDR + lr * D + 16 * n + 4 * lq) = acc[n];
    if (lq == 0) {
        part[lr] = m_run;
        part[G + lr] = l_run;
    }
}

template <int D, int G, int NS, bool WIDE = false>
__global__ __launch_bounds__(WIDE ? 512 : 64)
void split_f16(cf_decode_attn_args_t a) {
    constexpr int BP = WIDE ? 16 : 32;
    constexpr int TILE = BP * D;
    constexpr int QH = (G * D * 2 + 1023) / 1024 * 512;
    constexpr int WAVE_LDS = NS * 2 * TILE + QH;          // halves of one wave's ring + Q area
    __shared__ __attribute__((aligned(16))) _Float16 ring_all[(WIDE ? 8 : 1) * WAVE_LDS];
    const int kvh = WIDE ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : (int)blockIdx.y;   // wave-uniform
    _Float16* ring = ring_all + (WIDE ? kvh * WAVE_LDS : 0);
    if constexpr (WIDE) {
        if (a.balanced) {
            // Ragged lengths: one range of one sequence per workgroup (balanced_geom).
            const BalancedGeom geo = balanced_geom(a);
            if ((int)blockIdx.x >= geo.used) return;
            const BalancedRange r = balanced_range(a, geo, (int)blockIdx.x);
            float* part = r.ns == 1 ? nullptr
                                    : a.partials + ((size_t)blockIdx.x * a.H_kv + kvh) * part_stride(G, D);
            split_range<D, G, NS, WIDE>(a, ring, r.b, kvh, r.t0, r.t1, part);
            return;
        }
    }
    const int split = blockIdx.x;
    const int b = WIDE ? (int)blockIdx.y : (int)blockIdx.z;
    const int T_b = attended(a, b);
    const int t0 = split * a.chunk;
    if (t0 >= T_b) return;
    const int nsplit_b = (T_b + a.chunk - 1) / a.chunk;
    split_range<D, G, NS, WIDE>(a, ring, b, kvh, t0, min(t0 + a.chunk, T_b),
                                nsplit_b == 1 ? nullptr : partial_at(a, b * a.H_kv + kvh, split, G, D));
}

// The grouped kernel with K in registers (split_range_kv): a wave per KV head, each with
// an NSV-stage V ring; otherwise the same grid and ranges as split_f16<..., WIDE>.
// Config 2 (rotating KV sets, one box): split 44.85-44.88 us at 4 stages and 7 sets,
// 45.2-45.5 us at 5 stages (all 160 KB of LDS), 45.2 us with 5 sets; the K-and-V ring
// kernel 46.2 us.
constexpr int kKvStages = 4;    // V ring stages per wave (4 KB each at d = 128)
constexpr int kKvSets = 7;      // K register sets per wave (K runs 6 blocks ahead)
template <int D, int G, int NSV = kKvStages, int NSETS = kKvSets>
__global__ __launch_bounds__(512)
void split_f16_kv(cf_decode_attn_args_t a) {
    constexpr int WAVE_LDS = NSV * KvRing<D>::TILE;
    __shared__ __attribute__((aligned(16))) _Float16 ring_all[8 * WAVE_LDS];
    const int kvh = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    _Float16* ring = ring_all + kvh * WAVE_LDS;
    if (a.balanced) {
        const BalancedGeom geo = balanced_geom(a);
        if ((int)blockIdx.x >= geo.used) return;
        const BalancedRange r = balanced_range(a, geo, (int)blockIdx.x);
        float* part = r.ns == 1 ? nullptr : a.partials + ((size_t)blockIdx.x * a.H_kv + kvh) * part_stride(G, D);
        split_range_kv<D, G, NSV, NSETS>(a, ring, r.b, kvh, r.t0, r.t1, part);
        return;
    }
    const int split = blockIdx.x, b = blockIdx.y;
    const int T_b = attended(a, b);
    const int t0 = split * a.chunk;
    if (t0 >= T_b) return;
    const int nsplit_b = (T_b + a.chunk - 1) / a.chunk;
    split_range_kv<D, G, NSV, NSETS>(a, ring, b, kvh, t0, min(t0 + a.chunk, T_b),
                                             nsplit_b == 1 ? nullptr : partial_at(a, b * a.H_kv + kvh, split, G, D));
}

// ------------------------------------------------------------------ fp32 split ---
template <int D, int G>
__global__ __launch_bounds__(kF32Threads)
void split_f32(cf_decode_attn_args_t a) {
    constexpr int LPR = D / 4;                 // lanes per row (4 floats each)
    constexpr int RPW = 64 / LPR;
    constexpr int NW = kF32Threads / 64;
    constexpr int ROWS = NW * RPW;
    constexpr int PIT = ROWS * kF32Unroll;
    static_assert(G <= LPR, "one writer lane per head");
    static_assert(LPR == 16 || LPR == 32, "row reductions on DPP and the row swaps");
    extern __shared__ float smem[];

    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int T_b = attended(a, b);
    const int t0 = split * a.chunk;
    if (t0 >= T_b) return;
    const int t1 = min(t0 + a.chunk, T_b);
    const int npos = t1 - t0;
    const int nsplit_b = (T_b + a.chunk - 1) / a.chunk;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane / LPR, c = lane - r * LPR;

    const size_t row_stride = (size_t)a.H_kv * D;
    const size_t unit_off = ((size_t)b * a.max_seq * a.H_kv + kvh) * D + (size_t)c * 4;
    const float* __restrict__ kb = (const float*)a.k + unit_off;
    const float* __restrict__ vb = (const float*)a.v + unit_off;
    const int h0 = kvh * G;
    const int sc_floats = max(a.chunk * G, NW * G * D);
    float* sc = smem;
    float* red = smem + sc_floats;             // [2][NW][G]

    f4_t qv[G];
#pragma unroll
    for (int g = 0; g < G; g++) qv[g] = *(const f4_t*)((const float*)a.q + ((size_t)b * a.H_q + h0 + g) * D + c * 4);
    const float qk_scale = a.scale * kLog2e;

    // Rows are loaded unconditionally, clamped to the split's last row (a load under a
    // branch is waited for at the branch's end), and the first block's V rows go out with
    // its K rows, so a split of one block (config 1: 64 positions) reads K and V in one
    // round trip.
    auto load_rows = [&](const float* __restrict__ src, int base, f4_t (&dst)[kF32Unroll]) {
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++)
            dst[u] = *(const f4_t*)(src + (size_t)min(base + u * ROWS + wave * RPW + r, t1 - 1) * row_stride);
    };
    f4_t kv[kF32Unroll], v0[kF32Unroll];
    load_rows(kb, t0, kv);
    load_rows(vb, t0, v0);
    float mloc[G];
#pragma unroll
    for (int g = 0; g < G; g++) mloc[g] = -INFINITY;
    auto score_block = [&](int base) {
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++) {
            const int pos = base + u * ROWS + wave * RPW + r;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float s = qv[g][0] * kv[u][0];
                s = __builtin_fmaf(qv[g][1], kv[u][1], s);
                s = __builtin_fmaf(qv[g][2], kv[u][2], s);
                s = __builtin_fmaf(qv[g][3], kv[u][3], s);
                s = row_sum16(s);                  // the row's LPR lanes (DPP, no LDS trip)
                if constexpr (LPR == 32) s = add_xor16(s);
                s *= qk_scale;
                if (pos < t1) {
                    if (c == g) sc[(pos - t0) * G + g] = s;
                    mloc[g] = fmaxf(mloc[g], s);
                }
            }
        }
    };
    score_block(t0);
    for (int base = t0 + PIT; base < t1; base += PIT) {
        load_rows(kb, base, kv);
        score_block(base);
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = mloc[g];
        if constexpr (LPR == 16) m = max_xor16(m);
        m = max_xor32(m);
        if (lane == 0) red[wave * G + g] = m;
    }
    __syncthreads();
    float M[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = red[g];
#pragma unroll
        for (int w = 1; w < NW; w++) m = fmaxf(m, red[w * G + g]);
        M[g] = m;
    }
    float lsum = 0.0f;
    {
        const int gm = tid % G;
        float mg = M[0];
#pragma unroll
        for (int g = 1; g < G; g++) if (gm == g) mg = M[g];
        for (int i = tid; i < npos * G; i += kF32Threads) {
            const float p = exp2f(sc[i] - mg);
            sc[i] = p;
            lsum += p;
        }
    }
    lsum = sum_stride<G>(lsum);
    if (lane < G) red[NW * G + wave * G + lane] = lsum;
    __syncthreads();
    float L[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) l += red[NW * G + w * G + g];
        L[g] = l;
    }
    float acc[G][4];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[g][e] = 0.0f;
    auto acc_block = [&](int base, const f4_t (&vv)[kF32Unroll]) {
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++) {
            const int pos = base + u * ROWS + wave * RPW + r;
            if (pos < t1) {
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = sc[(pos - t0) * G + g];
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[g][e] = __builtin_fmaf(p, vv[u][e], acc[g][e]);
                }
            }
        }
    };
    acc_block(t0, v0);
    for (int base = t0 + PIT; base < t1; base += PIT) {
        f4_t vv[kF32Unroll];
        load_rows(vb, base, vv);
        acc_block(base, vv);
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = acc[g][e];
            if constexpr (LPR == 16) v = add_xor16(v);
            acc[g][e] = add_xor32(v);
        }
    __syncthreads();
    float* accbuf = smem;                      // [NW][G][D]
    if (r == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 4; e++) accbuf[(wave * G + g) * D + c * 4 + e] = acc[g][e];
    }
    __syncthreads();
    float* part = nsplit_b == 1 ? nullptr : partial_at(a, b * a.H_kv + kvh, split, G, D);
    float* out = (float*)a.o + ((size_t)b * a.H_q + h0) * D;
    for (int idx = tid; idx < G * D; idx += kF32Threads) {
        float s = accbuf[idx];
#pragma unroll
        for (int w = 1; w < NW; w++) s += accbuf[w * G * D + idx];
        const int g = idx / D;
        if (part) {
            part[part_hdr(G) + idx] = s;
        } else {
            float l = L[0];
#pragma unroll
            for (int gg = 1; gg < G; gg++) if (g == gg) l = L[gg];
            out[idx] = s / l;
        }
    }
    if (part && tid < G) {
        float m = M[0], l = L[0];
#pragma unroll
        for (int g = 1; g < G; g++) if (tid == g) { m = M[g]; l = L[g]; }
        part[tid] = m;
        part[G + tid] = l;
    }
}

// ---------------------------------------------------------------- generic split ---
template <typename T>
__global__ __launch_bounds__(kGenericThreads)
void split_generic(cf_decode_attn_args_t a) {
    extern __shared__ float smem[];
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int D = a.d;
    const int kvh = h / (a.H_q / a.H_kv);
    const int T_b = attended(a, b);
    const int t0 = split * a.chunk;
    if (t0 >= T_b) return;
    const int t1 = min(t0 + a.chunk, T_b);
    const int npos = t1 - t0;
    const int nsplit_b = (T_b + a.chunk - 1) / a.chunk;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int nw = kGenericThreads / 64;
    float* qs = smem;                 // [D]
    float* sc = smem + D;             // [chunk]
    float* red = sc + a.chunk;        // [2 * nw]

    const T* __restrict__ q = (const T*)a.q + ((size_t)b * a.H_q + h) * D;
    const float qk_scale = a.scale * kLog2e;
    for (int i = tid; i < D; i += kGenericThreads) qs[i] = to_f(q[i]) * qk_scale;
    __syncthreads();
    const size_t row_stride = (size_t)a.H_kv * D;
    const size_t unit_off = ((size_t)b * a.max_seq * a.H_kv + kvh) * D;
    const T* __restrict__ kb = (const T*)a.k + unit_off;
    const T* __restrict__ vb = (const T*)a.v + unit_off;
    float mloc = -INFINITY;
    for (int t = t0 + tid; t < t1; t += kGenericThreads) {
        const T* kr = kb + (size_t)t * row_stride;
        float s = 0.0f;
        for (int i = 0; i < D; i++) s = __builtin_fmaf(qs[i], to_f(kr[i]), s);
        sc[t - t0] = s;
        mloc = fmaxf(mloc, s);
    }
    for (int off = 1; off < 64; off <<= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, off));
    if (lane == 0) red[wave] = mloc;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < nw; w++) M = fmaxf(M, red[w]);
    float lsum = 0.0f;
    for (int i = tid; i < npos; i += kGenericThreads) {
        const float p = exp2f(sc[i] - M);
        sc[i] = p;
        lsum += p;
    }
    for (int off = 1; off < 64; off <<= 1) lsum += __shfl_xor(lsum, off);
    if (lane == 0) red[nw + wave] = lsum;
    __syncthreads();
    float L = 0.0f;
    for (int w = 0; w < nw; w++) L += red[nw + w];
    T* __restrict__ out = (T*)a.o + ((size_t)b * a.H_q + h) * D;
    float* part = partial_at(a, b * a.H_q + h, split, 1, D);
    for (int i = tid; i < D; i += kGenericThreads) {
        float acc = 0.0f;
        const T* vc = vb + (size_t)t0 * row_stride + i;
        for (int j = 0; j < npos; j++) acc = __builtin_fmaf(sc[j], to_f(vc[(size_t)j * row_stride]), acc);
        if (nsplit_b == 1) out[i] = from_f<T>(acc / L);
        else part[part_hdr(1) + i] = acc;
    }
    if (nsplit_b > 1 && tid == 0) { part[0] = M; part[1] = L; }
}

// ------------------------------------------------------------------------ merge ---
// One thread per output element (unit, head g, dim i); unit = (b, kv head) holding Gx
// heads, or (b, q head) with Gx = 1.  Each thread streams its splits 16 at a time with
// all loads of a group in flight together and folds them into a running
// (M, num, den) with the log-sum-exp rescale, so there is no LDS and no barrier.
template <typename T>
__global__ __launch_bounds__(kMergeThreads)
void merge_kernel(cf_decode_attn_args_t a, int Gx, int units_per_b, MergeDivs md) {
    const int D = a.d;
    const size_t idx = (size_t)blockIdx.x * kMergeThreads + threadIdx.x;
    const size_t total = (size_t)a.B * units_per_b * Gx * D;
    if (idx >= total) return;
    const int i = (int)(idx % D);
    const size_t ug = idx / D;
    const int g = (int)(ug % Gx);
    const int unit = (int)(ug / Gx);
    const int b = unit / units_per_b;
    const int stride = part_stride(Gx, D), hdr = part_hdr(Gx);
    const SplitRecords sr = split_records(a, b, unit, units_per_b, stride, md);
    const int nsplit = sr.n;
    if (nsplit <= 1) return;                       // finished by the split kernel
    constexpr int NB = 16;
    float M = -INFINITY, num = 0.0f, den = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += NB) {
        float mv[NB], lv[NB], av[NB];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const bool ok = s0 + j < nsplit;
            const float* ps = sr.first + (size_t)(ok ? s0 + j : 0) * sr.step;
            mv[j] = ok ? ps[g] : -INFINITY;
            lv[j] = ok ? ps[Gx + g] : 0.0f;
            av[j] = ok ? ps[hdr + g * D + i] : 0.0f;
        }
        float mc = mv[0];
#pragma unroll
        for (int j = 1; j < NB; j++) mc = fmaxf(mc, mv[j]);
        const float m_new = fmaxf(M, mc);
        const float rescale = exp2f(M - m_new);    // 0 on the first group (M = -inf)
        num *= rescale;
        den *= rescale;
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const float w = exp2f(mv[j] - m_new);  // 0 for padding entries
            num = __builtin_fmaf(w, av[j], num);
            den = __builtin_fmaf(w, lv[j], den);
        }
        M = m_new;
    }
    ((T*)a.o)[idx] = from_f<T>(num / den);
}

// Row merge (D % 4 == 0): DS workgroups per output row (unit, head g), each owning
// D / DS dims.  DV = D / (4 DS) threads own 4 dims each; the SG = 256/DV thread groups
// take splits sg, sg+SG, ... with NB records in flight per thread, so a sequence with
// hundreds of splits costs a few load rounds instead of one per 16 splits, and DS > 1
// spreads a row's records over more CUs.  The SG running results combine through LDS
// in a log-depth tree that folds the upper half of the live groups onto the lower half,
// so SG need not be a power of two (a serial pass over them cost ~1.5 us with hundreds
// of splits; 256 threads measured faster than 1024 per row).
template <typename T, int NT = kMergeThreads>
__global__ __launch_bounds__(NT)
void merge_rows(cf_decode_attn_args_t a, int Gx, int units_per_b, int ds, MergeDivs md) {
    const int D = a.d, DV = D / (4 * ds), SG = NT / DV;
    const int row = blockIdx.x / ds, part = blockIdx.x - row * ds;
    const int unit = fastdiv(row, md.gx), g = row - unit * Gx, b = fastdiv(unit, md.ub);
    const int stride = part_stride(Gx, D), hdr = part_hdr(Gx);
    const SplitRecords sr = split_records(a, b, unit, units_per_b, stride, md);
    const int nsplit = sr.n;
    if (nsplit <= 1) return;                       // finished by the split kernel
    const int tid = threadIdx.x, col = part * DV + tid % DV, sg = tid / DV;
    __shared__ float sm[NT], sd[NT];
    __shared__ f4_t sn[NT];
    float M = -INFINITY, den = 0.0f;
    f4_t num = {0.f, 0.f, 0.f, 0.f};
    if (sg < SG) {
        constexpr int NB = 8;
        // Unconditional loads (split index clamped to the last split, weight 0 below)
        // through a global pointer: one batch of loads per round, no branch between them.
        const CF_GLOBAL float* first = (const CF_GLOBAL float*)sr.first;
        for (int s0 = sg; s0 < nsplit; s0 += SG * NB) {
            float mv[NB], lv[NB];
            f4_t av[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const int sp = s0 + j * SG;
                const CF_GLOBAL float* ps = first + (size_t)min(sp, nsplit - 1) * sr.step;
                const float mr = ps[g], lr = ps[Gx + g];
                mv[j] = sp < nsplit ? mr : -INFINITY;
                lv[j] = sp < nsplit ? lr : 0.0f;
                av[j] = *(const CF_GLOBAL f4_t*)(ps + hdr + g * D + 4 * col);
            }
            float mc = mv[0];
#pragma unroll
            for (int j = 1; j < NB; j++) mc = fmaxf(mc, mv[j]);
            const float m_new = fmaxf(M, mc);      // finite: split s0 < nsplit is valid
            const float rescale = exp2f(M - m_new);
            den *= rescale;
            num *= rescale;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const float w = exp2f(mv[j] - m_new);
                den = __builtin_fmaf(w, lv[j], den);
                num += w * av[j];
            }
            M = m_new;
        }
    }
    // The SG groups' (M, den, num) of each column combine in a tree through LDS: with n
    // groups live, groups [h, n) (h = ceil(n / 2)) fold onto groups [0, n - h).
    sm[tid] = M;
    sd[tid] = den;
    sn[tid] = num;
    __syncthreads();
    for (int n = SG; n > 1;) {
        const int h = (n + 1) >> 1;
        if (sg < n - h) {
            const int o = tid + h * DV;
            const float m1 = sm[tid], m2 = sm[o];
            const float mx = fmaxf(m1, m2);
            const float w1 = m1 == -INFINITY ? 0.0f : exp2f(m1 - mx);
            const float w2 = m2 == -INFINITY ? 0.0f : exp2f(m2 - mx);
            sm[tid] = mx;
            sd[tid] = w1 * sd[tid] + w2 * sd[o];
            sn[tid] = w1 * sn[tid] + w2 * sn[o];
        }
        __syncthreads();
        n = h;
    }
    if (sg == 0) {
        T* out = (T*)a.o + (size_t)row * D + 4 * col;
        const float inv = 1.0f / sd[tid];
        const f4_t nn = sn[tid];
#pragma unroll
        for (int e = 0; e < 4; e++) out[e] = from_f<T>(nn[e] * inv);
    }
}

// Merge, one wave per output row (D = 64 or 128; DPL = D / 64 dims per lane; used up to
// 16 splits), four rows per workgroup, no LDS: lane s holds (m, l) of splits s, s + 64,
// ...; the wave reduces M = max m and den = sum 2^(m - M) l with shuffles, then
// accumulates the splits' accumulator rows weighted by 2^(m_s - M) (broadcast from lane
// s % 64), eight in flight.
template <typename T, int DPL>
__global__ __launch_bounds__(256)
void merge_wave(cf_decode_attn_args_t a, int Gx, int units_per_b, int rows, MergeDivs md) {
    constexpr int D = 64 * DPL;
    constexpr int MAXS = kMergeWaveSplits;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (row >= rows) return;
    const int unit = fastdiv(row, md.gx), g = row - unit * Gx, b = fastdiv(unit, md.ub);
    const int stride = part_stride(Gx, D), hdr = part_hdr(Gx);
    const SplitRecords sr = split_records(a, b, unit, units_per_b, stride, md);
    const int nsplit = sr.n;
    if (nsplit <= 1) return;                       // finished by the split kernel
    // Every load first (one round trip): lane s < nsplit holds split s's (m, l), and each
    // lane the DPL accumulator values of every split for its dims.  The loads are
    // unconditional, split indices clamped to the last split (weight 0 below), so that
    // no branch splits them into several waits.
    const int last = nsplit - 1;
    const CF_GLOBAL float* first = (const CF_GLOBAL float*)sr.first;
    const CF_GLOBAL float* ph = first + (size_t)min(lane, last) * sr.step + g;
    const float mr = ph[0], lr = ph[Gx];
    const float mv = lane < nsplit ? mr : -INFINITY, lv = lane < nsplit ? lr : 0.0f;
    float av[MAXS][DPL];
#pragma unroll
    for (int j = 0; j < MAXS; j++) {
        const CF_GLOBAL float* ps = first + (size_t)min(j, last) * sr.step + hdr + g * D + DPL * lane;
#pragma unroll
        for (int e = 0; e < DPL; e++) av[j][e] = ps[e];
    }
    // Reductions on DPP and the row swaps, weights broadcast by v_readlane: no LDS round
    // trip after the loads.
    const float M = wave_max(mv);
    const float w = lane < nsplit ? exp2f(mv - M) : 0.0f;
    const float den = wave_sum(w * lv);
    float num[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) num[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXS; j++) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));   // 0 for j >= nsplit
#pragma unroll
        for (int e = 0; e < DPL; e++) num[e] = __builtin_fmaf(wj, av[j][e], num[e]);
    }
    const float inv = 1.0f / den;
    T* out = (T*)a.o + (size_t)row * D + DPL * lane;
#pragma unroll
    for (int e = 0; e < DPL; e++) out[e] = from_f<T>(num[e] * inv);
}

bool fast_supported(int elem, int d, int G) {
    (void)elem;
    return (d == 64 || d == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

int quantum(int elem, int d) {
    if (elem == CF_ELEM_F16) return kF16Quantum;
    return (kF32Threads / 64) * (64 / (d / 4)) * kF32Unroll;
}

bool use_fast(const cf_decode_attn_args_t* a) {
    const int G = a->H_q / a->H_kv;
    const bool aligned = (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->v | (uintptr_t)a->o) % 16) == 0;
    // The fp16 kernel scales the max of the raw scores, which needs scale > 0.
    return aligned && fast_supported(a->elem, a->d, G) && (a->elem != CF_ELEM_F16 || a->scale > 0.0f);
}

int g_stages = 0;   // tuning override of the fp16 ring depth (2..4; 0 = kDecodeStages)
int g_merge_rows = 0;   // 1: use the workgroup-per-row merge for every head size (tests)
int g_merge_rows_ds = -1;   // tuning override of merge_rows' workgroups per row (-1 = automatic)

// Workgroups per row of merge_rows: the largest of 1, 2, 4 that divides d / 4 and leaves
// at least 16 threads (64 dims) per thread group.  Ragged config 4 (d = 128, up to ~100
// records per row) measured a 5.0 us merge at 2 per row against 5.7 us at 1 and 5.5 us
// at 4.
int merge_rows_dsplit(int d) {
    const int dv = d / 4;
    if (g_merge_rows_ds > 0 && dv % g_merge_rows_ds == 0) return g_merge_rows_ds;
    for (int ds = 4; ds > 1; ds >>= 1)
        if (dv % ds == 0 && dv / ds >= 16) return ds;
    return 1;
}
int g_merge_wave_wg = 2; // rows (waves) per merge_wave workgroup (2 and 1 measured 0.15-0.2 us faster than 4)

int g_wide = 1;     // 0: one workgroup per (split, KV head) even where the grouped kernel applies
int g_kreg = 1;     // 0: the grouped kernel keeps K in its LDS ring too (d = 128)

int f16_stages() { return g_stages >= 2 && g_stages <= 4 ? g_stages : kDecodeStages; }

// Static LDS of split_f16<D, G, NS>: the ring plus the Q area.
int f16_lds_bytes(int d, int G, int NS) {
    const int qh = (G * d * 2 + 1023) / 1024 * 512;
    return (NS * 2 * 32 * d + qh) * 2;
}

// The grouped (WIDE) fp16 split kernel: 2-stage rings of 16-position blocks, one wave per
// KV head, static LDS for 8 waves.
constexpr int kWideStages = 2;
constexpr int kWideMaxHeads = 8;
int wide_lds_bytes(int d, int G) {
    const int qh = (G * d * 2 + 1023) / 1024 * 512;
    return kWideMaxHeads * (kWideStages * 2 * 16 * d + qh) * 2;
}
// Uniform lengths only (given on the host, or held on the device and equal): with
// ragged lengths the grouped kernel's whole-row workgroups leave a partial last round
// (config 4: 67 us against 64.6 us one wave per KV head).
bool use_wide(const cf_decode_attn_args_t* a) {
    return g_wide && a->elem == CF_ELEM_F16 && (!a->seq_lens || a->lens_uniform || a->balanced) &&
           a->H_kv <= kWideMaxHeads && use_fast(a);
}

// split_f16_kv's vmcnt waits count the loads the kernel itself issues; a register
// spill would add scratch loads between them.  The build has none (checked once here,
// from the code object), else the K-and-V ring kernel runs instead.
template <int D, int G>
bool kv_kernel_ok() {
    static const bool ok = [] {
        hipFuncAttributes at;
        return hipFuncGetAttributes(&at, reinterpret_cast<const void*>(&split_f16_kv<D, G>)) == hipSuccess &&
               at.localSizeBytes == 0;
    }();
    return ok;
}

template <int D, int G>
hipError_t launch_split_fast(const cf_decode_attn_args_t& a, hipStream_t s) {
    dim3 grid((unsigned)a.n_split, (unsigned)a.H_kv, (unsigned)a.B);
    if (use_wide(&a)) {
        const dim3 wgrid = a.balanced ? dim3((unsigned)a.n_split) : dim3((unsigned)a.n_split, (unsigned)a.B);
        bool kreg = false;
        if constexpr (D == 128) {
            if (g_kreg && kv_kernel_ok<D, G>()) {
                kreg = true;
                hipLaunchKernelGGL((split_f16_kv<D, G>), wgrid, dim3(64 * (unsigned)a.H_kv), 0, s, a);
            }
        }
        if (!kreg) hipLaunchKernelGGL((split_f16<D, G, kWideStages, true>), wgrid, dim3(64 * (unsigned)a.H_kv), 0, s, a);
    } else if (a.elem == CF_ELEM_F16) {
        switch (f16_stages()) {
            case 2: hipLaunchKernelGGL((split_f16<D, G, 2>), grid, dim3(64), 0, s, a); break;
            case 3: hipLaunchKernelGGL((split_f16<D, G, 3>), grid, dim3(64), 0, s, a); break;
            default: hipLaunchKernelGGL((split_f16<D, G, 4>), grid, dim3(64), 0, s, a); break;
        }
    } else {
        const int NW = kF32Threads / 64;
        const int sc_floats = a.chunk * G > NW * G * D ? a.chunk * G : NW * G * D;
        const size_t lds = (size_t)(sc_floats + 2 * NW * G) * sizeof(float);
        hipLaunchKernelGGL((split_f32<D, G>), grid, dim3(kF32Threads), lds, s, a);
    }
    return hipGetLastError();
}

template <int D>
hipError_t launch_split_g(const cf_decode_attn_args_t& a, int G, hipStream_t s) {
    switch (G) {
        case 1: return launch_split_fast<D, 1>(a, s);
        case 2: return launch_split_fast<D, 2>(a, s);
        case 4: return launch_split_fast<D, 4>(a, s);
        default: return launch_split_fast<D, 8>(a, s);
    }
}

}  // namespace

extern "C" int32_t cf_decode_attn_chunk_quantum(int32_t elem, int32_t d, int32_t group) {
    return fast_supported(elem, d, group) ? quantum(elem, d) : 0;
}

extern "C" void cf_decode_attn_set_stages(int32_t stages) { g_stages = stages; }

extern "C" void cf_decode_attn_set_merge_rows(int32_t on) { g_merge_rows = on != 0; }
extern "C" void cf_decode_attn_set_merge_rows_split(int32_t ds) { g_merge_rows_ds = ds >= 1 && ds <= 4 ? ds : -1; }
extern "C" void cf_decode_attn_set_merge_wave_wg(int32_t rows) { g_merge_wave_wg = rows >= 1 && rows <= 4 ? rows : 2; }

extern "C" void cf_decode_attn_set_wide(int32_t on) { g_wide = on != 0; }

extern "C" void cf_decode_attn_set_kreg(int32_t on) { g_kreg = on != 0; }

extern "C" int32_t cf_decode_attn_kreg_ok(int32_t group) {
    switch (group) {
        case 1: return kv_kernel_ok<128, 1>();
        case 2: return kv_kernel_ok<128, 2>();
        case 4: return kv_kernel_ok<128, 4>();
        case 8: return kv_kernel_ok<128, 8>();
        default: return 0;
    }
}

extern "C" int32_t cf_decode_attn_wide_wgs_per_cu(int32_t elem, int32_t d, int32_t group, int32_t h_kv) {
    if (!g_wide || elem != CF_ELEM_F16 || h_kv > kWideMaxHeads || !fast_supported(elem, d, group)) return 0;
    const int n = kLdsPerCu / wide_lds_bytes(d, group);
    return n < 1 ? 1 : n;
}

extern "C" int32_t cf_decode_attn_balanced_ok(int32_t elem, int32_t d, int32_t group, int32_t h_kv, int32_t B) {
    // Every workgroup and the merge derive their ranges from the B lengths (one per lane),
    // and the partition needs n_split = CUs x workgroups per CU >= 2B.
    const int per_cu = cf_decode_attn_wide_wgs_per_cu(elem, d, group, h_kv);
    return per_cu > 0 && B <= 64 && (long long)cu_count() * per_cu >= 2LL * B ? 1 : 0;
}

extern "C" int32_t cf_decode_attn_wgs_per_cu(int32_t elem, int32_t d, int32_t group) {
    if (elem != CF_ELEM_F16 || !fast_supported(elem, d, group)) return 0;
    const int n = kLdsPerCu / f16_lds_bytes(d, group, f16_stages());
    return n < 1 ? 1 : n;
}

extern "C" int32_t cf_decode_attn_chunk_max(int32_t elem, int32_t d, int32_t group) {
    return elem == CF_ELEM_F16 && fast_supported(elem, d, group) ? kChunkMaxF16 : kChunkMax;
}

extern "C" size_t cf_decode_attn_partials_floats(int32_t B, int32_t H_q, int32_t H_kv, int32_t d,
                                                 int32_t n_split, int32_t elem) {
    // (b, kv head) units with G heads each, or (b, q head) units: the same total.
    (void)H_kv; (void)elem;
    return (size_t)B * H_q * n_split * (d + 4);   // >= units * n_split * part_stride(Gx, d)
}

extern "C" int cf_launch_decode_attn_split(const cf_decode_attn_args_t* a, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (a->chunk <= 0 || a->n_split <= 0) return (int)hipErrorInvalidValue;
    const bool f16_fast = a->elem == CF_ELEM_F16 && use_fast(a);
    if (a->chunk > (f16_fast ? kChunkMaxF16 : kChunkMax)) return (int)hipErrorInvalidValue;
    hipError_t err;
    if (use_fast(a)) {
        const int G = a->H_q / a->H_kv;
        err = a->d == 64 ? launch_split_g<64>(*a, G, s) : launch_split_g<128>(*a, G, s);
    } else {
        const size_t lds = (size_t)(a->d + a->chunk + 8) * sizeof(float);
        dim3 grid((unsigned)a->n_split, (unsigned)a->H_q, (unsigned)a->B);
        if (a->elem == CF_ELEM_F16)
            hipLaunchKernelGGL(split_generic<_Float16>, grid, dim3(kGenericThreads), lds, s, *a);
        else
            hipLaunchKernelGGL(split_generic<float>, grid, dim3(kGenericThreads), lds, s, *a);
        err = hipGetLastError();
    }
    return (int)err;
}

extern "C" int cf_launch_decode_attn_merge(const cf_decode_attn_args_t* a, void* stream) {
    if (a->n_split <= 1) return 0;
    hipStream_t s = (hipStream_t)stream;
    const bool fast = use_fast(a);
    const int Gx = fast ? a->H_q / a->H_kv : 1;
    const int units_per_b = fast ? a->H_kv : a->H_q;
    const int rows = a->B * units_per_b * Gx;
    const MergeDivs md{fastdiv_make(Gx), fastdiv_make(units_per_b), fastdiv_make(a->chunk > 0 ? a->chunk : 1)};
    // One wave per row while the splits fit a few rounds of eight loads; with many
    // splits (long or ragged caches) a whole workgroup per row keeps more in flight.
    if ((a->d == 64 || a->d == 128) && a->n_split <= kMergeWaveSplits && !g_merge_rows) {
        const int per = g_merge_wave_wg;
        const dim3 grid((unsigned)((rows + per - 1) / per)), blk(64 * per);
        if (a->elem == CF_ELEM_F16) {
            if (a->d == 64) hipLaunchKernelGGL((merge_wave<_Float16, 1>), grid, blk, 0, s, *a, Gx, units_per_b, rows, md);
            else hipLaunchKernelGGL((merge_wave<_Float16, 2>), grid, blk, 0, s, *a, Gx, units_per_b, rows, md);
        } else {
            if (a->d == 64) hipLaunchKernelGGL((merge_wave<float, 1>), grid, blk, 0, s, *a, Gx, units_per_b, rows, md);
            else hipLaunchKernelGGL((merge_wave<float, 2>), grid, blk, 0, s, *a, Gx, units_per_b, rows, md);
        }
        return (int)hipGetLastError();
    }
    if (a->d % 4 == 0 && a->d / 4 <= kMergeThreads) {
        const int ds = merge_rows_dsplit(a->d);
        dim3 grid((unsigned)((size_t)a->B * units_per_b * Gx * ds));
        if (a->elem == CF_ELEM_F16)
            hipLaunchKernelGGL((merge_rows<_Float16>), grid, dim3(kMergeThreads), 0, s, *a, Gx, units_per_b, ds, md);
        else
            hipLaunchKernelGGL((merge_rows<float>), grid, dim3(kMergeThreads), 0, s, *a, Gx, units_per_b, ds, md);
        return (int)hipGetLastError();
    }
    const size_t total = (size_t)a->B * units_per_b * Gx * a->d;
    dim3 grid((unsigned)((total + kMergeThreads - 1) / kMergeThreads));
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(merge_kernel<_Float16>, grid, dim3(kMergeThreads), 0, s, *a, Gx, units_per_b, md);
    else
        hipLaunchKernelGGL(merge_kernel<float>, grid, dim3(kMergeThreads), 0, s, *a, Gx, units_per_b, md);
    return (int)hipGetLastError();
}

extern "C" int cf_launch_decode_attn(const cf_decode_attn_args_t* a, void* stream) {
    int rc = cf_launch_decode_attn_split(a, stream);
    if (rc != 0) return rc;
    return cf_launch_decode_attn_merge(a, stream);
}

// ------------------------------------------------------------ fixed scratch ---
// Split partials for callers that cannot allocate (mha_decode_attn_f16_noalloc): a
// file-scope device array, one copy per GPU, held until the process ends.  Host code
// never passes `scratch` itself to a kernel (on the host the name is only a stand-in for
// the symbol): it looks up each device's address once, with that device current, and
// uses that pointer.
namespace {
constexpr size_t kScratchBytes = (size_t)16 << 20;
constexpr int kScratchDevices = 64;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
float* g_scratch_ptr[kScratchDevices];
}  // namespace

extern "C" size_t cf_decode_attn_scratch_bytes(void) { return kScratchBytes; }

extern "C" int cf_decode_attn_scratch_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kScratchDevices) return (int)hipErrorInvalidDevice;
    if (g_scratch_ptr[dev]) return 0;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    }
    g_scratch_ptr[dev] = (float*)p;
    return 0;
}

extern "C" float* cf_decode_attn_scratch(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) return nullptr;
    if (!g_scratch_ptr[dev] && cf_decode_attn_scratch_init() != 0) return nullptr;
    return g_scratch_ptr[dev];
}
