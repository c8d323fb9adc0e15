// decode_attn.hip — split-KV single-token attention over a KV cache for gfx950.
//
// Replaces the reference's one-block-per-batch-row decode kernel
// (src/operator/nn/mha_decode_cuda.cu:11-157).  Two launches:
//
// 1. split kernel, grid = (split, kv head, batch row).  A workgroup streams one `chunk`
//    of positions of one (b, kv head) and serves the whole GQA group of G query heads
//    (kv head = h / G, mha_decode.c:77) from a single read of every K and V row.
//    Inside a split the softmax is exact and two-pass over LDS-resident scores:
//      pass 1 streams K and stores s = q·k · scale·log2(e) (and its max),
//      pass 2 streams V with p = 2^(s - m)  -> partial (m, l = Σp, acc = Σ p·v).
//    fp16 (d = 64/128): one wave per workgroup.  Q·K^T runs on the matrix cores as
//      S^T(16 positions x 16 heads) = K(16 x 32 dims) · Q^T(32 dims x 16 heads) with
//      v_mfma_f32_16x16x32_f16, so a lane ends up holding 4 positions of ONE head and
//      no cross-lane reduction is needed; the K tile loads are double-buffered.  P·V is
//      on the VALU: a lane owns 8 dims of one V row and accumulates all G heads.
//    fp32 (d = 64/128): four waves, lanes own 4 dims of a row, dot products reduced
//      across the row's lanes.
//    Other head or group sizes: a generic kernel, one query head per workgroup.
// 2. merge kernel, one thread per output element: the log-sum-exp combine
//      O = Σ_s 2^(m_s - M)·acc_s / Σ_s 2^(m_s - M)·l_s
//    (the reference's split/merge formula, mha_fused_cuda.cu:847-863 and :895-931,
//    restated per (b, head) with the head index it lacked).  A sequence that fits in
//    one split is finished by the split kernel and skipped here.
// No fences or atomics: the kernel boundary orders the partials, which matters on
// MI355X where each XCD has its own L2.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kChunkMax = 4096;            // positions per split (LDS: chunk * G floats)
constexpr int kF16Quantum = 32;            // fp16 split kernel: positions per double-block
constexpr int kF32Threads = 256;
constexpr int kF32Unroll = 4;
constexpr int kGenericThreads = 128;
constexpr int kMergeThreads = 256;

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }

__device__ __forceinline__ int attended(const cf_decode_attn_args_t& a, int b) {
    const int cl = a.seq_lens ? a.seq_lens[b] : a.cache_len;
    return min(max(cl + 1, 1), a.max_seq);
}

// Partial record of one split: [m (Gx)] [l (Gx)] [acc (Gx*D)].
__device__ __forceinline__ float* partial_at(const cf_decode_attn_args_t& a, int unit, int split, int Gx, int D) {
    return a.partials + ((size_t)unit * a.n_split + split) * (size_t)(Gx * (D + 2));
}

// ------------------------------------------------------------------ fp16 split ---
template <int D, int G>
__global__ __launch_bounds__(64)
void split_f16(cf_decode_attn_args_t a) {
    constexpr int KT = D / 32;          // 32-dim MFMA steps
    constexpr int LPR = D / 8;          // lanes per V row (8 halves each)
    constexpr int RPW = 64 / LPR;       // V rows per wave load
    constexpr int VU = 4;               // V loads in flight per lane per step
    extern __shared__ float sc[];       // [chunk][G]

    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int T_b = attended(a, b);
    const int t0 = split * a.chunk;
    if (t0 >= T_b) return;
    const int t1 = min(t0 + a.chunk, T_b);
    const int npos = t1 - t0;
    const int nsplit_b = (T_b + a.chunk - 1) / a.chunk;
    const int lane = threadIdx.x, lr = lane & 15, lq = lane >> 4;

    const size_t row_stride = (size_t)a.H_kv * D;
    const _Float16* __restrict__ kb = (const _Float16*)a.k + ((size_t)b * a.max_seq * a.H_kv + kvh) * D;
    const _Float16* __restrict__ vb = (const _Float16*)a.v + ((size_t)b * a.max_seq * a.H_kv + kvh) * D;
    const int h0 = kvh * G;

    // B operand Q^T: lane (lr, lq) holds Q[head lr][32kt + 8lq .. +7]; heads >= G are 0.
    h8_t qf[KT];
#pragma unroll
    for (int kt = 0; kt < KT; kt++)
        qf[kt] = lr < G ? *(const h8_t*)((const _Float16*)a.q + ((size_t)b * a.H_q + h0 + lr) * D + 32 * kt + 8 * lq)
                        : h8_t{};
    const float qk_scale = a.scale * kLog2e;

    // ---- pass 1: scores, 16 positions per MFMA block, two blocks in flight.
    auto load_k = [&](int p0, h8_t (&kf)[KT]) {
        const int pos = p0 + lr;
#pragma unroll
        for (int kt = 0; kt < KT; kt++)
            kf[kt] = pos < t1 ? *(const h8_t*)(kb + (size_t)pos * row_stride + 32 * kt + 8 * lq) : h8_t{};
    };
    float mrun = -INFINITY;
    auto score = [&](int p0, const h8_t (&kf)[KT]) {
        f4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < KT; kt++) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kt], qf[kt], s, 0, 0, 0);
        if (lr < G) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int pos = p0 + 4 * lq + i;
                if (pos < t1) {
                    const float x = s[i] * qk_scale;
                    sc[(pos - t0) * G + lr] = x;
                    mrun = fmaxf(mrun, x);
                }
            }
        }
    };
    h8_t ka[KT], kc[KT];
    load_k(t0, ka);
    for (int p0 = t0; p0 < t1; p0 += 32) {
        load_k(p0 + 16, kc);
        score(p0, ka);
        if (p0 + 32 < t1) load_k(p0 + 32, ka);
        if (p0 + 16 < t1) score(p0 + 16, kc);
    }
    // First V rows go out now, so their latency overlaps the softmax pass below.
    const int r = lane / LPR, c = lane - (lane / LPR) * LPR;
    const _Float16* __restrict__ vrow = vb + 8 * c;
    auto load_v = [&](int p0, h8_t (&vv)[VU]) {
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int pos = p0 + u * RPW + r;
            vv[u] = pos < t1 ? *(const h8_t*)(vrow + (size_t)pos * row_stride) : h8_t{};
        }
    };
    h8_t va[VU], vc[VU];
    load_v(t0, va);
    // Max per head: lanes with equal lr hold the same head.
    mrun = fmaxf(mrun, __shfl_xor(mrun, 16));
    mrun = fmaxf(mrun, __shfl_xor(mrun, 32));
    float M[G];
#pragma unroll
    for (int g = 0; g < G; g++) M[g] = __shfl(mrun, g);
    __syncthreads();

    // ---- probabilities and their sums (64 % G == 0, so a lane always sees one head).
    float lsum = 0.0f;
    {
        const int gm = lane % G;
        float mg = M[0];
#pragma unroll
        for (int g = 1; g < G; g++) if (gm == g) mg = M[g];
        for (int i = lane; i < npos * G; i += 64) {
            const float p = exp2f(sc[i] - mg);
            sc[i] = p;
            lsum += p;
        }
    }
#pragma unroll
    for (int off = G; off < 64; off <<= 1) lsum += __shfl_xor(lsum, off);
    float L[G];
#pragma unroll
    for (int g = 0; g < G; g++) L[g] = __shfl(lsum, g);
    __syncthreads();

    // ---- pass 2: acc[g][e] += p[g] * V[pos][8c + e], VU rows in flight per lane.
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    auto accum = [&](int p0, const h8_t (&vv)[VU]) {
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int pos = p0 + u * RPW + r;
            if (pos < t1) {
                float p[G];
#pragma unroll
                for (int g = 0; g < G; g++) p[g] = sc[(pos - t0) * G + g];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float ve = (float)vv[u][e];
#pragma unroll
                    for (int g = 0; g < G; g++) acc[g][e] = __builtin_fmaf(p[g], ve, acc[g][e]);
                }
            }
        }
    };
    constexpr int VSTEP = VU * RPW;
    for (int p0 = t0; p0 < t1; p0 += 2 * VSTEP) {
        load_v(p0 + VSTEP, vc);
        accum(p0, va);
        if (p0 + 2 * VSTEP < t1) load_v(p0 + 2 * VSTEP, va);
        if (p0 + VSTEP < t1) accum(p0 + VSTEP, vc);
    }
    // Rows of the wave -> row 0.
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = acc[g][e];
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) v += __shfl_xor(v, off);
            acc[g][e] = v;
        }

    if (nsplit_b == 1) {
        if (r == 0) {
            _Float16* out = (_Float16*)a.o + ((size_t)b * a.H_q + h0) * D + 8 * c;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float inv = 1.0f / L[g];
                h8_t o;
#pragma unroll
                for (int e = 0; e < 8; e++) o[e] = (_Float16)(acc[g][e] * inv);
                *(h8_t*)(out + (size_t)g * D) = o;
            }
        }
        return;
    }
    float* part = partial_at(a, b * a.H_kv + kvh, split, G, D);
    if (r == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            f4_t lo = {acc[g][0], acc[g][1], acc[g][2], acc[g][3]};
            f4_t hi = {acc[g][4], acc[g][5], acc[g][6], acc[g][7]};
            *(f4_t*)(part + 2 * G + g * D + 8 * c) = lo;
            *(f4_t*)(part + 2 * G + g * D + 8 * c + 4) = hi;
        }
    }
    if (lane < G) {
        float m = M[0], l = L[0];
#pragma unroll
        for (int g = 1; g < G; g++) if (lane == g) { m = M[g]; l = L[g]; }
        part[lane] = m;
        part[G + lane] = l;
    }
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

    float mloc[G];
#pragma unroll
    for (int g = 0; g < G; g++) mloc[g] = -INFINITY;
    for (int base = t0; base < t1; base += PIT) {
        f4_t kv[kF32Unroll];
        int pos[kF32Unroll];
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++) {
            pos[u] = base + u * ROWS + wave * RPW + r;
            kv[u] = pos[u] < t1 ? *(const f4_t*)(kb + (size_t)pos[u] * row_stride) : f4_t{};
        }
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++)
#pragma unroll
            for (int g = 0; g < G; g++) {
                float s = qv[g][0] * kv[u][0];
                s = __builtin_fmaf(qv[g][1], kv[u][1], s);
                s = __builtin_fmaf(qv[g][2], kv[u][2], s);
                s = __builtin_fmaf(qv[g][3], kv[u][3], s);
#pragma unroll
                for (int m = 1; m < LPR; m <<= 1) s += __shfl_xor(s, m);
                s *= qk_scale;
                if (pos[u] < t1) {
                    if (c == g) sc[(pos[u] - t0) * G + g] = s;
                    mloc[g] = fmaxf(mloc[g], s);
                }
            }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = mloc[g];
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
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
#pragma unroll
    for (int off = G; off < 64; off <<= 1) lsum += __shfl_xor(lsum, off);
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
    for (int base = t0; base < t1; base += PIT) {
        f4_t vv[kF32Unroll];
        int pos[kF32Unroll];
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++) {
            pos[u] = base + u * ROWS + wave * RPW + r;
            vv[u] = pos[u] < t1 ? *(const f4_t*)(vb + (size_t)pos[u] * row_stride) : f4_t{};
        }
#pragma unroll
        for (int u = 0; u < kF32Unroll; u++)
            if (pos[u] < t1) {
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = sc[(pos[u] - t0) * G + g];
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[g][e] = __builtin_fmaf(p, vv[u][e], acc[g][e]);
                }
            }
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = acc[g][e];
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) v += __shfl_xor(v, off);
            acc[g][e] = v;
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
            part[2 * G + idx] = s;
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
        else part[2 + i] = acc;
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
void merge_kernel(cf_decode_attn_args_t a, int Gx, int units_per_b) {
    const int D = a.d;
    const size_t idx = (size_t)blockIdx.x * kMergeThreads + threadIdx.x;
    const size_t total = (size_t)a.B * units_per_b * Gx * D;
    if (idx >= total) return;
    const int i = (int)(idx % D);
    const size_t ug = idx / D;
    const int g = (int)(ug % Gx);
    const int unit = (int)(ug / Gx);
    const int b = unit / units_per_b;
    const int T_b = attended(a, b);
    const int nsplit = (T_b + a.chunk - 1) / a.chunk;
    if (nsplit <= 1) return;                       // finished by the split kernel
    const int stride = Gx * (D + 2);
    const float* part = a.partials + (size_t)unit * a.n_split * stride;
    constexpr int NB = 16;
    float M = -INFINITY, num = 0.0f, den = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += NB) {
        float mv[NB], lv[NB], av[NB];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const float* ps = part + (size_t)(s0 + j) * stride;
            const bool ok = s0 + j < nsplit;
            mv[j] = ok ? ps[g] : -INFINITY;
            lv[j] = ok ? ps[Gx + g] : 0.0f;
            av[j] = ok ? ps[2 * Gx + g * D + i] : 0.0f;
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
    return aligned && fast_supported(a->elem, a->d, G);
}

template <int D, int G>
hipError_t launch_split_fast(const cf_decode_attn_args_t& a, hipStream_t s) {
    dim3 grid((unsigned)a.n_split, (unsigned)a.H_kv, (unsigned)a.B);
    if (a.elem == CF_ELEM_F16) {
        const size_t lds = (size_t)a.chunk * G * sizeof(float);
        hipLaunchKernelGGL((split_f16<D, G>), grid, dim3(64), lds, s, a);
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

extern "C" int32_t cf_decode_attn_chunk_max(int32_t elem, int32_t d, int32_t group) {
    (void)elem; (void)d; (void)group;
    return kChunkMax;
}

extern "C" size_t cf_decode_attn_partials_floats(int32_t B, int32_t H_q, int32_t H_kv, int32_t d,
                                                 int32_t n_split, int32_t elem) {
    // (b, kv head) units with G heads each, or (b, q head) units: the same total.
    (void)H_kv; (void)elem;
    return (size_t)B * H_q * n_split * (d + 2);
}

extern "C" int cf_launch_decode_attn_split(const cf_decode_attn_args_t* a, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (a->chunk <= 0 || a->chunk > kChunkMax || a->n_split <= 0) return (int)hipErrorInvalidValue;
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
    const size_t total = (size_t)a->B * units_per_b * Gx * a->d;
    dim3 grid((unsigned)((total + kMergeThreads - 1) / kMergeThreads));
    if (a->elem == CF_ELEM_F16)
        hipLaunchKernelGGL(merge_kernel<_Float16>, grid, dim3(kMergeThreads), 0, s, *a, Gx, units_per_b);
    else
        hipLaunchKernelGGL(merge_kernel<float>, grid, dim3(kMergeThreads), 0, s, *a, Gx, units_per_b);
    return (int)hipGetLastError();
}

extern "C" int cf_launch_decode_attn(const cf_decode_attn_args_t* a, void* stream) {
    int rc = cf_launch_decode_attn_split(a, stream);
    if (rc != 0) return rc;
    return cf_launch_decode_attn_merge(a, stream);
}
