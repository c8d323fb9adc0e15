// decode_attn.hip — split-KV single-token attention over a KV cache for gfx950.
//
// Replaces the reference's one-block-per-batch-row decode kernel
// (src/operator/nn/mha_decode_cuda.cu:11-157) with a bandwidth-shaped design:
//
//  * grid = (split, kv head, batch row); each workgroup streams one `chunk` of
//    positions of one (b, kv head) and serves the whole GQA group of G query heads
//    from a single read of each K and V row (kv head = h / G, mha_decode.c:77);
//  * 16-byte loads per lane; a wave covers 64*16 B = RPW whole K rows per load and
//    keeps kUnroll loads in flight;
//  * inside a split the softmax is exact two-pass over LDS-resident scores: pass 1
//    streams K and writes s = q·k·scale·log2(e), pass 2 streams V with p = 2^(s - m),
//    so no running rescale is needed;
//  * the partial (m, l, acc) of every split goes to the workspace; the last workgroup
//    of a (b, kv head) — found with a device-scope counter — merges them with the
//    log-sum-exp rule  O = Σ 2^(m_s - M)·acc_s / Σ 2^(m_s - M)·l_s  and resets the
//    counter, so one launch produces the final output (mha_fused_cuda.cu:847-863 and
//    :895-931 give the reference's split/merge formula).
//
// A generic kernel (one query head per workgroup, element-wise loops) covers head
// sizes and group sizes the specialised kernel is not instantiated for.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 4;
constexpr int kFastChunkMax = 1024;
constexpr int kGenericThreads = 128;
constexpr int kGenericChunkMax = 4096;

template <typename T> struct VecOf;
template <> struct VecOf<_Float16> { using type = h8_t; static constexpr int n = 8; };
template <> struct VecOf<float>    { using type = f4_t; static constexpr int n = 4; };

__device__ __forceinline__ float dot_lane(const h8_t& a, const h8_t& b) {
    float s = 0.0f;
    s = __builtin_amdgcn_fdot2(h2_t{a[0], a[1]}, h2_t{b[0], b[1]}, s, false);
    s = __builtin_amdgcn_fdot2(h2_t{a[2], a[3]}, h2_t{b[2], b[3]}, s, false);
    s = __builtin_amdgcn_fdot2(h2_t{a[4], a[5]}, h2_t{b[4], b[5]}, s, false);
    s = __builtin_amdgcn_fdot2(h2_t{a[6], a[7]}, h2_t{b[6], b[7]}, s, false);
    return s;
}

__device__ __forceinline__ float dot_lane(const f4_t& a, const f4_t& b) {
    float s = a[0] * b[0];
    s = __builtin_fmaf(a[1], b[1], s);
    s = __builtin_fmaf(a[2], b[2], s);
    s = __builtin_fmaf(a[3], b[3], s);
    return s;
}

template <int W>
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
    for (int m = 1; m < W; m <<= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 from_f<_Float16>(float x) { return (_Float16)x; }

// Merge the partials of all splits of one unit (this workgroup is the last to finish).
// part layout per split: [m (Gx)] [l (Gx)] [acc (Gx*D)], stride Gx*(D+2) floats.
template <typename T>
__device__ void merge_splits(const float* __restrict__ part, int nsplit, int Gx, int D,
                             T* __restrict__ out, int out_head_stride) {
    const int stride = Gx * (D + 2);
    for (int idx = threadIdx.x; idx < Gx * D; idx += blockDim.x) {
        const int g = idx / D, i = idx - g * D;
        float mx = -INFINITY;
        for (int s = 0; s < nsplit; s++) mx = fmaxf(mx, part[(size_t)s * stride + g]);
        float num = 0.0f, den = 0.0f;
        for (int s = 0; s < nsplit; s++) {
            const float* ps = part + (size_t)s * stride;
            const float w = exp2f(ps[g] - mx);
            num = __builtin_fmaf(w, ps[2 * Gx + idx], num);
            den = __builtin_fmaf(w, ps[Gx + g], den);
        }
        out[(size_t)g * out_head_stride + i] = from_f<T>(num / den);
    }
}

// Publish this split's partial and report whether this workgroup is the last of its
// unit.  Every thread fences its own stores before the counter moves (release); the
// last workgroup fences again before reading the others' partials (acquire).
__device__ bool publish_and_check_last(uint32_t* counter, int nsplit) {
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(counter, 1u);
        const int last = (prev == (uint32_t)(nsplit - 1));
        if (last) atomicExch(counter, 0u);
        s_last = last;
    }
    __syncthreads();
    const bool last = s_last != 0;
    if (last) __threadfence();
    return last;
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads)
void decode_attn_fast(cf_decode_attn_args_t a) {
    using V = typename VecOf<T>::type;
    constexpr int VEC = VecOf<T>::n;
    constexpr int LPR = D / VEC;               // lanes per K/V row
    constexpr int RPW = 64 / LPR;              // rows one wave load covers
    constexpr int ROWS = kWaves * RPW;         // rows one workgroup load covers
    constexpr int PIT = ROWS * kUnroll;        // positions per pass
    static_assert(G <= LPR, "one writer lane per head");

    extern __shared__ float smem[];
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int T_b = min(max((a.seq_lens ? a.seq_lens[b] : a.cache_len) + 1, 1), a.max_seq);
    const int t0 = split * a.chunk;
    if (t0 >= T_b) return;
    const int t1 = min(t0 + a.chunk, T_b);
    const int npos = t1 - t0;
    const int nsplit_b = (T_b + a.chunk - 1) / a.chunk;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane / LPR, c = lane - r * LPR;

    const size_t row_stride = (size_t)a.H_kv * D;
    const size_t unit_off = ((size_t)b * a.max_seq * a.H_kv + kvh) * D + (size_t)c * VEC;
    const T* __restrict__ kbase = (const T*)a.k + unit_off;
    const T* __restrict__ vbase = (const T*)a.v + unit_off;
    const int h0 = kvh * G;

    const int sc_floats = max(a.chunk * G, kWaves * G * D);
    float* sc = smem;                          // [npos][G] scores, later probabilities
    float* red = smem + sc_floats;             // [2][kWaves][G]

    V qv[G];
#pragma unroll
    for (int g = 0; g < G; g++)
        qv[g] = *(const V*)((const T*)a.q + ((size_t)b * a.H_q + h0 + g) * D + (size_t)c * VEC);
    const float qk_scale = a.scale * kLog2e;

    // Pass 1: scores.
    float mloc[G];
#pragma unroll
    for (int g = 0; g < G; g++) mloc[g] = -INFINITY;
    for (int base = t0; base < t1; base += PIT) {
        V kv[kUnroll];
        int pos[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            pos[u] = base + u * ROWS + wave * RPW + r;
            if (pos[u] < t1) kv[u] = *(const V*)(kbase + (size_t)pos[u] * row_stride);
            else kv[u] = V{};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float s = xor_sum<LPR>(dot_lane(qv[g], kv[u])) * qk_scale;
                if (pos[u] < t1) {
                    if (c == g) sc[(pos[u] - t0) * G + g] = s;
                    mloc[g] = fmaxf(mloc[g], s);
                }
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
        for (int w = 1; w < kWaves; w++) m = fmaxf(m, red[w * G + g]);
        M[g] = m;
    }

    // Probabilities and their sum per head.
    float lsum = 0.0f;
    {
        const int gm = tid % G;
        float mg = M[0];
#pragma unroll
        for (int g = 1; g < G; g++) if (gm == g) mg = M[g];
        for (int i = tid; i < npos * G; i += kThreads) {
            const float p = exp2f(sc[i] - mg);
            sc[i] = p;
            lsum += p;
        }
    }
#pragma unroll
    for (int off = G; off < 64; off <<= 1) lsum += __shfl_xor(lsum, off);
    if (lane < G) red[kWaves * G + wave * G + lane] = lsum;
    __syncthreads();
    float L[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) l += red[kWaves * G + w * G + g];
        L[g] = l;
    }

    // Pass 2: acc[g][:] += p[g] * V.
    float acc[G][VEC];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < VEC; e++) acc[g][e] = 0.0f;
    for (int base = t0; base < t1; base += PIT) {
        V vv[kUnroll];
        int pos[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            pos[u] = base + u * ROWS + wave * RPW + r;
            if (pos[u] < t1) vv[u] = *(const V*)(vbase + (size_t)pos[u] * row_stride);
            else vv[u] = V{};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            if (pos[u] < t1) {
                const float* pp = sc + (pos[u] - t0) * G;
                float p[G];
#pragma unroll
                for (int g = 0; g < G; g++) p[g] = pp[g];
#pragma unroll
                for (int e = 0; e < VEC; e++) {
                    const float ve = to_f(vv[u][e]);
#pragma unroll
                    for (int g = 0; g < G; g++) acc[g][e] = __builtin_fmaf(p[g], ve, acc[g][e]);
                }
            }
        }
    }
    // Rows of a wave -> row 0, then waves -> LDS.
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            float v = acc[g][e];
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) v += __shfl_xor(v, off);
            acc[g][e] = v;
        }
    __syncthreads();                           // everyone is done with sc
    float* accbuf = smem;                      // [kWaves][G][D]
    if (r == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < VEC; e++) accbuf[(wave * G + g) * D + c * VEC + e] = acc[g][e];
    }
    __syncthreads();

    T* __restrict__ out = (T*)a.o + ((size_t)b * a.H_q + h0) * D;
    if (nsplit_b == 1) {
        for (int idx = tid; idx < G * D; idx += kThreads) {
            float s = accbuf[idx];
#pragma unroll
            for (int w = 1; w < kWaves; w++) s += accbuf[w * G * D + idx];
            const int g = idx / D;
            float l = L[0];
#pragma unroll
            for (int gg = 1; gg < G; gg++) if (g == gg) l = L[gg];
            out[idx] = from_f<T>(s / l);
        }
        return;
    }

    const int unit = b * a.H_kv + kvh;
    float* part = a.partials + ((size_t)unit * a.n_split + split) * (G * (D + 2));
    for (int idx = tid; idx < G * D; idx += kThreads) {
        float s = accbuf[idx];
#pragma unroll
        for (int w = 1; w < kWaves; w++) s += accbuf[w * G * D + idx];
        part[2 * G + idx] = s;
    }
    if (tid < G) {
        float m = M[0], l = L[0];
#pragma unroll
        for (int g = 1; g < G; g++) if (tid == g) { m = M[g]; l = L[g]; }
        part[tid] = m;
        part[G + tid] = l;
    }
    if (!publish_and_check_last(a.counters + unit, nsplit_b)) return;
    merge_splits<T>(a.partials + (size_t)unit * a.n_split * (G * (D + 2)), nsplit_b, G, D, out, D);
}

template <typename T>
__global__ __launch_bounds__(kGenericThreads)
void decode_attn_generic(cf_decode_attn_args_t a) {
    extern __shared__ float smem[];
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int D = a.d;
    const int kvh = h / (a.H_q / a.H_kv);
    const int T_b = min(max((a.seq_lens ? a.seq_lens[b] : a.cache_len) + 1, 1), a.max_seq);
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
    const int unit = b * a.H_q + h;
    float* part = a.partials + ((size_t)unit * a.n_split + split) * (D + 2);
    for (int i = tid; i < D; i += kGenericThreads) {
        float acc = 0.0f;
        const T* vc = vb + (size_t)t0 * row_stride + i;
        for (int j = 0; j < npos; j++) acc = __builtin_fmaf(sc[j], to_f(vc[(size_t)j * row_stride]), acc);
        if (nsplit_b == 1) out[i] = from_f<T>(acc / L);
        else part[2 + i] = acc;
    }
    if (nsplit_b == 1) return;
    if (tid == 0) { part[0] = M; part[1] = L; }
    if (!publish_and_check_last(a.counters + unit, nsplit_b)) return;
    merge_splits<T>(a.partials + (size_t)unit * a.n_split * (D + 2), nsplit_b, 1, D, out, D);
}

bool fast_supported(int elem, int d, int G) {
    (void)elem;
    return (d == 64 || d == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

int quantum(int elem, int d) {
    const int vec = elem == CF_ELEM_F16 ? 8 : 4;
    const int lpr = d / vec;
    return kWaves * (64 / lpr) * kUnroll;
}

template <typename T, int D, int G>
hipError_t launch_fast(const cf_decode_attn_args_t& a, hipStream_t s) {
    const int sc_floats = a.chunk * G > kWaves * G * D ? a.chunk * G : kWaves * G * D;
    const size_t lds = (size_t)(sc_floats + 2 * kWaves * G) * sizeof(float);
    dim3 grid((unsigned)a.n_split, (unsigned)a.H_kv, (unsigned)a.B);
    hipLaunchKernelGGL((decode_attn_fast<T, D, G>), grid, dim3(kThreads), lds, s, a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_fast_g(const cf_decode_attn_args_t& a, int G, hipStream_t s) {
    switch (G) {
        case 1: return launch_fast<T, D, 1>(a, s);
        case 2: return launch_fast<T, D, 2>(a, s);
        case 4: return launch_fast<T, D, 4>(a, s);
        default: return launch_fast<T, D, 8>(a, s);
    }
}

template <typename T>
hipError_t launch_fast_dg(const cf_decode_attn_args_t& a, int G, hipStream_t s) {
    return a.d == 64 ? launch_fast_g<T, 64>(a, G, s) : launch_fast_g<T, 128>(a, G, s);
}

}  // namespace

extern "C" int32_t cf_decode_attn_chunk_quantum(int32_t elem, int32_t d, int32_t group) {
    return fast_supported(elem, d, group) ? quantum(elem, d) : 0;
}

extern "C" int32_t cf_decode_attn_chunk_max(int32_t elem, int32_t d, int32_t group) {
    return fast_supported(elem, d, group) ? kFastChunkMax : kGenericChunkMax;
}

extern "C" size_t cf_decode_attn_partials_floats(int32_t B, int32_t H_q, int32_t H_kv, int32_t d,
                                                 int32_t n_split, int32_t elem) {
    const int G = H_q / H_kv;
    if (fast_supported(elem, d, G)) return (size_t)B * H_kv * n_split * G * (d + 2);
    return (size_t)B * H_q * n_split * (d + 2);
}

extern "C" size_t cf_decode_attn_counters(int32_t B, int32_t H_q, int32_t H_kv, int32_t d, int32_t elem) {
    // Worst case over both kernels (the launcher may pick the generic one for
    // unaligned pointers): one counter per (b, query head).
    (void)H_kv; (void)d; (void)elem;
    return (size_t)B * H_q;
}

extern "C" int cf_launch_decode_attn(const cf_decode_attn_args_t* a, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    const int G = a->H_q / a->H_kv;
    // The specialised kernel issues 16-byte loads of Q, K and V rows.
    const bool aligned = (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->v) % 16) == 0;
    hipError_t err;
    if (aligned && fast_supported(a->elem, a->d, G)) {
        err = a->elem == CF_ELEM_F16 ? launch_fast_dg<_Float16>(*a, G, s)
                                     : launch_fast_dg<float>(*a, G, s);
    } else {
        const size_t lds = (size_t)(a->d + a->chunk + 8) * sizeof(float);
        dim3 grid((unsigned)a->n_split, (unsigned)a->H_q, (unsigned)a->B);
        if (a->elem == CF_ELEM_F16)
            hipLaunchKernelGGL(decode_attn_generic<_Float16>, grid, dim3(kGenericThreads), lds, s, *a);
        else
            hipLaunchKernelGGL(decode_attn_generic<float>, grid, dim3(kGenericThreads), lds, s, *a);
        err = hipGetLastError();
    }
    return (int)err;
}
