// flash_attn.hip — prefill multi-head attention with an online softmax (gfx950).
//
// Computes, per (b, query head h), softmax(Q·K^T·scale)·V over keys 0..S-1 (or
// 0..i for causal query i, the rule of mha_fused_cuda.cu:336 / causal_mask.c:19),
// reading the projections the GEMM epilogue laid out head-major:
//   q (B,H_q,S,d), k (B,H_kv,S,d), vt (B,H_kv,d,S)  ->  o (B,S,H_q,d).
// kv head = h / (H_q/H_kv) (mha_decode.c:77).  The reference CPU semantics it must match
// are mha_fused.c:98-131 (two-pass softmax); the online form changes only rounding.
//
// fp16 path (d = 64 or 128): a workgroup owns 64 queries (4 waves x 16).  Key blocks of
// 64 are staged in LDS (K as [key][dim], V^T as [dim][key]).  Each wave computes
// S^T = K·Q^T with v_mfma_f32_16x16x32_f16, so a lane holds 16 scores of ONE query and
// the row max / row sum are lane-local plus a 4-lane exchange.  The probabilities are
// converted to fp16 in registers and fed straight back as the B operand of
// O^T += V^T·P^T; the key order inside each 32-key MFMA step is permuted so that the
// registers a lane already holds are exactly its B operand (V^T reads follow the same
// permutation).  No score or probability ever goes through LDS.
// Causal workgroups are issued heaviest-first.
//
// Generic path (fp32, or other head sizes): one thread per query, online softmax in
// fp32 with Q and the accumulator in LDS.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQB = 64;      // queries per workgroup
constexpr int kKB = 64;      // keys per block
constexpr int kThreads = 256;

template <int D>
__global__ __launch_bounds__(kThreads)
void flash_f16(cf_flash_args_t a) {
    constexpr int LDK = D + 8;        // halves per K row in LDS
    constexpr int LDV = kKB + 8;      // halves per V^T row in LDS
    constexpr int KT = D / 32;        // 32-dim steps of S^T
    constexpr int UT = D / 16;        // 16-dim tiles of O^T
    __shared__ __attribute__((aligned(16))) _Float16 Ks[kKB * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Vs[D * LDV];

    const int nqb = gridDim.x;
    const int qb = a.causal ? (nqb - 1 - (int)blockIdx.x) : (int)blockIdx.x;
    const int h = blockIdx.y, b = blockIdx.z;
    const int S = a.S;
    const int kvh = h / (a.H_q / a.H_kv);
    const int q0 = qb * kQB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int query = q0 + wave * 16 + lr;

    const _Float16* __restrict__ qp = (const _Float16*)a.q + (((size_t)b * a.H_q + h) * S) * D;
    const _Float16* __restrict__ kp = (const _Float16*)a.k + (((size_t)b * a.H_kv + kvh) * S) * D;
    const _Float16* __restrict__ vp = (const _Float16*)a.vt + (((size_t)b * a.H_kv + kvh) * D) * (size_t)S;

    h8_t qf[KT];
#pragma unroll
    for (int kt = 0; kt < KT; kt++)
        qf[kt] = query < S ? *(const h8_t*)(qp + (size_t)query * D + 32 * kt + 8 * lq) : h8_t{};

    const float c = a.scale * kLog2e;
    float m_run = -INFINITY, l_run = 0.0f;
    f4_t acc[UT];
#pragma unroll
    for (int u = 0; u < UT; u++) acc[u] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int k_end = a.causal ? min(S, q0 + kQB) : S;
    const bool v_vec = (S % 8) == 0;
    for (int k0 = 0; k0 < k_end; k0 += kKB) {
        // Stage K [key][dim] and V^T [dim][key].
        for (int ch = tid; ch < kKB * D / 8; ch += kThreads) {
            const int r = ch / (D / 8), cc = (ch % (D / 8)) * 8;
            h8_t v{};
            if (k0 + r < S) v = *(const h8_t*)(kp + (size_t)(k0 + r) * D + cc);
            *(h8_t*)&Ks[r * LDK + cc] = v;
        }
        for (int ch = tid; ch < D * (kKB / 8); ch += kThreads) {
            const int dm = ch / (kKB / 8), kc = (ch % (kKB / 8)) * 8;
            const _Float16* src = vp + (size_t)dm * S + k0 + kc;
            h8_t v{};
            if (v_vec && k0 + kc + 8 <= S) v = *(const h8_t*)src;
            else {
#pragma unroll
                for (int e = 0; e < 8; e++) if (k0 + kc + e < S) v[e] = src[e];
            }
            *(h8_t*)&Vs[dm * LDV + kc] = v;
        }
        __syncthreads();

        // S^T tiles: st[t][i] = score(key k0 + 16t + 4*lq + i, query).
        f4_t st[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            st[t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < KT; kt++) {
                const h8_t kf = *(const h8_t*)&Ks[(16 * t + lr) * LDK + 32 * kt + 8 * lq];
                st[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[kt], st[t], 0, 0, 0);
            }
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = k0 + 16 * t + 4 * lq + i;
                float x = st[t][i] * c;
                if (key >= S || (a.causal && key > query)) x = -INFINITY;
                st[t][i] = x;
                mloc = fmaxf(mloc, x);
            }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m_run - m_use);
        m_run = m_new;
        float psum = 0.0f;
        h8_t pf[2];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = exp2f(st[t][i] - m_use);
                psum += p;
                pf[t >> 1][(t & 1) * 4 + i] = (_Float16)p;
            }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int u = 0; u < UT; u++) acc[u] *= alpha;
        // O^T[16u + 4*lq + i][query] += Σ_keys V^T · P^T, key k-slot e of lane group lq
        // in step j is key 32j + 16*(e/4) + 4*lq + (e%4).
#pragma unroll
        for (int u = 0; u < UT; u++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const _Float16* vr = &Vs[(16 * u + lr) * LDV + 32 * j + 4 * lq];
                const h4_t lo = *(const h4_t*)vr;
                const h4_t hi = *(const h4_t*)(vr + 16);
                const h8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[j], acc[u], 0, 0, 0);
            }
        __syncthreads();
    }
    float l_tot = l_run + __shfl_xor(l_run, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (query < S) {
        const float inv = 1.0f / l_tot;
        _Float16* op = (_Float16*)a.o + (((size_t)b * S + query) * a.H_q + h) * D;
#pragma unroll
        for (int u = 0; u < UT; u++) {
            const h4_t ov = {(_Float16)(acc[u][0] * inv), (_Float16)(acc[u][1] * inv),
                             (_Float16)(acc[u][2] * inv), (_Float16)(acc[u][3] * inv)};
            *(h4_t*)(op + 16 * u + 4 * lq) = ov;
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

}  // namespace

extern "C" int cf_launch_flash_attn(const cf_flash_args_t* a, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (a->S <= 0 || a->d <= 0 || a->H_kv <= 0 || a->H_q % a->H_kv != 0) return (int)hipErrorInvalidValue;
    const bool aligned = ((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->vt | (uintptr_t)a->o) % 16 == 0;
    if (a->elem == CF_ELEM_F16 && aligned && (a->d == 64 || a->d == 128)) {
        dim3 grid((unsigned)((a->S + kQB - 1) / kQB), (unsigned)a->H_q, (unsigned)a->B);
        if (a->d == 64) hipLaunchKernelGGL(flash_f16<64>, grid, dim3(kThreads), 0, s, *a);
        else hipLaunchKernelGGL(flash_f16<128>, grid, dim3(kThreads), 0, s, *a);
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

