/*
 * oracle.h — CPU restatement of CudaForge's attention fallbacks.
 *
 * TEST INFRASTRUCTURE ONLY.  This code is the parity checker for the HIP operators:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and never as the thing measured or shipped.  The product library
 * (cudaforge_amd/libcudaforge_amd.so) does not link or call it.
 *
 * Functions follow the reference loop and arithmetic order:
 *   oracle_mha_decode_f32   src/operator/nn/mha_decode.c:11-125
 *   oracle_decode_attn_f32  src/operator/nn/mha_decode.c:88-114 (attention core, Q given)
 *   oracle_mha_fused_f32    src/operator/nn/mha_fused.c:32-176
 *   oracle_causal_mask_f32  src/operator/nn/causal_mask.c:8-23
 *   oracle_rope_f32, oracle_rope_at  src/operator/nn/rope.c:17-66
 *   oracle_layernorm_f32    src/operator/nn/layernorm.c:85-122 (scalar path)
 *   oracle_matmul_f32       src/operator/blas/matmul.c:14-50
 *   oracle_mha_decode_rope_f32  the decode op with rope.c's rotation of Q and K_new at
 *                               the token's position (a composition the reference runs as
 *                               two ops; no reference function computes it in one)
 * with the reference's fixed stack arrays (mha_decode.c:56,81,90,109) replaced by heap
 * buffers, GQA in the fused op (kv head = h / (H_q/H_kv), mha_decode.c:77), the causal
 * rule j <= i (mha_fused_cuda.cu:336, causal_mask.c:19) and ragged per-sequence cache
 * lengths for decode.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   - vs the reference C fallback itself, compiled from /root/reference into oracle/_ref
 *     (bit-exact where its fixed arrays allow: d <= 64, T <= 512, non-causal);
 *   - vs golden vectors written by that build (tests/golden/);
 *   - closed forms (T = 1, identical keys, one-hot scores), invariants (KV permutation,
 *     GQA == repeated-KV MHA, causal row == prefix attention, ragged == uniform) and a
 *     float64 brute force on tiny shapes;
 *   - LayerNorm and MatMul: bit-exact vs layernorm.c / matmul.c built into oracle/_ref
 *     (no USE_AVX2: the scalar path), plus closed forms (constant rows, identity matrices);
 *   - RoPE: bit-exact vs the reference's rope.c built into oracle/_ref, the known-answer
 *     inputs of tests/test_rope.c (srand(42)), norm preservation, position 0 = identity;
 *     decode with RoPE: position 0 equals plain decode bit for bit, and rotating the
 *     projection weights' output columns instead of Q and K_new gives the same result.
 */
#ifndef CF_ORACLE_H_
#define CF_ORACLE_H_

#include <stddef.h>
#include <stdint.h>
#include "mha_decode_int.h"
#include "mha_fused_int.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Full MHA_Decode op.  inputs/outputs use the operator slot layout
 * (mha_decode.c:1-5): [X_new, K_cache, V_cache, WQ, bQ, WK, bK, WV, bV, WO, bO] and
 * [Y, K_cache_out, V_cache_out]; biases may be NULL.  When p->cache_len < 0,
 * inputs[11] is a host int32 array of per-sequence cache lengths. */
int oracle_mha_decode_f32(const void* inputs[], void* outputs[], const mha_decode_params_t* p);

/* Attention core with Q given: Q (B, H_q, d), K/V (B, max_seq, H_kv, d), O (B, H_q, d).
 * Sequence b attends positions 0 .. attend[b]-1. */
int oracle_decode_attn_f32(const float* Q, const float* K, const float* V, float* O,
                           int64_t B, int64_t H_q, int64_t H_kv, int64_t d, int64_t max_seq,
                           const int32_t* attend, float scale);

/* Full MHA_Fused op: [X, R, WQ, bQ, WK, bK, WV, bV, WO, bO] -> [Y]. */
int oracle_mha_fused_f32(const void* inputs[], void* outputs[], const mha_fused_params_t* p);

void oracle_causal_mask_f32(float* mask, int64_t S);

/* LayerNorm over the last dimension: x, y (N, D); gamma, beta (D). */
int  oracle_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y,
                          int64_t N, int64_t D, float eps);
/* Batched MatMul with optional transposes and bias (bias may be NULL). */
int  oracle_matmul_f32(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                       int64_t K, int transpose_a, int transpose_b, int64_t batch, int64_t stride_a,
                       int64_t stride_b, int64_t stride_c);

/* RoPE (rope.c): in/out (S, H, d), row pos rotated by position pos; in == out allowed. */
int  oracle_rope_f32(const float* in, float* out, int64_t S, int64_t H, int64_t d, float base);
/* One position: the H heads of v (H x d) rotated in place by position pos. */
void oracle_rope_at(float* v, int64_t H, int64_t d, int64_t pos, float base);
/* MHA_Decode with RoPE on Q and K_new (same slots as oracle_mha_decode_f32). */
int  oracle_mha_decode_rope_f32(const void* inputs[], void* outputs[], const mha_decode_params_t* p,
                                float rope_base);

/* Seeded generators. */
uint64_t oracle_splitmix64(uint64_t* state);
void oracle_fill_normal(float* out, size_t n, uint64_t seed, float mean, float stddev);
void oracle_fill_uniform_int(int32_t* out, size_t n, uint64_t seed, int32_t lo, int32_t hi);
/* tests/test_mha_decode.c:50-55 (glibc srand/rand) */
void oracle_fill_glibc_rand(float* out, size_t n, int seed);
/* tests/test_bert_mha.c:58-64 and tests/test_utils.h:18-24 (LCG) */
void oracle_fill_lcg(float* out, size_t n, unsigned seed);

/* IEEE binary16 conversion, round-to-nearest-even (not the reference's truncating
 * cast.c:8-17). */
uint16_t oracle_f32_to_f16(float x);
float    oracle_f16_to_f32(uint16_t h);
void     oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void     oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* Operator-signature wrappers so tests can register the oracle as the CPU ops
 * "mha_decode_f32" / "mha_fused_f32" in the product's registry (the reference's
 * CPU registrations, operator_registry.def:35,37). */
int oracle_op_mha_decode_f32(const void* inputs[], void* outputs[], const void* params, void* stream);
int oracle_op_mha_fused_f32(const void* inputs[], void* outputs[], const void* params, void* stream);
int oracle_op_causal_mask_f32(const void* inputs[], void* outputs[], const void* params, void* stream);

/* Wall-clock seconds (CLOCK_MONOTONIC), for the CPU baseline. */
double oracle_now(void);

#ifdef __cplusplus
}
#endif

#endif /* CF_ORACLE_H_ */
