/*
 * mha_ops.h — the HIP operators of the attention hot path and their registrations.
 *
 * Every function has the operator_func_t signature (operator.h) and takes device
 * pointers.  Return: 0 on success, -1 on invalid arguments or workspace allocation
 * failure, a positive hipError_t value if a launch failed.  Work is enqueued on
 * stream->cuda_stream (NULL stream when `stream` is NULL) and not synchronised.
 */
#ifndef CF_MHA_OPS_H_
#define CF_MHA_OPS_H_

#include <stdint.h>
#include "operator.h"
#include "mha_decode_int.h"
#include "mha_fused_int.h"
#include "causal_mask_int.h"

#ifdef __cplusplus
extern "C" {
#endif

/* MHA_Decode, FP32 I/O.  Replaces mha_decode_f32_cuda (src/operator/nn/mha_decode_cuda.cu:159-190).
 * inputs  [X_new(B,1,D), K_cache(B,max_seq,H_kv,d), V_cache, WQ(D,D), bQ(D), WK(D,H_kv*d), bK,
 *          WV(D,H_kv*d), bV, WO(D,D), bO(D)] (+ [seq_lens int32 (B)] when cache_len < 0)
 * outputs [Y(B,1,D), K_cache_out, V_cache_out]
 * All eleven inputs must be non-NULL (mha_decode.c:15, mha_decode_cuda.cu:162).  The new
 * K/V row is written at position cache_len of the output caches; history is read from
 * the output caches, which are first filled from the input caches unless they alias
 * them (in-place update, the decode-loop use). */
int mha_decode_f32_cuda(const void* inputs[], void* outputs[],
                        const operator_params_t* params, stream_t* stream);
/* MHA_Decode with FP16 activations, caches and weights, fp32 accumulation (new; the
 * graph dispatches "<base>_f16_cuda" for an F16 output, graph.c:841-868). */
int mha_decode_f16_cuda(const void* inputs[], void* outputs[],
                        const operator_params_t* params, stream_t* stream);

/* Decode attention core, Q given (new entry; the split-KV core of the decode op).
 * inputs  [Q(B,H_q,d), K_cache(B,max_seq,H_kv,d), V_cache] (+ [seq_lens] when cache_len < 0)
 * outputs [O(B,H_q,d)]; sequence b attends positions 0..cache_len (or 0..seq_lens[b]).
 * params: mha_decode_params_t (hidden_size is ignored). */
int mha_decode_attn_f32_cuda(const void* inputs[], void* outputs[],
                             const operator_params_t* params, stream_t* stream);
int mha_decode_attn_f16_cuda(const void* inputs[], void* outputs[],
                             const operator_params_t* params, stream_t* stream);

/* Allocation-free variant of mha_decode_attn_f16_cuda.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments, plan, kernels
 * and result bits; the split partials live in a fixed 16 MiB device array per GPU
 * (cf. cf_decode_attn_scratch_bytes) instead of the stream workspace, and no call
 * allocates or frees anything.  A plan whose partials exceed that array returns -1 with
 * a message on stderr.  One caller at a time per GPU: every call on one GPU shares the
 * array, so calls that overlap there in time (different streams, or threads) race and
 * give undefined results; order them on one stream. */
int mha_decode_attn_f16_noalloc(const void* inputs[], void* outputs[],
                                const operator_params_t* params, stream_t* stream);

/* MHA_Fused, FP32 I/O.  Replaces mha_fused_f32_cuda (src/operator/nn/mha_fused_cuda.cu:938-1189).
 * inputs  [X(B,S,D), R(B,S,D) or NULL, WQ(D,D), bQ, WK(D,H_kv*d), bK, WV(D,H_kv*d), bV, WO(D,D), bO]
 * outputs [Y(B,S,D)]; honours causal and num_kv_heads (the reference CPU op ignores both). */
int mha_fused_f32_cuda(const void* inputs[], void* outputs[],
                       const operator_params_t* params, stream_t* stream);
/* MHA_Fused with FP16 arithmetic behind FP32 buffers: replaces mha_fused_f16_cuda
 * (src/operator/nn/mha_fused_f16_cuda.cu:209-244, registered "f32"), same slots and
 * buffer types.  Inputs are rounded to fp16, the fp16 path runs, Y is widened to fp32;
 * any S (the reference took S <= 64). */
int mha_fused_f16_cuda(const void* inputs[], void* outputs[],
                       const operator_params_t* params, stream_t* stream);
/* MHA_Fused with FP16 buffers and fp32 accumulation (registered "f16"): the op graphs of
 * F16 tensors dispatch MHA_Fused nodes to (the reference's graph named
 * mha_fused_f16_cuda there, graph.c:841-865, which read those buffers as floats).  Same
 * slots; every activation, weight and bias _Float16. */
int mha_fused_f16io_cuda(const void* inputs[], void* outputs[],
                         const operator_params_t* params, stream_t* stream);

/* CausalMask (src/operator/nn/causal_mask_cuda.cu:6-29): outputs [mask(S,S) f32]. */
int causal_mask_f32_cuda(const void* inputs[], void* outputs[],
                         const operator_params_t* params, stream_t* stream);

int register_mha_decode_f32_cuda(void);
int register_mha_decode_f16_cuda(void);
int register_mha_decode_attn_f32_cuda(void);
int register_mha_decode_attn_f16_cuda(void);
int register_mha_fused_f32_cuda(void);
int register_mha_fused_f16_cuda(void);
int register_mha_fused_f16io_cuda(void);
int register_causal_mask_f32_cuda(void);

/* Decode split planning.  Positions per split for the next calls: 0 = automatic (fill
 * every CU), otherwise rounded to the kernel's quantum.  Process-wide; for tuning and
 * split-invariance tests. */
void    mha_decode_set_split_chunk(int64_t chunk);
/* Prefill (mha_fused_f16io_cuda and mha_fused_f16_cuda): 1 (default) writes the QKV projection as one row-major
 * (B*S, (H + 2 H_kv) d) matrix that attention reads directly, where both kernels take it
 * (fp16, d = 64, S % 8 == 0); 0 always scatters q, k, v^T head-major.  Process-wide; for
 * tests and measurements. */
void    mha_fused_set_rowcat(int on);
/* The (chunk, n_split) the decode core would use for these params on this device. */
int     mha_decode_plan(const mha_decode_params_t* p, int elem_f16, int64_t* chunk, int64_t* n_split);

#ifdef __cplusplus
}
#endif

#endif /* CF_MHA_OPS_H_ */
