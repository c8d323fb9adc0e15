/*
 * rope_ops.h — rotary position encoding on the GPU: the reference's RoPE operator and a
 * decode operator with RoPE applied to the new token's Q and K.
 *
 * Angles follow rope.c:38-45 exactly: angle = pos / powf(base, 2i/d), with (cos, sin)
 * from glibc on the host, kept per device in a table of (n_pos, d/2) float pairs that
 * grows on demand (a synchronous upload the first time a (base, d) pair or a longer
 * range is used) and is freed by gpu_platform_finalize.  Pairs (2i, 2i+1) of each head
 * are rotated: x'[2i] = x[2i]·cos − x[2i+1]·sin, x'[2i+1] = x[2i]·sin + x[2i+1]·cos, in
 * fp32 without contraction (fp16 I/O rounds once).  Return codes as in mha_ops.h.
 */
#ifndef CF_ROPE_OPS_H_
#define CF_ROPE_OPS_H_

#include "operator.h"
#include "rope_int.h"
#include "mha_decode_int.h"

#ifdef __cplusplus
extern "C" {
#endif

/* RoPE, FP32.  Replaces rope_f32_cuda (src/operator/nn/rope_cuda.cu:35-51).
 * inputs [x (S, H, d)], outputs [y (S, H, d)], y may alias x (in place, OP_FLAG_IN_PLACE);
 * row pos is rotated by position pos.  Like the reference, one sequence (B = 1): a batch
 * is S·B rows only if positions restart per sequence, which they do not here. */
int rope_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);
/* RoPE with FP16 I/O (new; the graph dispatches "<base>_f16_cuda" for an F16 output). */
int rope_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);

/* MHA_Decode with RoPE (new; the reference runs RoPE as a separate op on the
 * projections, which its fused decode op cannot do).  Same slots, validation and
 * results as mha_decode_{f32,f16}_cuda, except that Q and K_new are rotated at the
 * token's position (cache_len, or seq_lens[b] in ragged mode) after the projection,
 * before K_new is stored and before the scores.  V is not rotated. */
typedef struct {
    mha_decode_params_t decode;
    float               rope_base;   /* > 0 */
    int32_t             reserved;    /* 0 */
} mha_decode_rope_params_t;

int mha_decode_rope_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params,
                             stream_t* stream);
int mha_decode_rope_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params,
                             stream_t* stream);

int register_rope_f32_cuda(void);
int register_rope_f16_cuda(void);
int register_mha_decode_rope_f32_cuda(void);
int register_mha_decode_rope_f16_cuda(void);

/* Device (cos, sin) table for (base, d) covering positions 0 .. n_pos-1 on the current
 * device (NULL on failure).  Owned by the library. */
const float* rope_table_device(float base, int64_t d, int64_t n_pos);

#ifdef __cplusplus
}
#endif

#endif /* CF_ROPE_OPS_H_ */
