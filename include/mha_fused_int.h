/*
 * mha_fused_int.h — params of the MHA_Fused operator.
 *
 * Layout-identical to src/operator/nn/mha_fused_int.h:7-17 of the reference.
 * The reference's FA_* tile constants (mha_fused_int.h:28-47) describe its CUDA
 * kernels and are not part of the interface; the MI355X tiles live with the kernels.
 */
#ifndef CF_MHA_FUSED_INT_H_
#define CF_MHA_FUSED_INT_H_

#include <stdint.h>
#include <stdbool.h>

typedef struct {
    int64_t batch_size;   /* B */
    int64_t seq_len;      /* S */
    int64_t hidden_size;  /* D */
    int64_t num_heads;    /* H_q */
    int64_t num_kv_heads; /* H_kv (<= 0 means H_q); WK/WV are (D, H_kv*d) */
    int64_t head_dim;     /* d */
    float   scale;        /* usually 1/sqrt(d) */
    bool    has_residual; /* add inputs[1] to the output when it is non-NULL */
    bool    causal;       /* key j is visible to query i iff j <= i */
} mha_fused_params_t;

#define MHA_FUSED_NUM_INPUTS  10
#define MHA_FUSED_NUM_OUTPUTS 1

#endif /* CF_MHA_FUSED_INT_H_ */
