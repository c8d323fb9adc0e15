/*
 * rope_int.h — params of the RoPE operator, layout-identical to the reference's
 * src/operator/nn/rope_int.h:6-11.
 */
#ifndef CF_ROPE_INT_H_
#define CF_ROPE_INT_H_

#include <stdint.h>

typedef struct {
    int64_t seq_len;    /* S: rows of the (S, H, d) tensor; row pos is position pos */
    int64_t head_dim;   /* d (even) */
    int64_t num_heads;  /* H */
    float   base;       /* theta base, typically 10000.0 */
} rope_params_t;

#endif /* CF_ROPE_INT_H_ */
