/*
 * causal_mask_int.h — params of the CausalMask operator (src/operator/nn/causal_mask_int.h:6-8).
 * Output is an (S, S) float mask: 0 where key j <= query i, -inf above the diagonal.
 */
#ifndef CF_CAUSAL_MASK_INT_H_
#define CF_CAUSAL_MASK_INT_H_

#include <stdint.h>

typedef struct {
    int64_t seq_len;
} causal_mask_params_t;

#endif /* CF_CAUSAL_MASK_INT_H_ */
