/* layernorm_int.h — params of the LayerNorm operator, layout-identical to the
 * reference's src/operator/nn/layernorm_int.h:6-10. */
#ifndef CF_LAYERNORM_INT_H_
#define CF_LAYERNORM_INT_H_

#include <stdint.h>

typedef struct {
    int64_t N;               /* rows (product of the dimensions before the normalised one) */
    int64_t normalized_size; /* D */
    float   epsilon;
} layernorm_params_t;

#endif /* CF_LAYERNORM_INT_H_ */
