/* matmul_int.h — params of the MatMul operator, layout-identical to the reference's
 * src/operator/blas/matmul_int.h:7-17. */
#ifndef CF_MATMUL_INT_H_
#define CF_MATMUL_INT_H_

#include <stdbool.h>
#include <stdint.h>

typedef struct {
    int64_t M, N, K;
    bool    transpose_a;    /* A given as (K, M) */
    bool    transpose_b;    /* B given as (N, K) */
    int64_t batch_size;     /* independent products (1 for 2-D) */
    int64_t stride_a;       /* elements between batch slices of A */
    int64_t stride_b;       /* ... of B */
    int64_t stride_c;       /* ... of C */
    int     tuning_config;  /* the reference's CUDA kernel choice; ignored here */
} matmul_params_t;

#endif /* CF_MATMUL_INT_H_ */
