/*
 * layer_ops.h — the operators next to attention in a transformer layer, on the GPU, so
 * an FP16 layer stays on the device between them: LayerNorm, Cast and MatMul in FP32 and
 * FP16.  Operator signature and return codes as in mha_ops.h (0; -1 invalid arguments
 * or workspace failure; a hipError_t value if a launch failed).
 */
#ifndef CF_LAYER_OPS_H_
#define CF_LAYER_OPS_H_

#include "operator.h"
#include "layernorm_int.h"
#include "cast_int.h"
#include "matmul_int.h"

#ifdef __cplusplus
extern "C" {
#endif

/* LayerNorm over the last dimension.  Replaces layernorm_f32_cuda
 * (src/operator/nn/layernorm_cuda.cu:107-133) and layernorm_f16_cuda
 * (src/operator/nn/norm_f16_cuda.cu:145-161): inputs [x (N, D), gamma (D), beta (D)],
 * outputs [y (N, D)]; y = (x - mean) / sqrt(var + eps) * gamma + beta with fp32
 * statistics (population variance); the _f16 op takes and writes F16. */
int layernorm_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);
int layernorm_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);

/* Cast.  Replaces cast_f32_cuda (src/operator/nn/cast_cuda.cu:33-64): INT64 <-> FLOAT,
 * FLOAT -> FLOAT16 (round to nearest even, as the reference's CUDA op; its CPU op
 * truncates), FLOAT16 -> FLOAT; any other pair copies numel * 4 bytes, as the
 * reference does. */
int cast_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);

/* MatMul C = A·B (+ bias), per batch slice.  Replaces matmul_f32_cuda
 * (src/operator/blas/matmul_cuda.cu:297-421) and matmul_f16_cuda
 * (src/operator/nn/matmul_f16_cuda.cu:27-43): inputs [A, B, bias (N) or NULL] — slot 2
 * is always read, as in the reference, so a direct caller passes three slots — and
 * outputs [C (M, N)].  Transposed operands, batches with strides and the bias are
 * honoured in both precisions (the reference's FP16 op ignored them).  K must be > 0. */
int matmul_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);
int matmul_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream);

int register_layernorm_f32_cuda(void);
int register_layernorm_f16_cuda(void);
int register_cast_f32_cuda(void);
int register_matmul_f32_cuda(void);
int register_matmul_f16_cuda(void);

#ifdef __cplusplus
}
#endif

#endif /* CF_LAYER_OPS_H_ */
