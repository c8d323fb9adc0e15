/* cast_int.h — params of the Cast operator, layout-identical to the reference's
 * src/operator/nn/cast_int.h:6-16 (ONNX TensorProto data type codes). */
#ifndef CF_CAST_INT_H_
#define CF_CAST_INT_H_

#include <stdint.h>

#define ONNX_DTYPE_FLOAT    1
#define ONNX_DTYPE_FLOAT16  10
#define ONNX_DTYPE_INT64    7

typedef struct {
    int     src_dtype;   /* ONNX data type of the input */
    int     dst_dtype;   /* ONNX data type of the output */
    int64_t numel;
} cast_params_t;

#endif /* CF_CAST_INT_H_ */
