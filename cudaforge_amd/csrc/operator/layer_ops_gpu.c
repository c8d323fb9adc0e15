/*
 * layer_ops_gpu.c — host side of the HIP LayerNorm, Cast and MatMul operators (the
 * reference's layernorm_cuda.cu:107-141, norm_f16_cuda.cu:145-168, cast_cuda.cu:33-71,
 * matmul_cuda.cu:297-429 and matmul_f16_cuda.cu:27-50).
 */
#include "layer_ops.h"
#include "gpu_ops.h"
#include "op_common.h"
#include "../kernels/kernels.h"

#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------ LayerNorm --- */

static int layernorm_op(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                        stream_t* stream) {
    if (!inputs || !inputs[0] || !inputs[1] || !inputs[2] || !outputs || !outputs[0] || !params) return -1;
    const layernorm_params_t* p = (const layernorm_params_t*)params;
    if (p->N < 0 || p->normalized_size <= 0 || p->normalized_size > INT32_MAX) return -1;
    cf_layernorm_args_t a;
    memset(&a, 0, sizeof(a));
    a.x = inputs[0];
    a.gamma = inputs[1];
    a.beta = inputs[2];
    a.y = outputs[0];
    a.N = p->N;
    a.D = (int32_t)p->normalized_size;
    a.eps = p->epsilon;
    a.elem = elem;
    return cf_launch_layernorm(&a, cf_stream_of(stream));
}

int layernorm_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    return layernorm_op(CF_ELEM_F32, inputs, outputs, params, stream);
}

int layernorm_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    return layernorm_op(CF_ELEM_F16, inputs, outputs, params, stream);
}

/* ------------------------------------------------------------------ Cast --- */

int cast_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    if (!inputs || !inputs[0] || !outputs || !outputs[0] || !params) return -1;
    const cast_params_t* p = (const cast_params_t*)params;
    if (p->numel < 0) return -1;
    void* st = cf_stream_of(stream);
    int kind = -1;
    if (p->src_dtype == ONNX_DTYPE_INT64 && p->dst_dtype == ONNX_DTYPE_FLOAT) kind = CF_CAST_I64_F32;
    else if (p->src_dtype == ONNX_DTYPE_FLOAT && p->dst_dtype == ONNX_DTYPE_INT64) kind = CF_CAST_F32_I64;
    else if (p->src_dtype == ONNX_DTYPE_FLOAT && p->dst_dtype == ONNX_DTYPE_FLOAT16) kind = CF_CAST_F32_F16;
    else if (p->src_dtype == ONNX_DTYPE_FLOAT16 && p->dst_dtype == ONNX_DTYPE_FLOAT) kind = CF_CAST_F16_F32;
    if (kind < 0) {
        /* Other pairs: a copy of numel floats (cast.c:70, cast_cuda.cu:58-62). */
        if (p->numel == 0 || inputs[0] == outputs[0]) return 0;
        return gpu_memcpy_d2d(outputs[0], inputs[0], (size_t)p->numel * sizeof(float), st);
    }
    return cf_launch_cast(inputs[0], outputs[0], p->numel, kind, st);
}

/* ------------------------------------------------------------------ MatMul --- */

static int matmul_op(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                     stream_t* stream) {
    if (!inputs || !inputs[0] || !inputs[1] || !outputs || !outputs[0] || !params) return -1;
    const matmul_params_t* p = (const matmul_params_t*)params;
    const int64_t M = p->M, N = p->N, K = p->K;
    const int64_t batch = p->batch_size > 0 ? p->batch_size : 1;
    if (M < 0 || N < 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return -1;
    if (M == 0 || N == 0) return 0;
    if (batch > 1 && (p->stride_a < 0 || p->stride_b < 0 || p->stride_c < 0)) return -1;
    const size_t esz = elem == CF_ELEM_F16 ? 2 : 4;
    void* st = cf_stream_of(stream);
    const char* A = (const char*)inputs[0];
    const char* B = (const char*)inputs[1];
    int64_t sa = batch > 1 ? p->stride_a : 0, sb = batch > 1 ? p->stride_b : 0;
    const int64_t sc = batch > 1 ? p->stride_c : 0;

    /* Transposed operands are first made row-major in the workspace
     * (matmul_cuda.cu:320-352 transposes into per-call allocations). */
    if (p->transpose_a || p->transpose_b) {
        size_t cur = 0;
        const size_t off_a = p->transpose_a ? cf_ws_take(&cur, (size_t)batch * M * K * esz) : 0;
        const size_t off_b = p->transpose_b ? cf_ws_take(&cur, (size_t)batch * K * N * esz) : 0;
        char* ws = (char*)gpu_workspace_get_stream(st, cur);
        if (!ws) return -1;
        int rc;
        if (p->transpose_a) {
            if ((rc = cf_launch_transpose(A, ws + off_a, K, M, batch, sa, M * K, (int32_t)esz, st)) != 0) return rc;
            A = ws + off_a;
            sa = M * K;
        }
        if (p->transpose_b) {
            if ((rc = cf_launch_transpose(B, ws + off_b, N, K, batch, sb, K * N, (int32_t)esz, st)) != 0) return rc;
            B = ws + off_b;
            sb = K * N;
        }
    }
    for (int64_t bi = 0; bi < batch; bi++) {
        cf_gemm_args_t g;
        memset(&g, 0, sizeof(g));
        g.a = A + (size_t)(bi * sa) * esz;
        g.M = (int32_t)M;
        g.K = (int32_t)K;
        g.nseg = 1;
        g.w[0] = B + (size_t)(bi * sb) * esz;
        g.bias[0] = inputs[2];
        g.n[0] = (int32_t)N;
        g.out_kind = CF_GEMM_OUT_ROWMAJOR;
        g.out[0] = (char*)outputs[0] + (size_t)(bi * sc) * esz;
        g.elem = elem;
        const int rc = cf_launch_gemm(&g, st);
        if (rc != 0) return rc;
    }
    return 0;
}

int matmul_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    return matmul_op(CF_ELEM_F32, inputs, outputs, params, stream);
}

int matmul_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    return matmul_op(CF_ELEM_F16, inputs, outputs, params, stream);
}

/* ------------------------------------------------------------------ registrations --- */

int register_layernorm_f32_cuda(void) {
    static const operator_registry_t reg = {"layernorm_f32_cuda", "f32", layernorm_f32_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_layernorm_f16_cuda(void) {
    static const operator_registry_t reg = {"layernorm_f16_cuda", "f16", layernorm_f16_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_cast_f32_cuda(void) {
    static const operator_registry_t reg = {"cast_f32_cuda", "f32", cast_f32_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_matmul_f32_cuda(void) {
    static const operator_registry_t reg = {"matmul_f32_cuda", "f32", matmul_f32_cuda, 3, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_matmul_f16_cuda(void) {
    static const operator_registry_t reg = {"matmul_f16_cuda", "f16", matmul_f16_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}
