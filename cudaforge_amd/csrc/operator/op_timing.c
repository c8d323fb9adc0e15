/* op_timing.c — event-timed loop over a registered operator (see include/op_timing.h). */
#include "op_timing.h"
#include "gpu_ops.h"
#include "../kernels/kernels.h"

int synthetic_fill_normal(void* dst, int64_t n, int elem_f16, uint64_t seed, float mean, float stddev,
                          stream_t* stream) {
    if (!dst || n < 0) return -1;
    return cf_launch_fill_normal(dst, (size_t)n, elem_f16 ? CF_ELEM_F16 : CF_ELEM_F32, seed, mean, stddev,
                                 stream ? stream->cuda_stream : NULL);
}

int operator_time(const char* name, const void* inputs[], void* outputs[],
                  const operator_params_t* params, stream_t* stream,
                  int warmup, int iters, float* ms_total) {
    if (!name || !ms_total || iters <= 0 || warmup < 0) return -1;
    const operator_registry_t* op = operator_find(name);
    if (!op) return -2;
    void* s = stream ? stream->cuda_stream : NULL;
    int rc;
    for (int i = 0; i < warmup; i++)
        if ((rc = op->func(inputs, outputs, params, stream)) != 0) return rc;
    if ((rc = gpu_stream_synchronize(s)) != 0) return rc;
    gpu_event_t e0 = NULL, e1 = NULL;
    if ((rc = gpu_event_create(&e0)) != 0) return rc;
    if ((rc = gpu_event_create(&e1)) != 0) { gpu_event_destroy(e0); return rc; }
    rc = gpu_event_record(e0, s);
    for (int i = 0; i < iters && rc == 0; i++) rc = op->func(inputs, outputs, params, stream);
    if (rc == 0) rc = gpu_event_record(e1, s);
    if (rc == 0) rc = gpu_event_synchronize(e1);
    if (rc == 0) rc = gpu_event_elapsed_ms(ms_total, e0, e1);
    gpu_event_destroy(e0);
    gpu_event_destroy(e1);
    return rc;
}

int operator_time_sets(const char* name, const void* const* input_sets, int n_inputs,
                       void* const* output_sets, int n_outputs, int n_sets,
                       const operator_params_t* params, stream_t* stream,
                       int warmup, int iters, float* ms_total) {
    if (!name || !input_sets || !output_sets || !ms_total || iters <= 0 || warmup < 0 || n_inputs <= 0 ||
        n_outputs <= 0 || n_sets < 1 || n_sets > 16)
        return -1;
    const operator_registry_t* op = operator_find(name);
    if (!op) return -2;
    void* s = stream ? stream->cuda_stream : NULL;
    int rc;
#define CF_SET_IN(j) ((const void**)&input_sets[((j) % n_sets) * n_inputs])
#define CF_SET_OUT(j) ((void**)&output_sets[((j) % n_sets) * n_outputs])
    for (int i = 0; i < warmup; i++)
        if ((rc = op->func(CF_SET_IN(i), CF_SET_OUT(i), params, stream)) != 0) return rc;
    if ((rc = gpu_stream_synchronize(s)) != 0) return rc;
    gpu_event_t e0 = NULL, e1 = NULL;
    if ((rc = gpu_event_create(&e0)) != 0) return rc;
    if ((rc = gpu_event_create(&e1)) != 0) { gpu_event_destroy(e0); return rc; }
    rc = gpu_event_record(e0, s);
    for (int i = 0; i < iters && rc == 0; i++) rc = op->func(CF_SET_IN(i), CF_SET_OUT(i), params, stream);
#undef CF_SET_IN
#undef CF_SET_OUT
    if (rc == 0) rc = gpu_event_record(e1, s);
    if (rc == 0) rc = gpu_event_synchronize(e1);
    if (rc == 0) rc = gpu_event_elapsed_ms(ms_total, e0, e1);
    gpu_event_destroy(e0);
    gpu_event_destroy(e1);
    return rc;
}
