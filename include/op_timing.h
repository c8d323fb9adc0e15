/*
 * op_timing.h — device-side timing of a registered operator (measurement utility).
 *
 * No counterpart in the reference, whose benches time graph_execute wall-clock with
 * clock_gettime including copies and allocations (tests/bench_bert_mha.c:198-232,
 * tests/bench_mha_decode.c:31-36).  Here the loop runs in C so that host-language
 * overhead does not enter the measurement, and time is read from HIP events recorded on
 * the stream the kernels are launched on.
 */
#ifndef CF_OP_TIMING_H_
#define CF_OP_TIMING_H_

#include "operator.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Calls operator `name` `warmup` times, then `iters` times between two events on
 * stream->cuda_stream, and stores the elapsed milliseconds of the timed calls in
 * *ms_total.  Returns 0, -2 if the op is not registered, -1 for bad arguments, or the
 * op's / HIP's nonzero status. */
int operator_time(const char* name, const void* inputs[], void* outputs[],
                  const operator_params_t* params, stream_t* stream,
                  int warmup, int iters, float* ms_total);

/* The decode attention core (mha_decode_attn_{f16,f32}_cuda, same arguments) run
 * `iters` times (<= 4096) after `warmup` calls, with HIP events recorded around its
 * split kernel and its merge kernel separately; stores the mean duration of each (ms).
 * elem_f16 selects the fp16 (1) or fp32 (0) entry. */
int mha_decode_attn_kernel_times(const void* inputs[], void* outputs[], const operator_params_t* params,
                                 stream_t* stream, int elem_f16, int warmup, int iters,
                                 float* ms_split, float* ms_merge);

#ifdef __cplusplus
}
#endif

#endif /* CF_OP_TIMING_H_ */
