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

/* As operator_time, rotating over `n_sets` (1..16) sets of `n_inputs` input and
 * `n_outputs` output pointers (input_sets[s * n_inputs + i], output_sets[s * n_outputs
 * + o]); call j uses set j % n_sets.  With a working set larger than the GPU's
 * last-level cache (256 MB Infinity Cache on MI355X) every call reads its inputs from
 * HBM, as a decode step does once the other layers of a model have run. */
int operator_time_sets(const char* name, const void* const* input_sets, int n_inputs,
                       void* const* output_sets, int n_outputs, int n_sets,
                       const operator_params_t* params, stream_t* stream,
                       int warmup, int iters, float* ms_total);

/* The decode attention core (mha_decode_attn_{f16,f32}_cuda, inputs as for that entry,
 * rotating over `n_sets` input sets laid out as in operator_time_sets): after `warmup`
 * full calls, its split kernel is launched `iters` times (<= 4096) back to back between
 * two HIP events, then its merge kernel likewise; stores the mean time per launch of
 * each (ms).  elem_f16 selects the fp16 (1) or fp32 (0) entry. */
int mha_decode_attn_kernel_times(const void* const* input_sets, int n_inputs, int n_sets,
                                 void* outputs[], const operator_params_t* params,
                                 stream_t* stream, int elem_f16, int warmup, int iters,
                                 float* ms_split, float* ms_merge);

/* MHA_Fused (mha_fused_{f16,f32}_cuda, inputs and params as for that entry): after
 * `warmup` full calls, each of its three kernels (QKV projection, attention, output
 * projection) is launched `iters` times (<= 4096) back to back between two HIP events;
 * ms[0..2] receive the mean time per launch of each. */
int mha_fused_kernel_times(const void* inputs[], void* outputs[], const operator_params_t* params,
                           stream_t* stream, int elem_f16, int warmup, int iters, float ms[3]);

/* Synthetic inputs for timing runs, generated on the device: `n` elements (fp16 when
 * elem_f16, else fp32) of N(mean, stddev) from splitmix64 seeded with `seed` and
 * Box-Muller with both outputs used, the generator of the CPU oracle's inputs
 * (oracle_fill_normal), so a seed names the same values on both sides up to the last bit
 * of the device's double-precision log/cos/sin.  Enqueued on stream->cuda_stream (NULL:
 * the default stream).  Returns 0, -1 for bad arguments, or HIP's status. */
int synthetic_fill_normal(void* dst, int64_t n, int elem_f16, uint64_t seed, float mean, float stddev,
                          stream_t* stream);

#ifdef __cplusplus
}
#endif

#endif /* CF_OP_TIMING_H_ */
