/*
 * gpu_ops.h — the MI355X platform module: a thin C-ABI over the HIP runtime.
 *
 * Replaces the reference's CUDA platform module (src/platform/include/cuda_ops.h:77-124,
 * src/platform/cuda/cuda_platform.h:10-27, cuda_device.cu, cuda_memory.cu, cuda_arena.cu)
 * with the same responsibilities: device select/reset, caps query, device and pinned
 * host memory, async copies, streams.  Two additions serve the operators directly:
 *   - a persistent per-device workspace (gpu_workspace_get) so that ops never allocate
 *     per call (the reference's unused arena, cuda_arena.cu:15-58, was the intent);
 *   - HIP events for timing on the stream the kernels run on.
 * Host code (C) includes only this header; nothing here exposes HIP types.
 */
#ifndef CF_GPU_OPS_H_
#define CF_GPU_OPS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* gpu_stream_t; /* hipStream_t; NULL = null stream */
typedef void* gpu_event_t;  /* hipEvent_t */

/* Runtime snapshot of the device (cuda_ops.h:77-103 restated for CDNA). */
typedef struct {
    int    device_id;
    char   name[256];
    char   arch[64];              /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int    cu_count;              /* compute units (256 on MI355X) */
    int    wavefront_size;        /* 64 */
    int    max_threads_per_block;
    int    max_threads_per_cu;
    int    regs_per_block;
    int    lds_per_block;         /* bytes */
    int    l2_bytes;
    int    clock_khz;             /* peak shader clock */
    int    mem_clock_khz;
    int    mem_bus_width;         /* bits */
    size_t total_memory;          /* bytes */
    double hbm_peak_gbs;          /* published HBM peak used for rooflines (8000 on MI355X) */
    double fp16_mfma_peak_tflops; /* dense fp16 MFMA peak (2500 on MI355X) */
    double fp32_peak_tflops;      /* vector fp32 peak (157.3 on MI355X) */
} gpu_caps_t;

/* Function table with the responsibilities of the reference's cuda_ops_t (cuda_ops.h:106-122). */
typedef struct {
    int   (*init)(int device_id);
    void  (*finalize)(void);
    void* (*device_alloc)(size_t size);
    void  (*device_free)(void* ptr);
    void* (*host_alloc_pinned)(size_t size);
    void  (*host_free_pinned)(void* ptr);
    int   (*memcpy_h2d)(void* dst, const void* src, size_t bytes, gpu_stream_t stream);
    int   (*memcpy_d2h)(void* dst, const void* src, size_t bytes, gpu_stream_t stream);
    int   (*memcpy_d2d)(void* dst, const void* src, size_t bytes, gpu_stream_t stream);
    int   (*stream_create)(gpu_stream_t* stream);
    int   (*stream_synchronize)(gpu_stream_t stream);
    int   (*stream_destroy)(gpu_stream_t stream);
    int   (*get_device_count)(int* count);
    int   (*get_gpu_caps)(gpu_caps_t* caps, int device_id);
} gpu_ops_t;

extern gpu_ops_t g_gpu;

/* Platform bring-up (cuda_platform.h:10-11).  gpu_platform_init selects the device and
 * fills g_gpu; it fails (returns nonzero) when no HIP device is present. */
int  gpu_platform_init(int device_id);
void gpu_platform_finalize(void);
int  gpu_print_caps(int device_id);

/* Flat entry points behind g_gpu (also usable directly through the C-ABI). */
int   gpu_init(int device_id);
int   gpu_available(void);                 /* 1 when at least one HIP device is usable */
void* gpu_device_alloc(size_t size);
void  gpu_device_free(void* ptr);
void* gpu_host_alloc_pinned(size_t size);
void  gpu_host_free_pinned(void* ptr);
int   gpu_memcpy_h2d(void* dst, const void* src, size_t bytes, gpu_stream_t stream);
int   gpu_memcpy_d2h(void* dst, const void* src, size_t bytes, gpu_stream_t stream);
int   gpu_memcpy_d2d(void* dst, const void* src, size_t bytes, gpu_stream_t stream);
int   gpu_memset(void* dst, int value, size_t bytes, gpu_stream_t stream);
int   gpu_stream_create(gpu_stream_t* stream);
int   gpu_stream_synchronize(gpu_stream_t stream);
int   gpu_stream_destroy(gpu_stream_t stream);
/* Stream capture into a replayable HIP graph (thread-local capture mode): between
 * gpu_capture_begin and gpu_capture_end, work enqueued on `stream` is recorded, not run.
 * gpu_capture_end instantiates the recording into *exec (0), or returns the capture's
 * error and keeps nothing.  gpu_graph_launch replays an instantiated recording on a
 * stream.  The graph executor uses these for repeated executions
 * (graph_set_replay in graph.h). */
int   gpu_capture_begin(gpu_stream_t stream);
int   gpu_capture_end(gpu_stream_t stream, void** exec);
int   gpu_graph_launch(void* exec, gpu_stream_t stream);
void  gpu_graph_exec_destroy(void* exec);
int   gpu_device_synchronize(void);
int   gpu_get_device_count(int* count);
int   gpu_current_device(void);          /* device id HIP calls on this thread go to */
int   gpu_get_gpu_caps(gpu_caps_t* caps, int device_id);
int   gpu_get_last_error(void);            /* clears and returns the sticky HIP error */
const char* gpu_error_string(int err);

/* Events (timing on the stream the kernels are launched on). */
int   gpu_event_create(gpu_event_t* ev);
int   gpu_event_destroy(gpu_event_t ev);
int   gpu_event_record(gpu_event_t ev, gpu_stream_t stream);
int   gpu_event_synchronize(gpu_event_t ev);
int   gpu_event_elapsed_ms(float* ms, gpu_event_t start, gpu_event_t stop);

/* Persistent scratch for split partials and projections, one per (current device,
 * stream): returns a 256-byte aligned device buffer of at least `bytes` bytes that only
 * work on `stream` uses, so operators on different streams may run concurrently.  It
 * grows (one synchronous reallocation) when a larger size is requested and is otherwise
 * reused; work on one stream is ordered, so successive operators there may share it.
 * Up to 16 streams per device keep their own buffer; a further stream takes over the
 * least recently used one after a device synchronisation.  Not thread-safe (like the
 * operator registry): one host thread drives a device.  NULL on allocation failure.
 * gpu_workspace_get(bytes) is the default stream's buffer. */
void*  gpu_workspace_get_stream(gpu_stream_t stream, size_t bytes);
void*  gpu_workspace_get(size_t bytes);
size_t gpu_workspace_size(void);     /* bytes held on the current device, all streams */
void   gpu_workspace_release(void);

/* Buffer generation: a counter bumped whenever a device buffer that recorded work
 * (a HIP graph) may hold a pointer to is freed or handed to another stream: workspace
 * growth, takeover and release, and operator tables rebuilt larger.  A recording made
 * at one generation must not be replayed at another (graph_execute re-records).
 * gpu_buffer_generation_bump is for operators that keep such buffers themselves. */
uint64_t gpu_buffer_generation(void);
void     gpu_buffer_generation_bump(void);

/* Registers fn to run at gpu_platform_finalize, before the workspaces are freed: for
 * device tables an operator keeps across calls (the RoPE angle tables).  Up to 8
 * callbacks; registering the same one again is a no-op.  0, or -1 when full. */
int    gpu_at_finalize(void (*fn)(void));

/* Allocation-failure injection for error-path tests: the next `n` device allocations
 * made through this module fail (return NULL).  n = 0 disables. */
void  gpu_inject_alloc_failures(int n);

#ifdef __cplusplus
}
#endif

#endif /* CF_GPU_OPS_H_ */
