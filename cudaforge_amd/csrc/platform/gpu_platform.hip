// gpu_platform.hip — the HIP runtime behind include/gpu_ops.h.
//
// Replaces the reference's CUDA platform module (src/platform/cuda/cuda_device.cu,
// cuda_memory.cu, cuda_arena.cu, cuda_platform_init.cu) with the same duties on HIP,
// plus a persistent per-device workspace so operators never allocate per call
// (the reference allocates per call, mha_fused_cuda.cu:976-1038).

#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include "gpu_ops.h"
#include "kernels.h"

namespace {

constexpr int kMaxDevices = 16;

// One workspace per (device, stream): operators on different streams may run at the
// same time, so each stream gets its own scratch.  kWsSlots streams per device; a new
// stream beyond that takes over the least recently used slot (after a device sync).
constexpr int kWsSlots = 16;
struct Workspace {
    void*         base = nullptr;
    size_t        bytes = 0;
    hipStream_t   stream = nullptr;
    bool          used = false;
    unsigned long last = 0;
};
Workspace g_ws[kMaxDevices][kWsSlots];
unsigned long g_ws_clock = 0;
int g_inject_failures = 0;
int g_initialized_device = -1;
// Bumped whenever a buffer that recorded work may point at is freed or handed to
// another stream (workspace slots, operator tables): recordings made before the bump
// must not be replayed.
uint64_t g_buffer_generation = 1;

int current_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    return dev;
}

int rc(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

}  // namespace

extern "C" {

gpu_ops_t g_gpu;

int gpu_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n > 0 ? 1 : 0;
}

int gpu_init(int device_id) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return e != hipSuccess ? (int)e : (int)hipErrorNoDevice;
    }
    if (device_id < 0 || device_id >= n) return (int)hipErrorInvalidDevice;
    e = hipSetDevice(device_id);
    if (e == hipSuccess) g_initialized_device = device_id;
    return rc(e);
}

void gpu_inject_alloc_failures(int n) { g_inject_failures = n > 0 ? n : 0; }

void* gpu_device_alloc(size_t size) {
    if (g_inject_failures > 0) {
        g_inject_failures--;
        return nullptr;
    }
    void* p = nullptr;
    if (size == 0) size = 1;
    if (hipMalloc(&p, size) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

void gpu_device_free(void* ptr) {
    if (ptr) (void)hipFree(ptr);
}

void* gpu_host_alloc_pinned(size_t size) {
    void* p = nullptr;
    if (hipHostMalloc(&p, size ? size : 1, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

void gpu_host_free_pinned(void* ptr) {
    if (ptr) (void)hipHostFree(ptr);
}

int gpu_memcpy_h2d(void* dst, const void* src, size_t bytes, gpu_stream_t stream) {
    if (bytes == 0) return 0;
    if (!dst || !src) return (int)hipErrorInvalidValue;
    return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
}

int gpu_memcpy_d2h(void* dst, const void* src, size_t bytes, gpu_stream_t stream) {
    if (bytes == 0) return 0;
    if (!dst || !src) return (int)hipErrorInvalidValue;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
    // Host memory may be pageable: the copy is complete only after the stream drains.
    return rc(hipStreamSynchronize((hipStream_t)stream));
}

int gpu_memcpy_d2d(void* dst, const void* src, size_t bytes, gpu_stream_t stream) {
    if (bytes == 0 || dst == src) return 0;
    if (!dst || !src) return (int)hipErrorInvalidValue;
    return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int gpu_memset(void* dst, int value, size_t bytes, gpu_stream_t stream) {
    if (bytes == 0) return 0;
    return rc(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
}

int gpu_stream_create(gpu_stream_t* stream) {
    if (!stream) return (int)hipErrorInvalidValue;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = (gpu_stream_t)s;
    return rc(e);
}

int gpu_stream_synchronize(gpu_stream_t stream) { return rc(hipStreamSynchronize((hipStream_t)stream)); }
int gpu_stream_destroy(gpu_stream_t stream) { return stream ? rc(hipStreamDestroy((hipStream_t)stream)) : 0; }
int gpu_device_synchronize(void) { return rc(hipDeviceSynchronize()); }

int gpu_capture_begin(gpu_stream_t stream) {
    if (!stream) return (int)hipErrorInvalidValue;   // the legacy stream cannot be captured
    return rc(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
}

int gpu_capture_end(gpu_stream_t stream, void** exec) {
    if (!exec) return (int)hipErrorInvalidValue;
    *exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &graph);
    if (e != hipSuccess || !graph) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipGetLastError();
        return e != hipSuccess ? (int)e : (int)hipErrorStreamCaptureInvalidated;
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return (int)e;
    }
    *exec = (void*)x;
    return 0;
}

int gpu_graph_launch(void* exec, gpu_stream_t stream) {
    if (!exec) return (int)hipErrorInvalidValue;
    return rc(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream));
}

void gpu_graph_exec_destroy(void* exec) {
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

int gpu_get_device_count(int* count) {
    if (!count) return (int)hipErrorInvalidValue;
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) { (void)hipGetLastError(); *count = 0; }
    return rc(e);
}

int gpu_current_device(void) { return current_device(); }

int gpu_get_last_error(void) { return (int)hipGetLastError(); }
const char* gpu_error_string(int err) { return hipGetErrorString((hipError_t)err); }

int gpu_get_gpu_caps(gpu_caps_t* caps, int device_id) {
    if (!caps) return (int)hipErrorInvalidValue;
    memset(caps, 0, sizeof(*caps));
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, device_id);
    if (e != hipSuccess) return (int)e;
    caps->device_id = device_id;
    snprintf(caps->name, sizeof(caps->name), "%s", p.name);
    snprintf(caps->arch, sizeof(caps->arch), "%s", p.gcnArchName);
    caps->cu_count = p.multiProcessorCount;
    caps->wavefront_size = p.warpSize;
    caps->max_threads_per_block = p.maxThreadsPerBlock;
    caps->max_threads_per_cu = p.maxThreadsPerMultiProcessor;
    caps->regs_per_block = p.regsPerBlock;
    caps->lds_per_block = (int)p.sharedMemPerBlock;
    caps->l2_bytes = p.l2CacheSize;
    caps->clock_khz = p.clockRate;
    caps->mem_clock_khz = p.memoryClockRate;
    caps->mem_bus_width = p.memoryBusWidth;
    caps->total_memory = p.totalGlobalMem;
    if (strncmp(p.gcnArchName, "gfx950", 6) == 0) {
        // MI355X published peaks: HBM3E 8 TB/s, dense fp16 MFMA 2.5 PFLOP/s, fp32 157.3 TFLOP/s.
        caps->hbm_peak_gbs = 8000.0;
        caps->fp16_mfma_peak_tflops = 2500.0;
        caps->fp32_peak_tflops = 157.3;
    } else {
        const double ghz = p.clockRate * 1e-6;
        caps->hbm_peak_gbs = 2.0 * p.memoryClockRate * 1e-6 * (p.memoryBusWidth / 8.0);
        caps->fp16_mfma_peak_tflops = p.multiProcessorCount * 2048.0 * ghz * 1e-3;
        caps->fp32_peak_tflops = p.multiProcessorCount * 256.0 * ghz * 1e-3;
    }
    return 0;
}

int gpu_event_create(gpu_event_t* ev) {
    if (!ev) return (int)hipErrorInvalidValue;
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreate(&e);
    *ev = (gpu_event_t)e;
    return rc(r);
}
int gpu_event_destroy(gpu_event_t ev) { return ev ? rc(hipEventDestroy((hipEvent_t)ev)) : 0; }
int gpu_event_record(gpu_event_t ev, gpu_stream_t stream) {
    return rc(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
}
int gpu_event_synchronize(gpu_event_t ev) { return rc(hipEventSynchronize((hipEvent_t)ev)); }
int gpu_event_elapsed_ms(float* ms, gpu_event_t start, gpu_event_t stop) {
    if (!ms) return (int)hipErrorInvalidValue;
    return rc(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}

void* gpu_workspace_get_stream(gpu_stream_t stream, size_t bytes) {
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    hipStream_t st = (hipStream_t)stream;
    Workspace* slot = nullptr;
    for (int i = 0; i < kWsSlots && !slot; i++)
        if (g_ws[dev][i].used && g_ws[dev][i].stream == st) slot = &g_ws[dev][i];
    for (int i = 0; i < kWsSlots && !slot; i++)
        if (!g_ws[dev][i].used) slot = &g_ws[dev][i];
    if (!slot) {
        slot = &g_ws[dev][0];
        for (int i = 1; i < kWsSlots; i++)
            if (g_ws[dev][i].last < slot->last) slot = &g_ws[dev][i];
        (void)hipDeviceSynchronize();   // its previous stream may still be using it
        g_buffer_generation++;          // ... and a recording on that stream may point at it
    }
    slot->used = true;
    slot->stream = st;
    slot->last = ++g_ws_clock;
    const size_t need = ((bytes + 255) / 256) * 256;
    if (slot->base && slot->bytes >= need) return slot->base;
    // Grow: in-flight kernels may still use the old buffer.
    if (slot->base) {
        (void)hipDeviceSynchronize();
        (void)hipFree(slot->base);
        slot->base = nullptr;
        slot->bytes = 0;
        g_buffer_generation++;
    }
    size_t grow = need < (size_t)64 << 20 ? (size_t)64 << 20 : need + need / 4;
    void* p = gpu_device_alloc(grow);
    if (!p) return nullptr;
    slot->base = p;
    slot->bytes = grow;
    return p;
}

void* gpu_workspace_get(size_t bytes) { return gpu_workspace_get_stream(nullptr, bytes); }

size_t gpu_workspace_size(void) {
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return 0;
    size_t total = 0;
    for (int i = 0; i < kWsSlots; i++) total += g_ws[dev][i].bytes;
    return total;
}

void gpu_workspace_release(void) {
    for (int d = 0; d < kMaxDevices; d++) {
        bool any = false;
        for (int i = 0; i < kWsSlots; i++) any = any || g_ws[d][i].base;
        if (!any) continue;
        int prev = current_device();
        (void)hipSetDevice(d);
        (void)hipDeviceSynchronize();
        for (int i = 0; i < kWsSlots; i++) {
            if (g_ws[d][i].base) (void)hipFree(g_ws[d][i].base);
            g_ws[d][i] = Workspace{};
        }
        g_buffer_generation++;
        (void)hipSetDevice(prev);
    }
}

extern "C" uint64_t gpu_buffer_generation(void) { return g_buffer_generation; }
extern "C" void gpu_buffer_generation_bump(void) { g_buffer_generation++; }

static void (*g_at_finalize[8])(void);

extern "C" int gpu_at_finalize(void (*fn)(void)) {
    if (!fn) return -1;
    for (auto& f : g_at_finalize) {
        if (f == fn) return 0;
        if (!f) { f = fn; return 0; }
    }
    return -1;
}

static void gpu_finalize_impl(void) {
    for (auto f : g_at_finalize)
        if (f) f();
    gpu_workspace_release();
    g_initialized_device = -1;
}

int gpu_platform_init(int device_id) {
    int e = gpu_init(device_id);
    if (e != 0) return e;
    // The allocation-free decode entry's fixed scratch: its address on this device.
    if ((e = cf_decode_attn_scratch_init()) != 0) return e;
    g_gpu.init = gpu_init;
    g_gpu.finalize = gpu_finalize_impl;
    g_gpu.device_alloc = gpu_device_alloc;
    g_gpu.device_free = gpu_device_free;
    g_gpu.host_alloc_pinned = gpu_host_alloc_pinned;
    g_gpu.host_free_pinned = gpu_host_free_pinned;
    g_gpu.memcpy_h2d = gpu_memcpy_h2d;
    g_gpu.memcpy_d2h = gpu_memcpy_d2h;
    g_gpu.memcpy_d2d = gpu_memcpy_d2d;
    g_gpu.stream_create = gpu_stream_create;
    g_gpu.stream_synchronize = gpu_stream_synchronize;
    g_gpu.stream_destroy = gpu_stream_destroy;
    g_gpu.get_device_count = gpu_get_device_count;
    g_gpu.get_gpu_caps = gpu_get_gpu_caps;
    return 0;
}

void gpu_platform_finalize(void) {
    if (g_gpu.finalize) g_gpu.finalize();
    memset(&g_gpu, 0, sizeof(g_gpu));
}

int gpu_print_caps(int device_id) {
    gpu_caps_t c;
    const int e = gpu_get_gpu_caps(&c, device_id);
    if (e != 0) return e;
    fprintf(stderr,
            "GPU %d: %s (%s)\n  CUs %d, wave%d, LDS/block %d B, L2 %d B, clock %d kHz\n"
            "  HBM %.1f GiB, peak %.0f GB/s, fp16 MFMA %.0f TFLOP/s, fp32 %.1f TFLOP/s\n",
            c.device_id, c.name, c.arch, c.cu_count, c.wavefront_size, c.lds_per_block, c.l2_bytes,
            c.clock_khz, c.total_memory / 1073741824.0, c.hbm_peak_gbs, c.fp16_mfma_peak_tflops,
            c.fp32_peak_tflops);
    return 0;
}

}  // extern "C"
