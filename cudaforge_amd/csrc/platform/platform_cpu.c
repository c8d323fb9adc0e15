/* platform_cpu.c — host platform ops (src/platform/cpu/platform_cpu.c:20-150 of the
 * reference): aligned allocation, cache-line size and core count, pinning. */
#define _GNU_SOURCE
#include "platform.h"

#include <sched.h>
#include <stdlib.h>
#include <unistd.h>

static int g_line = 64;
static int g_cores = 1;

static int host_init(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    g_cores = n > 0 ? (int)n : 1;
    long sz = sysconf(_SC_LEVEL1_DCACHE_LINESIZE);
    if (sz > 0) g_line = (int)sz;
    return 0;
}

static void host_finalize(void) {}

static void* host_alloc_aligned(size_t size, size_t align) {
    void* p = NULL;
    if (align < sizeof(void*)) align = sizeof(void*);
    if (posix_memalign(&p, align, size ? size : 1) != 0) return NULL;
    return p;
}

static void host_free_aligned(void* p) { free(p); }
static int host_line(void) { return g_line; }

static int host_simd(void) {
    int f = 0;
#if defined(__AVX2__)
    f |= SIMD_AVX2;
#endif
#if defined(__AVX512F__)
    f |= SIMD_AVX512;
#endif
    return f;
}

static int host_cores(void) { return g_cores; }

static int host_pin(int cpu) {
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(cpu, &set);
    return sched_setaffinity(0, sizeof(set), &set) == 0 ? 0 : -1;
}

static const platform_ops_t k_host = {
    .name = "x86",
    .init = host_init,
    .finalize = host_finalize,
    .alloc_aligned = host_alloc_aligned,
    .free_aligned = host_free_aligned,
    .get_cache_line_size = host_line,
    .get_simd_flags = host_simd,
    .get_core_count = host_cores,
    .pin_thread = host_pin,
};

const platform_ops_t* g_platform = NULL;

int platform_init(void) {
    g_platform = &k_host;
    return g_platform->init();
}

void platform_finalize(void) {
    if (g_platform) g_platform->finalize();
    g_platform = NULL;
}

int platform_get_cache_line_size(void) { return g_platform ? g_platform->get_cache_line_size() : 64; }
int platform_get_core_count(void) { return g_platform ? g_platform->get_core_count() : 1; }

/* Works before platform_init (tensors may be created first). */
void* platform_alloc_aligned(size_t size, size_t alignment) { return host_alloc_aligned(size, alignment); }
void platform_free_aligned(void* ptr) { host_free_aligned(ptr); }
