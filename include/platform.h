/*
 * platform.h — core host types of the engine: element types, tensors, streams.
 *
 * Layout-identical to the reference interface it replaces
 * (src/platform/include/platform.h:11-58, 63-107) so that code written against the
 * reference operator/graph API compiles unchanged.  The device side of a tensor
 * (`data_device`) is HIP device memory on MI355X; `stream_t` carries a hipStream_t.
 */
#ifndef CF_PLATFORM_H_
#define CF_PLATFORM_H_

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (same enumerator order as platform.h:11-20 of the reference). */
typedef enum {
    DATA_TYPE_F32 = 0,
    DATA_TYPE_F16,
    DATA_TYPE_BF16,
    DATA_TYPE_I32,
    DATA_TYPE_I8,
    DATA_TYPE_U8,
    DATA_TYPE_I64,
    DATA_TYPE_COUNT
} data_type_t;

typedef struct {
    const char* name;
    size_t      size;       /* bytes per element */
    int         is_float;
    int         is_signed;
} data_type_info_t;

const data_type_info_t* data_type_get_info(data_type_t dt);

/* Tensor: host buffer plus an optional HIP device mirror. */
#define MAX_TENSOR_DIMS 8

typedef struct {
    data_type_t dtype;
    int         ndim;
    int64_t     shape[MAX_TENSOR_DIMS];
    int64_t     strides[MAX_TENSOR_DIMS];
    int64_t     numel;
    void*       data;        /* host pointer */
    void*       data_device; /* HIP device pointer, NULL while not resident on the GPU */
} tensor_t;

tensor_t* tensor_create(data_type_t dtype, int ndim, const int64_t* shape);
void      tensor_destroy(tensor_t* t);
/* Allocate the device mirror and upload, once: a tensor that is already resident is
 * left unchanged (reference contract, tensor.c:50-68). */
int       tensor_copy_to_device(tensor_t* t);
/* Upload host data to the device every time (allocating on first use); used for graph
 * inputs whose host data changes between executions. */
int       tensor_upload(tensor_t* t);
/* Synchronous device -> host copy (no-op for a tensor without a device mirror). */
int       tensor_copy_to_host(tensor_t* t);
bool      tensor_allclose(const tensor_t* a, const tensor_t* b, float rtol, float atol);

/* Stream handle.  The single field holds a hipStream_t (NULL = the null stream); its
 * name is kept from platform.h:56-58 so existing callers that fill it keep compiling. */
typedef struct {
    void* cuda_stream;
} stream_t;

/* Host platform ops (platform.h:63-75). */
typedef struct {
    const char* name;
    int   (*init)(void);
    void  (*finalize)(void);
    void* (*alloc_aligned)(size_t size, size_t align);
    void  (*free_aligned)(void* ptr);
    int   (*get_cache_line_size)(void);
    int   (*get_simd_flags)(void);
    int   (*get_core_count)(void);
    int   (*pin_thread)(int cpu_id);
} platform_ops_t;

extern const platform_ops_t* g_platform;

#define SIMD_AVX2   (1 << 0)
#define SIMD_AVX512 (1 << 1)
#define SIMD_NEON   (1 << 2)
#define SIMD_SVE    (1 << 3)

int   platform_get_cache_line_size(void);
int   platform_get_core_count(void);
void* platform_alloc_aligned(size_t size, size_t alignment);
void  platform_free_aligned(void* ptr);
int   platform_init(void);
void  platform_finalize(void);

#ifdef __cplusplus
}
#endif

#endif /* CF_PLATFORM_H_ */
