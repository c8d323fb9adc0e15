/* tensor.c — host tensors with a HIP device mirror (src/platform/tensor.c:10-130 of the
 * reference).  Device memory comes from the platform module (gpu_ops.h). */
#include "platform.h"
#include "gpu_ops.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static size_t tensor_bytes(const tensor_t* t) {
    const data_type_info_t* info = data_type_get_info(t->dtype);
    return info ? (size_t)t->numel * info->size : 0;
}

tensor_t* tensor_create(data_type_t dtype, int ndim, const int64_t* shape) {
    if (ndim < 0 || ndim > MAX_TENSOR_DIMS || !shape) return NULL;
    const data_type_info_t* info = data_type_get_info(dtype);
    if (!info) return NULL;
    tensor_t* t = (tensor_t*)calloc(1, sizeof(tensor_t));
    if (!t) return NULL;
    t->dtype = dtype;
    t->ndim = ndim;
    t->numel = 1;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] < 0) { free(t); return NULL; }
        t->shape[i] = shape[i];
        t->numel *= shape[i];
    }
    int64_t stride = 1;
    for (int i = ndim - 1; i >= 0; i--) {
        t->strides[i] = stride;
        stride *= shape[i];
    }
    const size_t bytes = (size_t)t->numel * info->size;
    t->data = platform_alloc_aligned(bytes, 64);
    if (!t->data) { free(t); return NULL; }
    memset(t->data, 0, bytes);
    return t;
}

void tensor_destroy(tensor_t* t) {
    if (!t) return;
    platform_free_aligned(t->data);
    if (t->data_device) gpu_device_free(t->data_device);
    free(t);
}

/* Same contract as the reference (tensor.c:50-68): allocate and upload on first use;
 * a tensor that is already resident is left as is.  Callers whose host data changed
 * use tensor_upload. */
int tensor_copy_to_device(tensor_t* t) {
    if (!t || !t->data) return -1;
    if (t->data_device) return 0;
    const size_t bytes = tensor_bytes(t);
    t->data_device = gpu_device_alloc(bytes);
    if (!t->data_device) return -1;
    return gpu_memcpy_h2d(t->data_device, t->data, bytes, NULL) == 0 ? 0 : -1;
}

/* Always copies host -> device (allocating if needed). */
int tensor_upload(tensor_t* t) {
    if (!t || !t->data) return -1;
    const size_t bytes = tensor_bytes(t);
    if (!t->data_device) {
        t->data_device = gpu_device_alloc(bytes);
        if (!t->data_device) return -1;
    }
    return gpu_memcpy_h2d(t->data_device, t->data, bytes, NULL) == 0 ? 0 : -1;
}

int tensor_copy_to_host(tensor_t* t) {
    if (!t) return -1;
    if (!t->data_device) return 0;
    return gpu_memcpy_d2h(t->data, t->data_device, tensor_bytes(t), NULL) == 0 ? 0 : -1;
}

static float half_to_float(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu, m = (uint32_t)h & 0x3FFu, u;
    if (e == 0) {
        if (m == 0) u = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            u = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

static float element(const tensor_t* t, int64_t i) {
    switch (t->dtype) {
        case DATA_TYPE_F32: return ((const float*)t->data)[i];
        case DATA_TYPE_F16: return half_to_float(((const uint16_t*)t->data)[i]);
        case DATA_TYPE_I32: return (float)((const int32_t*)t->data)[i];
        default: return 0.0f;
    }
}

bool tensor_allclose(const tensor_t* a, const tensor_t* b, float rtol, float atol) {
    if (!a || !b || a->numel != b->numel || a->dtype != b->dtype) return false;
    for (int64_t i = 0; i < a->numel; i++) {
        const float x = element(a, i), y = element(b, i);
        const float diff = fabsf(x - y);
        if (diff > atol && diff > rtol * fmaxf(fabsf(x), fabsf(y))) return false;
    }
    return true;
}
