/*
 * rope_gpu.c — host side of the HIP RoPE operators (the reference's rope.c:17-66 and
 * rope_cuda.cu:35-59) and the per-device angle tables they share with
 * mha_decode_rope_*_cuda.
 */
#include "rope_ops.h"
#include "gpu_ops.h"
#include "op_common.h"
#include "../kernels/kernels.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ tables --- */

typedef struct {
    int      dev;
    float    base;
    int64_t  d;
    int64_t  n_pos;
    float*   table;     /* device */
} rope_table_t;

#define ROPE_TABLES 16
static rope_table_t g_tables[ROPE_TABLES];

static void rope_tables_release(void) {
    for (int i = 0; i < ROPE_TABLES; i++) {
        if (g_tables[i].table) gpu_device_free(g_tables[i].table);
        memset(&g_tables[i], 0, sizeof(g_tables[i]));
    }
    gpu_buffer_generation_bump();
}

/* (cos, sin) of angle = pos / powf(base, 2i/d), rope.c:38-45. */
static void fill_table(float* host, float base, int64_t d, int64_t n_pos) {
    const int64_t half = d / 2;
    for (int64_t pos = 0; pos < n_pos; pos++)
        for (int64_t i = 0; i < half; i++) {
            const float angle = (float)pos / powf(base, (float)(2 * i) / (float)d);
            host[2 * (pos * half + i)] = cosf(angle);
            host[2 * (pos * half + i) + 1] = sinf(angle);
        }
}

const float* rope_table_device(float base, int64_t d, int64_t n_pos) {
    if (!(base > 0.0f) || d <= 0 || (d & 1) || n_pos <= 0) return NULL;
    const int dev = gpu_current_device();
    rope_table_t* hit = NULL;
    rope_table_t* slot = NULL;
    for (int i = 0; i < ROPE_TABLES; i++) {
        rope_table_t* t = &g_tables[i];
        if (t->table && t->dev == dev && t->d == d && memcmp(&t->base, &base, sizeof(float)) == 0) hit = t;
        if (!t->table && !slot) slot = t;
    }
    if (hit && hit->n_pos >= n_pos) return hit->table;
    /* Grow to at least twice the old range so a decode loop that lengthens its cache
     * rebuilds rarely. */
    int64_t n = n_pos;
    if (hit && n < 2 * hit->n_pos) n = 2 * hit->n_pos;
    if (!hit && !slot) {
        /* All slots taken: reuse the first one (other entries stay valid). */
        slot = &g_tables[0];
    }
    const size_t bytes = (size_t)n * (size_t)(d / 2) * 2 * sizeof(float);
    float* host = (float*)malloc(bytes);
    if (!host) return NULL;
    fill_table(host, base, d, n);
    float* dptr = (float*)gpu_device_alloc(bytes);
    if (!dptr) { free(host); return NULL; }
    if (gpu_memcpy_h2d(dptr, host, bytes, NULL) != 0 || gpu_stream_synchronize(NULL) != 0) {
        free(host);
        gpu_device_free(dptr);
        return NULL;
    }
    free(host);
    rope_table_t* t = hit ? hit : slot;
    if (t->table) {
        /* Work already enqueued may still read the old table, and a recording may
         * point at it. */
        gpu_device_synchronize();
        gpu_device_free(t->table);
        gpu_buffer_generation_bump();
    }
    t->dev = dev;
    t->base = base;
    t->d = d;
    t->n_pos = n;
    t->table = dptr;
    gpu_at_finalize(rope_tables_release);
    return dptr;
}

/* ------------------------------------------------------------------ the op --- */

static int rope_op(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                   stream_t* stream) {
    if (!inputs || !inputs[0] || !outputs || !outputs[0] || !params) return -1;
    const rope_params_t* p = (const rope_params_t*)params;
    if (p->seq_len < 0 || p->num_heads <= 0 || p->head_dim <= 0 || (p->head_dim & 1) || !(p->base > 0.0f)) return -1;
    if (p->num_heads > (1 << 30) || p->head_dim > (1 << 30)) return -1;
    if (p->seq_len == 0) return 0;
    const float* table = rope_table_device(p->base, p->head_dim, p->seq_len);
    if (!table) return -1;
    cf_rope_args_t a;
    memset(&a, 0, sizeof(a));
    a.in = inputs[0];
    a.out = outputs[0];
    a.table = table;
    a.rows = p->seq_len;
    a.H = (int32_t)p->num_heads;
    a.d = (int32_t)p->head_dim;
    a.elem = elem;
    return cf_launch_rope(&a, cf_stream_of(stream));
}

int rope_f32_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    return rope_op(CF_ELEM_F32, inputs, outputs, params, stream);
}

int rope_f16_cuda(const void* inputs[], void* outputs[], const operator_params_t* params, stream_t* stream) {
    return rope_op(CF_ELEM_F16, inputs, outputs, params, stream);
}

/* Registrations (rope_cuda.cu:53-59; in place allowed). */
int register_rope_f32_cuda(void) {
    static const operator_registry_t reg = {"rope_f32_cuda", "f32", rope_f32_cuda, 1, OP_FLAG_IN_PLACE};
    return operator_register(&reg);
}

int register_rope_f16_cuda(void) {
    static const operator_registry_t reg = {"rope_f16_cuda", "f16", rope_f16_cuda, 1, OP_FLAG_IN_PLACE};
    return operator_register(&reg);
}
