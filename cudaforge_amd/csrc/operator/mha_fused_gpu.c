/*
 * mha_fused_gpu.c — host side of the HIP MHA_Fused operators.
 *
 * Contract of the reference fused op (src/operator/nn/mha_fused.c:7-31 for semantics,
 * mha_fused_cuda.cu:938-1197 and mha_fused_f16_cuda.cu:209-252 for the GPU entries),
 * executed as three launches on the caller's stream:
 *   1. QKV GEMM: X·[WQ | WK | WV] + b, scattered head-major (V transposed);
 *   2. attention with an online softmax (causal if params->causal);
 *   3. output GEMM: merged·WO + bO (+ R when has_residual and R != NULL).
 * Differences from the reference GPU op, by design: the FP32 entry computes in fp32 (the
 * reference silently ran FP16 WMMA unless MHA_FORCE_FP32 was set, mha_fused_cuda.cu:982);
 * causal and num_kv_heads are honoured at every S (the reference's S > 512 split path is
 * wrong, mha_fused_cuda.cu:720,852,905-929); no per-call allocation.
 */
#include "mha_ops.h"
#include "gpu_ops.h"
#include "op_common.h"
#include "../kernels/kernels.h"
#include "op_timing.h"

#include <string.h>

/* The three launches of one call, planned: QKV GEMM, attention, output GEMM. */
typedef struct {
    cf_gemm_args_t  qkv;
    cf_flash_args_t attn;
    cf_gemm_args_t  wo;
} fused_plan_t;

/* 1 (default): where both kernels take it, the QKV product is written row-concatenated,
 * (B*S, (H + 2 H_kv) d) with Q | K | V side by side, and attention reads that matrix;
 * 0: always the head-major scatter (q, k, v^T). */
static int g_rowcat = 1;
void mha_fused_set_rowcat(int on) { g_rowcat = on != 0; }

/* The shape of a call, checked as the plan needs it. */
typedef struct { int64_t B, S, D, H, d, H_kv, kvd; } fused_shape_t;

static int fused_shape(const operator_params_t* params, fused_shape_t* sh) {
    if (!params) return -1;
    const mha_fused_params_t* p = (const mha_fused_params_t*)params;
    const int64_t B = p->batch_size, S = p->seq_len, D = p->hidden_size;
    const int64_t H = p->num_heads, d = p->head_dim;
    const int64_t H_kv = p->num_kv_heads > 0 ? p->num_kv_heads : H;
    if (B <= 0 || S <= 0 || D <= 0 || H <= 0 || d <= 0 || H % H_kv != 0 || H * d != D) return -1;
    if (B > 65535 || H > 65535 || B * S > (1LL << 31) - 1 || D > (1 << 20)) return -1;
    *sh = (fused_shape_t){B, S, D, H, d, H_kv, H_kv * d};
    return 0;
}

/* Workspace areas of the intermediates (q, k, v, attention output), carved from *cur on. */
static void fused_carve(const fused_shape_t* sh, size_t esz, size_t* cur, size_t off[4]) {
    off[0] = cf_ws_take(cur, (size_t)(sh->B * sh->S * sh->D) * esz);
    off[1] = cf_ws_take(cur, (size_t)(sh->B * sh->S * sh->kvd) * esz);
    off[2] = cf_ws_take(cur, (size_t)(sh->B * sh->S * sh->kvd) * esz);
    off[3] = cf_ws_take(cur, (size_t)(sh->B * sh->S * sh->D) * esz);
}

static void fused_fill(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                       const fused_shape_t* sh, char* data, const size_t off[4], fused_plan_t* pl);

static int fused_plan(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                      void* st, fused_plan_t* pl) {
    if (!inputs || !inputs[0] || !outputs || !outputs[0] || !params) return -1;
    if (!inputs[2] || !inputs[4] || !inputs[6] || !inputs[8]) return -1;
    fused_shape_t sh;
    if (fused_shape(params, &sh) != 0) return -1;
    size_t cur = 0, off[4];
    fused_carve(&sh, elem == CF_ELEM_F16 ? 2 : 4, &cur, off);
    char* data = (char*)gpu_workspace_get_stream(st, cur);
    if (!data) return -1;
    fused_fill(elem, inputs, outputs, params, &sh, data, off, pl);
    return 0;
}

static void fused_fill(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                       const fused_shape_t* sh, char* data, const size_t off[4], fused_plan_t* pl) {
    const mha_fused_params_t* p = (const mha_fused_params_t*)params;
    const int64_t B = sh->B, S = sh->S, D = sh->D, H = sh->H, d = sh->d, H_kv = sh->H_kv, kvd = sh->kvd;
    const size_t off_q = off[0], off_k = off[1], off_v = off[2], off_o = off[3];

    memset(pl, 0, sizeof(*pl));
    cf_gemm_args_t* g = &pl->qkv;
    g->a = inputs[0];
    g->M = (int32_t)(B * S);
    g->K = (int32_t)D;
    g->nseg = 3;
    g->w[0] = inputs[2]; g->bias[0] = inputs[3]; g->n[0] = (int32_t)D;
    g->w[1] = inputs[4]; g->bias[1] = inputs[5]; g->n[1] = (int32_t)kvd;
    g->w[2] = inputs[6]; g->bias[2] = inputs[7]; g->n[2] = (int32_t)kvd;
    g->out_kind = CF_GEMM_OUT_QKV;
    g->out[0] = data + off_q;
    g->out[1] = data + off_k;
    g->out[2] = data + off_v;
    g->B = (int32_t)B; g->S = (int32_t)S; g->H_q = (int32_t)H; g->H_kv = (int32_t)H_kv; g->d = (int32_t)d;
    g->elem = elem;

    cf_flash_args_t* f = &pl->attn;
    f->q = data + off_q;
    f->k = data + off_k;
    f->vt = data + off_v;
    f->o = data + off_o;
    f->B = (int32_t)B; f->S = (int32_t)S; f->H_q = (int32_t)H; f->H_kv = (int32_t)H_kv; f->d = (int32_t)d;
    f->scale = p->scale;
    f->causal = p->causal ? 1 : 0;
    f->elem = elem;

    /* The row-concatenated layout: one (B*S, (H + 2 H_kv) d) matrix from the start of the
     * q area; the q, k and v areas follow one another (each start rounded up to 256 bytes),
     * so together they hold its B*S*(D + 2 kvd) elements. */
    if (g_rowcat && elem == CF_ELEM_F16) {
        cf_gemm_args_t rc = *g;
        rc.out_kind = CF_GEMM_OUT_ROWCAT;
        rc.out[0] = data + off_q;
        rc.out[1] = rc.out[2] = NULL;
        cf_flash_args_t fr = *f;
        fr.q = data + off_q;
        fr.k = fr.vt = NULL;
        fr.qkv_ld = (int32_t)(D + 2 * kvd);
        if (cf_gemm_rowcat_ok(&rc) && cf_flash_rowcat_ok(&fr)) {
            *g = rc;
            *f = fr;
        }
    }

    cf_gemm_args_t* o = &pl->wo;
    o->a = data + off_o;
    o->M = (int32_t)(B * S);
    o->K = (int32_t)D;
    o->nseg = 1;
    o->w[0] = inputs[8]; o->bias[0] = inputs[9]; o->n[0] = (int32_t)D;
    o->out_kind = CF_GEMM_OUT_ROWMAJOR;
    o->out[0] = outputs[0];
    o->residual = (p->has_residual && inputs[1]) ? inputs[1] : NULL;
    o->elem = elem;
}

static int fused_launch(const fused_plan_t* pl, int which, void* st) {
    switch (which) {
        case 0: return cf_launch_gemm(&pl->qkv, st);
        case 1: return cf_launch_flash_attn(&pl->attn, st);
        default: return cf_launch_gemm(&pl->wo, st);
    }
}

static int fused_op(int elem, const void* inputs[], void* outputs[],
                    const operator_params_t* params, stream_t* stream) {
    void* st = cf_stream_of(stream);
    fused_plan_t pl;
    int rc = fused_plan(elem, inputs, outputs, params, st, &pl);
    for (int k = 0; k < 3 && rc == 0; k++) rc = fused_launch(&pl, k, st);
    return rc;
}

int mha_fused_kernel_times(const void* inputs[], void* outputs[], const operator_params_t* params,
                           stream_t* stream, int elem_f16, int warmup, int iters, float ms[3]) {
    if (!ms || iters <= 0 || iters > 4096 || warmup < 0) return -1;
    void* st = cf_stream_of(stream);
    fused_plan_t pl;
    int rc = fused_plan(elem_f16 ? CF_ELEM_F16 : CF_ELEM_F32, inputs, outputs, params, st, &pl);
    for (int i = 0; i < warmup && rc == 0; i++)
        for (int k = 0; k < 3 && rc == 0; k++) rc = fused_launch(&pl, k, st);
    gpu_event_t ev[4] = {NULL, NULL, NULL, NULL};
    for (int i = 0; i < 4 && rc == 0; i++) rc = gpu_event_create(&ev[i]);
    if (rc == 0) rc = gpu_stream_synchronize(st);
    /* Each kernel `iters` times back to back between two events (its inputs are those
     * the previous kernel left, as in a call). */
    if (rc == 0) rc = gpu_event_record(ev[0], st);
    for (int k = 0; k < 3 && rc == 0; k++) {
        for (int i = 0; i < iters && rc == 0; i++) rc = fused_launch(&pl, k, st);
        if (rc == 0) rc = gpu_event_record(ev[k + 1], st);
    }
    if (rc == 0) rc = gpu_event_synchronize(ev[3]);
    for (int k = 0; k < 3 && rc == 0; k++) {
        float t = 0.0f;
        rc = gpu_event_elapsed_ms(&t, ev[k], ev[k + 1]);
        ms[k] = t / (float)iters;
    }
    for (int i = 0; i < 4; i++) if (ev[i]) gpu_event_destroy(ev[i]);
    return rc;
}

int mha_fused_f32_cuda(const void* inputs[], void* outputs[],
                       const operator_params_t* params, stream_t* stream) {
    return fused_op(CF_ELEM_F32, inputs, outputs, params, stream);
}

int mha_fused_f16io_cuda(const void* inputs[], void* outputs[],
                         const operator_params_t* params, stream_t* stream) {
    return fused_op(CF_ELEM_F16, inputs, outputs, params, stream);
}

/* The reference's contract for mha_fused_f16_cuda (mha_fused_f16_cuda.cu:209-244): FP32
 * buffers in and out, FP16 arithmetic inside.  X, R, the weights and biases are rounded
 * to fp16 (nearest even) into the stream's workspace, the fp16 path runs on them, and Y
 * is widened back to fp32.  Any S (the reference's kernel held a sequence in shared
 * memory, S <= 64). */
int mha_fused_f16_cuda(const void* inputs[], void* outputs[],
                       const operator_params_t* params, stream_t* stream) {
    if (!inputs || !inputs[0] || !outputs || !outputs[0] || !params) return -1;
    if (!inputs[2] || !inputs[4] || !inputs[6] || !inputs[8]) return -1;
    fused_shape_t sh;
    if (fused_shape(params, &sh) != 0) return -1;
    const mha_fused_params_t* p = (const mha_fused_params_t*)params;
    const int64_t BSD = sh.B * sh.S * sh.D, D = sh.D, kvd = sh.kvd;
    /* Elements of inputs 0..9 (X, R, WQ, bQ, WK, bK, WV, bV, WO, bO); R only when it is used. */
    const int64_t n_in[10] = {BSD, (p->has_residual && inputs[1]) ? BSD : 0, D * D, D, D * kvd, kvd,
                              D * kvd, kvd, D * D, D};
    size_t cur = 0, off_in[10], off_y, off[4];
    for (int i = 0; i < 10; i++) off_in[i] = cf_ws_take(&cur, (size_t)n_in[i] * 2);
    off_y = cf_ws_take(&cur, (size_t)BSD * 2);
    fused_carve(&sh, 2, &cur, off);
    void* st = cf_stream_of(stream);
    char* data = (char*)gpu_workspace_get_stream(st, cur);
    if (!data) return -1;
    const void* in16[10];
    for (int i = 0; i < 10; i++) {
        in16[i] = NULL;
        if (!inputs[i] || n_in[i] == 0) continue;
        if (cf_launch_cast(inputs[i], data + off_in[i], n_in[i], CF_CAST_F32_F16, st) != 0) return -1;
        in16[i] = data + off_in[i];
    }
    void* out16[1] = {data + off_y};
    fused_plan_t pl;
    fused_fill(CF_ELEM_F16, in16, out16, params, &sh, data, off, &pl);
    for (int k = 0; k < 3; k++)
        if (fused_launch(&pl, k, st) != 0) return -1;
    return cf_launch_cast(data + off_y, outputs[0], BSD, CF_CAST_F16_F32, st);
}

int causal_mask_f32_cuda(const void* inputs[], void* outputs[],
                         const operator_params_t* params, stream_t* stream) {
    (void)inputs;
    if (!outputs || !outputs[0] || !params) return -1;
    const causal_mask_params_t* p = (const causal_mask_params_t*)params;
    if (p->seq_len <= 0) return -1;
    return cf_launch_causal_mask((float*)outputs[0], p->seq_len, cf_stream_of(stream));
}

/* Registrations (mha_fused_cuda.cu:1191-1197, mha_fused_f16_cuda.cu:246-252,
 * causal_mask_cuda.cu).  mha_fused_f16_cuda declares "f32" I/O as the reference does;
 * the fp16-I/O op, which graphs of F16 tensors dispatch to, is mha_fused_f16io_cuda. */
int register_mha_fused_f32_cuda(void) {
    static const operator_registry_t reg = {"mha_fused_f32_cuda", "f32", mha_fused_f32_cuda, 6, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_mha_fused_f16_cuda(void) {
    static const operator_registry_t reg = {"mha_fused_f16_cuda", "f32", mha_fused_f16_cuda, 2, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_mha_fused_f16io_cuda(void) {
    static const operator_registry_t reg = {"mha_fused_f16io_cuda", "f16", mha_fused_f16io_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_causal_mask_f32_cuda(void) {
    static const operator_registry_t reg = {"causal_mask_f32_cuda", "f32", causal_mask_f32_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}
