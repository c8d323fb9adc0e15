/*
 * mha_decode_gpu.c — host side of the HIP MHA_Decode operators.
 *
 * Same contract as the reference decode op (src/operator/nn/mha_decode.c:11-125 for the
 * semantics, mha_decode_cuda.cu:159-198 for the GPU entry and registration), built as
 * three launches on the caller's stream:
 *   1. projection GEMV: X_new·[WQ | WK | WV] + b; Q goes to the workspace, K_new/V_new
 *      straight into row cache_len (or seq_lens[b]) of the output caches; the RoPE
 *      variant (mha_decode_rope_*) rotates Q and that K row as the projection's
 *      K-chunk sum stores them (or, with a single K chunk, in place afterwards);
 *   2. split-KV attention over positions 0..cache_len with the LSE merge;
 *   3. output GEMV: O·WO + bO -> Y.
 * Temporaries live in the persistent device workspace (no per-call allocation).
 */
#include "mha_ops.h"
#include "rope_ops.h"
#include "gpu_ops.h"
#include "op_common.h"
#include "../kernels/kernels.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "op_timing.h"

static int64_t g_chunk_override = 0;

void mha_decode_set_split_chunk(int64_t chunk) { g_chunk_override = chunk > 0 ? chunk : 0; }

typedef struct {
    int64_t B, D, H, H_kv, d, max_seq, cache_len;
    int ragged;        /* lengths come from the device array in slot 11 */
    int lens_uniform;  /* ... and the caller guarantees they are all equal (cache_len -2, -3) */
    int advance;       /* ... and the op adds one to each after the step (cache_len -3) */
} decode_shape_t;

/* Validation shared by the op and the core entry (mha_decode.c:14-24, plus the GPU
 * limits the launch grids need). */
static int decode_shape(const mha_decode_params_t* p, decode_shape_t* s) {
    if (!p) return -1;
    s->B = p->batch_size;
    s->D = p->hidden_size;
    s->H = p->num_heads;
    s->d = p->head_dim;
    s->H_kv = p->num_kv_heads > 0 ? p->num_kv_heads : p->num_heads;
    s->max_seq = p->max_seq;
    s->cache_len = p->cache_len;
    s->ragged = p->cache_len < 0;
    s->advance = p->cache_len == MHA_DECODE_CACHE_LEN_DEVICE_ADVANCE;
    s->lens_uniform = p->cache_len == MHA_DECODE_CACHE_LEN_DEVICE_UNIFORM || s->advance;
    if (s->B <= 0 || s->H <= 0 || s->d <= 0 || s->H_kv <= 0 || s->max_seq <= 0) return -1;
    if (s->H % s->H_kv != 0) return -1;
    if (!s->ragged && s->cache_len >= s->max_seq) return -1;
    if (s->B > 65535 || s->H > 65535 || s->d > 1024 || s->max_seq > (1 << 30)) return -1;
    return 0;
}

static void plan_split(int elem, const decode_shape_t* s, int64_t t_max, int64_t* chunk, int64_t* n_split) {
    const int G = (int)(s->H / s->H_kv);
    int64_t q = cf_decode_attn_chunk_quantum(elem, (int)s->d, G);
    const int fast = q > 0;
    if (!fast) q = 64;
    int64_t cmax = cf_decode_attn_chunk_max(elem, (int)s->d, G);
    cmax = cmax / q * q;
    int64_t c;
    if (g_chunk_override > 0) {
        c = cf_ceil_div(g_chunk_override, q) * q;
    } else {
        /* Enough workgroups to keep every CU's memory pipeline full.  The grouped fp16
         * kernel is one workgroup per (split, b) covering every KV head, the other fp16
         * kernel one wave per (split, b, KV head), each as many per CU as its LDS rings
         * allow; the others are 2-4 waves with registers as their only buffer. */
        const int spread = s->ragged && !s->lens_uniform;   /* lengths may differ */
        const int32_t wide_cu = spread ? 0 : cf_decode_attn_wide_wgs_per_cu(elem, (int)s->d, G, (int)s->H_kv);
        const int64_t units = wide_cu > 0 ? s->B : s->B * (fast ? s->H_kv : s->H);
        const int32_t ring_cu = wide_cu > 0 ? wide_cu : cf_decode_attn_wgs_per_cu(elem, (int)s->d, G);
        const int64_t per_cu = ring_cu > 0 ? ring_cu : 4;
        int64_t target = per_cu * (int64_t)cf_cu_count();
        /* Ragged: the grid spans max_seq, but a sequence only runs the splits its length
         * reaches, so plan four times as many (shorter) splits; the busy ones then fill
         * the CUs and rebalance as short sequences finish.  Measured on config 4 shapes:
         * 1-17 % faster than one split per CU slot. */
        if (spread) target *= 4;
        int64_t n = cf_ceil_div(target, units);
        const int64_t nmax = cf_ceil_div(t_max, q);
        if (n > nmax) n = nmax;
        if (n < 1) n = 1;
        c = cf_ceil_div(cf_ceil_div(t_max, n), q) * q;
    }
    if (c > cmax) c = cmax;
    if (c < q) c = q;
    /* At most 1024 splits: bounds the partials workspace and the merge's serial loop. */
    if (cf_ceil_div(t_max, c) > 1024) c = cf_ceil_div(cf_ceil_div(t_max, 1024), q) * q;
    *chunk = c;
    *n_split = cf_ceil_div(t_max, c);
}

int mha_decode_plan(const mha_decode_params_t* p, int elem_f16, int64_t* chunk, int64_t* n_split) {
    decode_shape_t s;
    if (!chunk || !n_split || decode_shape(p, &s) != 0) return -1;
    const int64_t t_max = s.ragged ? s.max_seq : s.cache_len + 1;
    plan_split(elem_f16 ? CF_ELEM_F16 : CF_ELEM_F32, &s, t_max, chunk, n_split);
    return 0;
}

/* Fill the attention-core launch arguments; returns the workspace bytes it needs.
 * `fast_ok`: the q/k/v/o pointers are 16-byte aligned and scale > 0, which the grouped
 * fp16 kernel needs.  Ragged lengths on that kernel split the batch's attended positions
 * evenly over one round of workgroups (balanced mode) instead of planning chunks over
 * max_seq, where short sequences leave most of their splits empty. */
static size_t attn_args(int elem, const decode_shape_t* s, const int32_t* lens, int fast_ok,
                        cf_decode_attn_args_t* a) {
    memset(a, 0, sizeof(*a));
    const int64_t t_max = s->ragged ? s->max_seq : s->cache_len + 1;
    int64_t chunk, n_split;
    plan_split(elem, s, t_max, &chunk, &n_split);
    const int G = (int)(s->H / s->H_kv);
    if (s->ragged && !s->lens_uniform && fast_ok &&
        cf_decode_attn_balanced_ok(elem, (int)s->d, G, (int)s->H_kv, (int)s->B)) {
        a->balanced = 1;
        n_split = (int64_t)cf_cu_count() * cf_decode_attn_wide_wgs_per_cu(elem, (int)s->d, G, (int)s->H_kv);
        chunk = cf_decode_attn_chunk_quantum(elem, (int)s->d, G);   /* unused by the balanced kernel */
    }
    a->seq_lens = lens;
    a->lens_uniform = s->lens_uniform;
    a->B = (int32_t)s->B;
    a->H_q = (int32_t)s->H;
    a->H_kv = (int32_t)s->H_kv;
    a->d = (int32_t)s->d;
    a->max_seq = (int32_t)s->max_seq;
    a->cache_len = s->ragged ? 0 : (int32_t)s->cache_len;
    a->chunk = (int32_t)chunk;
    a->n_split = (int32_t)n_split;
    a->elem = elem;
    if (a->balanced)   /* records per (workgroup, kv head); at most n_split (n_split + B kept as headroom) */
        return (size_t)(a->n_split + a->B) * (size_t)a->H_q * (size_t)(a->d + 4) * sizeof(float);
    return cf_decode_attn_partials_floats(a->B, a->H_q, a->H_kv, a->d, a->n_split, elem) * sizeof(float);
}

static int aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

/* Fill the core's launch arguments.  Partials come from the stream's workspace, or,
 * when `fixed` is non-NULL, from that buffer of `fixed_bytes` bytes (no allocation);
 * a plan whose partials exceed it is rejected with -1. */
static int attn_prepare(int elem, const void* inputs[], void* outputs[],
                        const operator_params_t* params, void* stream, cf_decode_attn_args_t* a,
                        float* fixed, size_t fixed_bytes) {
    if (!params || !inputs || !outputs) return -1;
    const mha_decode_params_t* p = (const mha_decode_params_t*)params;
    decode_shape_t s;
    if (decode_shape(p, &s) != 0 || s.advance) return -1;
    for (int i = 0; i < 3; i++) if (!inputs[i]) return -1;
    if (!outputs[0]) return -1;
    const int32_t* lens = NULL;
    if (s.ragged) {
        lens = (const int32_t*)inputs[3];
        if (!lens) return -1;
    }
    const int fast_ok = aligned16(inputs[0]) && aligned16(inputs[1]) && aligned16(inputs[2]) &&
                        aligned16(outputs[0]) && p->scale > 0.0f;
    const size_t part_bytes = attn_args(elem, &s, lens, fast_ok, a);
    if (fixed) {
        if (part_bytes > fixed_bytes) {
            fprintf(stderr,
                    "mha_decode_attn_f16_noalloc: split partials need %zu bytes, more than the %zu-byte fixed "
                    "scratch (B=%lld H_q=%lld d=%lld n_split=%d); use mha_decode_attn_f16_cuda\n",
                    part_bytes, fixed_bytes, (long long)s.B, (long long)s.H, (long long)s.d, a->n_split);
            return -1;
        }
        a->partials = fixed;
    } else {
        char* ws = (char*)gpu_workspace_get_stream(stream, part_bytes);
        if (!ws) return -1;
        a->partials = (float*)ws;
    }
    a->q = inputs[0];
    a->k = inputs[1];
    a->v = inputs[2];
    a->o = outputs[0];
    a->scale = p->scale;
    return 0;
}

int mha_decode_attn_kernel_times(const void* const* input_sets, int n_inputs, int n_sets,
                                 void* outputs[], const operator_params_t* params,
                                 stream_t* stream, int elem_f16, int warmup, int iters,
                                 float* ms_split, float* ms_merge) {
    if (!input_sets || !ms_split || !ms_merge || iters <= 0 || iters > 4096 || warmup < 0 ||
        n_inputs < 3 || n_sets < 1 || n_sets > 16)
        return -1;
    const int elem = elem_f16 ? CF_ELEM_F16 : CF_ELEM_F32;
    cf_decode_attn_args_t a[16];
    for (int s = 0; s < n_sets; s++) {
        const int rc = attn_prepare(elem, (const void**)&input_sets[s * n_inputs], outputs, params,
                                    cf_stream_of(stream), &a[s], NULL, 0);
        if (rc != 0) return rc;
    }
    void* st = cf_stream_of(stream);
    int rc = 0;
    for (int i = 0; i < warmup; i++)
        if ((rc = cf_launch_decode_attn(&a[i % n_sets], st)) != 0) return rc;
    /* `iters` split launches back to back between two events, then `iters` merge
     * launches: per-launch events would add the dispatch latency of every launch. */
    gpu_event_t ev[3] = {NULL, NULL, NULL};
    for (int i = 0; i < 3 && rc == 0; i++) rc = gpu_event_create(&ev[i]);
    if (rc == 0) rc = gpu_stream_synchronize(st);
    if (rc == 0) rc = gpu_event_record(ev[0], st);
    for (int i = 0; i < iters && rc == 0; i++) rc = cf_launch_decode_attn_split(&a[i % n_sets], st);
    if (rc == 0) rc = gpu_event_record(ev[1], st);
    for (int i = 0; i < iters && rc == 0; i++) rc = cf_launch_decode_attn_merge(&a[i % n_sets], st);
    if (rc == 0) rc = gpu_event_record(ev[2], st);
    if (rc == 0) rc = gpu_event_synchronize(ev[2]);
    float t1 = 0.0f, t2 = 0.0f;
    if (rc == 0) rc = gpu_event_elapsed_ms(&t1, ev[0], ev[1]);
    if (rc == 0) rc = gpu_event_elapsed_ms(&t2, ev[1], ev[2]);
    for (int i = 0; i < 3; i++) if (ev[i]) gpu_event_destroy(ev[i]);
    *ms_split = t1 / (float)iters;
    *ms_merge = t2 / (float)iters;
    return rc;
}

static int attn_core(int elem, const void* inputs[], void* outputs[],
                     const operator_params_t* params, stream_t* stream) {
    cf_decode_attn_args_t a;
    const int rc = attn_prepare(elem, inputs, outputs, params, cf_stream_of(stream), &a, NULL, 0);
    if (rc != 0) return rc;
    return cf_launch_decode_attn(&a, cf_stream_of(stream));
}

/* mha_decode_attn_f16_cuda with its split partials in the library's fixed per-GPU
 * scratch instead of the stream workspace: no allocation of any kind.  Same plan, same
 * kernels, so the same bits.  Calls that overlap on one GPU share the scratch and race. */
int mha_decode_attn_f16_noalloc(const void* inputs[], void* outputs[],
                                const operator_params_t* params, stream_t* stream) {
    float* fixed = cf_decode_attn_scratch();
    if (!fixed) return -1;
    cf_decode_attn_args_t a;
    const int rc = attn_prepare(CF_ELEM_F16, inputs, outputs, params, cf_stream_of(stream), &a, fixed,
                                cf_decode_attn_scratch_bytes());
    if (rc != 0) return rc;
    return cf_launch_decode_attn(&a, cf_stream_of(stream));
}

int mha_decode_attn_f32_cuda(const void* inputs[], void* outputs[],
                             const operator_params_t* params, stream_t* stream) {
    return attn_core(CF_ELEM_F32, inputs, outputs, params, stream);
}

int mha_decode_attn_f16_cuda(const void* inputs[], void* outputs[],
                             const operator_params_t* params, stream_t* stream) {
    return attn_core(CF_ELEM_F16, inputs, outputs, params, stream);
}

static int gemv_k_split(int elem, int64_t K, int64_t col_tiles, int64_t m_tiles) {
    const int64_t kstep = cf_gemv_k_step(elem);
    const int64_t target = 2 * (int64_t)cf_cu_count();
    int64_t ks = cf_ceil_div(target, col_tiles * m_tiles);
    int64_t kmax = K / (4 * kstep);  /* keep >= 4 k steps (one per wave) per chunk */
    if (ks > kmax) ks = kmax;
    if (ks > 32) ks = 32;            /* the reduce sums up to 32 chunks in one round trip */
    if (ks < 1) ks = 1;
    /* every chunk non-empty */
    while (ks > 1) {
        const int64_t chunk = cf_ceil_div(cf_ceil_div(K, ks), kstep) * kstep;
        if ((ks - 1) * chunk < K) break;
        ks--;
    }
    return (int)ks;
}

/* rope_base > 0: RoPE on Q and K_new between the projection and the attention. */
static int decode_op(int elem, const void* inputs[], void* outputs[],
                     const mha_decode_params_t* p, float rope_base, stream_t* stream) {
    if (!p || !inputs || !outputs) return -1;
    for (int i = 0; i < MHA_DECODE_NUM_INPUTS; i++) if (!inputs[i]) return -1;
    for (int i = 0; i < MHA_DECODE_NUM_OUTPUTS; i++) if (!outputs[i]) return -1;
    decode_shape_t s;
    if (decode_shape(p, &s) != 0) return -1;
    if (s.H * s.d != s.D) return -1;
    const float* rope_table = NULL;
    if (rope_base > 0.0f) {
        if (s.d & 1) return -1;
        if (!(rope_table = rope_table_device(rope_base, s.d, s.max_seq))) return -1;
    }
    const int32_t* lens = NULL;
    if (s.ragged) {
        lens = (const int32_t*)inputs[MHA_DECODE_SLOT_SEQLENS];
        if (!lens) return -1;
    }
    const size_t esz = elem == CF_ELEM_F16 ? 2 : 4;
    const int64_t kvd = s.H_kv * s.d;
    void* st = cf_stream_of(stream);

    /* Non-aliased output caches start as copies of the inputs (mha_decode.c:43-44). */
    const size_t cache_bytes = (size_t)s.B * (size_t)s.max_seq * (size_t)kvd * esz;
    int rc;
    if (outputs[1] != inputs[1] && (rc = gpu_memcpy_d2d(outputs[1], inputs[1], cache_bytes, st)) != 0) return rc;
    if (outputs[2] != inputs[2] && (rc = gpu_memcpy_d2d(outputs[2], inputs[2], cache_bytes, st)) != 0) return rc;

    /* Plan all three launches, then carve one workspace. */
    cf_gemv_args_t g1;
    memset(&g1, 0, sizeof(g1));
    g1.x = inputs[0];
    g1.M = (int32_t)s.B;
    g1.K = (int32_t)s.D;
    g1.nseg = 3;
    g1.seg[0] = (cf_gemv_seg_t){inputs[3], inputs[4], NULL, s.H * s.d, s.H * s.d, 0};
    g1.seg[1] = (cf_gemv_seg_t){inputs[5], inputs[6], outputs[1], kvd, s.max_seq * kvd, kvd};
    g1.seg[2] = (cf_gemv_seg_t){inputs[7], inputs[8], outputs[2], kvd, s.max_seq * kvd, kvd};
    g1.pos_lens = lens;
    g1.pos_uniform = s.ragged ? 0 : s.cache_len;
    g1.pos_limit = s.max_seq;
    g1.elem = elem;
    const int64_t m_tiles = cf_ceil_div(s.B, 16);
    const int64_t tile = cf_gemv_col_tile(elem);
    const int64_t ct1 = cf_ceil_div(s.H * s.d, tile) + 2 * cf_ceil_div(kvd, tile);
    g1.k_split = gemv_k_split(elem, s.D, ct1, m_tiles);
    /* RoPE rides in the projection's K-chunk sum when it has one (Q and K_new are rotated
     * before they are stored); otherwise a kernel of its own rotates them afterwards. */
    const int fuse_rope = rope_table && cf_gemv_fuses_rope(&g1);
    if (fuse_rope) {
        g1.rope_table = rope_table;
        g1.rope_d = (int32_t)s.d;
        g1.rope_segs = 3;              /* Q and K */
        g1.rope_rows = s.max_seq;
    }

    cf_decode_attn_args_t a;
    /* q and o live in the workspace (256-byte aligned). */
    const int fast_ok = aligned16(outputs[1]) && aligned16(outputs[2]) && p->scale > 0.0f;
    const size_t attn_part = attn_args(elem, &s, lens, fast_ok, &a);

    cf_gemv_args_t g2;
    memset(&g2, 0, sizeof(g2));
    g2.M = (int32_t)s.B;
    g2.K = (int32_t)(s.H * s.d);
    g2.nseg = 1;
    g2.seg[0] = (cf_gemv_seg_t){inputs[9], inputs[10], outputs[0], s.D, s.D, 0};
    g2.elem = elem;
    g2.k_split = gemv_k_split(elem, s.H * s.d, cf_ceil_div(s.D, tile), m_tiles);
    if (s.advance) {   /* nothing after the output projection reads the lengths */
        g2.advance = (int32_t*)lens;
        g2.advance_n = (int32_t)s.B;
    }

    size_t cur = 0;
    const size_t off_q = cf_ws_take(&cur, (size_t)s.B * s.H * s.d * esz);
    const size_t off_o = cf_ws_take(&cur, (size_t)s.B * s.H * s.d * esz);
    const size_t off_p1 = cf_ws_take(&cur, cf_gemv_partials_floats(&g1) * sizeof(float));
    const size_t off_pa = cf_ws_take(&cur, attn_part);
    const size_t off_p2 = cf_ws_take(&cur, cf_gemv_partials_floats(&g2) * sizeof(float));
    char* data = (char*)gpu_workspace_get_stream(st, cur);
    if (!data) return -1;

    g1.seg[0].out = data + off_q;
    g1.partials = (float*)(data + off_p1);
    if ((rc = cf_launch_gemv(&g1, st)) != 0) return rc;

    if (rope_table && !fuse_rope) {
        cf_rope_decode_args_t r;
        memset(&r, 0, sizeof(r));
        r.q = data + off_q;
        r.k_cache = outputs[1];
        r.table = rope_table;
        r.lens = lens;
        r.pos_uniform = s.ragged ? 0 : s.cache_len;
        r.max_seq = s.max_seq;
        r.B = (int32_t)s.B;
        r.H_q = (int32_t)s.H;
        r.H_kv = (int32_t)s.H_kv;
        r.d = (int32_t)s.d;
        r.elem = elem;
        if ((rc = cf_launch_rope_decode(&r, st)) != 0) return rc;
    }

    a.q = data + off_q;
    a.k = outputs[1];
    a.v = outputs[2];
    a.o = data + off_o;
    a.scale = p->scale;
    a.partials = (float*)(data + off_pa);
    if ((rc = cf_launch_decode_attn(&a, st)) != 0) return rc;

    g2.x = data + off_o;
    g2.partials = (float*)(data + off_p2);
    return cf_launch_gemv(&g2, st);
}

int mha_decode_f32_cuda(const void* inputs[], void* outputs[],
                        const operator_params_t* params, stream_t* stream) {
    return decode_op(CF_ELEM_F32, inputs, outputs, (const mha_decode_params_t*)params, 0.0f, stream);
}

int mha_decode_f16_cuda(const void* inputs[], void* outputs[],
                        const operator_params_t* params, stream_t* stream) {
    return decode_op(CF_ELEM_F16, inputs, outputs, (const mha_decode_params_t*)params, 0.0f, stream);
}

static int decode_rope(int elem, const void* inputs[], void* outputs[], const operator_params_t* params,
                       stream_t* stream) {
    const mha_decode_rope_params_t* rp = (const mha_decode_rope_params_t*)params;
    if (!rp || !(rp->rope_base > 0.0f)) return -1;
    return decode_op(elem, inputs, outputs, &rp->decode, rp->rope_base, stream);
}

int mha_decode_rope_f32_cuda(const void* inputs[], void* outputs[],
                             const operator_params_t* params, stream_t* stream) {
    return decode_rope(CF_ELEM_F32, inputs, outputs, params, stream);
}

int mha_decode_rope_f16_cuda(const void* inputs[], void* outputs[],
                             const operator_params_t* params, stream_t* stream) {
    return decode_rope(CF_ELEM_F16, inputs, outputs, params, stream);
}

int register_mha_decode_rope_f32_cuda(void) {
    static const operator_registry_t reg = {"mha_decode_rope_f32_cuda", "f32", mha_decode_rope_f32_cuda, 1,
                                            OP_FLAG_ALLOW_ALIAS};
    return operator_register(&reg);
}

int register_mha_decode_rope_f16_cuda(void) {
    static const operator_registry_t reg = {"mha_decode_rope_f16_cuda", "f16", mha_decode_rope_f16_cuda, 1,
                                            OP_FLAG_ALLOW_ALIAS};
    return operator_register(&reg);
}

/* Registrations (mha_decode_cuda.cu:192-198).  The attention-core entries are new. */
int register_mha_decode_f32_cuda(void) {
    static const operator_registry_t reg = {"mha_decode_f32_cuda", "f32", mha_decode_f32_cuda, 2, OP_FLAG_ALLOW_ALIAS};
    return operator_register(&reg);
}

int register_mha_decode_f16_cuda(void) {
    static const operator_registry_t reg = {"mha_decode_f16_cuda", "f16", mha_decode_f16_cuda, 1, OP_FLAG_ALLOW_ALIAS};
    return operator_register(&reg);
}

int register_mha_decode_attn_f32_cuda(void) {
    static const operator_registry_t reg = {"mha_decode_attn_f32_cuda", "f32", mha_decode_attn_f32_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}

int register_mha_decode_attn_f16_cuda(void) {
    static const operator_registry_t reg = {"mha_decode_attn_f16_cuda", "f16", mha_decode_attn_f16_cuda, 1, OP_FLAG_NONE};
    return operator_register(&reg);
}
