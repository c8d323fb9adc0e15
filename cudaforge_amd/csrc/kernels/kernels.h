/*
 * kernels.h — C-ABI between the host operator code (C) and the HIP kernels (gfx950).
 *
 * Every launcher validates nothing beyond what the kernel's indexing needs; the
 * operator layer (the csrc/operator C files) checks shapes and arguments first.  Launchers
 * return 0 or a positive hipError_t value.  All pointers are device pointers.
 */
#ifndef CF_KERNELS_H_
#define CF_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { CF_ELEM_F32 = 0, CF_ELEM_F16 = 1 };

/* ---------------------------------------------------------------------------------
 * Split-KV decode attention with a fused log-sum-exp combine.
 *
 * q: (B, H_q, d); k/v caches: (B, max_seq, H_kv, d); o: (B, H_q, d), all in `elem`.
 * Sequence b attends positions 0 .. T_b-1 with T_b = seq_lens ? seq_lens[b] + 1
 * : cache_len + 1.  The split kernel covers n_split splits of `chunk` positions per
 * (b, kv head) (a split past T_b exits at once) and writes partial (max, sum, acc)
 * tuples to `partials`; the merge kernel combines them.  A sequence with one split is
 * written directly by the split kernel.
 * ------------------------------------------------------------------------------- */
typedef struct {
    const void*    q;
    const void*    k;
    const void*    v;
    void*          o;
    const int32_t* seq_lens;   /* device, NULL = uniform cache_len */
    int32_t        lens_uniform; /* seq_lens all hold one value (a device-held uniform length) */
    int32_t        balanced;   /* ragged seq_lens on the grouped fp16 kernel: n_split workgroups
                                  (>= 2B) share the batch's attended positions about equally,
                                  each one range of one sequence (chunk unused); partial
                                  records: at most n_split x H_kv */
    float*         partials;   /* workspace */
    int32_t        B, H_q, H_kv, d;
    int32_t        max_seq, cache_len;
    int32_t        chunk, n_split;
    float          scale;
    int32_t        elem;
} cf_decode_attn_args_t;

/* Positions one workgroup pass covers (chunk must be a multiple); 0 = generic kernel. */
/* n / d (0 <= n < 2^31, d >= 1) by the multiply-and-shift divisor the kernels take at
 * launch, computed on the host (checks of that arithmetic). */
int32_t cf_fastdiv_quotient(int32_t n, int32_t d);
int32_t cf_decode_attn_chunk_quantum(int32_t elem, int32_t d, int32_t group);
int32_t cf_decode_attn_chunk_max(int32_t elem, int32_t d, int32_t group);
/* Workgroups of the fp16 split kernel that fit one CU (its LDS ring bounds it), or 0
 * where that kernel does not apply. */
int32_t cf_decode_attn_wgs_per_cu(int32_t elem, int32_t d, int32_t group);
/* Tuning override of the fp16 split kernel's LDS ring depth (2..4; 0 = default 3). */
void    cf_decode_attn_set_stages(int32_t stages);
/* The grouped fp16 split kernel (one workgroup per (split, b), one wave per KV head,
 * H_kv <= 8): workgroups per CU, or 0 where it does not apply.  The chunk planner sizes
 * the split count by it.  cf_decode_attn_set_wide(0) selects the one-wave-per-(split, KV
 * head) kernel everywhere (tests and measurements; default 1). */
int32_t cf_decode_attn_wide_wgs_per_cu(int32_t elem, int32_t d, int32_t group, int32_t h_kv);
void    cf_decode_attn_set_wide(int32_t on);
/* The grouped kernel at d = 128 loads K straight into registers and keeps only V in its
 * LDS ring (default 1); 0 selects the K-and-V ring (tests and measurements). */
void    cf_decode_attn_set_kreg(int32_t on);
/* 1 when that kernel's build for GQA group `group` (1, 2, 4, 8) holds no register spills,
 * which its load counting needs; else the K-and-V ring kernel runs in its place. */
int32_t cf_decode_attn_kreg_ok(int32_t group);
/* Tests: 1 selects the workgroup-per-row merge for every head size (0 = the one-wave
 * merge for d = 64 / 128). */
void    cf_decode_attn_set_merge_rows(int32_t on);
/* Tuning override: workgroups per row of the row merge, 1, 2 or 4 dividing d / 4
 * (0 = automatic: up to 4, keeping at least 64 dims per workgroup). */
void    cf_decode_attn_set_merge_rows_split(int32_t ds);
/* Tuning override: rows (one wave each) per workgroup of the one-wave merge, 1..4
 * (default 2). */
void    cf_decode_attn_set_merge_wave_wg(int32_t rows);
/* Workspace floats needed for the partials of a launch. */
size_t  cf_decode_attn_partials_floats(int32_t B, int32_t H_q, int32_t H_kv, int32_t d,
                                       int32_t n_split, int32_t elem);
/* 1 when ragged lengths of this shape take the balanced grouped kernel (then n_split
 * workgroups, as many as fit the CUs at once, share the attended positions equally). */
int32_t cf_decode_attn_balanced_ok(int32_t elem, int32_t d, int32_t group, int32_t h_kv, int32_t B);
/* Fixed device scratch for the split partials of the allocation-free decode entry: a
 * file-scope device array of cf_decode_attn_scratch_bytes() bytes, one per GPU.
 * cf_decode_attn_scratch_init looks up the current device's address of it once
 * (0 or a hipError_t value); cf_decode_attn_scratch returns that address, looking it up
 * on first use on a device, or NULL on failure. */
size_t  cf_decode_attn_scratch_bytes(void);
int     cf_decode_attn_scratch_init(void);
float*  cf_decode_attn_scratch(void);
int     cf_launch_decode_attn_split(const cf_decode_attn_args_t* a, void* stream);
int     cf_launch_decode_attn_merge(const cf_decode_attn_args_t* a, void* stream);
int     cf_launch_decode_attn(const cf_decode_attn_args_t* a, void* stream);  /* split + merge */

/* ---------------------------------------------------------------------------------
 * Skinny GEMM for decode projections: Y[m, n] = Σ_k X[m, k] W[k, n] + bias[n] for
 * M <= 16 rows per tile (grid covers ceil(M/16) tiles), W row-major (K, N).
 * Up to three column segments, each with its own W/bias and destination; segment s
 * covers global columns [col0_s, col0_s + n_s) and writes element (m, j) to
 *   out_s + m*ld_m_s + pos(m)*ld_pos_s + j,   pos(m) = pos_lens ? pos_lens[m] : pos_uniform.
 * That places decode's K_new / V_new rows straight into the KV cache.
 * K is split across `k_split` workgroups writing fp32 partials to the workspace; a
 * second kernel sums them, adds the bias and stores (k_split = 1: one kernel).
 * ------------------------------------------------------------------------------- */
#define CF_GEMV_MAX_SEGS 3
typedef struct {
    const void* w;
    const void* bias;   /* may be NULL */
    void*       out;
    int64_t     n;
    int64_t     ld_m;
    int64_t     ld_pos;
} cf_gemv_seg_t;

typedef struct {
    const void*    x;         /* (M, K) row-major */
    int32_t        M, K;
    int32_t        nseg;
    cf_gemv_seg_t  seg[CF_GEMV_MAX_SEGS];
    const int32_t* pos_lens;  /* device, may be NULL */
    int64_t        pos_uniform;
    int64_t        pos_limit; /* rows whose pos is outside [0, pos_limit) are not stored;
                                 0 = no limit */
    int32_t        k_split;   /* 1..32 (larger is taken as 32); K chunk = ceil(K / k_split)
                                 rounded to the k step (the fp16 DMA path and the small
                                 one-pass kernel plan their own) */
    float*         partials;  /* workspace */
    int32_t        elem;
    int32_t*       advance;   /* device, may be NULL: the launch's last kernel adds one to
                                 advance[0 .. advance_n) (nothing in it reads them) */
    int32_t        advance_n;
    /* RoPE on the stored values, in the K-chunk sum or the small one-pass kernel (other
     * single-chunk launches reject it, see cf_gemv_fuses_rope):
     * in segment s with bit s of rope_segs set, columns (2i, 2i+1) of each rope_d-wide
     * head are rotated by table[pos * rope_d/2 + i] (cos, sin) after the bias is added,
     * where pos is the row's position; a position outside [0, rope_rows) is not rotated. */
    const float*   rope_table;
    int32_t        rope_d;
    int32_t        rope_segs;
    int64_t        rope_rows;
} cf_gemv_args_t;

int32_t cf_gemv_col_tile(int32_t elem);
int32_t cf_gemv_k_step(int32_t elem);
size_t  cf_gemv_partials_floats(const cf_gemv_args_t* a);
int     cf_launch_gemv(const cf_gemv_args_t* a, void* stream);
/* Tuning override of the fp16 DMA path's column-tile width (64, 128 or 256; 0 =
 * automatic: 128 where it divides every segment, else 64). */
void    cf_gemv_set_dma_tile(int32_t bn);
/* Tuning override of the fp16 DMA path's K split (1..32; 0 = automatic). */
void    cf_gemv_set_dma_ksplit(int32_t ks);
/* The one-pass kernel for small projections (M <= 4, M * K <= 4096, every segment width
 * a multiple of 16, weights of at most 8 MB): 0 never, 1 automatic (default), 2 wherever
 * the shape allows it whatever the weight size (tests). */
void    cf_gemv_set_small(int32_t mode);
/* 1 when a launch with these arguments can apply RoPE (rope_table): the K-chunk sum or
 * the one-pass small kernel runs it; a single-chunk split-K launch cannot. */
int32_t cf_gemv_fuses_rope(const cf_gemv_args_t* a);

/* ---------------------------------------------------------------------------------
 * Prefill GEMM with fused epilogue: C = A·W + bias (+ residual), A (M, K) row-major,
 * W (K, N) row-major.  Output layouts:
 *   CF_GEMM_OUT_ROWMAJOR: out (M, N) row-major (+ residual (M, N) if non-NULL);
 *   CF_GEMM_OUT_QKV:      columns split into Q | K | V, written head-major as
 *                          q (B, H_q, S, d), k (B, H_kv, S, d), vt (B, H_kv, d, S)
 *                          (V transposed so attention reads keys contiguously);
 *                          M = B*S rows, W given as three segments.
 *   CF_GEMM_OUT_ROWCAT:   the nseg segments side by side in one row-major (M, sum n[s])
 *                          out[0], each with its own bias, no residual; fp16 on the
 *                          wave-specialised kernel only (cf_gemm_rowcat_ok says whether a
 *                          product can take it; cf_launch_gemm rejects it otherwise).
 * ------------------------------------------------------------------------------- */
enum { CF_GEMM_OUT_ROWMAJOR = 0, CF_GEMM_OUT_QKV = 1, CF_GEMM_OUT_ROWCAT = 2 };

typedef struct {
    const void* a;           /* (M, K) */
    int32_t     M, K;
    int32_t     nseg;        /* 1 (row-major) or 3 (QKV) */
    const void* w[3];
    const void* bias[3];
    int32_t     n[3];
    int32_t     out_kind;
    void*       out[3];      /* row-major: out[0]; QKV: q, k, vt */
    const void* residual;    /* row-major only, may be NULL */
    int32_t     B, S, H_q, H_kv, d;  /* QKV layout */
    int32_t     elem;        /* element type of a, w, bias, out, residual */
} cf_gemm_args_t;

int cf_launch_gemm(const cf_gemm_args_t* a, void* stream);
/* Tuning override of the fp16 direct-to-LDS GEMM's ring depth (3 or 4 stages; 0 =
 * automatic: 3, i.e. three workgroups per CU, when there are more than two tiles per CU). */
void cf_gemm_set_stages(int32_t stages);
/* Tuning override of the tile order's group height (M tiles per group; 0 = default). */
void cf_gemm_set_group_m(int32_t group_m);
/* Tuning/test override of the fp16 direct-to-LDS GEMM's tile width (96 or 128 columns;
 * 0 = automatic: the width that balances the tiles over the CUs). */
void cf_gemm_set_bn(int32_t bn);
/* Tuning/test override of its stage depth in k (32: 3-4 stages of 16 KB; 64: 2 stages of
 * 32 KB; 0 = automatic). */
void cf_gemm_set_bk(int32_t bk);
/* Tuning/test override of its k split inside a workgroup (1: one group of 4 waves per
 * tile; 2: two groups of 4 waves, each over half of K, where K % 128 == 0; 0 = automatic:
 * two groups when the grid has at most one tile per CU). */
void cf_gemm_set_ksplit(int32_t ks);
/* The fp16 wave-specialised GEMM (256- or 128-row tiles; 4 loader and 4 compute waves):
 * mode 0 = used wherever it applies, 1 = never (the other kernels run). */
void cf_gemm_set_ws(int32_t mode);
/* Tuning/test override of that kernel's tile (BM 256 or 128, BN among its widths; 0, 0 =
 * the cost model's choice).  A product the tile does not fit takes the cost model's. */
void cf_gemm_set_ws_shape(int32_t bm, int32_t bn);
int32_t cf_gemm_rowcat_ok(const cf_gemm_args_t* a);

/* ---------------------------------------------------------------------------------
 * Prefill attention (flash style, online softmax): q (B, H_q, S, d), k (B, H_kv, S, d),
 * vt (B, H_kv, d, S) -> o (B, S, H_q, d) == (B*S, H_q*d) row-major.
 * With qkv_ld > 0 the inputs are instead one row-major (B*S, qkv_ld) matrix at q whose
 * row holds Q (H_q*d) | K (H_kv*d) | V (H_kv*d) side by side, qkv_ld = (H_q + 2 H_kv) d
 * (the CF_GEMM_OUT_ROWCAT product); k and vt are unused.  Only the fp16 d = 64 kernel
 * with S % 8 == 0 reads that layout (cf_flash_rowcat_ok).
 * ------------------------------------------------------------------------------- */
typedef struct {
    const void* q;
    const void* k;
    const void* vt;
    void*       o;
    int32_t     B, S, H_q, H_kv, d;
    float       scale;
    int32_t     causal;
    int32_t     elem;
    int32_t     qkv_ld;
} cf_flash_args_t;

int cf_launch_flash_attn(const cf_flash_args_t* a, void* stream);
int32_t cf_flash_rowcat_ok(const cf_flash_args_t* a);
/* Selects the fp16 d = 64 prefill attention kernel (tuning and tests): 0 the register-
 * staged kernel, 1 / 2 the DMA-ring kernel with 32 / 16 queries per wave, 3 (default)
 * the DMA-ring kernel where it applies (S % 8 == 0) with the width chosen by size. */
void cf_flash_set_mode(int32_t mode);
/* Causal fp16 DMA attention: 1 runs each query block and its mirror in one workgroup;
 * 0 (default) one block per workgroup, heaviest first (tests and measurements). */
void cf_flash_set_causal_pairs(int32_t on);

/* CausalMask (S, S) float on the device. */
int cf_launch_causal_mask(float* mask, int64_t S, void* stream);

/* Copies `bytes` bytes with a kernel (either end may be pinned host memory, which the
 * device reads and writes directly): small stream-ordered transfers between kernels. */
int cf_launch_copy_bytes(void* dst, const void* src, size_t bytes, void* stream);

/* n elements (CF_ELEM_F16 or CF_ELEM_F32) of N(mean, stddev) from splitmix64 seeded with
 * `seed` and Box-Muller (synthetic benchmark inputs; misc.hip). */
int cf_launch_fill_normal(void* out, size_t n, int elem, uint64_t seed, float mean, float stddev, void* stream);

/* v[0..n) = value (add = 0) or += value (add = 1), as a kernel (graph decode lengths). */
int cf_launch_i32_update(int32_t* v, int32_t n, int32_t value, int32_t add, void* stream);

/* ---------------------------------------------------------------------------------
 * Layer-neighbour kernels (layer_ops.hip) for the FP16 path around attention.
 *
 * LayerNorm over the last dimension (layernorm.c:96-120): per row, mean, population
 * variance, y = (x - mean) / sqrt(var + eps) * gamma + beta, fp32 statistics.
 */
typedef struct {
    const void* x;         /* (N, D) */
    const void* gamma;     /* (D) */
    const void* beta;      /* (D) */
    void*       y;         /* (N, D); may equal x */
    int64_t     N;
    int32_t     D;
    float       eps;
    int32_t     elem;      /* all tensors CF_ELEM_F32 or all CF_ELEM_F16 */
} cf_layernorm_args_t;
int cf_launch_layernorm(const cf_layernorm_args_t* a, void* stream);

/* Element conversions of the Cast op (cast_cuda.cu:6-64): kind selects the pair;
 * f32 -> f16 rounds to nearest even, f32 -> i64 truncates toward zero. */
enum { CF_CAST_I64_F32 = 0, CF_CAST_F32_I64 = 1, CF_CAST_F32_F16 = 2, CF_CAST_F16_F32 = 3 };
int cf_launch_cast(const void* in, void* out, int64_t n, int32_t kind, void* stream);

/* out (cols, rows) = in (rows, cols)^T for `batch` slices (strides in elements);
 * elem_bytes 2 or 4. */
int cf_launch_transpose(const void* in, void* out, int64_t rows, int64_t cols, int64_t batch,
                        int64_t in_stride, int64_t out_stride, int32_t elem_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * Rotary position encoding (rope.hip).  Pair (2i, 2i+1) of every head at position pos
 * is rotated by the angle whose (cos, sin) is table[pos * d/2 + i] (float2), computed on
 * the host exactly as rope.c:38-45 does.  fp32 arithmetic without contraction, so the
 * rotation matches the reference's CPU op bit for bit on the same table.
 */
typedef struct {
    const void*  in;        /* (rows, H, d); rows = S */
    void*        out;       /* may equal in */
    const float* table;     /* (n_pos, d/2) x {cos, sin}; n_pos >= rows */
    int64_t      rows;
    int32_t      H, d;
    int32_t      elem;      /* CF_ELEM_F32 / CF_ELEM_F16 */
} cf_rope_args_t;
int cf_launch_rope(const cf_rope_args_t* a, void* stream);

/* Decode form: rotates, in place, Q (B, H_q, d) and the new K row of every sequence,
 * k_cache[b, pos_b, :, :] of a (B, max_seq, H_kv, d) cache, at pos_b = lens[b] (or
 * pos_uniform without lens); rows whose position is outside 0 .. max_seq-1 are skipped. */
typedef struct {
    void*          q;
    void*          k_cache;
    const float*   table;   /* n_pos >= max_seq */
    const int32_t* lens;    /* may be NULL */
    int64_t        pos_uniform;
    int64_t        max_seq;
    int32_t        B, H_q, H_kv, d;
    int32_t        elem;
} cf_rope_decode_args_t;
int cf_launch_rope_decode(const cf_rope_decode_args_t* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CF_KERNELS_H_ */
