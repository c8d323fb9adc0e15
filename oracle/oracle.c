/*
 * oracle.c — CPU restatement of the reference attention fallbacks (test infrastructure
 * only; see oracle.h for who may use it and how each function is pinned).
 */
#define _POSIX_C_SOURCE 199309L
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------------------------
 * MHA_Decode — follows src/operator/nn/mha_decode.c:11-125 statement by statement:
 *   copy caches (:43-44); per batch row: y = bO (:51); per kv head K_new/V_new = x·W + b
 *   written at row cache_len (:54-72); per query head: Q = x·WQ + bQ (:81-86),
 *   s_t = (Q·K_t)·scale with running max (:91-98), e_t = expf(s_t - max), sum (:101-105),
 *   clamp 1e-12 (:106), merged += (e_t / sum)·V_t (:109-114), y_j += Σ merged·WO (:117-121).
 * ---------------------------------------------------------------------------------- */
/* LayerNorm — src/operator/nn/layernorm.c:96-120 (the scalar path): per row, mean of x,
 * population variance of (x - mean), inv_std = 1 / sqrtf(var/D + eps),
 * y = (x - mean) * inv_std * gamma + beta, each sum accumulated in order. */
int oracle_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y,
                         int64_t N, int64_t D, float eps) {
    if (!x || !gamma || !beta || !y || N < 0 || D <= 0) return -1;
    for (int64_t n = 0; n < N; n++) {
        const float* xn = x + n * D;
        float* yn = y + n * D;
        float mean = 0.0f;
        for (int64_t d = 0; d < D; d++) mean += xn[d];
        mean /= (float)D;
        float var = 0.0f;
        for (int64_t d = 0; d < D; d++) {
            const float diff = xn[d] - mean;
            var += diff * diff;
        }
        var = var / (float)D + eps;
        const float inv_std = 1.0f / sqrtf(var);
        for (int64_t d = 0; d < D; d++) yn[d] = (xn[d] - mean) * inv_std * gamma[d] + beta[d];
    }
    return 0;
}

/* MatMul — src/operator/blas/matmul.c:14-50: per batch slice, C[i][j] = Σ_k a·b in k order
 * (+ bias[j]), A (M, K) or, transposed, (K, M); B (K, N) or, transposed, (N, K). */
int oracle_matmul_f32(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                      int64_t K, int transpose_a, int transpose_b, int64_t batch, int64_t stride_a,
                      int64_t stride_b, int64_t stride_c) {
    if (!A || !B || !C || M < 0 || N < 0 || K < 0) return -1;
    if (batch <= 0) batch = 1;
    for (int64_t bi = 0; bi < batch; bi++) {
        const float* Ab = A + bi * stride_a;
        const float* Bb = B + bi * stride_b;
        float* Cb = C + bi * stride_c;
        for (int64_t i = 0; i < M; i++)
            for (int64_t j = 0; j < N; j++) {
                float sum = 0.0f;
                for (int64_t k = 0; k < K; k++) {
                    const float av = transpose_a ? Ab[k * M + i] : Ab[i * K + k];
                    const float bv = transpose_b ? Bb[j * K + k] : Bb[k * N + j];
                    sum += av * bv;
                }
                Cb[i * N + j] = sum + (bias ? bias[j] : 0.0f);
            }
    }
    return 0;
}

/* RoPE of one position — src/operator/nn/rope.c:36-62: angle = pos / base^(2i/d) in
 * float with powf, cosf, sinf; pair (2i, 2i+1) of each of the H heads of v (H x d)
 * rotated by that angle. */
void oracle_rope_at(float* v, int64_t H, int64_t d, int64_t pos, float base) {
    const int64_t half_d = d / 2;
    for (int64_t h = 0; h < H; h++) {
        float* q = v + h * d;
        for (int64_t i = 0; i < half_d; i++) {
            const float angle = (float)pos / powf(base, (float)(2 * i) / (float)d);
            const float c = cosf(angle);
            const float s = sinf(angle);
            const float x0 = q[2 * i];
            const float x1 = q[2 * i + 1];
            q[2 * i] = x0 * c - x1 * s;
            q[2 * i + 1] = x0 * s + x1 * c;
        }
    }
}

/* RoPE op — src/operator/nn/rope.c:17-66: copy when not in place, then rotate row pos
 * (H heads of d) by position pos for pos = 0 .. S-1. */
int oracle_rope_f32(const float* in, float* out, int64_t S, int64_t H, int64_t d, float base) {
    if (!in || !out || S < 0 || H <= 0 || d <= 0 || (d & 1)) return -1;
    if (in != out) memcpy(out, in, (size_t)(S * H * d) * sizeof(float));
    for (int64_t pos = 0; pos < S; pos++) oracle_rope_at(out + pos * H * d, H, d, pos, base);
    return 0;
}

static int decode_impl(const void* inputs[], void* outputs[], const mha_decode_params_t* p, float rope_base);

int oracle_mha_decode_f32(const void* inputs[], void* outputs[], const mha_decode_params_t* p) {
    return decode_impl(inputs, outputs, p, 0.0f);
}

/* MHA_Decode with RoPE: the decode op above with rope.c's rotation applied to Q and to
 * K_new at the token's position (cache_len, or the sequence's length when ragged)
 * before K_new is appended and before the scores. */
int oracle_mha_decode_rope_f32(const void* inputs[], void* outputs[], const mha_decode_params_t* p,
                               float rope_base) {
    if (!(rope_base > 0.0f)) return -1;
    return decode_impl(inputs, outputs, p, rope_base);
}

static int decode_impl(const void* inputs[], void* outputs[], const mha_decode_params_t* p, float rope_base) {
    if (!p || !inputs || !outputs) return -1;
    for (int i = 0; i < 3; i++) if (!inputs[i]) return -1;
    if (!inputs[3] || !inputs[5] || !inputs[7] || !inputs[9]) return -1;
    for (int i = 0; i < 3; i++) if (!outputs[i]) return -1;

    const int64_t B = p->batch_size, D = p->hidden_size;
    const int64_t H = p->num_heads, d = p->head_dim;
    const int64_t H_kv = p->num_kv_heads > 0 ? p->num_kv_heads : H;
    const int64_t max_seq = p->max_seq;
    if (B <= 0 || D <= 0 || H <= 0 || d <= 0 || H % H_kv != 0 || max_seq <= 0) return -1;
    if (H * d != D) return -1;
    const int64_t kv_dim = H_kv * d;
    const int64_t group = H / H_kv;
    const int32_t* lens = NULL;
    if (p->cache_len < 0) {
        lens = (const int32_t*)inputs[MHA_DECODE_SLOT_SEQLENS];
        if (!lens) return -1;
    } else if (p->cache_len >= max_seq) {
        return -1;
    }

    const float* X  = (const float*)inputs[0];
    const float* Kc = (const float*)inputs[1];
    const float* Vc = (const float*)inputs[2];
    const float* WQ = (const float*)inputs[3];
    const float* bQ = (const float*)inputs[4];
    const float* WK = (const float*)inputs[5];
    const float* bK = (const float*)inputs[6];
    const float* WV = (const float*)inputs[7];
    const float* bV = (const float*)inputs[8];
    const float* WO = (const float*)inputs[9];
    const float* bO = (const float*)inputs[10];
    float* Y  = (float*)outputs[0];
    float* Ko = (float*)outputs[1];
    float* Vo = (float*)outputs[2];

    const size_t cache_elems = (size_t)B * (size_t)max_seq * (size_t)kv_dim;
    if (Ko != Kc) memcpy(Ko, Kc, cache_elems * sizeof(float));
    if (Vo != Vc) memcpy(Vo, Vc, cache_elems * sizeof(float));

    float* knew = (float*)malloc((size_t)d * sizeof(float));
    float* vnew = (float*)malloc((size_t)d * sizeof(float));
    float* q = (float*)malloc((size_t)d * sizeof(float));
    float* merged = (float*)malloc((size_t)d * sizeof(float));
    float* scores = (float*)malloc((size_t)max_seq * sizeof(float));
    if (!knew || !vnew || !q || !merged || !scores) {
        free(knew); free(vnew); free(q); free(merged); free(scores);
        return -1;
    }

    for (int64_t b = 0; b < B; b++) {
        const int64_t cache_len = lens ? (int64_t)lens[b] : p->cache_len;
        if (cache_len < 0 || cache_len >= max_seq) {
            free(knew); free(vnew); free(q); free(merged); free(scores);
            return -1;
        }
        const float* x = X + b * D;
        float* y = Y + b * D;
        for (int64_t j = 0; j < D; j++) y[j] = bO ? bO[j] : 0.0f;

        for (int64_t kvh = 0; kvh < H_kv; kvh++) {
            const int64_t kvo = kvh * d;
            for (int64_t di = 0; di < d; di++) {
                float ka = 0.0f, va = 0.0f;
                for (int64_t j = 0; j < D; j++) {
                    ka += x[j] * WK[j * kv_dim + kvo + di];
                    va += x[j] * WV[j * kv_dim + kvo + di];
                }
                knew[di] = ka + (bK ? bK[kvo + di] : 0.0f);
                vnew[di] = va + (bV ? bV[kvo + di] : 0.0f);
            }
            if (rope_base > 0.0f) oracle_rope_at(knew, 1, d, cache_len, rope_base);
            const int64_t row = (b * max_seq + cache_len) * kv_dim + kvo;
            for (int64_t di = 0; di < d; di++) {
                Ko[row + di] = knew[di];
                Vo[row + di] = vnew[di];
            }
        }

        for (int64_t h = 0; h < H; h++) {
            const int64_t ho = h * d;
            const int64_t kvo = (h / group) * d;
            for (int64_t di = 0; di < d; di++) {
                float acc = 0.0f;
                for (int64_t j = 0; j < D; j++) acc += x[j] * WQ[j * D + ho + di];
                q[di] = acc + (bQ ? bQ[ho + di] : 0.0f);
            }
            if (rope_base > 0.0f) oracle_rope_at(q, 1, d, cache_len, rope_base);
            const int64_t total = cache_len + 1;
            float mx = -1e38f;
            for (int64_t t = 0; t < total; t++) {
                float dot = 0.0f;
                const int64_t ko = (b * max_seq + t) * kv_dim + kvo;
                for (int64_t di = 0; di < d; di++) dot += q[di] * Ko[ko + di];
                scores[t] = dot * p->scale;
                if (scores[t] > mx) mx = scores[t];
            }
            float sum = 0.0f;
            for (int64_t t = 0; t < total; t++) {
                scores[t] = expf(scores[t] - mx);
                sum += scores[t];
            }
            if (sum < 1e-12f) sum = 1e-12f;
            for (int64_t di = 0; di < d; di++) merged[di] = 0.0f;
            for (int64_t t = 0; t < total; t++) {
                const float w = scores[t] / sum;
                const int64_t vo = (b * max_seq + t) * kv_dim + kvo;
                for (int64_t di = 0; di < d; di++) merged[di] += w * Vo[vo + di];
            }
            for (int64_t j = 0; j < D; j++) {
                float c = 0.0f;
                for (int64_t di = 0; di < d; di++) c += merged[di] * WO[(ho + di) * D + j];
                y[j] += c;
            }
        }
    }
    free(knew); free(vnew); free(q); free(merged); free(scores);
    return 0;
}

/* Attention core with Q given — the inner part of mha_decode.c:88-114, same order. */
int oracle_decode_attn_f32(const float* Q, const float* K, const float* V, float* O,
                           int64_t B, int64_t H_q, int64_t H_kv, int64_t d, int64_t max_seq,
                           const int32_t* attend, float scale) {
    if (!Q || !K || !V || !O || !attend) return -1;
    if (H_kv <= 0) H_kv = H_q;
    if (B <= 0 || H_q <= 0 || d <= 0 || H_q % H_kv != 0) return -1;
    const int64_t kv_dim = H_kv * d, group = H_q / H_kv;
    float* scores = (float*)malloc((size_t)max_seq * sizeof(float));
    if (!scores) return -1;
    for (int64_t b = 0; b < B; b++) {
        const int64_t total = attend[b];
        if (total < 1 || total > max_seq) { free(scores); return -1; }
        for (int64_t h = 0; h < H_q; h++) {
            const float* q = Q + (b * H_q + h) * d;
            float* o = O + (b * H_q + h) * d;
            const int64_t kvo = (h / group) * d;
            float mx = -1e38f;
            for (int64_t t = 0; t < total; t++) {
                float dot = 0.0f;
                const int64_t ko = (b * max_seq + t) * kv_dim + kvo;
                for (int64_t di = 0; di < d; di++) dot += q[di] * K[ko + di];
                scores[t] = dot * scale;
                if (scores[t] > mx) mx = scores[t];
            }
            float sum = 0.0f;
            for (int64_t t = 0; t < total; t++) {
                scores[t] = expf(scores[t] - mx);
                sum += scores[t];
            }
            if (sum < 1e-12f) sum = 1e-12f;
            for (int64_t di = 0; di < d; di++) o[di] = 0.0f;
            for (int64_t t = 0; t < total; t++) {
                const float w = scores[t] / sum;
                const int64_t vo = (b * max_seq + t) * kv_dim + kvo;
                for (int64_t di = 0; di < d; di++) o[di] += w * V[vo + di];
            }
        }
    }
    free(scores);
    return 0;
}

/* ------------------------------------------------------------------------------------
 * MHA_Fused — follows src/operator/nn/mha_fused.c:32-176: projections with the three
 * accumulators interleaved (:75-86), per (b, h, row) scores·scale and running max
 * (:104-113), expf and sum (:116-120), clamp and inv_sum (:121-122),
 * attn = Σ (e·inv_sum)·V (:125-131), merge heads, Y = merged·WO + bO (+R) (:152-171).
 * Additions: causal (keys j > i excluded, as the reference GPU kernels' -1e38 mask gives
 * exp = 0) and GQA (WK/WV of shape (D, H_kv·d)).
 * ---------------------------------------------------------------------------------- */
int oracle_mha_fused_f32(const void* inputs[], void* outputs[], const mha_fused_params_t* p) {
    if (!inputs || !inputs[0] || !outputs || !outputs[0] || !p) return -1;
    const float* X  = (const float*)inputs[0];
    const float* R  = (const float*)inputs[1];
    const float* WQ = (const float*)inputs[2];
    const float* bQ = (const float*)inputs[3];
    const float* WK = (const float*)inputs[4];
    const float* bK = (const float*)inputs[5];
    const float* WV = (const float*)inputs[6];
    const float* bV = (const float*)inputs[7];
    const float* WO = (const float*)inputs[8];
    const float* bO = (const float*)inputs[9];
    float* Y = (float*)outputs[0];
    if (!WQ || !WK || !WV || !WO) return -1;

    const int64_t B = p->batch_size, S = p->seq_len, D = p->hidden_size;
    const int64_t H = p->num_heads, d = p->head_dim;
    const int64_t H_kv = p->num_kv_heads > 0 ? p->num_kv_heads : H;
    if (B <= 0 || S <= 0 || D <= 0 || H <= 0 || d <= 0 || H % H_kv != 0) return -1;
    const int64_t kvd = H_kv * d, qd = H * d, group = H / H_kv;
    if (qd != D) return -1;
    const int causal = p->causal ? 1 : 0;

    float* Q = (float*)calloc((size_t)(B * S * qd), sizeof(float));
    float* Kb = (float*)calloc((size_t)(B * S * kvd), sizeof(float));
    float* V = (float*)calloc((size_t)(B * S * kvd), sizeof(float));
    float* attn = (float*)calloc((size_t)(B * H * S * d), sizeof(float));
    float* merged = (float*)calloc((size_t)(B * S * qd), sizeof(float));
    float* row = (float*)calloc((size_t)S, sizeof(float));
    if (!Q || !Kb || !V || !attn || !merged || !row) {
        free(Q); free(Kb); free(V); free(attn); free(merged); free(row);
        return -1;
    }

    for (int64_t bs = 0; bs < B * S; bs++) {
        const float* x = X + bs * D;
        for (int64_t j = 0; j < qd; j++) {
            float sq = 0.0f, sk = 0.0f, sv = 0.0f;
            const int kv_col = j < kvd;
            for (int64_t i = 0; i < D; i++) {
                const float xv = x[i];
                sq += xv * WQ[i * qd + j];
                if (kv_col) {
                    sk += xv * WK[i * kvd + j];
                    sv += xv * WV[i * kvd + j];
                }
            }
            Q[bs * qd + j] = sq + (bQ ? bQ[j] : 0.0f);
            if (kv_col) {
                Kb[bs * kvd + j] = sk + (bK ? bK[j] : 0.0f);
                V[bs * kvd + j] = sv + (bV ? bV[j] : 0.0f);
            }
        }
    }

    const float scale = p->scale;
    for (int64_t b = 0; b < B; b++) {
        for (int64_t h = 0; h < H; h++) {
            float* ab = attn + (b * H + h) * S * d;
            const int64_t kvo = (h / group) * d;
            for (int64_t si = 0; si < S; si++) {
                const int64_t nk = causal ? si + 1 : S;
                float mx = -1e38f;
                for (int64_t sj = 0; sj < nk; sj++) {
                    float dot = 0.0f;
                    for (int64_t di = 0; di < d; di++)
                        dot += Q[(b * S + si) * qd + h * d + di] * Kb[(b * S + sj) * kvd + kvo + di];
                    row[sj] = dot * scale;
                    if (row[sj] > mx) mx = row[sj];
                }
                float sum = 0.0f;
                for (int64_t sj = 0; sj < nk; sj++) {
                    row[sj] = expf(row[sj] - mx);
                    sum += row[sj];
                }
                if (sum < 1e-12f) sum = 1e-12f;
                const float inv = 1.0f / sum;
                for (int64_t di = 0; di < d; di++) {
                    float acc = 0.0f;
                    for (int64_t sj = 0; sj < nk; sj++)
                        acc += row[sj] * inv * V[(b * S + sj) * kvd + kvo + di];
                    ab[si * d + di] = acc;
                }
            }
        }
    }

    for (int64_t b = 0; b < B; b++)
        for (int64_t s = 0; s < S; s++)
            for (int64_t h = 0; h < H; h++)
                for (int64_t di = 0; di < d; di++)
                    merged[(b * S + s) * qd + h * d + di] = attn[(b * H + h) * S * d + s * d + di];

    for (int64_t bs = 0; bs < B * S; bs++) {
        float* y = Y + bs * D;
        const float* m = merged + bs * qd;
        for (int64_t j = 0; j < D; j++) {
            float acc = 0.0f;
            for (int64_t i = 0; i < qd; i++) acc += m[i] * WO[i * D + j];
            y[j] = acc + (bO ? bO[j] : 0.0f);
        }
        if (p->has_residual && R) {
            const float* r = R + bs * D;
            for (int64_t j = 0; j < D; j++) y[j] += r[j];
        }
    }

    free(Q); free(Kb); free(V); free(attn); free(merged); free(row);
    return 0;
}

/* src/operator/nn/causal_mask.c:17-21 */
void oracle_causal_mask_f32(float* mask, int64_t S) {
    for (int64_t i = 0; i < S; i++)
        for (int64_t j = 0; j < S; j++)
            mask[i * S + j] = (j <= i) ? 0.0f : -INFINITY;
}

/* ------------------------------------------------------------------------------------
 * Generators
 * ---------------------------------------------------------------------------------- */
uint64_t oracle_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Uniform double in (0, 1] from the top 53 bits. */
static double unit_open0(uint64_t* st) {
    return ((double)(oracle_splitmix64(st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

/* Box–Muller, both outputs used. */
void oracle_fill_normal(float* out, size_t n, uint64_t seed, float mean, float stddev) {
    uint64_t st = seed;
    size_t i = 0;
    while (i < n) {
        const double u1 = unit_open0(&st), u2 = unit_open0(&st);
        const double r = sqrt(-2.0 * log(u1));
        const double a = 6.283185307179586 * u2;
        out[i++] = (float)(mean + stddev * r * cos(a));
        if (i < n) out[i++] = (float)(mean + stddev * r * sin(a));
    }
}

void oracle_fill_uniform_int(int32_t* out, size_t n, uint64_t seed, int32_t lo, int32_t hi) {
    uint64_t st = seed;
    const uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)((int64_t)lo + (int64_t)(oracle_splitmix64(&st) % span));
}

void oracle_fill_glibc_rand(float* out, size_t n, int seed) {
    srand((unsigned)seed);
    for (size_t i = 0; i < n; i++) out[i] = ((float)rand() / (float)RAND_MAX - 0.5f) * 2.0f;
}

void oracle_fill_lcg(float* out, size_t n, unsigned seed) {
    unsigned st = seed;
    for (size_t i = 0; i < n; i++) {
        st = st * 1103515245u + 12345u;
        out[i] = ((float)(st & 0x7FFFFFFF) / 2147483648.0f) - 1.0f;
    }
}

/* ------------------------------------------------------------------------------------
 * binary16 <-> binary32 (IEEE 754, round to nearest even)
 * ---------------------------------------------------------------------------------- */
uint16_t oracle_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t ax = u & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* subnormal or zero half */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;                      /* 14 .. 24 */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu, u;
    if (e == 0) {
        if (m == 0) u = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3FFu;
            u = sign | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------------------
 * Operator-signature wrappers (CPU registrations for graph tests)
 * ---------------------------------------------------------------------------------- */
int oracle_op_mha_decode_f32(const void* inputs[], void* outputs[], const void* params, void* stream) {
    (void)stream;
    if (!params) return -1;
    return oracle_mha_decode_f32(inputs, outputs, (const mha_decode_params_t*)params);
}

int oracle_op_mha_fused_f32(const void* inputs[], void* outputs[], const void* params, void* stream) {
    (void)stream;
    if (!params) return -1;
    return oracle_mha_fused_f32(inputs, outputs, (const mha_fused_params_t*)params);
}

int oracle_op_causal_mask_f32(const void* inputs[], void* outputs[], const void* params, void* stream) {
    (void)inputs; (void)stream;
    if (!outputs || !outputs[0] || !params) return -1;
    oracle_causal_mask_f32((float*)outputs[0], *(const int64_t*)params);
    return 0;
}

double oracle_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}
