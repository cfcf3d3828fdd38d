/*
 * oracle.c - CPU restatement of Sapphire's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity reference, never the product). See oracle.h.
 *
 * Arithmetic-order notes. The reference is built by gcc with -O3 -mavx2 -mfma and
 * GNU C's default -ffp-contract=fast, so a few scalar expressions in the reference
 * are contracted into fused multiply-adds by the compiler. This file is built with
 * -ffp-contract=off and writes every fused operation as an explicit fmaf(); the
 * places where the reference's fusion comes from contraction rather than from an
 * _mm256_fmadd_ps intrinsic are marked "contracted", and each was pinned bitwise
 * against the compiled reference (tests/test_oracle_pin.py).
 *
 * How each function is pinned is stated in tests/test_oracle_pin.py and tests/test_oracle_math.py.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Block formats: include/kernels.h:29-38.                                     */
/* Q4_0 = { float scale; uint8_t q[16]; } (20 B), element 2j = q[j] & 0xF,     */
/* element 2j+1 = q[j] >> 4 (q4_0_avx.c:61-66), value = (nib - 8) * scale.     */
/* Q8_0 = { float scale; int8_t q[32]; } (36 B), value = q * scale.            */
/* ------------------------------------------------------------------------- */
typedef struct { float scale; uint8_t q[16]; } orc_q4_block;
typedef struct { float scale; uint8_t q[32]; } orc_q8_block;

static inline int q4_nibble(const orc_q4_block *b, int e) {
    uint8_t v = b->q[e >> 1];
    return (e & 1) ? (v >> 4) : (v & 0x0F);
}

void oracle_q4_0_unpack_ints(const void *blocks, int nblocks, int8_t *out) {
    const orc_q4_block *b = (const orc_q4_block *)blocks;
    for (int i = 0; i < nblocks; ++i)
        for (int e = 0; e < 32; ++e) out[i * 32 + e] = (int8_t)(q4_nibble(&b[i], e) - 8);
}

void oracle_q8_0_unpack_ints(const void *blocks, int nblocks, int8_t *out) {
    const orc_q8_block *b = (const orc_q8_block *)blocks;
    for (int i = 0; i < nblocks; ++i)
        for (int e = 0; e < 32; ++e) out[i * 32 + e] = (int8_t)b[i].q[e];
}

/* The dequantised float the reference feeds to its FMA: fl(int * scale)
 * (q4_0_avx.c:38-40: cvt, sub 8.0f, mul scale; q8_0_avx.c:50-59: cvt, mul scale). */
void oracle_dequant(int dtype, const void *blocks, int nblocks, float *out) {
    if (dtype == ORC_Q4_0) {
        const orc_q4_block *b = (const orc_q4_block *)blocks;
        for (int i = 0; i < nblocks; ++i)
            for (int e = 0; e < 32; ++e)
                out[i * 32 + e] = ((float)q4_nibble(&b[i], e) - 8.0f) * b[i].scale;
    } else {
        const orc_q8_block *b = (const orc_q8_block *)blocks;
        for (int i = 0; i < nblocks; ++i)
            for (int e = 0; e < 32; ++e)
                out[i * 32 + e] = (float)(int8_t)b[i].q[e] * b[i].scale;
    }
}

/* ------------------------------------------------------------------------- */
/* Row kernels.                                                                */
/* ------------------------------------------------------------------------- */

/* One Q4_0 block into a bank of four 8-lane accumulators: q4_0_avx.c:53-81.
 * acc[k][l] receives element 8k+l of the block (ilo, ilo>>8, ihi, ihi>>8). */
static inline void q4_block(const orc_q4_block *blk, const float *x, float acc[4][8]) {
    for (int k = 0; k < 4; ++k)
        for (int l = 0; l < 8; ++l) {
            int e = 8 * k + l;
            float w = ((float)q4_nibble(blk, e) - 8.0f) * blk->scale;   /* :38-40 */
            acc[k][l] = fmaf(w, x[e], acc[k][l]);                         /* :41 */
        }
}

/* quantized_gemv_q4_0_{aligned,unaligned}: q4_0_avx.c:102-148 (the two differ only
 * in how x is loaded). Even blocks go to bank 0..3, odd blocks to bank 4..7, an odd
 * tail block to bank 0..3 (:113-120); reduction tree :86-98. */
float oracle_q4_0_row(const void *w_row, const float *x, int block_count, int block_size) {
    if (block_size != 32 || !w_row || !x) return 0.0f;                    /* :103 */
    const orc_q4_block *blocks = (const orc_q4_block *)w_row;
    float acc[8][8];
    memset(acc, 0, sizeof acc);
    int b = 0;
    for (; b + 1 < block_count; b += 2) {
        q4_block(&blocks[b], x + b * 32, &acc[0]);
        q4_block(&blocks[b + 1], x + (b + 1) * 32, &acc[4]);
    }
    for (; b < block_count; ++b) q4_block(&blocks[b], x + b * 32, &acc[0]);
    float t[8];
    for (int l = 0; l < 8; ++l) {
        float s01 = acc[0][l] + acc[1][l], s23 = acc[2][l] + acc[3][l];
        float s45 = acc[4][l] + acc[5][l], s67 = acc[6][l] + acc[7][l];
        t[l] = (s01 + s23) + (s45 + s67);
    }
    return t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];         /* :97 */
}

/* quantized_gemv_q8_0_{aligned,unaligned}: q8_0_avx.c:16-136. Four accumulators,
 * acc[k] lane l <- element 8k+l of every block (:21-64); reduction :67-74. */
float oracle_q8_0_row(const void *w_row, const float *x, int block_count, int block_size) {
    if (block_size != 32 || !w_row || !x) return 0.0f;                    /* :17 */
    const orc_q8_block *blocks = (const orc_q8_block *)w_row;
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    for (int b = 0; b < block_count; ++b) {
        const orc_q8_block *blk = &blocks[b];
        for (int k = 0; k < 4; ++k)
            for (int l = 0; l < 8; ++l) {
                int e = 8 * k + l;
                float w = (float)(int8_t)blk->q[e] * blk->scale;          /* :50-59 */
                acc[k][l] = fmaf(w, x[b * 32 + e], acc[k][l]);            /* :61-64 */
            }
    }
    float t[8];
    for (int l = 0; l < 8; ++l) t[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    return t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];         /* :73 */
}

/* ------------------------------------------------------------------------- */
/* F32 / BF16 rows (the dtypes the reference loader produces).                  */
/* ------------------------------------------------------------------------- */

/* A scalar chain acc += w[j] * x[j], j = j0 .. j1-1, as the reference build compiles it: BF16
 * terms are fused (one FMA each); F32 loops are vectorised four wide, so the first
 * 4 * floor(n / 4) products are rounded before their in-order additions and the last n % 4
 * terms are fused. Both forms are pinned against the compiled reference (tests/test_oracle_pin.py). */
static float f_elem(int dtype, const void *w, int j);
static float scalar_chain(int dtype, const void *w, const float *x, int j0, int j1, float acc) {
    const int vec_end = dtype == ORC_F32 ? j0 + (j1 - j0) / 4 * 4 : j0;
    int j = j0;
    for (; j < vec_end; ++j) acc = acc + f_elem(dtype, w, j) * x[j];
    for (; j < j1; ++j) acc = fmaf(f_elem(dtype, w, j), x[j], acc);
    return acc;
}

/* element j of an F32 row, or of a BF16 row widened by a 16-bit shift (bf16_avx.c:30-33,
 * :77-79) */
static float f_elem(int dtype, const void *w, int j) {
    if (dtype == ORC_F32) return ((const float *)w)[j];
    uint32_t b = (uint32_t)((const uint16_t *)w)[j] << 16;
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

/* quantized_gemv_{bf16,f32}_avx2: bf16_avx.c:57-113, f32_avx.c:43-90. Chunks of 32: element
 * j + 8k + l goes to accumulator k, lane l (FMA); the remainder is one scalar_chain; the
 * lanes reduce as (a0 + a1) + (a2 + a3), then t0 + ... + t7 + remainder left to right. */
float oracle_f_row(int dtype, const void *w_row, const float *x, int cols) {
    if (!w_row || !x) return 0.0f;
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    int j = 0;
    for (; j + 32 <= cols; j += 32)
        for (int k = 0; k < 4; ++k)
            for (int l = 0; l < 8; ++l) acc[k][l] = fmaf(f_elem(dtype, w_row, j + 8 * k + l), x[j + 8 * k + l], acc[k][l]);
    const float rem = scalar_chain(dtype, w_row, x, j, cols, 0.0f);
    float t[8];
    for (int l = 0; l < 8; ++l) t[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    return t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7] + rem;
}

/* kernel_gemv without a context for F32 / BF16: gemv_f32 / gemv_bf16, dispatch.c:60-85, one
 * scalar_chain per row. */
float oracle_f_row_scalar(int dtype, const void *w_row, const float *x, int cols) {
    return scalar_chain(dtype, w_row, x, 0, cols, 0.0f);
}

/* kernel_gemm_{bf16,f32}_avx2 (bf16_avx.c:115-159, f32_avx.c): per sequence one accumulator
 * of eight lanes over chunks of 8, t0 + ... + t7 left to right, then the remainder added as a
 * scalar_chain. Y[b * ldy + r]. */
int oracle_gemm_f(int dtype, const void *W, int M, int K, const float *X, int batch, float *Y, int ldy) {
    if (!W || !X || !Y || M <= 0 || K <= 0 || batch <= 0 || (dtype != ORC_F32 && dtype != ORC_BF16)) return -1;
    const size_t es = dtype == ORC_F32 ? 4 : 2;
    for (int r = 0; r < M; ++r) {
        const void *w = (const unsigned char *)W + (size_t)r * K * es;
        for (int b = 0; b < batch; ++b) {
            const float *x = X + (size_t)b * K;
            float acc[8] = { 0 };
            int j = 0;
            for (; j + 8 <= K; j += 8)
                for (int l = 0; l < 8; ++l) acc[l] = fmaf(f_elem(dtype, w, j + l), x[j + l], acc[l]);
            float sum = acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
            sum = scalar_chain(dtype, w, x, j, K, sum);
            Y[(size_t)b * ldy + r] = sum;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Pooled GEMV: pool.c:270-362. Rows are independent (y[r] = kernel(row r),     */
/* pool.c:112-140); the partition (chunk = ceil(rows/threads), pool.c:326-329)  */
/* changes only which thread computes a row, never its value.                  */
/* ------------------------------------------------------------------------- */
typedef struct {
    int dtype, K, nb, r0, r1;
    size_t stride;
    const unsigned char *W;
    const float *x;
    float *y;
} gemv_task;

static void gemv_rows(const gemv_task *t) {
    for (int r = t->r0; r < t->r1; ++r) {
        const void *row = t->W + (size_t)r * t->stride;
        if (t->dtype == ORC_F32 || t->dtype == ORC_BF16)   /* count = cols, pool.c:116-121 */
            t->y[r] = oracle_f_row(t->dtype, row, t->x, t->K);
        else
            t->y[r] = (t->dtype == ORC_Q4_0) ? oracle_q4_0_row(row, t->x, t->nb, 32)
                                             : oracle_q8_0_row(row, t->x, t->nb, 32);
    }
}

static void *gemv_thread(void *arg) { gemv_rows((const gemv_task *)arg); return NULL; }

int oracle_gemv(int dtype, const void *W, int M, int K, const float *x, float *y, int nthreads) {
    if (!W || !x || !y || M <= 0 || K <= 0) return -1;                    /* dispatch.c:102-124 */
    if (dtype != ORC_Q4_0 && dtype != ORC_Q8_0 && dtype != ORC_F32 && dtype != ORC_BF16) return -1;
    int nb = (K + 31) / 32;                                               /* pool.c:285 */
    size_t stride = dtype == ORC_F32 ? (size_t)K * 4 : dtype == ORC_BF16 ? (size_t)K * 2   /* pool.c:303-312 */
                                     : (size_t)nb * (dtype == ORC_Q4_0 ? 20 : 36);        /* pool.c:297,301 */
    if (nthreads <= 1) {
        gemv_task t = { dtype, K, nb, 0, M, stride, (const unsigned char *)W, x, y };
        gemv_rows(&t);
        return 0;
    }
    int chunk = (M + nthreads - 1) / nthreads;                            /* pool.c:328 */
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    gemv_task *ts = (gemv_task *)malloc(sizeof(gemv_task) * (size_t)nthreads);
    if (!th || !ts) { free(th); free(ts); return -1; }
    int launched = 0;
    for (int i = 0; i < nthreads; ++i) {
        int r0 = i * chunk, r1 = r0 + chunk < M ? r0 + chunk : M;
        if (r0 >= M) break;
        ts[i] = (gemv_task){ dtype, K, nb, r0, r1, stride, (const unsigned char *)W, x, y };
        if (pthread_create(&th[launched], NULL, gemv_thread, &ts[i]) != 0) { gemv_rows(&ts[i]); continue; }
        ++launched;
    }
    for (int i = 0; i < launched; ++i) pthread_join(th[i], NULL);
    free(th);
    free(ts);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* RMSNorm: normalization.c.                                                   */
/* ------------------------------------------------------------------------- */

/* sum_sq_avx2: normalization.c:12-32. 8 FMA lanes, then (lo+hi) and two hadds:
 * ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7)); scalar tail (contracted). */
static float sum_sq(const float *in, int dim) {
    float s[8] = { 0 };
    int i = 0;
    for (; i + 8 <= dim; i += 8)
        for (int l = 0; l < 8; ++l) s[l] = fmaf(in[i + l], in[i + l], s[l]);
    float a0 = s[0] + s[4], a1 = s[1] + s[5], a2 = s[2] + s[6], a3 = s[3] + s[7];
    float sum = (a0 + a1) + (a2 + a3);
    for (; i < dim; ++i) sum = fmaf(in[i], in[i], sum);
    return sum;
}

/* rmsnorm: normalization.c:89-102; out = (in * rms_inv) * w. */
int oracle_rmsnorm(float *out, const float *in, const float *w, float eps, int dim) {
    if (!out || !in || !w || dim <= 0 || eps < 0.0f) return -1;
    float rms_inv = 1.0f / sqrtf(sum_sq(in, dim) / (float)dim + eps);
    for (int i = 0; i < dim; ++i) out[i] = (in[i] * rms_inv) * w[i];
    return 0;
}

/* rmsnorm_delta: normalization.c:104-117 (apply :48-62); out = (in * rms_inv) * (1 + w). */
int oracle_rmsnorm_delta(float *out, const float *in, const float *w, float eps, int dim) {
    if (!out || !in || !w || dim <= 0 || eps < 0.0f) return -1;
    float rms_inv = 1.0f / sqrtf(sum_sq(in, dim) / (float)dim + eps);
    for (int i = 0; i < dim; ++i) out[i] = (in[i] * rms_inv) * (1.0f + w[i]);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* RoPE: rope.c.                                                               */
/* ------------------------------------------------------------------------- */

/* rope_precompute_freqs: rope.c:41-63. Half-split tables [max_ctx][d_k]. */
int oracle_rope_precompute_freqs(float *cos_t, float *sin_t, int d_k, int max_ctx, float base) {
    if (!cos_t || !sin_t) return -1;
    int half = d_k / 2;
    for (int pos = 0; pos < max_ctx; ++pos)
        for (int m = 0; m < half; ++m) {
            float freq = 1.0f / powf(base, 2.0f * (float)m / (float)d_k);
            float angle = (float)pos * freq;
            float c = cosf(angle), s = sinf(angle);
            cos_t[pos * d_k + m] = c; cos_t[pos * d_k + m + half] = c;
            sin_t[pos * d_k + m] = s; sin_t[pos * d_k + m + half] = s;
        }
    return 0;
}

/* rope_apply_fast: rope.c:99-117 (half-split rotation). Both outputs are contracted
 * by the reference build as x0*c - x1*s -> fmaf(x0, c, -(x1*s)) and
 * x1*c + x0*s -> fmaf(x1, c, x0*s). */
void oracle_rope_apply_fast(float *x, int pos, int head_dim, const float *cos_t, const float *sin_t) {
    if (!x || !cos_t || !sin_t) return;
    const float *c = cos_t + pos * head_dim, *s = sin_t + pos * head_dim;
    int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        float x0 = x[i], x1 = x[i + half];
        x[i]        = fmaf(x0, c[i], -(x1 * s[i]));
        x[i + half] = fmaf(x1, c[i], x0 * s[i]);
    }
}

/* ------------------------------------------------------------------------- */
/* Activations: activations.c:64-82; FFN combine transformer.c:150-157.        */
/* ------------------------------------------------------------------------- */

/* gelu: activations.c:64-76. x + B*x*x*x is contracted to fmaf((B*x)*x, x, x). */
float oracle_gelu(float x) {
    const float A = 0.7978845608f, B = 0.044715f;
    float y = A * fmaf((B * x) * x, x, x);
    float t = tanhf(y);
    return 0.5f * x * (1.0f + t);
}

void oracle_gelu_mul(float *gate, const float *up, int n) {
    for (int i = 0; i < n; ++i) gate[i] = oracle_gelu(gate[i]);          /* gelu_inplace */
    for (int i = 0; i < n; ++i) gate[i] *= up[i];                         /* :154-156 */
}

/* silu: activations.c:16-20 (a divide, then a product; nothing to contract). */
float oracle_silu(float x) {
    const float sigmoid = 1.0f / (1.0f + expf(-x));
    return x * sigmoid;
}

/* geglu: activations.c:103-105. */
float oracle_geglu(float x, float y) { return x * oracle_gelu(y); }

/* apply_rope: rope.c:17-25 -> apply_positional_encoding (positional_encoding.c:76-104) with
 * rope_encoding_strategy (:16-40). Pair j/2 of (x[j], x[j+1]), j + 1 < head_dim, rotates by
 * theta = pos * powf(1/base, 2 (j/2) / head_dim); the reference build contracts the second
 * product of each line onto the first one's result (pinned against the compiled reference). */
void oracle_apply_rope(float *x, int pos, int head_dim, float base) {
    if (!x) return;
    for (int j = 0; j + 1 < head_dim; j += 2) {
        const float inv_freq = powf(1.0f / base, 2.0f * (float)(j / 2) / (float)head_dim);
        const float theta = (float)pos * inv_freq;
        const float c = cosf(theta), s = sinf(theta);
        const float xe = x[j], xo = x[j + 1];
        x[j] = fmaf(-xo, s, xe * c);
        x[j + 1] = fmaf(xo, c, xe * s);
    }
}

/* ------------------------------------------------------------------------- */
/* utils.c: softmax, argmax, vector ops.                                       */
/* ------------------------------------------------------------------------- */

/* softmax: utils.c:18-59. 8-lane max seeded with -1e38f, merged into scores[0];
 * sequential expf/sum; multiply by 1/sum. */
void oracle_softmax(float *x, int n) {
    if (n <= 0 || !x) return;
    float max_score = x[0];
    float lanes[8];
    for (int l = 0; l < 8; ++l) lanes[l] = -1e38f;
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) {
            /* _mm256_max_ps(a, b) returns b when either is NaN or a == b */
            float a = lanes[l], b = x[i + l];
            lanes[l] = (a > b) ? a : b;
        }
    for (int l = 0; l < 8; ++l) if (lanes[l] > max_score) max_score = lanes[l];
    for (; i < n; ++i) if (x[i] > max_score) max_score = x[i];
    float sum = 0.0f;
    for (i = 0; i < n; ++i) { x[i] = expf(x[i] - max_score); sum += x[i]; }
    float inv = 1.0f / sum;
    for (i = 0; i < n; ++i) x[i] *= inv;
}

/* sample_greedy: utils.c:145-156; strict '>' so the lowest index wins ties. */
int oracle_sample_greedy(const float *logits, int n) {
    if (!logits || n <= 0) return -1;
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < n; ++i) if (logits[i] > bv) { bv = logits[i]; best = i; }
    return best;
}

/* sample_temperature: utils.c:158-180. The max is seeded with logits[0] (strict '>'), the
 * weights expf((l - max) / T) overwrite the logits, their float sum runs left to right, and
 * the walk returns the first i with r <= cumsum (cumsum += w_i / sum in float), n - 1 if
 * none. r stands for (float)rand() / (float)RAND_MAX. */
int oracle_sample_temperature(float *logits, int n, float temperature, float r) {
    if (!logits || n <= 0) return -1;
    if (temperature <= 0.0f) return oracle_sample_greedy(logits, n);
    float mx = logits[0];
    for (int i = 1; i < n; ++i) if (logits[i] > mx) mx = logits[i];
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        logits[i] = expf((logits[i] - mx) / temperature);
        sum += logits[i];
    }
    float cum = 0.0f;
    for (int i = 0; i < n; ++i) {
        cum += logits[i] / sum;
        if (r <= cum) return i;
    }
    return n - 1;
}

/* perform_inference's draw (inference.c:262-266 and 297): the logits scaled by 1/T
 * (vec_scale, utils.c:87-92, which skips a factor of exactly 1) when T > 0, then
 * sample_temperature. */
int oracle_sample(float *logits, int n, float temperature, float r) {
    if (!logits || n <= 0) return -1;
    if (temperature > 0.0f) {
        const float inv = 1.0f / temperature;
        if (inv != 1.0f)
            for (int i = 0; i < n; ++i) logits[i] *= inv;
    }
    return oracle_sample_temperature(logits, n, temperature, r);
}

void oracle_vec_add(float *dst, const float *src, int n) {               /* utils.c:81-85 */
    for (int i = 0; i < n; ++i) dst[i] += src[i];
}

/* vec_dot: utils.c:100-117. 8 FMA lanes, lanes summed left to right, contracted tail. */
float oracle_vec_dot(const float *a, const float *b, int n) {
    float s[8] = { 0 };
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) s[l] = fmaf(a[i + l], b[i + l], s[l]);
    float f = s[0] + s[1] + s[2] + s[3] + s[4] + s[5] + s[6] + s[7];
    for (; i < n; ++i) f = fmaf(a[i], b[i], f);
    return f;
}

void oracle_bf16_to_f32(float *dst, const uint16_t *src, int n) {        /* utils.c:127-143 */
    for (int i = 0; i < n; ++i) {
        uint32_t bits = (uint32_t)src[i] << 16;
        memcpy(&dst[i], &bits, sizeof bits);
    }
}

/* ------------------------------------------------------------------------- */
/* Quantizer (the producer of Q4_0 / Q8_0 blocks).                             */
/* The reference has none: nothing in it creates quantized tensors            */
/* (tensor.c:108-110, safetensors_reader.c:406-414); its block structs are    */
/* ggml's. This restates ggml's published reference quantizer                 */
/* (llama.cpp ggml-quants.c, quantize_row_q8_0_ref / quantize_row_q4_0_ref),  */
/* adapted to the reference's block structs: an fp32 scale (kernels.h:29-38)  */
/* and the reference's Q4_0 nibble order, element 2j in the low nibble of     */
/* byte j and 2j+1 in the high nibble (q4_0_avx.c:61-66; ggml packs j and     */
/* j+16). Every product and sum is rounded on its own (no contraction):       */
/*   Q8_0: amax = max|x|; d = amax / 127; id = d ? 1/d : 0;                    */
/*         q = roundf(x * id) (ties away from zero).                           */
/*   Q4_0: max = the first x of largest |x| (+0 when all are zero);            */
/*         d = max / -8; id = d ? 1/d : 0;                                     */
/*         q = min(15, (int)(x * id + 8.5f)) (truncation: ties round up).      */
/* Inputs must be finite. Elements past K in the last block are zeros.         */
/* Parity pins: tests/test_oracle_quant.py (known answers, reconstruction     */
/* bounds, idempotence on representable blocks, and the layout through the    */
/* reference's own row kernels).                                              */
/* ------------------------------------------------------------------------- */

/* Integer codes of the rounded values. For blocks of normal scale these are ggml's
 * conversions, min(15, (int)v) and (int)v; the guards only define the blocks ggml leaves
 * undefined, whose scale is subnormal so that 1/d overflows: an infinite product saturates
 * and a NaN one (0 * inf) gives the code of zero. */
static int q8_code(float v) { return v != v ? 0 : v > 127.0f ? 127 : v < -127.0f ? -127 : (int)v; }
static int q4_code(float v) { return v != v ? 8 : v > 15.0f ? 15 : v < 0.0f ? 0 : (int)v; }

static void quantize_block(int dtype, const float *x, void *out) {
    if (dtype == ORC_Q8_0) {
        orc_q8_block *b = (orc_q8_block *)out;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        b->scale = d;
        for (int i = 0; i < 32; ++i) b->q[i] = (uint8_t)(int8_t)q8_code(roundf(x[i] * id));
    } else {
        orc_q4_block *b = (orc_q4_block *)out;
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < 32; ++i)
            if (amax < fabsf(x[i])) {
                amax = fabsf(x[i]);
                max = x[i];
            }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        b->scale = d;
        for (int j = 0; j < 16; ++j) {
            const int q0 = q4_code(x[2 * j] * id + 8.5f), q1 = q4_code(x[2 * j + 1] * id + 8.5f);
            b->q[j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

int oracle_quantize(int dtype, int src_dtype, const void *src, int M, int K, void *blocks) {
    if ((dtype != ORC_Q4_0 && dtype != ORC_Q8_0) || (src_dtype != ORC_F32 && src_dtype != ORC_BF16) || !src ||
        !blocks || M <= 0 || K <= 0)
        return -1;
    const int nb = (K + 31) / 32;
    const size_t bb = dtype == ORC_Q4_0 ? sizeof(orc_q4_block) : sizeof(orc_q8_block);
    uint8_t *out = (uint8_t *)blocks;
    float x[32];
    for (int r = 0; r < M; ++r)
        for (int j = 0; j < nb; ++j) {
            for (int e = 0; e < 32; ++e) {
                const int k = j * 32 + e;
                if (k >= K) x[e] = 0.0f;
                else if (src_dtype == ORC_F32) x[e] = ((const float *)src)[(size_t)r * K + k];
                else oracle_bf16_to_f32(&x[e], (const uint16_t *)src + (size_t)r * K + k, 1);
            }
            quantize_block(dtype, x, out + ((size_t)r * nb + j) * bb);
        }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Decode step.                                                                */
/* ------------------------------------------------------------------------- */

static int layer_is_global(const oracle_model_t *m, int l) {              /* attention.c:104-111 */
    if (m->global_mask) return ((m->global_mask >> (unsigned)l) & 1ULL) != 0ULL;
    return ((l + 1) % 6) == 0;
}

/* sapphire_attention_forward: attention.c:93-163 (one token, GQA, sliding window). */
static void attention(const oracle_model_t *m, int l, int pos, const float *q, float *out, float *scores) {
    int hd = m->head_dim, seq_len = pos + 1;
    int win = m->sliding_window > 0 ? m->sliding_window : 1024;
    const float *kc = m->k_cache + (size_t)l * m->n_kv_heads * m->max_ctx * hd;
    const float *vc = m->v_cache + (size_t)l * m->n_kv_heads * m->max_ctx * hd;
    size_t cache_stride = (size_t)m->max_ctx * hd;
    memset(out, 0, sizeof(float) * (size_t)m->n_heads * hd);
    int start = 0, len = seq_len;
    if (!layer_is_global(m, l) && seq_len > win) { start = seq_len - win; len = win; }
    float scal = m->query_pre_attn_scalar > 0.0f ? 1.0f / sqrtf(m->query_pre_attn_scalar)
                                                 : 1.0f / sqrtf((float)hd);
    int group = m->n_heads / m->n_kv_heads;
    for (int h = 0; h < m->n_heads; ++h) {
        int hk = h / group;
        const float *kb = kc + hk * cache_stride + (size_t)start * hd;
        const float *vb = vc + hk * cache_stride + (size_t)start * hd;
        const float *qh = q + (size_t)h * hd;
        for (int t = 0; t < len; ++t) scores[t] = oracle_vec_dot(qh, kb + (size_t)t * hd, hd) * scal;
        oracle_softmax(scores, len);
        float *ho = out + (size_t)h * hd;
        for (int t = 0; t < len; ++t) {
            float a = scores[t];
            const float *vv = vb + (size_t)t * hd;
            for (int d = 0; d < hd; ++d) ho[d] = fmaf(a, vv[d], ho[d]);  /* :156, contracted */
        }
    }
}

/* inference_forward_batch with batch 1: inference.c:616-651, composed of
 * compute_attention_stage (attention.c:311-375), compute_ffn_stage
 * (transformer.c:96-171), finalize_layer_output (transformer.c:211-283) and
 * lm_head (transformer.c:393-408), followed by sample_greedy. */
int oracle_decode_step(const oracle_model_t *m, int token, int pos, float *logits) {
    if (!m || !logits || token < 0 || token >= m->vocab || pos < 0 || pos >= m->max_ctx) return -1;
    int H = m->hidden, hd = m->head_dim, nq = m->n_heads * hd, nk = m->n_kv_heads * hd;
    float *hidden = calloc((size_t)H, sizeof(float));
    float *resid = calloc((size_t)H, sizeof(float));
    float *norm = calloc((size_t)H, sizeof(float));
    float *q = calloc((size_t)nq, sizeof(float));
    float *k = calloc((size_t)nk, sizeof(float));
    float *v = calloc((size_t)nk, sizeof(float));
    float *attn = calloc((size_t)nq, sizeof(float));
    float *gate = calloc((size_t)m->ffn, sizeof(float));
    float *up = calloc((size_t)m->ffn, sizeof(float));
    float *qs = calloc((size_t)nq, sizeof(float));
    float *ks = calloc((size_t)nk, sizeof(float));
    float *scores = calloc((size_t)m->max_ctx, sizeof(float));
    int rc = -1;
    if (!hidden || !resid || !norm || !q || !k || !v || !attn || !gate || !up || !qs || !ks || !scores)
        goto done;

    /* embedding: transformer.c:367-380 (bf16 row, times sqrtf(hidden)) */
    oracle_bf16_to_f32(hidden, m->embed_bf16 + (size_t)token * H, H);
    float es = sqrtf((float)H);
    if (es != 1.0f) for (int i = 0; i < H; ++i) hidden[i] *= es;

    for (int l = 0; l < m->n_layers; ++l) {
        int glob = layer_is_global(m, l);
        const float *rc_ = glob ? m->rope_cos_global : m->rope_cos_local;  /* inference.c:630-632 */
        const float *rs_ = glob ? m->rope_sin_global : m->rope_sin_local;

        /* attention stage: attention.c:316-366 */
        memcpy(resid, hidden, sizeof(float) * H);
        oracle_rmsnorm_delta(norm, hidden, m->norm_attn[l], m->eps, H);
        oracle_gemv(m->wdtype, m->wq[l], nq, H, norm, q, m->nthreads);
        oracle_gemv(m->wdtype, m->wk[l], nk, H, norm, k, m->nthreads);
        oracle_gemv(m->wdtype, m->wv[l], nk, H, norm, v, m->nthreads);
        /* QK-norm with a head_dim-long gamma broadcast to every head: attention.c:228-289 */
        for (int h = 0; m->q_norm && h < m->n_heads; ++h) {
            const float *g = m->q_norm[l] + (m->q_norm_len == nq ? (size_t)h * hd : 0);
            memcpy(qs, q + (size_t)h * hd, sizeof(float) * hd);
            oracle_rmsnorm_delta(q + (size_t)h * hd, qs, g, m->eps, hd);
        }
        for (int h = 0; m->k_norm && h < m->n_kv_heads; ++h) {
            const float *g = m->k_norm[l] + (m->k_norm_len == nk ? (size_t)h * hd : 0);
            memcpy(ks, k + (size_t)h * hd, sizeof(float) * hd);
            oracle_rmsnorm_delta(k + (size_t)h * hd, ks, g, m->eps, hd);
        }
        for (int h = 0; h < m->n_heads; ++h) oracle_rope_apply_fast(q + (size_t)h * hd, pos, hd, rc_, rs_);
        for (int h = 0; h < m->n_kv_heads; ++h) oracle_rope_apply_fast(k + (size_t)h * hd, pos, hd, rc_, rs_);
        /* kv_cache_write_token: kv_cache.c:252-278, layout [head][pos][dim] */
        for (int h = 0; h < m->n_kv_heads; ++h) {
            size_t off = (((size_t)l * m->n_kv_heads + h) * m->max_ctx + pos) * hd;
            memcpy(m->k_cache + off, k + (size_t)h * hd, sizeof(float) * hd);
            memcpy(m->v_cache + off, v + (size_t)h * hd, sizeof(float) * hd);
        }
        attention(m, l, pos, q, attn, scores);
        oracle_gemv(m->wdtype, m->wo[l], H, nq, attn, hidden, m->nthreads);
        oracle_rmsnorm_delta(norm, hidden, m->norm_attn_post[l], m->eps, H);
        oracle_vec_add(resid, norm, H);
        memcpy(hidden, resid, sizeof(float) * H);

        /* FFN stage: transformer.c:119-170 (pre-norm reads the residual) */
        oracle_rmsnorm_delta(norm, resid, m->norm_ffn[l], m->eps, H);
        oracle_gemv(m->wdtype, m->wgate[l], m->ffn, H, norm, gate, m->nthreads);
        oracle_gemv(m->wdtype, m->wup[l], m->ffn, H, norm, up, m->nthreads);
        oracle_gelu_mul(gate, up, m->ffn);
        oracle_gemv(m->wdtype, m->wdown[l], H, m->ffn, gate, hidden, m->nthreads);

        /* finalize: transformer.c:231-239 */
        oracle_rmsnorm_delta(norm, hidden, m->norm_ffn_post[l], m->eps, H);
        oracle_vec_add(resid, norm, H);
        memcpy(hidden, resid, sizeof(float) * H);
    }

    /* lm_head: transformer.c:393-408 (final rmsnorm_delta then GEMV) */
    oracle_rmsnorm_delta(norm, hidden, m->norm_final, m->eps, H);
    oracle_gemv(m->lm_dtype, m->lm_head, m->vocab, H, norm, logits, m->nthreads);
    rc = oracle_sample_greedy(logits, m->vocab);

done:
    free(hidden); free(resid); free(norm); free(q); free(k); free(v); free(attn);
    free(gate); free(up); free(qs); free(ks); free(scores);
    return rc;
}
