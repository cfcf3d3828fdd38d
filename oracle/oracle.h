/*
 * oracle.h - CPU restatement of Sapphire's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity reference the HIP path is compared
 * against; it is never linked into, loaded by, or called from the product library
 * (sapphire_amd/). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Every function restates one reference routine in the reference's own arithmetic
 * order (file:line cited at each definition in oracle.c), so that its outputs are
 * bit-identical to the compiled reference on the same host.
 */
#ifndef SAPPHIRE_ORACLE_H
#define SAPPHIRE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: identical to tensor_dtype_t in the reference include/tensor.h:17-23 */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_F16 = 2, ORC_Q4_0 = 3, ORC_Q8_0 = 4 };

/* ---- quantizer: F32 / BF16 rows [M][K] -> [M][ceil(K/32)] Q4_0 / Q8_0 blocks ---- */
int   oracle_quantize(int dtype, int src_dtype, const void *src, int M, int K, void *blocks);

/* ---- block formats and unpack (include/kernels.h:29-38) ---- */
void  oracle_q4_0_unpack_ints(const void *blocks, int nblocks, int8_t *out /* 32*nblocks */);
void  oracle_q8_0_unpack_ints(const void *blocks, int nblocks, int8_t *out /* 32*nblocks */);
void  oracle_dequant(int dtype, const void *blocks, int nblocks, float *out /* 32*nblocks */);

/* ---- row kernels (src/kernels/q4_0_avx.c, q8_0_avx.c) ---- */
float oracle_q4_0_row(const void *w_row, const float *x, int block_count, int block_size);
float oracle_q8_0_row(const void *w_row, const float *x, int block_count, int block_size);

/* ---- F32 / BF16 rows (src/kernels/f32_avx.c, bf16_avx.c, dispatch.c:60-85) ---- */
float oracle_f_row(int dtype, const void *w_row, const float *x, int cols);          /* pooled kernel */
float oracle_f_row_scalar(int dtype, const void *w_row, const float *x, int cols);   /* no context */
/* batched form: Y[b * ldy + r] = W[r] . X[b] (kernel_gemm_{f32,bf16}_avx2) */
int   oracle_gemm_f(int dtype, const void *W, int M, int K, const float *X, int batch, float *Y, int ldy);

/* ---- pooled GEMV (src/kernels/pool.c:270-362 + dispatch.c:101-156) ----
 * y[M] = W[M x K] . x[K]; W is the reference AoS block array, row stride ceil(K/32)*B_blk,
 * or an F32 / BF16 matrix with row stride K elements.
 * nthreads <= 1 runs on the calling thread. Returns 0, or -1 on bad arguments. */
int   oracle_gemv(int dtype, const void *W, int M, int K, const float *x, float *y, int nthreads);

/* ---- primitives ---- */
int   oracle_rmsnorm(float *out, const float *in, const float *w, float eps, int dim);
int   oracle_rmsnorm_delta(float *out, const float *in, const float *w, float eps, int dim);
int   oracle_rope_precompute_freqs(float *cos_t, float *sin_t, int d_k, int max_ctx, float base);
void  oracle_rope_apply_fast(float *x, int pos, int head_dim, const float *cos_t, const float *sin_t);
float oracle_gelu(float x);
void  oracle_gelu_mul(float *gate, const float *up, int n);   /* gate = gelu(gate) * up */
float oracle_silu(float x);
float oracle_geglu(float x, float y);                          /* x * gelu(y) */
void  oracle_apply_rope(float *x, int pos, int head_dim, float base);   /* interleaved pairs */
void  oracle_softmax(float *x, int n);
int   oracle_sample_greedy(const float *logits, int n);
/* sample_temperature (utils.c:158-180; logits overwritten with the weights) with r in place
 * of rand() / RAND_MAX, and perform_inference's draw: 1/T scaling, then sample_temperature */
int   oracle_sample_temperature(float *logits, int n, float temperature, float r);
int   oracle_sample(float *logits, int n, float temperature, float r);
void  oracle_vec_add(float *dst, const float *src, int n);
float oracle_vec_dot(const float *a, const float *b, int n);
void  oracle_bf16_to_f32(float *dst, const uint16_t *src, int n);

/* ---- one Gemma-3 decode step (src/inference/inference.c:616-651 order) ---- */
typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    int sliding_window;                 /* <= 0 -> 1024, attention.c:113 */
    unsigned long long global_mask;     /* bit l set -> layer l is global; 0 -> (l+1)%6==0 */
    float query_pre_attn_scalar;        /* <= 0 -> head_dim, attention.c:129 */
    float eps;                          /* 1e-6 at every reference call site */
    int wdtype;                         /* ORC_Q4_0 or ORC_Q8_0 for the 7 projections */
    int lm_dtype;                       /* dtype of lm_head */
    /* per-layer pointers, arrays of length n_layers */
    const void  **wq, **wk, **wv, **wo, **wgate, **wup, **wdown;
    const float **norm_attn, **norm_attn_post, **norm_ffn, **norm_ffn_post;
    const float **q_norm, **k_norm;     /* length head_dim (broadcast) or heads*head_dim */
    int q_norm_len, k_norm_len;
    const uint16_t *embed_bf16;         /* [vocab, hidden] */
    const float    *norm_final;         /* [hidden] */
    const void     *lm_head;            /* [vocab, hidden] blocks */
    float *k_cache, *v_cache;           /* [n_layers][n_kv_heads][max_ctx][head_dim] */
    const float *rope_cos_global, *rope_sin_global, *rope_cos_local, *rope_sin_local;
    int nthreads;
} oracle_model_t;

/* Runs embed -> layers -> final norm -> lm_head for one token at position pos.
 * Writes logits[vocab]; returns the greedy argmax (lowest index on ties), or -1. */
int   oracle_decode_step(const oracle_model_t *m, int token, int pos, float *logits);

#ifdef __cplusplus
}
#endif
#endif
