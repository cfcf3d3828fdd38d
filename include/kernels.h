/*
 * kernels.h - GEMV / primitive API exported by libsapphire_hip.so (MI355X, gfx950).
 *
 * Drop-in for the reference's include/kernels.h: same block structs, context type,
 * function names, argument meanings, return codes and legacy macro aliases. Every
 * call below takes HOST pointers and is synchronous, like the reference's pthread
 * pool; the work runs on the GPU (HIP kernels in sapphire_amd/csrc), with weights kept
 * resident in HBM after the first call that reads them. Device-pointer and
 * stream-ordered forms of the same operations are declared in sapphire_hip.h.
 *
 * The scalar activations silu/relu/gelu/geglu(float) are one value's host arithmetic (the
 * reference's formula with its compiler's contraction, libm expf/tanhf); the vector forms the
 * engine calls on its buffers (gelu_inplace, sapphire_geglu, ...) run on the GPU.
 *
 * The include guard is the reference's own (KERNELS_H), like tensor.h's.
 */
#ifndef KERNELS_H
#define KERNELS_H

#include <stddef.h>
#include <stdint.h>

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- weight block formats: reference include/kernels.h:29-38 ---- */
typedef struct {
    float scale;        /* fp32 block scale */
    uint8_t q_data[16]; /* element 2j = q_data[j] & 0xF, element 2j+1 = q_data[j] >> 4; w = (nib-8)*scale */
} ggml_block_q4_0;

typedef struct {
    float scale;
    uint8_t q_data[32]; /* int8 quants; w = (int8)q * scale */
} ggml_block_q8_0;

/* ---- context: reference include/kernels.h:45-72, src/kernels/pool.c:157-268 ----
 * The context owns one HIP stream on the current device, pinned staging buffers for
 * the host-pointer calls and the device scratch they need. num_threads <= 0 is
 * accepted like the reference (it sizes the host callback pool of
 * kernel_parallel_for); chunk_size is accepted and ignored. */
typedef struct sapphire_context kernel_context_t;

kernel_context_t *kernel_ctx_create(int num_threads, int chunk_size);  /* kernels.h:56 */
int kernel_ctx_init(kernel_context_t *ctx);                            /* kernels.h:66; 0 / -1 */
void kernel_ctx_destroy(kernel_context_t *ctx);                        /* kernels.h:72 */

typedef float (*kernel_fn_t)(const void *w_row, const float *x, int blocks, int block_size);
typedef float (*gemv_kernel_t)(const void *w_row, const float *x, int blocks, int block_size);

typedef struct {
    const void *w_row;
    const float *X;
    float *Y;
    int batch_size;
    int d_model;
    int out_stride;
    int blocks;
    int block_size;
} gemm_args_t;                                                         /* kernels.h:84-93 */

typedef void (*gemm_kernel_t)(const gemm_args_t *args);
typedef void (*parallel_for_fn_t)(void *arg, int idx);

/* Host callbacks fn(arg, i) for i in [0, n), each index exactly once, on the context's
 * host worker threads; returns when all are done. kernels.h:110, pool.c:364-396. */
int kernel_parallel_for(kernel_context_t *ctx, parallel_for_fn_t fn, void *arg, int n);

/* ---- single-row dot products: reference kernels.h:113-118 ----
 * dot(W_row[0..block_count), x[0..32*block_count)); 0.0f when block_size != 32 or a
 * pointer is NULL (q4_0_avx.c:103, q8_0_avx.c:17). Evaluated on the GPU (one row). */
float quantized_gemv_q4_0_aligned(const void *W_row, const float *x, int block_count, int block_size);
float quantized_gemv_q4_0_unaligned(const void *W_row, const float *x, int block_count, int block_size);
float quantized_gemv_q8_0_aligned(const void *W_row, const float *x, int block_count, int block_size);
float quantized_gemv_q8_0_unaligned(const void *W_row, const float *x, int block_count, int block_size);

/* ---- F32 / BF16 rows: reference kernels.h:121-126 ----
 * dot(W_row[0..cols), x[0..cols)) with cols = block_count when block_size == 1, else
 * block_count * block_size (f32_avx.c:21-83, bf16_avx.c:21-108); 0.0f when a pointer is
 * NULL or cols <= 0. The avx2 and scalar names compute the same dot on the GPU (one row); the
 * reference's two differ only in fp32 summation order. */
float quantized_gemv_bf16_avx2(const void *W_row, const float *x, int block_count, int block_size);
float quantized_gemv_bf16_scalar(const void *W_row, const float *x, int block_count, int block_size);
float quantized_gemv_f32_avx2(const void *W_row, const float *x, int block_count, int block_size);
float quantized_gemv_f32_scalar(const void *W_row, const float *x, int block_count, int block_size);

/* ---- one weight row times a batch: reference kernels.h:129-130 ----
 * Y[b * out_stride] = w_row[0..d_model) . X[b * d_model ..] for b < batch_size
 * (f32_avx.c:97-135, bf16_avx.c:110-150); nothing is written when an argument is NULL or a
 * size is not positive. */
void kernel_gemm_f32_avx2(const gemm_args_t *args);
void kernel_gemm_bf16_avx2(const gemm_args_t *args);

/* ---- tensor GEMV API: reference kernels.h:140-166, src/kernels/dispatch.c ---- */

/* y[M] = A[M,K] . x[K]. A: 2-D tensor of dtype Q4_0, Q8_0, F32 or BF16 (rows = outputs).
 * Returns 0, or -1 on NULL y/A/x, ndim != 2, non-positive shape, NULL ctx with a
 * quantized A, unsupported dtype, or a device error (dispatch.c:101-156). With a NULL
 * ctx, F32/BF16 use the library's default context (the reference runs a naive loop). */
int kernel_gemv(kernel_context_t *ctx, float *y, const tensor_t *A, const float *x);

/* Y[b*M + r] = A[r,:] . X[b*K : b*K+K] for b < batch_size (row stride of Y is M, as in
 * pool.c:127-136; out_stride is accepted and, as in the reference, not used as the
 * stride). Unlike the reference, which rejects quantized batching (pool.c:318-321),
 * Q4_0/Q8_0 are computed. dispatch.c:87-99. */
int kernel_gemm(kernel_context_t *ctx, float *Y, const tensor_t *A, const float *X, int batch_size, int out_stride);

/* y = A . x with y, x 1-D F32 tensors; shape checks of dispatch.c:158-198. */
int kernel_gemv_tensor(kernel_context_t *ctx, const tensor_t *y, const tensor_t *A, const tensor_t *x);

/* y += alpha * (A . x). dispatch.c:200-232. */
int kernel_gemv_add(kernel_context_t *ctx, float *y, const tensor_t *A, const float *x, float alpha);

/* Y[b] = A . X[b] for b < batch_size (X stride K, Y stride M). dispatch.c:234-266. */
int kernel_gemv_batch(kernel_context_t *ctx, float *Y, const tensor_t *A, const float *X, int batch_size);

/* Float padding granularity callers use to size scratch (dispatch.c:275-287):
 * 8 for F32/BF16/F16/Q4_0/Q8_0, 1 otherwise. */
int kernel_get_simd_lane_count(tensor_dtype_t dtype);

/* ---- activations & normalization: reference kernels.h:173-207 ---- */
float silu(float x);                                                  /* x / (1 + e^-x), activations.c:16-20 */
float relu(float x);                                                  /* activations.c:37-39 */
float gelu(float x);                       /* 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))), :64-76 */
float geglu(float x, float y);                                        /* x * gelu(y), :103-105 */
void gelu_inplace(float *x, int n);                                   /* activations.c:78-82 */
int sapphire_geglu(float *output, const float *input, size_t size);  /* [x|y] -> x*gelu(y); -1 on bad args */
void silu_inplace(float *x, int n);                                   /* activations.c:22-26 */
void relu_inplace(float *x, int n);                                   /* activations.c:41-45 */

/* out = (in / rms) * w and out = (in / rms) * (1 + w), rms = sqrt(mean(in^2) + eps);
 * -1 on NULL, dim <= 0 or eps < 0 (normalization.c:89-160). */
int rmsnorm(float *out, const float *in, const float *weight, float epsilon, int dim);
int rmsnorm_delta(float *out, const float *in, const float *weight, float epsilon, int dim);
int rmsnorm_batch(float *out, const float *in, const float *weight, float epsilon, int batch_size, int dim);

void softmax(float *scores, int n);                                   /* utils.c:18-59 */
void vec_softcap(float *x, int n, float cap);                         /* utils.c:119-125 */

/* ---- vector math: reference kernels.h:213-222 ---- */
void vec_add(float *dst, const float *src, int n);
void vec_scale(float *x, float s, int n);
void vec_copy(float *dst, const float *src, int n);
float vec_dot(const float *a, const float *b, int n);
void bf16_to_f32_vec(float *dst, const uint16_t *src, int n);
const float *get_norm_weights(const tensor_t *weight, float *scratch, int n);

/* ---- legacy aliases: reference kernels.h:228-238 ---- */
#define sapphire_context_create kernel_ctx_create
#define sapphire_context_destroy kernel_ctx_destroy
#define tensor_gemv_ctx_create kernel_ctx_create
#define tensor_gemv_ctx_destroy kernel_ctx_destroy
#define tensor_gemv_with_ctx kernel_gemv
#define tensor_gemm_with_ctx kernel_gemm
#define tensor_gemv_tensor_with_ctx kernel_gemv_tensor
#define tensor_gemv_add_with_ctx kernel_gemv_add
#define tensor_gemv_batch_with_ctx kernel_gemv_batch
#define tensor_gemv_simd_lane_count_for_dtype kernel_get_simd_lane_count
#define sapphire_batched_gemv kernel_gemv

#ifdef __cplusplus
}
#endif
#endif /* KERNELS_H */
