/*
 * sapphire_hip.h - device-pointer, stream-ordered API of libsapphire_hip.so.
 *
 * kernels.h keeps the reference's synchronous host-pointer contract. This header is the
 * MI355X-native layer beneath it: every operation takes device pointers and a HIP stream
 * (passed as void*; NULL = the null stream) and only enqueues work, so a host engine can
 * keep activations, logits and the KV cache resident in HBM and capture a whole decode
 * step in a hipGraph. All functions return 0 on success and -1 on bad arguments or a HIP
 * error (message via sapphire_last_error()).
 *
 * None of these entry points exists in the reference; each names the reference routine
 * whose semantics it implements.
 */
#ifndef SAPPHIRE_HIP_H
#define SAPPHIRE_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes are tensor_dtype_t's: F32 0, BF16 1, F16 2, Q4_0 3, Q8_0 4 */
enum { SAPPHIRE_F32 = 0, SAPPHIRE_BF16 = 1, SAPPHIRE_F16 = 2, SAPPHIRE_Q4_0 = 3, SAPPHIRE_Q8_0 = 4 };

/* Weight layouts in device memory for Q4_0/Q8_0.
 *  AOS    : the reference block array, rows contiguous, row stride ceil(K/32)*B_blk
 *           (B_blk 20 for Q4_0, 36 for Q8_0; include/kernels.h:29-38).
 *  PACKED : the same quants and scales split in two planes, built by
 *           sapphire_q_repack_dev: quants [M][nb][16|32] bytes (byte order of the
 *           reference block), then, at offset sapphire_q_scales_offset(), fp32
 *           scales [M][nb]. Values are bit-identical; only their placement differs.
 *  TILED  : the matrix-core layout (K a multiple of 128): 16-row tiles, 4-block groups,
 *           each group's quants stored in the order the MFMA operand registers of a wave
 *           take them (one contiguous KiB per load instruction), then fp32 scales
 *           [tile][group][block][row]. Rows past M are zero. The batch-1 GEMV runs on it
 *           for K/128 in {5, 8, 9}; the batched GEMM for every K. */
enum { SAPPHIRE_LAYOUT_AOS = 0, SAPPHIRE_LAYOUT_PACKED = 1, SAPPHIRE_LAYOUT_TILED = 2 };

const char *sapphire_last_error(void);
const char *sapphire_version(void);

/* ---- device memory / streams / events (thin wrappers over the HIP runtime) ---- */
int sapphire_device_count(void);
int sapphire_set_device(int device);
void *sapphire_malloc(size_t bytes);                 /* NULL on failure */
int sapphire_free(void *dev_ptr);
int sapphire_memcpy_h2d(void *dst_dev, const void *src_host, size_t bytes);
int sapphire_memcpy_d2h(void *dst_host, const void *src_dev, size_t bytes);
int sapphire_memcpy_d2d(void *dst_dev, const void *src_dev, size_t bytes, void *stream);
int sapphire_memset(void *dev_ptr, int value, size_t bytes);
int sapphire_synchronize(void);
void *sapphire_stream_create(void);                  /* default priority, non-blocking */
int sapphire_stream_destroy(void *stream);
int sapphire_stream_synchronize(void *stream);
void *sapphire_event_create(void);
int sapphire_event_destroy(void *event);
int sapphire_event_record(void *event, void *stream);
int sapphire_event_synchronize(void *event);
float sapphire_event_elapsed_ms(void *start, void *stop);   /* < 0 on error */

/* ---- quantized weights ---- */
size_t sapphire_q_aos_bytes(int dtype, int M, int K);
size_t sapphire_q_packed_bytes(int dtype, int M, int K);
size_t sapphire_q_scales_offset(int dtype, int M, int K);
/* AOS -> PACKED (both on device). */
int sapphire_q_repack_dev(int dtype, const void *w_aos, int M, int K, void *w_packed, void *stream);
/* Bytes of an M x K matrix in `layout` (0 if the layout cannot hold it), and the
 * conversion of an on-device AOS array into PACKED or TILED. */
size_t sapphire_q_layout_bytes(int dtype, int layout, int M, int K);
int sapphire_q_convert_dev(int dtype, const void *w_aos, int M, int K, int layout, void *out, void *stream);
/* Integer weight values (nib-8 or q) of every element, [M][nb*32] int8: the unpack
 * of q4_0_avx.c:61-66 / q8_0_avx.c:45-56. */
int sapphire_q_unpack_ints_dev(int dtype, int layout, const void *w, int M, int K, int8_t *out, void *stream);
/* Dequantised weights fl(int * scale), [M][nb*32] f32: q4_0_avx.c:38-40, q8_0_avx.c:50-59. */
int sapphire_q_dequant_dev(int dtype, int layout, const void *w, int M, int K, float *out, void *stream);

/* y[M] = W[M,K] . x[K]  (kernel_gemv semantics, dispatch.c:101-156). K must be a
 * multiple of 32 for Q4_0/Q8_0 (callers pad activations, as the reference's session
 * scratch does; inference.c:377-394). */
int sapphire_gemv_q_dev(int dtype, int layout, const void *w, int M, int K,
                        const float *x, float *y, void *stream);
/* y[M] = W[M,K] . x[K] for F32 or BF16 row-major W (f32_avx.c:44-83, bf16_avx.c:55-108). */
int sapphire_gemv_f_dev(int dtype, const void *w, int M, int K, const float *x, float *y, void *stream);
/* Y[b][r] = W[r,:] . X[b][:] for BF16 row-major W and `batch` fp32 vectors (rows of X with
 * stride ldx, rows of Y with stride ldy), on the matrix cores in passes of 16 vectors: the
 * batched form kernel_gemm_bf16_avx2 computes (bf16_avx.c:115-159). Needs K % 8 == 0, W
 * 16-byte aligned and M*K*2 below 4 GiB. */
int sapphire_gemm_bf16_dev(const void *w, int M, int K, const float *x, int ldx, int batch, float *y, int ldy,
                           void *stream);

/* Y[b][M] = W[M,K] . X[b][K] for b < batch: the batched GEMV of kernel_gemm /
 * kernel_gemv_batch (dispatch.c:87-99, 234-266) for Q4_0/Q8_0, which the reference
 * itself rejects (pool.c:318-321); its meaning is `batch` independent kernel_gemv calls.
 * X and Y are row-major [batch][K] / [batch][M]. On the TILED layout the rows run on the
 * fp16 matrix cores, 16 sequences per pass (longer batches loop), with `ws` holding
 * sapphire_gemm_workspace_bytes(dtype, M, K) bytes of device memory (K-split partial
 * sums); calls that share a workspace must be ordered on one stream. On AOS/PACKED it is
 * the vector kernel and ws may be NULL. */
size_t sapphire_gemm_workspace_bytes(int dtype, int M, int K);
int sapphire_gemm_q_dev(int dtype, int layout, const void *w, int M, int K, const float *X, int batch,
                        float *Y, void *ws, void *stream);

/* The batched LM head with the greedy pick fused: tokens[b] (device) = sample_greedy of
 * W . X[b] (utils.c:145-156: the first index of the maximum; 0 when row 0 is NaN or no row
 * is above -inf), for TILED weights with K <= 1152. The rows are formed as
 * sapphire_gemm_q_dev forms them but never stored: each workgroup keeps the best row per
 * sequence of the tiles it multiplies and leaves one partial in ws, and one short kernel picks
 * the tokens. ws as for sapphire_gemm_q_dev. batch <= 16. */
int sapphire_gemm_q_greedy_dev(int dtype, const void *w_tiled, int M, int K, const float *X, int batch,
                               int *tokens, void *ws, void *stream);

/* The batched GEMM with its input and output transforms, for a host engine that runs a
 * batched decode step (TILED weights only). Per sequence row b the input is formed while
 * the activations are staged:
 *   d = sum of the `nparts` rows parts[c * part_stride + b * ldp + k] (when parts is set),
 *   d = rmsnorm_delta(d, w_delta) when w_delta is set; h = x[b * ldx + k] (+ d);
 *   resid_out[b * ldr + k] = h when resid_out is set;
 *   input = rmsnorm_delta(h, w_norm) when w_norm is set, else h
 * (the residual of attention.c:356-366 / transformer.c:231-239 and the pre-norms of
 * attention.c:316-325 / transformer.c:119-121; rmsnorm_delta of normalization.c:104-117).
 * The residual's norm sums its squares in the reference's order (sum_sq_avx2,
 * normalization.c:12-32), so resid_out is the reference's bit for bit; the pre-norm's sum is a
 * tree over the row, whose last bits may differ from that order.
 * The norms need whole rows: K <= 1152 when w_delta or w_norm is set. Output: with
 * out.parts set, the K chunks' partial sums are left in parts[c][b][M] (c < the number
 * sapphire_gemm_splits(K) returns) for the next call's input; else y[b * ldy + r]. With
 * out.geglu, W's rows are gate and up rows interleaved by eight and y[b * ldy + j] =
 * gelu(gate_j) * up_j for j < M/2 (transformer.c:141-157). Pointers 16-byte aligned,
 * leading dimensions multiples of 4; ws as for sapphire_gemm_q_dev (NULL allowed when
 * K <= 1152 or out.parts is set). batch <= 16.
 * Block order (x_blocked, y_blocked): a vector set of 16 slots in which element k of
 * sequence b sits at (k / 32) * 512 + ((k / 8) % 4) * 128 + b * 8 + k % 8 (16 * K floats,
 * ldx / ldy unused), the order of the matrix-core operands, so a GEMM reads it with
 * contiguous loads. x_blocked only for a plain x (no parts, norms or resid_out); y_blocked
 * only when K <= 1152 and out.parts is unset (with geglu, over the M/2 outputs). A step
 * passes the GeGLU output to the down projection this way. */
typedef struct {
    const float *x;
    int ldx;
    const float *parts;
    int nparts, ldp;
    size_t part_stride;
    const float *w_delta;
    float *resid_out;
    int ldr;
    const float *w_norm;
    float eps;
    int x_blocked;
} sapphire_gemm_input_t;
typedef struct {
    float *y;
    int ldy;
    float *parts;
    int geglu;
    int y_blocked;
} sapphire_gemm_output_t;
int sapphire_gemm_splits(int K);
int sapphire_gemm_q_fused_dev(int dtype, const void *w_tiled, int M, int K, int batch, const sapphire_gemm_input_t *in,
                              const sapphire_gemm_output_t *out, void *ws, void *stream);

/* ---- LM-head epilogue ----
 * probs = softmax(logits) (utils.c:18-59) written to probs (may equal logits) and the
 * greedy token (utils.c:145-156: the first index of the maximum; 0 when logits[0] is NaN)
 * written to *argmax_dev. probs may be NULL to compute only the argmax. The partials use a
 * small per-device buffer (allocated on the device's first call): calls that overlap on one
 * device must be ordered on one stream. */
int sapphire_softmax_argmax_dev(const float *logits, int n, float *probs, int *argmax_dev, void *stream);

/* The LM head with its epilogue fused: logits = W . x as sapphire_gemv_q_dev, then probs
 * and the greedy token as sapphire_softmax_argmax_dev. On the TILED layout the GEMV's
 * workgroups leave (max, sum exp, argmax) partials and one short kernel finishes the
 * softmax, instead of two more passes over the logits. probs may be NULL (argmax only)
 * or equal logits. The partials use a small per-device buffer: calls that overlap on one
 * device must be ordered on one stream. */
int sapphire_gemv_softmax_dev(int dtype, int layout, const void *w, int M, int K, const float *x, float *logits,
                              float *probs, int *argmax_dev, void *stream);

/* sapphire_gemv_softmax_dev for callers that cannot allocate device memory (code under HIP
 * graph capture, fixed serving loops, hosts that forbid hipMalloc). No counterpart in the
 * reference. Same arguments, results and kernels; the reduction partials live in a fixed
 * 64 KiB array of the library's device code (one per GPU, kept until the process ends), so
 * nothing is allocated or freed. The array's device address is looked up on a device's first
 * call: make that call once before capturing. Sizes needing more partials than the array
 * holds are rejected (-1) before any launch; the TILED layout needs K/128 in {5, 8, 9}. Calls
 * that overlap on one GPU share the array and race: order them on one stream. */
int sapphire_gemv_softmax_noalloc_dev(int dtype, int layout, const void *w, int M, int K, const float *x,
                                      float *logits, float *probs, int *argmax_dev, void *stream);

/* ---- the next token ----
 * The next token of each of `batch` rows of logits (row b at logits + b * ld, ld >= n) as
 * perform_inference draws it (inference.c:262-266 and 297): temperature <= 0 gives
 * sample_greedy (utils.c:145-156); otherwise each row is scaled by 1.0f / temperature
 * (vec_scale, utils.c:87-92) and sample_temperature (utils.c:158-180) draws its token with
 * draws_dev[b] in place of (float)rand() / RAND_MAX. The result is the reference's token bit
 * for bit (its float sums included). As there, a sampled row is overwritten with the weights
 * expf((l / T - max) / T); a NaN or +inf among the scaled logits gives n - 1. tokens_dev[b]
 * receives the token. workspace: sapphire_sample_workspace_bytes(n, batch) bytes of device
 * memory (256-byte aligned, per-chunk sums and maps); calls sharing one must be ordered.
 * 1 <= n <= 2^21. */
size_t sapphire_sample_workspace_bytes(int n, int batch);
int sapphire_sample_dev(float *logits, int n, int batch, int ld, float temperature, const float *draws_dev,
                        int *tokens_dev, void *workspace, void *stream);

/* ---- device copies of tensor_t weights ----
 * The device-resident copy kernel_gemv keeps for a 2-D weight tensor (Q4_0/Q8_0 in the
 * PACKED layout, F32/BF16 as is), created on first use; *layout receives its layout.
 * NULL on error. sapphire_tensor_invalidate drops it (call after changing host data). */
const void *sapphire_tensor_device_data(const tensor_t *t, int *layout, void *stream);
int sapphire_tensor_invalidate(tensor_t *t);

/* ---- primitives on device vectors ---- */
/* out[b] = rmsnorm_delta(in[b]) for b < batch, rows of length dim (normalization.c:104-117). */
int sapphire_rmsnorm_delta_dev(float *out, const float *in, const float *w, float eps, int dim, int batch, void *stream);
int sapphire_rmsnorm_dev(float *out, const float *in, const float *w, float eps, int dim, int batch, void *stream);
/* Half-split rotation of n_heads consecutive heads at position pos (rope.c:99-117). */
int sapphire_rope_apply_dev(float *x, int n_heads, int head_dim, int pos,
                            const float *cos_table, const float *sin_table, void *stream);
/* gate[i] = gelu(gate[i]) * up[i] (transformer.c:150-157, activations.c:64-82). */
int sapphire_gelu_mul_dev(float *gate, const float *up, int n, void *stream);
/* Residual pattern n = rmsnorm_delta(h, w); resid += n; h = resid
 * (attention.c:358-366, transformer.c:231-239). */
int sapphire_norm_residual_dev(float *hidden, float *resid, const float *w, float eps, int dim, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* SAPPHIRE_HIP_H */
