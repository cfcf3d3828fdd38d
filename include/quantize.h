/*
 * quantize.h - the producer of Q4_0 / Q8_0 weights.
 *
 * The reference reads Q4_0 / Q8_0 block arrays (kernels.h:29-38) but has no function that
 * makes them: its loader yields F32 / BF16 tensors only (safetensors_reader.c:406-449) and
 * tensor_create makes no blocks (tensor.c:108-110). These entry points have no counterpart
 * in the reference; they are for the host engine's load path, which turns the F32 / BF16
 * projection and LM-head tensors of a checkpoint into the blocks kernel_gemv and the device
 * decoder consume.
 *
 * Algorithm: ggml's reference quantizer (quantize_row_q8_0_ref / quantize_row_q4_0_ref, the
 * library whose block structs the reference uses) with the reference's fp32 block scale and
 * its Q4_0 nibble order (element 2j in the low nibble of byte j, 2j+1 in the high nibble,
 * q4_0_avx.c:61-66):
 *   Q8_0: amax = max|x|; d = amax / 127; id = d ? 1/d : 0; q = roundf(x * id).
 *   Q4_0: max = the first x of largest |x| (+0 when all are zero); d = max / -8;
 *         id = d ? 1/d : 0; q = min(15, trunc(x * id + 8.5)).
 * Rows [M][K] become [M][ceil(K/32)] blocks; elements past K in a row's last block are zeros.
 * Inputs must be finite. A block whose scale is subnormal, so that 1/d overflows, saturates
 * infinite products to the largest code and codes NaN ones (0 * inf) as zero. 0 on success, -1 on bad arguments or a device error
 * (sapphire_last_error()).
 */
#ifndef SAPPHIRE_HIP_QUANTIZE_H
#define SAPPHIRE_HIP_QUANTIZE_H

#include "kernels.h"
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Host pointers, synchronous (the kernels.h contract): src is a 2-D F32 or BF16 tensor
 * [M, K]; blocks receives M * ceil(K/32) blocks of `dtype` (DTYPE_Q4_0 or DTYPE_Q8_0),
 * 20 or 36 bytes each. ctx may be NULL (the library's default context). */
int kernel_quantize(kernel_context_t *ctx, void *blocks, tensor_dtype_t dtype, const tensor_t *src);

/* Device pointers, enqueued on `stream` (NULL = the null stream): src_dtype 0 (F32) or
 * 1 (BF16) rows [M][K] into M * ceil(K/32) blocks of dst_dtype 3 (Q4_0) or 4 (Q8_0) at
 * `blocks` (4-byte aligned), the AOS layout of sapphire_hip.h. */
int sapphire_quantize_dev(int dst_dtype, int src_dtype, const void *src, int M, int K, void *blocks,
                          void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SAPPHIRE_HIP_QUANTIZE_H */
