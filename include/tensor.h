/*
 * tensor.h - opaque tensor carrier exported by libsapphire_hip.so.
 *
 * Drop-in for the reference's include/tensor.h: same enum values, same opaque type,
 * same function names, argument meanings and return conventions. The implementation
 * (sapphire_amd/csrc/tensor.cpp) replaces src/tensor/tensor.c; its private struct
 * additionally carries the device-resident copy of a weight tensor, created on the
 * first GPU operation that reads it and released with the tensor.
 *
 * Replaces (reference file:line):
 *   tensor_dtype_t / memory_layout_t ......... include/tensor.h:17-34
 *   tensor_t (opaque) ........................ include/tensor.h:40, src/tensor/tensor.c:8-17
 *   tensor_create / tensor_create_view ....... include/tensor.h:60,208; tensor.c:81-152
 *   tensor_clone / tensor_transpose .......... include/tensor.h:64-77; tensor.c:163-204
 *   accessors ................................ include/tensor.h:85-202; tensor.c:210-390
 *
 * The include guard is the reference's own (TENSOR_H): an engine translation unit that also
 * reaches the reference's tensor.h through a relative include sees one definition of the types.
 */
#ifndef TENSOR_H
#define TENSOR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    DTYPE_F32,   /* 32-bit float */
    DTYPE_BF16,  /* bfloat16 */
    DTYPE_F16,   /* IEEE half (no kernels, as in the reference) */
    DTYPE_Q4_0,  /* 20-byte blocks of 32 4-bit weights, fp32 scale */
    DTYPE_Q8_0,  /* 36-byte blocks of 32 int8 weights, fp32 scale */
} tensor_dtype_t;

typedef enum {
    LAYOUT_ROW_MAJOR,
    LAYOUT_COLUMN_MAJOR,
} memory_layout_t;

typedef struct tensor_t tensor_t;

/* Owning tensor, zero-initialised. Q4_0 holds ceil(numel/2) bytes and every other dtype
 * numel * dtype_element_size bytes, exactly as the reference (no room for block scales:
 * quantized weights are expected as views over block arrays). NULL on bad ndim/shape. */
tensor_t *tensor_create(int ndim, const int *shape, tensor_dtype_t dtype);

/* Non-owning view over caller memory (host memory, e.g. an mmap). nbytes is
 * numel * dtype_element_size, as in the reference (metadata only for block formats). */
tensor_t *tensor_create_view(tensor_dtype_t dtype, int ndim, const int *shape, void *data);

int tensor_transpose(const tensor_t *src, tensor_t **dst);   /* 2-D F32 only; 0 on success */
tensor_t *tensor_clone(const tensor_t *src);
size_t tensor_numel(const tensor_t *t);
size_t dtype_element_size(tensor_dtype_t dtype);              /* F32 4, BF16/F16 2, Q4_0/Q8_0 1 */
const char *dtype_name(tensor_dtype_t dtype);
float tensor_get_f32(const tensor_t *t, size_t idx);         /* F32 only; 0.0f otherwise */
int tensor_set_f32(tensor_t *t, size_t idx, float val);      /* F32 only; -1 otherwise */
void tensor_ref_inc(tensor_t *t);
void tensor_release(tensor_t *t);                            /* frees data unless a view */
void tensor_print_info(const tensor_t *t);
int tensor_ndim(const tensor_t *t);
const int *tensor_shape(const tensor_t *t);
const void *tensor_data(const tensor_t *t);
float *tensor_data_f32(const tensor_t *t);                   /* NULL unless F32 */
void *tensor_data_mutable(const tensor_t *t);
tensor_dtype_t tensor_dtype(const tensor_t *t);
size_t tensor_nbytes(const tensor_t *t);
int tensor_ref_count(const tensor_t *t);

#ifdef __cplusplus
}
#endif
#endif /* TENSOR_H */
