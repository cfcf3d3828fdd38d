/*
 * rope.h - rotary positional embedding API of libsapphire_hip.so (MI355X, gfx950).
 *
 * Drop-in for the reference's include/rope.h: the same types, names and argument meanings.
 * The library provides the four functions of the reference's src/transformer/rope.c:
 *   rope_precompute_freqs   (rope.c:41-63)  host tables, the reference's libm formula
 *   rope_apply_fast         (rope.c:99-117) half-split rotation, on the GPU
 *   apply_rope              (rope.c:17-25)  interleaved-pair rotation with the RoPE
 *                                           strategy's angles, on the GPU
 *   apply_rope_default      (rope.c:34-36)  apply_rope with base 1e6
 * The pluggable strategy interface (apply_positional_encoding, rope_encoding_strategy,
 * alibi_encoding_strategy; positional_encoding.c) is not on the decode path: it stays in the
 * engine's own positional_encoding.c and is declared here so that file compiles unchanged.
 */
#ifndef ROPE_H
#define ROPE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- strategy interface: reference rope.h:20-72 (defined by the engine) ---- */
typedef void (*PositionalEncodingStrategy)(int head_dim, int dim_pair, int pos, void *user_data, float *out_cos,
                                           float *out_sin);

void apply_positional_encoding(float *x, int pos, int head_dim, PositionalEncodingStrategy strategy,
                               void *user_data);
void rope_encoding_strategy(int head_dim, int dim_pair, int pos, void *user_data, float *out_cos, float *out_sin);
void alibi_encoding_strategy(int head_dim, int dim_pair, int pos, void *user_data, float *out_cos, float *out_sin);

/* ---- provided by libsapphire_hip.so ---- */

/* x[2p], x[2p+1] rotated by theta_p = pos * (1/base)^(2p/head_dim) for every pair with
 * 2p + 1 < head_dim (rope.c:17-25 through positional_encoding.c:16-40,76-104). Host x; no-op
 * when x is NULL. */
void apply_rope(float *x, int pos, int head_dim, float base);
void apply_rope_default(float *x, int pos, int head_dim);        /* base 1e6 (rope.c:7,34-36) */

/* freqs_cos / freqs_sin [max_context_len][d_k]: for m < d_k/2, freq = 1/powf(base, 2m/d_k),
 * angle = pos * freq, cos/sin stored at m and m + d_k/2 (rope.c:41-63). Host arrays; -1 when
 * a pointer is NULL, else 0. */
int rope_precompute_freqs(float *freqs_cos, float *freqs_sin, int d_k, int max_context_len, float rope_base);

/* x[i] = x0 c - x1 s, x[i + half] = x1 c + x0 s with c, s from row pos of the tables
 * (rope.c:99-117). Host pointers; no-op when one is NULL. */
void rope_apply_fast(float *x, int pos, int head_dim, const float *freqs_cos, const float *freqs_sin);

#ifdef __cplusplus
}
#endif

#endif /* ROPE_H */
