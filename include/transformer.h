/*
 * transformer.h - the engine-level decode API of libsapphire_hip.so (MI355X, gfx950).
 *
 * Drop-in for the reference's include/transformer.h: the same types and entry points, taking
 * the engine's own inference_session_t (inference.h), so the engine's inference_forward /
 * inference_forward_batch (inference.c:612-651) run their layers on the GPU unchanged. The
 * library replaces src/transformer/transformer.c and attention.c as a whole.
 *
 * Per session the library keeps device state, built on the first call: the projections (the
 * device copies kernel_gemv keeps for each tensor_t), the norm weights, the RoPE tables the
 * engine passes, and a mirror of the engine's KV cache (uploaded once; every K/V row a call
 * writes is also written back to the engine's cache). A call moves only its hidden vectors,
 * positions / tokens and logits across PCIe. The state is dropped when the engine releases the
 * session's KV cache (destroy_inference_session) or by sapphire_transformer_session_release.
 * The engine's kv_cache_get_keys / kv_cache_get_values must be visible to the library (an
 * executable linked with it exports them).
 *
 * Supported models: Q4_0 / Q8_0 projections sharing one dtype, every norm weight present
 * (F32 or BF16), QK-norm gammas of head_dim elements (broadcast over the heads), a BF16
 * embedding table (also the LM head, as lm_head computes it), hidden size up to 2048. A call
 * on another model returns -1 (or, for the void entry points, leaves its outputs unwritten)
 * with the reason in sapphire_last_error().
 */
#ifndef TRANSFORMER_H
#define TRANSFORMER_H

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "llm_model.h"            /* the engine's headers */
#include "gemma3_270m_config.h"

#ifdef __cplusplus
extern "C" {
#endif

struct inference_session_t;

typedef struct {
    const float *cos;
    const float *sin;
} transformer_rope_t;

/* One decoder layer for the token at token_pos: hidden [d_model] in, the layer's output out
 * (transformer.c:289-316). The token's K/V rows are written to the session's cache. 0 / -1. */
int sapphire_transformer_layer(struct inference_session_t *session, int layer_idx, int token_pos, float *hidden,
                               transformer_rope_t rope);

/* The same for batch_size (<= 32) tokens of one sequence at start_pos.. (rows d_model apart):
 * each token attends to the positions up to its own (transformer.c:318-345). */
int sapphire_transformer_layer_batch(struct inference_session_t *session, int layer_idx, int start_pos,
                                     int batch_size, float *hidden, transformer_rope_t rope);

/* hidden = bf16 embedding row of token_id times sqrtf(d_model) (no scale when the environment
 * sets SAPPHIRE_NO_EMBED_SCALE), transformer.c:347-380. */
void sapphire_embed_lookup(struct inference_session_t *session, int token_id, float *hidden);
void sapphire_embed_lookup_batch(struct inference_session_t *session, const int *token_ids, int batch_size,
                                 float *hidden);

/* logits [vocab] = embedding_weight . rmsnorm_delta(hidden, norm_final) (transformer.c:393-408). */
void lm_head(struct inference_session_t *session, const float *hidden, float *logits);

typedef struct layer_buffers {
    int pm, pi, pk, pf;
    int batch_size;
    float *residual, *norm_buf, *q_proj, *k_proj, *v_proj;
    float *attn_out, *ffn_gate_buf, *ffn_value_buf, *geglu_buf;
    float *weight_scratch;
} layer_buffers_t;

typedef struct transformer_layer_ctx {
    struct inference_session_t *session;
    model_layer_weights_t *layer;
    gemma3_270m_config_t *config;
    int layer_idx;
    int token_pos;
    int batch_size;
    int d_model;
    int head_dim;
} transformer_layer_ctx_t;

/* The stages of a layer on the engine's host buffers (attention.c:311-375, transformer.c:96-283):
 * attention: buf.residual <- hidden, hidden <- residual + post-norm(o-proj(attention));
 * ffn: hidden <- down(gelu(gate(n)) * up(n)), n = pre-norm(buf.residual);
 * finalize: buf.residual += post-norm(hidden), hidden <- buf.residual.
 * The other scratch buffers of buf are not written. */
void compute_attention_stage(layer_buffers_t buf, transformer_layer_ctx_t *ctx, float *hidden,
                             const float *rope_cos, const float *rope_sin);
void compute_ffn_stage(layer_buffers_t buf, transformer_layer_ctx_t *ctx, float *hidden);
void finalize_layer_output(layer_buffers_t buf, transformer_layer_ctx_t *ctx, float *hidden);
/* Placeholders in the reference (transformer.c:422-450): a warning, no computation. */
void compute_linear_attention_stage(layer_buffers_t buf, transformer_layer_ctx_t *ctx, float *hidden,
                                    const float *rope_cos, const float *rope_sin);
void compute_ssm_stage(layer_buffers_t buf, transformer_layer_ctx_t *ctx, float *hidden);

/* Drops the session's device state now (it is also dropped when the engine releases the
 * session's KV cache). No counterpart in the reference. 0. */
int sapphire_transformer_session_release(struct inference_session_t *session);

#ifdef __cplusplus
}
#endif

#endif /* TRANSFORMER_H */
