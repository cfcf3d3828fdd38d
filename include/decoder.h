/*
 * decoder.h - device-resident decode (greedy or temperature-sampled) of a Gemma-3-shaped
 * model on one MI355X.
 *
 * The reference runs a decode step as inference_forward (src/inference/inference.c:612-651):
 * sapphire_embed_lookup, then sapphire_transformer_layer for every layer (attention stage
 * attention.c:311-375, FFN stage transformer.c:96-171, finalize transformer.c:211-283),
 * then lm_head (transformer.c:393-408) and sample_greedy / sample_temperature (utils.c:145-180),
 * calling kernel_gemv and the vector primitives with host buffers. The library also exports
 * those transformer.h entry points on the engine's own session (one PCIe round trip per layer
 * call). This engine is the MI355X-native form of the whole step: weights, activations, the KV
 * cache and the sampled token stay in HBM, and one step is a captured HIP graph of fused
 * kernels. The host engine keeps its model loader and session and hands the weights over once
 * (sapphire_decoder_create below).
 *
 * Not a reference interface: the reference has no device engine. Semantics follow the
 * functions cited above; weights are the reference's Q4_0 / Q8_0 block arrays
 * (kernels.h:29-38), rows = outputs, exactly as the reference's tensor views hold them.
 */
#ifndef SAPPHIRE_HIP_DECODER_H
#define SAPPHIRE_HIP_DECODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    int sliding_window;             /* local layers' window; <= 0 -> 1024 (attention.c:113) */
    unsigned long long global_mask; /* bit l set -> layer l is global; 0 -> (l+1) % 6 == 0 */
    float query_pre_attn_scalar;    /* scores scaled by 1/sqrt(this); <= 0 -> head_dim (attention.c:129) */
    float rope_theta;               /* RoPE base of global layers (inference.c:477-483) */
    float rope_local_base;          /* RoPE base of local layers (inference.c:485-491) */
    float eps;                      /* RMSNorm epsilon; the reference uses 1e-6 everywhere */
    int wdtype;                     /* DTYPE_Q4_0 (3) or DTYPE_Q8_0 (4): the seven projections */
    int lm_dtype;                   /* DTYPE_Q4_0 or DTYPE_Q8_0: a separate LM head; DTYPE_BF16 (1):
                                     * the LM head is the embedding table (weight tying, as
                                     * lm_head does, transformer.c:393-408) */
} sapphire_decoder_config_t;

/* Host pointers, read once by sapphire_decoder_create. Projection arrays hold one pointer
 * per layer to that layer's block array ([rows][ceil(K/32)] blocks): wq [H*hd x hidden],
 * wk/wv [n_kv*hd x hidden], wo [hidden x H*hd], wgate/wup [ffn x hidden], wdown [hidden x ffn].
 * Norm weights are applied as (1 + w) (normalization.c:104-117); q_norm and k_norm are
 * head_dim long and shared by every head (attention.c:228-269). They are fp32, or, with
 * norm_dtype DTYPE_BF16, bf16 values (uint16_t arrays behind the same pointers, as a
 * safetensors checkpoint stores them), widened exactly as get_norm_weights does
 * (utils.c:218-225). */
typedef struct {
    const void *const *wq, *const *wk, *const *wv, *const *wo, *const *wgate, *const *wup, *const *wdown;
    const float *const *norm_attn, *const *norm_attn_post, *const *norm_ffn, *const *norm_ffn_post;
    const float *const *q_norm, *const *k_norm;
    const uint16_t *embed_bf16;     /* [vocab][hidden] bf16, scaled by sqrt(hidden) on lookup */
    const float *norm_final;        /* [hidden] */
    const void *lm_head;            /* [vocab][hidden] blocks of lm_dtype; ignored for DTYPE_BF16 */
    int norm_dtype;                 /* DTYPE_F32 (0) or DTYPE_BF16 (1): the element type of every norm
                                     * array above (norm_*, q_norm, k_norm, norm_final) */
} sapphire_decoder_weights_t;

typedef struct sapphire_decoder sapphire_decoder_t;

/* Uploads the weights to the current device (NULL on error; sapphire_last_error()). */
sapphire_decoder_t *sapphire_decoder_create(const sapphire_decoder_config_t *cfg,
                                            const sapphire_decoder_weights_t *w);
void sapphire_decoder_destroy(sapphire_decoder_t *dec);

/* The KV caches as [n_layers][n_kv_heads][max_ctx][head_dim] fp32 (kv_cache.c:101-106);
 * for a batched decoder [batch][n_layers][n_kv_heads][max_ctx][head_dim]. */
int sapphire_decoder_set_kv(sapphire_decoder_t *dec, const float *k, const float *v);
int sapphire_decoder_get_kv(sapphire_decoder_t *dec, float *k, float *v);

/* Decode: `steps` steps starting with `token` at position `pos`; step s feeds tokens_out[s-1]
 * back (token for s = 0). tokens_out[steps] receives every step's token: the greedy one (the
 * lowest index among equal maxima), or the sampled one (sapphire_decoder_set_sampling). logits_out, if not NULL, receives [steps][vocab] logits
 * (copied back after each step, which costs time). elapsed_ms, if not NULL, receives the
 * device time of the steps (HIP events on the decoder's stream). A call without logits_out on
 * the persistent step launches sixteen steps per captured graph where they fit. 0 / -1. */
int sapphire_decoder_generate(sapphire_decoder_t *dec, int token, int pos, int steps, int *tokens_out,
                              float *logits_out, float *elapsed_ms);

/* Prefill: tokens[0..n) at positions pos..pos+n-1 of sequence `seq` (0 for a one-sequence
 * decoder) run through every layer and leave their K/V rows in that sequence's cache, as
 * inference_forward_batch does for a prompt without logits (inference.c:236-244, 616-651:
 * every row of a chunk is written before its attention reads any, attention.c:292-309).
 * Chunks of up to 16 tokens run their projections as one matrix-core GEMM. No logits; the
 * next call is sapphire_decoder_generate with the prompt's last token at pos + n.
 * Needs hidden, n_heads*head_dim and ffn multiples of 128 and hidden <= 1152 (-1
 * otherwise). elapsed_ms, if not NULL, receives the device time. 0 / -1. */
int sapphire_decoder_prefill(sapphire_decoder_t *dec, int seq, const int *tokens, int n, int pos,
                             float *elapsed_ms);
/* The form of a one-sequence step. groups > 0: the layers run as one persistent kernel of
 * `groups` workgroups (all co-resident) whose stages exchange epoch-tagged vectors
 * instead of waiting for kernel boundaries; this is the default (128 workgroups, or the value
 * of the SAPPHIRE_DECODE_WORKGROUPS environment variable at create time) where the shapes and
 * the device allow it. groups == 0: six fused launches per layer in a HIP graph. Both forms
 * compute the same step. Returns -1 (and keeps the current form) when `groups` cannot run
 * these shapes on this device, and for a batched decoder. */
int sapphire_decoder_set_workgroups(sapphire_decoder_t *dec, int groups);
/* The current form: workgroups of the persistent step, 0 for the multi-launch step. */
int sapphire_decoder_workgroups(const sapphire_decoder_t *dec);
/* No counterpart in the reference; for tests of the persistent step and the batched step. The
 * persistent step's stages tag exchanged values with epochs (steps since the last reset x 8 x
 * (n_layers + 1) + stage) that must stay below 2^32; the batched step's fused QKV + attention
 * launch tags its q | k | v words with (steps since the last reset + 1) x 64 + layer + 1, whose
 * step count must stay below 2^26 - 1. generate starts them over (clearing every tagged word)
 * before a call would pass that. This sets the count of steps since the last reset, on the
 * device and the host, as if that many steps had run: a test can start just below the reset
 * and decode across it. No effect on the multi-launch step. 0 / -1 (count past the range). */
int sapphire_decoder_set_epoch_count(sapphire_decoder_t *dec, uint32_t steps);

/* How the following generate calls pick tokens (inference.c:262-266 and 297). temperature <= 0
 * (the default): greedy, sample_greedy (utils.c:145-156). temperature > 0: each step scales
 * its logits by 1.0f / temperature and draws as sample_temperature (utils.c:158-180), bit for
 * bit, with draws[s * batch + b] in place of (float)rand() / RAND_MAX for step s of a call and
 * sequence b; n_draws of them are copied here (at most max_ctx * batch), and a call may run at
 * most n_draws / batch steps. logits_out still receives the unscaled logits. The vocabulary
 * must be at most 2^21. NaN temperatures are rejected. 0 / -1. */
int sapphire_decoder_set_sampling(sapphire_decoder_t *dec, float temperature, const float *draws, int n_draws);

/* Stop tokens for the following generate calls (none by default; n = 0 clears them). The
 * reference's generation loop ends when it samples 1 (<eos>) or 106 (<end_of_turn>)
 * (inference.c:298-301); a host that mirrors it sets {1, 106}. On the device, the step that
 * picks a stop token logs it to tokens_out and marks its sequence done; every later step of
 * that sequence logs -1, leaves its position and its KV cache unchanged and, for a
 * one-sequence decoder, returns at once from its layers and its greedy LM head (the
 * multi-launch step and a batch whose other sequences go on still run their kernels). The
 * logits of such steps are unspecified. At most 8 tokens, each in [0, vocab). 0 / -1. */
int sapphire_decoder_set_stop_tokens(sapphire_decoder_t *dec, const int *ids, int n);

/* ---- batched decode ----
 * `batch` (2..16) independent sequences decoded in lock step, each with its own KV cache,
 * position and token: one step runs every projection as one matrix-core GEMM over
 * the batch (the reference decodes one sequence per inference_forward call). Shapes:
 * hidden, n_heads*head_dim and ffn multiples of 128, hidden <= 1152. Weights as for
 * sapphire_decoder_create. A decoder made by sapphire_decoder_create has batch 1; the
 * functions below accept it too. For Q4_0 projections, 4..16 sequences and the head shapes
 * of the Gemma-3 family, each layer's QKV GEMM and attention run as one launch (its
 * attention workgroups stream their K/V rows while the GEMM's workgroups run, then take
 * q | k | v from tagged words); the environment variable SAPPHIRE_FUSED_QKV_ATTN=0 at create
 * time keeps them two launches. Both forms compute the same step. */
sapphire_decoder_t *sapphire_decoder_create_batch(const sapphire_decoder_config_t *cfg,
                                                  const sapphire_decoder_weights_t *w, int batch);
int sapphire_decoder_batch(const sapphire_decoder_t *dec);
/* The KV caches of sequence `seq`, [n_layers][n_kv_heads][max_ctx][head_dim] fp32.
 * sapphire_decoder_set_kv / get_kv move all sequences at once, [batch][n_layers]... */
int sapphire_decoder_set_kv_seq(sapphire_decoder_t *dec, int seq, const float *k, const float *v);
int sapphire_decoder_get_kv_seq(sapphire_decoder_t *dec, int seq, float *k, float *v);
/* tokens[batch] and pos[batch] start every sequence; tokens_out receives [steps][batch]
 * tokens (greedy or sampled); logits_out, if not NULL, [steps][batch][vocab]. */
int sapphire_decoder_generate_batch(sapphire_decoder_t *dec, const int *tokens, const int *pos, int steps,
                                    int *tokens_out, float *logits_out, float *elapsed_ms);

#ifdef __cplusplus
}
#endif
#endif /* SAPPHIRE_HIP_DECODER_H */
