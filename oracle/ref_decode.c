/*
 * ref_decode.c - drives the compiled reference engine through one configurable
 * Gemma-3-shaped decode loop, for pinning the oracle's decode step.
 *
 * TEST INFRASTRUCTURE ONLY. Built by `make -C oracle ref` against the reference's own
 * headers and linked with oracle/_ref/libsapphire_ref.so (both compiled from the
 * reference sources); the output lives in oracle/_ref/ and is never shipped.
 *
 * Composition (reference public functions, in the reference's own order):
 *   inference_session_create(spec, max_ctx)            inference.c:499-584
 *   K/V prefill through kv_cache_get_keys/values         kv_cache.c:217-234
 *   per step:
 *     sapphire_embed_lookup(session, token, hidden)      transformer.c:347-365
 *     sapphire_transformer_layer(session, l, pos, ...)   transformer.c:289-316
 *       with the global/local RoPE table choice           inference.c:629-632
 *     rmsnorm_delta(final) + kernel_gemv(lm_head)         transformer.c:393-408
 *     sample_greedy                                      utils.c:145-156
 * lm_head() itself always projects through embedding_weight (transformer.c:407): a
 * BF16 (tied) LM head calls it; a quantized LM head is applied with the same two calls
 * lm_head makes, on a separate Q4_0/Q8_0 tensor view.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gemma3_270m_config.h"
#include "inference.h"
#include "kernels.h"
#include "kv_cache.h"
#include "llm_model.h"
#include "model_spec.h"
#include "tensor.h"
#include "transformer.h"
#include "utils.h"

typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    int sliding_window;
    unsigned long long global_mask;
    float query_pre_attn_scalar, rope_theta, rope_local_base;
    int wdtype, lm_dtype;
} ref_cfg_t;

typedef struct {
    /* each a concatenation over layers of the reference AoS block rows */
    const void *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;
    /* each [n_layers][len] f32 */
    const float *norm_attn, *norm_attn_post, *norm_ffn, *norm_ffn_post, *q_norm, *k_norm;
    int q_norm_len, k_norm_len;
    const uint16_t *embed_bf16;
    const float *norm_final;
    const void *lm_head;
} ref_weights_t;

static size_t row_bytes(int dtype, int k) { return (size_t)((k + 31) / 32) * (dtype == DTYPE_Q4_0 ? 20 : 36); }

static tensor_t *view2(int dtype, int rows, int cols, const void *data) {
    int shape[2] = { rows, cols };
    return tensor_create_view((tensor_dtype_t)dtype, 2, shape, (void *)data);
}

static tensor_t *view1(int dtype, int n, const void *data) {
    int shape[1] = { n };
    return tensor_create_view((tensor_dtype_t)dtype, 1, shape, (void *)data);
}

/* Returns 0 on success. tokens_out[steps]; logits_out[steps*vocab] may be NULL;
 * k_cache/v_cache [n_layers][n_kv][max_ctx][hd] are read in and written back. */
int ref_decode_run(const ref_cfg_t *c, const ref_weights_t *w, float *k_cache, float *v_cache,
                   int start_token, int start_pos, int steps, int *tokens_out, float *logits_out) {
    int L = c->n_layers, H = c->hidden, hd = c->head_dim;
    int nq = c->n_heads * hd, nk = c->n_kv_heads * hd;

    gemma3_270m_config_t cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.hidden_size = H;
    cfg.intermediate_size = c->ffn;
    cfg.num_attention_heads = c->n_heads;
    cfg.num_key_value_heads = c->n_kv_heads;
    cfg.num_hidden_layers = L;
    cfg.head_dim = hd;
    cfg.vocab_size = c->vocab;
    cfg.query_pre_attn_scalar = c->query_pre_attn_scalar;
    cfg.rope_theta = c->rope_theta;
    cfg.rope_local_base_freq = c->rope_local_base;
    cfg.sliding_window = c->sliding_window;
    cfg.layer_types_mask = c->global_mask;
    cfg.rms_norm_eps = 1e-6f;

    llm_model_t model;
    memset(&model, 0, sizeof model);
    model.layers = calloc((size_t)L, sizeof(model_layer_weights_t));
    if (!model.layers) return -1;
    for (int l = 0; l < L; ++l) {
        model_layer_weights_t *lw = &model.layers[l];
        lw->q_proj_weight = view2(c->wdtype, nq, H, (const char *)w->wq + (size_t)l * nq * row_bytes(c->wdtype, H));
        lw->k_proj_weight = view2(c->wdtype, nk, H, (const char *)w->wk + (size_t)l * nk * row_bytes(c->wdtype, H));
        lw->v_proj_weight = view2(c->wdtype, nk, H, (const char *)w->wv + (size_t)l * nk * row_bytes(c->wdtype, H));
        lw->out_proj_weight = view2(c->wdtype, H, nq, (const char *)w->wo + (size_t)l * H * row_bytes(c->wdtype, nq));
        lw->gate_proj_weight = view2(c->wdtype, c->ffn, H, (const char *)w->wgate + (size_t)l * c->ffn * row_bytes(c->wdtype, H));
        lw->up_proj_weight = view2(c->wdtype, c->ffn, H, (const char *)w->wup + (size_t)l * c->ffn * row_bytes(c->wdtype, H));
        lw->down_proj_weight = view2(c->wdtype, H, c->ffn, (const char *)w->wdown + (size_t)l * H * row_bytes(c->wdtype, c->ffn));
        lw->norm_attn_weight = view1(DTYPE_F32, H, w->norm_attn + (size_t)l * H);
        lw->norm_attn_post_weight = view1(DTYPE_F32, H, w->norm_attn_post + (size_t)l * H);
        lw->norm_ffn_weight = view1(DTYPE_F32, H, w->norm_ffn + (size_t)l * H);
        lw->norm_ffn_post_weight = view1(DTYPE_F32, H, w->norm_ffn_post + (size_t)l * H);
        lw->q_norm_weight = view1(DTYPE_F32, w->q_norm_len, w->q_norm + (size_t)l * w->q_norm_len);
        lw->k_norm_weight = view1(DTYPE_F32, w->k_norm_len, w->k_norm + (size_t)l * w->k_norm_len);
    }
    model.embedding_weight = view2(DTYPE_BF16, c->vocab, H, w->embed_bf16);
    model.norm_final_weight = view1(DTYPE_F32, H, w->norm_final);
    tensor_t *lm = view2(c->lm_dtype, c->vocab, H, w->lm_head);

    model_spec_t spec;
    memset(&spec, 0, sizeof spec);
    spec.model_id = "gemma3-shaped-synthetic";
    spec.llm_model = &model;
    spec.variant_config = &cfg;

    int rc = -1;
    float *norm = NULL, *logits = NULL;
    inference_session_t *s = inference_session_create(&spec, c->max_ctx);
    if (!s) goto out;
    if (posix_memalign((void **)&norm, 32, sizeof(float) * (size_t)((H + 7) & ~7)) != 0) goto out;
    logits = malloc(sizeof(float) * (size_t)c->vocab);
    if (!logits) goto out;

    size_t per_layer = (size_t)c->n_kv_heads * c->max_ctx * hd;
    for (int l = 0; l < L; ++l) {
        memcpy(tensor_data_mutable(kv_cache_get_keys(s->kv_cache, l)), k_cache + l * per_layer, per_layer * sizeof(float));
        memcpy(tensor_data_mutable(kv_cache_get_values(s->kv_cache, l)), v_cache + l * per_layer, per_layer * sizeof(float));
    }

    int token = start_token;
    for (int st = 0; st < steps; ++st) {
        int pos = start_pos + st;
        float *hidden = s->scratch_buffer;
        sapphire_embed_lookup(s, token, hidden);
        for (int l = 0; l < L; ++l) {
            int glob = s->layer_configs[l].config.attention.is_global;
            transformer_rope_t rope = { glob ? s->rope_freqs_cos_global : s->rope_freqs_cos_local,
                                        glob ? s->rope_freqs_sin_global : s->rope_freqs_sin_local };
            sapphire_transformer_layer(s, l, pos, hidden, rope);
        }
        if (c->lm_dtype == DTYPE_BF16) {
            lm_head(s, hidden, logits);       /* tied: projects through embedding_weight */
        } else {
            rmsnorm_delta(norm, hidden, (const float *)tensor_data(model.norm_final_weight), 1e-6f, H);
            if (kernel_gemv(s->gemv_ctx, logits, lm, norm) != 0) goto out;
        }
        token = sample_greedy(logits, c->vocab);
        tokens_out[st] = token;
        if (logits_out) memcpy(logits_out + (size_t)st * c->vocab, logits, sizeof(float) * (size_t)c->vocab);
    }
    for (int l = 0; l < L; ++l) {
        memcpy(k_cache + l * per_layer, tensor_data(kv_cache_get_keys(s->kv_cache, l)), per_layer * sizeof(float));
        memcpy(v_cache + l * per_layer, tensor_data(kv_cache_get_values(s->kv_cache, l)), per_layer * sizeof(float));
    }
    rc = 0;
out:
    if (s) destroy_inference_session(s);
    free(norm);
    free(logits);
    for (int l = 0; l < L; ++l) {
        model_layer_weights_t *lw = &model.layers[l];
        tensor_t *ts[] = { lw->q_proj_weight, lw->k_proj_weight, lw->v_proj_weight, lw->out_proj_weight,
                           lw->gate_proj_weight, lw->up_proj_weight, lw->down_proj_weight,
                           lw->norm_attn_weight, lw->norm_attn_post_weight, lw->norm_ffn_weight,
                           lw->norm_ffn_post_weight, lw->q_norm_weight, lw->k_norm_weight };
        for (size_t i = 0; i < sizeof ts / sizeof ts[0]; ++i) tensor_release(ts[i]);
    }
    free(model.layers);
    tensor_release(model.embedding_weight);
    tensor_release(model.norm_final_weight);
    tensor_release(lm);
    return rc;
}
