/*
 * ref_decode.c - drives an engine built from the reference's own sources through a
 * configurable Gemma-3-shaped model (synthetic weights handed over as raw arrays).
 *
 * TEST INFRASTRUCTURE ONLY, compiled twice from this one file:
 *  - `make -C oracle ref`: with the reference's headers, linked with
 *    oracle/_ref/libsapphire_ref.so (the whole reference engine) -> libref_decode.so, the
 *    checker that pins the oracle's decode step;
 *  - `make -C oracle engine`: with this repository's include/ first, linked with the
 *    reference's engine sources that libsapphire_hip.so does not replace (inference.c,
 *    kv_cache.c, the loaders, utils.c, log.c, ...) and with libsapphire_hip.so ->
 *    libref_engine_hip.so: the reference's own session and forward loop running its layers
 *    through the library's transformer.h, the thing the GPU tests compare with the oracle.
 * Outputs live in oracle/_ref/ and are never shipped.
 *
 * ref_decode_run composes the reference's public functions in the reference's own order:
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
 *
 * engine_forward_run runs the reference's inference_forward_batch over a prompt in chunks of
 * up to 32 tokens (as perform_inference does, inference.c:236-244), then inference_forward
 * + sample_greedy per step (inference.c:250-297 at temperature 0): embed, layers and lm_head
 * exactly as the engine calls them.
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

/* The engine-side model: configuration, tensor views over the caller's arrays, spec. */
typedef struct {
    gemma3_270m_config_t cfg;
    llm_model_t model;
    tensor_t *lm;
    model_spec_t spec;
} built_t;

static int build_model(const ref_cfg_t *c, const ref_weights_t *w, built_t *b) {
    int L = c->n_layers, H = c->hidden, hd = c->head_dim;
    int nq = c->n_heads * hd, nk = c->n_kv_heads * hd;
    memset(b, 0, sizeof *b);
    b->cfg.hidden_size = H;
    b->cfg.intermediate_size = c->ffn;
    b->cfg.num_attention_heads = c->n_heads;
    b->cfg.num_key_value_heads = c->n_kv_heads;
    b->cfg.num_hidden_layers = L;
    b->cfg.head_dim = hd;
    b->cfg.vocab_size = c->vocab;
    b->cfg.query_pre_attn_scalar = c->query_pre_attn_scalar;
    b->cfg.rope_theta = c->rope_theta;
    b->cfg.rope_local_base_freq = c->rope_local_base;
    b->cfg.sliding_window = c->sliding_window;
    b->cfg.layer_types_mask = c->global_mask;
    b->cfg.rms_norm_eps = 1e-6f;
    b->model.layers = calloc((size_t)L, sizeof(model_layer_weights_t));
    if (!b->model.layers) return -1;
    for (int l = 0; l < L; ++l) {
        model_layer_weights_t *lw = &b->model.layers[l];
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
    b->model.embedding_weight = view2(DTYPE_BF16, c->vocab, H, w->embed_bf16);
    b->model.norm_final_weight = view1(DTYPE_F32, H, w->norm_final);
    b->lm = view2(c->lm_dtype, c->vocab, H, w->lm_head);
    b->spec.model_id = "gemma3-shaped-synthetic";
    b->spec.llm_model = &b->model;
    b->spec.variant_config = &b->cfg;
    return 0;
}

static void free_model(const ref_cfg_t *c, built_t *b) {
    for (int l = 0; b->model.layers && l < c->n_layers; ++l) {
        model_layer_weights_t *lw = &b->model.layers[l];
        tensor_t *ts[] = { lw->q_proj_weight, lw->k_proj_weight, lw->v_proj_weight, lw->out_proj_weight,
                           lw->gate_proj_weight, lw->up_proj_weight, lw->down_proj_weight,
                           lw->norm_attn_weight, lw->norm_attn_post_weight, lw->norm_ffn_weight,
                           lw->norm_ffn_post_weight, lw->q_norm_weight, lw->k_norm_weight };
        for (size_t i = 0; i < sizeof ts / sizeof ts[0]; ++i) tensor_release(ts[i]);
    }
    free(b->model.layers);
    tensor_release(b->model.embedding_weight);
    tensor_release(b->model.norm_final_weight);
    tensor_release(b->lm);
}

static void kv_in(inference_session_t *s, const ref_cfg_t *c, const float *k_cache, const float *v_cache) {
    size_t per_layer = (size_t)c->n_kv_heads * c->max_ctx * c->head_dim;
    for (int l = 0; l < c->n_layers; ++l) {
        memcpy(tensor_data_mutable(kv_cache_get_keys(s->kv_cache, l)), k_cache + l * per_layer, per_layer * sizeof(float));
        memcpy(tensor_data_mutable(kv_cache_get_values(s->kv_cache, l)), v_cache + l * per_layer, per_layer * sizeof(float));
    }
}

static void kv_out(inference_session_t *s, const ref_cfg_t *c, float *k_cache, float *v_cache) {
    size_t per_layer = (size_t)c->n_kv_heads * c->max_ctx * c->head_dim;
    for (int l = 0; l < c->n_layers; ++l) {
        memcpy(k_cache + l * per_layer, tensor_data(kv_cache_get_keys(s->kv_cache, l)), per_layer * sizeof(float));
        memcpy(v_cache + l * per_layer, tensor_data(kv_cache_get_values(s->kv_cache, l)), per_layer * sizeof(float));
    }
}

/* The library's call for engines that change a tensor's host data behind tensor_set_f32
 * (absent from the reference, which reads host data on every call). */
extern int sapphire_tensor_invalidate(tensor_t *t) __attribute__((weak));

/* Changes to the model between the first and the second step (patch 1: every row's first
 * block scale of layer 0's q_proj negated in place, then sapphire_tensor_invalidate where the
 * library provides it; patch 2: 0.25f added to every element of layer 0's norm_attn through
 * tensor_set_f32). The caller's oracle applies the same change to its copy. */
static void apply_patch(built_t *b, const ref_cfg_t *c, int patch) {
    model_layer_weights_t *lw = &b->model.layers[0];
    if (patch == 1) {
        tensor_t *q = lw->q_proj_weight;
        int rows = c->n_heads * c->head_dim, nb = (c->hidden + 31) / 32;
        char *d = (char *)tensor_data_mutable(q);
        size_t bb = c->wdtype == DTYPE_Q4_0 ? 20 : 36;
        for (int r = 0; r < rows; ++r) {
            float *scale = (float *)(d + (size_t)r * nb * bb);   /* the block's leading fp32 scale */
            *scale = -*scale;
        }
        if (sapphire_tensor_invalidate) sapphire_tensor_invalidate(q);
    } else if (patch == 2) {
        tensor_t *n = lw->norm_attn_weight;
        for (int i = 0; i < c->hidden; ++i) tensor_set_f32(n, (size_t)i, tensor_get_f32(n, (size_t)i) + 0.25f);
    }
}

static int decode_run(const ref_cfg_t *c, const ref_weights_t *w, float *k_cache, float *v_cache, int start_token,
                      int start_pos, int steps, int *tokens_out, float *logits_out, int patch) {
    int L = c->n_layers, H = c->hidden;
    built_t b;
    if (build_model(c, w, &b) != 0) return -1;
    int rc = -1;
    float *norm = NULL, *logits = NULL;
    inference_session_t *s = inference_session_create(&b.spec, c->max_ctx);
    if (!s) goto out;
    if (posix_memalign((void **)&norm, 32, sizeof(float) * (size_t)((H + 7) & ~7)) != 0) goto out;
    logits = malloc(sizeof(float) * (size_t)c->vocab);
    if (!logits) goto out;
    kv_in(s, c, k_cache, v_cache);

    int token = start_token;
    for (int st = 0; st < steps; ++st) {
        int pos = start_pos + st;
        float *hidden = s->scratch_buffer;
        sapphire_embed_lookup(s, token, hidden);
        for (int l = 0; l < L; ++l) {
            int glob = s->layer_configs[l].config.attention.is_global;
            transformer_rope_t rope = { glob ? s->rope_freqs_cos_global : s->rope_freqs_cos_local,
                                        glob ? s->rope_freqs_sin_global : s->rope_freqs_sin_local };
            if (sapphire_transformer_layer(s, l, pos, hidden, rope) != 0) goto out;
        }
        if (c->lm_dtype == DTYPE_BF16) {
            lm_head(s, hidden, logits);       /* tied: projects through embedding_weight */
        } else {
            rmsnorm_delta(norm, hidden, (const float *)tensor_data(b.model.norm_final_weight), 1e-6f, H);
            if (kernel_gemv(s->gemv_ctx, logits, b.lm, norm) != 0) goto out;
        }
        token = sample_greedy(logits, c->vocab);
        tokens_out[st] = token;
        if (logits_out) memcpy(logits_out + (size_t)st * c->vocab, logits, sizeof(float) * (size_t)c->vocab);
        if (st == 0 && patch) apply_patch(&b, c, patch);
    }
    kv_out(s, c, k_cache, v_cache);
    rc = 0;
out:
    if (s) destroy_inference_session(s);
    free(norm);
    free(logits);
    free_model(c, &b);
    return rc;
}

/* Returns 0 on success. tokens_out[steps]; logits_out[steps*vocab] may be NULL;
 * k_cache/v_cache [n_layers][n_kv][max_ctx][hd] are read in and written back. */
int ref_decode_run(const ref_cfg_t *c, const ref_weights_t *w, float *k_cache, float *v_cache,
                   int start_token, int start_pos, int steps, int *tokens_out, float *logits_out) {
    return decode_run(c, w, k_cache, v_cache, start_token, start_pos, steps, tokens_out, logits_out, 0);
}

/* ref_decode_run with apply_patch(patch) between the first and the second step. */
int ref_decode_patch_run(const ref_cfg_t *c, const ref_weights_t *w, float *k_cache, float *v_cache,
                         int start_token, int start_pos, int steps, int *tokens_out, float *logits_out, int patch) {
    return decode_run(c, w, k_cache, v_cache, start_token, start_pos, steps, tokens_out, logits_out, patch);
}

/* The engine's own loop (tied BF16 LM head, as lm_head computes it): prompt[n_prompt] at
 * positions start_pos.. through inference_forward_batch in chunks of up to 32, then `steps`
 * inference_forward + sample_greedy steps from start_token at start_pos + n_prompt.
 * Returns 0; tokens_out[steps], logits_out[steps*vocab] (may be NULL); the caches are read in
 * and written back. */
int engine_forward_run(const ref_cfg_t *c, const ref_weights_t *w, float *k_cache, float *v_cache,
                       const int *prompt, int n_prompt, int start_token, int start_pos, int steps, int *tokens_out,
                       float *logits_out) {
    built_t b;
    if (build_model(c, w, &b) != 0) return -1;
    int rc = -1;
    float *logits = NULL;
    inference_session_t *s = inference_session_create(&b.spec, c->max_ctx);
    if (!s) goto out;
    logits = malloc(sizeof(float) * (size_t)c->vocab);
    if (!logits) goto out;
    kv_in(s, c, k_cache, v_cache);
    for (int p = 0; p < n_prompt; p += 32) {
        int n = n_prompt - p > 32 ? 32 : n_prompt - p;
        inference_forward_batch(s, prompt + p, start_pos + p, n, NULL);
    }
    int token = start_token;
    for (int st = 0; st < steps; ++st) {
        inference_forward(s, token, start_pos + n_prompt + st, logits);
        token = sample_greedy(logits, c->vocab);
        tokens_out[st] = token;
        if (logits_out) memcpy(logits_out + (size_t)st * c->vocab, logits, sizeof(float) * (size_t)c->vocab);
    }
    kv_out(s, c, k_cache, v_cache);
    rc = 0;
out:
    if (s) destroy_inference_session(s);
    free(logits);
    free_model(c, &b);
    return rc;
}


/* The buffers sapphire_transformer_layer(_batch) hands its stages: the scratch layout of
 * init_layer_buffers (transformer.c:19-76), which transformer.h's stage functions expect from
 * their caller. */
static layer_buffers_t stage_buffers(const inference_session_t *s, const gemma3_270m_config_t *cfg, int d_model,
                                     int head_dim, int batch) {
    layer_buffers_t buf;
    memset(&buf, 0, sizeof buf);
    const int max_batch = 32;
    buf.pm = s->padded_d_model;
    buf.pi = s->padded_d_inner;
    buf.pk = s->padded_d_kv;
    buf.pf = s->padded_d_ff;
    buf.batch_size = batch;
    size_t bm = (size_t)max_batch * buf.pm, bi = (size_t)max_batch * buf.pi, bk = (size_t)max_batch * buf.pk,
           bf = (size_t)max_batch * buf.pf;
    buf.residual = s->scratch_buffer + bm;
    buf.norm_buf = s->scratch_buffer + 2 * bm;
    buf.q_proj = s->scratch_buffer + 3 * bm;
    buf.k_proj = buf.q_proj + bi;
    buf.v_proj = buf.k_proj + bk;
    buf.attn_out = buf.v_proj + bk;
    buf.ffn_gate_buf = buf.attn_out + bi;
    buf.ffn_value_buf = buf.ffn_gate_buf + bf;
    buf.geglu_buf = buf.ffn_value_buf + bf;
    size_t scratch_floats = s->scratch_size / sizeof(float);
    int need = d_model, qn = cfg->num_attention_heads * head_dim, kn = cfg->num_key_value_heads * head_dim;
    if (qn > need) need = qn;
    if (kn > need) need = kn;
    buf.weight_scratch = (size_t)need <= scratch_floats ? s->scratch_buffer + (scratch_floats - need) : buf.q_proj;
    return buf;
}

/* One layer for `batch` tokens at positions pos.. as sapphire_transformer_layer_batch
 * composes its stages (transformer.c:318-345): attention, FFN, finalize. */
static void layer_by_stages(inference_session_t *s, int l, int pos, int batch, float *hidden, const float *cs,
                            const float *sn) {
    llm_model_t *model = (llm_model_t *)s->model_spec->llm_model;
    gemma3_270m_config_t *cfg = (gemma3_270m_config_t *)s->model_spec->variant_config;
    int d_model = cfg->hidden_size;
    int head_dim = cfg->head_dim > 0 ? cfg->head_dim : d_model / cfg->num_attention_heads;
    layer_buffers_t buf = stage_buffers(s, cfg, d_model, head_dim, batch);
    transformer_layer_ctx_t ctx;
    memset(&ctx, 0, sizeof ctx);
    ctx.session = s;
    ctx.layer = &model->layers[l];
    ctx.config = cfg;
    ctx.layer_idx = l;
    ctx.token_pos = pos;
    ctx.batch_size = batch;
    ctx.d_model = d_model;
    ctx.head_dim = head_dim;
    compute_attention_stage(buf, &ctx, hidden, cs, sn);
    compute_ffn_stage(buf, &ctx, hidden);
    finalize_layer_output(buf, &ctx, hidden);
}

/* engine_forward_run with every layer of every batch run through the three stage functions
 * (inference_forward_batch, inference.c:616-651, with sapphire_transformer_layer_batch
 * composed as transformer.c:318-345 composes it); tied BF16 LM head through lm_head. */
int engine_stage_run(const ref_cfg_t *c, const ref_weights_t *w, float *k_cache, float *v_cache, const int *prompt,
                     int n_prompt, int start_token, int start_pos, int steps, int *tokens_out, float *logits_out) {
    built_t b;
    if (build_model(c, w, &b) != 0) return -1;
    int rc = -1;
    float *logits = NULL;
    inference_session_t *s = inference_session_create(&b.spec, c->max_ctx);
    if (!s) goto out;
    logits = malloc(sizeof(float) * (size_t)c->vocab);
    if (!logits) goto out;
    kv_in(s, c, k_cache, v_cache);
    for (int p = 0; p <= n_prompt + steps - 1; ) {
        /* a prompt chunk of up to 32 tokens, then one token per step */
        int in_prompt = p < n_prompt;
        int n = in_prompt ? (n_prompt - p > 32 ? 32 : n_prompt - p) : 1;
        int st = p - n_prompt;
        const int *ids = in_prompt ? prompt + p : &start_token;
        sapphire_embed_lookup_batch(s, ids, n, s->scratch_buffer);
        for (int l = 0; l < c->n_layers; ++l) {
            int glob = s->layer_configs[l].config.attention.is_global;
            layer_by_stages(s, l, start_pos + p, n, s->scratch_buffer,
                            glob ? s->rope_freqs_cos_global : s->rope_freqs_cos_local,
                            glob ? s->rope_freqs_sin_global : s->rope_freqs_sin_local);
        }
        if (!in_prompt) {
            lm_head(s, s->scratch_buffer, logits);
            start_token = sample_greedy(logits, c->vocab);
            tokens_out[st] = start_token;
            if (logits_out) memcpy(logits_out + (size_t)st * c->vocab, logits, sizeof(float) * (size_t)c->vocab);
        }
        p += n;
    }
    kv_out(s, c, k_cache, v_cache);
    rc = 0;
out:
    if (s) destroy_inference_session(s);
    free(logits);
    free_model(c, &b);
    return rc;
}
