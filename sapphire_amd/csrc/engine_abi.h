// engine_abi.h - the host engine's structs that transformer.h's entry points receive, in the
// memory layout the engine compiles them with (not installed).
//
// sapphire_transformer_layer and its siblings take the engine's inference_session_t and read
// the model, its configuration and the KV cache through it. These definitions restate the
// fields and their order from the reference's headers (inference.h:57-87, model_spec.h
// struct model_spec, llm_model.h:31-58, gemma3_270m_config.h, transformer.h:68-93); only the
// layout matters, the library never allocates them. The KV cache stays opaque: its tensors are
// reached through the engine's kv_cache_get_keys / kv_cache_get_values (kv_cache.h).
#pragma once

#include <cstddef>

#include "../../include/tensor.h"

extern "C" {

typedef struct kv_cache_t kv_cache_t;
typedef struct sapphire_context kernel_context_t;

typedef struct {
    tensor_t *norm_attn_weight;
    tensor_t *norm_attn_post_weight;
    tensor_t *q_proj_weight;
    tensor_t *k_proj_weight;
    tensor_t *v_proj_weight;
    tensor_t *q_norm_weight;
    tensor_t *k_norm_weight;
    tensor_t *out_proj_weight;
    tensor_t *norm_ffn_weight;
    tensor_t *norm_ffn_post_weight;
    tensor_t *up_proj_weight;
    tensor_t *gate_proj_weight;
    tensor_t *down_proj_weight;
} model_layer_weights_t;

typedef struct {
    tensor_t *embedding_weight;
    tensor_t *norm_final_weight;
    tensor_t *lm_head_weight;
    model_layer_weights_t *layers;
    void *safetensors_handle;
} llm_model_t;

typedef struct {
    int sliding_window_pattern;
    const char *architectures_first;
    int attention_bias;
    float attention_dropout;
    float attn_logit_softcapping;
    int bos_token_id;
    int eos_token_id;
    float final_logit_softcapping;
    int head_dim;
    const char *hidden_activation;
    int hidden_size;
    float initializer_range;
    int intermediate_size;
    unsigned long long layer_types_mask;
    int layer_types_count;
    int max_position_embeddings;
    const char *model_type;
    int num_attention_heads;
    int num_hidden_layers;
    int num_key_value_heads;
    int pad_token_id;
    float query_pre_attn_scalar;
    float rms_norm_eps;
    float rope_local_base_freq;
    float rope_scaling;
    float rope_theta;
    int sliding_window;
    const char *torch_dtype;
    const char *transformers_version;
    int use_bidirectional_attention;
    int use_cache;
    int vocab_size;
} gemma3_270m_config_t;

struct model_spec {
    const char *model_id;
    const void *tensor_map;
    int tensor_map_size;
    const void *tokenizer_spec;
    void *tokenizer_handle;
    void *llm_model;
    const void *files;
    void *variant_config;
    const void *loader_hooks;
};
typedef struct model_spec model_spec_t;

typedef struct inference_session_t {
    model_spec_t *model_spec;
    kv_cache_t *kv_cache;
    float *scratch_buffer;
    size_t scratch_size;
    int padded_d_model;
    int padded_d_inner;
    int padded_d_kv;
    int padded_d_ff;
    float *attn_scores;
    float *attn_scores_raw;
    float *rope_freqs_cos_global;
    float *rope_freqs_sin_global;
    float *rope_freqs_cos_local;
    float *rope_freqs_sin_local;
    kernel_context_t *gemv_ctx;
    void *layer_configs;
    int num_layers;
} inference_session_t;

typedef struct {
    const float *cos;
    const float *sin;
} transformer_rope_t;

typedef struct layer_buffers {
    int pm, pi, pk, pf;
    int batch_size;
    float *residual, *norm_buf, *q_proj, *k_proj, *v_proj;
    float *attn_out, *ffn_gate_buf, *ffn_value_buf, *geglu_buf;
    float *weight_scratch;
} layer_buffers_t;

typedef struct transformer_layer_ctx {
    inference_session_t *session;
    model_layer_weights_t *layer;
    gemma3_270m_config_t *config;
    int layer_idx;
    int token_pos;
    int batch_size;
    int d_model;
    int head_dim;
} transformer_layer_ctx_t;

}  // extern "C"
