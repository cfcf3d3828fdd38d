// decode_kernels.h - launchers of the fused decode-step kernels (decode.hip), used by the
// device engine (decoder.cpp). Not installed.
#pragma once

#include "internal.h"

namespace sapphire {

// A Q4_0 / Q8_0 matrix in the PACKED layout: quants [M][K/32][16|32], scales [M][K/32].
struct QMat {
    const uint8_t *q = nullptr;
    const float *s = nullptr;
    int M = 0, K = 0;
};

// Input vector of a fused GEMV: h = resid_in (+ rmsnorm_delta(delta, w_delta) when delta is
// set: the residual pattern of attention.c:358-366 / transformer.c:231-239); workgroup 0
// writes h to resid_out when set; x = rmsnorm_delta(h, w_norm) when w_norm is set, else h.
struct GemvIn {
    const float *resid_in = nullptr;
    const float *delta = nullptr;
    const float *w_delta = nullptr;
    float *resid_out = nullptr;
    const float *w_norm = nullptr;
    float eps = 1e-6f;
};

constexpr int kDecMaxK = 2048;       // longest GEMV input of the fused kernels
constexpr int kAttnMaxQ = 2048;      // n_heads * head_dim
constexpr int kAttnMaxKV = 512;      // n_kv_heads * head_dim (at most two K/V heads)
constexpr int kAttnSplit = 64;       // workgroups over the positions of one attention
constexpr int kAttnSplitBatch = 16;  // the same per sequence of a batch (batch >= 4)

// y = W . x(in)  (rows M of w, K = w.K)
int dec_gemv(int dt, const QMat &w, const GemvIn &in, float *y, hipStream_t s);
// g = gelu(Wg . x(in)) * (Wu . x(in))  (transformer.c:141-157)
int dec_geglu(int dt, const QMat &wg, const QMat &wu, const GemvIn &in, float *g, hipStream_t s);
// out = x(in) for K elements (one workgroup): the final norm before the LM head
int dec_prologue_only(const GemvIn &in, int K, float *out, hipStream_t s);
// the same for `batch` sequences whose vectors (resid_in, delta, out) are `stride` floats apart;
// resid_out must be unset
int dec_prologue_batch(const GemvIn &in, int K, int batch, size_t stride, float *out, hipStream_t s);

struct AttnArgs {
    const float *qkv = nullptr;      // [nh*hd | nkv*hd | nkv*hd]: q, k, v projections
    const float *qn = nullptr, *kn = nullptr;   // [hd] QK-norm gammas (attention.c:221-226)
    const float *cos_t = nullptr, *sin_t = nullptr;   // [max_ctx][hd] RoPE tables of the layer
    float *kc = nullptr, *vc = nullptr;          // this layer's caches [nkv][max_ctx][hd]
    const int *d_pos = nullptr;      // position of the token (device)
    const int *d_done = nullptr;     // the sequence's done flag (device, may be NULL): set, no K/V row is written
    float *part = nullptr;           // [kAttnSplit][nh][hd + 2] partial (o, max, sum)
    int nh = 0, nkv = 0, hd = 0, max_ctx = 0;
    int window = 0;                  // sliding window of a local layer, 0 for a global one
    float scale = 1.f, eps = 1e-6f;
    // a batch of independent sequences: sequence b uses qkv + b*qkv_stride, the caches at
    // + b*kv_stride, d_pos[b], d_done[b], and its own partials; out + b*out_stride
    int batch = 1;
    size_t qkv_stride = 0, kv_stride = 0, out_stride = 0;
    // the K/V rows of every position already hold this batch's tokens (dec_kv_write ran):
    // the attention kernel writes none (a prefill chunk of one sequence, whose tokens read
    // each other's rows)
    bool kv_written = false;
    // the combined output in block order (block_order_index(b, h * hd + d), out_stride unused):
    // the input of a batched GEMM
    bool out_blocked = false;
};
// QK-norm, RoPE, KV write and split attention partials, then their combination into
// out[nh*hd] (attention.c:93-163, 271-309; kv_cache.c:252-278). part holds
// attn_part_floats(nh, hd) floats per sequence.
size_t attn_part_floats(int nh, int hd);
int dec_attention(const AttnArgs &a, float *out, hipStream_t s);
// A batched step's QKV GEMM (W [M][K] TILED, input `in` with norms or parts, as
// launch_gemm_tiled_ex) and its attention partials as one launch, then the combine into out:
// the GEMM's rows go to `tagged` ([batch][M] words, tagged with the step counter *epoch and
// `layer`), and the attention workgroups poll them while their K/V rows arrive. A poll longer
// than spin_limit counts in *err. qkv_attention_fusable tells whether the shapes allow it.
bool qkv_attention_fusable(int dt, int K, const AttnArgs &a);
int dec_qkv_attention(int dt, const void *w, int M, int K, const GemmIn &in, void *ws, uint64_t *tagged,
                      const AttnArgs &a, const uint32_t *epoch, int layer, int spin_limit, int *err, float *out,
                      hipStream_t s);
// The K/V rows of the batch only: K = rope(rmsnorm_delta(k, kn)) and V as projected, at
// d_pos[b] (attention.c:292-309 writes every row of a batch before its attention runs).
// Bit-identical to the rows dec_attention writes.
int dec_kv_write(const AttnArgs &a, hipStream_t s);

// resid[i] = bf16 row of *d_token * es (transformer.c:347-365); a token outside [0, vocab)
// reads row 0
int dec_embed(const uint16_t *embed, int hidden, int vocab, float es, const int *d_token, float *resid,
              hipStream_t s);
// Unless *d_done is set: log[*d_step] = *d_token; ++*d_step; ++*d_pos; ++*d_seq when d_seq is
// set; *d_done = 1 when the token is in `stop`
int dec_advance(const int *d_token, int *d_pos, int *d_step, int *log, uint32_t *d_seq, int *d_done,
                const StopSet &stop, hipStream_t s);

// ---- the layers of a step as one persistent kernel (decode_persist.hip) ----

// One layer's weights and caches, in device memory (an array of n_layers).
struct PLayer {
    QMat qkv, o, gate, up, down;
    const float *n_attn, *n_attn_post, *n_ffn, *n_ffn_post, *qn, *kn;
    const float *cos_t, *sin_t;      // RoPE rows of the layer's base (row p at p * rope_stride)
    float *kc, *vc;                  // [nkv][max_ctx][hd]
    int window;                      // sliding window, 0 for a global layer
};

// Exchanged vectors are 64-bit words: fp32 value in the low half, the producing stage's
// epoch in the high half (see decode_persist.hip).
struct PersistArgs {
    const PLayer *layers = nullptr;
    int n_layers = 0;
    const uint16_t *embed = nullptr;  // [vocab][H] bf16
    int vocab = 0;
    float es = 1.f;                   // embedding scale sqrt(H)
    const float *norm_final = nullptr;
    int H = 0, nh = 0, nkv = 0, hd = 0, ffn = 0, max_ctx = 0;
    int rope_stride = 0;              // floats between consecutive positions' rows of cos_t / sin_t
    int window = 0;                   // the local layers' sliding window (PLayer::window of a local layer)
    float scale = 1.f, eps = 1e-6f;
    const int *state = nullptr;       // [0] token, [1] position
    int *done = nullptr;              // the sequence's done flag: set, the kernel returns at once
    const uint32_t *seq = nullptr;    // step counter that makes the epochs unique
    // set: the token, position and epoch counter come from the previous step's LM head through
    // these slots instead of state and seq (the first step of a run takes tok0 and pos0); the
    // kernel logs that token in log and sets done on a token in stop
    TokenSlots *slots = nullptr;
    int *log = nullptr;
    StopSet stop;
    uint64_t *t_qkv = nullptr, *t_part = nullptr, *t_attn = nullptr, *t_o = nullptr, *t_g = nullptr,
             *t_dn = nullptr;
    float *xfin = nullptr;            // [H] final-norm output (the LM-head input)
    int *err = nullptr;               // incremented by a workgroup whose wait timed out
    int spin_limit = 0;
};
constexpr int kPersistMaxGroups = 256;
constexpr int kPersistMaxLayers = 48;   // layer descriptors the persistent step keeps in LDS
// 64-bit words of the tagged exchange buffers for a model shape (all six, contiguous in this
// order: qkv, partials for kPersistMaxGroups workgroups, attention output, o, g, down).
size_t persist_words(int H, int nh, int nkv, int hd, int ffn);
// Whether `groups` workgroups can run the persistent step for these shapes on the current
// device (co-residency included); sets the error message when not.
bool persist_supported(int dt, int groups, int n_layers, int H, int nh, int nkv, int hd, int ffn);
// Launch of the persistent step, all workgroups co-resident (capturable into a HIP graph).
int dec_persist(int dt, const PersistArgs &a, int groups, hipStream_t s);
// Epoch stride of one step: 8 stages per layer plus the final one.
__host__ __device__ inline uint32_t persist_epochs_per_step(int n_layers) { return 8u * (uint32_t)(n_layers + 1); }

// ---- batched decode (a batch of sequences in lock step) ----
// resid[b][i] = bf16 row of tokens[b] * es
int dec_embed_batch(const uint16_t *embed, int hidden, int vocab, float es, const int *d_tokens, int batch,
                    float *resid, hipStream_t s);
// tokens[b] = first index of the maximum of logits[b][0..n) (utils.c:145-156); part holds
// argmax_batch_part_floats(n, batch) floats
size_t argmax_batch_part_floats(int n, int batch);
int dec_argmax_batch(const float *logits, int n, int batch, float *part, int *d_tokens, hipStream_t s);
// For every b with done[b] clear: log[*d_step][b] = tokens[b]; ++pos[b]; done[b] = 1 when the
// token is in `stop`. Then ++*d_step, and ++*d_epoch when d_epoch is set.
int dec_advance_batch(const int *d_tokens, int *d_pos, int *d_step, int batch, int *log, int *d_done,
                      const StopSet &stop, uint32_t *d_epoch, hipStream_t s);

}  // namespace sapphire
