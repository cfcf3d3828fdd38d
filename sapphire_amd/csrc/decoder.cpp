// decoder.cpp - the device-resident decode engine of include/decoder.h.
//
// Weights are uploaded once: the seven projections as PACKED Q4_0/Q8_0 matrices (q, k and v
// concatenated into one QKV matrix), the LM head as TILED (matrix-core GEMV) where its
// width allows, else PACKED. One decode step is recorded once into a HIP graph and
// replayed: embedding of the token in device memory, 18 x (QKV GEMV, attention, o-proj,
// gate/up GEMV, down GEMV), final norm, LM head with its argmax epilogue writing the next
// token, and a one-thread kernel that logs the token and advances the position (a greedy
// TILED LM head does both in its own epilogue: its last workgroup picks the token). The host
// only launches the graph; nothing crosses PCIe between steps. By default the layers of the
// step run as one persistent kernel (decode_persist.hip) instead of six launches
// per layer; sapphire_decoder_set_workgroups selects either form.
//
// A batched decoder (sapphire_decoder_create_batch) runs 2..16 sequences in lock step, each
// with its own KV cache and position. Its projections are TILED matrices multiplied on the
// matrix cores as one GEMM over the batch (QKV stacked, gate and up interleaved by eight
// rows so that the GeGLU is the GEMM's epilogue), and the residual adds and RMSNorms are
// formed while each GEMM stages its input; a step is 4 GEMMs, 2 attention launches and the
// sum of the down projection's K-chunk partials per layer, the LM-head GEMM, a batched
// argmax and the advance.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/decoder.h"
#include "../../include/rope.h"
#include "decode_kernels.h"
#include "internal.h"

using namespace sapphire;

namespace {

struct Layer {
    QMat qkv, o, gate, up, down;
    // batched decoder: TILED matrices (QKV stacked; gate/up interleaved by eight rows)
    const void *t_qkv = nullptr, *t_o = nullptr, *t_gu = nullptr, *t_down = nullptr;
    const float *n_attn = nullptr, *n_attn_post = nullptr, *n_ffn = nullptr, *n_ffn_post = nullptr;
    const float *qn = nullptr, *kn = nullptr;
    bool global = false;
};

}  // namespace

struct sapphire_decoder {
    sapphire_decoder_config_t cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;  // the arena's chunks
    char *arena_cur = nullptr;
    size_t arena_left = 0;
    std::vector<Layer> layers;
    const uint16_t *embed = nullptr;
    const float *norm_final = nullptr;
    const void *lm = nullptr;
    int lm_layout = LAYOUT_PACKED;
    float *kc = nullptr, *vc = nullptr;
    float *cos_g = nullptr, *sin_g = nullptr, *cos_l = nullptr, *sin_l = nullptr;
    const float *rope_rows = nullptr;   // persistent step: [max_ctx][4][head_dim] (see create)
    float *resid[2] = {nullptr, nullptr};
    float *qkv = nullptr, *attn = nullptr, *o = nullptr, *g = nullptr, *ffn_out = nullptr, *xfin = nullptr;
    float *logits = nullptr, *attn_part = nullptr;
    void *lm_scratch = nullptr;
    // a greedy TILED LM head's per-workgroup keys and its 1 + kGreedyGroups counters (zero
    // between steps): the LM head that picks the token also advances the state
    unsigned long long *gkeys = nullptr;
    unsigned *gcount = nullptr;
    // the persistent step's greedy token hand-over (TokenSlots); graph_slots: the captured step
    // uses it
    TokenSlots *tslots = nullptr;
    bool graph_slots = false;
    int slot_run = kSlotRunSteps;   // steps per run (SAPPHIRE_TOKEN_SLOT_RUN at create time, for tests)
    // [0] token, [1] position, [2] step, [4] done; batched: tokens[B], pos[B], step, -, done[B]
    int *state = nullptr;
    int *log = nullptr;     // [max_ctx] tokens of the steps; batched: [max_ctx][B]
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // kMultiSteps steps captured back to back (calls that take no logits), and their form
    hipGraph_t graph_multi = nullptr;
    hipGraphExec_t exec_multi = nullptr;
    // whether the captured step writes the logits: a greedy batched step that returns no
    // logits picks its tokens inside the LM-head GEMM instead
    bool graph_logits = true;
    // batched: the captured step ends by looking up the next step's input rows (and does not
    // look up its own)
    bool graph_embeds_next = false;
    // batched decoder
    int batch = 1;
    float *dparts = nullptr;     // the down projection's K-chunk partial sums [splits][B][hidden]
    float *dout = nullptr;       // their sum [B][hidden]
    float *amax_part = nullptr;  // argmax partials
    void *gws = nullptr;         // GEMM workspace
    // persistent step (one sequence): workgroups (0: the multi-launch step), the layer
    // descriptors in device memory, the tagged exchange buffers, the epoch counter, the
    // wait-timeout counter and the steps run since the epochs were last reset
    int groups = 0;
    PLayer *players = nullptr;
    uint64_t *tbuf = nullptr;    // tagged exchange vectors
    size_t tbuf_words = 0;
    uint32_t *seq = nullptr;
    int *perr = nullptr;
    uint64_t persist_steps = 0;
    // batched step: the QKV GEMM and the attention in one launch (SAPPHIRE_FUSED_QKV_ATTN=0 turns
    // it off at create time), exchanging q | k | v as words tagged with the step counter bepoch
    // (starts at 1, advanced every step; the host restarts it before a tag would wrap)
    bool fuse_qkv_attn = true;
    uint64_t *tqkv = nullptr;
    uint32_t *bepoch = nullptr;
    uint64_t bepoch_steps = 0;
    // prefill (chunks of up to kPrefillChunk tokens of one sequence through the batched
    // GEMMs); pf_ok is false when the shapes do not fit the TILED GEMM
    bool pf_ok = false;
    float *pf_resid[2] = {nullptr, nullptr};
    float *pf_qkv = nullptr, *pf_attn = nullptr, *pf_o = nullptr, *pf_g = nullptr;
    float *pf_dparts = nullptr, *pf_dout = nullptr, *pf_part = nullptr;
    int *pf_tok = nullptr;       // [kPrefillChunk] tokens, then [kPrefillChunk] positions
    std::vector<hipGraph_t> pf_graph;          // per sequence: a full chunk's pass, captured once
    std::vector<hipGraphExec_t> pf_exec;
    // temperature sampling (temperature > 0): the draws of a generate call [max_ctx][B], the
    // sampler's weights [B][vocab] and workspace
    float temperature = 0.0f;
    // stop tokens (none by default): a sequence that logs one stops (done flag in the state)
    StopSet stop;
    float *draws = nullptr;
    int n_draws = 0;
    float *smp_w = nullptr;
    void *smp_ws = nullptr;
};

namespace {

// Device buffers are carved from large chunks (256-byte aligned pieces): a few big
// allocations instead of one per weight matrix and buffer.
constexpr size_t kArenaChunk = size_t(256) << 20;

bool dev_alloc(sapphire_decoder *d, void **p, size_t bytes, const char *what) {
    *p = nullptr;
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes == 0) bytes = 256;
    if (bytes > d->arena_left) {
        const size_t chunk = std::max(bytes, kArenaChunk);
        void *c = nullptr;
        if (!hip_ok(hipMalloc(&c, chunk), what)) return false;
        d->allocs.push_back(c);
        d->arena_cur = static_cast<char *>(c);
        d->arena_left = chunk;
    }
    *p = d->arena_cur;
    d->arena_cur += bytes;
    d->arena_left -= bytes;
    return true;
}

template <class T>
bool dev_alloc_t(sapphire_decoder *d, T **p, size_t count, const char *what) {
    void *v = nullptr;
    if (!dev_alloc(d, &v, count * sizeof(T), what)) return false;
    *p = static_cast<T *>(v);
    return true;
}

bool upload(sapphire_decoder *d, const void *host, size_t bytes, void **dst, const char *what) {
    if (!host) {
        set_error("decoder weights: %s is NULL", what);
        return false;
    }
    return dev_alloc(d, dst, bytes, what) && hip_ok(hipMemcpy(*dst, host, bytes, hipMemcpyHostToDevice), what);
}

const float *upload_f32(sapphire_decoder *d, const float *host, size_t n, const char *what) {
    void *p = nullptr;
    return upload(d, host, n * sizeof(float), &p, what) ? static_cast<const float *>(p) : nullptr;
}

// Block arrays (AOS, rows concatenated in order) -> one PACKED matrix of sum(rows) x K.
bool upload_packed(sapphire_decoder *d, int dt, std::initializer_list<std::pair<const void *, int>> parts, int K,
                   QMat *out, const char *what) {
    int M = 0;
    for (const auto &p : parts) {
        if (!p.first) {
            set_error("decoder weights: %s is NULL", what);
            return false;
        }
        M += p.second;
    }
    void *aos = nullptr;
    if (!hip_ok(hipMalloc(&aos, q_aos_bytes(dt, M, K)), what)) return false;
    size_t off = 0;
    bool ok = true;
    for (const auto &p : parts) {
        const size_t b = q_aos_bytes(dt, p.second, K);
        ok = ok && hip_ok(hipMemcpy(static_cast<char *>(aos) + off, p.first, b, hipMemcpyHostToDevice), what);
        off += b;
    }
    void *packed = nullptr;
    ok = ok && dev_alloc(d, &packed, q_packed_bytes(dt, M, K), what) &&
         launch_repack(dt, aos, M, K, packed, d->stream) == 0 && hip_ok(hipStreamSynchronize(d->stream), what);
    (void)hipFree(aos);
    if (!ok) return false;
    out->q = static_cast<const uint8_t *>(packed);
    out->s = reinterpret_cast<const float *>(static_cast<const uint8_t *>(packed) + q_scales_offset(dt, M, K));
    out->M = M;
    out->K = K;
    return true;
}

// Block arrays (AOS) -> one TILED matrix: the parts' rows concatenated in order, or, with
// interleave8, two equally long parts interleaved by eight rows (a0..a7, b0..b7, a8..).
bool upload_tiled(sapphire_decoder *d, int dt, std::initializer_list<std::pair<const void *, int>> parts, int K,
                  bool interleave8, const void **out, const char *what) {
    int M = 0;
    for (const auto &p : parts) {
        if (!p.first) {
            set_error("decoder weights: %s is NULL", what);
            return false;
        }
        M += p.second;
    }
    const size_t rb = q_aos_bytes(dt, 1, K);
    void *aos = nullptr;
    if (!hip_ok(hipMalloc(&aos, rb * M), what)) return false;
    bool ok = true;
    if (interleave8) {
        int i = 0;
        for (const auto &p : parts) {
            ok = ok && p.second % 8 == 0 && p.second * 2 == M &&
                 hip_ok(hipMemcpy2D(static_cast<char *>(aos) + (size_t)i * 8 * rb, 16 * rb, p.first, 8 * rb, 8 * rb,
                                    p.second / 8, hipMemcpyHostToDevice),
                        what);
            ++i;
        }
        if (!ok) set_error("decoder weights: %s cannot be interleaved", what);
    } else {
        size_t off = 0;
        for (const auto &p : parts) {
            ok = ok && hip_ok(hipMemcpy(static_cast<char *>(aos) + off, p.first, rb * p.second, hipMemcpyHostToDevice),
                              what);
            off += rb * p.second;
        }
    }
    void *t = nullptr;
    ok = ok && dev_alloc(d, &t, q_tiled_bytes(dt, M, K), what) && launch_to_tiled(dt, aos, M, K, t, d->stream) == 0 &&
         hip_ok(hipStreamSynchronize(d->stream), what);
    (void)hipFree(aos);
    if (!ok) return false;
    *out = t;
    return true;
}

// Half-split tables [max_ctx][hd] from rope_precompute_freqs (rope.c:41-63; host libm, as the
// reference computes them at session creation).
void rope_tables(int hd, int max_ctx, float base, std::vector<float> &c, std::vector<float> &s) {
    c.assign((size_t)max_ctx * hd, 0.f);
    s.assign((size_t)max_ctx * hd, 0.f);
    (void)rope_precompute_freqs(c.data(), s.data(), hd, max_ctx, base);
}

bool layer_is_global(const sapphire_decoder_config_t &c, int l) {   // attention.c:104-111
    if (c.global_mask) return ((c.global_mask >> (unsigned)l) & 1ULL) != 0ULL;
    return ((l + 1) % 6) == 0;
}

// Tokens of one prefill chunk: the batched GEMM's widest batch.
constexpr int kPrefillChunk = 16;
static_assert(kPrefillChunk == kGemmSeqs, "a prefill chunk is one batched GEMM pass (block-order buffers of 16 slots)");

// Shapes the TILED matrix-core GEMM takes: every projection K a multiple of 128 and the
// hidden size at most 36 blocks (the norms are formed inside one K chunk).
bool tiled_shapes_ok(const sapphire_decoder_config_t &c) {
    const int nq = c.n_heads * c.head_dim;
    return c.hidden % 128 == 0 && nq % 128 == 0 && c.ffn % 128 == 0 && c.hidden <= 1152;
}

// A persistent-step wait longer than this many polls (about a second) is a failure.
constexpr int kPersistSpinLimit = 1 << 19;
// the batched step counter's range (tags are counter << 6 | layer + 1 in 32 bits)
constexpr uint64_t kBatchEpochLimit = uint64_t(1) << 26;
// steps per launch of the persistent step's multi-step graph (each graph launch costs the GPU a
// gap of its own: 0.384 ms per token at one step per launch, 0.3829 at 8 and 0.3824 at 16 on
// one box)
constexpr int kMultiSteps = 16;
int batch_qkv_width(const sapphire_decoder_config_t &c) { return (c.n_heads + 2 * c.n_kv_heads) * c.head_dim; }

// Per sequence 1 once it has logged a stop token (the state's last B words).
int *done_flags(sapphire_decoder *d) { return d->state + 2 * d->batch + 2; }

// The sampled tokens of the step's logits into tokens[B] (perform_inference's draw,
// inference.c:262-266 and 297), the step's draws at d->draws[step * B].
int enqueue_sample(sapphire_decoder *d, const int *d_step, hipStream_t s) {
    const auto &c = d->cfg;
    return launch_sample(d->logits, c.vocab, d->batch, c.vocab, d->temperature, d->smp_w, c.vocab, d->draws, d_step,
                         d->state, d->smp_ws, s);
}

// Whether the persistent step hands its greedy token to the next step through d->tslots: a
// greedy TILED LM head over a vocabulary the slot keys can index.
bool use_token_slots(const sapphire_decoder *d) {
    return d->groups > 0 && d->batch == 1 && d->tslots && !(d->temperature > 0.0f) && d->cfg.lm_dtype != DT_BF16 &&
           d->lm_layout == LAYOUT_TILED && d->cfg.vocab <= kSlotMaxVocab;
}

// LM head on d->xfin with the greedy (or sampled) token into d->state[0], then the advance
// (for a greedy TILED head both happen in the LM head's own epilogue, or, with token slots, in
// the next step's layers kernel).
int enqueue_lm_head(sapphire_decoder *d) {
    const auto &c = d->cfg;
    hipStream_t s = d->stream;
    const int H = c.hidden;
    const bool greedy = !(d->temperature > 0.0f);
    if (use_token_slots(d))
        return launch_gemv_tiled_greedy_slots(c.lm_dtype, d->lm, c.vocab, H, d->xfin, d->logits, d->tslots,
                                              done_flags(d), s);
    if (c.lm_dtype == DT_BF16) {
        // weight tying: the logits are the embedding table times the final norm
        // (transformer.c:393-408 projects through embedding_weight)
        if (launch_gemv_f(DT_BF16, d->lm, c.vocab, H, d->xfin, d->logits, s) != 0) return -1;
        if (greedy &&
            launch_softmax_argmax(d->logits, c.vocab, nullptr, d->state, static_cast<float *>(d->lm_scratch), s) != 0)
            return -1;
    } else if (d->lm_layout == LAYOUT_TILED) {
        if (greedy) {
            // the logits, the token and the advance in one launch
            GreedyStep gs;
            gs.keys = d->gkeys;
            gs.count = d->gcount;
            gs.tok = d->state;
            gs.pos = d->state + 1;
            gs.step = d->state + 2;
            gs.log = d->log;
            gs.seq = d->groups > 0 ? d->seq : nullptr;
            gs.done = done_flags(d);
            gs.stop = d->stop;
            return launch_gemv_tiled_greedy_step(c.lm_dtype, d->lm, c.vocab, H, d->xfin, d->logits, gs, s);
        }
        if (launch_gemv_tiled(c.lm_dtype, d->lm, c.vocab, H, d->xfin, d->logits, s) != 0) return -1;
    } else {
        if (launch_gemv_q(c.lm_dtype, LAYOUT_PACKED, d->lm, c.vocab, H, d->xfin, d->logits, s) != 0) return -1;
        if (greedy &&
            launch_softmax_argmax(d->logits, c.vocab, nullptr, d->state, static_cast<float *>(d->lm_scratch), s) != 0)
            return -1;
    }
    if (!greedy && enqueue_sample(d, d->state + 2, s) != 0) return -1;
    return dec_advance(d->state, d->state + 1, d->state + 2, d->log, d->groups > 0 ? d->seq : nullptr, done_flags(d),
                       d->stop, s);
}

// One decode step, enqueued on d->stream (recorded into the graph).
int enqueue_step(sapphire_decoder *d) {
    const auto &c = d->cfg;
    hipStream_t s = d->stream;
    const int H = c.hidden, hd = c.head_dim;
    const float es = sqrtf((float)H);
    const float scale = 1.0f / sqrtf(c.query_pre_attn_scalar > 0.f ? c.query_pre_attn_scalar : (float)hd);
    const int win = c.sliding_window > 0 ? c.sliding_window : 1024;
    if (d->groups > 0) {
        PersistArgs pa;
        pa.layers = d->players;
        pa.n_layers = c.n_layers;
        pa.embed = d->embed;
        pa.vocab = c.vocab;
        pa.es = es;
        pa.norm_final = d->norm_final;
        pa.H = H;
        pa.nh = c.n_heads;
        pa.nkv = c.n_kv_heads;
        pa.hd = hd;
        pa.ffn = c.ffn;
        pa.max_ctx = c.max_ctx;
        pa.rope_stride = 4 * hd;
        pa.window = win;
        pa.scale = scale;
        pa.eps = c.eps;
        pa.state = d->state;
        pa.done = done_flags(d);
        pa.seq = d->seq;
        const size_t nqkv = (size_t)(c.n_heads + 2 * c.n_kv_heads) * hd;
        pa.t_qkv = d->tbuf;
        pa.t_part = pa.t_qkv + nqkv;
        pa.t_attn = pa.t_part + (size_t)kPersistMaxGroups * c.n_heads * (hd + 2);
        pa.t_o = pa.t_attn + (size_t)c.n_heads * hd;
        pa.t_g = pa.t_o + H;
        pa.t_dn = pa.t_g + c.ffn;
        pa.xfin = d->xfin;
        pa.err = d->perr;
        pa.spin_limit = kPersistSpinLimit;
        if (use_token_slots(d)) {
            pa.slots = d->tslots;
            pa.log = d->log;
            pa.stop = d->stop;
        }
        if (dec_persist(c.wdtype, pa, d->groups, s) != 0) return -1;
        return enqueue_lm_head(d);
    }
    if (dec_embed(d->embed, H, c.vocab, es, d->state, d->resid[0], s) != 0) return -1;
    int cur = 0;
    const size_t layer_kv = (size_t)c.n_kv_heads * c.max_ctx * hd;
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer &L = d->layers[l];
        // previous layer's finalize (transformer.c:231-239) + attention pre-norm (attention.c:316-325)
        GemvIn a_in;
        a_in.resid_in = d->resid[cur];
        a_in.eps = c.eps;
        a_in.w_norm = L.n_attn;
        if (l > 0) {
            a_in.delta = d->ffn_out;
            a_in.w_delta = d->layers[l - 1].n_ffn_post;
            a_in.resid_out = d->resid[1 - cur];
            cur = 1 - cur;
        }
        if (dec_gemv(c.wdtype, L.qkv, a_in, d->qkv, s) != 0) return -1;
        AttnArgs at;
        at.qkv = d->qkv;
        at.qn = L.qn;
        at.kn = L.kn;
        at.cos_t = L.global ? d->cos_g : d->cos_l;
        at.sin_t = L.global ? d->sin_g : d->sin_l;
        at.kc = d->kc + (size_t)l * layer_kv;
        at.vc = d->vc + (size_t)l * layer_kv;
        at.d_pos = d->state + 1;
        at.d_done = done_flags(d);
        at.part = d->attn_part;
        at.nh = c.n_heads;
        at.nkv = c.n_kv_heads;
        at.hd = hd;
        at.max_ctx = c.max_ctx;
        at.window = L.global ? 0 : win;
        at.scale = scale;
        at.eps = c.eps;
        if (dec_attention(at, d->attn, s) != 0) return -1;
        GemvIn o_in;
        o_in.resid_in = d->attn;
        if (dec_gemv(c.wdtype, L.o, o_in, d->o, s) != 0) return -1;
        // post-attention norm + residual (attention.c:356-366), FFN pre-norm (transformer.c:119-121)
        GemvIn f_in;
        f_in.resid_in = d->resid[cur];
        f_in.delta = d->o;
        f_in.w_delta = L.n_attn_post;
        f_in.resid_out = d->resid[1 - cur];
        f_in.w_norm = L.n_ffn;
        f_in.eps = c.eps;
        cur = 1 - cur;
        if (dec_geglu(c.wdtype, L.gate, L.up, f_in, d->g, s) != 0) return -1;
        GemvIn d_in;
        d_in.resid_in = d->g;
        if (dec_gemv(c.wdtype, L.down, d_in, d->ffn_out, s) != 0) return -1;
    }
    // last finalize + final norm (transformer.c:400-406), LM head + greedy token
    GemvIn fin;
    fin.resid_in = d->resid[cur];
    fin.delta = d->ffn_out;
    fin.w_delta = d->layers[c.n_layers - 1].n_ffn_post;
    fin.w_norm = d->norm_final;
    fin.eps = c.eps;
    if (dec_prologue_only(fin, H, d->xfin, s) != 0) return -1;
    return enqueue_lm_head(d);
}

// One batched pass over the layers: r.B token vectors, either the sequences of a batched
// decode step (each with its own cache and position) or a prefill chunk of one sequence (one
// cache, kv_stride 0, positions pos..pos+B-1, all K/V rows written before attention reads
// them, as attention.c:292-309 does for a batch). Leaves the last layer's down projection as
// K-chunk partials in r.dparts and returns the index of r.resid holding the residual stream.
struct BatchRun {
    int B = 0;
    const int *d_tokens = nullptr, *d_pos = nullptr;
    const int *d_done = nullptr;          // per sequence: set, its K/V rows are not written
    float *kc = nullptr, *vc = nullptr;   // layer 0 of the first sequence's caches
    size_t kv_stride = 0;                 // between sequences (0: one shared cache)
    bool prefill = false;
    float *resid[2] = {nullptr, nullptr};
    float *qkv = nullptr, *attn = nullptr, *o = nullptr, *g = nullptr, *dparts = nullptr, *dout = nullptr;
    float *part = nullptr;
    void *gws = nullptr;
    // the fused QKV + attention launch of a decode step (not set for a prefill chunk)
    uint64_t *tqkv = nullptr;
    const uint32_t *epoch = nullptr;
    int *err = nullptr;
    bool embedded = false;                // resid[0] already holds the tokens' embeddings
};

int enqueue_layers_batch(sapphire_decoder *d, const BatchRun &r) {
    const auto &c = d->cfg;
    hipStream_t s = d->stream;
    const int B = r.B, H = c.hidden, hd = c.head_dim;
    const int nq = c.n_heads * hd, nqkv = nq + 2 * c.n_kv_heads * hd;
    const float es = sqrtf((float)H);
    const float scale = 1.0f / sqrtf(c.query_pre_attn_scalar > 0.f ? c.query_pre_attn_scalar : (float)hd);
    const int win = c.sliding_window > 0 ? c.sliding_window : 1024;
    const size_t layer_kv = (size_t)c.n_kv_heads * c.max_ctx * hd;
    const int nsd = gemm_splits(c.ffn);
    if (!r.embedded && dec_embed_batch(d->embed, H, c.vocab, es, r.d_tokens, B, r.resid[0], s) != 0) return -1;
    int cur = 0;
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer &L = d->layers[l];
        // previous layer's finalize (transformer.c:231-239) + attention pre-norm (attention.c:316-325)
        GemmIn qi;
        qi.x = r.resid[cur];
        qi.ldx = H;
        qi.w_norm = L.n_attn;
        qi.eps = c.eps;
        qi.tree_norms = true;           // both norms as trees (the decode tolerance)
        if (l > 0) {
            // the previous down projection's K-chunk partial sums, added in chunk order by the
            // GEMM's input pass
            qi.parts = r.dparts;
            qi.nparts = nsd;
            qi.ldp = H;
            qi.part_stride = (size_t)B * H;
            qi.w_delta = d->layers[l - 1].n_ffn_post;
            qi.resid_out = r.resid[1 - cur];
            qi.ldr = H;
            cur = 1 - cur;
        }
        AttnArgs at;
        at.qkv = r.qkv;
        at.qn = L.qn;
        at.kn = L.kn;
        at.cos_t = L.global ? d->cos_g : d->cos_l;
        at.sin_t = L.global ? d->sin_g : d->sin_l;
        at.kc = r.kc + (size_t)l * layer_kv;
        at.vc = r.vc + (size_t)l * layer_kv;
        at.d_pos = r.d_pos;
        at.d_done = r.d_done;
        at.part = r.part;
        at.nh = c.n_heads;
        at.nkv = c.n_kv_heads;
        at.hd = hd;
        at.max_ctx = c.max_ctx;
        at.window = L.global ? 0 : win;
        at.scale = scale;
        at.eps = c.eps;
        at.batch = B;
        at.qkv_stride = (size_t)nqkv;
        at.kv_stride = r.kv_stride;
        at.out_stride = (size_t)nq;
        at.out_blocked = true;          // the o projection stages it with contiguous loads
        if (r.prefill) {
            if (launch_gemm_tiled_ex(c.wdtype, L.t_qkv, nqkv, H, B, qi, GemmOut{r.qkv, nqkv}, r.gws, s) != 0)
                return -1;
            if (dec_kv_write(at, s) != 0) return -1;
            at.kv_written = true;
            if (dec_attention(at, r.attn, s) != 0) return -1;
        } else if (d->fuse_qkv_attn && r.tqkv && l <= 62 && qkv_attention_fusable(c.wdtype, H, at)) {
            // one launch: the attention workgroups stream their K/V rows while the GEMM runs
            if (dec_qkv_attention(c.wdtype, L.t_qkv, nqkv, H, qi, r.gws, r.tqkv, at, r.epoch, l, kPersistSpinLimit,
                                  r.err, r.attn, s) != 0)
                return -1;
        } else {
            if (launch_gemm_tiled_ex(c.wdtype, L.t_qkv, nqkv, H, B, qi, GemmOut{r.qkv, nqkv}, r.gws, s) != 0)
                return -1;
            if (dec_attention(at, r.attn, s) != 0) return -1;
        }
        GemmIn oi;
        oi.x = r.attn;
        oi.x_blocked = true;
        GemmOut oo;
        oo.y = r.o;
        oo.ldy = H;
        if (launch_gemm_tiled_ex(c.wdtype, L.t_o, H, nq, B, oi, oo, r.gws, s) != 0) return -1;
        // post-attention norm + residual (attention.c:356-366), FFN pre-norm (transformer.c:119-121),
        // gate/up projections with the GeGLU (transformer.c:126-157)
        GemmIn fi;
        fi.x = r.resid[cur];
        fi.ldx = H;
        fi.parts = r.o;
        fi.nparts = 1;
        fi.ldp = H;
        fi.w_delta = L.n_attn_post;
        fi.resid_out = r.resid[1 - cur];
        fi.ldr = H;
        fi.w_norm = L.n_ffn;
        fi.eps = c.eps;
        fi.tree_norms = true;           // both norms as trees (the decode tolerance)
        cur = 1 - cur;
        GemmOut fo;
        fo.y = r.g;
        fo.geglu = true;
        fo.y_blocked = true;            // the down projection stages it with contiguous loads
        if (launch_gemm_tiled_ex(c.wdtype, L.t_gu, 2 * c.ffn, H, B, fi, fo, r.gws, s) != 0) return -1;
        GemmIn di;
        di.x = r.g;
        di.x_blocked = true;
        GemmOut dout;
        dout.parts = r.dparts;
        if (launch_gemm_tiled_ex(c.wdtype, L.t_down, H, c.ffn, B, di, dout, r.gws, s) != 0) return -1;
    }
    return cur;
}

// One step of the batched decoder, enqueued on d->stream (recorded into the graph).
int enqueue_step_batch(sapphire_decoder *d) {
    const auto &c = d->cfg;
    hipStream_t s = d->stream;
    const int B = d->batch, H = c.hidden;
    const int nsd = gemm_splits(c.ffn);
    BatchRun r;
    r.B = B;
    r.d_tokens = d->state;
    r.d_pos = d->state + B;
    r.d_done = done_flags(d);
    r.kc = d->kc;
    r.vc = d->vc;
    r.kv_stride = (size_t)c.n_layers * c.n_kv_heads * c.max_ctx * c.head_dim;
    r.resid[0] = d->resid[0];
    r.resid[1] = d->resid[1];
    r.qkv = d->qkv;
    r.attn = d->attn;
    r.o = d->o;
    r.g = d->g;
    r.dparts = d->dparts;
    r.dout = d->dout;
    r.part = d->attn_part;
    r.gws = d->gws;
    r.tqkv = d->tqkv;
    r.epoch = d->bepoch;
    r.err = d->perr;
    // the greedy GEMM form's finish looks up the next step's input rows: the step starts
    // from them (generate looks up the first step's before the first launch)
    const bool greedy_gemm =
        c.lm_dtype != DT_BF16 && d->temperature <= 0.0f && !d->graph_logits && gemm_splits(H) == 1;
    r.embedded = greedy_gemm;
    d->graph_embeds_next = greedy_gemm;
    const int cur = enqueue_layers_batch(d, r);
    if (cur < 0) return -1;
    // last finalize + final norm (transformer.c:400-406), LM head, greedy tokens
    if (c.lm_dtype == DT_BF16) {
        if (launch_sum_parts(d->dparts, nsd, (size_t)B * H, B, H, d->dout, H, s) != 0) return -1;
        // weight tying: the embedding table times the final norms, on the matrix cores
        GemvIn fin;
        fin.resid_in = d->resid[cur];
        fin.delta = d->dout;
        fin.w_delta = d->layers[c.n_layers - 1].n_ffn_post;
        fin.w_norm = d->norm_final;
        fin.eps = c.eps;
        if (dec_prologue_batch(fin, H, B, (size_t)H, d->xfin, s) != 0) return -1;
        if (launch_gemm_bf16(d->lm, c.vocab, H, d->xfin, H, B, d->logits, c.vocab, s) != 0) return -1;
        if ((d->temperature > 0.0f ? enqueue_sample(d, d->state + 2 * B, s)
                                   : dec_argmax_batch(d->logits, c.vocab, B, d->amax_part, d->state, s)) != 0)
            return -1;
        return dec_advance_batch(d->state, d->state + B, d->state + 2 * B, B, d->log, done_flags(d), d->stop, d->bepoch,
                             s);
    }
    GemmIn li;
    li.x = d->resid[cur];
    li.ldx = H;
    li.parts = d->dparts;
    li.nparts = nsd;
    li.ldp = H;
    li.part_stride = (size_t)B * H;
    li.w_delta = d->layers[c.n_layers - 1].n_ffn_post;
    li.w_norm = d->norm_final;
    li.eps = c.eps;
    li.tree_norms = true;
    GemmOut lo;
    if (greedy_gemm) {
        // greedy tokens straight from the LM-head GEMM: no logits written or read again; its
        // finish launch also advances the step and looks up the next step's input rows
        BatchAdvance adv;
        adv.pos = d->state + B;
        adv.step = d->state + 2 * B;
        adv.log = d->log;
        adv.done = done_flags(d);
        adv.epoch = d->bepoch;
        adv.stop = d->stop;
        adv.embed = d->embed;
        adv.hidden = H;
        adv.es = sqrtf((float)H);
        adv.resid = d->resid[0];
        lo.tokens = d->state;
        lo.advance = &adv;
        return launch_gemm_tiled_ex(c.lm_dtype, d->lm, c.vocab, H, B, li, lo, d->gws, s);
    }
    lo.y = d->logits;
    lo.ldy = c.vocab;
    if (launch_gemm_tiled_ex(c.lm_dtype, d->lm, c.vocab, H, B, li, lo, d->gws, s) != 0) return -1;
    if ((d->temperature > 0.0f ? enqueue_sample(d, d->state + 2 * B, s)
                               : dec_argmax_batch(d->logits, c.vocab, B, d->amax_part, d->state, s)) != 0)
        return -1;
    return dec_advance_batch(d->state, d->state + B, d->state + 2 * B, B, d->log, done_flags(d), d->stop, d->bepoch,
                             s);
}

bool valid_config(const sapphire_decoder_config_t &c) {
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.ffn <= 0 ||
        c.vocab <= 0 || c.max_ctx <= 0) {
        set_error("decoder config: non-positive dimension");
        return false;
    }
    if (!is_quant(c.wdtype) || (!is_quant(c.lm_dtype) && c.lm_dtype != DT_BF16)) {
        set_error("decoder config: projections must be Q4_0 or Q8_0, the LM head Q4_0, Q8_0 or BF16 (tied)");
        return false;
    }
    if (c.hidden % kBlock || (c.n_heads * c.head_dim) % kBlock || c.ffn % kBlock) {
        set_error("decoder config: hidden, n_heads*head_dim and ffn must be multiples of 32");
        return false;
    }
    if (c.hidden > kDecMaxK || c.n_heads * c.head_dim > kDecMaxK || c.ffn > kDecMaxK) {
        set_error("decoder config: GEMV inputs longer than %d are not supported", kDecMaxK);
        return false;
    }
    if (c.n_heads % c.n_kv_heads || (c.head_dim & 1)) {
        set_error("decoder config: heads must group evenly and head_dim be even");
        return false;
    }
    return true;
}

// Drops the captured step graphs (one step and kMultiSteps steps): the next generate captures
// them again with the decoder's current form, sampling and stop set.
void drop_step_graphs(sapphire_decoder *d) {
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    if (d->exec_multi) (void)hipGraphExecDestroy(d->exec_multi);
    if (d->graph_multi) (void)hipGraphDestroy(d->graph_multi);
    d->exec = d->exec_multi = nullptr;
    d->graph = d->graph_multi = nullptr;
}

}  // namespace

extern "C" {

void sapphire_decoder_destroy(sapphire_decoder_t *d) {
    if (!d) return;
    (void)hipSetDevice(d->device);
    if (d->stream) (void)hipStreamSynchronize(d->stream);
    drop_step_graphs(d);
    for (hipGraphExec_t e : d->pf_exec)
        if (e) (void)hipGraphExecDestroy(e);
    for (hipGraph_t g : d->pf_graph)
        if (g) (void)hipGraphDestroy(g);
    for (void *p : d->allocs) (void)hipFree(p);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    delete d;
}

}  // extern "C"

namespace {

// The batched decoder's extra shape rules: every projection K a multiple of 128 (TILED),
// the hidden size at most 36 blocks (the norms are formed inside one K chunk).
bool valid_batch_config(const sapphire_decoder_config_t &c, int batch) {
    const int nq = c.n_heads * c.head_dim;
    if (batch < 2 || batch > 16) {
        set_error("batched decoder: batch must be 2..16 (got %d)", batch);
        return false;
    }
    if (c.hidden % 128 || nq % 128 || c.ffn % 128 || c.hidden > 1152) {
        set_error("batched decoder: hidden, n_heads*head_dim and ffn must be multiples of 128, hidden <= 1152");
        return false;
    }
    if (c.n_heads % c.n_kv_heads || (c.head_dim & 1)) {
        set_error("decoder config: heads must group evenly and head_dim be even");
        return false;
    }
    return true;
}

bool setup_persistent(sapphire_decoder *d);

sapphire_decoder_t *create_decoder(const sapphire_decoder_config_t *cfg, const sapphire_decoder_weights_t *w,
                                   int batch) {
    if (!cfg || !w) {
        set_error("sapphire_decoder_create: NULL argument");
        return nullptr;
    }
    if (batch == 1 ? !valid_config(*cfg) : !valid_batch_config(*cfg, batch)) return nullptr;
    if (batch > 1 && (cfg->n_layers <= 0 || cfg->hidden <= 0 || cfg->n_heads <= 0 || cfg->n_kv_heads <= 0 ||
                      cfg->head_dim <= 0 || cfg->ffn <= 0 || cfg->vocab <= 0 || cfg->max_ctx <= 0 ||
                      !is_quant(cfg->wdtype) || (!is_quant(cfg->lm_dtype) && cfg->lm_dtype != DT_BF16))) {
        set_error("decoder config: non-positive dimension, projections not Q4_0/Q8_0 or LM head not Q4_0/Q8_0/BF16");
        return nullptr;
    }
    sapphire_decoder *d = new (std::nothrow) sapphire_decoder();
    if (!d) return nullptr;
    d->cfg = *cfg;
    d->batch = batch;
    d->pf_ok = tiled_shapes_ok(*cfg);
    const int B = batch;
    const auto &c = d->cfg;
    auto fail = [&]() -> sapphire_decoder_t * {
        sapphire_decoder_destroy(d);
        return nullptr;
    };
    if (!hip_ok(hipGetDevice(&d->device), "hipGetDevice") ||
        !hip_ok(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking), "hipStreamCreate"))
        return fail();
    const int H = c.hidden, hd = c.head_dim, nq = c.n_heads * hd, nk = c.n_kv_heads * hd;
    d->layers.resize((size_t)c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        Layer &L = d->layers[l];
        L.global = layer_is_global(c, l);
        if (!w->wq || !w->wk || !w->wv || !w->wo || !w->wgate || !w->wup || !w->wdown || !w->norm_attn ||
            !w->norm_attn_post || !w->norm_ffn || !w->norm_ffn_post || !w->q_norm || !w->k_norm) {
            set_error("decoder weights: a per-layer array is NULL");
            return fail();
        }
        if (B == 1) {
            if (!upload_packed(d, c.wdtype, {{w->wq[l], nq}, {w->wk[l], nk}, {w->wv[l], nk}}, H, &L.qkv, "wqkv") ||
                !upload_packed(d, c.wdtype, {{w->wo[l], H}}, nq, &L.o, "wo") ||
                !upload_packed(d, c.wdtype, {{w->wgate[l], c.ffn}}, H, &L.gate, "wgate") ||
                !upload_packed(d, c.wdtype, {{w->wup[l], c.ffn}}, H, &L.up, "wup") ||
                !upload_packed(d, c.wdtype, {{w->wdown[l], H}}, c.ffn, &L.down, "wdown"))
                return fail();
        }
        if (d->pf_ok) {   // TILED copies: the batched step and the prefill GEMMs
            if (!upload_tiled(d, c.wdtype, {{w->wq[l], nq}, {w->wk[l], nk}, {w->wv[l], nk}}, H, false, &L.t_qkv,
                              "wqkv") ||
                !upload_tiled(d, c.wdtype, {{w->wo[l], H}}, nq, false, &L.t_o, "wo") ||
                !upload_tiled(d, c.wdtype, {{w->wgate[l], c.ffn}, {w->wup[l], c.ffn}}, H, true, &L.t_gu, "wgate/wup") ||
                !upload_tiled(d, c.wdtype, {{w->wdown[l], H}}, c.ffn, false, &L.t_down, "wdown"))
                return fail();
        }
    }
    // Every layer's norm weights and QK gammas, and the final norm, in one block: the step
    // reads a few of them in every stage, and one block keeps them in one translation page.
    {
        const size_t vh = (H + 63) & ~size_t(63), vd = (hd + 63) & ~size_t(63);
        const size_t per = 4 * vh + 2 * vd;
        if (w->norm_dtype != DT_F32 && w->norm_dtype != DT_BF16) {
            set_error("decoder weights: norm_dtype %d (F32 or BF16)", w->norm_dtype);
            return fail();
        }
        // fp32 as given, or bf16 widened by its bits (get_norm_weights, utils.c:218-225)
        auto put = [&](float *dst, const float *src, int n) {
            if (w->norm_dtype == DT_F32) {
                memcpy(dst, src, sizeof(float) * n);
                return;
            }
            const uint16_t *b = reinterpret_cast<const uint16_t *>(src);
            for (int i = 0; i < n; ++i) {
                const uint32_t u = (uint32_t)b[i] << 16;
                memcpy(dst + i, &u, sizeof u);
            }
        };
        std::vector<float> hv((size_t)c.n_layers * per + vh, 0.f);
        for (int l = 0; l < c.n_layers; ++l) {
            float *o = hv.data() + (size_t)l * per;
            put(o, w->norm_attn[l], H);
            put(o + vh, w->norm_attn_post[l], H);
            put(o + 2 * vh, w->norm_ffn[l], H);
            put(o + 3 * vh, w->norm_ffn_post[l], H);
            put(o + 4 * vh, w->q_norm[l], hd);
            put(o + 4 * vh + vd, w->k_norm[l], hd);
        }
        if (!w->norm_final) {
            set_error("decoder weights: norm_final is NULL");
            return fail();
        }
        put(hv.data() + (size_t)c.n_layers * per, w->norm_final, H);
        const float *dv = upload_f32(d, hv.data(), hv.size(), "norm weights");
        if (!dv) return fail();
        for (int l = 0; l < c.n_layers; ++l) {
            Layer &L = d->layers[l];
            const float *o = dv + (size_t)l * per;
            L.n_attn = o;
            L.n_attn_post = o + vh;
            L.n_ffn = o + 2 * vh;
            L.n_ffn_post = o + 3 * vh;
            L.qn = o + 4 * vh;
            L.kn = o + 4 * vh + vd;
        }
        d->norm_final = dv + (size_t)c.n_layers * per;
    }
    void *p = nullptr;
    if (!upload(d, w->embed_bf16, (size_t)c.vocab * H * sizeof(uint16_t), &p, "embed")) return fail();
    d->embed = static_cast<const uint16_t *>(p);
    // LM head
    if (c.lm_dtype == DT_BF16) {
        if (B > 1 && !gemm_bf16_supported(d->embed, c.vocab, H)) {
            set_error("batched decoder: a BF16 LM head needs hidden %% 8 == 0 and a table below 4 GiB");
            return fail();
        }
        d->lm = d->embed;
        if (!dev_alloc(d, &d->lm_scratch, softmax_scratch_floats(c.vocab) * sizeof(float), "lm scratch"))
            return fail();
    } else {
        if (!w->lm_head) {
            set_error("decoder weights: lm_head is NULL");
            return fail();
        }
        void *aos = nullptr;
        const size_t ab = q_aos_bytes(c.lm_dtype, c.vocab, H);
        if (!hip_ok(hipMalloc(&aos, ab), "lm aos")) return fail();
        bool ok = hip_ok(hipMemcpy(aos, w->lm_head, ab, hipMemcpyHostToDevice), "lm upload");
        d->lm_layout = (B > 1 ? tiled_layout_ok(c.lm_dtype, c.vocab, H) : tiled_supported(c.lm_dtype, c.vocab, H))
                           ? LAYOUT_TILED
                           : LAYOUT_PACKED;
        if (B > 1 && d->lm_layout != LAYOUT_TILED) {
            (void)hipFree(aos);
            set_error("batched decoder: the LM head does not fit the TILED layout");
            return fail();
        }
        const size_t lb = d->lm_layout == LAYOUT_TILED ? q_tiled_bytes(c.lm_dtype, c.vocab, H)
                                                       : q_packed_bytes(c.lm_dtype, c.vocab, H);
        void *lm = nullptr;
        ok = ok && dev_alloc(d, &lm, lb, "lm") &&
             (d->lm_layout == LAYOUT_TILED ? launch_to_tiled(c.lm_dtype, aos, c.vocab, H, lm, d->stream)
                                           : launch_repack(c.lm_dtype, aos, c.vocab, H, lm, d->stream)) == 0 &&
             hip_ok(hipStreamSynchronize(d->stream), "lm repack");
        (void)hipFree(aos);
        if (!ok) return fail();
        d->lm = lm;
        const size_t sb = d->lm_layout == LAYOUT_TILED ? tiled_softmax_scratch_bytes(c.vocab)
                                                       : softmax_scratch_floats(c.vocab) * sizeof(float);
        if (!dev_alloc(d, &d->lm_scratch, sb, "lm scratch")) return fail();
    }
    // RoPE tables and the KV caches
    {
        std::vector<float> cs, sn;
        rope_tables(hd, c.max_ctx, c.rope_theta, cs, sn);
        if (!(d->cos_g = const_cast<float *>(upload_f32(d, cs.data(), cs.size(), "rope"))) ||
            !(d->sin_g = const_cast<float *>(upload_f32(d, sn.data(), sn.size(), "rope"))))
            return fail();
        std::vector<float> cl, sl;
        rope_tables(hd, c.max_ctx, c.rope_local_base, cl, sl);
        if (!(d->cos_l = const_cast<float *>(upload_f32(d, cl.data(), cl.size(), "rope"))) ||
            !(d->sin_l = const_cast<float *>(upload_f32(d, sl.data(), sl.size(), "rope"))))
            return fail();
        if (B == 1) {
            // the persistent step's copy, one row per position: [pos][global cos | global sin |
            // local cos | local sin][hd], so a step reads one 4*hd row instead of four tables
            std::vector<float> il((size_t)c.max_ctx * 4 * hd);
            for (int p = 0; p < c.max_ctx; ++p) {
                const size_t r = (size_t)p * hd;
                float *o = il.data() + (size_t)p * 4 * hd;
                memcpy(o, cs.data() + r, sizeof(float) * hd);
                memcpy(o + hd, sn.data() + r, sizeof(float) * hd);
                memcpy(o + 2 * hd, cl.data() + r, sizeof(float) * hd);
                memcpy(o + 3 * hd, sl.data() + r, sizeof(float) * hd);
            }
            if (!(d->rope_rows = upload_f32(d, il.data(), il.size(), "rope rows"))) return fail();
        }
    }
    const size_t kv = (size_t)B * c.n_layers * c.n_kv_heads * c.max_ctx * hd;
    if (!dev_alloc_t(d, &d->kc, kv, "k cache") || !dev_alloc_t(d, &d->vc, kv, "v cache") ||
        !hip_ok(hipMemset(d->kc, 0, kv * sizeof(float)), "kv zero") ||
        !hip_ok(hipMemset(d->vc, 0, kv * sizeof(float)), "kv zero"))
        return fail();
    const size_t b = (size_t)B;
    // a batched step keeps the attention output and the GeGLU output in block order (16 slots)
    const size_t bo = B > 1 ? (size_t)kGemmSeqs : b;
    if (!dev_alloc_t(d, &d->resid[0], b * H, "resid") || !dev_alloc_t(d, &d->resid[1], b * H, "resid") ||
        !dev_alloc_t(d, &d->qkv, b * (nq + 2 * nk), "qkv") || !dev_alloc_t(d, &d->attn, bo * nq, "attn") ||
        !dev_alloc_t(d, &d->o, b * H, "o") || !dev_alloc_t(d, &d->g, bo * c.ffn, "g") ||
        !dev_alloc_t(d, &d->ffn_out, H, "ffn_out") || !dev_alloc_t(d, &d->xfin, b * H, "xfin") ||
        !dev_alloc_t(d, &d->logits, b * c.vocab, "logits") ||
        !dev_alloc_t(d, &d->attn_part, b * attn_part_floats(c.n_heads, hd), "attn partials") ||
        !dev_alloc_t(d, &d->state, 3 * b + 2, "state") || !dev_alloc_t(d, &d->log, (size_t)c.max_ctx * b, "token log") ||
        !dev_alloc_t(d, &d->gkeys, tiled_greedy_key_slots(c.vocab), "greedy keys") ||
        !dev_alloc_t(d, &d->gcount, 1 + kGreedyGroups, "greedy counters") ||
        !hip_ok(hipMemset(d->gcount, 0, (1 + kGreedyGroups) * sizeof(unsigned)), "greedy counters zero") ||
        !hip_ok(hipDeviceSynchronize(), "greedy counters zero"))
        return fail();
    if (B > 1 || d->pf_ok) {
        const size_t wsb = std::max({gemm_workspace_bytes(H, c.ffn), gemm_workspace_bytes(H, nq),
                                     gemm_workspace_bytes(c.vocab, H)});
        if (!dev_alloc(d, &d->gws, wsb, "gemm workspace")) return fail();
    }
    if (B > 1) {
        if (!dev_alloc_t(d, &d->dparts, (size_t)gemm_splits(c.ffn) * b * H, "down partials") ||
            !dev_alloc_t(d, &d->dout, b * H, "down output") ||
            !dev_alloc_t(d, &d->amax_part, argmax_batch_part_floats(c.vocab, B), "argmax partials"))
            return fail();
        const uint32_t one = 1;
        if (const char *e = getenv("SAPPHIRE_FUSED_QKV_ATTN")) d->fuse_qkv_attn = atoi(e) != 0;
        if (!dev_alloc_t(d, &d->tqkv, b * (nq + 2 * nk), "tagged qkv") ||
            !hip_ok(hipMemset(d->tqkv, 0, b * (nq + 2 * nk) * sizeof(uint64_t)), "tagged qkv zero") ||
            !dev_alloc_t(d, &d->bepoch, 1, "step counter") ||
            !hip_ok(hipMemcpy(d->bepoch, &one, sizeof(uint32_t), hipMemcpyHostToDevice), "step counter") ||
            (!d->perr && (!dev_alloc_t(d, &d->perr, 1, "timeout counter") ||
                          !hip_ok(hipMemset(d->perr, 0, sizeof(int)), "timeout zero"))) ||
            !hip_ok(hipDeviceSynchronize(), "batched state zero"))
            return fail();
    }
    if (d->pf_ok) {
        const size_t p = kPrefillChunk;
        if (!dev_alloc_t(d, &d->pf_resid[0], p * H, "prefill resid") ||
            !dev_alloc_t(d, &d->pf_resid[1], p * H, "prefill resid") ||
            !dev_alloc_t(d, &d->pf_qkv, p * (nq + 2 * nk), "prefill qkv") ||
            !dev_alloc_t(d, &d->pf_attn, p * nq, "prefill attn") || !dev_alloc_t(d, &d->pf_o, p * H, "prefill o") ||
            !dev_alloc_t(d, &d->pf_g, p * c.ffn, "prefill g") ||
            !dev_alloc_t(d, &d->pf_dparts, (size_t)gemm_splits(c.ffn) * p * H, "prefill partials") ||
            !dev_alloc_t(d, &d->pf_dout, p * H, "prefill down") ||
            !dev_alloc_t(d, &d->pf_part, p * attn_part_floats(c.n_heads, hd), "prefill attention partials") ||
            !dev_alloc_t(d, &d->pf_tok, 2 * p, "prefill tokens"))
            return fail();
    }
    if (B == 1 && !setup_persistent(d)) return fail();
    // the zero fills above run on the null stream; the decoder's stream does not wait for it
    if (!hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize")) return fail();
    return d;
}

// Workgroups of the persistent step unless SAPPHIRE_DECODE_WORKGROUPS says otherwise.
constexpr int kDefaultGroups = 128;

// Device resources of the persistent step (one sequence) and its default workgroup count:
// kDefaultGroups when the shapes and the device allow it, else 0 (the multi-launch step).
bool setup_persistent(sapphire_decoder *d) {
    const auto &c = d->cfg;
    const int hd = c.head_dim, win = c.sliding_window > 0 ? c.sliding_window : 1024;
    const size_t layer_kv = (size_t)c.n_kv_heads * c.max_ctx * hd;
    std::vector<PLayer> pl((size_t)c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer &L = d->layers[l];
        PLayer &P = pl[l];
        P.qkv = L.qkv;
        P.o = L.o;
        P.gate = L.gate;
        P.up = L.up;
        P.down = L.down;
        P.n_attn = L.n_attn;
        P.n_attn_post = L.n_attn_post;
        P.n_ffn = L.n_ffn;
        P.n_ffn_post = L.n_ffn_post;
        P.qn = L.qn;
        P.kn = L.kn;
        // rows of 4 * hd: global cos, global sin, local cos, local sin
        P.cos_t = d->rope_rows + (L.global ? 0 : 2 * hd);
        P.sin_t = P.cos_t + hd;
        P.kc = d->kc + (size_t)l * layer_kv;
        P.vc = d->vc + (size_t)l * layer_kv;
        P.window = L.global ? 0 : win;
    }
    d->tbuf_words = persist_words(c.hidden, c.n_heads, c.n_kv_heads, hd, c.ffn);
    if (!dev_alloc_t(d, &d->players, pl.size(), "layer descriptors") ||
        !hip_ok(hipMemcpy(d->players, pl.data(), sizeof(PLayer) * pl.size(), hipMemcpyHostToDevice), "descriptors") ||
        !dev_alloc_t(d, &d->tbuf, d->tbuf_words, "exchange buffers") ||
        !hip_ok(hipMemset(d->tbuf, 0, d->tbuf_words * sizeof(uint64_t)), "exchange zero") ||
        !dev_alloc_t(d, &d->seq, 1, "epoch counter") || !hip_ok(hipMemset(d->seq, 0, sizeof(uint32_t)), "epoch zero") ||
        !dev_alloc_t(d, &d->tslots, 1, "token slots") ||
        !hip_ok(hipMemset(d->tslots, 0, sizeof(TokenSlots)), "token slots zero") ||
        !dev_alloc_t(d, &d->perr, 1, "timeout counter") || !hip_ok(hipMemset(d->perr, 0, sizeof(int)), "timeout zero"))
        return false;
    if (const char *e = getenv("SAPPHIRE_TOKEN_SLOT_RUN")) d->slot_run = std::min(std::max(atoi(e), 1), kSlotRunSteps);
    int g = kDefaultGroups;
    if (const char *e = getenv("SAPPHIRE_DECODE_WORKGROUPS")) g = atoi(e);
    d->groups = g > 0 && persist_supported(c.wdtype, g, c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, hd, c.ffn) ? g : 0;
    return true;
}

size_t seq_kv_floats(const sapphire_decoder_config_t &c) {
    return (size_t)c.n_layers * c.n_kv_heads * c.max_ctx * c.head_dim;
}

int kv_copy(sapphire_decoder_t *d, int seq, int nseq, const float *k_in, const float *v_in, float *k_out,
            float *v_out) {
    const size_t n = seq_kv_floats(d->cfg), off = (size_t)seq * n, bytes = (size_t)nseq * n * sizeof(float);
    SPH_CHECK(hipSetDevice(d->device));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    if (k_in) {
        SPH_CHECK(hipMemcpy(d->kc + off, k_in, bytes, hipMemcpyHostToDevice));
        SPH_CHECK(hipMemcpy(d->vc + off, v_in, bytes, hipMemcpyHostToDevice));
    } else {
        SPH_CHECK(hipMemcpy(k_out, d->kc + off, bytes, hipMemcpyDeviceToHost));
        SPH_CHECK(hipMemcpy(v_out, d->vc + off, bytes, hipMemcpyDeviceToHost));
    }
    return 0;
}

}  // namespace

extern "C" {

sapphire_decoder_t *sapphire_decoder_create(const sapphire_decoder_config_t *cfg, const sapphire_decoder_weights_t *w) {
    return create_decoder(cfg, w, 1);
}

sapphire_decoder_t *sapphire_decoder_create_batch(const sapphire_decoder_config_t *cfg,
                                                  const sapphire_decoder_weights_t *w, int batch) {
    return create_decoder(cfg, w, batch);
}

int sapphire_decoder_batch(const sapphire_decoder_t *d) { return d ? d->batch : 0; }

int sapphire_decoder_set_kv(sapphire_decoder_t *d, const float *k, const float *v) {
    if (!d || !k || !v) {
        set_error("sapphire_decoder_set_kv: NULL argument");
        return -1;
    }
    return kv_copy(d, 0, d->batch, k, v, nullptr, nullptr);
}

int sapphire_decoder_get_kv(sapphire_decoder_t *d, float *k, float *v) {
    if (!d || !k || !v) {
        set_error("sapphire_decoder_get_kv: NULL argument");
        return -1;
    }
    return kv_copy(d, 0, d->batch, nullptr, nullptr, k, v);
}

int sapphire_decoder_set_kv_seq(sapphire_decoder_t *d, int seq, const float *k, const float *v) {
    if (!d || !k || !v || seq < 0 || seq >= d->batch) {
        set_error("sapphire_decoder_set_kv_seq: bad arguments");
        return -1;
    }
    return kv_copy(d, seq, 1, k, v, nullptr, nullptr);
}

int sapphire_decoder_get_kv_seq(sapphire_decoder_t *d, int seq, float *k, float *v) {
    if (!d || !k || !v || seq < 0 || seq >= d->batch) {
        set_error("sapphire_decoder_get_kv_seq: bad arguments");
        return -1;
    }
    return kv_copy(d, seq, 1, nullptr, nullptr, k, v);
}

int sapphire_decoder_generate_batch(sapphire_decoder_t *d, const int *tokens, const int *pos, int steps,
                                    int *tokens_out, float *logits_out, float *elapsed_ms) {
    if (!d || !tokens || !pos || !tokens_out || steps <= 0) {
        set_error("sapphire_decoder_generate: bad arguments");
        return -1;
    }
    const auto &c = d->cfg;
    const int B = d->batch;
    for (int b = 0; b < B; ++b)
        if (tokens[b] < 0 || tokens[b] >= c.vocab || pos[b] < 0 || pos[b] + steps > c.max_ctx) {
            set_error("sapphire_decoder_generate: sequence %d: token %d / positions %d..%d out of range", b, tokens[b],
                      pos[b], pos[b] + steps - 1);
            return -1;
        }
    if (d->temperature > 0.0f && (size_t)steps * B > (size_t)d->n_draws) {
        set_error("sapphire_decoder_generate: %d steps of %d sequences need %d draws, %d were set", steps, B,
                  steps * B, d->n_draws);
        return -1;
    }
    SPH_CHECK(hipSetDevice(d->device));
    const bool want_logits = logits_out != nullptr || B == 1;
    if (d->exec && d->graph_logits != want_logits) drop_step_graphs(d);   // the LM head changes form
    // n steps back to back as one graph (every step's state lives on the device)
    auto capture = [&](int n, hipGraph_t *graph, hipGraphExec_t *exec) -> int {
        SPH_CHECK(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
        int rc = 0;
        for (int i = 0; i < n && rc == 0; ++i) rc = B == 1 ? enqueue_step(d) : enqueue_step_batch(d);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(d->stream, &g);
        if (rc != 0 || !hip_ok(e, "hipStreamEndCapture")) {
            if (g) (void)hipGraphDestroy(g);
            return -1;
        }
        *graph = g;
        SPH_CHECK(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
        return 0;
    };
    if (!d->exec) {
        d->graph_logits = want_logits;
        d->graph_slots = B == 1 && use_token_slots(d);
        if (capture(1, &d->graph, &d->exec) != 0) return -1;
    }
    // a persistent-form call that takes no logits runs its steps kMultiSteps to a launch where
    // it can (a batched step's graph of ~190 kernels measured slower captured eight times over)
    const bool multi = logits_out == nullptr && B == 1 && d->groups > 0 && steps >= kMultiSteps;
    if (multi && !d->exec_multi && capture(kMultiSteps, &d->graph_multi, &d->exec_multi) != 0) return -1;
    // state: token, position, step (one sequence) or tokens[B], positions[B], step; every done
    // flag clear
    std::vector<int> st((size_t)3 * B + 2, 0);
    if (B == 1) {
        st[0] = tokens[0];
        st[1] = pos[0];
    } else {
        for (int b = 0; b < B; ++b) {
            st[b] = tokens[b];
            st[B + b] = pos[b];
        }
    }
    SPH_CHECK(hipMemcpy(d->state, st.data(), sizeof(int) * st.size(), hipMemcpyHostToDevice));
    // with stop tokens, the steps after a sequence's stop log nothing: their entries read -1
    if (d->stop.n > 0) SPH_CHECK(hipMemsetAsync(d->log, 0xFF, sizeof(int) * (size_t)steps * B, d->stream));
    if (d->groups > 0) {
        // epochs must stay below 2^32: start them over (and clear every tag) before they would wrap
        const uint64_t per = persist_epochs_per_step(c.n_layers);
        if ((d->persist_steps + (uint64_t)steps + 1) * per > 0xFFFFFFFFull) {
            SPH_CHECK(hipMemsetAsync(d->tbuf, 0, d->tbuf_words * sizeof(uint64_t), d->stream));
            d->persist_steps = 0;
        }
        // the call's steps take the epoch counter from here on (one per step, whichever form
        // advances it)
        const uint32_t seq0 = (uint32_t)d->persist_steps;
        SPH_CHECK(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(d->seq), (int)seq0, 1, d->stream));
        if (d->graph_slots) {
            TokenSlots ts{};
            ts.tok0 = tokens[0];
            ts.pos0 = pos[0];
            ts.seq0 = seq0;
            SPH_CHECK(hipMemcpyAsync(d->tslots, &ts, sizeof(ts), hipMemcpyHostToDevice, d->stream));
            SPH_CHECK(hipStreamSynchronize(d->stream));   // ts is a local
        }
        SPH_CHECK(hipMemsetAsync(d->perr, 0, sizeof(int), d->stream));
        d->persist_steps += (uint64_t)steps;
    }
    if (B > 1) {
        // the fused QKV + attention launch tags its words with (step counter << 6) + layer + 1:
        // the counter starts over at 1 (and every word is cleared) before it would pass 2^26
        if (d->bepoch_steps + (uint64_t)steps + 1 >= kBatchEpochLimit) {
            SPH_CHECK(hipMemsetAsync(d->tqkv, 0, (size_t)B * batch_qkv_width(c) * sizeof(uint64_t), d->stream));
            SPH_CHECK(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(d->bepoch), 1, 1, d->stream));
            d->bepoch_steps = 0;
        }
        SPH_CHECK(hipMemsetAsync(d->perr, 0, sizeof(int), d->stream));
        d->bepoch_steps += (uint64_t)steps;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (elapsed_ms) {
        SPH_CHECK(hipEventCreate(&e0));
        SPH_CHECK(hipEventCreate(&e1));
        SPH_CHECK(hipEventRecord(e0, d->stream));
    }
    // a batched step that ends by looking up the next step's input rows needs the first's
    if (B > 1 && d->graph_embeds_next &&
        dec_embed_batch(d->embed, c.hidden, c.vocab, sqrtf((float)c.hidden), d->state, B, d->resid[0], d->stream) != 0)
        return -1;
    const size_t lstep = (size_t)B * c.vocab;
    for (int s = 0; s < steps;) {
        // kMultiSteps at once where they fit in the call and (token slots) inside one run
        const bool many = multi && s + kMultiSteps <= steps &&
                          (!d->graph_slots || s % d->slot_run + kMultiSteps <= d->slot_run);
        SPH_CHECK(hipGraphLaunch(many ? d->exec_multi : d->exec, d->stream));
        if (logits_out)
            SPH_CHECK(hipMemcpyAsync(logits_out + (size_t)s * lstep, d->logits, sizeof(float) * lstep,
                                     hipMemcpyDeviceToHost, d->stream));
        s += many ? kMultiSteps : 1;
        // token slots: a run's last token is logged after its last step
        if (d->graph_slots && (s % d->slot_run == 0 || s == steps) &&
            launch_token_slots_settle(d->tslots, c.vocab, d->log, done_flags(d), d->stop, d->perr, d->stream) != 0)
            return -1;
    }
    if (elapsed_ms) SPH_CHECK(hipEventRecord(e1, d->stream));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    if (elapsed_ms) {
        SPH_CHECK(hipEventElapsedTime(elapsed_ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
    }
    if (d->groups > 0 || B > 1) {
        int timeouts = 0;
        SPH_CHECK(hipMemcpy(&timeouts, d->perr, sizeof(int), hipMemcpyDeviceToHost));
        if (timeouts) {
            set_error("sapphire_decoder_generate: %d persistent-step waits timed out (or a step found no token); "
                      "results are invalid", timeouts);
            return -1;
        }
    }
    SPH_CHECK(hipMemcpy(tokens_out, d->log, sizeof(int) * (size_t)steps * B, hipMemcpyDeviceToHost));
    return 0;
}

int sapphire_decoder_set_workgroups(sapphire_decoder_t *d, int groups) {
    if (!d || groups < 0) {
        set_error("sapphire_decoder_set_workgroups: bad arguments");
        return -1;
    }
    if (groups > 0) {
        const auto &c = d->cfg;
        if (d->batch != 1) {
            set_error("sapphire_decoder_set_workgroups: the persistent step decodes one sequence");
            return -1;
        }
        SPH_CHECK(hipSetDevice(d->device));
        if (!persist_supported(c.wdtype, groups, c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn)) return -1;
    }
    if (groups == d->groups) return 0;
    SPH_CHECK(hipStreamSynchronize(d->stream));
    drop_step_graphs(d);
    d->groups = groups;
    return 0;
}

int sapphire_decoder_workgroups(const sapphire_decoder_t *d) { return d ? d->groups : -1; }

int sapphire_decoder_set_epoch_count(sapphire_decoder_t *d, uint32_t steps) {
    if (!d) {
        set_error("sapphire_decoder_set_epoch_count: bad arguments");
        return -1;
    }
    if (d->batch > 1) {
        if ((uint64_t)steps + 1 >= kBatchEpochLimit) {
            set_error("sapphire_decoder_set_epoch_count: %u steps are past the step counter's range", steps);
            return -1;
        }
        SPH_CHECK(hipSetDevice(d->device));
        SPH_CHECK(hipStreamSynchronize(d->stream));
        const uint32_t e = steps + 1u;
        SPH_CHECK(hipMemset(d->tqkv, 0, (size_t)d->batch * batch_qkv_width(d->cfg) * sizeof(uint64_t)));
        SPH_CHECK(hipMemcpy(d->bepoch, &e, sizeof(uint32_t), hipMemcpyHostToDevice));
        d->bepoch_steps = steps;
        return 0;
    }
    if (d->groups <= 0) return 0;
    if ((uint64_t)(steps + 1ull) * persist_epochs_per_step(d->cfg.n_layers) > 0xFFFFFFFFull) {
        set_error("sapphire_decoder_set_epoch_count: %u steps are past the epoch range", steps);
        return -1;
    }
    SPH_CHECK(hipSetDevice(d->device));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    // every exchange word is stale (tag 0) for any epoch above 0; the device counter and the
    // host's count of steps since the last reset move together
    SPH_CHECK(hipMemset(d->tbuf, 0, d->tbuf_words * sizeof(uint64_t)));
    SPH_CHECK(hipMemcpy(d->seq, &steps, sizeof(uint32_t), hipMemcpyHostToDevice));
    d->persist_steps = steps;
    return 0;
}

int sapphire_decoder_set_sampling(sapphire_decoder_t *d, float temperature, const float *draws, int n_draws) {
    if (!d || temperature != temperature || (temperature > 0.0f && (!draws || n_draws <= 0))) {
        set_error("sapphire_decoder_set_sampling: bad arguments");
        return -1;
    }
    const auto &c = d->cfg;
    const int B = d->batch;
    SPH_CHECK(hipSetDevice(d->device));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    if (temperature > 0.0f) {
        if (!sample_supported(c.vocab, B)) {
            set_error("sapphire_decoder_set_sampling: vocabulary %d too large to sample", c.vocab);
            return -1;
        }
        if ((size_t)n_draws > (size_t)c.max_ctx * B) {
            set_error("sapphire_decoder_set_sampling: at most max_ctx * batch = %zu draws", (size_t)c.max_ctx * B);
            return -1;
        }
        if (!d->smp_w && (!dev_alloc_t(d, &d->smp_w, (size_t)B * c.vocab, "sampling weights") ||
                          !dev_alloc(d, &d->smp_ws, sample_workspace_bytes(c.vocab, B), "sampling workspace") ||
                          !dev_alloc_t(d, &d->draws, (size_t)c.max_ctx * B, "draws"))) {
            d->smp_w = nullptr;
            return -1;
        }
        SPH_CHECK(hipMemcpy(d->draws, draws, sizeof(float) * n_draws, hipMemcpyHostToDevice));
    }
    const float t = temperature > 0.0f ? temperature : 0.0f;
    d->n_draws = t > 0.0f ? n_draws : 0;
    if (t != d->temperature) {
        // the step's kernels (and the temperature in their arguments) change: capture again
        drop_step_graphs(d);
        d->temperature = t;
    }
    return 0;
}

int sapphire_decoder_set_stop_tokens(sapphire_decoder_t *d, const int *ids, int n) {
    if (!d || n < 0 || n > kMaxStop || (n > 0 && !ids)) {
        set_error("sapphire_decoder_set_stop_tokens: bad arguments (at most %d tokens)", kMaxStop);
        return -1;
    }
    StopSet st;
    st.n = n;
    for (int i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= d->cfg.vocab) {
            set_error("sapphire_decoder_set_stop_tokens: token %d outside the vocabulary", ids[i]);
            return -1;
        }
        st.id[i] = ids[i];
    }
    SPH_CHECK(hipSetDevice(d->device));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    // the set is an argument of the step's advance: capture again
    drop_step_graphs(d);
    d->stop = st;
    return 0;
}

int sapphire_decoder_prefill(sapphire_decoder_t *d, int seq, const int *tokens, int n, int pos, float *elapsed_ms) {
    if (!d || !tokens || n <= 0 || seq < 0 || seq >= d->batch || pos < 0 || pos + n > d->cfg.max_ctx) {
        set_error("sapphire_decoder_prefill: bad arguments (sequence %d, %d tokens at position %d)", seq, n, pos);
        return -1;
    }
    if (!d->pf_ok) {
        set_error("sapphire_decoder_prefill: needs hidden, n_heads*head_dim and ffn multiples of 128, hidden <= 1152");
        return -1;
    }
    const auto &c = d->cfg;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.vocab) {
            set_error("sapphire_decoder_prefill: token %d (%d) outside the vocabulary", i, tokens[i]);
            return -1;
        }
    SPH_CHECK(hipSetDevice(d->device));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    // per chunk: its tokens, then its positions (the host array outlives the stream's reads)
    const int nchunks = (n + kPrefillChunk - 1) / kPrefillChunk;
    std::vector<int> host((size_t)nchunks * 2 * kPrefillChunk, 0);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (elapsed_ms) {
        SPH_CHECK(hipEventCreate(&e0));
        SPH_CHECK(hipEventCreate(&e1));
        SPH_CHECK(hipEventRecord(e0, d->stream));
    }
    const size_t seq_kv = (size_t)c.n_layers * c.n_kv_heads * c.max_ctx * c.head_dim;
    for (int k = 0; k < nchunks; ++k) {
        const int c0 = k * kPrefillChunk, m = std::min(kPrefillChunk, n - c0);
        int *h = host.data() + (size_t)k * 2 * kPrefillChunk;
        for (int i = 0; i < m; ++i) {
            h[i] = tokens[c0 + i];
            h[kPrefillChunk + i] = pos + c0 + i;
        }
        SPH_CHECK(hipMemcpyAsync(d->pf_tok, h, sizeof(int) * 2 * kPrefillChunk, hipMemcpyHostToDevice, d->stream));
        BatchRun r;
        const bool full = m == kPrefillChunk;
        r.B = m;
        r.d_tokens = d->pf_tok;
        r.d_pos = d->pf_tok + kPrefillChunk;
        r.kc = d->kc + (size_t)seq * seq_kv;
        r.vc = d->vc + (size_t)seq * seq_kv;
        r.kv_stride = 0;
        r.prefill = true;
        r.resid[0] = d->pf_resid[0];
        r.resid[1] = d->pf_resid[1];
        r.qkv = d->pf_qkv;
        r.attn = d->pf_attn;
        r.o = d->pf_o;
        r.g = d->pf_g;
        r.dparts = d->pf_dparts;
        r.dout = d->pf_dout;
        r.part = d->pf_part;
        r.gws = d->gws;
        if (!full) {   // the last, shorter chunk runs its launches directly
            if (enqueue_layers_batch(d, r) < 0) return -1;
            continue;
        }
        // a full chunk replays the sequence's captured pass (tokens and positions are device data)
        if (d->pf_exec.empty()) {
            d->pf_graph.assign((size_t)d->batch, nullptr);
            d->pf_exec.assign((size_t)d->batch, nullptr);
        }
        if (!d->pf_exec[seq]) {
            SPH_CHECK(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue_layers_batch(d, r);
            hipGraph_t g = nullptr;
            const hipError_t e = hipStreamEndCapture(d->stream, &g);
            if (rc < 0 || !hip_ok(e, "hipStreamEndCapture")) {
                if (g) (void)hipGraphDestroy(g);
                return -1;
            }
            d->pf_graph[seq] = g;
            SPH_CHECK(hipGraphInstantiate(&d->pf_exec[seq], g, nullptr, nullptr, 0));
        }
        SPH_CHECK(hipGraphLaunch(d->pf_exec[seq], d->stream));
    }
    if (elapsed_ms) SPH_CHECK(hipEventRecord(e1, d->stream));
    SPH_CHECK(hipStreamSynchronize(d->stream));
    if (elapsed_ms) {
        SPH_CHECK(hipEventElapsedTime(elapsed_ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
    }
    return 0;
}

int sapphire_decoder_generate(sapphire_decoder_t *d, int token, int pos, int steps, int *tokens_out, float *logits_out,
                              float *elapsed_ms) {
    if (d && d->batch != 1) {
        set_error("sapphire_decoder_generate: a batched decoder takes sapphire_decoder_generate_batch");
        return -1;
    }
    return sapphire_decoder_generate_batch(d, &token, &pos, steps, tokens_out, logits_out, elapsed_ms);
}

}  // extern "C"
