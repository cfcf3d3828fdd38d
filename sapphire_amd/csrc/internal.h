// internal.h - shared declarations of libsapphire_hip.so (not installed).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>

namespace sapphire {

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_Q4_0 = 3, DT_Q8_0 = 4 };
enum : int { LAYOUT_AOS = 0, LAYOUT_PACKED = 1, LAYOUT_TILED = 2 };

constexpr int kBlock = 32;                      // weights per quant block
constexpr int kTiledMinRows = 16384;            // weight matrices this long use the TILED layout
inline int quant_bytes(int dt) { return dt == DT_Q4_0 ? 16 : 32; }   // payload per block
inline int block_bytes(int dt) { return dt == DT_Q4_0 ? 20 : 36; }   // AoS block size
inline bool is_quant(int dt) { return dt == DT_Q4_0 || dt == DT_Q8_0; }

// Error reporting: the last message is kept per thread and also written to stderr.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
bool hip_ok(hipError_t e, const char *what);

#define SPH_CHECK(expr)                                   \
    do {                                                  \
        if (!::sapphire::hip_ok((expr), #expr)) return -1; \
    } while (0)

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ---- kernel launchers (device pointers, stream ordered); return 0 / -1 ----
size_t q_aos_bytes(int dt, int M, int K);
size_t q_scales_offset(int dt, int M, int K);
size_t q_packed_bytes(int dt, int M, int K);
int launch_repack(int dt, const void *aos, int M, int K, void *packed, hipStream_t s);
int launch_unpack_ints(int dt, int layout, const void *w, int M, int K, int8_t *out, hipStream_t s);
int launch_dequant(int dt, int layout, const void *w, int M, int K, float *out, hipStream_t s);
int launch_gemv_q(int dt, int layout, const void *w, int M, int K, const float *x, float *y, hipStream_t s);
int launch_gemm_q(int dt, int layout, const void *w, int M, int K, const float *X, float *Y, int batch,
                  hipStream_t s);
// TILED layout + matrix-core GEMV (gemv_mfma.hip). The layout needs K % 128 == 0 and
// fewer than 4 GiB (tiled_layout_ok); the GEMV also needs K/128 in {5, 8, 9} (tiled_supported).
bool tiled_layout_ok(int dt, int M, int K);
bool tiled_supported(int dt, int M, int K);
size_t q_tiled_scales_offset(int dt, int M, int K);
size_t q_tiled_bytes(int dt, int M, int K);
int launch_to_tiled(int dt, const void *aos, int M, int K, void *out, hipStream_t s);
int launch_tiled_unpack(int dt, const void *w, int M, int K, int8_t *ints, float *deq, hipStream_t s);
int launch_gemv_tiled(int dt, const void *w, int M, int K, const float *x, float *y, hipStream_t s);
// TILED GEMV with the softmax epilogue: logits, then probs (if not NULL) and the greedy
// token (if not NULL). scratch: tiled_softmax_scratch_bytes(M) bytes of device memory for
// the per-workgroup partials.
size_t tiled_softmax_scratch_bytes(int M);
int launch_gemv_tiled_softmax(int dt, const void *w, int M, int K, const float *x, float *logits, float *probs,
                              int *argmax, void *scratch, hipStream_t s);
// The decode state a greedy LM head advances (dec_advance_kernel's work). keys: one slot per
// workgroup (tiled_greedy_key_slots); count: 1 + kGreedyGroups counters that are 0 before the
// first launch and that every launch leaves at 0.
constexpr int kGreedyGroups = 8;
// Tokens that end a sequence (inference.c:298-301 stops on 1 and 106): the advance that logs
// one sets the sequence's done flag; later steps log nothing, advance nothing and skip their
// work (their log entries keep the caller's fill).
constexpr int kMaxStop = 8;
struct StopSet {
    int n = 0;
    int id[kMaxStop] = {};
    __host__ __device__ bool has(int t) const {
        bool r = false;
        for (int i = 0; i < kMaxStop; ++i) r |= i < n && id[i] == t;
        return r;
    }
};
struct TokenSlots;
struct GreedyStep {
    unsigned long long *keys = nullptr;  // each workgroup's best greedy key
    unsigned *count = nullptr;           // [0] groups done, [1 + g] workgroups of group g done
    int *tok = nullptr, *pos = nullptr, *step = nullptr, *log = nullptr;
    uint32_t *seq = nullptr;             // the persistent step's counter (may be NULL)
    int *done = nullptr;                 // the sequence's done flag (may be NULL): set, the launch does nothing
    StopSet stop;
    TokenSlots *slots = nullptr;         // set: the token goes through these (launch_gemv_tiled_greedy_slots)
};
size_t tiled_greedy_key_slots(int M);
// TILED GEMV whose epilogue writes the logits, picks the greedy token (sample_greedy's
// order) into *tok and log[*step], and advances *pos, *step and *seq (and sets *done when
// the token is in gs.stop): one launch for the LM head, the argmax and the advance. With
// *done set it returns at once. Launches that share the state must be ordered.
int launch_gemv_tiled_greedy_step(int dt, const void *w, int M, int K, const float *x, float *logits,
                                  const GreedyStep &gs, hipStream_t s);

// The greedy token handed from a step's LM head to the next step's layers kernel without a
// reduction inside the LM head. Its workgroups fold the greedy key of their rows into 64
// slots by atomic maxima (workgroup b into slot b mod 64, so that no address takes more than a
// few of them: atomics on one address from every XCD serialize), each key tagged with the step,
// so that the slots need no clearing between steps; the next step's layers kernel takes the
// largest, decodes the token, logs it and stops the sequence on a stop token. Two step words
// alternate, so that no launch writes a word its own workgroups read: the layers kernel reads
// `a` (steps of this run whose LM head has run) and writes b = a + 1; the LM head reads b, its
// tag, and writes a = b. A run covers at most kSlotRunSteps steps; launch_token_slots_settle
// logs a run's last token and starts the next run from it.
constexpr int kSlotIndexBits = 18, kSlotTagBits = 64 - 32 - kSlotIndexBits;
constexpr int kSlotMaxVocab = 1 << kSlotIndexBits;
constexpr int kSlotRunSteps = (1 << kSlotTagBits) - 1;
constexpr int kSlotCount = 64;               // one per lane of a wave, which reads them all at once
struct TokenSlots {
    unsigned long long key[kSlotCount];      // tag << 50 | ordered value << 18 | (2^18 - 1 - index)
    uint32_t a, b;
    int tok0, pos0;                          // the run's first token and position
    uint32_t seq0;                           // the persistent step's epoch counter at the run's start
    int logbase;                             // log index of the run's first step
};
// A slot key from greedy_key's (ordered value << 32 | ~index) for rows below kSlotMaxVocab.
__host__ __device__ inline unsigned long long slot_key(unsigned long long gk, uint32_t tag) {
    constexpr unsigned long long lo = (1ull << (64 - kSlotTagBits)) - 1;
    const unsigned long long body = gk ? ((gk >> 32) << kSlotIndexBits) | (gk & (kSlotMaxVocab - 1)) : 0ull;
    return ((unsigned long long)tag << (64 - kSlotTagBits)) | (body & lo);
}
// The token of the largest slot key k, which must carry `tag` (0 when no row had a key, as
// sample_greedy starts at index 0); false when it carries another tag.
__host__ __device__ inline bool slot_token(unsigned long long k, uint32_t tag, int vocab, int &tok) {
    constexpr unsigned long long lo = (1ull << (64 - kSlotTagBits)) - 1;
    const int r = (kSlotMaxVocab - 1) - (int)(k & (kSlotMaxVocab - 1));
    tok = (k & lo) != 0 && r < vocab ? r : 0;
    return (uint32_t)(k >> (64 - kSlotTagBits)) == tag;
}
// The TILED LM head of a persistent step whose token goes through `slots` (gs.done, if set,
// makes it return at once; gs.keys, count, tok, pos, step and log are not used).
int launch_gemv_tiled_greedy_slots(int dt, const void *w, int M, int K, const float *x, float *logits,
                                   TokenSlots *slots, const int *done, hipStream_t s);
// After a run's last step: logs its last token (log[logbase + a - 1]; done set on a stop token)
// and makes it the next run's first (tok0, pos0 + a, seq0 + a, logbase + a, a = b = 0, slots
// cleared). Does nothing once done is set; counts *err when the slots do not carry the run's
// last tag.
int launch_token_slots_settle(TokenSlots *slots, int vocab, int *log, int *done, const StopSet &stop, int *err,
                              hipStream_t s);
// Batched GEMM on the TILED layout (gemm_mfma.hip): Y[b][r] = W[r] . X[b] for b < batch, 16
// sequences per pass. ws: gemm_workspace_bytes(M, K) bytes of 256-byte aligned device memory
// (the K-split partial sums). Calls sharing a workspace must be ordered.
size_t gemm_workspace_bytes(int M, int K);
int launch_gemm_tiled(int dt, const void *w, int M, int K, const float *X, int batch, float *Y, void *ws,
                      hipStream_t s);
// Number of K chunks (partial sums) of a batched GEMM with inner dimension K.
int gemm_splits(int K);
// Sequences of one batched GEMM pass.
constexpr int kGemmSeqs = 16;
// The block order of a batched GEMM's activations: element k of sequence s (s < 16) at
// (k / 32) * 512 + ((k / 8) % 4) * 128 + s * 8 + k % 8, the order in which a K chunk's
// matrix-core operands sit (so a GEMM stages it with contiguous loads). 16 * K floats.
__host__ __device__ inline size_t block_order_index(int s, int k) {
    return (size_t)(k >> 5) * 512 + ((k >> 3) & 3) * 128 + s * 8 + (k & 7);
}
// y[b * ldy + r] = sum over c < nparts of parts[c * stride + b * M + r] (chunk order).
int launch_sum_parts(const float *parts, int nparts, size_t stride, int batch, int M, float *y, int ldy,
                     hipStream_t s);
// Input of a batched GEMM, formed per sequence row while the activations are staged (the
// residual pattern of attention.c:356-366 / transformer.c:231-239 and the pre-norms of
// attention.c:316-325 / transformer.c:119-121):
//   d = sum of `nparts` partial rows (when parts is set), d = rmsnorm_delta(d, w_delta) when
//   w_delta is set; h = x (+ d); resid_out <- h (workgroup (0, 0)); the GEMM input is
//   rmsnorm_delta(h, w_norm) when w_norm is set, else h.
// The norms need whole rows: K at most 36 blocks (one K chunk) when w_delta or w_norm is set.
struct GemmIn {
    const float *x = nullptr;        // [b * ldx + k]; may be NULL when parts is set
    int ldx = 0;
    const float *parts = nullptr;    // [c * part_stride + b * ldp + k], c < nparts
    int nparts = 0, ldp = 0;
    size_t part_stride = 0;
    const float *w_delta = nullptr;
    float *resid_out = nullptr;      // [b * ldr + k]
    int ldr = 0;
    const float *w_norm = nullptr;
    float eps = 1e-6f;
    // x in block order (block_order_index; ldx unused): only with neither parts, norms nor
    // resid_out
    bool x_blocked = false;
    // the delta norm's sum of squares as a tree over all threads too, not in the reference's
    // eight-lane order (resid_out then differs from it in the last bits, inside the decode
    // tolerance); the decoder's own steps set it
    bool tree_norms = false;
};
// Output of a batched GEMM. parts set: the K chunks' partial sums go to parts[c][b][M] (an
// input of the next GEMM's GemmIn), nothing else is written. geglu: the weight rows are
// interleaved by eight (gate rows 8i..8i+7, then the matching up rows) and
// y[b * ldy + j] = gelu(gate_j) * up_j for j < M / 2 (transformer.c:141-157).
// The batched step's end, done by the greedy LM head's finish launch (GemmOut.advance): for
// every sequence b that has not stopped, log[step * batch + b] = tokens[b], pos[b] + 1 and
// done[b] on a stop token, then step + 1 and epoch + 1 (dec_advance_batch's work); and for every
// b, resid[b] = the bf16 embedding row of tokens[b] times es, the next step's input
// (dec_embed_batch's work).
struct BatchAdvance {
    int *pos = nullptr, *step = nullptr, *log = nullptr, *done = nullptr;
    uint32_t *epoch = nullptr;
    StopSet stop{};
    const uint16_t *embed = nullptr;
    int hidden = 0;
    float es = 1.0f;
    float *resid = nullptr;
};

struct GemmOut {
    float *y = nullptr;
    int ldy = 0;
    // rows as epoch-tagged words for a consumer in the same launch (gemm_body.h):
    // tagged[b * ldy + r] = tag << 32 | bits(y[b][r]), stored with agent-scope atomics. One K
    // chunk, rows form only.
    uint64_t *tagged = nullptr;
    uint32_t tag = 0;
    float *parts = nullptr;
    bool geglu = false;
    // y in block order (block_order_index over the M or M / 2 outputs; ldy unused): one K
    // chunk only, no parts
    bool y_blocked = false;
    // greedy form: instead of y, tokens[b] = the first index of the maximum of sequence b's
    // rows (sample_greedy, utils.c:145-156). One K chunk only, no parts or GeGLU; the
    // workgroups' partials go to the workspace, which is then required.
    int *tokens = nullptr;
    float *amax = nullptr;   // set by the launch: the partials in the workspace
    // greedy form: the step's advance and next input in the finish launch (host pointer, read
    // by the launcher only; batch <= 16)
    const BatchAdvance *advance = nullptr;
};
int launch_gemm_tiled_ex(int dt, const void *w, int M, int K, int batch, const GemmIn &in, const GemmOut &out,
                         void *ws, hipStream_t s);
// The launch parameters of one batched GEMM pass (gemm_mfma.hip), for a kernel that runs the
// GEMM's workgroups beside other work (gemm_body.h): weights, K chunking (cb blocks per chunk,
// nsplit chunks), waves per tile ks, workgroups gx of nw waves, staging mode (0 full, 1
// prepared, 2 plain), the prepared operands and the partial-sum workspace.
struct GemmPlan {
    const uint8_t *wq = nullptr;
    uint32_t q_bytes = 0;
    const uint8_t *wsc = nullptr;
    uint32_t s_bytes = 0;
    int M = 0, K = 0, batch = 0, cb = 0, nsplit = 1, ks = 1, gx = 0, nw = 0, mode = 0;
    const void *prep = nullptr;
    float *Yp = nullptr;
};
// For an input with norms or parts and one K chunk: launches the input pass (gemm_prep_kernel)
// on s and returns the plan of the GEMM that consumes it (mode 1). ws as for
// launch_gemm_tiled_ex. 0 / -1.
int plan_gemm_tiled(int dt, const void *w, int M, int K, int batch, const GemmIn &in, void *ws, hipStream_t s,
                    GemmPlan *P);
int launch_gemv_f(int dt, const void *w, int M, int K, const float *x, float *y, hipStream_t s);
// BF16 W [M][K] times up to any number of fp32 vectors X[b][ldx] -> Y[b][ldy] on the matrix
// cores (gemm_bf16.hip); supported: K % 8 == 0, W 16-byte aligned, below 4 GiB
bool gemm_bf16_supported(const void *w, int M, int K);
int launch_gemm_bf16(const void *w, int M, int K, const float *x, int ldx, int batch, float *y, int ldy,
                     hipStream_t s);
// F32 / BF16 rows [M][K] -> [M][ceil(K/32)] Q4_0 / Q8_0 blocks (AOS), quantize.hip
int launch_quantize(int dst_dtype, int src_dtype, const void *src, int M, int K, void *blocks, hipStream_t s);

int launch_rmsnorm(float *out, const float *in, const float *w, float eps, int dim, int batch, bool delta,
                   hipStream_t s);
int launch_rope(float *x, int n_heads, int head_dim, int pos, const float *cos_t, const float *sin_t,
                hipStream_t s);
// Interleaved pairs: (x[2p], x[2p+1]) rotated by (cos_p[p], sin_p[p]) for p < npairs
// (positional_encoding.c:95-99).
int launch_rope_pairs(float *x, int npairs, const float *cos_p, const float *sin_p, hipStream_t s);
int launch_gelu_mul(float *gate, const float *up, int n, hipStream_t s);
int launch_softmax_argmax(const float *logits, int n, float *probs, int *argmax, float *scratch,
                          hipStream_t s);
size_t softmax_scratch_floats(int n);
// The current device's buffer for launch_softmax_argmax's partials (allocated once per device,
// kept until the process ends; calls that overlap on one device must share a stream). NULL on
// error.
float *softmax_partials_scratch();
// The next token of `batch` rows of logits (row b at logits + b * ld) as perform_inference
// draws it (sample.hip): temperature <= 0 is sample_greedy; otherwise sample_temperature after
// the 1/T scaling, bit for bit, with draws[step * batch + b] (step = *d_step, or 0 when d_step
// is NULL) in place of rand() / RAND_MAX. The weights go to w (row b at w + b * ldw; w may be
// the logits). ws: sample_workspace_bytes(n, batch) bytes, 256-byte aligned; calls sharing it
// must be ordered. n at most 2^21.
size_t sample_workspace_bytes(int n, int batch);
bool sample_supported(int n, int batch);
int launch_sample(const float *logits, int n, int batch, size_t ld, float temperature, float *w, size_t ldw,
                  const float *draws, const int *d_step, int *tokens, void *ws, hipStream_t s);
enum : int { UOP_GELU = 0, UOP_SILU = 1, UOP_RELU = 2, UOP_SCALE = 3, UOP_SOFTCAP = 4 };
int launch_unary(float *x, int n, int op, float a, hipStream_t s);
int launch_axpy(float *dst, const float *src, int n, float a, bool fused, hipStream_t s);
int launch_geglu_split(float *out, const float *in, int n, hipStream_t s);
int launch_bf16_to_f32(float *dst, const uint16_t *src, int n, hipStream_t s);
int launch_dot_ref(const float *a, const float *b, int n, float *out, hipStream_t s);
int launch_norm_residual(float *hidden, float *resid, const float *w, float eps, int dim, hipStream_t s);

}  // namespace sapphire
