// decode_persist.hip - the layers of one Gemma-3 decode step as one persistent kernel.
//
// The multi-launch step (decode.hip) separates its stages by kernel boundaries; each of its
// ~110 launches per token costs a launch and a cold start of its memory loads. Here one grid
// of G workgroups, all resident at once (the host checks the occupancy), runs every layer, and
// the stages are separated by data instead:
//
// * Every exchanged vector element is one 64-bit word: the fp32 value in the low half and the
//   epoch of the stage that produced it in the high half. Words are stored and loaded with
//   agent-scope atomics, which are coherent across the L2 caches of the eight XCDs.
// * A consumer polls exactly the words it needs until every tag equals the producer's epoch:
//   the poll is the data load, and no store acknowledgement is waited for. A workgroup's weight
//   and KV-cache loads for its next stage are issued before that wait, so their latency hides
//   behind it.
// * Every workgroup keeps its own copy of the residual stream in LDS. It is updated by the same
//   instructions from the same inputs, so the copies are bit-identical.
//
// Stages of layer l, epoch e = seq * 8 * (n_layers + 1) + 8 * l + stage (seq counts steps):
//   1 QKV GEMV       input: previous layer's down output (post-FFN norm + residual), pre-norm
//   2 attention      input: q, k, v; QK-norm, RoPE, KV write; partial of one head over a slice
//   3 combine        input: the slices' partials for this workgroup's attention elements
//   4 o-proj GEMV    input: attention output
//   5 gate/up GEMV   input: o (post-attention norm + residual, pre-FFN norm); epilogue gelu*up
//   6 down GEMV      input: g
// After the last layer the final finalize + norm run; workgroup 0 writes the LM-head input.
// The op order is that of inference_forward_batch (inference.c:616-651) with the stages of
// attention.c:311-375 and transformer.c:96-283, as in decode.hip.
//
// Every wait is bounded. A wait that exceeds spin_limit polls increments *err and ends its
// workgroup; every other workgroup then times out at its next wait. So the kernel always ends,
// and the host reports the failure.
#include "decode_device.h"

namespace sapphire {

namespace {

constexpr int kLpr = 16;                          // lanes per GEMV row
constexpr int kSlots = 4;                         // (wave-step, block) slots per lane in one GEMV stage
constexpr int kCombMax = 2048;                    // gathered partial words per workgroup in the combine
constexpr int kVecRegs = kDecMaxK / kThreads;     // vector elements per thread (longest vector)

__device__ __forceinline__ void put_tagged(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_tagged(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

constexpr int kAttnRows = 36;                     // K/V rows of one attention batch (9 per wave)

// The layer-invariant geometry of one GEMV stage for this workgroup (the same for every layer:
// all layers share their shapes), computed once per launch so that the stages do no integer
// division: rows in wave-steps of 64 / lpr rows, contiguous ranges of ceil(S / G) wave-steps
// per workgroup, wave w taking every fourth step; lane slot -> (step offset k, block round j).
struct StageGeom {
    int M, nb, bpl, s0, s1;
    int k[kSlots], j[kSlots];
};

__device__ __forceinline__ void stage_geom(StageGeom &g, int M, int K, int lpr) {
    const int rpw = kWave / lpr;
    g.M = M;
    g.nb = K / kBlock;
    g.bpl = (g.nb + lpr - 1) / lpr;
    const int S = (M + rpw - 1) / rpw, per = (S + (int)gridDim.x - 1) / (int)gridDim.x;
    g.s0 = min(S, (int)blockIdx.x * per);
    g.s1 = min(S, g.s0 + per);
    for (int slot = 0; slot < kSlots; ++slot) {
        g.k[slot] = slot / g.bpl;
        g.j[slot] = slot - g.k[slot] * g.bpl;
    }
}

struct CombGeom {
    int e0, e1, E, hb;     // elements [e0, e1), nominal E, first element of the range's second head
};

__device__ __forceinline__ void comb_geom(CombGeom &c, uint32_t *off, int nh, int hd) {
    const int nq = nh * hd, G = gridDim.x, S = G / nh;   // S slices: partial (b, h) of slice b
    c.E = (nq + G - 1) / G;
    c.e0 = min(nq, (int)blockIdx.x * c.E);
    c.e1 = min(nq, c.e0 + c.E);
    if (c.e0 >= c.e1) return;
    const int h_lo = c.e0 / hd, h_hi = (c.e1 - 1) / hd;   // E <= hd: at most two heads
    c.hb = (h_lo + 1) * hd;
    const int per = c.E + 4;
    for (int j = threadIdx.x; j < S * per; j += kThreads) {
        const int b = j / per, k = j - b * per;
        size_t o;
        if (k < c.E) {
            const int el = min(c.e0 + k, c.e1 - 1);
            o = ((size_t)b * nh + el / hd) * (hd + 2) + el % hd;
        } else {
            const int hh = (k - c.E) < 2 ? h_lo : h_hi;
            o = ((size_t)b * nh + hh) * (hd + 2) + hd + ((k - c.E) & 1);
        }
        off[j] = (uint32_t)o;
    }
}

enum { kGeomQkv = 0, kGeomO = 1, kGeomGu = 2, kGeomDown = 3 };

// The GEMV input in LDS: each 32-element block padded to 36 floats. The 16 (or 32) lanes of a
// row read 16 different blocks at once; at a 128-byte stride every second lane fell on the same
// four of the 64 four-byte banks (an 8-way conflict on every ds_read_b128), at 144 bytes the 16
// lanes of a row take 16 different bank quads.
constexpr int kXBlock = kBlock + 4;
__device__ __forceinline__ int xpad(int i) { return i + (i >> 5) * (kXBlock - kBlock); }

template <int NH, int DPL>
struct alignas(16) PersistLds {
    float resid[kDecMaxK];                       // the residual stream
    float xs[kDecMaxK / kBlock * kXBlock];       // input of the current GEMV (padded blocks, xpad)
    float dl[kDecMaxK];                          // gathered delta vector
    float comb[kCombMax];
    // K / V rows of the attention slice's current batch (natural dim order), filled by DMA
    float kvk[kAttnRows][kWave * DPL], kvv[kAttnRows][kWave * DPL];
    // the layer descriptors (PLayer), copied once per step: read from here, not with scalar
    // loads of global memory that a step's streaming has long evicted from every cache
    alignas(16) uint32_t layer_words[kPersistMaxLayers * sizeof(PLayer) / 4];
    StageGeom geom[4];                           // kGeomQkv, kGeomO, kGeomGu, kGeomDown
    int att_t[2][2];                             // attention slice [t0, t1) of local (0) / global (1) layers
    CombGeom cg;                                 // the combine's element range
    uint32_t comb_off[kCombMax];                 // the combine's gathered word offsets
    __device__ __forceinline__ const PLayer &layer(int l) const {
        return reinterpret_cast<const PLayer *>(layer_words)[l];
    }
    float sh[16];
    int flag;
};

// dst[j] = value of word *src(j) for j < n, once its tag equals `tag`; thread t takes
// j = t + 256 e. begin() issues the first load of every word; end() polls the stale words
// again until all have the tag. A stage issues begin() before its prefetch loads (weights,
// norm weights, K/V rows), so that the first check of the words waits only for their own
// loads: vector memory loads complete in issue order, and a check issued after the prefetch
// would wait for all of it. end() returns false when a word is still stale after spin_limit
// polls (and counts the failure in *err). It synchronises the workgroup; the result is the
// same in every thread. With sq set, the wave sums of the squares of the gathered values go
// to sq[0..3] before that barrier: each thread sums its own values in the order par_sum_sq
// takes them, so (sq[0] + sq[1]) + (sq[2] + sq[3]) afterwards is par_sum_sq(dst, n), bit for
// bit.
template <int MAXE, class Src>
struct Gather {
    uint64_t w[MAXE];

    __device__ __forceinline__ void begin(Src src, int n, uint32_t tag) {
#pragma unroll
        for (int e = 0; e < MAXE; ++e) {
            const int j = threadIdx.x + e * kThreads;
            w[e] = j < n ? get_tagged(src(j)) : (uint64_t)tag << 32;
        }
    }

    template <bool PAD = false>
    __device__ __forceinline__ bool end(Src src, int n, uint32_t tag, float *dst, int spin_limit, int *err,
                                        int *flag, float *sq = nullptr) {
        for (int spins = 0;; ++spins) {
            bool ready = true;
#pragma unroll
            for (int e = 0; e < MAXE; ++e) ready = ready && tag_is(w[e], tag);
            if (ready) break;
            if (spins >= spin_limit) {
                *flag = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
#pragma unroll
            for (int e = 0; e < MAXE; ++e) {
                const int j = threadIdx.x + e * kThreads;
                if (j < n && !tag_is(w[e], tag)) w[e] = get_tagged(src(j));
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < MAXE; ++e) {
            const int j = threadIdx.x + e * kThreads;
            if (j < n) {
                const float v = __uint_as_float((uint32_t)w[e]);
                dst[PAD ? xpad(j) : j] = v;
                acc = __builtin_fmaf(v, v, acc);
            }
        }
        if (sq) {
            acc = lanes::wave_sum(acc);
            if ((threadIdx.x & (kWave - 1)) == 0) sq[threadIdx.x / kWave] = acc;
        }
        __syncthreads();
        const bool ok = *flag == 0;
        if (!ok && threadIdx.x == 0) atomicAdd(err, 1);
        return ok;
    }
};

template <int MAXE, class Src>
__device__ __forceinline__ bool gather(Src src, int n, uint32_t tag, float *dst, int spin_limit, int *err,
                                       int *flag, float *sq = nullptr) {
    Gather<MAXE, Src> g;
    g.begin(src, n, tag);
    return g.end(src, n, tag, dst, spin_limit, err, flag, sq);
}

// gather() with during() run between the first loads of the words and their first check:
// loads it issues go out behind the polls, so the first check does not wait for them. PAD:
// dst is a GEMV input (element j at xpad(j)).
template <int MAXE, bool PAD = false, class Src, class F>
__device__ __forceinline__ bool gather_during(Src src, int n, uint32_t tag, float *dst, int spin_limit, int *err,
                                              int *flag, float *sq, F during) {
    Gather<MAXE, Src> g;
    g.begin(src, n, tag);
    during();
    return g.template end<PAD>(src, n, tag, dst, spin_limit, err, flag, sq);
}

struct Contig {
    const uint64_t *p;
    __device__ const uint64_t *operator()(int j) const { return p + j; }
};

// Elements t + 256 e of a K-long weight vector in registers (loaded before a wait). Every
// lane loads (from element K - 1 past the end) and the value is selected where it is used:
// a load into a register that other lanes of the wave then zero makes the compiler wait for
// every load in flight at that point.
template <int R>
struct VecRegs {
    float v[R];
    int K;
    __device__ __forceinline__ void load(const float *__restrict__ p, int n) {
        K = n;
#pragma unroll
        for (int e = 0; e < R; ++e) v[e] = as_global(p)[min((int)threadIdx.x + e * kThreads, n - 1)];
    }
    __device__ __forceinline__ float operator[](int e) const {
        return (int)threadIdx.x + e * kThreads < K ? v[e] : 0.f;
    }
};

// Sum of squares of v[0..K) (LDS) over the workgroup: per-thread FMA chains of at most
// K / 256 elements, DPP row sums, then the four waves in a fixed order. The reference sums
// in eight sequential lanes (normalization.c:12-32); this order is a tree (within the decode
// tolerance) and takes a few hundred cycles instead of a K/8-long dependent chain. Every
// thread gets the same value; the call synchronises the workgroup.
__device__ __forceinline__ float par_sum_sq(const float *v, int K, float *sh) {
    float acc = 0.f;
    for (int i = threadIdx.x; i < K; i += kThreads) acc = __builtin_fmaf(v[i], v[i], acc);
    acc = lanes::wave_sum(acc);
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = acc;
    __syncthreads();
    return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// xs = rmsnorm_delta(resid, w) (normalization.c:104-117), xs a GEMV input (xpad)
template <int R>
__device__ __forceinline__ void norm_to(float *xs, const float *resid, const VecRegs<R> &w, int K, float eps,
                                        float *sh) {
    const float r = rms_inv_of(par_sum_sq(resid, K, sh), K, eps);
#pragma unroll
    for (int e = 0; e < R; ++e) {
        const int i = threadIdx.x + e * kThreads;
        if (i < K) xs[xpad(i)] = __fmul_rn(__fmul_rn(resid[i], r), __fadd_rn(1.0f, w[e]));
    }
    __syncthreads();
}

// resid += rmsnorm_delta(dl, wd) (attention.c:358-366, transformer.c:231-239), then
// xs = rmsnorm_delta(resid, wn) with the arithmetic of norm_to. dl was gathered with its wave
// sums of squares in sh[0..3] (gather's sq). Each thread sums the squares of the residual
// elements it has just updated, which are the elements par_sum_sq gives it, in its order, so
// the second norm is bit-identical to norm_to on the stored residual but needs no barrier
// before its sum and no second read of the residual from LDS. Its wave sums go to sh[4..7]:
// other waves may still be reading sh[0..3].
template <int R>
__device__ __forceinline__ void add_norm_delta_norm(float *resid, float *xs, const float *dl, const VecRegs<R> &wd,
                                                    const VecRegs<R> &wn, int K, float eps, float *sh) {
    const float r1 = rms_inv_of((sh[0] + sh[1]) + (sh[2] + sh[3]), K, eps);
    float nv[R];
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < R; ++e) {
        const int i = threadIdx.x + e * kThreads;
        nv[e] = 0.f;
        if (i < K) {
            nv[e] = __fadd_rn(resid[i], __fmul_rn(__fmul_rn(dl[i], r1), __fadd_rn(1.0f, wd[e])));
            resid[i] = nv[e];
            acc = __builtin_fmaf(nv[e], nv[e], acc);
        }
    }
    acc = lanes::wave_sum(acc);
    if ((threadIdx.x & (kWave - 1)) == 0) sh[4 + threadIdx.x / kWave] = acc;
    __syncthreads();
    const float r2 = rms_inv_of((sh[4] + sh[5]) + (sh[6] + sh[7]), K, eps);
#pragma unroll
    for (int e = 0; e < R; ++e) {
        const int i = threadIdx.x + e * kThreads;
        if (i < K) xs[xpad(i)] = __fmul_rn(__fmul_rn(nv[e], r2), __fadd_rn(1.0f, wn[e]));
    }
    __syncthreads();
}

// The rows of one GEMV stage owned by this workgroup. A wave-step is 64 / LPR rows of LPR
// lanes (16, or 32 for the o-proj's and the down projection's longer rows); lane q of a row
// takes blocks q, q + LPR, ... (bpl = ceil(K / (32 LPR)) of them), and the row's lanes are
// summed by DPP. The S = ceil(M / (64 / LPR)) wave-steps are split into contiguous ranges of
// ceil(S / G) per workgroup; wave w takes every fourth step of its workgroup's range. A lane
// holds SL (step, block) slots, slot = step * bpl + block (steps per wave x bpl <= SL,
// checked by the host). load() issues the weight loads; finish() forms the rows.
template <int DT, bool GEGLU, int SL = kSlots, int LPR = kLpr>
struct GemvStage {
    static_assert(LPR == 16 || LPR == 32, "rows of 16 or 32 lanes");
    static constexpr int RPW = kWave / LPR;   // rows per wave-step
    LaneBlock<DT> b0[SL], b1[GEGLU ? SL : 1];
    const StageGeom *g;

    __device__ __forceinline__ void load(const QMat &w0, const QMat &w1, const StageGeom &geom) {
        g = &geom;
        const int M = g->M, nb = g->nb, s0 = g->s0, s1 = g->s1;
        const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
        const int q = lane & (LPR - 1), rin = lane / LPR;
        (void)M;
#pragma unroll
        for (int slot = 0; slot < SL; ++slot) {
            const int k = g->k[slot], j = g->j[slot];
            const int st = s0 + wid + 4 * k;
            if (st < s1) {
                const int blk = q + LPR * j;
                load_lane_block<DT>(w0, st * RPW + rin, blk, nb, blk < nb, b0[slot]);
                if constexpr (GEGLU) load_lane_block<DT>(w1, st * RPW + rin, blk, nb, blk < nb, b1[slot]);
            }
        }
    }

    // y[row] (tagged) = W0[row] . xs, or gelu(W0[row] . xs) * (W1[row] . xs) for the GeGLU form.
    // Ends with a workgroup barrier, after which xs may be overwritten.
    __device__ __forceinline__ void finish(const float *xs, uint64_t *y, uint32_t tag) {
        const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
        const int q = lane & (LPR - 1), rin = lane / LPR;
        const int M = g->M, nb = g->nb, bpl = g->bpl, s0 = g->s0, s1 = g->s1;
        float p0 = 0.f, p1 = 0.f;
#pragma unroll
        for (int slot = 0; slot < SL; ++slot) {
            const int k = g->k[slot], j = g->j[slot];
            const int st = s0 + wid + 4 * k;
            if (st < s1) {
                const int blk = q + LPR * j;
                const bool on = blk < nb;
                float xv[32];
                const float4 *xp = reinterpret_cast<const float4 *>(xs + blk * kXBlock);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 v = on ? xp[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                    xv[4 * i] = v.x;
                    xv[4 * i + 1] = v.y;
                    xv[4 * i + 2] = v.z;
                    xv[4 * i + 3] = v.w;
                }
                float xt[16];   // sum of the block's x as a tree (not a 32-long chain)
#pragma unroll
                for (int i = 0; i < 16; ++i) xt[i] = xv[2 * i] + xv[2 * i + 1];
#pragma unroll
                for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
                    for (int i = 0; i < w; ++i) xt[i] = xt[2 * i] + xt[2 * i + 1];
                const float xsum = xt[0];
                p0 += block_value<DT>(b0[slot], xv, xsum);
                if constexpr (GEGLU) p1 += block_value<DT>(b1[slot], xv, xsum);
                if (j == bpl - 1) {   // the step's last block: sum the row's lanes and store
                    p0 = row16_sum(p0);
                    if constexpr (GEGLU) p1 = row16_sum(p1);
                    if constexpr (LPR == 32) {   // the row's two 16-lane halves: the second's lanes
                        // add the first's sum (DPP row_bcast:15 into rows 1 and 3)
                        p0 += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(p0), 0x142, 0xA, 0xF, false));
                        if constexpr (GEGLU)
                            p1 += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(p1), 0x142, 0xA, 0xF, false));
                    }
                    const int row = st * RPW + rin;
                    if (q == (LPR == 32 ? 16 : 0) && row < M)
                        put_tagged(y + row, GEGLU ? __fmul_rn(gelu_ref(p0), p1) : p0, tag);
                    p0 = 0.f;
                    p1 = 0.f;
                }
            }
            // one slot's 32 x values live at a time
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    }
};

// Stage 2: QK-norm, RoPE and the KV write of the token, then this workgroup's partial
// (o, max in log2 units, sum) of one query head over one slice of the layer's positions
// (attention.c:140-158 over the slice). Workgroup b takes slice b % S and head b / S of
// S = G / NH slices, so the combine merges S partials per element instead of one per
// workgroup, and the NH workgroups of a slice read the same K/V rows on one XCD (b mod 8). Its four waves take the slice's positions in turn (wave w: positions t0 + w +
// 4j, K/V rows that the wave itself brought into LDS by DMA), each with the head's q and the
// token's k and v in registers (lane l holds dims l*DPL .. l*DPL+DPL-1), normalised by DPP
// sums and rotated with the partner dims in lane l ^ 32; the four running (max, sum, o) are
// merged through LDS. prefetch() loads the slice's first K/V rows, the gammas and the RoPE row
// entries; the kernel calls it a stage ahead, so the loads have returned when run() polls for
// q, k and v.
template <int DPL, int NH>
struct AttnStage {
    static constexpr int NW = kThreads / kWave;
    // K/V rows of positions t0 .. t0 + PF - 1 (one K/V head: rows [max_ctx][hd]); wave w
    // holds rows w, w + NW, ...
    static constexpr int PF = kAttnRows;
    static_assert(PF % NW == 0, "whole rows per wave");
    float gq[DPL], gk[DPL], cs[DPL], sn[DPL];
    int t0, t1;

    // DMA of this wave's K and V rows of the batch from tb into LDS (row pos is written by
    // this step and taken from registers instead)
    __device__ __forceinline__ void load_batch(const PLayer &L, int hd, int pos, int tb, PersistLds<NH, DPL> &s) {
        const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
#pragma unroll
        for (int j = 0; j < PF / NW; ++j) {
            const int r = wid + NW * j, t = tb + r;
            if (t < t1 && t != pos) {   // wave-uniform
                row_to_lds<DPL>(L.kc + (size_t)t * hd, s.kvk[r]);
                row_to_lds<DPL>(L.vc + (size_t)t * hd, s.kvv[r]);
            }
        }
    }

    // this workgroup's slice [t0, t1) of the positions a layer with sliding window `window`
    // (0: global) attends to at pos (attention.c:122-127); computed once per launch
    __device__ static void slice(int pos, int window, int &t0, int &t1) {
        const int seq = pos + 1;
        const int start = (window > 0 && seq > window) ? seq - window : 0;
        const int len = seq - start, S = (int)gridDim.x / NH;
        const int chunk = (len + S - 1) / S;
        t0 = min(seq, start + (int)(blockIdx.x % S) * chunk);
        t1 = min(seq, t0 + chunk);
    }

    // the slice of layer L's kind (local or global)
    __device__ __forceinline__ void set_slice(const PLayer &L, const PersistLds<NH, DPL> &s) {
        t0 = s.att_t[L.window > 0 ? 0 : 1][0];
        t1 = s.att_t[L.window > 0 ? 0 : 1][1];
    }

    // rows j0 <= j < j1 of this wave's part of the first batch (a third of it per stage of the
    // previous layer, so that no stage stalls long on issuing them)
    __device__ __forceinline__ void load_rows(const PLayer &L, int hd, int pos, int j0, int j1,
                                              PersistLds<NH, DPL> &s) {
        const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
#pragma unroll
        for (int j = 0; j < PF / NW; ++j) {
            const int r = wid + NW * j, t = t0 + r;
            if (j >= j0 && j < j1 && t < t1 && t != pos) {   // wave-uniform
                row_to_lds<DPL>(L.kc + (size_t)t * hd, s.kvk[r]);
                row_to_lds<DPL>(L.vc + (size_t)t * hd, s.kvv[r]);
            }
        }
    }

    __device__ __forceinline__ void prefetch(const PersistArgs &a, const PLayer &L, int pos, PersistLds<NH, DPL> &s) {
        set_slice(L, s);
        load_batch(L, a.hd, pos, t0, s);
        prefetch_regs(a, L, pos);
    }

    // the gammas and the RoPE row entries of layer L (its rows are loaded already)
    __device__ __forceinline__ void prefetch_regs(const PersistArgs &a, const PLayer &L, int pos) {
        const int lane = threadIdx.x & (kWave - 1), d0 = lane * DPL;
        // gammas (one head_dim vector for every q head, one for k: attention.c:228-269) and the
        // RoPE row of pos at (dim mod half) (rope.c:99-117)
        const size_t ci = (size_t)pos * a.rope_stride + (size_t)(lane & (kWave / 2 - 1)) * DPL;
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            gq[i] = as_global(L.qn)[d0 + i];
            gk[i] = as_global(L.kn)[d0 + i];
            cs[i] = as_global(L.cos_t)[ci + i];
            sn[i] = as_global(L.sin_t)[ci + i];
        }
    }

    // during() runs between the first loads of q, k, v and their first check (it issues the
    // next stage's loads, which then go out behind the polls).
    template <class F>
    __device__ __forceinline__ bool run(const PersistArgs &a, const PLayer &L, int pos, uint32_t tag_in,
                                        uint32_t tag_out, PersistLds<NH, DPL> &s, F during) {
        const int hd = a.hd;
        const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
        const int wu = __builtin_amdgcn_readfirstlane(wid);
        const int head = (int)blockIdx.x / ((int)gridDim.x / NH);
        const int d0 = lane * DPL;                     // this lane's first dim
        // q of the head, k and v (t_qkv holds q | k | v), 3 hd words, gathered once per
        // workgroup into LDS (s.xs is free between the QKV and o-proj stages) and read back by
        // every wave
        constexpr int NQW = (3 * kWave * DPL + kThreads - 1) / kThreads;
        auto src = [&](int j) -> const uint64_t * {
            const int v = j / hd, d = j - v * hd;
            const int vec = v == 0 ? head : NH + (v - 1);   // q head, k (NH) or v (NH + 1)
            return a.t_qkv + (size_t)vec * hd + d;
        };
        // this wave's K/V DMA was issued before the polls, so it has landed once they have
        if (!gather_during<NQW>(src, 3 * hd, tag_in, s.xs, a.spin_limit, a.err, &s.flag, nullptr, during))
            return false;
        float xv[3][DPL];
#pragma unroll
        for (int v = 0; v < 3; ++v)
#pragma unroll
            for (int i = 0; i < DPL; ++i) xv[v][i] = s.xs[v * hd + d0 + i];

        // rmsnorm_delta of the q head and of k over their hd dims (wave sums of the lanes'
        // squares), then the half-split rotation: dim d < half pairs with d + half in lane l ^ 32
        // (rope.c:113-115: x[i] = x0 c - x1 s, x[i + half] = x1 c + x0 s)
        const bool upper = lane >= kWave / 2;
        float qk[2][DPL];
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc = __builtin_fmaf(xv[v][i], xv[v][i], acc);
            const float r = rms_inv_of(lanes::wave_sum(acc), hd, a.eps);
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float g = v == 0 ? gq[i] : gk[i];
                const float xn = __fmul_rn(__fmul_rn(xv[v][i], r), __fadd_rn(1.0f, g));
                const float xp = __shfl_xor(xn, kWave / 2, kWave);
                qk[v][i] = upper ? __builtin_fmaf(xn, cs[i], __fmul_rn(xp, sn[i]))
                                 : __builtin_fmaf(xn, cs[i], -__fmul_rn(xp, sn[i]));
            }
        }
        const float *vnew = xv[2];
        // kv_cache_write_token: [head][pos][dim], once (head 0's workgroup of pos's slice)
        if (head == 0 && wid == 0 && t0 <= pos && pos < t1) {
            const size_t off = (size_t)pos * hd + d0;
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                as_global(L.kc)[off + i] = qk[1][i];
                as_global(L.vc)[off + i] = vnew[i];
            }
        }

        // scores in log2 units, so that every softmax weight is one exp2 (v_exp_f32)
        const float sl2 = __fmul_rn(a.scale, 1.44269504088896341f);
        float m = -INFINITY, sm = 0.f, o[DPL];
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] = 0.f;
        for (int tb = t0; tb < t1; tb += PF) {
            if (tb != t0) {   // a further batch into this wave's own rows (all read by now)
                load_batch(L, hd, pos, tb, s);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
#pragma unroll
            for (int j = 0; j < PF / NW; ++j) {
                const int r = wu + NW * j, t = tb + r;
                if (t < t1) {
                    float kr[DPL], vr[DPL];
                    if (t == pos) {   // the token's own row is in registers
#pragma unroll
                        for (int i = 0; i < DPL; ++i) {
                            kr[i] = qk[1][i];
                            vr[i] = vnew[i];
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < DPL; ++i) {
                            kr[i] = s.kvk[r][d0 + i];
                            vr[i] = s.kvv[r][d0 + i];
                        }
                    }
                    float dp = 0.f;
#pragma unroll
                    for (int i = 0; i < DPL; ++i) dp = __builtin_fmaf(qk[0][i], kr[i], dp);
                    const float score = __fmul_rn(lanes::wave_sum(dp), sl2);
                    const float mn = fmaxf(m, score);
                    const float c = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
                    const float p = __builtin_amdgcn_exp2f(score - mn);
                    sm = __builtin_fmaf(sm, c, p);
#pragma unroll
                    for (int i = 0; i < DPL; ++i) o[i] = __builtin_fmaf(o[i], c, p * vr[i]);
                    m = mn;
                }
            }
        }
        // the waves' running partials merged through LDS (s.dl is free until the o-proj's
        // residual stage): weights exp2(m_w - M), then one partial of the workgroup
        float *mo = s.dl;                              // [NW][hd] o, then (m, sum) per wave
#pragma unroll
        for (int i = 0; i < DPL; ++i) mo[wid * hd + d0 + i] = o[i];
        if (lane == 0) {
            mo[NW * hd + 2 * wid] = m;
            mo[NW * hd + 2 * wid + 1] = sm;
        }
        __syncthreads();
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < NW; ++v) M = fmaxf(M, mo[NW * hd + 2 * v]);
        float ew[NW], S = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) {
            const float mv = mo[NW * hd + 2 * v];
            ew[v] = mv == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv - M);
            S = __builtin_fmaf(mo[NW * hd + 2 * v + 1], ew[v], S);
        }
        // partial (slice, head) at (slice * NH + head) * (hd + 2)
        const int nsl = (int)gridDim.x / NH;
        uint64_t *out = a.t_part + ((size_t)(blockIdx.x % nsl) * NH + head) * (hd + 2);
        for (int d = threadIdx.x; d < hd; d += kThreads) {
            float O = 0.f;
#pragma unroll
            for (int v = 0; v < NW; ++v) O = __builtin_fmaf(mo[v * hd + d], ew[v], O);
            put_tagged(out + d, O, tag_out);
        }
        if (threadIdx.x == 0) {
            put_tagged(out + hd, M, tag_out);
            put_tagged(out + hd + 1, S, tag_out);
        }
        return true;
    }
};

// Stage 3: attention elements [e0, e1) of this workgroup, E = ceil(NH*hd / G) each:
// out = sum_b e_b o_b / sum_b e_b s_b with e_b = exp2(m_b - max_b m_b) over the partials b of
// the G / NH slices (attention.c:140-158; the maxima are in log2 units), reduced over 16 lanes. The
// gathered words are E values, then (m, s) of the range's first and last head, of every
// partial; their offsets (s.comb_off) and the range are computed once per launch.
template <int NH, int DPL, class D, class F>
__device__ __forceinline__ bool combine_stage(const PersistArgs &a, uint32_t tag_in, uint32_t tag_out,
                                              PersistLds<NH, DPL> &s, D during, F on_arrival) {
    const CombGeom c = s.cg;
    if (c.e0 >= c.e1) {
        during();
        on_arrival();
        return true;
    }
    const int S = (int)gridDim.x / NH, per = c.E + 4;   // partials per head: one per slice
    constexpr int NE = kCombMax / kThreads;
    uint32_t offs[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        const int j = threadIdx.x + e * kThreads;
        offs[e] = j < S * per ? s.comb_off[j] : 0u;
    }
    const uint64_t *part = a.t_part;
    auto src = [&](int j) -> const uint64_t * { return part + offs[(j - (int)threadIdx.x) / kThreads]; };
    if (!gather_during<NE>(src, S * per, tag_in, s.comb, a.spin_limit, a.err, &s.flag, nullptr, during)) return false;
    on_arrival();
    // 16-lane row r takes elements k = r, r + 16, ...; lane q of the row takes partials
    // b = q, q + 16, ...; max, weights and sums are reduced over the row by DPP
    const int q = threadIdx.x & 15;
    for (int k = threadIdx.x / 16; k < c.e1 - c.e0; k += kThreads / 16) {
        const int el = c.e0 + k, hk = el < c.hb ? 0 : 2;
        float M = -INFINITY;
        for (int b = q; b < S; b += 16) M = fmaxf(M, s.comb[b * per + c.E + hk]);
        M = row16_max(M);
        float Sw = 0.f, O = 0.f;
        for (int b = q; b < S; b += 16) {
            const float mb = s.comb[b * per + c.E + hk];
            const float e = mb == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mb - M);
            Sw = __builtin_fmaf(s.comb[b * per + c.E + hk + 1], e, Sw);
            O = __builtin_fmaf(s.comb[b * per + k], e, O);
        }
        Sw = row16_sum(Sw);
        O = row16_sum(O);
        if (q == 0) put_tagged(a.t_attn + el, O * (1.0f / Sw), tag_out);
    }
    __syncthreads();
    return true;
}

// HR: elements per thread of an H-long vector (the residual stream, its deltas, norm weights);
// the attention output (NH heads of 64 DPL) takes NQR, the FFN activations kVecRegs. SL: the
// weight slots per lane of the GEMV stages.
template <int DT, int DPL, int NH, int HR, int SL>
__global__ __launch_bounds__(kThreads) void dec_persist_kernel(PersistArgs a) {
    constexpr int NQR = (NH * kWave * DPL + kThreads - 1) / kThreads;
    __shared__ PersistLds<NH, DPL> s;
    // Every load the start needs goes out at once: each check below that returns would
    // otherwise hold the next load back by a memory round trip.
    const int lane0 = threadIdx.x & (kWave - 1);
    const int err0 = *a.err;
    const int done0 = a.done ? *a.done : 0;
    int tok, pos;
    uint32_t seq, st = 0;
    unsigned long long key = 0;
    if (a.slots) {
        const TokenSlots &ts = *a.slots;
        st = ts.a;
        static_assert(kSlotCount == kWave, "one slot per lane");
        key = ts.key[lane0];                       // lane l reads slot l
        tok = ts.tok0;
        pos = ts.pos0 + (int)st;
        seq = ts.seq0 + st;
    } else {
        tok = a.state[0];
        pos = a.state[1];
        seq = *a.seq;
    }
    {   // the layer descriptors into LDS (they do not depend on the token)
        static_assert(sizeof(PLayer) % 4 == 0, "descriptors copied as words");
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a.layers);
        uint32_t *dst = s.layer_words;
        const int nw = a.n_layers * (int)(sizeof(PLayer) / 4);
        for (int i = threadIdx.x; i < nw; i += kThreads) dst[i] = src[i];
    }
    // a wait of an earlier step of this generate call timed out: its results are void, and
    // every later step ends at once instead of timing out again
    if (err0 != 0) return;
    if (done0) return;                             // the sequence has stopped
    if (threadIdx.x == 0) s.flag = 0;
    const int H = a.H, nq = NH * a.hd;
    if (a.slots && st > 0) {
        // the previous step's LM head left its greedy key in the slots (none before a run's
        // first step): every workgroup decodes the same token (the wave's maximum by 64-bit
        // shuffles, no LDS, no barrier); workgroup 0 logs it (inference.c:297) and, on a stop
        // token (inference.c:298-301), marks the sequence done, and every workgroup returns
#pragma unroll
        for (int mask = 1; mask < kWave; mask <<= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)key, mask, kWave), hi = __shfl_xor((uint32_t)(key >> 32), mask, kWave);
            const unsigned long long o = ((unsigned long long)hi << 32) | lo;
            key = o > key ? o : key;
        }
        if (!slot_token(key, st, a.vocab, tok)) {
            if (threadIdx.x == 0) atomicAdd(a.err, 1);
            return;
        }
        const bool stop = a.stop.has(tok);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            a.log[a.slots->logbase + (int)st - 1] = tok;
            if (stop) *a.done = 1;
        }
        if (stop) return;
    }
    // nothing in this launch reads b; the LM head after it tags its keys with it
    if (a.slots && blockIdx.x == 0 && threadIdx.x == 0) a.slots->b = st + 1u;
    const uint32_t base = seq * persist_epochs_per_step(a.n_layers);
    {   // sapphire_embed_lookup (transformer.c:347-365)
        const size_t row = embed_row(tok, a.vocab, H);
        for (int i = threadIdx.x; i < H; i += kThreads) {
            const float v = __uint_as_float((uint32_t)a.embed[row + i] << 16);
            s.resid[i] = a.es != 1.0f ? __fmul_rn(v, a.es) : v;
        }
        // the stages' layer-invariant geometry
        CombGeom cg;
        comb_geom(cg, s.comb_off, NH, a.hd);
        if (threadIdx.x == 0) {
            stage_geom(s.geom[kGeomQkv], (NH + 2) * a.hd, H, kLpr);
            stage_geom(s.geom[kGeomO], H, nq, 32);
            stage_geom(s.geom[kGeomGu], a.ffn, H, kLpr);
            stage_geom(s.geom[kGeomDown], H, a.ffn, 32);
            AttnStage<DPL, NH>::slice(pos, a.window, s.att_t[0][0], s.att_t[0][1]);
            AttnStage<DPL, NH>::slice(pos, 0, s.att_t[1][0], s.att_t[1][1]);
            s.cg = cg;
        }
    }
    __syncthreads();
    // Every stage issues the next stage's weight loads as soon as its own input has arrived,
    // before its own arithmetic: the loads then return during that arithmetic and the next
    // wait, and the next stage's first check of its input (vector loads complete in issue
    // order) does not wait on them.
    GemvStage<DT, false, SL> gq;               // the layer's QKV
    VecRegs<HR> wn_attn, wd_prev;              // its pre-norm; the previous layer's post-FFN norm
    AttnStage<DPL, NH> at;                     // its attention (K/V rows in LDS, gammas, RoPE)
    gq.load(s.layer(0).qkv, s.layer(0).qkv, s.geom[kGeomQkv]);
    wn_attn.load(s.layer(0).n_attn, H);
    at.prefetch(a, s.layer(0), pos, s);
    for (int l = 0; l < a.n_layers; ++l) {
        const PLayer &L = s.layer(l);
        const uint32_t ep = base + 8u * (uint32_t)l;
        // 1: previous layer's finalize, pre-attention norm, QKV
        if (l > 0) {
            if (!gather<HR>(Contig{a.t_dn}, H, ep - 2, s.dl, a.spin_limit, a.err, &s.flag, s.sh)) return;
            add_norm_delta_norm(s.resid, s.xs, s.dl, wd_prev, wn_attn, H, a.eps, s.sh);
        } else {
            norm_to(s.xs, s.resid, wn_attn, H, a.eps, s.sh);
        }
        gq.finish(s.xs, a.t_qkv, ep + 1);
        // 2: attention (the o-proj's weights go out during its wait)
        GemvStage<DT, false, SL, 32> go;
        if (!at.run(a, L, pos, ep + 1, ep + 2, s, [&] { go.load(L.o, L.o, s.geom[kGeomO]); })) return;
        // The next layer's K/V rows go into LDS (this layer's attention is done with them) a
        // third at a time during the waits of stages 3, 4 and 5, behind each wait's first polls.
        const bool nx = l + 1 < a.n_layers;
        const PLayer &Ln = s.layer(nx ? l + 1 : l);
        if (nx) at.set_slice(Ln, s);
        constexpr int RPW = AttnStage<DPL, NH>::PF / (kThreads / kWave);   // rows per wave
        // 3: combine (the gate/up weights and the norm weights of stage 5 go out)
        GemvStage<DT, true, SL> gu;
        VecRegs<HR> wd_attn, wn_ffn;
        if (!combine_stage<NH, DPL>(
                a, ep + 2, ep + 3, s,
                [&] {
                    gu.load(L.gate, L.up, s.geom[kGeomGu]);
                    wd_attn.load(L.n_attn_post, H);
                    wn_ffn.load(L.n_ffn, H);
                    if (nx) at.load_rows(Ln, a.hd, pos, 0, RPW / 3, s);
                },
                [] {}))
            return;
        // 4: o-proj
        if (!gather_during<NQR, true>(Contig{a.t_attn}, nq, ep + 3, s.xs, a.spin_limit, a.err, &s.flag, nullptr,
                                [&] { if (nx) at.load_rows(Ln, a.hd, pos, RPW / 3, 2 * RPW / 3, s); }))
            return;
        go.finish(s.xs, a.t_o, ep + 4);
        // 5: post-attention norm + residual, pre-FFN norm, gate/up with the GeGLU (the down
        // projection's weights go out)
        GemvStage<DT, false, SL, 32> gd;
        if (!gather_during<HR>(Contig{a.t_o}, H, ep + 4, s.dl, a.spin_limit, a.err, &s.flag, s.sh, [&] {
                gd.load(L.down, L.down, s.geom[kGeomDown]);
                if (nx) at.load_rows(Ln, a.hd, pos, 2 * RPW / 3, RPW, s);
            }))
            return;
        add_norm_delta_norm(s.resid, s.xs, s.dl, wd_attn, wn_ffn, H, a.eps, s.sh);
        gu.finish(s.xs, a.t_g, ep + 5);
        // 6: down (the next layer's QKV and norm weights, or the final norm's, go out)
        if (!gather_during<kVecRegs, true>(Contig{a.t_g}, a.ffn, ep + 5, s.xs, a.spin_limit, a.err, &s.flag, nullptr, [&] {
                if (nx) {
                    gq.load(Ln.qkv, Ln.qkv, s.geom[kGeomQkv]);
                    wn_attn.load(Ln.n_attn, H);
                    at.prefetch_regs(a, Ln, pos);
                } else {
                    wn_attn.load(a.norm_final, H);
                }
                wd_prev.load(L.n_ffn_post, H);
            }))
            return;
        gd.finish(s.xs, a.t_dn, ep + 6);
    }
    // last finalize + final norm (transformer.c:400-406)
    const uint32_t ep_last = base + 8u * (uint32_t)(a.n_layers - 1) + 6u;
    if (!gather<HR>(Contig{a.t_dn}, H, ep_last, s.dl, a.spin_limit, a.err, &s.flag, s.sh)) return;
    add_norm_delta_norm(s.resid, s.xs, s.dl, wd_prev, wn_attn, H, a.eps, s.sh);
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < H; i += kThreads) a.xfin[i] = s.xs[xpad(i)];
}

using PersistKernel = void (*)(PersistArgs);

template <int DT, int HR, int SL>
PersistKernel pick(int dpl, int nh) {
#define SPH_PK(DPLV, NHV) \
    if (dpl == DPLV && nh == NHV) return dec_persist_kernel<DT, DPLV, NHV, HR, SL>;
    SPH_PK(1, 4) SPH_PK(2, 4) SPH_PK(4, 4) SPH_PK(1, 8) SPH_PK(2, 8) SPH_PK(4, 8)
#undef SPH_PK
    return nullptr;
}

// (wave-step, block) slots per lane of an M x K GEMV stage over `groups` workgroups.
int slots_per_lane(int M, int K, int groups, int lpr = kLpr) {
    const int rpw = kWave / lpr;
    const int S = (M + rpw - 1) / rpw, per = (S + groups - 1) / groups;
    const int bpl = (K / kBlock + lpr - 1) / lpr;
    return (per + 3) / 4 * bpl;
}

// Slots per lane the GEMV stages need (o-proj and down in rows of 32 lanes).
int light_slots(int groups, int H, int nh, int nkv, int hd, int ffn) {
    const int nq = nh * hd;
    return std::max({slots_per_lane(nq + 2 * nkv * hd, H, groups), slots_per_lane(H, nq, groups, 32),
                     slots_per_lane(ffn, H, groups), slots_per_lane(H, ffn, groups, 32)});
}

// H up to 1024 takes four elements per thread, longer vectors (up to kDecMaxK) eight, and the
// GEMV stages two weight slots per lane where two suffice: the registers
// held across every wait are those the model and the workgroup count need.
PersistKernel kernel_for(int dt, int nh, int hd, int H, int slots) {
    if (hd % kWave || H <= 0 || H > kDecMaxK) return nullptr;
    const int dpl = hd / kWave;
    if (H <= 4 * kThreads && slots <= 2)
        return dt == DT_Q4_0 ? pick<DT_Q4_0, 4, 2>(dpl, nh) : dt == DT_Q8_0 ? pick<DT_Q8_0, 4, 2>(dpl, nh) : nullptr;
    if (H <= 4 * kThreads)
        return dt == DT_Q4_0 ? pick<DT_Q4_0, 4, kSlots>(dpl, nh)
                             : dt == DT_Q8_0 ? pick<DT_Q8_0, 4, kSlots>(dpl, nh) : nullptr;
    return dt == DT_Q4_0 ? pick<DT_Q4_0, kVecRegs, kSlots>(dpl, nh)
                         : dt == DT_Q8_0 ? pick<DT_Q8_0, kVecRegs, kSlots>(dpl, nh) : nullptr;
}

}  // namespace

size_t persist_words(int H, int nh, int nkv, int hd, int ffn) {
    return (size_t)(nh + 2 * nkv) * hd + (size_t)kPersistMaxGroups * nh * (hd + 2) + (size_t)nh * hd + H + ffn + H;
}

bool persist_supported(int dt, int groups, int n_layers, int H, int nh, int nkv, int hd, int ffn) {
    const PersistKernel k = kernel_for(dt, nh, hd, H, light_slots(groups, H, nh, nkv, hd, ffn));
    const int nq = nh * hd;
    if (!k || nkv != 1 || nq > kAttnMaxQ || hd > kAttnMaxKV) {
        set_error("persistent decode: %d heads of dim %d / %d KV heads not instantiated (one KV head)", nh, hd, nkv);
        return false;
    }
    if (n_layers < 1 || n_layers > kPersistMaxLayers) {
        set_error("persistent decode: %d layers (at most %d)", n_layers, kPersistMaxLayers);
        return false;
    }
    if (groups < nh || groups > kPersistMaxGroups || groups % nh) {
        set_error("persistent decode: %d workgroups (a multiple of the %d heads, at most %d)", groups, nh,
                  kPersistMaxGroups);
        return false;
    }
    if (H % kBlock || nq % kBlock || ffn % kBlock || H > kDecMaxK || nq > kDecMaxK || ffn > kDecMaxK) {
        set_error("persistent decode: GEMV inputs must be multiples of 32 and at most %d", kDecMaxK);
        return false;
    }
    const int worst = light_slots(groups, H, nh, nkv, hd, ffn);
    const int E = (nq + groups - 1) / groups;
    if (worst > kSlots || groups / nh * (E + 4) > kCombMax) {
        set_error("persistent decode: %d workgroups are too few for these shapes", groups);
        return false;
    }
    int dev = 0, cus = 0, occ = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice") ||
        !hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count") ||
        !hip_ok(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, kThreads, 0), "occupancy"))
        return false;
    if (occ * cus < groups) {
        set_error("persistent decode: %d workgroups cannot be co-resident (%d per CU x %d CUs)", groups, occ, cus);
        return false;
    }
    return true;
}

int dec_persist(int dt, const PersistArgs &a, int groups, hipStream_t s) {
    if (a.slots && (!a.log || !a.done || a.vocab > kSlotMaxVocab)) {
        set_error("persistent decode: token slots need the log, the done flag and a vocabulary of at most %d",
                  kSlotMaxVocab);
        return -1;
    }
    const PersistKernel k = kernel_for(dt, a.nh, a.hd, a.H, light_slots(groups, a.H, a.nh, a.nkv, a.hd, a.ffn));
    if (!k) {
        set_error("persistent decode: shape not instantiated");
        return -1;
    }
    // An ordinary launch: persist_supported has checked that `groups` workgroups fit on the
    // device at once, so they are all dispatched together on an otherwise idle device; if
    // they were not, the bounded waits would end the kernel with an error, never a hang.
    hipLaunchKernelGGL(k, dim3(groups), dim3(kThreads), 0, s, a);
    return hip_ok(hipGetLastError(), "persistent decode launch") ? 0 : -1;
}

}  // namespace sapphire
