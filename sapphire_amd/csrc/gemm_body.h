// gemm_body.h - the device side of the batched Q4_0 / Q8_0 GEMM on the matrix cores
// (gemm_mfma.hip describes the method): operand formats, the staging of the activations and
// the body of one workgroup, so that a kernel of another file can run the GEMM beside other
// work in the same launch. Not installed.
#pragma once

#include <algorithm>
#include <climits>

#include "devmath.h"
#include "internal.h"
#include "lanes.h"
#include "nonfinite.h"

namespace sapphire {
namespace {
namespace gemmb {

constexpr int kWave = 64;
constexpr int kWaves = 8;                              // waves per workgroup (two per CU)
constexpr int kWavesWide = 16;                         // the same for a streaming launch (one per CU)
constexpr int kTileRows = 16;
constexpr int kGroupBlocks = 4;
constexpr int kChunkBlocks = 36;                       // A operands staged per workgroup (72 KiB)
constexpr int kBatchMax = 16;
constexpr int kRing = 6;                               // units in flight per wave
constexpr int kNT = 2;                                 // streaming (non-temporal) weight loads
constexpr int kMaxGrid = 1024;                         // workgroups over the tiles

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// k order of the 8 values a lane holds for one block, and the factor of its weight. Q8_0:
// elements 8m+0..7 in order, weights as they are. Q4_0: elements 8m + {0,4,1,5,2,6,3,7},
// the high nibbles (odd elements) left in place as 16 * (nib - 8), so their activations
// are staged divided by 16 (exact: a power of two).
template <int DT>
__device__ __forceinline__ int k_order(int i) {
    if constexpr (DT == DT_Q8_0) return i;
    else return (i >> 1) + 4 * (i & 1);
}
template <int DT>
__device__ __forceinline__ float k_factor(int i) {
    if constexpr (DT == DT_Q8_0) return 1.0f;
    else return (i & 2) ? 0.0625f : 1.0f;
}

// a ? (q ^ b) : b for every bit, in one v_bitop3_b32. Its 8-bit table is indexed by
// {S0, S1, S2} (S0 the most significant bit): with S0 = q, S1 = a, S2 = b that is
// ((0xf0 ^ 0xaa) & 0xcc) | (0xaa & ~0xcc) = 0x6a.
__device__ __forceinline__ uint32_t mask_xor_or(uint32_t q, uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x6a" : "=v"(d) : "v"(q), "v"(a), "v"(b));
    return d;
}

// Exact fp16 weights of block j of a lane's group registers, for the MFMA B operand.
template <int DT>
__device__ __forceinline__ h8 b_operand(const u32x4 (&a)[2], int j, uint32_t kLoMask, uint32_t kHiMask,
                                        uint32_t kLoBits, uint32_t kHiBits) {
    uint32_t w[4];
    _Float16 bias[4];
    if constexpr (DT == DT_Q4_0) {
        // TILED holds nib ^ 8. Halves 0x6400 | nib = 1024 + nib (low nibbles of bytes 0, 2 /
        // 1, 3) and 0x6400 | nib << 4 = 1024 + 16 nib (high nibbles)
        const uint32_t q = a[0][j], q8 = q >> 8;
        w[0] = mask_xor_or(q, kLoMask, kLoBits);
        w[1] = mask_xor_or(q, kHiMask, kHiBits);
        w[2] = mask_xor_or(q8, kLoMask, kLoBits);
        w[3] = mask_xor_or(q8, kHiMask, kHiBits);
        bias[0] = bias[2] = (_Float16)1032.0f;             // 1024 + 8
        bias[1] = bias[3] = (_Float16)1152.0f;             // 1024 + 16 * 8
    } else {
        const u32x4 h = a[j >> 1];
        const uint32_t lo = ((j & 1) ? h.z : h.x) ^ 0x80808080u, hi = ((j & 1) ? h.w : h.y) ^ 0x80808080u;
        // halves 0x64uu = 1024 + (q + 128)
        w[0] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
        w[1] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
        w[2] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
        w[3] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
        bias[0] = bias[1] = bias[2] = bias[3] = (_Float16)1152.0f;   // 1024 + 128
    }
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 v = __builtin_bit_cast(h2, w[i]) - h2{bias[i], bias[i]};   // exact small integers
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

// One ring slot: the weight quants (1 or 2 KiB per wave) and the four block scales of row n.
struct Unit {
    u32x4 a[2];
    float s[4];
};

// Loads of unit (tile, group) gb: the lane's 16 (or 2 x 16) quant bytes and row n's four
// block scales. The unit offset is wave-uniform (scalar offset), the lane part constant.
template <int DT>
__device__ __forceinline__ void unit_issue(Unit &u, __amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs,
                                           uint32_t gb, int lane, int n) {
    constexpr int NQ = DT == DT_Q8_0 ? 2 : 1;
#pragma unroll
    for (int h = 0; h < NQ; ++h)
        u.a[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u + h * 1024u, gb * (NQ * 1024u), kNT));
    if constexpr (NQ == 1) u.a[1] = u.a[0];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        u.s[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, n * 4u + j * 64u, gb * 256u, kNT));
}

struct BConst {
    uint32_t lo_mask, hi_mask, lo_bits, hi_bits;
};

template <int DT>
__device__ __forceinline__ void unit_mfma(const Unit &u, const h8 *__restrict__ xs, int bl, int lane, f4 &acc,
                                          const BConst &k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h8 bop = b_operand<DT>(u.a, j, k.lo_mask, k.hi_mask, k.lo_bits, k.hi_bits);
        f4 C = {0.f, 0.f, 0.f, 0.f};
        C = __builtin_amdgcn_mfma_f32_16x16x32_f16(xs[((bl + j) * 2 + 0) * kWave + lane], bop, C, 0, 0, 0);
        C = __builtin_amdgcn_mfma_f32_16x16x32_f16(xs[((bl + j) * 2 + 1) * kWave + lane], bop, C, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(C[r], u.s[j], acc[r]);
    }
}

// The same for two tiles at once (the same groups of two tiles): each A operand read from LDS
// feeds both tiles' MFMAs; per tile the arithmetic and its order are unit_mfma's.
template <int DT>
__device__ __forceinline__ void unit_mfma2(const Unit &ua, const Unit &ub, const h8 *__restrict__ xs, int bl,
                                           int lane, f4 &acca, f4 &accb, const BConst &k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h8 ahi = xs[((bl + j) * 2 + 0) * kWave + lane], alo = xs[((bl + j) * 2 + 1) * kWave + lane];
        const h8 ba = b_operand<DT>(ua.a, j, k.lo_mask, k.hi_mask, k.lo_bits, k.hi_bits);
        const h8 bb = b_operand<DT>(ub.a, j, k.lo_mask, k.hi_mask, k.lo_bits, k.hi_bits);
        f4 C = {0.f, 0.f, 0.f, 0.f}, D = {0.f, 0.f, 0.f, 0.f};
        C = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, ba, C, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bb, D, 0, 0, 0);
        C = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, ba, C, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bb, D, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acca[r] = __builtin_fmaf(C[r], ua.s[j], acca[r]);
            accb[r] = __builtin_fmaf(D[r], ub.s[j], accb[r]);
        }
    }
}

// Reference-order sums of squares of the staged rows (sum_sq_avx2, normalization.c:12-32:
// eight strided chains, then ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) and the tail), turned into
// the rmsnorm factor 1/sqrtf(sum/dim + eps) of every sequence. raw: [seq][ld] fp32 in LDS.
template <int U = 8>
__device__ void rows_rms_inv(const float *raw, int ld, int dim, int batch, float eps, float (*part)[8], float *rinv) {
    const int t = threadIdx.x;
    if (t < kBatchMax * 8) {
        const int seq = t >> 3, l = t & 7;
        float s = 0.f;
        if (seq < batch) {
            const float *r = raw + seq * ld + l;
            const int n8 = dim >> 3;
            int j = 0;
            for (; j + U <= n8; j += U) {   // U loads in flight, then the chain
                float x[U];
#pragma unroll
                for (int u = 0; u < U; ++u) x[u] = r[(j + u) * 8];
#pragma unroll
                for (int u = 0; u < U; ++u) s = __builtin_fmaf(x[u], x[u], s);
            }
            for (; j < n8; ++j) s = __builtin_fmaf(r[j * 8], r[j * 8], s);
        }
        part[seq][l] = s;
    }
    __syncthreads();
    if (t < batch) {
        const float *pp = part[t];
        const float a0 = pp[0] + pp[4], a1 = pp[1] + pp[5], a2 = pp[2] + pp[6], a3 = pp[3] + pp[7];
        float sum = (a0 + a1) + (a2 + a3);
        for (int i = dim & ~7; i < dim; ++i) sum = __builtin_fmaf(raw[t * ld + i], raw[t * ld + i], sum);
        rinv[t] = devmath::rms_inv_of(sum, dim, eps);
    }
    __syncthreads();
}

__device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const float4 lo = reinterpret_cast<const float4 *>(p)[0], hi = reinterpret_cast<const float4 *>(p)[1];
    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
    v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
}

// LDS of the staging: the A operands [block][hi/lo][lane 16m + seq] of a chunk, and, before
// them (same memory), the rows as fp32 [seq][K + 8] for the reference-order norm sums (the
// pad puts the rows of four sequences in different banks).
constexpr int kRawLd = kChunkBlocks * kBlock + 8;
constexpr int kStageH8 = (kBatchMax * kRawLd * 4 + 15) / 16 > kChunkBlocks * 2 * kWave
                             ? (kBatchMax * kRawLd * 4 + 15) / 16
                             : kChunkBlocks * 2 * kWave;

// Positions of the non-finite activations of a K chunk (at most kChunkBlocks blocks): per
// sequence a bit mask of the +inf and of the -inf elements of every block, and one bit per
// sequence that holds a NaN.
struct NfChunk {
    uint32_t inf[kBatchMax][2][kChunkBlocks];
    uint32_t nan;
};

// Row `row`'s share of the non-finite activations of sequence seq in this chunk (blocks
// b0 .. b0+nbl-1 of rows of nb blocks): NaN if one is NaN, else the fold of fl(w * +-inf)
// over the recorded positions (nonfinite.h).
template <int DT>
__device__ float chunk_fold(const NfChunk &c, const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wsc,
                            int nb, int b0, int nbl, int row, int seq) {
    if ((c.nan >> seq) & 1u) return __builtin_nanf("");
    float a = 0.f;
    for (int bl = 0; bl < nbl; ++bl)
        for (int sg = 0; sg < 2; ++sg)
            for (uint32_t m = c.inf[seq][sg][bl]; m != 0; m &= m - 1) {
                const int k = (b0 + bl) * kBlock + __builtin_ctz(m);
                const float w = nonfinite::weight_at<DT, LAYOUT_TILED>(wq, wsc, nb, row, k);
                a = __fadd_rn(a, __fmul_rn(w, sg ? -INFINITY : INFINITY));
            }
    return a;
}

// The staged operands of one K chunk, formed once per GEMM by gemm_prep_kernel instead of in
// every workgroup: the LDS image of the A operands [block][hi/lo][lane 16m + seq], and per
// sequence the range scale and the non-finite record (1 in nf when the sequence has a NaN or
// infinite activation in this chunk).
struct PrepChunk {
    h8 a[kChunkBlocks * 2 * kWave];
    float xsc[kBatchMax];
    uint32_t inf[kBatchMax][2][kChunkBlocks];
    int nan[kBatchMax];
    int nf[kBatchMax];
};

constexpr int kPrepThreads = 256;
constexpr int kPrepParts = 8;                  // partial sums in flight per prep thread
static_assert(kPrepThreads >= kChunkBlocks * 4, "one (block, quarter) pair per prep thread");

// grid.x: workgroups over the tiles (grid-stride), grid.y: K chunks of `cb` blocks.
// Four waves per SIMD (two workgroups of 8 waves, or one of 16, per CU): at most 128 VGPRs.
// How a workgroup forms its A operands: the full input transform, a copy of the chunk that
// gemm_prep_kernel formed, or a plain x (no sum of parts, norm or residual).
enum StageMode { kStageFull = 0, kStagePrepared = 1, kStagePlain = 2 };

// The LDS of one GEMM workgroup of NW waves.
template <int NW>
struct GemmLds {
    h8 xs[kStageH8];
    float wmax[NW][kBatchMax];
    float xsc[kBatchMax];
    float npart[kBatchMax][8];
    float rinv[kBatchMax];
    NfChunk nfc;
    int wnf[NW];
};

// The GEMM's work as workgroup (bx, by) of a (gdx, gdy) grid, with its LDS in L, so that a
// kernel can run it beside other work. GREEDY: the greedy form (out.tokens): rows are reduced
// to per-sequence partials, not stored.
template <int DT, int MODE, int NW, bool GREEDY>
__device__ __forceinline__ void gemm_body(GemmLds<NW> &L, int bx, int by, int gdx, int gdy,
                                          const uint8_t *__restrict__ wq, uint32_t q_bytes,
                                          const uint8_t *__restrict__ wsc, uint32_t s_bytes, const GemmIn &in,
                                          int batch, int M, int K, int cb, const GemmOut &out,
                                          float *__restrict__ Yp, const PrepChunk *__restrict__ prep, int ks) {
    constexpr int NT = NW * kWave;                 // threads
    constexpr int RING = DT == DT_Q8_0 ? kRing - 1 : kRing;   // Q8_0's units are larger
    constexpr int NP = (kChunkBlocks * 4 + NT / kBatchMax - 1) / (NT / kBatchMax);   // pairs per staging thread
    h8 *xs = L.xs;
    auto &wmax = L.wmax;
    float *xsc = L.xsc;
    auto &npart = L.npart;
    float *rinv = L.rinv;
    NfChunk &nfc = L.nfc;
    int *wnf = L.wnf;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    if (tid == 0) nfc.nan = 0;
    const int nb = K / kBlock, G = nb / kGroupBlocks;
    const int b0 = by * cb, b1 = min(nb, b0 + cb);

    // ---- the wave's units: (tile, 4-block group) pairs of this K chunk ----
    // Unit counters are wave-uniform (scalar registers, scalar branches).
    const int n = lane & 15, m = lane >> 4;
    const int ntiles = (M + kTileRows - 1) / kTileRows;
    const int g0 = b0 / kGroupBlocks, gc = (b1 - b0) / kGroupBlocks;
    // ks waves share a tile (ks <= gc, and then every wave has at most one tile): wave `part`
    // of tile slot `slot` takes groups gs .. gs + gcw - 1 of the chunk
    const int wu = __builtin_amdgcn_readfirstlane(wid);
    const int slot = wu / ks, part = wu - slot * ks;
    const int gs = part * gc / ks, gcw = (part + 1) * gc / ks - gs;
    const int tstride = gdx * (NW / ks);
    const int t0 = bx * (NW / ks) + slot;
    const bool idle = t0 >= ntiles;           // no tile: stages, then leaves
    const int U = idle ? 0 : (ntiles - t0 + tstride - 1) / tstride * gcw;   // units of this wave
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(wq, q_bytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wsc, s_bytes);

    // bit masks of the Q4_0 expansion: nibble fields (low / high nibble of bytes 0 and 2),
    // and outside them the fp16 exponent of 1024, inside them the bits that undo nib ^ 8
    BConst bk = {0x000F000Fu, 0x00F000F0u, 0x64086408u, 0x64806480u};
    asm volatile("" : "+v"(bk.lo_mask), "+v"(bk.hi_mask), "+v"(bk.lo_bits), "+v"(bk.hi_bits));
    // ---- the first RING-1 units' weight loads ----
    // Streaming form (16 waves, one wave per tile): the wave's tiles go in pairs (its tiles
    // 2i and 2i + 1), one pair-unit per group, RP pair-units through the ring.
    constexpr bool PAIR = NW == kWavesWide;
    constexpr int RP = DT == DT_Q8_0 ? 2 : 3;
    Unit ring[PAIR ? 2 * RP : RING];
    // issue pointer: group offset (tile * G + g) of unit u + RING - 1; loads past the last
    // unit repeat it. The offset goes in the scalar offset field, which the buffer range
    // check does not cover, so it must stay inside the matrix: an idle wave reads tile 0.
    int igb = idle ? g0 : t0 * G + g0 + gs, ig = 0, issued = 0;
    // pairs: the wave's tile count, pair-units, and the second tile's offset (a missing
    // second tile repeats the first's loads)
    const int ntw = idle ? 0 : (ntiles - t0 + tstride - 1) / tstride;
    const int PU = (ntw + 1) / 2 * gcw;
    int ip = 0, igb2 = ntw > 1 ? igb + tstride * G : igb;
    auto padvance = [&]() {
        if (issued < PU - 1) {
            ++issued;
            if (++ig == gcw) {
                ig = 0;
                ++ip;
                const int ta = t0 + 2 * ip * tstride;
                igb = ta * G + g0;
                igb2 = 2 * ip + 1 < ntw ? igb + tstride * G : igb;
            } else {
                ++igb;
                ++igb2;
            }
        }
    };
    auto prime = [&]() {
        if constexpr (PAIR) {
#pragma unroll
            for (int p = 0; p < RP - 1; ++p) {
                unit_issue<DT>(ring[2 * p], rq, rs, (uint32_t)igb, lane, n);
                unit_issue<DT>(ring[2 * p + 1], rq, rs, (uint32_t)igb2, lane, n);
                padvance();
            }
        } else {
#pragma unroll
            for (int p = 0; p < RING - 1; ++p) {
                unit_issue<DT>(ring[p], rq, rs, (uint32_t)igb, lane, n);
                if (issued < U - 1) {
                    ++issued;
                    if (++ig == gcw) { ig = 0; igb += tstride * G - (gcw - 1); } else { ++igb; }
                }
            }
        }
    };
    // ---- stage the chunk: input transform, range scale per sequence, hi/lo operands ----
    bool any_nf = false;                               // a NaN / inf activation in this chunk
    if constexpr (MODE == kStagePrepared) {
        // formed by gemm_prep_kernel: copy the chunk's operands (sequences past the batch
        // zero). The weight loads go out first: they do not wait for the operands.
        prime();
        const PrepChunk &pc = prep[by];
        const int na = (b1 - b0) * 2 * kWave;
        constexpr int kCopy = (kChunkBlocks * 2 * kWave + NT - 1) / NT;
        // all loads first: the range scales and non-finite flags with the operands
        const float sc = tid < batch ? pc.xsc[tid] : 1.0f;
        const int nfv = tid < batch ? pc.nf[tid] : 0;
        h8 val[kCopy];
#pragma unroll
        for (int j = 0; j < kCopy; ++j) {
            const int i = tid + j * NT;
            val[j] = i < na ? pc.a[i] : h8{};
        }
#pragma unroll
        for (int j = 0; j < kCopy; ++j) {
            const int i = tid + j * NT;
            if (i < na) xs[i] = (i & 15) < batch ? val[j] : h8{};
        }
        if (tid < kBatchMax) xsc[tid] = sc;
        if (tid < kWave) {                             // the sequences sit in wave 0
            const bool a = __any(nfv != 0) != 0;
            if (tid == 0) wnf[0] = a;
        }
        __syncthreads();
        any_nf = wnf[0] != 0;
        if (any_nf) {
            const int nbl = b1 - b0;
            for (int i = tid; i < batch * 2 * nbl; i += NT) {
                const int q = i / (2 * nbl), sg = (i / nbl) & 1, bl = i % nbl;
                nfc.inf[q][sg][bl] = pc.inf[q][sg][bl];
            }
            if (tid == 0) {
                uint32_t bits = 0;
                for (int q = 0; q < batch; ++q) bits |= (pc.nan[q] ? 1u : 0u) << q;
                nfc.nan = bits;
            }
            __syncthreads();
        }
    } else {
        constexpr bool plain = MODE == kStagePlain;
        // the weights do not wait for x either (Q8_0's larger units do not fit beside it)
        if constexpr (plain && DT == DT_Q4_0) prime();
        const int seq = tid & (kBatchMax - 1), q = tid / kBatchMax;   // q: 0..31
        const int pairs = (b1 - b0) * 4;
        const int kb = b0 * kBlock;
        float *raw = reinterpret_cast<float *>(xs);
        float v[NP][8];    // the delta (parts given), else h
        float xv[NP][8];   // x when it is added to the delta
        // every load of the staging's first stage goes out before any is used
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = q + i * (NT / kBatchMax);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = xv[i][e] = 0.f;
            if (p < pairs && seq < batch) {
                const int k = kb + p * 8;
                // block order: the 64 lanes of a wave read 2 KiB in one piece
                if (plain && in.x_blocked) load8(in.x + block_order_index(seq, k), v[i]);
                else if (in.x) load8(in.x + (size_t)seq * in.ldx + k, !plain && in.parts ? xv[i] : v[i]);
                if (!plain && in.parts) load8(in.parts + (size_t)seq * in.ldp + k, v[i]);
            }
        }
        if (!plain && in.parts) {
            for (int c = 1; c < in.nparts; ++c)
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = q + i * (NT / kBatchMax);
                    if (p < pairs && seq < batch) {
                        float t[8];
                        load8(in.parts + c * in.part_stride + (size_t)seq * in.ldp + kb + p * 8, t);
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[i][e] = __fadd_rn(v[i][e], t[e]);
                    }
                }
            if (in.w_delta) {
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = q + i * (NT / kBatchMax);
                    if (p < pairs)
#pragma unroll
                        for (int e = 0; e < 8; ++e) raw[seq * kRawLd + p * 8 + e] = v[i][e];
                }
                __syncthreads();
                rows_rms_inv(raw, kRawLd, K, batch, in.eps, npart, rinv);
                const float r = rinv[seq];
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = q + i * (NT / kBatchMax);
                    if (p < pairs && seq < batch) {
                        float w[8];
                        load8(in.w_delta + kb + p * 8, w);
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[i][e] = __fmul_rn(__fmul_rn(v[i][e], r), __fadd_rn(1.0f, w[e]));
                    }
                }
            }
            if (in.x)
#pragma unroll
                for (int i = 0; i < NP; ++i)
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[i][e] = __fadd_rn(xv[i][e], v[i][e]);
        }
        if (!plain && in.resid_out && bx == 0 && by == 0)
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = q + i * (NT / kBatchMax);
                if (p < pairs && seq < batch) {
                    float4 *dst = reinterpret_cast<float4 *>(in.resid_out + (size_t)seq * in.ldr + kb + p * 8);
                    dst[0] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
                    dst[1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
                }
            }
        if (!plain && in.w_norm) {
            __syncthreads();                           // raw may still be read by the delta norm
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = q + i * (NT / kBatchMax);
                if (p < pairs)
#pragma unroll
                    for (int e = 0; e < 8; ++e) raw[seq * kRawLd + p * 8 + e] = v[i][e];
            }
            __syncthreads();
            rows_rms_inv(raw, kRawLd, K, batch, in.eps, npart, rinv);
            const float r = rinv[seq];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = q + i * (NT / kBatchMax);
                if (p < pairs && seq < batch) {
                    float w[8];
                    load8(in.w_norm + kb + p * 8, w);
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[i][e] = __fmul_rn(__fmul_rn(v[i][e], r), __fadd_rn(1.0f, w[e]));
                }
            }
        }
        // the range and whether any value is NaN / inf: the largest exponent field is all ones
        // (one integer maximum per value; no per-value flag stays live for the rare path below)
        float mx = 0.f;
        uint32_t emax = 0;
#pragma unroll
        for (int i = 0; i < NP; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                mx = fmaxf(mx, fabsf(v[i][e]));
                emax = max(emax, __float_as_uint(v[i][e]) & 0x7f800000u);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const bool wbad = __any(emax == 0x7f800000u) != 0;
        if (lane < kBatchMax) wmax[wid][lane] = mx;
        if (lane == 0) wnf[wid] = wbad;
        __syncthreads();                               // also ends every read of raw
        mx = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, wmax[w][seq]);
        any_nf = false;
#pragma unroll
        for (int w = 0; w < NW; ++w) any_nf |= wnf[w] != 0;
        if (any_nf) {
            // NaN / inf activations (workgroup-uniform, rare): record where they are, zero them,
            // and take the range maxima again over the rest. Pairs p = 4 bl .. 4 bl + 3 of block
            // bl sit in the lanes 16 (p & 3) + seq of one wave.
            __syncthreads();                           // every wave has read wmax
            mx = 0.f;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = q + i * (NT / kBatchMax);
                uint32_t pinf = 0, ninf = 0;
                bool nan = false;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float t = v[i][e];
                    nan |= t != t;
                    pinf |= (t == INFINITY ? 1u : 0u) << e;
                    ninf |= (t == -INFINITY ? 1u : 0u) << e;
                    v[i][e] = nonfinite::is_nf(t) ? 0.f : t;
                    mx = fmaxf(mx, fabsf(v[i][e]));
                }
                if (nan && p < pairs && seq < batch) atomicOr(&nfc.nan, 1u << seq);
                pinf <<= 8 * (p & 3);
                ninf <<= 8 * (p & 3);
                pinf |= __shfl_xor(pinf, 16, kWave);
                ninf |= __shfl_xor(ninf, 16, kWave);
                pinf |= __shfl_xor(pinf, 32, kWave);
                ninf |= __shfl_xor(ninf, 32, kWave);
                if ((p & 3) == 0 && p < pairs) {
                    nfc.inf[seq][0][p >> 2] = pinf;
                    nfc.inf[seq][1][p >> 2] = ninf;
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            if (lane < kBatchMax) wmax[wid][lane] = mx;
            __syncthreads();
            mx = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) mx = fmaxf(mx, wmax[w][seq]);
        }
        // e: the chunk's largest |x| * 2^-e in [2^14, 2^15) (finite in fp16, lo term normal)
        int e = 0;
        if (mx > 0.f) {
            int ex;
            frexpf(mx, &ex);
            e = ex - 15;
        }
        if (q == 0) xsc[seq] = ldexpf(1.0f, e);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = q + i * (NT / kBatchMax);
            if (p < pairs) {
                h8 hv, lv;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float s = ldexpf(v[i][k_order<DT>(k)], -e) * k_factor<DT>(k);
                    const _Float16 h = (_Float16)s;
                    hv[k] = h;
                    lv[k] = (_Float16)(s - (float)h);
                }
                const int bl = p >> 2, m = p & 3;
                xs[(bl * 2 + 0) * kWave + m * 16 + seq] = hv;
                xs[(bl * 2 + 1) * kWave + m * 16 + seq] = lv;
            }
        }
        __syncthreads();
    }

    if constexpr (MODE == kStageFull || (MODE == kStagePlain && DT != DT_Q4_0)) prime();
    // ---- stream the tiles: units (tile, group) through the register ring ----
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = xsc[4 * m + r];
    // where this chunk's results go: final rows, or the partial sums of chunk by
    float *dst = out.y;
    int ldd = out.ldy;
    if (out.parts) {
        dst = out.parts + (size_t)by * batch * M;
        ldd = M;
    } else if (gdy > 1) {
        dst = Yp + (size_t)by * batch * M;
        ldd = M;
    }
    // greedy form: the best (value, row) so far of sequence 4m + r over the wave's tiles
    float bv[4];
    int bi[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        bv[r] = -INFINITY;
        bi[r] = INT_MAX;
    }
    // the results of tile ct: rows (or GeGLU pairs) times the range scales, plus the non-finite fold
    auto store_tile = [&](int ct, const f4 &a) {
        if constexpr (GREEDY) {
            // the tile's best row per sequence, over the 16 lanes n of each lane group m. A NaN in
            // row 0 wins outright (sample_greedy keeps index 0, as no value compares greater than
            // its starting NaN); other NaN rows and rows past M become (-inf, INT_MAX), which never
            // wins, so every pair compares and no lane keeps a NaN that blocks its partners.
            const int row = ct * kTileRows + n;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float val = a[r] * sc[r];
                int idx = row;
                if (row < M && any_nf && 4 * m + r < batch)
                    val += chunk_fold<DT>(nfc, wq, wsc, nb, b0, b1 - b0, row, 4 * m + r);
                if (row >= M || val != val) {
                    const bool first = row == 0;
                    val = first ? INFINITY : -INFINITY;
                    idx = first ? 0 : INT_MAX;
                }
                lanes::row16_best(val, idx, devmath::greedy_better);
                if (devmath::greedy_better(val, idx, bv[r], bi[r])) {
                    bv[r] = val;
                    bi[r] = idx;
                }
            }
            return;
        }
        if (out.geglu) {
            // lanes n < 8 hold gate rows 8t'+n, lanes n + 8 the matching up rows
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float val = a[r] * sc[r];
                if (any_nf && 4 * m + r < batch)
                    val += chunk_fold<DT>(nfc, wq, wsc, nb, b0, b1 - b0, ct * kTileRows + n, 4 * m + r);
                const float up = __shfl_xor(val, 8, kWave);
                const int j = ct * 8 + n;
                if (n < 8 && 4 * m + r < batch && 2 * j < M)
                    dst[out.y_blocked ? block_order_index(4 * m + r, j) : (size_t)(4 * m + r) * ldd + j] =
                        __fmul_rn(devmath::gelu_ref(val), up);
            }
        } else {
            const int row = ct * kTileRows + n;
            if (row < M)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (4 * m + r < batch) {
                        float val = a[r] * sc[r];
                        if (any_nf) val += chunk_fold<DT>(nfc, wq, wsc, nb, b0, b1 - b0, row, 4 * m + r);
                        if (out.tagged)
                            __hip_atomic_store(out.tagged + (size_t)(4 * m + r) * out.ldy + row,
                                               ((uint64_t)out.tag << 32) | __float_as_uint(val), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                        else
                            dst[out.y_blocked ? block_order_index(4 * m + r, row) : (size_t)(4 * m + r) * ldd + row] = val;
                    }
        }
    };
    // greedy form: the workgroup's best per sequence, from the waves' through LDS once every
    // wave is past its last operand read; one (value, index) partial per sequence and workgroup
    auto greedy_finish = [&]() {
        __syncthreads();
        float *wv = reinterpret_cast<float *>(xs);
        int *wi = reinterpret_cast<int *>(xs) + NW * kBatchMax;
        if (n == 0)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                wv[wid * kBatchMax + 4 * m + r] = bv[r];
                wi[wid * kBatchMax + 4 * m + r] = bi[r];
            }
        __syncthreads();
        if (tid < batch) {
            float v = wv[tid];
            int i = wi[tid];
            for (int w = 1; w < NW; ++w)
                if (devmath::greedy_better(wv[w * kBatchMax + tid], wi[w * kBatchMax + tid], v, i)) {
                    v = wv[w * kBatchMax + tid];
                    i = wi[w * kBatchMax + tid];
                }
            float *o = out.amax + ((size_t)tid * gdx + bx) * 2;
            o[0] = v;
            o[1] = __int_as_float(i);
        }
    };
    int ct = t0, cg = 0;                               // tile and group of the unit multiplied
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (PAIR) {
        f4 acc2 = {0.f, 0.f, 0.f, 0.f};
        int cp = 0;                                    // the pair being multiplied
        for (int base = 0; base < PU; base += RP) {
#pragma unroll
            for (int p = 0; p < RP; ++p) {
                const int sl = (p + RP - 1) % RP;
                unit_issue<DT>(ring[2 * sl], rq, rs, (uint32_t)igb, lane, n);
                unit_issue<DT>(ring[2 * sl + 1], rq, rs, (uint32_t)igb2, lane, n);
                padvance();
                if (base + p < PU) {
                    unit_mfma2<DT>(ring[2 * p], ring[2 * p + 1], xs, cg * kGroupBlocks, lane, acc, acc2, bk);
                    if (++cg == gcw) {
                        store_tile(ct, acc);
                        if (2 * cp + 1 < ntw) store_tile(ct + tstride, acc2);
                        acc = f4{0.f, 0.f, 0.f, 0.f};
                        acc2 = f4{0.f, 0.f, 0.f, 0.f};
                        cg = 0;
                        ++cp;
                        ct += 2 * tstride;
                    }
                }
            }
        }
        if constexpr (GREEDY) greedy_finish();
        return;
    }
    // Every pass issues the loads of all RING slots (past the last unit they repeat it), so
    // each path through the loop has the same load order and the waits stay RING-1 units
    // deep; only the multiplication of units past the end is skipped. (An idle wave has
    // U = 0.)
    for (int base = 0; base < U; base += RING) {
#pragma unroll
        for (int p = 0; p < RING; ++p) {
            unit_issue<DT>(ring[(p + RING - 1) % RING], rq, rs, (uint32_t)igb, lane, n);
            if (issued < U - 1) {
                ++issued;
                if (++ig == gcw) { ig = 0; igb += tstride * G - (gcw - 1); } else { ++igb; }
            }
            if (base + p < U) {
                unit_mfma<DT>(ring[p], xs, (gs + cg) * kGroupBlocks, lane, acc, bk);
                if (++cg == gcw && ks == 1) {
                    store_tile(ct, acc);
                    acc = f4{0.f, 0.f, 0.f, 0.f};
                    cg = 0;
                    ct += tstride;
                }
            }
        }
    }
    if (ks > 1) {
        // the tile's share sums, in part order, through LDS (the operands are no longer read)
        __syncthreads();
        f4 *red = reinterpret_cast<f4 *>(xs);
        if (part > 0 && !idle) red[(slot * (ks - 1) + part - 1) * kWave + lane] = acc;
        __syncthreads();
        if (part == 0 && !idle) {
            for (int q = 1; q < ks; ++q) acc += red[(slot * (ks - 1) + q - 1) * kWave + lane];
            store_tile(t0, acc);
        }
    }
    if constexpr (GREEDY) greedy_finish();
}

}  // namespace gemmb
}  // namespace
}  // namespace sapphire
