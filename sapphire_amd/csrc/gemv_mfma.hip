// gemv_mfma.hip - Q8_0 / Q4_0 GEMV on the CDNA4 matrix cores, for long weight matrices
// (the LM head: 262144 x 640 and 262144 x 1152).
//
// Semantics are those of the reference's kernel_gemv (dispatch.c:101-156 with the row
// kernels q4_0_avx.c:102-148 / q8_0_avx.c:16-136): y[r] = sum_b scale[r][b] * sum_e
// int(r, b, e) * x[32b + e], int = (nib - 8) for Q4_0 (element 2j = low nibble of byte j)
// and the int8 quant for Q8_0.
//
// Why the matrix cores. A fp32 GEMV spends two VALU operations per weight (convert +
// FMA); at 20 bytes per 32 Q4_0 weights that keeps the SIMDs as busy as HBM, and the two
// phases do not overlap well. Here the integer weights go straight into
// v_mfma_i32_16x16x32_i8, so the VALU work per block shrinks to applying its scale.
//
// x is turned into exact integers once per wave: per 32-element block, X = rint(x*2^sh)
// with sh chosen so that the block's largest |x| maps below 2^30 (an absolute error
// <= 2^-31 * max|x_block| per element, below the rounding of fp32 products), and X is
// split into four signed 8-bit digits, X = sum_d D_d * 256^d. The B operand of the MFMA
// holds the digits: column n = 4j + d (j = block of a 4-block group, d = digit), so one
// MFMA per block of the group leaves in C[row][4j+d] the exact integer sum_e int*D_d over
// block j. Each lane then applies scale[row][block] * 2^(8d - sh) to its four C values
// with one FMA each, and the sixteen columns of a row are summed across the lanes of a
// 16-lane row group with a ds_swizzle reduce-scatter.
//
// Weights live in the TILED layout (built by launch_convert), so every load instruction
// of a wave reads one contiguous KiB:
//   quants  [tile = 16 rows][group = 4 blocks][..][lane 64][16 B]
//     Q8_0: two 1 KiB halves per (tile, group); lane l = 16m + i holds, for blocks 2h and
//           2h+1 of the group, the 8 quants e = 8m..8m+7 of row i (the MFMA A operand).
//     Q4_0: one 1 KiB slab; lane l holds, for blocks 0..3 of the group, the 4 bytes
//           4m..4m+3 of row i's block (elements 8m..8m+7), each nibble stored as
//           nib ^ 8 (the 4-bit two's complement of nib - 8), expanded in registers.
//   scales  [tile][group][block 4][row 16] fp32, after the quants at a 256-byte boundary.
// Rows past M in the last tile are zero.
#include <algorithm>

#include "internal.h"
#include "lanes.h"
#include "nonfinite.h"

namespace sapphire {

namespace {

constexpr int kWave = 64;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kTileRows = 16;
constexpr int kGroupBlocks = 4;
constexpr int kNT = 2;   // nontemporal: the weights are streamed once

template <int DT> struct TL;
template <> struct TL<DT_Q4_0> { static constexpr int BB = 20; };   // AoS block bytes
template <> struct TL<DT_Q8_0> { static constexpr int BB = 36; };

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT));
}

template <int MASK>
__device__ __forceinline__ float swz_xor(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (MASK << 10)));
}

// Reduce-scatter over the 16 lanes of a row group (lanes 16m..16m+15): lane n enters with
// its column's contributions a[0..3] to rows 4m..4m+3 and leaves with the full row sum of
// row 4m + ((n >> 2) & 3). Lane bit 3 picks the row pair kept at the first exchange, bit
// 2 the row kept of that pair; bits 1 and 0 finish the sum.
__device__ __forceinline__ float row16_scatter(const float (&a)[4], int n) {
    const bool b3 = (n & 8) != 0, b2 = (n & 4) != 0;
    float k0 = b3 ? a[2] : a[0], k1 = b3 ? a[3] : a[1];
    const float s0 = b3 ? a[0] : a[2], s1 = b3 ? a[1] : a[3];
    k0 += swz_xor<8>(s0);
    k1 += swz_xor<8>(s1);
    float k = b2 ? k1 : k0;
    k += swz_xor<4>(b2 ? k0 : k1);
    k += swz_xor<2>(k);
    k += swz_xor<1>(k);
    return k;
}

// The MFMA B operand of this lane for group g (8 signed digits) and the factor
// 2^(8d - sh) of its column. Lane l supplies column n = l % 16 (block j = n / 4 of the
// group, digit d = n % 4) for the k-slots of lane group m = l / 16: elements 8m..8m+7 of
// block 4g + j, in the order the A operand holds them (natural for Q8_0; even then odd
// elements for Q4_0, whose A bytes are the low nibbles, then the high nibbles).
// NaN and infinite activations are zeroed here (nf is set): the row results get their fold
// added when they are stored.
template <int DT>
__device__ __forceinline__ void lane_digits(const float *__restrict__ x, int g, int lane, uint32_t &w0,
                                            uint32_t &w1, float &p, bool &nf) {
    const int n = lane & 15, m = lane >> 4;
    const int j = n >> 2, d = n & 3;
    const float4 *xp = reinterpret_cast<const float4 *>(x + (4 * g + j) * 32 + 8 * m);
    const float4 va = xp[0], vb = xp[1];
    float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
    int mexp = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        nf |= nonfinite::is_nf(v[i]);
        v[i] = nonfinite::is_nf(v[i]) ? 0.f : v[i];
        mexp = max(mexp, (int)((__float_as_uint(v[i]) >> 23) & 0xFFu));
    }
    // the block's 32 elements are held by lanes n, n+16, n+32, n+48
    mexp = max(mexp, __shfl_xor(mexp, 16, kWave));
    mexp = max(mexp, __shfl_xor(mexp, 32, kWave));
    const int sh = 156 - mexp;   // max |x_block| < 2^(mexp-126), so |X| < 2^30
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int src = DT == DT_Q8_0 ? i : (i < 4 ? 2 * i : 2 * (i - 4) + 1);
        const int X = (int)rintf(ldexpf(v[src], sh));
        const uint32_t U = ((uint32_t)X + 0x80808080u) ^ 0x80808080u;   // bytes = signed digits
        b[i] = (U >> (8 * d)) & 0xFFu;
    }
    w0 = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    w1 = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    // Q4_0 A bytes carry 16 * (nib - 8); the 1/16 is folded in here (exact)
    p = ldexpf(1.0f, 8 * d - sh - (DT == DT_Q4_0 ? 4 : 0));
}

// A operand of the MFMA for block jj of the group.
template <int DT>
__device__ __forceinline__ long a_operand(const u32x4 (&a)[2], int jj) {
    if constexpr (DT == DT_Q8_0) {
        const u32x4 h = a[jj >> 1];
        const uint32_t lo = (jj & 1) ? h.z : h.x, hi = (jj & 1) ? h.w : h.y;
        return (long)(((unsigned long)hi << 32) | lo);
    } else {
        const uint32_t q = a[0][jj];                    // nibbles stored as nib ^ 8
        const uint32_t even = (q << 4) & 0xF0F0F0F0u;   // int8 16*(nib-8) of elements 0,2,4,6
        const uint32_t odd = q & 0xF0F0F0F0u;           // ... of elements 1,3,5,7
        return (long)(((unsigned long)odd << 32) | even);
    }
}

// Registers of one tile's loads: the A operands of every group and the lane's scales.
template <int NG>
struct TileRegs {
    u32x4 a[NG][2];
    u32x4 sv[NG];
};

template <int DT, int NG>
__device__ __forceinline__ void tile_issue(TileRegs<NG> &R, __amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs,
                                           int t, int lane) {
    constexpr int NQ = DT == DT_Q8_0 ? 2 : 1;
    const int jc = (lane & 15) >> 2, m = lane >> 4;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const uint32_t gb = (uint32_t)(t * NG + g);
#pragma unroll
        for (int h = 0; h < NQ; ++h) R.a[g][h] = load16(rq, (gb * NQ + h) * 1024u + lane * 16u);
        R.sv[g] = load16(rs, ((gb * 4u + jc) * 16u + 4u * m) * 4u);
    }
}

// Four MFMAs per group (one per block; the lane's B digits enter only the MFMA of the
// block its column belongs to) and the scales applied to the C values: acc[r] = this
// lane's column of rows 4m + r.
template <int DT, int NG>
__device__ __forceinline__ void tile_mfma(const TileRegs<NG> &R, const long (&bop)[NG], const float (&p)[NG],
                                          int lane, float (&acc)[4]) {
    const int jc = (lane & 15) >> 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        i32x4 C = {0, 0, 0, 0};
#pragma unroll
        for (int jj = 0; jj < kGroupBlocks; ++jj)
            C = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_operand<DT>(R.a[g], jj), jc == jj ? bop[g] : 0L, C, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[r] = __builtin_fmaf((float)C[r], __uint_as_float(R.sv[g][r]) * p[g], acc[r]);
    }
}

// Running (max, sum of exp(v - max), first index of the max) of a stream of logits: the
// softmax / greedy-argmax partial of the rows a lane stores (utils.c:18-59, 145-156).
struct SoftPart {
    float m, s;
    int i;
};

// e^d as one v_exp_f32 of d * log2(e): the running sums only normalise the probabilities,
// which are formed with expf (1-ulp-class differences in the sum, far inside the softmax
// tolerance)
__device__ __forceinline__ float exp_fast(float d) { return __builtin_amdgcn_exp2f(d * 1.44269504088896341f); }

// A +inf logit contributes exp(inf - inf) = NaN to the sum, as in utils.c:43-46, so every
// probability of such a vector is NaN there and here.
__device__ __forceinline__ void soft_push(SoftPart &p, float v, int row) {
    if (v > p.m) {                      // strict: an equal later value keeps the earlier index
        p.s = (p.m == -INFINITY ? 0.f : p.s * exp_fast(p.m - v)) + exp_fast(v - v);
        p.m = v;
        p.i = row;
    } else {
        p.s += exp_fast(v - p.m);
    }
}

__device__ __forceinline__ SoftPart soft_merge(SoftPart a, SoftPart b) {
    const float m = fmaxf(a.m, b.m);
    SoftPart r;
    r.m = m;
    r.s = (a.m == -INFINITY ? 0.f : a.s * exp_fast(a.m - m)) + (b.m == -INFINITY ? 0.f : b.s * exp_fast(b.m - m));
    r.i = (b.m > a.m || (b.m == a.m && b.i < a.i)) ? b.i : a.i;
    return r;
}

template <int CTRL>
__device__ __forceinline__ SoftPart soft_dpp(const SoftPart &p) {
    return SoftPart{lanes::dpp_mov<CTRL>(p.m), lanes::dpp_mov<CTRL>(p.s),
                    __float_as_int(lanes::dpp_mov<CTRL>(__int_as_float(p.i)))};
}

__device__ __forceinline__ SoftPart soft_lane(const SoftPart &p, int l) {
    return SoftPart{__int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.m), l)),
                    __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.s), l)), __builtin_amdgcn_readlane(p.i, l)};
}

// The merge of the wave's 64 partials, the same in every lane: rows of 16 lanes by DPP
// (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror; each lane merges with a
// partner that holds the same set, and soft_merge is commutative, so a row's lanes agree), then
// the four rows' merges in row order.
__device__ __forceinline__ SoftPart soft_wave_fold(SoftPart p) {
    p = soft_merge(p, soft_dpp<0xB1>(p));
    p = soft_merge(p, soft_dpp<0x4E>(p));
    p = soft_merge(p, soft_dpp<0x141>(p));
    p = soft_merge(p, soft_dpp<0x140>(p));
    SoftPart r = soft_lane(p, 0);
    r = soft_merge(r, soft_lane(p, 16));
    r = soft_merge(r, soft_lane(p, 32));
    return soft_merge(r, soft_lane(p, 48));
}

// sample_greedy's order (utils.c:145-156: best = 0, then every later strictly greater value)
// as one unsigned 64-bit key, the larger key the better (value, index) pair: the value's
// bits mapped to an unsigned order (-0 taken as +0, which compares equal to it) in the high
// half, the complement of the index in the low half, so that equal values prefer the lower
// index. A NaN never wins, except at index 0, which sample_greedy keeps (no value compares
// greater than NaN): that key is the largest, and its low half decodes to index 0 too.
__device__ __forceinline__ unsigned long long greedy_key(float v, int row) {
    if (v != v) return row == 0 ? ~0ull : 0ull;
    uint32_t u = v == 0.f ? 0u : __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xFFFFFFFFu - (uint32_t)row);
}

// What tile_store needs for activations with NaN / inf elements (nf, wave-uniform): the
// weight planes, the blocks per row and x itself, for the fold of its non-finite elements.
struct NfCtx {
    const uint8_t *wq, *wsc;
    int nb;
    const float *x;
    bool nf;
};

// Epilogues of the TILED GEMV: the logits only; the logits and each workgroup's softmax /
// argmax partial; the logits and the greedy token with the decode step's advance.
constexpr int kEpNone = 0, kEpSoftmax = 1, kEpGreedyStep = 2, kEpGreedySlots = 3;
static_assert(kGreedyGroups == 8, "one counter per XCD-interleaved group of workgroups");

// The 16 columns of each row summed across the row group; lane 16m + 4r stores row
// 4m + r and folds it into its softmax partial (kEpSoftmax) or its greedy key (kEpGreedyStep).
template <int DT, int EP>
__device__ __forceinline__ void tile_store(const float (&acc)[4], float *__restrict__ y, int M, int t, int lane,
                                           SoftPart &sp, unsigned long long &key, const NfCtx &nc) {
    const int n = lane & 15;
    float v = row16_scatter(acc, n);
    const int row = t * kTileRows + 4 * (lane >> 4) + ((n >> 2) & 3);
    if ((n & 3) == 0 && row < M) {
        if (nc.nf) v += nonfinite::fold<DT, LAYOUT_TILED>(nc.wq, nc.wsc, nc.nb, row, nc.x);
        y[row] = v;
        if constexpr (EP == kEpSoftmax) soft_push(sp, v, row);
        if constexpr (EP == kEpGreedyStep || EP == kEpGreedySlots) {
            const unsigned long long k = greedy_key(v, row);
            key = k > key ? k : key;
        }
    }
}

// Waves walk the 16-row tiles with a grid stride. Where two tiles' loads fit in registers
// (DB) the next tile is loaded before the current one is consumed; otherwise its loads
// are issued as soon as the current tile's MFMAs have read their operands. Each wave
// builds its B digits once. With kEpSoftmax every workgroup also leaves the softmax/argmax
// partial of its rows in part[blockIdx.x] (folded by softmax_finish_parts). With
// kEpGreedyStep every workgroup leaves the greedy key of its rows in its slot of gs.keys and
// counts itself done; the last one takes the maximum key, decodes the token and advances the
// decode state (dec_advance_kernel's work), so the step needs no further launch. With
// kEpGreedySlots every workgroup folds its key into its group's slot of gs.slots, tagged with
// the step (gs.slots->b), and workgroup 0 writes gs.slots->a = b: the next step's layers
// kernel picks the token.
template <int DT, int NG, int EP>
__global__ __launch_bounds__(256) void gemv_mfma(const uint8_t *__restrict__ wq, uint32_t q_bytes,
                                                 const uint8_t *__restrict__ wsc, uint32_t s_bytes,
                                                 const float *__restrict__ x, float *__restrict__ y, int M,
                                                 int ntiles, SoftPart *__restrict__ part, GreedyStep gs) {
    constexpr int NQ = DT == DT_Q8_0 ? 2 : 1;
    constexpr bool DB = NG * (NQ + 1) * 4 * 2 <= 128;   // VGPRs of two tiles' loads
    const int lane = threadIdx.x & (kWave - 1), nw_blk = blockDim.x / kWave;
    const int wave = blockIdx.x * nw_blk + threadIdx.x / kWave;
    const int nwaves = gridDim.x * nw_blk;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(wq, q_bytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wsc, s_bytes);

    TileRegs<NG> RA;
    int t = wave;
    if (t < ntiles) tile_issue<DT, NG>(RA, rq, rs, t, lane);
    // a stopped sequence: the whole launch returns (every workgroup reads the same flag, so no
    // key slot or counter is touched); the check waits behind the first tile's loads
    if constexpr (EP == kEpGreedyStep || EP == kEpGreedySlots)
        if (gs.done && *gs.done) return;
    uint32_t tag = 0;
    if constexpr (EP == kEpGreedySlots) tag = gs.slots->b;

    float p[NG];
    long bop[NG];
    bool nfl = false;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        uint32_t w0, w1;
        lane_digits<DT>(x, g, lane, w0, w1, p[g], nfl);
        bop[g] = (long)(((unsigned long)w1 << 32) | w0);
    }
    // the wave's lanes cover all of x
    const NfCtx nc{wq, wsc, NG * kGroupBlocks, x, __any(nfl) != 0};

    float acc[4];
    SoftPart sp{-INFINITY, 0.f, 0x7fffffff};
    unsigned long long key = 0;
    if constexpr (DB) {
        TileRegs<NG> RB;
        while (t < ntiles) {
            if (t + nwaves < ntiles) tile_issue<DT, NG>(RB, rq, rs, t + nwaves, lane);
            tile_mfma<DT, NG>(RA, bop, p, lane, acc);
            tile_store<DT, EP>(acc, y, M, t, lane, sp, key, nc);
            t += nwaves;
            if (t >= ntiles) break;
            if (t + nwaves < ntiles) tile_issue<DT, NG>(RA, rq, rs, t + nwaves, lane);
            tile_mfma<DT, NG>(RB, bop, p, lane, acc);
            tile_store<DT, EP>(acc, y, M, t, lane, sp, key, nc);
            t += nwaves;
        }
    } else {
        while (t < ntiles) {
            tile_mfma<DT, NG>(RA, bop, p, lane, acc);
            const int tn = t + nwaves;
            if (tn < ntiles) tile_issue<DT, NG>(RA, rq, rs, tn, lane);
            tile_store<DT, EP>(acc, y, M, t, lane, sp, key, nc);
            t = tn;
        }
    }
    if constexpr (EP == kEpGreedyStep) {
        key = lanes::u64_wave_max(key);
        __shared__ unsigned long long wkeys[4];
        __shared__ int last;
        const int wid = threadIdx.x / kWave;
        if (lane == 0) wkeys[wid] = key;
        __syncthreads();
        const unsigned nb = gridDim.x, ng = nb < kGreedyGroups ? nb : kGreedyGroups;
        if (threadIdx.x == 0) {
            unsigned long long b = wkeys[0];
            for (int w = 1; w < nw_blk; ++w) b = wkeys[w] > b ? wkeys[w] : b;
            // this workgroup's key in its own slot, acknowledged before the workgroup counts
            // itself done: one count per workgroup on its group's counter (blockIdx % 8), one per
            // group on the top counter, so no address takes more than nb / 8 atomics
            __hip_atomic_store(gs.keys + blockIdx.x, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            const unsigned g = blockIdx.x % kGreedyGroups;
            const unsigned gsize = nb / kGreedyGroups + (g < nb % kGreedyGroups ? 1u : 0u);
            int is_last = 0;
            if (__hip_atomic_fetch_add(gs.count + 1 + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gsize - 1) {
                __hip_atomic_store(gs.count + 1 + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                is_last = __hip_atomic_fetch_add(gs.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ng - 1;
            }
            last = is_last;
        }
        __syncthreads();
        if (last) {
            // every workgroup's key has been acknowledged: the maximum, then the advance
            unsigned long long b = 0;
            for (unsigned i = threadIdx.x; i < nb; i += blockDim.x) {
                const unsigned long long k = __hip_atomic_load(gs.keys + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                b = k > b ? k : b;
            }
            b = lanes::u64_wave_max(b);
            if (lane == 0) wkeys[wid] = b;
            __syncthreads();
            if (threadIdx.x == 0) {
                unsigned long long k = wkeys[0];
                for (int w = 1; w < nw_blk; ++w) k = wkeys[w] > k ? wkeys[w] : k;
                const uint32_t r = 0xFFFFFFFFu - (uint32_t)k;
                const int tok = k != 0 && r < (uint32_t)M ? (int)r : 0;
                __hip_atomic_store(gs.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int s = *gs.step;
                *gs.tok = tok;
                gs.log[s] = tok;
                *gs.step = s + 1;
                *gs.pos = *gs.pos + 1;
                if (gs.seq) *gs.seq = *gs.seq + 1u;
                if (gs.done && gs.stop.has(tok)) *gs.done = 1;   // inference.c:298-301
            }
        }
    }
    if constexpr (EP == kEpGreedySlots) {
        key = lanes::u64_wave_max(key);
        __shared__ unsigned long long wkeys[4];
        const int wid = threadIdx.x / kWave;
        if (lane == 0) wkeys[wid] = key;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = wkeys[0];
            for (int w = 1; w < nw_blk; ++w) b = wkeys[w] > b ? wkeys[w] : b;
            // no return value: the launch's end waits for it, nothing in the launch does
            __hip_atomic_fetch_max(gs.slots->key + blockIdx.x % kSlotCount, slot_key(b, tag), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            if (blockIdx.x == 0) gs.slots->a = tag;
        }
    }
    if constexpr (EP == kEpSoftmax) {
        // lanes 16m + 4r hold the wave's partials (the others are still empty, and merge as
        // the identity)
        sp = soft_wave_fold(sp);
        __shared__ SoftPart wparts[4];
        const int wid = threadIdx.x / kWave;
        if (lane == 0) wparts[wid] = sp;
        __syncthreads();
        if (threadIdx.x == 0) {
            SoftPart b = wparts[0];
            for (int w = 1; w < nw_blk; ++w) b = soft_merge(b, wparts[w]);
            part[blockIdx.x] = b;
        }
    }
}

constexpr int kFinishVec = 1;   // float4 logits per thread and pass of softmax_finish_parts

// Every block folds the nparts partials (256 threads, then the block), block 0 writes the
// greedy token, and each block turns its chunk of logits into probabilities:
// probs[i] = exp(logits[i] - max) / sum (utils.c:43-58).
__global__ __launch_bounds__(256) void softmax_finish_parts(const float *__restrict__ logits, int n, int chunk,
                                                            const SoftPart *__restrict__ part, int nparts,
                                                            float *__restrict__ probs, int *__restrict__ argmax,
                                                            int aligned) {
    __shared__ SoftPart wp[4];
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    // the first pass's logits (and logits[0] for the token) are loaded before the partials are
    // folded (independent loads)
    const float l0 = blockIdx.x == 0 && threadIdx.x == 0 && argmax ? logits[0] : 0.f;
    constexpr int U = kFinishVec;
    const int begin = blockIdx.x * chunk, end = min(n, begin + chunk);
    float4 v0[U];
    if (probs && aligned)
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = begin + 4 * threadIdx.x + 4 * u * blockDim.x;
            v0[u] = i + 3 < end ? *reinterpret_cast<const float4 *>(logits + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    // four partials per thread and trip, all four loads issued before any is merged (the fold's
    // order changes only the rounding of the sum: ties keep the lower index whatever the order)
    const SoftPart none{-INFINITY, 0.f, 0x7fffffff};
    SoftPart b = none;
    for (int i = threadIdx.x; i < nparts; i += 4 * blockDim.x) {
        SoftPart q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = i + k * (int)blockDim.x < nparts ? part[i + k * blockDim.x] : none;
        b = soft_merge(b, soft_merge(soft_merge(q[0], q[1]), soft_merge(q[2], q[3])));
    }
    b = soft_wave_fold(b);
    if (lane == 0) wp[wid] = b;
    __syncthreads();
    // every thread folds the waves' partials in the same order (the same result everywhere)
    SoftPart t = wp[0];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) t = soft_merge(t, wp[w]);
    // sample_greedy (utils.c:145-156) starts at index 0 and only a greater logit replaces it:
    // 0 when logits[0] is NaN or no logit is above -inf, else the first maximum
    if (blockIdx.x == 0 && threadIdx.x == 0 && argmax) *argmax = (t.i >= 0 && t.i < n && !isnan(l0)) ? t.i : 0;
    if (!probs) return;
    const float m = t.m, inv = 1.0f / t.s;
    if (!aligned) {
        for (int i = begin + threadIdx.x; i < end; i += blockDim.x) probs[i] = expf(logits[i] - m) * inv;
        return;
    }
    // kFinishVec 16-byte loads in flight per thread, then their exps and stores
    for (int i0 = begin + 4 * threadIdx.x; i0 < end; i0 += 4 * U * blockDim.x) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + 4 * u * blockDim.x;
            v[u] = i0 == begin + 4 * (int)threadIdx.x ? v0[u]
                   : (i + 3 < end ? *reinterpret_cast<const float4 *>(logits + i) : make_float4(0.f, 0.f, 0.f, 0.f));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + 4 * u * blockDim.x;
            if (i + 3 < end) {
                const float4 r = make_float4(expf(v[u].x - m) * inv, expf(v[u].y - m) * inv, expf(v[u].z - m) * inv,
                                             expf(v[u].w - m) * inv);
                *reinterpret_cast<float4 *>(probs + i) = r;
            } else {
                for (int e = i; e < end && e < i + 4; ++e) probs[e] = expf(logits[e] - m) * inv;
            }
        }
    }
}

// One thread per (row, block) of the AoS array: scatter into the TILED layout.
template <int DT>
__global__ void to_tiled_kernel(const uint8_t *__restrict__ aos, uint8_t *__restrict__ q, float *__restrict__ sc,
                                int M, int nb) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)M * nb) return;
    const int r = (int)(idx / nb), b = (int)(idx - (long)r * nb);
    const int G = nb / kGroupBlocks;
    const int t = r / kTileRows, i = r % kTileRows, g = b / kGroupBlocks, j = b % kGroupBlocks;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(aos + (size_t)idx * TL<DT>::BB);
    const size_t gb = (size_t)t * G + g;
    sc[(gb * kGroupBlocks + j) * kTileRows + i] = __uint_as_float(src[0]);
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        if constexpr (DT == DT_Q8_0) {
            uint32_t *dst = reinterpret_cast<uint32_t *>(q + (gb * 2 + (j >> 1)) * 1024 + (mm * 16 + i) * 16 +
                                                         (j & 1) * 8);
            dst[0] = src[1 + 2 * mm];
            dst[1] = src[2 + 2 * mm];
        } else {
            uint32_t *dst = reinterpret_cast<uint32_t *>(q + gb * 1024 + (mm * 16 + i) * 16 + j * 4);
            dst[0] = src[1 + mm] ^ 0x88888888u;
        }
    }
}

// The reference block image (scale + quants) of block (r, b) read back from TILED.
template <int DT>
__global__ void tiled_unpack_kernel(const uint8_t *__restrict__ q, const float *__restrict__ sc, int M, int nb,
                                    int8_t *__restrict__ ints, float *__restrict__ deq) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)M * nb) return;
    const int r = (int)(idx / nb), b = (int)(idx - (long)r * nb);
    const int G = nb / kGroupBlocks;
    const int t = r / kTileRows, i = r % kTileRows, g = b / kGroupBlocks, j = b % kGroupBlocks;
    const size_t gb = (size_t)t * G + g;
    const float s = sc[(gb * kGroupBlocks + j) * kTileRows + i];
    uint8_t qb[32];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        if constexpr (DT == DT_Q8_0) {
            const uint8_t *p = q + (gb * 2 + (j >> 1)) * 1024 + (mm * 16 + i) * 16 + (j & 1) * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) qb[8 * mm + e] = p[e];
        } else {
            const uint8_t *p = q + gb * 1024 + (mm * 16 + i) * 16 + j * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) qb[4 * mm + e] = p[e] ^ 0x88u;
        }
    }
    for (int e = 0; e < 32; ++e) {
        int v;
        if constexpr (DT == DT_Q4_0) v = (int)((e & 1) ? (qb[e >> 1] >> 4) : (qb[e >> 1] & 0xFu)) - 8;
        else v = (int)(int8_t)qb[e];
        if (ints) ints[(size_t)idx * 32 + e] = (int8_t)v;
        if (deq) deq[(size_t)idx * 32 + e] = __fmul_rn((float)v, s);
    }
}

int cus_of_current_device() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}

// Waves per CU of the TILED GEMV. Measured on the 262144 x 640 LM head with cold weights:
// Q8_0 (11.5 KiB per tile) is fastest at 8 (two per SIMD, its register limit for the double
// buffer anyway), Q4_0 (6.4 KiB per tile, half the bytes per wave) at 12 (3 %).
constexpr int kWavesPerCuQ8 = 8, kWavesPerCuQ4 = 12;

unsigned tiled_blocks(int dt, int M) {
    const int ntiles = (M + kTileRows - 1) / kTileRows;
    const int per_cu = dt == DT_Q4_0 ? kWavesPerCuQ4 : kWavesPerCuQ8;
    const long waves = std::min<long>(ntiles, (long)cus_of_current_device() * per_cu);
    return (unsigned)((waves + 3) / 4);
}

template <int DT, int NG>
int launch_mfma_typed(const uint8_t *w, int M, int K, const float *x, float *y, SoftPart *part,
                      const GreedyStep *gs, hipStream_t st) {
    const int ntiles = (M + kTileRows - 1) / kTileRows;
    const size_t so = q_tiled_scales_offset(DT, M, K);
    const size_t sbytes = q_tiled_bytes(DT, M, K) - so;
    const unsigned blocks = tiled_blocks(DT, M);
    const GreedyStep g = gs ? *gs : GreedyStep{};
    if (gs && gs->slots)
        hipLaunchKernelGGL((gemv_mfma<DT, NG, kEpGreedySlots>), dim3(blocks), dim3(256), 0, st, w, (uint32_t)so,
                           w + so, (uint32_t)sbytes, x, y, M, ntiles, part, g);
    else if (gs)
        hipLaunchKernelGGL((gemv_mfma<DT, NG, kEpGreedyStep>), dim3(blocks), dim3(256), 0, st, w, (uint32_t)so,
                           w + so, (uint32_t)sbytes, x, y, M, ntiles, part, g);
    else if (part)
        hipLaunchKernelGGL((gemv_mfma<DT, NG, kEpSoftmax>), dim3(blocks), dim3(256), 0, st, w, (uint32_t)so, w + so,
                           (uint32_t)sbytes, x, y, M, ntiles, part, g);
    else
        hipLaunchKernelGGL((gemv_mfma<DT, NG, kEpNone>), dim3(blocks), dim3(256), 0, st, w, (uint32_t)so, w + so,
                           (uint32_t)sbytes, x, y, M, ntiles, part, g);
    return hip_ok(hipGetLastError(), "gemv_mfma launch") ? 0 : -1;
}

int launch_tiled(int dt, const void *w, int M, int K, const float *x, float *y, SoftPart *part, hipStream_t st,
                 const GreedyStep *gs = nullptr) {
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const int ng = K / (kGroupBlocks * kBlock);
#define SPH_TILED_CASE(DTV, NGV) \
    if (dt == DTV && ng == NGV) return launch_mfma_typed<DTV, NGV>(wb, M, K, x, y, part, gs, st);
    SPH_TILED_CASE(DT_Q4_0, 5) SPH_TILED_CASE(DT_Q4_0, 8) SPH_TILED_CASE(DT_Q4_0, 9)
    SPH_TILED_CASE(DT_Q8_0, 5) SPH_TILED_CASE(DT_Q8_0, 8) SPH_TILED_CASE(DT_Q8_0, 9)
#undef SPH_TILED_CASE
    set_error("TILED GEMV: K=%d is not supported (K/128 must be 5, 8 or 9)", K);
    return -1;
}

}  // namespace

bool tiled_layout_ok(int dt, int M, int K) {
    if (!is_quant(dt) || M <= 0 || K <= 0 || K % (kGroupBlocks * kBlock) != 0) return false;
    return q_tiled_bytes(dt, M, K) < (size_t(1) << 32) - 256;   // 32-bit buffer offsets
}

bool tiled_supported(int dt, int M, int K) {
    const int ng = K / (kGroupBlocks * kBlock);
    return tiled_layout_ok(dt, M, K) && (ng == 5 || ng == 8 || ng == 9);
}

size_t q_tiled_scales_offset(int dt, int M, int K) {
    const size_t tiles = (size_t)(M + kTileRows - 1) / kTileRows, groups = (size_t)K / (kGroupBlocks * kBlock);
    const size_t qbytes = tiles * groups * (dt == DT_Q4_0 ? 1024 : 2048);
    return (qbytes + 255) & ~size_t(255);
}

size_t q_tiled_bytes(int dt, int M, int K) {
    const size_t tiles = (size_t)(M + kTileRows - 1) / kTileRows, groups = (size_t)K / (kGroupBlocks * kBlock);
    return q_tiled_scales_offset(dt, M, K) + tiles * groups * kGroupBlocks * kTileRows * sizeof(float);
}

int launch_to_tiled(int dt, const void *aos, int M, int K, void *out, hipStream_t st) {
    const int nb = K / kBlock;
    uint8_t *q = static_cast<uint8_t *>(out);
    float *sc = reinterpret_cast<float *>(q + q_tiled_scales_offset(dt, M, K));
    if (!hip_ok(hipMemsetAsync(out, 0, q_tiled_bytes(dt, M, K), st), "tiled memset")) return -1;
    const long n = (long)M * nb;
    const dim3 g((unsigned)((n + 255) / 256)), b(256);
    if (dt == DT_Q4_0)
        hipLaunchKernelGGL(to_tiled_kernel<DT_Q4_0>, g, b, 0, st, static_cast<const uint8_t *>(aos), q, sc, M, nb);
    else
        hipLaunchKernelGGL(to_tiled_kernel<DT_Q8_0>, g, b, 0, st, static_cast<const uint8_t *>(aos), q, sc, M, nb);
    return hip_ok(hipGetLastError(), "to_tiled launch") ? 0 : -1;
}

int launch_tiled_unpack(int dt, const void *w, int M, int K, int8_t *ints, float *deq, hipStream_t st) {
    const int nb = K / kBlock;
    const uint8_t *q = static_cast<const uint8_t *>(w);
    const float *sc = reinterpret_cast<const float *>(q + q_tiled_scales_offset(dt, M, K));
    const long n = (long)M * nb;
    const dim3 g((unsigned)((n + 255) / 256)), b(256);
    if (dt == DT_Q4_0)
        hipLaunchKernelGGL(tiled_unpack_kernel<DT_Q4_0>, g, b, 0, st, q, sc, M, nb, ints, deq);
    else
        hipLaunchKernelGGL(tiled_unpack_kernel<DT_Q8_0>, g, b, 0, st, q, sc, M, nb, ints, deq);
    return hip_ok(hipGetLastError(), "tiled unpack launch") ? 0 : -1;
}

size_t tiled_softmax_scratch_bytes(int M) {
    return sizeof(SoftPart) * (size_t)std::max(tiled_blocks(DT_Q4_0, M), tiled_blocks(DT_Q8_0, M));
}

int launch_gemv_tiled_softmax(int dt, const void *w, int M, int K, const float *x, float *logits, float *probs,
                              int *argmax, void *scratch, hipStream_t st) {
    SoftPart *part = static_cast<SoftPart *>(scratch);
    if (launch_tiled(dt, w, M, K, x, logits, part, st) != 0) return -1;
    // 4 * kFinishVec * 256 logits per block (one pass of kFinishVec float4 per thread), so the
    // 262144-entry vocabulary spreads over 256 blocks; chunks are multiples of 4 floats so the
    // float4 accesses stay aligned
    constexpr int per_block = 4 * kFinishVec * 256;
    const int blocks = probs ? std::max(1, (M + per_block - 1) / per_block) : 1;
    const int chunk = ((M + blocks - 1) / blocks + 3) & ~3;
    const int aligned = ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(probs)) & 15u) == 0;
    hipLaunchKernelGGL(softmax_finish_parts, dim3(blocks), dim3(256), 0, st, logits, M, chunk, part,
                       (int)tiled_blocks(dt, M), probs, argmax, aligned);
    return hip_ok(hipGetLastError(), "softmax_finish_parts launch") ? 0 : -1;
}

int launch_gemv_tiled(int dt, const void *w, int M, int K, const float *x, float *y, hipStream_t st) {
    return launch_tiled(dt, w, M, K, x, y, nullptr, st);
}

size_t tiled_greedy_key_slots(int M) { return std::max(tiled_blocks(DT_Q4_0, M), tiled_blocks(DT_Q8_0, M)); }

int launch_gemv_tiled_greedy_step(int dt, const void *w, int M, int K, const float *x, float *logits,
                                  const GreedyStep &gs, hipStream_t st) {
    if (!gs.keys || !gs.count || !gs.tok || !gs.pos || !gs.step || !gs.log) {
        set_error("greedy LM head: missing state");
        return -1;
    }
    return launch_tiled(dt, w, M, K, x, logits, nullptr, st, &gs);
}

int launch_gemv_tiled_greedy_slots(int dt, const void *w, int M, int K, const float *x, float *logits,
                                   TokenSlots *slots, const int *done, hipStream_t st) {
    if (!slots || M > kSlotMaxVocab) {
        set_error("greedy LM head: token slots need a vocabulary of at most %d", kSlotMaxVocab);
        return -1;
    }
    GreedyStep gs;
    gs.slots = slots;
    gs.done = const_cast<int *>(done);
    return launch_tiled(dt, w, M, K, x, logits, nullptr, st, &gs);
}

namespace {
__global__ void token_slots_settle_kernel(TokenSlots *ts, int vocab, int *log, int *done, StopSet stop, int *err) {
    if (threadIdx.x != 0 || (done && *done)) return;
    const uint32_t a = ts->a;
    if (a == 0) return;
    unsigned long long k = 0;
    for (int i = 0; i < kSlotCount; ++i) k = ts->key[i] > k ? ts->key[i] : k;
    int tok = 0;
    if (!slot_token(k, a, vocab, tok)) {
        atomicAdd(err, 1);
        return;
    }
    log[ts->logbase + (int)a - 1] = tok;
    if (done && stop.has(tok)) *done = 1;   // inference.c:298-301
    ts->tok0 = tok;
    ts->pos0 += (int)a;
    ts->seq0 += a;
    ts->logbase += (int)a;
    ts->a = 0;
    ts->b = 0;
    for (int i = 0; i < kSlotCount; ++i) ts->key[i] = 0;
}
}  // namespace

int launch_token_slots_settle(TokenSlots *slots, int vocab, int *log, int *done, const StopSet &stop, int *err,
                              hipStream_t st) {
    hipLaunchKernelGGL(token_slots_settle_kernel, dim3(1), dim3(64), 0, st, slots, vocab, log, done, stop, err);
    return hip_ok(hipGetLastError(), "token slots settle launch") ? 0 : -1;
}

}  // namespace sapphire
