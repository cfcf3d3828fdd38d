// sample.hip - the next token as perform_inference draws it (inference.c:262-266, 297), for a
// batch of logit rows: temperature <= 0 is sample_greedy (utils.c:145-156); otherwise the
// logits are scaled by 1/T (vec_scale, utils.c:87-92) and sample_temperature (utils.c:158-180)
// draws: max seeded with logits[0] (strict >), w_i = expf((l_i - max) / T) in place, sum the
// w_i left to right in float, then walk cumsum += w_i / sum (float) and return the first i with
// r <= cumsum, n - 1 if there is none. r is the caller's draw in place of rand() / RAND_MAX.
//
// The token is the reference's bit for bit, so both float chains (the sum, and the running sum
// the draw is compared with) are reproduced exactly, in parallel:
// * while a chain v <- fl(v + x) (x >= 0) stays inside one binade [2^e, 2^(e+1)), whose
//   spacing is u, it is integer arithmetic on M = v / u: fl(v + x) = (M + k) u with k = x / u
//   rounded to nearest, and on a tie (x / u = f + 1/2) the even one of M + f and M + f + 1.
//   Each element is the map M -> M + d[M & 1] (k and the tie read from the element's float
//   bits in integer arithmetic); maps compose (associatively), so a sub-chunk of kSub elements
//   is one pair (d0, d1) for a given binade. The binades a chain can occupy at a sub-chunk's
//   start are fixed to at most two by the exact prefix sum and the error bound of recursive
//   summation (|fl-sum - sum| <= n 2^-24 sum for nonnegative terms);
// * one wave per row walks the sub-chunks with these maps, 64 at a time, and in a sub-chunk
//   where the binade changes or the draw is reached scans its lanes' maps (16 elements each)
//   to find the lane where that happens; that lane adds its elements with real float adds
//   (the reference's own operation).
// The weights come from libm_expf, glibc's expf bit for bit.
#include "internal.h"
#include "libm_expf.h"

#include <cmath>

namespace sapphire {
namespace {

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kPer = 4;                         // elements per thread in the grid kernels
constexpr int kSub = kThreads * kPer;           // elements per sub-chunk (one grid workgroup)
constexpr int kRun = kSub / kWave;              // consecutive elements per lane in the walk
constexpr int kMaxSubs = 2048;                  // n <= 2^21 keeps the error bound below 1/4
constexpr int kCap = 1 << 28;                   // saturation of map increments
constexpr int kZero = -1000, kSub_ = -127;      // binade ids of 0 and of the subnormals

struct SubStat {         // per row and sub-chunk
    float max;           // largest non-NaN scaled logit (+-inf included)
    int arg;             // its first index, -1 if the sub-chunk is all NaN
    int nan;             // whether the sub-chunk holds a NaN
    int nan0;            // sub-chunk 0 only: whether the row's first scaled logit is NaN
    double wsum;         // sum of the sub-chunk's weights (exact enough for the bounds)
};
struct SubMaps {         // per row and sub-chunk: its map for the chunk's (up to) two binades
    int reg[2];
    int d[2][2];
};
struct RowInfo {
    float m;             // the reference's max (NaN when logits[0] is NaN)
    int bad;             // a NaN weight (or an all -inf row): the token is n - 1
    float sum;           // the float sum of the weights
    int pad;
};

struct Reg {
    int id, uexp, mlim;  // binade id, exponent of its spacing, 2^24 (2^23 subnormal, 1 for zero)
};

__device__ __forceinline__ Reg reg_zero() { return {kZero, 0, 1}; }
__device__ __forceinline__ Reg reg_id(int id) {
    if (id == kZero) return reg_zero();
    if (id == kSub_) return {kSub_, -149, 1 << 23};
    return {id, id - 23, 1 << 24};
}
__device__ __forceinline__ Reg reg_of(float v) {
    if (v == 0.0f) return reg_zero();
    if (v < 0x1p-126f) return reg_id(kSub_);
    return reg_id(ilogbf(v));
}
__device__ __forceinline__ Reg reg_of_bound(double x) {
    if (!(x > 0.0)) return reg_zero();
    if (x < 0x1p-126) return reg_id(kSub_);
    return reg_id(min(ilogb(x), 127));
}
__device__ __forceinline__ int m_of(float v, const Reg &R) {
    return R.id == kZero ? 0 : (int)ldexp((double)v, -R.uexp);
}
__device__ __forceinline__ float val_of(int M, const Reg &R) {   // exact for M < R.mlim
    return R.id == kZero ? 0.0f : (float)ldexp((double)M, R.uexp);
}

struct Map {
    int d0, d1;
};
__device__ __forceinline__ Map map_id() { return {0, 0}; }
// a then b
__device__ __forceinline__ Map compose(Map a, Map b) {
    const int e = a.d0 + ((a.d0 & 1) ? b.d1 : b.d0);
    const int o = a.d1 + ((a.d1 & 1) ? b.d0 : b.d1);
    return {min(e, kCap), min(o, kCap)};
}
__device__ __forceinline__ int apply(int M, Map m) { return M + min((M & 1) ? m.d1 : m.d0, kCap); }

// The map of element x (bits xb of a float >= +0) in binade R: k = x / u rounded to nearest,
// a tie to the even sum. x = mx 2^e2, so x / u = mx 2^(e2 - uexp) in integers.
__device__ __forceinline__ Map elem_map(uint32_t xb, const Reg &R) {
    if (R.id == kZero) return xb ? Map{kCap, kCap} : map_id();
    const uint32_t ex = xb >> 23;
    const uint32_t mx = ex ? (xb & 0x7fffffu) | 0x800000u : xb;
    const int sh = (ex ? (int)ex - 150 : -149) - R.uexp;
    if (sh >= 0) {
        const uint64_t k = (uint64_t)mx << min(sh, 40);
        if (k >= (1u << 25)) return {kCap, kCap};
        return {(int)k, (int)k};
    }
    const int s = -sh;
    if (s >= 26) return map_id();              // x / u < 2^24 2^-26
    const uint32_t f = mx >> s, rem = mx & ((1u << s) - 1u), half = 1u << (s - 1);
    const int fi = (int)f;
    if (rem > half) return {fi + 1, fi + 1};
    if (rem < half) return {fi, fi};
    return {fi + (fi & 1), fi + ((fi & 1) ^ 1)};
}

__device__ __forceinline__ float scaled(float l, float inv_t, int scale) { return scale ? __fmul_rn(l, inv_t) : l; }

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return bi < 0 || (i >= 0 && (v > bv || (v == bv && i < bi)));
}

// grid (sub-chunks, batch): SubStat of each sub-chunk of the (scaled) logits
__global__ __launch_bounds__(kThreads) void smp_stats(const float *__restrict__ logits, int n, size_t ld,
                                                      float inv_t, int scale, SubStat *__restrict__ stats) {
    __shared__ float sv[kThreads / kWave];
    __shared__ int si[kThreads / kWave], sn[kThreads / kWave];
    const int nsub = gridDim.x, q = blockIdx.x, b = blockIdx.y;
    const float *x = logits + (size_t)b * ld;
    const int i0 = q * kSub + threadIdx.x * kPer;
    float bv = -INFINITY;
    int bi = -1, nan = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = i0 + k;
        if (i < n) {
            const float s = scaled(x[i], inv_t, scale);
            if (s != s) nan = 1;
            else if (bi < 0 || s > bv) {
                bv = s;
                bi = i;
            }
        }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
        nan |= __shfl_xor(nan, off, kWave);
    }
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) {
        sv[wid] = bv;
        si[wid] = bi;
        sn[wid] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / kWave; ++w) {
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
            nan |= sn[w];
        }
        SubStat st;
        st.max = bv;
        st.arg = bi;
        st.nan = nan;
        st.nan0 = q == 0 ? (int)(scaled(x[0], inv_t, scale) != scaled(x[0], inv_t, scale)) : 0;
        st.wsum = 0.0;
        stats[(size_t)b * nsub + q] = st;
    }
}

// The reference's max and the row's status from the sub-chunk statistics (all threads).
__device__ void row_max(const SubStat *__restrict__ st, int nsub, float *m_out, int *bad_out) {
    __shared__ float sm[kThreads / kWave];
    __shared__ int sb[kThreads / kWave];
    float m = -INFINITY;
    int nan = 0;
    for (int q = threadIdx.x; q < nsub; q += blockDim.x) {
        m = fmaxf(m, st[q].max);
        nan |= st[q].nan;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off, kWave));
        nan |= __shfl_xor(nan, off, kWave);
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sm[threadIdx.x / kWave] = m;
        sb[threadIdx.x / kWave] = nan;
    }
    __syncthreads();
    m = sm[0];
    nan = sb[0];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) {
        m = fmaxf(m, sm[w]);
        nan |= sb[w];
    }
    __syncthreads();
    if (st[0].nan0) m = __int_as_float(0x7fc00000);
    *m_out = m;
    // NaN anywhere, or max = +inf (inf - inf) or -inf (every weight NaN): the sum is NaN
    *bad_out = nan || m != m || m == INFINITY || m == -INFINITY;
}

// grid (sub-chunks, batch): w = expf((s - m) / T) written to w (may alias the logits), the
// sub-chunk's weight sum into its SubStat, the row's RowInfo (sub-chunk 0)
__global__ __launch_bounds__(kThreads) void smp_weights(const float *logits, int n, size_t ld, float inv_t,
                                                        int scale, float t, float *w, size_t ldw,
                                                        SubStat *__restrict__ stats, RowInfo *__restrict__ rows) {
    __shared__ double sd[kThreads / kWave];
    const int nsub = gridDim.x, q = blockIdx.x, b = blockIdx.y;
    SubStat *st = stats + (size_t)b * nsub;
    float m;
    int bad;
    row_max(st, nsub, &m, &bad);
    const float *x = logits + (size_t)b * ld;
    float *wr = w + (size_t)b * ldw;
    const int i0 = q * kSub + threadIdx.x * kPer;
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = i0 + k;
        if (i < n) {
            const float v = libm_expf(__fdiv_rn(__fsub_rn(scaled(x[i], inv_t, scale), m), t));
            wr[i] = v;
            sum += (double)v;
        }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) sd[threadIdx.x / kWave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kThreads / kWave; ++k) sum += sd[k];
        st[q].wsum = sum;
        if (q == 0) {
            RowInfo ri;
            ri.m = m;
            ri.bad = bad;
            ri.sum = 0.0f;
            ri.pad = 0;
            rows[b] = ri;
        }
    }
}

// Element x of a chain, as float bits: the weight (chain 0) or the weight over the float sum
// (chain 1).
__device__ __forceinline__ uint32_t chain_elem(float wv, int chain, float sum) {
    return __float_as_uint(chain ? __fdiv_rn(wv, sum) : wv);
}

// Ordered composition of the block's per-thread maps; the result in thread 0.
__device__ Map block_compose(Map m, Map *sh) {
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        Map o;
        o.d0 = __shfl_down(m.d0, off, kWave);
        o.d1 = __shfl_down(m.d1, off, kWave);
        if ((lane & (2 * off - 1)) == 0 && lane + off < kWave) m = compose(m, o);
    }
    if (lane == 0) sh[wid] = m;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < kThreads / kWave; ++k) m = compose(m, sh[k]);
    return m;
}

// grid (sub-chunks, batch): each sub-chunk's map (chain 0: the weight sum; chain 1: the
// running sum of the weights over the float sum) for the binades the chain can be in at the
// sub-chunk's start.
__global__ __launch_bounds__(kThreads) void smp_maps(const float *__restrict__ w, int n, size_t ldw, int chain,
                                                     const SubStat *__restrict__ stats,
                                                     const RowInfo *__restrict__ rows, SubMaps *__restrict__ maps) {
    __shared__ double sd[kThreads / kWave];
    __shared__ Map sm[2][kThreads / kWave];
    const int nsub = gridDim.x, q = blockIdx.x, b = blockIdx.y;
    const RowInfo ri = rows[b];
    if (ri.bad) return;
    const SubStat *st = stats + (size_t)b * nsub;
    // the exact sum of the weights before this sub-chunk
    double p = 0.0;
    for (int k = threadIdx.x; k < q; k += kThreads) p += st[k].wsum;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) p += __shfl_xor(p, off, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) sd[threadIdx.x / kWave] = p;
    __syncthreads();
    p = sd[0];
    for (int k = 1; k < kThreads / kWave; ++k) p += sd[k];
    // recursive summation of n nonnegative floats: relative error below (n + 2) 2^-24 (with
    // margin); the quotients w / sum add 2^-24 relative each, and subnormal ones 2^-150
    double rel = 2.0 * (n + 2) * 0x1p-24, abs_err = 0.0;
    if (chain) {
        p /= (double)ri.sum;
        rel += 0x1p-22;
        abs_err = (double)n * 0x1p-149;
    }
    const Reg lo = reg_of_bound(p * (1.0 - rel) - abs_err), hi = reg_of_bound(p * (1.0 + rel) + abs_err);
    const float *wr = w + (size_t)b * ldw;
    const int i0 = q * kSub + threadIdx.x * kPer;
    Map m0 = map_id(), m1 = map_id();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = i0 + k;
        if (i < n) {
            const uint32_t x = chain_elem(wr[i], chain, ri.sum);
            m0 = compose(m0, elem_map(x, lo));
            m1 = compose(m1, elem_map(x, hi));
        }
    }
    m0 = block_compose(m0, sm[0]);
    m1 = block_compose(m1, sm[1]);
    if (threadIdx.x == 0) {
        SubMaps cm;
        cm.reg[0] = lo.id;
        cm.d[0][0] = m0.d0;
        cm.d[0][1] = m0.d1;
        cm.reg[1] = hi.id;
        cm.d[1][0] = m1.d0;
        cm.d[1][1] = m1.d1;
        maps[(size_t)b * nsub + q] = cm;
    }
}

// One DPP move of both halves of a map; lanes without a source (and rows outside row_mask)
// read 0, the identity map.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ Map dpp_map(Map m) {
    return {__builtin_amdgcn_update_dpp(0, m.d0, CTRL, ROW_MASK, 0xf, true),
            __builtin_amdgcn_update_dpp(0, m.d1, CTRL, ROW_MASK, 0xf, true)};
}

// Inclusive scan of the wave's maps in lane order (lane l gets m_0 ... m_l composed): shifts
// by 1, 2, 4, 8 within each 16-lane row, then the last lane of row 0 (and of row 2) into the
// next row, then lane 31 into rows 2 and 3.
__device__ __forceinline__ Map wave_scan(Map m) {
    m = compose(dpp_map<0x111, 0xf>(m), m);   // row_shr:1
    m = compose(dpp_map<0x112, 0xf>(m), m);   // row_shr:2
    m = compose(dpp_map<0x114, 0xf>(m), m);   // row_shr:4
    m = compose(dpp_map<0x118, 0xf>(m), m);   // row_shr:8
    m = compose(dpp_map<0x142, 0xa>(m), m);   // row_bcast:15 into rows 1 and 3
    m = compose(dpp_map<0x143, 0xc>(m), m);   // row_bcast:31 into rows 2 and 3
    return m;
}

__device__ __forceinline__ int first_lane(unsigned long long bal) { return __builtin_ctzll(bal); }

// grid (batch), one wave per row: the chain walk. chain 0 stores the float sum of the weights
// in RowInfo; chain 1 finds the first index whose running sum reaches the row's draw r
// (draws[step * batch + b], step = *d_step or 0) and writes the token (n - 1 if none, or for
// a bad row). The wave takes 64 sub-chunks at a time, one per lane: a scan of their maps in
// the chain's binade finds the first sub-chunk in which the binade changes or r is reached
// (or whose binades were not prepared). In that sub-chunk each lane holds 16 consecutive
// elements, a scan of the lanes' maps finds the first lane where the same happens, and that
// lane adds its elements with real float adds; the scan resumes after it.
__global__ __launch_bounds__(kWave) void smp_walk(const float *__restrict__ w, int n, size_t ldw, int chain,
                                                  int nsub, const SubMaps *__restrict__ maps,
                                                  RowInfo *__restrict__ rows, const float *__restrict__ draws,
                                                  const int *__restrict__ d_step, int batch,
                                                  int *__restrict__ tokens) {
    __shared__ SubMaps cm[kMaxSubs];
    const int b = blockIdx.x, lane = threadIdx.x;
    const RowInfo ri = rows[b];
    if (ri.bad) {
        if (chain && lane == 0) tokens[b] = n - 1;
        return;
    }
    const float r = chain ? draws[(size_t)(d_step ? *d_step : 0) * batch + b] : INFINITY;
    const float *wr = w + (size_t)b * ldw;
    for (int k = lane; k < nsub; k += kWave) cm[k] = maps[(size_t)b * nsub + k];
    __syncthreads();
    float v = 0.0f;
    int q = 0, found = -1;
    while (q < nsub && found < 0) {
        // sub-chunks q .. q + 63 in the current binade
        {
            const Reg R = reg_of(v);
            const int M0 = m_of(v, R), qi = q + lane;
            Map m = map_id();
            if (qi < nsub) {
                const SubMaps &c = cm[qi];
                const int k = c.reg[0] == R.id ? 0 : (c.reg[1] == R.id ? 1 : -1);
                m = k < 0 ? Map{kCap, kCap} : Map{c.d[k][0], c.d[k][1]};
            }
            const int Me = apply(M0, wave_scan(m));
            const bool stop = qi < nsub && (Me >= R.mlim || r <= val_of(Me, R));
            const unsigned long long bal = __ballot(stop);
            if (bal == 0) {
                const int last = min(kWave, nsub - q) - 1;
                v = val_of(__shfl(Me, last, kWave), R);
                q += kWave;
                continue;
            }
            const int s = first_lane(bal);
            const int Mprev = __shfl(Me, s > 0 ? s - 1 : 0, kWave);
            if (s > 0) v = val_of(Mprev, R);
            q += s;
        }
        // sub-chunk q element by element: lane l holds elements base + 16 l .. + 15
        const int base = q * kSub, e0 = base + lane * kRun;
        uint32_t x[kRun];
#pragma unroll
        for (int j = 0; j < kRun; ++j) {
            const int i = e0 + j;
            x[j] = i < n ? chain_elem(wr[i], chain, ri.sum) : 0u;
        }
        const int nval = max(0, min(kRun, n - e0));   // this lane's elements
        int from = 0;                                  // the first lane not yet added
        while (from < kWave) {
            const Reg R = reg_of(v);
            const int M0 = m_of(v, R);
            Map m = map_id();
            if (lane >= from)
#pragma unroll
                for (int j = 0; j < kRun; ++j)
                    if (j < nval) m = compose(m, elem_map(x[j], R));
            const int Me = apply(M0, wave_scan(m));
            const bool stop = lane >= from && nval > 0 && (Me >= R.mlim || r <= val_of(Me, R));
            const unsigned long long bal = __ballot(stop);
            if (bal == 0) {                            // the rest of the sub-chunk stays in the binade
                const unsigned long long has = __ballot(nval > 0);
                const int last = has ? 63 - __builtin_clzll(has) : -1;
                if (last >= from) v = val_of(__shfl(Me, last, kWave), R);
                break;
            }
            const int s = first_lane(bal);
            const int Mprev = __shfl(Me, s > 0 ? s - 1 : 0, kWave);
            float vv = s > from ? val_of(Mprev, R) : v;
            int fnd = -1;
            if (lane == s) {
#pragma unroll
                for (int j = 0; j < kRun; ++j)
                    if (j < nval && fnd < 0) {
                        vv = __fadd_rn(vv, __uint_as_float(x[j]));
                        if (r <= vv) fnd = e0 + j;
                    }
            }
            v = __shfl(vv, s, kWave);
            fnd = __shfl(fnd, s, kWave);
            if (fnd >= 0) {
                found = fnd;
                break;
            }
            from = s + 1;
        }
        ++q;
    }
    if (lane == 0) {
        if (chain) tokens[b] = found >= 0 ? found : n - 1;
        else rows[b].sum = v;
    }
}

// grid (batch), one wave: sample_greedy from the sub-chunk statistics: the first maximum, 0
// when logits[0] is NaN
__global__ __launch_bounds__(kWave) void smp_greedy(const SubStat *__restrict__ stats, int nsub,
                                                    int *__restrict__ tokens) {
    const SubStat *st = stats + (size_t)blockIdx.x * nsub;
    float bv = -INFINITY;
    int bi = -1;
    for (int q = threadIdx.x; q < nsub; q += kWave)
        if (better(st[q].max, st[q].arg, bv, bi)) {
            bv = st[q].max;
            bi = st[q].arg;
        }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (threadIdx.x == 0) tokens[blockIdx.x] = st[0].nan0 || bi < 0 ? 0 : bi;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int subs_of(int n) { return (n + kSub - 1) / kSub; }

}  // namespace

size_t sample_workspace_bytes(int n, int batch) {
    const size_t cells = (size_t)subs_of(n) * batch;
    return align256(cells * sizeof(SubStat)) + 2 * align256(cells * sizeof(SubMaps)) +
           align256((size_t)batch * sizeof(RowInfo));
}

bool sample_supported(int n, int batch) { return n > 0 && batch > 0 && subs_of(n) <= kMaxSubs; }

int launch_sample(const float *logits, int n, int batch, size_t ld, float temperature, float *w, size_t ldw,
                  const float *draws, const int *d_step, int *tokens, void *ws, hipStream_t s) {
    if (!sample_supported(n, batch)) {
        set_error("sampling supports 1..%d logits per row", kMaxSubs * kSub);
        return -1;
    }
    const int nsub = subs_of(n);
    const size_t cells = (size_t)nsub * batch;
    char *p = static_cast<char *>(ws);
    auto *stats = reinterpret_cast<SubStat *>(p);
    p += align256(cells * sizeof(SubStat));
    auto *maps0 = reinterpret_cast<SubMaps *>(p);
    p += align256(cells * sizeof(SubMaps));
    auto *maps1 = reinterpret_cast<SubMaps *>(p);
    p += align256(cells * sizeof(SubMaps));
    auto *rows = reinterpret_cast<RowInfo *>(p);
    const dim3 grid(nsub, batch);
    if (temperature <= 0.0f) {
        hipLaunchKernelGGL(smp_stats, grid, dim3(kThreads), 0, s, logits, n, ld, 1.0f, 0, stats);
        if (!hip_ok(hipGetLastError(), "sample stats launch")) return -1;
        hipLaunchKernelGGL(smp_greedy, dim3(batch), dim3(kWave), 0, s, stats, nsub, tokens);
        return hip_ok(hipGetLastError(), "sample greedy launch") ? 0 : -1;
    }
    // vec_scale skips s == 1.0f; a product with 1.0f changes no value either way. A NaN
    // temperature (not scaled there) makes every weight NaN either way: token n - 1.
    const float inv_t = 1.0f / temperature;
    const int scale = inv_t != 1.0f;
    hipLaunchKernelGGL(smp_stats, grid, dim3(kThreads), 0, s, logits, n, ld, inv_t, scale, stats);
    if (!hip_ok(hipGetLastError(), "sample stats launch")) return -1;
    hipLaunchKernelGGL(smp_weights, grid, dim3(kThreads), 0, s, logits, n, ld, inv_t, scale, temperature, w, ldw,
                       stats, rows);
    if (!hip_ok(hipGetLastError(), "sample weights launch")) return -1;
    hipLaunchKernelGGL(smp_maps, grid, dim3(kThreads), 0, s, w, n, ldw, 0, stats, rows, maps0);
    if (!hip_ok(hipGetLastError(), "sample maps launch")) return -1;
    hipLaunchKernelGGL(smp_walk, dim3(batch), dim3(kWave), 0, s, w, n, ldw, 0, nsub, maps0, rows, draws, d_step,
                       batch, tokens);
    if (!hip_ok(hipGetLastError(), "sample sum walk launch")) return -1;
    hipLaunchKernelGGL(smp_maps, grid, dim3(kThreads), 0, s, w, n, ldw, 1, stats, rows, maps1);
    if (!hip_ok(hipGetLastError(), "sample maps launch")) return -1;
    hipLaunchKernelGGL(smp_walk, dim3(batch), dim3(kWave), 0, s, w, n, ldw, 1, nsub, maps1, rows, draws, d_step,
                       batch, tokens);
    return hip_ok(hipGetLastError(), "sample draw walk launch") ? 0 : -1;
}

}  // namespace sapphire
