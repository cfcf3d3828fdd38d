// decode_device.h - device helpers shared by the decode kernels (decode.hip) and the
// persistent decode kernel (decode_persist.hip). Not installed.
#pragma once

#include <cmath>

#include "decode_kernels.h"
#include "devmath.h"
#include "lanes.h"
#include "qdot.h"

namespace sapphire {
namespace {

using namespace devmath;
using namespace qdot;
using namespace lanes;

constexpr int kWave = 64;
constexpr int kThreads = 256;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Sum over the 64 lanes of a wave by an xor butterfly (the multi-launch GEMV's row sums).
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// One hd-long fp32 row (hd = 64 DPL) from global memory into LDS by DMA (no VGPRs): the
// wave's lanes load 16 B each (DPL 4) or 4 B per 64-dim chunk; the data lands in natural
// dim order at lds_row, which must be the same for the whole wave. Completion is counted by
// vmcnt like any other load.
template <int DPL>
__device__ __forceinline__ void row_to_lds(const float *src_row, float *lds_row) {
    const int lane = threadIdx.x & (kWave - 1);
    if constexpr (DPL == 4) {
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src_row + lane * 4),
                                         (__attribute__((address_space(3))) void *)lds_row, 16, 0, 0);
    } else {
#pragma unroll
        for (int c = 0; c < DPL; ++c)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src_row + c * kWave + lane),
                                             (__attribute__((address_space(3))) void *)(lds_row + c * kWave), 4, 0, 0);
    }
}

// Sum of squares of v[0..n) (LDS) in the reference order of sum_sq_avx2
// (normalization.c:12-32): eight sequential FMA lanes over elements l, l+8, ..., then
// ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7)) and a sequential fused tail. Threads 0..7 run the
// lanes, loading eight elements ahead of their FMA chain; the result is returned to every
// thread (the call synchronises the workgroup).
__device__ __forceinline__ float lds_sum_sq(const float *v, int n, float *sh) {
    const int t = threadIdx.x;
    if (t < 8) {
        float s = 0.f;
        const int full = n & ~7;
        int i = t;
        for (; i + 56 < full; i += 64) {
            float w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = v[i + 8 * u];
#pragma unroll
            for (int u = 0; u < 8; ++u) s = __builtin_fmaf(w[u], w[u], s);
        }
        for (; i < full; i += 8) s = __builtin_fmaf(v[i], v[i], s);
        sh[t] = s;
    }
    __syncthreads();
    if (t == 0) {
        const float a0 = sh[0] + sh[4], a1 = sh[1] + sh[5], a2 = sh[2] + sh[6], a3 = sh[3] + sh[7];
        float s = (a0 + a1) + (a2 + a3);
        for (int i = n & ~7; i < n; ++i) s = __builtin_fmaf(v[i], v[i], s);
        sh[8] = s;
    }
    __syncthreads();
    return sh[8];
}

template <int DT> struct QB;
template <> struct QB<DT_Q4_0> { static constexpr int BYTES = 16, WORDS = 4; };
template <> struct QB<DT_Q8_0> { static constexpr int BYTES = 32, WORDS = 8; };

// The quants and scale of this lane's block of `row` (zeros for a lane off the matrix),
// loaded before the input vector is staged so their latency overlaps the prologue.
template <int DT>
struct LaneBlock {
    uint32_t q[QB<DT>::WORDS];
    float s;
};

// p as a pointer into device memory: loads and stores through it compile to global_*
// instructions. A pointer the compiler cannot trace to a kernel argument (one read from LDS,
// as the persistent step's layer descriptors are) is otherwise generic, and flat instructions
// count in the LDS counter as well, so every later wait for an LDS result or a barrier would
// also wait for them to come back from memory.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *as_global(const T *p) {
    return (const __attribute__((address_space(1))) T *)p;
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T *as_global(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}

template <int DT>
__device__ __forceinline__ void load_lane_block(const QMat &w, int row, int blk, int nb, bool on, LaneBlock<DT> &b) {
    const bool ok = on && row < w.M;
    const size_t bi = ok ? (size_t)row * nb + blk : 0;
    const auto qp = as_global(reinterpret_cast<const u32x4 *>(w.q + bi * QB<DT>::BYTES));
#pragma unroll
    for (int i = 0; i < QB<DT>::WORDS / 4; ++i) {
        const u32x4 t = qp[i];
        b.q[4 * i + 0] = t.x; b.q[4 * i + 1] = t.y; b.q[4 * i + 2] = t.z; b.q[4 * i + 3] = t.w;
    }
    // loaded in every lane (block 0 stands in when !ok) and selected afterwards: a load that
    // only some lanes issue into a register the others then write makes the compiler wait
    // for every load in flight
    const float sv = as_global(w.s)[bi];
    b.s = ok ? sv : 0.f;
}

template <int DT>
__device__ __forceinline__ float block_value(const LaneBlock<DT> &b, const float (&xv)[32], float xsum) {
    if constexpr (DT == DT_Q4_0) return b.s * dot_q4(b.q, xv, xsum);
    else return b.s * dot_q8(b.q, xv, xsum);
}

// Sums of squares of nv consecutive vectors of length hd in LDS, each in the reference
// order of sum_sq_avx2 (eight sequential lanes, then the fixed tree and a sequential
// tail); eight threads per vector, loading eight elements ahead. Result in ss[v].
__device__ __forceinline__ void vectors_sum_sq(const float *base, int nv, int hd, float *part8, float *ss) {
    const int t = threadIdx.x;
    if (t < 8 * nv) {
        const int v = t / 8, l = t - 8 * v;
        const float *p = base + (size_t)v * hd;
        const int full = hd & ~7;
        float s = 0.f;
        int i = l;
        for (; i + 56 < full; i += 64) {
            float w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = p[i + 8 * u];
#pragma unroll
            for (int u = 0; u < 8; ++u) s = __builtin_fmaf(w[u], w[u], s);
        }
        for (; i < full; i += 8) s = __builtin_fmaf(p[i], p[i], s);
        part8[t] = s;
    }
    __syncthreads();
    if (t < nv) {
        const float *s8 = part8 + 8 * t;
        const float a0 = s8[0] + s8[4], a1 = s8[1] + s8[5], a2 = s8[2] + s8[6], a3 = s8[3] + s8[7];
        float s = (a0 + a1) + (a2 + a3);
        const float *p = base + (size_t)t * hd;
        for (int i = hd & ~7; i < hd; ++i) s = __builtin_fmaf(p[i], p[i], s);
        ss[t] = s;
    }
    __syncthreads();
}

// dst[v] = rope(rmsnorm_delta(src[v], g)) for nv head vectors held in LDS (attention.c:
// 221-309; rope_apply_fast rope.c:99-117 with the fused forms of the reference build).
__device__ __forceinline__ void norm_rope_heads(const float *src, int nv, int hd, const float *__restrict__ g,
                                                const float *__restrict__ cs, const float *__restrict__ sn, float eps,
                                                float *dst, float *part8, float *ss) {
    vectors_sum_sq(src, nv, hd, part8, ss);
    if (threadIdx.x < nv) ss[threadIdx.x] = rms_inv_of(ss[threadIdx.x], hd, eps);
    __syncthreads();
    const int half = hd / 2;
    for (int idx = threadIdx.x; idx < nv * half; idx += blockDim.x) {
        const int v = idx / half, i = idx - v * half;
        const float r = ss[v];
        const float *p = src + (size_t)v * hd;
        const float x0 = __fmul_rn(__fmul_rn(p[i], r), __fadd_rn(1.0f, g[i]));
        const float x1 = __fmul_rn(__fmul_rn(p[i + half], r), __fadd_rn(1.0f, g[i + half]));
        const float c = cs[i], s = sn[i];
        dst[v * hd + i] = __builtin_fmaf(x0, c, -__fmul_rn(x1, s));
        dst[v * hd + i + half] = __builtin_fmaf(x1, c, __fmul_rn(x0, s));
    }
    __syncthreads();
}

// The token is device data (the previous step's argmax): it is clamped into the vocabulary
// so that no value can address outside the table.
__device__ __forceinline__ size_t embed_row(int tok, int vocab, int hidden) {
    return (size_t)(tok >= 0 && tok < vocab ? tok : 0) * hidden;
}

}  // namespace
}  // namespace sapphire
