// gemv.hip - Q4_0 / Q8_0 / F32 / BF16 GEMV kernels for gfx950 (wave64).
//
// Semantics: y[r] = sum_k W[r,k] * x[k] with W in the reference block formats
// (include/kernels.h:29-38): Q4_0 element 2j = (q[j] & 0xF) - 8, element 2j+1 =
// (q[j] >> 4) - 8 (q4_0_avx.c:61-66); Q8_0 element e = (int8)q[e] (q8_0_avx.c:45-56);
// each times the block's fp32 scale. The reference accumulates fl(w*scale)*x in 32 or
// 64 fp32 FMA lanes (q4_0_avx.c:102-123, q8_0_avx.c:16-75); here each block's integer
// dot product sum(int*x) is accumulated first and multiplied by the block scale once,
// which differs from the reference only in fp32 rounding order.
//
// Kernel shapes
//  * gemv_q_cols  (nb = K/32 <= 64): lane l of a wave owns column block (l % nb) of
//    row (l / nb) of each wave-step; floor(64/nb) rows per step (3 for K=640, 2 for
//    K=1024, 1 for K=2048). The lane's 32 x values stay in VGPRs for the whole kernel,
//    so per block a lane issues one 16-B (Q4_0) or two 16-B (Q8_0) loads of quants and
//    one 4-B scale load; consecutive lanes read consecutive 16-B chunks. S wave-steps are
//    loaded before any is consumed (S*(1..2) dwordx4 in flight per lane). Per-row sums of
//    the nb block partials go through a per-wave LDS transpose.
//  * gemv_q_rows  (any K): one row per wave-step, lanes stride over the row's blocks,
//    x read through L1, wave-wide reduction.
//  * gemv_f16      (F32/BF16 rows, 16-byte aligned rows): 16 lanes per row, 4 rows per
//    wave-step; lane q reads the 16-byte chunks q, q+16, ... of its row (4 fp32 or 8 bf16
//    each), U chunks in flight, x from LDS; row sums by DPP.
//  * gemv_f       (F32/BF16, any K or alignment): lanes stride over the elements of one
//    row, wave-wide reduction.
#include <algorithm>
#include <cstdlib>

#include "internal.h"
#include "lanes.h"
#include "nonfinite.h"
#include "qdot.h"

namespace sapphire {

namespace {

constexpr int kWave = 64;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int DT> struct QT;
template <> struct QT<DT_Q4_0> { static constexpr int QB = 16, BB = 20, QD = 4; };
template <> struct QT<DT_Q8_0> { static constexpr int QB = 32, BB = 36, QD = 8; };

using namespace qdot;
using namespace lanes;

// Buffer descriptors over the quant and scale planes (gfx9-family word3 0x00020000).
// A byte offset at or beyond num_records returns zeros without touching memory.
constexpr uint32_t kOffNone = 0xFFFFFFF0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kNT = 2;   // nontemporal: weights are streamed once

template <int DT, int LAYOUT>
__device__ __forceinline__ void load_block_buf(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs, uint32_t bi,
                                               bool ok, uint32_t (&q)[QT<DT>::QD], float &s) {
    if constexpr (LAYOUT == LAYOUT_PACKED) {
        const uint32_t oq = ok ? bi * QT<DT>::QB : kOffNone;
        const uint32_t os = ok ? bi * 4u : kOffNone;
#pragma unroll
        for (int i = 0; i < QT<DT>::QD / 4; ++i) {
            const u32x4 t = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, oq + 16u * i, 0, kNT));
            q[4 * i + 0] = t.x; q[4 * i + 1] = t.y; q[4 * i + 2] = t.z; q[4 * i + 3] = t.w;
        }
        s = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, os, 0, kNT));
    } else {
        const uint32_t ob = ok ? bi * QT<DT>::BB : kOffNone;
        s = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rq, ob, 0, kNT));
#pragma unroll
        for (int i = 0; i < QT<DT>::QD / 4; ++i) {
            const u32x4 t =
                __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, ob + 4u + 16u * i, 0, kNT));
            q[4 * i + 0] = t.x; q[4 * i + 1] = t.y; q[4 * i + 2] = t.z; q[4 * i + 3] = t.w;
        }
    }
}

template <int DT, int LAYOUT>
__device__ __forceinline__ void load_block(const uint8_t *__restrict__ w, size_t sc_off, long bi,
                                           uint32_t (&q)[QT<DT>::QD], float &s) {
    if constexpr (LAYOUT == LAYOUT_PACKED) {
        const u32x4 *qp = reinterpret_cast<const u32x4 *>(w + (size_t)bi * QT<DT>::QB);
#pragma unroll
        for (int i = 0; i < QT<DT>::QD / 4; ++i) {
            const u32x4 t = __builtin_nontemporal_load(qp + i);
            q[4 * i + 0] = t.x; q[4 * i + 1] = t.y; q[4 * i + 2] = t.z; q[4 * i + 3] = t.w;
        }
        s = __builtin_nontemporal_load(reinterpret_cast<const float *>(w + sc_off) + bi);
    } else {
        const uint32_t *bp = reinterpret_cast<const uint32_t *>(w + (size_t)bi * QT<DT>::BB);
        s = __uint_as_float(bp[0]);
#pragma unroll
        for (int i = 0; i < QT<DT>::QD; ++i) q[i] = bp[1 + i];
    }
}

template <int DT>
__device__ __forceinline__ float block_dot(const uint32_t (&q)[QT<DT>::QD], const float (&xv)[32], float xs) {
    if constexpr (DT == DT_Q4_0) return dot_q4(q, xv, xs);
    else return dot_q8(q, xv, xs);
}

// Orders this wave's LDS traffic without a workgroup barrier: each wave only touches its
// own slice of the reduction buffer, and the LDS unit executes one wave's operations in
// issue order, so a compiler-level fence around the exchange is sufficient.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Each wave owns the contiguous rows [wave*rows_per_wave, +rows_per_wave) (a multiple of
// rps), walked in wave-steps of rps rows, S wave-steps per iteration. Matrices are
// addressed with 32-bit byte offsets (the launcher rejects planes of 4 GiB or more).
template <int DT, int LAYOUT, int S>
__global__ __launch_bounds__(256) void gemv_q_cols(const uint8_t *__restrict__ w, size_t sc_off, uint32_t q_bytes,
                                                   uint32_t s_bytes, const float *__restrict__ x,
                                                   float *__restrict__ y, int M, int nb, int rps, int rows_per_wave) {
    __shared__ float red[4][S * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int r_in = lane / nb;
    const int blk = lane - r_in * nb;
    const bool lane_on = r_in < rps;

    float xv[32];
    {
        const float4 *xp = reinterpret_cast<const float4 *>(x + blk * kBlock);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 t = lane_on ? xp[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[4 * i + 0] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
        }
    }
    float xs = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) xs += xv[i];
    // a NaN or infinite activation makes xs non-finite (so does an overflowing sum, for which
    // the fold below is 0): zero them for the block dots and add their fold to every row
    const bool nf = __any(nonfinite::is_nf(xs));
    if (nf) {
        xs = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            xv[i] = nonfinite::is_nf(xv[i]) ? 0.f : xv[i];
            xs += xv[i];
        }
    }

    const __amdgpu_buffer_rsrc_t rq = make_rsrc(w, q_bytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w + sc_off, s_bytes);
    const int wave = blockIdx.x * (blockDim.x / kWave) + wid;
    const int rbeg = wave * rows_per_wave;
    const int rend = min(M, rbeg + rows_per_wave);
    const uint32_t step_blocks = (uint32_t)(rps * nb);
    float *redw = red[wid];

    for (int row0 = rbeg; row0 < rend; row0 += S * rps) {
        const int row_l = row0 + r_in;
        const uint32_t bi0 = (uint32_t)row_l * (uint32_t)nb + (uint32_t)blk;
        uint32_t q[S][QT<DT>::QD];
        float s[S];
#pragma unroll
        for (int st = 0; st < S; ++st)
            load_block_buf<DT, LAYOUT>(rq, rs, bi0 + st * step_blocks, lane_on && row_l + st * rps < rend, q[st],
                                       s[st]);
        float part[S];
#pragma unroll
        for (int st = 0; st < S; ++st) part[st] = s[st] * block_dot<DT>(q[st], xv, xs);
        wave_lds_sync();
#pragma unroll
        for (int st = 0; st < S; ++st) redw[st * kWave + lane] = part[st];
        wave_lds_sync();
        if (lane < S * rps) {
            const int st = lane / rps;
            const int r = lane - st * rps;
            const float *rp = &redw[st * kWave + r * nb];
            float acc = 0.f;
            for (int b = 0; b < nb; ++b) acc += rp[b];
            const int row = row0 + lane;
            if (row < rend) y[row] = nf ? acc + nonfinite::fold<DT, LAYOUT>(w, w + sc_off, nb, row, x) : acc;
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <int DT, int LAYOUT>
__global__ __launch_bounds__(256) void gemv_q_rows(const uint8_t *__restrict__ w, size_t sc_off,
                                                   const float *__restrict__ X, float *__restrict__ Y, int M,
                                                   int nb, int rows_per_wave, int batch) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const long row_begin = ((long)blockIdx.x * (blockDim.x / kWave) + wid) * rows_per_wave;
    const int K = nb * kBlock;
    for (int r = 0; r < rows_per_wave; ++r) {
        const long row = row_begin + r;
        if (row >= M) break;
        for (int b = 0; b < batch; ++b) {
            const float *x = X + (size_t)b * K;
            float acc = 0.f;
            bool nfl = false;
            for (int blk = lane; blk < nb; blk += kWave) {
                uint32_t q[QT<DT>::QD];
                float s;
                load_block<DT, LAYOUT>(w, sc_off, row * nb + blk, q, s);
                float xv[32];
                const float4 *xp = reinterpret_cast<const float4 *>(x + blk * kBlock);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 t = xp[i];
                    xv[4 * i + 0] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
                }
                float xs = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) xs += xv[i];
                if (nonfinite::is_nf(xs)) {   // NaN / inf activations: zeroed here, folded in below
                    nfl = true;
                    xs = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        xv[i] = nonfinite::is_nf(xv[i]) ? 0.f : xv[i];
                        xs += xv[i];
                    }
                }
                acc = __builtin_fmaf(s, block_dot<DT>(q, xv, xs), acc);
            }
            acc = wave_sum(acc);
            const bool nf = __any(nfl);
            if (lane == 0)
                Y[(size_t)b * M + row] = nf ? acc + nonfinite::fold<DT, LAYOUT>(w, w + sc_off, nb, (int)row, x) : acc;
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void gemv_f(const void *__restrict__ w, const float *__restrict__ x,
                                              float *__restrict__ y, int M, int K, int rows_per_wave) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const long row_begin = ((long)blockIdx.x * (blockDim.x / kWave) + wid) * rows_per_wave;
    for (int r = 0; r < rows_per_wave; ++r) {
        const long row = row_begin + r;
        if (row >= M) break;
        float acc = 0.f;
        if constexpr (DT == DT_F32) {
            const float *wr = reinterpret_cast<const float *>(w) + (size_t)row * K;
            for (int k = lane; k < K; k += kWave) acc = __builtin_fmaf(wr[k], x[k], acc);
        } else {
            const uint16_t *wr = reinterpret_cast<const uint16_t *>(w) + (size_t)row * K;
            for (int k = lane; k < K; k += kWave)
                acc = __builtin_fmaf(__uint_as_float((uint32_t)wr[k] << 16), x[k], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) y[row] = acc;
    }
}

// F32 / BF16 rows of 16-byte aligned length. x is staged once per workgroup in LDS,
// zero-padded to xpad = a whole number of U-chunk rounds of 16 lanes; a chunk past the end
// of its row (or a row past M) is loaded from an out-of-range buffer offset, which returns
// zeros, and meets zero activations. Wave-steps of 4 rows are spread over all waves of the
// grid. Each product is fused into one of two accumulators (even / odd element of the
// chunk); the reference accumulates in its own lane order (bf16_avx.c:57-113,
// f32_avx.c:43-90), so sums agree to fp32 rounding.
template <int DT, int U>
__global__ __launch_bounds__(256) void gemv_f16(const uint8_t *__restrict__ w, uint32_t w_bytes, uint32_t row_bytes,
                                                const float *__restrict__ x, float *__restrict__ y, int M, int K,
                                                int xpad) {
    constexpr int E = DT == DT_F32 ? 4 : 8;   // elements per 16-byte chunk
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < xpad; i += blockDim.x) xs[i] = i < K ? x[i] : 0.f;
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int q = lane & 15, g = lane >> 4;
    const int nchunk = (int)(row_bytes / 16u);
    const int rounds = xpad / (16 * E);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const int nwaves = gridDim.x * (blockDim.x / kWave);
    const int steps = (M + 3) / 4;
    for (int st = blockIdx.x * (blockDim.x / kWave) + (int)(threadIdx.x / kWave); st < steps; st += nwaves) {
        const int row = st * 4 + g;
        const bool on = row < M;
        const uint32_t rbase = (uint32_t)row * row_bytes;
        float a0 = 0.f, a1 = 0.f;
        for (int r = 0; r < rounds; r += U) {
            u32x4 v[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int c = (r + j) * 16 + q;
                const uint32_t off = on && c < nchunk ? rbase + 16u * (uint32_t)c : kOffNone;
                v[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kNT));
            }
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const float *xp = xs + ((r + j) * 16 + q) * E;
                if constexpr (DT == DT_F32) {
                    const float4 xv = *reinterpret_cast<const float4 *>(xp);
                    a0 = __builtin_fmaf(__uint_as_float(v[j].x), xv.x, a0);
                    a1 = __builtin_fmaf(__uint_as_float(v[j].y), xv.y, a1);
                    a0 = __builtin_fmaf(__uint_as_float(v[j].z), xv.z, a0);
                    a1 = __builtin_fmaf(__uint_as_float(v[j].w), xv.w, a1);
                } else {
                    const float4 xl = *reinterpret_cast<const float4 *>(xp);
                    const float4 xh = *reinterpret_cast<const float4 *>(xp + 4);
                    a0 = __builtin_fmaf(__uint_as_float(v[j].x << 16), xl.x, a0);
                    a1 = __builtin_fmaf(__uint_as_float(v[j].x & 0xFFFF0000u), xl.y, a1);
                    a0 = __builtin_fmaf(__uint_as_float(v[j].y << 16), xl.z, a0);
                    a1 = __builtin_fmaf(__uint_as_float(v[j].y & 0xFFFF0000u), xl.w, a1);
                    a0 = __builtin_fmaf(__uint_as_float(v[j].z << 16), xh.x, a0);
                    a1 = __builtin_fmaf(__uint_as_float(v[j].z & 0xFFFF0000u), xh.y, a1);
                    a0 = __builtin_fmaf(__uint_as_float(v[j].w << 16), xh.z, a0);
                    a1 = __builtin_fmaf(__uint_as_float(v[j].w & 0xFFFF0000u), xh.w, a1);
                }
            }
        }
        const float acc = row16_sum(a0 + a1);
        if (on && q == 0) y[row] = acc;
    }
}

template <int DT>
__global__ void repack_kernel(const uint8_t *__restrict__ aos, uint8_t *__restrict__ qs, float *__restrict__ sc,
                              long nblocks) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(aos + (size_t)i * QT<DT>::BB);
    sc[i] = __uint_as_float(src[0]);
    uint32_t *dst = reinterpret_cast<uint32_t *>(qs + (size_t)i * QT<DT>::QB);
#pragma unroll
    for (int d = 0; d < QT<DT>::QD; ++d) dst[d] = src[1 + d];
}

// One thread per block: the 32 integer weight values, and optionally fl(int * scale).
template <int DT, int LAYOUT>
__global__ void unpack_kernel(const uint8_t *__restrict__ w, size_t sc_off, long nblocks, int8_t *__restrict__ ints,
                              float *__restrict__ deq) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    uint32_t q[QT<DT>::QD];
    float s;
    load_block<DT, LAYOUT>(w, sc_off, i, q, s);
    for (int e = 0; e < 32; ++e) {
        int v;
        if constexpr (DT == DT_Q4_0) {
            const uint32_t byte = (q[(e >> 1) >> 2] >> (8 * ((e >> 1) & 3))) & 0xFFu;
            v = (int)((e & 1) ? (byte >> 4) : (byte & 0xFu)) - 8;
        } else {
            v = (int)(int8_t)((q[e >> 2] >> (8 * (e & 3))) & 0xFFu);
        }
        if (ints) ints[(size_t)i * 32 + e] = (int8_t)v;
        if (deq) deq[(size_t)i * 32 + e] = __fmul_rn((float)v, s);
    }
}

inline unsigned grid_for(long n, int per) { return (unsigned)((n + per - 1) / per); }

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <int DT, int LAYOUT, int S>
void launch_cols(const uint8_t *w, size_t sc_off, int M, int nb, int rps, const float *x, float *y, hipStream_t st,
                 int waves_per_cu) {
    const long steps = (M + rps - 1) / rps;                       // wave-steps of rps rows
    const long want = std::max(1L, std::min((long)device_cus() * waves_per_cu, (steps + S - 1) / S));
    const long steps_per_wave = (steps + want - 1) / want;
    const long waves = (steps + steps_per_wave - 1) / steps_per_wave;
    const int rows_per_wave = (int)(steps_per_wave * rps);
    const int wpb = waves >= 4L * device_cus() ? 4 : 1;           // small problems: 1 wave per block
    const size_t nblk = (size_t)M * (size_t)nb;
    const uint32_t q_bytes = (uint32_t)(nblk * (LAYOUT == LAYOUT_PACKED ? QT<DT>::QB : QT<DT>::BB));
    hipLaunchKernelGGL((gemv_q_cols<DT, LAYOUT, S>), dim3((unsigned)((waves + wpb - 1) / wpb)), dim3(64 * wpb), 0,
                       st, w, sc_off, q_bytes, (uint32_t)(nblk * 4), x, y, M, nb, rps, rows_per_wave);
}

template <int DT, int LAYOUT>
int gemv_q_typed(const uint8_t *w, size_t sc_off, int M, int nb, const float *x, float *y, hipStream_t st) {
    if ((size_t)M * (size_t)nb * QT<DT>::BB >= (size_t(1) << 32) - 256) {
        set_error("weight matrix of %d x %d blocks exceeds the 4 GiB addressing of the GEMV kernels", M, nb);
        return -1;
    }
    const int rps = nb <= kWave ? kWave / nb : 0;
    if (rps > 0 && nb * rps * 4 >= kWave * 3) {   // >= 75% of lanes busy
        const long steps = (M + rps - 1) / rps;
        if (steps >= 8L * 16 * device_cus())
            launch_cols<DT, LAYOUT, 8>(w, sc_off, M, nb, rps, x, y, st, 16);
        else if (steps >= 2L * 16 * device_cus())
            launch_cols<DT, LAYOUT, 2>(w, sc_off, M, nb, rps, x, y, st, 16);
        else
            launch_cols<DT, LAYOUT, 1>(w, sc_off, M, nb, rps, x, y, st, 16);
    } else {
        const int rpw = M >= 65536 ? 4 : 1;
        const long waves = (M + rpw - 1) / rpw;
        hipLaunchKernelGGL((gemv_q_rows<DT, LAYOUT>), dim3(grid_for(waves, 4)), dim3(256), 0, st, w, sc_off, x, y,
                           M, nb, rpw, 1);
    }
    return hip_ok(hipGetLastError(), "gemv_q launch") ? 0 : -1;
}

}  // namespace

size_t q_aos_bytes(int dt, int M, int K) { return (size_t)M * (size_t)((K + 31) / 32) * (size_t)block_bytes(dt); }

size_t q_scales_offset(int dt, int M, int K) {
    const size_t qbytes = (size_t)M * (size_t)((K + 31) / 32) * (size_t)quant_bytes(dt);
    return (qbytes + 255) & ~size_t(255);
}

size_t q_packed_bytes(int dt, int M, int K) {
    return q_scales_offset(dt, M, K) + (size_t)M * (size_t)((K + 31) / 32) * sizeof(float);
}

int launch_repack(int dt, const void *aos, int M, int K, void *packed, hipStream_t st) {
    const long nblocks = (long)M * ((K + 31) / 32);
    uint8_t *qs = static_cast<uint8_t *>(packed);
    float *sc = reinterpret_cast<float *>(qs + q_scales_offset(dt, M, K));
    if (dt == DT_Q4_0)
        hipLaunchKernelGGL(repack_kernel<DT_Q4_0>, dim3(grid_for(nblocks, 256)), dim3(256), 0, st,
                           static_cast<const uint8_t *>(aos), qs, sc, nblocks);
    else
        hipLaunchKernelGGL(repack_kernel<DT_Q8_0>, dim3(grid_for(nblocks, 256)), dim3(256), 0, st,
                           static_cast<const uint8_t *>(aos), qs, sc, nblocks);
    return hip_ok(hipGetLastError(), "repack launch") ? 0 : -1;
}

static int launch_unpack(int dt, int layout, const void *w, int M, int K, int8_t *ints, float *deq,
                         hipStream_t st) {
    const long nblocks = (long)M * ((K + 31) / 32);
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const size_t so = q_scales_offset(dt, M, K);
    const dim3 g(grid_for(nblocks, 256)), b(256);
    if (dt == DT_Q4_0 && layout == LAYOUT_AOS)
        hipLaunchKernelGGL((unpack_kernel<DT_Q4_0, LAYOUT_AOS>), g, b, 0, st, wb, so, nblocks, ints, deq);
    else if (dt == DT_Q4_0)
        hipLaunchKernelGGL((unpack_kernel<DT_Q4_0, LAYOUT_PACKED>), g, b, 0, st, wb, so, nblocks, ints, deq);
    else if (layout == LAYOUT_AOS)
        hipLaunchKernelGGL((unpack_kernel<DT_Q8_0, LAYOUT_AOS>), g, b, 0, st, wb, so, nblocks, ints, deq);
    else
        hipLaunchKernelGGL((unpack_kernel<DT_Q8_0, LAYOUT_PACKED>), g, b, 0, st, wb, so, nblocks, ints, deq);
    return hip_ok(hipGetLastError(), "unpack launch") ? 0 : -1;
}

int launch_unpack_ints(int dt, int layout, const void *w, int M, int K, int8_t *out, hipStream_t st) {
    if (layout == LAYOUT_TILED) return launch_tiled_unpack(dt, w, M, K, out, nullptr, st);
    return launch_unpack(dt, layout, w, M, K, out, nullptr, st);
}

int launch_dequant(int dt, int layout, const void *w, int M, int K, float *out, hipStream_t st) {
    if (layout == LAYOUT_TILED) return launch_tiled_unpack(dt, w, M, K, nullptr, out, st);
    return launch_unpack(dt, layout, w, M, K, nullptr, out, st);
}

int launch_gemv_q(int dt, int layout, const void *w, int M, int K, const float *x, float *y, hipStream_t st) {
    if (layout == LAYOUT_TILED) return launch_gemv_tiled(dt, w, M, K, x, y, st);
    const int nb = K / kBlock;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const size_t so = q_scales_offset(dt, M, K);
    if (dt == DT_Q4_0)
        return layout == LAYOUT_PACKED ? gemv_q_typed<DT_Q4_0, LAYOUT_PACKED>(wb, so, M, nb, x, y, st)
                                       : gemv_q_typed<DT_Q4_0, LAYOUT_AOS>(wb, so, M, nb, x, y, st);
    return layout == LAYOUT_PACKED ? gemv_q_typed<DT_Q8_0, LAYOUT_PACKED>(wb, so, M, nb, x, y, st)
                                   : gemv_q_typed<DT_Q8_0, LAYOUT_AOS>(wb, so, M, nb, x, y, st);
}

int launch_gemm_q(int dt, int layout, const void *w, int M, int K, const float *X, float *Y, int batch,
                  hipStream_t st) {
    if (layout == LAYOUT_TILED) {
        for (int b = 0; b < batch; ++b)
            if (launch_gemv_tiled(dt, w, M, K, X + (size_t)b * K, Y + (size_t)b * M, st) != 0) return -1;
        return 0;
    }
    const int nb = K / kBlock;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const size_t so = q_scales_offset(dt, M, K);
    const int rpw = M >= 65536 ? 4 : 1;
    const dim3 g(grid_for((M + rpw - 1) / rpw, 4)), b(256);
    if (dt == DT_Q4_0 && layout == LAYOUT_AOS)
        hipLaunchKernelGGL((gemv_q_rows<DT_Q4_0, LAYOUT_AOS>), g, b, 0, st, wb, so, X, Y, M, nb, rpw, batch);
    else if (dt == DT_Q4_0)
        hipLaunchKernelGGL((gemv_q_rows<DT_Q4_0, LAYOUT_PACKED>), g, b, 0, st, wb, so, X, Y, M, nb, rpw, batch);
    else if (layout == LAYOUT_AOS)
        hipLaunchKernelGGL((gemv_q_rows<DT_Q8_0, LAYOUT_AOS>), g, b, 0, st, wb, so, X, Y, M, nb, rpw, batch);
    else
        hipLaunchKernelGGL((gemv_q_rows<DT_Q8_0, LAYOUT_PACKED>), g, b, 0, st, wb, so, X, Y, M, nb, rpw, batch);
    return hip_ok(hipGetLastError(), "gemm_q launch") ? 0 : -1;
}

namespace {

constexpr int kF16MaxX = 16384;   // floats of x in LDS (64 KiB)

template <int DT, int U>
void launch_f16_u(const uint8_t *w, uint32_t w_bytes, uint32_t row_bytes, const float *x, float *y, int M, int K,
                  int xpad, hipStream_t st) {
    const long steps = (M + 3) / 4;
    const long blocks = std::max(1L, std::min((steps + 3) / 4, 8L * device_cus()));
    hipLaunchKernelGGL((gemv_f16<DT, U>), dim3((unsigned)blocks), dim3(256), (size_t)xpad * sizeof(float), st, w,
                       w_bytes, row_bytes, x, y, M, K, xpad);
}

template <int DT>
void launch_f16(const uint8_t *w, uint32_t w_bytes, uint32_t row_bytes, const float *x, float *y, int M, int K,
                int rounds, int U, hipStream_t st) {
    constexpr int E = DT == DT_F32 ? 4 : 8;
    const int xpad = (rounds + U - 1) / U * U * 16 * E;
    switch (U) {
        case 1: launch_f16_u<DT, 1>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        case 2: launch_f16_u<DT, 2>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        case 3: launch_f16_u<DT, 3>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        case 4: launch_f16_u<DT, 4>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        case 5: launch_f16_u<DT, 5>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        case 6: launch_f16_u<DT, 6>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        case 7: launch_f16_u<DT, 7>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
        default: launch_f16_u<DT, 8>(w, w_bytes, row_bytes, x, y, M, K, xpad, st); break;
    }
}

// Chunks in flight per lane for `rounds` rounds of 16 chunks: all of them up to 8, else the
// depth in 4..8 that pads the fewest rounds (the deeper on a tie).
int f16_depth(int rounds) {
    if (rounds <= 8) return std::max(rounds, 1);
    int best = 8, waste = (rounds + 7) / 8 * 8 - rounds;
    for (int u = 7; u >= 4; --u) {
        const int wst = (rounds + u - 1) / u * u - rounds;
        if (wst < waste) best = u, waste = wst;
    }
    return best;
}

}  // namespace

int launch_gemv_f(int dt, const void *w, int M, int K, const float *x, float *y, hipStream_t st) {
    if (M <= 0) return 0;
    const size_t es = dt == DT_F32 ? 4 : 2;
    const size_t row_bytes = (size_t)K * es;
    const int E = (int)(16 / es);
    const int rounds = (int)((row_bytes / 16 + 15) / 16);
    const int U = f16_depth(rounds);
    const long xpad = (long)(rounds + U - 1) / U * U * 16 * E;
    if (K > 0 && row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 && xpad <= kF16MaxX) {
        // 32-bit buffer offsets: launches of at most 2^32 - 2^20 bytes of rows each
        const long rows_per = std::max(4L, (long)((((size_t)1 << 32) - ((size_t)1 << 20)) / row_bytes) & ~3L);
        const uint8_t *wb = static_cast<const uint8_t *>(w);
        for (long r0 = 0; r0 < M; r0 += rows_per) {
            const int m = (int)std::min<long>(rows_per, M - r0);
            const uint32_t wbytes = (uint32_t)((size_t)m * row_bytes);
            if (dt == DT_F32)
                launch_f16<DT_F32>(wb + (size_t)r0 * row_bytes, wbytes, (uint32_t)row_bytes, x, y + r0, m, K, rounds,
                                   U, st);
            else
                launch_f16<DT_BF16>(wb + (size_t)r0 * row_bytes, wbytes, (uint32_t)row_bytes, x, y + r0, m, K,
                                    rounds, U, st);
        }
        return hip_ok(hipGetLastError(), "gemv_f16 launch") ? 0 : -1;
    }
    const int rpw = M >= 65536 ? 4 : 1;
    const dim3 g(grid_for((M + rpw - 1) / rpw, 4)), b(256);
    if (dt == DT_F32)
        hipLaunchKernelGGL(gemv_f<DT_F32>, g, b, 0, st, w, x, y, M, K, rpw);
    else
        hipLaunchKernelGGL(gemv_f<DT_BF16>, g, b, 0, st, w, x, y, M, K, rpw);
    return hip_ok(hipGetLastError(), "gemv_f launch") ? 0 : -1;
}

}  // namespace sapphire
