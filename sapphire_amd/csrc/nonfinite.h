// nonfinite.h - IEEE behaviour of the quantized GEMV kernels for activations that are NaN or
// +-inf (shared device helpers; not installed).
//
// The reference accumulates w * x with fp32 FMAs (q4_0_avx.c:31-42, q8_0_avx.c:50-64), so a
// non-finite activation x_k reaches every row: its term fl(w_rk * x_k) is NaN (x_k NaN, or
// w_rk = 0 with x_k infinite) or +-inf, and from then on the row's accumulators stay
// non-finite; the final sum is NaN if any term is NaN or terms of both signs are infinite,
// else that infinity. The finite terms cannot change that result, so
//   y_r = sum over the non-finite x_k of fl(w_rk * x_k)   (in any order)
// whenever x has a non-finite element. (Finite sums that overflow to infinity are outside
// this argument; they need |x| near 1e36.)
//
// The fast kernels compute the finite dot products with algebraic shortcuts (integer digits,
// -8 * sum(x) offsets, range scales) that turn a non-finite x into the wrong special value.
// They therefore zero non-finite activations before those steps, detect them with one
// wave-uniform test, and in that (rare) case add fold() to the row's result: a finite number
// plus the fold is the fold.
#pragma once

#include <cstdint>

#include "internal.h"

namespace sapphire {
namespace nonfinite {

__device__ __forceinline__ bool is_nf(float v) { return (__float_as_uint(v) & 0x7f800000u) == 0x7f800000u; }

// fl(int * scale) of element k of row r (the dequantised weight, q4_0_avx.c:38-40 /
// q8_0_avx.c:50-59). wq: quants (AOS: the block array), wsc: scales (PACKED / TILED planes).
template <int DT, int LAYOUT>
__device__ float weight_at(const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wsc, int nb, int r, int k) {
    const int b = k >> 5, e = k & 31;
    uint32_t byte;
    float s;
    if constexpr (LAYOUT == LAYOUT_TILED) {
        // 16-row tiles, 4-block groups (gemv_mfma.hip / to_tiled_kernel)
        const int t = r >> 4, i = r & 15, g = b >> 2, j = b & 3;
        const size_t gb = (size_t)t * (size_t)(nb >> 2) + (size_t)g;
        s = reinterpret_cast<const float *>(wsc)[(gb * 4 + j) * 16 + i];
        if constexpr (DT == DT_Q8_0) {
            byte = wq[(gb * 2 + (j >> 1)) * 1024 + ((e >> 3) * 16 + i) * 16 + (j & 1) * 8 + (e & 7)];
        } else {
            const int bi = e >> 1;
            byte = wq[gb * 1024 + ((bi >> 2) * 16 + i) * 16 + j * 4 + (bi & 3)] ^ 0x88u;
        }
    } else {
        const size_t bi = (size_t)r * (size_t)nb + (size_t)b;
        const uint8_t *q;
        if constexpr (LAYOUT == LAYOUT_PACKED) {
            s = reinterpret_cast<const float *>(wsc)[bi];
            q = wq + bi * (size_t)(DT == DT_Q4_0 ? 16 : 32);
        } else {
            const uint8_t *blk = wq + bi * (size_t)(DT == DT_Q4_0 ? 20 : 36);
            s = *reinterpret_cast<const float *>(blk);
            q = blk + 4;
        }
        byte = DT == DT_Q8_0 ? q[e] : q[e >> 1];
    }
    int v;
    if constexpr (DT == DT_Q8_0) v = (int)(int8_t)byte;
    else v = (int)((e & 1) ? (byte >> 4) : (byte & 0xFu)) - 8;
    return __fmul_rn((float)v, s);
}

// Sum over the non-finite x[k], k < nb * 32, of fl(w_rk * x_k): row r's result whenever x
// has a non-finite element.
template <int DT, int LAYOUT>
__device__ float fold(const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wsc, int nb, int r,
                      const float *__restrict__ x) {
    float acc = 0.f;
    for (int k = 0; k < nb * 32; ++k) {
        const float xv = x[k];
        if (is_nf(xv)) acc = __fadd_rn(acc, __fmul_rn(weight_at<DT, LAYOUT>(wq, wsc, nb, r, k), xv));
    }
    return acc;
}

}  // namespace nonfinite
}  // namespace sapphire
