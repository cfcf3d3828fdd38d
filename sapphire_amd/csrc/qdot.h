// qdot.h - per-lane dot products of one Q4_0 / Q8_0 block with 32 fp32 activations held in
// registers (shared by the GEMV kernels; not installed).
#pragma once

#include <cstdint>

namespace sapphire {
namespace qdot {

// Opaque bitwise ops: the compiler would otherwise fold the nibble mask into later
// byte extracts (v_bfe_u32 + v_cvt_f32_ubyte0, two ops per weight). Behind an opaque
// v_and/v_xor every (v >> 8c) & 0xFF -> float becomes one v_cvt_f32_ubyte{c}.
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(m));
    return r;
}
__device__ __forceinline__ uint32_t xor_opaque(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_xor_b32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(m));
    return r;
}
template <int C>
__device__ __forceinline__ float cvt_ub(uint32_t v) { return (float)((v >> (8 * C)) & 0xFFu); }

// sum over the 32 elements of one Q4_0 block of (nib - 8) * x, x in registers.
// lo = q & 0x0F0F0F0F holds nib(2j) in byte j; hi = q & 0xF0F0F0F0 holds 16*nib(2j+1);
// the -8 offset is folded into -8*sum(x) (xs), precomputed once per lane. All products
// and the 1/16 rescale of the hi sum are exact; only the fp32 sums round.
__device__ __forceinline__ float dot_q4(const uint32_t (&q)[4], const float (&xv)[32], float xs) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t lo = and_opaque(q[d], 0x0F0F0F0Fu);
        const uint32_t hi = and_opaque(q[d], 0xF0F0F0F0u);
        const float *xd = &xv[8 * d];
        a0 = __builtin_fmaf(cvt_ub<0>(lo), xd[0], a0);
        a2 = __builtin_fmaf(cvt_ub<0>(hi), xd[1], a2);
        a1 = __builtin_fmaf(cvt_ub<1>(lo), xd[2], a1);
        a3 = __builtin_fmaf(cvt_ub<1>(hi), xd[3], a3);
        a0 = __builtin_fmaf(cvt_ub<2>(lo), xd[4], a0);
        a2 = __builtin_fmaf(cvt_ub<2>(hi), xd[5], a2);
        a1 = __builtin_fmaf(cvt_ub<3>(lo), xd[6], a1);
        a3 = __builtin_fmaf(cvt_ub<3>(hi), xd[7], a3);
    }
    const float lo_sum = a0 + a1;
    return __builtin_fmaf(a2 + a3, 0.0625f, __builtin_fmaf(-8.0f, xs, lo_sum));
}

// sum over one Q8_0 block of q * x. Bytes are flipped to q + 128 (0..255) so the
// unsigned converts apply; the +128 is removed as -128*sum(x) (xs).
__device__ __forceinline__ float dot_q8(const uint32_t (&q)[8], const float (&xv)[32], float xs) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        const uint32_t u = xor_opaque(q[d], 0x80808080u);
        a0 = __builtin_fmaf(cvt_ub<0>(u), xv[4 * d + 0], a0);
        a1 = __builtin_fmaf(cvt_ub<1>(u), xv[4 * d + 1], a1);
        a2 = __builtin_fmaf(cvt_ub<2>(u), xv[4 * d + 2], a2);
        a3 = __builtin_fmaf(cvt_ub<3>(u), xv[4 * d + 3], a3);
    }
    return __builtin_fmaf(-128.0f, xs, (a0 + a1) + (a2 + a3));
}

}  // namespace qdot
}  // namespace sapphire
