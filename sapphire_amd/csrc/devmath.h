// devmath.h - device functions shared by the primitive and decode kernels (not installed).
#pragma once

#include <hip/hip_runtime.h>

namespace sapphire {
namespace devmath {

// Bit-exact restatement of sum_sq_avx2 (normalization.c:12-32). Called by one lane.
__device__ inline float sum_sq_ref(const float *__restrict__ in, int dim) {
    float s[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) s[l] = 0.f;
    int i = 0;
    for (; i + 8 <= dim; i += 8) {
#pragma unroll
        for (int l = 0; l < 8; ++l) s[l] = __builtin_fmaf(in[i + l], in[i + l], s[l]);
    }
    const float a0 = s[0] + s[4], a1 = s[1] + s[5], a2 = s[2] + s[6], a3 = s[3] + s[7];
    float sum = (a0 + a1) + (a2 + a3);
    for (; i < dim; ++i) sum = __builtin_fmaf(in[i], in[i], sum);
    return sum;
}

// Correctly rounded fp32 square root. The fp32 sqrt lowers to v_sqrt_f32 (about 1 ulp);
// the fp64 one is Newton-refined with FMAs, and rounding its result to fp32 is exact-
// rounding safe because 53 >= 2*24 + 2.
__device__ __forceinline__ float sqrt_rn(float a) { return (float)__builtin_sqrt((double)a); }

__device__ __forceinline__ float rms_inv_of(float ss, int dim, float eps) {
    return __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)dim), eps)));
}

// Eight lanes each run one sequential chain so the loads of the eight chains overlap.
__device__ inline float block_sum_sq_ref(const float *__restrict__ in, int dim, float *sh) {
    const int t = threadIdx.x;
    if (t < 8) {
        float s = 0.f;
        int i = t;
        const int full = dim & ~7;
        for (; i < full; i += 8) s = __builtin_fmaf(in[i], in[i], s);
        sh[t] = s;
    }
    __syncthreads();
    if (t == 0) {
        const float a0 = sh[0] + sh[4], a1 = sh[1] + sh[5], a2 = sh[2] + sh[6], a3 = sh[3] + sh[7];
        float sum = (a0 + a1) + (a2 + a3);
        for (int i = dim & ~7; i < dim; ++i) sum = __builtin_fmaf(in[i], in[i], sum);
        sh[8] = sum;
    }
    __syncthreads();
    return sh[8];
}

// (value, index) order of sample_greedy (utils.c:145-156): a larger value wins, and of
// equal values the lower index. A NaN never wins.
__device__ __forceinline__ bool greedy_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// gelu of activations.c:64-76 (tanh form; x + B*x^3 fused as in the reference build).
__device__ __forceinline__ float gelu_ref(float x) {
    const float A = 0.7978845608f, B = 0.044715f;
    const float y = __fmul_rn(A, __builtin_fmaf(__fmul_rn(__fmul_rn(B, x), x), x, x));
    const float t = tanhf(y);
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, t));
}

}  // namespace devmath
}  // namespace sapphire
