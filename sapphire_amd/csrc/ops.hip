// ops.hip - RMSNorm, RoPE, GeGLU, softmax/argmax and residual kernels for gfx950.
//
// Rounding: RMSNorm reproduces the reference's sum-of-squares order exactly (eight
// sequential fp32 FMA lanes over elements l, l+8, ..., then ((s0+s4)+(s1+s5)) +
// ((s2+s6)+(s3+s7)) and a sequential fused tail; normalization.c:12-32) and the same
// correctly rounded sqrt/divide, so with identical inputs its output is bit-identical to
// the reference. RoPE applies the same two fused multiply-adds the reference build
// produces (rope.c:113-115). GELU/softmax use the device expf/tanhf, which may differ
// from glibc by an ulp; softmax sums in parallel rather than left to right.
#include <algorithm>

#include "devmath.h"
#include "internal.h"

namespace sapphire {

namespace {

using namespace devmath;

constexpr int kWave = 64;

template <bool DELTA>
__global__ __launch_bounds__(256) void rmsnorm_kernel(float *__restrict__ out, const float *__restrict__ in,
                                                      const float *__restrict__ w, float eps, int dim) {
    __shared__ float sh[16];
    const float *row = in + (size_t)blockIdx.x * dim;
    float *orow = out + (size_t)blockIdx.x * dim;
    const float ss = block_sum_sq_ref(row, dim, sh);
    const float r = rms_inv_of(ss, dim, eps);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        const float g = DELTA ? __fadd_rn(1.0f, w[i]) : w[i];
        orow[i] = __fmul_rn(__fmul_rn(row[i], r), g);
    }
}

// n = rmsnorm_delta(h, w); resid += n; h = resid  (attention.c:358-366, transformer.c:231-239)
__global__ __launch_bounds__(256) void norm_residual_kernel(float *__restrict__ hidden, float *__restrict__ resid,
                                                            const float *__restrict__ w, float eps, int dim) {
    __shared__ float sh[16];
    const float ss = block_sum_sq_ref(hidden, dim, sh);
    const float r = rms_inv_of(ss, dim, eps);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        const float n = __fmul_rn(__fmul_rn(hidden[i], r), __fadd_rn(1.0f, w[i]));
        const float v = __fadd_rn(resid[i], n);
        resid[i] = v;
        hidden[i] = v;
    }
}

// x[i] = x0*c - x1*s, x[i+half] = x1*c + x0*s, in the fused forms of the reference build.
__global__ void rope_kernel(float *__restrict__ x, int n_heads, int head_dim, int pos,
                            const float *__restrict__ cos_t, const float *__restrict__ sin_t) {
    const int half = head_dim / 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_heads * half) return;
    const int h = t / half, i = t - h * half;
    float *xh = x + (size_t)h * head_dim;
    const float c = cos_t[(size_t)pos * head_dim + i];
    const float s = sin_t[(size_t)pos * head_dim + i];
    const float x0 = xh[i], x1 = xh[i + half];
    xh[i] = __builtin_fmaf(x0, c, -__fmul_rn(x1, s));
    xh[i + half] = __builtin_fmaf(x1, c, __fmul_rn(x0, s));
}

// (x[2p], x[2p+1]) -> (xe c - xo s, xe s + xo c) (positional_encoding.c:95-99), in the fused
// forms of the reference build (the second product of each line fused onto the first).
__global__ void rope_pairs_kernel(float *__restrict__ x, int npairs, const float *__restrict__ cos_p,
                                  const float *__restrict__ sin_p) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npairs) return;
    const float c = cos_p[p], s = sin_p[p];
    const float xe = x[2 * p], xo = x[2 * p + 1];
    x[2 * p] = __builtin_fmaf(-xo, s, __fmul_rn(xe, c));
    x[2 * p + 1] = __builtin_fmaf(xo, c, __fmul_rn(xe, s));
}

__global__ void gelu_mul_kernel(float *__restrict__ gate, const float *__restrict__ up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = __fmul_rn(gelu_ref(gate[i]), up[i]);
}

// ---- softmax + argmax over a long vector, two passes over the partials ----
constexpr int kSmBlock = 256;
constexpr int kSmParts = 256;   // partial blocks of pass 1

struct MaxArg { float v; int i; };

__device__ __forceinline__ MaxArg better(MaxArg a, MaxArg b) {
    // larger value wins; equal values -> lower index (sample_greedy's strict '>')
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

__device__ __forceinline__ MaxArg wave_maxarg(MaxArg m) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        MaxArg o{__shfl_xor(m.v, off, kWave), __shfl_xor(m.i, off, kWave)};
        m = better(m, o);
    }
    return m;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Each thread visits elements i = i0 + u * stride (u < kSmVec) of [.., end) per trip. The loads
// go through an index clamped to end - 1 (in bounds, branch-free), so a trip's kSmVec loads are
// issued together; f sees the in-range ones in ascending order, as a plain strided loop would.
constexpr int kSmVec = 4;

template <typename T, typename F>
__device__ __forceinline__ void strided_visit(const T *__restrict__ a, int first, int end, int stride, F f) {
    for (int i0 = first; i0 < end; i0 += kSmVec * stride) {
        T v[kSmVec];
#pragma unroll
        for (int u = 0; u < kSmVec; ++u) v[u] = a[min(i0 + u * stride, end - 1)];
#pragma unroll
        for (int u = 0; u < kSmVec; ++u)
            if (i0 + u * stride < end) f(v[u], i0 + u * stride);
    }
}

// Pass 1: each block reduces a contiguous chunk to (max, first argmax, sum exp(x - max)).
__global__ __launch_bounds__(kSmBlock) void softmax_partials(const float *__restrict__ x, int n, int chunk,
                                                             float *__restrict__ pmax, float *__restrict__ psum,
                                                             int *__restrict__ parg) {
    __shared__ MaxArg smax[kSmBlock / kWave];
    __shared__ float ssum[kSmBlock / kWave];
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int begin = blockIdx.x * chunk;
    const int end = min(n, begin + chunk);
    MaxArg m{-INFINITY, 0x7fffffff};
    strided_visit(x, begin + (int)threadIdx.x, end, kSmBlock, [&](float v, int i) { m = better(m, MaxArg{v, i}); });
    m = wave_maxarg(m);
    if (lane == 0) smax[wid] = m;
    __syncthreads();
    MaxArg bm = smax[0];
    for (int k = 1; k < kSmBlock / kWave; ++k) bm = better(bm, smax[k]);
    float s = 0.f;
    if (bm.v > -INFINITY)
        strided_visit(x, begin + (int)threadIdx.x, end, kSmBlock, [&](float v, int) { s += expf(v - bm.v); });
    s = wave_sum(s);
    if (lane == 0) ssum[wid] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.f;
        for (int k = 0; k < kSmBlock / kWave; ++k) t += ssum[k];
        pmax[blockIdx.x] = bm.v;
        psum[blockIdx.x] = t;
        parg[blockIdx.x] = bm.i;
    }
}

// Pass 2: every block folds the partials (cheap, kSmParts values) and normalises its chunk. The
// chunk's first kSmVec values per thread are loaded before the fold (independent loads).
__global__ __launch_bounds__(kSmBlock) void softmax_finish(const float *__restrict__ x, int n, int chunk, int parts,
                                                           const float *__restrict__ pmax,
                                                           const float *__restrict__ psum,
                                                           const int *__restrict__ parg, float *__restrict__ probs,
                                                           int *__restrict__ argmax_out) {
    __shared__ float s_gmax, s_inv;
    const int begin = blockIdx.x * chunk;
    const int end = min(n, begin + chunk);
    const int first = begin + (int)threadIdx.x;
    float v0[kSmVec];
    if (probs && first < end)
#pragma unroll
        for (int u = 0; u < kSmVec; ++u) v0[u] = x[min(first + u * kSmBlock, end - 1)];
    static_assert(kSmParts <= kWave * kSmVec, "one trip of wave 0 covers the partials");
    if (threadIdx.x < kWave) {
        // lane l holds partials l + 64u (clamped loads, all issued together)
        float pm[kSmVec], ps[kSmVec];
        int pa[kSmVec];
#pragma unroll
        for (int u = 0; u < kSmVec; ++u) {
            const int p = min((int)threadIdx.x + u * kWave, parts - 1);
            pm[u] = pmax[p];
            ps[u] = psum[p];
            pa[u] = parg[p];
        }
        MaxArg m{-INFINITY, 0x7fffffff};
#pragma unroll
        for (int u = 0; u < kSmVec; ++u)
            if ((int)threadIdx.x + u * kWave < parts) m = better(m, MaxArg{pm[u], pa[u]});
        m = wave_maxarg(m);
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < kSmVec; ++u)
            if ((int)threadIdx.x + u * kWave < parts && pm[u] > -INFINITY) s += ps[u] * expf(pm[u] - m.v);
        s = wave_sum(s);
        if (threadIdx.x == 0) {
            s_gmax = m.v;
            s_inv = 1.0f / s;
            // sample_greedy (utils.c:145-156) starts at index 0 and only a greater logit
            // replaces it: 0 when x[0] is NaN or no logit is above -inf
            if (blockIdx.x == 0 && argmax_out) *argmax_out = (m.i >= 0 && m.i < n && !isnan(x[0])) ? m.i : 0;
        }
    }
    __syncthreads();
    if (!probs) return;
    const float gm = s_gmax, inv = s_inv;
    for (int i0 = first; i0 < end; i0 += kSmVec * kSmBlock) {
        float v[kSmVec];
#pragma unroll
        for (int u = 0; u < kSmVec; ++u) v[u] = i0 == first ? v0[u] : x[min(i0 + u * kSmBlock, end - 1)];
#pragma unroll
        for (int u = 0; u < kSmVec; ++u)
            if (i0 + u * kSmBlock < end) probs[i0 + u * kSmBlock] = expf(v[u] - gm) * inv;
    }
}


// ---- elementwise kernels behind the host-pointer API of kernels.h ----
__global__ void unary_kernel(float *__restrict__ x, int n, int op, float a) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r = v;
    switch (op) {
        case UOP_GELU: r = gelu_ref(v); break;                                       // activations.c:64-76
        case UOP_SILU: r = __fmul_rn(v, __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-v)))); break;  // :16-20
        case UOP_RELU: r = v > 0.0f ? v : 0.0f; break;                               // :37-39
        case UOP_SCALE: r = __fmul_rn(v, a); break;                                  // utils.c:87-92
        case UOP_SOFTCAP: r = __fmul_rn(a, tanhf(__fmul_rn(v, __fdiv_rn(1.0f, a)))); break;  // utils.c:119-125
        default: break;
    }
    x[i] = r;
}

// dst = a*src + dst (fused, as `y[i] += alpha * temp[i]` is built; dispatch.c:226-228); a=1 -> add
__global__ void axpy_kernel(float *__restrict__ dst, const float *__restrict__ src, int n, float a, int fused) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    dst[i] = fused ? __builtin_fmaf(a, src[i], dst[i]) : __fadd_rn(dst[i], src[i]);
}

// out[i] = in[i] * gelu(in[i + n])  (sapphire_geglu, activations.c:123-156)
__global__ void geglu_split_kernel(float *__restrict__ out, const float *__restrict__ in, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __fmul_rn(in[i], gelu_ref(in[i + n]));
}

__global__ void bf16_kernel(float *__restrict__ dst, const uint16_t *__restrict__ src, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = __uint_as_float((uint32_t)src[i] << 16);
}

// vec_dot in the reference order (utils.c:100-117): eight sequential FMA lanes, lanes
// summed left to right, fused tail. One block; eight lanes do the work.
__global__ void dot_ref_kernel(const float *__restrict__ a, const float *__restrict__ b, int n, float *out) {
    __shared__ float sh[8];
    const int t = threadIdx.x;
    if (t < 8) {
        float s = 0.f;
        const int full = n & ~7;
        for (int i = t; i < full; i += 8) s = __builtin_fmaf(a[i], b[i], s);
        sh[t] = s;
    }
    __syncthreads();
    if (t == 0) {
        float f = sh[0] + sh[1] + sh[2] + sh[3] + sh[4] + sh[5] + sh[6] + sh[7];
        for (int i = n & ~7; i < n; ++i) f = __builtin_fmaf(a[i], b[i], f);
        *out = f;
    }
}

}  // namespace

int launch_rmsnorm(float *out, const float *in, const float *w, float eps, int dim, int batch, bool delta,
                   hipStream_t s) {
    if (delta)
        hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(batch), dim3(256), 0, s, out, in, w, eps, dim);
    else
        hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(batch), dim3(256), 0, s, out, in, w, eps, dim);
    return hip_ok(hipGetLastError(), "rmsnorm launch") ? 0 : -1;
}

int launch_norm_residual(float *hidden, float *resid, const float *w, float eps, int dim, hipStream_t s) {
    hipLaunchKernelGGL(norm_residual_kernel, dim3(1), dim3(256), 0, s, hidden, resid, w, eps, dim);
    return hip_ok(hipGetLastError(), "norm_residual launch") ? 0 : -1;
}

int launch_rope(float *x, int n_heads, int head_dim, int pos, const float *cos_t, const float *sin_t,
                hipStream_t s) {
    const int n = n_heads * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, n_heads, head_dim, pos, cos_t, sin_t);
    return hip_ok(hipGetLastError(), "rope launch") ? 0 : -1;
}

int launch_rope_pairs(float *x, int npairs, const float *cos_p, const float *sin_p, hipStream_t s) {
    hipLaunchKernelGGL(rope_pairs_kernel, dim3((npairs + 255) / 256), dim3(256), 0, s, x, npairs, cos_p, sin_p);
    return hip_ok(hipGetLastError(), "rope_pairs launch") ? 0 : -1;
}

int launch_gelu_mul(float *gate, const float *up, int n, hipStream_t s) {
    hipLaunchKernelGGL(gelu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, gate, up, n);
    return hip_ok(hipGetLastError(), "gelu_mul launch") ? 0 : -1;
}

size_t softmax_scratch_floats(int) { return 3 * kSmParts; }

int launch_softmax_argmax(const float *logits, int n, float *probs, int *argmax, float *scratch, hipStream_t s) {
    const int parts = n < kSmParts * kSmBlock ? (n + kSmBlock - 1) / kSmBlock : kSmParts;
    const int chunk = (n + parts - 1) / parts;
    float *pmax = scratch, *psum = scratch + kSmParts;
    int *parg = reinterpret_cast<int *>(scratch + 2 * kSmParts);
    hipLaunchKernelGGL(softmax_partials, dim3(parts), dim3(kSmBlock), 0, s, logits, n, chunk, pmax, psum, parg);
    if (!hip_ok(hipGetLastError(), "softmax_partials launch")) return -1;
    const unsigned g2 = probs ? (unsigned)parts : 1u;
    hipLaunchKernelGGL(softmax_finish, dim3(g2), dim3(kSmBlock), 0, s, logits, n, chunk, parts, pmax, psum, parg,
                       probs, argmax);
    return hip_ok(hipGetLastError(), "softmax_finish launch") ? 0 : -1;
}

int launch_unary(float *x, int n, int op, float a, hipStream_t s) {
    hipLaunchKernelGGL(unary_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, n, op, a);
    return hip_ok(hipGetLastError(), "unary launch") ? 0 : -1;
}

int launch_axpy(float *dst, const float *src, int n, float a, bool fused, hipStream_t s) {
    hipLaunchKernelGGL(axpy_kernel, dim3((n + 255) / 256), dim3(256), 0, s, dst, src, n, a, fused ? 1 : 0);
    return hip_ok(hipGetLastError(), "axpy launch") ? 0 : -1;
}

int launch_geglu_split(float *out, const float *in, int n, hipStream_t s) {
    hipLaunchKernelGGL(geglu_split_kernel, dim3((n + 255) / 256), dim3(256), 0, s, out, in, n);
    return hip_ok(hipGetLastError(), "geglu launch") ? 0 : -1;
}

int launch_bf16_to_f32(float *dst, const uint16_t *src, int n, hipStream_t s) {
    hipLaunchKernelGGL(bf16_kernel, dim3((n + 255) / 256), dim3(256), 0, s, dst, src, n);
    return hip_ok(hipGetLastError(), "bf16 launch") ? 0 : -1;
}

int launch_dot_ref(const float *a, const float *b, int n, float *out, hipStream_t s) {
    hipLaunchKernelGGL(dot_ref_kernel, dim3(1), dim3(64), 0, s, a, b, n, out);
    return hip_ok(hipGetLastError(), "dot launch") ? 0 : -1;
}

}  // namespace sapphire
