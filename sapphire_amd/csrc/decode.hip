// decode.hip - fused kernels of one Gemma-3 decode step for the device engine.
//
// One step per layer is six launches (decoder.cpp captures them in a HIP graph):
//   dec_gemv  (QKV)    prologue: previous layer's post-FFN norm + residual, pre-attention norm
//   attention partials QK-norm, RoPE, KV write, scores/softmax/values over a slice of positions
//   combine            the slices of every head into the attention output
//   dec_gemv  (o-proj)
//   dec_geglu (gate/up) prologue: post-attention norm + residual, pre-FFN norm; epilogue gelu*up
//   dec_gemv  (down)
// in the op order of inference_forward_batch (inference.c:616-651) with the stages of
// attention.c:311-375 and transformer.c:96-283.
//
// GEMV body: the input vector is staged once per workgroup in LDS; each wave takes wave-steps
// of rps = 64 / nb rows (nb = K/32 blocks per row), lane l owning block l % nb of row l / nb,
// so a Q4_0 lane issues one 16-byte quant load per block and reads its 32 x values from LDS.
// Row sums are wave-wide shuffle reductions. These GEMVs are small (<= 2 MiB of weights):
// their cost is latency, hence the fusion of the vector work around them.
#include <cmath>

#include "decode_kernels.h"
#include "devmath.h"
#include "qdot.h"

namespace sapphire {

namespace {

using namespace devmath;
using namespace qdot;

constexpr int kWave = 64;
constexpr int kThreads = 256;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// xs[0..K) = x(in) (see GemvIn); every thread of the workgroup takes part.
__device__ void stage_input(const GemvIn &in, int K, float *xs, float *sh) {
    for (int i = threadIdx.x; i < K; i += blockDim.x) xs[i] = in.resid_in[i];
    if (in.delta) {
        const float r = rms_inv_of(block_sum_sq_ref(in.delta, K, sh), K, in.eps);
        for (int i = threadIdx.x; i < K; i += blockDim.x)
            xs[i] = __fadd_rn(xs[i], __fmul_rn(__fmul_rn(in.delta[i], r), __fadd_rn(1.0f, in.w_delta[i])));
    }
    __syncthreads();
    if (in.resid_out && blockIdx.x == 0)
        for (int i = threadIdx.x; i < K; i += blockDim.x) in.resid_out[i] = xs[i];
    if (in.w_norm) {
        const float r = rms_inv_of(block_sum_sq_ref(xs, K, sh), K, in.eps);   // synchronises
        for (int i = threadIdx.x; i < K; i += blockDim.x)
            xs[i] = __fmul_rn(__fmul_rn(xs[i], r), __fadd_rn(1.0f, in.w_norm[i]));
    }
    __syncthreads();
}

template <int DT> struct QB;
template <> struct QB<DT_Q4_0> { static constexpr int BYTES = 16, WORDS = 4; };
template <> struct QB<DT_Q8_0> { static constexpr int BYTES = 32, WORDS = 8; };

// This lane's block of `row` times x: scale * sum(int * x) (0 for a lane off the matrix).
template <int DT>
__device__ __forceinline__ float lane_block(const QMat &w, int row, int blk, int nb, const float (&xv)[32], float xsum,
                                            bool on) {
    if (!on || row >= w.M) return 0.f;
    const size_t bi = (size_t)row * nb + blk;
    uint32_t q[QB<DT>::WORDS];
    const u32x4 *qp = reinterpret_cast<const u32x4 *>(w.q + bi * QB<DT>::BYTES);
#pragma unroll
    for (int i = 0; i < QB<DT>::WORDS / 4; ++i) {
        const u32x4 t = __builtin_nontemporal_load(qp + i);
        q[4 * i + 0] = t.x; q[4 * i + 1] = t.y; q[4 * i + 2] = t.z; q[4 * i + 3] = t.w;
    }
    const float s = w.s[bi];
    if constexpr (DT == DT_Q4_0) return s * dot_q4(q, xv, xsum);
    else return s * dot_q8(q, xv, xsum);
}

template <int DT, bool GEGLU>
__global__ __launch_bounds__(kThreads) void dec_gemv_kernel(QMat w0, QMat w1, GemvIn in, float *__restrict__ y) {
    __shared__ float xs[kDecMaxK];
    __shared__ float sh[16];
    const int K = w0.K, M = w0.M;
    stage_input(in, K, xs, sh);
    const int nb = K / kBlock, rps = kWave / nb;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int r_in = lane / nb, blk = lane - r_in * nb;
    const bool on = r_in < rps;
    float xv[32];
    float xsum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        xv[i] = on ? xs[blk * kBlock + i] : 0.f;
        xsum += xv[i];
    }
    const int wsteps = (M + rps - 1) / rps;
    for (int st = blockIdx.x * (kThreads / kWave) + wid; st < wsteps; st += gridDim.x * (kThreads / kWave)) {
        const int row = st * rps + r_in;
        const float p0 = lane_block<DT>(w0, row, blk, nb, xv, xsum, on);
        float p1 = 0.f;
        if constexpr (GEGLU) p1 = lane_block<DT>(w1, row, blk, nb, xv, xsum, on);
        for (int r = 0; r < rps; ++r) {
            const float t0 = wave_sum(r_in == r ? p0 : 0.f);
            float v = t0;
            if constexpr (GEGLU) v = __fmul_rn(gelu_ref(t0), wave_sum(r_in == r ? p1 : 0.f));
            const int orow = st * rps + r;
            if (lane == r && orow < M) y[orow] = v;
        }
    }
}

__global__ __launch_bounds__(kThreads) void dec_prologue_kernel(GemvIn in, int K, float *__restrict__ out) {
    __shared__ float xs[kDecMaxK];
    __shared__ float sh[16];
    stage_input(in, K, xs, sh);
    for (int i = threadIdx.x; i < K; i += blockDim.x) out[i] = xs[i];
}

// ---- attention ----

// Sums of squares of nv consecutive vectors of length hd, each in the reference order of
// sum_sq_avx2 (eight sequential lanes, then the fixed tree and a sequential tail); eight
// threads per vector. Result in ss[v].
__device__ void vectors_sum_sq(const float *__restrict__ base, int nv, int hd, float *part8, float *ss) {
    const int t = threadIdx.x;
    if (t < 8 * nv) {
        const int v = t / 8, l = t - 8 * v;
        const float *p = base + (size_t)v * hd;
        float s = 0.f;
        for (int i = l; i < (hd & ~7); i += 8) s = __builtin_fmaf(p[i], p[i], s);
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

// dst[v] = rope(rmsnorm_delta(src[v], g)) for nv head vectors, into LDS (attention.c:221-309;
// rope_apply_fast rope.c:99-117 with the fused forms of the reference build).
__device__ void norm_rope_heads(const float *__restrict__ src, int nv, int hd, const float *__restrict__ g,
                                const float *__restrict__ cs, const float *__restrict__ sn, float eps, float *dst,
                                float *part8, float *ss) {
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

// Workgroup b takes positions [t0, t1) of the layer's attention range; each wave walks
// every fourth of them with a running (max, sum, weighted V) per head; the waves are then
// merged and the slice's partial stored. Lane l owns dims [l*DPL, l*DPL + DPL).
template <int DPL, int NH>
__global__ __launch_bounds__(kThreads) void dec_attn_part_kernel(AttnArgs a) {
    __shared__ float qs[kAttnMaxQ];
    __shared__ float ks[kAttnMaxKV];
    __shared__ float part8[8 * 16];
    __shared__ float ss[16];
    __shared__ float wm[kThreads / kWave][NH], wsum[kThreads / kWave][NH];
    __shared__ float wo[kThreads / kWave][NH][kWave * DPL];
    const int hd = a.hd, nkv = a.nkv;
    const int pos = *a.d_pos, seq = pos + 1;
    const int start = (a.window > 0 && seq > a.window) ? seq - a.window : 0;
    const float *cs = a.cos_t + (size_t)pos * hd, *sn = a.sin_t + (size_t)pos * hd;
    norm_rope_heads(a.qkv, NH, hd, a.qn, cs, sn, a.eps, qs, part8, ss);
    norm_rope_heads(a.qkv + NH * hd, nkv, hd, a.kn, cs, sn, a.eps, ks, part8, ss);
    const float *vnew = a.qkv + (NH + nkv) * hd;
    if (blockIdx.x == 0)   // kv_cache_write_token: [head][pos][dim]
        for (int i = threadIdx.x; i < nkv * hd; i += blockDim.x) {
            const int h = i / hd, d = i - h * hd;
            const size_t off = ((size_t)h * a.max_ctx + pos) * hd + d;
            a.kc[off] = ks[i];
            a.vc[off] = vnew[i];
        }

    const int len = seq - start, nsplit = gridDim.x;
    const int chunk = (len + nsplit - 1) / nsplit;
    const int t0 = start + blockIdx.x * chunk, t1 = min(seq, t0 + chunk);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int group = NH / nkv;
    float m[NH], s[NH], o[NH][DPL];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        m[h] = -INFINITY;
        s[h] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[h][d] = 0.f;
    }
    for (int t = t0 + wid; t < t1; t += kThreads / kWave) {
        float kv[DPL], vv[DPL];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            if (h % group == 0) {   // the heads of one group share a K/V row
                const int hk = h / group;
                const float *krow = t == pos ? ks + hk * hd : a.kc + ((size_t)hk * a.max_ctx + t) * hd;
                const float *vrow = t == pos ? vnew + hk * hd : a.vc + ((size_t)hk * a.max_ctx + t) * hd;
#pragma unroll
                for (int d = 0; d < DPL; ++d) {
                    kv[d] = krow[lane * DPL + d];
                    vv[d] = vrow[lane * DPL + d];
                }
            }
            float dp = 0.f;
#pragma unroll
            for (int d = 0; d < DPL; ++d) dp = __builtin_fmaf(qs[h * hd + lane * DPL + d], kv[d], dp);
            const float score = __fmul_rn(wave_sum(dp), a.scale);
            const float mn = fmaxf(m[h], score);
            const float c = m[h] == -INFINITY ? 0.f : expf(m[h] - mn);
            const float p = expf(score - mn);
            s[h] = __builtin_fmaf(s[h], c, p);
#pragma unroll
            for (int d = 0; d < DPL; ++d) o[h][d] = __builtin_fmaf(o[h][d], c, p * vv[d]);
            m[h] = mn;
        }
    }
    // merge the four waves
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        if (lane == 0) {
            wm[wid][h] = m[h];
            wsum[wid][h] = s[h];
        }
#pragma unroll
        for (int d = 0; d < DPL; ++d) wo[wid][h][lane * DPL + d] = o[h][d];
    }
    __syncthreads();
    float *out = a.part + (size_t)blockIdx.x * NH * (hd + 2);
    for (int idx = threadIdx.x; idx < NH * hd; idx += blockDim.x) {
        const int h = idx / hd, d = idx - h * hd;
        float M = -INFINITY;
        for (int w = 0; w < kThreads / kWave; ++w) M = fmaxf(M, wm[w][h]);
        float S = 0.f, O = 0.f;
        for (int w = 0; w < kThreads / kWave; ++w) {
            if (wm[w][h] == -INFINITY) continue;
            const float e = expf(wm[w][h] - M);
            S = __builtin_fmaf(wsum[w][h], e, S);
            O = __builtin_fmaf(wo[w][h][d], e, O);
        }
        out[h * (hd + 2) + d] = O;
        if (d == 0) {
            out[h * (hd + 2) + hd] = M;
            out[h * (hd + 2) + hd + 1] = S;
        }
    }
}

// out[h*hd + d] = sum_b e_b o_b[d] / sum_b e_b s_b with e_b = exp(m_b - max_b m_b): the
// softmax-weighted sum of values of attention.c:140-158 over all slices. One workgroup per
// head, one thread per dim.
__global__ __launch_bounds__(kThreads) void dec_attn_combine_kernel(const float *__restrict__ part, int nsplit, int nh,
                                                                    int hd, float *__restrict__ out) {
    const int h = blockIdx.x;
    float M = -INFINITY;
    for (int b = 0; b < nsplit; ++b) M = fmaxf(M, part[((size_t)b * nh + h) * (hd + 2) + hd]);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float S = 0.f, O = 0.f;
        for (int b = 0; b < nsplit; ++b) {
            const float *p = part + ((size_t)b * nh + h) * (hd + 2);
            if (p[hd] == -INFINITY) continue;
            const float e = expf(p[hd] - M);
            S = __builtin_fmaf(p[hd + 1], e, S);
            O = __builtin_fmaf(p[d], e, O);
        }
        out[h * hd + d] = O / S;
    }
}

__global__ void dec_embed_kernel(const uint16_t *__restrict__ embed, int hidden, float es, const int *__restrict__ tok,
                                 float *__restrict__ resid) {
    const size_t row = (size_t)(*tok) * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
        const float v = __uint_as_float((uint32_t)embed[row + i] << 16);
        resid[i] = es != 1.0f ? __fmul_rn(v, es) : v;
    }
}

__global__ void dec_advance_kernel(const int *__restrict__ tok, int *__restrict__ pos, int *__restrict__ step,
                                   int *__restrict__ log) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        const int s = *step;
        log[s] = *tok;
        *step = s + 1;
        *pos = *pos + 1;
    }
}

template <int DT, bool GEGLU>
int launch_gemv_kernel(const QMat &w0, const QMat &w1, const GemvIn &in, float *y, hipStream_t st) {
    const int nb = w0.K / kBlock;
    if (w0.K % kBlock != 0 || nb > kWave || w0.K > kDecMaxK) {
        set_error("fused decode GEMV needs K a multiple of 32 and at most %d (K=%d)", kDecMaxK, w0.K);
        return -1;
    }
    const int rps = kWave / nb;
    const int wsteps = (w0.M + rps - 1) / rps;
    const int blocks = (wsteps + 3) / 4;
    hipLaunchKernelGGL((dec_gemv_kernel<DT, GEGLU>), dim3(blocks), dim3(kThreads), 0, st, w0, w1, in, y);
    return hip_ok(hipGetLastError(), "dec_gemv launch") ? 0 : -1;
}

}  // namespace

int dec_gemv(int dt, const QMat &w, const GemvIn &in, float *y, hipStream_t s) {
    return dt == DT_Q4_0 ? launch_gemv_kernel<DT_Q4_0, false>(w, w, in, y, s)
                         : launch_gemv_kernel<DT_Q8_0, false>(w, w, in, y, s);
}

int dec_geglu(int dt, const QMat &wg, const QMat &wu, const GemvIn &in, float *g, hipStream_t s) {
    if (wg.M != wu.M || wg.K != wu.K) {
        set_error("gate and up projections differ in shape");
        return -1;
    }
    return dt == DT_Q4_0 ? launch_gemv_kernel<DT_Q4_0, true>(wg, wu, in, g, s)
                         : launch_gemv_kernel<DT_Q8_0, true>(wg, wu, in, g, s);
}

int dec_prologue_only(const GemvIn &in, int K, float *out, hipStream_t s) {
    if (K > kDecMaxK) {
        set_error("vector of %d floats exceeds %d", K, kDecMaxK);
        return -1;
    }
    hipLaunchKernelGGL(dec_prologue_kernel, dim3(1), dim3(kThreads), 0, s, in, K, out);
    return hip_ok(hipGetLastError(), "dec_prologue launch") ? 0 : -1;
}

int dec_attention(const AttnArgs &a, float *out, hipStream_t s) {
    if (a.nh * a.hd > kAttnMaxQ || a.nkv * a.hd > kAttnMaxKV || a.nkv <= 0 || a.nh % a.nkv != 0 ||
        a.hd % kWave != 0 || a.hd > 4 * kWave || a.nh + a.nkv > 16) {
        set_error("attention shape not supported (heads %d/%d, head_dim %d)", a.nh, a.nkv, a.hd);
        return -1;
    }
    const int dpl = a.hd / kWave;
#define SPH_ATTN(DPLV, NHV)                                                                                  \
    if (dpl == DPLV && a.nh == NHV) {                                                                        \
        hipLaunchKernelGGL((dec_attn_part_kernel<DPLV, NHV>), dim3(kAttnSplit), dim3(kThreads), 0, s, a); \
    } else
    SPH_ATTN(1, 4) SPH_ATTN(2, 4) SPH_ATTN(4, 4) SPH_ATTN(1, 8) SPH_ATTN(2, 8) SPH_ATTN(4, 8) {
        set_error("attention with %d heads of dim %d not instantiated", a.nh, a.hd);
        return -1;
    }
#undef SPH_ATTN
    if (!hip_ok(hipGetLastError(), "attention launch")) return -1;
    hipLaunchKernelGGL(dec_attn_combine_kernel, dim3(a.nh), dim3(kThreads), 0, s, a.part, kAttnSplit, a.nh, a.hd, out);
    return hip_ok(hipGetLastError(), "attention combine launch") ? 0 : -1;
}

int dec_embed(const uint16_t *embed, int hidden, float es, const int *d_token, float *resid, hipStream_t s) {
    hipLaunchKernelGGL(dec_embed_kernel, dim3((hidden + kThreads - 1) / kThreads), dim3(kThreads), 0, s, embed, hidden,
                       es, d_token, resid);
    return hip_ok(hipGetLastError(), "embed launch") ? 0 : -1;
}

int dec_advance(const int *d_token, int *d_pos, int *d_step, int *log, hipStream_t s) {
    hipLaunchKernelGGL(dec_advance_kernel, dim3(1), dim3(64), 0, s, d_token, d_pos, d_step, log);
    return hip_ok(hipGetLastError(), "advance launch") ? 0 : -1;
}

}  // namespace sapphire
