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
#include "decode_device.h"
#include "gemm_body.h"

namespace sapphire {

namespace {

// xs[0..K) = x(in) (see GemvIn); every thread of the workgroup takes part. dl is LDS
// scratch of K floats for the delta vector.
__device__ void stage_input(const GemvIn &in, int K, float *xs, float *dl, float *sh) {
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        xs[i] = in.resid_in[i];
        if (in.delta) dl[i] = in.delta[i];
    }
    __syncthreads();
    if (in.delta) {
        const float r = rms_inv_of(lds_sum_sq(dl, K, sh), K, in.eps);
        for (int i = threadIdx.x; i < K; i += blockDim.x)
            xs[i] = __fadd_rn(xs[i], __fmul_rn(__fmul_rn(dl[i], r), __fadd_rn(1.0f, in.w_delta[i])));
        __syncthreads();
    }
    if (in.resid_out && blockIdx.x == 0)
        for (int i = threadIdx.x; i < K; i += blockDim.x) in.resid_out[i] = xs[i];
    if (in.w_norm) {
        const float r = rms_inv_of(lds_sum_sq(xs, K, sh), K, in.eps);   // synchronises
        for (int i = threadIdx.x; i < K; i += blockDim.x)
            xs[i] = __fmul_rn(__fmul_rn(xs[i], r), __fadd_rn(1.0f, in.w_norm[i]));
    }
    __syncthreads();
}

// One wave-step per wave: rps rows of w0 (and of w1 for the GeGLU form).
template <int DT, bool GEGLU>
__global__ __launch_bounds__(kThreads) void dec_gemv_kernel(QMat w0, QMat w1, GemvIn in, float *__restrict__ y) {
    __shared__ float xs[kDecMaxK];
    __shared__ float dl[kDecMaxK];
    __shared__ float sh[16];
    const int K = w0.K, M = w0.M;
    const int nb = K / kBlock, rps = kWave / nb;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int r_in = lane / nb, blk = lane - r_in * nb;
    const bool on = r_in < rps;
    const int st = blockIdx.x * (kThreads / kWave) + wid;
    const int row = st * rps + r_in;
    LaneBlock<DT> b0, b1;
    load_lane_block<DT>(w0, row, blk, nb, on, b0);
    if constexpr (GEGLU) load_lane_block<DT>(w1, row, blk, nb, on, b1);
    stage_input(in, K, xs, dl, sh);
    float xv[32];
    float xsum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        xv[i] = on ? xs[blk * kBlock + i] : 0.f;
        xsum += xv[i];
    }
    const float p0 = block_value<DT>(b0, xv, xsum);
    float p1 = 0.f;
    if constexpr (GEGLU) p1 = block_value<DT>(b1, xv, xsum);
    for (int r = 0; r < rps; ++r) {
        const float t0 = xor_sum(r_in == r ? p0 : 0.f);
        float v = t0;
        if constexpr (GEGLU) v = __fmul_rn(gelu_ref(t0), xor_sum(r_in == r ? p1 : 0.f));
        const int orow = st * rps + r;
        if (lane == r && orow < M) y[orow] = v;
    }
}

// Sequence blockIdx.y of a batch: its vectors at + blockIdx.y * stride.
__global__ __launch_bounds__(kThreads) void dec_prologue_kernel(GemvIn in, int K, float *__restrict__ out,
                                                                size_t stride) {
    {
        const size_t o = blockIdx.y * stride;
        in.resid_in += o;
        if (in.delta) in.delta += o;
        out += o;
    }
    __shared__ float xs[kDecMaxK];
    __shared__ float dl[kDecMaxK];
    __shared__ float sh[16];
    stage_input(in, K, xs, dl, sh);
    for (int i = threadIdx.x; i < K; i += blockDim.x) out[i] = xs[i];
}

// ---- attention ----

// K/V rows of a batch (sequence blockIdx.x): the same norm_rope_heads on the same inputs
// as dec_attn_part_kernel, so the rows are bit-identical to the ones it writes.
__global__ __launch_bounds__(kThreads) void dec_kv_write_kernel(AttnArgs a) {
    const size_t b = blockIdx.x;
    const float *qkv = a.qkv + b * a.qkv_stride;
    float *kc = a.kc + b * a.kv_stride, *vc = a.vc + b * a.kv_stride;
    const int pos = a.d_pos[b];
    __shared__ float raw[kAttnMaxKV];
    __shared__ float ks[kAttnMaxKV];
    __shared__ float part8[8 * 16];
    __shared__ float ss[16];
    const int hd = a.hd, nkv = a.nkv, nq = a.nh * hd;
    for (int i = threadIdx.x; i < nkv * hd; i += blockDim.x) raw[i] = qkv[nq + i];
    __syncthreads();
    norm_rope_heads(raw, nkv, hd, a.kn, a.cos_t + (size_t)pos * hd, a.sin_t + (size_t)pos * hd, a.eps, ks, part8, ss);
    for (int i = threadIdx.x; i < nkv * hd; i += blockDim.x) {
        const int h = i / hd, d = i - h * hd;
        const size_t off = ((size_t)h * a.max_ctx + pos) * hd + d;
        kc[off] = ks[i];
        vc[off] = qkv[nq + nkv * hd + i];
    }
}

// p[0..DPL) as one vector load (p aligned to DPL floats).
template <int DPL>
struct Lanes {
    float v[DPL];
};
template <int DPL>
__device__ __forceinline__ Lanes<DPL> load_lanes(const float *p) {
    Lanes<DPL> r;
    if constexpr (DPL == 4) {
        const float4 x = *reinterpret_cast<const float4 *>(p);
        r.v[0] = x.x;
        r.v[1] = x.y;
        r.v[2] = x.z;
        r.v[3] = x.w;
    } else if constexpr (DPL == 2) {
        const float2 x = *reinterpret_cast<const float2 *>(p);
        r.v[0] = x.x;
        r.v[1] = x.y;
    } else {
        r.v[0] = p[0];
    }
    return r;
}

// Threads of the attention workgroup over a batch's slices (16 per sequence): eight waves.
// Measured on the Gemma-3-1B step with 16 sequences: 1.543 ms per step against 1.576 ms with
// four waves (one per SIMD, every dependent step of the position loop exposed) and 1.586 ms
// with sixteen (four positions in flight per wave to fit 128 VGPRs).
constexpr int kAttnThreadsBatch = 512;

// Workgroup b takes positions [t0, t1) of the layer's attention range; each of its NT / 64
// waves walks every (NT / 64)-th of them with a running (max, sum, weighted V) per head; the waves are then
// merged and the slice's partial stored. Lane l owns dims [l*DPL, l*DPL + DPL). Scores are
// summed by DPP into wave-uniform values and the weights are powers of two of log2-scaled
// scores (one exp2 each). NKV: the K/V heads (1 or 2, a.nkv).
template <int DPL, int NH, int NKV, int NT>
__global__ __launch_bounds__(NT) void dec_attn_part_kernel(AttnArgs a) {
    {   // sequence blockIdx.y of a batch
        const size_t b = blockIdx.y;
        a.qkv += b * a.qkv_stride;
        a.kc += b * a.kv_stride;
        a.vc += b * a.kv_stride;
        a.d_pos += b;
        if (a.d_done) a.d_done += b;
        a.part += b * (size_t)gridDim.x * NH * (a.hd + 2);
    }
    __shared__ float raw[kAttnMaxQ + 2 * kAttnMaxKV];   // q | k | v as projected
    __shared__ float qs[kAttnMaxQ];
    __shared__ float ks[kAttnMaxKV];
    __shared__ float part8[8 * 16];
    __shared__ float ss[16];
    __shared__ float wm[NT / kWave][NH], wsum[NT / kWave][NH];
    __shared__ float wo[NT / kWave][NH][kWave * DPL];
    __shared__ float wx[NT / kWave][NH];   // wave merge weights
    __shared__ float wmax[NH], wtot[NH];
    const int hd = a.hd, half = hd / 2;
    constexpr int nkv = NKV;
    // Loads that wait for nothing go out first: q | k | v as projected and the QK-norm gammas
    // (thread t applies the norm and RoPE to pair i = t mod hd/2 of every head, the same i for
    // every head as NT is a multiple of hd/2).
    constexpr int kRawRegs = (kAttnMaxQ + 2 * kAttnMaxKV) / NT;
    const int nraw = (NH + 2 * nkv) * hd;
    float rv[kRawRegs];
#pragma unroll
    for (int e = 0; e < kRawRegs; ++e) {
        const int i = threadIdx.x + e * NT;
        rv[e] = i < nraw ? a.qkv[i] : 0.f;
    }
    const int pi = threadIdx.x % half;
    const float gq0 = a.qn[pi], gq1 = a.qn[pi + half], gk0 = a.kn[pi], gk1 = a.kn[pi + half];
    const int pos = *a.d_pos, seq = pos + 1;
    const float rc = a.cos_t[(size_t)pos * hd + pi], rs = a.sin_t[(size_t)pos * hd + pi];
    const int start = (a.window > 0 && seq > a.window) ? seq - a.window : 0;
    const int len = seq - start, nsplit = gridDim.x;
    const int chunk = (len + nsplit - 1) / nsplit;
    const int t0 = start + blockIdx.x * chunk, t1 = min(seq, t0 + chunk);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    constexpr int group = NH / NKV;
    // The wave's positions t0 + wid + 4j, PF at a time. The rows of the next batch are loaded
    // while the current one is used (two register sets). Rows come from the cache; the row of
    // the current position is taken from this kernel's own K (after RoPE) and V.
    constexpr int PF = 8 / NKV;
    constexpr int NW = NT / kWave;
    float kr[PF][NKV][DPL], vr[PF][NKV][DPL];
    float nk[PF][NKV][DPL], nv[PF][NKV][DPL];   // the next batch
    // A row outside the slice (or the current position's) reads row 0 instead, in bounds, and
    // is dropped: every row is one vector load per lane.
    auto load_batch = [&](int tb, float(&K)[PF][NKV][DPL], float(&V)[PF][NKV][DPL]) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int t = tb + j * NW;
#pragma unroll
            for (int hk = 0; hk < NKV; ++hk) {
                const bool ok = t < t1 && t != pos;
                const size_t off = (ok ? ((size_t)hk * a.max_ctx + t) * hd : 0) + lane * DPL;
                const Lanes<DPL> kv = load_lanes<DPL>(a.kc + off);
                const Lanes<DPL> vv = load_lanes<DPL>(a.vc + off);
#pragma unroll
                for (int d = 0; d < DPL; ++d) {
                    K[j][hk][d] = ok ? kv.v[d] : 0.f;
                    V[j][hk][d] = ok ? vv.v[d] : 0.f;
                }
            }
        }
    };
    if (t0 + wid < t1) load_batch(t0 + wid, kr, vr);   // in flight during the prologue

#pragma unroll
    for (int e = 0; e < kRawRegs; ++e) {
        const int i = threadIdx.x + e * NT;
        if (i < nraw) raw[i] = rv[e];
    }
    __syncthreads();
    // QK-norm and RoPE of the query heads and the K heads in one pass: per head the
    // arithmetic of norm_rope_heads (the sums of squares of every head at once)
    vectors_sum_sq(raw, NH + nkv, hd, part8, ss);
    if (threadIdx.x < NH + nkv) ss[threadIdx.x] = rms_inv_of(ss[threadIdx.x], hd, a.eps);
    __syncthreads();
    for (int v = threadIdx.x / half; v < NH + nkv; v += NT / half) {
        const bool isq = v < NH;
        const float r = ss[v], g0 = isq ? gq0 : gk0, g1 = isq ? gq1 : gk1;
        const float *p = raw + (size_t)v * hd;
        const float x0 = __fmul_rn(__fmul_rn(p[pi], r), __fadd_rn(1.0f, g0));
        const float x1 = __fmul_rn(__fmul_rn(p[pi + half], r), __fadd_rn(1.0f, g1));
        float *dst = isq ? qs + v * hd : ks + (v - NH) * hd;
        dst[pi] = __builtin_fmaf(x0, rc, -__fmul_rn(x1, rs));
        dst[pi + half] = __builtin_fmaf(x1, rc, __fmul_rn(x0, rs));
    }
    __syncthreads();
    const float *vnew = raw + (NH + nkv) * hd;
    // kv_cache_write_token: [head][pos][dim] (a stopped sequence writes none)
    if (blockIdx.x == 0 && !a.kv_written && !(a.d_done && *a.d_done))
        for (int i = threadIdx.x; i < nkv * hd; i += blockDim.x) {
            const int h = i / hd, d = i - h * hd;
            const size_t off = ((size_t)h * a.max_ctx + pos) * hd + d;
            a.kc[off] = ks[i];
            a.vc[off] = vnew[i];
        }

    // scores in log2 units, so that every softmax weight is one exp2 (v_exp_f32); the
    // partial's maximum is stored in these units
    const float sl2 = __fmul_rn(a.scale, 1.44269504088896341f);
    float m[NH], s[NH], o[NH][DPL];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        m[h] = -INFINITY;
        s[h] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[h][d] = 0.f;
    }
    float qr[NH][DPL];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int d = 0; d < DPL; ++d) qr[h][d] = qs[h * hd + lane * DPL + d];
    // positions whose scores are formed together (independent wave sums), then one rescale per
    // head: the running maximum moves to the largest score of the group
    constexpr int SB = 32 / NH < PF ? 32 / NH : PF;
    for (int tb = t0 + wid; tb < t1; tb += PF * NW) {
        const int tn = tb + PF * NW;
        if (tn < t1) load_batch(tn, nk, nv);
        const int nj = min(PF, (t1 - tb + NW - 1) / NW);      // positions of this batch in the slice
#pragma unroll
        for (int j = 0; j < PF; ++j)
            if (j < nj && tb + j * NW == pos) {
#pragma unroll
                for (int hk = 0; hk < NKV; ++hk)
#pragma unroll
                    for (int d = 0; d < DPL; ++d) {
                        kr[j][hk][d] = ks[hk * hd + lane * DPL + d];
                        vr[j][hk][d] = vnew[hk * hd + lane * DPL + d];
                    }
            }
#pragma unroll
        for (int j0 = 0; j0 < PF; j0 += SB) {
            if (j0 >= nj) break;
            float sc[SB][NH];
#pragma unroll
            for (int jj = 0; jj < SB; ++jj)
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    const int hk = h / group;
                    float dp = 0.f;
#pragma unroll
                    for (int d = 0; d < DPL; ++d) dp = __builtin_fmaf(qr[h][d], kr[j0 + jj][hk][d], dp);
                    sc[jj][h] = j0 + jj < nj ? __fmul_rn(lanes::wave_sum(dp), sl2) : -INFINITY;
                }
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int hk = h / group;
                float mb = sc[0][h];
#pragma unroll
                for (int jj = 1; jj < SB; ++jj) mb = fmaxf(mb, sc[jj][h]);
                const float mn = fmaxf(m[h], mb);
                const float c = m[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[h] - mn);
                s[h] = __fmul_rn(s[h], c);
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[h][d] = __fmul_rn(o[h][d], c);
#pragma unroll
                for (int jj = 0; jj < SB; ++jj)
                    if (j0 + jj < nj) {
                        const float p = __builtin_amdgcn_exp2f(sc[jj][h] - mn);
                        s[h] = __fadd_rn(s[h], p);
#pragma unroll
                        for (int d = 0; d < DPL; ++d) o[h][d] = __builtin_fmaf(p, vr[j0 + jj][hk][d], o[h][d]);
                    }
                m[h] = mn;
            }
        }
        if (tn < t1) {
#pragma unroll
            for (int j = 0; j < PF; ++j)
#pragma unroll
                for (int hk = 0; hk < NKV; ++hk)
#pragma unroll
                    for (int d = 0; d < DPL; ++d) {
                        kr[j][hk][d] = nk[j][hk][d];
                        vr[j][hk][d] = nv[j][hk][d];
                    }
        }
    }
    // merge the four waves: the (wave, head) weights exp2(m_w - M) are formed once
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
    if (threadIdx.x < NH) {
        const int h = threadIdx.x;
        float M = -INFINITY;
        for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][h]);
        float S = 0.f;
        for (int w = 0; w < NW; ++w) {
            const float e = wm[w][h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm[w][h] - M);
            wx[w][h] = e;
            S = __builtin_fmaf(wsum[w][h], e, S);
        }
        wmax[h] = M;
        wtot[h] = S;
    }
    __syncthreads();
    float *out = a.part + (size_t)blockIdx.x * NH * (hd + 2);
    for (int idx = threadIdx.x; idx < NH * hd; idx += blockDim.x) {
        const int h = idx / hd, d = idx - h * hd;
        float O = 0.f;
        for (int w = 0; w < NW; ++w) O = __builtin_fmaf(wo[w][h][d], wx[w][h], O);
        out[h * (hd + 2) + d] = O;
        if (d == 0) {
            out[h * (hd + 2) + hd] = wmax[h];
            out[h * (hd + 2) + hd + 1] = wtot[h];
        }
    }
}

// The batch form with the K/V rows in LDS. A slice's rows go into LDS by DMA as soon as the
// position is known, before this token's q/k/v are used, so the whole slice (up to PB
// positions, 144 KiB) is in flight at once without holding it in registers; one workgroup per
// CU. Wave w takes positions rb + w + 8j of a round [rb, rb + PB) and loads exactly those rows,
// so it waits for its own DMA only; a slice longer than PB takes further rounds in the same
// slots. Arithmetic and order are those of dec_attn_part_kernel.
// PBMAX caps the positions per round (the LDS of a workgroup that shares its CU).
template <int DPL, int NH, int NKV, int PBMAX = 72>
struct AttnLdsShape {
    static constexpr int NT = kAttnThreadsBatch, NW = NT / kWave, HD = kWave * DPL;
    // raw q|k|v, the normed q and k, and (within 2 KiB) the small merge arrays
    static constexpr int kFixed = (2 * NH + 3 * NKV) * HD * 4 + 2048;
    static constexpr int kRoom = (160 * 1024 - kFixed) / (2 * NKV * HD * 4) / NW * NW;
    static constexpr int PB = kRoom < PBMAX ? kRoom : PBMAX;   // positions per round
    static_assert(PB >= NW, "at least one row per wave and round");
    static_assert(NW * NH <= 2 * PB * NKV, "the wave merge fits in the row space");
};

template <int DPL, int NH, int NKV, int PBMAX = 72>
struct AttnLds {
    using S = AttnLdsShape<DPL, NH, NKV, PBMAX>;
    alignas(16) float kvr[2][S::PB * NKV][S::HD];   // K rows | V rows of a round
    float raw[(NH + 2 * NKV) * S::HD];              // q | k | v as projected
    float qs[NH * S::HD];
    float ks[NKV * S::HD];
    float part8[8 * 16];
    float ss[16];
    float wm[S::NW][NH], wsum[S::NW][NH], wx[S::NW][NH];
    float wmax[NH], wtot[NH];
};

// Where a batch attention workgroup takes q | k | v from: a.qkv (written by an earlier
// launch), or epoch-tagged words that a GEMM in the same launch writes (words of sequence b at
// w + b * stride, polled until their tag equals `tag`; a wait longer than spin_limit polls
// counts in *err and goes on with what it has).
struct QkvTagged {
    const uint64_t *w = nullptr;
    size_t stride = 0;
    uint32_t tag = 0;
    int spin_limit = 0;
    int *err = nullptr;
};

// Slice bx of sequence by (gdx slices per sequence), with its LDS in L.
template <int DPL, int NH, int NKV, int PBMAX>
__device__ __forceinline__ void attn_lds_body(AttnLds<DPL, NH, NKV, PBMAX> &L, int bx, int by, int gdx, AttnArgs a,
                                              const QkvTagged &tq) {
    using S = AttnLdsShape<DPL, NH, NKV, PBMAX>;
    constexpr int NT = S::NT, NW = S::NW, HD = S::HD, PB = S::PB, PW = PB / NW;
    {   // sequence by of a batch
        const size_t b = by;
        a.qkv += b * a.qkv_stride;
        a.kc += b * a.kv_stride;
        a.vc += b * a.kv_stride;
        a.d_pos += b;
        if (a.d_done) a.d_done += b;
        a.part += b * (size_t)gdx * NH * (HD + 2);
    }
    auto &kvr = L.kvr;
    float *raw = L.raw, *qs = L.qs, *ks = L.ks, *part8 = L.part8, *ss = L.ss;
    auto &wm = L.wm;
    auto &wsum = L.wsum;
    auto &wx = L.wx;
    float *wmax = L.wmax, *wtot = L.wtot;
    constexpr int half = HD / 2, group = NH / NKV;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int wu = __builtin_amdgcn_readfirstlane(wid);
    // q | k | v and the QK-norm gammas wait for nothing (thread t takes pair i = t mod hd/2 of
    // every head)
    constexpr int nraw = (NH + 2 * NKV) * HD;
    constexpr int kRawRegs = (nraw + NT - 1) / NT;
    float rv[kRawRegs];
    if (!tq.w)
#pragma unroll
        for (int e = 0; e < kRawRegs; ++e) {
            const int i = threadIdx.x + e * NT;
            rv[e] = i < nraw ? a.qkv[i] : 0.f;
        }
    const int pi = threadIdx.x % half;
    const float gq0 = a.qn[pi], gq1 = a.qn[pi + half], gk0 = a.kn[pi], gk1 = a.kn[pi + half];
    const int pos = *a.d_pos, seq = pos + 1;
    const float rc = a.cos_t[(size_t)pos * HD + pi], rs = a.sin_t[(size_t)pos * HD + pi];
    const int start = (a.window > 0 && seq > a.window) ? seq - a.window : 0;
    const int len = seq - start, nsplit = gdx;
    const int chunk = (len + nsplit - 1) / nsplit;
    const int t0 = start + bx * chunk, t1 = min(seq, t0 + chunk);
    // this wave's rows of the round from rb into its own slots wu + NW j; the current
    // position's row is this kernel's own k and v
    auto issue = [&](int rb) {
        const int re = min(t1, rb + PB);
#pragma unroll
        for (int j = 0; j < PW; ++j) {
            const int t = rb + wu + NW * j;
            if (t < re && t != pos)
#pragma unroll
                for (int hk = 0; hk < NKV; ++hk) {
                    const size_t off = ((size_t)hk * a.max_ctx + t) * HD;
                    row_to_lds<DPL>(a.kc + off, kvr[0][(wu + NW * j) * NKV + hk]);
                    row_to_lds<DPL>(a.vc + off, kvr[1][(wu + NW * j) * NKV + hk]);
                }
        }
    };
    issue(t0);
    if (tq.w) {
        // the GEMM's words, polled behind the rows' DMA (whose loads the GEMM's run outlasts).
        // Until one word of this wave's share carries the tag, only one lane per wave polls
        // (the GEMM's workgroups share the CUs); then every thread loads its words.
        const uint64_t *src = tq.w + (size_t)by * tq.stride;
        if (lane == 0) {
            const uint64_t *sw = src + wu * (nraw / NW);
            for (int spins = 0; spins < tq.spin_limit; ++spins) {
                if ((uint32_t)(__hip_atomic_load(sw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32) == tq.tag)
                    break;
                __builtin_amdgcn_s_sleep(8);
            }
        }
        uint64_t w[kRawRegs];
#pragma unroll
        for (int e = 0; e < kRawRegs; ++e) {
            const int i = threadIdx.x + e * NT;
            w[e] = i < nraw ? __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : (uint64_t)tq.tag << 32;
        }
        for (int spins = 0;; ++spins) {
            bool ready = true;
#pragma unroll
            for (int e = 0; e < kRawRegs; ++e) ready = ready && (uint32_t)(w[e] >> 32) == tq.tag;
            if (ready) break;
            if (spins >= tq.spin_limit) {
                atomicAdd(tq.err, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
#pragma unroll
            for (int e = 0; e < kRawRegs; ++e) {
                const int i = threadIdx.x + e * NT;
                if (i < nraw && (uint32_t)(w[e] >> 32) != tq.tag)
                    w[e] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
#pragma unroll
        for (int e = 0; e < kRawRegs; ++e) rv[e] = __uint_as_float((uint32_t)w[e]);
    }

#pragma unroll
    for (int e = 0; e < kRawRegs; ++e) {
        const int i = threadIdx.x + e * NT;
        if (i < nraw) raw[i] = rv[e];
    }
    __syncthreads();
    // QK-norm and RoPE of the query heads and the K heads in one pass (norm_rope_heads'
    // arithmetic)
    vectors_sum_sq(raw, NH + NKV, HD, part8, ss);
    if (threadIdx.x < NH + NKV) ss[threadIdx.x] = rms_inv_of(ss[threadIdx.x], HD, a.eps);
    __syncthreads();
    for (int v = threadIdx.x / half; v < NH + NKV; v += NT / half) {
        const bool isq = v < NH;
        const float r = ss[v], g0 = isq ? gq0 : gk0, g1 = isq ? gq1 : gk1;
        const float *p = raw + (size_t)v * HD;
        const float x0 = __fmul_rn(__fmul_rn(p[pi], r), __fadd_rn(1.0f, g0));
        const float x1 = __fmul_rn(__fmul_rn(p[pi + half], r), __fadd_rn(1.0f, g1));
        float *dst = isq ? qs + v * HD : ks + (v - NH) * HD;
        dst[pi] = __builtin_fmaf(x0, rc, -__fmul_rn(x1, rs));
        dst[pi + half] = __builtin_fmaf(x1, rc, __fmul_rn(x0, rs));
    }
    __syncthreads();
    const float *vnew = raw + (NH + NKV) * HD;
    // kv_cache_write_token: [head][pos][dim] (a stopped sequence writes none)
    if (bx == 0 && !a.kv_written && !(a.d_done && *a.d_done))
        for (int i = threadIdx.x; i < NKV * HD; i += NT) {
            const int h = i / HD, d = i - h * HD;
            const size_t off = ((size_t)h * a.max_ctx + pos) * HD + d;
            a.kc[off] = ks[i];
            a.vc[off] = vnew[i];
        }

    const float sl2 = __fmul_rn(a.scale, 1.44269504088896341f);
    float m[NH], s[NH], o[NH][DPL], qr[NH][DPL];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        m[h] = -INFINITY;
        s[h] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            o[h][d] = 0.f;
            qr[h][d] = qs[h * HD + lane * DPL + d];
        }
    }
    constexpr int SB = 32 / NH < PW ? 32 / NH : PW;
    for (int rb = t0; rb < t1; rb += PB) {
        if (rb != t0) issue(rb);                       // the slots' previous rows are all read
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const int re = min(t1, rb + PB);
        const int nj = min(PW, max(0, (re - rb - wu + NW - 1) / NW));   // this wave's positions
#pragma unroll
        for (int j0 = 0; j0 < PW; j0 += SB) {
            if (j0 >= nj) break;
            float sc[SB][NH];
#pragma unroll
            for (int jj = 0; jj < SB; ++jj) {
                const int j = j0 + jj < PW ? j0 + jj : PW - 1;
                const bool cur = rb + wu + NW * j == pos;
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    const int hk = h / group;
                    const float *kp = cur ? ks + hk * HD : kvr[0][(wu + NW * j) * NKV + hk];
                    float dp = 0.f;
#pragma unroll
                    for (int d = 0; d < DPL; ++d) dp = __builtin_fmaf(qr[h][d], kp[lane * DPL + d], dp);
                    sc[jj][h] = j0 + jj < nj ? __fmul_rn(lanes::wave_sum(dp), sl2) : -INFINITY;
                }
            }
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int hk = h / group;
                float mb = sc[0][h];
#pragma unroll
                for (int jj = 1; jj < SB; ++jj) mb = fmaxf(mb, sc[jj][h]);
                const float mn = fmaxf(m[h], mb);
                const float c = m[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[h] - mn);
                s[h] = __fmul_rn(s[h], c);
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[h][d] = __fmul_rn(o[h][d], c);
#pragma unroll
                for (int jj = 0; jj < SB; ++jj)
                    if (j0 + jj < nj) {
                        const int j = j0 + jj;
                        const bool cur = rb + wu + NW * j == pos;
                        const float *vp = cur ? vnew + hk * HD : kvr[1][(wu + NW * j) * NKV + hk];
                        const float p = __builtin_amdgcn_exp2f(sc[jj][h] - mn);
                        s[h] = __fadd_rn(s[h], p);
#pragma unroll
                        for (int d = 0; d < DPL; ++d) o[h][d] = __builtin_fmaf(p, vp[lane * DPL + d], o[h][d]);
                    }
                m[h] = mn;
            }
        }
    }
    // merge the waves (their rows are no longer read: the merge takes their space)
    __syncthreads();
    float *wo = &kvr[0][0][0];                         // [NW][NH][HD]
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        if (lane == 0) {
            wm[wid][h] = m[h];
            wsum[wid][h] = s[h];
        }
#pragma unroll
        for (int d = 0; d < DPL; ++d) wo[(wid * NH + h) * HD + lane * DPL + d] = o[h][d];
    }
    __syncthreads();
    if (threadIdx.x < NH) {
        const int h = threadIdx.x;
        float M = -INFINITY;
        for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][h]);
        float Ssum = 0.f;
        for (int w = 0; w < NW; ++w) {
            const float e = wm[w][h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm[w][h] - M);
            wx[w][h] = e;
            Ssum = __builtin_fmaf(wsum[w][h], e, Ssum);
        }
        wmax[h] = M;
        wtot[h] = Ssum;
    }
    __syncthreads();
    float *out = a.part + (size_t)bx * NH * (HD + 2);
    for (int idx = threadIdx.x; idx < NH * HD; idx += NT) {
        const int h = idx / HD, d = idx - h * HD;
        float O = 0.f;
        for (int w = 0; w < NW; ++w) O = __builtin_fmaf(wo[(w * NH + h) * HD + d], wx[w][h], O);
        out[h * (HD + 2) + d] = O;
        if (d == 0) {
            out[h * (HD + 2) + HD] = wmax[h];
            out[h * (HD + 2) + HD + 1] = wtot[h];
        }
    }
}

template <int DPL, int NH, int NKV>
__global__ __launch_bounds__(kAttnThreadsBatch) void dec_attn_lds_kernel(AttnArgs a) {
    __shared__ AttnLds<DPL, NH, NKV> L;
    attn_lds_body<DPL, NH, NKV, 72>(L, blockIdx.x, blockIdx.y, gridDim.x, a, QkvTagged{});
}

// ---- the QKV GEMM and the attention partials of a batched step in one launch ----

constexpr int kQkvAttnRows = 32;   // K/V positions per round of a fused attention workgroup (~75 KiB LDS)

struct QkvAttnArgs {
    GemmPlan P;                  // the QKV GEMM (prepared input, one K chunk, 8-wave workgroups)
    GemmIn in;
    GemmOut out;                 // rows as tagged words: out.tagged, out.ldy
    AttnArgs at;
    int ns = 0;                  // attention slices per sequence
    const uint32_t *epoch = nullptr;   // the batched step counter that makes the tags unique
    int layer = 0;
    int spin_limit = 0;
    int *err = nullptr;
};

// Workgroups [0, P.gx) run the QKV GEMM (its rows stored as words tagged with this step and
// layer), the rest the attention partials of (slice, sequence), which bring their K/V rows
// into LDS while the GEMM runs and then poll for their sequence's q | k | v words. The GEMM's
// workgroups come first in dispatch order and wait for nothing, so the launch completes even
// when not every workgroup is resident; the union keeps both roles at two workgroups per CU.
template <int DT, int DPL, int NH, int NKV>
__global__ __launch_bounds__(kAttnThreadsBatch) __attribute__((amdgpu_waves_per_eu(4))) void dec_qkv_attn_kernel(
    QkvAttnArgs q) {
    __shared__ union Lds {
        gemmb::GemmLds<gemmb::kWaves> g;
        AttnLds<DPL, NH, NKV, kQkvAttnRows> a;
    } L;
    // the step counter by a vector load: a scalar one would share lgkmcnt with the LDS
    // accesses of the staging, whose every wait would then wait for it too
    const uint32_t tag = (__hip_atomic_load(q.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) << 6) +
                         (uint32_t)q.layer + 1u;
    const int ng = q.P.gx;
    if ((int)blockIdx.x < ng) {
        GemmOut o = q.out;
        o.tag = tag;
        gemmb::gemm_body<DT, gemmb::kStagePrepared, gemmb::kWaves, false>(
            L.g, blockIdx.x, 0, ng, 1, q.P.wq, q.P.q_bytes, q.P.wsc, q.P.s_bytes, q.in, q.P.batch, q.P.M, q.P.K,
            q.P.cb, o, q.P.Yp, static_cast<const gemmb::PrepChunk *>(q.P.prep), q.P.ks);
    } else {
        const int w = (int)blockIdx.x - ng;
        QkvTagged t;
        t.w = q.out.tagged;
        t.stride = (size_t)q.out.ldy;
        t.tag = tag;
        t.spin_limit = q.spin_limit;
        t.err = q.err;
        attn_lds_body<DPL, NH, NKV, kQkvAttnRows>(L.a, w % q.ns, w / q.ns, q.ns, q.at, t);
    }
}

// out[h*hd + d] = sum_b e_b o_b[d] / sum_b e_b s_b with e_b = exp2(m_b - max_b m_b) (the
// partials' maxima are in log2 units): the softmax-weighted sum of values of
// attention.c:140-158 over all slices. One workgroup per head, one thread per dim. Every load
// goes out at once: each wave forms the slice weights itself (lane b holds slice b's maximum
// and sum), so no load waits for another.
template <int NS>
__global__ __launch_bounds__(kThreads) void dec_attn_combine_kernel(const float *__restrict__ part, int nh, int hd,
                                                                    float *__restrict__ out, size_t out_stride,
                                                                    bool blocked) {
    static_assert(NS <= kWave, "one lane per slice");
    const int h = blockIdx.x, t = threadIdx.x, lane = t & (kWave - 1);
    part += (size_t)blockIdx.y * NS * nh * (hd + 2);   // sequence blockIdx.y
    if (!blocked) out += (size_t)blockIdx.y * out_stride;
    const size_t hs = (size_t)nh * (hd + 2);             // stride between slices
    const float *ph = part + (size_t)h * (hd + 2);
    const float mb = lane < NS ? ph[lane * hs + hd] : -INFINITY;
    const float sb = lane < NS ? ph[lane * hs + hd + 1] : 0.f;
    float o[NS];
    const int d = t;                                     // head_dim <= 256 = one dim per thread
#pragma unroll
    for (int b = 0; b < NS; ++b) o[b] = d < hd ? ph[b * hs + d] : 0.f;
    const float M = lanes::wave_max(mb);
    const float e = mb == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mb - M);
    const float inv = 1.0f / lanes::wave_sum(e * sb);
    float O = 0.f;
#pragma unroll
    for (int b = 0; b < NS; ++b) O = __builtin_fmaf(o[b], lane_value(e, b), O);
    if (d < hd) out[blocked ? block_order_index(blockIdx.y, h * hd + d) : (size_t)h * hd + d] = O * inv;
}

__global__ void dec_embed_kernel(const uint16_t *__restrict__ embed, int hidden, int vocab, float es,
                                 const int *__restrict__ tok, float *__restrict__ resid) {
    const size_t row = embed_row(*tok, vocab, hidden);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
        const float v = __uint_as_float((uint32_t)embed[row + i] << 16);
        resid[i] = es != 1.0f ? __fmul_rn(v, es) : v;
    }
}

__global__ void dec_advance_kernel(const int *__restrict__ tok, int *__restrict__ pos, int *__restrict__ step,
                                   int *__restrict__ log, uint32_t *__restrict__ seq, int *__restrict__ done,
                                   StopSet stop) {
    if (threadIdx.x == 0 && blockIdx.x == 0 && !(done && *done)) {
        const int s = *step, t = *tok;
        log[s] = t;
        *step = s + 1;
        *pos = *pos + 1;
        if (seq) *seq = *seq + 1u;
        if (done && stop.has(t)) *done = 1;   // inference.c:298-301
    }
}

// ---- batched decode: embedding, greedy token and position of a batch of sequences ----

__global__ void dec_embed_batch_kernel(const uint16_t *__restrict__ embed, int hidden, int vocab, float es,
                                       const int *__restrict__ tok, float *__restrict__ resid) {
    const size_t row = embed_row(tok[blockIdx.y], vocab, hidden);
    float *out = resid + (size_t)blockIdx.y * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
        const float v = __uint_as_float((uint32_t)embed[row + i] << 16);
        out[i] = es != 1.0f ? __fmul_rn(v, es) : v;
    }
}

constexpr int kArgmaxParts = 64;     // workgroups per sequence in the first argmax pass

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return greedy_better(v, i, bv, bi); }

__device__ __forceinline__ void wave_best(float &v, int &i) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, kWave);
        const int oi = __shfl_xor(i, off, kWave);
        if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
}

// grid (kArgmaxParts, batch): part[b][p] = best (value, index) of slice p of logits[b]
__global__ __launch_bounds__(kThreads) void dec_argmax_part_kernel(const float *__restrict__ logits, int n,
                                                                   float *__restrict__ part) {
    __shared__ float sv[kThreads / kWave];
    __shared__ int si[kThreads / kWave];
    const float *x = logits + (size_t)blockIdx.y * n;
    const int chunk = (n + gridDim.x - 1) / gridDim.x;
    const int i0 = blockIdx.x * chunk, i1 = min(n, i0 + chunk);
    float bv = -INFINITY;
    int bi = n;
    for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
        const float v = x[i];
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    wave_best(bv, bi);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) { sv[wid] = bv; si[wid] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / kWave; ++w)
            if (better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
        float *o = part + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 2;
        o[0] = bv;
        o[1] = __int_as_float(bi);
    }
}

// grid (batch), one wave: tokens[b] = best of the sequence's partials; 0 when logits[b][0] is
// NaN or no logit is above -inf, as sample_greedy (utils.c:145-156) starts at index 0 and
// only a greater logit replaces it
__global__ void dec_argmax_finish_kernel(const float *__restrict__ part, int nparts, int n,
                                         const float *__restrict__ logits, int *__restrict__ tokens) {
    const float *p = part + (size_t)blockIdx.x * nparts * 2;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int j = threadIdx.x; j < nparts; j += kWave) {
        const float v = p[2 * j];
        const int i = __float_as_int(p[2 * j + 1]);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    wave_best(bv, bi);
    if (threadIdx.x == 0)
        tokens[blockIdx.x] = (bi >= 0 && bi < n && !isnan(logits[(size_t)blockIdx.x * n])) ? bi : 0;
}

__global__ void dec_advance_batch_kernel(const int *__restrict__ tok, int *__restrict__ pos, int *__restrict__ step,
                                         int batch, int *__restrict__ log, int *__restrict__ done, StopSet stop,
                                         uint32_t *__restrict__ epoch) {
    const int s = *step;
    for (int b = threadIdx.x; b < batch; b += blockDim.x) {
        if (done && done[b]) continue;       // a stopped sequence: its entry keeps the fill
        const int t = tok[b];
        log[(size_t)s * batch + b] = t;
        pos[b] = pos[b] + 1;
        if (done && stop.has(t)) done[b] = 1;   // inference.c:298-301
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        *step = s + 1;
        if (epoch) *epoch = *epoch + 1u;
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
    const int blocks = (wsteps + 3) / 4;   // one wave-step per wave
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

int dec_prologue_batch(const GemvIn &in, int K, int batch, size_t stride, float *out, hipStream_t s) {
    if (K > kDecMaxK || batch <= 0 || in.resid_out) {
        set_error("batched prologue: %d floats (at most %d), %d sequences, no residual output", K, kDecMaxK, batch);
        return -1;
    }
    hipLaunchKernelGGL(dec_prologue_kernel, dim3(1, batch), dim3(kThreads), 0, s, in, K, out, stride);
    return hip_ok(hipGetLastError(), "dec_prologue launch") ? 0 : -1;
}

int dec_prologue_only(const GemvIn &in, int K, float *out, hipStream_t s) {
    if (K > kDecMaxK) {
        set_error("vector of %d floats exceeds %d", K, kDecMaxK);
        return -1;
    }
    hipLaunchKernelGGL(dec_prologue_kernel, dim3(1), dim3(kThreads), 0, s, in, K, out, (size_t)0);
    return hip_ok(hipGetLastError(), "dec_prologue launch") ? 0 : -1;
}

size_t attn_part_floats(int nh, int hd) { return (size_t)kAttnSplit * nh * (hd + 2); }

int dec_attention(const AttnArgs &a, float *out, hipStream_t s) {
    if (a.nh * a.hd > kAttnMaxQ || a.nkv * a.hd > kAttnMaxKV || a.nkv <= 0 || a.nkv > 2 || a.nh % a.nkv != 0 ||
        a.hd % kWave != 0 || a.hd > 4 * kWave || a.nh + a.nkv > 16 || a.batch < 1 || a.batch > 65535 ||
        (a.out_blocked && a.batch > kGemmSeqs)) {
        set_error("attention shape not supported (heads %d/%d, head_dim %d)", a.nh, a.nkv, a.hd);
        return -1;
    }
    const int dpl = a.hd / kWave;
    // splits per sequence: enough workgroups in total, without cutting a sequence's positions
    // into slivers once a batch fills the GPU
    const int ns = a.batch >= 4 ? kAttnSplitBatch : kAttnSplit;
    // a batch's slices are longer: eight waves per workgroup walk them (one wave per SIMD would
    // expose every dependent step of the position loop)
    const bool wide = ns == kAttnSplitBatch;
#define SPH_ATTN(DPLV, NHV, NKVV)                                                                              \
    if (dpl == DPLV && a.nh == NHV && a.nkv == NKVV) {                                                         \
        if (wide)                                                                                              \
            hipLaunchKernelGGL((dec_attn_lds_kernel<DPLV, NHV, NKVV>), dim3(ns, a.batch),                          \
                               dim3(kAttnThreadsBatch), 0, s, a);                                               \
        else                                                                                                   \
            hipLaunchKernelGGL((dec_attn_part_kernel<DPLV, NHV, NKVV, kThreads>), dim3(ns, a.batch),             \
                               dim3(kThreads), 0, s, a);                                                        \
    } else
    SPH_ATTN(1, 4, 1) SPH_ATTN(2, 4, 1) SPH_ATTN(4, 4, 1) SPH_ATTN(1, 8, 1) SPH_ATTN(2, 8, 1) SPH_ATTN(4, 8, 1)
    SPH_ATTN(1, 4, 2) SPH_ATTN(2, 4, 2) SPH_ATTN(4, 4, 2) SPH_ATTN(1, 8, 2) SPH_ATTN(2, 8, 2) SPH_ATTN(4, 8, 2) {
        set_error("attention with %d heads of dim %d not instantiated", a.nh, a.hd);
        return -1;
    }
#undef SPH_ATTN
    if (!hip_ok(hipGetLastError(), "attention launch")) return -1;
    if (ns == kAttnSplit)
        hipLaunchKernelGGL(dec_attn_combine_kernel<kAttnSplit>, dim3(a.nh, a.batch), dim3(kThreads), 0, s, a.part,
                           a.nh, a.hd, out, a.out_stride, a.out_blocked);
    else
        hipLaunchKernelGGL(dec_attn_combine_kernel<kAttnSplitBatch>, dim3(a.nh, a.batch), dim3(kThreads), 0, s,
                           a.part, a.nh, a.hd, out, a.out_stride, a.out_blocked);
    return hip_ok(hipGetLastError(), "attention combine launch") ? 0 : -1;
}

// The fused form is instantiated where both roles fit two workgroups per CU (LDS <= 80 KiB,
// <= 128 VGPRs, no scratch): Q4_0 weights, head_dim 64 or 128 with 4 or 8 query heads and 1 or
// 2 K/V heads, or head_dim 256 with 4 query heads and one K/V head (the Gemma-3 shapes). Q8_0's
// larger weight units and the larger attention shapes spill; they keep two launches.
bool qkv_attention_fusable(int dt, int K, const AttnArgs &a) {
    const int dpl = a.hd / kWave;
    const bool shape = a.hd % kWave == 0 && (((dpl == 1 || dpl == 2) && (a.nh == 4 || a.nh == 8) &&
                                              (a.nkv == 1 || a.nkv == 2)) ||
                                             (dpl == 4 && a.nh == 4 && a.nkv == 1));
    return dt == DT_Q4_0 && shape && a.batch >= 4 && a.batch <= kGemmSeqs && a.nh % a.nkv == 0 && !a.kv_written &&
           a.out_blocked && gemm_splits(K) == 1;
}

int dec_qkv_attention(int dt, const void *w, int M, int K, const GemmIn &in, void *ws, uint64_t *tagged,
                      const AttnArgs &a, const uint32_t *epoch, int layer, int spin_limit, int *err, float *out,
                      hipStream_t s) {
    // the tags are (step counter << 6) + layer + 1, so at most 63 layers
    if (!qkv_attention_fusable(dt, K, a) || !tagged || !epoch || !err || layer < 0 || layer > 62) {
        set_error("fused QKV + attention: unsupported shape");
        return -1;
    }
    QkvAttnArgs q;
    if (plan_gemm_tiled(dt, w, M, K, a.batch, in, ws, s, &q.P) != 0) return -1;
    if (q.P.nw != kAttnThreadsBatch / kWave || q.P.mode != gemmb::kStagePrepared || q.P.nsplit != 1) {
        set_error("fused QKV + attention: the QKV GEMM's launch form does not fit");
        return -1;
    }
    q.in = in;
    q.out.tagged = tagged;
    q.out.ldy = M;
    q.at = a;
    q.ns = kAttnSplitBatch;
    q.epoch = epoch;
    q.layer = layer;
    q.spin_limit = spin_limit;
    q.err = err;
    const dim3 grid((unsigned)(q.P.gx + q.ns * a.batch));
    const int dpl = a.hd / kWave;
#define SPH_QA(DTV, DPLV, NHV, NKVV)                                                                         \
    if (dt == DTV && dpl == DPLV && a.nh == NHV && a.nkv == NKVV)                                          \
        hipLaunchKernelGGL((dec_qkv_attn_kernel<DTV, DPLV, NHV, NKVV>), grid, dim3(kAttnThreadsBatch), 0, s, q); \
    else
    SPH_QA(DT_Q4_0, 1, 4, 1) SPH_QA(DT_Q4_0, 2, 4, 1) SPH_QA(DT_Q4_0, 4, 4, 1) SPH_QA(DT_Q4_0, 1, 8, 1)
    SPH_QA(DT_Q4_0, 2, 8, 1) SPH_QA(DT_Q4_0, 1, 4, 2) SPH_QA(DT_Q4_0, 2, 4, 2) SPH_QA(DT_Q4_0, 1, 8, 2)
    SPH_QA(DT_Q4_0, 2, 8, 2) {
        set_error("fused QKV + attention: shape not instantiated");
        return -1;
    }
#undef SPH_QA
    if (!hip_ok(hipGetLastError(), "fused QKV + attention launch")) return -1;
    hipLaunchKernelGGL(dec_attn_combine_kernel<kAttnSplitBatch>, dim3(a.nh, a.batch), dim3(kThreads), 0, s, a.part,
                       a.nh, a.hd, out, a.out_stride, a.out_blocked);
    return hip_ok(hipGetLastError(), "attention combine launch") ? 0 : -1;
}

int dec_kv_write(const AttnArgs &a, hipStream_t s) {
    if (a.nkv * a.hd > kAttnMaxKV || a.batch <= 0) {
        set_error("KV write: %d K/V heads of dim %d", a.nkv, a.hd);
        return -1;
    }
    hipLaunchKernelGGL(dec_kv_write_kernel, dim3(a.batch), dim3(kThreads), 0, s, a);
    return hip_ok(hipGetLastError(), "KV write launch") ? 0 : -1;
}

int dec_embed(const uint16_t *embed, int hidden, int vocab, float es, const int *d_token, float *resid,
              hipStream_t s) {
    hipLaunchKernelGGL(dec_embed_kernel, dim3((hidden + kThreads - 1) / kThreads), dim3(kThreads), 0, s, embed, hidden,
                       vocab, es, d_token, resid);
    return hip_ok(hipGetLastError(), "embed launch") ? 0 : -1;
}

int dec_advance(const int *d_token, int *d_pos, int *d_step, int *log, uint32_t *d_seq, int *d_done,
                const StopSet &stop, hipStream_t s) {
    hipLaunchKernelGGL(dec_advance_kernel, dim3(1), dim3(64), 0, s, d_token, d_pos, d_step, log, d_seq, d_done, stop);
    return hip_ok(hipGetLastError(), "advance launch") ? 0 : -1;
}

int dec_embed_batch(const uint16_t *embed, int hidden, int vocab, float es, const int *d_tokens, int batch,
                    float *resid, hipStream_t s) {
    hipLaunchKernelGGL(dec_embed_batch_kernel, dim3((hidden + kThreads - 1) / kThreads, batch), dim3(kThreads), 0, s,
                       embed, hidden, vocab, es, d_tokens, resid);
    return hip_ok(hipGetLastError(), "batched embed launch") ? 0 : -1;
}

size_t argmax_batch_part_floats(int n, int batch) {
    (void)n;
    return (size_t)batch * kArgmaxParts * 2;
}

int dec_argmax_batch(const float *logits, int n, int batch, float *part, int *d_tokens, hipStream_t s) {
    hipLaunchKernelGGL(dec_argmax_part_kernel, dim3(kArgmaxParts, batch), dim3(kThreads), 0, s, logits, n, part);
    if (!hip_ok(hipGetLastError(), "argmax launch")) return -1;
    hipLaunchKernelGGL(dec_argmax_finish_kernel, dim3(batch), dim3(kWave), 0, s, part, kArgmaxParts, n, logits,
                       d_tokens);
    return hip_ok(hipGetLastError(), "argmax finish launch") ? 0 : -1;
}

int dec_advance_batch(const int *d_tokens, int *d_pos, int *d_step, int batch, int *log, int *d_done,
                      const StopSet &stop, uint32_t *d_epoch, hipStream_t s) {
    hipLaunchKernelGGL(dec_advance_batch_kernel, dim3(1), dim3(kWave), 0, s, d_tokens, d_pos, d_step, batch, log,
                       d_done, stop, d_epoch);
    return hip_ok(hipGetLastError(), "batched advance launch") ? 0 : -1;
}

}  // namespace sapphire
