// gemm_mfma.hip - Q4_0 / Q8_0 weights times a batch of up to 16 activation vectors on the
// CDNA4 matrix cores: Y[b][r] = sum_k W[r][k] * X[b][k], the batched form of kernel_gemv
// (dispatch.c:101-156; the reference itself rejects quantized batches, pool.c:318-321, so
// its meaning here is 16 independent GEMVs).
//
// Operands of v_mfma_f32_16x16x32_f16, one MFMA per 32-weight block and activation term:
//  * B (16 columns = 16 weight rows of a TILED tile): the integer weights, converted exactly
//    to fp16 in registers: a nibble or a sign-flipped byte is placed under the fp16 exponent
//    of 1024 (0x64nn) with v_perm and the bias removed with one packed fp16 subtract.
//  * A (16 rows = the sequences): x split into fp16 hi + lo terms, x * 2^-e = hi + lo to
//    about 22 bits, with one power-of-two range scale e per sequence and K chunk, so that
//    the largest |x| of the chunk sits in [2^14, 2^15). Two MFMAs (hi, lo) per block.
//  * C: per lane the four sequences 4m..4m+3 of weight row n; the block's weight scale is
//    applied with one FMA per value, the chunk's 2^e when the tile's result is stored.
//
// A workgroup of eight waves converts its K chunk (at most 36 blocks) of the 16 activation
// vectors into the A operands in LDS once, then each wave streams whole tiles through it.
// A wave's (tile, 4-block group) units run through a ring of register buffers: the loads of
// the next kRing-1 units are in flight while one unit is multiplied. K longer than one
// chunk is split over workgroups (grid.y): each leaves its partial sums, which a short
// kernel adds in chunk order (or the next GEMM adds while staging its input). Adding them
// in the GEMM itself (last workgroup to finish) needs device-scope fences, i.e. L2
// write-backs across the XCDs, which cost more than the extra launch.
#include "gemm_body.h"

namespace sapphire {

namespace {

using namespace gemmb;

// grid (sequences, K chunks): the input transform of the staging below for one sequence and
// chunk, with the same arithmetic (so the operands are bit-identical): the delta's sum of
// parts and rmsnorm_delta, the residual, the pre-norm, the range scale over the finite values,
// the non-finite record, the hi / lo fp16 split. Thread t takes pair t (8 activations).
template <int DT>
__global__ __launch_bounds__(kPrepThreads) void gemm_prep_kernel(GemmIn in, int K, int cb, PrepChunk *prep) {
    __shared__ float raw[kRawLd];
    __shared__ float npart[kBatchMax][8];
    __shared__ float rinv[kBatchMax];
    __shared__ float wmx[kPrepThreads / kWave];
    __shared__ float wsq[2][kPrepThreads / kWave];
    __shared__ int wflag[kPrepThreads / kWave];
    const int seq = blockIdx.x, chunk = blockIdx.y, p = threadIdx.x;
    const int lane = p & (kWave - 1), wid = p / kWave;
    const int nb = K / kBlock, b0 = chunk * cb, b1 = min(nb, b0 + cb);
    const int pairs = (b1 - b0) * 4, kb = b0 * kBlock;
    const bool on = p < pairs;
    PrepChunk &pc = prep[chunk];
    // 1 / rms of this sequence's K values, summed as a tree: each thread's eight squares, one
    // wave sum each (lane 0's), then the waves in a fixed order (slot: which of the two norms,
    // so that the second does not overwrite sums the first may still be reading)
    auto tree_rms_inv = [&](const float (&x)[8], int slot) {
        float sq = 0.f;
        if (p < pairs)
#pragma unroll
            for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(x[e], x[e], sq);
        sq = lanes::wave_sum(sq);
        if (lane == 0) wsq[slot][wid] = sq;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < kPrepThreads / kWave; ++w) tot += wsq[slot][w];
        return devmath::rms_inv_of(tot, K, in.eps);
    };
    float v[8], xv[8], wd[8], wn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = xv[e] = wd[e] = wn[e] = 0.f;
    if (on) {                                          // every independent load goes out first
        const int k = kb + p * 8;
        if (in.x) load8(in.x + (size_t)seq * in.ldx + k, in.parts ? xv : v);
        if (in.parts) load8(in.parts + (size_t)seq * in.ldp + k, v);
        if (in.w_delta && in.parts) load8(in.w_delta + k, wd);
        if (in.w_norm) load8(in.w_norm + k, wn);
    }
    if (in.parts) {
        // every partial's loads go out before the sum (in chunk order) uses them
        for (int c0 = 1; c0 < in.nparts; c0 += kPrepParts) {
            float t[kPrepParts][8];
#pragma unroll
            for (int c = 0; c < kPrepParts; ++c)
                if (on && c0 + c < in.nparts) load8(in.parts + (c0 + c) * in.part_stride + (size_t)seq * in.ldp + kb + p * 8, t[c]);
#pragma unroll
            for (int c = 0; c < kPrepParts; ++c)
                if (on && c0 + c < in.nparts)
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = __fadd_rn(v[e], t[c][e]);
        }
        if (in.w_delta) {
            float r;
            if (in.tree_norms) {
                r = tree_rms_inv(v, 0);
            } else {
                if (on)
#pragma unroll
                    for (int e = 0; e < 8; ++e) raw[p * 8 + e] = v[e];
                __syncthreads();
                rows_rms_inv<36>(raw, kRawLd, K, 1, in.eps, npart, rinv);
                r = rinv[0];
            }
            if (on)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = __fmul_rn(__fmul_rn(v[e], r), __fadd_rn(1.0f, wd[e]));
        }
        if (in.x)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __fadd_rn(xv[e], v[e]);
    }
    if (in.resid_out && on) {
        float4 *dst = reinterpret_cast<float4 *>(in.resid_out + (size_t)seq * in.ldr + kb + p * 8);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (in.w_norm) {
        // The pre-norm's sum of squares as a tree (tree_rms_inv: no staging through LDS and no
        // K/8-long chain). Its last bits differ from the reference's eight-lane order, inside
        // the decode tolerance; the residual above keeps that order (unless tree_norms is set)
        // and stays bit-identical.
        const float r = tree_rms_inv(v, 1);
        if (on)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __fmul_rn(__fmul_rn(v[e], r), __fadd_rn(1.0f, wn[e]));
    }
    // non-finite activations recorded and zeroed, the range over the rest
    bool nan = false;
    uint32_t pinf = 0, ninf = 0;
    float mx = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float t = v[e];
        nan |= t != t;
        pinf |= (t == INFINITY ? 1u : 0u) << e;
        ninf |= (t == -INFINITY ? 1u : 0u) << e;
        v[e] = nonfinite::is_nf(t) ? 0.f : t;
        mx = fmaxf(mx, fabsf(v[e]));
    }
    mx = lanes::wave_max(mx);
    const bool wnan = __any(nan) != 0, wnf = __any(nan || pinf != 0 || ninf != 0) != 0;
    if (lane == 0) {
        wmx[wid] = mx;
        wflag[wid] = (wnan ? 1 : 0) | (wnf ? 2 : 0);
    }
    // the four pairs of a block sit in threads 4 bl .. 4 bl + 3
    pinf <<= 8 * (p & 3);
    ninf <<= 8 * (p & 3);
    pinf = lanes::quad_or(pinf);
    ninf = lanes::quad_or(ninf);
    if (on && (p & 3) == 0) {
        pc.inf[seq][0][p >> 2] = pinf;
        pc.inf[seq][1][p >> 2] = ninf;
    }
    __syncthreads();
    mx = 0.f;
    int fl = 0;
#pragma unroll
    for (int w = 0; w < kPrepThreads / kWave; ++w) {
        mx = fmaxf(mx, wmx[w]);
        fl |= wflag[w];
    }
    int e = 0;
    if (mx > 0.f) {
        int ex;
        frexpf(mx, &ex);
        e = ex - 15;
    }
    if (p == 0) {
        pc.xsc[seq] = ldexpf(1.0f, e);
        pc.nan[seq] = fl & 1;
        pc.nf[seq] = (fl >> 1) & 1;
    }
    if (on) {
        h8 hv, lv;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float s = ldexpf(v[k_order<DT>(k)], -e) * k_factor<DT>(k);
            const _Float16 h = (_Float16)s;
            hv[k] = h;
            lv[k] = (_Float16)(s - (float)h);
        }
        const int bl = p >> 2, m = p & 3;
        pc.a[(bl * 2 + 0) * kWave + m * 16 + seq] = hv;
        pc.a[(bl * 2 + 1) * kWave + m * 16 + seq] = lv;
    }
}

template <int DT, int MODE, int NW, bool GREEDY = false>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(4))) void gemm_mfma_kernel(
    const uint8_t *__restrict__ wq, uint32_t q_bytes, const uint8_t *__restrict__ wsc, uint32_t s_bytes, GemmIn in,
    int batch, int M, int K, int cb, GemmOut out, float *__restrict__ Yp, const PrepChunk *__restrict__ prep, int ks) {
    __shared__ GemmLds<NW> L;
    gemm_body<DT, MODE, NW, GREEDY>(L, blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, wq, q_bytes, wsc, s_bytes, in,
                                    batch, M, K, cb, out, Yp, prep, ks);
}

// grid (batch), one wave: tokens[b] = the best of sequence b's nparts workgroup partials
// (sample_greedy, utils.c:145-156; 0 when no row is above -inf)
__global__ void gemm_greedy_finish_kernel(const float *__restrict__ part, int nparts, int n, int *__restrict__ tokens) {
    const float *p = part + (size_t)blockIdx.x * nparts * 2;
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int j = threadIdx.x; j < nparts; j += kWave) {
        const float v = p[2 * j];
        const int i = __float_as_int(p[2 * j + 1]);
        if (devmath::greedy_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (devmath::greedy_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (threadIdx.x == 0) tokens[blockIdx.x] = bi >= 0 && bi < n ? bi : 0;
}

constexpr int kEmbedPasses = 4;   // 16-byte embedding loads per lane of the finish (hidden <= 2048)

// grid 1, one wave per sequence: wave b picks sequence b's token from its nparts workgroup
// partials (as gemm_greedy_finish_kernel), then the step ends as BatchAdvance describes. Every
// wave reads the step counter before the barrier, and thread 0 advances it after.
__global__ __launch_bounds__(kBatchMax *kWave) void gemm_greedy_finish_advance_kernel(
    const float *__restrict__ part, int nparts, int n, int *__restrict__ tokens, int batch, BatchAdvance a) {
    const int b = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int s = *a.step;
    const float *p = part + (size_t)b * nparts * 2;
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int j = lane; j < nparts; j += kWave) {
        const float v = p[2 * j];
        const int i = __float_as_int(p[2 * j + 1]);
        if (devmath::greedy_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    // rows of 16 lanes by DPP, then the four rows' bests in row order (a total order: every
    // order of the comparisons picks the same pair)
    lanes::row16_best(bv, bi, devmath::greedy_better);
    float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
    int i = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int r = 16; r < kWave; r += 16) {
        const float ov = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), r));
        const int oi = __builtin_amdgcn_readlane(bi, r);
        if (devmath::greedy_better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
    const int t = i >= 0 && i < n ? i : 0;
    if (lane == 0) {
        tokens[b] = t;
        if (!(a.done && a.done[b])) {               // a stopped sequence: its entry keeps the fill
            a.log[(size_t)s * batch + b] = t;
            a.pos[b] = a.pos[b] + 1;
            if (a.done && a.stop.has(t)) a.done[b] = 1;   // inference.c:298-301
        }
    }
    const uint16_t *row = a.embed + (size_t)t * a.hidden;
    float *out = a.resid + (size_t)b * a.hidden;
    auto widen = [&](uint32_t bits) {
        const float x = __uint_as_float(bits << 16);
        return a.es != 1.0f ? __fmul_rn(x, a.es) : x;
    };
    if (a.hidden % 8 == 0 && a.hidden <= kEmbedPasses * kWave * 8) {
        // eight bf16 (16 bytes) per lane and pass, every pass's load issued before any store
        // (rows are 16-byte aligned: the table and resid start so, and hidden % 8 == 0)
        const int chunks = a.hidden / 8;
        uint4 u[kEmbedPasses];
#pragma unroll
        for (int q = 0; q < kEmbedPasses; ++q) {
            const int c = lane + q * kWave;
            u[q] = c < chunks ? reinterpret_cast<const uint4 *>(row)[c] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < kEmbedPasses; ++q) {
            const int c = lane + q * kWave;
            if (c < chunks) {
                float4 *dst = reinterpret_cast<float4 *>(out + 8 * c);
                dst[0] = make_float4(widen(u[q].x & 0xFFFFu), widen(u[q].x >> 16), widen(u[q].y & 0xFFFFu),
                                     widen(u[q].y >> 16));
                dst[1] = make_float4(widen(u[q].z & 0xFFFFu), widen(u[q].z >> 16), widen(u[q].w & 0xFFFFu),
                                     widen(u[q].w >> 16));
            }
        }
    } else {
        for (int k = lane; k < a.hidden; k += kWave) out[k] = widen(row[k]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        *a.step = s + 1;
        if (a.epoch) *a.epoch = *a.epoch + 1u;
    }
}

// y[b * ldy + r] = sum over c of parts[c * stride + b * M + r], in chunk order.
__global__ void sum_parts_kernel(const float *__restrict__ parts, int nparts, size_t stride, int batch, int M,
                                 float *__restrict__ y, int ldy) {
    const size_t n = (size_t)batch * M;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float s = parts[i];
        for (int c = 1; c < nparts; ++c) s += parts[c * stride + i];
        y[(i / M) * ldy + i % M] = s;
    }
}

int cus() {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
        return 256;
    return c;
}

// K chunking: as few chunks of at most kChunkBlocks blocks as cover K, in whole groups,
// every chunk non-empty (only the last may be shorter).
void k_chunks(int K, int *nsplit, int *cb) {
    const int nb = K / kBlock;
    const int parts = (nb + kChunkBlocks - 1) / kChunkBlocks;
    const int per = (nb + parts - 1) / parts;
    *cb = (per + kGroupBlocks - 1) / kGroupBlocks * kGroupBlocks;
    *nsplit = (nb + *cb - 1) / *cb;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

size_t partials_bytes(int M, int nsplit) { return nsplit > 1 ? (size_t)nsplit * kBatchMax * M * sizeof(float) : 0; }
size_t prep_offset(int M, int nsplit) { return (partials_bytes(M, nsplit) + 255) & ~size_t(255); }
size_t prep_stride() { return (sizeof(PrepChunk) + 255) & ~size_t(255); }
// the greedy form's partials: (value, index) per sequence and workgroup, after the prep chunks
size_t amax_offset(int M, int nsplit) { return prep_offset(M, nsplit) + (size_t)nsplit * prep_stride(); }
constexpr size_t kAmaxBytes = (size_t)kBatchMax * kMaxGrid * 2 * sizeof(float);

// The launch of one pass of at most 16 sequences: K chunks, waves per tile, grid and staging
// mode. With `prep` the input transform runs once per sequence and chunk (gemm_prep_kernel,
// into the workspace, launched here) instead of in every workgroup.
int gemm_plan(int dt, const void *w, int M, int K, int batch, const GemmIn &in, void *ws, hipStream_t st,
              bool prep, GemmPlan *P) {
    int nsplit = 1, cb = 0;
    k_chunks(K, &nsplit, &cb);
    PrepChunk *pc = nullptr;
    if (prep) {
        pc = reinterpret_cast<PrepChunk *>(static_cast<char *>(ws) + prep_offset(M, nsplit));
        if (dt == DT_Q4_0)
            hipLaunchKernelGGL(gemm_prep_kernel<DT_Q4_0>, dim3(batch, nsplit), dim3(kPrepThreads), 0, st, in, K, cb, pc);
        else
            hipLaunchKernelGGL(gemm_prep_kernel<DT_Q8_0>, dim3(batch, nsplit), dim3(kPrepThreads), 0, st, in, K, cb, pc);
        if (!hip_ok(hipGetLastError(), "gemm_prep launch")) return -1;
    }
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const size_t so = q_tiled_scales_offset(dt, M, K);
    const size_t sbytes = q_tiled_bytes(dt, M, K) - so;
    const int ntiles = (M + kTileRows - 1) / kTileRows;
    // Waves per tile: a tile's groups are split over ks waves when then every wave still has
    // at most one tile and the launch fits on the CUs once (the layer shapes of a decode
    // step); a streaming launch (the LM head) keeps one wave per tile.
    const int nb = K / kBlock, min_gc = (nb - (nsplit - 1) * cb) / kGroupBlocks;   // the last chunk's groups
    int ks = 1;
    for (int k : {4, 2})
        if (k <= min_gc && (ntiles * k + kWaves - 1) / kWaves * nsplit <= cus()) {
            ks = k;
            break;
        }
    // A streaming launch (one wave per tile, at least two tiles per wave) runs one workgroup of
    // 16 waves per CU: the chunk is staged once per CU, and no second workgroup on the CU
    // finishes behind the first. Else workgroups of 8 waves, two per CU.
    const bool wide = ks == 1 && nsplit == 1 && ntiles >= 2 * kWavesWide * cus();
    const int nw = wide ? kWavesWide : kWaves;
    const int sets = (ntiles * ks + nw - 1) / nw;
    P->wq = wb;
    P->q_bytes = (uint32_t)so;
    P->wsc = wb + so;
    P->s_bytes = (uint32_t)sbytes;
    P->M = M;
    P->K = K;
    P->batch = batch;
    P->cb = cb;
    P->nsplit = nsplit;
    P->ks = ks;
    P->nw = nw;
    P->gx = ks > 1 ? sets : std::max(1, std::min({sets, ((wide ? 1 : 2) * cus() + nsplit - 1) / nsplit, kMaxGrid}));
    P->mode = pc ? kStagePrepared
                 : (!in.parts && !in.w_delta && !in.w_norm && !in.resid_out) ? kStagePlain : kStageFull;
    P->prep = pc;
    P->Yp = static_cast<float *>(ws);
    return 0;
}

int gemm_pass(int dt, const void *w, int M, int K, int batch, const GemmIn &in, const GemmOut &out, void *ws,
              hipStream_t st, bool prep = false) {
    GemmPlan P;
    if (gemm_plan(dt, w, M, K, batch, in, ws, st, prep, &P) != 0) return -1;
    const int mode = P.mode, nsplit = P.nsplit, gx = P.gx;
    const bool wide = P.nw == kWavesWide;
    if (out.tokens && mode == kStageFull) {
        set_error("batched GEMM: the greedy form needs a workspace");
        return -1;
    }
    decltype(&gemm_mfma_kernel<DT_Q4_0, kStageFull, kWaves>) kern;
#define SPH_GEMM_PICK(DTV, NWV)                                                                                    \
    kern = out.tokens ? (mode == kStagePrepared ? gemm_mfma_kernel<DTV, kStagePrepared, NWV, true>                 \
                                                : gemm_mfma_kernel<DTV, kStagePlain, NWV, true>)                   \
           : mode == kStagePrepared ? gemm_mfma_kernel<DTV, kStagePrepared, NWV>                                   \
           : mode == kStagePlain    ? gemm_mfma_kernel<DTV, kStagePlain, NWV>                                      \
                                    : gemm_mfma_kernel<DTV, kStageFull, NWV>;
    if (dt == DT_Q4_0) {
        if (wide) { SPH_GEMM_PICK(DT_Q4_0, kWavesWide) } else { SPH_GEMM_PICK(DT_Q4_0, kWaves) }
    } else {
        if (wide) { SPH_GEMM_PICK(DT_Q8_0, kWavesWide) } else { SPH_GEMM_PICK(DT_Q8_0, kWaves) }
    }
#undef SPH_GEMM_PICK
    GemmOut o = out;
    if (o.tokens) o.amax = reinterpret_cast<float *>(static_cast<char *>(ws) + amax_offset(M, nsplit));
    hipLaunchKernelGGL(kern, dim3((unsigned)gx, (unsigned)nsplit), dim3(P.nw * kWave), 0, st, P.wq, P.q_bytes, P.wsc,
                       P.s_bytes, in, batch, M, K, P.cb, o, P.Yp, (const PrepChunk *)P.prep, P.ks);
    if (!hip_ok(hipGetLastError(), "gemm_mfma launch")) return -1;
    if (o.tokens && o.advance)
        hipLaunchKernelGGL(gemm_greedy_finish_advance_kernel, dim3(1), dim3(batch * kWave), 0, st, o.amax, gx, M,
                           o.tokens, batch, *o.advance);
    else if (o.tokens)
        hipLaunchKernelGGL(gemm_greedy_finish_kernel, dim3(batch), dim3(kWave), 0, st, o.amax, gx, M, o.tokens);
    if (o.tokens) return hip_ok(hipGetLastError(), "greedy finish launch") ? 0 : -1;
    if (nsplit > 1 && !out.parts) return launch_sum_parts(P.Yp, nsplit, (size_t)batch * M, batch, M, out.y, out.ldy, st);
    return 0;
}

}  // namespace

int gemm_splits(int K) {
    int nsplit = 1, cb = 0;
    k_chunks(K, &nsplit, &cb);
    return nsplit;
}

size_t gemm_workspace_bytes(int M, int K) {
    const int nsplit = gemm_splits(K);
    return amax_offset(M, nsplit) + kAmaxBytes;
}

int launch_sum_parts(const float *parts, int nparts, size_t stride, int batch, int M, float *y, int ldy,
                     hipStream_t st) {
    const size_t n = (size_t)batch * M;
    hipLaunchKernelGGL(sum_parts_kernel, dim3((unsigned)std::min<size_t>(1024, (n + 255) / 256)), dim3(256), 0, st,
                       parts, nparts, stride, batch, M, y, ldy);
    return hip_ok(hipGetLastError(), "sum_parts launch") ? 0 : -1;
}

int launch_gemm_tiled_ex(int dt, const void *w, int M, int K, int batch, const GemmIn &in, const GemmOut &out,
                         void *ws, hipStream_t st) {
    const int nsplit = gemm_splits(K);
    const bool norms = in.w_delta || in.w_norm;
    const bool ok = batch >= 1 && batch <= kBatchMax && M > 0 && K > 0 && K % (kGroupBlocks * kBlock) == 0 &&
                    (in.x || in.parts) &&
                    (!in.x || (aligned16(in.x) && (in.x_blocked || (in.ldx % 4 == 0 && in.ldx >= K)))) &&
                    (!in.parts || (aligned16(in.parts) && in.nparts >= 1 && in.ldp % 4 == 0 && in.ldp >= K &&
                                   in.part_stride % 4 == 0)) &&
                    (!in.w_delta || in.parts) && (!in.resid_out || (aligned16(in.resid_out) && in.ldr % 4 == 0)) &&
                    (!norms || (nsplit == 1 && aligned16(in.w_delta ? in.w_delta : in.w_norm) &&
                                (!in.w_norm || aligned16(in.w_norm)))) &&
                    (out.parts || out.tokens || (out.y && (out.y_blocked || out.ldy >= (out.geglu ? M / 2 : M)))) &&
                    (!out.tokens || (nsplit == 1 && !out.parts && !out.geglu && !out.y_blocked && ws &&
                                     (reinterpret_cast<uintptr_t>(ws) & 255u) == 0)) &&
                    (!out.geglu || (nsplit == 1 && M % 16 == 0 && !out.parts)) &&
                    (out.parts || nsplit == 1 || ((reinterpret_cast<uintptr_t>(ws) & 255u) == 0 && ws)) &&
                    (!in.x_blocked || (in.x && !in.parts && !norms && !in.resid_out)) &&
                    (!out.y_blocked || (nsplit == 1 && !out.parts && out.y)) &&
                    (!out.advance || (out.tokens && out.advance->pos && out.advance->step && out.advance->log &&
                                      out.advance->embed && out.advance->resid && out.advance->hidden > 0));
    if (!ok) {
        set_error("batched GEMM: unsupported arguments (batch=%d M=%d K=%d nsplit=%d)", batch, M, K, nsplit);
        return -1;
    }
    // inputs with a sum of parts or a norm are prepared once; a plain x is staged by every
    // workgroup (a copy costs about what the prep launch would)
    return gemm_pass(dt, w, M, K, batch, in, out, ws, st, ws != nullptr && (norms || in.parts));
}

int plan_gemm_tiled(int dt, const void *w, int M, int K, int batch, const GemmIn &in, void *ws, hipStream_t st,
                    GemmPlan *P) {
    const bool norms = in.w_delta || in.w_norm;
    if (batch < 1 || batch > kBatchMax || M <= 0 || K <= 0 || K % (kGroupBlocks * kBlock) != 0 || !ws ||
        (reinterpret_cast<uintptr_t>(ws) & 255u) != 0 || gemm_splits(K) != 1 || !(norms || in.parts) ||
        (!in.x && !in.parts)) {
        set_error("batched GEMM plan: unsupported arguments (batch=%d M=%d K=%d)", batch, M, K);
        return -1;
    }
    return gemm_plan(dt, w, M, K, batch, in, ws, st, true, P);
}

int launch_gemm_tiled(int dt, const void *w, int M, int K, const float *X, int batch, float *Y, void *ws,
                      hipStream_t st) {
    if (batch < 1 || K % (kGroupBlocks * kBlock) != 0 || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0 ||
        !aligned16(X)) {
        set_error("batched GEMM: bad arguments (batch=%d K=%d ws=%p X=%p; K %% 128 == 0, ws 256-byte and X "
                  "16-byte aligned)", batch, K, ws, (const void *)X);
        return -1;
    }
    // passes of 16 sequences share the workspace; the stream orders them
    for (int b0 = 0; b0 < batch; b0 += kBatchMax) {
        GemmIn in;
        in.x = X + (size_t)b0 * K;
        in.ldx = K;
        GemmOut out;
        out.y = Y + (size_t)b0 * M;
        out.ldy = M;
        if (gemm_pass(dt, w, M, K, std::min(kBatchMax, batch - b0), in, out, ws, st)) return -1;
    }
    return 0;
}

}  // namespace sapphire
