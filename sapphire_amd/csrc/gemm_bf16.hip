// gemm_bf16.hip - BF16 weights times a batch of up to 16 fp32 activation vectors on the CDNA4
// matrix cores: Y[b][r] = sum_k W[r][k] * X[b][k], the batched form of kernel_gemv for BF16
// tensors (kernel_gemv_batch / kernel_gemm, dispatch.c:87-99,234-266; the reference computes it
// with kernel_gemm_bf16_avx2, bf16_avx.c:115-159).
//
// Operands of v_mfma_f32_16x16x32_bf16, three per 32-element block:
//  * B (16 columns = 16 weight rows of a tile): the BF16 weights as they are in memory, one
//    16-byte load per lane (lane l: row l % 16, elements 8 (l / 16) .. + 7 of the block).
//  * A (16 rows = the sequences): x split into three bf16 terms, x = t1 + t2 + t3 with
//    t1 = bf16(x), t2 = bf16(x - t1), t3 = bf16(x - t1 - t2) (each difference exact in fp32),
//    which carry 24 significant bits: every product of a term and a weight is exact in fp32.
//    bf16 has fp32's exponent range, so no range scaling is needed.
//  * C: per lane the four sequences 4m..4m+3 (m = l / 16) of weight row l % 16, accumulated
//    over the blocks in order, three terms per block.
// A workgroup of four waves stages a 256-element chunk of all 16 vectors' terms into LDS
// (24 KiB) and each wave multiplies its tiles (grid-stride, at most kMaxTiles per wave, their
// accumulators held across the chunks). The weight loads of a tile's eight blocks are issued
// together, up to three tiles ahead of the one being multiplied (across chunk boundaries too).
#include <algorithm>

#include "internal.h"

namespace sapphire {

namespace {

constexpr int kWave = 64;
constexpr int kWavesPerWg = 4;
constexpr int kThreads = kWave * kWavesPerWg;
constexpr int kTileRows = 16;
constexpr int kChunk = 256;                 // elements of K staged at a time
constexpr int kChunkBlocks = kChunk / 32;
constexpr int kTerms = 3;
constexpr int kMaxTiles = 8;                // tiles per wave (accumulators in registers)
constexpr int kBatch = 16;
constexpr uint32_t kOffNone = 0xFFFFFFF0u;  // out of range: the buffer load returns zeros
constexpr int kNT = 0;                      // plain loads: a row's two 64-byte halves meet in L2

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// fp32 -> bf16 bits, rounded to nearest even (finite inputs)
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_to_f(uint32_t b) { return __uint_as_float(b << 16); }

template <int NTW>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(const uint16_t *__restrict__ w, uint32_t w_bytes, int M,
                                                             int K, const float *__restrict__ x, int ldx, int batch,
                                                             float *__restrict__ y, int ldy) {
    __shared__ u32x4 as[kTerms][kChunkBlocks][kWave];   // the A operands of a chunk (24 KiB)
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    const int n = lane & 15, m = lane >> 4;
    const int ntiles = (M + kTileRows - 1) / kTileRows;
    const int nwaves = gridDim.x * kWavesPerWg;
    const int wave = blockIdx.x * kWavesPerWg + wid;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w_bytes);
    const uint32_t row_bytes = (uint32_t)K * 2u;

    f4 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

    // A ring of R tile loads: unit u = (chunk, tile i) sits in bw[u % R] = bw[i % R] (NTW is a
    // multiple of R), and unit u + R - 1 is issued while unit u is multiplied, across chunk
    // boundaries too, so R - 1 tiles' loads are in flight during every multiply and staging.
    constexpr int R = NTW >= 4 ? 4 : NTW;
    u32x4 bw[R][kChunkBlocks];
    // the weight loads of tile i of the chunk at k0 (offsets past the matrix load zeros)
    auto issue = [&](int k0, int i, u32x4 (&dst)[kChunkBlocks]) {
        const int t = wave + i * nwaves;
        const uint32_t rowoff = (uint32_t)(t * kTileRows + n) * row_bytes;
#pragma unroll
        for (int b = 0; b < kChunkBlocks; ++b) {
            const int k = k0 + b * 32 + m * 8;
            const uint32_t off = (t < ntiles && t * kTileRows + n < M && k < K) ? rowoff + (uint32_t)k * 2u : kOffNone;
            dst[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kNT));
        }
    };
#pragma unroll
    for (int j = 0; j + 1 < R; ++j) issue(0, j, bw[j]);   // in flight during the first staging
    for (int k0 = 0; k0 < K; k0 += kChunk) {
        // ---- stage: thread (seq, q) converts elements k0 + 16q .. + 15 of vector seq ----
        {
            const int seq = tid & 15, q = tid >> 4;
            const int bl = q >> 1;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int g = (q & 1) * 2 + h;                  // 8-element group of the block
                const int kk = k0 + bl * 32 + g * 8;
                uint32_t t[kTerms][4];
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    float v[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int k = kk + e + u;
                        v[u] = (seq < batch && k < K) ? x[(size_t)seq * ldx + k] : 0.f;
                    }
                    uint32_t b[kTerms][2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        b[0][u] = bf16_rne(v[u]);
                        const float r1 = v[u] - bf16_to_f(b[0][u]);
                        b[1][u] = bf16_rne(r1);
                        const float r2 = r1 - bf16_to_f(b[1][u]);
                        b[2][u] = bf16_rne(r2);
                    }
#pragma unroll
                    for (int tt = 0; tt < kTerms; ++tt) t[tt][e / 2] = b[tt][0] | (b[tt][1] << 16);
                }
#pragma unroll
                for (int tt = 0; tt < kTerms; ++tt)
                    as[tt][bl][g * 16 + seq] = u32x4{t[tt][0], t[tt][1], t[tt][2], t[tt][3]};
            }
        }
        __syncthreads();
        const int nbl = min(kChunkBlocks, (K - k0 + 31) / 32);
        // ---- multiply the wave's tiles ----
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int ia = i + R - 1;   // the unit issued now: R - 1 ahead
            if (ia < NTW) issue(k0, ia, bw[ia % R]);
            else if (k0 + kChunk < K) issue(k0 + kChunk, ia - NTW, bw[ia % R]);
            if (wave + i * nwaves < ntiles) {
#pragma unroll
                for (int b = 0; b < kChunkBlocks; ++b) {
                    if (b < nbl) {
                        const bf16x8 bop = __builtin_bit_cast(bf16x8, bw[i % R][b]);
#pragma unroll
                        for (int tt = 0; tt < kTerms; ++tt)
                            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, as[tt][b][lane]), bop, acc[i], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();   // the chunk's A operands are read before the next staging
    }
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
        const int t = wave + i * nwaves;
        const int row = t * kTileRows + n;
        if (t < ntiles && row < M)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * m + r < batch) y[(size_t)(4 * m + r) * ldy + row] = acc[i][r];
    }
}

int cus_bf16() {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
        return 256;
    return c;
}

}  // namespace

bool gemm_bf16_supported(const void *w, int M, int K) {
    return M > 0 && K > 0 && K % 8 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
           (size_t)M * (size_t)K * 2 < ((size_t)1 << 32) - 256;
}

int launch_gemm_bf16(const void *w, int M, int K, const float *x, int ldx, int batch, float *y, int ldy,
                     hipStream_t st) {
    if (!gemm_bf16_supported(w, M, K) || batch <= 0 || !x || !y || ldx < K || ldy < M) {
        set_error("BF16 GEMM: unsupported arguments (M=%d K=%d batch=%d)", M, K, batch);
        return -1;
    }
    static const int cus = cus_bf16();
    const long ntiles = (M + kTileRows - 1) / kTileRows;
    const uint32_t wb = (uint32_t)((size_t)M * K * 2);
    for (int b0 = 0; b0 < batch; b0 += kBatch) {
        const int nb = std::min(kBatch, batch - b0);
        // waves: up to eight per CU, enough that no wave has more than kMaxTiles tiles
        const long waves = std::max(std::min(ntiles, 8L * cus), (ntiles + kMaxTiles - 1) / kMaxTiles);
        const int ntw = (int)((ntiles + waves - 1) / waves);
        const dim3 grid((unsigned)((waves + kWavesPerWg - 1) / kWavesPerWg)), blk(kThreads);
        const float *xb = x + (size_t)b0 * ldx;
        float *yb = y + (size_t)b0 * ldy;
        const uint16_t *wp = static_cast<const uint16_t *>(w);
        switch (ntw) {
            case 1: hipLaunchKernelGGL(gemm_bf16_kernel<1>, grid, blk, 0, st, wp, wb, M, K, xb, ldx, nb, yb, ldy); break;
            case 2: hipLaunchKernelGGL(gemm_bf16_kernel<2>, grid, blk, 0, st, wp, wb, M, K, xb, ldx, nb, yb, ldy); break;
            case 3:
            case 4: hipLaunchKernelGGL(gemm_bf16_kernel<4>, grid, blk, 0, st, wp, wb, M, K, xb, ldx, nb, yb, ldy); break;
            default: hipLaunchKernelGGL(gemm_bf16_kernel<8>, grid, blk, 0, st, wp, wb, M, K, xb, ldx, nb, yb, ldy); break;
        }
        if (!hip_ok(hipGetLastError(), "gemm_bf16 launch")) return -1;
    }
    return 0;
}

}  // namespace sapphire
