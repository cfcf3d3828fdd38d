// quantize.hip - the producer of Q4_0 / Q8_0 weights: F32 / BF16 rows [M][K] into the
// reference's block arrays [M][ceil(K/32)] (include/kernels.h:29-38), elements past K in the
// last block of a row taken as zeros.
//
// The reference has no quantizer (it only reads blocks: tensor.c:108-110,
// safetensors_reader.c:406-414); its block structs are ggml's, and this follows ggml's
// published reference quantizer (quantize_row_q8_0_ref / quantize_row_q4_0_ref) with the
// reference's fp32 scale and its Q4_0 nibble order (element 2j in the low nibble of byte j,
// 2j+1 in the high nibble, q4_0_avx.c:61-66):
//   Q8_0: amax = max|x|; d = amax / 127; id = d ? 1/d : 0; q = roundf(x * id).
//   Q4_0: max = the first x of largest |x| (+0 when all are zero); d = max / -8;
//         id = d ? 1/d : 0; q = min(15, trunc(x * id + 8.5)).
// Each product and sum is rounded on its own (the library is built without contraction) and
// divisions are correctly rounded. Inputs must be finite; a block whose scale is subnormal
// (1/d overflows) saturates infinite products and codes NaN ones (0 * inf) as zero.
//
// Layout of the work: four lanes per block, lane l holding elements 8l..8l+7 (two 16-byte
// fp32 loads or one 16-byte bf16 load, consecutive lanes on consecutive bytes); the block's
// maximum goes through two DPP steps inside the quad. A Q4_0 lane stores one dword of
// nibbles, a Q8_0 lane two dwords of quants, lane 0 the scale (plain stores, so the L2
// merges a wave's partial lines before they go to HBM). Each lane group loads 128
// bytes of source (4 fp32 or 8 bf16 blocks) before it quantizes any of them.
#include <algorithm>

#include "internal.h"
#include "lanes.h"

namespace sapphire {

namespace {

constexpr int kQThreads = 256;
constexpr int kLanes = 4;   // lanes per block, eight elements each
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// max / min over the 4 lanes of a quad (quad_perm [1,0,3,2], then [2,3,0,1])
__device__ __forceinline__ float max4(float v) {
    v = fmaxf(v, lanes::dpp_mov<0xB1>(v));
    return fmaxf(v, lanes::dpp_mov<0x4E>(v));
}
__device__ __forceinline__ int min4(int v) {
    v = min(v, dpp_int<0xB1>(v));
    return min(v, dpp_int<0x4E>(v));
}

// Integer codes of the rounded values: ggml's conversions for blocks of normal scale; for a
// subnormal scale (1/d overflows) an infinite product saturates and a NaN one (0 * inf)
// gives the code of zero.
__device__ __forceinline__ int q8_code(float v) {
    return v != v ? 0 : v > 127.0f ? 127 : v < -127.0f ? -127 : (int)v;
}
__device__ __forceinline__ int q4_code(float v) { return v != v ? 8 : v > 15.0f ? 15 : v < 0.0f ? 0 : (int)v; }

// Elements e0..e0+7 of a row (zeros past K), without branches: VEC (K % 8 == 0, 16-byte
// aligned rows) loads the eight at a clamped address and zeroes them past the row; otherwise
// each element is loaded from a clamped index and zeroed past the row.
template <int SRC, bool VEC>
__device__ __forceinline__ void load8(const void *__restrict__ src, size_t base, int e0, int K, float (&x)[8]) {
    const bool in = e0 < K;
    if constexpr (VEC) {
        const size_t off = base + (in ? e0 : 0);
        float v[8];
        if constexpr (SRC == DT_F32) {
            const f32x4 *p = reinterpret_cast<const f32x4 *>(static_cast<const float *>(src) + off);
            const f32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const u32x4 t =
                __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(src) + off));
            const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float(w[i] << 16);
                v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = in ? v[i] : 0.f;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + i;
            const size_t at = base + (size_t)min(e, K - 1);
            float v;
            if constexpr (SRC == DT_F32) v = static_cast<const float *>(src)[at];
            else v = __uint_as_float((uint32_t) static_cast<const uint16_t *>(src)[at] << 16);
            x[i] = e < K ? v : 0.f;
        }
    }
}

// DENSE: K % 32 == 0, so block b starts at element 32b. Otherwise row and block come from a
// 32-bit division (the launcher keeps such matrices below 2^31 blocks).
template <int DST, int SRC, bool VEC, bool DENSE, int U>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(const void *__restrict__ src, int K, int nb,
                                                            long nblocks, uint8_t *__restrict__ dst) {
    constexpr int BB = DST == DT_Q4_0 ? 20 : 36;
    const int lq = threadIdx.x & (kLanes - 1);
    const long group = ((long)blockIdx.x * kQThreads + threadIdx.x) / kLanes;
    const long stride = ((long)gridDim.x * kQThreads) / kLanes;
    for (long b0 = group; b0 < nblocks; b0 += U * stride) {
        // every lane loads U blocks (past the end: the last block again), then quantizes them
        float x[U][8];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long b = min(b0 + u * stride, nblocks - 1);
            if constexpr (DENSE) {
                load8<SRC, VEC>(src, (size_t)b * 32, lq * 8, 32, x[u]);
            } else {
                const uint32_t row = (uint32_t)b / (uint32_t)nb;
                const int blk = (int)((uint32_t)b - row * (uint32_t)nb);
                load8<SRC, VEC>(src, (size_t)row * K, blk * 32 + lq * 8, K, x[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long b = b0 + u * stride;
            const bool store = b < nblocks;   // the same for the four lanes of a block
            uint8_t *out = dst + (size_t)min(b, nblocks - 1) * BB;
            float la = 0.f;
            int lkey = 0x7FFFFFFF;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float a = fabsf(x[u][i]);
                const bool gt = la < a;   // the first element of the lane's largest |x|
                la = gt ? a : la;
                if constexpr (DST == DT_Q4_0)
                    lkey = gt ? (((lq * 8 + i) << 1) | (int)(__float_as_uint(x[u][i]) >> 31)) : lkey;
            }
            const float amax = max4(la);
            if constexpr (DST == DT_Q8_0) {
                const float d = amax / 127.0f;
                const float id = d != 0.f ? 1.0f / d : 0.f;
                uint32_t w[2] = {0u, 0u};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int q = q8_code(roundf(__fmul_rn(x[u][i], id)));
                    w[i >> 2] |= (uint32_t)(q & 0xFF) << (8 * (i & 3));
                }
                if (store) {
                    uint32_t *o = reinterpret_cast<uint32_t *>(out + 4) + 2 * lq;
                    o[0] = w[0];
                    o[1] = w[1];
                    if (lq == 0) *reinterpret_cast<float *>(out) = d;
                }
            } else {
                // the first element (in block order) whose |x| is the block's maximum, and its sign
                const int key = min4(la == amax ? lkey : 0x7FFFFFFF);
                const float mx = amax == 0.f ? 0.f : ((key & 1) ? -amax : amax);
                const float d = mx / -8.0f;
                const float id = d != 0.f ? 1.0f / d : 0.f;
                uint32_t w = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    w |= (uint32_t)q4_code(__fadd_rn(__fmul_rn(x[u][i], id), 8.5f)) << (4 * i);
                if (store) {
                    reinterpret_cast<uint32_t *>(out + 4)[lq] = w;
                    if (lq == 0) *reinterpret_cast<float *>(out) = d;
                }
            }
        }
    }
}

int device_cus_q() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

template <int DST, int SRC>
int launch_typed(const void *src, int M, int K, void *dst, hipStream_t st) {
    constexpr int U = SRC == DT_F32 ? 4 : 8;   // 128 bytes of source per lane in flight
    const int nb = (K + 31) / 32;
    const long nblocks = (long)M * nb;
    const bool vec = K % 8 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
    if (K % 32 != 0 && nblocks >= (1L << 31)) {
        set_error("quantize: rows of a partial block need fewer than 2^31 blocks per call");
        return -1;
    }
    const long per_wg = (long)(kQThreads / kLanes) * U;
    static int cus = device_cus_q();
    const long grid = std::max(1L, std::min((nblocks + per_wg - 1) / per_wg, 8L * cus));
    uint8_t *d = static_cast<uint8_t *>(dst);
    const dim3 g((unsigned)grid), t(kQThreads);
    if (vec && K % 32 == 0)
        hipLaunchKernelGGL((quantize_kernel<DST, SRC, true, true, U>), g, t, 0, st, src, K, nb, nblocks, d);
    else if (vec)
        hipLaunchKernelGGL((quantize_kernel<DST, SRC, true, false, U>), g, t, 0, st, src, K, nb, nblocks, d);
    else if (K % 32 == 0)
        hipLaunchKernelGGL((quantize_kernel<DST, SRC, false, true, U>), g, t, 0, st, src, K, nb, nblocks, d);
    else
        hipLaunchKernelGGL((quantize_kernel<DST, SRC, false, false, U>), g, t, 0, st, src, K, nb, nblocks, d);
    return 0;
}

}  // namespace

int launch_quantize(int dst_dtype, int src_dtype, const void *src, int M, int K, void *blocks, hipStream_t st) {
    if ((dst_dtype != DT_Q4_0 && dst_dtype != DT_Q8_0) || (src_dtype != DT_F32 && src_dtype != DT_BF16) || !src ||
        !blocks || M <= 0 || K <= 0) {
        set_error("quantize: source must be F32 or BF16, destination Q4_0 or Q8_0, with positive shape");
        return -1;
    }
    if (reinterpret_cast<uintptr_t>(blocks) & 3) {
        set_error("quantize: the block array must be 4-byte aligned");
        return -1;
    }
    int rc;
    if (dst_dtype == DT_Q4_0 && src_dtype == DT_F32) rc = launch_typed<DT_Q4_0, DT_F32>(src, M, K, blocks, st);
    else if (dst_dtype == DT_Q4_0) rc = launch_typed<DT_Q4_0, DT_BF16>(src, M, K, blocks, st);
    else if (src_dtype == DT_F32) rc = launch_typed<DT_Q8_0, DT_F32>(src, M, K, blocks, st);
    else rc = launch_typed<DT_Q8_0, DT_BF16>(src, M, K, blocks, st);
    if (rc != 0) return -1;
    return hip_ok(hipGetLastError(), "quantize launch") ? 0 : -1;
}

}  // namespace sapphire
