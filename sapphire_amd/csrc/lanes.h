// lanes.h - cross-lane sums and maxima by DPP over rows of 16 lanes and whole waves (shared by
// the GEMV, GEMM and decode kernels; not installed).
#pragma once

namespace sapphire {
namespace lanes {

// DPP move of v (dpp_ctrl CTRL, every row and bank enabled).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over each row of 16 lanes, left in every lane of the row: quad_perm [1,0,3,2] and
// [2,3,0,1], then row_half_mirror and row_mirror. Each step adds a lane to its partner in
// the other half, so every lane of the row ends with the same bits (fp addition commutes).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    return v;
}

// Maximum over each row of 16 lanes, left in every lane of the row (as row16_sum).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return v;
}

// Sum over the 64 lanes of a wave, the same bits in every lane: row16_sum, then the four
// rows' sums (read from lanes 0, 16, 32, 48) added as a pair of pairs.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// Maximum over the 64 lanes of a wave, in every lane (as wave_sum).
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Bitwise OR over each quad of lanes (4 q .. 4 q + 3), left in every lane of the quad:
// quad_perm [1,0,3,2], then [2,3,0,1].
__device__ __forceinline__ uint32_t quad_or(uint32_t v) {
    v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    return v;
}

// The largest unsigned 64-bit value of the wave, in every lane: rows of 16 lanes by DPP on
// both halves (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror), then the four
// rows' maxima read from lanes 0, 16, 32 and 48.
template <int CTRL>
__device__ __forceinline__ unsigned long long u64_dpp(unsigned long long k) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)k, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(k >> 32), CTRL, 0xF, 0xF, false);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ unsigned long long u64_lane(unsigned long long k, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ unsigned long long u64_wave_max(unsigned long long k) {
    auto mx = [](unsigned long long a, unsigned long long b) { return a > b ? a : b; };
    k = mx(k, u64_dpp<0xB1>(k));
    k = mx(k, u64_dpp<0x4E>(k));
    k = mx(k, u64_dpp<0x141>(k));
    k = mx(k, u64_dpp<0x140>(k));
    return mx(mx(u64_lane(k, 0), u64_lane(k, 16)), mx(u64_lane(k, 32), u64_lane(k, 48)));
}

// The greedy (value, index) best over each row of 16 lanes, left in every lane of the row: the
// steps of row16_max, each pairing a lane with a partner that takes the same pair, under
// `better` (a total order on (value, index) pairs, so every lane ends with the same pair).
template <class Better>
__device__ __forceinline__ void row16_best(float &v, int &i, Better better) {
    auto step = [&](float ov, int oi) {
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    };
    step(dpp_mov<0xB1>(v), __float_as_int(dpp_mov<0xB1>(__int_as_float(i))));
    step(dpp_mov<0x4E>(v), __float_as_int(dpp_mov<0x4E>(__int_as_float(i))));
    step(dpp_mov<0x141>(v), __float_as_int(dpp_mov<0x141>(__int_as_float(i))));
    step(dpp_mov<0x140>(v), __float_as_int(dpp_mov<0x140>(__int_as_float(i))));
}

}  // namespace lanes
}  // namespace sapphire
