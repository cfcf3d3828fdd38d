// lanes.h - cross-lane sums and maxima over rows of 16 lanes by DPP (shared by the GEMV and
// decode kernels; not installed).
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
