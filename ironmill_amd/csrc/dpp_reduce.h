// dpp_reduce.h -- reductions over one DPP row (16 consecutive lanes of a wave)
// with data-parallel-primitive moves: no LDS traffic, 4 steps, the result in
// every lane of the row.  Steps: quad butterflies (quad_perm [1,0,3,2] and
// [2,3,0,1]), then row rotations by 4 and 8; lane 0 of a row always combines
// in the same order, so sums are deterministic.
#pragma once

#include <hip/hip_runtime.h>

namespace imh_dpp {

constexpr int kQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kRowRor4 = 0x124;
constexpr int kRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<kQuadXor1>(v);
    v += dpp_mov<kQuadXor2>(v);
    v += dpp_mov<kRowRor4>(v);
    v += dpp_mov<kRowRor8>(v);
    return v;
}

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<kQuadXor1>(v));
    v = fmaxf(v, dpp_mov<kQuadXor2>(v));
    v = fmaxf(v, dpp_mov<kRowRor4>(v));
    v = fmaxf(v, dpp_mov<kRowRor8>(v));
    return v;
}

// The same reductions for code where all 16 lanes of the row are active: the
// moves leave the lanes' old values undefined (every source lane of these
// patterns lies inside the row), so the compiler can fold each move into the
// add or max as a DPP operand instead of first zeroing the destination.
template <int CTRL>
__device__ __forceinline__ float dpp_mov_full(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum_full(float v) {
    v += dpp_mov_full<kQuadXor1>(v);
    v += dpp_mov_full<kQuadXor2>(v);
    v += dpp_mov_full<kRowRor4>(v);
    v += dpp_mov_full<kRowRor8>(v);
    return v;
}

__device__ __forceinline__ float row16_max_full(float v) {
    v = fmaxf(v, dpp_mov_full<kQuadXor1>(v));
    v = fmaxf(v, dpp_mov_full<kQuadXor2>(v));
    v = fmaxf(v, dpp_mov_full<kRowRor4>(v));
    v = fmaxf(v, dpp_mov_full<kRowRor8>(v));
    return v;
}

// the value in the wave's first active lane, as a wave-uniform scalar
__device__ __forceinline__ float first_lane(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

}  // namespace imh_dpp
