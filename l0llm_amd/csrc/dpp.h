// Cross-lane helpers shared by the gfx950 kernels: DPP lane permutations and the wave / lane-group
// reductions built on them, and the hardware 2^x.
#pragma once

#include <hip/hip_runtime.h>

namespace l0h {
namespace {

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave, returned to every lane (wave-uniform).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_src<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_src<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_src<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_src<0x140, 0xf>(v);  // row_mirror
    v += dpp_src<0x142, 0xa>(v);  // row_bcast15 into rows 1, 3
    v += dpp_src<0x143, 0xc>(v);  // row_bcast31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// 2^x as one v_exp_f32. exp2f wraps the instruction in a range reduction (compare, select, add,
// ldexp) so that results below 2^-126 come out as denormals instead of zero; every softmax weight
// here is summed against a running total of at least 1, where such a value changes nothing, and
// for x >= -126 both give the same bits.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum over the LPP lanes that share a position (2, 4 or 8 lanes of a row, or the full 16-lane
// row), left in every lane of the group.
template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_src<0xB1, 0xf>(v);  // quad_perm [1,0,3,2]
    if constexpr (LPP >= 4) v += dpp_src<0x4E, 0xf>(v);  // quad_perm [2,3,0,1]
    if constexpr (LPP == 8) {
        v += dpp_src<0x141, 0xf>(v);  // row_half_mirror: quad 0 <-> quad 1
    } else if constexpr (LPP == 16) {
        v += dpp_src<0x124, 0xf>(v);  // row_ror:4
        v += dpp_src<0x128, 0xf>(v);  // row_ror:8
    }
    return v;
}

// Reduction over the position slots of a wave: lanes lane % LPP == const. Within a 16-lane row
// the slots are LPP lanes apart (DPP row rotations), then rows are combined with the gfx950 row
// swaps: permlane16_swap(v, v) yields rows (r0, r0, r2, r2) and (r1, r1, r3, r3), permlane32_swap
// the two 32-lane halves, so op(first, second) reduces across them.
template <int LPP, bool MAX>
__device__ __forceinline__ float slot_reduce(float v) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    if constexpr (LPP <= 8) v = op(v, dpp_src<0x120 + (LPP <= 8 ? LPP : 1), 0xf>(v));   // row_ror:LPP
    if constexpr (LPP <= 4) v = op(v, dpp_src<0x120 + (LPP <= 4 ? 2 * LPP : 1), 0xf>(v));  // row_ror:2 LPP
    if constexpr (LPP <= 2) v = op(v, dpp_src<0x120 + (LPP <= 2 ? 4 * LPP : 1), 0xf>(v));  // row_ror:4 LPP
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// Lane j of each 16-lane row, in every lane of that row (DPP row_newbcast).
template <int J>
__device__ __forceinline__ float row_lane(float v) {
    return dpp_src<0x150 + J, 0xf>(v);
}

}  // namespace
}  // namespace l0h
