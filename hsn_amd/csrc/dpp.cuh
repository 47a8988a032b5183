// Reductions over aligned groups of L consecutive lanes of a 64-lane wavefront, with DPP.
//
// Within a 16-lane row, gfx9 DPP reaches lane i^1 and i^2 (quad_perm), the mirror within an
// 8-lane half row (row_half_mirror) and the rotation by 8 (row_ror:8), so groups of up to 16
// lanes reduce with one v_*_dpp instruction per step and no LDS traffic; each step combines a
// lane with its partner symmetrically, so every lane of the group ends with the bit-identical
// result. Wider groups (32, 64 lanes) join rows with gfx950's permlane swaps.
#pragma once

#include "common.cuh"

namespace hsn {

namespace dpp {
constexpr int kXor1 = 0xB1;        // quad_perm:[1,0,3,2]
constexpr int kXor2 = 0x4E;        // quad_perm:[2,3,0,1]
constexpr int kHalfMirror = 0x141;  // lane i <- lane 7-i within each 8 lanes
constexpr int kRor8 = 0x128;       // lane i <- lane (i+8) mod 16 within each row
}  // namespace dpp

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false));
}

// The partner row of every lane (gfx950 v_permlane16_swap / v_permlane32_swap, no LDS): the
// swap of a value with itself returns, in every lane, {the value in the even row, the value in
// the odd row} of the lane's pair of 16-lane rows (lanes l and l^16), resp. of its pair of
// 32-lane halves (lanes l and l^32). Both lanes of a pair get the same two operands in the same
// order, so a combination of them is bit-identical in both.
struct RowPair {
    uint32_t lo, hi;
};
__device__ __forceinline__ RowPair pair16(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return {static_cast<uint32_t>(r[0]), static_cast<uint32_t>(r[1])};
}
__device__ __forceinline__ RowPair pair32(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return {static_cast<uint32_t>(r[0]), static_cast<uint32_t>(r[1])};
}
__device__ __forceinline__ float sum16(float v) {
    const RowPair r = pair16(__float_as_uint(v));
    return __uint_as_float(r.lo) + __uint_as_float(r.hi);
}
__device__ __forceinline__ float sum32(float v) {
    const RowPair r = pair32(__float_as_uint(v));
    return __uint_as_float(r.lo) + __uint_as_float(r.hi);
}

// Sum over each aligned group of L lanes; every lane of a group gets the group's sum.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(L == 1 || L == 2 || L == 4 || L == 8 || L == 16 || L == 32 || L == 64, "L");
    if constexpr (L >= 2) v += dpp_f32<dpp::kXor1>(v);
    if constexpr (L >= 4) v += dpp_f32<dpp::kXor2>(v);
    if constexpr (L >= 8) v += dpp_f32<dpp::kHalfMirror>(v);
    if constexpr (L >= 16) v += dpp_f32<dpp::kRor8>(v);
    if constexpr (L >= 32) v = sum16(v);
    if constexpr (L >= 64) v = sum32(v);
    return v;
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Unsigned max over each aligned group of L lanes.
template <int L>
__device__ __forceinline__ uint32_t group_max(uint32_t v) {
    if constexpr (L >= 2) v = umax(v, dpp_u32<dpp::kXor1>(v));
    if constexpr (L >= 4) v = umax(v, dpp_u32<dpp::kXor2>(v));
    if constexpr (L >= 8) v = umax(v, dpp_u32<dpp::kHalfMirror>(v));
    if constexpr (L >= 16) v = umax(v, dpp_u32<dpp::kRor8>(v));
    if constexpr (L >= 32) {
        const RowPair r = pair16(v);
        v = umax(r.lo, r.hi);
    }
    if constexpr (L >= 64) {
        const RowPair r = pair32(v);
        v = umax(r.lo, r.hi);
    }
    return v;
}

// Unsigned max over the whole wavefront of a value already uniform within aligned groups of L
// lanes: finish the row with DPP, join the four 16-lane rows with row_bcast:15 / row_bcast:31
// (gfx9 DPP), and read the result from lane 63.
template <int L>
__device__ __forceinline__ uint32_t wave_max_from_groups(uint32_t v) {
    if constexpr (L < 2) v = umax(v, dpp_u32<dpp::kXor1>(v));
    if constexpr (L < 4) v = umax(v, dpp_u32<dpp::kXor2>(v));
    if constexpr (L < 8) v = umax(v, dpp_u32<dpp::kHalfMirror>(v));
    if constexpr (L < 16) v = umax(v, dpp_u32<dpp::kRor8>(v));
    if constexpr (L < 32) {
        const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            static_cast<int>(v), static_cast<int>(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
        v = umax(v, a);
    }
    if constexpr (L < 64) {
        const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            static_cast<int>(v), static_cast<int>(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
        v = umax(v, a);
    }
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// ------------------------------------------------------------------------------------------
// Activations, branch-free, from exp2 and reciprocal (v_exp_f32 / v_rcp_f32, about 1 ulp each):
//   sigmoid(x) = 1 / (1 + 2^(-x log2 e))
//   tanh(x)    = 2 sigmoid(2x) - 1
// The tanh form has an absolute error of a few ulps of 1 everywhere (its relative error grows
// as |x| -> 0, where tanh(x) ~ x), well inside the 1e-5 parity bar |err| <= 1e-5 max(|want|, 1).
// Both saturate correctly: exp2 overflows to +inf (reciprocal 0) or underflows to 0.
// ------------------------------------------------------------------------------------------

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float fast_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2e * x));
}

__device__ __forceinline__ float fast_tanh(float x) {
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.0f * kLog2e * x));
    return 2.0f * s - 1.0f;
}

}  // namespace hsn
