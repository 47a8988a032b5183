// Device helpers shared by the window kernels (gfx950 / CDNA4, 64-lane wavefronts).
//
// Everything here is written for one wavefront of 64 lanes: cross-lane work uses the
// wavefront-wide shuffle / ballot intrinsics, never 32-lane warp idioms.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hsn_window.h"

namespace hsn {

constexpr int kWave = 64;

// ------------------------------------------------------------------------------------------
// Storage types. fp32 state is the rule; inputs and per-slot outputs may be stored as bf16
// (upper half of an fp32, widened exactly, narrowed round-to-nearest-even).
// ------------------------------------------------------------------------------------------

struct bf16_t {
    uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);

template <>
__device__ __forceinline__ float from_f32<float>(float x) {
    return x;
}

// Round-to-nearest-even narrowing of an fp32 to bf16 (the IEEE rounding every framework uses
// for this cast): gfx950's v_cvt_pk_bf16_f32, one instruction under the default round-to-nearest
// mode with fp32 denormals kept; a NaN stays a NaN.
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
    bf16_t r;
    r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
    return r;
}

__device__ __forceinline__ float to_f32(_Float16 x) { return static_cast<float>(x); }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) {
    return static_cast<_Float16>(x);
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p, int64_t i) {
    return to_f32(p[i]);
}

template <typename T>
__device__ __forceinline__ void store_f32(T* p, int64_t i, float v) {
    p[i] = from_f32<T>(v);
}

// ------------------------------------------------------------------------------------------
// Wavefront primitives.
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ float wave_shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ int wave_shfl_xor(int v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ uint32_t wave_shfl_xor(uint32_t v, int mask) {
    return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), mask, kWave));
}

__device__ __forceinline__ int readlane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ uint32_t readlane(uint32_t v, int lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
__device__ __forceinline__ float readlane(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// A branch taken rarely (a reset, a padded slot, a new slice maximum). The hint moves its block
// out of the straight-line code of an unrolled loop, so the hot path stays contiguous in the
// instruction cache instead of jumping over the cold code at every step.
__device__ __forceinline__ bool unlikely(bool c) { return __builtin_expect(c, false); }

// Number of set bits of `mask` below this lane (an exclusive prefix count).
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

// ------------------------------------------------------------------------------------------
// Floating point with the reductions' NaN conventions.
// ------------------------------------------------------------------------------------------

// min / max that return NaN when either operand is NaN (torch's amin / amax).
__device__ __forceinline__ float nan_min(float a, float b) {
    return (a != a || b != b) ? __int_as_float(0x7fc00000) : fminf(a, b);
}
__device__ __forceinline__ float nan_max(float a, float b) {
    return (a != a || b != b) ? __int_as_float(0x7fc00000) : fmaxf(a, b);
}

// A total order on fp32 scores as a stable descending sort sees them: NaN above +inf (all NaNs
// equal), -0 equal to +0, otherwise the numeric order. Larger key = earlier in the order.
// Selects only (no branch): a negative score flips every bit, a non-negative one sets the top bit.
__device__ __forceinline__ uint32_t score_key(float s) {
    const uint32_t u0 = __float_as_uint(s);
    const uint32_t u = u0 == 0x80000000u ? 0u : u0;  // -0 sorts with +0
    const uint32_t k = u ^ (static_cast<uint32_t>(static_cast<int32_t>(u) >> 31) | 0x80000000u);
    return s != s ? 0xffffffffu : k;
}
constexpr uint32_t kKeyPosInf = 0xff800000u;  // score_key(+inf)

// The row's max |h| is kept as the integer order of the bit patterns of |h| (non-negative
// floats order like their bits; any NaN is above +inf, so a NaN anywhere wins).
__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

// ------------------------------------------------------------------------------------------
// Activations of the round: the candidate c = tanh(pre) and the write gate b = sigmoid(gate).
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ float act_tanh(float x) { return tanhf(x); }
__device__ __forceinline__ float act_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace hsn
