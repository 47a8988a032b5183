// Buffer-resource loads and stores (MUBUF) for the sweeps.
//
// A row's tensor is one buffer resource (its base and byte size in SGPRs). A lane addresses its
// element with a 32-bit voffset and the position with a uniform soffset (an SGPR), so a load or
// a store costs no per-lane address arithmetic. Raw buffers check voffset against the size: a
// voffset past it (kOob) reads 0 and drops a store, which masks inactive lanes without a branch,
// and a resource of size 0 (an absent optional tensor) reads zeros and drops every store. The
// soffset is not part of that check on this architecture family: every soffset stays inside the
// tensor's row, and only the voffset masks.
#pragma once

#include "common.cuh"

namespace hsn {

using rsrc_t = __amdgpu_buffer_rsrc_t;

constexpr uint32_t kOob = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // the gfx9 raw-buffer descriptor's fourth word

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), kRsrcWord3);
}

template <typename T>
__device__ __forceinline__ T bload(rsrc_t r, uint32_t voff, uint32_t soff);

template <>
__device__ __forceinline__ float bload<float>(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
template <>
__device__ __forceinline__ bf16_t bload<bf16_t>(rsrc_t r, uint32_t voff, uint32_t soff) {
    bf16_t v;
    v.bits = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
    return v;
}
template <>
__device__ __forceinline__ int32_t bload<int32_t>(rsrc_t r, uint32_t voff, uint32_t soff) {
    return static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
template <>
__device__ __forceinline__ int64_t bload<int64_t>(rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    return static_cast<int64_t>((static_cast<uint64_t>(v[1]) << 32) | v[0]);
}
template <>
__device__ __forceinline__ uint8_t bload<uint8_t>(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
}

__device__ __forceinline__ void bstore(float v, rsrc_t r, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
}
__device__ __forceinline__ void bstore(bf16_t v, rsrc_t r, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b16(v.bits, r, voff, soff, 0);
}

template <typename T>
__device__ __forceinline__ void bstore_f32(float v, rsrc_t r, uint32_t voff, uint32_t soff) {
    bstore(from_f32<T>(v), r, voff, soff);
}

}  // namespace hsn
