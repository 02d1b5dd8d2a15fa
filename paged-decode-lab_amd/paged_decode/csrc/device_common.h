// Device-side building blocks shared by the partition and merge kernels of
// the gfx950 decode library: vector types, wave64 lane primitives (DPP,
// ds_swizzle, permlane swaps), the exp2 used for the softmax, and the element
// type of the FP32 vector-ALU kernel. Included by every translation unit of
// the library (decode.hip and the partial_*.hip format units).
#ifndef PAGED_DECODE_DEVICE_COMMON_H
#define PAGED_DECODE_DEVICE_COMMON_H

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "paged_decode.h"
#include "partition_map.h"

namespace pd {

constexpr float kNoToken = -FLT_MAX;  // running max before any live token
constexpr float kLog2e = 1.4426950408889634f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Note: reinterpret whole vectors (bit_cast of a u32x4 to f16x8 / f32x4), never
// a single element: clang 22 lowers __builtin_bit_cast of a vector-element
// lvalue to a read of element 0.

// ---------------------------------------------------------------------------
// Wave64 lane primitives.
// DPP controls: quad_perm [1,0,3,2] and [2,3,0,1] swap neighbours at distance
// 1 and 2; row_half_mirror reverses each 8-lane half-row; row_mirror reverses
// each 16-lane row. Applied in that order, a sum/max reaches every lane of an
// aligned 8- or 16-lane group. ds_swizzle in bit mode with xor 0x10 exchanges
// lanes 16 apart within each 32-lane half.
constexpr int kDppQuadSwap1 = 0xB1;
constexpr int kDppQuadSwap2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kSwizzleSwap16 = 0x401F;

template <int kCtrl>
__device__ __forceinline__ float dpp_move(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float swizzle_swap16(float x) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), kSwizzleSwap16));
}

// Sum over each aligned group of kLanes (8, 16 or 32) lanes, result in every lane.
template <int kLanes>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(kLanes == 8 || kLanes == 16 || kLanes == 32, "unsupported group");
    x += dpp_move<kDppQuadSwap1>(x);
    x += dpp_move<kDppQuadSwap2>(x);
    x += dpp_move<kDppRowHalfMirror>(x);
    if constexpr (kLanes >= 16) x += dpp_move<kDppRowMirror>(x);
    if constexpr (kLanes >= 32) x += swizzle_swap16(x);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_move<kDppQuadSwap1>(x));
    x = fmaxf(x, dpp_move<kDppQuadSwap2>(x));
    x = fmaxf(x, dpp_move<kDppRowHalfMirror>(x));
    x = fmaxf(x, dpp_move<kDppRowMirror>(x));
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
    x = group_sum<16>(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// gfx950 v_permlane32_swap / v_permlane16_swap on float pairs. For (a, b):
//   swap32: lanes 0-31 get (a[l], a[l+32]), lanes 32-63 get (b[l-32], b[l]);
//   swap16: even 16-lane rows get (a[l], a[l+16]), odd rows (b[l-16], b[l]).
// The pair's sum is a + partner's a in the lower half (even rows) and
// b + partner's b in the upper half (odd rows): one reduce-scatter step.
// The builtins return a two-element vector; its elements are copied into
// scalars before the bit cast (a bit cast of a vector-element lvalue reads
// element 0 with this compiler).
struct FloatPair {
    float first, second;
};

__device__ __forceinline__ FloatPair permlane32_swap(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                    false, false);
    const unsigned first = r[0], second = r[1];
    return {__builtin_bit_cast(float, first), __builtin_bit_cast(float, second)};
}

__device__ __forceinline__ FloatPair permlane16_swap(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                    false, false);
    const unsigned first = r[0], second = r[1];
    return {__builtin_bit_cast(float, first), __builtin_bit_cast(float, second)};
}

__device__ __forceinline__ float swap32_sum(float a, float b) {
    const FloatPair r = permlane32_swap(a, b);
    return r.first + r.second;
}

__device__ __forceinline__ float swap16_sum(float a, float b) {
    const FloatPair r = permlane16_swap(a, b);
    return r.first + r.second;
}

// Max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48, result in every lane.
__device__ __forceinline__ float max_over_lane_groups(float x) {
    const FloatPair r = permlane32_swap(x, x);
    x = fmaxf(r.first, r.second);
    const FloatPair s = permlane16_swap(x, x);
    return fmaxf(s.first, s.second);
}

__device__ __forceinline__ float sum_over_lane_groups(float x) {
    x = swap32_sum(x, x);
    return swap16_sum(x, x);
}

// State j of a row, read as one 8-byte load. Callers clamp j into the row and
// mask the result, so loads are unconditional and issue back to back.
__device__ __forceinline__ float2 read_state(const float2* st, int j) {
    return __builtin_bit_cast(float2, reinterpret_cast<const uint64_t*>(st)[j]);
}

// ---------------------------------------------------------------------------
// Element types of the vector-ALU kernel. A lane moves 16 bytes per load: 4 floats.
template <typename T>
struct Elem;

template <>
struct Elem<float> {
    static constexpr int kPerLoad = 4;
    static __device__ __forceinline__ float dot(const u32x4& a, const u32x4& b) {
        const f32x4 af = __builtin_bit_cast(f32x4, a);
        const f32x4 bf = __builtin_bit_cast(f32x4, b);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = fmaf(af[i], bf[i], acc);
        return acc;
    }
    static __device__ __forceinline__ void widen(const u32x4& x, float (&f)[4]) {
        const f32x4 v = __builtin_bit_cast(f32x4, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = v[i];
    }
};

}  // namespace pd

#endif  // PAGED_DECODE_DEVICE_COMMON_H
