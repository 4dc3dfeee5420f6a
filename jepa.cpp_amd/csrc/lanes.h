// lanes.h - cross-lane helpers for wave64 on gfx950.
#pragma once
#include <hip/hip_runtime.h>

// f(x[l], x[l ^ 32]) in every lane l, for a commutative f: v_permlane32_swap exchanges the two
// 32-lane halves of a register pair in the VALU, without the LDS round trip of ds_bpermute
// (__shfl_xor) and its latency. Both halves see the same operand pair, so lane l and lane l ^ 32
// get the same bits.
__device__ __forceinline__ float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The same for values that are never NaN, with a plain v_max_f32: fmaxf on the swapped values would
// first canonicalize both (IEEE mode), two more VALU ops.
__device__ __forceinline__ float halves_max_nonan(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    float m;
    asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(r[0]), "v"(r[1]));
    return m;
}
__device__ __forceinline__ float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ uint32_t halves_min_u32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return min((uint32_t) r[0], (uint32_t) r[1]);
}
