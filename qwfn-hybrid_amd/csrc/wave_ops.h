// Wave-wide sums without LDS on gfx950: DPP within each row of 16 lanes (quad
// swaps, the mirrored half-row, the mirrored row), then across the rows with
// the permlane16 / permlane32 swaps. Every lane gets the sum. The f64 forms
// move both halves of a double with the same pattern.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qwfn {
namespace wave {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// x + the value of the lane that a permlane16 / permlane32 swap brings
template <bool P32>
__device__ __forceinline__ float swap_add(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = P32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false) : __builtin_amdgcn_permlane16_swap(u, u, false, false);
    unsigned p = r[0], q = r[1];
    asm volatile("" : "+v"(p), "+v"(q));
    return __builtin_bit_cast(float, p) + __builtin_bit_cast(float, q);
}

// sum over the wave, in every lane: within each row of 16 (quad swaps, the
// mirrored half-row, the mirrored row), then across rows (permlane swaps)
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_f<0xB1>(x);    // quad_perm [1,0,3,2]
    x += dpp_f<0x4E>(x);    // quad_perm [2,3,0,1]
    x += dpp_f<0x141>(x);   // row_half_mirror
    x += dpp_f<0x140>(x);   // row_mirror
    x = swap_add<false>(x);
    return swap_add<true>(x);
}

// the same for a double: both halves move with the same pattern
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) (u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);
}
template <bool P32>
__device__ __forceinline__ double swap_add_d(double x) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const unsigned lo = (unsigned) u, hi = (unsigned) (u >> 32);
    const auto rl = P32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false) : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = P32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false) : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    unsigned l0 = rl[0], l1 = rl[1], h0 = rh[0], h1 = rh[1];
    asm volatile("" : "+v"(l0), "+v"(l1), "+v"(h0), "+v"(h1));
    return __builtin_bit_cast(double, ((uint64_t) h0 << 32) | l0) + __builtin_bit_cast(double, ((uint64_t) h1 << 32) | l1);
}
__device__ __forceinline__ double wave_sum_d(double x) {
    x += dpp_d<0xB1>(x);
    x += dpp_d<0x4E>(x);
    x += dpp_d<0x141>(x);
    x += dpp_d<0x140>(x);
    x = swap_add_d<false>(x);
    return swap_add_d<true>(x);
}

// sum over the 16 lanes of each DPP row (every lane of the row gets its row's sum)
__device__ __forceinline__ double row16_sum_d(double x) {
    x += dpp_d<0xB1>(x);
    x += dpp_d<0x4E>(x);
    x += dpp_d<0x141>(x);
    x += dpp_d<0x140>(x);
    return x;
}

}  // namespace wave
}  // namespace qwfn
