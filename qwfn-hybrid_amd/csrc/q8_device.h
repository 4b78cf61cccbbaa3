// Device helpers for ggml's q8_0 format on gfx950 (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qwfn {
namespace dev {

// DPP controls (GCN/CDNA encoding).
constexpr int DPP_QUAD_1032   = 0xB1;   // quad_perm [1,0,3,2]: lane ^ 1
constexpr int DPP_QUAD_2301   = 0x4E;   // quad_perm [2,3,0,1]: lane ^ 2
constexpr int DPP_HALF_MIRROR = 0x141;  // row_half_mirror: lane i <-> 7-i within 8

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t) __builtin_amdgcn_update_dpp((int) v, (int) v, CTRL, 0xF, 0xF, false);
}

// x86 AVX/AVX2 quantize_row_q8_0 element: _mm256_round_ps(NEAREST) (ties to
// even) then _mm256_cvtps_epi32 (out of int32 range or NaN -> 0x80000000) and
// the two saturating packs to int8.
__device__ __forceinline__ int32_t q8_round_x86(float v) {
    const float r = __builtin_rintf(v);
    if (!(__builtin_fabsf(r) < 2147483648.0f)) return -128;
    const int32_t i = (int32_t) r;
    return i > 127 ? 127 : (i < -128 ? -128 : i);
}

// quantize_row_q8_0_ref element: roundf (ties away from zero).
__device__ __forceinline__ int32_t q8_round_ref(float v) {
    float r = roundf(v);
    if (!(r == r)) r = 0.0f;
    r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
    return (int32_t) r;
}

// Scale and inverse scale of one block from its amax, per variant.
//   d  = amax / 127                       (both variants; stored as fp16 RNE)
//   id = amax ? 127 / amax : 0            (x86)
//   id = d ? 1 / d : 0                    (ref)
// IEEE division: hipcc keeps fp32 '/' correctly rounded by default.
struct q8_scale { float d; float id; };

__device__ __forceinline__ q8_scale q8_block_scale(float amax, bool x86) {
    q8_scale s;
    s.d = amax / 127.0f;
    if (x86) s.id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else     s.id = s.d != 0.0f ? 1.0f / s.d : 0.0f;
    return s;
}

// The low bytes of four int32 in one dword (byte j from q[j]): two byte
// permutes and an or.
__device__ __forceinline__ uint32_t pack_low_bytes(const int32_t q[4]) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t) q[1], (uint32_t) q[0], 0x0c0c0400u);   // q0.b0, q1.b0, 0, 0
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t) q[3], (uint32_t) q[2], 0x04000c0cu);   // 0, 0, q2.b0, q3.b0
    return lo | hi;
}

__device__ __forceinline__ uint32_t q8_pack4(const float x[4], float id, bool x86) {
    int32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float v = x[j] * id;
        q[j] = x86 ? q8_round_x86(v) : q8_round_ref(v);
    }
    return pack_low_bytes(q);
}

// x86 element for a block whose amax is a finite float of at least 2^-100:
// then |x * id| <= 127 * (1 + 2^-22), so rint lands in [-127, 127] and neither
// the range check nor the saturation of q8_round_x86 can act.
__device__ __forceinline__ uint32_t q8_pack4_x86_normal(const float x[4], float id) {
    int32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) q[j] = (int32_t) __builtin_rintf(x[j] * id);
    return pack_low_bytes(q);
}
constexpr uint32_t Q8_AMAX_NORMAL_MIN = 0x0d800000u;   // 2^-100 as float bits

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16) f);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float) __builtin_bit_cast(_Float16, h);
}

// Quantise V consecutive values held by this lane as part of a 32-value block
// spread over L = 32 / V consecutive lanes (lane % L == position of the group).
// w[m] gets the packed int8 quads of values 4m .. 4m+3; *d16 the block's fp16
// scale bits and *dq its fp32 value (fp16 -> fp32, as ggml's vec_dot reads it).
template <int V>
__device__ __forceinline__ void q8_quantize_lanes(const float (&x)[V], bool x86, uint32_t (&w)[V / 4], uint16_t * d16,
                                                  float * dq) {
    static_assert(V == 4 || V == 8 || V == 16 || V == 32, "a block is 32 values");
    constexpr int L = 32 / V;
    // |x| max over the block: non-negative IEEE floats order like their bit
    // patterns, so an unsigned max is exact; the lanes of a block combine by
    // quad butterfly, then the two quads of each half-row
    uint32_t am = 0;
#pragma unroll
    for (int j = 0; j < V; j++) am = max(am, __builtin_bit_cast(uint32_t, x[j]) & 0x7fffffffu);
    if constexpr (L >= 2) am = max(am, dpp_u32<DPP_QUAD_1032>(am));
    if constexpr (L >= 4) am = max(am, dpp_u32<DPP_QUAD_2301>(am));
    if constexpr (L >= 8) am = max(am, dpp_u32<DPP_HALF_MIRROR>(am));
    const float amax = __builtin_bit_cast(float, am);
    const q8_scale s = q8_block_scale(amax, x86);
    *d16 = f32_to_f16_bits(s.d);
    *dq = f16_bits_to_f32(*d16);
    if (x86 && am >= Q8_AMAX_NORMAL_MIN && am < 0x7f800000u) {
#pragma unroll
        for (int m = 0; m < V / 4; m++) w[m] = q8_pack4_x86_normal(&x[4 * m], s.id);
    } else {
#pragma unroll
        for (int m = 0; m < V / 4; m++) w[m] = q8_pack4(&x[4 * m], s.id, x86);
    }
}

// The same for 4 values per lane over 8 lanes; returns the packed quad.
__device__ __forceinline__ uint32_t q8_quantize_lane4(const float x[4], bool x86, uint16_t * d16, float * dq) {
    const float (&xv)[4] = *reinterpret_cast<const float (*)[4]>(x);
    uint32_t w[1];
    q8_quantize_lanes<4>(xv, x86, w, d16, dq);
    return w[0];
}

}  // namespace dev
}  // namespace qwfn
