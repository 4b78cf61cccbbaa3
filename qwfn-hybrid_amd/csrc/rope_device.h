// Device-side RMS norm and multi-section rotary embedding with ggml-cpu's
// float arithmetic (ggml_rms_norm; ggml_rope_multi with GGML_ROPE_TYPE_IMROPE,
// as graph_builder::rope and qsa_pool_blocks call it, qwfn_graph.cpp:129-132,
// :297-299): freq_scale 1, ext_factor 0, attn_factor 1.
//
// Rope pair k (values k and k + n_dims/2, neox order) of a head turns by
// theta_s(k) = pos_s * theta_scale^k, the power being the running float
// product ggml forms pair by pair (theta_scale = powf(freq_base, -2/n_dims),
// computed on the host with the C library, as ggml does). The section s of a
// pair follows Qwen3-VL's interleaved layout for IMROPE (t, h, w, t, h, w, ...
// within sections[0..2] each, then e) or contiguous sections for MROPE. cos
// and sin are taken in double and rounded to float (correctly rounded).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qwfn {

struct rope_params {
    int32_t n_dims;         // rotated values per head (even)
    int32_t sections[4];    // t, h, w, e
    int32_t imrope;         // 1: interleaved sections (IMROPE), 0: contiguous (MROPE)
    float   theta_scale;    // powf(freq_base, -2.0f / n_dims)
};

__host__ __device__ inline int rope_section(const rope_params & p, int k) {
    const int sect_dims = p.sections[0] + p.sections[1] + p.sections[2] + p.sections[3];
    const int sector = k % sect_dims;
    if (p.imrope) {
        if (sector % 3 == 1 && sector < 3 * p.sections[1]) return 1;
        if (sector % 3 == 2 && sector < 3 * p.sections[2]) return 2;
        if (sector % 3 == 0 && sector < 3 * p.sections[0]) return 0;
        return 3;
    }
    const int sec_w = p.sections[0] + p.sections[1];
    return sector < p.sections[0] ? 0 : sector < sec_w ? 1 : sector < sec_w + p.sections[2] ? 2 : 3;
}

// cos and sin of pair k's angle for positions pos[4] (t, h, w, e)
__device__ inline void rope_cos_sin(const rope_params & p, const int32_t pos[4], int k, float * c, float * s) {
    float th = (float) pos[rope_section(p, k)];
    for (int j = 0; j < k; j++) th = __fmul_rn(th, p.theta_scale);
    double sd, cd;
    sincos((double) th, &sd, &cd);
    *c = (float) cd;
    *s = (float) sd;
}

// (x0, x1) of pair k rotated: x0 c - x1 s, x0 s + x1 c, each product rounded
// before the sum (no contraction)
__device__ inline void rope_rotate(float x0, float x1, float c, float s, float * y0, float * y1) {
    *y0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    *y1 = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
}

}  // namespace qwfn
