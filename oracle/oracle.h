/*
 * CPU oracle for the q8_0 KV-cache path. TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it. The product path (libqwfn_kv.so) never
 * links, loads or calls it.
 *
 * It restates, in plain C, the ggml-cpu semantics the reference engine relies on
 * (ggml from unslothai/llama.cpp @ ca1426903, not vendored in the reference tree,
 * see scripts/build.sh:8-16 and CMakeLists.txt:20-31 of the reference):
 *   - block_q8_0 = { fp16 d; int8 qs[32]; }  (34 bytes per 32 values)
 *   - quantize_row_q8_0: scalar "_ref" variant and the x86 AVX/AVX2 variant
 *   - dequantize_row_q8_0, vec_dot_q8_0_q8_0 (scalar and x86 summation order)
 *   - set_rows / cpy F32 -> Q8_0 (reference call sites qwfn_graph.cpp:370-384,
 *     :612-628), get_rows on I32 words (qwfn_graph.cpp:632-645)
 *   - flash_attn_ext, the CPU one-chunk loop (Q requantised to q8_0, online
 *     softmax with expf, V dequantised to F32), as called at qwfn_graph.cpp:469
 *     and :698
 *   - an fp64 textbook attention used as a second referee
 *   - snapshot part layout (qwfn_engine.cpp:988-999)
 *
 * Pinning status of each function is recorded next to its declaration.
 */
#ifndef QWFN_ORACLE_H
#define QWFN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_QK8_0 32
#define ORACLE_Q8_0_BLOCK_BYTES 34

enum { ORACLE_Q8_REF = 0, ORACLE_Q8_X86 = 1 };

/* ---- deterministic PRNG: SplitMix64-seeded xoshiro256**, Box-Muller in double ----
 * Pinned by the published xoshiro256** / SplitMix64 reference outputs (tests). */
typedef struct { uint64_t s[4]; } oracle_rng;
void     oracle_rng_seed(oracle_rng * r, uint64_t seed);
uint64_t oracle_rng_next(oracle_rng * r);
uint64_t oracle_splitmix64(uint64_t * state);
/* stream key for per-tensor sub-streams: hash(seed, a, b, c) */
uint64_t oracle_stream_key(uint64_t seed, uint64_t a, uint64_t b, uint64_t c);
/* n normal values N(0, stddev^2) rounded to float */
void oracle_fill_normal(uint64_t key, float * out, int64_t n, double stddev);
/* n uniform values in [0, 1) as float (top 24 bits) */
void oracle_fill_uniform(uint64_t key, float * out, int64_t n);

/* ---- fp16 <-> fp32, IEEE round-to-nearest-even (ggml's GGML_FP32_TO_FP16).
 * Pinned against numpy.float16 over all 2^16 patterns and random floats. */
uint16_t oracle_fp32_to_fp16(float f);
float    oracle_fp16_to_fp32(uint16_t h);

/* ---- q8_0 quantisation.  variant: ORACLE_Q8_REF or ORACLE_Q8_X86.
 * Pinned by closed-form invariants, crafted tie / 1-ulp cases, brute force. */
void  oracle_quantize_row_q8_0(const float * x, void * y, int64_t k, int variant);
void  oracle_dequantize_row_q8_0(const void * x, float * y, int64_t k);
/* variant selects the summation order: REF = scalar, X86 = AVX2 8-lane fma order */
float oracle_vec_dot_q8_0_q8_0(int64_t n, const void * x, const void * y, int variant);

/* ---- set_rows / cpy / get_rows.  Return 0 or a negative error code. ---- */
int oracle_set_rows_q8_0(void * dst, size_t dst_nb1, int64_t dst_rows,
                         const float * src, size_t src_nb1, int64_t ne0,
                         const int32_t * idx, int64_t n, int variant);
int oracle_cpy_f32_q8_0(void * dst, size_t dst_nb1, int64_t first_row, int64_t dst_rows,
                        const float * src, size_t src_nb1, int64_t ne0, int64_t n, int variant);
int oracle_get_rows(const void * src, size_t src_nb1, int64_t src_rows, size_t row_bytes,
                    const int32_t * idx, int64_t n, void * dst, size_t dst_nb1);

/* ---- attention ----
 * A ggml-style view: ne[4] elements, nb[4] byte strides. For q8_0 tensors
 * ne[0] counts values and nb[0] is 34 (one block). */
typedef struct {
    const void * data;
    int64_t ne[4];
    size_t  nb[4];
} oracle_view;

/* ggml flash_attn_ext (CPU one-chunk loop), F32 Q, q8_0 K/V, optional F16 mask.
 * dst is F32 [DV, n_head, T, B] contiguous.  q_variant / dot_variant select the
 * quantiser used for Q and the vec_dot summation order.  n_threads >= 1. */
int oracle_flash_attn_ext_q8_0(const oracle_view * q, const oracle_view * k, const oracle_view * v,
                               const oracle_view * mask, float scale, float * dst,
                               int q_variant, int dot_variant, int n_threads);

/* fp64 textbook softmax(Q K^T * scale + mask) V over dequantised K/V.
 * quantize_q: 0 uses the F32 Q as given, 1/2 requantises Q with REF/X86 first.
 * Fully masked rows give 0 (as ggml).  dst as above, in double. */
int oracle_attn_f64(const oracle_view * q, const oracle_view * k, const oracle_view * v,
                    const oracle_view * mask, double scale, double * dst, int quantize_q);

/* ---- QSA index producer (qwfn_graph.cpp:282-301 qsa_pool_blocks, :529-554
 * qsa_dec_index, :478-495 qsa_pool_rebuild) ----
 * ggml_rms_norm (ggml-cpu): the squares summed in double, mean = (float)
 * (sum / n), y = x * (1.0f / sqrtf(mean + eps)).  Pinned by its closed form. */
void oracle_rms_norm_f32(const float * x, float * y, int64_t n, float eps);
/* ggml_rope_multi on one head of ne0 values, GGML_ROPE_TYPE_IMROPE (imrope = 1)
 * or MROPE (imrope = 0), freq_scale 1, ext_factor 0, attn_factor 1: the first
 * n_dims values rotate in neox pairs (i, i + n_dims/2); pair i turns by
 * theta_s * theta_scale^i (a running float product) for the position of its
 * section s, theta_scale = powf(freq_base, -2/n_dims); the rest pass through.
 * pos = {t, h, w, e}.  Pinned by the reduction to standard neox rope at equal
 * positions, norm preservation, relative-position invariance and an fp64
 * restatement (tests). */
void oracle_rope_multi_f32(const float * x, float * y, int64_t ne0, int n_dims, const int32_t pos[4],
                           const int sections[4], int imrope, float freq_base);
/* F32 rows to F16 rows (ggml_set_rows into an F16 tensor): dst row idx[i] =
 * fp16(src row i).  Returns 0, or -1 for an index outside [0, dst_rows). */
int oracle_set_rows_f16(uint16_t * dst, int64_t dst_rows, int64_t ne0, const float * src, const int32_t * idx,
                        int64_t n);
/* qsa_pool_blocks for n_blk blocks: block b pools the F16 index-cache rows
 * members[b*r .. b*r+r-1] (mean: sequential adds, then * (1.0f/r)), RMS-norms
 * with eps, multiplies by k_norm_w, ropes at pos4[4*b .. 4*b+3] (t, h, w, e),
 * and stores fp16 of the result at out[b]. */
void oracle_qsa_pool_blocks(const uint16_t * ic, int64_t idx_dim, const int32_t * members, int64_t r, int64_t n_blk,
                            const float * k_norm_w, const int32_t * pos4, const int sections[4], float eps,
                            float freq_base, int n_dims, uint16_t * out);

/* The attention layer's K/V producer (qwfn_graph.cpp:441-451, :129-132,
 * :370-384) for T tokens: K = attn_k . cur, V = attn_v . cur with F16
 * weights [kv_dim][E] and cur rounded to F16 (ggml_mul_mat's conversion of
 * src1), the products summed in double and rounded to float (ggml-cpu sums in
 * float lanes: the difference is float rounding); each 256-value K head RMS
 * normed, times k_norm_w, IMROPE at pos[s*T + t]; then both quantised (q8_0,
 * variant) into k_rows / v_rows (T rows of kv_dim/32*34 bytes). k_f32 / v_f32
 * (may be NULL) receive the float rows before quantisation. */
void oracle_kv_produce_q8_0(const float * cur, int64_t E, int64_t T, const uint16_t * wk, const uint16_t * wv,
                            int64_t kv_dim, const float * k_norm_w, const int32_t * pos, const int sections[4],
                            int n_dims, float freq_base, float eps, void * k_rows, void * v_rows, float * k_f32,
                            float * v_f32, int variant, int w_bf16);
/* w_bf16: the weights are BF16 bits and the rows are rounded to BF16 (round
 * to nearest even) instead of F16. */
uint16_t oracle_fp32_to_bf16(float f);
float    oracle_bf16_to_fp32(uint16_t h);

/* Gated delta rule (ggml_gated_delta_net as qwfn_graph.cpp:258 calls it; the
 * op lives in the reference's llama.cpp fork, absent here, so this restates
 * the published recurrence of Gated DeltaNet -- Yang, Kautz, Hatamizadeh
 * 2024, as HF Qwen3-Next's recurrent form writes it): per value head h
 * (key head h / (n_v / n_k)), state S [dk][dv] (dv contiguous), token t:
 *   S = S * exp(g[t][h]);  m[c] = sum_r S[r][c] k[r]
 *   S[r][c] += k[r] * (v[c] - m[c]) * beta[t][h]
 *   out[t][h][c] = sum_r S[r][c] * q[r] * scale
 * q, k: [T][n_k][dk] at token strides q_ts / k_ts floats; v: [T][n_v][dv] at
 * v_ts; g, beta: [T][n_v]; state [n_v][dk][dv] in/out (the final state);
 * snap (may be NULL): n_snap slots of [n_v][dk][dv], slot s-1 the state s
 * tokens back (after token T-1-s), s = 1 .. n_snap <= T-1 (the rollback
 * snapshots of deltanet_write_state, :208-238). Sums run over r in order, in
 * float. */
void oracle_gated_delta_net(const float * q, int64_t q_ts, const float * k, int64_t k_ts, const float * v, int64_t v_ts,
                            const float * g, const float * beta, float * state, float * out, float * snap,
                            int64_t n_snap, int64_t T, int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, float scale);

#ifdef __cplusplus
}
#endif
#endif
