/*
 * CPU oracle for the q8_0 KV-cache path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg to check results,
 * never by the product library.
 *
 * Restates ggml-cpu semantics (ggml from unslothai/llama.cpp @ ca1426903, MIT
 * licence; not present in the reference tree or in this image) for:
 *   block_q8_0, quantize_row_q8_0[_ref], dequantize_row_q8_0,
 *   ggml_vec_dot_q8_0_q8_0, set_rows/cpy F32->Q8_0, get_rows (I32),
 *   flash_attn_ext one-chunk CPU loop, rms_norm, rope_multi (IMROPE),
 *   set_rows F32->F16, the QSA block pooling, the attention layer's K/V
 *   producer and the gated delta rule (ggml_gated_delta_net, an op of the
 *   reference's ggml fork: parity unpinned, see oracle_gated_delta_net).
 * The reference's use of them: qwfn_graph.cpp:370-384 (cpy append),
 * :612-628 (set_rows append), :632-645 (raw get_rows gather), :458-475 and
 * :697-701 (flash_attn_ext), qwfn_state.cpp:48-91 (cache layout).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off; FMAs are written out
 * explicitly where ggml's x86 build emits them).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ PRNG */

uint64_t oracle_splitmix64(uint64_t * state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void oracle_rng_seed(oracle_rng * r, uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; i++) r->s[i] = oracle_splitmix64(&sm);
}

uint64_t oracle_rng_next(oracle_rng * r) {
    uint64_t * s = r->s;
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

uint64_t oracle_stream_key(uint64_t seed, uint64_t a, uint64_t b, uint64_t c) {
    uint64_t st = seed ^ 0x51ed270b27a3c1f5ULL;
    uint64_t h = oracle_splitmix64(&st);
    st = h ^ (a * 0x9e3779b97f4a7c15ULL); h = oracle_splitmix64(&st);
    st = h ^ (b * 0xc2b2ae3d27d4eb4fULL); h = oracle_splitmix64(&st);
    st = h ^ (c * 0x165667b19e3779f9ULL); h = oracle_splitmix64(&st);
    return h;
}

void oracle_fill_normal(uint64_t key, float * out, int64_t n, double stddev) {
    oracle_rng r;
    oracle_rng_seed(&r, key);
    const double two_pi = 6.283185307179586476925286766559;
    int64_t i = 0;
    while (i < n) {
        /* u1 in (0, 1], u2 in [0, 1) */
        const double u1 = (double) ((oracle_rng_next(&r) >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double) (oracle_rng_next(&r) >> 11) * 0x1.0p-53;
        const double rad = sqrt(-2.0 * log(u1));
        out[i++] = (float) (stddev * rad * cos(two_pi * u2));
        if (i < n) out[i++] = (float) (stddev * rad * sin(two_pi * u2));
    }
}

void oracle_fill_uniform(uint64_t key, float * out, int64_t n) {
    oracle_rng r;
    oracle_rng_seed(&r, key);
    for (int64_t i = 0; i < n; i++) out[i] = (float) (oracle_rng_next(&r) >> 40) * 0x1.0p-24f;
}

/* ------------------------------------------------------------- fp16 */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_fp32_to_fp16(float f) {
    const uint32_t x    = f32_bits(f);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax   = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t) (sign | 0x7e00u);          /* NaN -> quiet NaN */
    if (ax == 0x7f800000u) return (uint16_t) (sign | 0x7c00u);         /* inf */
    if (ax < 0x38800000u) {
        /* below 2^-14: the f16 result is subnormal (or zero). Scaling by 2^24 is
         * exact; round the scaled value to an integer, ties to even. */
        const float scaled = bits_f32(ax) * 16777216.0f;
        const float r = nearbyintf(scaled);
        return (uint16_t) (sign | (uint16_t) r);                        /* 1024 -> 0x400, the min normal */
    }
    const int32_t  e = (int32_t) (ax >> 23) - 127 + 15;
    if (e >= 31) return (uint16_t) (sign | 0x7c00u);
    const uint32_t m   = ax & 0x7fffffu;
    uint32_t       h   = ((uint32_t) e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;            /* carry may reach inf: correct */
    return (uint16_t) (sign | h);
}

float oracle_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e    = ((uint32_t) h >> 10) & 0x1fu;
    const uint32_t m    = (uint32_t) h & 0x3ffu;
    if (e == 0) {
        const float v = (float) m * 0x1.0p-24f;                          /* exact */
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* ------------------------------------------------------------- q8_0 */

typedef struct { uint16_t d; int8_t qs[ORACLE_QK8_0]; } __attribute__((packed)) q8_block;
_Static_assert(sizeof(q8_block) == ORACLE_Q8_0_BLOCK_BYTES, "q8_0 block is 34 bytes");

/* _mm256_round_ps(.., NEAREST) + _mm256_cvtps_epi32 + packs_epi32 + packs_epi16:
 * ties to even; a value outside int32 (or NaN) becomes the integer-indefinite
 * 0x80000000, and the two saturating packs clamp to [-128, 127]. */
static inline int8_t q_x86(float v) {
    const float r = nearbyintf(v);
    int32_t i;
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) i = INT32_MIN;
    else i = (int32_t) r;
    if (i > 127) i = 127;
    if (i < -128) i = -128;
    return (int8_t) i;
}

/* quantize_row_q8_0_ref: roundf (ties away from zero) of x * (1/d). Values are
 * within [-127, 127] for finite inputs; the clamp only guards the conversion. */
static inline int8_t q_ref(float v) {
    float r = roundf(v);
    if (!(r == r)) r = 0.0f;
    if (r > 127.0f) r = 127.0f;
    if (r < -128.0f) r = -128.0f;
    return (int8_t) r;
}

void oracle_quantize_row_q8_0(const float * x, void * vy, int64_t k, int variant) {
    q8_block * y = (q8_block *) vy;
    const int64_t nb = k / ORACLE_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * ORACLE_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < ORACLE_QK8_0; j++) {
            const float a = fabsf(xb[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / 127.0f;
        y[i].d = oracle_fp32_to_fp16(d);
        if (variant == ORACLE_Q8_X86) {
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            for (int j = 0; j < ORACLE_QK8_0; j++) y[i].qs[j] = q_x86(xb[j] * id);
        } else {
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < ORACLE_QK8_0; j++) y[i].qs[j] = q_ref(xb[j] * id);
        }
    }
}

void oracle_dequantize_row_q8_0(const void * vx, float * y, int64_t k) {
    const q8_block * x = (const q8_block *) vx;
    const int64_t nb = k / ORACLE_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float d = oracle_fp16_to_fp32(x[i].d);
        for (int j = 0; j < ORACLE_QK8_0; j++) y[i * ORACLE_QK8_0 + j] = (float) x[i].qs[j] * d;
    }
}

float oracle_vec_dot_q8_0_q8_0(int64_t n, const void * vx, const void * vy, int variant) {
    const q8_block * x = (const q8_block *) vx;
    const q8_block * y = (const q8_block *) vy;
    const int64_t nb = n / ORACLE_QK8_0;
    if (variant == ORACLE_Q8_X86) {
        /* AVX2 order: 8 float lanes, lane l accumulates fma(dx*dy, sum of the
         * products of elements 4l..4l+3, acc); then hsum_float_8. */
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t ib = 0; ib < nb; ib++) {
            const float d = oracle_fp16_to_fp32(x[ib].d) * oracle_fp16_to_fp32(y[ib].d);
            for (int l = 0; l < 8; l++) {
                int32_t s = 0;
                for (int j = 4 * l; j < 4 * l + 4; j++) s += (int32_t) x[ib].qs[j] * (int32_t) y[ib].qs[j];
                acc[l] = fmaf(d, (float) s, acc[l]);
            }
        }
        const float r0 = acc[4] + acc[0], r1 = acc[5] + acc[1], r2 = acc[6] + acc[2], r3 = acc[7] + acc[3];
        const float s0 = r0 + r2, s1 = r1 + r3;
        return s0 + s1;
    }
    float sumf = 0.0f;
    for (int64_t ib = 0; ib < nb; ib++) {
        int32_t sumi = 0;
        for (int j = 0; j < ORACLE_QK8_0; j++) sumi += (int32_t) x[ib].qs[j] * (int32_t) y[ib].qs[j];
        const float dd = oracle_fp16_to_fp32(x[ib].d) * oracle_fp16_to_fp32(y[ib].d);
        const float t = (float) sumi * dd;
        sumf += t;
    }
    return sumf;
}

/* --------------------------------------------------- set_rows / cpy / get_rows */

int oracle_set_rows_q8_0(void * dst, size_t dst_nb1, int64_t dst_rows,
                         const float * src, size_t src_nb1, int64_t ne0,
                         const int32_t * idx, int64_t n, int variant) {
    if (ne0 % ORACLE_QK8_0) return -1;
    for (int64_t i = 0; i < n; i++)
        if (idx[i] < 0 || idx[i] >= dst_rows) return -2;
    for (int64_t i = 0; i < n; i++) {
        const float * row = (const float *) ((const char *) src + (size_t) i * src_nb1);
        oracle_quantize_row_q8_0(row, (char *) dst + (size_t) idx[i] * dst_nb1, ne0, variant);
    }
    return 0;
}

int oracle_cpy_f32_q8_0(void * dst, size_t dst_nb1, int64_t first_row, int64_t dst_rows,
                        const float * src, size_t src_nb1, int64_t ne0, int64_t n, int variant) {
    if (ne0 % ORACLE_QK8_0) return -1;
    if (first_row < 0 || first_row + n > dst_rows) return -2;
    for (int64_t i = 0; i < n; i++) {
        const float * row = (const float *) ((const char *) src + (size_t) i * src_nb1);
        oracle_quantize_row_q8_0(row, (char *) dst + (size_t) (first_row + i) * dst_nb1, ne0, variant);
    }
    return 0;
}

int oracle_get_rows(const void * src, size_t src_nb1, int64_t src_rows, size_t row_bytes,
                    const int32_t * idx, int64_t n, void * dst, size_t dst_nb1) {
    for (int64_t i = 0; i < n; i++)
        if (idx[i] < 0 || idx[i] >= src_rows) return -2;
    for (int64_t i = 0; i < n; i++)
        memcpy((char *) dst + (size_t) i * dst_nb1, (const char *) src + (size_t) idx[i] * src_nb1, row_bytes);
    return 0;
}

/* ------------------------------------------------------------- attention */

typedef struct {
    const oracle_view * q, * k, * v, * mask;
    float scale;
    float * dst;
    int q_variant, dot_variant;
    int64_t r0, r1;
} fa_job;

static void * fa_rows(void * arg) {
    const fa_job * J = (const fa_job *) arg;
    const oracle_view * q = J->q, * k = J->k, * v = J->v, * mask = J->mask;
    const int64_t DK = q->ne[0], DV = v->ne[0];
    const int64_t neq1 = q->ne[1], neq2 = q->ne[2];
    const int64_t nek1 = k->ne[1];
    const int64_t rk2 = neq2 / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    const int64_t rv2 = neq2 / v->ne[2], rv3 = q->ne[3] / v->ne[3];

    float * VKQ32 = (float *) malloc(sizeof(float) * (size_t) DV);
    float * V32   = (float *) malloc(sizeof(float) * (size_t) DV);
    q8_block * Q_q = (q8_block *) malloc(sizeof(q8_block) * (size_t) (DK / ORACLE_QK8_0));
    float * qrow  = (float *) malloc(sizeof(float) * (size_t) DK);

    for (int64_t ir = J->r0; ir < J->r1; ir++) {
        const int64_t iq3 = ir / (neq2 * neq1);
        const int64_t iq2 = (ir - iq3 * neq2 * neq1) / neq1;
        const int64_t iq1 = ir - iq3 * neq2 * neq1 - iq2 * neq1;

        float S = 0.0f;
        float M = -INFINITY;
        memset(VKQ32, 0, sizeof(float) * (size_t) DV);

        const uint16_t * mp = mask ? (const uint16_t *) ((const char *) mask->data + iq1 * mask->nb[1]
                                      + (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3])
                                   : NULL;
        const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3;
        const int64_t iv2 = iq2 / rv2, iv3 = iq3 / rv3;

        const char * pq = (const char *) q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3];
        for (int64_t d = 0; d < DK; d++) qrow[d] = *(const float *) (pq + d * q->nb[0]);
        oracle_quantize_row_q8_0(qrow, Q_q, DK, J->q_variant);

        for (int64_t ic = 0; ic < nek1; ic++) {
            const float mv = mp ? oracle_fp16_to_fp32(mp[ic]) : 0.0f;
            if (mv == -INFINITY) continue;

            const char * k_data = (const char *) k->data + ic * k->nb[1] + ik2 * k->nb[2] + ik3 * k->nb[3];
            float s = oracle_vec_dot_q8_0_q8_0(DK, k_data, Q_q, J->dot_variant);
            s = s * J->scale;
            s += mv;

            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            const char * v_data = (const char *) v->data + ic * v->nb[1] + iv2 * v->nb[2] + iv3 * v->nb[3];
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                for (int64_t d = 0; d < DV; d++) VKQ32[d] *= ms;
            } else {
                vs = expf(s - M);
            }
            oracle_dequantize_row_q8_0(v_data, V32, DV);
            for (int64_t d = 0; d < DV; d++) VKQ32[d] = fmaf(V32[d], vs, VKQ32[d]);
            S = fmaf(S, ms, vs);
        }

        const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
        for (int64_t d = 0; d < DV; d++) VKQ32[d] *= S_inv;

        /* dst [DV, n_head, T, B]: permute(0, 2, 1, 3) of the natural order */
        float * out = J->dst + (size_t) (iq3 * neq2 * neq1 + iq2 + iq1 * neq2) * (size_t) DV;
        memcpy(out, VKQ32, sizeof(float) * (size_t) DV);
    }
    free(VKQ32); free(V32); free(Q_q); free(qrow);
    return NULL;
}

static int fa_check(const oracle_view * q, const oracle_view * k, const oracle_view * v, const oracle_view * mask) {
    if (!q || !k || !v) return -1;
    if (q->ne[0] != k->ne[0] || q->ne[0] % ORACLE_QK8_0 || v->ne[0] % ORACLE_QK8_0) return -1;
    if (k->ne[1] != v->ne[1]) return -1;
    if (k->ne[2] <= 0 || q->ne[2] % k->ne[2] || v->ne[2] <= 0 || q->ne[2] % v->ne[2]) return -1;
    if (k->ne[3] <= 0 || q->ne[3] % k->ne[3] || v->ne[3] <= 0 || q->ne[3] % v->ne[3]) return -1;
    if (mask && (mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1])) return -1;
    if (k->nb[0] != ORACLE_Q8_0_BLOCK_BYTES || v->nb[0] != ORACLE_Q8_0_BLOCK_BYTES) return -1;
    return 0;
}

int oracle_flash_attn_ext_q8_0(const oracle_view * q, const oracle_view * k, const oracle_view * v,
                               const oracle_view * mask, float scale, float * dst,
                               int q_variant, int dot_variant, int n_threads) {
    if (fa_check(q, k, v, mask)) return -1;
    const int64_t nr = q->ne[1] * q->ne[2] * q->ne[3];
    if (n_threads < 1) n_threads = 1;
    if (n_threads > nr) n_threads = (int) (nr > 0 ? nr : 1);
    fa_job * jobs = (fa_job *) calloc((size_t) n_threads, sizeof(fa_job));
    pthread_t * th = (pthread_t *) calloc((size_t) n_threads, sizeof(pthread_t));
    const int64_t per = (nr + n_threads - 1) / n_threads;
    for (int t = 0; t < n_threads; t++) {
        jobs[t] = (fa_job) { q, k, v, mask, scale, dst, q_variant, dot_variant,
                             t * per, (t + 1) * per < nr ? (t + 1) * per : nr };
        if (jobs[t].r0 > jobs[t].r1) jobs[t].r0 = jobs[t].r1;
    }
    for (int t = 1; t < n_threads; t++) pthread_create(&th[t], NULL, fa_rows, &jobs[t]);
    fa_rows(&jobs[0]);
    for (int t = 1; t < n_threads; t++) pthread_join(th[t], NULL);
    free(jobs); free(th);
    return 0;
}

int oracle_attn_f64(const oracle_view * q, const oracle_view * k, const oracle_view * v,
                    const oracle_view * mask, double scale, double * dst, int quantize_q) {
    if (fa_check(q, k, v, mask)) return -1;
    const int64_t DK = q->ne[0], DV = v->ne[0];
    const int64_t neq1 = q->ne[1], neq2 = q->ne[2], neq3 = q->ne[3];
    const int64_t nek1 = k->ne[1];
    const int64_t rk2 = neq2 / k->ne[2], rk3 = neq3 / k->ne[3];
    const int64_t rv2 = neq2 / v->ne[2], rv3 = neq3 / v->ne[3];
    float * qrow = (float *) malloc(sizeof(float) * (size_t) DK);
    q8_block * Q_q = (q8_block *) malloc(sizeof(q8_block) * (size_t) (DK / ORACLE_QK8_0));
    float * kd = (float *) malloc(sizeof(float) * (size_t) DK);
    float * vd = (float *) malloc(sizeof(float) * (size_t) DV);
    double * s = (double *) malloc(sizeof(double) * (size_t) (nek1 > 0 ? nek1 : 1));
    double * acc = (double *) malloc(sizeof(double) * (size_t) DV);
    for (int64_t iq3 = 0; iq3 < neq3; iq3++)
    for (int64_t iq2 = 0; iq2 < neq2; iq2++)
    for (int64_t iq1 = 0; iq1 < neq1; iq1++) {
        const char * pq = (const char *) q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3];
        for (int64_t d = 0; d < DK; d++) qrow[d] = *(const float *) (pq + d * q->nb[0]);
        if (quantize_q) {
            oracle_quantize_row_q8_0(qrow, Q_q, DK, quantize_q == 2 ? ORACLE_Q8_X86 : ORACLE_Q8_REF);
            oracle_dequantize_row_q8_0(Q_q, qrow, DK);
        }
        const uint16_t * mp = mask ? (const uint16_t *) ((const char *) mask->data + iq1 * mask->nb[1]
                                      + (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3])
                                   : NULL;
        double mx = -INFINITY;
        for (int64_t ic = 0; ic < nek1; ic++) {
            const double mv = mp ? (double) oracle_fp16_to_fp32(mp[ic]) : 0.0;
            if (mv == -INFINITY) { s[ic] = -INFINITY; continue; }
            const char * kp = (const char *) k->data + ic * k->nb[1] + (iq2 / rk2) * k->nb[2] + (iq3 / rk3) * k->nb[3];
            oracle_dequantize_row_q8_0(kp, kd, DK);
            double dot = 0.0;
            for (int64_t d = 0; d < DK; d++) dot += (double) qrow[d] * (double) kd[d];
            s[ic] = dot * scale + mv;
            if (s[ic] > mx) mx = s[ic];
        }
        for (int64_t d = 0; d < DV; d++) acc[d] = 0.0;
        double l = 0.0;
        if (mx != -INFINITY) {
            for (int64_t ic = 0; ic < nek1; ic++) {
                if (s[ic] == -INFINITY) continue;
                const double p = exp(s[ic] - mx);
                l += p;
                const char * vp = (const char *) v->data + ic * v->nb[1] + (iq2 / rv2) * v->nb[2] + (iq3 / rv3) * v->nb[3];
                oracle_dequantize_row_q8_0(vp, vd, DV);
                for (int64_t d = 0; d < DV; d++) acc[d] += p * (double) vd[d];
            }
        }
        double * out = dst + (size_t) (iq3 * neq2 * neq1 + iq2 + iq1 * neq2) * (size_t) DV;
        for (int64_t d = 0; d < DV; d++) out[d] = l > 0.0 ? acc[d] / l : 0.0;
    }
    free(qrow); free(Q_q); free(kd); free(vd); free(s); free(acc);
    return 0;
}

/* ------------------------------------------------------ QSA index producer */

/* ggml_rms_norm (then the caller's ggml_mul by the weight): the squares summed
 * in double, the mean rounded to float, scale = 1 / sqrtf(mean + eps).
 * Used at qwfn_graph.cpp:124-126 (rms), :443 (attn_k_norm), :295 (pooled keys). */
void oracle_rms_norm_f32(const float * x, float * y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double) (x[i] * x[i]);
    const float mean = (float) (sum / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * scale;
}

/* ggml_rope_multi, neox pairs (k, k + n_dims/2), GGML_ROPE_TYPE_IMROPE sections
 * interleaved t, h, w over the pairs (qwfn_graph.cpp:128-131, :297-299,
 * :911-913); the angle is pos * theta_scale^k as a running float product,
 * theta_scale = powf(freq_base, -2 / n_dims), cos / sin of the float angle. */
void oracle_rope_multi_f32(const float * x, float * y, int64_t ne0, int n_dims, const int32_t pos[4],
                           const int sections[4], int imrope, float freq_base) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    const int sect_dims = sections[0] + sections[1] + sections[2] + sections[3];
    const int sec_w = sections[0] + sections[1];
    float th[4] = {(float) pos[0], (float) pos[1], (float) pos[2], (float) pos[3]};
    for (int64_t i = n_dims; i < ne0; i++) y[i] = x[i];
    for (int k = 0; k < n_dims / 2; k++) {
        const int sector = k % sect_dims;
        int s;
        if (imrope) {
            if (sector % 3 == 1 && sector < 3 * sections[1]) s = 1;
            else if (sector % 3 == 2 && sector < 3 * sections[2]) s = 2;
            else if (sector % 3 == 0 && sector < 3 * sections[0]) s = 0;
            else s = 3;
        } else {
            s = sector < sections[0] ? 0 : sector < sec_w ? 1 : sector < sec_w + sections[2] ? 2 : 3;
        }
        const float theta = th[s];
        const float c = cosf(theta), sn = sinf(theta);
        const float x0 = x[k], x1 = x[k + n_dims / 2];
        y[k] = x0 * c - x1 * sn;
        y[k + n_dims / 2] = x0 * sn + x1 * c;
        for (int j = 0; j < 4; j++) th[j] *= theta_scale;
    }
}

int oracle_set_rows_f16(uint16_t * dst, int64_t dst_rows, int64_t ne0, const float * src, const int32_t * idx,
                        int64_t n) {
    for (int64_t i = 0; i < n; i++)
        if (idx[i] < 0 || idx[i] >= dst_rows) return -1;
    for (int64_t i = 0; i < n; i++)
        for (int64_t j = 0; j < ne0; j++) dst[(size_t) idx[i] * ne0 + j] = oracle_fp32_to_fp16(src[(size_t) i * ne0 + j]);
    return 0;
}

void oracle_qsa_pool_blocks(const uint16_t * ic, int64_t idx_dim, const int32_t * members, int64_t r, int64_t n_blk,
                            const float * k_norm_w, const int32_t * pos4, const int sections[4], float eps,
                            float freq_base, int n_dims, uint16_t * out) {
    float * acc = malloc(sizeof(float) * (size_t) idx_dim * 3);
    float * nrm = acc + idx_dim;
    float * rot = nrm + idx_dim;
    const float inv_r = 1.0f / (float) r;
    for (int64_t b = 0; b < n_blk; b++) {
        for (int64_t d = 0; d < idx_dim; d++) acc[d] = oracle_fp16_to_fp32(ic[(size_t) members[b * r] * idx_dim + d]);
        for (int64_t m = 1; m < r; m++)
            for (int64_t d = 0; d < idx_dim; d++)
                acc[d] = acc[d] + oracle_fp16_to_fp32(ic[(size_t) members[b * r + m] * idx_dim + d]);
        for (int64_t d = 0; d < idx_dim; d++) acc[d] = acc[d] * inv_r;
        oracle_rms_norm_f32(acc, nrm, idx_dim, eps);
        for (int64_t d = 0; d < idx_dim; d++) nrm[d] = nrm[d] * k_norm_w[d];
        oracle_rope_multi_f32(nrm, rot, idx_dim, n_dims, pos4 + 4 * b, sections, 1, freq_base);
        for (int64_t d = 0; d < idx_dim; d++) out[(size_t) b * idx_dim + d] = oracle_fp32_to_fp16(rot[d]);
    }
    free(acc);
}

/* ----------------------------------------------------- K/V producer */

/* The attention layer's K/V producer for T tokens (qwfn_graph.cpp:441-451 for
 * the projections, attn_k_norm and rope; :370-384 / :623-624 for the q8_0
 * append): ggml_mul_mat with F16 weights (the F32 rows converted to F16, the
 * F16 products summed) or BF16 weights (w_bf16: the rows converted to BF16;
 * the products summed; summed in double here, which ggml's F32 accumulation
 * order matches to within a float rounding: parity of the projection is to a
 * tolerance, of everything after it bit for bit), K rms-normed times the
 * weight and roped, then both quantised with quantize_row_q8_0 (variant). */

/* F32 -> BF16: the upper 16 bits after rounding to nearest, ties to even; a
 * NaN keeps its sign and top payload bits and is made quiet. BF16 -> F32 is
 * the exact inverse placement of the 16 bits. */
uint16_t oracle_fp32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 0x40u);
    return (uint16_t) ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float oracle_bf16_to_fp32(uint16_t h) {
    const uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void oracle_kv_produce_q8_0(const float * cur, int64_t E, int64_t T, const uint16_t * wk, const uint16_t * wv,
                            int64_t kv_dim, const float * k_norm_w, const int32_t * pos, const int sections[4],
                            int n_dims, float freq_base, float eps, void * k_rows, void * v_rows, float * k_f32,
                            float * v_f32, int variant, int w_bf16) {
    const int64_t hd = 256;
    const size_t row_bytes = (size_t) (kv_dim / ORACLE_QK8_0) * 34;
    float * c16 = malloc(sizeof(float) * (size_t) E);
    float * k = malloc(sizeof(float) * (size_t) kv_dim * 2);
    float * v = k + kv_dim;
    float * tmp = malloc(sizeof(float) * (size_t) hd * 2);
    for (int64_t t = 0; t < T; t++) {
        /* ggml_mul_mat converts src1 to the weights' vec_dot type: F16 or BF16 */
        for (int64_t e = 0; e < E; e++)
            c16[e] = w_bf16 ? oracle_bf16_to_fp32(oracle_fp32_to_bf16(cur[t * E + e]))
                            : oracle_fp16_to_fp32(oracle_fp32_to_fp16(cur[t * E + e]));
        for (int64_t o = 0; o < kv_dim; o++) {
            double sk = 0.0, sv = 0.0;
            for (int64_t e = 0; e < E; e++) {
                const float a = w_bf16 ? oracle_bf16_to_fp32(wk[o * E + e]) : oracle_fp16_to_fp32(wk[o * E + e]);
                const float b = w_bf16 ? oracle_bf16_to_fp32(wv[o * E + e]) : oracle_fp16_to_fp32(wv[o * E + e]);
                sk += (double) a * (double) c16[e];
                sv += (double) b * (double) c16[e];
            }
            k[o] = (float) sk;
            v[o] = (float) sv;
        }
        const int32_t p4[4] = {pos[t], pos[T + t], pos[2 * T + t], pos[3 * T + t]};
        for (int64_t h = 0; h < kv_dim / hd; h++) {
            float * kh = k + h * hd;
            oracle_rms_norm_f32(kh, tmp, hd, eps);
            for (int64_t d = 0; d < hd; d++) tmp[d] = tmp[d] * k_norm_w[d];
            oracle_rope_multi_f32(tmp, kh, hd, n_dims, p4, sections, 1, freq_base);
        }
        if (k_f32) memcpy(k_f32 + t * kv_dim, k, sizeof(float) * (size_t) kv_dim);
        if (v_f32) memcpy(v_f32 + t * kv_dim, v, sizeof(float) * (size_t) kv_dim);
        oracle_quantize_row_q8_0(k, (char *) k_rows + (size_t) t * row_bytes, kv_dim, variant);
        oracle_quantize_row_q8_0(v, (char *) v_rows + (size_t) t * row_bytes, kv_dim, variant);
    }
    free(c16);
    free(k);
    free(tmp);
}

/* ----------------------------------------------------- gated delta rule */

/* The recurrence of ggml_gated_delta_net as the reference calls it
 * (qwfn_graph.cpp:240-278; snapshots for rollback :210-238): per value head h
 * (key head h / (n_v / n_k)), per token, S *= exp(g); m = S^T k;
 * S += k (v - m)^T beta; out = S^T q * scale; snapshot s = the state after
 * token T - 1 - s. The op belongs to the reference's ggml fork, which is not in
 * the reference tree or this image: the head broadcast rule and the float
 * order are restated from its call site and the gated delta rule's published
 * definition (parity unpinned beyond the fp64 brute force and closed forms of
 * tests/test_oracle_deltanet.py). */

void oracle_gated_delta_net(const float * q, int64_t q_ts, const float * k, int64_t k_ts, const float * v, int64_t v_ts,
                            const float * g, const float * beta, float * state, float * out, float * snap,
                            int64_t n_snap, int64_t T, int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, float scale) {
    const int64_t rep = n_v / n_k;
    float * m = malloc(sizeof(float) * (size_t) dv);
    for (int64_t h = 0; h < n_v; h++) {
        float * S = state + (size_t) h * dk * dv;
        const int64_t hk = h / rep;
        for (int64_t t = 0; t < T; t++) {
            const float * qt = q + t * q_ts + hk * dk;
            const float * kt = k + t * k_ts + hk * dk;
            const float * vt = v + t * v_ts + h * dv;
            const float a = expf(g[t * n_v + h]);
            const float b = beta[t * n_v + h];
            for (int64_t i = 0; i < dk * dv; i++) S[i] = S[i] * a;
            for (int64_t c = 0; c < dv; c++) {
                float acc = 0.0f;
                for (int64_t r = 0; r < dk; r++) acc = acc + S[r * dv + c] * kt[r];
                m[c] = acc;
            }
            for (int64_t c = 0; c < dv; c++) {
                const float d = (vt[c] - m[c]) * b;
                for (int64_t r = 0; r < dk; r++) S[r * dv + c] = S[r * dv + c] + kt[r] * d;
            }
            for (int64_t c = 0; c < dv; c++) {
                float acc = 0.0f;
                for (int64_t r = 0; r < dk; r++) acc = acc + S[r * dv + c] * (qt[r] * scale);
                out[(t * n_v + h) * dv + c] = acc;
            }
            const int64_t sb = T - 1 - t;
            if (snap && sb >= 1 && sb <= n_snap)
                memcpy(snap + ((size_t) (sb - 1) * n_v + h) * dk * dv, S, sizeof(float) * (size_t) dk * dv);
        }
    }
    free(m);
}
