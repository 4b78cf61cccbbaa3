// The attention layer's K/V producer for a decode or verify step, two launches:
// the K and V projections of the step's hidden rows, RMS norm of each K head
// times attn_k_norm, IMROPE at the tokens' positions, and the q8_0 append of
// both into the caches -- the ops qwfn_graph.cpp:441-451 (attn_k / attn_v
// mul_mat, rms), :129-132 / :446-451 (rope) and :370-384 (kv_append: cpy
// F32 -> q8_0) emit one by one.
//
// Projection: ggml_mul_mat with F16 weights converts the F32 hidden rows to
// F16 and sums the F16 products in F32; with BF16 weights it converts them to
// BF16 (round to nearest even) and sums the BF16 products in F32 (both kinds
// of products are exact in F32). Each wave computes one output row for
// all T tokens: the row's 16-byte weight loads are issued before the block
// stages the hidden rows (F16) in LDS, then per-lane F32 partial sums and a
// wave reduction. The rows land in a device-resident staging buffer. The
// second launch takes one (token, head) per wave: K heads are normed, weighted
// and roped (rope_device.h, ggml-cpu's float order; one lane per rope pair
// computes its cos / sin), then quantised with the cache quantiser
// (q8_device.h) into row first_row + t; V heads are quantised as they are. (A single launch whose
// last workgroup runs the epilogue needs a device-scope release per
// workgroup, an L2 write-back each: measured 13 us more than the second
// launch.)
#include "q8_device.h"
#include "qwfn_common.h"
#include "qwfn_state.h"
#include "rope_device.h"
#include "wave_ops.h"

#include <cmath>
#include <mutex>

namespace qwfn {
namespace {

using wave::wave_sum;
using wave::wave_sum_d;

constexpr int KVP_MAX_T = 16;            // tokens per call
constexpr int KVP_MAX_HKV = 8;           // KV heads
constexpr int KVP_HD = 256;              // head size
constexpr int KVP_WAVES = 4;
constexpr int KVP_MAX_EMBD = 8192;       // hidden size, at most (the F16 rows of all tokens fit LDS)
constexpr int KVP_MAX_PAIRS = 128;       // rope pairs per head, at most
constexpr int KVP_STAGE = KVP_MAX_T * 2 * KVP_MAX_HKV * KVP_HD;   // F32 projected rows

// projected rows of the current call ([t][K rows | V rows]), one buffer per
// device: calls that overlap on one device race
__device__ float g_kvp_rows[KVP_STAGE];

struct kvp_args {
    const float *    cur;         // F32 [n_embd] per token, token stride cur_nb1 bytes
    size_t           cur_nb1;
    int32_t          n_embd;
    int32_t          T;
    const uint16_t * wk;          // F16 or BF16 [n_embd] per output row (kv_dim rows), row stride w_nb1 bytes
    const uint16_t * wv;
    size_t           wk_nb1, wv_nb1;
    int32_t          nh_kv;
    int32_t          kv_dim;      // nh_kv * 256
    const float *    k_norm_w;    // F32 [256]
    float            eps;
    rope_params      rp;
    const int32_t *  pos;         // I32 [4 * T]: t positions, then h, w, e (ggml_rope_multi's layout)
    char *           kc;          // q8_0 caches, row stride k_nb1 / v_nb1 bytes
    char *           vc;
    size_t           k_nb1, v_nb1;
    int64_t          first_row;
    int32_t          x86;
    float *          rows;        // g_kvp_rows
};

__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }

// c + a * b for the low (or high) f16 halves of a and b, in f32 with one
// rounding: f16 values are exact in f32, so this is fmaf(float(a), float(b), c)
__device__ __forceinline__ float fma_mix_lo(uint32_t a, uint32_t b, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t a, uint32_t b, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// F32 -> BF16, round to nearest even (a NaN stays a quiet NaN)
__device__ __forceinline__ uint32_t f32_to_bf16(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// c + a * b for the low (or high) BF16 halves of a and b: a BF16 value is the
// upper half of an F32, and the product of two is exact in F32
__device__ __forceinline__ float fma_bf16_lo(uint32_t a, uint32_t b, float c) {
    return __builtin_fmaf(__builtin_bit_cast(float, a << 16), __builtin_bit_cast(float, b << 16), c);
}
__device__ __forceinline__ float fma_bf16_hi(uint32_t a, uint32_t b, float c) {
    return __builtin_fmaf(__builtin_bit_cast(float, a & 0xffff0000u), __builtin_bit_cast(float, b & 0xffff0000u), c);
}

// the hidden values 4 i .. 4 i + 3 of the call's rows, F32 -> F16 (or BF16),
// into LDS
template <bool BF16>
__device__ __forceinline__ void stage_hidden4(uint16_t * cur16, int idx, const float4 & x) {
    uint32_t lo, hi;
    if constexpr (BF16) {
        lo = f32_to_bf16(x.x) | (f32_to_bf16(x.y) << 16);
        hi = f32_to_bf16(x.z) | (f32_to_bf16(x.w) << 16);
    } else {
        lo = __builtin_bit_cast(uint16_t, (_Float16) x.x) | ((uint32_t) __builtin_bit_cast(uint16_t, (_Float16) x.y) << 16);
        hi = __builtin_bit_cast(uint16_t, (_Float16) x.z) | ((uint32_t) __builtin_bit_cast(uint16_t, (_Float16) x.w) << 16);
    }
    *(uint2 *) &cur16[idx] = make_uint2(lo, hi);
}

template <bool BF16, int NJ>      // NJ = ceil(n_embd / 512) weight loads a lane
__global__ __launch_bounds__(KVP_WAVES * 64) void k_kv_project(kvp_args a) {
    extern __shared__ uint16_t cur16[];          // [T][n_embd] F16 (or BF16) hidden rows
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int T = a.T, E = a.n_embd;
    const int n_out = 2 * a.kv_dim;
    constexpr int NT = KVP_WAVES * 64;
    const int n4 = T * E / 4;
    const uint32_t e4_mul = (uint32_t) (((uint64_t(1) << 32) + (uint64_t) (E / 4) - 1) / (uint64_t) (E / 4));
    auto hidden4 = [&](int i) -> float4 {          // values 4 i .. 4 i + 3 (i < n4)
        const int t = E / 4 == 1 ? i : (int) __umulhi((uint32_t) i, e4_mul);
        const int e = 4 * (i - t * (E / 4));
        return *(const float4 *) ((const char *) a.cur + (size_t) t * a.cur_nb1 + (size_t) e * 4);
    };

    // ---- the first 8 hidden loads a thread go out first (one round for up
    //      to 8192 values), then the weights: wave w of block b takes output
    //      row 4b + w of [K rows | V rows], lane l the 8 hidden values
    //      8 l + 512 j. Loads return in order, so the conversion below waits
    //      only for the hidden rows (mostly L2 hits) while the weights stream ----
    float4 x[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int i = threadIdx.x + NT * u;
        x[u] = hidden4(i < n4 ? i : n4 - 1);
    }
    const int o = blockIdx.x * KVP_WAVES + wv;
    const int oc = o < n_out ? o : n_out - 1;
    const uint16_t * wrow = oc < a.kv_dim ? (const uint16_t *) ((const char *) a.wk + (size_t) oc * a.wk_nb1)
                                          : (const uint16_t *) ((const char *) a.wv + (size_t) (oc - a.kv_dim) * a.wv_nb1);
    uint4 wq[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) wq[j] = *(const uint4 *) (wrow + (512 * j + 8 * lane < E ? 512 * j + 8 * lane : 0));
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int i = threadIdx.x + NT * u;
        if (i < n4) stage_hidden4<BF16>(cur16, 4 * i, x[u]);
    }
    // more than 8192 values: the rest, 8 loads in flight at a time
    for (int i0 = threadIdx.x + NT * 8; i0 < n4; i0 += NT * 8) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + NT * u;
            x[u] = hidden4(i < n4 ? i : n4 - 1);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + NT * u;
            if (i < n4) stage_hidden4<BF16>(cur16, 4 * i, x[u]);
        }
    }
    __syncthreads();

    // ---- projection ----
    float acc[KVP_MAX_T];
#pragma unroll
    for (int t = 0; t < KVP_MAX_T; t++) acc[t] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e0 = 512 * j + 8 * lane;
        if (e0 >= E) continue;
        const uint32_t ww[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
#pragma unroll
        for (int t = 0; t < KVP_MAX_T; t++) {
            if (t >= T) continue;
            const uint4 cq = *(const uint4 *) &cur16[t * E + e0];
            const uint32_t cw[4] = {cq.x, cq.y, cq.z, cq.w};
            float s = acc[t];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if constexpr (BF16) {
                    s = fma_bf16_lo(ww[q], cw[q], s);
                    s = fma_bf16_hi(ww[q], cw[q], s);
                } else {
                    s = fma_mix_lo(ww[q], cw[q], s);
                    s = fma_mix_hi(ww[q], cw[q], s);
                }
            }
            acc[t] = s;
        }
    }
#pragma unroll
    for (int t = 0; t < KVP_MAX_T; t++) {
        if (t >= T) continue;
        const float v = wave_sum(acc[t]);
        if (lane == 0 && o < n_out) a.rows[t * n_out + o] = v;
    }
}

// The epilogue: wave w of block b takes (token, head) task 4b + w (K heads,
// then V heads, of each token).
__global__ __launch_bounds__(KVP_WAVES * 64) void k_kv_epilogue(kvp_args a) {
    __shared__ float head[KVP_WAVES][KVP_HD];
    __shared__ float csw[KVP_WAVES][2][KVP_MAX_PAIRS];
    // wv through readfirstlane: the task, and so the position loads, are
    // scalar, and the cos / sin need not wait for the vector loads
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int T = a.T;
    const int n_out = 2 * a.kv_dim;
    const int half = a.rp.n_dims / 2;
    const int n_tasks = T * 2 * a.nh_kv;                 // (token, K heads then V heads)
    float * hx = head[wv];
    const int task = blockIdx.x * KVP_WAVES + wv;
    if (task < n_tasks) {
        const int t = task / (2 * a.nh_kv), hh = task - t * 2 * a.nh_kv;
        const bool is_k = hh < a.nh_kv;
        const int h = is_k ? hh : hh - a.nh_kv;
        const float * src = a.rows + t * n_out + (is_k ? 0 : a.kv_dim) + h * KVP_HD;
        // every load first (the row, the norm weight, the positions), then the
        // rope's cos / sin while they are in flight: one round trip, not three
        float x[4], nw[4];
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = src[4 * lane + i];
#pragma unroll
        for (int i = 0; i < 4; i++) nw[i] = a.k_norm_w[4 * lane + i];
        int32_t pos[4];
#pragma unroll
        for (int s = 0; s < 4; s++) pos[s] = a.pos[s * T + t];
        if (is_k) {
            // lane k computes pair k's cos / sin
            for (int k = lane; k < half; k += 64) rope_cos_sin(a.rp, pos, k, &csw[wv][0][k], &csw[wv][1][k]);
            // RMS norm (squares summed in double), times the weight
            double sq = 0.0;
#pragma unroll
            for (int i = 0; i < 4; i++) sq += (double) __fmul_rn(x[i], x[i]);
            sq = wave_sum_d(sq);
            const float mean = (float) (sq / (double) KVP_HD);
            const float scale = 1.0f / sqrtf(__fadd_rn(mean, a.eps));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[i] = __fmul_rn(__fmul_rn(x[i], scale), nw[i]);
                hx[4 * lane + i] = x[i];
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            // each lane rotates its values 4 lane + i that lie in the first n_dims
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d = 4 * lane + i;
                if (d < a.rp.n_dims) {
                    const int k = d < half ? d : d - half;
                    float y0, y1;
                    rope_rotate(hx[k], hx[k + half], csw[wv][0][k], csw[wv][1][k], &y0, &y1);
                    x[i] = d < half ? y0 : y1;
                }
            }
        }
        // q8_0 of the head row: 8 lanes per block
        uint16_t d16;
        float dqa;
        const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dqa);
        char * row = (is_k ? a.kc + (size_t) (a.first_row + t) * a.k_nb1 : a.vc + (size_t) (a.first_row + t) * a.v_nb1) +
                     (size_t) h * (KVP_HD / QK) * QBLOCK;
        char * bp = row + (lane >> 3) * QBLOCK;
        uint16_t * qp = (uint16_t *) (bp + 2 + (lane & 7) * 4);
        qp[0] = (uint16_t) (q4 & 0xffffu);
        qp[1] = (uint16_t) (q4 >> 16);
        if ((lane & 7) == 0) *(uint16_t *) bp = d16;
    }
}

constexpr int KVP_MAX_NJ = KVP_MAX_EMBD / 512;

// k_kv_project<BF16, nj> for nj = NJ .. KVP_MAX_NJ
template <bool BF16, int NJ = 1>
void launch_project(int nj, dim3 grid, size_t lds, hipStream_t stream, const kvp_args & a) {
    if constexpr (NJ <= KVP_MAX_NJ) {
        if (nj == NJ) hipLaunchKernelGGL((k_kv_project<BF16, NJ>), grid, dim3(KVP_WAVES * 64), lds, stream, a);
        else          launch_project<BF16, NJ + 1>(nj, grid, lds, stream, a);
    }
}

// the hidden rows of up to 16 tokens take more than 64 KB of LDS
template <bool BF16, int NJ = 1>
int allow_project_lds() {
    if constexpr (NJ <= KVP_MAX_NJ) {
        if (int rc = hip_check(hipFuncSetAttribute((const void *) k_kv_project<BF16, NJ>,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024),
                               "hipFuncSetAttribute"))
            return rc;
        return allow_project_lds<BF16, NJ + 1>();
    }
    return 0;
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" int qwfn_kv_produce_q8_0(const qwfn_tensor * cur, const qwfn_tensor * wk, const qwfn_tensor * wv,
                                    const float * k_norm_w, const int32_t * pos, const qwfn_rope_cfg * rope,
                                    const qwfn_tensor * k_cache, const qwfn_tensor * v_cache, int64_t first_row,
                                    int variant, void * stream) {
    return ::qwfn::abi_call("kv_produce_q8_0", [&]() -> int {
        if (!cur || !wk || !wv || !k_norm_w || !pos || !rope || !k_cache || !v_cache || !cur->data || !wk->data ||
            !wv->data || !k_cache->data || !v_cache->data)
            return set_error(QWFN_EINVAL, "kv_produce: NULL argument");
        const bool bf16 = wk->type == QWFN_TYPE_BF16;
        if (cur->type != QWFN_TYPE_F32 || (wk->type != QWFN_TYPE_F16 && wk->type != QWFN_TYPE_BF16) ||
            wv->type != wk->type || k_cache->type != QWFN_TYPE_Q8_0 || v_cache->type != QWFN_TYPE_Q8_0)
            return set_error(QWFN_EINVAL, "kv_produce: cur f32, weights both f16 or both bf16, caches q8_0");
        if (variant != QWFN_Q8_REF && variant != QWFN_Q8_X86) return set_error(QWFN_EINVAL, "kv_produce: unknown variant");
        const int64_t E = cur->ne[0], T = cur->ne[1];
        if (cur->nb[0] != 4 || wk->nb[0] != 2 || wv->nb[0] != 2) return set_error(QWFN_EINVAL, "kv_produce: rows must be contiguous");
        if (E < 8 || E % 8 || E > KVP_MAX_EMBD) return set_error(QWFN_ENOTSUP, "kv_produce: n_embd must be a multiple of 8, at most 8192");
        if (T < 1 || T > KVP_MAX_T) return set_error(QWFN_ENOTSUP, "kv_produce: 1 to 16 tokens per call");
        if (T * E * 2 > 128 * 1024) return set_error(QWFN_ENOTSUP, "kv_produce: T * n_embd must be at most 65536");
        if (wk->ne[0] != E || wv->ne[0] != E || wk->ne[1] != wv->ne[1])
            return set_error(QWFN_EINVAL, "kv_produce: weights must be [n_embd, kv_dim] for K and V alike");
        const int64_t kv_dim = wk->ne[1];
        if (kv_dim % KVP_HD || kv_dim / KVP_HD < 1 || kv_dim / KVP_HD > KVP_MAX_HKV)
            return set_error(QWFN_ENOTSUP, "kv_produce: kv_dim must be 256 * n_head_kv, 1 to 8 heads");
        if (k_cache->ne[0] != kv_dim || v_cache->ne[0] != kv_dim || k_cache->nb[0] != QBLOCK || v_cache->nb[0] != QBLOCK)
            return set_error(QWFN_EINVAL, "kv_produce: caches must be q8_0 rows of kv_dim values");
        if (k_cache->nb[1] < (size_t) kv_dim / QK * QBLOCK || v_cache->nb[1] < (size_t) kv_dim / QK * QBLOCK)
            return set_error(QWFN_EINVAL, "kv_produce: cache rows overlap");
        if (first_row < 0 || first_row + T > k_cache->ne[1] || first_row + T > v_cache->ne[1])
            return set_error(QWFN_ERANGE, "kv_produce: rows first_row .. first_row + T - 1 must lie in the caches");
        if (rope->n_dims < 2 || rope->n_dims % 2 || rope->n_dims > 2 * KVP_MAX_PAIRS || !(rope->freq_base > 0.f) ||
            !(rope->rms_eps >= 0.f))
            return set_error(QWFN_EINVAL, "kv_produce: rope n_dims must be even and at most 256, freq_base positive");
        int sect = 0;
        for (int s = 0; s < 4; s++) {
            if (rope->sections[s] < 0) return set_error(QWFN_EINVAL, "kv_produce: negative rope section");
            sect += rope->sections[s];
        }
        if (sect <= 0) return set_error(QWFN_EINVAL, "kv_produce: rope sections must not all be zero");
        if (!is_aligned(cur->data, 16) || cur->nb[1] % 16 || !is_aligned(wk->data, 16) || !is_aligned(wv->data, 16) ||
            wk->nb[1] % 16 || wv->nb[1] % 16 || !is_aligned(k_norm_w, 4) || !is_aligned(pos, 4) ||
            !is_aligned(k_cache->data, 2) || !is_aligned(v_cache->data, 2) || k_cache->nb[1] % 2 || v_cache->nb[1] % 2)
            return set_error(QWFN_EALIGN, "kv_produce: cur and weights 16-byte aligned rows, 4-byte i32 / weight, 2-byte cache rows");
        kvp_args a{};
        a.cur = (const float *) cur->data; a.cur_nb1 = cur->nb[1]; a.n_embd = (int32_t) E; a.T = (int32_t) T;
        a.wk = (const uint16_t *) wk->data; a.wv = (const uint16_t *) wv->data; a.wk_nb1 = wk->nb[1]; a.wv_nb1 = wv->nb[1];
        a.nh_kv = (int32_t) (kv_dim / KVP_HD); a.kv_dim = (int32_t) kv_dim;
        a.k_norm_w = k_norm_w; a.eps = rope->rms_eps;
        a.rp.n_dims = rope->n_dims;
        for (int s = 0; s < 4; s++) a.rp.sections[s] = rope->sections[s];
        a.rp.imrope = 1;
        a.rp.theta_scale = powf(rope->freq_base, -2.0f / (float) rope->n_dims);
        a.pos = pos;
        a.kc = (char *) k_cache->data; a.vc = (char *) v_cache->data; a.k_nb1 = k_cache->nb[1]; a.v_nb1 = v_cache->nb[1];
        a.first_row = first_row; a.x86 = variant == QWFN_Q8_X86;
        // the staging buffer, per device (its address, not the symbol)
        int dev = 0;
        if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
        static float * rows_ptr[64];
        static std::mutex mu;
        if (dev < 0 || dev >= 64) return set_error(QWFN_ENOTSUP, "kv_produce: device index beyond 63");
        std::lock_guard<std::mutex> lock(mu);
        if (!rows_ptr[dev]) {
            void * p = nullptr;
            if (int rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(g_kvp_rows)), "hipGetSymbolAddress")) return rc;
            if (int rc = allow_project_lds<false>()) return rc;
            if (int rc = allow_project_lds<true>()) return rc;
            rows_ptr[dev] = (float *) p;
        }
        a.rows = rows_ptr[dev];
        const int64_t n_out = 2 * kv_dim;
        const int64_t blocks = (n_out + KVP_WAVES - 1) / KVP_WAVES;
        const size_t lds = (size_t) T * E * 2;
        const int nj = (int) ((E + 511) / 512);
        if (bf16) launch_project<true>(nj, dim3((unsigned) blocks), lds, as_stream(stream), a);
        else      launch_project<false>(nj, dim3((unsigned) blocks), lds, as_stream(stream), a);
        if (int rc = hip_check(hipGetLastError(), "kv_produce launch")) return rc;
        const int64_t tasks = T * 2 * (kv_dim / KVP_HD);
        hipLaunchKernelGGL(k_kv_epilogue, dim3((unsigned) ((tasks + KVP_WAVES - 1) / KVP_WAVES)), dim3(KVP_WAVES * 64), 0,
                           as_stream(stream), a);
        return hip_check(hipGetLastError(), "kv_produce epilogue launch");
    });
}
