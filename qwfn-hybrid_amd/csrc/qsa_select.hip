// Decode-time block selection of Qwen Sparse Attention: the scores of the
// pooled block keys against the indexer query, the top k_blocks blocks, and
// their cells (graph_builder::qsa_dec_cells, qwfn_graph.cpp:556-581):
//
//   score[b] = sum over indexer heads h of relu(pool[b] . q16[h]) + bias[b]
//   top      = ggml_top_k(score, k_blocks)   (block indices, best first)
//   cells    = blk_cells[top[j] * ratio + m] for m < ratio
//
// q16 is the query rounded to f16: ggml's mul_mat of an F16 matrix converts
// its F32 operand to F16 before the dot products, which accumulate in f32.
//
// Two kernels. k_qsa_score spreads the pool cache (n_blocks x 128 f16, up to
// 4.7 MB per query) over many workgroups: 16 lanes per block, 16 bytes of the
// key each, 4 heads' partial dots reduced across the 16 lanes with DPP. The
// scores land in a workspace. k_qsa_topk, one workgroup per query, finds the
// k-th largest score by a radix select over order-preserving keys of the
// float bits (histograms in LDS), gathers the blocks above it and as many
// equal to it as needed, lowest block first, sorts those by score, best first
// (ties: lower block first), and writes their cells.
#include "qwfn_common.h"
#include "qwfn_state.h"

#include <algorithm>

namespace qwfn {
namespace {

constexpr int IDX_DIM = 128;             // indexer key length (hparams::idx_key_len)
constexpr int MAX_IDX_HEADS = 8;
constexpr int SCORE_THREADS = 256;        // 16 blocks per workgroup pass
constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_MAX = 1024;            // k_blocks per query, at most
constexpr int RADIX_BITS = 8;

struct score_args {
    const uint16_t * pool;        // F16 [IDX_DIM] per block, block stride pool_nb1 bytes
    size_t           pool_nb1;
    int64_t          n_blocks;
    const float *    q;           // F32 [IDX_DIM][n_heads] per query, query stride q_nb2 bytes
    size_t           q_nb2;
    int32_t          n_heads;
    const float *    bias;        // F32 [n_blocks] per query, query stride bias_nb1 bytes
    size_t           bias_nb1;
    float *          score;       // [T][n_blocks]
};

__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }

// q16: the query rounded to f16 (the conversion of ggml's F16 mul_mat), then
// back to f32 for the products.
__global__ __launch_bounds__(SCORE_THREADS) void k_qsa_score(score_args a) {
    __shared__ float qs[MAX_IDX_HEADS][IDX_DIM];
    const int t = blockIdx.y;
    const float * q = (const float *) ((const char *) a.q + (size_t) t * a.q_nb2);
    for (int i = threadIdx.x; i < a.n_heads * IDX_DIM; i += SCORE_THREADS)
        qs[i / IDX_DIM][i % IDX_DIM] = (float) (_Float16) q[i];   // round to nearest even
    __syncthreads();
    const int sub = threadIdx.x & 15;                  // 8 dims of the key
    const int64_t step = (int64_t) gridDim.x * (SCORE_THREADS / 16);
    for (int64_t b = (int64_t) blockIdx.x * (SCORE_THREADS / 16) + (threadIdx.x >> 4); b < a.n_blocks; b += step) {
        const uint4 raw = *(const uint4 *) ((const char *) a.pool + (size_t) b * a.pool_nb1 + 16 * sub);
        float k[8];
        k[0] = h2f(raw.x & 0xffff); k[1] = h2f(raw.x >> 16); k[2] = h2f(raw.y & 0xffff); k[3] = h2f(raw.y >> 16);
        k[4] = h2f(raw.z & 0xffff); k[5] = h2f(raw.z >> 16); k[6] = h2f(raw.w & 0xffff); k[7] = h2f(raw.w >> 16);
        float s = 0.f;
        for (int h = 0; h < a.n_heads; h++) {
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) d = fmaf(k[i], qs[h][8 * sub + i], d);
            // sum over the 16 lanes of the block: butterflies within 16-lane rows
            d += __shfl_xor(d, 1, 16);
            d += __shfl_xor(d, 2, 16);
            d += __shfl_xor(d, 4, 16);
            d += __shfl_xor(d, 8, 16);
            s += d > 0.f ? d : 0.f;                   // relu, then the sum over heads
        }
        if (sub == 0) {
            const float bb = *(const float *) ((const char *) a.bias + (size_t) t * a.bias_nb1 + (size_t) b * 4);
            a.score[(size_t) t * a.n_blocks + b] = s + bb;
        }
    }
}

struct topk_args {
    const float *   score;        // [T][n_blocks]
    int64_t         n_blocks;
    int32_t         k;            // blocks kept
    const int32_t * blk_cells;    // [n_blocks_max * ratio]
    int32_t         ratio;
    int32_t *       cells;        // [T][k * ratio]
    int32_t *       top;          // [T][k] or null
};

// float -> uint32 whose unsigned order is the float order (NaN never occurs:
// scores are sums of products of finite values plus a finite or -inf bias)
__device__ __forceinline__ uint32_t okey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(TOPK_THREADS) void k_qsa_topk(topk_args a) {
    __shared__ uint32_t hist[1 << RADIX_BITS];
    __shared__ uint32_t sel_key[TOPK_MAX];
    __shared__ int32_t  sel_idx[TOPK_MAX];
    __shared__ uint32_t s_prefix, s_need, n_above, n_equal;
    const int t = blockIdx.x;
    const float * sc = a.score + (size_t) t * a.n_blocks;
    const int64_t n = a.n_blocks;
    const int k = a.k;

    // radix select, most significant digit first: the k-th largest key
    uint32_t prefix = 0, mask = 0, need = (uint32_t) k;
    for (int shift = 32 - RADIX_BITS; shift >= 0; shift -= RADIX_BITS) {
        for (int i = threadIdx.x; i < (1 << RADIX_BITS); i += TOPK_THREADS) hist[i] = 0;
        __syncthreads();
        for (int64_t i = threadIdx.x; i < n; i += TOPK_THREADS) {
            const uint32_t key = okey(sc[i]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & ((1u << RADIX_BITS) - 1)], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t acc = 0;
            int d = (1 << RADIX_BITS) - 1;
            for (; d > 0; d--) {                       // from the largest digit down
                if (acc + hist[d] >= need) break;
                acc += hist[d];
            }
            s_prefix = prefix | ((uint32_t) d << shift);
            s_need = need - acc;
        }
        __syncthreads();
        prefix = s_prefix;
        need = s_need;
        mask |= ((1u << RADIX_BITS) - 1) << shift;
        __syncthreads();
    }
    // prefix is the k-th largest key; `need` of the keys equal to it are kept
    // (the lowest blocks), every key above it is kept
    if (threadIdx.x == 0) { n_above = 0; n_equal = 0; }
    __syncthreads();
    const uint32_t kth = prefix;
    const uint32_t keep_equal = need;
    for (int64_t i0 = 0; i0 < n; i0 += TOPK_THREADS) {
        const int64_t i = i0 + threadIdx.x;
        const uint32_t key = i < n ? okey(sc[i]) : 0u;
        if (i < n && key > kth) {
            const uint32_t slot = atomicAdd(&n_above, 1u);
            sel_key[slot] = key;
            sel_idx[slot] = (int32_t) i;
        }
        // equal keys in block order: a ballot per wave, waves in order
        const bool eq = i < n && key == kth;
        const unsigned long long bal = __ballot(eq);
        __shared__ uint32_t wave_eq[TOPK_THREADS / 64];
        const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
        if (lane == 0) wave_eq[w] = (uint32_t) __popcll(bal);
        __syncthreads();
        uint32_t before = n_equal;
        for (int w2 = 0; w2 < w; w2++) before += wave_eq[w2];
        const uint32_t rank = before + (uint32_t) __popcll(bal & ((1ull << lane) - 1ull));
        if (eq && rank < keep_equal) {
            const uint32_t slot = (uint32_t) k - keep_equal + rank;   // after the keys above
            sel_key[slot] = key;
            sel_idx[slot] = (int32_t) i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t tot = 0;
            for (int w2 = 0; w2 < TOPK_THREADS / 64; w2++) tot += wave_eq[w2];
            n_equal += tot;
        }
        __syncthreads();
    }
    // sort the k kept blocks by key, best first, lower block first on ties
    // (bitonic over the next power of two; padding sorts last)
    int np = 1;
    while (np < k) np <<= 1;
    for (int i = k + threadIdx.x; i < np; i += TOPK_THREADS) { sel_key[i] = 0u; sel_idx[i] = 0x7fffffff; }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np; i += TOPK_THREADS) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const uint32_t ki = sel_key[i], kj = sel_key[j];
                    const int32_t ii = sel_idx[i], ij = sel_idx[j];
                    // "i before j" in the final order: larger key, then lower block
                    const bool i_first = ki > kj || (ki == kj && ii < ij);
                    if (desc ? !i_first : i_first) {
                        sel_key[i] = kj; sel_key[j] = ki;
                        sel_idx[i] = ij; sel_idx[j] = ii;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int j = threadIdx.x; j < k; j += TOPK_THREADS) {
        const int32_t blk = sel_idx[j];
        if (a.top) a.top[(size_t) t * k + j] = blk;
        for (int m = 0; m < a.ratio; m++)
            a.cells[((size_t) t * k + j) * a.ratio + m] = a.blk_cells[(size_t) blk * a.ratio + m];
    }
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" size_t qwfn_qsa_select_workspace_size(int64_t n_blocks, int32_t T) {
    return (size_t) std::max<int64_t>(1, n_blocks) * (size_t) std::max(1, T) * sizeof(float);
}

extern "C" int qwfn_qsa_select_cells(const uint16_t * pool, size_t pool_nb1, int64_t n_blocks, const float * q,
                                     int32_t n_heads, size_t q_nb2, const float * bias, size_t bias_nb1, int32_t T,
                                     int32_t k_blocks, const int32_t * blk_cells, int32_t ratio, int32_t * cells,
                                     int32_t * top, void * ws, size_t ws_bytes, void * stream) {
    if (!pool || !q || !bias || !blk_cells || !cells) return set_error(QWFN_EINVAL, "qsa_select_cells: NULL pointer");
    if (n_blocks < 1 || T < 1 || ratio < 1) return set_error(QWFN_EINVAL, "qsa_select_cells: empty input");
    if (n_heads < 1 || n_heads > MAX_IDX_HEADS) return set_error(QWFN_ENOTSUP, "qsa_select_cells: 1 to 8 indexer heads");
    if (k_blocks < 1 || k_blocks > n_blocks || k_blocks > TOPK_MAX)
        return set_error(QWFN_EINVAL, "qsa_select_cells: need 1 <= k_blocks <= min(n_blocks, 1024)");
    if (pool_nb1 < IDX_DIM * 2 || pool_nb1 % 16 || !is_aligned(pool, 16))
        return set_error(QWFN_EALIGN, "qsa_select_cells: pooled keys must be 128 f16 at a 16-byte aligned stride");
    if (q_nb2 < (size_t) n_heads * IDX_DIM * 4 || !is_aligned(q, 4) || q_nb2 % 4 || bias_nb1 % 4 || !is_aligned(bias, 4))
        return set_error(QWFN_EALIGN, "qsa_select_cells: q [128, n_heads] f32 per query, f32 bias");
    if (!ws || ws_bytes < qwfn_qsa_select_workspace_size(n_blocks, T) || !is_aligned(ws, 4))
        return set_error(QWFN_ENOMEM, "qsa_select_cells: workspace too small");
    if (n_blocks * ratio > INT32_MAX) return set_error(QWFN_ERANGE, "qsa_select_cells: too many cells");
    hipStream_t st = as_stream(stream);
    score_args sa{pool, pool_nb1, n_blocks, q, q_nb2, n_heads, bias, bias_nb1, (float *) ws};
    const int64_t per = SCORE_THREADS / 16;
    const unsigned gx = (unsigned) std::max<int64_t>(1, std::min<int64_t>((n_blocks + per - 1) / per, 1024));
    hipLaunchKernelGGL(k_qsa_score, dim3(gx, (unsigned) T), dim3(SCORE_THREADS), 0, st, sa);
    if (int rc = hip_check(hipGetLastError(), "qsa score launch")) return rc;
    topk_args ta{(const float *) ws, n_blocks, k_blocks, blk_cells, ratio, cells, top};
    hipLaunchKernelGGL(k_qsa_topk, dim3((unsigned) T), dim3(TOPK_THREADS), 0, st, ta);
    return hip_check(hipGetLastError(), "qsa top-k launch");
}
