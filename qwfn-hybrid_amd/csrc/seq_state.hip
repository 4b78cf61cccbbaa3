// Per-sequence state around the q8_0 KV path, and the small per-step inputs
// of the attention layers, built on the device.
//
// State (qwfn::state, qwfn_state.cpp:21-173): per attention layer a K, a V and
// an indexer-key cache (1-D, token-major), per Gated-DeltaNet layer a
// recurrent state [d_state, d_state, dt_rank] and a conv history
// [d_conv-1, conv_dim], plus the PLE conv history. Here every device tensor
// lives in one arena. The caches come first; the recurrent tensors follow as
// one contiguous region, so the reset (qwfn_state.cpp:113-121) is one fill
// kernel. The engine's rollback snapshots (qwfn_engine.cpp:355-371) are kept
// as whole images of that region, slot after slot with the same layout, so a
// rollback (qwfn_engine.cpp:3629-3660) is one contiguous device copy instead
// of one copy per tensor.
//
// Step inputs: the reference fills masks and the decode-time sparse-attention
// inputs on the host and copies them over (qwfn_engine.cpp:1072-1105,
// :1261-1271, :2093-2098, :3415-3440; the cell mask is a chain of ggml ops,
// qwfn_graph.cpp:668-693). Here each is one small kernel whose only inputs are
// kernel arguments, so a decode step sends nothing over the host link.
#include "qwfn_common.h"
#include "qwfn_state.h"
#include "qsa_steps.h"
#include "state_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

namespace qwfn {
namespace {

constexpr size_t ARENA_ALIGN = 256;
constexpr int    FILL_THREADS = 256;
constexpr int    CELL_BATCH = 8;     // cells a thread loads before it sets their bits (one round of loads)
constexpr uint16_t F16_ZERO = 0x0000u;
constexpr uint16_t F16_NINF = 0xFC00u;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------- kernels

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// a 16-byte store that does not keep the line in the caches (the mask is read
// by later launches only; 5.4 -> 4.9 us for a 512 x 16896 mask)
__device__ __forceinline__ void store_nt16(void * p, uint4 v) {
    __builtin_nontemporal_store(v4u{v.x, v.y, v.z, v.w}, (v4u *) p);
}

// p[0 .. n16) = 0, 16 bytes per store
__global__ __launch_bounds__(FILL_THREADS) void k_zero16(uint4 * p, int64_t n16) {
    for (int64_t i = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x; i < n16; i += (int64_t) gridDim.x * FILL_THREADS)
        p[i] = make_uint4(0u, 0u, 0u, 0u);   // (plain stores: non-temporal ones ran 20% slower here)
}

int launch_zero(void * p, size_t bytes, hipStream_t stream) {
    // arena offsets and region sizes are multiples of ARENA_ALIGN
    const int64_t n16 = (int64_t) (bytes / 16);
    if (n16 == 0) return QWFN_OK;
    const int64_t grid = std::min<int64_t>((n16 + FILL_THREADS - 1) / FILL_THREADS, 8192);
    hipLaunchKernelGGL(k_zero16, dim3((unsigned) grid), dim3(FILL_THREADS), 0, stream, (uint4 *) p, n16);
    return hip_check(hipGetLastError(), "state zero launch");
}

// Causal mask: thread = (row, group of 8 keys). A group wholly inside the row
// and 16-byte aligned is one store, otherwise 2-byte stores.
// Row i0 + blockIdx.y (query i), 16-byte groups blockIdx.x * FILL_THREADS + tid
// and on in steps of the grid: a 2-D grid, so no 64-bit division splits a flat
// index.
__global__ __launch_bounds__(FILL_THREADS) void k_causal_mask(char * mask, int64_t n_kv, int64_t n_past, size_t row_stride,
                                                             int64_t groups_per_row, int64_t i0) {
    const int64_t i = i0 + blockIdx.y;
    const int64_t row_elems = (int64_t) (row_stride / 2);
    const int64_t vis = n_past + i;   // last visible key
    uint16_t * row = (uint16_t *) (mask + (size_t) i * row_stride);
    for (int64_t g = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x; g < groups_per_row; g += (int64_t) gridDim.x * FILL_THREADS) {
        const int64_t j0 = g * 8;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int64_t j = j0 + e;
            v[e] = (j <= vis && j < n_kv) ? F16_ZERO : F16_NINF;
        }
        if (j0 + 8 <= row_elems && ((uintptr_t) (row + j0) & 15) == 0) {
            uint4 w;
            w.x = v[0] | ((uint32_t) v[1] << 16);
            w.y = v[2] | ((uint32_t) v[3] << 16);
            w.z = v[4] | ((uint32_t) v[5] << 16);
            w.w = v[6] | ((uint32_t) v[7] << 16);
            store_nt16(row + j0, w);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (j0 + e < row_elems) row[j0 + e] = v[e];
        }
    }
}

// Decode cell mask and padded cell list; j < n_pad <= 2 n_cells (host-checked).
__global__ __launch_bounds__(FILL_THREADS) void k_cell_mask(const int32_t * cells, int64_t n_cells, int64_t n_pad,
                                                           int32_t n_past, uint16_t * mask, int32_t * gcells) {
    for (int64_t j = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x; j < n_pad; j += (int64_t) gridDim.x * FILL_THREADS) {
        const bool real = j < n_cells;
        const int32_t c = cells[real ? j : j - n_cells];
        mask[j] = (real && c <= n_past) ? F16_ZERO : F16_NINF;
        if (gcells) gcells[j] = c;
    }
}

struct qsa_prep_args {
    qwfn_qsa_inputs qd;
    const float *   prev;    // previous position's bias, or null (window in place)
    int32_t         n_past;
};

__global__ __launch_bounds__(FILL_THREADS) void k_qsa_prepare(qsa_prep_args a) {
    const int64_t r = a.qd.ratio;
    const int64_t b_last = a.n_past / r;
    const int64_t n_bid = ((int64_t) a.n_past + 1) / r;
    const int64_t b0 = b_last > 0 ? b_last - 1 : 0;
    const int64_t t0 = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x;
    const int64_t stride = (int64_t) gridDim.x * FILL_THREADS;
    if (a.prev) {
        for (int64_t b = t0; b < a.qd.n_blocks_max; b += stride)
            a.qd.bias[b] = (b >= b0 && b <= b_last + 1) ? bias_of(b, b_last, n_bid) : a.prev[b];
    } else if (t0 < 3) {
        const int64_t b = b0 + t0;
        if (b <= b_last + 1 && b < a.qd.n_blocks_max) a.qd.bias[b] = bias_of(b, b_last, n_bid);
    }
    for (int64_t m = t0; m < r; m += stride) a.qd.member_idx[m] = (int32_t) (b_last * r + m);
    if (t0 < 4) a.qd.blk_pos[t0] = (int32_t) (b_last * r);
    if (t0 == 0) {
        *a.qd.write_idx = a.n_past;
        *a.qd.blk_idx = (int32_t) b_last;
        *a.qd.npast_f = (float) a.n_past;
    }
}

// The inputs of T consecutive positions n_past .. n_past + T - 1 in one
// launch: k_qsa_prepare for position n_past, then for each later position
// from the previous one's bias (prepare_steps_range, qsa_steps.h).
__global__ __launch_bounds__(FILL_THREADS) void k_qsa_prepare_steps(qsa_prep_steps_args a) {
    prepare_steps_range(a, (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x, (int64_t) gridDim.x * FILL_THREADS);
}

__global__ __launch_bounds__(FILL_THREADS) void k_qsa_bias(float * bias, int64_t nb_max, int32_t n_past, int32_t ratio) {
    const int64_t b_last = n_past < 0 ? -1 : n_past / ratio;
    const int64_t n_bid = n_past < 0 ? 0 : ((int64_t) n_past + 1) / ratio;
    for (int64_t b = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x; b < nb_max; b += (int64_t) gridDim.x * FILL_THREADS)
        bias[b] = n_past < 0 ? -INFINITY : bias_of(b, b_last, n_bid);
}

struct qsa_tables_args {
    int32_t * blk_cells;
    int64_t   n_blocks_max;
    int32_t   ratio;
    float *   cell_pos;
    int64_t   n_ctx;
    int32_t * blk_pos_all;
    int64_t   n_whole;
};

__global__ __launch_bounds__(FILL_THREADS) void k_qsa_tables(qsa_tables_args a) {
    const int64_t stride = (int64_t) gridDim.x * FILL_THREADS;
    const int64_t t0 = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x;
    if (a.blk_cells)
        for (int64_t i = t0; i < a.n_blocks_max * a.ratio; i += stride) a.blk_cells[i] = (int32_t) i;
    if (a.cell_pos)
        for (int64_t i = t0; i < a.n_ctx; i += stride) a.cell_pos[i] = (float) i;
    if (a.blk_pos_all)
        for (int64_t i = t0; i < 4 * a.n_whole; i += stride) a.blk_pos_all[i] = (int32_t) ((i % a.n_whole) * a.ratio);
}

// ---- the prefill chunk's sparse-attention inputs (engine::fill_chunk_qsa,
//      qwfn_engine.cpp:1276-1320), closed form per element. n_kv = n_past_c +
//      Tc, n_blocks = ceil(n_kv / ratio), n_bid = n_kv / ratio whole blocks,
//      dead = the partial tail block (n_bid) if there is one, else the last.
struct qsa_chunk_args {
    int32_t * cell_blk;    // [n_kv] or null
    int32_t * blk_cells;   // [n_blocks * ratio] or null
    int32_t * blk_pos;     // [4 * n_blocks] or null
    float *   bias;        // [Tc][n_blocks], rows bias_ld floats apart, or null
    int64_t   bias_ld;
    int32_t   bias_vec;    // bias and bias_ld 16-byte aligned: 4 blocks a thread, one 16-byte store
    int64_t   n_past_c, Tc, n_blocks;
    int32_t   ratio;
};

// Row i (query q = n_past_c + i) of the bias at block b: the reference's fills
// (0 before tail_b = min(n_bid, (q+1)/ratio), 1e9 up to n_bid, -inf after, the
// dead block 1e9) followed by its -1e9 for positive entries of blocks wholly
// after q.
// tail_b = min((q + 1) / r, n_bid): the whole blocks that end at or before q
__device__ __forceinline__ float chunk_bias(int64_t b, int64_t q, int64_t r, int64_t tail_b, int64_t n_bid, int64_t dead,
                                            bool have_dead) {
    float v = b < tail_b ? 0.0f : (b < n_bid ? 1e9f : -INFINITY);
    if (have_dead && b == dead) v = 1e9f;
    if (b >= tail_b && v > 0.0f && b * r > q) v = -1e9f;
    return v;
}

// blockIdx.y < Tc: bias row blockIdx.y; blockIdx.y == Tc: the three tables.
__global__ __launch_bounds__(FILL_THREADS) void k_qsa_chunk(qsa_chunk_args a) {
    const int64_t r = a.ratio, n_kv = a.n_past_c + a.Tc, n_bid = n_kv / r;
    const bool have_dead = n_bid < a.n_blocks;
    const int64_t dead = have_dead ? n_bid : a.n_blocks - 1;
    const int64_t t0 = (int64_t) blockIdx.x * FILL_THREADS + threadIdx.x;
    const int64_t stride = (int64_t) gridDim.x * FILL_THREADS;
    if ((int64_t) blockIdx.y < a.Tc) {
        if (!a.bias) return;
        const int64_t q = a.n_past_c + blockIdx.y;
        const int64_t tail_b = (q + 1) / r < n_bid ? (q + 1) / r : n_bid;
        float * row = a.bias + (size_t) blockIdx.y * (size_t) a.bias_ld;
        if (a.bias_vec) {
            for (int64_t b = 4 * t0; b < a.n_blocks; b += 4 * stride) {
                if (b + 4 <= a.n_blocks) {
                    *(float4 *) (row + b) = make_float4(chunk_bias(b, q, r, tail_b, n_bid, dead, have_dead),
                                                        chunk_bias(b + 1, q, r, tail_b, n_bid, dead, have_dead),
                                                        chunk_bias(b + 2, q, r, tail_b, n_bid, dead, have_dead),
                                                        chunk_bias(b + 3, q, r, tail_b, n_bid, dead, have_dead));
                } else {
                    for (int64_t e = b; e < a.n_blocks; e++) row[e] = chunk_bias(e, q, r, tail_b, n_bid, dead, have_dead);
                }
            }
        } else {
            for (int64_t b = t0; b < a.n_blocks; b += stride) row[b] = chunk_bias(b, q, r, tail_b, n_bid, dead, have_dead);
        }
        return;
    }
    if (a.cell_blk)
        for (int64_t j = t0; j < n_kv; j += stride) a.cell_blk[j] = (int32_t) (j < n_bid * r ? j / r : dead);
    if (a.blk_cells)
        for (int64_t i = t0; i < a.n_blocks * r; i += stride) {
            const int64_t b = i / r;
            // whole blocks: their own cells; the partial tail block: its real
            // cells, the last one repeated (n_blocks = ceil(n_kv / ratio), so no
            // block lies past it)
            a.blk_cells[i] = (int32_t) (b < n_bid ? i : (i < n_kv - 1 ? i : n_kv - 1));
        }
    if (a.blk_pos)
        for (int64_t i = t0; i < 4 * a.n_blocks; i += stride) a.blk_pos[i] = (int32_t) ((i % a.n_blocks) * r);
}

// ---- the prefill's selection mask (graph_builder::qsa_mask, qwfn_graph.cpp:
//      388-414): -inf everywhere, 0 at the query's selected cells, plus the
//      causal mask. Block = query row t: its selected cells become a bitmap in
//      LDS, then every 8-key group of the row is written once: the causal
//      value where the key is selected, -inf elsewhere (and in the padding
//      past n_kv). Cells outside [0, n_kv) are skipped and flagged.
__global__ __launch_bounds__(FILL_THREADS) void k_qsa_mask(const int32_t * cells, int64_t width, int64_t cells_ld,
                                                          const uint16_t * causal, int64_t causal_ld, int64_t n_kv,
                                                          uint16_t * mask, int64_t mask_ld, uint32_t * status) {
    extern __shared__ uint32_t sel[];   // ceil(n_kv / 32) words
    const int64_t t = blockIdx.x;
    const int64_t n_words = (n_kv + 31) / 32;
    for (int64_t w = threadIdx.x; w < n_words; w += FILL_THREADS) sel[w] = 0u;
    __syncthreads();
    const int32_t * crow = cells + (size_t) t * (size_t) cells_ld;
    bool bad = false;
    // a thread's cells 8 at a time, all 8 loaded before any atomic
    for (int64_t j0 = threadIdx.x; j0 < width; j0 += (int64_t) FILL_THREADS * CELL_BATCH) {
        int32_t cb[CELL_BATCH];
#pragma unroll
        for (int u = 0; u < CELL_BATCH; u++) {
            const int64_t j = j0 + (int64_t) u * FILL_THREADS;
            cb[u] = j < width ? crow[j] : 0;
        }
#pragma unroll
        for (int u = 0; u < CELL_BATCH; u++) {
            if (j0 + (int64_t) u * FILL_THREADS >= width) break;
            const int64_t c = cb[u];
            if (c < 0 || c >= n_kv) { bad = true; continue; }
            atomicOr(&sel[c >> 5], 1u << (c & 31));
        }
    }
    if (__any(bad) && (threadIdx.x & 63) == 0 && status) atomicOr(status, DEVERR_SET_ROWS_INDEX);
    __syncthreads();
    const uint16_t * src = causal + (size_t) t * (size_t) causal_ld;
    uint16_t * dst = mask + (size_t) t * (size_t) mask_ld;
    const int64_t groups = (mask_ld + 7) / 8;
    const bool src_al = ((uintptr_t) src & 15) == 0;
    // a thread's groups in batches of MB: their causal values are loaded as
    // 16-byte vectors (where the group lies inside the row, is aligned and
    // holds a selected key) before any is used, so a batch waits for one
    // round of loads
    constexpr int MB = 8;
    for (int64_t gb = threadIdx.x; gb < groups; gb += (int64_t) FILL_THREADS * MB) {
        uint4 cw[MB];
#pragma unroll
        for (int u = 0; u < MB; u++) {
            const int64_t j0 = (gb + (int64_t) u * FILL_THREADS) * 8;
            // only groups holding a selected key are read
            const bool any = j0 + 8 <= n_kv && ((sel[j0 >> 5] >> (j0 & 31)) & 0xffu) != 0u;
            cw[u] = (src_al && any) ? *(const uint4 *) (src + j0) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < MB; u++) {
            const int64_t g = gb + (int64_t) u * FILL_THREADS;
            if (g >= groups) break;
            const int64_t j0 = g * 8;
            const bool vec = src_al && j0 + 8 <= n_kv;
            const uint32_t cwv[4] = {cw[u].x, cw[u].y, cw[u].z, cw[u].w};
            uint16_t v[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int64_t j = j0 + e;
                const bool on = j < n_kv && ((sel[j >> 5] >> (j & 31)) & 1u);
                // selected: f16(+0 + c), which is c except that -0 becomes +0
                const uint16_t c = on ? (vec ? (uint16_t) (cwv[e >> 1] >> (16 * (e & 1))) : src[j]) : F16_NINF;
                v[e] = c == 0x8000u ? F16_ZERO : c;
            }
            if (j0 + 8 <= mask_ld && ((uintptr_t) (dst + j0) & 15) == 0) {
                uint4 w;
                w.x = v[0] | ((uint32_t) v[1] << 16);
                w.y = v[2] | ((uint32_t) v[3] << 16);
                w.z = v[4] | ((uint32_t) v[5] << 16);
                w.w = v[6] | ((uint32_t) v[7] << 16);
                store_nt16(dst + j0, w);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (j0 + e < mask_ld) dst[j0 + e] = v[e];
            }
        }
    }
}

// ---- the keys each query of a QSA-on prefill chunk sees: the zeros of the
//      selection mask (graph_builder::qsa_mask, qwfn_graph.cpp:388-414) over
//      the chunk's causal mask (0 up to the query's position, -inf after,
//      qwfn_engine.cpp:1261-1270), as a list: the distinct cells query t
//      selected at or before its position n_past + t, ascending. Block =
//      query row t: its cells become a bitmap in LDS; thread i counts the set
//      bits of its run of words, the counts are scanned across the block, and
//      each thread writes its cells from its offset on. ----
__global__ __launch_bounds__(FILL_THREADS) void k_qsa_visible(const int32_t * cells, int64_t width, int64_t cells_ld,
                                                             int64_t n_kv, int64_t n_past, int32_t * lists,
                                                             int64_t lists_ld, int32_t * counts, uint32_t * status) {
    extern __shared__ uint32_t vis[];   // ceil(n_vis / 32) words
    __shared__ uint32_t wsum[FILL_THREADS / 64];
    const int64_t t = blockIdx.x;
    const int64_t n_vis = n_past + t + 1 < n_kv ? n_past + t + 1 : n_kv;   // keys at or before the position
    const int64_t n_words = (n_vis + 31) / 32;
    for (int64_t w = threadIdx.x; w < n_words; w += FILL_THREADS) vis[w] = 0u;
    __syncthreads();
    const int32_t * crow = cells + (size_t) t * (size_t) cells_ld;
    bool bad = false;
    // a thread's cells 8 at a time, all 8 loaded before any atomic
    for (int64_t j0 = threadIdx.x; j0 < width; j0 += (int64_t) FILL_THREADS * CELL_BATCH) {
        int32_t cb[CELL_BATCH];
#pragma unroll
        for (int u = 0; u < CELL_BATCH; u++) {
            const int64_t j = j0 + (int64_t) u * FILL_THREADS;
            cb[u] = j < width ? crow[j] : 0;
        }
#pragma unroll
        for (int u = 0; u < CELL_BATCH; u++) {
            if (j0 + (int64_t) u * FILL_THREADS >= width) break;
            const int64_t c = cb[u];
            if (c < 0 || c >= n_kv) { bad = true; continue; }
            if (c < n_vis) atomicOr(&vis[c >> 5], 1u << (c & 31));
        }
    }
    if (__any(bad) && (threadIdx.x & 63) == 0 && status) atomicOr(status, DEVERR_SET_ROWS_INDEX);
    __syncthreads();
    const int64_t per = (n_words + FILL_THREADS - 1) / FILL_THREADS;
    const int64_t w0 = (int64_t) threadIdx.x * per, w1 = w0 + per < n_words ? w0 + per : n_words;
    uint32_t cnt = 0;
    for (int64_t w = w0; w < w1; w++) cnt += (uint32_t) __popc(vis[w]);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(inc, o);
        if (lane >= o) inc += y;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (int k = 0; k < FILL_THREADS / 64; k++) {
        if (k < wv) base += wsum[k];
        total += wsum[k];
    }
    int32_t * orow = lists + (size_t) t * (size_t) lists_ld;
    uint32_t off = base + inc - cnt;
    for (int64_t w = w0; w < w1; w++) {
        uint32_t bits = vis[w];
        while (bits) {
            const int b = __ffs((int) bits) - 1;
            orow[off++] = (int32_t) (w * 32 + b);
            bits &= bits - 1u;
        }
    }
    if (threadIdx.x == 0) counts[t] = (int32_t) total;
}

unsigned grid_for(int64_t n) {
    return (unsigned) std::max<int64_t>(1, std::min<int64_t>((n + FILL_THREADS - 1) / FILL_THREADS, 4096));
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

// ------------------------------------------------------------ state owner

namespace qwfn {
namespace {

int add_entry(qwfn_state & st, int32_t kind, uint32_t il, bool host, int32_t type, std::initializer_list<int64_t> ne,
              size_t & cursor) {
    qwfn_state::entry e{};
    e.kind = kind; e.il = il; e.host = host; e.type = type;
    int d = 0;
    for (int64_t n : ne) e.ne[d++] = n;
    for (; d < 4; d++) e.ne[d] = 1;
    e.nb[0] = type_size(type);
    e.nb[1] = e.nb[0] * (size_t) (e.ne[0] / type_blck(type));
    for (int i = 2; i < 4; i++) e.nb[i] = e.nb[i - 1] * (size_t) e.ne[i - 1];
    e.bytes = e.nb[3] * (size_t) e.ne[3];
    cursor = align_up(cursor, ARENA_ALIGN);
    e.off = cursor;
    cursor += e.bytes;
    st.entries.push_back(e);
    return (int) st.entries.size() - 1;
}

int validate_config(const qwfn_state_config & c) {
    if (c.n_ctx < 1 || c.n_ctx > (1u << 24))
        return set_error(QWFN_EINVAL, "state: n_ctx must be in [1, 2^24] (cell positions are exact in f32)");
    if (c.n_layer < 1 || c.n_layer > 4096) return set_error(QWFN_EINVAL, "state: n_layer must be in [1, 4096]");
    if (c.type_k != QWFN_TYPE_Q8_0 && c.type_k != QWFN_TYPE_F16)
        return set_error(QWFN_ENOTSUP, "state: type_k must be q8_0 or f16");
    if (c.type_v != QWFN_TYPE_Q8_0 && c.type_v != QWFN_TYPE_F16)
        return set_error(QWFN_ENOTSUP, "state: type_v must be q8_0 or f16");
    if (c.type_idx != QWFN_TYPE_F16 && c.type_idx != QWFN_TYPE_F32)
        return set_error(QWFN_ENOTSUP, "state: type_idx must be f16 or f32");
    bool any_attn = false, any_dn = false;
    for (uint32_t il = 0; il < c.n_layer; il++) {
        const bool a = c.full_attention_interval > 0 && ((il + 1) % c.full_attention_interval) == 0;
        any_attn |= a;
        any_dn |= !a;
    }
    if (any_attn) {
        if (c.n_head_kv < 1 || c.n_embd_head_k < 1 || c.n_embd_head_v < 1 || c.idx_key_len < 1)
            return set_error(QWFN_EINVAL, "state: attention layers need n_head_kv, head sizes and idx_key_len");
        if ((c.type_k == QWFN_TYPE_Q8_0 && (c.n_embd_head_k * c.n_head_kv) % QK) ||
            (c.type_v == QWFN_TYPE_Q8_0 && (c.n_embd_head_v * c.n_head_kv) % QK))
            return set_error(QWFN_EINVAL, "state: a q8_0 cache row must be whole 32-value blocks");
    }
    if (any_dn && (c.ssm_d_state < 1 || c.ssm_n_group < 1 || c.ssm_dt_rank < 1 || c.ssm_d_conv < 2))
        return set_error(QWFN_EINVAL, "state: DeltaNet layers need d_state, n_group, dt_rank and d_conv >= 2");
    if (c.ple_n_head > 0 && (c.ple_conv_kernel < 2 || c.ple_ngram_size < 1 || c.hc_count < 1 || c.n_embd < 1))
        return set_error(QWFN_EINVAL, "state: the PLE history needs conv_kernel >= 2, ngram_size, hc_count and n_embd");
    if (c.n_rollback > 64) return set_error(QWFN_EINVAL, "state: at most 64 rollback slots");
    return QWFN_OK;
}

// declare_tensors (qwfn_state.cpp:48-91): caches per attention layer in layer
// order, then the recurrent region.
void plan(qwfn_state & st) {
    const qwfn_state_config & c = st.cfg;
    const uint32_t L = c.n_layer;
    st.k.assign(L, -1); st.v.assign(L, -1); st.idx.assign(L, -1); st.rs.assign(L, -1); st.conv.assign(L, -1);
    const int64_t n_ctx = c.n_ctx;
    const int64_t kv_dim = (int64_t) c.n_embd_head_k * c.n_head_kv;
    const int64_t v_dim = (int64_t) c.n_embd_head_v * c.n_head_kv;
    const int64_t hv = c.ssm_d_state;
    const int64_t conv_dim = (int64_t) c.ssm_d_state * c.ssm_n_group * 2 + (int64_t) c.ssm_d_state * c.ssm_dt_rank;
    const int64_t hc_dim = (int64_t) c.hc_count * c.n_embd;
    size_t dcur = 0, hcur = 0;
    for (uint32_t il = 0; il < L; il++) {
        if (!st.is_attn(il)) continue;
        st.k[il] = add_entry(st, QWFN_STATE_K, il, c.kv_host, c.type_k, {kv_dim * n_ctx}, c.kv_host ? hcur : dcur);
        st.v[il] = add_entry(st, QWFN_STATE_V, il, c.kv_host, c.type_v, {v_dim * n_ctx}, c.kv_host ? hcur : dcur);
        st.idx[il] = add_entry(st, QWFN_STATE_IDX, il, c.idx_host, c.type_idx, {(int64_t) c.idx_key_len * n_ctx},
                               c.idx_host ? hcur : dcur);
    }
    dcur = align_up(dcur, ARENA_ALIGN);
    st.rec_off = dcur;
    for (uint32_t il = 0; il < L; il++) {
        if (st.is_attn(il)) continue;
        st.rs[il] = add_entry(st, QWFN_STATE_RS, il, false, QWFN_TYPE_F32, {hv, hv, (int64_t) c.ssm_dt_rank}, dcur);
        st.conv[il] = add_entry(st, QWFN_STATE_CONV, il, false, QWFN_TYPE_F32, {(int64_t) c.ssm_d_conv - 1, conv_dim}, dcur);
    }
    if (c.ple_n_head > 0) {
        const int64_t hist = (int64_t) (c.ple_conv_kernel - 1) * c.ple_ngram_size;
        st.ple = add_entry(st, QWFN_STATE_PLE_CONV, 0, false, QWFN_TYPE_F32, {hist, hc_dim}, dcur);
    }
    dcur = align_up(dcur, ARENA_ALIGN);
    st.rec_bytes = dcur - st.rec_off;
    st.dev_bytes = dcur;
    st.host_bytes = align_up(hcur, ARENA_ALIGN);
}

}  // namespace

int zero_recurrent(qwfn_state & st, hipStream_t stream) {
    if (!st.dev) return set_error(QWFN_EINVAL, "state: created with QWFN_LAYOUT_ONLY, it has no memory");
    return launch_zero(st.dev + st.rec_off, st.rec_bytes, stream);
}

namespace {

void fill_desc(const qwfn_state & st, const qwfn_state::entry & e, int32_t slot, qwfn_tensor * out) {
    *out = qwfn_tensor{};
    out->data = st.addr(e, slot);
    out->type = e.type;
    for (int i = 0; i < 4; i++) { out->ne[i] = e.ne[i]; out->nb[i] = e.nb[i]; }
}

// snapshot_parts over one state (qwfn_engine.cpp:990-999)
}  // namespace

void parts_of(const qwfn_state & st, int32_t n, std::vector<qwfn_part> & out, std::vector<bool> * host_side) {
    auto push = [&](int ei, bool positional) {
        if (ei < 0) return;
        const qwfn_state::entry & e = st.entries[(size_t) ei];
        const size_t b = positional ? std::min(e.bytes, (size_t) n * st.row_bytes(e)) : e.bytes;
        out.push_back(qwfn_part{st.addr(e, -1), b});
        if (host_side) host_side->push_back(e.host);
    };
    for (uint32_t il = 0; il < st.cfg.n_layer; il++) {
        push(st.k[il], true);
        push(st.v[il], true);
        push(st.idx[il], true);
        push(st.rs[il], false);
        push(st.conv[il], false);
    }
    push(st.ple, false);
}

// Copies parts between state tensors and caller buffers: device<->device parts
// in batched kernels, anything that touches host memory with the copy engine.
// Allocates nothing (callers rely on that after they have changed their own
// bookkeeping).
int copy_parts(const std::vector<const char *> & src, const std::vector<char *> & dst, const std::vector<size_t> & bytes,
               const std::vector<bool> & host_side, hipStream_t stream) {
    constexpr int BATCH = 96;   // one launch of the single-destination copy kernel
    const char * ks[BATCH];
    char * kd[BATCH];
    size_t kb[BATCH];
    int n = 0;
    for (size_t k = 0; k < src.size(); k++) {
        if (!bytes[k]) continue;
        if (host_side[k]) {
            QWFN_HIP_TRY(hipMemcpyAsync(dst[k], src[k], bytes[k], hipMemcpyDefault, stream));
            continue;
        }
        ks[n] = src[k]; kd[n] = dst[k]; kb[n] = bytes[k];
        if (++n == BATCH) {
            if (int rc = restore_device(ks, kb, kd, n, 1, 0, stream)) return rc;
            n = 0;
        }
    }
    return n ? restore_device(ks, kb, kd, n, 1, 0, stream) : QWFN_OK;
}

int check_states(const qwfn_state * const * sts, int32_t n_sts, bool need_memory, const char * what) {
    if (!sts || n_sts < 1) return set_error(QWFN_EINVAL, std::string(what) + ": no states");
    for (int32_t i = 0; i < n_sts; i++) {
        if (!sts[i]) return set_error(QWFN_EINVAL, std::string(what) + ": NULL state");
        if (need_memory && !sts[i]->dev)
            return set_error(QWFN_EINVAL, std::string(what) + ": a state created with QWFN_LAYOUT_ONLY has no memory");
        if (need_memory && sts[i]->device != sts[0]->device)
            return set_error(QWFN_EINVAL, std::string(what) + ": states on different devices");
    }
    return QWFN_OK;
}

}  // namespace qwfn

extern "C" {

void qwfn_state_config_default(qwfn_state_config * c, uint32_t n_ctx) {
    if (!c) return;
    *c = qwfn_state_config{};
    c->n_ctx = n_ctx;
    c->n_layer = 48;
    c->full_attention_interval = 4;
    c->n_head_kv = 2;
    c->n_embd_head_k = 256;
    c->n_embd_head_v = 256;
    c->idx_key_len = 128;
    c->ssm_d_state = 128;
    c->ssm_n_group = 16;
    c->ssm_dt_rank = 48;
    c->ssm_d_conv = 4;
    c->hc_count = 4;
    c->n_embd = 2560;
    c->ple_n_head = 16;
    c->ple_conv_kernel = 4;
    c->ple_ngram_size = 3;
    c->type_k = QWFN_TYPE_Q8_0;
    c->type_v = QWFN_TYPE_Q8_0;
    c->type_idx = QWFN_TYPE_F16;
}

int qwfn_state_create(const qwfn_state_config * cfg, int device, qwfn_state ** out) {
    return ::qwfn::abi_call("state_create", [&]() -> int {
        if (!cfg || !out) return set_error(QWFN_EINVAL, "state_create: NULL argument");
        *out = nullptr;
        if (int rc = validate_config(*cfg)) return rc;
        if (device < QWFN_LAYOUT_ONLY) return set_error(QWFN_EINVAL, "state_create: bad device");
        std::unique_ptr<qwfn_state> st(new (std::nothrow) qwfn_state());
        if (!st) return set_error(QWFN_ENOMEM, "state_create: out of host memory");
        st->cfg = *cfg;
        plan(*st);
        if (device == QWFN_LAYOUT_ONLY) {
            *out = st.release();
            return QWFN_OK;
        }
        int n = 0;
        QWFN_HIP_TRY(hipGetDeviceCount(&n));
        if (device >= n) return set_error(QWFN_EINVAL, "state_create: device " + std::to_string(device) + " of " + std::to_string(n));
        st->device = device;
        device_scope ds(device);
        if (ds.rc) return ds.rc;
        void * p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(st->dev_bytes, ARENA_ALIGN)) != hipSuccess)
            return set_error(QWFN_ENOMEM, "failed to allocate state buffer");
        st->dev = (char *) p;
        if (st->host_bytes) {
            // mapped so that the device kernels can address the caches over the host link
            if (hipHostMalloc(&p, st->host_bytes, hipHostMallocMapped | hipHostMallocPortable) != hipSuccess)
                return set_error(QWFN_ENOMEM, "failed to allocate the host state buffer");
            st->host = (char *) p;
            void * dp = nullptr;
            QWFN_HIP_TRY(hipHostGetDevicePointer(&dp, p, 0));
            st->host_dev = (char *) dp;
        }
        if (cfg->n_rollback) {
            if (hipMalloc(&p, (size_t) cfg->n_rollback * std::max<size_t>(st->rec_bytes, ARENA_ALIGN)) != hipSuccess)
                return set_error(QWFN_ENOMEM, "no device memory for the rollback snapshots");
            st->rb = (char *) p;
        }
        // recurrent state and conv history start at zero; the caches need not
        if (int rc = zero_recurrent(*st, nullptr)) return rc;
        QWFN_HIP_TRY(hipStreamSynchronize(nullptr));
        *out = st.release();
        return QWFN_OK;
    });
}

void qwfn_state_destroy(qwfn_state * st) { delete st; }

int qwfn_state_tensor(const qwfn_state * st, int32_t kind, uint32_t il, int32_t slot, qwfn_tensor * out) {
    return ::qwfn::abi_call("state_tensor", [&]() -> int {
        if (!st || !out) return set_error(QWFN_EINVAL, "state_tensor: NULL argument");
        *out = qwfn_tensor{};
        const bool recurrent = kind == QWFN_STATE_RS || kind == QWFN_STATE_CONV || kind == QWFN_STATE_PLE_CONV;
        if (kind < QWFN_STATE_K || kind > QWFN_STATE_PLE_CONV) return set_error(QWFN_EINVAL, "state_tensor: unknown kind");
        if (slot < -1 || (slot >= 0 && (!recurrent || slot >= (int32_t) st->cfg.n_rollback)))
            return set_error(QWFN_ERANGE, "state_tensor: no such rollback slot");
        int ei = -1;
        if (kind == QWFN_STATE_PLE_CONV) ei = st->ple;
        else if (il < st->cfg.n_layer) {
            switch (kind) {
                case QWFN_STATE_K:    ei = st->k[il]; break;
                case QWFN_STATE_V:    ei = st->v[il]; break;
                case QWFN_STATE_IDX:  ei = st->idx[il]; break;
                case QWFN_STATE_RS:   ei = st->rs[il]; break;
                default:              ei = st->conv[il]; break;
            }
        }
        if (ei < 0) return 0;
        fill_desc(*st, st->entries[(size_t) ei], slot, out);
        return 1;
    });
}

size_t qwfn_state_bytes(const qwfn_state * st) { return st ? st->dev_bytes : 0; }
size_t qwfn_state_host_bytes(const qwfn_state * st) { return st ? st->host_bytes : 0; }
size_t qwfn_state_rollback_bytes(const qwfn_state * st) { return st ? (size_t) st->cfg.n_rollback * st->rec_bytes : 0; }
uint32_t qwfn_state_n_ctx(const qwfn_state * st) { return st ? st->cfg.n_ctx : 0; }
int32_t qwfn_state_n_past(const qwfn_state * st) { return st ? st->n_past : 0; }
int32_t qwfn_state_rollback_depth(const qwfn_state * st) { return st ? st->rb_depth : 0; }

int qwfn_state_summary(const qwfn_state * st, char * buf, size_t cap) {
    return ::qwfn::abi_call("state_summary", [&]() -> int {
        if (!st || (!buf && cap)) return set_error(QWFN_EINVAL, "state_summary: NULL argument");
        size_t kv = 0, ix = 0, rs = 0, cv = 0;
        for (const auto & e : st->entries) {
            if (e.kind == QWFN_STATE_K || e.kind == QWFN_STATE_V) kv += e.bytes;
            else if (e.kind == QWFN_STATE_IDX) ix += e.bytes;
            else if (e.kind == QWFN_STATE_RS) rs += e.bytes;
            else cv += e.bytes;
        }
        // qwfn_state.cpp:154-173; doubles printed as an ostream does by default (%g)
        std::string s = "state @ " + std::to_string(st->cfg.n_ctx) + " ctx: ";
        char tmp[512];
        snprintf(tmp, sizeof tmp, "KV %g GB (%s), indexer %g GB, deltanet %g MB (constant), conv %g MB  =>  total %g GB on the device",
                 kv / 1e9, type_name(st->cfg.type_k), ix / 1e9, rs / 1e6, cv / 1e6, st->dev_bytes / 1e9);
        s += tmp;
        if (st->host_bytes) {
            snprintf(tmp, sizeof tmp, " + %g GB in pinned host memory", st->host_bytes / 1e9);
            s += tmp;
        }
        if (cap) {
            const size_t n = std::min(cap - 1, s.size());
            memcpy(buf, s.data(), n);
            buf[n] = '\0';
        }
        return (int) s.size();
    });
}

int qwfn_state_step_done(qwfn_state * st, int32_t T, int32_t verified) {
    return ::qwfn::abi_call("state_step_done", [&]() -> int {
        if (!st) return set_error(QWFN_EINVAL, "state_step_done: NULL state");
        if (T < 1) return set_error(QWFN_EINVAL, "state_step_done: a step has at least one position");
        if ((int64_t) st->n_past + T > (int64_t) st->cfg.n_ctx) return set_error(QWFN_ERANGE, "context exhausted");
        st->rb_depth = (verified && T >= 2 && st->cfg.n_rollback > 0) ? std::min<int32_t>(T - 1, (int32_t) st->cfg.n_rollback) : 0;
        st->n_past += T;
        return QWFN_OK;
    });
}

int qwfn_state_reset(qwfn_state * st, void * stream) {
    return ::qwfn::abi_call("state_reset", [&]() -> int {
        if (!st) return set_error(QWFN_EINVAL, "state_reset: NULL state");
        device_scope ds(st->device);
        if (ds.rc) return ds.rc;
        if (st->dev)   // a QWFN_LAYOUT_ONLY state has only its bookkeeping
            if (int rc = zero_recurrent(*st, as_stream(stream))) return rc;
        st->n_past = 0;
        st->rb_depth = 0;
        return QWFN_OK;
    });
}

int qwfn_state_rollback(qwfn_state * st, int32_t n_back, void * stream) {
    return ::qwfn::abi_call("state_rollback", [&]() -> int {
        if (!st) return set_error(QWFN_EINVAL, "state_rollback: NULL state");
        if (n_back < 1 || n_back > st->rb_depth)
            return set_error(QWFN_ERANGE, "rollback: no snapshot of the state " + std::to_string(n_back) + " tokens back");
        if (!st->dev || !st->rb) return set_error(QWFN_EINVAL, "state_rollback: the state has no rollback memory");
        device_scope ds(st->device);
        if (ds.rc) return ds.rc;
        const char * src = st->rb + (size_t) (n_back - 1) * st->rec_bytes;
        char * dst = st->dev + st->rec_off;
        const size_t b = st->rec_bytes;
        if (int rc = restore_device(&src, &b, &dst, 1, 1, 0, as_stream(stream))) return rc;
        st->n_past -= n_back;
        st->rb_depth = 0;
        return QWFN_OK;
    });
}

int qwfn_snapshot_parts(const qwfn_state * const * sts, int32_t n_sts, int32_t n_past, qwfn_part * parts,
                        int32_t max_parts, int32_t * n_parts) {
    return ::qwfn::abi_call("snapshot_parts", [&]() -> int {
        if (!n_parts || (max_parts > 0 && !parts) || max_parts < 0) return set_error(QWFN_EINVAL, "snapshot_parts: bad output array");
        if (int rc = check_states(sts, n_sts, false, "snapshot_parts")) return rc;
        if (n_past < 0) return set_error(QWFN_EINVAL, "snapshot_parts: a position count");
        std::vector<qwfn_part> all;
        for (int32_t i = 0; i < n_sts; i++) parts_of(*sts[i], n_past, all, nullptr);
        *n_parts = (int32_t) all.size();
        for (int32_t k = 0; k < std::min<int32_t>(max_parts, (int32_t) all.size()); k++) parts[k] = all[(size_t) k];
        return QWFN_OK;
    });
}

int qwfn_snapshot_save(const qwfn_state * const * sts, int32_t n_sts, void * const * dst, const size_t * dst_bytes,
                       int32_t n_dst, int32_t dst_kind, int32_t * n_past_out, void * stream) {
    return ::qwfn::abi_call("snapshot_save", [&]() -> int {
        if (int rc = check_states(sts, n_sts, true, "snapshot_save")) return rc;
        if (dst_kind != QWFN_MEM_DEVICE && dst_kind != QWFN_MEM_HOST) return set_error(QWFN_EINVAL, "snapshot_save: unknown destination kind");
        const int32_t n_past = sts[0]->n_past;
        for (int32_t i = 1; i < n_sts; i++)
            if (sts[i]->n_past != n_past) return set_error(QWFN_EINVAL, "snapshot_save: the states disagree on n_past");
        std::vector<qwfn_part> parts;
        std::vector<bool> host_side;
        for (int32_t i = 0; i < n_sts; i++) parts_of(*sts[i], n_past, parts, &host_side);
        if (n_dst != (int32_t) parts.size() || (n_dst && (!dst || !dst_bytes)))
            return set_error(QWFN_ESIZE, "snapshot_save: " + std::to_string(parts.size()) + " parts, " + std::to_string(n_dst) + " buffers");
        std::vector<const char *> src;
        std::vector<char *> d;
        std::vector<size_t> b;
        for (size_t k = 0; k < parts.size(); k++) {
            if (dst_bytes[k] != parts[k].bytes)
                return set_error(QWFN_ESIZE, "snapshot_save: buffer " + std::to_string(k) + " has " + std::to_string(dst_bytes[k]) +
                                                 " bytes, the part " + std::to_string(parts[k].bytes));
            if (parts[k].bytes && !dst[k]) return set_error(QWFN_EINVAL, "snapshot_save: NULL buffer " + std::to_string(k));
            src.push_back((const char *) parts[k].data);
            d.push_back((char *) dst[k]);
            b.push_back(parts[k].bytes);
            if (dst_kind == QWFN_MEM_HOST) host_side[k] = true;
        }
        device_scope ds(sts[0]->device);
        if (ds.rc) return ds.rc;
        if (int rc = copy_parts(src, d, b, host_side, as_stream(stream))) return rc;
        if (n_past_out) *n_past_out = n_past;
        return QWFN_OK;
    });
}

int qwfn_snapshot_load(qwfn_state * const * sts, int32_t n_sts, int32_t n_past, const void * const * src,
                       const size_t * src_bytes, int32_t n_src, int32_t src_kind, void * stream) {
    return ::qwfn::abi_call("snapshot_load", [&]() -> int {
        if (int rc = check_states(sts, n_sts, true, "snapshot_load")) return rc;
        if (src_kind != QWFN_MEM_DEVICE && src_kind != QWFN_MEM_HOST) return set_error(QWFN_EINVAL, "snapshot_load: unknown source kind");
        for (int32_t i = 0; i < n_sts; i++)
            if (n_past < 0 || n_past > (int32_t) sts[i]->cfg.n_ctx) return set_error(QWFN_ERANGE, "snapshot_load: n_past outside the context");
        device_scope ds(sts[0]->device);
        if (ds.rc) return ds.rc;
        hipStream_t s = as_stream(stream);
        // engine::snapshot_load resets before it checks the parts (qwfn_engine.cpp:1034-1040)
        for (int32_t i = 0; i < n_sts; i++)
            if (int rc = qwfn_state_reset(sts[i], stream)) return rc;
        std::vector<qwfn_part> parts;
        std::vector<bool> host_side;
        for (int32_t i = 0; i < n_sts; i++) parts_of(*sts[i], n_past, parts, &host_side);
        if (n_src != (int32_t) parts.size() || (n_src && (!src || !src_bytes)))
            return set_error(QWFN_ESIZE, "snapshot_load: " + std::to_string(n_src) + " parts given, " + std::to_string(parts.size()) + " expected");
        std::vector<const char *> sp;
        std::vector<char *> dp;
        std::vector<size_t> b;
        for (size_t k = 0; k < parts.size(); k++) {
            if (src_bytes[k] != parts[k].bytes)
                return set_error(QWFN_ESIZE, "snapshot_load: part " + std::to_string(k) + " has " + std::to_string(src_bytes[k]) +
                                                 " bytes, expected " + std::to_string(parts[k].bytes));
            if (parts[k].bytes && !src[k]) return set_error(QWFN_EINVAL, "snapshot_load: NULL part " + std::to_string(k));
            sp.push_back((const char *) src[k]);
            dp.push_back((char *) parts[k].data);
            b.push_back(parts[k].bytes);
            if (src_kind == QWFN_MEM_HOST) host_side[k] = true;
        }
        if (int rc = copy_parts(sp, dp, b, host_side, s)) return rc;
        for (int32_t i = 0; i < n_sts; i++) sts[i]->n_past = n_past;
        return QWFN_OK;
    });
}

// ---------------------------------------------------------------- masks

int qwfn_causal_mask_f16(uint16_t * mask, int64_t n_kv, int64_t T, int64_t n_past, size_t row_stride, void * stream) {
    return ::qwfn::abi_call("causal_mask_f16", [&]() -> int {
        if (!mask) return set_error(QWFN_EINVAL, "causal_mask: NULL mask");
        if (n_kv < 0 || T < 0 || n_past < 0) return set_error(QWFN_EINVAL, "causal_mask: negative size");
        if (row_stride % 2 || row_stride < (size_t) n_kv * 2 || !is_aligned(mask, 2))
            return set_error(QWFN_EALIGN, "causal_mask: row_stride must be even and hold n_kv keys");
        const int64_t groups = (int64_t) ((row_stride / 2 + 7) / 8);
        if (T == 0 || groups == 0) return QWFN_OK;
        const int64_t gx = std::min<int64_t>((groups + FILL_THREADS - 1) / FILL_THREADS, 1024);
        for (int64_t i0 = 0; i0 < T; i0 += 65535) {   // grid rows: at most 65535 a launch
            const int64_t nr = std::min<int64_t>(T - i0, 65535);
            hipLaunchKernelGGL(k_causal_mask, dim3((unsigned) gx, (unsigned) nr), dim3(FILL_THREADS), 0, as_stream(stream),
                               (char *) mask, n_kv, n_past, row_stride, groups, i0);
        }
        return hip_check(hipGetLastError(), "causal_mask launch");
    });
}

int qwfn_cell_mask_f16(const int32_t * cells, int64_t n_cells, int64_t n_pad, int32_t n_past, uint16_t * mask,
                       int32_t * gcells, void * stream) {
    return ::qwfn::abi_call("cell_mask_f16", [&]() -> int {
        if (!cells || !mask) return set_error(QWFN_EINVAL, "cell_mask: NULL pointer");
        if (n_cells < 1 || n_pad < n_cells || n_pad > 2 * n_cells)
            return set_error(QWFN_EINVAL, "cell_mask: need 1 <= n_cells <= n_pad <= 2 n_cells");
        if (n_past < 0) return set_error(QWFN_EINVAL, "cell_mask: negative n_past");
        if (!is_aligned(cells, 4) || !is_aligned(mask, 2) || (gcells && !is_aligned(gcells, 4)))
            return set_error(QWFN_EALIGN, "cell_mask: misaligned pointer");
        hipLaunchKernelGGL(k_cell_mask, dim3(grid_for(n_pad)), dim3(FILL_THREADS), 0, as_stream(stream), cells, n_cells, n_pad,
                           n_past, mask, gcells);
        return hip_check(hipGetLastError(), "cell_mask launch");
    });
}

int qwfn_qsa_chunk_inputs(int64_t n_past_c, int64_t Tc, int32_t ratio, int32_t * cell_blk, int32_t * blk_cells,
                          int32_t * blk_pos, float * bias, size_t bias_nb1, void * stream) {
    return ::qwfn::abi_call("qsa_chunk_inputs", [&]() -> int {
        if (n_past_c < 0 || Tc < 1 || ratio < 1) return set_error(QWFN_EINVAL, "qsa_chunk_inputs: need n_past_c >= 0, Tc >= 1, ratio >= 1");
        if (Tc > 65535 - 1) return set_error(QWFN_ENOTSUP, "qsa_chunk_inputs: at most 65534 queries per chunk");
        const int64_t n_kv = n_past_c + Tc;
        if (n_kv >= (int64_t(1) << 31)) return set_error(QWFN_ENOTSUP, "qsa_chunk_inputs: n_kv must fit int32");
        const int64_t n_blocks = (n_kv + ratio - 1) / ratio;
        if (bias && (bias_nb1 % 4 || bias_nb1 < (size_t) n_blocks * 4))
            return set_error(QWFN_EINVAL, "qsa_chunk_inputs: bias rows must be float [n_blocks] at a 4-byte multiple stride");
        if ((cell_blk && !is_aligned(cell_blk, 4)) || (blk_cells && !is_aligned(blk_cells, 4)) ||
            (blk_pos && !is_aligned(blk_pos, 4)) || (bias && !is_aligned(bias, 4)))
            return set_error(QWFN_EALIGN, "qsa_chunk_inputs: misaligned pointer");
        qsa_chunk_args a{};
        a.cell_blk = cell_blk; a.blk_cells = blk_cells; a.blk_pos = blk_pos; a.bias = bias;
        a.bias_ld = (int64_t) (bias_nb1 / 4);
        a.bias_vec = bias && is_aligned(bias, 16) && bias_nb1 % 16 == 0;
        a.n_past_c = n_past_c; a.Tc = Tc; a.n_blocks = n_blocks; a.ratio = ratio;
        // sized for a bias row (4 blocks a thread when aligned): the table row
        // (blockIdx.y == Tc) strides over its longer tables
        const dim3 g(grid_for(a.bias_vec ? (n_blocks + 3) / 4 : n_blocks), (unsigned) (Tc + 1));
        hipLaunchKernelGGL(k_qsa_chunk, g, dim3(FILL_THREADS), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_chunk_inputs launch");
    });
}

int qwfn_qsa_mask_f16(const int32_t * cells, int64_t width, size_t cells_nb1, const uint16_t * causal,
                      size_t causal_nb1, int64_t n_kv, int64_t T, uint16_t * mask, size_t mask_nb1, void * stream) {
    return ::qwfn::abi_call("qsa_mask_f16", [&]() -> int {
        if (!cells || !causal || !mask) return set_error(QWFN_EINVAL, "qsa_mask: NULL pointer");
        if (width < 0 || n_kv < 1 || T < 1) return set_error(QWFN_EINVAL, "qsa_mask: need width >= 0, n_kv >= 1, T >= 1");
        if (cells_nb1 % 4 || cells_nb1 < (size_t) width * 4 || causal_nb1 % 2 || causal_nb1 < (size_t) n_kv * 2 ||
            mask_nb1 % 2 || mask_nb1 < (size_t) n_kv * 2)
            return set_error(QWFN_EINVAL, "qsa_mask: rows must hold width cells, n_kv causal values and n_kv mask values");
        if (!is_aligned(cells, 4) || !is_aligned(causal, 2) || !is_aligned(mask, 2))
            return set_error(QWFN_EALIGN, "qsa_mask: misaligned pointer");
        if (T > 0x7fffffff) return set_error(QWFN_ENOTSUP, "qsa_mask: too many rows");
        const size_t lds = (size_t) ((n_kv + 31) / 32) * 4;
        if (lds > 64 * 1024) return set_error(QWFN_ENOTSUP, "qsa_mask: n_kv beyond 524288 keys");
        // the output (T whole rows) must not overlap the causal mask it reads
        const char * m0 = (const char *) mask, * m1 = m0 + (size_t) T * mask_nb1;
        const char * c0 = (const char *) causal, * c1 = c0 + (size_t) (T - 1) * causal_nb1 + (size_t) n_kv * 2;
        if (m0 < c1 && c0 < m1) return set_error(QWFN_EINVAL, "qsa_mask: mask and causal overlap");
        uint32_t * status = nullptr;
        if (int rc = status_word(&status)) return rc;
        hipLaunchKernelGGL(k_qsa_mask, dim3((unsigned) T), dim3(FILL_THREADS), lds, as_stream(stream), cells, width,
                           (int64_t) (cells_nb1 / 4), causal, (int64_t) (causal_nb1 / 2), n_kv, mask,
                           (int64_t) (mask_nb1 / 2), status);
        return hip_check(hipGetLastError(), "qsa_mask launch");
    });
}

int qwfn_qsa_visible_cells(const int32_t * cells, int64_t width, size_t cells_nb1, int64_t n_kv, int64_t T,
                           int64_t n_past, int32_t * lists, size_t lists_nb1, int32_t * counts, void * stream) {
    return ::qwfn::abi_call("qsa_visible_cells", [&]() -> int {
        if (!cells || !lists || !counts) return set_error(QWFN_EINVAL, "qsa_visible_cells: NULL pointer");
        if (width < 0 || n_kv < 1 || T < 1 || n_past < 0)
            return set_error(QWFN_EINVAL, "qsa_visible_cells: need width >= 0, n_kv >= 1, T >= 1, n_past >= 0");
        if (cells_nb1 % 4 || cells_nb1 < (size_t) width * 4 || lists_nb1 % 4 || lists_nb1 < (size_t) width * 4)
            return set_error(QWFN_EINVAL, "qsa_visible_cells: rows of cells and lists must hold width int32");
        if (!is_aligned(cells, 4) || !is_aligned(lists, 4) || !is_aligned(counts, 4))
            return set_error(QWFN_EALIGN, "qsa_visible_cells: misaligned pointer");
        if (T > 0x7fffffff || n_kv > 0x7fffffff) return set_error(QWFN_ENOTSUP, "qsa_visible_cells: too many rows or keys");
        const size_t lds = (size_t) ((n_kv + 31) / 32) * 4;
        if (lds > 64 * 1024) return set_error(QWFN_ENOTSUP, "qsa_visible_cells: n_kv beyond 524288 keys");
        // the lists (T whole rows) and counts must not overlap the cells they read
        const char * c0 = (const char *) cells, * c1 = c0 + (size_t) (T - 1) * cells_nb1 + (size_t) width * 4;
        const char * l0 = (const char *) lists, * l1 = l0 + (size_t) (T - 1) * lists_nb1 + (size_t) width * 4;
        const char * n0 = (const char *) counts, * n1 = n0 + (size_t) T * 4;
        if ((width > 0 && l0 < c1 && c0 < l1) || (n0 < c1 && c0 < n1) || (width > 0 && n0 < l1 && l0 < n1))
            return set_error(QWFN_EINVAL, "qsa_visible_cells: cells, lists and counts must not overlap");
        uint32_t * status = nullptr;
        if (int rc = status_word(&status)) return rc;
        hipLaunchKernelGGL(k_qsa_visible, dim3((unsigned) T), dim3(FILL_THREADS), lds, as_stream(stream), cells, width,
                           (int64_t) (cells_nb1 / 4), n_kv, n_past, lists, (int64_t) (lists_nb1 / 4), counts, status);
        return hip_check(hipGetLastError(), "qsa_visible_cells launch");
    });
}

// ------------------------------------------- decode-time sparse-attention inputs

int64_t qwfn_qsa_bucket(int32_t n_past, int32_t ratio, int64_t n_blocks_max) {
    return ::qwfn::abi_value<int64_t>("qsa_bucket", 0, [&]() -> int64_t {
        if (ratio < 1 || n_past < 0 || n_blocks_max < 1) return 0;
        const int64_t b_last = n_past / ratio;
        int64_t nb = (b_last + 1 + 255) / 256 * 256;
        nb = std::max<int64_t>(nb, 768);
        return std::min<int64_t>(nb, n_blocks_max);
    });
}

int qwfn_qsa_decode_prepare(const qwfn_qsa_inputs * qd, const float * prev_bias, int32_t n_past, void * stream) {
    return ::qwfn::abi_call("qsa_decode_prepare", [&]() -> int {
        if (!qd || !qd->bias || !qd->write_idx || !qd->member_idx || !qd->blk_pos || !qd->blk_idx || !qd->npast_f)
            return set_error(QWFN_EINVAL, "qsa_decode_prepare: NULL tensor");
        if (qd->ratio < 1 || qd->n_blocks_max < 1 || n_past < 0)
            return set_error(QWFN_EINVAL, "qsa_decode_prepare: need ratio >= 1, n_blocks_max >= 1, n_past >= 0");
        qsa_prep_args a{};
        a.qd = *qd;
        a.prev = prev_bias == qd->bias ? nullptr : prev_bias;
        a.n_past = n_past;
        const int64_t n = std::max<int64_t>(a.prev ? qd->n_blocks_max : 4, qd->ratio);
        hipLaunchKernelGGL(k_qsa_prepare, dim3(grid_for(n)), dim3(FILL_THREADS), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_decode_prepare launch");
    });
}

int qwfn_qsa_decode_prepare_steps(const qwfn_qsa_inputs * qd, int32_t T, int32_t n_past, void * stream) {
    return ::qwfn::abi_call("qsa_decode_prepare_steps", [&]() -> int {
        qsa_prep_steps_args a;
        if (int rc = prep_steps_args(qd, T, n_past, "qsa_decode_prepare_steps", &a)) return rc;
        const int64_t n = std::max<int64_t>(qd[0].n_blocks_max, T);
        hipLaunchKernelGGL(k_qsa_prepare_steps, dim3(grid_for(n)), dim3(FILL_THREADS), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_decode_prepare_steps launch");
    });
}

int qwfn_qsa_bias_rebuild(float * bias, int64_t n_blocks_max, int32_t n_past, int32_t ratio, void * stream) {
    return ::qwfn::abi_call("qsa_bias_rebuild", [&]() -> int {
        if (!bias) return set_error(QWFN_EINVAL, "qsa_bias_rebuild: NULL bias");
        if (n_blocks_max < 1 || ratio < 1 || n_past < -1) return set_error(QWFN_EINVAL, "qsa_bias_rebuild: bad sizes");
        hipLaunchKernelGGL(k_qsa_bias, dim3(grid_for(n_blocks_max)), dim3(FILL_THREADS), 0, as_stream(stream), bias,
                           n_blocks_max, n_past, ratio);
        return hip_check(hipGetLastError(), "qsa_bias_rebuild launch");
    });
}

int qwfn_qsa_tables(int32_t * blk_cells, int64_t n_blocks_max, int32_t ratio, float * cell_pos, int64_t n_ctx,
                    int32_t * blk_pos_all, int64_t n_whole, void * stream) {
    return ::qwfn::abi_call("qsa_tables", [&]() -> int {
        if (ratio < 1 || n_blocks_max < 0 || n_ctx < 0 || n_whole < 0) return set_error(QWFN_EINVAL, "qsa_tables: bad sizes");
        if (n_blocks_max * ratio > INT32_MAX || n_ctx > (int64_t) 1 << 24 || n_whole * ratio > INT32_MAX)
            return set_error(QWFN_ERANGE, "qsa_tables: cell ids must fit int32 (positions exact in f32)");
        qsa_tables_args a{blk_cells, n_blocks_max, ratio, cell_pos, n_ctx, blk_pos_all, n_whole};
        const int64_t n = std::max({blk_cells ? n_blocks_max * ratio : 0, cell_pos ? n_ctx : 0, blk_pos_all ? 4 * n_whole : 0});
        if (n == 0) return QWFN_OK;
        hipLaunchKernelGGL(k_qsa_tables, dim3(grid_for(n)), dim3(FILL_THREADS), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_tables launch");
    });
}

}  // extern "C"
