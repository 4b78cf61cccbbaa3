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
// Two kernels. k_qsa_score reads the pool cache (n_blocks x 128 f16, 4.7 MB
// at 18432 blocks) once for up to 8 queries and computes the dot products on
// the matrix cores, one wave per 16 blocks (per 32 to 128 blocks when many
// queries keep the grid full); the scores land in a workspace, the bias
// added there for up to 8 queries and by k_qsa_topk as it loads them for
// more. k_qsa_topk, one workgroup per query, holds the scores in registers as
// order-preserving keys of the float bits, and writes the cells of the k
// best blocks, best first (ties: lower block first). Usually a threshold
// from a sample of the scores leaves under 1024 candidates, which one
// bitonic sort orders; otherwise a radix select (histograms in LDS) finds the
// k-th largest and the k are placed and sorted.
#include "qwfn_common.h"
#include "qwfn_state.h"

#include <algorithm>

namespace qwfn {
namespace {

constexpr int IDX_DIM = 128;             // indexer key length (hparams::idx_key_len)
constexpr int MAX_IDX_HEADS = 8;
constexpr int SCORE_THREADS = 256;        // 16 blocks per workgroup pass
constexpr int SCORE_T = 8;                // queries scored per pass over the pool
constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_MAX = 1024;            // k_blocks per query, at most
constexpr int TOPK_MAX_KPT = 48;          // scores per thread: n_blocks <= 49152
constexpr int RADIX_BITS = 8;
constexpr int RATIO_MAX = 16;             // cells per block, at most
constexpr int SUBH_LD = 36;               // words per bin of the sub-histograms: 32 counts + 4, rows 16-byte aligned

// scores of query t sit at score[t * ld + b]; ld is n_blocks rounded up to 64
__host__ __device__ constexpr int64_t score_ld(int64_t n) { return (n + 63) / 64 * 64; }

struct score_args {
    const uint16_t * pool;        // F16 [IDX_DIM] per block, block stride pool_nb1 bytes
    size_t           pool_nb1;
    int64_t          n_blocks;
    const float *    q;           // F32 [IDX_DIM][n_heads] per query, query stride q_nb2 bytes
    size_t           q_nb2;
    int32_t          n_heads;
    int32_t          head_bits;   // columns per query: 2^head_bits >= n_heads
    int32_t          T;
    const float *    bias;        // null: the sums over heads alone (k_qsa_topk adds the bias), else F32
    size_t           bias_nb1;    // [n_blocks] per query, query stride bias_nb1 bytes
    float *          score;       // [T][score_ld(n_blocks)]
    int32_t          mb;          // 16-block tiles per wave
};

// sum over the 16 lanes of a DPP row, the same tree as butterflies over lane
// masks 1, 2, 4, 8 (quad swaps, then half-row and row mirrors), so every lane
// of the row holds the same sum
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) x, CTRL, ROW_MASK, 0xf, false);
}

// inclusive prefix sum over the 64 lanes of a wave: shifts within rows of 16,
// then row 0's total into row 1, row 2's into row 3, lanes 0-31's into rows 2-3
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    v += dpp_u<0x111>(v);          // row_shr:1
    v += dpp_u<0x112>(v);          // row_shr:2
    v += dpp_u<0x114>(v);          // row_shr:4
    v += dpp_u<0x118>(v);          // row_shr:8
    v += dpp_u<0x142, 0xa>(v);     // row_bcast:15, rows 1 and 3
    v += dpp_u<0x143, 0xc>(v);     // row_bcast:31, rows 2 and 3
    return v;
}

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float    v4f __attribute__((ext_vector_type(4)));

// Scores as a GEMM on the matrix cores: D[block][col] = pool[block] . q16[col]
// with v_mfma_f32_16x16x32_f16, one wave per a.mb tiles of 16 blocks. The
// columns of a tile are (query, head) pairs, 2^head_bits columns per query
// (heads past n_heads are zero), so a query's heads are adjacent lanes of a
// DPP row. B (the query heads, rounded to f16) is loaded once per wave into
// registers, all of the workgroup's queries: lane (lg, ln) holds dims
// [32 s + 8 lg, +8) of column ln for k-step s. A (the keys) likewise for block
// ln of each 16-block tile, the next tile's keys loaded while the current one
// is scored. D: lane (lg, ln) holds blocks 4 lg + r of column ln. relu, then
// the sum over a query's heads across its lanes; the first lane of each query
// adds the bias and writes 4 scores. No LDS, no barriers: a wave past the
// last block leaves at once.
// 16-column tiles of a pass's query columns, at most: 8 queries of 8 columns
constexpr int SCORE_MAX_QT = SCORE_T * MAX_IDX_HEADS / 16;

__device__ __forceinline__ void score_keys(const score_args & a, int64_t blk, int lg, v8h (&kr)[4]) {
#pragma unroll
    for (int st = 0; st < 4; st++) {
        uint4 raw = make_uint4(0u, 0u, 0u, 0u);
        if (blk < a.n_blocks) raw = *(const uint4 *) ((const char *) a.pool + (size_t) blk * a.pool_nb1 + (32 * st + 8 * lg) * 2);
        kr[st] = __builtin_bit_cast(v8h, raw);
    }
}

__global__ __launch_bounds__(SCORE_THREADS) void k_qsa_score(score_args a) {
    const int lane = threadIdx.x & 63;
    const int ln = lane & 15, lg = lane >> 4;
    const int64_t n = a.n_blocks;
    const int64_t tile0 = ((int64_t) blockIdx.x * (SCORE_THREADS / 64) + (threadIdx.x >> 6)) * a.mb;
    if (tile0 * 16 >= n) return;
    const int t0 = blockIdx.y * SCORE_T;
    const int nt = a.T - t0 < SCORE_T ? a.T - t0 : SCORE_T;
    const int hb = a.head_bits, Hp = 1 << hb;
    const int QT = 16 >> hb;                                      // queries per tile of 16 columns
    const int n_tiles = (nt + QT - 1) / QT;
    const int h = ln & (Hp - 1);
    v8h qb[SCORE_MAX_QT][4];
#pragma unroll
    for (int tile = 0; tile < SCORE_MAX_QT; tile++) {
        const int tl = tile * QT + (ln >> hb);                    // query of this lane's column
        const bool colv = tile < n_tiles && tl < nt && h < a.n_heads;
        const float * qp = (const float *) ((const char *) a.q + (size_t) (t0 + (colv ? tl : 0)) * a.q_nb2)
                           + (colv ? h : 0) * IDX_DIM + 8 * lg;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
            if (colv) { x = *(const float4 *) (qp + 32 * st); y = *(const float4 *) (qp + 32 * st + 4); }
            qb[tile][st] = v8h{(_Float16) x.x, (_Float16) x.y, (_Float16) x.z, (_Float16) x.w,
                               (_Float16) y.x, (_Float16) y.y, (_Float16) y.z, (_Float16) y.w};   // round to nearest even
        }
    }
    const int64_t ld = score_ld(n);
    v8h kr[4];
    score_keys(a, tile0 * 16 + ln, lg, kr);
    for (int mt = 0; mt < a.mb; mt++) {
        const int64_t m0 = (tile0 + mt) * 16;
        if (m0 >= n) break;
        v8h kn[4];
        score_keys(a, m0 + 16 + ln, lg, kn);                      // past the wave's last tile: not used
        const int64_t ob = m0 + 4 * lg;                           // blocks ob .. ob + 3 of this lane's D rows
#pragma unroll
        for (int tile = 0; tile < SCORE_MAX_QT; tile++) {
            if (tile >= n_tiles) break;
            const int tl = tile * QT + (ln >> hb);
            const bool writer = h == 0 && tl < nt;
            float bias4[4] = {0.f, 0.f, 0.f, 0.f};
            if (a.bias) {
                const char * brow = (const char *) a.bias + (size_t) (t0 + (writer ? tl : 0)) * a.bias_nb1;
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (writer && ob + r < n) bias4[r] = *(const float *) (brow + (size_t) (ob + r) * 4);
            }
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; st++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[st], qb[tile][st], acc, 0, 0, 0);
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                v[r] = acc[r] > 0.f ? acc[r] : 0.f;               // relu per head
                if (hb >= 1) v[r] += dpp_f<0xB1>(v[r]);           // quad_perm 1,0,3,2
                if (hb >= 2) v[r] += dpp_f<0x4E>(v[r]);           // quad_perm 2,3,0,1
                if (hb >= 3) v[r] += dpp_f<0x141>(v[r]);          // row_half_mirror
                if (a.bias) v[r] += bias4[r];
            }
            // score rows are 64 floats apart in a 16-byte aligned workspace
            float * srow = a.score + (size_t) (t0 + (writer ? tl : 0)) * ld;
            if (writer && ob + 3 < n) {
                *(float4 *) (srow + ob) = make_float4(v[0], v[1], v[2], v[3]);
            } else if (writer) {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (ob + r < n) srow[ob + r] = v[r];
            }
        }
#pragma unroll
        for (int st = 0; st < 4; st++) kr[st] = kn[st];
    }
}

// Many queries (a prefill chunk): the same scores as k_qsa_score, tiled as a
// GEMM so that the pool and the queries are each read a few times instead of
// once per 8 queries. A workgroup holds QBW = 256 / 2^head_bits queries (64 at
// 4 heads), rounded to f16, in LDS ([query][head][128 dims], rows padded to 272
// bytes so that the 16 columns of an operand read hit distinct banks), and its
// 8 waves take mb tiles of 16 blocks each; per tile a wave keeps the keys in
// registers and runs the workgroup's 16-column tiles past them. The operand
// layout per lane and k-step is k_qsa_score's, so the scores are the same bits.
// The bias is left to the top-k.
constexpr int SQ_COLS = 256;                          // (query, head) columns of a workgroup
constexpr int SQ_ROWB = IDX_DIM * 2 + 16;             // 272: LDS bytes per column
constexpr int SQ_THREADS = 512;                       // 8 waves: two workgroups a CU hold 4 waves a SIMD

__global__ __launch_bounds__(SQ_THREADS) void k_qsa_score_tiled(score_args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sq_lds[];   // SQ_COLS * SQ_ROWB
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ln = lane & 15, lg = lane >> 4;
    const int64_t n = a.n_blocks;
    const int hb = a.head_bits, Hp = 1 << hb;
    const int QBW = SQ_COLS >> hb;                       // queries of the workgroup
    const int t0 = blockIdx.y * QBW;
    const int nt = a.T - t0 < QBW ? a.T - t0 : QBW;
    // ---- the workgroup's queries into LDS as f16: column c = query c >> hb,
    //      head c & (Hp - 1) (heads past n_heads and queries past T: zeros);
    //      thread i takes 8-dim pieces i, i + 256, ... ----
    // in two rounds of 8 pieces a thread, every load of a round issued before
    // any of its conversions and stores
    constexpr int SQ_PIECES = SQ_COLS * (IDX_DIM / 8) / SQ_THREADS;   // 8
    constexpr int SQ_ROUND = 8;
#pragma unroll
    for (int r0 = 0; r0 < SQ_PIECES; r0 += SQ_ROUND) {
        // unconditional loads (a piece past the queries or the heads reads
        // query 0, head 0 and is zeroed after): no branch holds a wait
        float4 x[SQ_ROUND], y[SQ_ROUND];
        bool ok[SQ_ROUND];
#pragma unroll
        for (int u = 0; u < SQ_ROUND; u++) {
            const int pc = (r0 + u) * SQ_THREADS + threadIdx.x;
            const int c = pc >> 4, d8 = (pc & 15) * 8;
            const int tl = c >> hb, hh = c & (Hp - 1);
            ok[u] = tl < nt && hh < a.n_heads;
            const float * qp = (const float *) ((const char *) a.q + (size_t) (t0 + (ok[u] ? tl : 0)) * a.q_nb2) +
                               (ok[u] ? hh : 0) * IDX_DIM + d8;
            x[u] = *(const float4 *) qp;
            y[u] = *(const float4 *) (qp + 4);
        }
#pragma unroll
        for (int u = 0; u < SQ_ROUND; u++) {
            const int pc = (r0 + u) * SQ_THREADS + threadIdx.x;
            const int c = pc >> 4, d8 = (pc & 15) * 8;
            const float4 xx = ok[u] ? x[u] : make_float4(0.f, 0.f, 0.f, 0.f), yy = ok[u] ? y[u] : make_float4(0.f, 0.f, 0.f, 0.f);
            const v8h hv = v8h{(_Float16) xx.x, (_Float16) xx.y, (_Float16) xx.z, (_Float16) xx.w,
                               (_Float16) yy.x, (_Float16) yy.y, (_Float16) yy.z, (_Float16) yy.w};   // round to nearest even
            *(v8h *) (sq_lds + c * SQ_ROWB + d8 * 2) = hv;
        }
    }
    static_assert(SQ_PIECES % SQ_ROUND == 0, "whole rounds");
    __syncthreads();
    const int QT = 16 >> hb;                              // queries per 16-column tile
    const int n_ct = (nt * Hp + 15) / 16;                 // the workgroup's column tiles holding a query
    const int h = ln & (Hp - 1);
    const int64_t ld = score_ld(n);
    const int64_t tile0 = ((int64_t) blockIdx.x * (SQ_THREADS / 64) + wave) * a.mb;
    v8h kr[4];
    score_keys(a, tile0 * 16 + ln, lg, kr);
    for (int mt = 0; mt < a.mb; mt++) {
        const int64_t m0 = (tile0 + mt) * 16;
        if (m0 >= n) break;
        v8h kn[4];
        score_keys(a, m0 + 16 + ln, lg, kn);              // the next tile's keys (past the wave's last: unused)
        const int64_t ob = m0 + 4 * lg;
        // 4 column tiles at a time: their 16 MFMAs interleave (each accumulator
        // still takes the k-steps 0..3 in order: the same bits)
        for (int ct0 = 0; ct0 < n_ct; ct0 += 4) {
            v4f acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int st = 0; st < 4; st++) {
                v8h bq[4];
#pragma unroll
                for (int c = 0; c < 4; c++)   // columns past n_ct read other LDS columns: unused
                    bq[c] = *(const v8h *) (sq_lds + ((ct0 + c) * 16 + ln) * SQ_ROWB + 16 * lg + 64 * st);
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[st], bq[c], acc[c], 0, 0, 0);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int ct = ct0 + c;
                if (ct >= n_ct) break;
                const int tl = ct * QT + (ln >> hb);      // query of this lane's column
                const bool writer = h == 0 && tl < nt;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    v[r] = acc[c][r] > 0.f ? acc[c][r] : 0.f;   // relu per head
                    if (hb >= 1) v[r] += dpp_f<0xB1>(v[r]);     // quad_perm 1,0,3,2
                    if (hb >= 2) v[r] += dpp_f<0x4E>(v[r]);     // quad_perm 2,3,0,1
                    if (hb >= 3) v[r] += dpp_f<0x141>(v[r]);    // row_half_mirror
                }
                float * srow = a.score + (size_t) (t0 + (writer ? tl : 0)) * ld;
                if (writer && ob + 3 < n) {
                    *(float4 *) (srow + ob) = make_float4(v[0], v[1], v[2], v[3]);
                } else if (writer) {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (ob + r < n) srow[ob + r] = v[r];
                }
            }
        }
#pragma unroll
        for (int st = 0; st < 4; st++) kr[st] = kn[st];
    }
}

struct topk_args {
    const float *   score;        // [T][score_ld(n_blocks)]: the sums over heads
    const float *   bias;         // null: the scores are complete; else F32 [n_blocks] per query
    size_t          bias_nb1;     // (query stride bias_nb1 bytes), added as the scores load
    int32_t         bias_vec;     // bias and bias_nb1 16-byte aligned
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

// exclusive prefix over the workgroup of (x, y), in thread order
__device__ __forceinline__ void block_scan2(uint32_t x, uint32_t y, uint32_t & ex, uint32_t & ey, uint2 * wsum) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t ix = wave_incl_scan(x), iy = wave_incl_scan(y);
    if (lane == 63) wsum[w] = make_uint2(ix, iy);
    __syncthreads();
    uint32_t bx = 0, by = 0;
#pragma unroll
    for (int w2 = 0; w2 < TOPK_THREADS / 64; w2++) {
        const uint2 t = wsum[w2];
        if (w2 < w) { bx += t.x; by += t.y; }
    }
    ex = bx + ix - x;
    ey = by + iy - y;
}

constexpr int CAND_MAX = 2 * TOPK_THREADS;   // LDS words of the candidates (the sort's two buffers)

struct topk_lds {
    uint32_t sub_hist[(1 << RADIX_BITS) * SUBH_LD];
    uint64_t sel[TOPK_MAX];
    uint64_t cand[CAND_MAX];
    uint2    wsum[TOPK_THREADS / 64];
    uint32_t hist[1 << RADIX_BITS];
    int32_t  order[TOPK_MAX];
    uint32_t s_digit, s_need, s_done, n_cand;
};

// Radix select over the keys key[j] (j < nv) of every thread, most significant
// 8-bit digit first, for the need-th largest, down to the digit at bit
// last_shift at most. Each pass counts digits into 32 sub-histograms, one per
// lane mod 32, whose rows are SUBH_LD words apart: lanes with the same digit
// hit distinct banks, so clustered digits (the exponent byte of similar
// scores) cost no serialised atomics. A pass whose boundary bin is kept whole
// ends the select early (done). Out: the digits found (prefix, the bits below
// them zero) and the need left within the boundary bin. sub_hist is all
// zeros at entry and at exit.
template <int KK>
__device__ __forceinline__ void radix_passes(const uint32_t (&key)[KK], int nv, uint32_t need, int last_shift, topk_lds & L,
                                             uint32_t & prefix_out, uint32_t & need_out, bool & done_out) {
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t prefix = 0, mask = 0;
    bool done = false;
#pragma unroll 1
    for (int shift = 32 - RADIX_BITS; shift >= last_shift; shift -= RADIX_BITS) {
        uint32_t * mine = L.sub_hist + (lane & 31);
#pragma unroll
        for (int j = 0; j < KK; j++)
            if (j < nv && (key[j] & mask) == prefix)
                atomicAdd(&mine[((key[j] >> shift) & ((1u << RADIX_BITS) - 1)) * SUBH_LD], 1u);
        __syncthreads();
        {
            // 4 threads per bin sum its 32 counts and clear them for the next pass
            const int bin = tid >> 2, qq = tid & 3;
            uint4 * p = (uint4 *) (L.sub_hist + bin * SUBH_LD + qq * 8);
            const uint4 x = p[0], y = p[1];
            p[0] = make_uint4(0u, 0u, 0u, 0u);
            p[1] = make_uint4(0u, 0u, 0u, 0u);
            uint32_t c = x.x + x.y + x.z + x.w + y.x + y.y + y.z + y.w;
            c += dpp_u<0xB1>(c);                          // quad_perm 1,0,3,2
            c += dpp_u<0x4E>(c);                          // quad_perm 2,3,0,1
            if (qq == 0) L.hist[bin] = c;
        }
        __syncthreads();
        if (tid < 64) {
            // lane l holds bins 255-4l down to 252-4l; s = keys in bins >= 252-4l
            const int top = 255 - 4 * lane;
            const uint32_t c3 = L.hist[top], c2 = L.hist[top - 1], c1 = L.hist[top - 2], c0 = L.hist[top - 3];
            const uint32_t tot = c0 + c1 + c2 + c3;
            const uint32_t sc = wave_incl_scan(tot);
            const uint32_t above = sc - tot;          // keys in bins above this lane's
            if (above < need && need <= sc) {         // the one lane whose bins hold the need-th key
                uint32_t acc = above, d, cd;
                if (acc + c3 >= need) { d = 3; cd = c3; }
                else {
                    acc += c3;
                    if (acc + c2 >= need) { d = 2; cd = c2; }
                    else {
                        acc += c2;
                        if (acc + c1 >= need) { d = 1; cd = c1; }
                        else { acc += c1; d = 0; cd = c0; }
                    }
                }
                L.s_digit = (uint32_t) (top - 3) + d;
                L.s_need = need - acc;
                L.s_done = (need - acc == cd) ? 1u : 0u;   // the whole bin is kept
            }
        }
        __syncthreads();
        prefix |= L.s_digit << shift;
        need = L.s_need;
        mask |= ((1u << RADIX_BITS) - 1) << shift;
        done = L.s_done != 0;
        if (done) break;   // (the next pass writes the result words only after two more barriers)
    }
    prefix_out = prefix;
    need_out = need;
    done_out = done;
}

// The k-th largest key `kth` and how many keys equal to it are kept (`keep`)
// from a full radix select: a select that ended on a bin kept whole keeps
// every key >= prefix (the bin's keys have prefix's top bits and any low
// bits): the keys above prefix - 1, and none equal to it; valid keys are
// never 0, so prefix 0 keeps them all.
__device__ __forceinline__ void kth_keep(uint32_t prefix, uint32_t need, bool done, uint32_t & kth, uint32_t & keep) {
    if (done) { kth = prefix ? prefix - 1 : 0u; keep = 0; }
    else      { kth = prefix; keep = need; }
}

// Keys above kth, then the kept equal keys (the lowest blocks), into
// sel[0, k), packed with their block as (key << 32 | ~block), so that the
// larger packed value comes first (ties: the lower block). Key j of thread
// tid is block blk(j), and blocks rise in the order (j / 4, tid, j % 4) (the
// top-k's interleaved layout). The keys above kth go in thread order (one
// exclusive scan: their order is the sort's business); the equal ones one
// group of 4 keys at a time, a scan per group, so that the first `keep` of
// them in block order are the ones kept.
template <int KK, typename Blk>
__device__ __forceinline__ void place(const uint32_t (&key)[KK], Blk blk, int nv, uint32_t kth, uint32_t keep, int k,
                                      topk_lds & L) {
    static_assert(KK % 4 == 0, "groups of 4 keys");
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    // exclusive prefix of x over the workgroup in thread order, and the total
    auto scan_total = [&](uint32_t x, uint32_t & ex) -> uint32_t {
        const uint32_t ix = wave_incl_scan(x);
        __syncthreads();                                 // the previous scan's readers are done with wsum
        if (lane == 63) L.wsum[w].x = ix;
        __syncthreads();
        uint32_t bx = 0, tot = 0;
#pragma unroll
        for (int w2 = 0; w2 < TOPK_THREADS / 64; w2++) {
            const uint32_t t = L.wsum[w2].x;
            if (w2 < w) bx += t;
            tot += t;
        }
        ex = bx + ix - x;
        return tot;
    };
    uint32_t na = 0;
#pragma unroll
    for (int j = 0; j < KK; j++) na += (j < nv && key[j] > kth) ? 1u : 0u;
    uint32_t pa;
    scan_total(na, pa);
    const uint32_t first_equal = (uint32_t) k - keep;        // the keys above take the slots before
#pragma unroll
    for (int j = 0; j < KK; j++)
        if (j < nv && key[j] > kth) {
            if (pa < first_equal) L.sel[pa] = ((uint64_t) key[j] << 32) | (uint32_t) ~blk(j);
            pa++;
        }
    uint32_t placed = 0;                                     // equal keys of the groups before (uniform)
#pragma unroll
    for (int g = 0; g < KK / 4; g++) {
        if (placed >= keep) break;
        uint32_t ne = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) ne += (4 * g + e < nv && key[4 * g + e] == kth) ? 1u : 0u;
        uint32_t pe;
        const uint32_t tot = scan_total(ne, pe);
        pe += placed;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int j = 4 * g + e;
            if (j < nv && key[j] == kth) {
                if (pe < keep && first_equal + pe < (uint32_t) k) L.sel[first_equal + pe] = ((uint64_t) key[j] << 32) | (uint32_t) ~blk(j);
                pe++;
            }
        }
        placed += tot;
    }
}

// One compare-exchange step of a bitonic sort with the element of lane ^ D
// (D < 64, in the wave): every lane gets max or min of the pair. The pair
// comes back as {a, b} = {own, partner} in either order (the permlane swaps
// return it so); the larger is taken iff take_max.
template <int D>
__device__ __forceinline__ uint64_t bitonic_lane_step(uint64_t v, bool take_max) {
    const uint32_t lo = (uint32_t) v, hi = (uint32_t) (v >> 32);
    uint32_t alo = lo, ahi = hi, blo, bhi;
    if constexpr (D == 1 || D == 2 || D == 8) {
        constexpr int CTRL = D == 1 ? 0xB1 : D == 2 ? 0x4E : 0x128;   // quad_perm [1,0,3,2], [2,3,0,1], row_ror:8
        blo = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) lo, CTRL, 0xF, 0xF, false);
        bhi = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) hi, CTRL, 0xF, 0xF, false);
    } else if constexpr (D == 16 || D == 32) {
        const auto rl = D == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                                : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto rh = D == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                                : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        alo = rl[0]; blo = rl[1]; ahi = rh[0]; bhi = rh[1];
    } else {
        static_assert(D == 4, "lane strides 1 to 32");
        // lane ^ 4 within a row of 16: row_ror:12 brings lane + 4 (lanes with
        // bit 2 clear), row_ror:4 lane - 4 (bit 2 set)
        const bool up = (threadIdx.x & 4) != 0;
        const uint32_t l4 = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) lo, 0x124, 0xF, 0xF, false);
        const uint32_t l12 = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) lo, 0x12C, 0xF, 0xF, false);
        const uint32_t h4 = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) hi, 0x124, 0xF, 0xF, false);
        const uint32_t h12 = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) hi, 0x12C, 0xF, 0xF, false);
        blo = up ? l4 : l12;
        bhi = up ? h4 : h12;
    }
    const uint64_t a = ((uint64_t) ahi << 32) | alo, b = ((uint64_t) bhi << 32) | blo;
    return (take_max == (a > b)) ? a : b;
}

// Bitonic sort, largest first, of the TOPK_THREADS values v (one a thread,
// element tid): strides below 64 exchange within the wave, larger ones
// through the two LDS buffers buf[0 .. 2 * TOPK_THREADS), one barrier a step.
// Returns the element of rank tid.
__device__ __forceinline__ uint64_t bitonic_sort_block(uint64_t v, uint64_t * buf) {
    const int tid = threadIdx.x;
    int cur = 0;
#pragma unroll
    for (int size = 2; size <= TOPK_THREADS; size <<= 1) {
        const bool up = (tid & size) == 0;   // this run of `size` is sorted largest first
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const bool take_max = up == ((tid & stride) == 0);
            if (stride >= 64) {
                buf[cur * TOPK_THREADS + tid] = v;
                __syncthreads();
                const uint64_t o = buf[cur * TOPK_THREADS + (tid ^ stride)];
                v = (take_max == (v > o)) ? v : o;
                cur ^= 1;
            } else if (stride == 32) v = bitonic_lane_step<32>(v, take_max);
            else if (stride == 16)   v = bitonic_lane_step<16>(v, take_max);
            else if (stride == 8)    v = bitonic_lane_step<8>(v, take_max);
            else if (stride == 4)    v = bitonic_lane_step<4>(v, take_max);
            else if (stride == 2)    v = bitonic_lane_step<2>(v, take_max);
            else                     v = bitonic_lane_step<1>(v, take_max);
        }
    }
    return v;
}

// One workgroup per query. Thread i holds scores [i * KPT, i * KPT + KPT) as
// order-preserving keys in registers, packed with their block as
// (key << 32 | ~block): the larger packed value comes first, ties to the
// lower block, and no two are equal. Fast path: a threshold tau such that
// between k and TOPK_THREADS keys are >= tau -- every key when there are at
// most TOPK_THREADS, else the 16-bit digits of the sample key (two a thread)
// ranked to leave about (k + TOPK_THREADS) / 2 keys in expectation -- the
// keys >= tau gathered into LDS (in any order), one bitonic sort of them, and
// thread i holds rank i. Otherwise (the sample missed, k above 3/4 of
// TOPK_THREADS, or more than 32 keys a thread): a radix select over every key
// finds the k-th largest, the keys above it and the lowest-block equal ones
// are placed by a scan, and those k are sorted in runs of 64 per wave, then
// merged by rank.
template <int KPT>
__global__ __launch_bounds__(TOPK_THREADS, KPT <= 16 ? 8 : 1) void k_qsa_topk(topk_args a) {
    __shared__ __align__(16) topk_lds L;
    const int tid = threadIdx.x, lane = tid & 63;
    const int64_t n = a.n_blocks;
    const int k = a.k;
    // key j of this thread is block kidx(j) = 4 tid + 4096 (j / 4) + j % 4: a
    // wave's float4 loads cover 1 KB runs, and a thread's valid keys are a
    // prefix of its j (the blocks rise with j)
    auto kidx = [&](int j) -> int64_t { return 4 * (int64_t) tid + 4 * TOPK_THREADS * (int64_t) (j >> 2) + (j & 3); };
    const float * sc = a.score + (size_t) blockIdx.x * score_ld(n);
    const float * br = a.bias ? (const float *) ((const char *) a.bias + (size_t) blockIdx.x * a.bias_nb1) : nullptr;

    for (int i = tid; i < (1 << RADIX_BITS) * SUBH_LD / 4; i += TOPK_THREADS)
        ((uint4 *) L.sub_hist)[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) L.n_cand = 0;
    uint32_t key[KPT];
#pragma unroll
    for (int j = 0; j < KPT; j += 4) {
        const int64_t b0 = kidx(j);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f), bv = v;
        if (b0 < n) v = *(const float4 *) (sc + b0);             // score_ld keeps the float4 inside the row
        if (br) {
            if (a.bias_vec && b0 + 3 < n) {
                bv = *(const float4 *) (br + b0);
            } else {
                if (b0 < n) bv.x = br[b0];
                if (b0 + 1 < n) bv.y = br[b0 + 1];
                if (b0 + 2 < n) bv.z = br[b0 + 2];
                if (b0 + 3 < n) bv.w = br[b0 + 3];
            }
            // score = the sum over heads + the bias, one f32 addition
            v.x += bv.x; v.y += bv.y; v.z += bv.z; v.w += bv.w;
        }
        key[j] = okey(v.x); key[j + 1] = okey(v.y); key[j + 2] = okey(v.z); key[j + 3] = okey(v.w);
    }
    int nv = 0;                                                 // valid keys of this thread: j < nv
#pragma unroll
    for (int j = 0; j < KPT; j += 4) {
        const int64_t r = n - kidx(j);
        nv += r <= 0 ? 0 : (r < 4 ? (int) r : 4);
    }
    __syncthreads();

    bool sorted_all = false;
    uint64_t mine = 0;                                          // fast path: the element of rank tid
    if (KPT <= 32 && (n <= TOPK_THREADS || 4 * k <= 3 * TOPK_THREADS)) {   // (barriers: the conditions are uniform)
        uint32_t tau = 0;                                       // valid keys are never 0: all of them
        if (n > TOPK_THREADS) {
            // the sample: keys j1 = tid % KPT and j2 = (tid + KPT / 2) % KPT of
            // each thread, so that it spreads over every part of the pool
            const int nn = (int) n;                             // at most 32 * 1024 here
            const int j1 = tid % KPT, j2 = (tid + KPT / 2) % KPT;
            uint32_t k1 = key[0], k2 = key[0];
#pragma unroll
            for (int j = 1; j < KPT; j++) {
                k1 = j == j1 ? key[j] : k1;
                k2 = j == j2 ? key[j] : k2;
            }
            const bool v1 = j1 < nv, v2 = j2 < nv;
            // the valid sample keys, counted with a ballot per wave
            const uint32_t c1 = (uint32_t) __popcll(__ballot(v1)), c2 = (uint32_t) __popcll(__ballot(v2));
            if (lane == 0) L.wsum[tid >> 6] = make_uint2(c1, c2);
            __syncthreads();
            int m = 0;
#pragma unroll
            for (int w2 = 0; w2 < TOPK_THREADS / 64; w2++) m += (int) (L.wsum[w2].x + L.wsum[w2].y);
            __syncthreads();                                    // wsum is free again
            // the sample rank, in float (an estimate serves: any tau with between
            // k and TOPK_THREADS keys at or above it gives the exact answer)
            const float want = 0.5f * (float) (k + TOPK_THREADS);
            uint32_t S = (uint32_t) ceilf(want * (float) m / (float) nn);
            S = S < 1 ? 1u : (S > (uint32_t) m ? (uint32_t) m : S);
            const uint32_t sk[2] = {v1 ? k1 : k2, v1 ? k2 : k1};   // the valid ones first
            uint32_t nd;
            bool dn;
            radix_passes<2>(sk, (v1 ? 1 : 0) + (v2 ? 1 : 0), S, 16, L, tau, nd, dn);
        }
        // the keys >= tau into L.cand, each wave's at an offset it takes with one atomic
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < KPT; j++) c += (j < nv && key[j] >= tau) ? 1u : 0u;
        const uint32_t incl = wave_incl_scan(c);
        uint32_t wbase = 0;
        if (lane == 63) wbase = atomicAdd(&L.n_cand, incl);
        wbase = (uint32_t) __builtin_amdgcn_readlane((int) wbase, 63);
        uint32_t pos = wbase + incl - c;
#pragma unroll
        for (int j = 0; j < KPT; j++)
            if (j < nv && key[j] >= tau) {
                if (pos < (uint32_t) TOPK_THREADS) L.cand[pos] = ((uint64_t) key[j] << 32) | (uint32_t) ~(uint32_t) kidx(j);
                pos++;
            }
        __syncthreads();
        const uint32_t total = L.n_cand;
        if (total >= (uint32_t) k && total <= (uint32_t) TOPK_THREADS) {
            sorted_all = true;
            uint64_t v = (uint32_t) tid < total ? L.cand[tid] : 0ull;   // 0: below every packed key
            __syncthreads();                                    // L.cand becomes the sort's buffers
            mine = bitonic_sort_block(v, L.cand);
        }
    }
    if (sorted_all) {
        if (tid < k) {
            const int32_t ix = (int32_t) ~(uint32_t) mine;
            const size_t o = (size_t) blockIdx.x * k + tid;
            const bool ok = ix >= 0 && ix < n;
            int32_t cv[RATIO_MAX];
#pragma unroll
            for (int m = 0; m < RATIO_MAX; m++) cv[m] = (ok && m < a.ratio) ? a.blk_cells[(size_t) ix * a.ratio + m] : -1;
            if (a.top) a.top[o] = ok ? ix : -1;
#pragma unroll
            for (int m = 0; m < RATIO_MAX; m++)
                if (m < a.ratio) a.cells[o * a.ratio + m] = cv[m];
        }
        return;
    }
    {
        uint32_t pfx, need, kth, keep;
        bool done;
        radix_passes<KPT>(key, nv, (uint32_t) k, 0, L, pfx, need, done);
        kth_keep(pfx, need, done, kth, keep);
        place<KPT>(key, [&](int j) { return (uint32_t) kidx(j); }, nv, kth, keep, k, L);
    }
    // order: every wave sorts a run of 64 values in registers (bitonic over
    // lane swaps, best first); then each value's place is its index in its
    // run plus, for every other run, the number of values above it there
    // (a binary search). Padding (0) sorts last and is never placed.
    const int kpad = (k + 63) & ~63;
    const int n_runs = kpad >> 6;
    for (int j = k + tid; j < kpad; j += TOPK_THREADS) L.sel[j] = 0;
    __syncthreads();
    const int wv = tid >> 6;
    if (wv < n_runs) {                                            // wave-uniform
        uint64_t x = L.sel[tid];
#pragma unroll
        for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
            for (int d = size >> 1; d > 0; d >>= 1) {
                const uint32_t ylo = (uint32_t) __shfl_xor((int) (uint32_t) x, d);
                const uint32_t yhi = (uint32_t) __shfl_xor((int) (uint32_t) (x >> 32), d);
                const uint64_t y = ((uint64_t) yhi << 32) | ylo;
                const bool take_max = ((lane & d) == 0) == ((lane & size) == 0);
                x = take_max ? (x > y ? x : y) : (x < y ? x : y);
            }
        }
        L.sel[tid] = x;
    }
    __syncthreads();
    if (wv < n_runs) {
        const uint64_t v = L.sel[tid];
        uint32_t rank = (uint32_t) lane;
        for (int r = 0; r < n_runs; r++) {
            if (r == wv) continue;
            const uint64_t * run = L.sel + 64 * r;
            int pos = 0;
#pragma unroll
            for (int step = 32; step >= 1; step >>= 1)
                if (run[pos + step - 1] > v) pos += step;
            pos += run[pos] > v ? 1 : 0;                          // pos <= 63 here: all 64 above
            rank += (uint32_t) pos;
        }
        if (v != 0 && rank < (uint32_t) k) L.order[rank] = (int32_t) ~(uint32_t) v;
    }
    __syncthreads();
    if (tid < k) {
        const int32_t ix = L.order[tid];
        const size_t o = (size_t) blockIdx.x * k + tid;
        const bool ok = ix >= 0 && ix < n;                      // always, for distinct ranks; never read outside blk_cells
        // all of the block's cells are loaded before any is stored (cells may alias blk_cells)
        int32_t c[RATIO_MAX];
#pragma unroll
        for (int m = 0; m < RATIO_MAX; m++) c[m] = (ok && m < a.ratio) ? a.blk_cells[(size_t) ix * a.ratio + m] : -1;
        if (a.top) a.top[o] = ok ? ix : -1;
#pragma unroll
        for (int m = 0; m < RATIO_MAX; m++)
            if (m < a.ratio) a.cells[o * a.ratio + m] = c[m];
    }
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" size_t qwfn_qsa_select_workspace_size(int64_t n_blocks, int32_t T) {
    return ::qwfn::abi_value<size_t>("qsa_select_workspace_size", 0, [&]() -> size_t {
        return (size_t) score_ld(std::max<int64_t>(1, n_blocks)) * (size_t) std::max(1, T) * sizeof(float);
    });
}

extern "C" int qwfn_qsa_select_cells(const uint16_t * pool, size_t pool_nb1, int64_t n_blocks, const float * q,
                                     int32_t n_heads, size_t q_nb2, const float * bias, size_t bias_nb1, int32_t T,
                                     int32_t k_blocks, const int32_t * blk_cells, int32_t ratio, int32_t * cells,
                                     int32_t * top, void * ws, size_t ws_bytes, void * stream) {
    return ::qwfn::abi_call("qsa_select_cells", [&]() -> int {
        if (!pool || !q || !bias || !blk_cells || !cells) return set_error(QWFN_EINVAL, "qsa_select_cells: NULL pointer");
        if (n_blocks < 1 || T < 1 || ratio < 1) return set_error(QWFN_EINVAL, "qsa_select_cells: empty input");
        if (ratio > RATIO_MAX) return set_error(QWFN_ENOTSUP, "qsa_select_cells: at most 16 cells per block");
        if (n_heads < 1 || n_heads > MAX_IDX_HEADS) return set_error(QWFN_ENOTSUP, "qsa_select_cells: 1 to 8 indexer heads");
        if (k_blocks < 1 || k_blocks > n_blocks || k_blocks > TOPK_MAX)
            return set_error(QWFN_EINVAL, "qsa_select_cells: need 1 <= k_blocks <= min(n_blocks, 1024)");
        if (pool_nb1 < IDX_DIM * 2 || pool_nb1 % 16 || !is_aligned(pool, 16))
            return set_error(QWFN_EALIGN, "qsa_select_cells: pooled keys must be 128 f16 at a 16-byte aligned stride");
        if (q_nb2 < (size_t) n_heads * IDX_DIM * 4 || !is_aligned(q, 16) || q_nb2 % 16 || bias_nb1 % 4 || !is_aligned(bias, 4))
            return set_error(QWFN_EALIGN, "qsa_select_cells: q [128, n_heads] f32 per query, f32 bias");
        if (!ws || ws_bytes < qwfn_qsa_select_workspace_size(n_blocks, T))
            return set_error(QWFN_ENOMEM, "qsa_select_cells: workspace too small");
        if (!is_aligned(ws, 16)) return set_error(QWFN_EALIGN, "qsa_select_cells: workspace must be 16-byte aligned");
        if (n_blocks > (int64_t) TOPK_THREADS * TOPK_MAX_KPT)
            return set_error(QWFN_ENOTSUP, "qsa_select_cells: at most 49152 blocks");
        if (n_blocks * ratio > INT32_MAX) return set_error(QWFN_ERANGE, "qsa_select_cells: too many cells");
        hipStream_t st = as_stream(stream);
        int head_bits = 0;
        while ((1 << head_bits) < n_heads) head_bits++;
        // one pass over the pool (up to 8 queries): one 16-block tile a wave
        const int64_t n_tile = (n_blocks + 15) / 16, ny = (T + SCORE_T - 1) / SCORE_T;
        const int32_t mb = 1;
        // the bias: added by the score kernel for one pass over the pool (up to 8
        // queries: decode, verify), whose top-k then reads only scores it has just
        // written; by the top-k for more (a prefill chunk), which keeps the score
        // kernel's tile loop free of dependent loads (8 tiles a wave at 512
        // queries x 4224 blocks: 32.0 -> 24.0 us, the top-k 14.9 -> 16.3 us; at
        // 3 queries x 18432 blocks the top-k took 13.3 -> 15.4 us)
        const bool bias_in_score = ny == 1;
        score_args sa{pool, pool_nb1, n_blocks, q, q_nb2, n_heads, head_bits, T, bias_in_score ? bias : nullptr,
                      bias_nb1, (float *) ws, mb};
        if (bias_in_score) {
            const int64_t per = SCORE_THREADS / 64 * 16 * mb;        // blocks per workgroup: 16 mb per wave
            const unsigned gx = (unsigned) ((n_blocks + per - 1) / per);
            hipLaunchKernelGGL(k_qsa_score, dim3(gx, (unsigned) ny), dim3(SCORE_THREADS), 0, st, sa);
        } else {
            // more than 8 queries: the tiled kernel, 256 >> head_bits queries a
            // workgroup; tiles a wave so that the grid fits in one round of two
            // workgroups a CU (512): 520 workgroups at 16512 blocks x 512
            // queries took 44 us, the 8 past the round costing a whole wave
            // lifetime
            const int64_t nyq = (T + (SQ_COLS >> head_bits) - 1) / (SQ_COLS >> head_bits);
            sa.mb = (int32_t) std::max<int64_t>(1, std::min<int64_t>(64, (n_tile * nyq + 8 * 512 - 1) / (8 * 512)));
            const int64_t per = SQ_THREADS / 64 * 16 * (int64_t) sa.mb;
            const unsigned gx = (unsigned) ((n_blocks + per - 1) / per);
            hipLaunchKernelGGL(k_qsa_score_tiled, dim3(gx, (unsigned) nyq), dim3(SQ_THREADS), SQ_COLS * SQ_ROWB, st, sa);
        }
        if (int rc = hip_check(hipGetLastError(), "qsa score launch")) return rc;
        const int32_t bias_vec = is_aligned(bias, 16) && bias_nb1 % 16 == 0;
        topk_args ta{(const float *) ws, bias_in_score ? nullptr : bias, bias_nb1, bias_vec, n_blocks, k_blocks,
                     blk_cells, ratio, cells, top};
        const int64_t kpt = (n_blocks + TOPK_THREADS - 1) / TOPK_THREADS;
        // the smallest multiple of 4 that holds n_blocks / 1024 (18432 blocks: 20)
        auto topk = kpt <= 8 ? k_qsa_topk<8> : kpt <= 12 ? k_qsa_topk<12> : kpt <= 16 ? k_qsa_topk<16>
                  : kpt <= 20 ? k_qsa_topk<20> : kpt <= 24 ? k_qsa_topk<24> : kpt <= 32 ? k_qsa_topk<32>
                  : kpt <= 40 ? k_qsa_topk<40> : k_qsa_topk<48>;
        hipLaunchKernelGGL(topk, dim3((unsigned) T), dim3(TOPK_THREADS), 0, st, ta);
        return hip_check(hipGetLastError(), "qsa top-k launch");
    });
}
