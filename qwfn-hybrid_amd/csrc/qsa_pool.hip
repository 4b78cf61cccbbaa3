// The QSA index producer on the device: the decode step's raw indexer key into
// the F16 index cache and the pooled key of its block into the pool cache
// (graph_builder::qsa_dec_index, qwfn_graph.cpp:529-554), the rebuild of every
// whole block's pooled key after a prefill or restore (engine::qsa_pool_rebuild
// qwfn_engine.cpp:1107-1148 -> graph_builder::qsa_pool_rebuild,
// qwfn_graph.cpp:478-495), and ggml_set_rows of F32 rows into an F16 tensor.
//
// A pooled key (qsa_pool_blocks, qwfn_graph.cpp:282-301): the block's r member
// rows of the index cache (F16 -> F32) added in member order, times 1/r, RMS
// normed (squares summed in double), times the k_norm weight, roped at the
// block's first cell (all four sections), rounded to F16. One wave per block:
// the block's key sits in LDS; lane k < n_dims/2 rotates pair k.
#include "qsa_steps.h"
#include "qwfn_common.h"
#include "qwfn_state.h"
#include "rope_device.h"
#include "wave_ops.h"

#include <algorithm>
#include <cmath>

namespace qwfn {
namespace {

constexpr int POOL_MAX_DIM = 256;     // index key length, at most

// fp16 <-> fp32 (IEEE; the f32 -> f16 conversion rounds to nearest even)
__device__ __forceinline__ uint16_t f2h(float x) { return __builtin_bit_cast(uint16_t, (_Float16) x); }
__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
constexpr int POOL_WAVES = 4;         // blocks per workgroup

struct pool_args {
    uint16_t *       ic;          // F16 [ic_rows][dim]
    int64_t          ic_rows;
    uint16_t *       pool;        // F16 [pool_rows][dim]
    int64_t          pool_rows;
    int32_t          dim;
    int32_t          r;
    float            inv_r;       // 1.0f / r (host float division, as ggml_scale's argument)
    float            eps;
    const float *    w;           // k_norm weight F32 [dim]
    rope_params      rp;
    int64_t          n_blk;       // rebuild: blocks 0 .. n_blk-1
    // decode: one block from the per-token inputs (device)
    const float *    k_raw;       // F32 [dim] or null
    const int32_t *  write_idx;
    const int32_t *  member_idx;  // [r]
    const int32_t *  blk_pos;     // [4]
    const int32_t *  blk_idx;
    uint32_t *       status;
};

// What the pooled block's tail needs besides the member mean, which a caller
// may fetch while the members load: the norm weights (lane + 64 i) and the
// cos / sin of rope pair `lane` at positions pos[0..3] (lanes past the pairs:
// pair 0's, unused).
struct pool_tail_in {
    float wr[POOL_MAX_DIM / 64];
    float c, s;
};
__device__ __forceinline__ void pool_prefetch(const pool_args & a, int lane, const int32_t (&pos)[4], pool_tail_in & in) {
#pragma unroll
    for (int i = 0; i < POOL_MAX_DIM / 64; i++) in.wr[i] = lane + 64 * i < a.dim ? a.w[lane + 64 * i] : 0.f;
    rope_cos_sin(a.rp, pos, lane < a.rp.n_dims / 2 ? lane : 0, &in.c, &in.s);
}

// The pooled block's tail, for the mean x[0 .. dim) of its member rows (one
// wave): RMS norm (the squares in float, summed in double across the wave),
// times the weight, IMROPE, F16 into pool row orow.
__device__ __forceinline__ void pool_finish_with(const pool_args & a, float * x, int lane, int64_t orow,
                                                 const pool_tail_in & in) {
    const int dim = a.dim;
    double sq = 0.0;
    for (int d = lane; d < dim; d += 64) sq += (double) __fmul_rn(x[d], x[d]);
    sq = wave::wave_sum_d(sq);
    const float mean = (float) (sq / (double) dim);
    const float scale = 1.0f / sqrtf(__fadd_rn(mean, a.eps));
#pragma unroll
    for (int i = 0; i < POOL_MAX_DIM / 64; i++) {
        const int d = lane + 64 * i;
        if (d < dim) x[d] = __fmul_rn(__fmul_rn(x[d], scale), in.wr[i]);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const bool ook = orow >= 0 && orow < a.pool_rows;
    if (!ook) {
        if (lane == 0) atomicOr(a.status, DEVERR_SET_ROWS_INDEX);
        return;
    }
    uint16_t * out = a.pool + (size_t) orow * dim;
    const int half = a.rp.n_dims / 2;
    if (lane < half) {
        float y0, y1;
        rope_rotate(x[lane], x[lane + half], in.c, in.s, &y0, &y1);
        out[lane] = f2h(y0);
        out[lane + half] = f2h(y1);
    }
    for (int d = a.rp.n_dims + lane; d < dim; d += 64) out[d] = f2h(x[d]);
}

__device__ __forceinline__ void pool_finish(const pool_args & a, float * x, int lane, const int32_t (&pos)[4], int64_t orow) {
    pool_tail_in in;
    pool_prefetch(a, lane, pos, in);
    pool_finish_with(a, x, lane, orow, in);
}

template <bool DECODE>
__global__ __launch_bounds__(POOL_WAVES * 64) void k_qsa_pool(pool_args a) {
    __shared__ float xs[POOL_WAVES][POOL_MAX_DIM];
    __shared__ uint16_t key16[POOL_WAVES][POOL_MAX_DIM];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t blk = (int64_t) blockIdx.x * POOL_WAVES + wv;
    if (!DECODE && blk >= a.n_blk) return;
    if (DECODE && blk > 0) return;
    float * x = xs[wv];
    const int dim = a.dim;

    int32_t wrow = -1;
    if constexpr (DECODE) {
        // the raw key into the index cache at write_idx (F32 -> F16, RNE); the
        // pooling below takes it from registers, not from memory
        wrow = *a.write_idx;
        const bool wok = wrow >= 0 && wrow < a.ic_rows;
        if (a.k_raw) {
            for (int d = lane; d < dim; d += 64) {
                const uint16_t h = f2h(a.k_raw[d]);
                key16[wv][d] = h;
                if (wok) a.ic[(size_t) wrow * dim + d] = h;
            }
            if (!wok && lane == 0) atomicOr(a.status, DEVERR_SET_ROWS_INDEX);
        } else {
            wrow = -1;
        }
    }
    // mean of the member rows, in member order
    for (int d = lane; d < dim; d += 64) {
        float acc = 0.f;
        for (int m = 0; m < a.r; m++) {
            const int64_t row = DECODE ? (int64_t) a.member_idx[m] : blk * a.r + m;
            float v;
            if (DECODE && row == wrow) {
                v = h2f(key16[wv][d]);
            } else if (row >= 0 && row < a.ic_rows) {
                v = h2f(a.ic[(size_t) row * dim + d]);
            } else {
                v = 0.f;
                if (d == lane && lane == 0) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
            }
            acc = m == 0 ? v : __fadd_rn(acc, v);
        }
        x[d] = __fmul_rn(acc, a.inv_r);
    }
    int32_t pos[4];
    int64_t orow;
    if constexpr (DECODE) {
        for (int s = 0; s < 4; s++) pos[s] = a.blk_pos[s];
        orow = *a.blk_idx;
    } else {
        for (int s = 0; s < 4; s++) pos[s] = (int32_t) (blk * a.r);
        orow = blk;
    }
    pool_finish(a, x, lane, pos, orow);
}

// qsa_dec_index for the T positions of a step, one wave each (wave w of
// workgroup g: position 4 g + w): the same caches as T k_qsa_pool<true>
// calls in position order. Every position writes its raw key; only the last
// position of each block pools it, since an earlier position's pooled row
// would be overwritten by the later one's. A member row that a position of
// this call at or before the pooling one writes is taken from that
// position's key (rounded to F16, as written), never from memory; a block's
// members never include a later position (they are cells of the block up to
// its position).
constexpr int POOL_MAX_T = 16;
struct pool_steps_args {
    pool_args       p;                        // caches, geometry, norm and rope constants, status
    const float *   k_raw;                    // F32 [T][dim], rows k_ld floats apart, or null (no keys)
    int64_t         k_ld;
    const int32_t * write_idx[POOL_MAX_T];
    const int32_t * member_idx[POOL_MAX_T];
    const int32_t * blk_pos[POOL_MAX_T];
    const int32_t * blk_idx[POOL_MAX_T];
    int32_t         T;
};

// One position's wave of the step's pooling (position t, lane `lane`, x its
// LDS row of dim floats). The indices come from the device inputs that the
// preparation wrote (CLOSED false) or from their closed forms of n_past
// (CLOSED true, qsa_steps.h: position p = n_past + t writes row p into block
// p / r, whose members are the rows (p / r) r + m and whose rope positions
// are (p / r) r), the same values without the round trips that read them.
template <int NI, bool CLOSED>      // dim <= 64 * NI
__device__ __forceinline__ void pool_step_wave(const pool_steps_args & s, int32_t n_past, float * x, int t, int lane) {
    const pool_args & a = s.p;
    const int dim = a.dim;
    // every position's write row and block (lane u holds position u's), this
    // position's members (lane m holds member m's row) and block positions,
    // all before the write so that their loads overlap it
    int32_t wi = -1, bi = -1;
    int32_t my_row = -1;
    int32_t pos[4];
    const int32_t * mem = nullptr;
    int64_t mem0 = 0;                   // CLOSED: member m is row mem0 + m
    if constexpr (CLOSED) {
        if (lane < s.T) {
            wi = s.k_raw ? n_past + lane : -1;
            bi = (int32_t) (((int64_t) n_past + lane) / a.r);
        }
        mem0 = (((int64_t) n_past + t) / a.r) * a.r;
        my_row = lane < a.r ? (int32_t) (mem0 + lane) : -1;
        for (int q = 0; q < 4; q++) pos[q] = (int32_t) mem0;
    } else {
        // both pointers, then both values: two round trips
        if (lane < s.T) {
            const int32_t * pb = s.blk_idx[lane];
            const int32_t * pw = s.k_raw ? s.write_idx[lane] : pb;
            const int32_t w = *pw;
            bi = *pb;
            wi = s.k_raw ? w : -1;
        }
        mem = s.member_idx[t];
        my_row = lane < a.r ? mem[lane & 63] : -1;
        for (int q = 0; q < 4; q++) pos[q] = s.blk_pos[t][q];
    }
    const int32_t wrow = __shfl(wi, t), blk = __shfl(bi, t);
    // src >= 0 only with k_raw; otherwise the loads from kr read the norm
    // weights' first word, which is discarded
    const auto kr = gptr(s.k_raw ? s.k_raw : a.w);
    const auto ic = gptr(a.ic);
    // the written key row, loaded first
    float kv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) kv[i] = kr[(s.k_raw && lane + 64 * i < dim) ? (size_t) t * s.k_ld + lane + 64 * i : 0];
    auto write_row = [&]() {
        if (!s.k_raw) return;
        const bool wok = wrow >= 0 && wrow < a.ic_rows;
#pragma unroll
        for (int i = 0; i < NI; i++)
            if (wok && lane + 64 * i < dim) ic[(size_t) wrow * dim + lane + 64 * i] = f2h(kv[i]);
        if (!wok && lane == 0) atomicOr(a.status, DEVERR_SET_ROWS_INDEX);
    };
    bool last = true;
    for (int u = t + 1; u < s.T; u++) last &= __shfl(bi, u) != blk;
    if (!last) {
        write_row();
        return;
    }
    if (a.r <= 64) {
        // lane m holds member m's row and the latest position at or before t
        // that writes it; then every member's values are loaded, 8 members a
        // round, before they are summed in member order (one round trip a
        // round, not one a member). The first round's loads go out before the
        // write, the tail's weights and cos / sin are fetched behind them: a
        // member row that this call writes is taken from k_raw, so the order of
        // the write and these reads does not matter.
        int my_src = -1;
        if (s.k_raw)
            for (int u = 0; u <= t; u++) my_src = __shfl(wi, u) == my_row ? u : my_src;
        float acc[NI];
        bool bad_row = false;
        uint16_t vi[8][NI];
        float vr[8][NI];
        int src[8];
        bool rok[8];
        auto load_round = [&](int m0) {
#pragma unroll
            for (int mm = 0; mm < 8; mm++) {
                const int m = m0 + mm;
                const bool mok = m < a.r;
                const int32_t row = __shfl(my_row, m & 63);
                src[mm] = __shfl(my_src, m & 63);
                rok[mm] = row >= 0 && row < a.ic_rows;
                bad_row |= mok && src[mm] < 0 && !rok[mm];
#pragma unroll
                for (int i = 0; i < NI; i++) {
                    const int d = lane + 64 * i;
                    const bool dok = mok && d < dim;
                    // unconditional loads at a valid address (row 0, dim 0 otherwise)
                    vi[mm][i] = ic[(dok && rok[mm]) ? (size_t) row * dim + d : 0];
                    vr[mm][i] = kr[(dok && src[mm] >= 0) ? (size_t) src[mm] * s.k_ld + d : 0];
                }
            }
        };
        // selects, not a break: a branch would put each member's loads behind
        // the previous member's wait
        auto sum_round = [&](int m0) {
#pragma unroll
            for (int mm = 0; mm < 8; mm++) {
                const int m = m0 + mm;
#pragma unroll
                for (int i = 0; i < NI; i++) {
                    const float v = src[mm] >= 0 ? h2f(f2h(vr[mm][i])) : (rok[mm] ? h2f(vi[mm][i]) : 0.f);
                    const float sum = __fadd_rn(acc[i], v);
                    acc[i] = m == 0 ? v : (m < a.r ? sum : acc[i]);
                }
            }
        };
        load_round(0);
        pool_tail_in in;
        pool_prefetch(a, lane, pos, in);
        write_row();
        __builtin_amdgcn_sched_barrier(0);
        sum_round(0);
        for (int m0 = 8; m0 < a.r; m0 += 8) {
            load_round(m0);
            __builtin_amdgcn_sched_barrier(0);        // every load of the round before the first sum waits
            sum_round(m0);
        }
        if (bad_row && lane == 0) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
#pragma unroll
        for (int i = 0; i < NI; i++)
            if (lane + 64 * i < dim) x[lane + 64 * i] = __fmul_rn(acc[i], a.inv_r);
        pool_finish_with(a, x, lane, blk, in);
        return;
    } else {
        write_row();
        for (int d = lane; d < dim; d += 64) {
            float acc = 0.f;
            for (int m = 0; m < a.r; m++) {
                const int64_t row = CLOSED ? mem0 + m : (int64_t) mem[m];
                int src = -1;                              // the latest position at or before t writing this row
                for (int u = 0; u <= t; u++) src = __shfl(wi, u) == row ? u : src;
                float v;
                if (src >= 0) {
                    v = h2f(f2h(s.k_raw[(size_t) src * s.k_ld + d]));
                } else if (row >= 0 && row < a.ic_rows) {
                    v = h2f(a.ic[(size_t) row * dim + d]);
                } else {
                    v = 0.f;
                    if (d == lane && lane == 0) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
                }
                acc = m == 0 ? v : __fadd_rn(acc, v);
            }
            x[d] = __fmul_rn(acc, a.inv_r);
        }
    }
    pool_finish(a, x, lane, pos, blk);
}

template <int NI>
__global__ __launch_bounds__(POOL_WAVES * 64) void k_qsa_pool_steps(pool_steps_args s) {
    __shared__ float xs[POOL_WAVES][POOL_MAX_DIM];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = (int) blockIdx.x * POOL_WAVES + wv;
    if (t < s.T) pool_step_wave<NI, false>(s, 0, xs[wv], t, lane);
}

// The step's preparation and pooling in one launch: workgroups below
// pool_blocks pool (4 positions each, indices in closed form), the others
// write the bias rows and the small inputs (prepare_steps_range). Neither
// part reads what the other writes.
struct prep_pool_args {
    pool_steps_args     s;
    qsa_prep_steps_args prep;
    int32_t             pool_blocks;
};

template <int NI>
__global__ __launch_bounds__(POOL_WAVES * 64) void k_qsa_prepare_pool_steps(prep_pool_args a) {
    __shared__ float xs[POOL_WAVES][POOL_MAX_DIM];
    if ((int) blockIdx.x < a.pool_blocks) {
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const int t = (int) blockIdx.x * POOL_WAVES + wv;
        if (t < a.s.T) pool_step_wave<NI, true>(a.s, a.prep.n_past, xs[wv], t, lane);
        return;
    }
    constexpr int64_t NT = POOL_WAVES * 64;
    prepare_steps_range(a.prep, (int64_t) (blockIdx.x - a.pool_blocks) * NT + threadIdx.x,
                        (int64_t) (gridDim.x - a.pool_blocks) * NT);
}

// The rebuild with 16-byte lanes, for dim / 8 a power of two and 16-byte
// aligned caches: a lane holds 8 dims of one block, summed over the block's r
// member rows in member order, and a wave holds 64 / (dim / 8) blocks (4 at
// dim 128). The normalised keys pass through LDS so that the rotation takes
// one (block, pair) per lane: the wave's fp64 sin / cos work is shared by all
// of its blocks (2 blocks per pass at n_dims 64) instead of one block leaving
// half the lanes idle. Per value the arithmetic is k_qsa_pool's.
constexpr int RB_WAVES = 4;
constexpr int RB_PRE = 4;       // member rows loaded ahead of the rope's cos / sin
constexpr int RB_TASKS = 4;     // rotation tasks a lane: bpw * n_dims / 2 <= 256
typedef unsigned v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(RB_WAVES * 64) void k_qsa_pool_rebuild(pool_args a) {
    __shared__ __align__(16) float xs[RB_WAVES][512];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int dim = a.dim, lpb = dim >> 3, bpw = 64 / lpb;
    const int lb = lane / lpb, lj = lane % lpb;
    const int64_t blk0 = ((int64_t) blockIdx.x * RB_WAVES + wv) * bpw;
    if (blk0 >= a.n_blk) return;   // wave-uniform
    const int64_t blk = blk0 + lb;
    const bool live = blk < a.n_blk;
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = 0.f;
    // the first RB_PRE member rows' loads go out first (unconditional, at
    // block 0 / member 0 where there is no such row); the rope's cos / sin,
    // which depend on the block positions alone, are computed while they land
    const uint16_t * src = a.ic + (size_t) (live ? blk : 0) * (size_t) a.r * (size_t) dim + 8 * lj;
    uint4 u[RB_PRE];
#pragma unroll
    for (int m = 0; m < RB_PRE; m++) u[m] = *(const uint4 *) (src + (size_t) (m < a.r ? m : 0) * dim);
    // lane task q: (block, pair) lane + 64 q of the wave's bpw blocks (at most
    // 4: bpw * n_dims / 2 <= 256); unused tasks keep cos 1, sin 0
    const int half = a.rp.n_dims / 2;
    float cq[RB_TASKS], sq4[RB_TASKS];
#pragma unroll
    for (int q = 0; q < RB_TASKS; q++) {
        const int idx = lane + 64 * q, b = idx / half, k = idx - b * half;
        cq[q] = 1.f;
        sq4[q] = 0.f;
        if (idx < bpw * half && blk0 + b < a.n_blk) {
            const int32_t p = (int32_t) ((blk0 + b) * a.r);
            const int32_t pos[4] = {p, p, p, p};
            rope_cos_sin(a.rp, pos, k, &cq[q], &sq4[q]);
        }
    }
    if (live) {
        auto add_row = [&](const uint4 & w, int m) {
            const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float v = h2f((uint16_t) (w4[i >> 1] >> (16 * (i & 1))));
                x[i] = m == 0 ? v : __fadd_rn(x[i], v);
            }
        };
#pragma unroll
        for (int m = 0; m < RB_PRE; m++)
            if (m < a.r) add_row(u[m], m);
        for (int m = RB_PRE; m < a.r; m++) add_row(*(const uint4 *) (src + (size_t) m * dim), m);
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = __fmul_rn(x[i], a.inv_r);
    }
    // RMS norm over the block's lpb lanes: the squares (float) summed in double
    double sq = 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) sq += (double) __fmul_rn(x[i], x[i]);
    if (lpb == 16) sq = wave::row16_sum_d(sq);   // a block's lanes are one DPP row
    else
        for (int off = lpb >> 1; off >= 1; off >>= 1) sq += __shfl_xor(sq, off);
    const float mean = (float) (sq / (double) dim);
    const float scale = 1.0f / sqrtf(__fadd_rn(mean, a.eps));
    float * xw = xs[wv] + lb * dim + 8 * lj;
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = __fmul_rn(__fmul_rn(x[i], scale), a.w[8 * lj + i]);
    *(float4 *) xw = make_float4(x[0], x[1], x[2], x[3]);
    *(float4 *) (xw + 4) = make_float4(x[4], x[5], x[6], x[7]);
    // the dims past the rotated ones go out from registers
    if (live) {
        uint16_t * out = a.pool + (size_t) blk * dim + 8 * lj;
        if (8 * lj >= a.rp.n_dims) {
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = (uint32_t) f2h(x[2 * i]) | ((uint32_t) f2h(x[2 * i + 1]) << 16);
            __builtin_nontemporal_store(v4u{o[0], o[1], o[2], o[3]}, (v4u *) out);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (8 * lj + i >= a.rp.n_dims) out[i] = f2h(x[i]);
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // rotation: lane -> (block, pair), the wave's blocks in turn
#pragma unroll
    for (int q = 0; q < RB_TASKS; q++) {
        const int idx = lane + 64 * q, b = idx / half, k = idx - b * half;
        const int64_t bk = blk0 + b;
        if (idx >= bpw * half || bk >= a.n_blk) break;   // idx only grows: every later task is past the end too
        float y0, y1;
        const float * xb = xs[wv] + b * dim;
        rope_rotate(xb[k], xb[k + half], cq[q], sq4[q], &y0, &y1);
        uint16_t * out = a.pool + (size_t) bk * dim;
        out[k] = f2h(y0);
        out[k + half] = f2h(y1);
    }
}

// ggml_set_rows F32 -> F16: row idx[i] of dst = fp16(row i of src)
struct f16_rows_args {
    uint16_t *      dst;
    size_t          dst_nb1;   // bytes
    int64_t         dst_rows;
    const float *   src;
    size_t          src_nb1;   // bytes
    int64_t         ne0;
    const int32_t * idx;
    int64_t         n;
    uint32_t *      status;
};

__global__ __launch_bounds__(256) void k_set_rows_f16(f16_rows_args a) {
    const int64_t i = blockIdx.y;
    const int32_t row = a.idx[i];
    if (row < 0 || row >= a.dst_rows) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(a.status, DEVERR_SET_ROWS_INDEX);
        return;
    }
    const float * s = (const float *) ((const char *) a.src + (size_t) i * a.src_nb1);
    uint16_t * d = (uint16_t *) ((char *) a.dst + (size_t) row * a.dst_nb1);
    for (int64_t j = (int64_t) blockIdx.x * 256 + threadIdx.x; j < a.ne0; j += (int64_t) gridDim.x * 256)
        d[j] = f2h(s[j]);
}

int pool_cfg_args(const qwfn_qsa_pool_cfg * cfg, int32_t ratio, const float * w, pool_args * a) {
    if (!cfg || !w) return set_error(QWFN_EINVAL, "qsa_pool: NULL cfg or k_norm weight");
    if (cfg->idx_dim < 2 || cfg->idx_dim > POOL_MAX_DIM || cfg->idx_dim % 2)
        return set_error(QWFN_ENOTSUP, "qsa_pool: idx_dim must be even and at most 256");
    if (cfg->n_dims < 2 || cfg->n_dims % 2 || cfg->n_dims > cfg->idx_dim || cfg->n_dims > 128)
        return set_error(QWFN_EINVAL, "qsa_pool: n_dims must be even, at most idx_dim and 128");
    int sect = 0;
    for (int s = 0; s < 4; s++) {
        if (cfg->sections[s] < 0) return set_error(QWFN_EINVAL, "qsa_pool: negative rope section");
        sect += cfg->sections[s];
    }
    if (sect <= 0) return set_error(QWFN_EINVAL, "qsa_pool: rope sections must not all be zero");
    if (!(cfg->freq_base > 0.f) || !std::isfinite(cfg->freq_base) || !(cfg->rms_eps >= 0.f))
        return set_error(QWFN_EINVAL, "qsa_pool: freq_base must be positive and rms_eps non-negative");
    if (ratio < 1 || ratio > 4096) return set_error(QWFN_EINVAL, "qsa_pool: ratio must lie in [1, 4096]");
    a->dim = cfg->idx_dim;
    a->r = ratio;
    a->inv_r = 1.0f / (float) ratio;
    a->eps = cfg->rms_eps;
    a->w = w;
    a->rp.n_dims = cfg->n_dims;
    for (int s = 0; s < 4; s++) a->rp.sections[s] = cfg->sections[s];
    a->rp.imrope = 1;
    a->rp.theta_scale = powf(cfg->freq_base, -2.0f / (float) cfg->n_dims);
    return QWFN_OK;
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" void qwfn_qsa_pool_cfg_default(qwfn_qsa_pool_cfg * cfg) {
    if (!cfg) return;
    cfg->idx_dim = 128;
    cfg->n_dims = 64;
    cfg->sections[0] = 11; cfg->sections[1] = 11; cfg->sections[2] = 10; cfg->sections[3] = 0;
    cfg->freq_base = 10000000.0f;
    cfg->rms_eps = 1e-6f;
}

extern "C" int qwfn_set_rows_f16(const qwfn_tensor * dst, const qwfn_tensor * src, const qwfn_tensor * idx,
                                 void * stream) {
    return ::qwfn::abi_call("set_rows_f16", [&]() -> int {
        if (!dst || !src || !idx || !dst->data || !src->data || !idx->data)
            return set_error(QWFN_EINVAL, "set_rows_f16: NULL tensor");
        if (dst->type != QWFN_TYPE_F16 || src->type != QWFN_TYPE_F32 || idx->type != QWFN_TYPE_I32)
            return set_error(QWFN_EINVAL, "set_rows_f16: dst must be f16, src f32, idx i32");
        if (dst->nb[0] != 2 || src->nb[0] != 4 || idx->nb[0] != 4)
            return set_error(QWFN_EINVAL, "set_rows_f16: rows must be contiguous");
        if (dst->ne[0] != src->ne[0] || src->ne[1] != idx->ne[0] || src->ne[2] != 1 || src->ne[3] != 1 ||
            dst->ne[2] != 1 || dst->ne[3] != 1 || idx->ne[1] != 1)
            return set_error(QWFN_EINVAL, "set_rows_f16: dst [ne0, rows], src [ne0, n], idx [n]");
        if (!is_aligned(dst->data, 2) || !is_aligned(src->data, 4) || !is_aligned(idx->data, 4) || dst->nb[1] % 2 ||
            src->nb[1] % 4)
            return set_error(QWFN_EALIGN, "set_rows_f16: element alignment");
        if (src->ne[1] > 65535) return set_error(QWFN_ENOTSUP, "set_rows_f16: at most 65535 rows per call");
        if (src->ne[0] == 0 || src->ne[1] == 0) return QWFN_OK;
        f16_rows_args a{};
        a.dst = (uint16_t *) dst->data; a.dst_nb1 = dst->nb[1]; a.dst_rows = dst->ne[1];
        a.src = (const float *) src->data; a.src_nb1 = src->nb[1]; a.ne0 = src->ne[0];
        a.idx = (const int32_t *) idx->data; a.n = src->ne[1];
        if (int rc = status_word(&a.status)) return rc;
        const unsigned gx = (unsigned) std::min<int64_t>((a.ne0 + 255) / 256, 64);
        hipLaunchKernelGGL(k_set_rows_f16, dim3(gx, (unsigned) a.n), dim3(256), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "set_rows_f16 launch");
    });
}

extern "C" int qwfn_qsa_pool_decode(uint16_t * idx_cache, int64_t ic_rows, const float * k_raw,
                                    const int32_t * write_idx, const int32_t * member_idx, int32_t ratio,
                                    const int32_t * blk_pos, const int32_t * blk_idx, const float * k_norm_w,
                                    uint16_t * pool, int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg, void * stream) {
    return ::qwfn::abi_call("qsa_pool_decode", [&]() -> int {
        pool_args a{};
        if (int rc = pool_cfg_args(cfg, ratio, k_norm_w, &a)) return rc;
        if (!idx_cache || !member_idx || !blk_pos || !blk_idx || !pool || (k_raw && !write_idx))
            return set_error(QWFN_EINVAL, "qsa_pool_decode: NULL pointer");
        if (ic_rows < 1 || pool_rows < 1) return set_error(QWFN_EINVAL, "qsa_pool_decode: empty cache");
        if (!is_aligned(idx_cache, 2) || !is_aligned(pool, 2) || !is_aligned(k_norm_w, 4) ||
            (k_raw && !is_aligned(k_raw, 4)))
            return set_error(QWFN_EALIGN, "qsa_pool_decode: element alignment");
        a.ic = idx_cache; a.ic_rows = ic_rows; a.pool = pool; a.pool_rows = pool_rows;
        a.k_raw = k_raw; a.write_idx = write_idx; a.member_idx = member_idx; a.blk_pos = blk_pos; a.blk_idx = blk_idx;
        a.n_blk = 1;
        if (int rc = status_word(&a.status)) return rc;
        hipLaunchKernelGGL(k_qsa_pool<true>, dim3(1), dim3(POOL_WAVES * 64), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_pool_decode launch");
    });
}

namespace qwfn {
namespace {

// Checks the pooling arguments of a step (qwfn_qsa_pool_decode_steps) and
// fills the kernel arguments; `who` names the entry point in the messages,
// `pointers`: the kernel reads the indices from qd (else their closed forms).
int pool_steps_fill(uint16_t * idx_cache, int64_t ic_rows, const float * k_raw, size_t k_raw_nb1, const qwfn_qsa_inputs * qd,
                    int32_t T, const float * k_norm_w, uint16_t * pool, int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg,
                    const char * who, bool pointers, pool_steps_args * sa) {
    if (!qd) return set_error2(QWFN_EINVAL, who, ": NULL inputs");
    if (T < 1 || T > POOL_MAX_T) return set_error2(QWFN_ENOTSUP, who, ": 1 to 16 positions");
    *sa = pool_steps_args{};
    if (int rc = pool_cfg_args(cfg, qd[0].ratio, k_norm_w, &sa->p)) return rc;
    if (!idx_cache || !pool) return set_error2(QWFN_EINVAL, who, ": NULL pointer");
    if (ic_rows < 1 || pool_rows < 1) return set_error2(QWFN_EINVAL, who, ": empty cache");
    if (!is_aligned(idx_cache, 2) || !is_aligned(pool, 2) || !is_aligned(k_norm_w, 4) ||
        (k_raw && (!is_aligned(k_raw, 4) || k_raw_nb1 % 4 || k_raw_nb1 < (size_t) sa->p.dim * 4)))
        return set_error2(QWFN_EALIGN, who, ": element alignment, or k_raw rows shorter than idx_dim");
    for (int t = 0; t < T; t++) {
        if (qd[t].ratio != qd[0].ratio) return set_error2(QWFN_EINVAL, who, ": positions of different ratios");
        if (!pointers) continue;
        if (!qd[t].member_idx || !qd[t].blk_pos || !qd[t].blk_idx || (k_raw && !qd[t].write_idx))
            return set_error2(QWFN_EINVAL, who, ": NULL tensor");
        sa->write_idx[t] = qd[t].write_idx;
        sa->member_idx[t] = qd[t].member_idx;
        sa->blk_pos[t] = qd[t].blk_pos;
        sa->blk_idx[t] = qd[t].blk_idx;
    }
    sa->p.ic = idx_cache; sa->p.ic_rows = ic_rows; sa->p.pool = pool; sa->p.pool_rows = pool_rows;
    sa->k_raw = k_raw;
    sa->k_ld = (int64_t) (k_raw_nb1 / 4);
    sa->T = T;
    return status_word(&sa->p.status);
}

}  // namespace
}  // namespace qwfn

extern "C" int qwfn_qsa_pool_decode_steps(uint16_t * idx_cache, int64_t ic_rows, const float * k_raw, size_t k_raw_nb1,
                                          const qwfn_qsa_inputs * qd, int32_t T, const float * k_norm_w, uint16_t * pool,
                                          int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg, void * stream) {
    return ::qwfn::abi_call("qsa_pool_decode_steps", [&]() -> int {
        pool_steps_args sa;
        if (int rc = pool_steps_fill(idx_cache, ic_rows, k_raw, k_raw_nb1, qd, T, k_norm_w, pool, pool_rows, cfg,
                                     "qsa_pool_decode_steps", true, &sa))
            return rc;
        const dim3 grid((unsigned) ((T + POOL_WAVES - 1) / POOL_WAVES));
        if (sa.p.dim <= 128)
            hipLaunchKernelGGL(k_qsa_pool_steps<2>, grid, dim3(POOL_WAVES * 64), 0, as_stream(stream), sa);
        else
            hipLaunchKernelGGL(k_qsa_pool_steps<POOL_MAX_DIM / 64>, grid, dim3(POOL_WAVES * 64), 0, as_stream(stream), sa);
        return hip_check(hipGetLastError(), "qsa_pool_decode_steps launch");
    });
}

extern "C" int qwfn_qsa_decode_prepare_pool_steps(const qwfn_qsa_inputs * qd, int32_t T, int32_t n_past, uint16_t * idx_cache,
                                                  int64_t ic_rows, const float * k_raw, size_t k_raw_nb1,
                                                  const float * k_norm_w, uint16_t * pool, int64_t pool_rows,
                                                  const qwfn_qsa_pool_cfg * cfg, void * stream) {
    return ::qwfn::abi_call("qsa_decode_prepare_pool_steps", [&]() -> int {
        prep_pool_args a{};
        if (int rc = prep_steps_args(qd, T, n_past, "qsa_decode_prepare_pool_steps", &a.prep)) return rc;
        if (int rc = pool_steps_fill(idx_cache, ic_rows, k_raw, k_raw_nb1, qd, T, k_norm_w, pool, pool_rows, cfg,
                                     "qsa_decode_prepare_pool_steps", false, &a.s))
            return rc;
        a.pool_blocks = (T + POOL_WAVES - 1) / POOL_WAVES;
        const int64_t n = std::max<int64_t>(qd[0].n_blocks_max, T);
        const int64_t prep_blocks = std::max<int64_t>(1, std::min<int64_t>((n + POOL_WAVES * 64 - 1) / (POOL_WAVES * 64), 4096));
        const dim3 grid((unsigned) (a.pool_blocks + prep_blocks));
        if (a.s.p.dim <= 128)
            hipLaunchKernelGGL(k_qsa_prepare_pool_steps<2>, grid, dim3(POOL_WAVES * 64), 0, as_stream(stream), a);
        else
            hipLaunchKernelGGL(k_qsa_prepare_pool_steps<POOL_MAX_DIM / 64>, grid, dim3(POOL_WAVES * 64), 0,
                               as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_decode_prepare_pool_steps launch");
    });
}

extern "C" int qwfn_qsa_pool_rebuild(const uint16_t * idx_cache, int64_t ic_rows, int64_t n_past, int32_t ratio,
                                     const float * k_norm_w, uint16_t * pool, int64_t pool_rows,
                                     const qwfn_qsa_pool_cfg * cfg, void * stream) {
    return ::qwfn::abi_call("qsa_pool_rebuild", [&]() -> int {
        pool_args a{};
        if (int rc = pool_cfg_args(cfg, ratio, k_norm_w, &a)) return rc;
        if (!idx_cache || !pool) return set_error(QWFN_EINVAL, "qsa_pool_rebuild: NULL pointer");
        if (n_past < 0) return set_error(QWFN_EINVAL, "qsa_pool_rebuild: negative n_past");
        const int64_t n_whole = n_past / ratio;
        if (n_whole * ratio > ic_rows) return set_error(QWFN_ERANGE, "qsa_pool_rebuild: n_past beyond the index cache");
        if (n_whole > pool_rows) return set_error(QWFN_ERANGE, "qsa_pool_rebuild: more whole blocks than pool rows");
        if (n_whole * ratio >= (int64_t(1) << 31)) return set_error(QWFN_ENOTSUP, "qsa_pool_rebuild: positions beyond 2^31");
        if (!is_aligned(idx_cache, 2) || !is_aligned(pool, 2) || !is_aligned(k_norm_w, 4))
            return set_error(QWFN_EALIGN, "qsa_pool_rebuild: element alignment");
        if (n_whole == 0) return QWFN_OK;
        a.ic = const_cast<uint16_t *>(idx_cache); a.ic_rows = ic_rows; a.pool = pool; a.pool_rows = pool_rows;
        a.n_blk = n_whole;
        if (int rc = status_word(&a.status)) return rc;
        const int lpb = a.dim / 8;
        if (a.dim % 8 == 0 && (lpb & (lpb - 1)) == 0 && is_aligned(idx_cache, 16) && is_aligned(pool, 16)) {
            const int64_t waves = (n_whole + 64 / lpb - 1) / (64 / lpb);
            const int64_t grid = (waves + RB_WAVES - 1) / RB_WAVES;
            hipLaunchKernelGGL(k_qsa_pool_rebuild, dim3((unsigned) grid), dim3(RB_WAVES * 64), 0, as_stream(stream), a);
            return hip_check(hipGetLastError(), "qsa_pool_rebuild launch");
        }
        const int64_t grid = (n_whole + POOL_WAVES - 1) / POOL_WAVES;
        hipLaunchKernelGGL(k_qsa_pool<false>, dim3((unsigned) grid), dim3(POOL_WAVES * 64), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "qsa_pool_rebuild launch");
    });
}
