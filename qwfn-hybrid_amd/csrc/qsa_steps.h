// The decode step inputs of Qwen Sparse Attention for a verify step's
// positions n_past .. n_past + T - 1, shared by the preparation alone
// (seq_state.hip) and the preparation fused with the index pooling
// (qsa_pool.hip). Every value is a closed form of the position p = n_past + t
// and the ratio r (engine::qsa_decode_prepare, qwfn_engine.cpp:1072-1105):
// write_idx = p, blk_idx = p / r, member_idx[m] = (p / r) r + m, blk_pos = 4 x
// (p / r) r, npast_f = p, and the bias of block b: 0 for whole blocks, 1e9 for
// the incomplete block of p, -inf past it, within the window p / r - 1 ..
// p / r + 1 of the previous position's bias.
#pragma once

#include "qwfn_common.h"
#include "qwfn_state.h"

#include <cmath>
#include <cstdint>

namespace qwfn {

// The decode bias of block b at n_past (b_last = n_past / ratio, n_bid =
// (n_past + 1) / ratio): 0 whole block, 1e9 the incomplete block of n_past,
// -inf beyond (qwfn_engine.cpp:1093-1096 for the window, :1115-1120 for all).
__device__ __forceinline__ float bias_of(int64_t b, int64_t b_last, int64_t n_bid) {
    return b < n_bid ? 0.0f : (b == b_last ? 1e9f : -INFINITY);
}

constexpr int PREP_MAX_T = 16;
struct qsa_prep_steps_args {
    qwfn_qsa_inputs qd[PREP_MAX_T];
    int32_t         T;
    int32_t         n_past;
};

// qwfn_qsa_decode_prepare(&qd[0], NULL, n_past) then qwfn_qsa_decode_prepare(
// &qd[t], qd[t-1].bias, n_past + t) for t = 1 .. T-1, for the blocks t0,
// t0 + stride, .. of the bias rows and, from the threads t0 < T, position t0's
// small inputs: row t's block b is the value of the latest window at or before
// t that holds b, else the running bias qd[0].bias[b], which the thread reads
// before it writes (the window of position 0 lands in place in qd[0].bias).
__device__ __forceinline__ void prepare_steps_range(const qsa_prep_steps_args & a, int64_t t0, int64_t stride) {
    const int64_t r = a.qd[0].ratio, nbm = a.qd[0].n_blocks_max;
    for (int64_t b = t0; b < nbm; b += stride) {
        float v = gptr(a.qd[0].bias)[b];
        for (int t = 0; t < a.T; t++) {
            const int64_t p = (int64_t) a.n_past + t, b_last = p / r, n_bid = (p + 1) / r;
            const int64_t lo = b_last > 0 ? b_last - 1 : 0;
            const bool win = b >= lo && b <= b_last + 1;
            if (win) v = bias_of(b, b_last, n_bid);
            if (t == 0) {
                if (win) gptr(a.qd[0].bias)[b] = v;
            } else {
                gptr(a.qd[t].bias)[b] = v;
            }
        }
    }
    if (t0 < a.T) {
        const int t = (int) t0;
        const int64_t p = (int64_t) a.n_past + t, b_last = p / r;
        const qwfn_qsa_inputs & q = a.qd[t];
        for (int64_t m = 0; m < r; m++) gptr(q.member_idx)[m] = (int32_t) (b_last * r + m);
        for (int i = 0; i < 4; i++) gptr(q.blk_pos)[i] = (int32_t) (b_last * r);
        *gptr(q.write_idx) = (int32_t) p;
        *gptr(q.blk_idx) = (int32_t) b_last;
        *gptr(q.npast_f) = (float) p;
    }
}

// Checks the step inputs of qwfn_qsa_decode_prepare_steps and fills the
// kernel arguments; `who` names the entry point in the error messages.
inline int prep_steps_args(const qwfn_qsa_inputs * qd, int32_t T, int32_t n_past, const char * who,
                           qsa_prep_steps_args * a) {
    if (!qd) return set_error2(QWFN_EINVAL, who, ": NULL inputs");
    if (T < 1 || T > PREP_MAX_T) return set_error2(QWFN_ENOTSUP, who, ": 1 to 16 positions");
    if (n_past < 0 || (int64_t) n_past + T - 1 > INT32_MAX) return set_error2(QWFN_EINVAL, who, ": positions outside [0, 2^31)");
    *a = qsa_prep_steps_args{};
    for (int t = 0; t < T; t++) {
        const qwfn_qsa_inputs & q = qd[t];
        if (!q.bias || !q.write_idx || !q.member_idx || !q.blk_pos || !q.blk_idx || !q.npast_f)
            return set_error2(QWFN_EINVAL, who, ": NULL tensor");
        if (q.ratio < 1 || q.n_blocks_max < 1 || q.ratio != qd[0].ratio || q.n_blocks_max != qd[0].n_blocks_max)
            return set_error2(QWFN_EINVAL, who, ": every position needs the same ratio >= 1 and n_blocks_max >= 1");
        for (int u = 0; u < t; u++) {
            const char * x0 = (const char *) q.bias, * x1 = x0 + q.n_blocks_max * 4;
            const char * y0 = (const char *) qd[u].bias, * y1 = y0 + q.n_blocks_max * 4;
            if (x0 < y1 && y0 < x1) return set_error2(QWFN_EINVAL, who, ": bias rows overlap");
        }
        a->qd[t] = q;
    }
    a->T = T;
    a->n_past = n_past;
    return QWFN_OK;
}

}  // namespace qwfn
