// The Gated DeltaNet recurrent update of a step, with its rollback snapshots
// written by the kernel itself: the ggml_gated_delta_net of
// graph_builder::deltanet (qwfn_graph.cpp:240-278) and the state copies of
// deltanet_write_state (:208-238) in one launch.
//
// Per value head h (key head h / (n_v / n_k)) the state S [dk][dv] (dv
// contiguous) evolves token by token (the gated delta rule):
//   S = S * exp(g);  m[c] = sum_r S[r][c] k[r];  S[r][c] += k[r] (v[c] - m[c]) beta
//   out[c] = sum_r S[r][c] q[r] scale
// Columns c are independent: a workgroup takes 32 columns of one head, 8 lanes
// per column (16 rows each, the sums over r finished by a butterfly across the
// 8 lanes), so each state column stays in registers for the whole step and the
// state is read and written once. After token T-1-s the state is also stored
// to rollback slot s-1 (s = 1 .. n_snap): the state s tokens back.
#include "qwfn_common.h"
#include "qwfn_state.h"

#include <cmath>

namespace qwfn {
namespace {

constexpr int DN_D = 128;                  // key and value head size (ssm_d_state)
constexpr int DN_COLS = 32;                // state columns per workgroup
constexpr int DN_SLICES = 8;               // lanes per column
constexpr int DN_RPS = DN_D / DN_SLICES;   // rows per lane

struct dn_args {
    const float * q;  int64_t q_ts;        // [T] x [n_k][dk], token stride in floats
    const float * k;  int64_t k_ts;
    const float * v;  int64_t v_ts;        // [T] x [n_v][dv]
    const float * g;                       // [T][n_v] log decay
    const float * beta;                    // [T][n_v]
    float *       state;                   // [n_v][dk][dv], in place
    float *       out;                     // [T][n_v][dv]
    float *       snap;                    // slot s: snap + s * snap_stride floats, [n_v][dk][dv]
    int64_t       snap_stride;
    int32_t       n_snap;
    int32_t       T, n_k, n_v, rep;
    float         scale;
};

__device__ __forceinline__ float sum8(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    return x;
}

__global__ __launch_bounds__(DN_COLS * DN_SLICES) void k_gated_delta_net(dn_args a) {
    const int h = blockIdx.x / (DN_D / DN_COLS), cb = blockIdx.x % (DN_D / DN_COLS);
    const int j = threadIdx.x & (DN_SLICES - 1);
    const int c = cb * DN_COLS + (int) (threadIdx.x >> 3);
    const int r0 = DN_RPS * j;
    float * Sg = a.state + (size_t) h * DN_D * DN_D;
    float S[DN_RPS];
#pragma unroll
    for (int i = 0; i < DN_RPS; i++) S[i] = Sg[(size_t) (r0 + i) * DN_D + c];
    const int hk = h / a.rep;
    for (int t = 0; t < a.T; t++) {
        const float4 * kp = (const float4 *) (a.k + t * a.k_ts + (int64_t) hk * DN_D + r0);
        const float4 * qp = (const float4 *) (a.q + t * a.q_ts + (int64_t) hk * DN_D + r0);
        float kk[DN_RPS], qq[DN_RPS];
#pragma unroll
        for (int i = 0; i < DN_RPS / 4; i++) {
            const float4 k4 = kp[i], q4 = qp[i];
            kk[4 * i] = k4.x; kk[4 * i + 1] = k4.y; kk[4 * i + 2] = k4.z; kk[4 * i + 3] = k4.w;
            qq[4 * i] = q4.x; qq[4 * i + 1] = q4.y; qq[4 * i + 2] = q4.z; qq[4 * i + 3] = q4.w;
        }
        const float e = expf(a.g[(int64_t) t * a.n_v + h]);
        const float b = a.beta[(int64_t) t * a.n_v + h];
        const float vc = a.v[t * a.v_ts + (int64_t) h * DN_D + c];
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < DN_RPS; i++) {
            S[i] = S[i] * e;
            m = __fmaf_rn(S[i], kk[i], m);
        }
        m = sum8(m);
        const float d = (vc - m) * b;
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < DN_RPS; i++) {
            S[i] = __fmaf_rn(kk[i], d, S[i]);
            o = __fmaf_rn(S[i], qq[i] * a.scale, o);
        }
        o = sum8(o);
        if (j == 0) a.out[((int64_t) t * a.n_v + h) * DN_D + c] = o;
        const int sb = a.T - 1 - t;
        if (sb >= 1 && sb <= a.n_snap) {
            float * sp = a.snap + (sb - 1) * a.snap_stride + (size_t) h * DN_D * DN_D;
#pragma unroll
            for (int i = 0; i < DN_RPS; i++) sp[(size_t) (r0 + i) * DN_D + c] = S[i];
        }
    }
#pragma unroll
    for (int i = 0; i < DN_RPS; i++) Sg[(size_t) (r0 + i) * DN_D + c] = S[i];
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" int qwfn_gated_delta_net(const float * q, int64_t q_token_stride, const float * k, int64_t k_token_stride,
                                    const float * v, int64_t v_token_stride, const float * g, const float * beta,
                                    int32_t T, int32_t n_k_heads, int32_t n_v_heads, int32_t head_dim, float scale,
                                    float * state, float * out, float * snap, size_t snap_stride_bytes, int32_t n_snap,
                                    void * stream) {
    return ::qwfn::abi_call("gated_delta_net", [&]() -> int {
        if (!q || !k || !v || !g || !beta || !state || !out) return set_error(QWFN_EINVAL, "gated_delta_net: NULL pointer");
        if (head_dim != DN_D) return set_error(QWFN_ENOTSUP, "gated_delta_net: head_dim must be 128");
        if (T < 1 || n_k_heads < 1 || n_v_heads < 1 || n_v_heads % n_k_heads)
            return set_error(QWFN_EINVAL, "gated_delta_net: T >= 1 and n_v_heads a multiple of n_k_heads");
        if (q_token_stride < (int64_t) n_k_heads * DN_D || k_token_stride < (int64_t) n_k_heads * DN_D ||
            v_token_stride < (int64_t) n_v_heads * DN_D)
            return set_error(QWFN_EINVAL, "gated_delta_net: token strides shorter than a token's heads");
        if (n_snap < 0 || n_snap > T - 1) return set_error(QWFN_EINVAL, "gated_delta_net: n_snap must lie in [0, T-1]");
        const size_t state_bytes = (size_t) n_v_heads * DN_D * DN_D * sizeof(float);
        if (n_snap > 0 && (!snap || snap_stride_bytes < state_bytes || snap_stride_bytes % 4))
            return set_error(QWFN_EINVAL, "gated_delta_net: snapshot slots must hold the state (stride a multiple of 4)");
        if (!is_aligned(q, 16) || !is_aligned(k, 16) || q_token_stride % 4 || k_token_stride % 4 || !is_aligned(v, 4) ||
            !is_aligned(g, 4) || !is_aligned(beta, 4) || !is_aligned(state, 4) || !is_aligned(out, 4) ||
            (snap && !is_aligned(snap, 4)))
            return set_error(QWFN_EALIGN, "gated_delta_net: q, k 16-byte aligned (token strides multiples of 4), the rest 4");
        dn_args a{};
        a.q = q; a.q_ts = q_token_stride; a.k = k; a.k_ts = k_token_stride; a.v = v; a.v_ts = v_token_stride;
        a.g = g; a.beta = beta; a.state = state; a.out = out;
        a.snap = snap; a.snap_stride = (int64_t) (snap_stride_bytes / sizeof(float)); a.n_snap = n_snap;
        a.T = T; a.n_k = n_k_heads; a.n_v = n_v_heads; a.rep = n_v_heads / n_k_heads; a.scale = scale;
        const unsigned blocks = (unsigned) n_v_heads * (DN_D / DN_COLS);
        hipLaunchKernelGGL(k_gated_delta_net, dim3(blocks), dim3(DN_COLS * DN_SLICES), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "gated_delta_net launch");
    });
}
