// The Gated DeltaNet recurrent update of a step, with its rollback snapshots
// written by the kernel itself: the ggml_gated_delta_net of
// graph_builder::deltanet (qwfn_graph.cpp:240-278) and the state copies of
// deltanet_write_state (:208-238) in one launch.
//
// Per value head h (key head h / (n_v / n_k)) the state S [dk][dv] (dv
// contiguous) evolves token by token (the gated delta rule):
//   S = S * exp(g);  m[c] = sum_r S[r][c] k[r];  S[r][c] += k[r] (v[c] - m[c]) beta
//   out[c] = sum_r S[r][c] q[r] scale
// Columns c are independent: a workgroup takes 32 columns of one head and
// splits the 128 rows into 16 slices of 8; lane l of wave w holds column
// 32 cb + (l & 31) of slice 2 w + (l >> 5), so every state load and store of a
// wave covers two whole 128-byte row pieces. A column stays in registers for
// the whole step and the state is read and written once. The sums over r
// are finished across the two halves of the wave (permlane32 swap) and then
// across the 8 waves through LDS, in a fixed order; one barrier a token (a
// token's output sums share the next token's barrier) and one at the end. The inputs of up to DN_TC
// tokens (k and q of the key head in LDS, v, the decay and beta in registers)
// are loaded together with the state. After token T-1-s the state is also
// stored to rollback slot s-1 (s = 1 .. n_snap): the state s tokens back.
#include "qwfn_common.h"
#include "qwfn_state.h"

#include <cmath>

namespace qwfn {
namespace {

constexpr int DN_D = 128;                  // key and value head size (ssm_d_state)
constexpr int DN_COLS = 32;                // state columns per workgroup: 128 bytes of each state row
constexpr int DN_TC = 4;                   // tokens whose inputs are loaded at once
constexpr int DN_SLICES = 16;              // row slices per column
constexpr int DN_WAVES = DN_SLICES / 2;    // two slices a wave
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

// x plus the value of the lane 32 away (the same column, the other slice)
__device__ __forceinline__ float sum_halves(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    unsigned p = r[0], q = r[1];
    asm volatile("" : "+v"(p), "+v"(q));
    return __builtin_bit_cast(float, p) + __builtin_bit_cast(float, q);
}

static_assert(DN_COLS == 32 && DN_WAVES * 64 == DN_COLS * DN_SLICES, "a wave: 32 columns x 2 slices");

// the waves' partial sums of column cl, in a fixed order (pairs, then pairs
// of pairs)
__device__ __forceinline__ float red_sum(const float (*red)[DN_COLS], int cl) {
    float x[DN_WAVES];
#pragma unroll
    for (int i = 0; i < DN_WAVES; i++) x[i] = red[i][cl];
#pragma unroll
    for (int n = DN_WAVES; n > 1; n >>= 1)
#pragma unroll
        for (int i = 0; i < n / 2; i++) x[i] = x[2 * i] + x[2 * i + 1];
    return x[0];
}

__global__ __launch_bounds__(DN_WAVES * 64) void k_gated_delta_net(dn_args a) {
    __shared__ float4 kq[DN_TC][2][DN_D / 4];   // [token][k, q][rows / 4]
    // the waves' partial sums, two buffers each by token parity: token t's
    // output sums are read after token t + 1's first barrier (or the last one)
    __shared__ float red_m[2][DN_WAVES][DN_COLS], red_o[2][DN_WAVES][DN_COLS];
    const int h = blockIdx.x / (DN_D / DN_COLS), cb = blockIdx.x % (DN_D / DN_COLS);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int cl = lane & 31;
    const int c = cb * DN_COLS + cl;
    const int r0 = DN_RPS * (2 * w + (lane >> 5));
    float * Sg = a.state + (size_t) h * DN_D * DN_D;
    float S[DN_RPS];
#pragma unroll
    for (int i = 0; i < DN_RPS; i++) S[i] = Sg[(size_t) (r0 + i) * DN_D + c];
    const int hk = h / a.rep;
    for (int t0 = 0; t0 < a.T; t0 += DN_TC) {
        const int nt = a.T - t0 < DN_TC ? a.T - t0 : DN_TC;
        if (t0 > 0) __syncthreads();   // every lane has read the previous tokens' k and q
        for (int u = (int) threadIdx.x; u < nt * 2 * (DN_D / 4); u += DN_WAVES * 64) {
            const int tt = u / (2 * (DN_D / 4)), kqs = (u / (DN_D / 4)) & 1, e4 = u % (DN_D / 4);
            const float * src = kqs ? a.q + (int64_t) (t0 + tt) * a.q_ts : a.k + (int64_t) (t0 + tt) * a.k_ts;
            kq[tt][kqs][e4] = *(const float4 *) (src + (int64_t) hk * DN_D + 4 * e4);
        }
        float vv[DN_TC], ee[DN_TC], bb[DN_TC];
#pragma unroll
        for (int tt = 0; tt < DN_TC; tt++) {
            vv[tt] = ee[tt] = bb[tt] = 0.f;
            if (tt < nt) {
                const int64_t t = t0 + tt;
                vv[tt] = a.v[t * a.v_ts + (int64_t) h * DN_D + c];
                ee[tt] = expf(a.g[t * a.n_v + h]);
                bb[tt] = a.beta[t * a.n_v + h];
            }
        }
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < DN_TC; tt++) {
            if (tt >= nt) break;
            const int t = t0 + tt;
            float kk[DN_RPS], qq[DN_RPS];
#pragma unroll
            for (int i = 0; i < DN_RPS / 4; i++) {
                const float4 k4 = kq[tt][0][r0 / 4 + i], q4 = kq[tt][1][r0 / 4 + i];
                kk[4 * i] = k4.x; kk[4 * i + 1] = k4.y; kk[4 * i + 2] = k4.z; kk[4 * i + 3] = k4.w;
                qq[4 * i] = q4.x; qq[4 * i + 1] = q4.y; qq[4 * i + 2] = q4.z; qq[4 * i + 3] = q4.w;
            }
            const float e = ee[tt], b = bb[tt], vc = vv[tt];
            float m = 0.f;
#pragma unroll
            for (int i = 0; i < DN_RPS; i++) {
                S[i] = S[i] * e;
                m = __fmaf_rn(S[i], kk[i], m);
            }
            m = sum_halves(m);
            if (lane < 32) red_m[t & 1][w][cl] = m;
            __syncthreads();
            if (t > 0 && w == 0 && lane < 32)
                a.out[((int64_t) (t - 1) * a.n_v + h) * DN_D + c] = red_sum(red_o[(t - 1) & 1], cl);
            m = red_sum(red_m[t & 1], cl);
            const float d = (vc - m) * b;
            float o = 0.f;
#pragma unroll
            for (int i = 0; i < DN_RPS; i++) {
                S[i] = __fmaf_rn(kk[i], d, S[i]);
                o = __fmaf_rn(S[i], qq[i] * a.scale, o);
            }
            o = sum_halves(o);
            if (lane < 32) red_o[t & 1][w][cl] = o;
            const int sb = a.T - 1 - t;
            if (sb >= 1 && sb <= a.n_snap) {
                float * sp = a.snap + (sb - 1) * a.snap_stride + (size_t) h * DN_D * DN_D;
#pragma unroll
                for (int i = 0; i < DN_RPS; i++) __builtin_nontemporal_store(S[i], &sp[(size_t) (r0 + i) * DN_D + c]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < DN_RPS; i++) __builtin_nontemporal_store(S[i], &Sg[(size_t) (r0 + i) * DN_D + c]);
    __syncthreads();
    if (w == 0 && lane < 32)
        a.out[((int64_t) (a.T - 1) * a.n_v + h) * DN_D + c] = red_sum(red_o[(a.T - 1) & 1], cl);
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
        hipLaunchKernelGGL(k_gated_delta_net, dim3(blocks), dim3(DN_WAVES * 64), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "gated_delta_net launch");
    });
}
