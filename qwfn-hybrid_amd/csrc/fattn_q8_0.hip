// Flash attention straight from the raw q8_0 KV cache, for decode and MTP
// verify (T * n_head/n_head_kv <= 64 query rows per KV head), on gfx950.
//
// Semantics: ggml_flash_attn_ext with q8_0 K/V and F32 accumulation, as the
// reference calls it at qwfn_graph.cpp:469-471 (dense / MTP head / QSA-off
// decode and verify) and :698-699 (QSA decode over gathered cells). The CPU
// one-chunk loop of ggml (the oracle) requantises Q to q8_0, takes
// s = sum_b d_k[b]*d_q[b]*isum_b, skips keys whose mask is -inf, runs an online
// softmax and accumulates dequantised V rows. This kernel keeps that arithmetic:
// Q is requantised with the same quantiser, the integer block dot products are
// exact (i8 MFMA), only the float accumulation order differs.
//
// Work decomposition (flash-decoding):
//   grid   : (batch, KV head, key split), ordered so that the KV heads of one
//            split run on the same XCD (their rows share cache lines).
//   block  : 4 wavefronts. A 128-key chunk of K and V rows (272-byte head
//            segments) is staged into LDS with 16-byte loads; wave w owns keys
//            [32w, 32w+32) of the chunk.
//   QK^T   : v_mfma_i32_16x16x32_i8, A = 16 keys x one 32-value block of K,
//            B = the block of 16 requantised query rows; the int32 tile is
//            scaled by d_q*d_k per block (one FMA per element) into F32 scores.
//   softmax: online, base 2, per query row; row max reduced over the 4 lane
//            groups with cross-lane swaps.
//   PV     : v_mfma_f32_16x16x32_f16, A = V^T (16 dims x 32 keys, exact int8 ->
//            f16 via SDWA byte-select conversion), B = P*d_v for one V block.
//   merge  : the 4 waves merge in LDS; the key splits merge in a second kernel
//            (LSE merge), or in place when there is a single split.
#include "q8_device.h"
#include "qwfn_common.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace qwfn {
namespace {

typedef int      v4i __attribute__((ext_vector_type(4)));
typedef float    v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int D      = 256;            // head size (values per head row)
constexpr int NBLK   = D / QK;         // 8 q8_0 blocks per head row
constexpr int SEG    = NBLK * QBLOCK;  // 272 bytes per head row
constexpr int PIECES = SEG / 16;       // 17 16-byte pieces per head row
constexpr int WAVES  = 4;
constexpr int THREADS = WAVES * 64;
constexpr int KW     = 32;             // keys per wave per chunk
constexpr int CK     = WAVES * KW;     // keys per chunk
constexpr int MAX_RW = 32;             // query rows per block (2 MFMA row tiles)
constexpr float LOG2E = 1.4426950408889634f;

struct fa_args {
    const char * q;  size_t q_nb1, q_nb2, q_nb3;
    const char * k;  size_t k_nb1, k_nb2, k_nb3;
    const char * v;  size_t v_nb1, v_nb2, v_nb3;
    const char * mask; size_t m_nb1, m_nb2, m_nb3;
    int32_t m_ne2, m_ne3;
    float *  dst;          // [D, nh, T, B]
    float *  part_o;       // [B][nh_kv][ns][R][D] (tile order)
    float2 * part_ml;      // [B][nh_kv][ns][R]
    int64_t  n_kv;
    int32_t  T, nh, nh_kv, gqa, R, B;
    int32_t  kb, vb;       // K/V batch extents (ne[3]); batch b reads b % kb
    int32_t  ns;           // key splits
    int32_t  split_len;    // keys per split, multiple of CK
    int32_t  rw;           // query rows per block (row group size)
    int32_t  n_rg;         // row groups per KV head
    float    scale;
    int32_t  x86;
};

// Dim of the element at tile position pos (0..255) of the PV output.
// Tile (block b, half e) holds, in row m, dim 32b + 4(m%8) + 2e + m/8; the
// MFMA output lane (n, g) holds rows 4g..4g+3. pos = 32b + 16e + 4g + i.
__host__ __device__ __forceinline__ int pos_to_dim(int pos) {
    const int b = pos >> 5, e = (pos >> 4) & 1, m = pos & 15;
    return 32 * b + 4 * (m & 7) + 2 * e + (m >> 3);
}

// Two int8 values (byte 0 or 2 of a and of b) -> packed f16 pair, exact.
__device__ __forceinline__ uint32_t cvt_i8x2_f16_b0(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0"
        : "=&v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t cvt_i8x2_f16_b2(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_2"
        : "=&v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t * p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);   // gfx950 LDS reads any alignment in one ds_read_b32
    return v;
}
__device__ __forceinline__ uint64_t lds_u64(const uint8_t * p) {
    uint64_t v;
    __builtin_memcpy(&v, p, 8);
    return v;
}

__device__ __forceinline__ float xmax(float a, float b) { return a > b ? a : b; }

__device__ __forceinline__ float h2f(uint64_t four, int i) {
    return dev::f16_bits_to_f32((uint16_t) (four >> (16 * i)));
}

typedef __attribute__((address_space(3))) void lds_void;

// LDS layout of one block (bytes).
struct lds_layout {
    static constexpr int KS = 0;                          // K rows  [CK][272]
    static constexpr int VS = KS + CK * SEG;              // V rows  [CK][272]
    static constexpr int KD = VS + CK * SEG;              // K scales [8][CK] fp16
    static constexpr int VD = KD + CK * NBLK * 2;         // V scales [8][CK] fp16
    static constexpr int MS = VD + CK * NBLK * 2;         // mask [n_mrows][CK] fp16
    static constexpr int MAX_MROWS = 32;
    static constexpr int END = MS + MAX_MROWS * CK * 2;
    // Aliases used before / after the key loop.
    static constexpr int QS = 0;                          // Q int8 [32][256]
    static constexpr int QD = QS + 32 * D;                // Q scales [32][8] f32
    static constexpr int OB = 0;                          // merge buffer [32][256] f32
    static constexpr int ML = OB + 32 * D * 4;            // per-wave (m, l) [4][32]
};
static_assert(lds_layout::QD + 32 * NBLK * 4 <= lds_layout::MS, "Q staging fits below the mask");
static_assert(lds_layout::ML + WAVES * 32 * 8 <= lds_layout::MS, "merge buffer fits below the mask");
static_assert(CK * PIECES % 64 == 0, "staging is whole wave instructions");

template <int RT>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_fattn_q8_0(fa_args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int ln = lane & 15;       // MFMA row/col within a 16-tile
    const int lg = lane >> 4;       // lane group (k-chunk / output row quad)

    // ---- block -> (b, kvh, row group, split); a split's heads and row groups share an XCD ----
    const int id   = blockIdx.x;
    const int xcd  = id & 7;
    const int j    = id >> 3;
    const int hgn  = a.nh_kv * a.n_rg;
    const int hg   = j % hgn;
    const int kvh  = hg / a.n_rg;
    const int rg   = hg - kvh * a.n_rg;
    const int u    = (j / hgn) * 8 + xcd;
    const int b    = u / a.ns;
    const int split = u - b * a.ns;
    if (b >= a.B) return;
    const int64_t k_lo = (int64_t) split * a.split_len;
    const int64_t k_hi = std::min<int64_t>(a.n_kv, k_lo + a.split_len);
    const int r0 = rg * a.rw;                          // first query row of this block
    const int RW = std::min(a.rw, a.R - r0);          // rows in this block
    const int t0 = r0 / a.gqa;
    const int n_mrows = a.m_ne2 == 1 ? (r0 + RW - 1) / a.gqa - t0 + 1 : RW;

    // ---- stage Q: requantise the block's query rows to q8_0 ----
    {
        uint32_t * qs = (uint32_t *) (lds + lds_layout::QS);
        float *    qd = (float *) (lds + lds_layout::QD);
        const int sub = lane & 7;       // 4-value group in a block
        const int blk = lane >> 3;      // block in the row
        for (int rl = wave; rl < RT * 16; rl += WAVES) {
            float x[4] = {0.f, 0.f, 0.f, 0.f};
            if (rl < RW) {
                const int r = r0 + rl;
                const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
                const float4 v = *(const float4 *) (a.q + (size_t) t * a.q_nb1 + (size_t) h * a.q_nb2 +
                                                    (size_t) b * a.q_nb3 + (size_t) (blk * QK + sub * 4) * 4);
                x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
            }
            uint16_t d16;
            float dq;
            const uint32_t w = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dq);
            qs[rl * (D / 4) + blk * 8 + sub] = w;
            if (sub == 0) qd[rl * NBLK + blk] = dq;
        }
    }
    __syncthreads();

    long  qB[RT][NBLK];
    float dqr[RT][NBLK];
    int   mrow[RT];     // staged mask row of this lane's query row; -1 for padding rows
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int rl = rt * 16 + ln;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            qB[rt][bb] = (long) lds_u64(lds + lds_layout::QS + rl * D + bb * QK + lg * 8);
            dqr[rt][bb] = ((const float *) (lds + lds_layout::QD))[rl * NBLK + bb];
        }
        mrow[rt] = rl >= RW ? -1 : (a.m_ne2 == 1 ? (r0 + rl) / a.gqa - t0 : rl);
    }

    // ---- online softmax state ----
    v4f   O[RT][NBLK][2];
    float m_run[RT], l_run[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.f;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) { O[rt][bb][0] = v4f{0, 0, 0, 0}; O[rt][bb][1] = v4f{0, 0, 0, 0}; }
    }

    const char * kbase = a.k + (size_t) (b % a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) (b % a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;
    const uint16_t * ms = (const uint16_t *) (lds + lds_layout::MS);
    const int wk = wave * KW;   // this wave's first key in a chunk
    int keyj[8];                // k-slot order: j<4 -> key 4g+j, j>=4 -> key 16+4g+j-4
#pragma unroll
    for (int jj = 0; jj < 8; jj++) keyj[jj] = wk + (jj >> 2) * 16 + lg * 4 + (jj & 3);
    const int aoff = 2 + 4 * (ln & 7) + (ln >> 3);   // V^T row m: dims 4(m%8) (+1 byte for m >= 8)

    for (int64_t c0 = k_lo; c0 < k_hi; c0 += CK) {
        __syncthreads();   // previous chunk (or Q staging) fully consumed
        // ---- stage raw K/V rows straight into LDS (keys past k_hi repeat the last key) ----
        for (int i = wave; i < CK * PIECES / 64; i += WAVES) {
            const int p = i * 64 + lane;
            const int key = p / PIECES, part = p - key * PIECES;
            const int64_t kk = std::min<int64_t>(c0 + key, k_hi - 1);
            __builtin_amdgcn_global_load_lds((const void *) (kbase + (size_t) kk * a.k_nb1 + part * 16),
                                             (lds_void *) (lds + lds_layout::KS + i * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void *) (vbase + (size_t) kk * a.v_nb1 + part * 16),
                                             (lds_void *) (lds + lds_layout::VS + i * 1024), 16, 0, 0);
        }
        // ---- stage mask values (F16 bits); keys past k_hi are -inf ----
        for (int e = threadIdx.x; e < n_mrows * CK; e += THREADS) {
            const int mr = e / CK, key = e - mr * CK;
            const int64_t kk = c0 + key;
            uint16_t mv = 0xFC00;   // -inf
            if (kk < k_hi) {
                if (a.mask) {
                    int t, hq;
                    if (a.m_ne2 == 1) { t = t0 + mr; hq = 0; }
                    else { const int r = r0 + mr; t = r / a.gqa; hq = (kvh * a.gqa + (r - t * a.gqa)) % a.m_ne2; }
                    mv = *(const uint16_t *) (a.mask + (size_t) t * a.m_nb1 + (size_t) hq * a.m_nb2 +
                                              (size_t) (b % a.m_ne3) * a.m_nb3 + (size_t) kk * 2);
                } else {
                    mv = 0;
                }
            }
            ((uint16_t *) (lds + lds_layout::MS))[mr * CK + key] = mv;
        }
        __builtin_amdgcn_s_waitcnt(0);   // LDS-DMA writes are counted by vmcnt
        __syncthreads();
        // ---- per-block scales, transposed to [block][key] ----
        for (int e = threadIdx.x; e < CK * NBLK; e += THREADS) {
            const int key = e >> 3, bb = e & 7;
            ((uint16_t *) (lds + lds_layout::KD))[bb * CK + key] = *(const uint16_t *) (lds + lds_layout::KS + key * SEG + bb * QBLOCK);
            ((uint16_t *) (lds + lds_layout::VD))[bb * CK + key] = *(const uint16_t *) (lds + lds_layout::VS + key * SEG + bb * QBLOCK);
        }
        __syncthreads();

        // ---- S = Q K^T for 2 tiles of 16 keys ----
        float s[RT][2][4];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            const int kr = wk + kt * 16 + ln;                 // A-operand key row
            const int k4 = wk + kt * 16 + lg * 4;             // output keys k4..k4+3
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) s[rt][kt][i] = 0.f;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                const long kA = (long) lds_u64(lds + lds_layout::KS + kr * SEG + bb * QBLOCK + 2 + lg * 8);
                const uint64_t dk4 = lds_u64(lds + lds_layout::KD + (bb * CK + k4) * 2);
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(kA, qB[rt][bb], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        s[rt][kt][i] = __builtin_fmaf((float) c[i], dqr[rt][bb] * h2f(dk4, i), s[rt][kt][i]);
                }
            }
        }

        // ---- mask, scale, online softmax (base 2) ----
        float p[RT][8];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            float sv[8];
            float mloc = -INFINITY;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {
                const float mv = mrow[rt] >= 0 ? dev::f16_bits_to_f32(ms[mrow[rt] * CK + keyj[jj]]) : -INFINITY;
                const float x = (mv == -INFINITY) ? -INFINITY : (s[rt][jj >> 2][jj & 3] * a.scale + mv) * LOG2E;
                sv[jj] = x;
                mloc = xmax(mloc, x);
            }
            mloc = xmax(mloc, __shfl_xor(mloc, 16));
            mloc = xmax(mloc, __shfl_xor(mloc, 32));
            const float m_new = xmax(m_run[rt], mloc);
            const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run[rt] - m_new);
            float lsum = 0.f;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {
                const float pv = (sv[jj] == -INFINITY) ? 0.f : exp2f(sv[jj] - m_new);
                p[rt][jj] = pv;
                lsum += pv;
            }
            l_run[rt] = l_run[rt] * alpha + lsum;
            m_run[rt] = m_new;
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[rt][bb][0] *= alpha; O[rt][bb][1] *= alpha; }
            }
        }

        // ---- O += V^T P (per V block: B = P * d_v) ----
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            uint32_t w[8];
#pragma unroll
            for (int jj = 0; jj < 8; jj++) w[jj] = lds_u32(lds + lds_layout::VS + keyj[jj] * SEG + bb * QBLOCK + aoff);
            uint32_t a0[4], a1[4];
#pragma unroll
            for (int q2 = 0; q2 < 4; q2++) {
                a0[q2] = cvt_i8x2_f16_b0(w[2 * q2], w[2 * q2 + 1]);
                a1[q2] = cvt_i8x2_f16_b2(w[2 * q2], w[2 * q2 + 1]);
            }
            const v8h A0 = __builtin_bit_cast(v8h, uint4{a0[0], a0[1], a0[2], a0[3]});
            const v8h A1 = __builtin_bit_cast(v8h, uint4{a1[0], a1[1], a1[2], a1[3]});
            const uint64_t dvlo = lds_u64(lds + lds_layout::VD + (bb * CK + keyj[0]) * 2);
            const uint64_t dvhi = lds_u64(lds + lds_layout::VD + (bb * CK + keyj[4]) * 2);
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                v8h Bp;
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    Bp[jj] = (_Float16) (p[rt][jj] * h2f(jj < 4 ? dvlo : dvhi, jj & 3));
                O[rt][bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bp, O[rt][bb][0], 0, 0, 0);
                O[rt][bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bp, O[rt][bb][1], 0, 0, 0);
            }
        }
    }

    // ---- merge the 4 waves' partial states in LDS (deterministic order) ----
    __syncthreads();   // staging area becomes the merge buffer
    float * ob = (float *) (lds + lds_layout::OB);
    float2 * ml = (float2 *) (lds + lds_layout::ML);
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        float l = l_run[rt];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        l_run[rt] = l;
        if (lg == 0) ml[wave * 32 + rt * 16 + ln] = make_float2(m_run[rt], l);
    }
    __syncthreads();
    float mw[RT], lw[RT], fw[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int rl = rt * 16 + ln;
        float M = -INFINITY;
        for (int w2 = 0; w2 < WAVES; w2++) M = xmax(M, ml[w2 * 32 + rl].x);
        float L = 0.f;
        for (int w2 = 0; w2 < WAVES; w2++) {
            const float2 e = ml[w2 * 32 + rl];
            L += (e.x == -INFINITY) ? 0.f : e.y * exp2f(e.x - M);
        }
        mw[rt] = M;
        lw[rt] = L;
        fw[rt] = (m_run[rt] == -INFINITY) ? 0.f : exp2f(m_run[rt] - M);
    }
    __syncthreads();   // every wave has read ml before row 0's (M, L) overwrite it below
    for (int w2 = 0; w2 < WAVES; w2++) {
        if (wave == w2) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int rl = rt * 16 + ln;
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++)
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        float4 * dstp = (float4 *) (ob + rl * D + bb * 32 + e * 16 + lg * 4);
                        const v4f val = O[rt][bb][e] * fw[rt];
                        if (w2 == 0) {
                            *dstp = make_float4(val[0], val[1], val[2], val[3]);
                        } else {
                            float4 cur = *dstp;
                            cur.x += val[0]; cur.y += val[1]; cur.z += val[2]; cur.w += val[3];
                            *dstp = cur;
                        }
                    }
            }
            if (w2 == 0 && lg == 0) {
#pragma unroll
                for (int rt = 0; rt < RT; rt++) ml[rt * 16 + ln] = make_float2(mw[rt], lw[rt]);
            }
        }
        __syncthreads();
    }

    // ---- write the block's result ----
    const size_t bh = (size_t) b * a.nh_kv + kvh;
    if (a.ns == 1) {
        // single split: normalised final output, dims restored
        for (int e = threadIdx.x; e < RW * D; e += THREADS) {
            const int rl = e / D, pos = e - rl * D;
            const int r = r0 + rl;
            const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
            const float L = ml[rl].y;
            const float o = L > 0.f ? ob[rl * D + pos] / L : 0.f;
            a.dst[(((size_t) b * a.T + t) * a.nh + h) * D + pos_to_dim(pos)] = o;
        }
    } else {
        float * po = a.part_o + ((bh * a.ns + split) * a.R + r0) * D;
        for (int e = threadIdx.x; e < RW * D / 4; e += THREADS)
            ((float4 *) po)[e] = ((const float4 *) ob)[e];
        for (int rl = threadIdx.x; rl < RW; rl += THREADS)
            a.part_ml[(bh * a.ns + split) * a.R + r0 + rl] = ml[rl];
    }
}

// One block per (b, kvh, r): LSE merge of the ns split partials.
__global__ __launch_bounds__(256) void k_fattn_merge(fa_args a) {
    const int row = blockIdx.x;                  // ((b * nh_kv + kvh) * R + r)
    const int r = row % a.R;
    const int bh = row / a.R;
    const int kvh = bh % a.nh_kv, b = bh / a.nh_kv;
    const float2 * ml = a.part_ml + (size_t) bh * a.ns * a.R + r;
    float M = -INFINITY;
    for (int s2 = 0; s2 < a.ns; s2++) M = xmax(M, ml[(size_t) s2 * a.R].x);
    float L = 0.f, acc = 0.f;
    const int pos = threadIdx.x;
    const float * po = a.part_o + ((size_t) bh * a.ns * a.R + r) * D + pos;
    for (int s2 = 0; s2 < a.ns; s2++) {
        const float2 e = ml[(size_t) s2 * a.R];
        if (e.x == -INFINITY) continue;
        const float f = exp2f(e.x - M);
        L += e.y * f;
        acc += po[(size_t) s2 * a.R * D] * f;
    }
    const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
    a.dst[(((size_t) b * a.T + t) * a.nh + h) * D + pos_to_dim(pos)] = L > 0.f ? acc / L : 0.f;
}

// Blocks use more than the default 64 KB of dynamic LDS (gfx950 has 160 KB).
template <int RT>
int launch_fa(int64_t grid, size_t shmem, hipStream_t st, const fa_args & a) {
    static bool attr_set = false;
    if (!attr_set) {
        QWFN_HIP_TRY(hipFuncSetAttribute((const void *) k_fattn_q8_0<RT>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds_layout::END));
        attr_set = true;
    }
    hipLaunchKernelGGL(k_fattn_q8_0<RT>, dim3((unsigned) grid), dim3(THREADS), shmem, st, a);
    return QWFN_OK;
}

// ---------------------------------------------------------------- planning

struct fa_plan {
    int32_t R, RT, gqa, rw, n_rg, ns, split_len, n_mrows;
    size_t  ws_bytes;
};

int env_int(const char * name, int dflt) {
    const char * s = std::getenv(name);
    return s && *s ? std::atoi(s) : dflt;
}

int plan_fattn(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v, const qwfn_tensor * mask,
               fa_plan * pl) {
    if (!q || !k || !v) return set_error(QWFN_EINVAL, "flash_attn_ext: NULL q/k/v");
    if (q->type != QWFN_TYPE_F32) return set_error(QWFN_EINVAL, "flash_attn_ext: q must be f32");
    if (k->type != QWFN_TYPE_Q8_0 || v->type != QWFN_TYPE_Q8_0)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: k and v must be q8_0");
    if (q->ne[0] != D || k->ne[0] != D || v->ne[0] != D)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: head size must be 256");
    if (q->nb[0] != 4 || k->nb[0] != QBLOCK || v->nb[0] != QBLOCK)
        return set_error(QWFN_EINVAL, "flash_attn_ext: q nb[0] must be 4, k/v nb[0] must be 34");
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2])
        return set_error(QWFN_EINVAL, "flash_attn_ext: k and v must have the same n_kv and n_head_kv");
    if (k->ne[2] <= 0 || q->ne[2] % k->ne[2])
        return set_error(QWFN_EINVAL, "flash_attn_ext: n_head must be a multiple of n_head_kv");
    if (k->ne[3] <= 0 || v->ne[3] <= 0 || q->ne[3] % k->ne[3] || q->ne[3] % v->ne[3])
        return set_error(QWFN_EINVAL, "flash_attn_ext: batch of q must be a multiple of the batch of k/v");
    const int64_t T = q->ne[1], nh = q->ne[2], nh_kv = k->ne[2];
    if (T <= 0 || nh <= 0 || q->ne[3] <= 0) return set_error(QWFN_EINVAL, "flash_attn_ext: empty q");
    const int64_t gqa = nh / nh_kv;
    const int64_t R = T * gqa;
    // 16-byte aligned rows and heads: the kernel stages K/V with 16-byte loads.
    if (!is_aligned(k->data, 16) || !is_aligned(v->data, 16) || k->nb[1] % 16 || k->nb[2] % 16 || k->nb[3] % 16 ||
        v->nb[1] % 16 || v->nb[2] % 16 || v->nb[3] % 16)
        return set_error(QWFN_EALIGN, "flash_attn_ext: k/v data and strides must be 16-byte aligned");
    if (!is_aligned(q->data, 16) || q->nb[1] % 16 || q->nb[2] % 16 || q->nb[3] % 16)
        return set_error(QWFN_EALIGN, "flash_attn_ext: q data and strides must be 16-byte aligned");
    int n_mrows = (int) T;
    if (mask) {
        if (!mask->data) return set_error(QWFN_EINVAL, "flash_attn_ext: mask has no data");
        if (mask->type != QWFN_TYPE_F16) return set_error(QWFN_EINVAL, "flash_attn_ext: mask must be f16");
        if (mask->nb[0] != 2) return set_error(QWFN_EINVAL, "flash_attn_ext: mask rows must be contiguous");
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < T)
            return set_error(QWFN_EINVAL, "flash_attn_ext: mask must be at least [n_kv, T]");
        if (mask->ne[2] <= 0 || nh % mask->ne[2] || mask->ne[3] <= 0 || q->ne[3] % mask->ne[3])
            return set_error(QWFN_EINVAL, "flash_attn_ext: mask must broadcast over heads and batch");
        if (!is_aligned(mask->data, 2)) return set_error(QWFN_EALIGN, "flash_attn_ext: mask must be 2-byte aligned");
        n_mrows = mask->ne[2] == 1 ? (int) T : (int) R;
    }
    // Query rows per block: up to 32 (two 16-row MFMA tiles); more rows are
    // split into row groups that read the same K/V (L2-shared on one XCD).
    int rw = (int) std::min<int64_t>(R, MAX_RW);
    if (const int force = env_int("QWFN_FA_ROWS", 0)) rw = std::max(1, std::min(rw, force));
    pl->R = (int32_t) R;
    pl->rw = rw;
    pl->n_rg = (int32_t) ((R + rw - 1) / rw);
    pl->RT = (rw + 15) / 16;
    pl->gqa = (int32_t) gqa;
    pl->n_mrows = (mask && mask->ne[2] != 1) ? rw : (int) std::min<int64_t>(T, (rw + gqa - 1) / gqa + 1);
    (void) n_mrows;
    const int64_t n_kv = k->ne[1];
    const int64_t B = q->ne[3];
    // Splits: enough blocks to cover the chip about twice, each at least one chunk.
    const int64_t target_blocks = env_int("QWFN_FA_BLOCKS", 512);
    int64_t ns = std::max<int64_t>(1, target_blocks / std::max<int64_t>(1, nh_kv * B * pl->n_rg));
    ns = std::min<int64_t>(ns, std::max<int64_t>(1, (n_kv + CK - 1) / CK));
    if (const int force = env_int("QWFN_FA_SPLITS", 0)) ns = force;
    int64_t split_len = (n_kv + ns - 1) / ns;
    split_len = std::max<int64_t>(CK, (split_len + CK - 1) / CK * CK);
    ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
    pl->ns = (int32_t) ns;
    pl->split_len = (int32_t) split_len;
    pl->ws_bytes = ns > 1 ? (size_t) (B * nh_kv * ns * R) * (D * sizeof(float) + sizeof(float2)) + 256 : 0;
    return QWFN_OK;
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" size_t qwfn_fattn_workspace_size(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v) {
    fa_plan pl{};
    if (plan_fattn(q, k, v, nullptr, &pl)) return 0;
    return pl.ws_bytes;
}

extern "C" int qwfn_flash_attn_ext_q8_0(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                        const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                        const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                        void * stream) {
    if (max_bias != 0.0f) return set_error(QWFN_ENOTSUP, "flash_attn_ext: max_bias (ALiBi) is not supported");
    if (logit_softcap != 0.0f) return set_error(QWFN_ENOTSUP, "flash_attn_ext: logit_softcap is not supported");
    if (!(std::isfinite(scale))) return set_error(QWFN_EINVAL, "flash_attn_ext: scale must be finite");
    if (variant != QWFN_Q8_REF && variant != QWFN_Q8_X86) return set_error(QWFN_EINVAL, "flash_attn_ext: unknown variant");
    fa_plan pl{};
    if (int rc = plan_fattn(q, k, v, mask, &pl)) return rc;
    if (!dst || !dst->data || dst->type != QWFN_TYPE_F32) return set_error(QWFN_EINVAL, "flash_attn_ext: dst must be f32");
    if (dst->ne[0] != D || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != q->ne[3])
        return set_error(QWFN_EINVAL, "flash_attn_ext: dst must be [256, n_head, T, B]");
    if (dst->nb[0] != 4 || dst->nb[1] != (size_t) D * 4 || dst->nb[2] != dst->nb[1] * (size_t) dst->ne[1] ||
        dst->nb[3] != dst->nb[2] * (size_t) dst->ne[2])
        return set_error(QWFN_EINVAL, "flash_attn_ext: dst must be contiguous");
    if (!is_aligned(dst->data, 4)) return set_error(QWFN_EALIGN, "flash_attn_ext: dst must be 4-byte aligned");
    if (pl.ns > 1) {
        if (ws) {
            if (ws_bytes < pl.ws_bytes) return set_error(QWFN_ENOMEM, "flash_attn_ext: workspace too small");
            if (!is_aligned(ws, 256)) return set_error(QWFN_EALIGN, "flash_attn_ext: workspace must be 256-byte aligned");
        } else if (int rc = library_workspace(pl.ws_bytes, &ws)) {
            return rc;
        }
    }
    const int64_t n_kv = k->ne[1];
    if (n_kv == 0) {
        QWFN_HIP_TRY(hipMemsetAsync(dst->data, 0, view_bytes(*dst), as_stream(stream)));
        return QWFN_OK;
    }

    fa_args a{};
    a.q = (const char *) q->data; a.q_nb1 = q->nb[1]; a.q_nb2 = q->nb[2]; a.q_nb3 = q->nb[3];
    a.k = (const char *) k->data; a.k_nb1 = k->nb[1]; a.k_nb2 = k->nb[2]; a.k_nb3 = k->nb[3];
    a.v = (const char *) v->data; a.v_nb1 = v->nb[1]; a.v_nb2 = v->nb[2]; a.v_nb3 = v->nb[3];
    if (mask) {
        a.mask = (const char *) mask->data; a.m_nb1 = mask->nb[1]; a.m_nb2 = mask->nb[2]; a.m_nb3 = mask->nb[3];
        a.m_ne2 = (int32_t) mask->ne[2]; a.m_ne3 = (int32_t) mask->ne[3];
    } else {
        a.mask = nullptr; a.m_ne2 = 1; a.m_ne3 = 1;
    }
    a.dst = (float *) dst->data;
    const size_t n_part = (size_t) q->ne[3] * k->ne[2] * pl.ns * pl.R;
    a.part_o = (float *) ws;
    a.part_ml = ws ? (float2 *) ((char *) ws + n_part * D * sizeof(float)) : nullptr;
    a.n_kv = n_kv;
    a.T = (int32_t) q->ne[1]; a.nh = (int32_t) q->ne[2]; a.nh_kv = (int32_t) k->ne[2];
    a.gqa = pl.gqa; a.R = pl.R; a.B = (int32_t) q->ne[3];
    a.kb = (int32_t) k->ne[3]; a.vb = (int32_t) v->ne[3];
    a.ns = pl.ns; a.split_len = pl.split_len; a.rw = pl.rw; a.n_rg = pl.n_rg;
    a.scale = scale; a.x86 = variant == QWFN_Q8_X86;

    const int64_t units = ((int64_t) a.B * a.ns + 7) / 8 * 8;
    const int64_t grid = units * a.nh_kv * a.n_rg;
    if (grid > 0x7fffffff) return set_error(QWFN_EINVAL, "flash_attn_ext: grid too large");
    hipStream_t st = as_stream(stream);
    const size_t shmem = (size_t) lds_layout::MS + (size_t) pl.n_mrows * CK * 2;
    if (pl.RT == 1) {
        if (int rc = launch_fa<1>(grid, shmem, st, a)) return rc;
    } else {
        if (int rc = launch_fa<2>(grid, shmem, st, a)) return rc;
    }
    if (int rc = hip_check(hipGetLastError(), "flash_attn launch")) return rc;
    if (a.ns > 1) {
        const int64_t rows = (int64_t) a.B * a.nh_kv * a.R;
        hipLaunchKernelGGL(k_fattn_merge, dim3((unsigned) rows), dim3(256), 0, st, a);
        if (int rc = hip_check(hipGetLastError(), "flash_attn merge launch")) return rc;
    }
    return QWFN_OK;
}
