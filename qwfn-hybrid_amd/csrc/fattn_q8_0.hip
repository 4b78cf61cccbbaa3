// Flash attention straight from the raw q8_0 KV cache, for decode, MTP verify
// and (through row groups) longer query blocks, on gfx950.
//
// Semantics: ggml_flash_attn_ext with q8_0 K/V and F32 accumulation, as the
// reference calls it at qwfn_graph.cpp:469-471 (dense / MTP head / QSA-off
// decode and verify) and :698-699 (QSA decode over gathered cells). The CPU
// one-chunk loop of ggml (the oracle) requantises Q to q8_0, takes
// s = sum_b d_k[b]*d_q[b]*isum_b, skips keys whose mask is -inf, runs an online
// softmax and accumulates dequantised V rows. This kernel keeps that arithmetic:
// Q is requantised with the same quantiser and the integer block dot products
// are exact (i8 MFMA); only the float accumulation order differs. P*d_v enters
// the f16 PV matrix cores as a hi + lo pair of f16 values (~22 bits).
//
// Work decomposition (flash-decoding):
//   grid   : (batch, KV head, row group, key split); the KV heads and row
//            groups of one split sit on the same XCD and are dispatched next to
//            each other, so the cache lines two heads share (a 272-byte head row
//            is not line aligned) come from one L2.
//   block  : RT 16-row query tiles x 2 key groups = 2*RT wavefronts. Keys are
//            streamed in 64-key chunks of raw 272-byte head rows with gfx950's
//            LDS DMA (global_load_lds_dwordx4) into a two-stage ring: chunk c+1
//            is in flight while chunk c is computed. Wave (tile t, group g) owns
//            query rows 16t..16t+15 and keys 32g..32g+31 of every chunk.
//   QK^T   : v_mfma_i32_16x16x64_i8 per q8_0 block. The A operand is four
//            16-byte aligned pieces of the raw K row that cover the block's 32
//            quants (a 64-byte window); the B operand is the requantised query
//            laid out on the same window, zero outside the block, so the integer
//            sum is exactly the block's dot product and no LDS read is ever
//            misaligned. The int32 tile is scaled by d_q*d_k.
//   softmax: online, base 2, per query row; row max across the 4 lane groups.
//   PV     : v_mfma_f32_16x16x32_f16, A = V^T (int8 -> f16 exact, SDWA byte
//            select from naturally aligned 2-byte LDS reads), B = P*d_v of one V
//            block as f16 hi + lo.
//   merge  : the two key groups merge in LDS; key splits merge in a second
//            kernel (log-sum-exp weights).
#include "q8_device.h"
#include "qwfn_common.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace qwfn {
namespace {

typedef int      v4i __attribute__((ext_vector_type(4)));
typedef float    v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2  __attribute__((ext_vector_type(2)));
typedef uint16_t us2 __attribute__((ext_vector_type(2)));

constexpr int D      = 256;            // head size (values per head row)
constexpr int NBLK   = D / QK;         // 8 q8_0 blocks per head row
constexpr int SEG    = NBLK * QBLOCK;  // 272 bytes per head row
constexpr int KW     = 16;             // keys per wave per chunk (one QK tile, one PV MFMA depth)
constexpr int KG     = 4;              // key groups = waves of a block
constexpr int CK     = KG * KW;        // keys per chunk
constexpr int CHUNK_BYTES = CK * SEG;  // one tensor's rows of a chunk (17408)
constexpr int DMA_PER_TENSOR = CHUNK_BYTES / 1024;   // wave-wide 16-byte LDS-DMA loads per tensor (17)
constexpr int MASK_ROWS = 16;          // mask rows a block streams with each chunk
constexpr int MASK_BYTES = MASK_ROWS * CK * 2;       // a chunk's mask slice in LDS (2048)
constexpr int STAGE_BYTES = 2 * CHUNK_BYTES + MASK_BYTES;   // one ring stage: K rows, V rows, mask slice
constexpr int DMA_SLOTS = 2 * DMA_PER_TENSOR + MASK_BYTES / 1024;   // wave-wide DMAs per chunk (36)
constexpr int QROWS_IMG = 32;          // d_q rows per row group in the query image (one 1 KB DMA)
constexpr int QWIN   = 64;             // bytes of one block's query window
constexpr int MAX_SPLITS = 1024;       // key splits per (batch, KV head, row group)
constexpr float LOG2E = 1.4426950408889634f;
static_assert(CHUNK_BYTES % 1024 == 0, "a chunk is whole wave-wide DMA instructions");

// First 16-byte piece of the 64-byte window of block b inside a 272-byte head
// row. Block b's quants occupy bytes [34b+2, 34b+34); the window
// [16*w(b), 16*w(b)+64) contains them and stays inside the row.
__host__ __device__ constexpr int win_piece(int b) { return b == 0 ? 0 : b == 1 ? 1 : b == 7 ? 13 : 2 * b; }
// Window byte of quant 0 of block b.
__host__ __device__ constexpr int win_off(int b) { return QBLOCK * b + 2 - 16 * win_piece(b); }
static_assert(win_off(0) >= 0 && win_off(7) + QK <= QWIN, "windows cover the blocks");

struct fa_args {
    const char * q;  size_t q_nb1, q_nb2, q_nb3;
    const char * k;  size_t k_nb1, k_nb2, k_nb3;
    const char * v;  size_t v_nb1, v_nb2, v_nb3;
    const char * mask; size_t m_nb1, m_nb2, m_nb3;
    int32_t m_ne2, m_ne3;
    float *  dst;          // [D, nh, T, B]
    float *  part_o;       // [B][nh_kv][ns][R][D]
    float2 * part_ml;      // [B][nh_kv][ns][R]: (running max in log2 units, sum)
    uint4 *  qimg;         // [B][nh_kv][n_rg][RT][64 lanes][NBLK]: lane's 16-byte query window slices
    float *  dqimg;        // [B][nh_kv][n_rg][32 rows][NBLK]: d_q * scale * log2(e)
    uint16_t * mimg;       // [m_ne3][m_ne2][T][n_kv_pad] F16 mask copy, -inf past n_kv (or null)
    int64_t  n_kv;
    int64_t  n_kv_pad;     // n_kv rounded up to a chunk
    int32_t  T, nh, nh_kv, gqa, R, B;
    int32_t  kb, vb;       // K/V batch extents (ne[3]); batch b reads b % kb
    int32_t  ns;           // key splits
    int32_t  split_len;    // keys per split, multiple of CK
    int32_t  rw;           // query rows per block (16 * RT)
    int32_t  n_rg;         // row groups per KV head
    float    scale;
    int32_t  x86;
    int32_t  dst_vec;      // dst is 16-byte aligned: float4 stores
};

// The compiler's hazard recognizer does not see the VALU writes inside inline
// asm, and an MFMA that reads a VGPR needs two wait states after a VALU wrote
// it. Every asm below whose result can feed an MFMA operand therefore ends
// with s_nop 1.

// One V block's A operands for the lane's 4 keys: w[q] holds dims 2m, 2m+1
// of keys 2q (bytes 0-1) and 2q+1 (bytes 2-3); a0[q] = f16 pair (dim 2m of
// both keys), a1[q] = f16 pair (dim 2m+1). int8 -> f16 is exact.
__device__ __forceinline__ void cvt_v_block(const uint32_t w[2], uint32_t a0[2], uint32_t a1[2]) {
#define QWFN_SDWA(D, S, DSEL, UNUSED, SSEL) "v_cvt_f16_i16_sdwa " D ", sext(" S ") dst_sel:" DSEL " dst_unused:" UNUSED " src0_sel:" SSEL "\n\t"
#define QWFN_PAIR(D, S, B0, B1) QWFN_SDWA(D, S, "WORD_0", "UNUSED_PAD", B0) QWFN_SDWA(D, S, "WORD_1", "UNUSED_PRESERVE", B1)
    asm volatile(QWFN_PAIR("%0", "%4", "BYTE_0", "BYTE_2") QWFN_PAIR("%1", "%5", "BYTE_0", "BYTE_2")
                 QWFN_PAIR("%2", "%4", "BYTE_1", "BYTE_3") QWFN_PAIR("%3", "%5", "BYTE_1", "BYTE_3")
                 "s_nop 1"
                 : "=&v"(a0[0]), "=&v"(a0[1]), "=&v"(a1[0]), "=&v"(a1[1])
                 : "v"(w[0]), "v"(w[1]));
#undef QWFN_PAIR
#undef QWFN_SDWA
}

// B operands of one V block: for key pairs q (keys 2q, 2q+1), P*d_v as an f16
// hi pair, bh[q] = f16(p*d_v) (RNE), and a lo pair, bl[q] = f16(p*d_v - hi),
// each from one fused v_fma_mix (the product is exact before its rounding).
// dv[q] holds the two keys' fp16 d_v.
__device__ __forceinline__ void pdv_hilo(const float p[4], const uint32_t dv[2], uint32_t bh[2], uint32_t bl[2]) {
#define QWFN_HILO(H, L, P0, P1, DV)                                                                   \
    "v_fma_mixlo_f16 " H ", " P0 ", " DV ", 0 op_sel:[0,0,0] op_sel_hi:[0,1,0]\n\t"                     \
    "v_fma_mixhi_f16 " H ", " P1 ", " DV ", 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"                     \
    "v_fma_mixlo_f16 " L ", " P0 ", " DV ", -" H " op_sel:[0,0,0] op_sel_hi:[0,1,1]\n\t"                \
    "v_fma_mixhi_f16 " L ", " P1 ", " DV ", -" H " op_sel:[0,1,1] op_sel_hi:[0,1,1]\n\t"
    asm volatile(QWFN_HILO("%0", "%2", "%4", "%5", "%8") QWFN_HILO("%1", "%3", "%6", "%7", "%9")
                 "s_nop 1"
                 : "=&v"(bh[0]), "=&v"(bh[1]), "=&v"(bl[0]), "=&v"(bl[1])
                 : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(dv[0]), "v"(dv[1]));
#undef QWFN_HILO
}

// x * f16 (low or high half of a packed dword), one v_fma_mix_f32.
__device__ __forceinline__ float mul_f16lo(float x, uint32_t h) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,0,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(h));
    return r;
}
__device__ __forceinline__ float mul_f16hi(float x, uint32_t h) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(h));
    return r;
}
// x + f16 * c (f16 in the low or high half of a packed dword), one v_fma_mix_f32.
__device__ __forceinline__ float fma_f16lo(uint32_t h, float c, float x) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(c), "v"(x));
    return r;
}
__device__ __forceinline__ float fma_f16hi(uint32_t h, float c, float x) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(c), "v"(x));
    return r;
}
__device__ __forceinline__ float xmax(float a, float b) { return a > b ? a : b; }

// Reductions over the 4 lanes l, l^16, l^32, l^48 (the four lane groups
// holding one MFMA column), with gfx950's cross-row swaps instead of LDS
// permutes: a swap pair holds lanes l and l^16 (or l^32) between its two
// results. The two results pass through an empty asm: without it the
// compiler's IR folds the second result into the first (r[0] op r[1] becomes
// r[0] op r[0]), which silently turns the reduction into x op x.
template <typename Op>
__device__ __forceinline__ float reduce_lanes16_32(float x, Op op) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    unsigned a = r16[0], b = r16[1];
    asm volatile("" : "+v"(a), "+v"(b));
    x = op(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    const unsigned w = __builtin_bit_cast(unsigned, x);
    const auto r32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    unsigned c = r32[0], d = r32[1];
    asm volatile("" : "+v"(c), "+v"(d));
    return op(__builtin_bit_cast(float, c), __builtin_bit_cast(float, d));
}
__device__ __forceinline__ float xmax_lanes16_32(float x) {
    return reduce_lanes16_32(x, [](float a, float b) { return xmax(a, b); });
}
__device__ __forceinline__ float sum_lanes16_32(float x) {
    return reduce_lanes16_32(x, [](float a, float b) { return a + b; });
}

// s_waitcnt that waits for vmcnt <= n only (gfx9 encoding: vmcnt[3:0] in
// bits 3:0, vmcnt[5:4] in bits 15:14, expcnt and lgkmcnt left at their max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// One wave-wide LDS-DMA load: each lane copies 16 bytes from gptr to
// LDS[lds_base + 16 * lane]; lds_base is wave-uniform. Issued as inline asm:
// the compiler neither reorders memory operations across it nor tracks it, and
// the kernel waits for it explicitly (vmcnt) before the barrier that publishes
// the data. No other vector-memory load is in flight while DMAs are, so the
// explicit counts are exact.
__device__ __forceinline__ void dma16(const void * gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\t"
                 "global_load_lds_dwordx4 %0, off"
                 :: "v"(gptr), "s"(lds_base) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void * p) {
    return (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) void *) p;
}

// LDS writes of this wave become visible to its other lanes (LDS operations of
// one wave complete in order; the fences keep the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row of the mask copy that staged row mr of a block reads: query position
// t0 + mr for a shared mask, query row r0 + mr for a per-head mask.
__device__ __forceinline__ int64_t mask_img_row(const fa_args & a, int mr, int t0, int r0, int kvh, int b) {
    int t, hq;
    if (a.m_ne2 == 1) { t = t0 + mr; hq = 0; }
    else { const int r = r0 + mr; t = r / a.gqa; hq = (kvh * a.gqa + (r - t * a.gqa)) % a.m_ne2; }
    return ((int64_t) (b % a.m_ne3) * a.m_ne2 + hq) * a.T + t;
}

// f[0 .. n) = 0 (dst is only 4-byte aligned, so plain f32 stores).
__global__ void k_zero_f32(float * f, int64_t n) {
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) f[i] = 0.f;
}

// Per-call preparation shared by every key split:
//  * blocks [0, n_qblocks): one (batch, KV head, row group) each. The query
//    rows are requantised to q8_0 (ggml-cpu's quantiser, `x86` variant) and
//    each q8_0 block is laid out on its 64-byte window (zero outside the
//    block); the result is stored in the order the attention lanes load it as
//    MFMA B operands, with d_q * scale * log2(e) beside it.
//  * blocks past that: the F16 mask rows [0, T) of every (head, batch) slice
//    are copied to a 16-byte aligned image padded with -inf up to n_kv_pad, so
//    the attention kernel can stream each chunk's slice with the K/V DMA.
template <int RT>
__global__ __launch_bounds__(256) void k_fattn_prep(fa_args a, int n_qblocks) {
    constexpr int ROWS = 16 * RT;
    if ((int) blockIdx.x >= n_qblocks) {
        if (!a.mask) return;
        const int64_t rows = (int64_t) a.m_ne3 * a.m_ne2 * a.T;
        const int64_t units = rows * (a.n_kv_pad / 8);            // 8 keys (16 bytes) per unit
        const int64_t stride = (int64_t) (gridDim.x - n_qblocks) * 256;
        for (int64_t e = (int64_t) (blockIdx.x - n_qblocks) * 256 + threadIdx.x; e < units; e += stride) {
            const int64_t row = e / (a.n_kv_pad / 8);
            const int64_t k0 = (e - row * (a.n_kv_pad / 8)) * 8;
            const int t = (int) (row % a.T);
            const int64_t hs = row / a.T;
            const int hq = (int) (hs % a.m_ne2), bm = (int) (hs / a.m_ne2);
            const uint16_t * src = (const uint16_t *) (a.mask + (size_t) t * a.m_nb1 + (size_t) hq * a.m_nb2 + (size_t) bm * a.m_nb3);
            uint16_t v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = k0 + i < a.n_kv ? src[k0 + i] : (uint16_t) 0xFC00;
            uint4 w;
            w.x = v[0] | ((uint32_t) v[1] << 16); w.y = v[2] | ((uint32_t) v[3] << 16);
            w.z = v[4] | ((uint32_t) v[5] << 16); w.w = v[6] | ((uint32_t) v[7] << 16);
            *(uint4 *) (a.mimg + row * a.n_kv_pad + k0) = w;
        }
        return;
    }
    __shared__ __attribute__((aligned(16))) uint8_t qwin[ROWS * NBLK * QWIN];
    const int bkr = blockIdx.x;                    // (b * nh_kv + kvh) * n_rg + rg
    const int rg = bkr % a.n_rg, kvh = (bkr / a.n_rg) % a.nh_kv, b = bkr / (a.n_rg * a.nh_kv);
    const int r0 = rg * a.rw;
    const int RW = min(a.rw, a.R - r0);
    for (int e = threadIdx.x; e < ROWS * NBLK * QWIN / 16; e += 256) ((uint4 *) qwin)[e] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane & 7, blk = lane >> 3;
    const float fs = a.scale * LOG2E;
    for (int rl = wave; rl < ROWS; rl += 4) {
        const int r = r0 + min(rl, RW - 1);
        const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
        float4 v4 = *(const float4 *) (a.q + (size_t) t * a.q_nb1 + (size_t) h * a.q_nb2 + (size_t) b * a.q_nb3 +
                                       (size_t) (blk * QK + sub * 4) * 4);
        if (rl >= RW) v4 = make_float4(0.f, 0.f, 0.f, 0.f);
        const float x[4] = {v4.x, v4.y, v4.z, v4.w};
        uint16_t d16;
        float dq;
        const uint32_t w = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dq);
        uint16_t * wp = (uint16_t *) (qwin + (rl * NBLK + blk) * QWIN + win_off(blk) + 4 * sub);
        wp[0] = (uint16_t) w;
        wp[1] = (uint16_t) (w >> 16);
        if (sub == 0) a.dqimg[((size_t) bkr * QROWS_IMG + rl) * NBLK + blk] = dq * fs;
    }
    __syncthreads();
    // lane (ln, lg) of row tile `tile` reads slice lg of row 16*tile + ln's window, per block
    for (int e = threadIdx.x; e < RT * 64 * NBLK; e += 256) {
        const int tile = e / (64 * NBLK), ln_ = (e / NBLK) & 63, bb = e % NBLK;
        const int row = tile * 16 + (ln_ & 15), lg_ = ln_ >> 4;
        a.qimg[(size_t) bkr * RT * 64 * NBLK + e] = *(const uint4 *) (qwin + (row * NBLK + bb) * QWIN + 16 * lg_);
    }
}

// 16-byte global load into registers, issued as inline asm so that its
// completion is tracked by the kernel's own vmcnt waits (like the LDS DMAs)
// rather than by compiler-inserted ones.
__device__ __forceinline__ v4i gload16_asm(const void * p) {
    v4i r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}

template <int RT>
__global__ __launch_bounds__(KG * 64)
void k_fattn_q8_0(fa_args a) {
    constexpr int WAVES = KG;
    constexpr int ROWS = 16 * RT;
    constexpr int DPW = DMA_SLOTS / WAVES;         // DMAs per wave per chunk
    static_assert(DMA_SLOTS % WAVES == 0, "every wave issues the same number of DMAs");
    // two ring stages, each K rows [CK][272], V rows [CK][272], mask [MASK_ROWS][CK] F16
    __shared__ __attribute__((aligned(16))) uint8_t ring[2][STAGE_BYTES];
    // per-wave scale tables of the current chunk: [K|V][block][key of the wave] fp16
    __shared__ __attribute__((aligned(16))) uint16_t scl[WAVES][2][NBLK][KW];
    __shared__ __attribute__((aligned(16))) float dql[QROWS_IMG][NBLK];     // d_q * scale * log2(e) per row and block
    static_assert(ROWS * D * 4 + WAVES * ROWS * 8 <= STAGE_BYTES, "merge buffer fits in stage 0");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
    const int ln = lane & 15;       // MFMA row/col within a 16-tile
    const int lg = lane >> 4;       // lane group (k-slice / output row quad)
    const int kgrp = wave;          // key group: keys 16*kgrp .. 16*kgrp+15 of every chunk

    // ---- block -> (b, kvh, row group, split) ----
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
    const int n_chunks = (int) ((k_hi - k_lo + CK - 1) / CK);
    const int r0 = rg * a.rw;                          // first query row of this block
    const int RW = std::min(a.rw, a.R - r0);          // rows in this block
    const int t0 = r0 / a.gqa;
    const int n_mrows = a.m_ne2 == 1 ? (r0 + RW - 1) / a.gqa - t0 + 1 : RW;   // <= MASK_ROWS (planned)
    const int bkr = (b * a.nh_kv + kvh) * a.n_rg + rg;

    const char * kbase = a.k + (size_t) (b % a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) (b % a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;

    // Issue part of chunk c into stage dstb: the chunk is DMA_SLOTS wave-wide
    // 16-byte DMAs, DPW per wave, issued as slots [n0, n1) of the wave. Wave w
    // issues slots w, w + WAVES, ...: slots 0-16 are K pieces, 17-33 V pieces
    // (piece p = 64*i + lane of a tensor's chunk is byte 16*(p % 17) of key
    // p / 17; keys past the split are loaded and masked while they exist, past
    // n_kv they repeat the last key), 34-35 the chunk's mask slice, rows 0-7 and
    // 8-15. Only a wave's last slot can be a mask slot; without a mask it
    // repeats the wave's first piece.
    static_assert((DPW - 1) * WAVES + WAVES - 1 < DMA_SLOTS && (DPW - 1) * WAVES <= 2 * DMA_PER_TENSOR,
                  "the mask slots are the last slot of some waves");
    auto issue_part = [&](int c, uint8_t * dstb, auto n0c, auto n1c) __attribute__((always_inline)) {
        constexpr int n0 = decltype(n0c)::value, n1 = decltype(n1c)::value;
        const int64_t c0 = k_lo + (int64_t) c * CK;
        const bool clamp = c0 + CK > a.n_kv;   // the cache's last chunk: no rows past n_kv
        const int last = (int) std::min<int64_t>(CK - 1, a.n_kv - 1 - c0);
        int ln_o = lane;
        asm volatile("" : "+v"(ln_o));          // recomputed per chunk: no hoisted per-piece addresses
        const char * kc0 = kbase + (size_t) c0 * a.k_nb1;
        const char * vc0 = vbase + (size_t) c0 * a.v_nb1;
        auto kv_piece = [&](int i) __attribute__((always_inline)) {
            const int tensor = i >= DMA_PER_TENSOR;
            const int ii = i - tensor * DMA_PER_TENSOR;
            const unsigned p = (unsigned) (ii * 64) + (unsigned) ln_o;      // < 1088
            // p / 17 and p % 17 with full-rate 24-bit multiplies: (p * 3856) >> 16
            // is exact for p < 1088
            unsigned key = __umul24(p, 3856u) >> 16;
            const unsigned part = p - __umul24(key, 17u);
            if (clamp) key = std::min(key, (unsigned) last);
            // row strides are < 2^24 (checked on the host): 24-bit multiplies suffice
            const char * src = (tensor ? vc0 + __umul24(key, (unsigned) a.v_nb1) : kc0 + __umul24(key, (unsigned) a.k_nb1)) + part * 16;
            dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(dstb + tensor * CHUNK_BYTES + ii * 1024)));
        };
#pragma unroll
        for (int n = n0; n < (n1 < DPW - 1 ? n1 : DPW - 1); n++) kv_piece(wave + n * WAVES);
        if constexpr (n1 < DPW) return;
        const int il = wave + (DPW - 1) * WAVES;
        if (il < 2 * DMA_PER_TENSOR) {
            kv_piece(il);
        } else if (a.mask) {
            const int m = il - 2 * DMA_PER_TENSOR;
            const int mr = std::min(m * 8 + (ln_o >> 3), n_mrows - 1);
            const uint16_t * src = a.mimg + mask_img_row(a, mr, t0, r0, kvh, b) * a.n_kv_pad + c0 + (ln_o & 7) * 8;
            dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(dstb + 2 * CHUNK_BYTES + m * 1024)));
        } else {
            kv_piece(wave);
        }
    };

    // ---- prologue: the lane's query operands (prepared once per call) and
    //      chunk 0, one wait for both. Chunk c+1 is then issued during chunk c's
    //      compute, in three parts, so the DMA queue drains while the wave works ----
    v4i qw[RT][NBLK];                                   // B operands of QK: window slice lg of each block, per row tile
    {
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const uint4 * qp = a.qimg + ((size_t) bkr * RT * 64 + t * 64 + lane) * NBLK;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) qw[t][bb] = gload16_asm(qp + bb);
        }
        if (wave == 0) dma16(a.dqimg + (size_t) bkr * QROWS_IMG * NBLK + lane * 4, __builtin_amdgcn_readfirstlane(lds_addr(&dql[0][0])));
    }
    issue_part(0, ring[0], std::integral_constant<int, 0>{}, std::integral_constant<int, DPW>{});
    wait_vmcnt<0>();
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) asm volatile("" : "+v"(qw[t][bb]));   // loaded: usable from here on
    // the lane's query row in tile t is 16t + ln; padded rows (>= RW) read mask
    // row 0 and are never stored
    int mrow[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const int rl = t * 16 + ln;
        mrow[t] = rl >= RW ? 0 : (a.m_ne2 == 1 ? (r0 + rl) / a.gqa - t0 : rl);
    }

    // ---- online softmax state per row tile ----
    v4f   O[RT][NBLK][2];
    float m_run[RT], l_run[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        m_run[t] = -INFINITY;
        l_run[t] = 0.f;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) { O[t][bb][0] = v4f{0, 0, 0, 0}; O[t][bb][1] = v4f{0, 0, 0, 0}; }
    }

    const int wk = kgrp * KW;   // this wave's first key in a chunk
    const int span = (int) (k_hi - k_lo);                       // keys of this split (<= split_len)
    uint16_t (*sw)[NBLK][KW] = scl[wave];

    // One chunk: `cur` holds chunk c; chunk c+1 goes to `nxt`. Called with the
    // ring stages literally so the compiler can tell them apart.
    constexpr int P1 = DPW / 3, P2 = 2 * DPW / 3;
    auto chunk_step = [&](int c, uint8_t * cur, uint8_t * nxt) __attribute__((always_inline)) {
        // chunk c was the last thing issued (during step c-1): wait for all of
        // it; the barrier publishes it and also tells every wave that `nxt`
        // (chunk c-1's stage) is no longer read
        wait_vmcnt<0>();
        __syncthreads();
        const bool more = c + 1 < n_chunks;
        const uint8_t * ks = cur;
        const uint8_t * vs = cur + CHUNK_BYTES;
        // this wave's keys' block scales, transposed to [block][key] (all reads
        // issued before the writes: the two LDS arrays could alias as far as the
        // compiler knows, so interleaving would serialise them)
        {
            // entry n of this lane: tensor n / 2, key (n % 2) * 8 + lane / 8, block lane % 8
            const uint8_t * src = cur + (wk + (lane >> 3)) * SEG + (lane & 7) * QBLOCK;
            uint16_t * dstw = &sw[0][lane & 7][lane >> 3];
            uint16_t sv[4];
#pragma unroll
            for (int n = 0; n < 4; n++) sv[n] = *(const uint16_t *) (src + (n >> 1) * CHUNK_BYTES + (n & 1) * 8 * SEG);
#pragma unroll
            for (int n = 0; n < 4; n++) dstw[(n >> 1) * NBLK * KW + (n & 1) * 8] = sv[n];
        }
        wave_lds_sync();
        if (more) issue_part(c + 1, nxt, std::integral_constant<int, 0>{}, std::integral_constant<int, P1>{});

        // ---- S = Q K^T: one 16-key tile (the MFMA rows) x RT row tiles ----
        float s[RT][4];
        {
            const uint8_t * krow = ks + (wk + ln) * SEG + 16 * lg;   // A operand: key row ln, slice lg
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) s[t][i] = 0.f;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                const v4i kA = *(const v4i *) (krow + 16 * win_piece(bb));
                const uint2 dk = *(const uint2 *) &sw[0][bb][lg * 4];   // the lane's 4 keys' fp16 d_k
#pragma unroll
                for (int t = 0; t < RT; t++) {
                    const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA, qw[t][bb], v4i{0, 0, 0, 0}, 0, 0, 0);
                    const float dq = dql[t * 16 + ln][bb];
                    s[t][0] = __builtin_fmaf((float) cc[0], mul_f16lo(dq, dk.x), s[t][0]);
                    s[t][1] = __builtin_fmaf((float) cc[1], mul_f16hi(dq, dk.x), s[t][1]);
                    s[t][2] = __builtin_fmaf((float) cc[2], mul_f16lo(dq, dk.y), s[t][2]);
                    s[t][3] = __builtin_fmaf((float) cc[3], mul_f16hi(dq, dk.y), s[t][3]);
                }
            }
        }
        if (more) issue_part(c + 1, nxt, std::integral_constant<int, P1>{}, std::integral_constant<int, P2>{});

        // ---- mask, online softmax (base 2; scores are already in log2 units).
        //      A masked key has x = -inf, so its p is exp2(-inf) = 0 ----
        float p[RT][4];
        const int kin = c * CK + wk + lg * 4;                     // first of the lane's 4 keys in the split
        const bool tail = (c + 1) * CK > span;                     // keys past the split in this chunk
#pragma unroll
        for (int t = 0; t < RT; t++) {
            uint2 mv = make_uint2(0, 0);
            if (a.mask) mv = *(const uint2 *) (cur + 2 * CHUNK_BYTES + (mrow[t] * CK + wk + lg * 4) * 2);
            float x[4];
            float mloc = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t mh = i < 2 ? mv.x : mv.y;
                float xi = (i & 1) ? fma_f16hi(mh, LOG2E, s[t][i]) : fma_f16lo(mh, LOG2E, s[t][i]);
                if (tail && kin + i >= span) xi = -INFINITY;
                x[i] = xi;
                mloc = xmax(mloc, xi);
            }
            mloc = xmax_lanes16_32(mloc);
            const float m_new = xmax(m_run[t], mloc);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;   // all keys masked so far
            const float alpha = __builtin_amdgcn_exp2f(m_run[t] - m_use);
            float lsum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[t][i] = __builtin_amdgcn_exp2f(x[i] - m_use);
                lsum += p[t][i];
            }
            l_run[t] = l_run[t] * alpha + lsum;
            m_run[t] = m_new;
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[t][bb][0] *= alpha; O[t][bb][1] *= alpha; }
            }
        }
        if (more) issue_part(c + 1, nxt, std::integral_constant<int, P2>{}, std::integral_constant<int, DPW>{});

        // ---- O += V^T P per V block. Tile e of block bb holds dims 32bb + 2m + e
        //      (m = MFMA row); the A operand of lane (m, g) is dims 2m, 2m+1 of the
        //      lane's 4 keys (4g..4g+3 of the wave's 16), one naturally aligned
        //      2-byte LDS read per key, shared by every row tile ----
        const uint8_t * vrow = vs + (wk + lg * 4) * SEG + 2 + 2 * ln;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            // keys 2q and 2q+1 share a register: dims 2m, 2m+1 of key 2q in bytes 0-1,
            // of key 2q+1 in bytes 2-3
            uint32_t w[2];
#pragma unroll
            for (int q2 = 0; q2 < 2; q2++) {
                const uint8_t * r0p = vrow + (2 * q2) * SEG + bb * QBLOCK;
                us2 tv;
                tv.x = *(const uint16_t *) r0p;
                tv.y = *(const uint16_t *) (r0p + SEG);
                w[q2] = __builtin_bit_cast(uint32_t, tv);
            }
            const uint2 dv2 = *(const uint2 *) &sw[1][bb][lg * 4];
            const uint32_t dv[2] = {dv2.x, dv2.y};
            uint32_t a0[2], a1[2];
            cvt_v_block(w, a0, a1);
            const v4h A0 = __builtin_bit_cast(v4h, make_uint2(a0[0], a0[1]));
            const v4h A1 = __builtin_bit_cast(v4h, make_uint2(a1[0], a1[1]));
#pragma unroll
            for (int t = 0; t < RT; t++) {
                uint32_t bh[2], bl[2];
                pdv_hilo(p[t], dv, bh, bl);
                const v4h Bh = __builtin_bit_cast(v4h, make_uint2(bh[0], bh[1]));
                const v4h Bl = __builtin_bit_cast(v4h, make_uint2(bl[0], bl[1]));
                O[t][bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bh, O[t][bb][0], 0, 0, 0);
                O[t][bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bh, O[t][bb][1], 0, 0, 0);
                O[t][bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bl, O[t][bb][0], 0, 0, 0);
                O[t][bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bl, O[t][bb][1], 0, 0, 0);
            }
        }
    };
    for (int c = 0; c < n_chunks; c += 2) {
        chunk_step(c, ring[0], ring[1]);
        if (c + 1 < n_chunks) chunk_step(c + 1, ring[1], ring[0]);
    }
    __syncthreads();   // every wave is done with the last chunk: stage 0 becomes the merge buffer

    // ---- merge the 4 key groups in LDS: each wave publishes (max, sum) per row,
    //      then adds its weighted O into the buffer in turn; wave 0 adds last and
    //      writes the block's result ----
    float * ob = (float *) ring[0];                                // [ROWS][256] f32, natural dim order
    float2 * ml = (float2 *) (ring[0] + ROWS * D * 4);             // [WAVES][ROWS]
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const float l = sum_lanes16_32(l_run[t]);
        if (lg == 0) ml[wave * ROWS + t * 16 + ln] = make_float2(m_run[t], l);
    }
    __syncthreads();
    float M[RT], L[RT], fw[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        float mx = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) mx = xmax(mx, ml[w2 * ROWS + t * 16 + ln].x);
        float ls = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; w2++) {
            const float2 e = ml[w2 * ROWS + t * 16 + ln];
            ls += e.x == -INFINITY ? 0.f : e.y * exp2f(e.x - mx);
        }
        M[t] = mx;
        L[t] = ls;
        fw[t] = (m_run[t] == -INFINITY) ? 0.f : exp2f(m_run[t] - mx);
    }
    // Lane (ln, lg) holds, for row tile t and block bb, dims 32bb + 8lg + 2i + e
    // of row 16t + ln in O[t][bb][e][i]. Lane indices are re-derived here (an
    // opaque copy of the thread id), so no output address stays live through
    // the key loop.
    int tid_e = (int) threadIdx.x;
    asm volatile("" : "+v"(tid_e));
    const int ln_e = tid_e & 15, lg_e = (tid_e >> 4) & 3;
    for (int w2 = WAVES - 1; w2 >= 1; w2--) {
        if (wave == w2) {
#pragma unroll
            for (int t = 0; t < RT; t++) {
                float * orow = ob + (t * 16 + ln_e) * D + 8 * lg_e;
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) {
                    const v4f o0 = O[t][bb][0] * fw[t], o1 = O[t][bb][1] * fw[t];
                    float4 * d0 = (float4 *) (orow + 32 * bb);
                    float4 * d1 = (float4 *) (orow + 32 * bb + 4);
                    if (w2 == WAVES - 1) {
                        *d0 = make_float4(o0[0], o1[0], o0[1], o1[1]);
                        *d1 = make_float4(o0[2], o1[2], o0[3], o1[3]);
                    } else {
                        float4 x0 = *d0, x1 = *d1;
                        x0.x += o0[0]; x0.y += o1[0]; x0.z += o0[1]; x0.w += o1[1];
                        x1.x += o0[2]; x1.y += o1[2]; x1.z += o0[3]; x1.w += o1[3];
                        *d0 = x0;
                        *d1 = x1;
                    }
                }
            }
        }
        __syncthreads();
    }
    if (wave != 0) return;
    const size_t bh = (size_t) b * a.nh_kv + kvh;
    const bool vec = a.ns > 1 || a.dst_vec;
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const int rl = t * 16 + ln_e;
        if (rl >= RW) continue;
        const int r = r0 + rl;
        const int tq = r / a.gqa, h = kvh * a.gqa + (r - tq * a.gqa);
        float * out;
        float oscale;
        if (a.ns == 1) {
            out = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + 8 * lg_e;
            oscale = L[t] > 0.f ? 1.f / L[t] : 0.f;
        } else {
            out = a.part_o + ((bh * a.ns + split) * a.R + r) * D + 8 * lg_e;
            oscale = 1.f;
            if (lg_e == 0) a.part_ml[(bh * a.ns + split) * a.R + r] = make_float2(M[t], L[t]);
        }
        const float * orow = ob + rl * D + 8 * lg_e;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            const float4 p0 = *(const float4 *) (orow + 32 * bb), p1 = *(const float4 *) (orow + 32 * bb + 4);
            const v4f o0 = O[t][bb][0] * fw[t], o1 = O[t][bb][1] * fw[t];
            const float4 w0 = make_float4((o0[0] + p0.x) * oscale, (o1[0] + p0.y) * oscale, (o0[1] + p0.z) * oscale, (o1[1] + p0.w) * oscale);
            const float4 w1 = make_float4((o0[2] + p1.x) * oscale, (o1[2] + p1.y) * oscale, (o0[3] + p1.z) * oscale, (o1[3] + p1.w) * oscale);
            if (vec) {
                *(float4 *) (out + 32 * bb) = w0;
                *(float4 *) (out + 32 * bb + 4) = w1;
            } else {
                float * o = out + 32 * bb;
                o[0] = w0.x; o[1] = w0.y; o[2] = w0.z; o[3] = w0.w;
                o[4] = w1.x; o[5] = w1.y; o[6] = w1.z; o[7] = w1.w;
            }
        }
    }
}

// LSE merge of the ns split partials of one query row. All (max, sum) pairs
// are read into LDS at once while the partial rows are already in flight;
// thread (group g, quad q) then folds splits g, g+4, ... of dims 4q..4q+3 and
// the four groups add up through LDS.
constexpr int MERGE_GROUPS = 4;
constexpr int MERGE_BATCH = 8;

__global__ __launch_bounds__(256) void k_fattn_merge(fa_args a) {
    __shared__ float wsh[MAX_SPLITS];
    __shared__ float red[256 / 64];
    __shared__ float4 acc_sh[MERGE_GROUPS - 1][64];
    const int row = blockIdx.x;                               // (b * nh_kv + kvh) * R + r
    const int r = row % a.R;
    const int bh = row / a.R;
    const int kvh = bh % a.nh_kv, b = bh / a.nh_kv;
    const int g = threadIdx.x >> 6, q = threadIdx.x & 63;
    const float2 * ml = a.part_ml + (size_t) bh * a.ns * a.R + r;
    const float4 * po = (const float4 *) (a.part_o + ((size_t) bh * a.ns * a.R + r) * D) + q;
    const size_t sstride = (size_t) a.R * D / 4;              // float4s between splits

    // first batch of partial rows in flight before the weights are known
    float4 ob[MERGE_BATCH];
#pragma unroll
    for (int i = 0; i < MERGE_BATCH; i++) {
        const int s = g + i * MERGE_GROUPS;
        ob[i] = s < a.ns ? po[(size_t) s * sstride] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mloc = -INFINITY;
    for (int s = threadIdx.x; s < a.ns; s += 256) {
        const float2 e = ml[(size_t) s * a.R];
        wsh[s] = e.x;
        mloc = xmax(mloc, e.x);
    }
    for (int o = 32; o >= 1; o >>= 1) mloc = xmax(mloc, __shfl_xor(mloc, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mloc;
    __syncthreads();
    const float M = xmax(xmax(red[0], red[1]), xmax(red[2], red[3]));
    float lpart = 0.f;
    for (int s = threadIdx.x; s < a.ns; s += 256) {
        const float m = wsh[s];
        const float w = m == -INFINITY ? 0.f : exp2f(m - M);
        lpart += w * ml[(size_t) s * a.R].y;
        wsh[s] = w;
    }
    for (int o = 32; o >= 1; o >>= 1) lpart += __shfl_xor(lpart, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lpart;
    __syncthreads();
    const float L = (red[0] + red[1]) + (red[2] + red[3]);

    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < a.ns; s0 += MERGE_GROUPS * MERGE_BATCH) {
        if (s0 > 0) {
#pragma unroll
            for (int i = 0; i < MERGE_BATCH; i++) {
                const int s = s0 + g + i * MERGE_GROUPS;
                ob[i] = s < a.ns ? po[(size_t) s * sstride] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int i = 0; i < MERGE_BATCH; i++) {
            const int s = s0 + g + i * MERGE_GROUPS;
            const float w = s < a.ns ? wsh[s] : 0.f;
            acc.x += w * ob[i].x; acc.y += w * ob[i].y; acc.z += w * ob[i].z; acc.w += w * ob[i].w;
        }
    }
    if (g > 0) acc_sh[g - 1][q] = acc;
    __syncthreads();
    if (g == 0) {
        const float4 a1 = acc_sh[0][q], a2 = acc_sh[1][q], a3 = acc_sh[2][q];
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const float4 o = make_float4(((acc.x + a1.x) + (a2.x + a3.x)) * inv, ((acc.y + a1.y) + (a2.y + a3.y)) * inv,
                                     ((acc.z + a1.z) + (a2.z + a3.z)) * inv, ((acc.w + a1.w) + (a2.w + a3.w)) * inv);
        const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
        float * d = a.dst + (((size_t) b * a.T + t) * a.nh + h) * D + 4 * q;
        if (a.dst_vec) {
            *(float4 *) d = o;
        } else {
            d[0] = o.x; d[1] = o.y; d[2] = o.z; d[3] = o.w;
        }
    }
}

// ---------------------------------------------------------------- planning

struct fa_plan {
    int32_t R, RT, gqa, rw, n_rg, ns, split_len;
    int64_t n_kv_pad;
    size_t  off_ml, off_qimg, off_dq, off_mimg;   // workspace sections (bytes)
    size_t  ws_bytes;
};

int env_int(const char * name, int dflt) {
    const char * s = std::getenv(name);
    return s && *s ? std::atoi(s) : dflt;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// The key loop hand-counts its outstanding vector-memory operations (the LDS
// DMAs and the query-operand loads are inline asm the compiler does not see),
// so a build of the attention kernel that spills to scratch would break that
// count: refuse to run one.
int check_no_scratch() {
    static const int rc = [] {
        for (const void * f : {(const void *) k_fattn_q8_0<1>, (const void *) k_fattn_q8_0<2>}) {
            hipFuncAttributes at{};
            if (int e = hip_check(hipFuncGetAttributes(&at, f), "hipFuncGetAttributes")) return e;
            if (at.localSizeBytes != 0)
                return set_error(QWFN_EDEVICE, "flash_attn_ext: attention kernel was built with " +
                                                   std::to_string(at.localSizeBytes) + " B of scratch per lane");
        }
        return (int) QWFN_OK;
    }();
    if (rc) set_error(rc, "flash_attn_ext: attention kernel uses scratch memory (build is unusable)");
    return rc;
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
    if (k->nb[1] >= (size_t(1) << 24) || v->nb[1] >= (size_t(1) << 24))
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: k/v row strides must be below 16 MiB");
    bool per_head_mask = false;
    int64_t m_slices = 0;
    if (mask) {
        if (!mask->data) return set_error(QWFN_EINVAL, "flash_attn_ext: mask has no data");
        if (mask->type != QWFN_TYPE_F16) return set_error(QWFN_EINVAL, "flash_attn_ext: mask must be f16");
        if (mask->nb[0] != 2) return set_error(QWFN_EINVAL, "flash_attn_ext: mask rows must be contiguous");
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < T)
            return set_error(QWFN_EINVAL, "flash_attn_ext: mask must be at least [n_kv, T]");
        if (mask->ne[2] <= 0 || nh % mask->ne[2] || mask->ne[3] <= 0 || q->ne[3] % mask->ne[3])
            return set_error(QWFN_EINVAL, "flash_attn_ext: mask must broadcast over heads and batch");
        if (!is_aligned(mask->data, 2)) return set_error(QWFN_EALIGN, "flash_attn_ext: mask must be 2-byte aligned");
        per_head_mask = mask->ne[2] != 1;
        m_slices = mask->ne[2] * mask->ne[3];
    }
    // Query rows per block: one or two 16-row tiles. A block streams at most
    // MASK_ROWS mask rows per chunk: one per query row for a per-head mask, one
    // per query position for a shared one.
    int rw = R > 16 ? 32 : 16;
    if (const int force = env_int("QWFN_FA_ROWS", 0)) rw = force >= 32 ? 32 : 16;
    if (mask && rw == 32 && (per_head_mask || (32 + gqa - 1) / gqa + 1 > MASK_ROWS)) rw = 16;
    pl->R = (int32_t) R;
    pl->rw = rw;
    pl->RT = rw / 16;
    pl->n_rg = (int32_t) ((R + rw - 1) / rw);
    pl->gqa = (int32_t) gqa;
    const int64_t n_kv = k->ne[1];
    const int64_t B = q->ne[3];
    pl->n_kv_pad = (n_kv + CK - 1) / CK * CK;
    // Splits: about one block per CU (256), each at least one chunk.
    const int64_t target_blocks = env_int("QWFN_FA_BLOCKS", 256);
    int64_t ns = std::max<int64_t>(1, target_blocks / std::max<int64_t>(1, nh_kv * B * pl->n_rg));
    ns = std::min<int64_t>(ns, std::max<int64_t>(1, (n_kv + CK - 1) / CK));
    if (const int force = env_int("QWFN_FA_SPLITS", 0)) ns = force;
    int64_t split_len = (n_kv + ns - 1) / ns;
    split_len = std::max<int64_t>(CK, (split_len + CK - 1) / CK * CK);
    ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
    if (ns > MAX_SPLITS)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: " + std::to_string(ns) + " key splits requested, at most " +
                                           std::to_string(MAX_SPLITS) + " supported");
    pl->ns = (int32_t) ns;
    pl->split_len = (int32_t) split_len;
    // workspace: split partials (when ns > 1), the query image, the mask image
    const int64_t n_bkr = B * nh_kv * pl->n_rg;
    const size_t n_part = ns > 1 ? (size_t) (B * nh_kv * ns * R) : 0;
    size_t off = align256(n_part * D * sizeof(float));
    pl->off_ml = off;
    off = align256(off + n_part * sizeof(float2));
    pl->off_qimg = off;
    off = align256(off + (size_t) n_bkr * pl->RT * 64 * NBLK * 16);
    pl->off_dq = off;
    off = align256(off + (size_t) n_bkr * QROWS_IMG * NBLK * sizeof(float));
    pl->off_mimg = off;
    off = align256(off + (size_t) m_slices * T * pl->n_kv_pad * 2);
    pl->ws_bytes = off;
    return QWFN_OK;
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" size_t qwfn_fattn_workspace_size(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                            const qwfn_tensor * mask) {
    fa_plan pl{};
    if (plan_fattn(q, k, v, mask, &pl)) return 0;
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
    const int64_t n_kv = k->ne[1];
    if (n_kv == 0) {
        // no keys: ggml-cpu divides 0 by S = 0 only for rows it visits; the
        // result of an empty attention is defined here as zeros (a fill kernel,
        // not a memset node, so the call stays capturable into a HIP graph)
        const int64_t n = (int64_t) (view_bytes(*dst) / 4);
        hipLaunchKernelGGL(k_zero_f32, dim3((unsigned) std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 4096))),
                           dim3(256), 0, as_stream(stream), (float *) dst->data, n);
        return hip_check(hipGetLastError(), "flash_attn zero fill");
    }
    if (ws) {
        if (ws_bytes < pl.ws_bytes) return set_error(QWFN_ENOMEM, "flash_attn_ext: workspace too small");
        if (!is_aligned(ws, 256)) return set_error(QWFN_EALIGN, "flash_attn_ext: workspace must be 256-byte aligned");
    } else if (int rc = library_workspace(pl.ws_bytes, &ws)) {
        return rc;
    }
    if (int rc = check_no_scratch()) return rc;

    fa_args a{};
    a.q = (const char *) q->data; a.q_nb1 = q->nb[1]; a.q_nb2 = q->nb[2]; a.q_nb3 = q->nb[3];
    a.k = (const char *) k->data; a.k_nb1 = k->nb[1]; a.k_nb2 = k->nb[2]; a.k_nb3 = k->nb[3];
    a.v = (const char *) v->data; a.v_nb1 = v->nb[1]; a.v_nb2 = v->nb[2]; a.v_nb3 = v->nb[3];
    char * w = (char *) ws;
    if (mask) {
        a.mask = (const char *) mask->data; a.m_nb1 = mask->nb[1]; a.m_nb2 = mask->nb[2]; a.m_nb3 = mask->nb[3];
        a.m_ne2 = (int32_t) mask->ne[2]; a.m_ne3 = (int32_t) mask->ne[3];
        a.mimg = (uint16_t *) (w + pl.off_mimg);
    } else {
        a.mask = nullptr; a.m_ne2 = 1; a.m_ne3 = 1; a.mimg = nullptr;
    }
    a.dst = (float *) dst->data;
    a.part_o = (float *) w;
    a.part_ml = (float2 *) (w + pl.off_ml);
    a.qimg = (uint4 *) (w + pl.off_qimg);
    a.dqimg = (float *) (w + pl.off_dq);
    a.n_kv = n_kv;
    a.n_kv_pad = pl.n_kv_pad;
    a.T = (int32_t) q->ne[1]; a.nh = (int32_t) q->ne[2]; a.nh_kv = (int32_t) k->ne[2];
    a.gqa = pl.gqa; a.R = pl.R; a.B = (int32_t) q->ne[3];
    a.kb = (int32_t) k->ne[3]; a.vb = (int32_t) v->ne[3];
    a.ns = pl.ns; a.split_len = pl.split_len; a.rw = pl.rw; a.n_rg = pl.n_rg;
    a.scale = scale; a.x86 = variant == QWFN_Q8_X86;
    a.dst_vec = is_aligned(dst->data, 16) ? 1 : 0;

    const int64_t units = ((int64_t) a.B * a.ns + 7) / 8 * 8;
    const int64_t grid = units * a.nh_kv * a.n_rg;
    if (grid > 0x7fffffff) return set_error(QWFN_EINVAL, "flash_attn_ext: grid too large");
    hipStream_t st = as_stream(stream);
    const int n_qblocks = a.B * a.nh_kv * a.n_rg;
    const int n_mblocks = mask ? 64 : 0;
    if (pl.RT == 1) hipLaunchKernelGGL(k_fattn_prep<1>, dim3(n_qblocks + n_mblocks), dim3(256), 0, st, a, n_qblocks);
    else            hipLaunchKernelGGL(k_fattn_prep<2>, dim3(n_qblocks + n_mblocks), dim3(256), 0, st, a, n_qblocks);
    if (int rc = hip_check(hipGetLastError(), "flash_attn prep launch")) return rc;
    if (pl.RT == 1) hipLaunchKernelGGL(k_fattn_q8_0<1>, dim3((unsigned) grid), dim3(KG * 64), 0, st, a);
    else            hipLaunchKernelGGL(k_fattn_q8_0<2>, dim3((unsigned) grid), dim3(KG * 64), 0, st, a);
    if (int rc = hip_check(hipGetLastError(), "flash_attn launch")) return rc;
    if (a.ns > 1) {
        const int64_t blocks = (int64_t) a.B * a.nh_kv * a.R;
        hipLaunchKernelGGL(k_fattn_merge, dim3((unsigned) blocks), dim3(256), 0, st, a);
        if (int rc = hip_check(hipGetLastError(), "flash_attn merge launch")) return rc;
    }
    return QWFN_OK;
}
