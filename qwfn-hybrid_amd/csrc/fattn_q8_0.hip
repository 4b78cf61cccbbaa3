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

namespace qwfn {
namespace {

typedef int      v4i __attribute__((ext_vector_type(4)));
typedef float    v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2  __attribute__((ext_vector_type(2)));

constexpr int D      = 256;            // head size (values per head row)
constexpr int NBLK   = D / QK;         // 8 q8_0 blocks per head row
constexpr int SEG    = NBLK * QBLOCK;  // 272 bytes per head row
constexpr int KW     = 32;             // keys per wave per chunk (one PV MFMA depth)
constexpr int KG     = 2;              // key groups (waves along the keys of a chunk)
constexpr int CK     = KG * KW;        // keys per chunk
constexpr int CHUNK_BYTES = CK * SEG;  // one tensor's rows of a chunk (17408)
constexpr int DMA_PER_TENSOR = CHUNK_BYTES / 1024;   // wave-wide 16-byte LDS-DMA loads per tensor (17)
constexpr int MASK_LDS = 2048;         // staged mask values per block (rows x keys of its split)
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
    int64_t  n_kv;
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

// Two int8 values (byte SEL of a and of b) -> packed f16 pair, exact.
#define QWFN_CVT_I8X2(NAME, SEL)                                                                  \
    __device__ __forceinline__ uint32_t NAME(uint32_t a, uint32_t b) {                            \
        uint32_t r;                                                                               \
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:" SEL  \
            "\n\tv_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:" SEL \
            : "=&v"(r) : "v"(a), "v"(b));                                                         \
        return r;                                                                                 \
    }
QWFN_CVT_I8X2(cvt_i8x2_f16_b0, "BYTE_0")
QWFN_CVT_I8X2(cvt_i8x2_f16_b1, "BYTE_1")
#undef QWFN_CVT_I8X2

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
// Split two f32 values into f16 hi parts (RNE) and f16 lo = f16(x - hi):
// returns {hi pair, lo pair} as packed dwords.
__device__ __forceinline__ uint2 split_f16x2(float x0, float x1) {
    uint32_t hi, lo;
    asm("v_cvt_pk_f16_f32 %0, %2, %3\n\t"
        "v_fma_mixlo_f16 %1, %2, 1.0, -%0 op_sel:[0,0,0] op_sel_hi:[0,0,1]\n\t"
        "v_fma_mixhi_f16 %1, %3, 1.0, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=&v"(hi), "=&v"(lo) : "v"(x0), "v"(x1));
    return make_uint2(hi, lo);
}

__device__ __forceinline__ float xmax(float a, float b) { return a > b ? a : b; }

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

// Base of staged mask row mr of this block (F16 row over keys), or nullptr.
// Row mr is query position t0 + mr for a shared mask, query row r0 + mr for a
// per-head mask.
__device__ __forceinline__ const uint16_t * mask_row(const fa_args & a, int mr, int t0, int r0, int kvh, int b) {
    if (!a.mask) return nullptr;
    int t, hq;
    if (a.m_ne2 == 1) { t = t0 + mr; hq = 0; }
    else { const int r = r0 + mr; t = r / a.gqa; hq = (kvh * a.gqa + (r - t * a.gqa)) % a.m_ne2; }
    return (const uint16_t *) (a.mask + (size_t) t * a.m_nb1 + (size_t) hq * a.m_nb2 + (size_t) (b % a.m_ne3) * a.m_nb3);
}

// f[0 .. n) = 0 (dst is only 4-byte aligned, so plain f32 stores).
__global__ void k_zero_f32(float * f, int64_t n) {
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) f[i] = 0.f;
}

template <int RT>
__global__ __launch_bounds__(RT * KG * 64)
void k_fattn_q8_0(fa_args a) {
    constexpr int WAVES = RT * KG;
    constexpr int THREADS = WAVES * 64;
    constexpr int ROWS = 16 * RT;
    constexpr int DPW = (2 * DMA_PER_TENSOR + WAVES - 1) / WAVES;   // DMAs per wave per chunk
    // two chunk buffers, each K rows [CK][272] then V rows [CK][272]
    __shared__ __attribute__((aligned(16))) uint8_t ring[2][2 * CHUNK_BYTES];
    // per-wave scale tables of the current chunk: [K|V][block][key of the wave] fp16
    __shared__ __attribute__((aligned(16))) uint16_t scl[WAVES][2][NBLK][KW];
    __shared__ __attribute__((aligned(16))) uint16_t msk[MASK_LDS];         // mask of the block's split [row][key]
    // prologue scratch in ring stage 1 (before chunk 1's DMA): query windows
    // [ROWS][NBLK][64] int8, then d_q [ROWS][NBLK] f32
    static_assert(ROWS * NBLK * QWIN + ROWS * NBLK * 4 <= 2 * CHUNK_BYTES, "query scratch fits in stage 1");
    static_assert(ROWS * D * 4 + WAVES * 16 * 8 <= 2 * CHUNK_BYTES, "merge buffer fits in stage 0");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
    const int ln = lane & 15;       // MFMA row/col within a 16-tile
    const int lg = lane >> 4;       // lane group (k-slice / output row quad)
    const int tile = wave % RT;     // query row tile of this wave
    const int kgrp = wave / RT;     // key group of each chunk

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
    const int n_mrows = a.m_ne2 == 1 ? (r0 + RW - 1) / a.gqa - t0 + 1 : RW;

    const char * kbase = a.k + (size_t) (b % a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) (b % a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;

    // Issue chunk c's K/V rows into buffer dstb. Every wave issues exactly DPW
    // instructions (surplus ones repeat an instruction another wave covers,
    // writing identical bytes), so the number of loads in flight is known at
    // compile time. Piece p = 64*i + lane of a tensor's chunk is byte
    // 16*(p % 17) of key p / 17. Keys past the split are loaded (and masked)
    // while they exist; past n_kv they repeat the last key.
    uint32_t doff[DPW];             // per-lane byte offset of piece n within a chunk
#pragma unroll
    for (int n = 0; n < DPW; n++) {
        int i = wave + n * WAVES;
        if (i >= 2 * DMA_PER_TENSOR) i = 2 * DMA_PER_TENSOR - 1 - (i - 2 * DMA_PER_TENSOR);
        const int tensor = i >= DMA_PER_TENSOR;
        const int p = (i - tensor * DMA_PER_TENSOR) * 64 + lane;
        doff[n] = (uint32_t) ((p / 17) * (tensor ? a.v_nb1 : a.k_nb1) + (p % 17) * 16);
    }
    auto issue_chunk = [&](int c, uint8_t * dstb) __attribute__((always_inline)) {
        const int64_t c0 = k_lo + (int64_t) c * CK;
        const bool clamp = c0 + CK > a.n_kv;   // the cache's last chunk: no rows past n_kv
        const int last = (int) std::min<int64_t>(CK - 1, a.n_kv - 1 - c0);
#pragma unroll
        for (int n = 0; n < DPW; n++) {
            int i = wave + n * WAVES;
            if (i >= 2 * DMA_PER_TENSOR) i = 2 * DMA_PER_TENSOR - 1 - (i - 2 * DMA_PER_TENSOR);
            const int tensor = i >= DMA_PER_TENSOR;
            const int ii = i - tensor * DMA_PER_TENSOR;
            const char * base = tensor ? vbase + (size_t) c0 * a.v_nb1 : kbase + (size_t) c0 * a.k_nb1;
            uint32_t off = doff[n];
            if (clamp) {
                const int p = ii * 64 + lane;
                off = (uint32_t) (std::min(p / 17, last) * (tensor ? a.v_nb1 : a.k_nb1) + (p % 17) * 16);
            }
            dma16(base + off, __builtin_amdgcn_readfirstlane(lds_addr(dstb + tensor * CHUNK_BYTES + ii * 1024)));
        }
    };
    const int span = (int) (k_hi - k_lo);                       // keys of this split (<= split_len)
    const int mstride = a.split_len;                            // LDS row stride of the staged mask

    // ---- prologue: chunk 0's DMA first, then the block's Q rows and its mask.
    //      Waiting for the (later) ordinary loads also lands chunk 0. ----
    issue_chunk(0, ring[0]);
    const int sub = lane & 7;       // 4-value group of a q8_0 block (Q staging)
    const int blk = lane >> 3;      // q8_0 block of the row (Q staging)
    float4 xv[ROWS / WAVES];
#pragma unroll
    for (int q = 0; q < ROWS / WAVES; q++) {
        const int rl = wave + q * WAVES;
        const int r = r0 + std::min(rl, RW - 1);
        const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
        xv[q] = *(const float4 *) (a.q + (size_t) t * a.q_nb1 + (size_t) h * a.q_nb2 + (size_t) b * a.q_nb3 +
                                   (size_t) (blk * QK + sub * 4) * 4);
    }
    if (a.mask) {
        constexpr int MB = 8;                                   // loads in flight per thread
        for (int e0 = threadIdx.x; e0 < n_mrows * mstride; e0 += MB * THREADS) {
            uint16_t mv[MB];
#pragma unroll
            for (int q = 0; q < MB; q++) {
                const int e = e0 + q * THREADS;
                const int mr = std::min(e / mstride, n_mrows - 1);
                const int key = std::min(e - (e / mstride) * mstride, span - 1);
                mv[q] = mask_row(a, mr, t0, r0, kvh, b)[k_lo + key];
            }
#pragma unroll
            for (int q = 0; q < MB; q++) {
                const int e = e0 + q * THREADS;
                if (e < n_mrows * mstride) msk[e] = mv[q];
            }
        }
    }

    // ---- requantise the block's query rows to q8_0 and lay each block out on
    //      its 64-byte window (zero elsewhere), in ring stage 1 ----
    uint8_t * qwin = ring[1];
    float *   dqs  = (float *) (ring[1] + ROWS * NBLK * QWIN);
    for (int e = threadIdx.x; e < ROWS * NBLK * QWIN / 16; e += THREADS) ((uint4 *) qwin)[e] = make_uint4(0, 0, 0, 0);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < ROWS / WAVES; q++) {
        const int rl = wave + q * WAVES;
        const float4 v4 = rl < RW ? xv[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float x[4] = {v4.x, v4.y, v4.z, v4.w};
        uint16_t d16;
        float dq;
        const uint32_t w = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dq);
        uint16_t * wp = (uint16_t *) (qwin + (rl * NBLK + blk) * QWIN + win_off(blk) + 4 * sub);
        wp[0] = (uint16_t) w;
        wp[1] = (uint16_t) (w >> 16);
        if (sub == 0) dqs[rl * NBLK + blk] = dq;
    }
    __syncthreads();
    const int rl_lane = tile * 16 + ln;                 // this lane's query row (MFMA column)
    v4i qw[NBLK];                                       // B operand of QK: window slice lg of each block
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) qw[bb] = *(const v4i *) (qwin + (rl_lane * NBLK + bb) * QWIN + 16 * lg);
    float dqr[NBLK];                                    // d_q * scale * log2(e)
    {
        const float4 d0 = *(const float4 *) (dqs + rl_lane * NBLK), d1 = *(const float4 *) (dqs + rl_lane * NBLK + 4);
        const float f = a.scale * LOG2E;
        dqr[0] = d0.x * f; dqr[1] = d0.y * f; dqr[2] = d0.z * f; dqr[3] = d0.w * f;
        dqr[4] = d1.x * f; dqr[5] = d1.y * f; dqr[6] = d1.z * f; dqr[7] = d1.w * f;
    }
    __syncthreads();                                    // stage 1 is free again
    if (n_chunks > 1) issue_chunk(1, ring[1]);
    // padded rows (rl_lane >= RW) read mask row 0: their results are never stored
    const int mrow = rl_lane >= RW ? 0 : (a.m_ne2 == 1 ? (r0 + rl_lane) / a.gqa - t0 : rl_lane);

    // ---- online softmax state (one 16-row tile per wave) ----
    v4f   O[NBLK][2];
    float m_run = -INFINITY, l_run = 0.f;
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) { O[bb][0] = v4f{0, 0, 0, 0}; O[bb][1] = v4f{0, 0, 0, 0}; }

    const int wk = kgrp * KW;   // this wave's first key in a chunk
    uint16_t (*sw)[NBLK][KW] = scl[wave];

    // One chunk: `cur` holds chunk c. Called with ring[0] / ring[1] literally so
    // the compiler can tell the buffer being read from the one the DMA fills.
    auto chunk_step = [&](int c, uint8_t * cur) __attribute__((always_inline)) {
        if (c + 1 < n_chunks) {
            // chunk c+1's DMA is the only one issued after chunk c's: once at most
            // that many loads are outstanding, chunk c has landed
            wait_vmcnt<DPW>();
        } else {
            wait_vmcnt<0>();
        }
        __syncthreads();
        const uint8_t * ks = cur;
        const uint8_t * vs = cur + CHUNK_BYTES;
        // this wave's keys' block scales, transposed to [block][key]
#pragma unroll
        for (int n = 0; n < 2 * NBLK * KW / 64; n++) {
            const int e = n * 64 + lane;
            const int tensor = e / (NBLK * KW), kk = (e / NBLK) % KW, bb = e % NBLK;
            sw[tensor][bb][kk] = *(const uint16_t *) (cur + tensor * CHUNK_BYTES + (wk + kk) * SEG + bb * QBLOCK);
        }
        wave_lds_sync();

        // ---- S = Q K^T for 2 tiles of 16 keys ----
        float s[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            const uint8_t * krow = ks + (wk + kt * 16 + ln) * SEG + 16 * lg;   // A operand: key row ln, slice lg
            v4i cc[NBLK];
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++)
                cc[bb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i *) (krow + 16 * win_piece(bb)), qw[bb],
                                                               v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) s[kt][i] = 0.f;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                const uint2 dk = *(const uint2 *) &sw[0][bb][kt * 16 + lg * 4];   // 4 keys' fp16 d_k
                s[kt][0] = __builtin_fmaf((float) cc[bb][0], mul_f16lo(dqr[bb], dk.x), s[kt][0]);
                s[kt][1] = __builtin_fmaf((float) cc[bb][1], mul_f16hi(dqr[bb], dk.x), s[kt][1]);
                s[kt][2] = __builtin_fmaf((float) cc[bb][2], mul_f16lo(dqr[bb], dk.y), s[kt][2]);
                s[kt][3] = __builtin_fmaf((float) cc[bb][3], mul_f16hi(dqr[bb], dk.y), s[kt][3]);
            }
            __builtin_amdgcn_sched_barrier(0);   // one key tile's accumulators live at a time
        }

        // ---- mask, online softmax (base 2; scores are already in log2 units).
        //      A masked key has x = -inf, so its p is exp2(-inf) = 0 ----
        float p[8];
        {
            float x[8];
            float mloc = -INFINITY;
            const bool tail = (c + 1) * CK > span;                     // keys past the split in this chunk
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const int kin = c * CK + wk + kt * 16 + lg * 4;          // first of the lane's 4 keys in the split
                uint2 mv = make_uint2(0, 0);
                if (a.mask) mv = *(const uint2 *) (msk + mrow * mstride + kin);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t mh = i < 2 ? mv.x : mv.y;
                    float xi = (i & 1) ? fma_f16hi(mh, LOG2E, s[kt][i]) : fma_f16lo(mh, LOG2E, s[kt][i]);
                    if (tail && kin + i >= span) xi = -INFINITY;
                    x[kt * 4 + i] = xi;
                    mloc = xmax(mloc, xi);
                }
            }
            mloc = xmax(mloc, __shfl_xor(mloc, 16));
            mloc = xmax(mloc, __shfl_xor(mloc, 32));
            const float m_new = xmax(m_run, mloc);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;   // all keys masked so far
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
            float lsum = 0.f;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {
                p[jj] = __builtin_amdgcn_exp2f(x[jj] - m_use);
                lsum += p[jj];
            }
            l_run = l_run * alpha + lsum;
            m_run = m_new;
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[bb][0] *= alpha; O[bb][1] *= alpha; }
            }
        }
        // ---- O += V^T P per V block. Tile e of block bb holds dims 32bb + 2m + e
        //      (m = MFMA row); the A operand of lane (m, g) is dims 2m, 2m+1 of the
        //      lane's 8 keys, one naturally aligned 2-byte LDS read per key ----
        const uint8_t * vrow = vs + (wk + lg * 4) * SEG + 2 + 2 * ln;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            uint32_t w[8];
#pragma unroll
            for (int jj = 0; jj < 8; jj++)
                w[jj] = *(const uint16_t *) (vrow + ((jj >> 2) * 16 + (jj & 3)) * SEG + bb * QBLOCK);
            const uint2 dv0 = *(const uint2 *) &sw[1][bb][lg * 4];
            const uint2 dv1 = *(const uint2 *) &sw[1][bb][16 + lg * 4];
            const uint32_t dv[4] = {dv0.x, dv0.y, dv1.x, dv1.y};
            uint32_t bh[4], bl[4];
#pragma unroll
            for (int q2 = 0; q2 < 4; q2++) {
                const uint2 hl = split_f16x2(mul_f16lo(p[2 * q2], dv[q2]), mul_f16hi(p[2 * q2 + 1], dv[q2]));
                bh[q2] = hl.x;
                bl[q2] = hl.y;
            }
            uint32_t a0[4], a1[4];
#pragma unroll
            for (int q2 = 0; q2 < 4; q2++) {
                a0[q2] = cvt_i8x2_f16_b0(w[2 * q2], w[2 * q2 + 1]);
                a1[q2] = cvt_i8x2_f16_b1(w[2 * q2], w[2 * q2 + 1]);
            }
            const v8h A0 = __builtin_bit_cast(v8h, uint4{a0[0], a0[1], a0[2], a0[3]});
            const v8h A1 = __builtin_bit_cast(v8h, uint4{a1[0], a1[1], a1[2], a1[3]});
            const v8h Bh = __builtin_bit_cast(v8h, uint4{bh[0], bh[1], bh[2], bh[3]});
            const v8h Bl = __builtin_bit_cast(v8h, uint4{bl[0], bl[1], bl[2], bl[3]});
            O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bh, O[bb][0], 0, 0, 0);
            O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bh, O[bb][1], 0, 0, 0);
            O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bl, O[bb][0], 0, 0, 0);
            O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bl, O[bb][1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);   // bound the V reads hoisted ahead
        }
        __syncthreads();   // chunk c consumed: its buffer may be overwritten
        if (c + 2 < n_chunks) issue_chunk(c + 2, cur);
    };
    for (int c = 0; c < n_chunks; c += 2) {
        chunk_step(c, ring[0]);
        if (c + 1 < n_chunks) chunk_step(c + 1, ring[1]);
    }

    // ---- merge the two key groups in LDS: group 1 adds its weighted O to the
    //      buffer, group 0 adds its own and writes the block's result ----
    float * ob = (float *) ring[0];                                // [ROWS][256] f32, natural dim order
    float2 * ml = (float2 *) (ring[0] + ROWS * D * 4);             // [WAVES][16]
    {
        float l = l_run;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        l_run = l;
        if (lg == 0) ml[wave * 16 + ln] = make_float2(m_run, l);
    }
    __syncthreads();
    float M, L, fw;
    {
        const float2 e0 = ml[tile * 16 + ln], e1 = ml[(RT + tile) * 16 + ln];
        M = xmax(e0.x, e1.x);
        L = (e0.x == -INFINITY ? 0.f : e0.y * exp2f(e0.x - M)) + (e1.x == -INFINITY ? 0.f : e1.y * exp2f(e1.x - M));
        fw = (m_run == -INFINITY) ? 0.f : exp2f(m_run - M);
    }
    // lane (ln, lg) holds, for block bb, dims 32bb + 8lg + 2i + e in O[bb][e][i]
    float * orow = ob + rl_lane * D + 8 * lg;
    if (kgrp == 1) {
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            const v4f o0 = O[bb][0] * fw, o1 = O[bb][1] * fw;
            *(float4 *) (orow + 32 * bb)     = make_float4(o0[0], o1[0], o0[1], o1[1]);
            *(float4 *) (orow + 32 * bb + 4) = make_float4(o0[2], o1[2], o0[3], o1[3]);
        }
    }
    __syncthreads();
    if (kgrp != 0 || rl_lane >= RW) return;
    const int r = r0 + rl_lane;
    const int t = r / a.gqa, h = kvh * a.gqa + (r - t * a.gqa);
    const size_t bh = (size_t) b * a.nh_kv + kvh;
    float * out;
    float oscale;
    if (a.ns == 1) {
        out = a.dst + (((size_t) b * a.T + t) * a.nh + h) * D + 8 * lg;
        oscale = L > 0.f ? 1.f / L : 0.f;
    } else {
        out = a.part_o + ((bh * a.ns + split) * a.R + r) * D + 8 * lg;
        oscale = 1.f;
        if (lg == 0) a.part_ml[(bh * a.ns + split) * a.R + r] = make_float2(M, L);
    }
    const bool vec = a.ns > 1 || a.dst_vec;
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        const float4 p0 = *(const float4 *) (orow + 32 * bb), p1 = *(const float4 *) (orow + 32 * bb + 4);
        const v4f o0 = O[bb][0] * fw, o1 = O[bb][1] * fw;
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
    size_t  ws_bytes;
};

int env_int(const char * name, int dflt) {
    const char * s = std::getenv(name);
    return s && *s ? std::atoi(s) : dflt;
}

// The key loop hand-counts its outstanding vector-memory operations (the LDS
// DMAs are inline asm the compiler does not see), so a build of the attention
// kernel that spills to scratch would break that count: refuse to run one.
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
    bool per_head_mask = false;
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
    }
    // Query rows per block: one or two 16-row tiles. A per-head mask stages one
    // mask row per query row, so it keeps blocks at 16 rows.
    int rw = (R > 16 && !per_head_mask) ? 32 : 16;
    if (const int force = env_int("QWFN_FA_ROWS", 0)) rw = (force >= 32 && !per_head_mask) ? 32 : 16;
    pl->R = (int32_t) R;
    pl->rw = rw;
    pl->RT = rw / 16;
    pl->n_rg = (int32_t) ((R + rw - 1) / rw);
    pl->gqa = (int32_t) gqa;
    const int64_t n_kv = k->ne[1];
    const int64_t B = q->ne[3];
    // Splits: about one block per CU (256), each at least one chunk.
    const int64_t target_blocks = env_int("QWFN_FA_BLOCKS", 256);
    int64_t ns = std::max<int64_t>(1, target_blocks / std::max<int64_t>(1, nh_kv * B * pl->n_rg));
    ns = std::min<int64_t>(ns, std::max<int64_t>(1, (n_kv + CK - 1) / CK));
    if (const int force = env_int("QWFN_FA_SPLITS", 0)) ns = force;
    int64_t split_len = (n_kv + ns - 1) / ns;
    split_len = std::max<int64_t>(CK, (split_len + CK - 1) / CK * CK);
    if (mask) {
        // a block stages its split's mask rows in LDS: rows x split_len <= MASK_LDS
        const int64_t mrows = per_head_mask ? rw : std::min<int64_t>(T, (rw + gqa - 1) / gqa + 1);
        if (mrows * CK > MASK_LDS) return set_error(QWFN_ENOTSUP, "flash_attn_ext: too many mask rows per block");
        const int64_t cap = std::max<int64_t>(CK, MASK_LDS / mrows / CK * CK);
        split_len = std::min(split_len, cap);
    }
    ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
    if (ns > MAX_SPLITS) {
        // long caches with a mask: widen the splits (the mask cap above) no further
        // than MAX_SPLITS allows; such a call is refused rather than truncated
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: " + std::to_string(ns) + " key splits needed, at most " +
                                           std::to_string(MAX_SPLITS) + " supported");
    }
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
        // no keys: ggml-cpu divides 0 by S = 0 only for rows it visits; the
        // result of an empty attention is defined here as zeros (a fill kernel,
        // not a memset node, so the call stays capturable into a HIP graph)
        const int64_t n = (int64_t) (view_bytes(*dst) / 4);
        hipLaunchKernelGGL(k_zero_f32, dim3((unsigned) std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 4096))),
                           dim3(256), 0, as_stream(stream), (float *) dst->data, n);
        return hip_check(hipGetLastError(), "flash_attn zero fill");
    }
    if (int rc = check_no_scratch()) return rc;

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
    a.dst_vec = is_aligned(dst->data, 16) ? 1 : 0;

    const int64_t units = ((int64_t) a.B * a.ns + 7) / 8 * 8;
    const int64_t grid = units * a.nh_kv * a.n_rg;
    if (grid > 0x7fffffff) return set_error(QWFN_EINVAL, "flash_attn_ext: grid too large");
    hipStream_t st = as_stream(stream);
    if (pl.RT == 1) hipLaunchKernelGGL(k_fattn_q8_0<1>, dim3((unsigned) grid), dim3(1 * KG * 64), 0, st, a);
    else            hipLaunchKernelGGL(k_fattn_q8_0<2>, dim3((unsigned) grid), dim3(2 * KG * 64), 0, st, a);
    if (int rc = hip_check(hipGetLastError(), "flash_attn launch")) return rc;
    if (a.ns > 1) {
        const int64_t blocks = (int64_t) a.B * a.nh_kv * a.R;
        hipLaunchKernelGGL(k_fattn_merge, dim3((unsigned) blocks), dim3(256), 0, st, a);
        if (int rc = hip_check(hipGetLastError(), "flash_attn merge launch")) return rc;
    }
    return QWFN_OK;
}
