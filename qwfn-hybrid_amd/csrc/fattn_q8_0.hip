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
// Work decomposition (flash-decoding), one launch plus a split merge:
//   grid   : (batch, KV head, row group, key split); the KV heads and row
//            groups of one split sit on the same XCD and are dispatched next to
//            each other, so the cache lines two heads share (a 272-byte head row
//            is not line aligned) come from one L2.
//   block  : 4 wavefronts, two blocks per CU (RT 16-row query tiles x 4/RT
//            key groups of 16 or 32 keys), or 8 wavefronts, one block per CU
//            (8/RT key groups of 16 keys). Keys stream in chunks of raw 272-byte
//            head rows through gfx950's LDS DMA (buffer_load_dwordx4 ... lds)
//            into a ring of 2 or 3 stages, so one or two chunks are in flight
//            while one is computed. Query rows and split masks arrive by the
//            same DMA ahead of the first chunks, and the block requantises its
//            query rows while those chunks load.
//   QK^T   : v_mfma_i32_16x16x64_i8 per q8_0 block. The A operand is four
//            16-byte aligned pieces of the raw K row that cover the block's 32
//            quants (a 64-byte window); the B operand is the requantised query
//            laid out on the same window, zero outside the block, so the integer
//            sum is exactly the block's dot product and no LDS read is ever
//            misaligned. The int32 tile is scaled by d_q*d_k.
//   softmax: online, base 2, per query row; row max across the 4 lane groups
//            with cross-row lane swaps. The running max may lag the true max by
//            up to 2^8 (p <= 256), so the accumulators are rescaled only when
//            the max jumps by more than that.
//   PV     : v_mfma_f32_16x16x16_f16 (16-key waves) or 16x16x32 (32-key
//            waves), A = V^T (int8 -> f16 exact, SDWA byte select from
//            naturally aligned 2-byte LDS reads), B = P*d_v of one V block as
//            f16 hi + lo.
//   merge  : the key groups of a block merge in LDS; key splits merge in a
//            second kernel (log-sum-exp weights), one block per quarter row.
#include "q8_device.h"
#include "qwfn_common.h"

#include <algorithm>
#include <cmath>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <type_traits>

namespace qwfn {
namespace {

typedef int      v4i __attribute__((ext_vector_type(4)));
typedef float    v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef uint16_t us2 __attribute__((ext_vector_type(2)));

constexpr int D      = 256;            // head size (values per head row)
constexpr int NBLK   = D / QK;         // 8 q8_0 blocks per head row
constexpr int SEG    = NBLK * QBLOCK;  // 272 bytes per head row
constexpr int WAVES  = 8;              // wavefronts per block, one block per CU (two per SIMD)
constexpr int WAVES_PAIR = 4;          // wavefronts per block, two blocks per CU
constexpr int QWIN   = 64;             // bytes of one block's query window
constexpr int MAX_SPLITS = 1024;       // key splits per (batch, KV head, row group)
constexpr int RAGGED_MAX_B = 16;       // sequences of a call with per-sequence key counts
constexpr int GATHER_MAX_HEADS = 8;    // KV heads of a call with cell lists
constexpr int GATHER_MAX_LISTS = 32;   // (sequence, KV head) cell lists of a call
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_SLACK = 8.f;   // log2 units the running max may lag the true max
constexpr int PV_BATCH = 4;            // 16-key V block tiles whose LDS reads are issued together
constexpr int MASK_LDS = 8192;         // LDS bytes for a block's mask rows over its whole split
constexpr int MASK_ROWS_PAIR = 7;      // mask-tile rows of a 4-wave two-tile block
enum { MASK_NONE = 0, MASK_SPLIT = 1, MASK_TILE = 2 };

// Chunk geometry for RT query tiles per block of NW waves; MT: the mask
// travels with each chunk (MASK_TILE).
template <int RT, bool MT, int NW, int KWV>
struct fa_cfg {
    static constexpr int ROWS  = 16 * RT;                   // query rows per block
    static constexpr int KG    = NW / RT;                   // key groups
    static constexpr int NKT   = KWV / 16;                  // 16-key tiles per wave
    static constexpr int CK    = KG * KWV;                  // keys per chunk (64 or 128)
    // MASK_SPLIT bytes (none with MASK_TILE; half where 32-key waves leave
    // two blocks per CU no more room)
    static constexpr int MLDS  = MT ? 16 : KWV == 32 ? MASK_LDS / 2 : MASK_LDS;
    static constexpr int CHUNK = CK * SEG;                  // one tensor's rows of a chunk
    static constexpr int DMA_T = (CHUNK + 1023) / 1024;     // wave-wide 16-byte DMAs per tensor
    static constexpr int VOFF  = DMA_T * 1024;              // V rows' offset in a stage (K rows padded to whole DMAs)
    // MASK_TILE: a chunk's mask rows travel with it as 16-byte granules from
    // the 16-byte aligned address at or below each row's first key
    static constexpr int MGR   = 2 * CK / 16 + 1;           // granules per mask row
    // mask rows of a block, at most: every row, except for 4-wave blocks of two
    // tiles, which take mask tiles only for masks shared by the heads (a
    // block's rows then span at most MASK_ROWS_PAIR query positions)
    static constexpr int MROWS = NW == WAVES_PAIR && KWV == 32 ? MASK_ROWS_PAIR : ROWS;
    static constexpr int MDMA  = MT ? (MROWS * MGR + 63) / 64 : 0;   // wave-wide DMAs for them
    static constexpr int MTILE = MDMA * 1024;               // their bytes in a stage
    static constexpr int STAGE = 2 * VOFF + MTILE;          // one ring stage: K rows, V rows, mask tile
    static constexpr int SLOTS = 2 * DMA_T + MDMA;          // DMAs per chunk (the mask ones as needed)
    static constexpr int SPW   = (SLOTS + NW - 1) / NW;     // DMA slots per wave
    static constexpr int NS    = RT == 2 && NW == WAVES && KWV == 16 ? 3 : 2;   // ring stages (chunks in flight + 1)
    static_assert(SPW * NW - SLOTS < NW, "only a wave's last slot can be absent");
    static_assert(KWV == 16 || KWV == 32, "one or two 16-key tiles per wave");
};

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
    const char * mask; size_t m_nb1, m_nb2, m_nb3;   // F16 [n_kv, T, m_ne2, m_ne3] or null
    int32_t m_ne2, m_ne3;
    uint32_t m_slice;      // bytes of one batch slice of the mask (last row's end)
    int32_t  mask_mode;    // MASK_NONE, MASK_SPLIT (whole split in LDS) or MASK_TILE (with each chunk)
    float *  dst;          // [D, nh, T, B]
    float *  part_o;       // [B][nh_kv][ns][R][D]
    float2 * part_ml;      // [B][nh_kv][ns][R]: (running max in log2 units, sum)
    int64_t  n_kv;
    int32_t  T, nh, nh_kv, gqa, R, B;
    int32_t  kb, vb;       // K/V batch extents (ne[3]); batch b reads b % kb
    int32_t  ns;           // key splits
    int32_t  split_len;    // keys per split, a multiple of the chunk (the last split runs to n_kv)
    int32_t  rw;           // query rows per block (16 * RT)
    int32_t  n_rg;         // row groups per KV head
    float    scale;
    int32_t  x86;
    int32_t  dst_vec;      // dst is 16-byte aligned: float4 stores
    uint32_t q_slice;      // bytes of one batch slice of q (last row's end)
    uint32_t gqa_mul;      // ceil(2^32 / gqa): r / gqa = mulhi(r, gqa_mul) for gqa > 1
    int32_t  m_gran;       // MASK_SPLIT: 16-byte granules per mask row of a split (split_len / 8 + 1)
    uint32_t m_gran_mul;   // ceil(2^32 / m_gran)
    uint32_t ns_mul, hgn_mul, nrg_mul;   // ceil(2^32 / d) for ns, nh_kv * n_rg, n_rg
    // k_fa_pre block order: 0 puts the row groups of a (batch, KV head,
    // split) unit on one XCD (they share its K/V rows), 1 puts the splits of
    // a (batch, KV head, row group) on one XCD (they share its query rows)
    int32_t  pre_rgmap;
    uint32_t nbh_mul;      // ceil(2^32 / (B * nh_kv))
    // fused append (app_n > 0): F32 rows [nh_kv * D] of K and V quantised into
    // cache rows app_row0 .. app_row0 + app_n - 1 before they are attended
    const char * app_k;
    const char * app_v;
    size_t   app_nb1;
    int64_t  app_row0;
    int32_t  app_n;
    // per-sequence key counts (ragged != 0): sequence b attends keys
    // [0, r_n_kv[b]) in r_ns[b] splits of r_split_len[b] keys, which are units
    // r_ustart[b] .. r_ustart[b+1]-1; ns above is the largest r_ns (the stride
    // of the split partials)
    int32_t  ragged;
    int32_t  r_units;      // units of all sequences (r_ustart[B])
    int32_t  r_ustart[RAGGED_MAX_B + 1];
    int32_t  r_ns[RAGGED_MAX_B];
    int32_t  r_split_len[RAGGED_MAX_B];
    int64_t  r_n_kv[RAGGED_MAX_B];
    // gathered keys (k_fa_dec / k_fa_vd <.., GATHER>): KV head h of sequence b
    // attends cache rows g_cells[b * g_bstride + h * g_hstride + j],
    // j < g_n[b * nh_kv + h]; query t of sequence b sees a row only if it is
    // at most g_pos0 + b + t (one list per KV head: B = 1; one list per query
    // position: each position is a sequence of one query, T = 1). The cache
    // has g_rows rows.
    const int32_t * g_cells;
    int64_t  g_bstride, g_hstride;
    int64_t  g_pos0;
    int64_t  g_rows;
    int32_t  g_n[GATHER_MAX_LISTS];
    uint32_t * status;     // device flags (DEVERR_GET_ROWS_INDEX: a cell outside the cache)
    // output gate (or null): dst = attention * sigmoid(gate), gate laid out as dst
    const float * gate;
    // split merge inside the attention kernel (k_fa_dec, k_fa_vd; null: a
    // k_fattn_merge launch follows): per (batch, KV head) group two words,
    // [arrived splits] and [claimed rows], each (call epoch << 16) | count;
    // m_ebase = this call's epoch << 16; the last m_nm splits to arrive may merge
    unsigned long long * mctr;
    unsigned long long m_ebase;
    int32_t  m_nm;
};

__device__ __forceinline__ uint32_t div_gqa(const fa_args & a, uint32_t r) {
    return udiv(r, (uint32_t) a.gqa, a.gqa_mul);
}
// v * sigmoid(gate) for the 4 dst values at d (16-byte aligned), sigmoid(x) =
// 1 / (1 + exp(-x)) as ggml_sigmoid, then ggml_mul's product; v as is
// without a gate
__device__ __forceinline__ float4 apply_gate(const fa_args & a, const float * d, float4 v) {
    if (!a.gate) return v;
    const float4 g = *(const float4 *) (a.gate + (d - a.dst));
    v.x = __fmul_rn(v.x, 1.0f / (1.0f + expf(-g.x)));
    v.y = __fmul_rn(v.y, 1.0f / (1.0f + expf(-g.y)));
    v.z = __fmul_rn(v.z, 1.0f / (1.0f + expf(-g.z)));
    v.w = __fmul_rn(v.w, 1.0f / (1.0f + expf(-g.w)));
    return v;
}
// b % n for a batch index b and a broadcast extent n (n is 1 or B in practice)
__device__ __forceinline__ int bmod(int b, int n) {
    return b < n ? b : b % n;
}

// The compiler's hazard recognizer does not see the VALU writes inside inline
// asm, and an MFMA that reads a VGPR needs two wait states after a VALU wrote
// it. Every asm below whose result can feed an MFMA operand therefore ends
// with s_nop 1.

// One V block's A operands for the lane's 4 keys: v[j] holds dims 2m, 2m+1 of
// key j in its low two bytes (one 2-byte LDS read each); a0[q] = f16 pair
// (dim 2m of keys 2q, 2q+1), a1[q] = f16 pair (dim 2m+1). int8 -> f16 is exact.
__device__ __forceinline__ void cvt_v_block(const uint32_t v[4], uint32_t a0[2], uint32_t a1[2]) {
#define QWFN_SDWA(D, S, DSEL, UNUSED, SSEL) "v_cvt_f16_i16_sdwa " D ", sext(" S ") dst_sel:" DSEL " dst_unused:" UNUSED " src0_sel:" SSEL "\n\t"
#define QWFN_PAIR(D, S0, S1, B) QWFN_SDWA(D, S0, "WORD_0", "UNUSED_PAD", B) QWFN_SDWA(D, S1, "WORD_1", "UNUSED_PRESERVE", B)
    asm(QWFN_PAIR("%0", "%4", "%5", "BYTE_0") QWFN_PAIR("%1", "%6", "%7", "BYTE_0")
        QWFN_PAIR("%2", "%4", "%5", "BYTE_1") QWFN_PAIR("%3", "%6", "%7", "BYTE_1")
        "s_nop 1"
        : "=&v"(a0[0]), "=&v"(a0[1]), "=&v"(a1[0]), "=&v"(a1[1])
        : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
#undef QWFN_PAIR
#undef QWFN_SDWA
}

// B operands of one V block: for key pairs q (keys 2q, 2q+1), P*d_v as an f16
// hi pair and an f16 lo pair. hi = f16(P16 * d_v) with P16 = P rounded toward
// zero to f16 (one packed multiply per pair; p16[q] is computed once per
// chunk); lo = f16(p*d_v - hi), each from one fused v_fma_mix on the f32 p, so
// hi + lo carries p*d_v to about 2^-21 whatever the rounding of hi. dv[q] holds
// the two keys' fp16 d_v.
__device__ __forceinline__ void pdv_hilo(const float p[4], const uint32_t p16[2], const uint32_t dv[2], uint32_t bh[2],
                                         uint32_t bl[2]) {
#define QWFN_HILO(H, L, P0, P1, P16, DV)                                                              \
    "v_pk_mul_f16 " H ", " P16 ", " DV "\n\t"                                                           \
    "v_fma_mixlo_f16 " L ", " P0 ", " DV ", -" H " op_sel:[0,0,0] op_sel_hi:[0,1,1]\n\t"                \
    "v_fma_mixhi_f16 " L ", " P1 ", " DV ", -" H " op_sel:[0,1,1] op_sel_hi:[0,1,1]\n\t"
    asm(QWFN_HILO("%0", "%2", "%4", "%5", "%8", "%10") QWFN_HILO("%1", "%3", "%6", "%7", "%9", "%11")
                 "s_nop 1"
                 : "=&v"(bh[0]), "=&v"(bh[1]), "=&v"(bl[0]), "=&v"(bl[1])
                 : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p16[0]), "v"(p16[1]), "v"(dv[0]), "v"(dv[1]));
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
// max of two scores (finite or -inf, never NaN) in one v_max_f32: fmaxf on an
// asm result gets both operands canonicalised first, and the ternary above is
// a compare plus a select
__device__ __forceinline__ float vmax(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

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
    return reduce_lanes16_32(x, [](float a, float b) { return vmax(a, b); });
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
// The same for a wave-uniform runtime count below 32 (a compare chain: for
// the prologue's one wait).
template <int N = 0>
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
    if constexpr (N < 32) {
        if (n == N) {
            wait_vmcnt<N>();
            return;
        }
        wait_vmcnt_upto<N + 1>(n);
    } else {
        wait_vmcnt<0>();
    }
}
// The counts a wave can leave in flight in the key loop (anything else waits
// for everything).
__device__ __forceinline__ void wait_vmcnt_n(int n) {
    switch (n) {
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        default: wait_vmcnt<0>(); break;
    }
}

// Buffer resource of `bytes` bytes at base (raw, 32-bit data format). Loads
// at offsets past `bytes` return zeros instead of touching memory.
__device__ __forceinline__ v4i make_rsrc(const void * base, uint32_t bytes) {
    const uint64_t p = (uint64_t) (uintptr_t) base;
    v4i r;
    r[0] = (int) (uint32_t) p;
    r[1] = (int) ((uint32_t) (p >> 32) & 0xffffu);   // stride 0
    r[2] = (int) bytes;
    r[3] = 0x00020000;                               // DATA_FORMAT 32
    return r;
}

// One wave-wide LDS-DMA load: lane i copies the 16 bytes at offset off of the
// buffer to LDS[lds_base + 16 * i] (zeros past the buffer's size). Issued as
// inline asm: the compiler neither reorders memory operations across it nor
// tracks it, and the kernel waits for it explicitly (vmcnt) before the barrier
// that publishes the data. No other vector-memory load is in flight while DMAs
// are, so the explicit counts are exact.
__device__ __forceinline__ void dma16_buf(v4i rsrc, uint32_t off, uint32_t lds_base) {
    // an LDS DMA reads M0 one wait state after the SALU write at the earliest
    // The asm writes M0 only (a reserved register that the compiler uses for
    // nothing else in these kernels): no instruction in it touches SCC, so the
    // compiler may keep a carry or a branch condition live across it.
    asm volatile("s_mov_b32 m0, %2\n\t"
                 "s_nop 0\n\t"
                 "buffer_load_dwordx4 %0, %1, 0 offen lds"
                 :: "v"(off), "s"(rsrc), "s"(lds_base) : "memory");
}

// The same with the LDS destination lds_base + lds_off, lds_off a constant.
// The addition is the compiler's: a scalar add in the asm would overwrite SCC,
// which the compiler may hold across the asm (the carry of a 64-bit pointer
// increment split around it), and a lost carry moves a buffer base by 4 GiB.
template <uint32_t LDS_OFF>
__device__ __forceinline__ void dma16_buf_at(v4i rsrc, uint32_t off, uint32_t lds_base) {
    dma16_buf(rsrc, off, lds_base + LDS_OFF);
}

// r with every component read from the first lane: a resource that the
// compiler cannot prove uniform (a value merged across branches, at low
// optimisation levels) is moved to scalar registers for the DMA asm; where it
// is already scalar, nothing is emitted.
__device__ __forceinline__ v4i uniform_rsrc(v4i r) {
    return v4i{__builtin_amdgcn_readfirstlane(r[0]), __builtin_amdgcn_readfirstlane(r[1]),
               __builtin_amdgcn_readfirstlane(r[2]), __builtin_amdgcn_readfirstlane(r[3])};
}

// num_records of a buffer resource for `rem` bytes (at most 2^32 - 1).
__device__ __forceinline__ uint32_t rsrc_bytes(int64_t rem) {
    uint32_t hi = (uint32_t) ((uint64_t) rem >> 32);
    asm("" : "+s"(hi));   // a 32-bit scalar test (the 64-bit compare it would fold into is a vector one)
    return hi ? 0xffffffffu : (uint32_t) rem;
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

// 16-byte store marked non-temporal (p 16-byte aligned).
__device__ __forceinline__ void store_nt4(float * p, float4 v) {
    __builtin_nontemporal_store(v4f{v.x, v.y, v.z, v.w}, (v4f *) p);
}

__device__ __forceinline__ float4 load_nt4(const float4 * p) {
    const v4f v = __builtin_nontemporal_load((const v4f *) p);
    return make_float4(v[0], v[1], v[2], v[3]);
}

// Device-scope (sc1) access to the split partials of an in-kernel merge
// (fa_merge_tail): the cache policy of the compiler's agent-scope relaxed
// atomics, under which a store is written through to where the loads of every
// XCD read and a load never returns another XCD's stale L2 copy. So the
// partials need no L2 write-back on the writer's side and no L2 invalidate on
// the merger's. Offsets are bytes from the resource's base (below 4 GiB: the
// host checks the partials' extent).
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
constexpr int CPOL_DEV = 16;   // sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void * base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, -1, 0x00020000);
}
__device__ __forceinline__ void store_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v4f{v.x, v.y, v.z, v.w}), r, (int) off, 0, CPOL_DEV);
}
__device__ __forceinline__ void store_dev2(__amdgpu_buffer_rsrc_t r, uint32_t off, float2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), r, (int) off, 0, CPOL_DEV);
}
__device__ __forceinline__ float4 load_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const v4f v = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, (int) off, 0, CPOL_DEV));
    return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float2 load_dev2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, (int) off, 0, CPOL_DEV));
}

// f[0 .. n) = 0 (dst is only 4-byte aligned, so plain f32 stores).
__global__ void k_zero_f32(float * f, int64_t n) {
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) f[i] = 0.f;
}

// RG: per-sequence splits (the ragged table of fa_args); a template parameter
// so that the block mapping of the other calls carries none of it
template <int RT, bool MT, int NW, int KWV, bool RG>
__global__ __launch_bounds__(NW * 64, NW / 4 > 2 ? NW / 4 : 2) void k_fattn_q8_0(fa_args a) {
    using C = fa_cfg<RT, MT, NW, KWV>;
    // the argument block's pointers are loaded with the rest, in one round of
    // scalar loads (not a second round after the exit of padding blocks)
    asm volatile("" :: "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.mask), "s"(a.m_ne2), "s"(a.mask_mode), "s"(a.part_o));
    constexpr int WAVES = NW;
    constexpr int KW = KWV;              // keys per wave per chunk
    constexpr int NKT = C::NKT;
    constexpr int ROWS = C::ROWS, KG = C::KG, CK = C::CK, VOFF = C::VOFF, DMA_T = C::DMA_T;
    constexpr int SLOTS = C::SLOTS, SPW = C::SPW, NS = C::NS;
    // NS ring stages, each K rows [CK][272] and V rows [CK][272]
    __shared__ __attribute__((aligned(16))) uint8_t ring[NS][C::STAGE];
    // per-wave scale tables of the current chunk: [K|V][block][key of the wave] fp16
    __shared__ __attribute__((aligned(16))) uint16_t scl[WAVES][2][NBLK][KW];
    // the block's mask rows over its whole split (MASK_SPLIT mode): [row][split_len] F16
    __shared__ __attribute__((aligned(16))) uint16_t mlds[C::MLDS / 2];
    static_assert(ROWS * NBLK * QWIN + ROWS * NBLK * 4 <= C::STAGE, "query image fits in the last stage");
    static_assert(ROWS * (D + 4) * 4 + WAVES * 16 * 8 <= C::STAGE, "merge buffer fits in stage 0");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
    const int ln = lane & 15;       // MFMA row/col within a 16-tile
    const int lg = lane >> 4;       // lane group (k-slice / output row quad)
    const int tile = wave % RT;     // query rows 16*tile .. 16*tile+15 of the block
    const int kg = wave / RT;       // keys 16*kg .. 16*kg+15 of every chunk

    // ---- block -> (b, kvh, row group, split). With at least 8 (batch, split)
    //      units, the KV heads and row groups of one unit go to one XCD
    //      (blockIdx % 8); with fewer, consecutive blocks spread them ----
    const int id   = blockIdx.x;
    const int hgn  = a.nh_kv * a.n_rg;
    const int n_units = RG ? a.r_units : a.B * a.ns;
    int hg, u;
    if (n_units >= 8) {
        const int j = id >> 3;
        const int jq = (int) udiv((uint32_t) j, (uint32_t) hgn, a.hgn_mul);
        hg = j - jq * hgn;
        u  = jq * 8 + (id & 7);
    } else {
        u  = (int) udiv((uint32_t) id, (uint32_t) hgn, a.hgn_mul);
        hg = id - u * hgn;
    }
    const int kvh  = (int) udiv((uint32_t) hg, (uint32_t) a.n_rg, a.nrg_mul);
    const int rg   = hg - kvh * a.n_rg;
    if (u >= n_units) return;                      // padding of the XCD mapping
    int b, split;
    int64_t k_lo, k_hi;
    if constexpr (RG) {
        // the sequence whose units hold u; constant indices keep the table
        // reads scalar (an indexed read of the argument block is not)
        int32_t us = 0, nsb = 1, slb = 0;
        int64_t nkb = 0;
        b = 0;
#pragma unroll
        for (int i = 0; i < RAGGED_MAX_B; i++)
            if (i < a.B && u >= a.r_ustart[i]) {
                b = i; us = a.r_ustart[i]; nsb = a.r_ns[i]; slb = a.r_split_len[i]; nkb = a.r_n_kv[i];
            }
        split = u - us;
        k_lo = (int64_t) split * slb;
        const int64_t e = k_lo + slb;     // ternaries, not std::min: its reference result put a copy on the stack
        k_hi = split == nsb - 1 ? nkb : (nkb < e ? nkb : e);
    } else {
        b = (int) udiv((uint32_t) u, (uint32_t) a.ns, a.ns_mul);
        split = u - b * a.ns;
        k_lo = (int64_t) split * a.split_len;
        // the last split runs to n_kv (it may hold up to one chunk more than split_len)
        const int64_t e = k_lo + a.split_len;
        k_hi = split == a.ns - 1 ? a.n_kv : (a.n_kv < e ? a.n_kv : e);
    }
    const int n_chunks = (int) ((k_hi - k_lo + CK - 1) / CK);
    const int r0 = rg * a.rw;                          // first query row of this block
    const int RW = std::min(a.rw, a.R - r0);          // rows in this block
    const int t0 = (int) div_gqa(a, (uint32_t) r0);

    const char * kbase = a.k + (size_t) bmod(b, a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) bmod(b, a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;
    // Mask rows of this block: query position t0 + mr for a shared mask, query
    // row r0 + mr for a per-head one. Byte offset of row mr from the mask's
    // batch slice (`mslice`, its start rounded down to 16 bytes).
    const int n_mrows = a.mask_mode == MASK_NONE ? 0 : (a.m_ne2 == 1 ? (int) div_gqa(a, (uint32_t) (r0 + RW - 1)) - t0 + 1 : RW);
    const char * mslice = a.mask + (size_t) bmod(b, a.m_ne3) * a.m_nb3;
    const char * mslice_al = (const char *) ((uintptr_t) mslice & ~(uintptr_t) 15);
    auto mrow_off = [&](int mr) -> uint32_t {
        int t = t0 + mr, hq = 0;
        if (a.m_ne2 != 1) {
            const int r = r0 + mr;
            t = (int) div_gqa(a, (uint32_t) r);
            hq = (kvh * a.gqa + (r - t * a.gqa)) % a.m_ne2;
        }
        return (uint32_t) (mslice - mslice_al) + (uint32_t) ((size_t) t * a.m_nb1 + (size_t) hq * a.m_nb2);
    };
    const int n_mdma = MT ? (n_mrows * C::MGR + 63) / 64 : 0;

    // ---- prologue. What the block needs before its key loop travels as LDS
    //      DMA, in this order: its query rows (f32, into the last ring stage),
    //      its MASK_SPLIT mask rows, chunk 0 (and chunk 1 with three stages).
    //      One wait that leaves the chunk DMAs in flight covers the first two
    //      (the counter is in order), and the block requantises its query rows
    //      while the chunks arrive ----
    uint8_t * qstage = ring[NS - 1];    // [ROWS][D] f32 query rows, then the window image below
    {
        // one wave-wide DMA (1 KB) per query row; wave w takes rows w, w + NW, ...
        const v4i rq = make_rsrc(a.q + (size_t) b * a.q_nb3, a.q_slice);
#pragma unroll
        for (int j = 0; j < (ROWS + WAVES - 1) / WAVES; j++) {
            const int rl = wave + WAVES * j;
            if (rl >= RW) break;
            const uint32_t r = (uint32_t) (r0 + rl);
            const uint32_t t = div_gqa(a, r), h = (uint32_t) (kvh * a.gqa) + (r - t * (uint32_t) a.gqa);
            dma16_buf(rq, t * (uint32_t) a.q_nb1 + h * (uint32_t) a.q_nb2 + 16u * (uint32_t) lane,
                      __builtin_amdgcn_readfirstlane(lds_addr(qstage + rl * 1024)));
        }
    }
    // MASK_SPLIT: mask row mr of the split lands at byte mr * mstride of mlds as
    // the 16-byte granules from the aligned address at or below its first key,
    // which sits `mis` bytes into the LDS row. Granule g = 64m + lane is granule
    // g % m_gran of row g / m_gran; lanes past the last granule re-read it, so
    // every LDS byte a DMA writes lies inside mlds.
    const bool msplit = !MT && a.mask_mode == MASK_SPLIT;
    const uint32_t mstride = 16u * (uint32_t) a.m_gran;
    if (msplit) {
        const int n_g = n_mrows * a.m_gran;
        const v4i rm = make_rsrc(mslice_al, a.m_slice + (uint32_t) (mslice - mslice_al));
        for (int m = wave; m * 64 < n_g; m += WAVES) {
            const uint32_t g = (uint32_t) std::min(m * 64 + lane, n_g - 1);
            const uint32_t row = __umulhi(g, a.m_gran_mul);
            const uint32_t k = g - row * (uint32_t) a.m_gran;
            const uint32_t src = ((mrow_off((int) row) + 2u * (uint32_t) k_lo) & ~15u) + 16u * k;
            dma16_buf(rm, src, __builtin_amdgcn_readfirstlane(lds_addr((uint8_t *) mlds + m * 1024)));
        }
    }

    // A chunk is SLOTS wave-wide 16-byte DMAs; slot s lands at byte 1024*s of
    // the stage: slots [0, DMA_T) are the K rows (piece p = 64*s + lane is byte
    // 16*(p % 17) of key p / 17; when the rows end inside the last DMA, its
    // remaining lanes read the next rows into the padding before VOFF), the
    // next DMA_T the V rows, then (MASK_TILE) the mask rows, granule
    // G = 64*m + lane being granule G % MGR of row G / MGR. Wave w issues slots
    // w, w + NW, ... The lane offsets within a chunk are the same for every
    // chunk.
    auto slot_off = [&](int slot) -> uint32_t {
        if (slot < 2 * DMA_T) {
            const int tensor = slot >= DMA_T;
            const unsigned p = (unsigned) ((slot - tensor * DMA_T) * 64 + lane);
            const unsigned key = p / 17u, part = p - key * 17u;
            return key * (unsigned) (tensor ? a.v_nb1 : a.k_nb1) + part * 16u;
        }
        if (MT && slot < SLOTS) {
            const int g = (slot - 2 * DMA_T) * 64 + lane;
            const int mr = std::min(g / C::MGR, n_mrows - 1);   // lanes past the rows re-read the last one
            return (mrow_off(mr) & ~15u) + 16u * (unsigned) (g % C::MGR);
        }
        return 0u;
    };
    auto slot_live = [&](int slot) -> bool {
        return slot < 2 * DMA_T || (MT && slot < SLOTS && slot - 2 * DMA_T < n_mdma);
    };
    uint32_t doff[SPW];
#pragma unroll
    for (int s = 0; s < SPW; s++) doff[s] = slot_off(wave + WAVES * s);
    // DMAs this wave issues per chunk: the count a wait leaves in flight for
    // the chunk issued after the one it waits for
    int ops_per_chunk = 0;
#pragma unroll
    for (int s = 0; s < SPW; s++) ops_per_chunk += slot_live(wave + WAVES * s) ? 1 : 0;
    // the lane's own mask row in a MASK_TILE stage: row start plus the row's
    // offset from its 16-byte granule
    const int rl_lane0 = 16 * tile + ln;
    const int mrow0 = rl_lane0 >= RW ? 0 : (a.m_ne2 == 1 ? (int) div_gqa(a, (uint32_t) (r0 + rl_lane0)) - t0 : rl_lane0);
    const uint32_t mtile_off = MT ? (uint32_t) (mrow0 * C::MGR * 16) + (mrow_off(mrow0) & 15u) : 0u;
    // the lane's mask row in mlds (MASK_SPLIT)
    const uint32_t mlds_row = msplit ? (uint32_t) mrow0 * mstride + ((mrow_off(mrow0) + 2u * (uint32_t) k_lo) & 15u) : 0u;

    // Chunk c is read through buffer resources based at its first key and
    // ending at the split's last key: rows past the split arrive as zeros
    // without a memory access, and those keys are masked.
    const int64_t k_bytes = k_hi * (int64_t) a.k_nb1, v_bytes = k_hi * (int64_t) a.v_nb1;
    auto issue_chunk = [&](int c, uint8_t * dstb) __attribute__((always_inline)) {
        const int64_t c0 = k_lo + (int64_t) c * CK;
        const int64_t kc = c0 * (int64_t) a.k_nb1, vc = c0 * (int64_t) a.v_nb1;
        const v4i rk = make_rsrc(kbase + kc, (uint32_t) std::min<int64_t>(k_bytes - kc, 0xffffffffll));
        const v4i rv = make_rsrc(vbase + vc, (uint32_t) std::min<int64_t>(v_bytes - vc, 0xffffffffll));
#pragma unroll
        for (int s = 0; s < SPW; s++) {
            const int slot = wave + WAVES * s;
            if (slot >= 2 * DMA_T) continue;
            dma16_buf(slot < DMA_T ? rk : rv, doff[s], __builtin_amdgcn_readfirstlane(lds_addr(dstb + slot * 1024)));
        }
        if constexpr (MT) {
            // mask granules: the chunk's first key (a multiple of 8) is 16-byte aligned within a row
            const v4i rm = make_rsrc(mslice_al + c0 * 2, (uint32_t) (a.m_slice + (uint32_t) (mslice - mslice_al) - c0 * 2));
#pragma unroll
            for (int s = 0; s < SPW; s++) {
                const int slot = wave + WAVES * s;
                if (slot < 2 * DMA_T || !slot_live(slot)) continue;
                dma16_buf(rm, doff[s], __builtin_amdgcn_readfirstlane(lds_addr(dstb + slot * 1024)));
            }
        }
    };

    // Fused append: a block whose keys include appended rows quantises its KV
    // head's part of them into the cache (the arithmetic of k_append_q8_0, 8
    // lanes per q8_0 block) and waits for the stores before any of its chunk
    // DMAs, which then read the new rows from memory. Blocks of other row
    // groups write the same bytes; each reads only after its own stores.
    if (a.app_n > 0) {
        const int64_t alo = std::max<int64_t>(a.app_row0, k_lo), ahi = std::min<int64_t>(a.app_row0 + a.app_n, k_hi);
        if (alo < ahi) {
            const int units = (int) (ahi - alo) * NBLK * 2;   // rows x blocks x {K, V}
            const int sub = threadIdx.x & 7;
            for (int u0 = 0; u0 < units; u0 += WAVES * 8) {
                const int u = u0 + (int) (threadIdx.x >> 3);
                const bool live = u < units;                  // whole 8-lane groups: DPP partners exist
                const int uu = live ? u : 0;
                const int tensor = uu & 1, jb = (uu >> 1) % NBLK;
                const int64_t row = alo + (uu >> 1) / NBLK;
                const float4 xv = *(const float4 *) ((tensor ? a.app_v : a.app_k) + (size_t) (row - a.app_row0) * a.app_nb1 +
                                                     (size_t) (kvh * D + QK * jb + 4 * sub) * 4);
                float x[4] = {xv.x, xv.y, xv.z, xv.w};
                uint16_t d16;
                float dqa;
                const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dqa);
                if (live) {
                    char * bp = (char *) (tensor ? vbase + (size_t) row * a.v_nb1 : kbase + (size_t) row * a.k_nb1) + jb * QBLOCK;
                    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
                    qp[0] = (uint16_t) (q4 & 0xffffu);
                    qp[1] = (uint16_t) (q4 >> 16);
                    if (sub == 0) *(uint16_t *) bp = d16;
                }
            }
            wait_vmcnt<0>();      // this wave's stores (and its query DMAs) are done
            __syncthreads();      // ... and every wave's
        }
    }

    issue_chunk(0, ring[0]);
    int chunk_ops = ops_per_chunk;
    if constexpr (NS > 2) {
        if (n_chunks > 1) {
            issue_chunk(1, ring[1]);
            chunk_ops += ops_per_chunk;
        }
    }
    wait_vmcnt_upto(chunk_ops);   // this wave's query and mask DMAs have landed
    __syncthreads();              // ... and every wave's

    // Requantisation: QL lanes per (row, block), QV values each; wave w takes
    // blocks w, w + NW, ... for all rows (QL * ROWS = 64 lanes).
    constexpr int QL = 64 / ROWS, QV = 32 / QL, QIT = (NBLK + WAVES - 1) / WAVES;
    static_assert(QL * ROWS == 64 && (NBLK % WAVES == 0 || WAVES > NBLK), "one block of all rows per wave and iteration");
    const int qrl = lane / QL, qh = lane % QL;
    float qx[QIT][QV];
#pragma unroll
    for (int it = 0; it < QIT; it++) {
        const int blk = std::min(wave + WAVES * it, NBLK - 1);      // waves past the blocks read one, unused
        const float4 * src = (const float4 *) (qstage + qrl * 1024 + (QK * blk + QV * qh) * 4);
#pragma unroll
        for (int m = 0; m < QV / 4; m++) {
            const float4 v = qrl < RW ? src[m] : make_float4(0.f, 0.f, 0.f, 0.f);
            qx[it][4 * m] = v.x; qx[it][4 * m + 1] = v.y; qx[it][4 * m + 2] = v.z; qx[it][4 * m + 3] = v.w;
        }
    }
    __syncthreads();   // every query value is in registers: the stage becomes the window image

    uint8_t * qwin = qstage;                                        // [ROWS][NBLK][QWIN] windows
    float * dql = (float *) (qstage + ROWS * NBLK * QWIN);          // [ROWS][NBLK] d_q * scale * log2(e)
    {
        const float fs = a.scale * LOG2E;
#pragma unroll
        for (int it = 0; it < QIT; it++) {
            const int blk = wave + WAVES * it;
            if (WAVES > NBLK && blk >= NBLK) break;
            uint8_t * wrow = qwin + (qrl * NBLK + blk) * QWIN;
            // the lane's share of the window is zeroed first; the quants that
            // follow (written by lanes of this wave, whose LDS writes complete
            // in order) overwrite their part of it
#pragma unroll
            for (int z = 0; z < 4 / QL; z++) ((uint4 *) wrow)[qh * (4 / QL) + z] = make_uint4(0, 0, 0, 0);
            wave_lds_sync();
            uint32_t w[QV / 4];
            uint16_t d16;
            float dq = 0.f;
            if (a.x86) dev::q8_quantize_lanes<QV>(qx[it], true, w, &d16, &dq);
            else       dev::q8_quantize_lanes<QV>(qx[it], false, w, &d16, &dq);
            if (qrl < RW) {                                     // padding rows keep zero windows
                uint16_t * wp = (uint16_t *) (wrow + win_off(blk) + QV * qh);
#pragma unroll
                for (int m = 0; m < QV / 4; m++) {
                    wp[2 * m] = (uint16_t) w[m];
                    wp[2 * m + 1] = (uint16_t) (w[m] >> 16);
                }
            }
            if (qh == 0) dql[qrl * NBLK + blk] = qrl < RW ? dq * fs : 0.f;
        }
    }
    __syncthreads();
    const int rl_lane = 16 * tile + ln;                 // this lane's query row (MFMA column)
    v4i qw[NBLK];                                       // B operands of QK: window slice lg of each block
    float dq[NBLK];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        qw[bb] = *(const v4i *) (qwin + (rl_lane * NBLK + bb) * QWIN + 16 * lg);
        dq[bb] = dql[rl_lane * NBLK + bb];
    }
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) asm volatile("" : "+v"(qw[bb]), "+v"(dq[bb]));   // read before the stage is reused


    // ---- online softmax state of the lane's row ----
    v4f   O[NBLK][2];
    float m_run = -INFINITY, l_run = 0.f;
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) { O[bb][0] = v4f{0, 0, 0, 0}; O[bb][1] = v4f{0, 0, 0, 0}; }

    const int span = (int) (k_hi - k_lo);               // keys of this split
    uint16_t (*sw)[NBLK][KW] = scl[wave];

    // One chunk: `cur` holds chunk c; chunk c+NS-1 goes to `nxt` (chunk c-1's
    // stage). Called with the ring stages literally so the compiler can tell
    // them apart.
    auto chunk_step = [&](int c, uint8_t * cur, uint8_t * nxt) __attribute__((always_inline)) {
        // Wait for chunk c; with three stages chunk c+1 (issued one step
        // earlier) may stay in flight. The barrier publishes every wave's part
        // and tells all of them that `nxt` is no longer read.
        if (NS > 2 && c + 1 < n_chunks) wait_vmcnt_n(ops_per_chunk);
        else wait_vmcnt<0>();
        __syncthreads();
        if (c + NS - 1 < n_chunks) issue_chunk(c + NS - 1, nxt);

        // A wave whose keys are all past the split, or (MASK_TILE, where long
        // causal masks come) all masked (-inf) for all its rows, has nothing
        // to add for this chunk. The lane's keys are 16*kt + 4*lg + i of the
        // wave's KW (key tile kt, i = 0..3).
        const int kin = c * CK + kg * KW + lg * 4;               // the lane's first key of tile 0 in the split
        uint32_t mv[NKT][4];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) mv[kt][i] = 0;
        if constexpr (MT) {
            const uint8_t * mp = cur + 2 * VOFF + mtile_off + 2 * (kg * KW + lg * 4);
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) mv[kt][i] = *(const uint16_t *) (mp + 32 * kt + 2 * i);
            bool live = false;
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) live |= kin + 16 * kt + i < span && mv[kt][i] != 0xFC00u;
            if (!__any(live)) return;
        } else if (c * CK + kg * KW >= span) {
            return;
        }
        // The rest of the step, for the wave's first NL key tiles: a tile
        // whose keys are all past the split (the last chunk of a split) is
        // neither multiplied nor converted.
        auto compute = [&](auto nl_tag) __attribute__((always_inline)) {
        constexpr int NL = decltype(nl_tag)::value;
        // this wave's keys' block scales, transposed to [block][key]: entry n of
        // a lane is tensor n / (2 NKT), key (n % (2 NKT)) * 8 + lane / 8, block lane % 8
        {
            constexpr int NE = 4 * NKT;
            const uint8_t * src = cur + (kg * KW + (lane >> 3)) * SEG + (lane & 7) * QBLOCK;
            uint16_t * dstw = &sw[0][lane & 7][lane >> 3];
            uint16_t sv[NE];
#pragma unroll
            for (int n = 0; n < NE; n++) sv[n] = *(const uint16_t *) (src + (n / (2 * NKT)) * VOFF + (n % (2 * NKT)) * 8 * SEG);
#pragma unroll
            for (int n = 0; n < NE; n++) dstw[(n / (2 * NKT)) * NBLK * KW + (n % (2 * NKT)) * 8] = sv[n];
        }
        wave_lds_sync();

        // ---- S = Q K^T for the wave's key tiles (MFMA rows) x 16 query rows ----
        float s[NKT][4];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) s[kt][i] = 0.f;
        // QKB blocks at a time: their K and scale reads, then their MFMAs, then
        // the scaling, so the reads' and the MFMAs' latencies overlap (with two
        // key tiles, all eight blocks at once would not fit the registers)
        constexpr int QKB = NKT == 1 ? NBLK : NBLK / 2;
#pragma unroll
        for (int b0 = 0; b0 < NBLK; b0 += QKB) {
            v4i kA[QKB][NKT];
            uint2 dk[QKB][NKT];
#pragma unroll
            for (int u = 0; u < QKB; u++)
#pragma unroll
                for (int kt = 0; kt < NL; kt++) {
                    // A operand: key row 16*kt + ln of the wave, window slice lg
                    const uint8_t * krow = cur + (kg * KW + 16 * kt + ln) * SEG + 16 * lg;
                    kA[u][kt] = *(const v4i *) (krow + 16 * win_piece(b0 + u));
                    dk[u][kt] = *(const uint2 *) &sw[0][b0 + u][16 * kt + lg * 4];   // the lane's 4 keys' fp16 d_k
                }
            v4i cc[QKB][NKT];
#pragma unroll
            for (int u = 0; u < QKB; u++)
#pragma unroll
                for (int kt = 0; kt < NL; kt++)
                    cc[u][kt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[u][kt], qw[b0 + u], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int u = 0; u < QKB; u++)
#pragma unroll
                for (int kt = 0; kt < NL; kt++) {
                    const float d = dq[b0 + u];
                    if constexpr (NKT == 1) {
                        s[kt][0] = __builtin_fmaf((float) cc[u][kt][0], mul_f16lo(d, dk[u][kt].x), s[kt][0]);
                        s[kt][1] = __builtin_fmaf((float) cc[u][kt][1], mul_f16hi(d, dk[u][kt].x), s[kt][1]);
                        s[kt][2] = __builtin_fmaf((float) cc[u][kt][2], mul_f16lo(d, dk[u][kt].y), s[kt][2]);
                        s[kt][3] = __builtin_fmaf((float) cc[u][kt][3], mul_f16hi(d, dk[u][kt].y), s[kt][3]);
                    } else {
                        // (sum * d_q) * d_k: no scale product is formed (and
                        // held) ahead of the MFMA results (the register budget
                        // of 32-key waves)
                        s[kt][0] = fma_f16lo(dk[u][kt].x, (float) cc[u][kt][0] * d, s[kt][0]);
                        s[kt][1] = fma_f16hi(dk[u][kt].x, (float) cc[u][kt][1] * d, s[kt][1]);
                        s[kt][2] = fma_f16lo(dk[u][kt].y, (float) cc[u][kt][2] * d, s[kt][2]);
                        s[kt][3] = fma_f16hi(dk[u][kt].y, (float) cc[u][kt][3] * d, s[kt][3]);
                    }
                }
            if (b0 + QKB < NBLK) __builtin_amdgcn_sched_barrier(0);
        }

        // ---- mask, online softmax (base 2; scores are already in log2 units).
        //      A masked key has x = -inf, so its p is exp2(-inf) = 0 ----
        float p[NKT][4];
        uint32_t p16[NKT][2];   // p rounded toward zero to f16, key pairs (0,1), (2,3)
        {
            const bool tail = (c + 1) * CK > span;                // keys past the split in this chunk
            float x[NKT][4];
            float mloc = -INFINITY;
            if (msplit) {
                const uint16_t * mp = (const uint16_t *) ((const uint8_t *) mlds + mlds_row) + kin;
#pragma unroll
                for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) mv[kt][i] = mp[16 * kt + i];
            }
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    x[kt][i] = a.mask_mode != MASK_NONE ? fma_f16lo(mv[kt][i], LOG2E, s[kt][i]) : s[kt][i];
            if (tail) {   // uniform: only the last chunk of a split has keys past its end
#pragma unroll
                for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (kin + 16 * kt + i >= span) x[kt][i] = -INFINITY;
            }
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) mloc = vmax(mloc, x[kt][i]);
            mloc = xmax_lanes16_32(mloc);
            // the running max moves only when the chunk's max exceeds it by more
            // than RESCALE_SLACK (or it is still -inf), so p <= 2^RESCALE_SLACK
            const bool grow = mloc > m_run + RESCALE_SLACK;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(m_run - mloc);
                m_run = mloc;
            }
            const float m_use = m_run == -INFINITY ? 0.f : m_run;   // all keys masked so far
            float lsum = 0.f;
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    p[kt][i] = __builtin_amdgcn_exp2f(x[kt][i] - m_use);
                    lsum += p[kt][i];
                }
            l_run = l_run * alpha + lsum;
#pragma unroll
            for (int kt = 0; kt < NKT; kt++) {
                p16[kt][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[kt][0], p[kt][1]));
                p16[kt][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[kt][2], p[kt][3]));
            }
            if (__any(grow)) {
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[bb][0] *= alpha; O[bb][1] *= alpha; }
            }
        }

        // ---- O += V^T P per V block. Tile e of block bb holds dims 32bb + 2m + e
        //      (m = MFMA row); the A operand of lane (m, g) is dims 2m, 2m+1 of the
        //      lane's keys (16kt + 4g .. 16kt + 4g + 3), one naturally aligned
        //      2-byte LDS read per key. With two key tiles the reduction index
        //      4kt + i of the 16x16x32 MFMA is key 16kt + 4g + i, in the A and the
        //      B operand alike ----
        const uint8_t * vrow = cur + VOFF + (kg * KW + lg * 4) * SEG + 2 + 2 * ln;
        // PVB blocks at a time: all their LDS reads first (one 2-byte read per
        // key and block, each in its own register), so their latencies overlap
        constexpr int PVB = PV_BATCH;
#pragma unroll
        for (int b0 = 0; b0 < NBLK; b0 += PVB) {
            uint32_t w[PVB][NKT][4];
            uint2 dv2[PVB][NKT];
#pragma unroll
            for (int u = 0; u < PVB; u++)
#pragma unroll
                for (int kt = 0; kt < NL; kt++) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        w[u][kt][j] = *(const uint16_t *) (vrow + (16 * kt + j) * SEG + (b0 + u) * QBLOCK);
                    dv2[u][kt] = *(const uint2 *) &sw[1][b0 + u][16 * kt + lg * 4];
                }
#pragma unroll
            for (int u = 0; u < PVB; u++) {
                const int bb = b0 + u;
                uint32_t a0[NKT][2], a1[NKT][2], bh[NKT][2], bl[NKT][2];
#pragma unroll
                for (int kt = 0; kt < NKT; kt++) {
                    if (kt < NL) {
                        const uint32_t dv[2] = {dv2[u][kt].x, dv2[u][kt].y};
                        cvt_v_block(w[u][kt], a0[kt], a1[kt]);
                        pdv_hilo(p[kt], p16[kt], dv, bh[kt], bl[kt]);
                    } else {
                        // a key tile wholly past the split: zero operands
                        a0[kt][0] = a0[kt][1] = a1[kt][0] = a1[kt][1] = 0u;
                        bh[kt][0] = bh[kt][1] = bl[kt][0] = bl[kt][1] = 0u;
                    }
                }
                if constexpr (NKT == 1) {
                    const v4h A0 = __builtin_bit_cast(v4h, make_uint2(a0[0][0], a0[0][1]));
                    const v4h A1 = __builtin_bit_cast(v4h, make_uint2(a1[0][0], a1[0][1]));
                    const v4h Bh = __builtin_bit_cast(v4h, make_uint2(bh[0][0], bh[0][1]));
                    const v4h Bl = __builtin_bit_cast(v4h, make_uint2(bl[0][0], bl[0][1]));
                    O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bh, O[bb][0], 0, 0, 0);
                    O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bh, O[bb][1], 0, 0, 0);
                    O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bl, O[bb][0], 0, 0, 0);
                    O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bl, O[bb][1], 0, 0, 0);
                } else {
                    const v8h A0 = __builtin_bit_cast(v8h, make_uint4(a0[0][0], a0[0][1], a0[1][0], a0[1][1]));
                    const v8h A1 = __builtin_bit_cast(v8h, make_uint4(a1[0][0], a1[0][1], a1[1][0], a1[1][1]));
                    const v8h Bh = __builtin_bit_cast(v8h, make_uint4(bh[0][0], bh[0][1], bh[1][0], bh[1][1]));
                    const v8h Bl = __builtin_bit_cast(v8h, make_uint4(bl[0][0], bl[0][1], bl[1][0], bl[1][1]));
                    O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bh, O[bb][0], 0, 0, 0);
                    O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bh, O[bb][1], 0, 0, 0);
                    O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bl, O[bb][0], 0, 0, 0);
                    O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bl, O[bb][1], 0, 0, 0);
                }
            }
        }
        };
        if constexpr (NKT == 2) {
            if (c * CK + kg * KW + 16 >= span) {
                compute(std::integral_constant<int, 1>{});
                return;
            }
        }
        compute(std::integral_constant<int, NKT>{});
    };
    if constexpr (NS == 3) {
        for (int c = 0; c < n_chunks; c += 3) {
            chunk_step(c, ring[0], ring[2]);
            if (c + 1 < n_chunks) chunk_step(c + 1, ring[1], ring[0]);
            if (c + 2 < n_chunks) chunk_step(c + 2, ring[2], ring[1]);
        }
    } else {
        for (int c = 0; c < n_chunks; c += 2) {
            chunk_step(c, ring[0], ring[1]);
            if (c + 1 < n_chunks) chunk_step(c + 1, ring[1], ring[0]);
        }
    }
    // ---- merge the key groups of each row tile: every wave publishes (max,
    //      sum) per row in its own scale table (no other wave uses it), and
    //      after one barrier the groups 1 .. KG-1 store their weighted O into
    //      buffers of their own in the ring; after a second, group 0 adds them
    //      to its own and writes the block's result ----
    {
        const float l = sum_lanes16_32(l_run);
        float2 * mlw = (float2 *) &scl[wave][0][0][0];
        if (lg == 0) mlw[ln] = make_float2(m_run, l);
    }
    __syncthreads();   // every wave is done with the last chunk, and its (max, sum) are out
    // [NBUF][ROWS][OBS] f32, natural dim order; the padded row stride puts the
    // 16 rows a float4 access touches on different banks. With more groups
    // than buffers fit in the ring, they take turns (ROUNDS).
    constexpr int OBS = D + 4;
    constexpr int NBUF = std::min(KG - 1, NS * C::STAGE / (ROWS * OBS * 4));
    constexpr int ROUNDS = KG == 1 ? 0 : (KG - 1 + NBUF - 1) / NBUF;
    static_assert(KG == 1 || NBUF >= 1, "a group buffer fits in the ring");
    float M = -INFINITY, L = 0.f;
#pragma unroll
    for (int k2 = 0; k2 < KG; k2++) M = xmax(M, ((const float2 *) &scl[k2 * RT + tile][0][0][0])[ln].x);
#pragma unroll
    for (int k2 = 0; k2 < KG; k2++) {
        const float2 e = ((const float2 *) &scl[k2 * RT + tile][0][0][0])[ln];
        L += e.x == -INFINITY ? 0.f : e.y * exp2f(e.x - M);
    }
    const float fw = m_run == -INFINITY ? 0.f : exp2f(m_run - M);
    // Lane (ln, lg) holds dims 32bb + 8lg + 2i + e of row 16*tile + ln in
    // O[bb][e][i]. Lane indices are re-derived here (an opaque copy of the
    // thread id), so no output address stays live through the key loop.
    int tid_e = (int) threadIdx.x;
    asm volatile("" : "+v"(tid_e));
    const int ln_e = tid_e & 15, lg_e = (tid_e >> 4) & 3;
    const int rl = 16 * tile + ln_e;
    float * ob = (float *) &ring[0][0];
    const int orow = rl * OBS + 8 * lg_e;          // the lane's first float in a group buffer
    // the lane's 8 dims of block bb in natural order: acc[bb][0] dims 0..3, acc[bb][1] dims 4..7
    float4 acc[NBLK][2];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        const v4f o0 = O[bb][0] * fw, o1 = O[bb][1] * fw;
        acc[bb][0] = make_float4(o0[0], o1[0], o0[1], o1[1]);
        acc[bb][1] = make_float4(o0[2], o1[2], o0[3], o1[3]);
    }
    for (int rd = 0; rd < ROUNDS; rd++) {
        if (kg != 0 && (kg - 1) / NBUF == rd) {
            float * d = ob + ((kg - 1) % NBUF) * ROWS * OBS + orow;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                *(float4 *) (d + 32 * bb) = acc[bb][0];
                *(float4 *) (d + 32 * bb + 4) = acc[bb][1];
            }
        }
        __syncthreads();
        if (kg == 0 && rl < RW) {
            const int nb = std::min(NBUF, KG - 1 - rd * NBUF);
            for (int k2 = 0; k2 < nb; k2++) {
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) {
                    const float * src = ob + k2 * ROWS * OBS + orow + 32 * bb;
                    const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
                    acc[bb][0].x += x0.x; acc[bb][0].y += x0.y; acc[bb][0].z += x0.z; acc[bb][0].w += x0.w;
                    acc[bb][1].x += x1.x; acc[bb][1].y += x1.y; acc[bb][1].z += x1.z; acc[bb][1].w += x1.w;
                }
            }
        }
        if (rd + 1 < ROUNDS) __syncthreads();   // the buffers are read before the next round overwrites them
    }
    if (kg != 0 || rl >= RW) return;
    const size_t bh = (size_t) b * a.nh_kv + kvh;
    const bool vec = a.ns > 1 || a.dst_vec;
    const int r = r0 + rl;
    const int tq = (int) div_gqa(a, (uint32_t) r), h = kvh * a.gqa + (r - tq * a.gqa);
    float * out;
    float oscale;
    if (a.ns == 1) {
        out = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + 8 * lg_e;
        oscale = L > 0.f ? 1.f / L : 0.f;
    } else {
        out = a.part_o + ((bh * a.ns + split) * a.R + r) * D + 8 * lg_e;
        oscale = 1.f;
        if (lg_e == 0) {
            float2 * mlp = &a.part_ml[(bh * a.ns + split) * a.R + r];
            __builtin_nontemporal_store(M, &mlp->x);
            __builtin_nontemporal_store(L, &mlp->y);
        }
    }
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        const float4 p0 = acc[bb][0], p1 = acc[bb][1];
        const float4 w0 = make_float4(p0.x * oscale, p0.y * oscale, p0.z * oscale, p0.w * oscale);
        const float4 w1 = make_float4(p1.x * oscale, p1.y * oscale, p1.z * oscale, p1.w * oscale);
        if (a.ns > 1) {
            // split partials are read once, by the merge: streamed past the caches
            store_nt4(out + 32 * bb, w0);
            store_nt4(out + 32 * bb + 4, w1);
        } else if (vec) {
            *(float4 *) (out + 32 * bb) = apply_gate(a, out + 32 * bb, w0);
            *(float4 *) (out + 32 * bb + 4) = apply_gate(a, out + 32 * bb + 4, w1);
        } else {
            float * o = out + 32 * bb;
            o[0] = w0.x; o[1] = w0.y; o[2] = w0.z; o[3] = w0.w;
            o[4] = w1.x; o[5] = w1.y; o[6] = w1.z; o[7] = w1.w;
        }
    }
}

// LSE merge of the ns split partials. One block per (query row, quarter of
// the head dims): thread (group g, quad q) folds splits g, g + 16, ... of dims
// 4q..4q+3 of the quarter, with the first 8 partials of each group in flight
// before the weights are known; the 16 groups add up through LDS.
constexpr int MERGE_GROUPS = 16;
constexpr int MERGE_BATCH = 8;

// Wave-wide reduction without LDS: a butterfly within each row of 16 lanes
// (DPP: lane ^ 1, lane ^ 2, the mirrored half of 8, the mirrored row of 16),
// then the four rows' results through scalar reads.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
    auto dpp = [](float v, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), decltype(ctrl)::value,
                                                                     0xF, 0xF, false));
    };
    x = op(x, dpp(x, std::integral_constant<int, 0xB1>{}));    // quad_perm [1,0,3,2]
    x = op(x, dpp(x, std::integral_constant<int, 0x4E>{}));    // quad_perm [2,3,0,1]
    x = op(x, dpp(x, std::integral_constant<int, 0x141>{}));   // row_half_mirror
    x = op(x, dpp(x, std::integral_constant<int, 0x140>{}));   // row_mirror
    const int u = __builtin_bit_cast(int, x);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 48));
    return op(op(r0, r1), op(r2, r3));
}

template <bool RG>
__global__ __launch_bounds__(256) void k_fattn_merge(fa_args a) {
    __shared__ float wsh[MAX_SPLITS];
    __shared__ float red[4];
    __shared__ float4 acc_sh[MERGE_GROUPS][16];
    const int row = blockIdx.x >> 2, quarter = blockIdx.x & 3;   // row = (b * nh_kv + kvh) * R + r
    const int r = row % a.R;
    const int bh = row / a.R;
    const int kvh = bh % a.nh_kv, b = bh / a.nh_kv;
    int ns = a.ns;                                               // this sequence's splits (a.ns is the stride)
    if constexpr (RG) {
#pragma unroll
        for (int i = 0; i < RAGGED_MAX_B; i++)
            if (i == b) ns = a.r_ns[i];
    }
    const int g = threadIdx.x >> 4, q = threadIdx.x & 15;
    const float2 * ml = a.part_ml + (size_t) bh * a.ns * a.R + r;
    const float4 * po = (const float4 *) (a.part_o + ((size_t) bh * a.ns * a.R + r) * D + 64 * quarter) + q;
    const size_t sstride = (size_t) a.R * D / 4;              // float4s between splits

    // every split's (max, sum), read once: thread i holds splits i + 256 j.
    // All loads are unconditional (indices clamped to the last split) so the
    // counter waits stay exact: the (max, sum) pairs first, then the first
    // MERGE_BATCH partials of the thread's group, which stay in flight while
    // the weights are formed.
    constexpr int MLJ = MAX_SPLITS / 256;
    float2 e[MLJ];
#pragma unroll
    for (int j = 0; j < MLJ; j++) e[j] = ml[(size_t) std::min((int) threadIdx.x + 256 * j, ns - 1) * a.R];
    float4 ob[MERGE_BATCH];
#pragma unroll
    for (int i = 0; i < MERGE_BATCH; i++) ob[i] = load_nt4(po + (size_t) std::min(g + i * MERGE_GROUPS, ns - 1) * sstride);
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < MLJ; j++) {
        if ((int) threadIdx.x + 256 * j >= ns) e[j] = make_float2(-INFINITY, 0.f);
        mloc = xmax(mloc, e[j].x);
    }
    mloc = wave_reduce(mloc, [](float x, float y) { return xmax(x, y); });
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mloc;
    __syncthreads();
    const float M = xmax(xmax(red[0], red[1]), xmax(red[2], red[3]));
    float lpart = 0.f;
#pragma unroll
    for (int j = 0; j < MLJ; j++) {
        const int s = (int) threadIdx.x + 256 * j;
        const float w = e[j].x == -INFINITY ? 0.f : exp2f(e[j].x - M);
        lpart += w * e[j].y;
        if (s < ns) wsh[s] = w;
    }
    lpart = wave_reduce(lpart, [](float x, float y) { return x + y; });
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lpart;
    __syncthreads();
    const float L = (red[0] + red[1]) + (red[2] + red[3]);

    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < ns; s0 += MERGE_GROUPS * MERGE_BATCH) {
        if (s0 > 0) {
#pragma unroll
            for (int i = 0; i < MERGE_BATCH; i++) ob[i] = load_nt4(po + (size_t) std::min(s0 + g + i * MERGE_GROUPS, ns - 1) * sstride);
        }
#pragma unroll
        for (int i = 0; i < MERGE_BATCH; i++) {
            const int s = s0 + g + i * MERGE_GROUPS;
            const float w = s < ns ? wsh[s] : 0.f;
            acc.x += w * ob[i].x; acc.y += w * ob[i].y; acc.z += w * ob[i].z; acc.w += w * ob[i].w;
        }
    }
    acc_sh[g][q] = acc;
    __syncthreads();
    if (g == 0) {
        float4 o = acc_sh[0][q];
#pragma unroll
        for (int g2 = 1; g2 < MERGE_GROUPS; g2++) {
            const float4 e = acc_sh[g2][q];
            o.x += e.x; o.y += e.y; o.z += e.z; o.w += e.w;
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        o.x *= inv; o.y *= inv; o.z *= inv; o.w *= inv;
        const int t = (int) div_gqa(a, (uint32_t) r), h = kvh * a.gqa + (r - t * a.gqa);
        float * d = a.dst + (((size_t) b * a.T + t) * a.nh + h) * D + 64 * quarter + 4 * q;
        if (a.dst_vec) {
            *(float4 *) d = apply_gate(a, d, o);
        } else {
            d[0] = o.x; d[1] = o.y; d[2] = o.z; d[3] = o.w;
        }
    }
}

// LSE merge for many query rows over few splits (k_fa_pre's key splits, at
// most MERGE_ROWS_SPLITS): one 64-lane group (one wave) per row, a lane per 4
// dims. The (max, sum) pairs are loaded first; a split in which the row saw
// no key (max -inf) has no O partial (k_fa_pre does not write it), so only
// the live splits' partials are loaded, all before any is used.
constexpr int MERGE_ROWS_SPLITS = 16;

__global__ __launch_bounds__(256) void k_fattn_merge_rows(fa_args a) {
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);   // (b * nh_kv + kvh) * R + r
    const uint32_t n_rows = (uint32_t) a.B * (uint32_t) a.nh_kv * (uint32_t) a.R;
    if (row >= n_rows) return;
    const int q4 = threadIdx.x & 63;
    const uint32_t bh = row / (uint32_t) a.R, r = row - bh * (uint32_t) a.R;
    const uint32_t b = bh / (uint32_t) a.nh_kv, kvh = bh - b * (uint32_t) a.nh_kv;
    const float2 * ml = a.part_ml + (size_t) bh * a.ns * a.R + r;
    const float4 * po = (const float4 *) (a.part_o + ((size_t) bh * a.ns * a.R + r) * D) + q4;
    const size_t sstride = (size_t) a.R * D / 4;
    float2 e[MERGE_ROWS_SPLITS];
    float4 o[MERGE_ROWS_SPLITS];
#pragma unroll
    for (int s = 0; s < MERGE_ROWS_SPLITS; s++) e[s] = s < a.ns ? ml[(size_t) s * a.R] : make_float2(-INFINITY, 0.f);
#pragma unroll
    for (int s = 0; s < MERGE_ROWS_SPLITS; s++)
        o[s] = e[s].x != -INFINITY ? load_nt4(po + (size_t) s * sstride) : make_float4(0.f, 0.f, 0.f, 0.f);
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < MERGE_ROWS_SPLITS; s++) M = xmax(M, e[s].x);
    float L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < MERGE_ROWS_SPLITS; s++) {
        const float w = e[s].x == -INFINITY ? 0.f : exp2f(e[s].x - M);
        L += w * e[s].y;
        acc.x += w * o[s].x; acc.y += w * o[s].y; acc.z += w * o[s].z; acc.w += w * o[s].w;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
    const uint32_t t = div_gqa(a, r), h = kvh * (uint32_t) a.gqa + (r - t * (uint32_t) a.gqa);
    float * d = a.dst + (((size_t) b * a.T + t) * a.nh + h) * D + 4 * q4;
    if (a.dst_vec) {
        *(float4 *) d = apply_gate(a, d, acc);
    } else {
        d[0] = acc.x; d[1] = acc.y; d[2] = acc.z; d[3] = acc.w;
    }
}

// ================================================================ split merge inside the attention kernel
//
// Every block of a (batch, KV head) group writes its split's partials, then
// takes a ticket from the group's arrival word. The block with the last ticket
// knows that every split is written; it claims rows of the group one at a
// time from the group's claim word and merges each (the same LSE merge as
// k_fattn_merge) until none is left. The blocks with the m_nm - 1 tickets
// before it poll the arrival word for a bounded time: one that sees every
// split arrive claims rows too, one that does not simply leaves. So no block
// ever waits for a block that may not be resident, every row is merged once,
// and the merge costs no launch.
// Ordering across XCDs: the partials are written and read with device-scope
// accesses (store_dev4 and friends), and each writer waits until its stores
// have completed before the block arrives; a merger reads them only after it
// has seen the last arrival.
// Counters: one library-owned array (g_merge_ctr), zero when loaded. A call
// takes consecutive slots of it (one per group) and an epoch from a 48-bit
// per-device sequence; each word holds (epoch << 16) | count, and the call's
// first atomic max on a word installs its epoch with count 0, so no word is
// ever reset. Calls in flight at once get disjoint slots unless more than
// MERGE_SLOTS groups are in flight.

constexpr int      MERGE_SLOTS    = 16384;            // (batch, KV head) groups in flight at once, at most
constexpr uint32_t MERGE_SPIN_MAX = 1u << 13;         // polls of a waiting merger (s_sleep 2 each): ~0.4 ms
__device__ __align__(256) static unsigned long long g_merge_ctr[2 * MERGE_SLOTS];

// LDS of the fused merge (floats): 16 words of tickets, the split weights, a
// reduction row and 8 x 64 float4 column sums
constexpr int FMERGE_LDS = 16 + MAX_SPLITS + 16 + 8 * 64 * 4;

// One row r of group (b, kvh) by a block of NT threads: thread t folds
// float4 column t % 64 of splits t / 64 + (NT / 64) i, 16 partials in flight
// per batch (the first batch is issued with the (max, sum) loads).
template <int NT>
__device__ __forceinline__ void fa_merge_row(const fa_args & a, int b, int kvh, int r, float * sm) {
    constexpr int NG = NT / 64, MB = 16, MLJ = (MAX_SPLITS + NT - 1) / NT;
    static_assert(NG <= 8, "column sums hold 8 groups");
    const int S = a.ns;
    const int t = (int) threadIdx.x, sg = t >> 6, c = t & 63;
    const size_t bh = (size_t) b * a.nh_kv + kvh;
    // the group's partials: (max, sum) of split s at 8 (s R + r), its O row at 4 D (s R + r)
    const __amdgpu_buffer_rsrc_t mr = dev_rsrc(a.part_ml + bh * a.ns * a.R);
    const __amdgpu_buffer_rsrc_t orr = dev_rsrc(a.part_o + bh * a.ns * a.R * D);
    const uint32_t mst = 8u * (uint32_t) a.R, ost = 4u * D * (uint32_t) a.R;
    const uint32_t m0 = 8u * (uint32_t) r, o0 = 4u * D * (uint32_t) r + 16u * (uint32_t) c;
    float * wsh = sm + 16;
    float * red = wsh + MAX_SPLITS;
    float4 * colsum = (float4 *) (red + 16);
    float2 e[MLJ];
#pragma unroll
    for (int j = 0; j < MLJ; j++) e[j] = load_dev2(mr, m0 + mst * (uint32_t) std::min(t + NT * j, S - 1));
    float4 ob[MB];
#pragma unroll
    for (int i = 0; i < MB; i++) ob[i] = load_dev4(orr, o0 + ost * (uint32_t) std::min(sg + NG * i, S - 1));
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < MLJ; j++) {
        if (t + NT * j >= S) e[j] = make_float2(-INFINITY, 0.f);
        mloc = xmax(mloc, e[j].x);
    }
    mloc = wave_reduce(mloc, [](float x, float y) { return xmax(x, y); });
    if ((t & 63) == 0) red[sg] = mloc;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int g = 1; g < NG; g++) M = xmax(M, red[g]);
    float lpart = 0.f;
#pragma unroll
    for (int j = 0; j < MLJ; j++) {
        const int s = t + NT * j;
        const float w = e[j].x == -INFINITY ? 0.f : exp2f(e[j].x - M);
        lpart += w * e[j].y;
        if (s < S) wsh[s] = w;
    }
    lpart = wave_reduce(lpart, [](float x, float y) { return x + y; });
    if ((t & 63) == 0) red[8 + sg] = lpart;
    __syncthreads();
    float L = 0.f;
#pragma unroll
    for (int g = 0; g < NG; g++) L += red[8 + g];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < S; s0 += NG * MB) {
        if (s0 > 0) {
#pragma unroll
            for (int i = 0; i < MB; i++) ob[i] = load_dev4(orr, o0 + ost * (uint32_t) std::min(s0 + sg + NG * i, S - 1));
        }
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const int s = s0 + sg + NG * i;
            const float w = s < S ? wsh[s] : 0.f;
            acc.x += w * ob[i].x; acc.y += w * ob[i].y; acc.z += w * ob[i].z; acc.w += w * ob[i].w;
        }
    }
    colsum[sg * 64 + c] = acc;
    __syncthreads();
    if (sg == 0) {
        float4 o = colsum[c];
#pragma unroll
        for (int g = 1; g < NG; g++) {
            const float4 x = colsum[g * 64 + c];
            o.x += x.x; o.y += x.y; o.z += x.z; o.w += x.w;
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        o.x *= inv; o.y *= inv; o.z *= inv; o.w *= inv;
        const int tq = (int) div_gqa(a, (uint32_t) r), h = kvh * a.gqa + (r - tq * a.gqa);
        float * d = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + 4 * c;
        if (a.dst_vec) {
            *(float4 *) d = apply_gate(a, d, o);
        } else {
            d[0] = o.x; d[1] = o.y; d[2] = o.z; d[3] = o.w;
        }
    }
    __syncthreads();   // wsh, red and colsum are the next row's
}

// The tail of a k_fa_dec / k_fa_vd block of NT threads once its partials are
// stored (every thread of the block calls it); sm: FMERGE_LDS floats of LDS
// the block no longer uses.
template <int NT>
__device__ void fa_merge_tail(const fa_args & a, int b, int kvh, float * sm) {
    unsigned long long * arrive = a.mctr + 2 * ((size_t) b * a.nh_kv + kvh);
    unsigned long long * claim = arrive + 1;
    const unsigned long long e = a.m_ebase;
    const int S = a.ns;
    int * si = (int *) sm;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's device-scope partial stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_max(arrive, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int tk = (int) (__hip_atomic_fetch_add(arrive, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 0xFFFFu);
        int go = tk == S - 1;
        if (!go && tk >= S - a.m_nm) {
            for (uint32_t polls = 0; polls < MERGE_SPIN_MAX; polls++) {
                if (__hip_atomic_load(arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (e | (unsigned) S)) {
                    go = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        if (go) __hip_atomic_fetch_max(claim, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        si[0] = go;
    }
    __syncthreads();
    if (!si[0]) return;
    for (;;) {
        __syncthreads();   // every thread has read si[1]
        if (threadIdx.x == 0)
            si[1] = (int) (__hip_atomic_fetch_add(claim, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 0xFFFFu);
        __syncthreads();
        const int r = si[1];
        if (r >= a.R) break;
        fa_merge_row<NT>(a, b, kvh, r, sm);
    }
}

// ================================================================ decode / verify
//
// k_fa_dec: row groups of at most 32 query rows per KV head (decode, MTP
// verify, batch decode), one block of 8 waves per CU. Wave (row tile t, key
// group g) owns query rows 16t .. 16t+15 of the block and its tiles
// g, g + KG, g + 2KG, ... of 16 keys. It streams them through a ring of two
// stages of its own: LDS DMA that only this wave waits for (its own vmcnt), so
// the key loop has no block barrier. Waves drift apart, and one wave's matrix
// core work overlaps another's vector work. The RT waves of a key group each
// load the same keys; the second load comes from L2. The arithmetic per tile
// is that of k_fattn_q8_0's 16-key waves (exact i8 block dots, per-block
// d_q*d_k scaling, online base-2 softmax, hi + lo f16 P*d_v).

constexpr int DEC_WAVES = 8;
constexpr int DEC_TK    = 16;                         // keys per tile
constexpr int DEC_KB    = DEC_TK * SEG;               // 4352: one tensor's rows of a tile
constexpr int DEC_TDMA  = (DEC_KB / 16 + 63) / 64;    // 5 wave DMAs per tensor (the last one with 16 lanes)
constexpr int DEC_MOFF  = 2 * DEC_KB;                 // a tile's mask granules follow its K and V rows
constexpr int DEC_MGR   = 3;                          // 16-byte granules per mask row of a tile (32 bytes, 2-byte aligned)
constexpr int DEC_STAGE = DEC_MOFF + 1024;            // 9728 bytes
constexpr int DEC_OBS   = D + 4;                      // merge buffer row stride (floats)
constexpr int DEC_QROW  = 1024 + 16;                  // query row stride in the prologue's staging (bank spread)
constexpr int DEC_GATHER_SPLIT = 512;                 // cells of a block's split, at most (gathered keys)
static_assert(DEC_KB / 16 - 64 * (DEC_TDMA - 1) == 16, "the last DMA of a tensor has 16 lanes");
static_assert(16 * DEC_MGR <= 64, "a wave's mask rows of a tile are one DMA");

// GATHER: the keys of KV head h are the cache rows its cell list names (the
// reference's raw get_rows of the selected cells, qwfn_graph.cpp:632-651,
// fused: the rows are DMA'd straight from the cache), and a query sees a row
// only if it is at most its own position (the decode cell mask, :668-675)
template <int RT, bool MASKED, bool RG, bool GATHER>
__global__ __launch_bounds__(DEC_WAVES * 64, 2) void k_fa_dec(fa_args a) {
    constexpr int ROWS = 16 * RT, KG = DEC_WAVES / RT;
    constexpr int OPS = 2 * DEC_TDMA + (MASKED ? 1 : 0);   // DMAs per tile of one wave
    asm volatile("" :: "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.mask), "s"(a.m_ne2), "s"(a.part_o));
    // ring[stage][wave]: stage 1 of all waves is one contiguous region, which
    // the prologue uses for the query rows and their window image
    __shared__ __attribute__((aligned(16))) uint8_t ring[2][DEC_WAVES][DEC_STAGE];
    __shared__ __attribute__((aligned(16))) uint16_t scl[DEC_WAVES][2][NBLK][DEC_TK];
    // GATHER: the block's part of its KV head's cell list
    __shared__ __attribute__((aligned(16))) int32_t gcell[GATHER ? DEC_GATHER_SPLIT : 4];
    static_assert(!(GATHER && (MASKED || RG)), "gathered keys carry their own mask, one sequence");
    static_assert(ROWS * DEC_QROW <= DEC_WAVES * DEC_STAGE, "query rows fit stage 1");
    static_assert(ROWS * NBLK * QWIN + ROWS * NBLK * 4 <= DEC_WAVES * DEC_STAGE, "query image fits stage 1");
    static_assert((KG - 1) * ROWS * DEC_OBS * 4 <= 2 * DEC_WAVES * DEC_STAGE, "merge buffers fit the ring");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const int tile = wave % RT, kg = wave / RT;

    // ---- block -> (b, kvh, split): as k_fattn_q8_0 (one row group) ----
    const int id = blockIdx.x;
    const int hgn = a.nh_kv;
    const int n_units = RG ? a.r_units : a.B * a.ns;
    int kvh, u;
    if (n_units >= 8) {
        const int j = id >> 3;
        const int jq = (int) udiv((uint32_t) j, (uint32_t) hgn, a.hgn_mul);
        kvh = j - jq * hgn;
        u = jq * 8 + (id & 7);
    } else {
        u = (int) udiv((uint32_t) id, (uint32_t) hgn, a.hgn_mul);
        kvh = id - u * hgn;
    }
    if (u >= n_units) return;
    int b, split;
    int64_t k_lo, k_hi;
    if constexpr (RG) {
        int32_t us = 0, nsb = 1, slb = 0;
        int64_t nkb = 0;
        b = 0;
#pragma unroll
        for (int i = 0; i < RAGGED_MAX_B; i++)
            if (i < a.B && u >= a.r_ustart[i]) {
                b = i; us = a.r_ustart[i]; nsb = a.r_ns[i]; slb = a.r_split_len[i]; nkb = a.r_n_kv[i];
            }
        split = u - us;
        k_lo = (int64_t) split * slb;
        const int64_t e = k_lo + slb;
        k_hi = split == nsb - 1 ? nkb : (nkb < e ? nkb : e);
    } else {
        b = (int) udiv((uint32_t) u, (uint32_t) a.ns, a.ns_mul);
        split = u - b * a.ns;
        k_lo = (int64_t) split * a.split_len;
        const int64_t e = k_lo + a.split_len;
        k_hi = split == a.ns - 1 ? a.n_kv : (a.n_kv < e ? a.n_kv : e);
    }
    if constexpr (GATHER) {
        // this list's own cell count (constant indices keep the table scalar)
        const int li = b * a.nh_kv + kvh;
        int64_t nh = 0;
#pragma unroll
        for (int i = 0; i < GATHER_MAX_LISTS; i++)
            if (i == li) nh = a.g_n[i];
        k_hi = k_hi < nh ? k_hi : nh;
        k_lo = k_lo < k_hi ? k_lo : k_hi;
    }
    const int span = (int) (k_hi - k_lo);
    const int n_tiles = (span + DEC_TK - 1) / DEC_TK;
    const int RW = a.R < ROWS ? a.R : ROWS;             // rows of this block (one row group)
    const int wr0 = 16 * tile;                          // the wave's first row in the block

    const char * kbase = a.k + (size_t) bmod(b, a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) bmod(b, a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;

    // ---- the wave's mask rows: query position for a mask shared by the heads,
    //      query row for a per-head mask; byte offsets from the mask slice
    //      rounded down to 16 bytes ----
    const char * mslice = MASKED ? a.mask + (size_t) bmod(b, a.m_ne3) * a.m_nb3 : nullptr;
    const char * mslice_al = (const char *) ((uintptr_t) mslice & ~(uintptr_t) 15);
    const int wt0 = (int) div_gqa(a, (uint32_t) wr0);   // first query position of the wave's rows
    auto mrow_off = [&](int mr) -> uint32_t {           // mask row mr of the wave
        int t = wt0 + mr, hq = 0;
        if (a.m_ne2 != 1) {
            const int r = wr0 + mr;
            t = (int) div_gqa(a, (uint32_t) r);
            hq = (kvh * a.gqa + (r - t * a.gqa)) % a.m_ne2;
        }
        return (uint32_t) (mslice - mslice_al) + (uint32_t) ((size_t) t * a.m_nb1 + (size_t) hq * a.m_nb2);
    };
    int n_mrows = 0;
    uint32_t m_goff = 0, m_lane = 0;
    if constexpr (MASKED) {
        const int wlast = (wr0 + 15 < RW ? wr0 + 15 : RW - 1);
        n_mrows = wr0 >= RW ? 1 : (a.m_ne2 == 1 ? (int) div_gqa(a, (uint32_t) wlast) - wt0 + 1 : wlast - wr0 + 1);
        // DMA lane g: granule g % 3 of mask row g / 3 (lanes past the rows re-read the last granule)
        const int g = lane < n_mrows * DEC_MGR ? lane : n_mrows * DEC_MGR - 1;
        m_goff = (mrow_off(g / DEC_MGR) & ~15u) + 16u * (uint32_t) (g % DEC_MGR);
        // the lane's own row in the stage's mask area
        const int rl = wr0 + ln < RW ? wr0 + ln : wr0;
        const int mi = a.m_ne2 == 1 ? (int) div_gqa(a, (uint32_t) rl) - wt0 : rl - wr0;
        m_lane = (uint32_t) (DEC_MOFF + mi * DEC_MGR * 16) + (mrow_off(mi) & 15u) + 8u * (uint32_t) lg;
    }

    // ---- per-lane DMA offsets of a tile's pieces: piece p = 64s + lane is byte
    //      16 (p % 17) of key p / 17; the same for every tile ----
    uint32_t koff[DEC_TDMA], voff[DEC_TDMA];
#pragma unroll
    for (int s = 0; s < DEC_TDMA; s++) {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u, part = p - key * 17u;
        koff[s] = key * (uint32_t) a.k_nb1 + part * 16u;
        voff[s] = key * (uint32_t) a.v_nb1 + part * 16u;
    }
    const int64_t k_bytes = k_hi * (int64_t) a.k_nb1, v_bytes = k_hi * (int64_t) a.v_nb1;
    // LDS addresses of the wave's two stages, in 32-bit arithmetic from the
    // ring's own address (casting a computed generic pointer tests it for null
    // at every use)
    const uint32_t stl0 = lds_addr(&ring[0][0][0]) + (uint32_t) wave * DEC_STAGE;
    const uint32_t stl1 = stl0 + DEC_WAVES * DEC_STAGE;
    // the wave's tiles kg, kg + KG, ... are issued in that order, each once:
    // their K, V and mask resources start where the previous one's did plus
    // a stride of KG tiles, and what is left of the split shrinks by as much
    const int64_t key_first = k_lo + (int64_t) kg * DEC_TK;
    const char * k_next = kbase + key_first * (int64_t) a.k_nb1;
    const char * v_next = vbase + key_first * (int64_t) a.v_nb1;
    const char * m_next = mslice_al + key_first * 2;
    int64_t k_rem = k_bytes - key_first * (int64_t) a.k_nb1, v_rem = v_bytes - key_first * (int64_t) a.v_nb1;
    int64_t m_rem = (int64_t) a.m_slice + (mslice - mslice_al) - key_first * 2;
    const int64_t k_step = (int64_t) (KG * DEC_TK) * a.k_nb1, v_step = (int64_t) (KG * DEC_TK) * a.v_nb1;
    constexpr int64_t m_step = KG * DEC_TK * 2;
    // GATHER: the DMA offsets of tile ti follow its cells (in LDS): piece p of
    // slot s is byte 16 (p % 17) of row gcell[16 ti + p / 17]; a cell outside
    // the cache, or a key past the split, gets an offset past the buffer, so
    // its bytes arrive as zeros (and the key is masked); the cache is below
    // 2 GiB per call, so 2^31 is past it
    const uint32_t g_kbytes = GATHER ? (uint32_t) (a.g_rows * (int64_t) a.k_nb1) : 0u;
    const uint32_t g_vbytes = GATHER ? (uint32_t) (a.g_rows * (int64_t) a.v_nb1) : 0u;
    auto gather_off = [&](int ti, int s, uint32_t nb1) -> uint32_t {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u, part = p - key * 17u;
        const int kk = ti * DEC_TK + (int) key;
        const uint32_t row = kk < span ? (uint32_t) gcell[kk] : 0xffffffffu;
        return row < (uint32_t) a.g_rows ? row * nb1 + part * 16u : 0x80000000u;
    };
    // tile ti of the split (keys 16 ti .. 16 ti + 15) into stage buffer st, in
    // two halves: the K rows (free once the tile's QK is done) and the V rows
    // with the mask granules (free once its PV is done). Keys past the split
    // arrive as zeros (buffer bounds) and are masked.
    auto issue_k = [&](int ti, uint32_t stl) __attribute__((always_inline)) {
        v4i rk;
        uint32_t o[DEC_TDMA];
        if constexpr (GATHER) {
#pragma unroll
            for (int s = 0; s < DEC_TDMA; s++) o[s] = gather_off(ti, s, (uint32_t) a.k_nb1);
            rk = make_rsrc(kbase, g_kbytes);
        } else {
#pragma unroll
            for (int s = 0; s < DEC_TDMA; s++) o[s] = koff[s];
            rk = make_rsrc(k_next, rsrc_bytes(k_rem));
            k_next += k_step;
            k_rem -= k_step;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): (the cells are read and) this wave's reads of the stage are done
        dma16_buf_at<0>(rk, o[0], stl);
        dma16_buf_at<1024>(rk, o[1], stl);
        dma16_buf_at<2048>(rk, o[2], stl);
        dma16_buf_at<3072>(rk, o[3], stl);
        static_assert(DEC_TDMA == 5, "five DMAs per tensor");
        if (lane < 16) dma16_buf_at<4096>(rk, o[4], stl);
    };
    auto issue_v = [&](int ti, uint32_t stl) __attribute__((always_inline)) {
        v4i rv;
        uint32_t o[DEC_TDMA];
        if constexpr (GATHER) {
#pragma unroll
            for (int s = 0; s < DEC_TDMA; s++) o[s] = gather_off(ti, s, (uint32_t) a.v_nb1);
            rv = make_rsrc(vbase, g_vbytes);
        } else {
#pragma unroll
            for (int s = 0; s < DEC_TDMA; s++) o[s] = voff[s];
            rv = make_rsrc(v_next, rsrc_bytes(v_rem));
            v_next += v_step;
            v_rem -= v_step;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        dma16_buf_at<DEC_KB>(rv, o[0], stl);
        dma16_buf_at<DEC_KB + 1024>(rv, o[1], stl);
        dma16_buf_at<DEC_KB + 2048>(rv, o[2], stl);
        dma16_buf_at<DEC_KB + 3072>(rv, o[3], stl);
        if (lane < 16) dma16_buf_at<DEC_KB + 4096>(rv, o[4], stl);
        if constexpr (MASKED) {
            const v4i rm = make_rsrc(m_next, (uint32_t) m_rem);
            m_next += m_step;
            m_rem -= m_step;
            if (lane < n_mrows * DEC_MGR) dma16_buf_at<DEC_MOFF>(rm, m_goff, stl);
        }
    };
    auto issue_tile = [&](int ti, uint32_t stl) __attribute__((always_inline)) {
        issue_k(ti, stl);
        issue_v(ti, stl);
    };

    // ---- prologue: the block's query rows (f32, one wave DMA per row) into
    //      stage 1, then the fused append (if any), then every wave's first tile ----
    uint8_t * qstage = &ring[1][0][0];
    {
        const v4i rq = make_rsrc(a.q + (size_t) b * a.q_nb3, a.q_slice);
#pragma unroll
        for (int j = 0; j < (ROWS + DEC_WAVES - 1) / DEC_WAVES; j++) {
            const int rl = wave + DEC_WAVES * j;
            if (rl >= RW) break;
            const uint32_t r = (uint32_t) rl;
            const uint32_t t = div_gqa(a, r), h = (uint32_t) (kvh * a.gqa) + (r - t * (uint32_t) a.gqa);
            dma16_buf(rq, t * (uint32_t) a.q_nb1 + h * (uint32_t) a.q_nb2 + 16u * (uint32_t) lane,
                      __builtin_amdgcn_readfirstlane(lds_addr(qstage + rl * DEC_QROW)));
        }
    }
    const int first0 = kg < n_tiles ? kg : -1, first1 = kg + KG < n_tiles ? kg + KG : -1;
    __shared__ uint32_t g_bad;   // GATHER: a cell of the block lies outside the cache
    if constexpr (GATHER) {
        // the block's cells [k_lo, k_hi): wave w takes 256-cell pieces w, w + NW, ...
        const int32_t * cl = a.g_cells + (size_t) b * a.g_bstride + (size_t) kvh * a.g_hstride + k_lo;
        const v4i rc = make_rsrc(cl, (uint32_t) span * 4u);
        for (int m = wave; m * 256 < span; m += DEC_WAVES)
            dma16_buf(rc, (uint32_t) (m * 1024 + 16 * lane), __builtin_amdgcn_readfirstlane(lds_addr(&gcell[m * 256])));
        if (threadIdx.x == 0) g_bad = 0;
        wait_vmcnt<0>();   // this wave's cells (and query rows) have landed
        __syncthreads();   // ... and every wave's: the first tiles' DMA offsets follow them
        if ((int) threadIdx.x < span && (uint32_t) gcell[threadIdx.x] >= (uint32_t) a.g_rows) g_bad = 1;
    }
    if (a.app_n > 0) {
        // as in k_fattn_q8_0: the blocks whose keys hold appended rows quantise
        // their KV head's part of them first, and read them back only after
        // their own stores are done
        const int64_t alo = std::max<int64_t>(a.app_row0, k_lo), ahi = std::min<int64_t>(a.app_row0 + a.app_n, k_hi);
        if (alo < ahi) {
            const int units = (int) (ahi - alo) * NBLK * 2;
            const int sub = threadIdx.x & 7;
            for (int u0 = 0; u0 < units; u0 += DEC_WAVES * 8) {
                const int uu0 = u0 + (int) (threadIdx.x >> 3);
                const bool live = uu0 < units;
                const int uu = live ? uu0 : 0;
                const int tensor = uu & 1, jb = (uu >> 1) % NBLK;
                const int64_t row = alo + (uu >> 1) / NBLK;
                const float4 xv = *(const float4 *) ((tensor ? a.app_v : a.app_k) + (size_t) (row - a.app_row0) * a.app_nb1 +
                                                     (size_t) (kvh * D + QK * jb + 4 * sub) * 4);
                float x[4] = {xv.x, xv.y, xv.z, xv.w};
                uint16_t d16;
                float dqa;
                const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dqa);
                if (live) {
                    char * bp = (char *) (tensor ? vbase + (size_t) row * a.v_nb1 : kbase + (size_t) row * a.k_nb1) + jb * QBLOCK;
                    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
                    qp[0] = (uint16_t) (q4 & 0xffffu);
                    qp[1] = (uint16_t) (q4 >> 16);
                    if (sub == 0) *(uint16_t *) bp = d16;
                }
            }
            wait_vmcnt<0>();
            __syncthreads();
        }
    }
    if (first0 >= 0) issue_tile(first0, stl0);
    if (first0 >= 0) wait_vmcnt<OPS>();                 // the query DMAs have landed (the tile's may not)
    else wait_vmcnt<0>();
    __syncthreads();

    // ---- requantisation of the query rows (ggml's quantiser): wave w takes
    //      q8_0 block w of every row, QL lanes per (row, block) ----
    constexpr int QL = 64 / ROWS, QV = 32 / QL;
    static_assert(NBLK == DEC_WAVES, "one block of all rows per wave");
    static_assert(win_off(0) == 2 && win_off(1) == 20 && win_off(2) == 6 && win_off(3) == 8 && win_off(4) == 10 &&
                  win_off(5) == 12 && win_off(6) == 14 && win_off(7) == 32, "the packed window offsets");
    const int qrl = lane / QL, qh = lane % QL;
    float qx[QV];
    {
        const float4 * src = (const float4 *) (qstage + qrl * DEC_QROW + (QK * wave + QV * qh) * 4);
#pragma unroll
        for (int m = 0; m < QV / 4; m++) {
            const float4 v = qrl < RW ? src[m] : make_float4(0.f, 0.f, 0.f, 0.f);
            qx[4 * m] = v.x; qx[4 * m + 1] = v.y; qx[4 * m + 2] = v.z; qx[4 * m + 3] = v.w;
        }
    }
    __syncthreads();   // every query value is in registers: stage 1 becomes the window image
    // window image [block][16-byte slice][row]: the 16 rows a lane group of the
    // MFMA operand reads are consecutive 16-byte pieces (no bank conflicts)
    uint8_t * qwin = qstage;
    auto qslice = [&](int bb, int sl, int row) { return qwin + ((bb * 4 + sl) * ROWS + row) * 16; };
    float * dql = (float *) (qstage + NBLK * QWIN * ROWS);        // [ROWS][NBLK]
    {
#pragma unroll
        for (int z = 0; z < 4 / QL; z++) *(uint4 *) qslice(wave, qh * (4 / QL) + z, qrl) = make_uint4(0, 0, 0, 0);
        wave_lds_sync();
        uint32_t w[QV / 4];
        uint16_t d16;
        float dqv = 0.f;
        if (a.x86) dev::q8_quantize_lanes<QV>(qx, true, w, &d16, &dqv);
        else       dev::q8_quantize_lanes<QV>(qx, false, w, &d16, &dqv);
        if (qrl < RW) {
            // win_off(wave), read from a packed table (no scalar branch chain)
            const int woff = (int) ((0x200E0C0A08061402ull >> (8 * wave)) & 0xff);
#pragma unroll
            for (int m = 0; m < QV / 2; m++) {   // 2-byte pieces never straddle a slice
                const int o = woff + QV * qh + 2 * m;
                *(uint16_t *) (qslice(wave, o >> 4, qrl) + (o & 15)) = (uint16_t) (w[m >> 1] >> (16 * (m & 1)));
            }
        }
        if (qh == 0) dql[qrl * NBLK + wave] = qrl < RW ? dqv * (a.scale * LOG2E) : 0.f;
    }
    __syncthreads();
    const int rl_lane = wr0 + ln;
    v4i qw[NBLK];
    float dq[NBLK];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        qw[bb] = *(const v4i *) qslice(bb, lg, rl_lane);
        dq[bb] = dql[rl_lane * NBLK + bb];
    }
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) asm volatile("" : "+v"(qw[bb]), "+v"(dq[bb]));
    __syncthreads();   // every wave has its operands: stage 1 is free
    if (first1 >= 0) issue_tile(first1, stl1);

    // ---- the key loop ----
    v4f O[NBLK][2];
    float m_run = -INFINITY, l_run = 0.f;
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) { O[bb][0] = v4f{0, 0, 0, 0}; O[bb][1] = v4f{0, 0, 0, 0}; }
    uint16_t (*sw)[NBLK][DEC_TK] = scl[wave];
    // GATHER: the position of the lane's query row
    const int64_t q_pos = GATHER ? a.g_pos0 + b + (int64_t) div_gqa(a, (uint32_t) (wr0 + ln)) : 0;

    // tile ti from stage st; nx >= 0: tile nx goes into the same stage, its K
    // rows as soon as the QK is done, its V rows and mask after the PV
    auto tile_step = [&](int ti, uint8_t * st, uint32_t stl, int nx) __attribute__((always_inline)) {
        const int kin = ti * DEC_TK + lg * 4;   // the lane's first key, within the split
        // the tile's block scales, transposed to [tensor][block][key]
        {
            const uint8_t * src = st + (lane >> 3) * SEG + (lane & 7) * QBLOCK;
            uint16_t * dstw = &sw[0][lane & 7][lane >> 3];
            uint16_t sv[4];
#pragma unroll
            for (int n = 0; n < 4; n++) sv[n] = *(const uint16_t *) (src + (n >> 1) * DEC_KB + (n & 1) * 8 * SEG);
#pragma unroll
            for (int n = 0; n < 4; n++) dstw[(n >> 1) * NBLK * DEC_TK + (n & 1) * 8] = sv[n];
        }
        wave_lds_sync();
        // ---- S = K Q^T: keys (MFMA rows) x the wave's 16 query rows. Each
        //      block's MFMA is issued two blocks ahead of its scaling, so the
        //      matrix core runs while the vector unit scales ----
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        {
            v4i kA[NBLK];
            uint2 dk[NBLK];
            const uint8_t * krow = st + ln * SEG + 16 * lg;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                kA[bb] = *(const v4i *) (krow + 16 * win_piece(bb));
                dk[bb] = *(const uint2 *) &sw[0][bb][lg * 4];
            }
            v4i cc[NBLK];
            cc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[0], qw[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            cc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[1], qw[1], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                if (bb + 2 < NBLK)
                    cc[bb + 2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[bb + 2], qw[bb + 2], v4i{0, 0, 0, 0}, 0, 0, 0);
                const float d = dq[bb];
                s[0] = __builtin_fmaf((float) cc[bb][0], mul_f16lo(d, dk[bb].x), s[0]);
                s[1] = __builtin_fmaf((float) cc[bb][1], mul_f16hi(d, dk[bb].x), s[1]);
                s[2] = __builtin_fmaf((float) cc[bb][2], mul_f16lo(d, dk[bb].y), s[2]);
                s[3] = __builtin_fmaf((float) cc[bb][3], mul_f16hi(d, dk[bb].y), s[3]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (nx >= 0) issue_k(nx, stl);
        // ---- mask, online softmax (base 2) ----
        float p[4];
        uint32_t p16[2];
        {
            float x[4];
            if constexpr (MASKED) {
                const uint16_t * mp = (const uint16_t *) (st + m_lane);
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = fma_f16lo((uint32_t) mp[i], LOG2E, s[i]);
            } else if constexpr (GATHER) {
                // a cell is seen by the queries at or after its position (keys
                // past the split read a cell that the tail check below masks)
                const int4 c = *(const int4 *) &gcell[kin < DEC_GATHER_SPLIT - 3 ? kin : 0];
                const int cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    x[i] = (uint32_t) cv[i] < (uint32_t) a.g_rows && (int64_t) cv[i] <= q_pos ? s[i] : -INFINITY;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = s[i];
            }
            if ((ti + 1) * DEC_TK > span) {   // the split's last tile: keys past its end
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (kin + i >= span) x[i] = -INFINITY;
            }
            float mloc = vmax(vmax(x[0], x[1]), vmax(x[2], x[3]));
            mloc = xmax_lanes16_32(mloc);
            const bool grow = mloc > m_run + RESCALE_SLACK;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(m_run - mloc);
                m_run = mloc;
            }
            const float m_use = m_run == -INFINITY ? 0.f : m_run;
            float lsum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
                lsum += p[i];
            }
            l_run = l_run * alpha + lsum;
            p16[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[0], p[1]));
            p16[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[2], p[3]));
            if (__any(grow)) {
                // a real branch (taken when the running max moves by more than
                // the slack): if-converted, every tile would pay the 64 multiplies
                asm volatile("" ::: "memory");
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[bb][0] *= alpha; O[bb][1] *= alpha; }
            }
        }
        // ---- O += V^T (P d_v) per V block. All V reads first; then block b's
        //      MFMAs are interleaved with the conversions of block b + 1, so
        //      the matrix core runs while the vector unit converts ----
        const uint8_t * vrow = st + DEC_KB + (lg * 4) * SEG + 2 + 2 * ln;
        uint32_t w[NBLK][4];
        uint2 dv2[NBLK];
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
#pragma unroll
            for (int jj = 0; jj < 4; jj++) w[bb][jj] = *(const uint16_t *) (vrow + jj * SEG + bb * QBLOCK);
            dv2[bb] = *(const uint2 *) &sw[1][bb][lg * 4];
        }
        uint32_t a0[2], a1[2], bh[2], bl[2];
        {
            const uint32_t dv[2] = {dv2[0].x, dv2[0].y};
            cvt_v_block(w[0], a0, a1);
            pdv_hilo(p, p16, dv, bh, bl);
        }
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            const v4h A0 = __builtin_bit_cast(v4h, make_uint2(a0[0], a0[1]));
            const v4h A1 = __builtin_bit_cast(v4h, make_uint2(a1[0], a1[1]));
            const v4h Bh = __builtin_bit_cast(v4h, make_uint2(bh[0], bh[1]));
            const v4h Bl = __builtin_bit_cast(v4h, make_uint2(bl[0], bl[1]));
            O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bh, O[bb][0], 0, 0, 0);
            O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bh, O[bb][1], 0, 0, 0);
            if (bb + 1 < NBLK) {
                const uint32_t dv[2] = {dv2[bb + 1].x, dv2[bb + 1].y};
                cvt_v_block(w[bb + 1], a0, a1);
                pdv_hilo(p, p16, dv, bh, bl);
            }
            O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bl, O[bb][0], 0, 0, 0);
            O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bl, O[bb][1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (nx >= 0) issue_v(nx, stl);
    };
    // key group kg takes tiles kg, kg + KG, ... in that order (a fixed order:
    // the result is reproducible bit for bit); the two stages alternate. The
    // DMAs of the tile after next follow each tile (its K half mid-step), so
    // the ones issued after a tile's own are exactly the next tile's.
    // Two waves share a SIMD (waves w and w + 4) and the older one wins its
    // issue slots, so it would finish its tiles long before the other, which
    // then runs alone at half the vector rate: the wave priority alternates
    // with the tile count, in opposite phase for the two waves of a SIMD, so
    // that on the same tile the two take turns and a wave that falls a tile
    // behind is served first.
    const bool young = wave >= DEC_WAVES / 2;
    for (int j = 0; kg + j * KG < n_tiles; j += 2) {
        const int t0 = kg + j * KG, t1 = t0 + KG, t2 = t1 + KG, t3 = t2 + KG;
        if (t1 < n_tiles) wait_vmcnt<OPS>();
        else wait_vmcnt<0>();
        if (young) __builtin_amdgcn_s_setprio(0); else __builtin_amdgcn_s_setprio(1);
        tile_step(t0, &ring[0][wave][0], stl0, t2 < n_tiles ? t2 : -1);
        if (t1 < n_tiles) {
            if (t2 < n_tiles) wait_vmcnt<OPS>();
            else wait_vmcnt<0>();
            if (young) __builtin_amdgcn_s_setprio(1); else __builtin_amdgcn_s_setprio(0);
            tile_step(t1, &ring[1][wave][0], stl1, t3 < n_tiles ? t3 : -1);
        }
    }
    __builtin_amdgcn_s_setprio(0);

    // ---- merge the key groups of each row tile (as k_fattn_q8_0's epilogue) ----
    {
        const float l = sum_lanes16_32(l_run);
        float2 * mlw = (float2 *) &scl[wave][0][0][0];
        if (lg == 0) mlw[ln] = make_float2(m_run, l);
    }
    __syncthreads();   // every wave is done with its ring stages, and its (max, sum) are out
    float M = -INFINITY, L = 0.f;
#pragma unroll
    for (int k2 = 0; k2 < KG; k2++) M = xmax(M, ((const float2 *) &scl[k2 * RT + tile][0][0][0])[ln].x);
#pragma unroll
    for (int k2 = 0; k2 < KG; k2++) {
        const float2 e = ((const float2 *) &scl[k2 * RT + tile][0][0][0])[ln];
        L += e.x == -INFINITY ? 0.f : e.y * exp2f(e.x - M);
    }
    const float fw = m_run == -INFINITY ? 0.f : exp2f(m_run - M);
    int tid_e = (int) threadIdx.x;
    asm volatile("" : "+v"(tid_e));
    const int ln_e = tid_e & 15, lg_e = (tid_e >> 4) & 3;
    const int rl = wr0 + ln_e;
    float * ob = (float *) &ring[0][0][0];
    const int orow = rl * DEC_OBS + 8 * lg_e;
    float4 acc[NBLK][2];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        const v4f o0 = O[bb][0] * fw, o1 = O[bb][1] * fw;
        acc[bb][0] = make_float4(o0[0], o1[0], o0[1], o1[1]);
        acc[bb][1] = make_float4(o0[2], o1[2], o0[3], o1[3]);
    }
    if (kg != 0) {
        float * d = ob + (kg - 1) * ROWS * DEC_OBS + orow;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            *(float4 *) (d + 32 * bb) = acc[bb][0];
            *(float4 *) (d + 32 * bb + 4) = acc[bb][1];
        }
    }
    __syncthreads();
    if constexpr (GATHER) {
        if (threadIdx.x == 0 && g_bad && a.status) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
    }
    if (kg == 0 && rl < RW) {
#pragma unroll 1
        for (int k2 = 0; k2 < KG - 1; k2++) {
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                const float * src = ob + k2 * ROWS * DEC_OBS + orow + 32 * bb;
                const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
                acc[bb][0].x += x0.x; acc[bb][0].y += x0.y; acc[bb][0].z += x0.z; acc[bb][0].w += x0.w;
                acc[bb][1].x += x1.x; acc[bb][1].y += x1.y; acc[bb][1].z += x1.z; acc[bb][1].w += x1.w;
            }
        }
        const size_t bh = (size_t) b * a.nh_kv + kvh;
        const int r = rl;
        const int tq = (int) div_gqa(a, (uint32_t) r), h = kvh * a.gqa + (r - tq * a.gqa);
        float * out;
        float oscale;
        const bool nsplit = a.ns > 1;
        if (!nsplit) {
            out = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + 8 * lg_e;
            oscale = L > 0.f ? 1.f / L : 0.f;
        } else {
            out = a.part_o + ((bh * a.ns + split) * a.R + r) * D + 8 * lg_e;
            oscale = 1.f;
            if (lg_e == 0) {
                float2 * mlp = &a.part_ml[(bh * a.ns + split) * a.R + r];
                if (a.mctr) {
                    store_dev2(dev_rsrc(a.part_ml), (uint32_t) ((const char *) mlp - (const char *) a.part_ml),
                               make_float2(M, L));
                } else {
                    __builtin_nontemporal_store(M, &mlp->x);
                    __builtin_nontemporal_store(L, &mlp->y);
                }
            }
        }
        const __amdgpu_buffer_rsrc_t prs = dev_rsrc(a.part_o);
        const uint32_t poff = (uint32_t) ((const char *) out - (const char *) a.part_o);
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            const float4 p0 = acc[bb][0], p1 = acc[bb][1];
            const float4 w0 = make_float4(p0.x * oscale, p0.y * oscale, p0.z * oscale, p0.w * oscale);
            const float4 w1 = make_float4(p1.x * oscale, p1.y * oscale, p1.z * oscale, p1.w * oscale);
            if (nsplit && a.mctr) {
                store_dev4(prs, poff + 128 * bb, w0);
                store_dev4(prs, poff + 128 * bb + 16, w1);
            } else if (nsplit) {
                store_nt4(out + 32 * bb, w0);
                store_nt4(out + 32 * bb + 4, w1);
            } else if (a.dst_vec) {
                *(float4 *) (out + 32 * bb) = apply_gate(a, out + 32 * bb, w0);
                *(float4 *) (out + 32 * bb + 4) = apply_gate(a, out + 32 * bb + 4, w1);
            } else {
                float * o = out + 32 * bb;
                o[0] = w0.x; o[1] = w0.y; o[2] = w0.z; o[3] = w0.w;
                o[4] = w1.x; o[5] = w1.y; o[6] = w1.z; o[7] = w1.w;
            }
        }
    }
    if (a.mctr) fa_merge_tail<DEC_WAVES * 64>(a, b, kvh, (float *) &ring[0][0][0]);
}

// ================================================================ many per-position cell lists
//
// k_fa_qc<KG> (KG = 2, 4, 8): attention of many query positions, each over its own list of
// cache cells (the keys a query of a QSA-on prefill chunk sees: its selected
// cells at or before its position, qwfn_graph.cpp:388-414 and :466-471), with
// the list lengths on the device. A unit is one (position, KV head) list and
// its n_head / n_head_kv query rows (at most 16: one MFMA tile, rows past the
// group zero). A block of 8 waves takes 8 / KG units of one KV head; the KG
// waves of a unit take its 16-key tiles round robin, each through a private
// two-stage LDS-DMA ring as k_fa_dec's waves do, with the same arithmetic per
// tile (exact i8 block dots of the requantised query, d_q*d_k per block,
// online base-2 softmax, P*d_v as f16 hi + lo). No key splits: the KG waves
// merge in LDS and the unit's rows go straight to dst (times sigmoid(gate)).
// Blocks alternate over the KV heads, so with 2 KV heads each XCD's L2 serves
// one head's rows.
//
// The tile's cells come by LDS DMA too, into four slots per wave, so every
// vector-memory load of the key loop is a DMA and the explicit counts stay
// exact: a step issues the K and V rows of the wave's tile two ahead (5 DMAs
// each) and the cells of the tile four ahead (1 DMA), 11 in all, including
// tiles past the list (their offsets lie past the buffers: zeros, no memory
// access). So when step j starts, the ops issued after tile j's V rows are
// the cells of tile j + 2, tile j + 1's K and V and the cells of tile j + 3:
// vmcnt <= 12 means tile j has landed, and <= 11 that tile j + 2's cells have.

constexpr int QC_WAVES  = 8;
constexpr int QC_STAGE  = 2 * DEC_KB;                 // 8704: a tile's K and V rows
constexpr int QC_SLOTS  = 4;                          // cell slots of a wave (16 cells each)
constexpr int QC_AHEAD  = 2 * DEC_TDMA + 2;           // 12: DMAs issued after a tile's V rows when its step starts

struct qc_args {
    const char *    q;            // F32 [256, T, n_head]: position stride q_nb1, head stride q_nb2
    uint32_t        q_nb1, q_nb2, q_bytes;
    const char *    k;            // q8_0 cache rows: row stride k_nb1, KV head offset k_nb2
    const char *    v;
    uint32_t        k_nb1, v_nb1, k_nb2, v_nb2;
    uint32_t        k_bytes, v_bytes;   // n_rows * row stride
    int64_t         n_rows;
    const int32_t * cells;        // list of position t at cells + t * cell_stride
    int64_t         cell_stride;
    const int32_t * counts;       // [T] list lengths (device)
    int64_t         pos0;         // position of query 0
    int32_t         T, nh, nh_kv, gqa;
    float           scale_log2;   // scale * log2(e)
    int32_t         x86;
    float *         dst;          // F32 [256, n_head, T] contiguous
    const float *   gate;         // null or dst's layout
    uint32_t *      status;
};

template <int KG>
__global__ __launch_bounds__(QC_WAVES * 64, 1) void k_fa_qc(qc_args a) {
    constexpr int UPB = QC_WAVES / KG;                 // units of a block
    constexpr int QR = 16 * UPB;                       // query rows staged by the block
    constexpr int OPS = 2 * DEC_TDMA + 1;              // DMAs of a step
    static_assert(QC_AHEAD == OPS + 1, "a step's DMAs and the cells issued before the next tile");
    __shared__ __attribute__((aligned(16))) uint8_t ring[2][QC_WAVES][QC_STAGE];
    __shared__ __attribute__((aligned(16))) uint16_t scl[QC_WAVES][2][NBLK][DEC_TK];
    __shared__ __attribute__((aligned(16))) int32_t cslot[QC_WAVES][QC_SLOTS][DEC_TK];
    static_assert(QR * DEC_QROW <= QC_WAVES * QC_STAGE, "query rows fit stage 1");
    static_assert(QR * NBLK * QWIN + QR * NBLK * 4 <= QC_WAVES * QC_STAGE, "query image fits stage 1");
    static_assert((KG - 1) * QR * DEC_OBS * 4 <= 2 * QC_WAVES * QC_STAGE, "merge buffers fit the ring");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const int unit = wave / KG, kg = wave % KG;
    const int kvh = (int) (blockIdx.x % (unsigned) a.nh_kv);
    const int t0 = (int) (blockIdx.x / (unsigned) a.nh_kv) * UPB;   // the block's first position
    const int t = t0 + unit;
    const bool live = t < a.T;
    const int tq = live ? t : a.T - 1;                 // a unit past the last position reads its rows, stores nothing
    int64_t n = live ? (int64_t) a.counts[t] : 0;
    bool bad = n < 0 || n > a.cell_stride;             // a count outside [0, cell_stride] is clipped and flagged
    n = n < 0 ? 0 : (n > a.cell_stride ? a.cell_stride : n);
    const int span = (int) n;
    const int n_tiles = (span + DEC_TK - 1) / DEC_TK;
    const int J = kg < n_tiles ? (n_tiles - kg + KG - 1) / KG : 0;   // the wave's tiles kg, kg + KG, ...
    const char * kbase = a.k + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) kvh * a.v_nb2;
    const v4i rk = make_rsrc(kbase, a.k_bytes), rv = make_rsrc(vbase, a.v_bytes);
    const v4i rc = make_rsrc(a.cells + (size_t) tq * (size_t) a.cell_stride, (uint32_t) span * 4u);
    // the query's position, clipped to int32 (cells are int32)
    const int32_t q_pos = a.pos0 + tq < INT32_MAX ? (int32_t) (a.pos0 + tq) : INT32_MAX;

    // ---- DMA issue: piece p = 64 s + lane of a tile is byte 16 (p % 17) of
    //      the row of its key p / 17; keys past the list, and cells outside
    //      the cache, get an offset past the buffer (zeros, and the key is
    //      masked) ----
    const uint32_t stl0 = lds_addr(&ring[0][0][0]) + (uint32_t) wave * QC_STAGE;
    const uint32_t stl1 = stl0 + QC_WAVES * QC_STAGE;
    const uint32_t csl = lds_addr(&cslot[wave][0][0]);
    // per lane and DMA slot s: the key (p / 17) and the byte within its row
    uint32_t skey[DEC_TDMA], spart[DEC_TDMA];
#pragma unroll
    for (int s = 0; s < DEC_TDMA; s++) {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u;
        skey[s] = (key < DEC_TK ? key : 0u) * 4u;          // byte offset in the slot (lanes past the tile: key 0)
        spart[s] = (p - key * 17u) * 16u;
    }
    // the rows of the wave's tile j: a key past the list reads a cell that is
    // 0 or another cell of the list (the DMA of the cells zero-fills past the
    // list) and is masked by the key check; a cell outside the cache gets
    // offsets past the buffer (zeros, no memory access)
    uint32_t srow[DEC_TDMA];
    auto load_rows = [&](int j) __attribute__((always_inline)) {
        const uint8_t * sl = (const uint8_t *) &cslot[wave][j & (QC_SLOTS - 1)][0];
#pragma unroll
        for (int s = 0; s < DEC_TDMA; s++) {
            const uint32_t row = *(const uint32_t *) (sl + skey[s]);
            srow[s] = row < (uint32_t) a.n_rows ? row : 0xffffffffu;
        }
    };
    auto issue_rows = [&](uint32_t stl, v4i r, uint32_t nb1, auto base_c) __attribute__((always_inline)) {
        constexpr uint32_t B = decltype(base_c)::value;
        uint32_t o[DEC_TDMA];
#pragma unroll
        for (int s = 0; s < DEC_TDMA; s++) o[s] = srow[s] != 0xffffffffu ? srow[s] * nb1 + spart[s] : 0x80000000u;
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the cells are read and this wave's reads of the stage are done
        dma16_buf_at<B>(r, o[0], stl);
        dma16_buf_at<B + 1024>(r, o[1], stl);
        dma16_buf_at<B + 2048>(r, o[2], stl);
        dma16_buf_at<B + 3072>(r, o[3], stl);
        static_assert(DEC_TDMA == 5, "five DMAs per tensor");
        if (lane < 16) dma16_buf_at<B + 4096>(r, o[4], stl);
    };
    // K rows of tile j (reads its cells), then V rows of the same tile
    auto issue_k = [&](int j, uint32_t stl) __attribute__((always_inline)) {
        load_rows(j);
        issue_rows(stl, rk, a.k_nb1, std::integral_constant<uint32_t, 0>{});
    };
    auto issue_v = [&](uint32_t stl) __attribute__((always_inline)) {
        issue_rows(stl, rv, a.v_nb1, std::integral_constant<uint32_t, DEC_KB>{});
    };
    // the 16 cells of the wave's tile j into slot j % 4 (lanes 0-3, 16 bytes each)
    auto issue_cells = [&](int j) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's reads of the slot are done
        if (lane < 4)
            dma16_buf(rc, (uint32_t) (((kg + j * KG) * DEC_TK + 4 * lane) * 4),
                      csl + (uint32_t) ((j & (QC_SLOTS - 1)) * DEC_TK * 4));
    };

    // ---- prologue: the block's query rows (one wave DMA per row) into stage 1
    //      and the cells of the wave's first four tiles; then tile 0 ----
    uint8_t * qstage = &ring[1][0][0];
    {
        const v4i rq = make_rsrc(a.q, a.q_bytes);
#pragma unroll
        for (int jr = 0; jr < QR / QC_WAVES; jr++) {
            const int rl = wave + QC_WAVES * jr, U = rl / 16, r = rl % 16;
            const int tU = t0 + U < a.T ? t0 + U : a.T - 1;
            if (r < a.gqa)
                dma16_buf(rq, (uint32_t) tU * a.q_nb1 + (uint32_t) (kvh * a.gqa + r) * a.q_nb2 + 16u * (uint32_t) lane,
                          __builtin_amdgcn_readfirstlane(lds_addr(qstage + rl * DEC_QROW)));
        }
        // own tiles 0..3: lane l takes piece l % 4 of tile l / 4
        if (lane < 16)
            dma16_buf(rc, (uint32_t) (((kg + (lane >> 2) * KG) * DEC_TK + 4 * (lane & 3)) * 4), csl);
    }
    wait_vmcnt<0>();   // this wave's query rows and cells have landed
    __syncthreads();   // ... and every wave's: the query rows are read across the block
    issue_k(0, stl0);
    issue_v(stl0);

    // ---- requantisation of the query rows (ggml's quantiser): wave w takes
    //      q8_0 block w of every row, QL lanes per row ----
    constexpr int QL = 64 / QR, QV = 32 / QL;
    static_assert(NBLK == QC_WAVES, "one block of all rows per wave");
    static_assert(QR * QL == 64, "QL lanes per row");
    const int qrow = lane / QL, qh = lane % QL;
    const bool qv = (qrow % 16) < a.gqa;               // rows past the head group stay zero
    float qx[QV];
    {
        const float4 * src = (const float4 *) (qstage + qrow * DEC_QROW + (QK * wave + QV * qh) * 4);
#pragma unroll
        for (int m = 0; m < QV / 4; m++) {
            const float4 v = qv ? src[m] : make_float4(0.f, 0.f, 0.f, 0.f);
            qx[4 * m] = v.x; qx[4 * m + 1] = v.y; qx[4 * m + 2] = v.z; qx[4 * m + 3] = v.w;
        }
    }
    __syncthreads();   // every query value is in registers: stage 1 becomes the window image
    uint8_t * qwin = qstage;
    auto qslice = [&](int bb, int sl, int row) { return qwin + ((bb * 4 + sl) * QR + row) * 16; };
    float * dql = (float *) (qstage + NBLK * QWIN * QR);          // [QR][NBLK]
    {
#pragma unroll
        for (int z = 0; z < 4 / QL; z++) *(uint4 *) qslice(wave, qh * (4 / QL) + z, qrow) = make_uint4(0, 0, 0, 0);
        wave_lds_sync();
        uint32_t w[QV / 4];
        uint16_t d16;
        float dqv = 0.f;
        if (a.x86) dev::q8_quantize_lanes<QV>(qx, true, w, &d16, &dqv);
        else       dev::q8_quantize_lanes<QV>(qx, false, w, &d16, &dqv);
        if (qv) {
            const int woff = (int) ((0x200E0C0A08061402ull >> (8 * wave)) & 0xff);   // win_off(wave)
#pragma unroll
            for (int m = 0; m < QV / 2; m++) {   // 2-byte pieces never straddle a slice
                const int o = woff + QV * qh + 2 * m;
                *(uint16_t *) (qslice(wave, o >> 4, qrow) + (o & 15)) = (uint16_t) (w[m >> 1] >> (16 * (m & 1)));
            }
        }
        if (qh == 0) dql[qrow * NBLK + wave] = qv ? dqv * a.scale_log2 : 0.f;
    }
    static_assert(win_off(0) == 2 && win_off(1) == 20 && win_off(2) == 6 && win_off(3) == 8 && win_off(4) == 10 &&
                  win_off(5) == 12 && win_off(6) == 14 && win_off(7) == 32, "the packed window offsets");
    __syncthreads();
    const int rl_lane = unit * 16 + ln;
    v4i qw[NBLK];
    float dq[NBLK];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        qw[bb] = *(const v4i *) qslice(bb, lg, rl_lane);
        dq[bb] = dql[rl_lane * NBLK + bb];
    }
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) asm volatile("" : "+v"(qw[bb]), "+v"(dq[bb]));
    __syncthreads();   // every wave has its operands: stage 1 is free
    // the order of a steady step (tile 0's V rows, then tile 2's cells, tile
    // 1's K and V, tile 3's cells): tiles 2 and 3's cells are already in
    // their slots and arrive again, unchanged
    issue_cells(2);
    issue_k(1, stl1);
    issue_v(stl1);
    issue_cells(3);

    // ---- the key loop ----
    v4f O[NBLK][2];
    float m_run = -INFINITY, l_run = 0.f;
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) { O[bb][0] = v4f{0, 0, 0, 0}; O[bb][1] = v4f{0, 0, 0, 0}; }
    uint16_t (*sw)[NBLK][DEC_TK] = scl[wave];

    // the wave's tile j from stage st; then tile j + 2 into the same stage
    // (its K rows once the QK is done, its V rows after the PV) and tile j +
    // 4's cells into tile j's slot
    auto tile_step = [&](int j, uint8_t * st, uint32_t stl) __attribute__((always_inline)) {
        const int kin = (kg + j * KG) * DEC_TK + lg * 4;   // the lane's first key, within the list
        {
            const uint8_t * src = st + (lane >> 3) * SEG + (lane & 7) * QBLOCK;
            uint16_t * dstw = &sw[0][lane & 7][lane >> 3];
            uint16_t sv[4];
#pragma unroll
            for (int nn = 0; nn < 4; nn++) sv[nn] = *(const uint16_t *) (src + (nn >> 1) * DEC_KB + (nn & 1) * 8 * SEG);
#pragma unroll
            for (int nn = 0; nn < 4; nn++) dstw[(nn >> 1) * NBLK * DEC_TK + (nn & 1) * 8] = sv[nn];
        }
        wave_lds_sync();
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        {
            v4i kA[NBLK];
            uint2 dk[NBLK];
            const uint8_t * krow = st + ln * SEG + 16 * lg;
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                kA[bb] = *(const v4i *) (krow + 16 * win_piece(bb));
                dk[bb] = *(const uint2 *) &sw[0][bb][lg * 4];
            }
            v4i cc[NBLK];
            cc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[0], qw[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            cc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[1], qw[1], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                if (bb + 2 < NBLK)
                    cc[bb + 2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kA[bb + 2], qw[bb + 2], v4i{0, 0, 0, 0}, 0, 0, 0);
                const float d = dq[bb];
                s[0] = __builtin_fmaf((float) cc[bb][0], mul_f16lo(d, dk[bb].x), s[0]);
                s[1] = __builtin_fmaf((float) cc[bb][1], mul_f16hi(d, dk[bb].x), s[1]);
                s[2] = __builtin_fmaf((float) cc[bb][2], mul_f16lo(d, dk[bb].y), s[2]);
                s[3] = __builtin_fmaf((float) cc[bb][3], mul_f16hi(d, dk[bb].y), s[3]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        wait_vmcnt<QC_AHEAD - 1>();   // tile j + 2's cells have landed
        issue_k(j + 2, stl);
        float p[4];
        uint32_t p16[2];
        {
            // a cell is seen by the queries at or after its position; keys
            // past the list and cells outside the cache are masked (and the
            // latter flagged)
            const int4 c = *(const int4 *) &cslot[wave][j & (QC_SLOTS - 1)][lg * 4];
            const int cv[4] = {c.x, c.y, c.z, c.w};
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bool in = kin + i < span;
                const bool row_ok = (uint32_t) cv[i] < (uint32_t) a.n_rows;
                bad |= in && !row_ok;
                x[i] = in && row_ok && cv[i] <= q_pos ? s[i] : -INFINITY;
            }
            float mloc = vmax(vmax(x[0], x[1]), vmax(x[2], x[3]));
            mloc = xmax_lanes16_32(mloc);
            const bool grow = mloc > m_run + RESCALE_SLACK;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(m_run - mloc);
                m_run = mloc;
            }
            const float m_use = m_run == -INFINITY ? 0.f : m_run;
            float lsum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
                lsum += p[i];
            }
            l_run = l_run * alpha + lsum;
            p16[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[0], p[1]));
            p16[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[2], p[3]));
            if (__any(grow)) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[bb][0] *= alpha; O[bb][1] *= alpha; }
            }
        }
        const uint8_t * vrow = st + DEC_KB + (lg * 4) * SEG + 2 + 2 * ln;
        uint32_t w[NBLK][4];
        uint2 dv2[NBLK];
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
#pragma unroll
            for (int jj = 0; jj < 4; jj++) w[bb][jj] = *(const uint16_t *) (vrow + jj * SEG + bb * QBLOCK);
            dv2[bb] = *(const uint2 *) &sw[1][bb][lg * 4];
        }
        uint32_t a0[2], a1[2], bh[2], bl[2];
        {
            const uint32_t dv[2] = {dv2[0].x, dv2[0].y};
            cvt_v_block(w[0], a0, a1);
            pdv_hilo(p, p16, dv, bh, bl);
        }
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            const v4h A0 = __builtin_bit_cast(v4h, make_uint2(a0[0], a0[1]));
            const v4h A1 = __builtin_bit_cast(v4h, make_uint2(a1[0], a1[1]));
            const v4h Bh = __builtin_bit_cast(v4h, make_uint2(bh[0], bh[1]));
            const v4h Bl = __builtin_bit_cast(v4h, make_uint2(bl[0], bl[1]));
            O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bh, O[bb][0], 0, 0, 0);
            O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bh, O[bb][1], 0, 0, 0);
            if (bb + 1 < NBLK) {
                const uint32_t dv[2] = {dv2[bb + 1].x, dv2[bb + 1].y};
                cvt_v_block(w[bb + 1], a0, a1);
                pdv_hilo(p, p16, dv, bh, bl);
            }
            O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bl, O[bb][0], 0, 0, 0);
            O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bl, O[bb][1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        issue_v(stl);                  // the rows issue_k(j + 2) read
        issue_cells(j + 4);
    };
    // Waves w and w + 4 share a SIMD: their priorities alternate with the tile,
    // in opposite phase, so that neither runs its tiles ahead of the other
    // and then finishes alone at half the vector rate.
    const bool young = wave >= QC_WAVES / 2;
    for (int j = 0; j < J; j += 2) {
        wait_vmcnt<QC_AHEAD>();
        if (young) __builtin_amdgcn_s_setprio(0); else __builtin_amdgcn_s_setprio(1);
        tile_step(j, &ring[0][wave][0], stl0);
        if (j + 1 < J) {
            wait_vmcnt<QC_AHEAD>();
            if (young) __builtin_amdgcn_s_setprio(1); else __builtin_amdgcn_s_setprio(0);
            tile_step(j + 1, &ring[1][wave][0], stl1);
        }
    }
    __builtin_amdgcn_s_setprio(0);
    wait_vmcnt<0>();   // every DMA of the wave has landed (those past the list included)

    // ---- merge the KG waves of each unit ----
    {
        const float l = sum_lanes16_32(l_run);
        float2 * mlw = (float2 *) &scl[wave][0][0][0];   // the wave's own scale table, done with
        if (lg == 0) mlw[ln] = make_float2(m_run, l);
    }
    if (__any(bad) && lane == 0 && a.status) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
    __syncthreads();   // every wave is done with its ring stages, and its (max, sum) are out
    float M = -INFINITY, L = 0.f;
#pragma unroll
    for (int k2 = 0; k2 < KG; k2++) M = xmax(M, ((const float2 *) &scl[unit * KG + k2][0][0][0])[ln].x);
#pragma unroll
    for (int k2 = 0; k2 < KG; k2++) {
        const float2 e = ((const float2 *) &scl[unit * KG + k2][0][0][0])[ln];
        L += e.x == -INFINITY ? 0.f : e.y * exp2f(e.x - M);
    }
    const float fw = m_run == -INFINITY ? 0.f : exp2f(m_run - M);
    int tid_e = (int) threadIdx.x;
    asm volatile("" : "+v"(tid_e));
    const int ln_e = tid_e & 15, lg_e = (tid_e >> 4) & 3;
    float * ob = (float *) &ring[0][0][0];
    const int orow = ln_e * DEC_OBS + 8 * lg_e;
    float4 acc[NBLK][2];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        const v4f o0 = O[bb][0] * fw, o1 = O[bb][1] * fw;
        acc[bb][0] = make_float4(o0[0], o1[0], o0[1], o1[1]);
        acc[bb][1] = make_float4(o0[2], o1[2], o0[3], o1[3]);
    }
    if (KG > 1 && kg != 0) {
        float * d = ob + (unit * (KG - 1) + kg - 1) * 16 * DEC_OBS + orow;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            *(float4 *) (d + 32 * bb) = acc[bb][0];
            *(float4 *) (d + 32 * bb + 4) = acc[bb][1];
        }
    }
    __syncthreads();
    if (kg == 0 && live && ln_e < a.gqa) {
#pragma unroll 1
        for (int k2 = 0; k2 < KG - 1; k2++) {
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                const float * src = ob + (unit * (KG - 1) + k2) * 16 * DEC_OBS + orow + 32 * bb;
                const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
                acc[bb][0].x += x0.x; acc[bb][0].y += x0.y; acc[bb][0].z += x0.z; acc[bb][0].w += x0.w;
                acc[bb][1].x += x1.x; acc[bb][1].y += x1.y; acc[bb][1].z += x1.z; acc[bb][1].w += x1.w;
            }
        }
        const int h = kvh * a.gqa + ln_e;
        const size_t o = ((size_t) t * (size_t) a.nh + (size_t) h) * D + 8 * lg_e;
        float * out = a.dst + o;
        const float oscale = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            const float4 p0 = acc[bb][0], p1 = acc[bb][1];
            float4 w0 = make_float4(p0.x * oscale, p0.y * oscale, p0.z * oscale, p0.w * oscale);
            float4 w1 = make_float4(p1.x * oscale, p1.y * oscale, p1.z * oscale, p1.w * oscale);
            if (a.gate) {
                const float4 g0 = *(const float4 *) (a.gate + o + 32 * bb), g1 = *(const float4 *) (a.gate + o + 32 * bb + 4);
                w0.x = __fmul_rn(w0.x, 1.0f / (1.0f + expf(-g0.x)));
                w0.y = __fmul_rn(w0.y, 1.0f / (1.0f + expf(-g0.y)));
                w0.z = __fmul_rn(w0.z, 1.0f / (1.0f + expf(-g0.z)));
                w0.w = __fmul_rn(w0.w, 1.0f / (1.0f + expf(-g0.w)));
                w1.x = __fmul_rn(w1.x, 1.0f / (1.0f + expf(-g1.x)));
                w1.y = __fmul_rn(w1.y, 1.0f / (1.0f + expf(-g1.y)));
                w1.z = __fmul_rn(w1.z, 1.0f / (1.0f + expf(-g1.z)));
                w1.w = __fmul_rn(w1.w, 1.0f / (1.0f + expf(-g1.w)));
            }
            *(float4 *) (out + 32 * bb) = w0;
            *(float4 *) (out + 32 * bb + 4) = w1;
        }
    }
}

// ================================================================ decode / verify in 32-key steps
//
// k_fa_vd<NF, PK, MASKED, RG, GATHER>: at most 24 query rows per KV head
// (decode, MTP verify, batch decode, sparse cells), one block of 8 waves per
// CU. Every wave holds all of the block's query rows and takes its own steps
// of 32 keys: two 16-key sub-tiles, one per stage of a private two-stage ring
// filled by LDS DMA. Each K/V row of the block is therefore DMA'd, its block
// scales tabulated and its V quants converted once (k_fa_dec does all three
// once per 16-row tile). The rows sit in up to two MFMA tiles:
//   full tile (NF = 1): query rows 0..15, one 16x16 score tile per sub-tile;
//   packed tile (PK = 1): the next 8 rows. Its score tile holds each of them
//     twice: column r for the keys of sub-tile 0, column r + 8 for sub-tile 1.
//     Its QK^T is two MFMAs, one per sub-tile, whose query operand is zero in
//     the other half's columns; its PV operand holds P*d_v of the column's
//     own sub-tile and zeros for the other. The two columns of a row share one
//     running max (a lane swap across the halves) and add up in the epilogue.
// 24 rows (3 tokens x 8 heads) take one tile of each kind, and no vector
// instruction works on a padding column. PV runs on v_mfma_f32_16x16x32_f16:
// the reduction index 8g + 4u + i of lane group g is key 4g + i of sub-tile u,
// in the V^T operand and in P*d_v alike. The arithmetic per score is
// k_fa_dec's: exact i8 block dots of the requantised query, d_q*d_k scaling
// per block, online base-2 softmax, P*d_v as f16 hi + lo.
// Sub-tiles go to the waves round robin (wave w takes sub-tiles w, w + 8,
// w + 16, ...) and a step pairs two of a wave's sub-tiles, 8 apart. A wave
// left with one sub-tile runs a half step: one 16-key sub-tile, PV on
// v_mfma_f32_16x16x16_f16, about 55% of a step's vector work. So a split of
// 16 keys more than 8 steps' worth costs one half step, not one step, and a
// split of 128 keys keeps all 8 waves busy.

constexpr int VD_WAVES  = 8;
constexpr int VD_STEP   = 32;                                   // keys of a step: two 16-key sub-tiles
constexpr int VD_GAP    = VD_WAVES;                             // sub-tiles from a step's first to its second
constexpr int VD_MROWS  = 4;                                    // mask rows (query positions) of a block, at most
constexpr int VD_MBYTES = 2 * VD_MROWS * DEC_MGR * 16;          // a wave's mask granules of one step
constexpr int VD_OBS    = D + 4;                                // epilogue buffer row stride (floats)
constexpr int VD_OBUF   = 32 * VD_OBS;                          // one epilogue buffer: 32 rows (floats)
constexpr int VD_QROW   = 1024;                                 // f32 query row in the prologue's staging
constexpr int VD_ROWS   = 24;                                   // query rows per KV head, at most
static_assert(VD_ROWS * VD_QROW <= VD_WAVES * DEC_KB, "the query rows fit sub-tile 1's V region");
static_assert(4 * VD_OBUF * 4 <= 2 * 2 * VD_WAVES * DEC_KB, "the epilogue buffers fit the ring");

// DPP row_ror:8: lane i of each 16-lane row reads lane i ^ 8 of the same row
__device__ __forceinline__ float swap_halves8(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xF, 0xF, false));
}

template <int NF, int PK, bool MASKED, bool RG, bool GATHER>
__global__ __launch_bounds__(VD_WAVES * 64, 2) void k_fa_vd(fa_args a) {
    static_assert(NF >= 0 && NF <= 1 && PK >= 0 && PK <= 1 && NF + PK >= 1, "a full tile, a packed tile or both");
    static_assert(!(GATHER && (MASKED || RG)), "gathered keys carry their own mask, one sequence");
    constexpr int IR  = 16 * NF + 8 * PK;                  // query rows of the block, at most
    constexpr int NKD = 2 * DEC_TDMA;                      // K DMAs of a step
    constexpr int NVD = 2 * DEC_TDMA + (MASKED ? 1 : 0);   // V and mask DMAs of a step
    asm volatile("" :: "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.mask), "s"(a.m_ne2), "s"(a.part_o));

    // kvr[tensor][u][wave]: sub-tile u's K (tensor 0) or V rows of a wave's
    // step (sub-tile 1 at a fixed offset below 64 KB from sub-tile 0, so one
    // address register serves both). The V rows of sub-tile 1 of all waves are
    // one contiguous region, which holds the block's f32 query rows during the
    // prologue.
    __shared__ __attribute__((aligned(16))) uint8_t kvr[2][2][VD_WAVES][DEC_KB];
    __shared__ __attribute__((aligned(16))) uint8_t mgr[MASKED ? VD_WAVES : 1][MASKED ? VD_MBYTES : 16];
    // query window images [block][16-byte slice][row] of the full tile and of
    // the packed tile; qzero has the packed image's layout and holds zeros
    __shared__ __attribute__((aligned(16))) uint8_t qimf[NF ? NBLK : 1][4][16][16];
    __shared__ __attribute__((aligned(16))) uint8_t qimp[PK ? NBLK : 1][4][8][16];
    __shared__ __attribute__((aligned(16))) uint8_t qzero[PK ? NBLK : 1][4][8][16];
    // one tensor's block scales of a wave's step, [block][key]; after the key
    // loop each wave's (max, sum) per row
    __shared__ __attribute__((aligned(16))) uint16_t stab[VD_WAVES][NBLK][VD_STEP];
    // the query rows' d_q * scale * log2(e), [row][block]
    __shared__ __attribute__((aligned(16))) float dqs[IR][NBLK];
    __shared__ __attribute__((aligned(16))) int32_t gcell[GATHER ? DEC_GATHER_SPLIT : 4];
    __shared__ uint32_t g_bad;   // GATHER: a cell of the block lies outside the cache

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const int hs = ln >> 3;                                // packed tile: the column's sub-tile

    // ---- block -> (b, kvh, split), as k_fa_dec ----
    const int id = blockIdx.x;
    const int hgn = a.nh_kv;
    const int n_units = RG ? a.r_units : a.B * a.ns;
    int kvh, unit;
    if (n_units >= 8) {
        const int j = id >> 3;
        const int jq = (int) udiv((uint32_t) j, (uint32_t) hgn, a.hgn_mul);
        kvh = j - jq * hgn;
        unit = jq * 8 + (id & 7);
    } else {
        unit = (int) udiv((uint32_t) id, (uint32_t) hgn, a.hgn_mul);
        kvh = id - unit * hgn;
    }
    if (unit >= n_units) return;
    int b, split;
    int64_t k_lo, k_hi;
    if constexpr (RG) {
        int32_t us = 0, nsb = 1, slb = 0;
        int64_t nkb = 0;
        b = 0;
#pragma unroll
        for (int i = 0; i < RAGGED_MAX_B; i++)
            if (i < a.B && unit >= a.r_ustart[i]) {
                b = i; us = a.r_ustart[i]; nsb = a.r_ns[i]; slb = a.r_split_len[i]; nkb = a.r_n_kv[i];
            }
        split = unit - us;
        k_lo = (int64_t) split * slb;
        const int64_t e = k_lo + slb;
        k_hi = split == nsb - 1 ? nkb : (nkb < e ? nkb : e);
    } else {
        b = (int) udiv((uint32_t) unit, (uint32_t) a.ns, a.ns_mul);
        split = unit - b * a.ns;
        k_lo = (int64_t) split * a.split_len;
        const int64_t e = k_lo + a.split_len;
        k_hi = split == a.ns - 1 ? a.n_kv : (a.n_kv < e ? a.n_kv : e);
    }
    if constexpr (GATHER) {
        const int li = b * a.nh_kv + kvh;
        int64_t nh = 0;
#pragma unroll
        for (int i = 0; i < GATHER_MAX_LISTS; i++)
            if (i == li) nh = a.g_n[i];
        k_hi = k_hi < nh ? k_hi : nh;
        k_lo = k_lo < k_hi ? k_lo : k_hi;
    }
    const int span = (int) (k_hi - k_lo);
    const int n_sub = (span + DEC_TK - 1) / DEC_TK;         // 16-key sub-tiles of the split
    const int RW = a.R;                                    // the block's rows: all of the KV head's

    const char * kbase = a.k + (size_t) bmod(b, a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) bmod(b, a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;

    // ---- mask (shared by the heads): n_mr query positions. One DMA a step
    //      brings 3 granules of 16 bytes per (sub-tile, position) from the
    //      16-byte aligned address at or below the sub-tile's first key; the
    //      lane's keys 4lg.. of a sub-tile then sit at m_lf (full tile,
    //      sub-tile 0; + 48 n_mr for sub-tile 1) or m_lp (packed tile) ----
    const char * mslice = MASKED ? a.mask + (size_t) bmod(b, a.m_ne3) * a.m_nb3 : nullptr;
    const char * mslice_al = (const char *) ((uintptr_t) mslice & ~(uintptr_t) 15);
    const uint32_t mb_off = (uint32_t) (mslice - mslice_al);
    int n_mr = 1;
    uint32_t m_goff = 0, m_lf = 0, m_lp = 0;
    if constexpr (MASKED) {
        n_mr = (int) div_gqa(a, (uint32_t) (RW - 1)) + 1;
        const int gmax = 2 * n_mr * DEC_MGR;
        const int g = lane < gmax ? lane : gmax - 1;
        const int su = g / (n_mr * DEC_MGR), mr = (g / DEC_MGR) % n_mr;
        m_goff = ((mb_off + (uint32_t) mr * (uint32_t) a.m_nb1) & ~15u) + (uint32_t) (VD_GAP * DEC_TK * 2) * (uint32_t) su +
                 16u * (uint32_t) (g % DEC_MGR);
        auto lane_at = [&](int row, int su2) -> uint32_t {
            const int mr2 = (int) div_gqa(a, (uint32_t) (row < RW ? row : RW - 1));
            return (uint32_t) ((su2 * n_mr + mr2) * DEC_MGR * 16) + ((mb_off + (uint32_t) mr2 * (uint32_t) a.m_nb1) & 15u) +
                   8u * (uint32_t) lg;
        };
        if constexpr (NF) m_lf = lane_at(ln, 0);
        if constexpr (PK) m_lp = lane_at(16 * NF + (ln & 7), hs);
    }

    // ---- per-lane DMA offsets of a sub-tile's pieces: piece p = 64s + lane is
    //      byte 16 (p % 17) of key p / 17 ----
    //      (K and V rows have the same stride: one table serves both)
    uint32_t koff[DEC_TDMA];
#pragma unroll
    for (int s = 0; s < DEC_TDMA; s++) {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u, part = p - key * 17u;
        koff[s] = key * (uint32_t) a.k_nb1 + part * 16u;
    }
    const uint32_t k_sub = (uint32_t) (VD_GAP * DEC_TK) * (uint32_t) a.k_nb1;   // sub-tile 1 of a step
    // the wave's steps start at sub-tiles wave, wave + 16, ... : resources
    // start at the step's first key and end at the split's end (keys past it
    // arrive as zeros, without memory traffic)
    const int64_t key_first = k_lo + (int64_t) wave * DEC_TK;
    const char * k_next = kbase + key_first * (int64_t) a.k_nb1;
    const char * v_next = vbase + key_first * (int64_t) a.v_nb1;
    const char * m_next = mslice_al + key_first * 2;
    int64_t k_rem = (k_hi - key_first) * (int64_t) a.k_nb1, v_rem = (k_hi - key_first) * (int64_t) a.v_nb1;
    int64_t m_rem = (int64_t) a.m_slice + mb_off - key_first * 2;
    const int64_t k_step = (int64_t) (2 * VD_GAP * DEC_TK) * a.k_nb1, v_step = (int64_t) (2 * VD_GAP * DEC_TK) * a.v_nb1;
    constexpr int64_t m_step = 2 * VD_GAP * DEC_TK * 2;
    // GATHER: the DMA offsets of sub-tile ti follow its cells (as k_fa_dec)
    const uint32_t g_kbytes = GATHER ? (uint32_t) (a.g_rows * (int64_t) a.k_nb1) : 0u;
    const uint32_t g_vbytes = GATHER ? (uint32_t) (a.g_rows * (int64_t) a.v_nb1) : 0u;
    auto gather_off = [&](int ti, int s, uint32_t nb1) -> uint32_t {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u, part = p - key * 17u;
        const int kk = ti * DEC_TK + (int) key;
        const uint32_t row = kk < span ? (uint32_t) gcell[kk] : 0xffffffffu;
        return row < (uint32_t) a.g_rows ? row * nb1 + part * 16u : 0x80000000u;
    };
    const uint32_t l_kv = lds_addr(&kvr[0][0][0][0]);
    const uint32_t l_k0 = l_kv + (uint32_t) (0 * VD_WAVES + wave) * DEC_KB, l_k1 = l_kv + (uint32_t) (1 * VD_WAVES + wave) * DEC_KB;
    const uint32_t l_v0 = l_kv + (uint32_t) (2 * VD_WAVES + wave) * DEC_KB, l_v1 = l_kv + (uint32_t) (3 * VD_WAVES + wave) * DEC_KB;
    const uint32_t l_m = lds_addr(&mgr[0][0]) + (uint32_t) (MASKED ? wave * VD_MBYTES : 0);

    auto rsrc_k = [&]() __attribute__((always_inline)) -> v4i {
        if constexpr (GATHER) return make_rsrc(kbase, g_kbytes);
        const v4i r = make_rsrc(k_next, rsrc_bytes(k_rem));
        k_next += k_step;
        k_rem -= k_step;
        return r;
    };
    auto rsrc_v = [&]() __attribute__((always_inline)) -> v4i {
        if constexpr (GATHER) return make_rsrc(vbase, g_vbytes);
        const v4i r = make_rsrc(v_next, rsrc_bytes(v_rem));
        v_next += v_step;
        v_rem -= v_step;
        return r;
    };
    // K rows of the two sub-tiles of the step that starts at sub-tile t0 (10 DMAs)
    auto issue_k = [&](int t0, v4i rk) __attribute__((always_inline)) {
        rk = uniform_rsrc(rk);
        uint32_t o0[DEC_TDMA], o1[DEC_TDMA];
#pragma unroll
        for (int s = 0; s < DEC_TDMA; s++) {
            if constexpr (GATHER) {
                o0[s] = gather_off(t0, s, (uint32_t) a.k_nb1);
                o1[s] = gather_off(t0 + VD_GAP, s, (uint32_t) a.k_nb1);
            } else {
                o0[s] = koff[s];
                o1[s] = koff[s] + k_sub;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's reads of the regions are done
        static_assert(DEC_TDMA == 5, "five DMAs per sub-tile and tensor");
        dma16_buf_at<0>(rk, o0[0], l_k0);
        dma16_buf_at<1024>(rk, o0[1], l_k0);
        dma16_buf_at<2048>(rk, o0[2], l_k0);
        dma16_buf_at<3072>(rk, o0[3], l_k0);
        if (lane < 16) dma16_buf_at<4096>(rk, o0[4], l_k0);
        dma16_buf_at<0>(rk, o1[0], l_k1);
        dma16_buf_at<1024>(rk, o1[1], l_k1);
        dma16_buf_at<2048>(rk, o1[2], l_k1);
        dma16_buf_at<3072>(rk, o1[3], l_k1);
        if (lane < 16) dma16_buf_at<4096>(rk, o1[4], l_k1);
    };
    // V rows of sub-tile su of the step that starts at sub-tile t0 (5 DMAs)
    auto issue_vs = [&](int t0, int su, v4i rv) __attribute__((always_inline)) {
        rv = uniform_rsrc(rv);
        uint32_t o[DEC_TDMA];
#pragma unroll
        for (int s = 0; s < DEC_TDMA; s++) {
            if constexpr (GATHER) o[s] = gather_off(t0 + (su ? VD_GAP : 0), s, (uint32_t) a.v_nb1);
            else o[s] = koff[s] + (su ? k_sub : 0u);
        }
        const uint32_t lv = su ? l_v1 : l_v0;
        __builtin_amdgcn_s_waitcnt(0xC07F);
        dma16_buf_at<0>(rv, o[0], lv);
        dma16_buf_at<1024>(rv, o[1], lv);
        dma16_buf_at<2048>(rv, o[2], lv);
        dma16_buf_at<3072>(rv, o[3], lv);
        if (lane < 16) dma16_buf_at<4096>(rv, o[4], lv);
    };
    // mask granules of a step (one DMA), the next step's resource after it
    auto issue_m = [&]() __attribute__((always_inline)) {
        if constexpr (MASKED) {
            const v4i rm = uniform_rsrc(make_rsrc(m_next, (uint32_t) m_rem));
            m_next += m_step;
            m_rem -= m_step;
            if (lane < 2 * n_mr * DEC_MGR) dma16_buf(rm, m_goff, l_m);
        }
    };

    // ---- prologue: the block's f32 query rows (one wave DMA per row, wave w
    //      takes rows w, w + 8, w + 16) and the cell list (GATHER) first, and
    //      waited for before any K/V DMA: queued behind the K/V requests of
    //      every CU they would arrive microseconds later. Then the fused
    //      append, the first step's K rows, sub-tile 0's V rows and the mask,
    //      which load while the query rows are requantised; sub-tile 1's V
    //      region holds the query rows until then, its DMA follows. ----
    uint8_t * qst = &kvr[1][1][0][0];
    const int first = wave < n_sub ? wave : -1;
    if constexpr (GATHER) {
        const int32_t * cl = a.g_cells + (size_t) b * a.g_bstride + (size_t) kvh * a.g_hstride + k_lo;
        const v4i rc = make_rsrc(cl, (uint32_t) span * 4u);
        for (int m = wave; m * 256 < span; m += VD_WAVES)
            dma16_buf(rc, (uint32_t) (m * 1024 + 16 * lane), __builtin_amdgcn_readfirstlane(lds_addr(&gcell[m * 256])));
        if (threadIdx.x == 0) g_bad = 0;
    }
    {
        const v4i rq = make_rsrc(a.q + (size_t) b * a.q_nb3, a.q_slice);
#pragma unroll
        for (int j = 0; j < (IR + VD_WAVES - 1) / VD_WAVES; j++) {
            const int rl = wave + VD_WAVES * j;
            if (rl >= RW) break;
            const uint32_t r = (uint32_t) rl;
            const uint32_t t = div_gqa(a, r), h = (uint32_t) (kvh * a.gqa) + (r - t * (uint32_t) a.gqa);
            dma16_buf(rq, t * (uint32_t) a.q_nb1 + h * (uint32_t) a.q_nb2 + 16u * (uint32_t) lane,
                      __builtin_amdgcn_readfirstlane(lds_addr(qst + rl * VD_QROW)));
        }
    }
    if (a.app_n > 0) {
        // as in k_fa_dec: the blocks whose keys hold appended rows quantise
        // their KV head's part of them first, and read them back only after
        // their own stores are done
        const int64_t alo = std::max<int64_t>(a.app_row0, k_lo), ahi = std::min<int64_t>(a.app_row0 + a.app_n, k_hi);
        if (alo < ahi) {
            const int units = (int) (ahi - alo) * NBLK * 2;
            const int sub = threadIdx.x & 7;
            for (int u0 = 0; u0 < units; u0 += VD_WAVES * 8) {
                const int uu0 = u0 + (int) (threadIdx.x >> 3);
                const bool live = uu0 < units;
                const int uu = live ? uu0 : 0;
                const int tensor = uu & 1, jb = (uu >> 1) % NBLK;
                const int64_t row = alo + (uu >> 1) / NBLK;
                const float4 xv = *(const float4 *) ((tensor ? a.app_v : a.app_k) + (size_t) (row - a.app_row0) * a.app_nb1 +
                                                     (size_t) (kvh * D + QK * jb + 4 * sub) * 4);
                float x[4] = {xv.x, xv.y, xv.z, xv.w};
                uint16_t d16;
                float dqa;
                const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dqa);
                if (live) {
                    char * bp = (char *) (tensor ? vbase + (size_t) row * a.v_nb1 : kbase + (size_t) row * a.k_nb1) + jb * QBLOCK;
                    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
                    qp[0] = (uint16_t) (q4 & 0xffffu);
                    qp[1] = (uint16_t) (q4 >> 16);
                    if (sub == 0) *(uint16_t *) bp = d16;
                }
            }
        }
    }
    wait_vmcnt<0>();   // this wave's query rows (cells, appended rows) have landed
    __syncthreads();   // ... and every wave's
    if constexpr (GATHER) {
        if ((int) threadIdx.x < span && (uint32_t) gcell[threadIdx.x] >= (uint32_t) a.g_rows) g_bad = 1;
    }
    v4i rv_first{0, 0, 0, 0};
    if (first >= 0) {
        issue_k(first, rsrc_k());
        rv_first = rsrc_v();
        issue_vs(first, 0, rv_first);
        issue_m();
    }

    // ---- requantisation of the query rows (ggml's quantiser): wave w takes
    //      q8_0 block w of every row, two lanes per row ----
    static_assert(NBLK == VD_WAVES, "one block of all rows per wave");
    const int qrow = lane >> 1, qh = lane & 1;
    float qx[16];
    {
        const float4 * src = (const float4 *) (qst + qrow * VD_QROW + (QK * wave + 16 * qh) * 4);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4 v = qrow < RW ? src[m] : make_float4(0.f, 0.f, 0.f, 0.f);
            qx[4 * m] = v.x; qx[4 * m + 1] = v.y; qx[4 * m + 2] = v.z; qx[4 * m + 3] = v.w;
        }
    }
    __syncthreads();   // every query value is in registers: the staging region becomes sub-tile 1's V rows
    if (first >= 0) issue_vs(first, 1, rv_first);
    {
        // zero this wave's block of both images and its share of the zero image
        if constexpr (NF) *(uint4 *) &qimf[wave][lane >> 4][lane & 15][0] = make_uint4(0, 0, 0, 0);
        if constexpr (PK) {
            if (lane < 32) *(uint4 *) &qimp[wave][lane >> 3][lane & 7][0] = make_uint4(0, 0, 0, 0);
            else           *(uint4 *) &qzero[wave][(lane - 32) >> 3][lane & 7][0] = make_uint4(0, 0, 0, 0);
        }
        wave_lds_sync();
        uint32_t w[4];
        uint16_t d16;
        float dqv = 0.f;
        if (a.x86) dev::q8_quantize_lanes<16>(qx, true, w, &d16, &dqv);
        else       dev::q8_quantize_lanes<16>(qx, false, w, &d16, &dqv);
        if (qrow < RW) {
            const int woff = (int) ((0x200E0C0A08061402ull >> (8 * wave)) & 0xff);   // win_off(wave)
            const bool full = qrow < 16 * NF;
            uint8_t * s0 = full ? &qimf[wave][0][NF ? qrow : 0][0] : &qimp[wave][0][PK ? qrow - 16 * NF : 0][0];
            const int sstride = full ? 16 * 16 : 8 * 16;    // bytes between the slices of a row
#pragma unroll
            for (int m = 0; m < 8; m++) {   // 2-byte pieces never straddle a slice
                const int o = woff + 16 * qh + 2 * m;
                *(uint16_t *) (s0 + (o >> 4) * sstride + (o & 15)) = (uint16_t) (w[m >> 1] >> (16 * (m & 1)));
            }
        }
        if (qh == 0 && qrow < IR) dqs[qrow][wave] = qrow < RW ? dqv * (a.scale * LOG2E) : 0.f;
    }
    __syncthreads();   // the images and the d_q table are complete

    // ---- the key loop ----
    v4f Of[NF ? NBLK : 1][2], Op[PK ? NBLK : 1][2];
#pragma unroll
    for (int bb = 0; bb < (NF ? NBLK : 1); bb++) { Of[bb][0] = v4f{0, 0, 0, 0}; Of[bb][1] = v4f{0, 0, 0, 0}; }
#pragma unroll
    for (int bb = 0; bb < (PK ? NBLK : 1); bb++) { Op[bb][0] = v4f{0, 0, 0, 0}; Op[bb][1] = v4f{0, 0, 0, 0}; }
    float mfr = -INFINITY, lfr = 0.f, mpr = -INFINITY, lpr = 0.f;
    // per-lane LDS addresses (block bb at + bb * stride)
    constexpr int SUB1 = VD_WAVES * DEC_KB;                                  // sub-tile 1's region from sub-tile 0's
    const uint8_t * kr0 = &kvr[0][0][wave][0] + ln * SEG + 16 * lg;         // K window slices of key ln
    const uint8_t * vr0 = &kvr[1][0][wave][0] + (4 * lg) * SEG + 2 + 2 * ln;   // V dims 2ln, 2ln+1 of keys 4lg..
    const float * dqf_l = &dqs[NF ? ln : 0][0];                             // the full tile's row
    const float * dqp_l = &dqs[PK ? 16 * NF + (ln & 7) : 0][0];             // the packed tile's row
    const uint8_t * qf_l = &qimf[0][lg][NF ? ln : 0][0];                   // + 1024 bb
    const uint8_t * qp0_l = hs == 0 ? &qimp[0][lg][ln & 7][0] : &qzero[0][lg][ln & 7][0];   // + 512 bb
    const uint8_t * qp1_l = hs == 1 ? &qimp[0][lg][ln & 7][0] : &qzero[0][lg][ln & 7][0];
    const uint8_t * tab = (const uint8_t *) &stab[wave][0][0];
    const uint8_t * tf_l = tab + 8 * lg;                                    // keys 4lg.. of sub-tile 0; + 64 bb (+ 32: sub-tile 1)
    const uint8_t * tp_l = tab + 32 * hs + 8 * lg;                          // the packed column's sub-tile
    const uint8_t * tz = &qzero[0][0][0][0];
    const uint8_t * tpv0_l = hs == 0 ? tp_l : tz;                           // d_v of the packed columns, zero for
    const uint8_t * tpv1_l = hs == 1 ? tp_l : tz;                           // the other half's sub-tile
    const uint8_t * mg = &mgr[MASKED ? wave : 0][0];
    // GATHER: the position of the lane's query rows
    const int64_t qpos_f = GATHER ? a.g_pos0 + b + (int64_t) div_gqa(a, (uint32_t) (NF ? ln : 0)) : 0;
    const int64_t qpos_p = GATHER ? a.g_pos0 + b + (int64_t) div_gqa(a, (uint32_t) (16 * NF + (ln & 7))) : 0;

    // one tensor's block scales of the step into the wave's table [block][key]
    auto tab_fill = [&](int tensor, auto half_tag) __attribute__((always_inline)) {
        constexpr bool HALF = decltype(half_tag)::value;
        const int bq = lane & 7, kq = lane >> 3;
        constexpr int NN = HALF ? 2 : 4;
        uint16_t sv[4];
#pragma unroll
        for (int n = 0; n < NN; n++)
            sv[n] = *(const uint16_t *) (&kvr[tensor][n >> 1][wave][0] + (kq + 8 * (n & 1)) * SEG + bq * QBLOCK);
#pragma unroll
        for (int n = 0; n < NN; n++) stab[wave][bq][16 * (n >> 1) + kq + 8 * (n & 1)] = sv[n];
    };

    // one step from the sub-tiles t0 and t0 + 8 (HALF: t0 only); the next
    // step of the wave starts at sub-tile tn
    auto step = [&](int t0, int tn, auto half_tag) __attribute__((always_inline)) {
        constexpr bool HALF = decltype(half_tag)::value;
        constexpr int NU = HALF ? 1 : 2;                   // sub-tiles of the step
        const bool nx = tn < n_sub;
        wait_vmcnt<NVD>();   // the step's K rows have landed
        tab_fill(0, half_tag);
        wave_lds_sync();

        // ---- S = K Q^T per sub-tile: MFMA rows are keys, columns the rows of
        //      the tile. Each block's MFMAs are issued one block ahead of its
        //      scaling ----
        float sf[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, sp[4] = {0.f, 0.f, 0.f, 0.f};
        {
            v4i cf[2][2], cp[2];
            float4 dq4f[2], dq4p[2];
            auto qk_mfma = [&](int bb) __attribute__((always_inline)) {
                const int sl = bb & 1;
                const v4i a0 = *(const v4i *) (kr0 + 16 * win_piece(bb));
                v4i a1{0, 0, 0, 0};
                if constexpr (!HALF) a1 = *(const v4i *) (kr0 + SUB1 + 16 * win_piece(bb));
                if constexpr (NF) {
                    const v4i qv = *(const v4i *) (qf_l + bb * 1024);
                    cf[sl][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, qv, v4i{0, 0, 0, 0}, 0, 0, 0);
                    if constexpr (!HALF) cf[sl][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, qv, v4i{0, 0, 0, 0}, 0, 0, 0);
                }
                if constexpr (PK) {
                    const v4i q0 = *(const v4i *) (qp0_l + bb * 512);
                    cp[sl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, q0, v4i{0, 0, 0, 0}, 0, 0, 0);
                    if constexpr (!HALF) {
                        const v4i q1 = *(const v4i *) (qp1_l + bb * 512);
                        cp[sl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, q1, cp[sl], 0, 0, 0);
                    }
                }
            };
            auto dq_at = [](const float4 & v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; };
            auto qk_scale = [&](int bb) __attribute__((always_inline)) {
                const int sl = bb & 1;
                if constexpr (NF) {
                    const float d = dq_at(dq4f[bb >> 2], bb & 3);
#pragma unroll
                    for (int su = 0; su < NU; su++) {
                        const uint2 dk = *(const uint2 *) (tf_l + bb * 64 + 32 * su);
                        sf[su][0] = __builtin_fmaf((float) cf[sl][su][0], mul_f16lo(d, dk.x), sf[su][0]);
                        sf[su][1] = __builtin_fmaf((float) cf[sl][su][1], mul_f16hi(d, dk.x), sf[su][1]);
                        sf[su][2] = __builtin_fmaf((float) cf[sl][su][2], mul_f16lo(d, dk.y), sf[su][2]);
                        sf[su][3] = __builtin_fmaf((float) cf[sl][su][3], mul_f16hi(d, dk.y), sf[su][3]);
                    }
                }
                if constexpr (PK) {
                    const uint2 dk = *(const uint2 *) (tp_l + bb * 64);
                    const float d = dq_at(dq4p[bb >> 2], bb & 3);
                    sp[0] = __builtin_fmaf((float) cp[sl][0], mul_f16lo(d, dk.x), sp[0]);
                    sp[1] = __builtin_fmaf((float) cp[sl][1], mul_f16hi(d, dk.x), sp[1]);
                    sp[2] = __builtin_fmaf((float) cp[sl][2], mul_f16lo(d, dk.y), sp[2]);
                    sp[3] = __builtin_fmaf((float) cp[sl][3], mul_f16hi(d, dk.y), sp[3]);
                }
            };
            if constexpr (NF) { dq4f[0] = *(const float4 *) dqf_l; dq4f[1] = *(const float4 *) (dqf_l + 4); }
            if constexpr (PK) { dq4p[0] = *(const float4 *) dqp_l; dq4p[1] = *(const float4 *) (dqp_l + 4); }
            qk_mfma(0);
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                if (bb + 1 < NBLK) qk_mfma(bb + 1);
                qk_scale(bb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // the scores are complete here: otherwise the compiler sinks the
        // scaling past the DMA branch below, keeping every block's integer
        // dots and scale products live at once
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+v"(sf[0][i]), "+v"(sf[1][i]), "+v"(sp[i]));
        if (nx) {
            issue_k(tn, rsrc_k());
            wait_vmcnt<NKD>();   // the step's V rows and mask have landed
        } else {
            wait_vmcnt<0>();
        }
        tab_fill(1, half_tag);
        wave_lds_sync();

        // ---- mask, online softmax (base 2) over the step's keys; sub-tile u
        //      starts at key kb[u] of the split ----
        const int kb0 = DEC_TK * t0, kb1 = DEC_TK * (t0 + VD_GAP);
        auto kb = [&](int su) { return su ? kb1 : kb0; };
        float pf[2][4], pp[4];
        uint32_t pf16[2][2], pp16[2];
        if constexpr (NF) {
            float x[2][4];
#pragma unroll
            for (int su = 0; su < NU; su++) {
#pragma unroll
                for (int i = 0; i < 4; i++) x[su][i] = sf[su][i];
                if constexpr (MASKED) {
                    const uint8_t * mp = mg + m_lf + su * (n_mr * DEC_MGR * 16);
#pragma unroll
                    for (int i = 0; i < 4; i++) x[su][i] = fma_f16lo((uint32_t) *(const uint16_t *) (mp + 2 * i), LOG2E, x[su][i]);
                } else if constexpr (GATHER) {
                    const int kin = kb(su) + 4 * lg;
                    const int4 c = *(const int4 *) &gcell[kin < DEC_GATHER_SPLIT - 3 ? kin : 0];
                    const int cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        x[su][i] = (uint32_t) cv[i] < (uint32_t) a.g_rows && (int64_t) cv[i] <= qpos_f ? x[su][i] : -INFINITY;
                }
                if (kb(su) + DEC_TK > span) {   // the split's last sub-tile: keys past its end
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (kb(su) + 4 * lg + i >= span) x[su][i] = -INFINITY;
                }
            }
            float mloc = vmax(vmax(x[0][0], x[0][1]), vmax(x[0][2], x[0][3]));
            if constexpr (!HALF) mloc = vmax(mloc, vmax(vmax(x[1][0], x[1][1]), vmax(x[1][2], x[1][3])));
            mloc = xmax_lanes16_32(mloc);
            const bool grow = mloc > mfr + RESCALE_SLACK;
            const bool rescale = grow && mfr != -INFINITY;   // the accumulators hold something to rescale
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(mfr - mloc);
                mfr = mloc;
            }
            const float m_use = mfr == -INFINITY ? 0.f : mfr;
            float lsum = 0.f;
#pragma unroll
            for (int su = 0; su < NU; su++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    pf[su][i] = __builtin_amdgcn_exp2f(x[su][i] - m_use);
                    lsum += pf[su][i];
                }
                pf16[su][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pf[su][0], pf[su][1]));
                pf16[su][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pf[su][2], pf[su][3]));
            }
            lfr = lfr * alpha + lsum;
            if (__any(rescale)) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { Of[bb][0] *= alpha; Of[bb][1] *= alpha; }
            }
        }
        if constexpr (PK) {
            float x[4];
            const int kbp = HALF || hs == 0 ? kb0 : kb1;   // the packed column's sub-tile (HALF: only sub-tile 0 has keys)
#pragma unroll
            for (int i = 0; i < 4; i++) x[i] = sp[i];
            if constexpr (MASKED) {
                const uint8_t * mp = mg + m_lp;
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = fma_f16lo((uint32_t) *(const uint16_t *) (mp + 2 * i), LOG2E, x[i]);
            } else if constexpr (GATHER) {
                const int kin = kbp + 4 * lg;
                const int4 c = *(const int4 *) &gcell[kin < DEC_GATHER_SPLIT - 3 ? kin : 0];
                const int cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    x[i] = (uint32_t) cv[i] < (uint32_t) a.g_rows && (int64_t) cv[i] <= qpos_p ? x[i] : -INFINITY;
            }
            if (HALF && hs) {
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = -INFINITY;   // no sub-tile 1 in a half step
            } else if (kbp + DEC_TK > span) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (kbp + 4 * lg + i >= span) x[i] = -INFINITY;
            }
            float mloc = vmax(vmax(x[0], x[1]), vmax(x[2], x[3]));
            mloc = xmax_lanes16_32(mloc);
            mloc = vmax(mloc, swap_halves8(mloc));      // both sub-tiles of the row
            const bool grow = mloc > mpr + RESCALE_SLACK;
            const bool rescale = grow && mpr != -INFINITY;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(mpr - mloc);
                mpr = mloc;
            }
            const float m_use = mpr == -INFINITY ? 0.f : mpr;
            float lsum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pp[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
                lsum += pp[i];
            }
            pp16[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pp[0], pp[1]));
            pp16[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pp[2], pp[3]));
            lpr = lpr * alpha + lsum;
            if (__any(rescale)) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { Op[bb][0] *= alpha; Op[bb][1] *= alpha; }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+v"(pf[0][i]), "+v"(pf[1][i]), "+v"(pp[i]));
        asm volatile("" : "+v"(pf16[0][0]), "+v"(pf16[0][1]), "+v"(pf16[1][0]), "+v"(pf16[1][1]), "+v"(pp16[0]), "+v"(pp16[1]));

        // ---- O += V^T (P d_v) per V block over the step's keys. Block bb + 1's
        //      V quants are read while bb is computed ----
        {
            uint32_t w[2][2][4];
            auto load_v = [&](int bb, uint32_t (&ww)[2][4]) __attribute__((always_inline)) {
#pragma unroll
                for (int jv = 0; jv < 4; jv++) {
                    ww[0][jv] = *(const uint16_t *) (vr0 + jv * SEG + bb * QBLOCK);
                    if constexpr (!HALF) ww[1][jv] = *(const uint16_t *) (vr0 + SUB1 + jv * SEG + bb * QBLOCK);
                }
            };
            load_v(0, w[0]);
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                const int cb = bb & 1;
                if (bb + 1 < NBLK) load_v(bb + 1, w[cb ^ 1]);
                uint32_t a00[2], a10[2], a01[2], a11[2];
                cvt_v_block(w[cb][0], a00, a10);
                if constexpr (!HALF) cvt_v_block(w[cb][1], a01, a11);
                if constexpr (NF) {
                    uint32_t bh[2][2], bl[2][2];
#pragma unroll
                    for (int su = 0; su < NU; su++) {
                        const uint2 d = *(const uint2 *) (tf_l + bb * 64 + 32 * su);
                        const uint32_t dv[2] = {d.x, d.y};
                        pdv_hilo(pf[su], pf16[su], dv, bh[su], bl[su]);
                    }
                    if constexpr (HALF) {
                        const v4h A0 = __builtin_bit_cast(v4h, make_uint2(a00[0], a00[1]));
                        const v4h A1 = __builtin_bit_cast(v4h, make_uint2(a10[0], a10[1]));
                        const v4h Bh = __builtin_bit_cast(v4h, make_uint2(bh[0][0], bh[0][1]));
                        const v4h Bl = __builtin_bit_cast(v4h, make_uint2(bl[0][0], bl[0][1]));
                        Of[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bh, Of[bb][0], 0, 0, 0);
                        Of[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bh, Of[bb][1], 0, 0, 0);
                        Of[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bl, Of[bb][0], 0, 0, 0);
                        Of[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bl, Of[bb][1], 0, 0, 0);
                    } else {
                        const v8h A0 = __builtin_bit_cast(v8h, make_uint4(a00[0], a00[1], a01[0], a01[1]));
                        const v8h A1 = __builtin_bit_cast(v8h, make_uint4(a10[0], a10[1], a11[0], a11[1]));
                        const v8h Bh = __builtin_bit_cast(v8h, make_uint4(bh[0][0], bh[0][1], bh[1][0], bh[1][1]));
                        const v8h Bl = __builtin_bit_cast(v8h, make_uint4(bl[0][0], bl[0][1], bl[1][0], bl[1][1]));
                        Of[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bh, Of[bb][0], 0, 0, 0);
                        Of[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bh, Of[bb][1], 0, 0, 0);
                        Of[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bl, Of[bb][0], 0, 0, 0);
                        Of[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bl, Of[bb][1], 0, 0, 0);
                    }
                }
                if constexpr (PK) {
                    uint32_t bh[2][2], bl[2][2];
#pragma unroll
                    for (int su = 0; su < NU; su++) {
                        const uint2 e = *(const uint2 *) ((su ? tpv1_l : tpv0_l) + bb * 64);
                        const uint32_t dv[2] = {e.x, e.y};
                        pdv_hilo(pp, pp16, dv, bh[su], bl[su]);
                    }
                    if constexpr (HALF) {
                        const v4h A0 = __builtin_bit_cast(v4h, make_uint2(a00[0], a00[1]));
                        const v4h A1 = __builtin_bit_cast(v4h, make_uint2(a10[0], a10[1]));
                        const v4h Bh = __builtin_bit_cast(v4h, make_uint2(bh[0][0], bh[0][1]));
                        const v4h Bl = __builtin_bit_cast(v4h, make_uint2(bl[0][0], bl[0][1]));
                        Op[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bh, Op[bb][0], 0, 0, 0);
                        Op[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bh, Op[bb][1], 0, 0, 0);
                        Op[bb][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, Bl, Op[bb][0], 0, 0, 0);
                        Op[bb][1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, Bl, Op[bb][1], 0, 0, 0);
                    } else {
                        const v8h A0 = __builtin_bit_cast(v8h, make_uint4(a00[0], a00[1], a01[0], a01[1]));
                        const v8h A1 = __builtin_bit_cast(v8h, make_uint4(a10[0], a10[1], a11[0], a11[1]));
                        const v8h Bh = __builtin_bit_cast(v8h, make_uint4(bh[0][0], bh[0][1], bh[1][0], bh[1][1]));
                        const v8h Bl = __builtin_bit_cast(v8h, make_uint4(bl[0][0], bl[0][1], bl[1][0], bl[1][1]));
                        Op[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bh, Op[bb][0], 0, 0, 0);
                        Op[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bh, Op[bb][1], 0, 0, 0);
                        Op[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bl, Op[bb][0], 0, 0, 0);
                        Op[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bl, Op[bb][1], 0, 0, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (nx) {
            const v4i rv = rsrc_v();
            issue_vs(tn, 0, rv);
            issue_vs(tn, 1, rv);
            issue_m();
        }
    };

    // The wave's steps. Two waves share a SIMD (waves w and w + 4) and the
    // older one wins its issue slots: the wave priority alternates with the
    // step count, in opposite phase for the two waves of a SIMD.
    const bool young = wave >= VD_WAVES / 2;
    int jj = 0, t0 = first;
    for (; t0 >= 0 && t0 + VD_GAP < n_sub; t0 += 2 * VD_GAP, jj++) {
        if (young == (bool) (jj & 1)) __builtin_amdgcn_s_setprio(1); else __builtin_amdgcn_s_setprio(0);
        step(t0, t0 + 2 * VD_GAP, std::false_type{});
    }
    if (t0 >= 0 && t0 < n_sub) {   // the wave's last sub-tile alone
        if (young == (bool) (jj & 1)) __builtin_amdgcn_s_setprio(1); else __builtin_amdgcn_s_setprio(0);
        step(t0, t0 + 2 * VD_GAP, std::true_type{});
    }
    __builtin_amdgcn_s_setprio(0);

    // ---- epilogue: the waves' (max, sum) per row, each wave's O scaled to the
    //      block max, then summed in two rounds through LDS (waves 4..7 into
    //      0..3, then 0..3 into four buffers that every thread reads) ----
    {
        float2 * mlw = (float2 *) &stab[wave][0][0];           // [row]
        if constexpr (NF) {
            const float l = sum_lanes16_32(lfr);
            if (lg == 0) mlw[ln] = make_float2(mfr, l);
        }
        if constexpr (PK) {
            float l = sum_lanes16_32(lpr);
            l += swap_halves8(l);
            if (lg == 0 && hs == 0) mlw[16 * NF + ln] = make_float2(mpr, l);
        }
    }
    __syncthreads();   // every wave is done with its ring stages, and its (max, sum) are out
    auto block_ml = [&](int row, float & M, float & L) __attribute__((always_inline)) {
        M = -INFINITY;
        L = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < VD_WAVES; w2++) M = xmax(M, ((const float2 *) &stab[w2][0][0])[row].x);
#pragma unroll
        for (int w2 = 0; w2 < VD_WAVES; w2++) {
            const float2 e = ((const float2 *) &stab[w2][0][0])[row];
            L += e.x == -INFINITY ? 0.f : e.y * __builtin_amdgcn_exp2f(e.x - M);
        }
    };
    if constexpr (NF) {
        float M, L;
        block_ml(ln, M, L);
        const float fw = mfr == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mfr - M);
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) { Of[bb][0] *= fw; Of[bb][1] *= fw; }
    }
    if constexpr (PK) {
        float M, L;
        block_ml(16 * NF + (ln & 7), M, L);
        const float fw = mpr == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mpr - M);
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) { Op[bb][0] *= fw; Op[bb][1] *= fw; }
    }
    // buffer rows: the full tile's column c at row c, the packed tile's at 16 NF + c
    float * ob = (float *) &kvr[0][0][0][0];
    int tid_e = (int) threadIdx.x;
    asm volatile("" : "+v"(tid_e));
    const int ln_e = tid_e & 15, lg_e = (tid_e >> 4) & 3;
    auto dump = [&](float * buf) __attribute__((always_inline)) {
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            if constexpr (NF) {
                float * d = buf + ln_e * VD_OBS + 32 * bb + 8 * lg_e;
                *(float4 *) d = make_float4(Of[bb][0][0], Of[bb][1][0], Of[bb][0][1], Of[bb][1][1]);
                *(float4 *) (d + 4) = make_float4(Of[bb][0][2], Of[bb][1][2], Of[bb][0][3], Of[bb][1][3]);
            }
            if constexpr (PK) {
                float * d = buf + (16 * NF + ln_e) * VD_OBS + 32 * bb + 8 * lg_e;
                *(float4 *) d = make_float4(Op[bb][0][0], Op[bb][1][0], Op[bb][0][1], Op[bb][1][1]);
                *(float4 *) (d + 4) = make_float4(Op[bb][0][2], Op[bb][1][2], Op[bb][0][3], Op[bb][1][3]);
            }
        }
    };
    auto add = [&](const float * buf) __attribute__((always_inline)) {
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            if constexpr (NF) {
                const float * d = buf + ln_e * VD_OBS + 32 * bb + 8 * lg_e;
                const float4 x0 = *(const float4 *) d, x1 = *(const float4 *) (d + 4);
                Of[bb][0][0] += x0.x; Of[bb][1][0] += x0.y; Of[bb][0][1] += x0.z; Of[bb][1][1] += x0.w;
                Of[bb][0][2] += x1.x; Of[bb][1][2] += x1.y; Of[bb][0][3] += x1.z; Of[bb][1][3] += x1.w;
            }
            if constexpr (PK) {
                const float * d = buf + (16 * NF + ln_e) * VD_OBS + 32 * bb + 8 * lg_e;
                const float4 x0 = *(const float4 *) d, x1 = *(const float4 *) (d + 4);
                Op[bb][0][0] += x0.x; Op[bb][1][0] += x0.y; Op[bb][0][1] += x0.z; Op[bb][1][1] += x0.w;
                Op[bb][0][2] += x1.x; Op[bb][1][2] += x1.y; Op[bb][0][3] += x1.z; Op[bb][1][3] += x1.w;
            }
        }
    };
    if (wave >= VD_WAVES / 2) dump(ob + (wave - VD_WAVES / 2) * VD_OBUF);
    __syncthreads();
    if (wave < VD_WAVES / 2) {
        add(ob + wave * VD_OBUF);
        dump(ob + wave * VD_OBUF);
    }
    __syncthreads();
    if constexpr (GATHER) {
        if (threadIdx.x == 0 && g_bad && a.status) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
    }
    // ---- the block's rows: thread (row, q) adds dims 16q .. 16q + 15 of the
    //      four buffers (and both columns of a packed row) ----
    const int frow = tid_e >> 4, fq = tid_e & 15;
    if (frow < RW) {
        const bool prow = frow >= 16 * NF;
        const int br = prow ? 16 * NF + (frow - 16 * NF) : frow;
        float4 acc[4];
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w4 = 0; w4 < VD_WAVES / 2; w4++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 x = *(const float4 *) (ob + w4 * VD_OBUF + br * VD_OBS + 16 * fq + 4 * c);
                acc[c].x += x.x; acc[c].y += x.y; acc[c].z += x.z; acc[c].w += x.w;
            }
            if (prow) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float4 x = *(const float4 *) (ob + w4 * VD_OBUF + (br + 8) * VD_OBS + 16 * fq + 4 * c);
                    acc[c].x += x.x; acc[c].y += x.y; acc[c].z += x.z; acc[c].w += x.w;
                }
            }
        }
        float M, L;
        block_ml(frow, M, L);
        const size_t bh = (size_t) b * a.nh_kv + kvh;
        const int tq = (int) div_gqa(a, (uint32_t) frow), h = kvh * a.gqa + (frow - tq * a.gqa);
        if (a.ns > 1) {
            float * out = a.part_o + ((bh * a.ns + split) * a.R + frow) * D + 16 * fq;
            float2 * mlp = &a.part_ml[(bh * a.ns + split) * a.R + frow];
            if (a.mctr) {
                const __amdgpu_buffer_rsrc_t prs = dev_rsrc(a.part_o);
                const uint32_t poff = (uint32_t) ((const char *) out - (const char *) a.part_o);
#pragma unroll
                for (int c = 0; c < 4; c++) store_dev4(prs, poff + 16 * c, acc[c]);
                if (fq == 0)
                    store_dev2(dev_rsrc(a.part_ml), (uint32_t) ((const char *) mlp - (const char *) a.part_ml),
                               make_float2(M, L));
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) store_nt4(out + 4 * c, acc[c]);
                if (fq == 0) {
                    __builtin_nontemporal_store(M, &mlp->x);
                    __builtin_nontemporal_store(L, &mlp->y);
                }
            }
        } else {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            float * out = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + 16 * fq;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 o = make_float4(acc[c].x * inv, acc[c].y * inv, acc[c].z * inv, acc[c].w * inv);
                if (a.dst_vec) {
                    *(float4 *) (out + 4 * c) = apply_gate(a, out + 4 * c, o);
                } else {
                    float * p = out + 4 * c;
                    p[0] = o.x; p[1] = o.y; p[2] = o.z; p[3] = o.w;
                }
            }
        }
    }
    if (a.mctr) fa_merge_tail<VD_WAVES * 64>(a, b, kvh, ob);
}

// ================================================================ decode / verify, value dims split across the waves
//
// k_fa_vs<NF, PK, MASKED, RG, GATHER>: the shapes of k_fa_vd (at most 24
// query rows per KV head, one block of 8 waves per CU), with the work of a
// block split so that no wave holds O for all 256 dims. The keys go in rounds
// of 128: in a round, wave w computes the scores of sub-tile w (16 keys) for
// all rows, the waves agree on each row's running max through LDS, wave w
// publishes its P (its lanes' values are already in the layout the PV
// operand wants, so the exchange is one float4 per lane), and then wave w
// computes O for its own V block (32 dims) over all 128 keys of the round.
// So O is 16 registers a lane instead of 96, no cross-wave reduction of O is
// needed at the end, and each K/V row is still read from HBM once. K and V
// go through two-stage rings (the next round's DMAs are issued as soon as
// every wave has finished the previous round), and the requantised query
// rows stay in registers. The arithmetic per score is k_fa_vd's: exact i8
// block dots, d_q*d_k per block, online base-2 softmax with the running max
// allowed to lag by RESCALE_SLACK (the same decision in every wave: they see
// the same block max), P*d_v as f16 hi + lo. The packed tile (rows 16..23)
// covers one sub-tile per wave: its columns 8..15 are empty in the scores,
// and in PV they carry the odd sub-tiles of each 32-key pair (column c + 8
// for rows of sub-tile 2j+1), which a lane swap adds at the end.

constexpr int VS_WAVES = 8;
constexpr int VS_ROUND = VS_WAVES * DEC_TK;               // 128 keys: one sub-tile per wave
constexpr int VS_MG    = VD_MROWS * DEC_MGR * 16;         // a wave's mask granules of a round
constexpr int VS_QROW  = 1024;                            // f32 query row in the prologue's staging
constexpr int64_t VS_AUTO_MAX_KEYS = 36864;               // the planner's k_fa_vs range (8 rows, one sequence)
static_assert(VD_ROWS * VS_QROW <= VS_WAVES * DEC_KB, "the query rows fit V stage 1");

template <int NF, int PK, bool MASKED, bool RG, bool GATHER>
__global__ __launch_bounds__(VS_WAVES * 64, 2) void k_fa_vs(fa_args a) {
    static_assert(NF >= 0 && NF <= 1 && PK >= 0 && PK <= 1 && NF + PK >= 1, "a full tile, a packed tile or both");
    static_assert(!(GATHER && (MASKED || RG)), "gathered keys carry their own mask, one sequence");
    static_assert(NBLK == VS_WAVES, "one V block per wave");
    constexpr int IR  = 16 * NF + 8 * PK;                  // query rows of the block, at most
    constexpr int NKD = DEC_TDMA + (MASKED ? 1 : 0);       // K and mask DMAs of a wave's round
    constexpr int NVD = DEC_TDMA;                          // V DMAs of a wave's round
    asm volatile("" :: "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.mask), "s"(a.m_ne2), "s"(a.part_o));

    // kr / vr[stage][wave]: sub-tile `wave`'s K (V) rows of a round. V stage 1
    // holds the f32 query rows in the prologue.
    __shared__ __attribute__((aligned(16))) uint8_t kr[2][VS_WAVES][DEC_KB];
    __shared__ __attribute__((aligned(16))) uint8_t vr[2][VS_WAVES][DEC_KB];
    __shared__ __attribute__((aligned(16))) uint8_t mgr[MASKED ? 2 : 1][MASKED ? VS_WAVES : 1][MASKED ? VS_MG : 16];
    // P of a round by sub-tile: the full tile's lanes, the packed tile's lanes
    // with a row (hs = 0) at 8 lg + c
    __shared__ __attribute__((aligned(16))) float4 pxf[NF ? VS_WAVES : 1][NF ? 64 : 1];
    __shared__ __attribute__((aligned(16))) float4 pxp[PK ? VS_WAVES : 1][PK ? 32 : 1];
    __shared__ __attribute__((aligned(16))) uint16_t ktab[VS_WAVES][NBLK][DEC_TK];   // a wave's d_k [block][key]
    __shared__ __attribute__((aligned(16))) uint16_t vtab[VS_WAVES][NBLK][DEC_TK];   // a sub-tile's d_v [block][key]
    __shared__ __attribute__((aligned(16))) float mx[IR][VS_WAVES];   // the waves' row maxima (row sums at the end)
    __shared__ __attribute__((aligned(16))) float dqs[IR][NBLK];      // d_q * scale * log2(e) [row][block]
    __shared__ __attribute__((aligned(16))) int32_t gcell[GATHER ? DEC_GATHER_SPLIT : 4];
    __shared__ uint32_t g_bad;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const int hs = ln >> 3;

    // ---- block -> (b, kvh, split), as k_fa_vd ----
    const int id = blockIdx.x;
    const int hgn = a.nh_kv;
    const int n_units = RG ? a.r_units : a.B * a.ns;
    int kvh, unit;
    if (n_units >= 8) {
        const int j = id >> 3;
        const int jq = (int) udiv((uint32_t) j, (uint32_t) hgn, a.hgn_mul);
        kvh = j - jq * hgn;
        unit = jq * 8 + (id & 7);
    } else {
        unit = (int) udiv((uint32_t) id, (uint32_t) hgn, a.hgn_mul);
        kvh = id - unit * hgn;
    }
    if (unit >= n_units) return;
    int b, split;
    int64_t k_lo, k_hi;
    if constexpr (RG) {
        int32_t us = 0, nsb = 1, slb = 0;
        int64_t nkb = 0;
        b = 0;
#pragma unroll
        for (int i = 0; i < RAGGED_MAX_B; i++)
            if (i < a.B && unit >= a.r_ustart[i]) {
                b = i; us = a.r_ustart[i]; nsb = a.r_ns[i]; slb = a.r_split_len[i]; nkb = a.r_n_kv[i];
            }
        split = unit - us;
        k_lo = (int64_t) split * slb;
        const int64_t e = k_lo + slb;
        k_hi = split == nsb - 1 ? nkb : (nkb < e ? nkb : e);
    } else {
        b = (int) udiv((uint32_t) unit, (uint32_t) a.ns, a.ns_mul);
        split = unit - b * a.ns;
        k_lo = (int64_t) split * a.split_len;
        const int64_t e = k_lo + a.split_len;
        k_hi = split == a.ns - 1 ? a.n_kv : (a.n_kv < e ? a.n_kv : e);
    }
    if constexpr (GATHER) {
        const int li = b * a.nh_kv + kvh;
        int64_t nh = 0;
#pragma unroll
        for (int i = 0; i < GATHER_MAX_LISTS; i++)
            if (i == li) nh = a.g_n[i];
        k_hi = k_hi < nh ? k_hi : nh;
        k_lo = k_lo < k_hi ? k_lo : k_hi;
    }
    const int span = (int) (k_hi - k_lo);
    const int n_sub = (span + DEC_TK - 1) / DEC_TK;          // 16-key sub-tiles of the split
    const int n_rounds = (n_sub + VS_WAVES - 1) / VS_WAVES;  // block-uniform
    const int RW = a.R;

    const char * kbase = a.k + (size_t) bmod(b, a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) bmod(b, a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;

    // ---- mask (shared by the heads): n_mr query positions; one DMA a round
    //      brings 3 granules of 16 bytes per position from the 16-byte aligned
    //      address at or below the sub-tile's first key ----
    const char * mslice = MASKED ? a.mask + (size_t) bmod(b, a.m_ne3) * a.m_nb3 : nullptr;
    const char * mslice_al = (const char *) ((uintptr_t) mslice & ~(uintptr_t) 15);
    const uint32_t mb_off = (uint32_t) (mslice - mslice_al);
    int n_mr = 1;
    uint32_t m_goff = 0, m_lf = 0, m_lp = 0;
    if constexpr (MASKED) {
        n_mr = (int) div_gqa(a, (uint32_t) (RW - 1)) + 1;
        const int gmax = n_mr * DEC_MGR;
        const int g = lane < gmax ? lane : gmax - 1;
        const int mr = g / DEC_MGR;
        m_goff = ((mb_off + (uint32_t) mr * (uint32_t) a.m_nb1) & ~15u) + 16u * (uint32_t) (g % DEC_MGR);
        auto lane_at = [&](int row) -> uint32_t {
            const int mr2 = (int) div_gqa(a, (uint32_t) (row < RW ? row : RW - 1));
            return (uint32_t) (mr2 * DEC_MGR * 16) + ((mb_off + (uint32_t) mr2 * (uint32_t) a.m_nb1) & 15u) + 8u * (uint32_t) lg;
        };
        if constexpr (NF) m_lf = lane_at(ln);
        if constexpr (PK) m_lp = lane_at(16 * NF + (ln & 7));
    }

    // ---- DMA: piece p = 64 s + lane of a sub-tile is byte 16 (p % 17) of key
    //      p / 17 (K and V rows have the same stride) ----
    uint32_t koff[DEC_TDMA];
#pragma unroll
    for (int s = 0; s < DEC_TDMA; s++) {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u, part = p - key * 17u;
        koff[s] = key * (uint32_t) a.k_nb1 + part * 16u;
    }
    // the wave's sub-tiles are wave, wave + 8, ...: resources start at the
    // sub-tile's first key and end at the split's end (keys past it arrive as
    // zeros); a sub-tile past the split issues nothing
    const int64_t key_first = k_lo + (int64_t) wave * DEC_TK;
    const char * k_next = kbase + key_first * (int64_t) a.k_nb1;
    const char * v_next = vbase + key_first * (int64_t) a.v_nb1;
    const char * m_next = mslice_al + key_first * 2;
    int64_t k_rem = (k_hi - key_first) * (int64_t) a.k_nb1, v_rem = (k_hi - key_first) * (int64_t) a.v_nb1;
    int64_t m_rem = (int64_t) a.m_slice + mb_off - key_first * 2;
    const int64_t k_step = (int64_t) VS_ROUND * a.k_nb1, v_step = (int64_t) VS_ROUND * a.v_nb1;
    constexpr int64_t m_step = VS_ROUND * 2;
    const uint32_t g_kbytes = GATHER ? (uint32_t) (a.g_rows * (int64_t) a.k_nb1) : 0u;
    const uint32_t g_vbytes = GATHER ? (uint32_t) (a.g_rows * (int64_t) a.v_nb1) : 0u;
    auto gather_off = [&](int ti, int s, uint32_t nb1) -> uint32_t {
        const uint32_t p = (uint32_t) (64 * s + lane), key = p / 17u, part = p - key * 17u;
        const int kk = ti * DEC_TK + (int) key;
        const uint32_t row = kk < span ? (uint32_t) gcell[kk] : 0xffffffffu;
        return row < (uint32_t) a.g_rows ? row * nb1 + part * 16u : 0x80000000u;
    };
    // sub-tile ti's K rows, mask granules and V rows into stage st (11 DMAs at most)
    // sub-tile ti's K rows and mask granules into stage st (6 DMAs at most),
    // then the resources of the wave's next sub-tile
    auto issue_km = [&](int ti, int st) __attribute__((always_inline)) {
        v4i rk;
        if constexpr (GATHER) rk = make_rsrc(kbase, g_kbytes);
        else                  rk = make_rsrc(k_next, rsrc_bytes(k_rem));
        rk = uniform_rsrc(rk);
        uint32_t ok[DEC_TDMA];
#pragma unroll
        for (int s = 0; s < DEC_TDMA; s++) {
            if constexpr (GATHER) ok[s] = gather_off(ti, s, (uint32_t) a.k_nb1);
            else                  ok[s] = koff[s];
        }
        const uint32_t lk = __builtin_amdgcn_readfirstlane(lds_addr(&kr[st][wave][0]));
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's reads of the stage are done
        static_assert(DEC_TDMA == 5, "five DMAs per sub-tile and tensor");
        dma16_buf_at<0>(rk, ok[0], lk);
        dma16_buf_at<1024>(rk, ok[1], lk);
        dma16_buf_at<2048>(rk, ok[2], lk);
        dma16_buf_at<3072>(rk, ok[3], lk);
        if (lane < 16) dma16_buf_at<4096>(rk, ok[4], lk);
        if constexpr (MASKED) {
            const v4i rm = uniform_rsrc(make_rsrc(m_next, (uint32_t) m_rem));
            if (lane < n_mr * DEC_MGR) dma16_buf(rm, m_goff, __builtin_amdgcn_readfirstlane(lds_addr(&mgr[st][wave][0])));
        }
        k_next += k_step; k_rem -= k_step;
        m_next += m_step; m_rem -= m_step;
    };
    // sub-tile ti's V rows into stage st (5 DMAs), then the next sub-tile's resource
    auto issue_v = [&](int ti, int st) __attribute__((always_inline)) {
        v4i rv;
        if constexpr (GATHER) rv = make_rsrc(vbase, g_vbytes);
        else                  rv = make_rsrc(v_next, rsrc_bytes(v_rem));
        rv = uniform_rsrc(rv);
        uint32_t ov[DEC_TDMA];
#pragma unroll
        for (int s = 0; s < DEC_TDMA; s++) {
            if constexpr (GATHER) ov[s] = gather_off(ti, s, (uint32_t) a.v_nb1);
            else                  ov[s] = koff[s];
        }
        const uint32_t lv = __builtin_amdgcn_readfirstlane(lds_addr(&vr[st][wave][0]));
        __builtin_amdgcn_s_waitcnt(0xC07F);
        dma16_buf_at<0>(rv, ov[0], lv);
        dma16_buf_at<1024>(rv, ov[1], lv);
        dma16_buf_at<2048>(rv, ov[2], lv);
        dma16_buf_at<3072>(rv, ov[3], lv);
        if (lane < 16) dma16_buf_at<4096>(rv, ov[4], lv);
        v_next += v_step; v_rem -= v_step;
    };

    // ---- prologue: the cell list (GATHER) and the query rows (V stage 1),
    //      the fused append; then round 0's K, mask and V rows and round 1's K
    //      and mask, which load while the rows are requantised into images
    //      (in the P exchange buffers) and from there into registers ----
    uint8_t * qst = &vr[1][0][0];
    if constexpr (GATHER) {
        const int32_t * cl = a.g_cells + (size_t) b * a.g_bstride + (size_t) kvh * a.g_hstride + k_lo;
        const v4i rc = make_rsrc(cl, (uint32_t) span * 4u);
        for (int m = wave; m * 256 < span; m += VS_WAVES)
            dma16_buf(rc, (uint32_t) (m * 1024 + 16 * lane), __builtin_amdgcn_readfirstlane(lds_addr(&gcell[m * 256])));
        if (threadIdx.x == 0) g_bad = 0;
    }
    {
        const v4i rq = make_rsrc(a.q + (size_t) b * a.q_nb3, a.q_slice);
#pragma unroll
        for (int j = 0; j < (IR + VS_WAVES - 1) / VS_WAVES; j++) {
            const int rl = wave + VS_WAVES * j;
            if (rl >= RW) break;
            const uint32_t r = (uint32_t) rl;
            const uint32_t t = div_gqa(a, r), h = (uint32_t) (kvh * a.gqa) + (r - t * (uint32_t) a.gqa);
            dma16_buf(rq, t * (uint32_t) a.q_nb1 + h * (uint32_t) a.q_nb2 + 16u * (uint32_t) lane,
                      __builtin_amdgcn_readfirstlane(lds_addr(qst + rl * VS_QROW)));
        }
    }
    if (a.app_n > 0) {
        // as in k_fa_vd: the blocks whose keys hold appended rows quantise
        // their KV head's part of them first, and read them back only after
        // their own stores are done
        const int64_t alo = std::max<int64_t>(a.app_row0, k_lo), ahi = std::min<int64_t>(a.app_row0 + a.app_n, k_hi);
        if (alo < ahi) {
            const int units = (int) (ahi - alo) * NBLK * 2;
            const int sub = threadIdx.x & 7;
            for (int u0 = 0; u0 < units; u0 += VS_WAVES * 8) {
                const int uu0 = u0 + (int) (threadIdx.x >> 3);
                const bool live = uu0 < units;
                const int uu = live ? uu0 : 0;
                const int tensor = uu & 1, jb = (uu >> 1) % NBLK;
                const int64_t row = alo + (uu >> 1) / NBLK;
                const float4 xv = *(const float4 *) ((tensor ? a.app_v : a.app_k) + (size_t) (row - a.app_row0) * a.app_nb1 +
                                                     (size_t) (kvh * D + QK * jb + 4 * sub) * 4);
                float x[4] = {xv.x, xv.y, xv.z, xv.w};
                uint16_t d16;
                float dqa;
                const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dqa);
                if (live) {
                    char * bp = (char *) (tensor ? vbase + (size_t) row * a.v_nb1 : kbase + (size_t) row * a.k_nb1) + jb * QBLOCK;
                    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
                    qp[0] = (uint16_t) (q4 & 0xffffu);
                    qp[1] = (uint16_t) (q4 >> 16);
                    if (sub == 0) *(uint16_t *) bp = d16;
                }
            }
        }
    }
    wait_vmcnt<0>();   // this wave's query rows (cells, appended rows) have landed
    __syncthreads();   // ... and every wave's
    if constexpr (GATHER) {
        if ((int) threadIdx.x < span && (uint32_t) gcell[threadIdx.x] >= (uint32_t) a.g_rows) g_bad = 1;
    }
    if (wave < n_sub) {
        issue_km(wave, 0);
        issue_v(wave, 0);
    }
    if (wave + VS_WAVES < n_sub) issue_km(wave + VS_WAVES, 1);

    // requantisation (ggml's quantiser): wave w takes q8_0 block w of every
    // row, two lanes per row; the images [block][16-byte slice][row] of the
    // full tile go to pxf, the packed tile's to pxp
    uint8_t * qimf = (uint8_t *) &pxf[0][0];
    uint8_t * qimp = (uint8_t *) &pxp[0][0];
    static_assert(!NF || NBLK * 4 * 16 * 16 <= (int) sizeof(pxf), "the full tile's image fits pxf");
    static_assert(!PK || NBLK * 4 * 8 * 16 <= (int) sizeof(pxp), "the packed tile's image fits pxp");
    const int qrow = lane >> 1, qh = lane & 1;
    {
        float qx[16];
        const float4 * src = (const float4 *) (qst + qrow * VS_QROW + (QK * wave + 16 * qh) * 4);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4 v = qrow < RW ? src[m] : make_float4(0.f, 0.f, 0.f, 0.f);
            qx[4 * m] = v.x; qx[4 * m + 1] = v.y; qx[4 * m + 2] = v.z; qx[4 * m + 3] = v.w;
        }
        // zero this wave's block of both images
        if constexpr (NF) *(uint4 *) (qimf + wave * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
        if constexpr (PK) if (lane < 32) *(uint4 *) (qimp + wave * 512 + lane * 16) = make_uint4(0, 0, 0, 0);
        wave_lds_sync();
        uint32_t w[4];
        uint16_t d16;
        float dqv = 0.f;
        if (a.x86) dev::q8_quantize_lanes<16>(qx, true, w, &d16, &dqv);
        else       dev::q8_quantize_lanes<16>(qx, false, w, &d16, &dqv);
        if (qrow < RW) {
            const int woff = (int) ((0x200E0C0A08061402ull >> (8 * wave)) & 0xff);   // win_off(wave)
            const bool full = qrow < 16 * NF;
            uint8_t * s0 = full ? qimf + wave * 1024 + (NF ? qrow : 0) * 16 : qimp + wave * 512 + (PK ? qrow - 16 * NF : 0) * 16;
            const int sstride = full ? 16 * 16 : 8 * 16;    // bytes between the slices of a row
#pragma unroll
            for (int m = 0; m < 8; m++) {   // 2-byte pieces never straddle a slice
                const int o = woff + 16 * qh + 2 * m;
                *(uint16_t *) (s0 + (o >> 4) * sstride + (o & 15)) = (uint16_t) (w[m >> 1] >> (16 * (m & 1)));
            }
        }
        if (qh == 0 && qrow < IR) dqs[qrow][wave] = qrow < RW ? dqv * (a.scale * LOG2E) : 0.f;
    }
    __syncthreads();   // the images and the d_q table are complete
    // the query operands in registers (read before the first round's barrier,
    // after which pxf and pxp carry P): the full tile's row ln, the packed
    // tile's row 16 + (ln & 7) in columns 0..7 (zeros in 8..15)
    v4i qf[NF ? NBLK : 1], qp[PK ? NBLK : 1];
    float dqf[NF ? NBLK : 1], dqp[PK ? NBLK : 1];
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
        if constexpr (NF) {
            qf[bb] = *(const v4i *) (qimf + bb * 1024 + lg * 256 + ln * 16);
            dqf[bb] = dqs[ln][bb];
        }
        if constexpr (PK) {
            const v4i v = *(const v4i *) (qimp + bb * 512 + lg * 128 + (ln & 7) * 16);
            qp[bb] = hs == 0 ? v : v4i{0, 0, 0, 0};
            dqp[bb] = dqs[16 * NF + (ln & 7)][bb];
        }
    }

    // ---- the rounds ----
    v4f Of[2] = {v4f{0, 0, 0, 0}, v4f{0, 0, 0, 0}}, Op[2] = {v4f{0, 0, 0, 0}, v4f{0, 0, 0, 0}};
    float mfr = -INFINITY, lfr = 0.f, mpr = -INFINITY, lpr = 0.f;
    const int64_t qpos_f = GATHER ? a.g_pos0 + b + (int64_t) div_gqa(a, (uint32_t) (NF ? ln : 0)) : 0;
    const int64_t qpos_p = GATHER ? a.g_pos0 + b + (int64_t) div_gqa(a, (uint32_t) (16 * NF + (ln & 7))) : 0;
    const int prow = 16 * NF + (ln & 7);                 // the packed tile's row of the lane
#pragma unroll 1
    for (int r = 0; r < n_rounds; r++) {
        const int st = r & 1;
        const int sub = VS_WAVES * r + wave;             // this wave's sub-tile
        const int kb0 = DEC_TK * sub;                    // its first key in the split
        const bool mine = sub < n_sub;
        const bool mine_nx = sub + VS_WAVES < n_sub;        // the wave's sub-tile of the next round
        const bool mine_nx2 = sub + 2 * VS_WAVES < n_sub;   // ... and of the one after
        // The wave issues K and mask rows two rounds ahead (after its scores
        // of a round, into the stage they leave) and V rows one round ahead
        // (after the round's first barrier, when every wave is done with the
        // stage): K0 M0 V0 K1 M1 | K2 M2 V1 | K3 M3 V2 | ... The sub-tile's K
        // rows and mask have landed once at most the next round's K, mask and
        // this round's V rows are in flight.
        if (mine_nx) wait_vmcnt<NKD + NVD>();
        else         wait_vmcnt<NVD>();

        // the sub-tile's K block scales, [block][key]
        {
            const int bq = lane & 7, kq = lane >> 3;
            const uint16_t s0 = *(const uint16_t *) (&kr[st][wave][0] + kq * SEG + bq * QBLOCK);
            const uint16_t s1 = *(const uint16_t *) (&kr[st][wave][0] + (kq + 8) * SEG + bq * QBLOCK);
            ktab[wave][bq][kq] = s0;
            ktab[wave][bq][kq + 8] = s1;
        }
        wave_lds_sync();

        // ---- S = K Q^T for the sub-tile: MFMA rows are keys, columns rows;
        //      block bb + 1's MFMAs are issued while bb is scaled ----
        float sf[4] = {0.f, 0.f, 0.f, 0.f}, sp[4] = {0.f, 0.f, 0.f, 0.f};
        {
            // every block's K window and scales first: one LDS latency a round
            const uint8_t * kr0 = &kr[st][wave][0] + ln * SEG + 16 * lg;
            const uint8_t * tk = (const uint8_t *) &ktab[wave][0][0] + 8 * lg;   // + 32 bb
            v4i kw[NBLK];
            uint2 dkw[NBLK];
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) kw[bb] = *(const v4i *) (kr0 + 16 * win_piece(bb));
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) dkw[bb] = *(const uint2 *) (tk + 32 * bb);
            v4i cf[2], cp[2];
            auto qk_mfma = [&](int bb) __attribute__((always_inline)) {
                if constexpr (NF) cf[bb & 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kw[bb], qf[bb], v4i{0, 0, 0, 0}, 0, 0, 0);
                if constexpr (PK) cp[bb & 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kw[bb], qp[bb], v4i{0, 0, 0, 0}, 0, 0, 0);
            };
            qk_mfma(0);
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) {
                if (bb + 1 < NBLK) qk_mfma(bb + 1);
                const uint2 dk = dkw[bb];
                if constexpr (NF) {
                    const float d = dqf[bb];
                    const v4i c = cf[bb & 1];
                    sf[0] = __builtin_fmaf((float) c[0], mul_f16lo(d, dk.x), sf[0]);
                    sf[1] = __builtin_fmaf((float) c[1], mul_f16hi(d, dk.x), sf[1]);
                    sf[2] = __builtin_fmaf((float) c[2], mul_f16lo(d, dk.y), sf[2]);
                    sf[3] = __builtin_fmaf((float) c[3], mul_f16hi(d, dk.y), sf[3]);
                }
                if constexpr (PK) {
                    const float d = dqp[bb];
                    const v4i c = cp[bb & 1];
                    sp[0] = __builtin_fmaf((float) c[0], mul_f16lo(d, dk.x), sp[0]);
                    sp[1] = __builtin_fmaf((float) c[1], mul_f16hi(d, dk.x), sp[1]);
                    sp[2] = __builtin_fmaf((float) c[2], mul_f16lo(d, dk.y), sp[2]);
                    sp[3] = __builtin_fmaf((float) c[3], mul_f16hi(d, dk.y), sp[3]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" : "+v"(sf[i]), "+v"(sp[i]));

        // ---- mask; the sub-tile's maxima per row out to LDS ----
        float xf[4], xp[4];
        const uint8_t * mg = &mgr[MASKED ? st : 0][MASKED ? wave : 0][0];
        if constexpr (NF) {
#pragma unroll
            for (int i = 0; i < 4; i++) xf[i] = sf[i];
            if constexpr (MASKED) {
#pragma unroll
                for (int i = 0; i < 4; i++) xf[i] = fma_f16lo((uint32_t) *(const uint16_t *) (mg + m_lf + 2 * i), LOG2E, xf[i]);
            } else if constexpr (GATHER) {
                const int kin = kb0 + 4 * lg;
                const int4 c = *(const int4 *) &gcell[kin < DEC_GATHER_SPLIT - 3 ? kin : 0];
                const int cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    xf[i] = (uint32_t) cv[i] < (uint32_t) a.g_rows && (int64_t) cv[i] <= qpos_f ? xf[i] : -INFINITY;
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (!mine || kb0 + 4 * lg + i >= span) xf[i] = -INFINITY;
            float m = vmax(vmax(xf[0], xf[1]), vmax(xf[2], xf[3]));
            m = xmax_lanes16_32(m);
            if (lg == 0) mx[ln][wave] = m;
        }
        if constexpr (PK) {
#pragma unroll
            for (int i = 0; i < 4; i++) xp[i] = sp[i];
            if constexpr (MASKED) {
#pragma unroll
                for (int i = 0; i < 4; i++) xp[i] = fma_f16lo((uint32_t) *(const uint16_t *) (mg + m_lp + 2 * i), LOG2E, xp[i]);
            } else if constexpr (GATHER) {
                const int kin = kb0 + 4 * lg;
                const int4 c = *(const int4 *) &gcell[kin < DEC_GATHER_SPLIT - 3 ? kin : 0];
                const int cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    xp[i] = (uint32_t) cv[i] < (uint32_t) a.g_rows && (int64_t) cv[i] <= qpos_p ? xp[i] : -INFINITY;
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (hs || !mine || kb0 + 4 * lg + i >= span) xp[i] = -INFINITY;   // columns 8..15 hold no row
            float m = vmax(vmax(xp[0], xp[1]), vmax(xp[2], xp[3]));
            m = xmax_lanes16_32(m);
            if (lg == 0 && hs == 0) mx[prow][wave] = m;
        }
        if (mine_nx2) issue_km(sub + 2 * VS_WAVES, st);   // the stage's K rows and mask are used
        __syncthreads();   // B1: the maxima are out; every wave is done with the previous round
        if (mine_nx) issue_v(sub + VS_WAVES, st ^ 1);

        // ---- the block's max per row (the same in every wave), P, the
        //      running sums; P out to LDS ----
        if constexpr (NF) {
            const float4 m0 = *(const float4 *) &mx[ln][0], m1 = *(const float4 *) &mx[ln][4];
            const float mloc = vmax(vmax(vmax(m0.x, m0.y), vmax(m0.z, m0.w)), vmax(vmax(m1.x, m1.y), vmax(m1.z, m1.w)));
            const bool grow = mloc > mfr + RESCALE_SLACK;
            const bool rescale = grow && mfr != -INFINITY;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(mfr - mloc);
                mfr = mloc;
            }
            const float m_use = mfr == -INFINITY ? 0.f : mfr;
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(xf[i] - m_use);
            lfr = lfr * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
            if (__any(rescale)) { Of[0] *= alpha; Of[1] *= alpha; }
            pxf[wave][lane] = make_float4(p[0], p[1], p[2], p[3]);
        }
        if constexpr (PK) {
            const float4 m0 = *(const float4 *) &mx[prow][0], m1 = *(const float4 *) &mx[prow][4];
            const float mloc = vmax(vmax(vmax(m0.x, m0.y), vmax(m0.z, m0.w)), vmax(vmax(m1.x, m1.y), vmax(m1.z, m1.w)));
            const bool grow = mloc > mpr + RESCALE_SLACK;
            const bool rescale = grow && mpr != -INFINITY;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(mpr - mloc);
                mpr = mloc;
            }
            const float m_use = mpr == -INFINITY ? 0.f : mpr;
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(xp[i] - m_use);
            lpr = lpr * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
            if (__any(rescale)) { Op[0] *= alpha; Op[1] *= alpha; }
            if (hs == 0) pxp[wave][8 * lg + ln] = make_float4(p[0], p[1], p[2], p[3]);
        }
        // this round's V rows have landed: after them come K and mask two
        // rounds ahead and V one round ahead
        if (mine_nx2)     wait_vmcnt<NKD + NVD>();
        else if (mine_nx) wait_vmcnt<NVD>();
        else              wait_vmcnt<0>();
        // the sub-tile's V block scales, [block][key]: zeros for a sub-tile
        // past the split (its ring stage holds an older round's rows); keys
        // past the split's end arrived as zero rows
        {
            const int bq = lane & 7, kq = lane >> 3;
            const uint16_t s0 = *(const uint16_t *) (&vr[st][wave][0] + kq * SEG + bq * QBLOCK);
            const uint16_t s1 = *(const uint16_t *) (&vr[st][wave][0] + (kq + 8) * SEG + bq * QBLOCK);
            vtab[wave][bq][kq] = mine ? s0 : (uint16_t) 0;
            vtab[wave][bq][kq + 8] = mine ? s1 : (uint16_t) 0;
        }
        __syncthreads();   // B2: every wave's P, V rows and V scales of the round

        // ---- O += V^T (P d_v) over the round's keys, two sub-tiles a step;
        //      a step's LDS operands are read one step ahead ----
        {
            const uint8_t * tv = (const uint8_t *) &vtab[0][wave][0] + 8 * lg;   // keys 4lg.. of sub-tile u: + 256 u
            const uint8_t * vb = &vr[st][0][0] + (4 * lg) * SEG + 2 + 2 * ln + wave * QBLOCK;   // + DEC_KB u
            struct pv_ops {
                uint32_t w0[4], w1[4];   // V dims 2ln, 2ln+1 of keys 4lg.. of the two sub-tiles
                uint2 d0, d1;            // their d_v
                float4 f0, f1;           // the full tile's P
                float4 pq;               // the packed tile's P (the column's sub-tile)
            };
            auto pv_load = [&](int j, pv_ops & x) __attribute__((always_inline)) {
                const int u0 = 2 * j, u1 = 2 * j + 1;
#pragma unroll
                for (int jv = 0; jv < 4; jv++) {
                    x.w0[jv] = *(const uint16_t *) (vb + u0 * DEC_KB + jv * SEG);
                    x.w1[jv] = *(const uint16_t *) (vb + u1 * DEC_KB + jv * SEG);
                }
                x.d0 = *(const uint2 *) (tv + 256 * u0);
                x.d1 = *(const uint2 *) (tv + 256 * u1);
                if constexpr (NF) {
                    x.f0 = pxf[u0][lane];
                    x.f1 = pxf[u1][lane];
                }
                if constexpr (PK) x.pq = pxp[hs ? u1 : u0][8 * lg + (ln & 7)];
            };
            pv_ops cur, nxt;
            pv_load(0, cur);
#pragma unroll
            for (int j = 0; j < VS_WAVES / 2; j++) {
                if (j + 1 < VS_WAVES / 2) pv_load(j + 1, nxt);
                uint32_t a00[2], a10[2], a01[2], a11[2];
                cvt_v_block(cur.w0, a00, a10);
                cvt_v_block(cur.w1, a01, a11);
                const v8h A0 = __builtin_bit_cast(v8h, make_uint4(a00[0], a00[1], a01[0], a01[1]));
                const v8h A1 = __builtin_bit_cast(v8h, make_uint4(a10[0], a10[1], a11[0], a11[1]));
                const uint32_t dv0[2] = {cur.d0.x, cur.d0.y}, dv1[2] = {cur.d1.x, cur.d1.y};
                if constexpr (NF) {
                    const float p0[4] = {cur.f0.x, cur.f0.y, cur.f0.z, cur.f0.w}, p1[4] = {cur.f1.x, cur.f1.y, cur.f1.z, cur.f1.w};
                    const uint32_t p016[2] = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p0[0], p0[1])),
                                              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p0[2], p0[3]))};
                    const uint32_t p116[2] = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p1[0], p1[1])),
                                              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p1[2], p1[3]))};
                    uint32_t bh0[2], bl0[2], bh1[2], bl1[2];
                    pdv_hilo(p0, p016, dv0, bh0, bl0);
                    pdv_hilo(p1, p116, dv1, bh1, bl1);
                    const v8h Bh = __builtin_bit_cast(v8h, make_uint4(bh0[0], bh0[1], bh1[0], bh1[1]));
                    const v8h Bl = __builtin_bit_cast(v8h, make_uint4(bl0[0], bl0[1], bl1[0], bl1[1]));
                    Of[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bh, Of[0], 0, 0, 0);
                    Of[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bh, Of[1], 0, 0, 0);
                    Of[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bl, Of[0], 0, 0, 0);
                    Of[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bl, Of[1], 0, 0, 0);
                }
                if constexpr (PK) {
                    // column c < 8: row 16 + c over sub-tile u0's keys; c >= 8: over u1's
                    const float pz[4] = {0.f, 0.f, 0.f, 0.f};
                    const float pq[4] = {cur.pq.x, cur.pq.y, cur.pq.z, cur.pq.w};
                    const uint32_t pq16[2] = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pq[0], pq[1])),
                                              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pq[2], pq[3]))};
                    const uint32_t z16[2] = {0u, 0u};
                    uint32_t bh0[2], bl0[2], bh1[2], bl1[2];
                    pdv_hilo(hs ? pz : pq, hs ? z16 : pq16, dv0, bh0, bl0);
                    pdv_hilo(hs ? pq : pz, hs ? pq16 : z16, dv1, bh1, bl1);
                    const v8h Bh = __builtin_bit_cast(v8h, make_uint4(bh0[0], bh0[1], bh1[0], bh1[1]));
                    const v8h Bl = __builtin_bit_cast(v8h, make_uint4(bl0[0], bl0[1], bl1[0], bl1[1]));
                    Op[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bh, Op[0], 0, 0, 0);
                    Op[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bh, Op[1], 0, 0, 0);
                    Op[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bl, Op[0], 0, 0, 0);
                    Op[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bl, Op[1], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                cur = nxt;
            }
        }
    }

    // ---- epilogue: the row sums over the waves; the packed columns c and
    //      c + 8 of a row added; O of the wave's V block written ----
    __syncthreads();   // every wave is done with the round maxima
    if constexpr (NF) {
        const float l = sum_lanes16_32(lfr);
        if (lg == 0) mx[ln][wave] = l;
    }
    if constexpr (PK) {
        float l = sum_lanes16_32(lpr);
        if (lg == 0 && hs == 0) mx[prow][wave] = l;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            Op[0][v] += swap_halves8(Op[0][v]);
            Op[1][v] += swap_halves8(Op[1][v]);
        }
    }
    __syncthreads();
    if constexpr (GATHER) {
        if (threadIdx.x == 0 && g_bad && a.status) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
    }
    const size_t bh = (size_t) b * a.nh_kv + kvh;
    auto store_row = [&](int row, float M, const v4f & o0, const v4f & o1) __attribute__((always_inline)) {
        const float4 l0 = *(const float4 *) &mx[row][0], l1 = *(const float4 *) &mx[row][4];
        const float L = ((l0.x + l0.y) + (l0.z + l0.w)) + ((l1.x + l1.y) + (l1.z + l1.w));
        const int dim0 = QK * wave + 8 * lg;
        float4 w0 = make_float4(o0[0], o1[0], o0[1], o1[1]), w1 = make_float4(o0[2], o1[2], o0[3], o1[3]);
        if (a.ns > 1) {
            float * out = a.part_o + ((bh * a.ns + split) * a.R + row) * D + dim0;
            if (a.mctr) {
                const __amdgpu_buffer_rsrc_t prs = dev_rsrc(a.part_o);
                const uint32_t poff = (uint32_t) ((const char *) out - (const char *) a.part_o);
                store_dev4(prs, poff, w0);
                store_dev4(prs, poff + 16, w1);
                if (wave == 0 && lg == 0)
                    store_dev2(dev_rsrc(a.part_ml),
                               (uint32_t) (((bh * a.ns + split) * a.R + row) * sizeof(float2)), make_float2(M, L));
            } else {
                store_nt4(out, w0);
                store_nt4(out + 4, w1);
                if (wave == 0 && lg == 0) {
                    float2 * mlp = &a.part_ml[(bh * a.ns + split) * a.R + row];
                    __builtin_nontemporal_store(M, &mlp->x);
                    __builtin_nontemporal_store(L, &mlp->y);
                }
            }
        } else {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            w0.x *= inv; w0.y *= inv; w0.z *= inv; w0.w *= inv;
            w1.x *= inv; w1.y *= inv; w1.z *= inv; w1.w *= inv;
            const int tq = (int) div_gqa(a, (uint32_t) row), h = kvh * a.gqa + (row - tq * a.gqa);
            float * out = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + dim0;
            if (a.dst_vec) {
                *(float4 *) out = apply_gate(a, out, w0);
                *(float4 *) (out + 4) = apply_gate(a, out + 4, w1);
            } else {
                out[0] = w0.x; out[1] = w0.y; out[2] = w0.z; out[3] = w0.w;
                out[4] = w1.x; out[5] = w1.y; out[6] = w1.z; out[7] = w1.w;
            }
        }
    };
    if constexpr (NF) {
        if (ln < RW) store_row(ln, mfr, Of[0], Of[1]);
    }
    if constexpr (PK) {
        if (hs == 0 && prow < RW) store_row(prow, mpr, Op[0], Op[1]);
    }
    if (a.mctr) fa_merge_tail<VS_WAVES * 64>(a, b, kvh, (float *) &kr[0][0][0]);
}

// ================================================================ prefill
//
// k_fa_pre: long query blocks (more than 32 query rows per KV head: prefill
// chunks, long verify blocks) with a mask shared by the heads or none, GQA >= 4.
// One block of 8 waves per CU holds 128 query rows of one KV head (16 rows a
// wave: 16 tokens x 8 heads at GQA 8). Keys stream in chunks of 64 through LDS
// DMA into a two-stage ring that the 8 waves share, so a block reads each K/V
// row once for its 128 rows; the row groups of one (KV head, key split) are
// placed on one XCD, whose L2 then serves the same rows to all of them. Per
// chunk the block converts V to f16 once, transposed to [dim][key] (the PV A
// operand of a lane is one 16-byte LDS read), repacks the K quants to
// [block][key][32 + 8 padding] (the QK A operand of a lane is one aligned 8-byte read),
// and tabulates the K and V block scales; then each wave takes its 16 rows
// over the 64 keys: exact i8 block dots (v_mfma_i32_16x16x32_i8, one q8_0
// block each) scaled by d_q*d_k, one online-softmax step, and hi + lo f16
// P*d_v on v_mfma_f32_16x16x32_f16 (32 keys a step). The LDS reads of the
// next key tile (QK) and V block (PV) are issued ahead of the current one's
// arithmetic. A wave whose rows see none of the
// chunk's keys (a causal mask's upper triangle) skips it.

constexpr int PRE_WAVES = 8;
constexpr int PRE_ROWS  = 16 * PRE_WAVES;                 // 128 query rows per block
constexpr int PRE_CK    = 64;                             // keys per chunk
constexpr int PRE_KB    = PRE_CK * SEG;                   // 17408: one tensor's rows of a chunk
constexpr int PRE_TDMA  = PRE_KB / 1024;                  // 17 wave DMAs per tensor
constexpr int PRE_MGR   = 2 * PRE_CK / 16 + 1;            // 9 granules per mask row of a chunk
constexpr int PRE_MROWS = PRE_ROWS / 4 + 1;               // 33 mask rows of a block at most (GQA >= 4)
constexpr int PRE_MDMA  = (PRE_MROWS * PRE_MGR + 63) / 64;   // 5 wave DMAs for them
constexpr int PRE_MOFF  = 2 * PRE_KB;                     // mask granules follow the K and V rows
constexpr int PRE_STAGE = PRE_MOFF + PRE_MDMA * 1024;     // 39936 bytes
constexpr int PRE_SLOTS = 2 * PRE_TDMA + PRE_MDMA;        // 39 DMA slots per chunk
constexpr int PRE_SPW   = (PRE_SLOTS + PRE_WAVES - 1) / PRE_WAVES;   // 5 per wave
// LDS rows are padded so that the wave-wide operand reads meet no bank
// conflict on gfx950 (measured): 16-byte reads of 16 rows need a row stride of
// 16 bytes times 2 mod 4, 8-byte reads of 16 rows one of 8 bytes times an odd
// number (the unpadded 128- and 32-byte strides ran 1.8x and 3.8x slower)
constexpr int PRE_VTS   = 2 * PRE_CK + 32;                // 160: bytes per dim row of V^T
constexpr int PRE_VT    = D * PRE_VTS;                    // 40960
constexpr int PRE_KQS   = QK + 8;                         // 40: bytes per key row of the repacked K quants
constexpr int PRE_KQ    = NBLK * PRE_CK * PRE_KQS;        // 20480: a chunk's K quants [block][key][32 + 8]
constexpr int PRE_SKV   = 2 * NBLK * PRE_CK * 2;          // 2048: K and V scales [K|V][block][key] fp16
constexpr int PRE_QIMG  = NBLK * 16 * QK;                 // 4096: a wave's query quants [block][row][32]
constexpr int PRE_QW    = PRE_QIMG + 16 * NBLK * 4;       // + d_q [row][block]
// LDS: V^T | K quants | scales | stage 0 | stage 1. The regions the key loop
// reads most end below 64 KB, so that their offsets fit the 16-bit offset of
// an LDS instruction and one base register serves many accesses.
constexpr int PRE_LDS   = PRE_VT + PRE_KQ + PRE_SKV + 2 * PRE_STAGE;   // 143360
static_assert(PRE_VT + PRE_KQ + PRE_SKV <= 65536, "V^T, K quants and scales sit below 64 KB");
static_assert(PRE_KB % 1024 == 0, "a tensor's rows of a chunk are whole wave DMAs");
static_assert(PRE_WAVES * PRE_QW <= PRE_VT + PRE_KQ, "the query images fit V^T and the K quants");
static_assert(PRE_CK == 64 && NBLK == PRE_WAVES, "the conversion pass: wave w takes V block w of every key");

// V^T rows hold a chunk's keys in this order: key k = 32h + 16tt + 4g + i
// (half h, key tile tt of the half, lane group g, i = 0..3) sits at position
// 32h + 8g + 4tt + i, so the 8 keys a lane group's PV operand needs are
// consecutive.

// f16 pair (lo: byte B of s0, hi: byte B of s1) from two int8 values, exact.
template <int B>
__device__ __forceinline__ uint32_t cvt_i8_pair(uint32_t s0, uint32_t s1) {
    uint32_t d;
    if constexpr (B == 0)
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
            "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0"
            : "=&v"(d) : "v"(s0), "v"(s1));
    else if constexpr (B == 1)
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
            "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1"
            : "=&v"(d) : "v"(s0), "v"(s1));
    else if constexpr (B == 2)
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
            "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_2"
            : "=&v"(d) : "v"(s0), "v"(s1));
    else
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
            "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
            : "=&v"(d) : "v"(s0), "v"(s1));
    return d;
}

template <bool MASKED>
__global__ __launch_bounds__(PRE_WAVES * 64, 2) void k_fa_pre(fa_args a) {
    asm volatile("" :: "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.mask), "s"(a.part_o));
    // V^T | K quants | scales | stage 0 | stage 1; the query images of the
    // prologue use V^T and the K quants
    __shared__ __attribute__((aligned(16))) uint8_t lds[PRE_LDS];
    uint8_t * const vt = lds;
    uint8_t * const kq = vt + PRE_VT;
    uint16_t (* const skv)[NBLK][PRE_CK] = (uint16_t (*)[NBLK][PRE_CK]) (kq + PRE_KQ);   // [K|V][block][key] fp16 scales
    uint8_t * const stg = kq + PRE_KQ + PRE_SKV;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;

    // ---- block -> (b, kvh, split, row group), blocks x, x + 8, ... on XCD x.
    //      pre_rgmap 0: unit (b, kvh, split) = x + 8 u, its n_rg row groups
    //      consecutive; 1: row group unit (rg, b, kvh) = x + 8 u (bh fastest, so
    //      an XCD holds one KV head when B * nh_kv divides 8), its ns splits
    //      consecutive ----
    const int id = blockIdx.x;
    const int xcd = id & 7, j = id >> 3;
    const int nbh = a.B * a.nh_kv;
    int bh, split, rg;
    if (a.pre_rgmap) {
        const int ul = (int) udiv((uint32_t) j, (uint32_t) a.ns, a.ns_mul);
        split = j - ul * a.ns;
        const int rgu = xcd + 8 * ul;
        if (rgu >= nbh * a.n_rg) return;
        rg = (int) udiv((uint32_t) rgu, (uint32_t) nbh, a.nbh_mul);
        bh = rgu - rg * nbh;
    } else {
        const int ul = (int) udiv((uint32_t) j, (uint32_t) a.n_rg, a.nrg_mul);
        rg = j - ul * a.n_rg;
        const int unit = xcd + 8 * ul;
        if (unit >= nbh * a.ns) return;
        bh = (int) udiv((uint32_t) unit, (uint32_t) a.ns, a.ns_mul);
        split = unit - bh * a.ns;
    }
    const int b = bh / a.nh_kv, kvh = bh - b * a.nh_kv;
    const int64_t k_lo = (int64_t) split * a.split_len;
    const int64_t k_e = k_lo + a.split_len;
    const int64_t k_hi = split == a.ns - 1 ? a.n_kv : (a.n_kv < k_e ? a.n_kv : k_e);
    const int span = (int) (k_hi - k_lo);
    const int n_chunks = (span + PRE_CK - 1) / PRE_CK;
    const int r0 = rg * PRE_ROWS;
    const int RW = a.R - r0 < PRE_ROWS ? a.R - r0 : PRE_ROWS;   // rows of this block
    const int wr0 = 16 * wave;                                  // the wave's first row in the block
    const int t0 = (int) div_gqa(a, (uint32_t) r0);

    const char * kbase = a.k + (size_t) bmod(b, a.kb) * a.k_nb3 + (size_t) kvh * a.k_nb2;
    const char * vbase = a.v + (size_t) bmod(b, a.vb) * a.v_nb3 + (size_t) kvh * a.v_nb2;
    // mask rows: query positions t0 .. t0 + n_mrows - 1 (one row per position)
    const char * mslice = MASKED ? a.mask + (size_t) bmod(b, a.m_ne3) * a.m_nb3 : nullptr;
    const char * mslice_al = (const char *) ((uintptr_t) mslice & ~(uintptr_t) 15);
    auto mrow_off = [&](int mr) -> uint32_t {
        return (uint32_t) (mslice - mslice_al) + (uint32_t) ((size_t) (t0 + mr) * a.m_nb1);
    };
    const int n_mrows = MASKED ? (int) div_gqa(a, (uint32_t) (r0 + RW - 1)) - t0 + 1 : 0;
    const int n_mdma = (n_mrows * PRE_MGR + 63) / 64;

    // ---- DMA slots of a chunk: slot s lands at byte 1024 s of the stage. Slots
    //      [0, 17) are the K rows (piece p = 64 s + lane is byte 16 (p % 17) of
    //      key p / 17), [17, 34) the V rows, then the mask granules (granule
    //      G = 64 m + lane is granule G % 9 of row G / 9; lanes past the rows
    //      re-read the last one). Wave w issues slots w, w + 8, ... ----
    uint32_t doff[PRE_SPW];
    bool dlive[PRE_SPW];
#pragma unroll
    for (int s = 0; s < PRE_SPW; s++) {
        const int slot = wave + PRE_WAVES * s;
        uint32_t off = 0;
        bool live = false;
        if (slot < 2 * PRE_TDMA) {
            const int tensor = slot >= PRE_TDMA;
            const uint32_t p = (uint32_t) ((slot - tensor * PRE_TDMA) * 64 + lane), key = p / 17u, part = p - key * 17u;
            off = key * (uint32_t) (tensor ? a.v_nb1 : a.k_nb1) + part * 16u;
            live = true;
        } else if (MASKED && slot < PRE_SLOTS && slot - 2 * PRE_TDMA < n_mdma) {
            const int g = (slot - 2 * PRE_TDMA) * 64 + lane;
            const int gc = g < n_mrows * PRE_MGR ? g : n_mrows * PRE_MGR - 1;
            off = (mrow_off(gc / PRE_MGR) & ~15u) + 16u * (uint32_t) (gc % PRE_MGR);
            live = true;
        }
        doff[s] = off;
        dlive[s] = live;
    }
    const int64_t k_bytes = k_hi * (int64_t) a.k_nb1, v_bytes = k_hi * (int64_t) a.v_nb1;
    // chunk c through resources based at its first key and ending at the
    // split's end: keys past the split arrive as zeros (and are masked)
    auto issue_chunk = [&](int c, uint8_t * st) __attribute__((always_inline)) {
        const int64_t c0 = k_lo + (int64_t) c * PRE_CK;
        const int64_t kc = c0 * (int64_t) a.k_nb1, vc = c0 * (int64_t) a.v_nb1;
        const v4i rk = make_rsrc(kbase + kc, (uint32_t) std::min<int64_t>(k_bytes - kc, 0xffffffffll));
        const v4i rv = make_rsrc(vbase + vc, (uint32_t) std::min<int64_t>(v_bytes - vc, 0xffffffffll));
        v4i rm = rk;
        if constexpr (MASKED)
            rm = make_rsrc(mslice_al + c0 * 2, (uint32_t) (a.m_slice + (uint32_t) (mslice - mslice_al) - c0 * 2));
#pragma unroll
        for (int s = 0; s < PRE_SPW; s++) {
            const int slot = wave + PRE_WAVES * s;
            if (!dlive[s]) continue;
            dma16_buf(slot < PRE_TDMA ? rk : slot < 2 * PRE_TDMA ? rv : rm, doff[s],
                      __builtin_amdgcn_readfirstlane(lds_addr(st + slot * 1024)));
        }
    };
    // fused append (as in k_fa_dec): the blocks whose keys hold appended rows
    // quantise their KV head's part of them first, and their chunk DMAs read
    // the rows only after these stores are done
    if (a.app_n > 0) {
        const int64_t alo = std::max<int64_t>(a.app_row0, k_lo), ahi = std::min<int64_t>(a.app_row0 + a.app_n, k_hi);
        if (alo < ahi) {
            const int units = (int) (ahi - alo) * NBLK * 2;
            const int sub = threadIdx.x & 7;
            for (int u0 = 0; u0 < units; u0 += PRE_WAVES * 8) {
                const int uu0 = u0 + (int) (threadIdx.x >> 3);
                const bool live = uu0 < units;
                const int uu = live ? uu0 : 0;
                const int tensor = uu & 1, jb = (uu >> 1) % NBLK;
                const int64_t row = alo + (uu >> 1) / NBLK;
                const float4 xv = *(const float4 *) ((tensor ? a.app_v : a.app_k) + (size_t) (row - a.app_row0) * a.app_nb1 +
                                                     (size_t) (kvh * D + QK * jb + 4 * sub) * 4);
                float x[4] = {xv.x, xv.y, xv.z, xv.w};
                uint16_t d16;
                float dqa;
                const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dqa);
                if (live) {
                    char * bp = (char *) (tensor ? vbase + (size_t) row * a.v_nb1 : kbase + (size_t) row * a.k_nb1) + jb * QBLOCK;
                    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
                    qp[0] = (uint16_t) (q4 & 0xffffu);
                    qp[1] = (uint16_t) (q4 >> 16);
                    if (sub == 0) *(uint16_t *) bp = d16;
                }
            }
            wait_vmcnt<0>();
            __syncthreads();
        }
    }
    if (n_chunks > 0) issue_chunk(0, stg);

    // ---- prologue: each wave requantises its own 16 query rows (ggml's
    //      quantiser; 4 lanes per (row, block)) into an image of its own, from
    //      which lane (ln, lg) takes quants 8 lg .. 8 lg + 7 of each block of row ln ----
    uint8_t * qimg = lds + wave * PRE_QW;                   // [block][row][32] int8
    float * dql = (float *) (qimg + PRE_QIMG);                  // [16 rows][NBLK]
    long qw[NBLK];
    float dq[NBLK];
    {
        const int qrow = lane >> 2, ql = lane & 3;              // (row, quarter of a block)
        const int r = r0 + wr0 + qrow;
        const bool live = wr0 + qrow < RW;
        const char * qp = a.q;
        if (live) {
            const uint32_t t = div_gqa(a, (uint32_t) r), h = (uint32_t) (kvh * a.gqa) + ((uint32_t) r - t * (uint32_t) a.gqa);
            qp = a.q + (size_t) b * a.q_nb3 + (size_t) t * a.q_nb1 + (size_t) h * a.q_nb2 + (size_t) (8 * ql) * 4;
        }
        float4 xv[NBLK][2];
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            xv[bb][0] = live ? *(const float4 *) (qp + QK * bb * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[bb][1] = live ? *(const float4 *) (qp + QK * bb * 4 + 16) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const float fs = a.scale * LOG2E;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            float x[8] = {xv[bb][0].x, xv[bb][0].y, xv[bb][0].z, xv[bb][0].w,
                          xv[bb][1].x, xv[bb][1].y, xv[bb][1].z, xv[bb][1].w};
            uint32_t w[2];
            uint16_t d16;
            float dqv;
            if (a.x86) dev::q8_quantize_lanes<8>(x, true, w, &d16, &dqv);
            else       dev::q8_quantize_lanes<8>(x, false, w, &d16, &dqv);
            // padding rows quantise zeros: all-zero quants and d_q = 0
            *(uint2 *) (qimg + (bb * 16 + qrow) * QK + 8 * ql) = make_uint2(w[0], w[1]);
            if (ql == 0) dql[qrow * NBLK + bb] = live ? dqv * fs : 0.f;
        }
        wave_lds_sync();
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) {
            qw[bb] = *(const long *) (qimg + (bb * 16 + ln) * QK + 8 * lg);
            dq[bb] = dql[ln * NBLK + bb];
        }
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++) asm volatile("" : "+v"(qw[bb]), "+v"(dq[bb]));
    }

    // the lane's mask row in a stage: its query position's granules, plus the
    // row's offset within its first granule
    const int rl_lane = wr0 + ln < RW ? wr0 + ln : 0;
    const int mrow = MASKED ? (int) div_gqa(a, (uint32_t) (r0 + rl_lane)) - t0 : 0;
    const uint32_t m_lane = MASKED ? (uint32_t) (PRE_MOFF + mrow * PRE_MGR * 16) + (mrow_off(mrow) & 15u) + 8u * (uint32_t) lg : 0u;
    const bool wave_rows = wr0 < RW;   // the wave has rows of its own

    v4f O[NBLK][2];
    float m_run = -INFINITY, l_run = 0.f;
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) { O[bb][0] = v4f{0, 0, 0, 0}; O[bb][1] = v4f{0, 0, 0, 0}; }

    // ---- the key loop: chunk c in stage c % 2; chunk c + 1 loads while chunk c
    //      is converted and computed ----
    for (int c = 0; c < n_chunks; c++) {
        uint8_t * st = stg + (c & 1) * PRE_STAGE;
        wait_vmcnt<0>();
        __syncthreads();   // chunk c has landed; every wave is done with chunk c - 1 (and the prologue)
        if (c + 1 < n_chunks) issue_chunk(c + 1, stg + ((c + 1) & 1) * PRE_STAGE);
        // conversion pass: wave w takes V block w (dims 32w .. 32w+31) of the
        // 64 keys: lane (key pair kp, half dh) converts dims 32w + 16dh .. +15 of
        // the keys at V^T positions 2kp, 2kp + 1, and K block w of key `lane`
        // into the repacked quants; lane k also tabulates the K and V scales of
        // block w of key k. Block w's quants start 2 bytes into a word when w
        // is even and on a word boundary when w is odd (34w + 2 = 0 mod 4): the
        // lanes read whole words from the word at or before them and realign
        // them with alignbyte (shift 2 or 0), with no branch on the parity.
        // Rows sit 272 bytes (68 words, 4 banks mod 32) apart, so reads of one
        // offset in many rows would meet in 8 banks: each lane reads its run of
        // words starting at a rotated word (slot i holds word (i + rot) mod n,
        // the word past the run sits in slot n), so that one read's lanes cover
        // every bank. Every read is issued before the first conversion.
        {
            const int kp = lane & 31, dh = lane >> 5;
            const int p0 = 2 * kp;
            // the key at position p0 (its neighbour p0 + 1 is the next key)
            const int key0 = 32 * (p0 >> 5) + 16 * ((p0 >> 2) & 1) + 4 * ((p0 >> 3) & 3) + (p0 & 3);
            const int odd = wave & 1;
            const uint32_t sh = odd ? 0u : 2u;
            const uint8_t * v0 = st + PRE_KB + key0 * SEG + QBLOCK * wave + 16 * dh + 2 * odd;
            const uint8_t * k0 = st + lane * SEG + QBLOCK * wave + 2 * odd;
            const int vrot = (kp >> 3) & 3, krot = (lane >> 3) & 7;
            uint32_t x[5], y[5], kw[9];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = (i + vrot) & 3;
                x[i] = *(const uint32_t *) (v0 + 4 * t);
                y[i] = *(const uint32_t *) (v0 + SEG + 4 * t);
            }
            x[4] = *(const uint32_t *) (v0 + 16);
            y[4] = *(const uint32_t *) (v0 + SEG + 16);
#pragma unroll
            for (int i = 0; i < 8; i++) kw[i] = *(const uint32_t *) (k0 + 4 * ((i + krot) & 7));
            kw[8] = *(const uint32_t *) (k0 + 32);
            const uint16_t dk16 = *(const uint16_t *) (st + lane * SEG + QBLOCK * wave);
            const uint16_t dv16 = *(const uint16_t *) (st + PRE_KB + lane * SEG + QBLOCK * wave);
            // V: word t of the lane's 16 bytes holds dims 16dh + 4t .. + 3 of keys key0 / key0 + 1
            uint8_t * vrow = vt + (32 * wave + 16 * dh) * PRE_VTS + 2 * p0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = (i + vrot) & 3;
                const uint32_t xa = __builtin_amdgcn_alignbyte(t == 3 ? x[4] : x[(i + 1) & 3], x[i], sh);
                const uint32_t ya = __builtin_amdgcn_alignbyte(t == 3 ? y[4] : y[(i + 1) & 3], y[i], sh);
                uint8_t * d = vrow + 4 * t * PRE_VTS;
                *(uint32_t *) (d) = cvt_i8_pair<0>(xa, ya);
                *(uint32_t *) (d + PRE_VTS) = cvt_i8_pair<1>(xa, ya);
                *(uint32_t *) (d + 2 * PRE_VTS) = cvt_i8_pair<2>(xa, ya);
                *(uint32_t *) (d + 3 * PRE_VTS) = cvt_i8_pair<3>(xa, ya);
            }
            // K: word j of block w of key `lane` (quants 4j .. 4j + 3) to kq[w][lane]
            uint8_t * kd = kq + (wave * PRE_CK + lane) * PRE_KQS;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int t = (i + krot) & 7;
                *(uint32_t *) (kd + 4 * t) = __builtin_amdgcn_alignbyte(t == 7 ? kw[8] : kw[(i + 1) & 7], kw[i], sh);
            }
            skv[0][wave][lane] = dk16;
            skv[1][wave][lane] = dv16;
        }
        __syncthreads();   // V^T and the scale tables of chunk c are complete

        // ---- the wave's 16 rows over the chunk's keys: the lane's keys are
        //      16 kt + 4 lg + i (key tile kt, i = 0..3) ----
        // mask pairs: mv[kt][j] holds the f16 mask of keys 16 kt + 4 lg + 2j (low
        // half) and + 1 (high half); a pair of two -inf is 0xFC00FC00. Keys past
        // the split (the last chunk only) arrive as zeros and are not live.
        const int kin = c * PRE_CK + 4 * lg;
        const bool tail = (c + 1) * PRE_CK > span;
        uint32_t mv[4][2];
        bool live = !MASKED;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                mv[kt][j] = MASKED ? *(const uint32_t *) (st + m_lane + 32 * kt + 4 * j) : 0u;
                if (MASKED) live |= mv[kt][j] != 0xFC00FC00u;
            }
        if (tail) {
            live = false;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    live |= kin + 16 * kt + i < span && (!MASKED || ((mv[kt][i >> 1] >> (16 * (i & 1))) & 0xffffu) != 0xFC00u);
        }
        if (!wave_rows || !__any(live)) continue;

        // S = K Q^T per key tile (MFMA rows: keys; columns: the wave's rows);
        // tile kt + 1's quants and scales are read while tile kt is computed
        float s[4][4];
        {
            long kA[2][NBLK];
            uint2 dk[2][NBLK];
            auto load_tile = [&](int kt, long (&ka)[NBLK], uint2 (&dkk)[NBLK]) __attribute__((always_inline)) {
                const uint8_t * kr = kq + (16 * kt + ln) * PRE_KQS + 8 * lg;
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) {
                    ka[bb] = *(const long *) (kr + bb * PRE_CK * PRE_KQS);
                    dkk[bb] = *(const uint2 *) &skv[0][bb][16 * kt + 4 * lg];
                }
            };
            load_tile(0, kA[0], dk[0]);
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                const int cb = kt & 1;
                if (cb) __builtin_amdgcn_s_setprio(0); else __builtin_amdgcn_s_setprio(1);
                if (kt + 1 < 4) load_tile(kt + 1, kA[cb ^ 1], dk[cb ^ 1]);
                v4i cc[NBLK];
                cc[0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(kA[cb][0], qw[0], v4i{0, 0, 0, 0}, 0, 0, 0);
                cc[1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(kA[cb][1], qw[1], v4i{0, 0, 0, 0}, 0, 0, 0);
                float sa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) {
                    if (bb + 2 < NBLK)
                        cc[bb + 2] = __builtin_amdgcn_mfma_i32_16x16x32_i8(kA[cb][bb + 2], qw[bb + 2], v4i{0, 0, 0, 0}, 0, 0, 0);
                    const float d = dq[bb];
                    sa[0] = __builtin_fmaf((float) cc[bb][0], mul_f16lo(d, dk[cb][bb].x), sa[0]);
                    sa[1] = __builtin_fmaf((float) cc[bb][1], mul_f16hi(d, dk[cb][bb].x), sa[1]);
                    sa[2] = __builtin_fmaf((float) cc[bb][2], mul_f16lo(d, dk[cb][bb].y), sa[2]);
                    sa[3] = __builtin_fmaf((float) cc[bb][3], mul_f16hi(d, dk[cb][bb].y), sa[3]);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) s[kt][i] = sa[i];
            }
        }

        // ---- mask, online softmax (base 2) over the chunk's 64 keys ----
        float p[4][4];
        uint32_t p16[4][2];
        {
            float x[4][4];
            float mloc = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    x[kt][i] = !MASKED ? s[kt][i]
                             : (i & 1) ? fma_f16hi(mv[kt][i >> 1], LOG2E, s[kt][i]) : fma_f16lo(mv[kt][i >> 1], LOG2E, s[kt][i]);
            if (tail) {
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (kin + 16 * kt + i >= span) x[kt][i] = -INFINITY;
            }
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) mloc = vmax(mloc, x[kt][i]);
            mloc = xmax_lanes16_32(mloc);
            const bool grow = mloc > m_run + RESCALE_SLACK;
            float alpha = 1.f;
            if (grow) {
                alpha = __builtin_amdgcn_exp2f(m_run - mloc);
                m_run = mloc;
            }
            const float m_use = m_run == -INFINITY ? 0.f : m_run;
            float lsum = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    p[kt][i] = __builtin_amdgcn_exp2f(x[kt][i] - m_use);
                    lsum += p[kt][i];
                }
                p16[kt][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[kt][0], p[kt][1]));
                p16[kt][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[kt][2], p[kt][3]));
            }
            l_run = l_run * alpha + lsum;
            if (__any(grow)) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++) { O[bb][0] *= alpha; O[bb][1] *= alpha; }
            }
        }

        // ---- O += V^T (P d_v): per half of 32 keys (key tiles 2h, 2h + 1) and V
        //      block, A = V^T rows 32bb + 16e + ln at the lane group's 8
        //      positions, B = the same 8 keys' P d_v as f16 hi + lo. A step's
        //      lo MFMAs accumulate into what its hi MFMAs just wrote, and an
        //      MFMA whose accumulator was written a few MFMAs before stalls for
        //      the result: the next step's B operands are formed between the
        //      two pairs. Step n + 1's V^T and step n + 2's d_v are read while
        //      step n is computed ----
        {
            v8h A[2][2];
            uint2 dvv[3][2];
            v8h Bh[2], Bl[2];
            auto load_a = [&](int n, v8h (&aa)[2]) __attribute__((always_inline)) {
                const int h = n >> 3, bb = n & 7;
                const uint8_t * va = vt + (32 * bb + ln) * PRE_VTS + (32 * h + 8 * lg) * 2;
                aa[0] = *(const v8h *) va;
                aa[1] = *(const v8h *) (va + 16 * PRE_VTS);
            };
            auto load_dv = [&](int n, uint2 (&dd)[2]) __attribute__((always_inline)) {
                const int h = n >> 3, bb = n & 7;
                dd[0] = *(const uint2 *) &skv[1][bb][32 * h + 4 * lg];
                dd[1] = *(const uint2 *) &skv[1][bb][32 * h + 16 + 4 * lg];
            };
            auto form_b = [&](int n, const uint2 (&dd)[2], v8h & bh, v8h & bl) __attribute__((always_inline)) {
                const int h = n >> 3;
                uint32_t bh0[2], bl0[2], bh1[2], bl1[2];
                {
                    const uint32_t dv[2] = {dd[0].x, dd[0].y};
                    pdv_hilo(p[2 * h], p16[2 * h], dv, bh0, bl0);
                }
                {
                    const uint32_t dv[2] = {dd[1].x, dd[1].y};
                    pdv_hilo(p[2 * h + 1], p16[2 * h + 1], dv, bh1, bl1);
                }
                bh = __builtin_bit_cast(v8h, make_uint4(bh0[0], bh0[1], bh1[0], bh1[1]));
                bl = __builtin_bit_cast(v8h, make_uint4(bl0[0], bl0[1], bl1[0], bl1[1]));
            };
            load_a(0, A[0]);
            load_dv(0, dvv[0]);
            load_dv(1, dvv[1]);
            form_b(0, dvv[0], Bh[0], Bl[0]);
#pragma unroll
            for (int n = 0; n < 2 * NBLK; n++) {
                const int cb = n & 1, bb = n & 7;
                if (cb) __builtin_amdgcn_s_setprio(0); else __builtin_amdgcn_s_setprio(1);
                if (n + 1 < 2 * NBLK) load_a(n + 1, A[cb ^ 1]);
                if (n + 2 < 2 * NBLK) load_dv(n + 2, dvv[(n + 2) % 3]);
                // the next reads are issued before this step's arithmetic
                __builtin_amdgcn_sched_barrier(0);
                O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[cb][0], Bh[cb], O[bb][0], 0, 0, 0);
                O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[cb][1], Bh[cb], O[bb][1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (n + 1 < 2 * NBLK) form_b(n + 1, dvv[(n + 1) % 3], Bh[cb ^ 1], Bl[cb ^ 1]);
                __builtin_amdgcn_sched_barrier(0);
                O[bb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[cb][0], Bl[cb], O[bb][0], 0, 0, 0);
                O[bb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[cb][1], Bl[cb], O[bb][1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
    }

    // ---- epilogue: lane (ln, lg) holds dims 32bb + 16e + 4lg + i of row ln in
    //      O[bb][e][i] ----
    const float L = sum_lanes16_32(l_run);
    if (!wave_rows) return;
    int tid_e = (int) threadIdx.x;
    asm volatile("" : "+v"(tid_e));
    const int ln_e = tid_e & 15, lg_e = (tid_e >> 4) & 3;
    const int rl = wr0 + ln_e;
    if (rl >= RW) return;
    const int r = r0 + rl;
    const int tq = (int) div_gqa(a, (uint32_t) r), h = kvh * a.gqa + (r - tq * a.gqa);
    float * out;
    float oscale;
    const bool nsplit = a.ns > 1;
    if (!nsplit) {
        out = a.dst + (((size_t) b * a.T + tq) * a.nh + h) * D + 4 * lg_e;
        oscale = L > 0.f ? 1.f / L : 0.f;
    } else {
        const size_t bhs = (size_t) bh * a.ns + split;
        out = a.part_o + (bhs * a.R + r) * D + 4 * lg_e;
        oscale = 1.f;
        if (lg_e == 0) {
            float2 * mlp = &a.part_ml[bhs * a.R + r];
            __builtin_nontemporal_store(m_run, &mlp->x);
            __builtin_nontemporal_store(L, &mlp->y);
        }
        // a row that saw no key of this split (a causal split above its
        // diagonal) leaves its O partial unwritten: k_fattn_merge_rows loads
        // only the partials whose max is finite (k_fattn_merge, for more
        // splits, reads them all)
        if (m_run == -INFINITY && a.ns <= MERGE_ROWS_SPLITS) return;
    }
#pragma unroll
    for (int bb = 0; bb < NBLK; bb++) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const v4f o = O[bb][e] * oscale;
            float * op = out + 32 * bb + 16 * e;
            if (nsplit) {
                store_nt4(op, make_float4(o[0], o[1], o[2], o[3]));
            } else if (a.dst_vec) {
                *(float4 *) op = apply_gate(a, op, make_float4(o[0], o[1], o[2], o[3]));
            } else {
                op[0] = o[0]; op[1] = o[1]; op[2] = o[2]; op[3] = o[3];
            }
        }
    }
}

// ---------------------------------------------------------------- planning

// Attention kernel shapes: waves per block, query tiles, keys per wave.
enum fa_kind {
    FA_VD,        // k_fa_vd: at most 24 query rows per KV head, 8 waves, one block per CU, 32-key steps
    FA_VS,        // k_fa_vs: the shapes of k_fa_vd, 128-key rounds, each wave one V block (32 dims)
    FA_DEC,       // k_fa_dec: at most 32 query rows per KV head, 8 waves, one block per CU
    FA_PRE,       // k_fa_pre: longer query blocks, mask shared by the heads (or none), GQA >= 4
    FA_P4_T1,     // 4 waves, one tile, 64-key chunks, two blocks per CU
    FA_P4_T2,     // 4 waves, two tiles, 32 keys per wave, two blocks per CU; mask tiles of
                  // more than MASK_ROWS_PAIR rows go to 8 waves over the same 64-key chunks
};

struct fa_plan {
    int32_t R, RT, gqa, rw, n_rg, ns, split_len;
    int32_t max_span;                 // keys of the longest split, whole chunks
    int32_t pre_rgmap;                // k_fa_pre block order (fa_args::pre_rgmap)
    fa_kind kind;
    size_t  off_ml;                   // workspace section of the split (max, sum) pairs (bytes)
    size_t  ws_bytes;
    // per-sequence key counts: splits of each sequence (ns is the largest)
    int32_t ragged;
    int32_t r_ustart[RAGGED_MAX_B + 1], r_ns[RAGGED_MAX_B], r_split_len[RAGGED_MAX_B];
    int64_t r_n_kv[RAGGED_MAX_B];
};

// A forced key-split count for later calls (0: the planner's choice); set by
// qwfn_fattn_force_splits, read once per call.
std::atomic<int32_t> g_force_splits{0};
// A forced kernel family (QWFN_FA_KERNEL_*, 0: the planner's choice); set by
// qwfn_fattn_force_kernel, read once per call.
std::atomic<int32_t> g_force_kernel{0};
// The attention kernel the calling thread's last attention call launched
// (qwfn_fattn_last_kernel).
thread_local const char * g_last_kernel = "";
// A forced split-merge path (QWFN_FA_MERGE_*, 0: the planner's choice); set by
// qwfn_fattn_force_merge, read once per call; and the path the calling
// thread's last call took (qwfn_fattn_last_merge).
std::atomic<int32_t> g_force_merge{0};
thread_local int32_t g_last_merge = QWFN_FA_MERGE_NONE;

// The fused merge's counter slots on each device: g_merge_ctr's address there
// (hipGetSymbolAddress, once per device, with the device current) and the next
// free slot. A call takes one slot per (batch, KV head) group, consecutive and
// not wrapping round the end; calls in flight at once (on several streams)
// get disjoint slots unless more than MERGE_SLOTS groups are in flight.
constexpr int MERGE_MAX_DEVICES = 64;
std::mutex            g_merge_mu;
unsigned long long *  g_merge_addr[MERGE_MAX_DEVICES];
std::atomic<uint64_t> g_merge_next[MERGE_MAX_DEVICES];
std::atomic<uint64_t> g_merge_epoch[MERGE_MAX_DEVICES];   // the last epoch handed out (48 bits, from 1)

int merge_slots(int64_t groups, unsigned long long ** out, unsigned long long * ebase) {
    int dev = 0;
    QWFN_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MERGE_MAX_DEVICES) return set_error(QWFN_ENOTSUP, "flash_attn_ext: device index beyond the merge table");
    if (groups < 1 || groups > MERGE_SLOTS) return set_error(QWFN_EINVAL, "flash_attn_ext: merge groups out of range");
    unsigned long long * base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_merge_mu);
        if (!g_merge_addr[dev]) {
            void * p = nullptr;
            QWFN_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(g_merge_ctr)));
            if (!p) return set_error(QWFN_EDEVICE, "flash_attn_ext: merge counters have no device address");
            g_merge_addr[dev] = (unsigned long long *) p;
        }
        base = g_merge_addr[dev];
    }
    uint64_t first = g_merge_next[dev].fetch_add((uint64_t) groups, std::memory_order_relaxed) % MERGE_SLOTS;
    if (first + (uint64_t) groups > (uint64_t) MERGE_SLOTS) first = 0;
    *out = base + 2 * first;
    const uint64_t ep = (g_merge_epoch[dev].fetch_add(1, std::memory_order_relaxed) + 1) & ((uint64_t(1) << 48) - 1);
    *ebase = (unsigned long long) ep << 16;
    return QWFN_OK;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Bytes from the start of a mask batch slice to the end of its last row.
size_t mask_slice_bytes(const qwfn_tensor & m) {
    return (size_t) (m.ne[1] - 1) * m.nb[1] + (size_t) (m.ne[2] - 1) * m.nb[2] + (size_t) m.ne[0] * 2;
}

// Bytes from the start of a q batch slice to the end of its last row.
size_t q_slice_bytes(const qwfn_tensor & q) {
    return (size_t) (q.ne[1] - 1) * q.nb[1] + (size_t) (q.ne[2] - 1) * q.nb[2] + (size_t) q.ne[0] * 4;
}

// ceil(2^32 / d) for d > 1 (0 for d = 1, which divides without it).
// The key loop hand-counts its outstanding vector-memory operations (the LDS
// DMAs are inline asm the compiler does not see), so a build of the attention
// kernel that spills to scratch would break that count: refuse to run one.
int check_no_scratch() {
    static const int rc = [] {
        for (const void * f : {(const void *) k_fa_dec<1, false, false, false>, (const void *) k_fa_dec<1, true, false, false>,
                               (const void *) k_fa_dec<2, false, false, false>, (const void *) k_fa_dec<2, true, false, false>,
                               (const void *) k_fa_dec<1, false, true, false>, (const void *) k_fa_dec<1, true, true, false>,
                               (const void *) k_fa_dec<2, false, true, false>, (const void *) k_fa_dec<2, true, true, false>,
                               (const void *) k_fa_dec<1, false, false, true>, (const void *) k_fa_dec<2, false, false, true>,
                               (const void *) k_fa_vd<0, 1, false, false, false>, (const void *) k_fa_vd<0, 1, true, false, false>,
                               (const void *) k_fa_vd<0, 1, false, true, false>, (const void *) k_fa_vd<0, 1, true, true, false>,
                               (const void *) k_fa_vd<0, 1, false, false, true>,
                               (const void *) k_fa_vd<1, 0, false, false, false>, (const void *) k_fa_vd<1, 0, true, false, false>,
                               (const void *) k_fa_vd<1, 0, false, true, false>, (const void *) k_fa_vd<1, 0, true, true, false>,
                               (const void *) k_fa_vd<1, 0, false, false, true>,
                               (const void *) k_fa_vd<1, 1, false, false, false>, (const void *) k_fa_vd<1, 1, true, false, false>,
                               (const void *) k_fa_vd<1, 1, false, true, false>, (const void *) k_fa_vd<1, 1, true, true, false>,
                               (const void *) k_fa_vd<1, 1, false, false, true>,
                               (const void *) k_fa_vs<0, 1, false, false, false>, (const void *) k_fa_vs<0, 1, true, false, false>,
                               (const void *) k_fa_vs<0, 1, false, true, false>, (const void *) k_fa_vs<0, 1, true, true, false>,
                               (const void *) k_fa_vs<0, 1, false, false, true>,
                               (const void *) k_fa_vs<1, 0, false, false, false>, (const void *) k_fa_vs<1, 0, true, false, false>,
                               (const void *) k_fa_vs<1, 0, false, true, false>, (const void *) k_fa_vs<1, 0, true, true, false>,
                               (const void *) k_fa_vs<1, 0, false, false, true>,
                               (const void *) k_fa_vs<1, 1, false, false, false>, (const void *) k_fa_vs<1, 1, true, false, false>,
                               (const void *) k_fa_vs<1, 1, false, true, false>, (const void *) k_fa_vs<1, 1, true, true, false>,
                               (const void *) k_fa_vs<1, 1, false, false, true>,
                               (const void *) k_fa_pre<false>, (const void *) k_fa_pre<true>,
                               (const void *) k_fa_qc<2>, (const void *) k_fa_qc<4>, (const void *) k_fa_qc<8>,
                               (const void *) k_fattn_q8_0<2, true, WAVES, 16, false>,
                               (const void *) k_fattn_q8_0<1, false, WAVES_PAIR, 16, false>,
                               (const void *) k_fattn_q8_0<1, true, WAVES_PAIR, 16, false>,
                               (const void *) k_fattn_q8_0<2, false, WAVES_PAIR, 32, false>,
                               (const void *) k_fattn_q8_0<2, true, WAVES_PAIR, 32, false>,
                               (const void *) k_fattn_q8_0<1, false, WAVES_PAIR, 16, true>,
                               (const void *) k_fattn_q8_0<1, true, WAVES_PAIR, 16, true>,
                               (const void *) k_fattn_q8_0<2, false, WAVES_PAIR, 32, true>,
                               (const void *) k_fattn_q8_0<2, true, WAVES_PAIR, 32, true>,
                               (const void *) k_fattn_q8_0<2, true, WAVES, 16, true>}) {
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
               fa_plan * pl, const int64_t * seq_n_kv = nullptr, int64_t ns_cap = MAX_SPLITS, bool gather = false) {
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
    // row indices divide by gqa through a 32-bit reciprocal (exact while R * gqa < 2^32)
    if (R * gqa >= (int64_t(1) << 32)) return set_error(QWFN_ENOTSUP, "flash_attn_ext: T * n_head * gqa too large");
    // query rows travel as 32-bit offsets within one batch slice
    if (q_slice_bytes(*q) >= (size_t(1) << 32))
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: q batch slices must be below 4 GiB");
    // 16-byte aligned rows and heads: the kernel stages K/V with 16-byte loads.
    if (!is_aligned(k->data, 16) || !is_aligned(v->data, 16) || k->nb[1] % 16 || k->nb[2] % 16 || k->nb[3] % 16 ||
        v->nb[1] % 16 || v->nb[2] % 16 || v->nb[3] % 16)
        return set_error(QWFN_EALIGN, "flash_attn_ext: k/v data and strides must be 16-byte aligned");
    if (!is_aligned(q->data, 16) || q->nb[1] % 16 || q->nb[2] % 16 || q->nb[3] % 16)
        return set_error(QWFN_EALIGN, "flash_attn_ext: q data and strides must be 16-byte aligned");
    if (k->nb[1] >= (size_t(1) << 24) || v->nb[1] >= (size_t(1) << 24))
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: k/v row strides must be below 16 MiB");
    const int64_t n_kv = k->ne[1];
    if (mask) {
        if (!mask->data) return set_error(QWFN_EINVAL, "flash_attn_ext: mask has no data");
        if (mask->type != QWFN_TYPE_F16) return set_error(QWFN_EINVAL, "flash_attn_ext: mask must be f16");
        if (mask->nb[0] != 2) return set_error(QWFN_EINVAL, "flash_attn_ext: mask rows must be contiguous");
        if (mask->ne[0] < n_kv || mask->ne[1] < T)
            return set_error(QWFN_EINVAL, "flash_attn_ext: mask must be at least [n_kv, T]");
        if (mask->ne[2] <= 0 || nh % mask->ne[2] || mask->ne[3] <= 0 || q->ne[3] % mask->ne[3])
            return set_error(QWFN_EINVAL, "flash_attn_ext: mask must broadcast over heads and batch");
        if (!is_aligned(mask->data, 2)) return set_error(QWFN_EALIGN, "flash_attn_ext: mask must be 2-byte aligned");
        // per-lane mask offsets are 32-bit within one batch slice (plus a chunk of slack)
        if (mask_slice_bytes(*mask) >= (size_t(1) << 31))
            return set_error(QWFN_ENOTSUP, "flash_attn_ext: mask batch slices must be below 2 GiB");
    }
    // Query rows per block: one or two 16-row tiles. Up to 32 rows per KV head
    // (decode, verify, batch decode) take k_fa_dec, 8-wave blocks, one per CU;
    // longer query blocks k_fattn_q8_0's 4-wave blocks, two per CU (their
    // prologues and phases overlap).
    const int rw = R > 16 ? 32 : 16;
    const int64_t B = q->ne[3];
    const bool dec = R <= 32;
    pl->kind = dec ? FA_DEC : rw == 16 ? FA_P4_T1 : FA_P4_T2;
    // k_fa_vd: up to 24 rows (a full and a packed tile), K and V rows of one
    // stride, and a mask shared by the heads over at most VD_MROWS query
    // positions (its granules travel with each step)
    const bool vd_ok = dec && R <= VD_ROWS && k->nb[1] == v->nb[1] &&
                       (!mask || (mask->ne[2] == 1 && (R - 1) / gqa + 1 <= VD_MROWS));
    const bool pre_ok = !dec && !gather && !seq_n_kv && (!mask || mask->ne[2] == 1) && gqa >= 4;
    const int32_t fk = g_force_kernel.load(std::memory_order_relaxed);
    switch (fk) {
        case QWFN_FA_KERNEL_VD:
            if (!vd_ok) return set_error(QWFN_ENOTSUP, "flash_attn_ext: the forced VD kernel cannot take this shape");
            break;
        case QWFN_FA_KERNEL_VS:
            if (!vd_ok) return set_error(QWFN_ENOTSUP, "flash_attn_ext: the forced VS kernel cannot take this shape");
            break;
        case QWFN_FA_KERNEL_DEC:
            if (!dec) return set_error(QWFN_ENOTSUP, "flash_attn_ext: the forced DEC kernel takes at most 32 rows per KV head");
            break;
        case QWFN_FA_KERNEL_GENERAL:
            if (gather) return set_error(QWFN_ENOTSUP, "flash_attn_ext: the forced GENERAL kernel takes no cell lists");
            pl->kind = rw == 16 ? FA_P4_T1 : FA_P4_T2;
            break;
        case QWFN_FA_KERNEL_PRE:
            if (!pre_ok) return set_error(QWFN_ENOTSUP, "flash_attn_ext: the forced PRE kernel cannot take this shape");
            break;
        default:
            break;
    }
    // k_fa_vd measures slower than k_fa_dec at every depth so far (its
    // prologue and epilogue cost more than its steps save): callers reach it
    // only by forcing it. k_fa_vs measures faster than k_fa_dec for one
    // sequence of at most 8 rows per KV head (one position, GQA 8) up to
    // 32K keys (kernel + merge, 2 KV heads: 1K 14.9 against 15.3 us, 16K
    // 16.5 against 17.3, 32K 21.0 against 21.4), slower past it (64K 28.5
    // against 27.0) and slower for 24 rows at every depth (16K 19.5
    // against 18.9)
    if (vd_ok && fk == QWFN_FA_KERNEL_VD) pl->kind = FA_VD;
    if (vd_ok && fk == QWFN_FA_KERNEL_VS) pl->kind = FA_VS;
    if (vd_ok && fk == QWFN_FA_KERNEL_AUTO && R <= 8 && B == 1 && !seq_n_kv && !gather && n_kv <= VS_AUTO_MAX_KEYS)
        pl->kind = FA_VS;
    if (pre_ok && (fk == QWFN_FA_KERNEL_AUTO || fk == QWFN_FA_KERNEL_PRE)) {
        // k_fa_pre: 128-row blocks; key splits of whole 64-key chunks (at least
        // two per split), about one block per CU; the row groups of a (batch,
        // KV head, split) unit share an XCD
        pl->kind = FA_PRE;
        pl->R = (int32_t) R;
        pl->rw = PRE_ROWS;
        pl->RT = PRE_WAVES;
        pl->n_rg = (int32_t) ((R + PRE_ROWS - 1) / PRE_ROWS);
        pl->gqa = (int32_t) gqa;
        const int64_t per = nh_kv * B * pl->n_rg;
        int64_t ns = std::max<int64_t>(1, (256 + per - 1) / per);
        ns = std::min<int64_t>(ns, std::max<int64_t>(1, n_kv / (2 * PRE_CK)));
        if (const int32_t force = g_force_splits.load(std::memory_order_relaxed)) ns = force;
        ns = std::max<int64_t>(1, std::min<int64_t>(ns, ns_cap));
        int64_t split_len = (n_kv + ns - 1) / ns;
        split_len = std::max<int64_t>(PRE_CK, (split_len + PRE_CK - 1) / PRE_CK * PRE_CK);
        ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
        if (ns > MAX_SPLITS)
            return set_error(QWFN_ENOTSUP, "flash_attn_ext: " + std::to_string(ns) + " key splits requested, at most " +
                                               std::to_string(MAX_SPLITS) + " supported");
        pl->ns = (int32_t) ns;
        pl->split_len = (int32_t) split_len;
        pl->max_span = split_len;
        pl->ragged = 0;
        // block order: the bytes an XCD's L2 cannot share. Units on an XCD read
        // each KV head's f32 query rows once per split; row groups on an XCD
        // (one KV head an XCD) read its K/V rows once per XCD holding its rows
        const int64_t nbh = B * nh_kv;
        const double q_rep = (double) R * D * 4 * (double) (ns - 1);
        const double kv_rep = (double) n_kv * (2.0 * (D / 32) * 34) * (double) (std::max<int64_t>(1, 8 / nbh) - 1);
        pl->pre_rgmap = ns > 1 && q_rep > kv_rep ? 1 : 0;
        const size_t n_part = ns > 1 ? (size_t) (B * nh_kv * ns * R) : 0;
        size_t off = align256(n_part * D * sizeof(float));
        pl->off_ml = off;
        off = align256(off + n_part * sizeof(float2));
        pl->ws_bytes = std::max<size_t>(off, 256);
        return QWFN_OK;
    }
    const bool vs = pl->kind == FA_VS;
    const bool vd = pl->kind == FA_VD || vs, kdec = pl->kind == FA_DEC;
    pl->R = (int32_t) R;
    pl->rw = vd ? VD_ROWS : rw;
    pl->RT = vd ? 1 : rw / 16;
    pl->n_rg = vd ? 1 : (int32_t) ((R + rw - 1) / rw);
    pl->gqa = (int32_t) gqa;
    // k_fa_vd: splits of whole 16-key sub-tiles, at least one per wave;
    // k_fa_dec: whole 16-key tiles, at least one tile per key group;
    // k_fattn_q8_0: whole chunks.
    const int64_t ck = vd ? DEC_TK : kdec ? DEC_TK
                     : pl->kind == FA_P4_T1 ? fa_cfg<1, false, WAVES_PAIR, 16>::CK : fa_cfg<2, false, WAVES_PAIR, 32>::CK;
    // (gathered cells with one row tile, T <= 2 at GQA 8: splits down to one
    // 16-key tile, so that the grid reaches a block per CU although most
    // waves of a block then idle; shared list, T = 1, kernel + merge: 1024
    // cells 13.8 -> 12.9 us, 2052 14.1 -> 13.1, 4096 15.0 -> 13.9, 8192 15.6 ->
    // 14.3. With two row tiles the same grid is slower: 3 x 2052, 64 splits
    // 22.6 against 16.3 us)
    const int64_t min_split = vd ? DEC_TK * VD_WAVES
                            : kdec ? (gather && pl->RT == 1 ? DEC_TK : DEC_TK * (DEC_WAVES / pl->RT)) : ck;
    // Splits: about one block per CU slot (256 for the one-block-per-CU
    // kernels, 512 otherwise).
    const int64_t target_blocks = vd || kdec ? 256 : 512;
    int64_t ns = std::max<int64_t>(1, target_blocks / std::max<int64_t>(1, nh_kv * B * pl->n_rg));
    if (vd) ns = std::min<int64_t>(ns, std::max<int64_t>(1, n_kv / min_split));
    else    ns = std::min<int64_t>(ns, std::max<int64_t>(1, (n_kv + min_split - 1) / min_split));
    const int32_t forced_ns = g_force_splits.load(std::memory_order_relaxed);
    if (forced_ns) ns = forced_ns;
    ns = std::min<int64_t>(ns, std::max<int64_t>(1, ns_cap));
    if (gather) {
        // gathered keys: a block's cells fit its LDS list
        if (!vd && !kdec) return set_error(QWFN_ENOTSUP, "flash_attn_ext_cells: at most 32 query rows per KV head (T * n_head / n_head_kv)");
        ns = std::max<int64_t>(ns, (n_kv + DEC_GATHER_SPLIT - 1) / DEC_GATHER_SPLIT);
    }
    int64_t split_len;
    if (vd && !gather) {
        const int64_t per = std::max<int64_t>(1, nh_kv * B);
        if (vs) {
            // Every wave of a k_fa_vs block takes ceil(s / 8) rounds for a
            // split of s sub-tiles, so splits are whole rounds of 128 keys,
            // as many as fill one block per CU, and the last split takes the
            // keys past the others' (n_kv = 2^k + T: one short round more in
            // one block, rather than a block more than the CUs)
            const int64_t rk = DEC_TK * VS_WAVES;
            const int64_t want = forced_ns ? (int64_t) forced_ns : std::max<int64_t>(1, target_blocks / per);
            const int64_t rounds = std::max<int64_t>(1, n_kv / rk);
            split_len = (rounds + want - 1) / want * rk;
            ns = forced_ns ? (n_kv + split_len - 1) / split_len : n_kv / split_len;
            ns = std::max<int64_t>(1, ns);
        } else {
            // The slowest wave of a split of s sub-tiles takes ceil(s / 8) of
            // them: pairs as steps, an odd one as a half step. The fewest
            // sub-tiles per split with every block on a CU of its own (the
            // last split takes what is left, fewer keys) give the shortest
            // slowest wave; a forced split count takes the sub-tiles that it
            // implies.
            int64_t sub = std::max<int64_t>(VD_WAVES, (n_kv + ck * ns - 1) / (ck * ns));
            if (!forced_ns)
                while ((n_kv + ck * sub - 1) / (ck * sub) * per > target_blocks) sub++;
            split_len = ck * sub;
            ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
        }
        if (ns > ns_cap) {
            split_len = (n_kv + ns_cap - 1) / ns_cap;
            split_len = (split_len + ck - 1) / ck * ck;
            ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
        }
    } else {
        // Splits are whole chunks. When the keys exceed two or more chunks per
        // split by less than one chunk (n_kv = 2^k + T), the last split takes the
        // rest; otherwise every split rounds up and there are fewer.
        split_len = n_kv / (ns * ck) * ck;
        if (gather || split_len < (kdec ? min_split : 2 * ck) || n_kv - ns * split_len >= (kdec ? min_split : ck)) {
            split_len = (n_kv + ns - 1) / ns;
            split_len = std::max<int64_t>(ck, (split_len + ck - 1) / ck * ck);
            ns = std::max<int64_t>(1, (n_kv + split_len - 1) / split_len);
        }
    }
    // keys of the longest split (the last may be longer), rounded up to whole chunks
    pl->max_span = std::max<int64_t>(split_len, n_kv - (ns - 1) * split_len);
    pl->max_span = (pl->max_span + ck - 1) / ck * ck;
    pl->ragged = 0;
    if (seq_n_kv) {
        // Per-sequence key counts: each sequence gets splits in proportion to its
        // keys, so every block streams about the same number of chunks whatever
        // the spread of the depths. Splits round up to whole chunks.
        if (B > RAGGED_MAX_B)
            return set_error(QWFN_ENOTSUP, "flash_attn_ext_seq: at most " + std::to_string(RAGGED_MAX_B) + " sequences");
        int64_t total = 0;
        for (int64_t b = 0; b < B; b++) {
            if (seq_n_kv[b] < 0 || seq_n_kv[b] > n_kv)
                return set_error(QWFN_ERANGE, "flash_attn_ext_seq: sequence key counts must lie in [0, n_kv]");
            total += seq_n_kv[b];
        }
        // (a forced split count asks for that many splits per sequence on average)
        const int64_t units = std::max<int64_t>(1, std::min<int64_t>(forced_ns ? forced_ns * B
                                                                               : target_blocks / std::max<int64_t>(1, nh_kv * pl->n_rg),
                                                                     ns_cap * B));
        int64_t ns_max = 1, span = ck, ustart = 0;
        for (int64_t b = 0; b < B; b++) {
            const int64_t nk = seq_n_kv[b];
            int64_t nsb = total > 0 ? std::max<int64_t>(1, (units * nk + total / 2) / total) : 1;
            nsb = std::min<int64_t>(nsb, std::max<int64_t>(1, (nk + min_split - 1) / min_split));
            int64_t sl = (nk + nsb - 1) / nsb;
            sl = std::max<int64_t>(ck, (sl + ck - 1) / ck * ck);
            nsb = std::max<int64_t>(1, (nk + sl - 1) / sl);
            pl->r_ustart[b] = (int32_t) ustart;
            pl->r_ns[b] = (int32_t) nsb;
            pl->r_split_len[b] = (int32_t) sl;
            pl->r_n_kv[b] = nk;
            ustart += nsb;
            ns_max = std::max(ns_max, nsb);
            span = std::max(span, sl);
        }
        pl->r_ustart[B] = (int32_t) ustart;
        pl->ragged = 1;
        ns = ns_max;
        split_len = span;
        pl->max_span = (int32_t) span;
    }
    if (ns > MAX_SPLITS)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: " + std::to_string(ns) + " key splits requested, at most " +
                                           std::to_string(MAX_SPLITS) + " supported");
    pl->ns = (int32_t) ns;
    pl->split_len = (int32_t) split_len;
    // workspace: split partials (when ns > 1)
    const size_t n_part = ns > 1 ? (size_t) (B * nh_kv * ns * R) : 0;
    size_t off = align256(n_part * D * sizeof(float));
    pl->off_ml = off;
    off = align256(off + n_part * sizeof(float2));
    pl->ws_bytes = std::max<size_t>(off, 256);
    return QWFN_OK;
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" size_t qwfn_fattn_workspace_size(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                            const qwfn_tensor * mask) {
    return ::qwfn::abi_value<size_t>("fattn_workspace_size", 0, [&]() -> size_t {
        fa_plan pl{};
        if (plan_fattn(q, k, v, mask, &pl)) return 0;
        return pl.ws_bytes;
    });
}

namespace {

struct fa_append {
    const qwfn_tensor * src_k;
    const qwfn_tensor * src_v;
    int64_t first_row;
};

int check_append(const fa_append & ap, const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v) {
    const qwfn_tensor * srcs[2] = {ap.src_k, ap.src_v};
    for (const qwfn_tensor * s : srcs) {
        if (!s || !s->data) return set_error(QWFN_EINVAL, "flash_attn_ext_append: src is NULL");
        if (s->type != QWFN_TYPE_F32 || s->nb[0] != 4) return set_error(QWFN_EINVAL, "flash_attn_ext_append: src must be contiguous f32 rows");
        if (s->ne[2] != 1 || s->ne[3] != 1) return set_error(QWFN_ENOTSUP, "flash_attn_ext_append: src must be 2-D");
        if (s->ne[0] != (int64_t) D * k->ne[2]) return set_error(QWFN_EINVAL, "flash_attn_ext_append: src rows must hold every KV head (256 * n_head_kv values)");
        if (!is_aligned(s->data, 16) || s->nb[1] % 16) return set_error(QWFN_EALIGN, "flash_attn_ext_append: src rows must be 16-byte aligned");
    }
    if (ap.src_k->ne[1] != ap.src_v->ne[1] || ap.src_k->nb[1] != ap.src_v->nb[1])
        return set_error(QWFN_EINVAL, "flash_attn_ext_append: src_k and src_v must have the same shape");
    const int64_t n = ap.src_k->ne[1];
    if (n < 1 || n > 64) return set_error(QWFN_ENOTSUP, "flash_attn_ext_append: 1 to 64 appended rows");
    if (ap.first_row < 0 || ap.first_row + n > k->ne[1])
        return set_error(QWFN_ERANGE, "flash_attn_ext_append: the appended rows must lie inside the attended keys");
    if (q->ne[3] != 1 || k->ne[3] != 1 || v->ne[3] != 1) return set_error(QWFN_ENOTSUP, "flash_attn_ext_append: one sequence (B = 1)");
    const size_t seg = (size_t) D / QK * QBLOCK;
    if (k->nb[2] != seg || v->nb[2] != seg)
        return set_error(QWFN_EINVAL, "flash_attn_ext_append: K/V heads must be consecutive 272-byte segments of a cache row");
    return QWFN_OK;
}

// Workspace of the allocation-free entry point (qwfn_flash_attn_ext_q8_0_noalloc):
// device memory of the library's code object, one copy per GPU, held until
// the process ends. In host code `scratch` only names the symbol; its device
// address on the current GPU comes from hipGetSymbolAddress (scratch_address).
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(16) << 20;
__device__ __align__(256) static char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *     g_scratch_addr[SCRATCH_MAX_DEVICES];   // scratch's address on each device, once looked up

// scratch's device address on the current device: looked up once per device
// (with that device current) on the first call there.
int scratch_address(void ** out) {
    int dev = 0;
    QWFN_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return set_error(QWFN_ENOTSUP, "flash_attn_ext_noalloc: device index beyond the library's table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void * p = nullptr;
        QWFN_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p || !is_aligned(p, 256)) return set_error(QWFN_EDEVICE, "flash_attn_ext_noalloc: scratch has no usable device address");
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return QWFN_OK;
}

// Where the split partials go: the caller's workspace (or the library-owned
// buffer when ws is NULL), or the library's static scratch.
enum ws_mode { WS_CALLER, WS_SCRATCH };

// Gathered keys: per KV head a list of cache rows (qwfn_flash_attn_ext_q8_0_cells).
struct fa_gather {
    const int32_t * cells;
    const int64_t * n_cells;   // host: one count per KV head, or per query position (per_query)
    int64_t stride;            // between the lists of consecutive heads, or positions (per_query)
    int64_t pos0;
    int64_t n_rows;            // rows of the cache
    bool    per_query = false; // one list per query position, shared by the KV heads
};

// Launch of an attention kernel of the fa_args `a` in scope, recording its
// name for qwfn_fattn_last_kernel.
#define QWFN_FA_LAUNCH(G, BD, ST, ...)                              \
    do {                                                            \
        g_last_kernel = #__VA_ARGS__;                               \
        hipLaunchKernelGGL((__VA_ARGS__), G, BD, 0, ST, a);         \
    } while (0)

// k_fa_vd with NF full and PK packed tiles, by mask, per-sequence counts and cell lists
template <int NF, int PK, bool M, bool RG, bool G>
void launch_vd1(const fa_args & a, dim3 g, hipStream_t st) {
    static const std::string name = "k_fa_vd<" + std::to_string(NF) + ", " + std::to_string(PK) + ", " +
                                    (M ? "true" : "false") + ", " + (RG ? "true" : "false") + ", " + (G ? "true" : "false") + ">";
    g_last_kernel = name.c_str();
    hipLaunchKernelGGL((k_fa_vd<NF, PK, M, RG, G>), g, dim3(VD_WAVES * 64), 0, st, a);
}
template <int NF, int PK>
void launch_vd(const fa_args & a, bool msk, bool rg, bool gat, dim3 g, hipStream_t st) {
    if (gat)      launch_vd1<NF, PK, false, false, true>(a, g, st);
    else if (rg)  { if (msk) launch_vd1<NF, PK, true, true, false>(a, g, st);
                    else     launch_vd1<NF, PK, false, true, false>(a, g, st); }
    else          { if (msk) launch_vd1<NF, PK, true, false, false>(a, g, st);
                    else     launch_vd1<NF, PK, false, false, false>(a, g, st); }
}
// k_fa_vs, likewise
template <int NF, int PK, bool M, bool RG, bool G>
void launch_vs1(const fa_args & a, dim3 g, hipStream_t st) {
    static const std::string name = "k_fa_vs<" + std::to_string(NF) + ", " + std::to_string(PK) + ", " +
                                    (M ? "true" : "false") + ", " + (RG ? "true" : "false") + ", " + (G ? "true" : "false") + ">";
    g_last_kernel = name.c_str();
    hipLaunchKernelGGL((k_fa_vs<NF, PK, M, RG, G>), g, dim3(VS_WAVES * 64), 0, st, a);
}
template <int NF, int PK>
void launch_vs(const fa_args & a, bool msk, bool rg, bool gat, dim3 g, hipStream_t st) {
    if (gat)      launch_vs1<NF, PK, false, false, true>(a, g, st);
    else if (rg)  { if (msk) launch_vs1<NF, PK, true, true, false>(a, g, st);
                    else     launch_vs1<NF, PK, false, true, false>(a, g, st); }
    else          { if (msk) launch_vs1<NF, PK, true, false, false>(a, g, st);
                    else     launch_vs1<NF, PK, false, false, false>(a, g, st); }
}

int fattn_run(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v, const qwfn_tensor * mask, float scale,
              float max_bias, float logit_softcap, const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
              void * stream, const fa_append * app, const int64_t * seq_n_kv = nullptr, ws_mode wsm = WS_CALLER,
              const fa_gather * gat = nullptr, const qwfn_tensor * gate = nullptr) {
    if (max_bias != 0.0f) return set_error(QWFN_ENOTSUP, "flash_attn_ext: max_bias (ALiBi) is not supported");
    if (logit_softcap != 0.0f) return set_error(QWFN_ENOTSUP, "flash_attn_ext: logit_softcap is not supported");
    if (!(std::isfinite(scale))) return set_error(QWFN_EINVAL, "flash_attn_ext: scale must be finite");
    if (variant != QWFN_Q8_REF && variant != QWFN_Q8_X86) return set_error(QWFN_EINVAL, "flash_attn_ext: unknown variant");
    fa_plan pl{};
    if (int rc = plan_fattn(q, k, v, mask, &pl, seq_n_kv, MAX_SPLITS, gat != nullptr)) return rc;
    if (wsm == WS_SCRATCH && pl.ws_bytes > NOALLOC_SCRATCH_BYTES) {
        // fewer key splits, so that their partials fit the scratch
        const size_t per_split = (size_t) q->ne[3] * k->ne[2] * pl.R * (D * sizeof(float) + sizeof(float2));
        const int64_t cap = std::max<int64_t>(1, (int64_t) ((NOALLOC_SCRATCH_BYTES - 512) / std::max<size_t>(per_split, 1)));
        if (int rc = plan_fattn(q, k, v, mask, &pl, seq_n_kv, cap, gat != nullptr)) return rc;
        if (pl.ws_bytes > NOALLOC_SCRATCH_BYTES)
            return set_error(QWFN_ENOMEM, "flash_attn_ext_noalloc: the split partials need more than the 16 MiB scratch");
    }
    if (app)
        if (int rc = check_append(*app, q, k, v)) return rc;
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
    if (wsm == WS_SCRATCH) {
        if (int rc = scratch_address(&ws)) return rc;
    } else if (ws) {
        if (ws_bytes < pl.ws_bytes) return set_error(QWFN_ENOMEM, "flash_attn_ext: workspace too small");
        if (!is_aligned(ws, 256)) return set_error(QWFN_EALIGN, "flash_attn_ext: workspace must be 256-byte aligned");
    } else if (int rc = library_workspace(pl.ws_bytes, as_stream(stream), &ws)) {
        return rc;
    }
    if (int rc = check_no_scratch()) return rc;

    fa_args a{};
    a.q = (const char *) q->data; a.q_nb1 = q->nb[1]; a.q_nb2 = q->nb[2]; a.q_nb3 = q->nb[3];
    a.k = (const char *) k->data; a.k_nb1 = k->nb[1]; a.k_nb2 = k->nb[2]; a.k_nb3 = k->nb[3];
    a.v = (const char *) v->data; a.v_nb1 = v->nb[1]; a.v_nb2 = v->nb[2]; a.v_nb3 = v->nb[3];
    char * w = (char *) ws;
    a.n_kv = n_kv;
    a.T = (int32_t) q->ne[1]; a.nh = (int32_t) q->ne[2]; a.nh_kv = (int32_t) k->ne[2];
    int64_t mrows = 0;    // mask rows a block can span, at most
    if (mask) {
        a.mask = (const char *) mask->data; a.m_nb1 = mask->nb[1]; a.m_nb2 = mask->nb[2]; a.m_nb3 = mask->nb[3];
        a.m_ne2 = (int32_t) mask->ne[2]; a.m_ne3 = (int32_t) mask->ne[3];
        a.m_slice = (uint32_t) mask_slice_bytes(*mask);
        // MASK_SPLIT: each mask row of a split as 16-byte granules from the
        // aligned address at or below its first key, all in LDS at once
        mrows = mask->ne[2] == 1 ? ((int64_t) pl.rw + pl.gqa - 1) / pl.gqa + 1 : pl.rw;
        const int64_t mlds = pl.kind == FA_P4_T2 ? fa_cfg<2, false, WAVES_PAIR, 32>::MLDS : MASK_LDS;
        a.m_gran = pl.max_span / 8 + 1;
        a.m_gran_mul = recip32(a.m_gran);
        a.mask_mode = mrows * 16 * a.m_gran <= mlds ? MASK_SPLIT : MASK_TILE;
    } else {
        a.mask = nullptr; a.m_ne2 = 1; a.m_ne3 = 1; a.m_slice = 0; a.mask_mode = MASK_NONE;
    }
    a.dst = (float *) dst->data;
    a.part_o = (float *) w;
    a.part_ml = (float2 *) (w + pl.off_ml);
    a.gqa = pl.gqa; a.R = pl.R; a.B = (int32_t) q->ne[3];
    a.kb = (int32_t) k->ne[3]; a.vb = (int32_t) v->ne[3];
    a.ns = pl.ns; a.split_len = pl.split_len; a.rw = pl.rw; a.n_rg = pl.n_rg;
    a.pre_rgmap = pl.kind == FA_PRE ? pl.pre_rgmap : 0;
    a.ragged = pl.ragged;
    if (pl.ragged) {
        for (int b = 0; b <= a.B; b++) a.r_ustart[b] = pl.r_ustart[b];
        a.r_units = pl.r_ustart[a.B];
        for (int b = 0; b < a.B; b++) {
            a.r_ns[b] = pl.r_ns[b]; a.r_split_len[b] = pl.r_split_len[b]; a.r_n_kv[b] = pl.r_n_kv[b];
        }
    }
    a.scale = scale; a.x86 = variant == QWFN_Q8_X86;
    a.dst_vec = is_aligned(dst->data, 16) ? 1 : 0;
    if (gate) {
        if (!gate->data || gate->type != QWFN_TYPE_F32) return set_error(QWFN_EINVAL, "flash_attn_ext_gated: gate must be f32");
        for (int i = 0; i < 4; i++)
            if (gate->ne[i] != dst->ne[i] || gate->nb[i] != dst->nb[i])
                return set_error(QWFN_EINVAL, "flash_attn_ext_gated: gate must have dst's shape and strides");
        const bool contiguous = dst->nb[0] == 4 && dst->nb[1] == (size_t) D * 4 && dst->nb[2] == dst->nb[1] * dst->ne[1] &&
                                dst->nb[3] == dst->nb[2] * dst->ne[2];
        if (!contiguous || !is_aligned(dst->data, 16) || !is_aligned(gate->data, 16))
            return set_error(QWFN_EALIGN, "flash_attn_ext_gated: dst and gate must be contiguous and 16-byte aligned");
        a.gate = (const float *) gate->data;
    }
    a.q_slice = (uint32_t) q_slice_bytes(*q);
    a.gqa_mul = recip32(pl.gqa);
    if (gat) {
        a.g_cells = gat->cells;
        a.g_bstride = gat->per_query ? gat->stride : 0;
        a.g_hstride = gat->per_query ? 0 : gat->stride;
        a.g_pos0 = gat->pos0;
        a.g_rows = gat->n_rows;
        for (int64_t b = 0; b < a.B; b++)
            for (int64_t h = 0; h < a.nh_kv; h++)
                a.g_n[b * a.nh_kv + h] = (int32_t) gat->n_cells[gat->per_query ? b : h];
        if (int rc = status_word(&a.status)) return rc;
    }
    if (app) {
        a.app_k = (const char *) app->src_k->data;
        a.app_v = (const char *) app->src_v->data;
        a.app_nb1 = app->src_k->nb[1];
        a.app_row0 = app->first_row;
        a.app_n = (int32_t) app->src_k->ne[1];
    }

    if (pl.kind == FA_PRE) {
        const int64_t units = (int64_t) a.B * a.nh_kv * a.ns;
        const int64_t rgus = (int64_t) a.B * a.nh_kv * a.n_rg;
        const int64_t grid = a.pre_rgmap ? 8 * (int64_t) a.ns * ((rgus + 7) / 8) : 8 * (int64_t) a.n_rg * ((units + 7) / 8);
        if (grid >= (int64_t(1) << 31) || grid * a.n_rg >= (int64_t(1) << 32) || units * a.ns >= (int64_t(1) << 32))
            return set_error(QWFN_ENOTSUP, "flash_attn_ext: grid too large");
        a.ns_mul = recip32(a.ns);
        a.nrg_mul = recip32(a.n_rg);
        a.nbh_mul = recip32(a.B * a.nh_kv);
        const dim3 g((unsigned) grid), bd(PRE_WAVES * 64);
        if (a.mask) QWFN_FA_LAUNCH(g, bd, as_stream(stream), k_fa_pre<true>);
        else        QWFN_FA_LAUNCH(g, bd, as_stream(stream), k_fa_pre<false>);
        g_last_merge = a.ns > 1 ? QWFN_FA_MERGE_KERNEL : QWFN_FA_MERGE_NONE;
        if (int rc = hip_check(hipGetLastError(), "flash_attn launch")) return rc;
        if (a.ns > 1) {
            const int64_t rows = (int64_t) a.B * a.nh_kv * a.R;
            if (rows * 4 > 0x7fffffff) return set_error(QWFN_EINVAL, "flash_attn_ext: merge grid too large");
            if (a.ns <= MERGE_ROWS_SPLITS)
                hipLaunchKernelGGL(k_fattn_merge_rows, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, as_stream(stream), a);
            else
                hipLaunchKernelGGL(k_fattn_merge<false>, dim3((unsigned) (rows * 4)), dim3(256), 0, as_stream(stream), a);
            if (int rc = hip_check(hipGetLastError(), "flash_attn merge launch")) return rc;
        }
        return QWFN_OK;
    }
    if (pl.kind == FA_DEC || pl.kind == FA_VD || pl.kind == FA_VS) a.n_rg = 1;
    // the split merge: a k_fattn_merge launch unless the in-kernel merge is
    // forced. The launch measures faster (16384 keys, T = 3: 20.0 against
    // 27.1 us per op; 65536: 33.2 against 39.1): after the last split, the
    // in-kernel merge waits out a chain of device-scope round trips (the
    // partials' store completion, the arrival, a row claim, the partials'
    // loads) that costs more than the launch boundary it replaces
    const int32_t fm = g_force_merge.load(std::memory_order_relaxed);
    const int64_t groups = (int64_t) a.B * a.nh_kv;
    const bool fuse = (pl.kind == FA_DEC || pl.kind == FA_VD || pl.kind == FA_VS) && !a.ragged && a.ns > 1 && groups <= MERGE_SLOTS &&
                      pl.off_ml < (size_t(1) << 32) && fm == QWFN_FA_MERGE_FUSED;
    if (fuse) {
        if (int rc = merge_slots(groups, &a.mctr, &a.m_ebase)) return rc;
        a.m_nm = std::min<int32_t>(a.R, a.ns);
    }
    g_last_merge = a.ns <= 1 ? QWFN_FA_MERGE_NONE : fuse ? QWFN_FA_MERGE_FUSED : QWFN_FA_MERGE_KERNEL;
    const int64_t n_units = a.ragged ? (int64_t) a.r_units : (int64_t) a.B * a.ns;
    const int64_t units = n_units >= 8 ? (n_units + 7) / 8 * 8 : n_units;
    const int64_t hgn = (int64_t) a.nh_kv * a.n_rg;
    const int64_t grid = units * hgn;
    // block indices divide by ns, nh_kv * n_rg and n_rg through 32-bit reciprocals
    if (grid * hgn >= (int64_t(1) << 32) || units * a.ns >= (int64_t(1) << 32))
        return set_error(QWFN_ENOTSUP, "flash_attn_ext: grid too large");
    a.ns_mul = recip32(a.ns);
    a.hgn_mul = recip32(hgn);
    a.nrg_mul = recip32(a.n_rg);
    hipStream_t st = as_stream(stream);
    const bool mt = a.mask_mode == MASK_TILE;
    const dim3 g((unsigned) grid), b8(WAVES * 64), b4(WAVES_PAIR * 64);
    if (pl.kind == FA_VD) {
        // tiles: a packed one for up to 8 rows, a full one for up to 16, both for up to 24
        const bool msk = a.mask != nullptr;
        if (a.R <= 8)       launch_vd<0, 1>(a, msk, a.ragged != 0, gat != nullptr, g, st);
        else if (a.R <= 16) launch_vd<1, 0>(a, msk, a.ragged != 0, gat != nullptr, g, st);
        else                launch_vd<1, 1>(a, msk, a.ragged != 0, gat != nullptr, g, st);
    } else if (pl.kind == FA_VS) {
        const bool msk = a.mask != nullptr;
        if (a.R <= 8)       launch_vs<0, 1>(a, msk, a.ragged != 0, gat != nullptr, g, st);
        else if (a.R <= 16) launch_vs<1, 0>(a, msk, a.ragged != 0, gat != nullptr, g, st);
        else                launch_vs<1, 1>(a, msk, a.ragged != 0, gat != nullptr, g, st);
    } else if (pl.kind == FA_DEC) {
        const dim3 bd(DEC_WAVES * 64);
        const bool msk = a.mask != nullptr;
#define QWFN_DEC(RT_, M_, RG_) QWFN_FA_LAUNCH(g, bd, st, k_fa_dec<RT_, M_, RG_, false>)
        if (gat) {
            if (pl.RT == 1) QWFN_FA_LAUNCH(g, bd, st, k_fa_dec<1, false, false, true>);
            else            QWFN_FA_LAUNCH(g, bd, st, k_fa_dec<2, false, false, true>);
        } else if (pl.RT == 1) {
            if (a.ragged) { if (msk) QWFN_DEC(1, true, true); else QWFN_DEC(1, false, true); }
            else          { if (msk) QWFN_DEC(1, true, false); else QWFN_DEC(1, false, false); }
        } else {
            if (a.ragged) { if (msk) QWFN_DEC(2, true, true); else QWFN_DEC(2, false, true); }
            else          { if (msk) QWFN_DEC(2, true, false); else QWFN_DEC(2, false, false); }
        }
#undef QWFN_DEC
    } else if (a.ragged) {
        // per-sequence splits: the 4-wave kernels (and the 8-wave mask-tile one)
        switch (pl.kind) {
            case FA_P4_T1:
                if (mt) QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<1, true, WAVES_PAIR, 16, true>);
                else    QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<1, false, WAVES_PAIR, 16, true>);
                break;
            default:
                if (mt && mrows > MASK_ROWS_PAIR) QWFN_FA_LAUNCH(g, b8, st, k_fattn_q8_0<2, true, WAVES, 16, true>);
                else if (mt) QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<2, true, WAVES_PAIR, 32, true>);
                else    QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<2, false, WAVES_PAIR, 32, true>);
                break;
        }
    } else {
    switch (pl.kind) {
        case FA_DEC:
        case FA_PRE:
            break;
        case FA_P4_T1:
            if (mt) QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<1, true, WAVES_PAIR, 16, false>);
            else    QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<1, false, WAVES_PAIR, 16, false>);
            break;
        case FA_P4_T2:
            // mask tiles of at most MASK_ROWS_PAIR rows fit next to two stages;
            // more rows (per-head masks, small gqa) take the 8-wave kernel over
            // the same 64-key chunks
            if (mt && mrows > MASK_ROWS_PAIR) QWFN_FA_LAUNCH(g, b8, st, k_fattn_q8_0<2, true, WAVES, 16, false>);
            else if (mt) QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<2, true, WAVES_PAIR, 32, false>);
            else    QWFN_FA_LAUNCH(g, b4, st, k_fattn_q8_0<2, false, WAVES_PAIR, 32, false>);
            break;
    }
    }
    if (int rc = hip_check(hipGetLastError(), "flash_attn launch")) return rc;
    if (a.ns > 1 && !a.mctr) {
        const int64_t blocks = (int64_t) a.B * a.nh_kv * a.R * 4;
        if (blocks > 0x7fffffff) return set_error(QWFN_EINVAL, "flash_attn_ext: merge grid too large");
        if (a.ragged) hipLaunchKernelGGL(k_fattn_merge<true>, dim3((unsigned) blocks), dim3(256), 0, st, a);
        else          hipLaunchKernelGGL(k_fattn_merge<false>, dim3((unsigned) blocks), dim3(256), 0, st, a);
        if (int rc = hip_check(hipGetLastError(), "flash_attn merge launch")) return rc;
    }
    return QWFN_OK;
}

}  // namespace

extern "C" int qwfn_flash_attn_ext_q8_0(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                        const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                        const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                        void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0", [&]() -> int {
        return fattn_run(q, k, v, mask, scale, max_bias, logit_softcap, dst, variant, ws, ws_bytes, stream, nullptr);
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_noalloc(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                                const qwfn_tensor * mask, float scale, float max_bias,
                                                float logit_softcap, const qwfn_tensor * dst, int variant, void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_noalloc", [&]() -> int {
        return fattn_run(q, k, v, mask, scale, max_bias, logit_softcap, dst, variant, nullptr, 0, stream, nullptr, nullptr,
                         WS_SCRATCH);
    });
}

namespace {
// Checks of a gathered call; kk / vv get the longest list's length as their key count.
int gather_args(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v, const int32_t * cells,
                const int64_t * n_cells, int64_t cell_stride, int64_t pos0, qwfn_tensor * kk, qwfn_tensor * vv,
                fa_gather * g) {
    if (!q || !k || !v || !cells || !n_cells) return set_error(QWFN_EINVAL, "flash_attn_ext_cells: NULL argument");
    if (!is_aligned(cells, 16)) return set_error(QWFN_EALIGN, "flash_attn_ext_cells: cells must be 16-byte aligned");
    if (k->ne[2] < 1 || k->ne[2] > GATHER_MAX_HEADS)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext_cells: 1 to 8 KV heads");
    if (q->ne[3] != 1 || k->ne[3] != 1 || v->ne[3] != 1) return set_error(QWFN_ENOTSUP, "flash_attn_ext_cells: one sequence (B = 1)");
    if (cell_stride < 0 || cell_stride % 4)
        return set_error(QWFN_EALIGN, "flash_attn_ext_cells: cell_stride must be 0 (one shared list) or a positive multiple of 4");
    if (pos0 < 0) return set_error(QWFN_EINVAL, "flash_attn_ext_cells: negative pos0");
    if (k->ne[1] != v->ne[1]) return set_error(QWFN_EINVAL, "flash_attn_ext_cells: k and v must have the same rows");
    if ((uint64_t) k->ne[1] * std::max(k->nb[1], v->nb[1]) >= (uint64_t(1) << 31))
        return set_error(QWFN_ENOTSUP, "flash_attn_ext_cells: the cache must be below 2 GiB (rows * row stride)");
    int64_t mx = 0;
    for (int64_t h = 0; h < k->ne[2]; h++) {
        if (n_cells[h] < 0 || (cell_stride > 0 && n_cells[h] > cell_stride))
            return set_error(QWFN_ERANGE, "flash_attn_ext_cells: each head's cell count must lie in [0, cell_stride]");
        mx = std::max(mx, n_cells[h]);
    }
    *kk = *k;
    *vv = *v;
    kk->ne[1] = vv->ne[1] = mx;
    *g = fa_gather{cells, n_cells, cell_stride, pos0, k->ne[1]};
    return QWFN_OK;
}
}  // namespace

extern "C" size_t qwfn_fattn_workspace_size_cells(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                                  const int64_t * n_cells, int64_t cell_stride) {
    return ::qwfn::abi_value<size_t>("fattn_workspace_size_cells", 0, [&]() -> size_t {
        qwfn_tensor kk, vv;
        fa_gather g{};
        static const int32_t dummy[4] = {0, 0, 0, 0};
        if (gather_args(q, k, v, dummy, n_cells, cell_stride, 0, &kk, &vv, &g)) return 0;
        fa_plan pl{};
        if (plan_fattn(q, &kk, &vv, nullptr, &pl, nullptr, MAX_SPLITS, true)) return 0;
        return pl.ws_bytes;
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_cells(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                              const int32_t * cells, const int64_t * n_cells, int64_t cell_stride,
                                              int64_t pos0, float scale, const qwfn_tensor * dst, int variant, void * ws,
                                              size_t ws_bytes, void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_cells", [&]() -> int {
        qwfn_tensor kk, vv;
        fa_gather g{};
        if (int rc = gather_args(q, k, v, cells, n_cells, cell_stride, pos0, &kk, &vv, &g)) return rc;
        return fattn_run(q, &kk, &vv, nullptr, scale, 0.0f, 0.0f, dst, variant, ws, ws_bytes, stream, nullptr, nullptr,
                         WS_CALLER, &g);
    });
}

namespace {
// Checks of a call with one cell list per query position, and the views that
// present position t as sequence t of one query: q [256, 1, n_head, T], dst
// and gate [256, n_head, 1, T] over the same memory; kk / vv get the longest
// list's length as their key count.
int query_cells_args(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v, const int32_t * cells,
                     const int64_t * n_cells, int64_t cell_stride, int64_t pos0, const qwfn_tensor * dst,
                     const qwfn_tensor * gate, qwfn_tensor * qq, qwfn_tensor * kk, qwfn_tensor * vv, qwfn_tensor * dd,
                     qwfn_tensor * gg, fa_gather * g) {
    if (!q || !k || !v || !cells || !n_cells) return set_error(QWFN_EINVAL, "flash_attn_ext_query_cells: NULL argument");
    if (!is_aligned(cells, 16)) return set_error(QWFN_EALIGN, "flash_attn_ext_query_cells: cells must be 16-byte aligned");
    if (k->ne[2] < 1 || k->ne[2] > GATHER_MAX_HEADS)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext_query_cells: 1 to 8 KV heads");
    if (q->ne[3] != 1 || k->ne[3] != 1 || v->ne[3] != 1)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext_query_cells: one sequence (q, k and v with ne[3] = 1)");
    const int64_t T = q->ne[1];
    if (T < 1 || T * k->ne[2] > GATHER_MAX_LISTS)
        return set_error(QWFN_ENOTSUP, "flash_attn_ext_query_cells: T * n_head_kv must lie in [1, 32]");
    if (cell_stride < 0 || cell_stride % 4)
        return set_error(QWFN_EALIGN, "flash_attn_ext_query_cells: cell_stride must be 0 (one list for every position) or a positive multiple of 4");
    if (pos0 < 0) return set_error(QWFN_EINVAL, "flash_attn_ext_query_cells: negative pos0");
    if (k->ne[1] != v->ne[1]) return set_error(QWFN_EINVAL, "flash_attn_ext_query_cells: k and v must have the same rows");
    if ((uint64_t) k->ne[1] * std::max(k->nb[1], v->nb[1]) >= (uint64_t(1) << 31))
        return set_error(QWFN_ENOTSUP, "flash_attn_ext_query_cells: the cache must be below 2 GiB (rows * row stride)");
    int64_t mx = 0;
    for (int64_t t = 0; t < T; t++) {
        if (n_cells[t] < 0 || (cell_stride > 0 && n_cells[t] > cell_stride))
            return set_error(QWFN_ERANGE, "flash_attn_ext_query_cells: each position's cell count must lie in [0, cell_stride]");
        mx = std::max(mx, n_cells[t]);
    }
    if (!dst || dst->ne[0] != D || dst->ne[1] != q->ne[2] || dst->ne[2] != T || dst->ne[3] != 1 || dst->nb[0] != 4 ||
        dst->nb[1] != (size_t) D * 4 || dst->nb[2] != dst->nb[1] * (size_t) dst->ne[1])
        return set_error(QWFN_EINVAL, "flash_attn_ext_query_cells: dst must be contiguous f32 [256, n_head, T, 1]");
    *qq = *q;
    qq->ne[1] = 1; qq->ne[3] = T; qq->nb[3] = q->nb[1];
    *kk = *k;
    *vv = *v;
    kk->ne[1] = vv->ne[1] = mx;
    *dd = *dst;
    dd->ne[2] = 1; dd->ne[3] = T; dd->nb[3] = dst->nb[2];
    if (gate) {
        *gg = *gate;
        if (gate->ne[2] != T || gate->ne[3] != 1 || gate->nb[2] != dst->nb[2])
            return set_error(QWFN_EINVAL, "flash_attn_ext_query_cells: gate must have dst's shape and strides");
        gg->ne[2] = 1; gg->ne[3] = T; gg->nb[3] = gate->nb[2];
    }
    *g = fa_gather{cells, n_cells, cell_stride, pos0, k->ne[1], true};
    return QWFN_OK;
}
}  // namespace

extern "C" size_t qwfn_fattn_workspace_size_query_cells(const qwfn_tensor * q, const qwfn_tensor * k,
                                                        const qwfn_tensor * v, const int64_t * n_cells,
                                                        int64_t cell_stride) {
    return ::qwfn::abi_value<size_t>("fattn_workspace_size_query_cells", 0, [&]() -> size_t {
        if (!q) return 0;
        qwfn_tensor qq, kk, vv, dd, gg;
        fa_gather g{};
        static const int32_t dummy[4] = {0, 0, 0, 0};
        qwfn_tensor dst = *q;   // a contiguous [256, n_head, T, 1] stand-in: only the plan is wanted
        dst.type = QWFN_TYPE_F32;
        dst.ne[0] = D; dst.ne[1] = q->ne[2]; dst.ne[2] = q->ne[1]; dst.ne[3] = 1;
        dst.nb[0] = 4; dst.nb[1] = (size_t) D * 4; dst.nb[2] = dst.nb[1] * (size_t) dst.ne[1]; dst.nb[3] = dst.nb[2] * (size_t) dst.ne[2];
        if (query_cells_args(q, k, v, dummy, n_cells, cell_stride, 0, &dst, nullptr, &qq, &kk, &vv, &dd, &gg, &g))
            return 0;
        fa_plan pl{};
        if (plan_fattn(&qq, &kk, &vv, nullptr, &pl, nullptr, MAX_SPLITS, true)) return 0;
        return pl.ws_bytes;
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_query_cells(const qwfn_tensor * q, const qwfn_tensor * k,
                                                    const qwfn_tensor * v, const int32_t * cells,
                                                    const int64_t * n_cells, int64_t cell_stride, int64_t pos0,
                                                    float scale, const qwfn_tensor * gate, const qwfn_tensor * dst,
                                                    int variant, void * ws, size_t ws_bytes, void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_query_cells", [&]() -> int {
        qwfn_tensor qq, kk, vv, dd, gg;
        fa_gather g{};
        if (int rc = query_cells_args(q, k, v, cells, n_cells, cell_stride, pos0, dst, gate, &qq, &kk, &vv, &dd, &gg, &g))
            return rc;
        return fattn_run(&qq, &kk, &vv, nullptr, scale, 0.0f, 0.0f, &dd, variant, ws, ws_bytes, stream, nullptr, nullptr,
                         WS_CALLER, &g, gate ? &gg : nullptr);
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_query_cells_dev(const qwfn_tensor * q, const qwfn_tensor * k,
                                                        const qwfn_tensor * v, const int32_t * cells,
                                                        const int32_t * counts, int64_t cell_stride, int64_t pos0,
                                                        float scale, const qwfn_tensor * gate, const qwfn_tensor * dst,
                                                        int variant, void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_query_cells_dev", [&]() -> int {
        const char * fn = "flash_attn_ext_query_cells_dev: ";
        auto fail = [&](int code, const char * what) { return set_error(code, std::string(fn) + what); };
        if (!q || !k || !v || !cells || !counts || !dst) return fail(QWFN_EINVAL, "NULL argument");
        if (q->type != QWFN_TYPE_F32 || q->ne[0] != D || q->nb[0] != 4) return fail(QWFN_EINVAL, "q must be F32 [256, T, n_head, 1]");
        if (k->type != QWFN_TYPE_Q8_0 || v->type != QWFN_TYPE_Q8_0) return fail(QWFN_ENOTSUP, "k and v must be q8_0");
        if (k->ne[0] != D || v->ne[0] != D || k->nb[0] != QBLOCK || v->nb[0] != QBLOCK)
            return fail(QWFN_ENOTSUP, "k and v rows must be 256 q8_0 values");
        if (q->ne[3] != 1 || k->ne[3] != 1 || v->ne[3] != 1) return fail(QWFN_ENOTSUP, "one sequence (ne[3] = 1)");
        if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2]) return fail(QWFN_EINVAL, "k and v must have the same rows and KV heads");
        const int64_t T = q->ne[1], nh = q->ne[2], nh_kv = k->ne[2], n_rows = k->ne[1];
        if (T < 1 || nh < 1 || nh_kv < 1 || n_rows < 1) return fail(QWFN_EINVAL, "empty q or cache");
        if (nh % nh_kv || nh / nh_kv > 16) return fail(QWFN_ENOTSUP, "n_head must be a multiple of n_head_kv, at most 16 times it");
        if (T > INT32_MAX / 2) return fail(QWFN_ENOTSUP, "too many positions");
        if (!is_aligned(q->data, 16) || q->nb[1] % 16 || q->nb[2] % 16)
            return fail(QWFN_EALIGN, "q data and strides must be 16-byte aligned");
        const uint64_t q_bytes = (uint64_t) (T - 1) * q->nb[1] + (uint64_t) (nh - 1) * q->nb[2] + (uint64_t) D * 4;
        if (q_bytes >= (uint64_t(1) << 32)) return fail(QWFN_ENOTSUP, "q must span below 4 GiB");
        if (!is_aligned(k->data, 16) || !is_aligned(v->data, 16) || k->nb[1] % 16 || v->nb[1] % 16 || k->nb[2] % 16 ||
            v->nb[2] % 16)
            return fail(QWFN_EALIGN, "k/v data and strides must be 16-byte aligned");
        if ((uint64_t) (nh_kv - 1) * k->nb[2] + SEG > k->nb[1] || (uint64_t) (nh_kv - 1) * v->nb[2] + SEG > v->nb[1])
            return fail(QWFN_EINVAL, "the KV heads must lie within a cache row");
        if ((uint64_t) n_rows * std::max(k->nb[1], v->nb[1]) >= (uint64_t(1) << 31))
            return fail(QWFN_ENOTSUP, "the cache must be below 2 GiB (rows * row stride)");
        if (!is_aligned(cells, 16) || cell_stride < 4 || cell_stride % 4 || cell_stride > (int64_t(1) << 28))
            return fail(QWFN_EALIGN, "cells must be 16-byte aligned rows of cell_stride int32, a positive multiple of 4");
        if (!is_aligned(counts, 4)) return fail(QWFN_EALIGN, "counts must be int32");
        if (pos0 < 0) return fail(QWFN_EINVAL, "negative pos0");
        if (dst->type != QWFN_TYPE_F32 || dst->ne[0] != D || dst->ne[1] != nh || dst->ne[2] != T || dst->ne[3] != 1 ||
            dst->nb[0] != 4 || dst->nb[1] != (size_t) D * 4 || dst->nb[2] != dst->nb[1] * (size_t) nh || !is_aligned(dst->data, 16))
            return fail(QWFN_EINVAL, "dst must be contiguous 16-byte aligned F32 [256, n_head, T, 1]");
        if (gate && (gate->type != QWFN_TYPE_F32 || gate->ne[0] != D || gate->ne[1] != nh || gate->ne[2] != T ||
                     gate->nb[0] != 4 || gate->nb[1] != dst->nb[1] || gate->nb[2] != dst->nb[2] || !is_aligned(gate->data, 16)))
            return fail(QWFN_EINVAL, "gate must have dst's shape and strides, 16-byte aligned");
        if (int rc = check_no_scratch()) return rc;
        qc_args a{};
        a.q = (const char *) q->data; a.q_nb1 = (uint32_t) q->nb[1]; a.q_nb2 = (uint32_t) q->nb[2];
        a.q_bytes = (uint32_t) q_bytes;
        a.k = (const char *) k->data; a.v = (const char *) v->data;
        a.k_nb1 = (uint32_t) k->nb[1]; a.v_nb1 = (uint32_t) v->nb[1];
        a.k_nb2 = (uint32_t) k->nb[2]; a.v_nb2 = (uint32_t) v->nb[2];
        a.k_bytes = (uint32_t) ((uint64_t) n_rows * k->nb[1]); a.v_bytes = (uint32_t) ((uint64_t) n_rows * v->nb[1]);
        a.n_rows = n_rows;
        a.cells = cells; a.cell_stride = cell_stride; a.counts = counts; a.pos0 = pos0;
        a.T = (int32_t) T; a.nh = (int32_t) nh; a.nh_kv = (int32_t) nh_kv; a.gqa = (int32_t) (nh / nh_kv);
        a.scale_log2 = scale * LOG2E;
        a.x86 = variant == QWFN_Q8_X86;
        a.dst = (float *) dst->data;
        a.gate = gate ? (const float *) gate->data : nullptr;
        if (int rc = status_word(&a.status)) return rc;
        // waves per list: the (position, KV head) lists over about 256 blocks
        // of 8 waves (one a CU), at least 2 waves a list
        const int64_t lists = T * nh_kv;
        const int kg = lists >= 1024 ? 2 : lists >= 512 ? 4 : 8;
        const int64_t upb = QC_WAVES / kg;
        const int64_t blocks = (T + upb - 1) / upb * nh_kv;
        if (blocks > INT32_MAX) return fail(QWFN_ENOTSUP, "too many positions");
        auto kern = kg == 2 ? k_fa_qc<2> : kg == 4 ? k_fa_qc<4> : k_fa_qc<8>;
        hipLaunchKernelGGL(kern, dim3((unsigned) blocks), dim3(QC_WAVES * 64), 0, as_stream(stream), a);
        return hip_check(hipGetLastError(), "flash_attn_ext_query_cells_dev launch");
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_gated(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                              const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                              const qwfn_tensor * dst, const qwfn_tensor * gate, int variant, void * ws,
                                              size_t ws_bytes, void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_gated", [&]() -> int {
        if (!gate) return set_error(QWFN_EINVAL, "flash_attn_ext_gated: NULL gate");
        return fattn_run(q, k, v, mask, scale, max_bias, logit_softcap, dst, variant, ws, ws_bytes, stream, nullptr,
                         nullptr, WS_CALLER, nullptr, gate);
    });
}

extern "C" size_t qwfn_fattn_workspace_size_seq(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                                const qwfn_tensor * mask, const int64_t * seq_n_kv) {
    return ::qwfn::abi_value<size_t>("fattn_workspace_size_seq", 0, [&]() -> size_t {
        fa_plan pl{};
        if (!seq_n_kv || plan_fattn(q, k, v, mask, &pl, seq_n_kv)) return 0;
        return pl.ws_bytes;
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_seq(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                            const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                            const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                            const int64_t * seq_n_kv, void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_seq", [&]() -> int {
        if (!seq_n_kv) return set_error(QWFN_EINVAL, "flash_attn_ext_seq: seq_n_kv is NULL");
        return fattn_run(q, k, v, mask, scale, max_bias, logit_softcap, dst, variant, ws, ws_bytes, stream, nullptr, seq_n_kv);
    });
}

extern "C" int qwfn_flash_attn_ext_q8_0_append(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                               const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                               const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                               const qwfn_tensor * src_k, const qwfn_tensor * src_v, int64_t first_row,
                                               void * stream) {
    return ::qwfn::abi_call("flash_attn_ext_q8_0_append", [&]() -> int {
        const fa_append app{src_k, src_v, first_row};
        return fattn_run(q, k, v, mask, scale, max_bias, logit_softcap, dst, variant, ws, ws_bytes, stream, &app);
    });
}

extern "C" void qwfn_fattn_force_splits(int32_t n_splits) {
    g_force_splits.store(n_splits > 0 ? std::min<int32_t>(n_splits, MAX_SPLITS) : 0, std::memory_order_relaxed);
}

extern "C" void qwfn_fattn_force_kernel(int32_t kind) {
    g_force_kernel.store(kind >= QWFN_FA_KERNEL_AUTO && kind <= QWFN_FA_KERNEL_VS ? kind : QWFN_FA_KERNEL_AUTO,
                         std::memory_order_relaxed);
}

extern "C" const char * qwfn_fattn_last_kernel(void) {
    return g_last_kernel;
}

extern "C" void qwfn_fattn_force_merge(int32_t mode) {
    g_force_merge.store(mode == QWFN_FA_MERGE_FUSED || mode == QWFN_FA_MERGE_KERNEL ? mode : QWFN_FA_MERGE_AUTO,
                        std::memory_order_relaxed);
}

extern "C" int32_t qwfn_fattn_last_merge(void) {
    return g_last_merge;
}
