/*
 * qwfn_kv.h -- C ABI of the MI355X (gfx950) q8_0 KV-cache path.
 *
 * This library replaces, behind a plain C boundary, the device work that the
 * reference engine (thomaskleiven/QwFN-hybrid) hands to ggml-cuda for its
 * attention layers:
 *
 *   ggml_cpy      F32 -> Q8_0   cache append at n_past      qwfn_graph.cpp:376-383, :916-921
 *   ggml_set_rows F32 -> Q8_0   decode append at write_idx  qwfn_graph.cpp:623-624
 *   ggml_get_rows on I32 words  raw gather of cache rows    qwfn_graph.cpp:638-645
 *   ggml_flash_attn_ext         decode / verify / prefill   qwfn_graph.cpp:469-471, :698-699
 *   ggml_backend_tensor_set/copy snapshot restore           qwfn_engine.cpp:1029-1053
 *
 * Conventions
 *   - Tensors are described ggml-style: ne[4] element counts, nb[4] byte
 *     strides, a type code using ggml's numbering, and a device address. For
 *     Q8_0, ne[0] counts values (a multiple of 32) and nb[0] is 34, one block
 *     { fp16 d; int8 qs[32]; }.
 *   - Every entry point returns QWFN_OK (0) or a negative QWFN_E* code and sets
 *     a thread-local message readable with qwfn_last_error(). No exception
 *     crosses the boundary.
 *   - Shapes, strides, alignment and host-visible index ranges are validated on
 *     the host BEFORE anything is launched, so an invalid call never touches
 *     the GPU. Indices that live in device memory are bounds-checked by the
 *     kernels: an out-of-range index is skipped (never dereferenced) and raises
 *     a device flag read by qwfn_device_status().
 *   - The caller owns all memory. Calls are stream-ordered and asynchronous on
 *     the given stream (a hipStream_t passed as void*; NULL is the null stream).
 */
#ifndef QWFN_KV_H
#define QWFN_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWFN_KV_ABI_VERSION 2

/* ggml type numbering (ggml.h: GGML_TYPE_F32 = 0, F16 = 1, Q8_0 = 8, I32 = 26) */
enum qwfn_type {
    QWFN_TYPE_F32  = 0,
    QWFN_TYPE_F16  = 1,
    QWFN_TYPE_Q8_0 = 8,
    QWFN_TYPE_I32  = 26,
    QWFN_TYPE_BF16 = 30,
};

enum qwfn_status {
    QWFN_OK      =  0,
    QWFN_EINVAL  = -1,  /* bad argument, shape or type            */
    QWFN_ERANGE  = -2,  /* index or row outside the tensor        */
    QWFN_EALIGN  = -3,  /* misaligned address, stride or row size */
    QWFN_ENOTSUP = -4,  /* valid in ggml, not supported here      */
    QWFN_EDEVICE = -5,  /* HIP runtime error                      */
    QWFN_ENOMEM  = -6,  /* allocation failure / workspace too small */
    QWFN_ESIZE   = -7,  /* snapshot part count or size mismatch   */
};

/* q8_0 quantiser rounding variant (ggml-cpu has two; they differ on ties and
 * on 1-ulp differences of the inverse scale):
 *   QWFN_Q8_X86 : quantize_row_q8_0 x86 AVX/AVX2 path: id = 127/amax, round half to even
 *   QWFN_Q8_REF : quantize_row_q8_0_ref:               id = 1/(amax/127), round half away from 0 */
enum qwfn_q8_variant { QWFN_Q8_REF = 0, QWFN_Q8_X86 = 1 };

typedef struct qwfn_tensor {
    void *   data;   /* device address of element [0,0,0,0]  */
    int32_t  type;   /* enum qwfn_type                       */
    int32_t  pad_;
    int64_t  ne[4];  /* elements per dimension               */
    size_t   nb[4];  /* byte stride per dimension            */
} qwfn_tensor;

/* ----------------------------------------------------------------- runtime */

int          qwfn_abi_version(void);
const char * qwfn_last_error(void);
/* Make `device` current for this thread and create the per-device status word. */
int          qwfn_init(int device);
/* Synchronise `stream`, then read and clear the device-side error flags
 * (bit 0: set_rows index out of range; bit 1: get_rows index out of range). */
int          qwfn_device_status(void * stream, uint32_t * flags);

/* ------------------------------------------------------------ cache append */

/* ggml_set_rows(dst, src, idx): dst Q8_0 [ne0, n_rows] (row stride nb[1]),
 * src F32 [ne0, n] (nb[0] == 4), idx I32 [n] in device memory. Row i of src is
 * quantised into row idx[i] of dst. Replaces qwfn_graph.cpp:623-624
 * (qsa_dec_kv_write) and the MTP head's decode append. */
int qwfn_set_rows_q8_0(const qwfn_tensor * dst, const qwfn_tensor * src, const qwfn_tensor * idx,
                       int variant, void * stream);

/* ggml_cpy(src, dst): src F32 [ne0, n], dst Q8_0 [ne0, n] (a view whose rows
 * start at the append position). Replaces qwfn_graph.cpp:376-383 (kv_append)
 * and :916-921 (mtp_head_kv). */
int qwfn_cpy_f32_q8_0(const qwfn_tensor * src, const qwfn_tensor * dst, int variant, void * stream);

/* The K and the V append of one layer in one launch: the two adjacent
 * ggml_set_rows nodes with the same idx at qwfn_graph.cpp:623-624
 * (qsa_dec_kv_write), or the two adjacent ggml_cpy nodes at :376-383
 * (kv_append) and :916-921 (mtp_head_kv). Each pair is checked as two calls of
 * the single-tensor entry point would be, and src_k and src_v must have the
 * same shape; the result is byte-identical to those two calls. */
int qwfn_set_rows_q8_0_kv(const qwfn_tensor * dst_k, const qwfn_tensor * src_k, const qwfn_tensor * dst_v,
                          const qwfn_tensor * src_v, const qwfn_tensor * idx, int variant, void * stream);
int qwfn_cpy_f32_q8_0_kv(const qwfn_tensor * src_k, const qwfn_tensor * dst_k, const qwfn_tensor * src_v,
                         const qwfn_tensor * dst_v, int variant, void * stream);

/* -------------------------------------------------------------- gather */

/* ggml_get_rows(src, idx) on I32 words: src I32 [ne0, n_rows], idx I32 [n]
 * (device), dst I32 [ne0, n]. Copies raw cache bytes, no dequantisation.
 * Replaces qwfn_graph.cpp:638-645 (qsa_gather, raw branch). */
int qwfn_get_rows_i32(const qwfn_tensor * src, const qwfn_tensor * idx, const qwfn_tensor * dst,
                      void * stream);

/* Per-segment gather for per-KV-head selections: for each segment s in
 * [0, n_seg) and i in [0, n_idx), copy seg_bytes bytes starting at byte
 * seg_off + s*seg_stride of row idx[s*n_idx + i] of src into
 * dst + s*dst_seg_stride + i*dst_row_stride. idx is device memory.
 * seg_bytes, offsets and strides must be multiples of 4. No ggml counterpart:
 * it is the reference's raw get_rows (qwfn_graph.cpp:638-645) applied per KV
 * head instead of once for both heads. */
int qwfn_kv_gather_segments(const void * src, size_t src_row_stride, int64_t src_rows,
                            size_t seg_off, size_t seg_stride, size_t seg_bytes, int32_t n_seg,
                            const int32_t * idx, int64_t n_idx,
                            void * dst, size_t dst_row_stride, size_t dst_seg_stride, void * stream);

/* qwfn_kv_gather_segments of the K cache into dst_k and of the V cache into
 * dst_v with the same indices and geometry, in one launch: the reference's
 * qsa_gather gathers K and V with the same index (qwfn_graph.cpp:632-645),
 * two get_rows; the same bytes as the two calls. dst_k and dst_v must not
 * overlap. */
int qwfn_kv_gather_segments_kv(const void * src_k, const void * src_v, size_t src_row_stride, int64_t src_rows,
                               size_t seg_off, size_t seg_stride, size_t seg_bytes, int32_t n_seg,
                               const int32_t * idx, int64_t n_idx, void * dst_k, void * dst_v,
                               size_t dst_row_stride, size_t dst_seg_stride, void * stream);

/* ------------------------------------------------------- flash attention */

/* ggml_flash_attn_ext(q, k, v, mask, scale, max_bias, logit_softcap) with F32
 * accumulation (ggml_prec_set_acc(.., GGML_PREC_F32), qwfn_graph.cpp:471, :699):
 *   q    F32  [D, T, n_head, B]          (nb[0] == 4; any other strides)
 *   k, v Q8_0 [D, n_kv, n_head_kv, B|1] (nb[0] == 34; nb[1] row, nb[2] head stride)
 *   mask F16  [n_kv', T', mh, mb] or NULL; n_kv' >= n_kv, T' >= T,
 *             n_head % mh == 0, B % mb == 0 (broadcast as in ggml)
 *   dst  F32  [D, n_head, T, B] contiguous
 * D must be 256 (the model's head size). n_head % n_head_kv == 0.
 * max_bias and logit_softcap must be 0 (the reference never sets them).
 * Semantics follow ggml-cpu's q8_0 path: Q is requantised to q8_0 with
 * `variant`, scores are sum_b d_k*d_q*isum_b, masked (-inf) keys are skipped,
 * softmax is online, V is dequantised q*d. A fully masked row gives 0.
 * ws: device workspace of at least qwfn_fattn_workspace_size(q, k, v, mask)
 * bytes, or NULL to use a library-owned buffer: one per device, allocated on
 * first use and regrown (after a device synchronisation) when a call needs
 * more. ws == NULL returns QWFN_EINVAL while `stream` is being captured into
 * a graph, and every ws == NULL call on a device shares that one buffer, so
 * such calls must not overlap (serialise them on one stream). The workspace
 * holds the split partials when the keys are split across workgroups (at
 * least 256 bytes are asked for otherwise); its contents need not be
 * preserved between calls. Calls that run at the same time need distinct
 * workspaces. */
size_t qwfn_fattn_workspace_size(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                 const qwfn_tensor * mask);
int qwfn_flash_attn_ext_q8_0(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                             const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                             const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes, void * stream);

/* qwfn_flash_attn_ext_q8_0 without a workspace argument and without any
 * device allocation: no counterpart in the reference; for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The split partials go to a 16 MiB scratch array inside the
 * library's code object (one per GPU, held until the process ends); when a
 * call's partials would not fit, it uses fewer key splits (the result then
 * differs from qwfn_flash_attn_ext_q8_0's only by float rounding). Every call on
 * a GPU shares that GPU's scratch: calls that overlap on one GPU (two streams,
 * or two threads) race and give wrong results. */
int qwfn_flash_attn_ext_q8_0_noalloc(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                     const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                     const qwfn_tensor * dst, int variant, void * stream);

/* Force the key-split count of later attention calls in this process (any
 * thread; 0 returns to the planner's choice, values are capped at 1024). For
 * split-invariance tests and tuning sweeps; the results do not depend on it
 * beyond float rounding. No counterpart in the reference (ggml picks its own
 * partition). */
void qwfn_fattn_force_splits(int32_t n_splits);

/* Force the attention kernel family of later calls in this process (any
 * thread): QWFN_FA_KERNEL_AUTO returns to the planner's choice. A call whose
 * shape the forced family cannot take returns QWFN_ENOTSUP. For parity tests
 * that reach every kernel family on the same inputs, and for A/B timing; the
 * results do not depend on it beyond float rounding. No counterpart in the
 * reference (ggml picks its own kernel).
 *   VD:      at most 24 query rows per KV head, a mask shared by the heads
 *            over at most 4 query positions (or none)
 *   DEC:     at most 32 query rows per KV head
 *   GENERAL: any shape but gathered cells
 *   PRE:     more than 32 query rows per KV head, a mask shared by the heads
 *            (or none), n_head / n_head_kv >= 4, one batch, no cells
 *   VS:      the shapes of VD (the value dims split across the waves) */
enum {
    QWFN_FA_KERNEL_AUTO    = 0,
    QWFN_FA_KERNEL_VD      = 1,
    QWFN_FA_KERNEL_DEC     = 2,
    QWFN_FA_KERNEL_GENERAL = 3,
    QWFN_FA_KERNEL_PRE     = 4,
    QWFN_FA_KERNEL_VS      = 5
};
void qwfn_fattn_force_kernel(int32_t kind);

/* The attention kernel that the calling thread's last attention call launched,
 * as its template instantiation ("k_fa_vd<1, 1, true, false, false>"), or ""
 * before the first launch; the string lives as long as the library. For the
 * tests that check that every kernel instantiation is reached. No counterpart
 * in the reference. */
const char * qwfn_fattn_last_kernel(void);

/* Force how later calls merge their key splits (any thread): AUTO lets the
 * planner choose (today the merge launch, which measures faster), FUSED
 * merges inside k_fa_dec / k_fa_vd (the last blocks of each (batch, KV head)
 * to finish fold all of its splits; other kernels, and batches of several
 * depths, still use a merge launch), KERNEL always launches the separate
 * merge kernel. qwfn_fattn_last_merge reports what the
 * calling thread's last attention call did (NONE: one split, nothing to
 * merge). For parity tests of both merge paths and for A/B timing; results
 * do not depend on it beyond float rounding. No counterpart in the reference
 * (ggml's CPU kernel keeps one partial per thread chunk). */
enum {
    QWFN_FA_MERGE_AUTO   = 0,
    QWFN_FA_MERGE_FUSED  = 1,
    QWFN_FA_MERGE_KERNEL = 2,
    QWFN_FA_MERGE_NONE   = 3
};
void    qwfn_fattn_force_merge(int32_t mode);
int32_t qwfn_fattn_last_merge(void);

/* Batched decode over sequences of different depths: as
 * qwfn_flash_attn_ext_q8_0, except that sequence b (q batch index) attends
 * only keys [0, seq_n_kv[b]) -- the same result as masking its later keys with
 * -inf, which is how a mask-only call expresses ragged batches (a [n_kv, 1,
 * 1, B] mask of 0 then -inf). seq_n_kv is a host array of B counts in
 * [0, n_kv], B <= 16. The keys are split per sequence in proportion to its
 * count, so every workgroup streams about the same number of chunks and no
 * workgroup reads keys past its sequence's end. A mask, if given, still
 * applies. Size ws with qwfn_fattn_workspace_size_seq. */
size_t qwfn_fattn_workspace_size_seq(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                     const qwfn_tensor * mask, const int64_t * seq_n_kv);
int qwfn_flash_attn_ext_q8_0_seq(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                 const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                 const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                 const int64_t * seq_n_kv, void * stream);

/* Sparse decode attention over selected cache cells, the gather fused into
 * the attention: replaces the raw get_rows of the selected cells' K and V
 * words (qsa_gather, qwfn_graph.cpp:632-645), the cell mask
 * (:668-675, padding :688-693) and the ggml_flash_attn_ext over the gathered
 * copy (:694-699). The rows are read straight from the cache; nothing is
 * materialised.
 *
 * k, v: the q8_0 cache views [256, n_rows, n_head_kv, 1] (nb1 = the cache row
 * stride, nb2 = the head offset), n_rows * row stride < 2 GiB, 1 <= n_head_kv
 * <= 8. cells: device int32, 16-byte aligned; KV head h attends the rows
 * cells[h * cell_stride + j], j < n_cells[h] (n_cells: host array of
 * n_head_kv counts). cell_stride = 0 gives every head the same list, the
 * reference's one list shared by both KV heads; otherwise it is a multiple of
 * 4 and at least every count. Query t (q [256, T, n_head, 1], T * n_head /
 * n_head_kv <= 32) sees a cell only if the cell is at most pos0 + t (cells are
 * positions, qwfn_engine.cpp:682). A cell outside [0, n_rows) is masked and
 * sets bit 1 (get_rows index) of qwfn_device_status. Lists may repeat
 * cells (each copy counts, as ggml's attention over a gathered copy counts
 * it) and need no padding. A query row that sees no cell is 0. Size ws with
 * qwfn_fattn_workspace_size_cells (ws NULL: the library's buffer). */
size_t qwfn_fattn_workspace_size_cells(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                       const int64_t * n_cells, int64_t cell_stride);
int qwfn_flash_attn_ext_q8_0_cells(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                   const int32_t * cells, const int64_t * n_cells, int64_t cell_stride, int64_t pos0,
                                   float scale, const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                   void * stream);

/* The attention of the reference's default verify step (QSA on), one list of
 * cells per query position: engine::attn_decode (qwfn_engine.cpp:2259-2280)
 * chains T sparse_attn_decode calls, and call k attends the k_blocks * ratio
 * cells its own top-k selected (qwfn_graph.cpp:653-705) through a raw gather
 * of whole cache rows (both KV heads read the same list, :694-699), masked to
 * cells at most the query's position (:668-675), scaled by 1/sqrt(256), and
 * multiplies the result by sigmoid(gate) (:701). Here all T positions run in
 * one launch and one merge: query t (position pos0 + t) attends cache rows
 * cells[t * cell_stride + j], j < n_cells[t] (n_cells: host array of T
 * counts), those at most pos0 + t; cell_stride = 0 gives every position the
 * same list. Lists may repeat cells and need no padding (the reference pads
 * to a multiple of 256 with masked duplicates, which add nothing). q: F32
 * [256, T, n_head, 1]; k, v: the q8_0 cache views [256, n_rows, n_head_kv, 1]
 * (nb1 the row stride, nb2 the head offset), n_rows * row stride < 2 GiB,
 * T * n_head_kv <= 32; cells: device int32, 16-byte aligned, cell_stride a
 * multiple of 4 and at least every count; dst: contiguous F32 [256, n_head,
 * T, 1]; gate: NULL or F32 of dst's shape and strides (then dst = attention *
 * sigmoid(gate), both 16-byte aligned). A cell outside [0, n_rows) is masked
 * and sets bit 1 of qwfn_device_status; a query that sees no cell gets 0.
 * Size ws with qwfn_fattn_workspace_size_query_cells (ws NULL: the library's
 * buffer). */
/* Many query positions, each over its own cell list, the list lengths on
 * the device: the attention of the reference's QSA-on prefill chunk
 * (ggml_flash_attn_ext over the selection mask, qwfn_graph.cpp:466-471)
 * given the keys each query sees as lists (qwfn_qsa_visible_cells), and, with
 * gate, the ggml_mul by sigmoid(gate) after it (:474). Query t (position
 * pos0 + t) attends cache rows cells[t * cell_stride + j], j < counts[t]
 * (counts: device int32 [T]), those at most pos0 + t, scaled by `scale`; a
 * cell outside [0, n_rows) is masked and sets bit 1 of qwfn_device_status, a
 * count outside [0, cell_stride] is clipped to it and sets the same bit, and a
 * query that sees no cell gets 0. Lists may repeat cells (each copy counts).
 * q: F32 [256, T, n_head, 1], 16-byte aligned strides; k, v: the q8_0 cache
 * views [256, n_rows, n_head_kv, 1] (nb1 the row stride, nb2 the head
 * offset), n_rows * row stride < 2 GiB, n_head / n_head_kv <= 16; cells:
 * device int32, 16-byte aligned, cell_stride a positive multiple of 4; dst:
 * contiguous F32 [256, n_head, T, 1], 16-byte aligned; gate: NULL or F32 of
 * dst's shape and strides. No workspace: every list is one unit of k_fa_qc,
 * with no key splits. */
int qwfn_flash_attn_ext_q8_0_query_cells_dev(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                             const int32_t * cells, const int32_t * counts, int64_t cell_stride,
                                             int64_t pos0, float scale, const qwfn_tensor * gate,
                                             const qwfn_tensor * dst, int variant, void * stream);

size_t qwfn_fattn_workspace_size_query_cells(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                             const int64_t * n_cells, int64_t cell_stride);
int qwfn_flash_attn_ext_q8_0_query_cells(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                         const int32_t * cells, const int64_t * n_cells, int64_t cell_stride,
                                         int64_t pos0, float scale, const qwfn_tensor * gate, const qwfn_tensor * dst,
                                         int variant, void * ws, size_t ws_bytes, void * stream);

/* Rope and norm constants of the attention layers (qwfn_hparams.h:26,
 * :34-36): n_dims = rope_dim (64), sections = mrope_sections {11, 11, 10, 0},
 * freq_base = rope_freq_base (1e7), rms_eps (1e-6). */
typedef struct qwfn_rope_cfg {
    int32_t n_dims;
    int32_t sections[4];
    float   freq_base;
    float   rms_eps;
} qwfn_rope_cfg;

/* The layer's K/V producer for a decode or verify step (two launches: the
 * projections, then norm, rope and quantisation): K =
 * attn_k . cur and V = attn_v . cur (ggml_mul_mat with F16 weights: cur
 * converted to F16, F16 products summed in F32; with BF16 weights: cur
 * converted to BF16, round to nearest even, BF16 products summed in F32),
 * each K head RMS-normed and
 * multiplied by k_norm_w (F32 [256]), roped (IMROPE at pos, I32 [4 * T]
 * device: the T t positions, then h, w, e, as ggml_rope_multi reads them),
 * then K and V quantised (q8_0, variant as in qwfn_set_rows_q8_0) into cache
 * rows first_row .. first_row + T - 1. Replaces qwfn_graph.cpp:441-451 (the
 * mul_mats and rms), :446-451 / :129-132 (rope) and :370-384 (kv_append).
 * cur: F32 [n_embd, T] (T <= 16, n_embd a multiple of 8, T * n_embd <=
 * 65536, 16-byte aligned rows); wk, wv: both F16 or both BF16 [n_embd,
 * kv_dim] (kv_dim = 256 * n_head_kv <= 2048, 16-byte aligned rows). Weights
 * stored quantised (the reference model's GGUF holds one F16 tensor, 484 BF16
 * and the rest in k-quant / i-quant types; which of these attn_k and attn_v
 * are is not recorded in its logs) must be converted by the caller to F16
 * (or BF16) once at load: ggml would instead quantise cur to q8_K for them,
 * so for such weights parity with ggml's projection is unpinned.
 * caches: q8_0 [kv_dim, n_rows]. The projected rows
 * pass through a device-resident staging buffer of the library (one per GPU):
 * calls that overlap on one GPU race. The K/V bytes equal ggml's quantiser on
 * the F32 rows this kernel computes; those rows differ from ggml-cpu's only
 * in float summation order. */
int qwfn_kv_produce_q8_0(const qwfn_tensor * cur, const qwfn_tensor * wk, const qwfn_tensor * wv, const float * k_norm_w,
                         const int32_t * pos, const qwfn_rope_cfg * rope, const qwfn_tensor * k_cache,
                         const qwfn_tensor * v_cache, int64_t first_row, int variant, void * stream);

/* Attention with the output gate of the reference's attention layers fused
 * into its last store: dst = attention * sigmoid(gate), sigmoid(x) = 1 / (1 +
 * exp(-x)) -- the ggml_sigmoid and ggml_mul after flash_attn_ext
 * (qwfn_graph.cpp:474, :701). gate: F32 with dst's shape and strides, dst
 * and gate contiguous and 16-byte aligned. Otherwise as
 * qwfn_flash_attn_ext_q8_0 (same workspace). */
int qwfn_flash_attn_ext_q8_0_gated(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                   const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                   const qwfn_tensor * dst, const qwfn_tensor * gate, int variant, void * ws,
                                   size_t ws_bytes, void * stream);

/* The layer's K and V append followed by its attention, in one launch: the
 * two ggml_cpy / ggml_set_rows nodes that write the step's rows
 * (qwfn_graph.cpp:376-383, :623-624, :916-921) and the ggml_flash_attn_ext
 * that reads them (:469-471, :697-701), adjacent in the graph. src_k and src_v
 * are F32 [256 * n_head_kv, n] (n <= 64, 16-byte aligned rows); they are
 * quantised with `variant` into rows first_row .. first_row + n - 1 of the
 * caches that k and v view (heads as consecutive 272-byte segments of a row,
 * as in the reference's cache), which must lie inside the attended keys; then
 * the attention runs as qwfn_flash_attn_ext_q8_0. The cache bytes and dst are
 * identical to qwfn_cpy_f32_q8_0_kv followed by qwfn_flash_attn_ext_q8_0.
 * One sequence (B = 1). The blocks whose keys hold the new rows write them
 * before reading, so no separate append launch is needed. */
int qwfn_flash_attn_ext_q8_0_append(const qwfn_tensor * q, const qwfn_tensor * k, const qwfn_tensor * v,
                                    const qwfn_tensor * mask, float scale, float max_bias, float logit_softcap,
                                    const qwfn_tensor * dst, int variant, void * ws, size_t ws_bytes,
                                    const qwfn_tensor * src_k, const qwfn_tensor * src_v, int64_t first_row,
                                    void * stream);

/* ------------------------------------------------------ snapshot restore */

enum qwfn_copy_src { QWFN_SRC_DEVICE = 0, QWFN_SRC_HOST = 1 };

/* Restore snapshot parts into n_slots sequence slots:
 *   for p in [0, n_parts), s in [0, n_slots): copy bytes[p] bytes from src[p]
 *   to dst[s*n_parts + p].
 * src_kind QWFN_SRC_DEVICE: one fused kernel reads every source byte once and
 * writes it to all slots. QWFN_SRC_HOST: src are host pointers (pinned for
 * asynchronous copies); slot 0 is filled over the host link, slots 1.. by the
 * device broadcast from slot 0. Replaces the per-part ggml_backend_tensor_set
 * loop of engine::snapshot_load (qwfn_engine.cpp:1039-1042). */
int qwfn_state_restore(const void * const * src, const size_t * bytes, void * const * dst,
                       int32_t n_parts, int32_t n_slots, int32_t src_kind, void * stream);

#ifdef __cplusplus
}
#endif
#endif
