/*
 * qwfn_state.h -- C ABI of the per-sequence state around the q8_0 KV path:
 * the cache/recurrent-state owner, its reset, MTP-verify rollback, session
 * snapshots, and the small per-step inputs of the attention layers (masks and
 * the decode-time sparse-attention inputs), all built on the device.
 *
 *   qwfn::state (init, k_cache/v_cache/idx_cache/rs_state/rs_conv/ple_conv,
 *                reset, bytes, summary, n_ctx)          qwfn_state.h:28-92, qwfn_state.cpp:21-173
 *   engine::init_state rollback slots                  qwfn_engine.cpp:343-374
 *   engine::rollback_n                                  qwfn_engine.cpp:3629-3660
 *   snapshot_parts / snapshot_save / snapshot_load      qwfn_engine.cpp:988-1053
 *   engine::reset                                       qwfn_engine.cpp:1055-1066
 *   saved-sequence pool of the server                   tools/qwfn_server.cpp:767-793, :1380-1424
 *   block scores, top-k and cells of the decode QSA     qwfn_graph.cpp:556-581
 *   decode cell mask and padded cell list               qwfn_graph.cpp:668-675, :681-693
 *   causal masks of prefill chunks, steps, MTP drafts   qwfn_engine.cpp:1261-1271, :2093-2098, :3415-3440
 *   qsa_decode_prepare / _k, qsa_pool_rebuild (bias),
 *   init_qsa_tables                                     qwfn_engine.cpp:1072-1105, :3582-3614, :1107-1125, :672-684
 *
 * Conventions are those of qwfn_kv.h: QWFN_OK or a negative code with a
 * thread-local message (qwfn_last_error), host-side validation before any
 * launch, stream-ordered asynchronous device work, caller-owned buffers except
 * the state's own arenas.
 */
#ifndef QWFN_STATE_H
#define QWFN_STATE_H

#include "qwfn_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ state owner */

/* Hyper-parameters that size the state (hparams fields of qwfn_hparams.h:14-80
 * that qwfn_state.cpp:48-91 reads) and the state_config fields. */
typedef struct qwfn_state_config {
    uint32_t n_ctx;                    /* state_config::n_ctx                        */
    uint32_t n_layer;                  /* 48                                         */
    uint32_t full_attention_interval;  /* 4: layer il is attention if (il+1) % 4 == 0 */
    uint32_t n_head_kv;                /* 2                                          */
    uint32_t n_embd_head_k;            /* 256                                        */
    uint32_t n_embd_head_v;            /* 256                                        */
    uint32_t idx_key_len;              /* 128                                        */
    uint32_t ssm_d_state;              /* 128                                        */
    uint32_t ssm_n_group;              /* 16                                         */
    uint32_t ssm_dt_rank;              /* 48                                         */
    uint32_t ssm_d_conv;               /* 4                                          */
    uint32_t hc_count;                 /* 4                                          */
    uint32_t n_embd;                   /* 2560                                       */
    uint32_t ple_n_head;               /* 16; 0 = no PLE convolution history         */
    uint32_t ple_conv_kernel;          /* 4                                          */
    uint32_t ple_ngram_size;           /* 3                                          */
    int32_t  type_k;                   /* QWFN_TYPE_Q8_0 or QWFN_TYPE_F16            */
    int32_t  type_v;                   /* QWFN_TYPE_Q8_0 or QWFN_TYPE_F16            */
    int32_t  type_idx;                 /* QWFN_TYPE_F16 or QWFN_TYPE_F32             */
    uint32_t kv_host;                  /* K/V caches in pinned host memory           */
    uint32_t idx_host;                 /* indexer caches in pinned host memory       */
    uint32_t n_rollback;               /* rollback slots (engine's rb_nsnap_); 0 = none */
} qwfn_state_config;

/* The model's values above (qwfn_hparams.h comments), with n_ctx, q8_0 K/V,
 * F16 indexer keys and no rollback slots. */
void qwfn_state_config_default(qwfn_state_config * cfg, uint32_t n_ctx);

typedef struct qwfn_state qwfn_state;

/* Create a state on `device` and zero its recurrent part (state::init). All
 * device tensors live in one arena, each 256-byte aligned; the recurrent
 * tensors (rs and conv of every DeltaNet layer, then the PLE history) are
 * contiguous, and each rollback slot is a separate image of that region with
 * the same layout. device = QWFN_LAYOUT_ONLY allocates nothing: tensor
 * descriptors then carry byte offsets from 0 instead of addresses, which is
 * enough for sizes, summaries and snapshot part lists (no device needed). */
#define QWFN_LAYOUT_ONLY (-1)
int  qwfn_state_create(const qwfn_state_config * cfg, int device, qwfn_state ** out);
void qwfn_state_destroy(qwfn_state * st);

enum qwfn_state_kind {
    QWFN_STATE_K        = 0,  /* q8_0/f16 1-D [kv_dim * n_ctx], attention layers */
    QWFN_STATE_V        = 1,
    QWFN_STATE_IDX      = 2,  /* f16 1-D [idx_key_len * n_ctx], attention layers */
    QWFN_STATE_RS       = 3,  /* f32 [d_state, d_state, dt_rank], DeltaNet layers */
    QWFN_STATE_CONV     = 4,  /* f32 [d_conv - 1, conv_dim], DeltaNet layers      */
    QWFN_STATE_PLE_CONV = 5,  /* f32 [(kernel - 1) * ngram, hc_count * n_embd]    */
};

/* Descriptor of a state tensor. slot = -1: the live tensor; slot s >= 0: the
 * tensor's image in rollback slot s (RS, CONV, PLE_CONV only; slot s holds the
 * state s+1 tokens back). Returns 1 and fills *out when the tensor exists, 0
 * (and a zeroed *out) when the layer has no such tensor -- k_cache() etc.
 * returning null in qwfn_state.cpp:123-148 -- or a negative code. */
int      qwfn_state_tensor(const qwfn_state * st, int32_t kind, uint32_t il, int32_t slot, qwfn_tensor * out);
size_t   qwfn_state_bytes(const qwfn_state * st);           /* device arena, without rollback slots */
size_t   qwfn_state_host_bytes(const qwfn_state * st);      /* pinned host arena (kv_host / idx_host) */
size_t   qwfn_state_rollback_bytes(const qwfn_state * st);  /* all rollback slots */
uint32_t qwfn_state_n_ctx(const qwfn_state * st);
/* state::summary(); writes at most cap bytes including the terminating NUL and
 * returns the full length (snprintf convention), or a negative code. */
int      qwfn_state_summary(const qwfn_state * st, char * buf, size_t cap);

/* ------------------------------------------------- position bookkeeping */

int32_t qwfn_state_n_past(const qwfn_state * st);
int32_t qwfn_state_rollback_depth(const qwfn_state * st);
/* After a step of T positions (eval_batch, qwfn_engine.cpp:2033-2035):
 * n_past += T; the rollback depth becomes min(T-1, n_rollback) for a verified
 * decode step of T >= 2 positions, else 0. QWFN_ERANGE if n_past + T > n_ctx. */
int qwfn_state_step_done(qwfn_state * st, int32_t T, int32_t verified);

/* engine::reset minus the engine-only flags: zero the recurrent tensors (one
 * fill kernel; the caches are not cleared), n_past = 0, rollback depth 0. A
 * QWFN_LAYOUT_ONLY state only has its bookkeeping reset. */
int qwfn_state_reset(qwfn_state * st, void * stream);

/* engine::rollback_n: copy rollback slot n_back-1 over the live recurrent
 * tensors (one contiguous device copy), n_past -= n_back, depth 0.
 * QWFN_ERANGE (message "rollback: no snapshot of the state N tokens back")
 * unless 1 <= n_back <= rollback depth. */
int qwfn_state_rollback(qwfn_state * st, int32_t n_back, void * stream);

/* ---------------------------------------------------------- snapshots */

typedef struct qwfn_part {
    void * data;    /* device address (or arena offset for QWFN_LAYOUT_ONLY) */
    size_t bytes;   /* bytes of the part that belong to the first n_past positions */
} qwfn_part;

enum qwfn_mem_kind { QWFN_MEM_DEVICE = 0, QWFN_MEM_HOST = 1 };

/* snapshot_parts (qwfn_engine.cpp:990-999) over the states in order (the
 * trunk, then the MTP head's state): per layer K, V, idx with
 * min(nbytes, n_past * row bytes), then rs and conv whole; then the PLE
 * history. Writes up to max_parts entries and sets *n_parts to the count
 * (call with max_parts = 0 to size the array). */
int qwfn_snapshot_parts(const qwfn_state * const * sts, int32_t n_sts, int32_t n_past,
                        qwfn_part * parts, int32_t max_parts, int32_t * n_parts);

/* snapshot_save: copy every part of the states' first n_past positions
 * (n_past of sts[0]; all states must agree) into dst[k] (dst_bytes[k] must
 * equal the part's size; n_dst the part count). dst_kind QWFN_MEM_DEVICE: one
 * batched device copy; QWFN_MEM_HOST: host buffers (pinned ones make the copy
 * asynchronous). Stream-ordered: synchronise before reading dst. */
int qwfn_snapshot_save(const qwfn_state * const * sts, int32_t n_sts, void * const * dst,
                       const size_t * dst_bytes, int32_t n_dst, int32_t dst_kind,
                       int32_t * n_past_out, void * stream);

/* snapshot_load: reset every state first (as the reference does, so a
 * rejected snapshot leaves a reset state), then QWFN_ESIZE if n_src differs
 * from the part count for n_past or any src_bytes[k] from its part's size;
 * else copy each part in and set n_past on every state. */
int qwfn_snapshot_load(qwfn_state * const * sts, int32_t n_sts, int32_t n_past, const void * const * src,
                       const size_t * src_bytes, int32_t n_src, int32_t src_kind, void * stream);

/* ------------------------------------------------- saved-sequence pool */

/* The server's saved sequences (saved_seq, save_seq, best_saved,
 * tools/qwfn_server.cpp:767-793; restore_or_reset, :1380-1400;
 * shared_prefix_split, :1401-1424) with the snapshots held in HBM instead of
 * host vectors. At most max_entries (the reference: 4) sequences whose
 * snapshot bytes sum to at most cap_bytes (QWFN_SNAP_MB), least recently used
 * first. The pool arena is 2 x (cap + slack) bytes of device memory, allocated
 * once; device = QWFN_LAYOUT_ONLY keeps the bookkeeping and copies nothing. */
typedef struct qwfn_snap_pool qwfn_snap_pool;
int     qwfn_snap_pool_create(size_t cap_bytes, int32_t max_entries, int device, qwfn_snap_pool ** out);
void    qwfn_snap_pool_destroy(qwfn_snap_pool * pool);
int32_t qwfn_snap_pool_count(const qwfn_snap_pool * pool);
size_t  qwfn_snap_pool_bytes(const qwfn_snap_pool * pool);   /* snapshot bytes held */
/* Entry k (0 = least recently used): token count, n_past, snapshot bytes, and
 * up to tok_cap of its tokens. */
int     qwfn_snap_pool_entry(const qwfn_snap_pool * pool, int32_t k, int32_t * n_tok, int32_t * n_past,
                             size_t * bytes, int32_t * tok, int32_t tok_cap);
/* save_seq: snapshot the states (at their n_past) under the token sequence.
 * Returns 1 if kept, 0 if larger than the cap (not kept), or a negative code.
 * An entry with the same tokens is replaced, then the least recently used go
 * until the count and the bytes are within the limits. */
int     qwfn_snap_pool_save(qwfn_snap_pool * pool, const qwfn_state * const * sts, int32_t n_sts,
                            const int32_t * tok, int32_t n_tok, void * stream);
/* best_saved: the longest saved sequence the prompt strictly extends, or -1
 * (always -1 for a prompt with images). */
int32_t qwfn_snap_pool_best(const qwfn_snap_pool * pool, const int32_t * tok, int32_t n_tok, int32_t has_images);
/* snapshot_load of entry k into the states (reset first; QWFN_ESIZE if the
 * states' parts differ from the saved ones); the entry becomes the most
 * recently used. */
int     qwfn_snap_pool_load(qwfn_snap_pool * pool, int32_t k, qwfn_state * const * sts, int32_t n_sts, void * stream);
/* shared_prefix_split: where a fresh prefill of `prompt` should stop once so
 * that its prefix shared with a saved sequence can be saved; 0 for none. */
int32_t qwfn_snap_pool_split(const qwfn_snap_pool * pool, const int32_t * prompt, int32_t n_prompt, int32_t n_consumed,
                             int32_t has_images);
/* restore_or_reset: save the consumed sequence when it has >= 2048 tokens and
 * no images, then load the best saved sequence the prompt extends (*n_restored
 * = its token count; it is now the last entry), or reset the states
 * (*n_restored = 0). The states' n_past must equal n_consumed. */
int     qwfn_snap_pool_restore_or_reset(qwfn_snap_pool * pool, qwfn_state * const * sts, int32_t n_sts,
                                        const int32_t * consumed, int32_t n_consumed, int32_t consumed_has_images,
                                        const int32_t * prompt, int32_t n_prompt, int32_t prompt_has_images,
                                        int32_t * n_restored, void * stream);

/* ------------------------------------------------- sparse block selection */

/* qsa_dec_cells (qwfn_graph.cpp:556-581) for T queries: for query t,
 *   score[b] = sum_h relu(pool[b] . f16(q[t][h])) + bias[t][b]   (b < n_blocks)
 *   top      = the k_blocks best blocks, best first            (ggml_top_k)
 *   cells[t][j * ratio + m] = blk_cells[top[j] * ratio + m]
 * pool: F16 [128] per block at pool_nb1 bytes (the pooled, normed, roped block
 * keys of the layer's pool cache); q: F32 [128, n_heads] per query at q_nb2
 * bytes, 16-byte aligned (the roped indexer query, n_heads <= 8); bias: F32
 * [n_blocks] per query at bias_nb1 bytes; blk_cells: I32 [n_blocks * ratio],
 * ratio <= 16; top (optional): I32
 * [T][k_blocks]. k_blocks <= min(n_blocks, 1024), n_blocks <= 49152. Equal
 * scores keep the lower block first. ws: at least
 * qwfn_qsa_select_workspace_size(n_blocks, T) bytes of 16-byte aligned device
 * memory (the scores; for more than 8 queries without the bias, which the
 * top-k adds). All pointers are device memory. */
size_t qwfn_qsa_select_workspace_size(int64_t n_blocks, int32_t T);
int qwfn_qsa_select_cells(const uint16_t * pool, size_t pool_nb1, int64_t n_blocks, const float * q, int32_t n_heads,
                          size_t q_nb2, const float * bias, size_t bias_nb1, int32_t T, int32_t k_blocks,
                          const int32_t * blk_cells, int32_t ratio, int32_t * cells, int32_t * top, void * ws,
                          size_t ws_bytes, void * stream);

/* ------------------------------------------------- Gated DeltaNet state */

/* The recurrent update of a DeltaNet layer for T tokens with its rollback
 * snapshots, one launch: ggml_gated_delta_net (qwfn_graph.cpp:258, inside
 * graph_builder::deltanet :240-278) and the state copies of
 * deltanet_write_state (:208-238). Per value head h (key head
 * h / (n_v_heads / n_k_heads)), state S [head_dim][head_dim] (the second index
 * contiguous), token t:
 *   S = S * exp(g[t][h]);  m[c] = sum_r S[r][c] k[r]
 *   S[r][c] += k[r] * (v[c] - m[c]) * beta[t][h]
 *   out[t][h][c] = sum_r S[r][c] * q[r] * scale
 * (the gated delta rule; q and k L2-normed by the caller as the reference's
 * deltanet_conv_qkv does, scale 1/sqrt(head_dim)). q, k: F32 [n_k][head_dim]
 * per token at q_token_stride / k_token_stride floats (the views of the conv
 * output), v: [n_v][head_dim] per token at v_token_stride; g (log decay) and
 * beta: F32 [T][n_v]; state: F32 [n_v][head_dim][head_dim], updated in place
 * (rs_state); out: F32 [T][n_v][head_dim]; snap: n_snap <= T-1 slots at
 * snap_stride_bytes, slot s-1 receiving the state s tokens back (the
 * rollback slots rb_rs_). head_dim = 128. Device memory throughout. */
int qwfn_gated_delta_net(const float * q, int64_t q_token_stride, const float * k, int64_t k_token_stride,
                         const float * v, int64_t v_token_stride, const float * g, const float * beta, int32_t T,
                         int32_t n_k_heads, int32_t n_v_heads, int32_t head_dim, float scale, float * state, float * out,
                         float * snap, size_t snap_stride_bytes, int32_t n_snap, void * stream);

/* ------------------------------------------------- QSA index producer */

/* The indexer's key geometry and the rope / norm constants of the model
 * (qwfn_hparams.h:26, :34-36, :53): idx_dim = idx_key_len (128), n_dims =
 * rope_dim (64), sections = mrope_sections {11, 11, 10, 0}, freq_base =
 * rope_freq_base (1e7), rms_eps (1e-6). */
typedef struct qwfn_qsa_pool_cfg {
    int32_t idx_dim;
    int32_t n_dims;
    int32_t sections[4];
    float   freq_base;
    float   rms_eps;
} qwfn_qsa_pool_cfg;
void qwfn_qsa_pool_cfg_default(qwfn_qsa_pool_cfg * cfg);

/* ggml_set_rows of F32 rows into an F16 tensor (IEEE round to nearest even):
 * dst F16 [ne0, rows] (row stride nb[1]), src F32 [ne0, n], idx I32 [n]
 * (device). An index outside [0, rows) skips its row and sets bit 0 of
 * qwfn_device_status. The decode step's raw indexer key into the index cache
 * (qwfn_graph.cpp:536-543) is this op with n = 1. */
int qwfn_set_rows_f16(const qwfn_tensor * dst, const qwfn_tensor * src, const qwfn_tensor * idx, void * stream);

/* qsa_dec_index (qwfn_graph.cpp:529-554) for one decode position, one launch:
 * the raw key k_raw (F32 [idx_dim], device; NULL: no key is written) into row
 * *write_idx of the index cache (F16 [ic_rows][idx_dim]), then the block's
 * pooled key -- qsa_pool_blocks (:282-301): the mean of index-cache rows
 * member_idx[0 .. ratio-1] (the new key among them read from the call's own
 * value), RMS norm, times k_norm_w (F32 [idx_dim]), IMROPE at positions
 * blk_pos[0..3] -- rounded to F16 into row *blk_idx of the pool cache (F16
 * [pool_rows][idx_dim]). write_idx, member_idx, blk_pos and blk_idx are the
 * device inputs qwfn_qsa_decode_prepare writes. Out-of-range rows are
 * skipped and flagged in qwfn_device_status. Both caches are rows packed at
 * idx_dim values (row r at element r * idx_dim): there is no row stride. */
int qwfn_qsa_pool_decode(uint16_t * idx_cache, int64_t ic_rows, const float * k_raw, const int32_t * write_idx,
                         const int32_t * member_idx, int32_t ratio, const int32_t * blk_pos, const int32_t * blk_idx,
                         const float * k_norm_w, uint16_t * pool, int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg,
                         void * stream);

/* The pooled keys of every whole block after a prefill or a restore
 * (engine::qsa_pool_rebuild, qwfn_engine.cpp:1121-1145, through
 * graph_builder::qsa_pool_rebuild, qwfn_graph.cpp:478-495): block b <
 * n_past / ratio pools index-cache rows b*ratio .. b*ratio + ratio - 1 at
 * position b*ratio into pool row b. One launch for all blocks. Rows packed
 * at idx_dim values, as in qwfn_qsa_pool_decode. */
int qwfn_qsa_pool_rebuild(const uint16_t * idx_cache, int64_t ic_rows, int64_t n_past, int32_t ratio,
                          const float * k_norm_w, uint16_t * pool, int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg,
                          void * stream);

/* ---------------------------------------------------------------- masks */

/* Causal F16 mask of T query rows over n_kv keys, row i at byte i*row_stride:
 * key j is visible (0x0000) iff j <= n_past + i, else -inf (0xFC00); keys
 * n_kv .. row_stride/2 - 1 of a padded row are -inf. The masks of
 * build_attn_inputs (qwfn_engine.cpp:1261-1271), build_step_inputs (:2093-2098)
 * and mtp_mask (:3415-3421) with n_past = n_past_c / n_past / pos. */
int qwfn_causal_mask_f16(uint16_t * mask, int64_t n_kv, int64_t T, int64_t n_past, size_t row_stride,
                         void * stream);

/* Decode cell mask (qwfn_graph.cpp:668-675, :681-693): for j < n_pad,
 * mask[j] = 0 if j < n_cells and cells[j] <= n_past, else -inf; and, when
 * gcells is not NULL, the padded cell list gcells[j] = cells[j] for
 * j < n_cells, cells[j - n_cells] after (the reference's concat of the list
 * with its own head; needs n_pad <= 2 n_cells). cells, mask and gcells are
 * device memory. */
int qwfn_cell_mask_f16(const int32_t * cells, int64_t n_cells, int64_t n_pad, int32_t n_past,
                       uint16_t * mask, int32_t * gcells, void * stream);

/* The prefill chunk's sparse-attention inputs, engine::fill_chunk_qsa
 * (qwfn_engine.cpp:1276-1320), written on the device in one launch. n_kv =
 * n_past_c + Tc keys, n_blocks = ceil(n_kv / ratio) blocks, n_bid = n_kv /
 * ratio whole ones; the dead block is the partial tail block n_bid when there
 * is one, else the last. Any pointer may be NULL.
 *   cell_blk  I32 [n_kv]:          j / ratio for the cells of whole blocks, dead after
 *   blk_cells I32 [n_blocks*ratio]: b*ratio + k; the tail block's real cells,
 *                                   the last one repeated
 *   blk_pos   I32 [4*n_blocks]:    b*ratio in each of the 4 rope sections
 *   bias      F32 [Tc][n_blocks] (rows bias_nb1 bytes apart), row i for query
 *             q = n_past_c + i: 0 for whole blocks ending at or before q, 1e9
 *             for the block holding q when q is not its last cell and for the
 *             dead block unless it lies wholly after q, -1e9 for blocks wholly
 *             after q, -inf for none (every block is one of the above).
 * Tc <= 65534, n_kv < 2^31. */
int qwfn_qsa_chunk_inputs(int64_t n_past_c, int64_t Tc, int32_t ratio, int32_t * cell_blk, int32_t * blk_cells,
                          int32_t * blk_pos, float * bias, size_t bias_nb1, void * stream);

/* The prefill's selection mask, graph_builder::qsa_mask (qwfn_graph.cpp:
 * 388-414): F16 mask [T rows of mask_nb1 bytes] = -inf everywhere, then 0 at
 * the cells query t selected (cells: I32 [T][width], rows cells_nb1 bytes
 * apart: the qsa_top_k output), plus the causal mask (F16 [T][>= n_kv], rows
 * causal_nb1 bytes apart). So key j < n_kv of row t is causal[t][j] where
 * selected, -inf elsewhere; the row's padding past n_kv is -inf. Repeated
 * cells are harmless; a cell outside [0, n_kv) is skipped and sets bit 0 of
 * qwfn_device_status. mask must not overlap causal (the reference adds in
 * place into a separate selection tensor). n_kv <= 524288. */
int qwfn_qsa_mask_f16(const int32_t * cells, int64_t width, size_t cells_nb1, const uint16_t * causal,
                      size_t causal_nb1, int64_t n_kv, int64_t T, uint16_t * mask, size_t mask_nb1, void * stream);

/* The keys each query of a QSA-on prefill chunk sees, as lists: the zeros of
 * qwfn_qsa_mask_f16's mask over the chunk's causal mask (qwfn_graph.cpp:
 * 388-414 over the mask of qwfn_engine.cpp:1261-1270, 0 up to the query's
 * position). Row t of lists (lists_nb1 bytes apart) gets the distinct cells
 * of cells row t (I32 [T][width], rows cells_nb1 bytes apart: the
 * qsa_top_k output) that are at most n_past + t, ascending; counts[t] their
 * number (device int32). With qwfn_flash_attn_ext_q8_0_query_cells_dev over
 * them (pos0 = n_past) it replaces qsa_mask and the flash attention over it:
 * the same keys, no mask. A cell outside [0, n_kv) is skipped and sets bit 0
 * of qwfn_device_status. No counterpart in the reference: its callers build
 * the dense mask. lists_nb1 >= width * 4; cells, lists and counts must not
 * overlap; n_kv <= 524288. */
int qwfn_qsa_visible_cells(const int32_t * cells, int64_t width, size_t cells_nb1, int64_t n_kv, int64_t T,
                           int64_t n_past, int32_t * lists, size_t lists_nb1, int32_t * counts, void * stream);

/* ------------------------------------------- decode-time sparse-attention inputs */

/* qsa_decode_inputs (qwfn_graph.h:71-84): device tensors written per token. */
typedef struct qwfn_qsa_inputs {
    float *   bias;          /* F32 [n_blocks_max]                         */
    int32_t * write_idx;     /* I32 [1]                                    */
    int32_t * member_idx;    /* I32 [ratio]                                */
    int32_t * blk_pos;       /* I32 [4]                                    */
    int32_t * blk_idx;       /* I32 [1]                                    */
    float *   npast_f;       /* F32 [1]                                    */
    int32_t   ratio;         /* cells per block                            */
    int32_t   pad_;
    int64_t   n_blocks_max;  /* bias ne[0] (NBmax)                         */
} qwfn_qsa_inputs;

/* The block bucket the decode graph is shaped for at n_past:
 * clamp(roundup256(n_past / ratio + 1), 768, n_blocks_max)
 * (qwfn_engine.cpp:1099-1101). Host only. */
int64_t qwfn_qsa_bucket(int32_t n_past, int32_t ratio, int64_t n_blocks_max);

/* qsa_decode_prepare (prev_bias NULL; the bias window around the block of
 * n_past is updated in place) or qsa_decode_prepare_k (prev_bias = the
 * previous position's bias: copied, then this position's window on top), in
 * one launch: write_idx = n_past, member_idx = the cells of n_past's block,
 * blk_pos = 4 x its first cell, blk_idx, npast_f; bias 0 for whole blocks,
 * 1e9 for the incomplete block of n_past, -inf past it. */
int qwfn_qsa_decode_prepare(const qwfn_qsa_inputs * qd, const float * prev_bias, int32_t n_past, void * stream);

/* The inputs of a verify step's T positions n_past .. n_past + T - 1 in one
 * launch (engine::attn_decode's T chained preparations, qwfn_engine.cpp:
 * 2259-2280 through :1072-1105 and :3582-3614): the same values as
 * qwfn_qsa_decode_prepare(&qd[0], NULL, n_past) followed by
 * qwfn_qsa_decode_prepare(&qd[t], qd[t-1].bias, n_past + t) for t = 1 ..
 * T-1. qd: host array of T input sets with the same ratio and n_blocks_max
 * and bias rows that do not overlap; qd[0].bias holds the running bias.
 * T <= 16. No counterpart in the reference, which prepares one position a
 * call; for engines that batch the step's positions. */
int qwfn_qsa_decode_prepare_steps(const qwfn_qsa_inputs * qd, int32_t T, int32_t n_past, void * stream);

/* qsa_dec_index for the T positions of a verify step in one launch (the T
 * chained sparse_attn_decode calls of engine::attn_decode, qwfn_engine.cpp:
 * 2259-2280, each through qwfn_graph.cpp:529-554): the same index cache and
 * pool as qwfn_qsa_pool_decode for position 0, 1, .. T-1 in order, with
 * position t's raw key in row t of k_raw (F32, rows k_raw_nb1 bytes apart;
 * NULL: no keys are written) and its device inputs in qd[t] (host array, as
 * qwfn_qsa_decode_prepare or _steps wrote them; qd[t].bias is not read).
 * Only the last position of each block pools it, with the keys of this call
 * taken from k_raw. T <= 16. No counterpart in the reference, which runs one
 * position a call; for engines that batch the step's positions. */
int qwfn_qsa_pool_decode_steps(uint16_t * idx_cache, int64_t ic_rows, const float * k_raw, size_t k_raw_nb1,
                               const qwfn_qsa_inputs * qd, int32_t T, const float * k_norm_w, uint16_t * pool,
                               int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg, void * stream);

/* qwfn_qsa_decode_prepare_steps(qd, T, n_past) followed by
 * qwfn_qsa_pool_decode_steps(idx_cache, ic_rows, k_raw, k_raw_nb1, qd, T,
 * k_norm_w, pool, pool_rows, cfg), in one launch: the same bias rows, small
 * inputs, index cache rows and pooled rows. The pooling takes its indices in
 * the closed forms the preparation writes (position p = n_past + t writes
 * index row p of block p / ratio, whose members are the rows
 * (p / ratio) ratio + m) instead of reading them back. No counterpart in the
 * reference, whose engine fills these inputs on the host (qwfn_engine.cpp:
 * 1072-1105) before the graph pools (qwfn_graph.cpp:529-554); for engines
 * that run the step's preparation and pooling back to back. */
int qwfn_qsa_decode_prepare_pool_steps(const qwfn_qsa_inputs * qd, int32_t T, int32_t n_past, uint16_t * idx_cache,
                                       int64_t ic_rows, const float * k_raw, size_t k_raw_nb1, const float * k_norm_w,
                                       uint16_t * pool, int64_t pool_rows, const qwfn_qsa_pool_cfg * cfg, void * stream);

/* The full bias rewrite of qsa_pool_rebuild (qwfn_engine.cpp:1115-1120):
 * 0 for blocks < (n_past+1)/ratio, the block of n_past 0 or 1e9, -inf after.
 * n_past = -1 writes -inf everywhere (engine::reset, init_qsa_tables). */
int qwfn_qsa_bias_rebuild(float * bias, int64_t n_blocks_max, int32_t n_past, int32_t ratio, void * stream);

/* Static tables of init_qsa_tables (qwfn_engine.cpp:676-681) and the block
 * positions of qsa_pool_rebuild (:1121-1124), any pointer may be NULL:
 * blk_cells[b*ratio + k] = b*ratio + k for b < n_blocks_max; cell_pos[i] = i
 * (F32) for i < n_ctx; blk_pos_all[s*n_whole + b] = b*ratio for s < 4,
 * b < n_whole. */
int qwfn_qsa_tables(int32_t * blk_cells, int64_t n_blocks_max, int32_t ratio, float * cell_pos, int64_t n_ctx,
                    int32_t * blk_pos_all, int64_t n_whole, void * stream);

#ifdef __cplusplus
}
#endif
#endif
