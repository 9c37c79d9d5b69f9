/*
 * libdsa: MI355X (gfx950) block-sparse self-attention hot path, C ABI.
 *
 * Drop-in device layer under the reference study's attention backends
 * (yangshuo1230/DiT_Sparse_Atten, attention_backends/).  The reference is
 * Python; its Python callers bind these symbols with ctypes (see
 * dit_sparse_atten_amd/_lib.py).  Conventions:
 *   - tensors are device pointers; bf16 is IEEE bfloat16, route/boolean
 *     tensors are one byte per entry (0 / 1), indices are int32;
 *   - q/k/v/o use [batch, tokens, heads, head_dim] logical order with
 *     arbitrary batch/token/head strides (in elements) and a contiguous head dim;
 *   - every call is asynchronous on `stream`, allocates nothing, and returns
 *     0 on success or a negative status (DSA_EINVAL = -1 invalid argument,
 *     DSA_EUNSUPPORTED = -2 valid but unsupported shape, DSA_ELAUNCH = -3 HIP
 *     error); dsa_last_error() describes the last failure on this thread.
 */
#ifndef DSA_H_
#define DSA_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version (1). */
int dsa_version(void);

/* Message of the last failed call on the calling thread ("" if none). */
const char* dsa_last_error(void);

/* Element types of the attention inputs (the `dtype` arguments). */
#define DSA_DTYPE_BF16 0
#define DSA_DTYPE_F16 1
/* fp32: dsa_bsa_fwd, dsa_bsa_fwd_noalloc, dsa_bsa_fwd_tile_stats and
 * dsa_bsa_fwd_block_mass (tokens a multiple of 128) only. */
#define DSA_DTYPE_F32 2

/*
 * Block-sparse attention forward, bf16, fp16 or fp32 in and out (dtype), fp32
 * online softmax; the matrix products run in the input type with fp32
 * accumulation (fp32 inputs: fp32 products on v_mfma_f32_32x32x2_f32, the
 * probabilities unrounded).
 * Replaces FlexAttention over a BlockMask (attention_backends/flex.py:379-399
 * `_flex_output`, flex.py:360-376) and, with row_ptr == col_idx == NULL, dense
 * SDPA (attention_backends/dense.py:14-48).
 *   strides[12]: q (b,t,h), k (b,t,h), v (b,t,h), o (b,t,h), in elements,
 *                each a multiple of 8; pointers 16-byte aligned.
 *   head_dim: a multiple of 8 up to 256 (dims past it are zero-filled in the
 *                kernel; the matrix products run at 128).  Head dims 136..256
 *                run the fp32-compute kernel for every dtype: S over 256
 *                dims, O in two launches of 128 dims.  block_size: 1..128
 *                tokens per query block and per key
 *                block (128 for the flex_reuse route; the spatial tile size of
 *                the matrix-sparse backend, sparse.py:51-103, 670-751).
 *   row_ptr/col_idx: CSR over rows ((rb * heads + h) * q_blocks + qb), rb <
 *                route_batches (1 = shared by all batch items, else = batch);
 *                col_idx lists key blocks (ascending order not required).
 *                Requires q_tokens == kv_tokens.  Out-of-range key blocks are
 *                skipped; a row with no key blocks yields zeros.
 *   scale: softmax scale (d^-1/2 for softmax_scale=None).
 *   causal: 1 for SDPA's is_causal (query t attends keys k <= t, top-left
 *                aligned when q_tokens != kv_tokens); dense calls only (the
 *                reference sends causal calls to its dense backend,
 *                flex.py:655-668, dense.py:40-47).
 *   deterministic: 1 for results reproducible bit for bit from run to run;
 *                0 lets a routed call that has the launch order (below) and
 *                at most 65,535 key blocks start each row's key walk where
 *                the workgroups resident on its XCD are reading (an aligned
 *                walk, for L2 reuse), so its fp32 accumulation order, and the
 *                last bits of O and LSE, depend on timing.  Dense calls are
 *                always reproducible.
 *   lse: optional [batch, heads, q_tokens] fp32 natural-log LSE, or NULL.
 *   workspace: optional device scratch (NULL with workspace_bytes == 0, or
 *                16-byte aligned).  Its front (only with q_blocks <= 8,192
 *                and at most 262,144 blocks in all) holds a 256-byte work
 *                queue, from which the workgroups of a call of more than one
 *                round take their slots in start order (the XCDs do not run
 *                equally fast), then the launch order of the query blocks
 *                (batch * heads * q_blocks int32, rounded up to 256 bytes;
 *                routed calls: each (batch, head)'s blocks, longest row
 *                first), 4,096 bytes of aligned-walk positions, and 64 fp32
 *                key-norm maxima per (batch, head) (rounded up to 256 bytes;
 *                at most 4,096 pairs), written by a pre-pass over K: with
 *                them a row skips its max on every 64-key half-tile whose
 *                scores the Cauchy-Schwarz bound |q| max|k| keeps within 2^32
 *                (bf16) or 2^15 (fp16) of its running reference (the same
 *                softmax; fp32 rounding can differ in the last bits).  Not used by plain-stream
 *                blocks whose last half-tile holds 1..32 keys.  The rest
 *                holds the fp32 partials
 *                of the query blocks in the last, partial round of workgroups
 *                (two per CU of the stream's device), which then run as 2..8
 *                key ranges merged by a second launch: at most rest / 66,560
 *                partials (128 x 130 fp32 each) and at most 1,024.  With less
 *                room (none: natural order, unsplit) the result can differ in
 *                the last bits, since a split row's fp32 accumulation order
 *                differs.  Contents need no initialisation and are dead after
 *                the call.  V is read in place; no transposed copy is made.
 * Keys past kv_tokens in a partial last block are masked.
 */
int dsa_bsa_fwd(const void* q, const void* k, const void* v, void* o, int32_t dtype,
                const int64_t* strides, int32_t batch, int32_t q_tokens, int32_t kv_tokens,
                int32_t heads, int32_t head_dim, int32_t block_size, const int32_t* row_ptr,
                const int32_t* col_idx, int32_t route_batches, float scale, int32_t causal,
                int32_t deterministic, float* lse, void* workspace, size_t workspace_bytes,
                hipStream_t stream);

/* Workspace bytes that let a self-attention dsa_bsa_fwd with 128-token
 * blocks order its launch and split its last round as far as it ever does:
 * the front (256 bytes of work queue, batch * heads * kv_blocks int32 of
 * launch order rounded up to 256, 4,096 bytes of aligned-walk positions, and
 * batch * heads * 64 fp32 of key-norm maxima rounded up to 256, none above
 * 4,096 (batch, head) pairs; 0 where the call is not ordered)
 * plus 68,157,440 (1,024 partials of 128 x 130 fp32) when the key range holds
 * at least 16 blocks (two parts of at least 8 key blocks each; none
 * otherwise, e.g. over 512 text tokens); 0 for invalid sizes.  No counterpart in the reference, whose FlexAttention
 * allocates internally. */
size_t dsa_bsa_workspace_bytes(int32_t batch, int32_t heads, int32_t kv_tokens,
                               int32_t head_dim);

/* The same for any block_size in 1..128 (key blocks of block_size tokens). */
size_t dsa_bsa_workspace_bytes_block(int32_t batch, int32_t heads, int32_t kv_tokens,
                                     int32_t head_dim, int32_t block_size);

/*
 * dsa_bsa_fwd without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Same arguments,
 * semantics and results as dsa_bsa_fwd given a workspace of
 * dsa_bsa_workspace_bytes_block() bytes; it calls no hipMalloc / hipFree.  The
 * work queue, the launch order, the aligned-walk positions, the key-norm
 * maxima and the split partials live in a library-owned device array of
 * 70,258,944 bytes (256 bytes of queue, 1 MiB of order, 4 KiB of positions,
 * 1 MiB of norms, then 1,024 partials of 128 x 130 fp32), one per device the
 * library runs on, held until the process ends; no call ever needs more, so
 * no call size is refused for want of scratch.  Every call on a device
 * shares that device's array: calls that overlap on one device (on
 * different streams) race; calls ordered on one stream do not.  Nothing in
 * the array needs clearing: a call clears its queue and writes every order
 * entry, norm and partial it reads, and a stale walk position only moves
 * where a row's walk starts.
 */
int dsa_bsa_fwd_noalloc(const void* q, const void* k, const void* v, void* o, int32_t dtype,
                        const int64_t* strides, int32_t batch, int32_t q_tokens,
                        int32_t kv_tokens, int32_t heads, int32_t head_dim, int32_t block_size,
                        const int32_t* row_ptr, const int32_t* col_idx, int32_t route_batches,
                        float scale, int32_t causal, int32_t deterministic, float* lse,
                        hipStream_t stream);

/*
 * Dense attention with dropout on the attention probabilities: the
 * reference's DenseBackend with dropout_p > 0, which hands dropout_p to SDPA
 * (attention_backends/dense.py:40-47; flex_reuse sends such calls to dense,
 * flex.py:655-668).  O[b,t,h] = sum_k keep[b,h,t,k] p[b,h,t,k] v[b,k,h] /
 * (1 - dropout_p) with p the softmax of scale q.k (every key counts in the
 * normaliser, as dropout after the softmax does) and keep = (u >=
 * round(dropout_p 2^32)) for the uniform u of key k: word k % 4 of
 * Philox4x32-10 with counter (k / 4, t, b * heads + h, offset) and key
 * (seed & 0xffffffff, seed >> 32) (Salmon et al., SC 2011).  Arguments as
 * dsa_bsa_fwd for a dense call (no route; causal allowed); dropout_p in
 * (0, 1).  Computes in fp32 for every dtype (the fp32-compute kernel) and
 * takes no workspace.  The reference's random stream is torch's and is not
 * reproduced: the same seed gives the same mask here, not the same mask as
 * SDPA.
 */
int dsa_bsa_fwd_dropout(const void* q, const void* k, const void* v, void* o, int32_t dtype,
                        const int64_t* strides, int32_t batch, int32_t q_tokens,
                        int32_t kv_tokens, int32_t heads, int32_t head_dim, float scale,
                        int32_t causal, float dropout_p, uint64_t seed, uint32_t offset,
                        float* lse, hipStream_t stream);

/*
 * Sampled block-mass estimate for one batch-1 self-attention call, bf16 or
 * fp16 Q/K (dtype).  Replaces `_sampled_block_mass`
 * (attention_backends/flex.py:205-251): `samples` evenly spaced tokens per
 * block, scores rounded like a matmul and a scale multiply in the input type,
 * fp32 softmax over all sampled keys plus log(block size / samples),
 * mass[h, qb, kb] = mean over query samples of the sum over key samples.
 * strides[4]: q (t, h), k (t, h) in elements.  samples: 1..block_size;
 * block_size <= 128; head_dim a multiple of 8 up to 256.  mass: [heads,
 * blocks, blocks], deterministic.
 */
int dsa_sampled_mass(const void* q, const void* k, int32_t dtype, const int64_t* strides,
                     int32_t tokens, int32_t heads, int32_t head_dim, int32_t block_size,
                     int32_t samples, float scale, float* mass, hipStream_t stream);

/*
 * Exact block attention mass of one batch-1 self-attention call, bf16 or fp16
 * Q/K (dtype).
 * Replaces `_block_attention_mass` and its Triton `_exact_block_mass_kernel`
 * (attention_backends/flex.py:96-202): mass[h, qb, kb] = sum over the valid
 * query tokens t of block qb and key tokens s of block kb of
 * exp(scale * <q_t, k_s> - lse[h, t]).  lse: [heads, tokens] fp32 natural-log
 * normaliser of the same Q/K and scale (dsa_bsa_fwd's lse output), head
 * stride lse_head_stride >= tokens.  strides[4]: q (t, h), k (t, h) in
 * elements.  head_dim a multiple of 8 up to 256, block_size 128.  mass:
 * [heads, blocks, blocks], every entry written (no initialisation needed);
 * deterministic.
 */
int dsa_block_mass(const void* q, const void* k, int32_t dtype, const int64_t* strides,
                   int32_t tokens,
                   int32_t heads, int32_t head_dim, int32_t block_size, const float* lse,
                   int64_t lse_head_stride, float scale, float* mass, hipStream_t stream);

/*
 * Spatial-tile attention statistics of one batch-1 self-attention call over
 * tile-major tokens, bf16 or fp16 Q/K (dtype) (tile_h * tile_w <= 128 tokens per tile, tokens a whole
 * number of tiles, at most 16384 tiles).  Replaces the statistics of the
 * matrix-sparse backend: `_dense_route` (attention_backends/sparse.py:184-233)
 * with row_ptr == col_idx == NULL, `sparse_chunk` (sparse.py:718-750) with the
 * CSR of the tiles each (head, query tile) row attended, and the
 * normalisations of sparse.py:859-864, 908-922.  lse: [heads, tokens]
 * natural-log normaliser of that same attention (dsa_bsa_fwd with
 * block_size = tile_h * tile_w).  Outputs [heads, tiles, tiles]: mass (fp32,
 * mass / tokens, required), mass_f16 (the same in fp16) and the four
 * centroids moment / max(mass, 1e-12) in fp16 (each optional).  Cells a CSR
 * row does not list are written as zeros; a row must not repeat a tile.
 */
int dsa_tile_stats(const void* q, const void* k, int32_t dtype, const int64_t* strides,
                   int32_t tokens,
                   int32_t heads, int32_t head_dim, int32_t tile_h, int32_t tile_w,
                   const float* lse, int64_t lse_head_stride, const int32_t* row_ptr,
                   const int32_t* col_idx, float scale, float* mass, void* mass_f16,
                   void* centroid_q_y, void* centroid_q_x, void* centroid_k_y,
                   void* centroid_k_x, hipStream_t stream);

/*
 * One step of the matrix-sparse backend: attention over spatial tiles
 * together with that attention's tile statistics.  Replaces `sparse_chunk`
 * (attention_backends/sparse.py:670-751: output plus the statistics of the
 * same softmax), `_sparse_stats_kernel` (sparse.py:498-578, the Triton path's
 * second pass over QK^T) and, with row_ptr == col_idx == NULL, the dense
 * attention and statistics of `_dense_route` (sparse.py:184-233).  The
 * arguments are those of dsa_bsa_fwd with batch 1, q_tokens = kv_tokens =
 * tokens (tile-major, a whole number of tile_h x tile_w tiles of at most 128
 * tokens) and the CSR of the kept tiles (route_batches 1) or none, and those
 * of dsa_tile_stats with lse required (written: [heads, tokens] fp32) and
 * lse_head_stride = tokens.
 *   entries: at least the CSR's entry count row_ptr[heads * tiles] (the
 *            cells of entries past it read as zeros); dense: at least
 *            heads * tiles * tiles.
 * The statistics come from the attention's own probabilities in the same
 * launch (the key-side sums on the matrix cores beside P V, per query row
 * and key tile, into the workspace), combined per cell by a short second
 * launch; no second QK pass runs.  Routed calls attend over blocks of one
 * tile.  Dense calls with tiles of 64..128 tokens, a multiple of 8, attend
 * over 128-token blocks and run unsplit; other dense calls attend over
 * blocks of one tile.  Head dims 136..256 (and fp32 inputs) run the
 * fp32-compute kernel on blocks of one tile.
 *   workspace: dsa_bsa_fwd_tile_stats_workspace_bytes(...) bytes, 16-byte
 *            aligned: entries * tile * 8 bytes of per-row statistics
 *            (rounded up to 256), then dsa_bsa_fwd's workspace.
 */
int dsa_bsa_fwd_tile_stats(const void* q, const void* k, const void* v, void* o, int32_t dtype,
                           const int64_t* strides, int32_t tokens, int32_t heads,
                           int32_t head_dim, int32_t tile_h, int32_t tile_w,
                           const int32_t* row_ptr, const int32_t* col_idx, int64_t entries,
                           float scale, int32_t deterministic, float* lse, float* mass,
                           void* mass_f16, void* centroid_q_y, void* centroid_q_x,
                           void* centroid_k_y, void* centroid_k_x, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes dsa_bsa_fwd_tile_stats needs (0 for invalid sizes).  No
 * counterpart in the reference. */
size_t dsa_bsa_fwd_tile_stats_workspace_bytes(int32_t heads, int32_t tokens, int32_t head_dim,
                                              int32_t tile_h, int32_t tile_w, int64_t entries);

/*
 * Dense attention with its exact block mass, for the exact route estimate:
 * the reference's `_dense_bootstrap` / exact refresh pair of a dense
 * FlexAttention with `return_lse=True` (attention_backends/flex.py:254-272,
 * 776-801) and `_block_attention_mass` (flex.py:158-202).  The arguments are
 * those of dsa_bsa_fwd for a dense batch-1 self-attention (q_tokens =
 * kv_tokens = tokens), with lse required (written: [heads, tokens] fp32) and
 * mass [heads, blocks, blocks] fp32 (blocks = ceil(tokens / 128)): the sum of
 * exp(scale * <q, k> - lse) over each pair of 128-token blocks, as
 * dsa_block_mass writes it.  When tokens is a multiple of 128, the mass
 * comes from the attention launch's own row sums per query row and key
 * block (then a short second launch; head dims above 128 on the
 * fp32-compute kernel); otherwise the call runs the attention and then
 * dsa_block_mass.  fp32 takes tokens a multiple of 128.
 *   workspace: dsa_bsa_fwd_block_mass_workspace_bytes(...) bytes, 16-byte
 *            aligned: heads * blocks^2 * 128 * 4 bytes of per-row log-masses
 *            when fused (rounded up to 256), then dsa_bsa_fwd's workspace.
 */
int dsa_bsa_fwd_block_mass(const void* q, const void* k, const void* v, void* o, int32_t dtype,
                           const int64_t* strides, int32_t tokens, int32_t heads,
                           int32_t head_dim, float scale, float* lse, float* mass,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes dsa_bsa_fwd_block_mass needs (0 for invalid sizes).  No
 * counterpart in the reference. */
size_t dsa_bsa_fwd_block_mass_workspace_bytes(int32_t heads, int32_t tokens, int32_t head_dim);

/*
 * Persistence prior + top-mass selection + first-frame sink, per row.
 * Replaces the prior of `_sampled_route` (flex.py:535-541), `_top_mass_route`
 * (flex.py:83-94, == sparse.py:171-181 `_row_mask`) and `_add_first_frame_sink`
 * (flex.py:550-566).  mass: [rows, keys] fp32, non-negative; previous: [rows,
 * keys] bytes or NULL (no prior); cap = max(1, ceil(keys * keep)); the first
 * sink_blocks columns are set after the cap.  keys <= 16384.  Outputs route
 * [rows, keys] bytes and counts [rows] (selected blocks per row, sink included).
 */
int dsa_route_select(const float* mass, const uint8_t* previous, int32_t rows, int32_t keys,
                     float rho, float target, int32_t cap, int32_t sink_blocks, uint8_t* route,
                     int32_t* counts, hipStream_t stream);

/*
 * Frontier of a route: selected cells (h, q, k) with an unselected valid
 * neighbour along the query axis (route[h, nb[q][d], k]) or the key axis
 * (route[h, q, nb[k][d]]).  Replaces `frontier_mask`
 * (attention_backends/routing.py:10-41).  route, frontier: [heads, blocks,
 * blocks] bytes; neighbors: [blocks, 4] int32 (-1 = none), blocks <= 16384.
 * count (optional, device) receives the number of frontier cells.
 */
int dsa_frontier_mask(const uint8_t* route, int32_t heads, int32_t blocks,
                      const int32_t* neighbors, uint8_t* frontier, unsigned long long* count,
                      hipStream_t stream);

/*
 * Frontier-aware directional route update with a per-row budget.
 * Replaces `directional_budget_update` (attention_backends/routing.py:92-168,
 * with `_sparse_best_targets` 53-80 and `_select_fixed_budget` 83-89) and the
 * first-frame sink that flex.py:544-546 applies to its result.
 *   mass: [heads, blocks, blocks] fp32, non-negative; previous: route bytes;
 *   previous_frontier: bytes or NULL (then the frontier of previous);
 *   neighbors: [blocks, 4] int32, blocks <= 16384; cap = max(1, ceil(blocks *
 *   keep)); explore_count = 0 or max(1, ceil(blocks * exploration_fraction));
 *   expand_flags: 1 query axis, 2 key axis, 4 joint.
 * Outputs (bytes, [heads, blocks, blocks]): route (selection, then the first
 * sink_blocks columns set), candidates (required, 16-byte aligned; also the
 * scatter scratch), and optionally exploration, dropped and added (before
 * the sink, as the reference's result dict); counts [heads, blocks] = set
 * entries per route row.
 */
int dsa_directional_update(const float* mass, const uint8_t* previous,
                           const uint8_t* previous_frontier, const int32_t* neighbors,
                           int32_t heads, int32_t blocks, int32_t cap, float persistence,
                           float min_ratio, float candidate_bonus, float budget_scale,
                           int32_t explore_count, int32_t expand_flags, int32_t sink_blocks,
                           uint8_t* route, int32_t* counts, uint8_t* candidates,
                           uint8_t* exploration, uint8_t* dropped, uint8_t* added,
                           hipStream_t stream);

/*
 * Next-step route of the matrix-sparse backend: drop low-mass tiles, keep one
 * tile in any row the drop emptied, then set the first sink_tiles columns.
 * Replaces `_drop_low_mass` + `_preserve_one_per_row`
 * (attention_backends/sparse.py:327-348) and the sink of sparse.py:883-884.
 *   mask, out: [heads, tiles, tiles] bytes; mass: the same shape, fp16
 *   (mass_is_f16 = 1, the reference's stored route mass) or fp32 (0);
 *   drop_factor > 0; head_scratch: device float[4 * heads], 8-byte aligned;
 *   counts: [heads, tiles] entries set per output row.
 */
int dsa_drop_low_mass(const uint8_t* mask, const void* mass, int32_t mass_is_f16, int32_t heads,
                      int32_t tiles, float drop_factor, int32_t sink_tiles, float* head_scratch,
                      uint8_t* out, int32_t* counts, hipStream_t stream);

/*
 * Predicted next-step mask of the matrix-sparse backend.  Replaces `_expand`
 * (attention_backends/sparse.py:350-373) for policy 1 ("all": eight coupled
 * query/key spatial neighbours of every routed tile, `_spatial_neighbors`
 * 258-276) and policy 2 ("directional": the eight neighbours of tiles whose
 * mass is at least huge_factor times the head's mean selected mass, and up to
 * three one-step moves of the others along their fp16 centroid directions,
 * `_apply_directional_steps` 285-324).  Tiles are numbered frame-major over
 * frames x blocks_h x blocks_w; mask, out: [heads, tiles, tiles] bytes;
 * mass_f16 and the centroids: fp16 of the same shape (directional only);
 * head_scratch: device float[4 * heads], 8-byte aligned (directional only).
 */
int dsa_expand_route(const uint8_t* mask, const void* mass_f16, const void* centroid_q_y,
                     const void* centroid_q_x, const void* centroid_k_y,
                     const void* centroid_k_x, int32_t heads, int32_t frames, int32_t blocks_h,
                     int32_t blocks_w, int32_t policy, float centroid_threshold,
                     float huge_factor, float* head_scratch, uint8_t* out, hipStream_t stream);

/*
 * Boolean route rows -> CSR (ascending key blocks per row).
 * Replaces the KV half of `_build_block_mask` / `_pack_route`
 * (flex.py:275-338; full_kv_num_blocks / full_kv_indices).  counts may be
 * given (e.g. from dsa_route_select) or NULL, in which case counts_out
 * receives them.  row_ptr: [rows + 1]; col_idx: capacity >= number of set
 * entries; nnz (optional, device int64) receives the total.
 */
int dsa_route_to_csr(const uint8_t* route, int32_t rows, int32_t keys,
                     const int32_t* counts_or_null, int32_t* counts_out, int32_t* row_ptr,
                     int32_t* col_idx, int64_t* nnz, hipStream_t stream);

/*
 * Stable partition of boolean rows: per row, the selected column ids
 * ascending, then the unselected ones ascending; counts = selected per row.
 * Replaces `pack_boolean_rows` (attention_backends/layout_ops.py:128-151).
 * indices: [rows, keys] int32.
 */
int dsa_pack_rows(const uint8_t* route, int32_t rows, int32_t keys, int32_t* counts,
                  int32_t* indices, hipStream_t stream);

/*
 * Token gather for 1-3 tensors: dst[n][b, t, h, :] = src[n][b, perm[t], h, :].
 * Replaces `reorder_qkv` (attention_backends/layout_ops.py:86-125) with the
 * permutation, and `SpatialTokenLayout.restore` (spatial.py:91-93) with the
 * inverse.  Strides are in BYTES: [n*3 + (b, t, h)]; row_bytes (head_dim *
 * element size) and strides multiples of 16.  Rows whose perm entry is out of
 * range are left untouched.
 */
int dsa_permute_rows(int32_t tensors, const void* const* src, void* const* dst,
                     const int64_t* src_strides, const int64_t* dst_strides,
                     const int32_t* perm, int32_t batch, int32_t tokens, int32_t heads,
                     int32_t row_bytes, hipStream_t stream);

/*
 * Non-GEMM work of the Wan DiT block around the attention call, for the
 * end-to-end denoising loop (the reference runs it through Diffusers'
 * WanTransformerBlock, wan_diffusers.py:75-191).  Rows are bf16 [rows, dim]
 * (dim a multiple of 8, <= 8192; row strides in elements; 16-byte aligned);
 * fp32 parameter vectors 16-byte aligned; arithmetic in fp32; in-place use
 * (out == x) is allowed.  One wave per row, 16 rows per workgroup.
 *
 * dsa_layernorm_modulate: out = LN(x) [* weight + bias] [* (1 + scale) + shift]
 *   (LayerNorm without or with affine; shift/scale fp32 [groups, dim], row r
 *   using group r / rows_per_group) - norm1/norm3 + modulation and norm2.
 * dsa_rmsnorm_rope: out = rope(x * rsqrt(mean(x^2) + eps) * weight) - the
 *   q/k RMSNorm, then (cos_sin != NULL, fp32 [tokens, head_dim / 2, 2]) the
 *   rotation of every head's consecutive (even, odd) pairs for token r % tokens.
 * dsa_gated_residual: out = x + gate * y (gate fp32 [groups, dim] or NULL = 1).
 */
int dsa_layernorm_modulate(const void* x, int64_t x_stride, int32_t rows, int32_t dim,
                           const float* weight, const float* bias, const float* shift,
                           const float* scale, int32_t rows_per_group, float eps, void* out,
                           int64_t out_stride, hipStream_t stream);
int dsa_rmsnorm_rope(const void* x, int64_t x_stride, int32_t rows, int32_t dim,
                     int32_t head_dim, const float* weight, const float* cos_sin,
                     int32_t tokens, float eps, void* out, int64_t out_stride,
                     hipStream_t stream);
int dsa_gated_residual(const void* x, int64_t x_stride, const void* y, int64_t y_stride,
                       const float* gate, int32_t rows, int32_t dim, int32_t rows_per_group,
                       void* out, int64_t out_stride, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_H_ */
