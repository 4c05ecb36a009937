/*
 * treeverify.h - C ABI of the MI355X (gfx950) tree-verification hot path.
 *
 * These device operations replace the Triton/PyTorch operations that the
 * nano-vllm-jetspec speculative runner calls per verify round:
 *
 *   tv_store_kvcache      slot-mapped K/V append
 *                         replaces layers/attention.py:38-45 (store_kvcache) and
 *                         the eager tree scatter models/qwen3.py:255-258
 *   tv_tree_attention     ragged packed tree-verify attention over a paged KV pool
 *                         replaces speculative/jetspec/paged_backend.py:240-306
 *                         (packed_tree_attention) and its kernels
 *                         paged_backend.py:116-213, tree_prefix.py:303-441,
 *                         tree_gqa.py:32-111
 *   tv_copy_accepted_kv   accepted-only KV commit across both KV axes and all layers
 *                         replaces speculative/jetspec/state.py:64-86
 *   tv_commit_slots       the batch's commit source/destination slots in one launch,
 *                         replaces the per-request maps of state.py:746-798
 *   tv_rope_scatter       HF-order RoPE of the tree Q/K fused with the scratch
 *                         scatter of K/V, replaces speculative/jetspec/
 *                         tree_fusion.py:181-199 (rope_scatter_prevalidated)
 *   tv_argmax_rows,       greedy acceptance: the target argmax and the tree walk,
 *   tv_tree_accept        replaces speculative/jetspec/serving_ops.py:55-90
 *   tv_truncate_accepted  max_new_tokens / EOS cut of the accepted outputs and the
 *                         packed commit paths, replaces batch_runtime.py:636-655
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless its name ends in _host.
 *   - Strides are in ELEMENTS, never bytes.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream).
 *   - Every entry point only enqueues work: no host synchronisation and no device
 *     allocation.  Caller-owned workspaces are passed in explicitly.
 *   - Return value: TV_OK (0) or a negative TV_ERR_* code; tv_last_error() gives
 *     the message of the last failing call made by the calling thread.
 *   - `status` (optional, may be NULL) is a device int32 that kernels OR error
 *     bits into (TV_STATUS_*) when they meet an out-of-range page or slot.  The
 *     offending K/V row is then neither read nor written, so a bad index can never
 *     fault the GPU; the result for that row is unspecified.
 */
#ifndef TREEVERIFY_H
#define TREEVERIFY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TV_ABI_VERSION 4

enum tv_error {
    TV_OK = 0,
    TV_ERR_INVALID = -1,      /* malformed arguments (shape, stride, pointer, count) */
    TV_ERR_UNSUPPORTED = -2,  /* well-formed but outside what the kernels implement */
    TV_ERR_LAUNCH = -3,       /* the HIP runtime refused a launch */
    TV_ERR_CAPACITY = -4      /* a caller-provided buffer is too small */
};

enum tv_dtype { TV_BF16 = 0, TV_F16 = 1, TV_F32 = 2 };

enum tv_status_bits {
    TV_STATUS_BAD_PAGE = 1,     /* a block-table page or tree slot outside the pool */
    TV_STATUS_BAD_SLOT = 2,     /* a store/commit slot outside the pool */
    TV_STATUS_BAD_REQUEST = 4,  /* metadata row that names a nonexistent request */
    TV_STATUS_BAD_POSITION = 8, /* a RoPE position outside the cos/sin cache */
    TV_STATUS_BAD_DEPTH = 16,   /* an accepted path node off its canonical depth */
    TV_STATUS_BAD_BIAS = 32,    /* a qq_bias entry other than 0 / -inf packed into visibility
                                   bits (finite values need tv_tree_attention_fp32) */
    TV_STATUS_STALE_PLAN = 64   /* an attention plan that no longer matches the live metadata:
                                   a request's prefix length or node count changed after the
                                   plan was made (tv_tree_attention_plan reads host copies) */
};

/* ABI version of the loaded library (TV_ABI_VERSION at build time). */
int tv_abi_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* tv_last_error(void);

/* sizeof(tv_tree_attention_args) as compiled into the library, so bindings can
 * verify their struct layout before the first call. */
int64_t tv_sizeof_tree_attention_args(void);

/* ------------------------------------------------------------------------- */
/* store_kvcache  (layers/attention.py:15-45)                                 */
/* ------------------------------------------------------------------------- */
/*
 * For each row i < num_rows with slot = slot_mapping[i] != -1, copy row_elems
 * contiguous elements of key[i] and value[i] to k_cache/v_cache at element
 * offset slot * row_elems (the reference's `slot * D` addressing, which assumes a
 * cache whose slot rows are dense: stride(1) == row_elems).  Bit-exact copy.
 *   key/value row i starts at element i * key_row_stride / i * value_row_stride.
 *   slot_mapping is int32 (slot_is_int64 == 0) or int64.
 *   num_cache_slots bounds the slot; slots outside [0, num_cache_slots) other than
 *   -1 are skipped and reported through `status`.
 */
int tv_store_kvcache(const void* key, int64_t key_row_stride,
                     const void* value, int64_t value_row_stride,
                     void* k_cache, void* v_cache, int64_t num_cache_slots,
                     const void* slot_mapping, int32_t slot_is_int64,
                     int64_t num_rows, int64_t row_elems, int32_t elem_bytes,
                     int32_t* status, void* stream);

/* ------------------------------------------------------------------------- */
/* copy_accepted_kv  (speculative/jetspec/state.py:64-86)                     */
/* ------------------------------------------------------------------------- */
/*
 * kv_pool has shape [2, L, N, B, H, D] with the given element strides; a slot row
 * (H*D elements) must be dense: stride[5] == 1 and stride[4] == D.
 * For every kv in {0,1}, layer l < L and i < num_slots:
 *     pool[kv, l, dst[i] / B, dst[i] % B] = pool[kv, l, src[i] / B, src[i] % B]
 * with the reference's gather-then-scatter semantics: if any destination slot is
 * also a source slot, all sources are read before any destination is written
 * (through `workspace`), otherwise the rows are copied directly.  Destination
 * slots must be distinct: which source lands in a repeated destination is
 * unspecified, as in the reference's indexed assignment on the GPU.  Sources
 * may repeat.
 * workspace must hold tv_copy_accepted_kv_workspace_bytes(...) bytes.
 * On success *payload_bytes (host, may be NULL) receives 2*L*num_slots*H*D*elem,
 * the reference's return value.
 */
int64_t tv_copy_accepted_kv_workspace_bytes(int64_t num_slots, int64_t num_layers,
                                            int64_t row_elems, int32_t elem_bytes);

int tv_copy_accepted_kv(void* kv_pool, const int64_t pool_shape[6],
                        const int64_t pool_stride[6], int32_t elem_bytes,
                        const int64_t* source_slots, const int64_t* destination_slots,
                        int64_t num_slots, void* workspace, int64_t workspace_bytes,
                        int64_t* payload_bytes_host, int32_t* status, void* stream);

/*
 * The commit maps of a whole batch in one launch, replacing the per-request host
 * construction of speculative/jetspec/state.py:746-798 (`source =
 * nodes.index_select(0, path)`, :780; `destination = _slots_for_blocks(owned +
 * pending, len(path), B, start=cache_len)`, :782-785 with :54-61).  For request
 * r < num_requests and i < len_r = path_offsets[r+1] - path_offsets[r]:
 *     source_slots[path_offsets[r] + i]      = tree_slots[cu_seqlens[r] + paths[path_offsets[r] + i]]
 *     pos = cache_lens[r] + i
 *     destination_slots[path_offsets[r] + i] = block_tables[r*table_stride + pos/B]*B + pos%B
 * (all int32 inputs; slots int64).  A path that is empty, does not start at node 0, repeats a
 * node or names a node outside its tree (the reference's ValueErrors, :755-772), or a
 * position past the row's table_width pages or a page outside [0, num_blocks), sets
 * TV_STATUS_BAD_SLOT and writes -1 for every row of that request, so the following
 * tv_copy_accepted_kv writes nothing.
 */
int tv_commit_slots(const int64_t* tree_slots, const int32_t* cu_seqlens, const int32_t* paths,
                    const int32_t* path_offsets, const int32_t* block_tables, int64_t table_stride,
                    int32_t table_width, const int32_t* cache_lens, int32_t num_requests,
                    int32_t block_size, int64_t num_blocks, int64_t* source_slots,
                    int64_t* destination_slots, int32_t* status, void* stream);

/* ------------------------------------------------------------------------- */
/* HF-order RoPE + tree K/V scatter  (speculative/jetspec/tree_fusion.py)     */
/* ------------------------------------------------------------------------- */
/*
 * Replaces rope_scatter_prevalidated (tree_fusion.py:181-199) and its kernel
 * _rope_scatter_hf_order (tree_fusion.py:20-82); called per layer by
 * models/qwen3.py:223-240 in place of the eager RoPE + scatter of :241-258.
 * For every row i < rows, with pos = positions[i] and the cache row
 * cache[pos] = [cos_0..cos_{D/2-1} | sin_0..sin_{D/2-1}]:
 *     out[i, h]             = rope(q[i, h])        for every query head h
 *     k_pool[slot_i, h]     = rope(k[i, h])        for every KV head h
 *     v_pool[slot_i, h]     = v[i, h]              (bit copy)
 * where slot_i = node_slots[i] addresses page slot_i / page_size, offset
 * slot_i % page_size, and rope(x) = [x1*cos - x2*sin | x2*cos + x1*sin] over the
 * halves x1 = x[:D/2], x2 = x[D/2:] in HF order: for bf16 operands cos/sin are
 * first rounded to bf16, each of the four products is rounded to bf16 before the
 * add/subtract, and the result is rounded to bf16 (round to nearest even; a NaN
 * becomes 0x7FC0); for fp32 operands every product and sum is a separate fp32
 * operation (no fused multiply-add).
 * Elements are addressed through element strides (all positive); dtype is
 * TV_BF16 or TV_F32 for q/k/v/out/pools, cache_dtype TV_BF16 or TV_F32.
 * Node slots must be unique (one writer per K/V row); a position or slot out of
 * range sets TV_STATUS_BAD_POSITION / TV_STATUS_BAD_SLOT and that row writes
 * nothing.
 */
typedef struct tv_rope_scatter_args {
    const void* q;           int64_t q_stride[3];      /* [rows, q_heads, D] */
    const void* k;           int64_t k_stride[3];      /* [rows, kv_heads, D] */
    const void* v;           int64_t v_stride[3];
    const void* positions;   int64_t positions_stride; int32_t positions_is_int64;
    const void* cache;       int64_t cache_rows, cache_stride_row, cache_stride_elem;
    int32_t cache_dtype;
    void* k_pool;            int64_t k_pool_stride[4]; /* [pages, page_size, kv_heads, D] */
    void* v_pool;            int64_t v_pool_stride[4];
    int64_t pool_pages, page_size;
    const void* node_slots;  int64_t slots_stride;     int32_t slots_is_int64;
    void* out;               int64_t out_stride[3];    /* [rows, q_heads, D] */
    int64_t rows;
    int32_t q_heads, kv_heads, head_dim, dtype;
    int32_t* status;         /* optional */
} tv_rope_scatter_args;

int64_t tv_sizeof_rope_scatter_args(void);

int tv_rope_scatter(const tv_rope_scatter_args* args, void* stream);

/* ------------------------------------------------------------------------- */
/* greedy acceptance  (speculative/jetspec/serving_ops.py:55-90)              */
/* ------------------------------------------------------------------------- */
/*
 * out[r] = argmax_j logits[r * row_stride + j], j < vocab, in torch.argmax's order
 * (a NaN beats every number; equal values, or two NaNs, go to the lower index).
 * Replaces the `logits.argmax(-1)` of serving_ops.py:62.  dtype TV_BF16 or TV_F32.
 */
int tv_argmax_rows(const void* logits, int64_t rows, int64_t vocab, int64_t row_stride,
                   int32_t dtype, int64_t* out, void* stream);

/*
 * The per-request greedy walk of serving_ops.py:78-89 on the device.  Request r owns
 * packed rows [cu_seqlens[r], cu_seqlens[r+1]) holding its tree nodes in order
 * (node 0 = root); token_ids/parents/depths are per node (parents request-local,
 * -1 at the root), greedy is the per-row argmax.  From the root, the next node is
 * the child of the current node whose token equals greedy[current]; among sibling
 * nodes with that token the last one wins.  The walk stops at a miss or after
 * max_depth + 1 path nodes.  Writes paths[r * (max_depth + 1) + i] (root-inclusive,
 * -1 padded), lengths[r] = path nodes - 1 and corrections[r] = greedy of the last
 * path node.  A path node whose depth differs from its path index sets
 * TV_STATUS_BAD_DEPTH (the reference raises RuntimeError, serving_ops.py:84-85).
 */
int tv_tree_accept(const int64_t* greedy, const void* token_ids, int32_t tokens_is_int64,
                   const void* parents, int32_t parents_is_int64,
                   const void* depths, int32_t depths_is_int64,
                   const int32_t* cu_seqlens, int32_t num_requests, int32_t max_depth,
                   int32_t* paths, int32_t* lengths, int64_t* corrections,
                   int32_t* status, void* stream);

/*
 * The cut of each request's accepted outputs before its commit, replacing the host
 * loop of speculative/jetspec/batch_runtime.py:636-655, on tv_tree_accept's outputs.
 * For request r (path row r of path_stride int32, root-inclusive; lengths[r] draft
 * tokens accepted; token_ids per packed node, int32 or int64):
 *     values = token_ids[cu[r] + path[1..lengths[r]]] followed by corrections[r]
 *     limit  = min(len(values), budgets[r])          (max_new_tokens - len(output_ids))
 *     unless ignore_eos[r]: the first values[j], j < limit, equal to one of the
 *     num_eos eos_token_ids sets limit = j + 1.
 * Writes limits[r], emitted[r * path_stride + j] = values[j] for j < limit (-1 after),
 * and the cut paths path[0..limit) back to back: commit_paths[commit_offsets[r] + j],
 * commit_offsets[0..num_requests] (exclusive prefix sums of the limits), the packed
 * paths tv_commit_slots takes; commit_paths needs room for num_requests * path_stride.
 * A budget below 1, a length outside [0, path_stride) or a path node outside its
 * tree sets TV_STATUS_BAD_REQUEST and gives that request limit 0 (no committed rows).
 * One workgroup; num_requests == 0 writes nothing.
 */
int tv_truncate_accepted(const int32_t* paths, int32_t path_stride, const int32_t* lengths,
                         const int64_t* corrections, const void* token_ids, int32_t tokens_is_int64,
                         const int32_t* cu_seqlens, int32_t num_requests, const int32_t* budgets,
                         const uint8_t* ignore_eos, const int64_t* eos_token_ids, int32_t num_eos,
                         int32_t* limits, int64_t* emitted, int32_t* commit_paths,
                         int32_t* commit_offsets, int32_t* status, void* stream);

/* ------------------------------------------------------------------------- */
/* packed tree attention  (speculative/jetspec/paged_backend.py:240-306)      */
/* ------------------------------------------------------------------------- */
/*
 * Work plan.  Splits the ragged batch into work items (request, KV-head group,
 * node block, prefix key range) ordered longest first, and merge groups for
 * requests whose prefix is split.  Pure host computation on the metadata's host
 * copies (PackedTreeMetadata.prefix_lengths / node_counts_host).
 * Call once with NULL outputs to learn the sizes (written to *info), then again
 * with buffers of at least info->num_items * 8 and info->num_groups * 8 int32.
 *   queries_per_kv: query heads per KV head, G (1 to 8, or 16); a work item holds
 *               256 score rows = (8 / HPW) * floor(32 / G) nodes x G heads x HPW KV heads
 *               (plus padding rows when G does not divide 32).
 *   num_compute_units: CUs of the target device (256 on MI355X).
 *   chunk_keys: 0 = automatic; > 0 forces every prefix chunk to that many keys
 *               (a multiple of 32), which makes per-request results independent
 *               of the rest of the batch.
 * Each request has 1 to 2048 tree nodes (a work item caches its tree's scratch slots in
 * LDS); larger trees return TV_ERR_UNSUPPORTED and run tv_tree_attention_fp32.
 * An item is 8 int32: request, first KV head, first node, prefix key begin, key end,
 * flags, partial-result slot (-1: unsplit), KV heads per item.  Flags: bit 0 = last
 * prefix chunk (that item also covers the tree), bit 1 = last node block of its
 * request, bits 8-15 = queries_per_kv.  tv_tree_attention checks every item against the
 * live device metadata: an item outside its request's prefix, or made for another
 * queries_per_kv, sets TV_STATUS_BAD_REQUEST and is skipped; a last chunk that ends
 * before the live prefix length, or a last node block that ends before the live node
 * count, sets TV_STATUS_STALE_PLAN (the plan's keys and rows are computed, the rest of
 * the grown request is not).  A merge group is 8 int32: request, first KV head, first
 * node, KV heads per item, first partial slot, partial count, queries_per_kv, 0; a group
 * made for another queries_per_kv sets TV_STATUS_BAD_REQUEST and writes nothing.
 */
typedef struct tv_attention_plan_info {
    int32_t num_items;
    int32_t num_groups;
    int32_t num_partial_slots;
    int32_t ancestor_words_per_row;  /* ceil(max node count / 64) */
    int64_t workspace_bytes;         /* device workspace tv_tree_attention needs (head_dim <= 128) */
} tv_attention_plan_info;

int tv_tree_attention_plan(const int32_t* prefix_lens_host, const int32_t* node_counts_host,
                           int32_t num_requests, int32_t num_kv_heads, int32_t queries_per_kv,
                           int32_t block_size,
                           int32_t num_compute_units, int32_t chunk_keys,
                           int32_t* items_host, int32_t* groups_host,
                           tv_attention_plan_info* info);

/*
 * The plan of a slot-addressed launch (tv_tree_attention_args.prefix_slots set): the same
 * items, with every prefix chunk at most 2048 keys (the keys' slots are cached per work
 * item, beside at most 1024 tree nodes per request) and no page-size constraint.  Replaces the grid of the legacy single-request
 * kernel, paged_backend.py:343-348.
 */
int tv_tree_attention_plan_slots(const int32_t* prefix_lens_host, const int32_t* node_counts_host,
                                 int32_t num_requests, int32_t num_kv_heads, int32_t queries_per_kv,
                                 int32_t num_compute_units, int32_t chunk_keys,
                                 int32_t* items_host, int32_t* groups_host,
                                 tv_attention_plan_info* info);

/*
 * Device-side planner: the same items and groups as tv_tree_attention_plan, item for
 * item, computed on the device from device prefix_lens / node_counts, so a launch
 * sequence keeps fixed grids while prefix lengths change (HIP graph replay, the
 * equivalent of target_graph.py:95-167 reading live metadata).  No counterpart kernel
 * in the reference: its Triton kernels read prefix lengths in every program.
 * tv_tree_attention_plan_capacity gives capacities that hold for any prefix length up
 * to max_prefix with these node counts (items <= the smaller of 2 x CUs + sum of
 * node-block groups x (1 + chunks forced by the LDS page cache) and groups x
 * ceil(max_prefix / 64), or groups x ceil(max_prefix / chunk_keys) for a forced chunk
 * length), and the workspace those need.
 * tv_tree_attention_plan_device writes items [item_capacity, 8], groups
 * [group_capacity, 8] and counts[4] = {items, groups, partial slots, error}; on overflow
 * it writes zero counts and error 1 instead of overrunning the arrays.
 */
int tv_tree_attention_plan_capacity(const int32_t* node_counts_host, int32_t num_requests,
                                    int32_t num_kv_heads, int32_t queries_per_kv, int32_t block_size,
                                    int32_t num_compute_units, int32_t chunk_keys, int64_t max_prefix,
                                    tv_attention_plan_info* info);

int tv_tree_attention_plan_device(const int32_t* prefix_lens, const int32_t* node_counts,
                                  int32_t num_requests, int32_t num_kv_heads, int32_t queries_per_kv,
                                  int32_t block_size,
                                  int32_t num_compute_units, int32_t chunk_keys, int32_t item_capacity,
                                  int32_t group_capacity, int32_t slot_capacity, int32_t* items,
                                  int32_t* groups, int32_t* counts, void* stream);

/*
 * Capacities like tv_tree_attention_plan_capacity, but holding for EVERY batch of one
 * graph signature of speculative/jetspec/target_graph.py:24-27: num_requests requests,
 * total_queries packed rows and (when > 0) sum_node_squares = sum_r T_r^2 (the
 * qq_bias element count), whatever the individual node counts.  The reference's
 * PackedTargetGraph replays one captured graph for all of them (target_graph.py:150-167),
 * so a captured launch must be sized for the whole class:
 *     max T <= min(2048, Q - (R - 1), floor(sqrt(sum T^2)))
 *     node blocks <= Hkv * min((Q + (N - 1) R) / N, R * ceil(max T / N)),
 * N = 256 / queries_per_kv nodes per one-head work item.
 */
int tv_tree_attention_plan_capacity_packed(int32_t total_queries, int32_t num_requests,
                                           int64_t sum_node_squares, int32_t num_kv_heads,
                                           int32_t queries_per_kv, int32_t block_size,
                                           int32_t num_compute_units,
                                           int32_t chunk_keys, int64_t max_prefix,
                                           tv_attention_plan_info* info);

/*
 * Whether `stream` is being captured into a graph: *capturing = 1 while capture is
 * active, 0 when it is not, -1 when the capture was invalidated; *capture_id identifies
 * the capture sequence (0 when not capturing).  The drop-in attention wrapper uses it
 * to enqueue the live-metadata preparation (ancestor words + device plan) once at the
 * start of each captured graph, so replays follow the metadata staged into the
 * captured buffers (target_graph.py:55-75,150-167), as the reference's kernels do by
 * reading prefix_lens in every program (paged_backend.py:138).
 */
int tv_stream_capture_info(void* stream, int32_t* capturing, uint64_t* capture_id);

/*
 * Packs the request-local additive ancestor bias of PackedTreeMetadata
 * (qq_bias f32, 0 = visible / -inf = hidden, row-major [local_q * T + node] at
 * qq_bias_offsets[r]; packed_metadata.py:93-100) into one bit per (row, node):
 * words[q * words_per_row + w] bit b is set iff node m = 64w + b satisfies
 * m < T, m <= local_q and qq_bias[...] == 0.  An entry with m <= local_q that is
 * neither 0 nor -inf (the reference would add it to the score) sets
 * TV_STATUS_BAD_BIAS: bits cannot carry it.
 */
int tv_pack_ancestor_words(const float* qq_bias, const int64_t* qq_bias_offsets,
                           const int32_t* query_to_request, const int32_t* query_local_row,
                           const int32_t* node_counts, int32_t total_queries,
                           int32_t num_requests, int32_t words_per_row,
                           uint64_t* words, int32_t* status, void* stream);

/*
 * Device-side construction of the same bits from the tree topology, replacing the
 * host-built f32 bias of packed_metadata.py:185-195 on the serving path: parents
 * holds every packed node's request-local parent (-1 at node 0, else < the node),
 * request r owns rows [cu_seqlens[r], cu_seqlens[r+1]) with at most max_nodes
 * (<= 1024) nodes, and words_per_row >= ceil(max_nodes / 64) (<= 16).
 * words[q * words_per_row + w] bit b is set iff node 64w + b is q itself or one of
 * its ancestors.  A malformed parent sets TV_STATUS_BAD_REQUEST (that node is then
 * treated as a root).
 */
int tv_ancestor_words_from_parents(const int32_t* parents, const int32_t* cu_seqlens,
                                   int32_t num_requests, int32_t max_nodes, int32_t words_per_row,
                                   uint64_t* words, int32_t* status, void* stream);

/*
 * The reference's additive bias (packed_metadata.py:96-100) from ancestor words:
 * qq_bias[qq_bias_offsets[r] + i * T + m] = 0 if bit m of row (r, i) is set, else
 * -inf, for every packed row q = (query_to_request[q], query_local_row[q]).
 */
int tv_bias_from_ancestor_words(const uint64_t* words, int32_t words_per_row,
                                const int32_t* query_to_request, const int32_t* query_local_row,
                                const int32_t* node_counts, const int64_t* qq_bias_offsets,
                                int32_t total_queries, float* qq_bias, void* stream);

typedef struct tv_tree_attention_args {
    /* q [Q, Hq, D]; head dim contiguous */
    const void* q;
    int64_t q_stride_row, q_stride_head;
    /* k/v pools [N, B, Hkv, D]; stride[3] must be 1 */
    const void* k_pool;
    const void* v_pool;
    int64_t k_stride[4];
    int64_t v_stride[4];
    int64_t num_blocks;
    int32_t in_dtype;                    /* TV_BF16 or TV_F16 */
    /* out [Q, Hq, D]; head dim contiguous */
    void* out;
    int64_t out_stride_row, out_stride_head;
    int32_t out_dtype;                   /* in_dtype or TV_F32 */
    /* PackedTreeMetadata device buffers (packed_metadata.py:17-26) */
    const int32_t* cu_seqlens_q;         /* [R+1] */
    const int32_t* prefix_lens;          /* [R] */
    const int32_t* node_counts;          /* [R] */
    const int32_t* block_tables;         /* [R, table_stride], pad -1 */
    int64_t block_table_stride;
    const int64_t* tree_slots;           /* [Q] */
    /* derived per metadata: tv_pack_ancestor_words */
    const uint64_t* ancestor_words;
    int32_t ancestor_words_per_row;
    /* geometry */
    int32_t num_requests, total_queries, num_q_heads, num_kv_heads, head_dim, block_size;
    float scale;
    /* plan: tv_tree_attention_plan, copied to the device */
    const int32_t* items;
    int32_t num_items;
    const int32_t* groups;
    int32_t num_groups;
    int32_t num_partial_slots;
    void* workspace;
    int64_t workspace_bytes;
    int32_t* status;                     /* optional */
    /* optional: counts written by tv_tree_attention_plan_device ({items, groups, slots, error}).
     * When set, num_items / num_groups / num_partial_slots are launch capacities and the
     * kernels read the live counts from here (a graph-capturable launch). */
    const int32_t* device_counts;
    /* optional: slot addressing of the prefix, the legacy single-request form of
     * paged_backend.py:20-113 (a logical slot per key instead of a page table).  When set,
     * prefix key k of request r is read at slot prefix_slots[r * prefix_slots_stride + k]
     * (int64 if prefix_slots_is_int64, else int32; page slot / block_size, offset
     * slot % block_size), block_tables is not read, block_size may be any positive value,
     * the plan must come from tv_tree_attention_plan_slots, and exact_probabilities must
     * be set (the legacy kernel is an FP32 one). */
    const void* prefix_slots;
    int64_t prefix_slots_stride;
    int32_t prefix_slots_is_int64;
    /* nonzero: keep each probability to ~2^-17 relative in the P.V product (two MFMAs:
     * its operand-type rounding and the rounding of the remainder) and sum them in fp32,
     * for the reference's FP32 entries (tree_attention.py:1-10, paged_backend.py:248-256:
     * "never BF16 probabilities"); zero: one operand-type rounding (tree_gqa.py:102-105). */
    int32_t exact_probabilities;
} tv_tree_attention_args;

/*
 * out[q, h, :] = softmax_k(scale * q[q,h,:] . K[k, h/G, :]) V[k, h/G, :] over the
 * keys visible to packed row q of request r: every committed prefix position
 * < prefix_lens[r] (addressed through block_tables), plus every tree node m of r
 * whose ancestor bit is set (addressed through tree_slots).  bf16/f16 operands,
 * fp32 accumulation and online softmax, probabilities rounded to the operand
 * type for the P.V product (tree_gqa.py:102-105).
 * Implemented geometry: num_q_heads == G * num_kv_heads with head_dim 128 and G in
 * 1..8 or 16, or head_dim 64 or 256 and G in 1, 2, 4, 8, 16 (the reference's grouped
 * kernel takes powers of two up to 16 and pads the head size to a power of two,
 * tree_gqa.py:124-135; its FP32 kernel any geometry, as tv_tree_attention_fp32 does),
 * block_size % 32 == 0 (any positive block_size with prefix_slots), at most 2048 tree
 * nodes per request (1024 with prefix_slots) and ancestor_words_per_row <= 32.  The plan must
 * have been made for the same G; plans do not depend on head_dim.  workspace_bytes must
 * be at least tv_tree_attention_workspace_bytes(num_partial_slots, head_dim).
 */
int tv_tree_attention(const tv_tree_attention_args* args, void* stream);

/*
 * Split-prefix workspace tv_tree_attention needs for a plan with num_partial_slots partial
 * slots at head size head_dim: the plan's workspace_bytes for head sizes up to 128, twice
 * its partial-row area at 256.  No counterpart in the reference (its kernels keep no
 * partial results).
 */
int64_t tv_tree_attention_workspace_bytes(int32_t num_partial_slots, int32_t head_dim);

/*
 * FP32 tree attention for every geometry the reference accepts: the MI355X form of
 * the reference's scalar FP32 kernel _packed_paged_tree_fp32 (paged_backend.py:116-213),
 * which its dispatcher runs for every batch outside its fast kernel's geometry
 * (paged_backend.py:288-306), and of the legacy slot-addressed kernel
 * (paged_backend.py:20-113).  Replaces them where tv_tree_attention's MFMA kernel does
 * not apply: f32 operands, head sizes other than 64, 128 and 256 (1..512), query-head groups
 * the MFMA instances do not take (any number per KV head), page sizes that are not
 * multiples of 32, trees above 2048 nodes (above 1024 beside slot-addressed prefixes), and
 * finite qq_bias values (added to the score, as the reference does).
 *
 * out[q, h, :] = sum_k p_k V[k, h/G, :] / sum_k p_k with p_k = exp(s_k - max s) and
 * s_k = scale * q[q,h,:] . K[k, h/G, :] (+ qq_bias[bias_off[r] + local * T + j] for tree
 * key j); key position pos of request r is visible iff pos <= P + local.  Arithmetic,
 * probabilities and the online softmax are fp32.  No plan or workspace: one wave per
 * (packed row, KV head), reading every metadata value from device memory, so the launch
 * is graph-capturable as is.  Out-of-range pages or slots set TV_STATUS_BAD_PAGE and
 * that key is skipped; a row naming a nonexistent request sets TV_STATUS_BAD_REQUEST.
 */
typedef struct tv_tree_attention_fp32_args {
    /* q [Q, Hq, D], head dim contiguous */
    const void* q;
    int64_t q_stride_row, q_stride_head;
    /* k/v pools [N, B, Hkv, D], any element strides */
    const void* k_pool;
    const void* v_pool;
    int64_t k_stride[4];
    int64_t v_stride[4];
    int64_t num_blocks;
    int32_t in_dtype;                    /* TV_F32, TV_BF16 or TV_F16 (q, k and v) */
    /* out [Q, Hq, D], head dim contiguous */
    void* out;
    int64_t out_stride_row, out_stride_head;
    int32_t out_dtype;                   /* TV_F32, TV_BF16 or TV_F16 */
    /* PackedTreeMetadata device buffers (packed_metadata.py:17-26) */
    const int32_t* cu_seqlens_q;         /* [R+1] */
    const int32_t* query_to_request;     /* [Q] */
    const int32_t* query_local_row;      /* [Q] */
    const int32_t* prefix_lens;          /* [R] */
    const int32_t* node_counts;          /* [R] */
    const int32_t* block_tables;         /* [R, table_stride]; unused with prefix_slots */
    int64_t block_table_stride;
    const int64_t* tree_slots;           /* [Q] */
    const float* qq_bias;                /* per request [T, T], added to tree-key scores */
    const int64_t* qq_bias_offsets;      /* [R+1] */
    /* optional slot addressing of the prefix (legacy form), as in tv_tree_attention_args */
    const void* prefix_slots;
    int64_t prefix_slots_stride;
    int32_t prefix_slots_is_int64;
    int32_t num_requests, total_queries, num_q_heads, num_kv_heads, head_dim, block_size;
    float scale;
    int32_t* status;                     /* optional */
} tv_tree_attention_fp32_args;

int tv_tree_attention_fp32(const tv_tree_attention_fp32_args* args, void* stream);
/* sizeof(tv_tree_attention_fp32_args) as compiled, for binding layout checks. */
int64_t tv_sizeof_tree_attention_fp32_args(void);

/*
 * Allocation-free variant of tv_tree_attention.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under graph capture, tight serving
 * loops, harnesses that forbid allocation).  Same arguments, except that `workspace` and
 * `workspace_bytes` are ignored: split prefixes keep their partial results in a scratch
 * array built into the library, one per device, of tv_tree_attention_noalloc_max_workspace()
 * bytes (64 MiB: 504 partial slots up to head size 128, 254 at 256; about two rounds of work
 * items on 256 CUs), held until
 * the process ends.  A plan whose partial slots need more returns TV_ERR_CAPACITY and
 * launches nothing.  Every call on one device shares that device's scratch, so calls that
 * overlap on one device (concurrent streams) race; calls ordered on one stream do not.
 * The scratch is the one of the device that `stream` belongs to; its address is looked up
 * (hipGetSymbolAddress, with that device current) on the first call for that device, which
 * may happen under graph capture.
 * No hipMalloc, hipFree or allocating library routine is called.
 */
int tv_tree_attention_noalloc(const tv_tree_attention_args* args, void* stream);

int64_t tv_tree_attention_noalloc_max_workspace(void);

#ifdef __cplusplus
}
#endif

#endif /* TREEVERIFY_H */
