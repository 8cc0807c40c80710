/*
 * beam_engine_amd -- C ABI of the MI355X (gfx950) beam-decode hot path.
 *
 * Plain C: no C++ types, no exceptions, no torch types.  Device pointers are
 * passed as void* / typed pointers, streams as void* (a hipStream_t, NULL for
 * the default stream).  Every function returns a be_status; on failure
 * be_last_error() returns a message for the calling thread.  The library
 * never allocates or frees device memory: the caller owns every buffer,
 * including the workspace.
 *
 * Reference interfaces replaced (paths relative to brian030128/beam_engine):
 *   be_kv_append      flashinfer.page.append_paged_kv_cache as called by
 *                     PageTable.write_blocks_vectorized (src/beam_engine/page_table.py:167-209)
 *   be_rope_qkv_append apply_rotary_pos_emb + write_blocks_vectorized of a decode layer
 *                     (src/beam_engine/models/modeling_llama.py:460-465, 506-514)
 *   be_page_copy      PageTable.copy_block's per-layer copy loop
 *                     (src/beam_engine/page_table.py:96-106), batched over forks and layers
 *   be_page_copy_counted  the same with the copy count read on the device (graph capture)
 *   be_attn_plan      MultiLevelCascadeAttentionWrapper.plan
 *                     (src/beam_engine/models/modeling_llama.py:732-755); over the levels of
 *                     be_trie_levels it is also the vnode layout step of FastTree's
 *                     prepare_fasttree_metadata_for_paged_cache
 *                     (src/beam_engine/attention/fasttree/preparation.py:107-225)
 *   be_attn_run       MultiLevelCascadeAttentionWrapper.run (models/modeling_llama.py:362); on a
 *                     plan of FastTree levels, fasttree_decode's two stages
 *                     (src/beam_engine/attention/fasttree/kernel.py:288-348), reading the paged
 *                     cache in place of the K / V copies of models/modeling_llama.py:369-425
 *   be_trie_levels    FastTree's per-edge SplitQ / SplitK decision over the trie
 *                     (src/beam_engine/attention/fasttree/preparation.py:34-105) with its inputs
 *                     (BeamState.get_fasttree_input, src/beam_engine/beam_state.py:414-633), the
 *                     flat / split / per-step-picked decompositions, and the cascade levels
 *   be_trie_plan_kind the per-step metadata + plan of either reference kernel_type
 *                     (src/beam_engine/beam.py:168-206; models/modeling_llama.py:732-773)
 *   be_merge_states   the log-sum-exp merge inside the cascade wrapper and FastTree stage 2
 *                     (src/beam_engine/attention/fasttree/kernel.py:188-285)
 *   be_beam_topk      log_softmax + per-row topk (src/beam_engine/beam.py:269-276, prefill
 *                     :105-141) and VanillaBeamSearchStrategy.select_candidates
 *                     (src/beam_engine/beam_strategy.py:433-488)
 *   be_diverse_select DiverseBeamSearchStrategy.select_candidates, Hamming diversity
 *                     (src/beam_engine/beam_strategy.py:173-312)
 *   be_trie_cascade   BeamState.get_cascade_input (src/beam_engine/beam_state.py:211-412) and the
 *                     per-step write locations / position ids (src/beam_engine/beam.py:180-221)
 *   be_pages_*        PageTable.allocate_block / free_block (src/beam_engine/page_table.py:77-124)
 *   be_trie_*         BeamState.add_root_sequence / add_filtered_results
 *                     (src/beam_engine/beam_state.py:76-209)
 */
#ifndef BEAM_ENGINE_AMD_H
#define BEAM_ENGINE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage dtypes of K/V, queries, outputs and logits. */
enum be_dtype { BE_F32 = 0, BE_F16 = 1, BE_BF16 = 2 };

enum be_status {
  BE_OK = 0,
  BE_ERR_INVALID = 1,     /* bad argument or inconsistent indices (ValueError) */
  BE_ERR_HIP = 2,         /* a HIP runtime call failed (RuntimeError)          */
  BE_ERR_CAPACITY = 3,    /* caller buffer / workspace too small               */
  BE_ERR_UNSUPPORTED = 4  /* shape or dtype this build has no kernel for       */
};

/* Library version (major*10000 + minor*100 + patch). */
int be_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* be_last_error(void);

/* ------------------------------------------------------------------ KV cache
 * Per-layer cache layout (the reference's FlashInfer "NHD" layout,
 * page_table.py:62-72):  [num_pages, 2, page_size, num_kv_heads, head_dim],
 * K at index 0, V at index 1, head_dim contiguous.
 *
 * be_kv_append: for i < n, writes k[i] and v[i] ([num_kv_heads, head_dim] each,
 * element strides k_stride_n/k_stride_h, v_stride_n/v_stride_h, head_dim
 * contiguous) into slot pos[i] of page page_idx[i] of kv_layer.
 * Replaces append_paged_kv_cache (page_table.py:199-209).  num_pages bounds
 * the page ids (checked on the device: out-of-range entries are skipped and
 * counted in *err_count when err_count is non-NULL, a device int32).
 */
int be_kv_append(void* kv_layer, int dtype, int num_pages, int page_size, int num_kv_heads,
                 int head_dim, const int32_t* page_idx, const int32_t* pos, const void* k,
                 int64_t k_stride_n, int64_t k_stride_h, const void* v, int64_t v_stride_n,
                 int64_t v_stride_h, int n, int32_t* err_count, void* stream);

/* be_page_copy: for every c < n and every layer l < num_layers, copies the
 * first len[c] slots of K and of V of page src[c] into page dst[c].  Layer l's
 * cache starts at (char*)kv_pool + l * layer_stride_bytes.  src/dst/len are
 * device int32 arrays.  Replaces copy_block's loop over layers
 * (page_table.py:96-106) with one launch for all forks of a step.
 * Bounds (page ids < num_pages, 0 <= len <= page_size) are checked on the
 * device; offending entries are skipped and counted in *err_count. */
int be_page_copy(void* kv_pool, int64_t layer_stride_bytes, int num_layers, int dtype,
                 int num_pages, int page_size, int num_kv_heads, int head_dim,
                 const int32_t* src, const int32_t* dst, const int32_t* len, int n,
                 int32_t* err_count, void* stream);

/* be_page_copy_counted: be_page_copy over entries c < *count (count a device
 * int32, read by the kernel) of arrays holding max_n entries: a launch whose
 * size does not change with the number of copies, so that it can be captured
 * in a HIP graph once and replayed with each step's copy list written into
 * the same device arrays (the decode step's fork copies inside the step
 * graph).  *count must lie in [0, max_n]; the same checks as be_page_copy.
 * Replaces the same loop (page_table.py:96-106). */
int be_page_copy_counted(void* kv_pool, int64_t layer_stride_bytes, int num_layers, int dtype,
                         int num_pages, int page_size, int num_kv_heads, int head_dim,
                         const int32_t* src, const int32_t* dst, const int32_t* len,
                         const int32_t* count, int max_n, int32_t* err_count, void* stream);

/* be_rope_qkv_append: decode-step rotary embedding fused with the append.
 * qkv is the fused projection [n, (Hq + 2 Hkv) * head_dim] (row stride in
 * elements; q heads, then k heads, then v heads).  For every candidate i:
 * q_out[i] ([Hq, head_dim] contiguous) = RoPE(q, positions[i]); RoPE(k) and v
 * go to slot slot[i] of page page_idx[i] of kv_layer.  RoPE is the HF
 * rotate_half form with cos/sin tables [max_position, head_dim] in the storage
 * dtype, rounded like the eager tensor code:
 * round(round(x*cos) + round(rotate_half(x)*sin)).  Replaces
 * apply_rotary_pos_emb + write_blocks_vectorized of the decode layer
 * (src/beam_engine/models/modeling_llama.py:460-465, 506-514;
 * page_table.py:167-209).  Out-of-range positions / pages / slots are
 * skipped and counted in *err_count (device int32, may be NULL). */
int be_rope_qkv_append(const void* qkv, int64_t qkv_stride_n, int dtype, int n, int num_qo_heads,
                       int num_kv_heads, int head_dim, const int64_t* positions,
                       const void* cos_table, const void* sin_table, int max_position, void* q_out,
                       void* kv_layer, int num_pages, int page_size, const int32_t* page_idx,
                       const int32_t* slot, int32_t* err_count, void* stream);

/* ------------------------------------------------------------------ attention
 * One level of a cascade (FlashInfer's per-level index arrays as built by
 * BeamState.get_cascade_input, src/beam_engine/beam_state.py:211-412): group
 * j owns queries qo_indptr[j]..qo_indptr[j+1] and pages
 * kv_indices[kv_indptr[j]..kv_indptr[j+1]]; every page but the last is full
 * and the last holds last_page_len[j] tokens (0..page_size).  Host pointers.
 */
typedef struct be_level {
  const int32_t* qo_indptr;      /* num_groups + 1 */
  const int32_t* kv_indptr;      /* num_groups + 1 */
  const int32_t* kv_indices;     /* kv_indptr[num_groups] */
  const int32_t* last_page_len;  /* num_groups */
  int32_t num_groups;
} be_level;

/* Plan flags. */
#define BE_PLAN_FORCE_VALU 1     /* use the VALU kernel even where MFMA applies            */
#define BE_PLAN_FUSED_MERGE 2    /* merge split-K partials in the attention kernel's last-
                                    arriving workgroup instead of a second kernel (every
                                    workgroup then pays a device-scope release fence, an
                                    L2 writeback on gfx950, so this is off by default)    */
#define BE_PLAN_TILE_KERNEL 4    /* one workgroup per (work item, KV head) tile kernel even
                                    where the persistent streaming kernel applies         */
#define BE_PLAN_NO_TAIL 8        /* streaming kernel: keep short groups of few queries in the
                                    persistent kernel's tiles instead of tail chunks       */
#define BE_PLAN_TAIL_ROLE 16     /* streaming kernel: attend tail chunks in tail-role
                                    workgroups of the persistent kernel rather than in the
                                    merge kernel, whatever their count (by default: when a
                                    plan with streamed groups has at most 2 per query, or
                                    tail work of at least two thirds of its streamed tiles') */
#define BE_PLAN_NO_REGS 32       /* streaming kernel: the direct-load loop whatever the runs'
                                    lengths and roles (no register-staged loop; the 256-row
                                    wide roles otherwise stage through registers)           */
#define BE_PLAN_NO_WIDE 64       /* streaming kernel: no wide wave roles (32 rows per wave)
                                    and no 128-row segments for long many-query groups      */
#define BE_PLAN_CAUSAL 128       /* causal groups on the last level: query q0 + i of a group
                                    of n queries over kv_len tokens sees its first
                                    kv_len - n + i + 1 tokens (FlashInfer's causal prefill
                                    alignment; such plans run the tile / VALU kernels)     */

#define BE_PLAN_ROWS 256         /* decode plans: the merge-free row-block kernel (each workgroup
                                    owns up to 16 rows -- queries x GQA heads of one KV head --
                                    and all their groups on every level; no partials, one
                                    kernel) whenever it applies                             */
#define BE_PLAN_NO_ROWS 512      /* never the row-block kernel                               */
#define BE_PLAN_NO_WIDE256 1024  /* streaming kernel: wide roles on 128-row segments only    */
                                 /* (no 256-row segments for groups of >= 256 rows)         */
#define BE_PLAN_NO_TAIL_ROLE 2048 /* streaming kernel: tail chunks always in the merge kernel */

/* Fixed-capacity plan layout (for HIP-graph capture): every region of the
 * device plan sits at an offset that depends only on these capacities, the
 * live counts sit in a device header, and be_attn_run launches capacity-sized
 * grids whose surplus workgroups exit at once.  A plan that exceeds a capacity
 * fails with BE_ERR_CAPACITY. */
typedef struct be_plan_caps {
  int32_t max_items, max_queries, max_pages, max_merge, max_merge_rows, max_zero;
  int32_t tile_rows;       /* fixed rows per workgroup tile: 16, 32, 64 or 128 */
  int32_t max_tails;       /* streaming kernel: tail chunk entries (and tail-role items) */
} be_plan_caps;

/* Filled by be_attn_plan; passed back to be_attn_run unchanged. */
typedef struct be_attn_plan_info {
  int32_t num_items;       /* work items (grid.x of the attention kernel)      */
  int32_t num_part_rows;   /* partial rows: tile kernel [Hq, D] fp32 + [Hq] fp32 lse each;
                              streaming kernel (slots) [g, D] in the KV's 16-bit type + [g] fp32 lse */
  int32_t num_merge;       /* queries merged by the merge kernel               */
  int32_t num_queries;
  int32_t num_qo_heads, num_kv_heads, head_dim, page_size, num_pages, dtype;
  int32_t kernel;          /* 0 = VALU, 1 = MFMA tile, 2 = MFMA streaming (persistent),
                              3 = MFMA row blocks (one kernel, no merge)           */
  int32_t tile_rows;       /* rows (queries x GQA group) per MFMA tile: 16/32  */
  int32_t chunk_tokens;    /* split-K chunk length                             */
  int32_t plan_ints;       /* int32 words of the device plan                    */
  int32_t off_items, off_qindex, off_pages, off_merge_q, off_merge_ptr, off_merge_rows;
  int32_t off_q_merge;     /* per query: index into the merge list, or -1      */
  int32_t fused_merge;     /* 1: the attention kernel merges (no second kernel) */
  int32_t num_zero;        /* queries with no keys at all: o = 0, lse = -inf   */
  int32_t off_zero_q, off_zero_ptr;
  int32_t static_layout;   /* 1: fixed-capacity layout, counts in the device header */
  int32_t grid_items, grid_merge, grid_zero;   /* launch sizes (= counts, or capacities) */
  int32_t part_rows_cap;   /* partial rows the scratch is laid out for          */
  int64_t partial_bytes;   /* device scratch: partial o + lse + merge counters */
  int64_t counter_offset;  /* byte offset of the int32 merge counters in the scratch;
                              the caller zeroes counter_bytes there once after planning
                              (every run leaves them at zero again)            */
  int64_t counter_bytes;
  int64_t kv_bytes;        /* algorithmic K+V bytes: distinct (page, head) valid tokens */
  int64_t qo_bytes;        /* Q + O bytes                                       */
  double flops;            /* 4 * D * sum_q sum_h kv_len(q)                     */
  /* streaming kernel (kernel == 2): one workgroup per CU walks a contiguous,
   * byte-balanced run of (query tile, KV head, 64-token tile) segments;
   * partial results go to per-(query, KV head) slots merged by records.
   * num_items = segments, num_part_rows = slots, num_merge = records.   */
  int32_t num_wg;          /* persistent workgroups (grid of the attention kernel) */
  int32_t off_wg;          /* [num_wg][4]: first segment, segments, tiles, 0       */
  int32_t off_records;     /* [grid_merge][8]: query, KV head, first slot entry, slots,
                              first tail entry, tail entries, 0, 0                  */
  int32_t off_record_slots;/* slot ids of every record                             */
  /* Groups of at most 128 tokens and at most 4 queries (page_size a multiple of
   * 16) skip the persistent kernel: the merge kernel attends them per (query,
   * KV head) before it combines the slots.  Tail entries are 16-token chunks,
   * [num_tails][2]: page id, in-page token offset | valid tokens << 16. */
  int32_t num_tails;
  int32_t off_tails;
  int32_t tail_waves;      /* waves per record in the tail-and-merge kernel: 1, 2 or 4 */
  /* With BE_PLAN_TAIL_ROLE, the tail chunks are attended by tail-role
   * workgroups of the streaming kernel instead: items [n][8] (query, KV head,
   * first tail entry, entries, slot) whose results join the records as slots. */
  int32_t num_tail_items;
  int32_t off_tail_items;
  int32_t stream_loop;     /* streaming kernel's loop: 0 direct global->LDS loads, 1 register-staged */
  int32_t off_seg_causal;  /* causal plans: per segment, the tokens its first query sees (query j
                              of the segment sees that + j); 0 when the plan has no causal group */
} be_attn_plan_info;

/* be_attn_plan (host only): validates the levels against num_queries,
 * num_pages and page_size, splits every group into work items (query tiles x
 * KV chunks) and writes the device plan into host_plan[0..info->plan_ints).
 * The caller copies that prefix to device memory (stream-ordered before
 * be_attn_run) and provides info->partial_bytes of device scratch.
 * num_cus sizes the split-K chunking (pass the device's CU count).  caps
 * NULL gives a compact layout sized to this plan; non-NULL the fixed layout
 * above (the fused merge is not available with it). */
int be_attn_plan(const be_level* levels, int num_levels, int num_queries, int num_qo_heads,
                 int num_kv_heads, int head_dim, int page_size, int num_pages, int dtype,
                 int flags, int num_cus, const be_plan_caps* caps, int32_t* host_plan,
                 int64_t host_plan_capacity, be_attn_plan_info* info);

/* be_diverse_select: diverse beam search selection with the Hamming penalty
 * (DiverseBeamSearchStrategy.select_candidates, src/beam_engine/beam_strategy.py:173-312)
 * over the row top-k that be_beam_topk wrote (row_vals / row_idx, [n_rows, k],
 * rows in candidate order).  Per request (rows [req_row_ptr[r], req_row_ptr[r+1]),
 * or all rows when req_row_ptr is NULL and n_req == 1): num_groups groups pick
 * max(1, beam / num_groups) choices each, by log_prob - diversity_penalty when
 * an earlier group took the token, ties to the higher log_prob, then the
 * earlier (row, rank); the picks come out grouped by row (children in pick
 * order), at most beam of them: out_* [n_req * beam] as be_beam_topk's (parent
 * = global row, -1 for unused entries; score = parent_scores[row] + log_prob). */
int be_diverse_select(const float* row_vals, const int32_t* row_idx, int n_rows, int k, const double* parent_scores,
                      int n_req, const int32_t* req_row_ptr, int max_req_rows, int beam, int num_groups,
                      double diversity_penalty, int32_t* out_parent, int32_t* out_token, double* out_score,
                      void* stream);

/* ------------------------------------------------------------------ trie metadata
 * be_trie_cascade (host only): the per-level cascade index arrays of a live
 * beam trie -- what the reference's BeamState.get_cascade_input builds by
 * walking every candidate's path in Python (beam_state.py:211-412), with its
 * grouping, ordering and last_page_len rules -- plus each candidate's query
 * token, write page / slot and position (beam.py:180-221).
 * The trie is a node table: node n has parent[n] (-1 for a root, else an
 * older live node), page[n], ntok[n] tokens, last_tok[n] (its last token)
 * and alive[n]; leaves[c] is candidate c's node.  out receives int32 words:
 * [num_levels L, off_cand], L records [groups, off_qo, off_kv_indptr,
 * off_kv_indices, off_last_page_len] (word offsets into out), the arrays,
 * and at off_cand four arrays of num_cands: query tokens, write pages, write
 * slots, positions.  *out_used is the word count (also on BE_ERR_CAPACITY). */
int be_trie_cascade(const int32_t* parent, const int32_t* page, const int32_t* ntok, const int32_t* last_tok,
                    const uint8_t* alive, int num_nodes, const int32_t* leaves, int num_cands, int32_t* out,
                    int64_t out_capacity, int64_t* out_used);

/* Strategy kinds of be_trie_levels / be_trie_plan_kind. */
#define BE_KIND_CASCADE 0  /* the reference's cascade levels (be_trie_cascade)                  */
#define BE_KIND_FLAT 1     /* one pass per candidate over its whole path                        */
#define BE_KIND_SPLIT 2    /* one pass per trie segment, merged                                  */
#define BE_KIND_TREE 3     /* each edge absorbed or split by the cost model's edge decision      */
#define BE_KIND_AUTO 4     /* the cheapest of flat, split and tree under the fitted costs        */
#define BE_EDGES_FITTED 0  /* edge decisions by this build's fitted kernel costs                 */
#define BE_EDGES_FASTTREE 1 /* edge decisions by FastTree's padded-tile model (preparation.py:34-57) */

/* Kernel costs (microseconds per layer, the whole GPU) and the edge model of
 * the tree decompositions: tile_nt[i] one 64-token tile of one KV head with
 * i + 1 16-row MFMA tiles filled, seg a segment start, slot a partial slot
 * and its merge, tail a 16-token tail chunk, fixed a step's launches,
 * tile_w128 / tile_w256 a tile of the wide segments a group of more than 64
 * rows takes when it has at least 8 tiles and 64 x 256 tiles of 64 rows over
 * its KV heads; alpha, beta, gamma FastTree's Cmm constants
 * (metadata.py:12-17). */
typedef struct be_tree_model {
  double tile_nt[4];
  double seg, slot, tail, fixed;
  double alpha, beta, gamma;
  double tile_w128, tile_w256;   /* a 64-token tile of a 128 / 256-row wide segment, one KV head */
  double tile_sib;               /* a 64-token tile of a group's second or later 64-row query tile, one
                                    KV head (its K/V comes from the L2 its first tile's reads filled) */
  int32_t num_qo_heads, num_kv_heads;
  int32_t edge_model;
  int32_t reserved;
} be_tree_model;

/* be_trie_levels (host only): the levels of one strategy for the live trie,
 * laid out as be_trie_cascade lays them out (with the same candidate block).
 * BE_KIND_CASCADE is be_trie_cascade (include_self must be 0).  The other
 * kinds attend every candidate to its root-to-leaf path exactly once --
 * with its newest token when include_self is set (FastTree's req_to_token
 * covers the whole path, beam_state.py:512-564), without it otherwise (the
 * cascade convention) -- as passes over the trie's segments: flat absorbs
 * every edge, split none, tree decides each edge top down with the model
 * (FastTree's rule, attention/fasttree/preparation.py:60-105), auto builds the
 * cheapest of the three under the fitted costs.  model is needed for
 * BE_KIND_TREE and BE_KIND_AUTO.  *chosen receives the kind built;
 * option_costs (3 doubles, optional) the modelled flat / split / tree costs
 * under BE_KIND_AUTO. */
int be_trie_levels(const int32_t* parent, const int32_t* page, const int32_t* ntok, const int32_t* last_tok,
                   const uint8_t* alive, int num_nodes, const int32_t* leaves, int num_cands, int page_size, int kind,
                   int include_self, const be_tree_model* model, int32_t* out, int64_t out_capacity,
                   int64_t* out_used, int32_t* chosen, double* option_costs);

/* ------------------------------------------------------------------ page pool and beam trie (host only)
 * be_page_pool replaces the reference PageTable's allocator
 * (src/beam_engine/page_table.py:77-124): a FIFO free list (oldest free page
 * first, freed pages to the back) with a holder count per page.
 * be_pages_allocate fails with BE_ERR_CAPACITY ("No free pages available",
 * the reference's MemoryError); be_pages_release drops one holder and puts
 * the page back at zero, *state = 1 (freed), 0 (still held) or -1 (was not
 * allocated: the reference only warns); be_pages_share adds a holder;
 * be_pages_reserve takes one given free page out of the list; be_pages_free_list
 * copies up to cap free pages in list order and returns the free count. */
typedef struct be_page_pool be_page_pool;
be_page_pool* be_pages_create(int num_pages);
void be_pages_destroy(be_page_pool* pool);
int be_pages_allocate(be_page_pool* pool, int32_t* page);
int be_pages_share(be_page_pool* pool, int page, int32_t* count);
int be_pages_release(be_page_pool* pool, int page, int32_t* state);
int be_pages_reserve(be_page_pool* pool, int page);
int be_pages_num_free(const be_page_pool* pool);
int be_pages_ref_count(const be_page_pool* pool, int page);
int be_pages_free_list(const be_page_pool* pool, int32_t* out, int cap);

/* be_beam_trie replaces the reference BeamState's trie and its update
 * (src/beam_engine/beam_state.py:76-209, add_root_sequence and
 * add_filtered_results), with pages from a be_page_pool.
 * be_trie_add_root: a prompt's pages (one per page_size tokens, written to
 * pages_out) and its candidate (score 0).
 * be_trie_apply: one step's selection in emission order -- entry e gives
 * the parent candidate (-1: unused entry), the token and the accumulated
 * score; a candidate's children are its entries in order.  Childless
 * candidates are pruned first (leaf upward, freeing pages), then candidates
 * are expanded in order by the reference's fork rules; the fork copies
 * (source page, new page, tokens to copy) go to copies (3 words each, room
 * for n_entries needed), *n_copies their count.  eos_token >= 0 finishes a
 * beam on that token (kept with its whole sequence) instead of expanding it.
 * *n_release_warnings counts frees of pages the pool did not hold.
 * be_trie_sizes: [nodes, candidates, finished, finished tokens, page_size] and
 * the state's version (bumped by every change).  be_trie_candidates /
 * be_trie_export copy the candidates and the node table (parent, page,
 * token count, alive, page_size tokens per node) and the finished beams
 * (request, score, token offsets, tokens).  be_trie_metadata is
 * be_trie_cascade over the trie. */
typedef struct be_beam_trie be_beam_trie;
be_beam_trie* be_trie_create(int page_size, be_page_pool* pool);
void be_trie_destroy(be_beam_trie* trie);
int be_trie_add_root(be_beam_trie* trie, const int32_t* tokens, int n, int request_id, int32_t* pages_out);
int be_trie_apply(be_beam_trie* trie, const int32_t* sel_parent, const int32_t* sel_token, const double* sel_score,
                  int n_entries, int eos_token, int32_t* copies, int copies_cap, int* n_copies,
                  int* n_release_warnings);
int be_trie_sizes(const be_beam_trie* trie, int32_t* out5, int64_t* version);
int be_trie_candidates(const be_beam_trie* trie, int32_t* node, int32_t* request, double* score);
int be_trie_export(const be_beam_trie* trie, int32_t* parent, int32_t* page, int32_t* ntok, uint8_t* alive,
                   int32_t* tokens, int32_t* fin_req, double* fin_score, int32_t* fin_off, int32_t* fin_tokens);
int be_trie_metadata(const be_beam_trie* trie, int32_t* out, int64_t out_capacity, int64_t* out_used);
/* be_trie_metadata_kind: be_trie_levels over the trie (any strategy kind). */
int be_trie_metadata_kind(const be_beam_trie* trie, int kind, int include_self, const be_tree_model* model,
                          int32_t* out, int64_t out_capacity, int64_t* out_used, int32_t* chosen,
                          double* option_costs);
/* be_trie_plan: be_trie_metadata into meta, then be_attn_plan of its levels
 * (the cascade wrapper's plan of the step: causal mask on the last level when
 * a group there holds more than one query; num_pages from the largest page
 * id named, returned in *max_page) -- a cascade decode step's host work in
 * one call.  BE_ERR_CAPACITY for meta or host_plan as the two calls give it. */
int be_trie_plan(const be_beam_trie* trie, int num_qo_heads, int num_kv_heads, int head_dim, int dtype, int flags,
                 int num_cus, const be_plan_caps* caps, int32_t* meta, int64_t meta_capacity, int64_t* meta_used,
                 int32_t* host_plan, int64_t host_plan_capacity, be_attn_plan_info* info, int32_t* max_page);
/* be_trie_plan_kind: be_trie_plan for any strategy kind -- be_trie_levels
 * over the trie into meta, then be_attn_plan of its levels (the causal mask
 * only for BE_KIND_CASCADE, as be_trie_plan decides it; the other kinds'
 * multi-query groups are shared segments, not causal blocks).  Replaces the
 * reference's per-step dispatch on kernel_type (beam.py:168-206) with
 * get_cascade_input or get_fasttree_input + prepare_fasttree_metadata_for_paged_cache
 * (attention/fasttree/preparation.py:11-225) and the wrapper's plan. */
int be_trie_plan_kind(const be_beam_trie* trie, int kind, int include_self, const be_tree_model* model,
                      int num_qo_heads, int num_kv_heads, int head_dim, int dtype, int flags, int num_cus,
                      const be_plan_caps* caps, int32_t* meta, int64_t meta_capacity, int64_t* meta_used,
                      int32_t* host_plan, int64_t host_plan_capacity, be_attn_plan_info* info, int32_t* max_page,
                      int32_t* chosen, double* option_costs);

/* be_attn_run: o[i, h] = softmax(sm_scale * q[i, h] . K^T) V over query i's
 * groups on every level, merged by log-sum-exp; query head h reads KV head
 * h / (Hq / Hkv).  q and out are [num_queries, Hq, D] with element strides
 * (n, h) and D contiguous; out has the plan's dtype.  lse (optional, device
 * float [num_queries, Hq]) receives the natural-log log-sum-exp; a query with
 * no keys gets o = 0 and lse = -inf.  dev_plan is the device copy of the plan,
 * partials points at info->partial_bytes of device scratch.  Runs of one plan
 * must be stream-ordered (they share the scratch and its merge counters).
 * phases selects the kernels launched (BE_RUN_ATTENTION | BE_RUN_MERGE for a
 * full run; the two halves may be issued separately, in that order). */
#define BE_RUN_ATTENTION 1   /* phases: the attention kernel                     */
#define BE_RUN_MERGE 2       /* phases: the split-K merge and zero-fill kernels   */
int be_attn_run(const be_attn_plan_info* info, const int32_t* dev_plan, void* partials,
                const void* q, int64_t q_stride_n, int64_t q_stride_h, const void* kv_layer,
                void* out, int64_t o_stride_n, int64_t o_stride_h, float* lse, float sm_scale,
                int phases, void* stream);

/* be_merge_states: (o, lse) <- merge((o_a, lse_a), (o_b, lse_b)) for n x heads
 * rows of head_dim; o_* are float [n, heads, D] contiguous, lse natural log.
 * o_out/lse_out may alias o_a/lse_a. */
int be_merge_states(const float* o_a, const float* lse_a, const float* o_b, const float* lse_b,
                    float* o_out, float* lse_out, int n, int heads, int head_dim, void* stream);

/* ------------------------------------------------------------------ beam top-k
 * be_beam_topk: one decode-step selection over logits [n_rows, vocab]
 * (dtype, row stride in elements).  The reference scales by the temperature
 * with `logits / temperature` when it is not 1 (src/beam_engine/beam.py:107,
 * :270); temp_mode picks the arithmetic of that division:
 *   BE_TEMP_RECIPROCAL  x' = round_dtype(x * fl32(1.0 / T)), the reciprocal taken in
 *                       double and rounded to float -- what torch runs for a
 *                       device tensor divided by a Python float (measured on
 *                       MI355X; the reference's logits live on the GPU);
 *   BE_TEMP_DIVIDE      x' = round_dtype(x / fl32(T)), correctly rounded in fp32 --
 *                       torch's CPU tensor division;
 * both leave x unchanged when T == 1.  Then
 *   logp = round_dtype(fl32(fl32(x' - max) - fl32(ln sum exp(x' - max))))
 *          with the exponential sum accumulated in float64;
 *   per row the k best (logp desc, index asc) -> row_vals/row_idx [n_rows, k];
 *   when beam > 0, for every request q < n_req (its rows are
 *   [req_row_ptr[q], req_row_ptr[q+1]), a device int32 array; NULL with
 *   n_req = 1 means all rows): the beam best of the request's pool
 *   total = parent_scores[r] + (double)row_vals[r, j] by (total desc,
 *   r*k + j asc), emitted grouped by row ascending and, within a row, in
 *   selection order, into out_parent (global row) / out_token (int32) and
 *   out_score (double) [n_req * beam].  max_req_rows bounds the rows of any
 *   request (host-side pool capacity check).
 * All pointers are device pointers.  workspace must hold
 * be_beam_topk_workspace_bytes(n_rows, vocab, k) bytes; its contents need no
 * initialisation (the call clears the per-request arrival counters at its
 * start), and calls that share one workspace must be stream-ordered.
 * Parity contract: the exponential sum is accumulated in float64 in a
 * reduction order of this library's own; L = fl32(ln S) then equals the
 * float64 oracle's whenever ln S lies more than ~1e-13 (relative) from an
 * fp32 rounding boundary -- torch's fp32 log_softmax agrees with this
 * contract to about 4e-6, so a near-tie whose order the fp32 rounding of L
 * decides may rank differently from the reference's GPU. */
#define BE_TEMP_RECIPROCAL 0
#define BE_TEMP_DIVIDE 1
int64_t be_beam_topk_workspace_bytes(int n_rows, int vocab, int k);
int be_beam_topk(const void* logits, int dtype, int n_rows, int vocab, int64_t row_stride,
                 double temperature, int temp_mode, int k, const double* parent_scores, int beam, int n_req,
                 const int32_t* req_row_ptr, int max_req_rows, float* row_vals, int32_t* row_idx,
                 int32_t* out_parent, int32_t* out_token, double* out_score, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* be_beam_topk_noalloc: be_beam_topk without a workspace argument and without
 * any allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Its scratch is a static 8 MiB
 * device array inside the library, one per GPU, held until the process ends
 * (its address looked up once per device on the first call there).  Shapes
 * whose be_beam_topk_workspace_bytes exceed 8 MiB are rejected with
 * BE_ERR_CAPACITY (e.g. 128 rows of a 128256 vocabulary with k = 32 need
 * 0.55 MB).  Every call on one GPU shares that scratch: calls that overlap on
 * one GPU (other streams, other host threads) race and must be serialised by
 * the caller.  Results are those of be_beam_topk with the same arguments. */
int be_beam_topk_noalloc(const void* logits, int dtype, int n_rows, int vocab, int64_t row_stride,
                         double temperature, int temp_mode, int k, const double* parent_scores, int beam,
                         int n_req, const int32_t* req_row_ptr, int max_req_rows, float* row_vals,
                         int32_t* row_idx, int32_t* out_parent, int32_t* out_token, double* out_score,
                         void* stream);

/* ------------------------------------------------------------------ measurement
 * be_read_probe: no counterpart in the reference -- the roofline measurement's
 * read ceiling.  Reads rows of row_bytes (16 bytes times a power of two, at
 * most 32 KiB) once with 16-byte loads, row r at base + (r % inner) * inner_stride + (r / inner) *
 * outer_stride bytes, over grid workgroups of 256 threads, and writes one
 * fold of the data per workgroup to sink[grid] (device uint32) so that no load
 * is dead.  One KV head's rows of a layer [P, 2, page, Hkv, D] at a time:
 * inner = P * 2 * page, inner_stride = Hkv * D * es, outer_stride = D * es,
 * row_bytes = D * es; a contiguous read: inner = rows, inner_stride =
 * row_bytes.  bench.py --workload read-ns times it over the north-star
 * layer. */
int be_read_probe(const void* base, int64_t rows, int64_t inner, int64_t inner_stride, int64_t outer_stride,
                  int row_bytes, uint32_t* sink, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BEAM_ENGINE_AMD_H */
