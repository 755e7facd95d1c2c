/*
 * vflorence_amd.h -- C ABI of the MI355X (gfx950) decode-step attention library and the
 * decoder-step kernels around it (residual + LayerNorm, log-softmax + rules + top-k,
 * the decoder's projections for a decode step's rows).
 *
 * Every entry point takes plain device pointers, element strides and sizes, and a
 * hipStream_t passed as `void *` (NULL = the legacy default stream).  No entry point
 * allocates device memory; the one that needs scratch space (vfl_copy_blocks with
 * overlapping pairs) takes it from the caller, or from a buffer the library holds in
 * each GPU's memory (vfl_copy_blocks_noalloc).  All work is enqueued asynchronously
 * on `stream`, in call order, so a caller that issues copy_blocks ->
 * reshape_and_cache -> attention_with_kv_cache on one stream gets the reference's
 * ordering.
 *
 * Return value: VFL_OK (0) or a negative VFL_E_* code; vfl_last_error() then holds
 * a message for the calling thread.  Arguments are validated on the host before
 * any launch; out-of-range block ids or slots found on the device are skipped
 * rather than dereferenced (see each entry point).
 *
 * Cache layout: tensors of the reference's shape [num_blocks][num_heads][block_size]
 *   [head_dim] (vflorence/engine/model_runner.py:66-77), contiguous, one per layer and
 *   per K / V.  K: token t of block b, head h at ((b * H + h) * block_size + t) *
 *   head_dim.  V: the same for fp32 pools; 16-bit pools store each [block][head] slice
 *   with tokens interleaved in groups of four, dim d of token t at
 *   (b * H + h) * head_dim * block_size + ((t / 4) * head_dim + d) * 4 + t % 4, so the
 *   matrix-core kernel reads 4 tokens of a dim as one 8-byte operand and a token's
 *   write spans one 512-byte run (head_dim 64).  The reference leaves the inside
 *   of a block to its attention backend ("internal layout determined by the selected
 *   ISA", AGENTS.md section 5.3); only these entry points address it, and whole-block
 *   operations (copy_blocks, zero-filling a pool) are layout-independent.
 */
#ifndef VFLORENCE_AMD_H
#define VFLORENCE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of caches, queries and outputs */
enum vfl_dtype { VFL_FLOAT32 = 0, VFL_BFLOAT16 = 1, VFL_FLOAT16 = 2 };

/*
 * What the rows of a row group share (vfl_get_scheduler_metadata's group_tables):
 *   VFL_GROUP_SHARED_TABLE  the group's rows are read through its first row's block
 *                           table and length (cross-attention: the beams of a request
 *                           over one encoder page list);
 *   VFL_GROUP_OWN_TABLES    every row keeps its own table and length; a block that
 *                           several rows of the group list at the same position is
 *                           read once for all of them (decoder self-attention: beams
 *                           whose copy-on-write forks share prefix blocks).  Any
 *                           partition of the rows gives the same results.
 */
enum vfl_group_tables { VFL_GROUP_SHARED_TABLE = 0, VFL_GROUP_OWN_TABLES = 1 };

/* bytes of the per-GPU staging buffer behind vfl_copy_blocks_noalloc (64 MiB) */
#define VFL_NOALLOC_STAGING_BYTES (64u << 20)

/* status codes */
enum vfl_status {
  VFL_OK = 0,
  VFL_E_INVALID = -1,     /* bad argument (shape, dtype, alignment, size)   */
  VFL_E_UNSUPPORTED = -2, /* valid but not built (head_dim, block_size ...) */
  VFL_E_LAUNCH = -3       /* HIP reported an error at launch                */
};

/* Message for the last failing call on this thread ("" if none). */
const char *vfl_last_error(void);

/* Library version, major * 10000 + minor * 100 + patch. */
int vfl_version(void);

/*
 * Replaces vllm_cpu_attn.get_isa(dtype, block_size, head_dim)
 * (vflorence/engine/model_runner.py:38).  There is one code path, so this returns
 * the GPU target the library was built for ("gfx950"), or NULL when the
 * (dtype, block_size, head_dim) combination has no kernel.  Kernels exist for fp32,
 * bf16 and fp16, block sizes 16 and 32 (the reference's aarch64 and x86 sizes,
 * vflorence/config.py:42), and the reference's head sizes (32, 48, 64, 80, 96, 112,
 * 128, 160, 192, 224, 256, 512: vflorence/layers/attention.py:6).  Row groups keeping
 * their own tables, group plans and the fused KV write have kernels for 16-bit caches
 * of head size 64 and 128 in 16-token blocks; other calls give the same results
 * through the one-row kernels (and a separate KV write).
 */
const char *vfl_get_isa(int dtype, int block_size, int head_dim);

/*
 * Replaces vllm_cpu_attn.reshape_and_cache(key, value, k_cache, v_cache,
 * slot_mapping, isa=) (vflorence/layers/attention.py:55-57 and
 * vflorence/engine/model_runner.py:252-259):
 *
 *   for t < num_tokens with 0 <= slot_mapping[t] < num_blocks * block_size:
 *     k_cache[slot / bs][h][slot % bs][:] = key[t][h][:]      (same for value)
 *
 * key / value are [num_tokens][num_heads][head_dim] with arbitrary token and head
 * strides (in elements) and a contiguous last dimension -- the strided views a
 * fused qkv projection produces.  Negative slots are skipped (padding tokens), as
 * are slots past the end of the pool.  Bit-exact copy.  block_size must be 16 or
 * 32, the block sizes the attention kernels read (VFL_E_UNSUPPORTED otherwise,
 * nothing launched).
 */
int vfl_reshape_and_cache(const void *key, const void *value,
                          int64_t key_stride_token, int64_t key_stride_head,
                          int64_t value_stride_token, int64_t value_stride_head,
                          void *k_cache, void *v_cache, const int64_t *slot_mapping,
                          int64_t num_tokens, int num_heads, int head_dim,
                          int block_size, int64_t num_blocks, int dtype, void *stream);

/*
 * Launch plan for vfl_attention_with_kv_cache.  Replaces
 * vllm_cpu_attn.get_scheduler_metadata(...) (vflorence/layers/attention.py:18-29,
 * vflorence/engine/model_runner.py:308-319): the CPU work partition becomes the
 * number of waves that split one (row group, head) context inside a workgroup.
 * Pure host computation; no device memory is touched.
 */
typedef struct vfl_sched_meta {
  int64_t num_rows;            /* query rows the plan was made for                  */
  int64_t num_groups;          /* row groups the plan was made for                  */
  int32_t num_heads;           /* heads the plan was made for                       */
  int32_t head_dim;            /* head size the plan was made for                   */
  int32_t max_blocks_per_seq;  /* block-table width; longer contexts are clamped    */
  int32_t waves_per_workgroup; /* waves splitting one (group, head) context: 1..8   */
  int32_t max_group_size;      /* largest row group (beams)                         */
  int32_t group_tables;        /* enum vfl_group_tables                             */
  /* Optional group plan (own-table groups, 16-bit caches): set by the caller after
   * vfl_get_scheduler_metadata, which leaves it NULL.  A device copy of what
   * vfl_build_group_plan wrote for this call's tables, lengths and groups; the launch
   * then reads each group's distinct blocks from it instead of walking the tables,
   * and runs group_plan_slots x num_heads workgroups.  For shared-table groups the same
   * fields carry slot descriptors (vfl_build_slot_descriptors). */
  const int32_t *group_plan;
  int64_t group_plan_stride;   /* words per slot (vfl_group_plan_stride)            */
  int64_t group_plan_slots;    /* slots the plan holds (>= its groups)              */
} vfl_sched_meta;

/*
 * num_rows:            query rows (sequences, beams included)
 * num_groups:          row groups (== num_rows when no rows are grouped)
 * max_blocks_per_seq:  width of the block table
 * max_group_size:      largest group, 1..8
 * waves_per_workgroup: 0 picks the library default, else 1, 2, 4 or 8
 * group_tables:        VFL_GROUP_SHARED_TABLE or VFL_GROUP_OWN_TABLES (what a
 *                      group's rows share; ignored when calls pass no group_start)
 */
int vfl_get_scheduler_metadata(int64_t num_rows, int64_t num_groups, int num_heads,
                               int head_dim, int block_size,
                               int64_t max_blocks_per_seq, int max_group_size,
                               int dtype, int waves_per_workgroup, int group_tables,
                               vfl_sched_meta *meta);

/*
 * Group plans: the per-step schedule of own-table row groups (a request's beams)
 * that the reference's get_scheduler_metadata computes per decode step
 * (vflorence/engine/model_runner.py:308-319), made once on the host and read by every
 * layer's self-attention launch.  Words of one slot for groups of up to
 * max_group_size rows (1..8) over block tables max_blocks_per_seq wide (<= 65536);
 * 0 for sizes out of range.
 */
int64_t vfl_group_plan_stride(int max_group_size, int64_t max_blocks_per_seq);

/*
 * Host function (all pointers host memory; no device call).  Writes plan, of
 * 4 + num_slots * stride int32: plan[0] = num_groups, then one slot per dispatch
 * position s < num_slots: group group_order[s] (s when group_order is NULL) for
 * s < num_groups, empty after.  A slot holds its group's first row and row count and,
 * position by position, each distinct block id in [0, num_blocks) that the group's
 * rows list there, with the rows that list it.  Arguments as for
 * vfl_attention_with_kv_cache (block_table / seq_lens / group_start / group_order of
 * the same call).  Fails when a group has more than 8 rows or stride is too small.
 */
int vfl_build_group_plan(const int32_t *block_table, int64_t block_table_stride,
                         int max_blocks_per_seq, const int32_t *seq_lens, int64_t num_rows,
                         const int32_t *group_start, const int32_t *group_order,
                         int64_t num_groups, int block_size, int64_t num_blocks,
                         int32_t *plan, int64_t num_slots, int64_t stride);

/*
 * Slot descriptors for shared-table row groups (the beams of a request reading its
 * encoder pages, vflorence/layers/attention.py:9-39 stage_cross): the per-batch part of
 * the reference's scheduler metadata for cross-attention, made on the host once per
 * batch composition.  Words of one slot for tables max_blocks_per_seq wide (0 when out
 * of range).  vfl_build_slot_descriptors (host memory, no device call) writes desc, of
 * num_slots * stride int32: slot s < num_groups holds group group_order[s] (s when
 * group_order is NULL) as [first row, rows, seq_lens[first row], 0, block_table[first
 * row][0 .. max_blocks_per_seq)], later slots [0, 0, 0, 0].  Passed (device copy) as
 * vfl_sched_meta.group_plan with VFL_GROUP_SHARED_TABLE groups and group_plan_stride /
 * group_plan_slots set, vfl_attention_with_kv_cache's 16-bit head-size-64/128 launch
 * reads each workgroup's group from its slot in one dependent load instead of three
 * (dispatch order, group start, then length and table); the call's group_start,
 * group_order, seq_lens and block_table must describe the same groups.
 */
int64_t vfl_slot_descriptor_stride(int64_t max_blocks_per_seq);
int vfl_build_slot_descriptors(const int32_t *block_table, int64_t block_table_stride,
                               int max_blocks_per_seq, const int32_t *seq_lens,
                               int64_t num_rows, const int32_t *group_start,
                               const int32_t *group_order, int64_t num_groups, int32_t *desc,
                               int64_t num_slots, int64_t stride);

/*
 * Host function (all pointers host memory; no device call).  Folds a decode step's
 * copy-on-write pairs into its group plan -- the batched block copy that replaces the
 * loop of vflorence/engine/model_runner.py:162-167, which the reference runs before the
 * step's KV writes (:284-286).  For each pair the plan entry holding block dst[i] gets
 * a copy flag and src[i] in place of dst[i]; vfl_self_attention_with_kv_write with that
 * plan then reads the source block, stores it whole with the row's new token in place
 * to the block of the row's slot -- dst[i], by the fused write's contract (a row's slot
 * is at its last context position, in a block no other row reads) -- in each layer's
 * launch for its own pools, and the step needs no vfl_copy_blocks launch.  Only the
 * fused launch may read a folded plan (the plain attention launch would read the
 * sources as the rows' blocks).  plan: the used slots of vfl_build_group_plan's output
 * (num_slots and stride as given to it).  Refused (VFL_E_INVALID, plan unchanged) when
 * a block is out of
 * [0, num_blocks), a destination repeats or is also a source, or a destination is not
 * exactly one single-row entry of the plan at that row's last position; the caller then
 * copies the pairs itself.
 */
int vfl_fold_plan_copies(int32_t *plan, int64_t num_slots, int64_t stride,
                         const int64_t *src, const int64_t *dst, int64_t num_pairs,
                         int64_t num_blocks);

/*
 * Replaces vllm_cpu_attn.attention_with_kv_cache(query, k_cache, v_cache, out,
 * query_start_loc, seq_lens, scale=, causal=, block_table=, scheduler_metadata=)
 * on its decode path (vflorence/layers/attention.py:61-72 for self-attention,
 * :98-109 for cross-attention): one query row per sequence,
 *
 *   out[r][h][:] = softmax_j(scale * <query[r][h], K_r[j][h]>) V_r[j][h]
 *
 * over j < seq_lens[r], where token j of row r lives in block
 * block_table[r][j / block_size] at offset j % block_size.  Decode queries sit at
 * the end of their context, so the reference's causal flag changes nothing here.
 *
 * Row groups: when group_start is non-NULL, group g owns rows group_start[g] ..
 * group_start[g+1]-1 (at most 8).  With meta->group_tables VFL_GROUP_SHARED_TABLE
 * (cross-attention beams) the rows must share one block-table row and one length, and
 * the kernel reads that row's K/V once for the whole group.  With
 * VFL_GROUP_OWN_TABLES every row keeps its own table and length, and each block that
 * several rows of a group list at the same position is read once (fp32 caches run
 * such groups row by row).  With group_start NULL every row is its own group
 * (num_groups == num_rows).
 * group_order (optional, int32 [num_groups]): a permutation of the groups giving
 * the dispatch order; NULL = natural order.  Longest first balances the tail of a
 * launch that runs in several rounds.  When every (group, head) workgroup is resident
 * at once, a CU receives the groups at order positions p, p + CUs / heads, ...; then
 * reversing every other run of CUs / heads groups of the longest-first order pairs long
 * with short groups on each CU.
 *
 * query: [num_rows][num_heads][head_dim], token / head strides in elements.
 * out:   [num_rows][num_heads][head_dim], contiguous.
 * block_table: int32, row stride block_table_stride >= meta->max_blocks_per_seq;
 *   only entries below min(ceil(seq_lens[r] / bs), meta->max_blocks_per_seq) are
 *   read (longer contexts are clamped to the table width).
 * Block ids outside [0, num_blocks) contribute nothing.  seq_lens[r] <= 0 gives a
 * zero output row.  Accumulation is fp32 for every element type.  One kernel
 * launch; no scratch memory.
 * meta: from vfl_get_scheduler_metadata for the same num_rows, num_groups,
 *   num_heads and head_dim (checked).
 */
int vfl_attention_with_kv_cache(const void *query, int64_t query_stride_token,
                                int64_t query_stride_head, const void *k_cache,
                                const void *v_cache, void *out,
                                const int32_t *seq_lens, const int32_t *block_table,
                                int64_t block_table_stride,
                                const int32_t *group_start, const int32_t *group_order,
                                int64_t num_rows, int64_t num_groups, int num_heads,
                                int head_dim, int block_size, int64_t num_blocks,
                                float scale, int dtype, const vfl_sched_meta *meta,
                                void *stream);

/*
 * The body of the reference's vflorence::self_attention op in one launch
 * (vflorence/layers/attention.py:53-73: reshape_and_cache of key/value at
 * slot_mapping, then attention_with_kv_cache over the updated cache), for one query
 * row per sequence.
 *
 * Precondition (what the block manager's copy-on-write guarantees,
 * vflorence/engine/block_manager.py:44-59): for every row r, slot_mapping[r] is
 * either negative, or the cache slot of position seq_lens[r]-1 of row r's block
 * table, or a slot that no row of this call attends to; and the block holding a
 * row's new token is read by no other row.  Then the result -- cache contents and
 * out -- equals reshape_and_cache followed by attention_with_kv_cache.  Callers that
 * cannot vouch for it use those two entry points.  fp32 caches, and head sizes other
 * than 64 and 128, run the two steps.
 *
 * key / value: [num_rows][num_heads][head_dim] with token / head strides in
 * elements (the strided views of a fused qkv projection).  Other arguments as for
 * vfl_attention_with_kv_cache; row groups (group_start non-NULL) need metadata made
 * with VFL_GROUP_OWN_TABLES.
 */
int vfl_self_attention_with_kv_write(const void *query, int64_t query_stride_token,
                                     int64_t query_stride_head, const void *key,
                                     int64_t key_stride_token, int64_t key_stride_head,
                                     const void *value, int64_t value_stride_token,
                                     int64_t value_stride_head, const int64_t *slot_mapping,
                                     void *k_cache, void *v_cache, void *out,
                                     const int32_t *seq_lens, const int32_t *block_table,
                                     int64_t block_table_stride, const int32_t *group_start,
                                     const int32_t *group_order, int64_t num_rows,
                                     int64_t num_groups, int num_heads, int head_dim,
                                     int block_size, int64_t num_blocks, float scale,
                                     int dtype, const vfl_sched_meta *meta, void *stream);

/*
 * Replaces ModelRunner._copy_blocks (vflorence/engine/model_runner.py:162-167):
 * for every cache c < num_caches and pair p < num_pairs,
 *   caches[c][dst[p]] = caches[c][src[p]]          (block_bytes bytes per block)
 * with the reference's gather-then-scatter semantics: every source is read before
 * any destination is written when `staging` is non-NULL (staging must hold
 * num_caches * num_pairs * block_bytes bytes); with staging NULL the caller
 * guarantees that no dst block is also a src block.  `caches` is a DEVICE array of
 * num_caches cache base pointers.  Pairs with an id outside [0, num_blocks) are
 * skipped.  block_bytes must be a multiple of 16 and every cache 16-byte aligned.
 */
int vfl_copy_blocks(void *const *caches, int num_caches, const int64_t *src,
                    const int64_t *dst, int64_t num_pairs, int64_t block_bytes,
                    int64_t num_blocks, void *staging, void *stream);

/*
 * No counterpart in the reference: vfl_copy_blocks for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same copy and semantics; with `staged` non-zero the
 * gather-then-scatter goes through a staging buffer of VFL_NOALLOC_STAGING_BYTES
 * bytes that is part of the library's code object: every GPU on which the library's
 * module is loaded (at its first kernel launch of any entry point) holds it until the
 * process ends, whether or not this entry point is ever called.
 * num_caches * num_pairs * block_bytes beyond that size is
 * refused with VFL_E_INVALID before anything is launched.  No device memory is
 * allocated.  Calls that overlap on one GPU (other streams, other threads) share that
 * buffer and race; serialise them.  The buffer keeps the last call's contents and
 * needs no clearing (every staged byte is written before it is read).
 */
int vfl_copy_blocks_noalloc(void *const *caches, int num_caches, const int64_t *src,
                            const int64_t *dst, int64_t num_pairs, int64_t block_bytes,
                            int64_t num_blocks, int staged, void *stream);

/*
 * The decoder layer's residual + LayerNorm (vflorence/models/bart.py:192-201:
 * `layer_norm(hidden + sublayer(hidden))`, torch ops in the reference, no
 * vllm_cpu_attn counterpart):
 *   out[r] = (s - mean(s)) / sqrt(var(s) + eps) * weight + bias,  s = x[r] + residual[r]
 * with s rounded to the element type first (the stored sum of a separate add), the
 * statistics (biased variance) in fp32.  Rows are `dim` contiguous elements at the
 * given row strides (elements); dim a multiple of 4, at most 4096; rows and
 * weight / bias aligned to 4 elements.  `out` may alias `x` or `residual`.
 */
int vfl_add_layer_norm(const void *x, int64_t x_stride, const void *residual,
                       int64_t residual_stride, const void *weight, const void *bias, void *out,
                       int64_t out_stride, int64_t rows, int dim, float eps, int dtype,
                       void *stream);

/*
 * The decoder's input embedding in one launch, replacing the lookups and LayerNorm of
 * vflorence/models/bart.py:260-264 (embed_tokens :24-39, embed_positions :12-21):
 *   t = token_table[ids[r]] * token_scale   (rounded to the element type; none at 1)
 *   p = position_table[positions[r] + position_offset]        (BART: offset 2)
 *   out[r] = LayerNorm(p + t) * weight + bias
 * with vfl_add_layer_norm's arithmetic (the sum rounded to the element type, fp32
 * statistics).  ids and positions are DEVICE int64 arrays of `rows` entries; a row whose
 * token or position index falls outside its table (token_rows, position_rows) is written
 * as NaN instead of reading past the table.  Same dim, alignment and stride rules as
 * vfl_add_layer_norm for the tables and out.
 */
int vfl_embed_layer_norm(const int64_t *ids, const int64_t *positions, int64_t rows,
                         const void *token_table, int64_t token_rows, int64_t token_stride,
                         float token_scale, const void *position_table, int64_t position_rows,
                         int64_t position_stride, int64_t position_offset, const void *weight,
                         const void *bias, void *out, int64_t out_stride, int dim, float eps,
                         int dtype, void *stream);

/*
 * Replaces the device work of ModelRunner._sample / _beam_search
 * (vflorence/engine/model_runner.py:355-398) and LogitsProcessor
 * (vflorence/layers/logits_processor.py:24-51) for the rules that need no token
 * history: per row r of `logits` ([rows][vocab], row stride in elements)
 *   score(t) = log_softmax(logits[r])(t)          (log_softmax != 0; else logits[r][t])
 * then, in the processors' order, with len = lengths[r]:
 *   len < min_length            -> the EOS tokens score -inf
 *   len == 1                    -> only the forced-BOS tokens remain, at score 0
 *   len == max_length - 1       -> only the forced-EOS tokens remain, at score 0
 *   always                      -> the suppressed tokens score -inf
 *   len == begin_index          -> the begin-suppressed tokens score -inf
 * and writes the k best (score, token) pairs, best first (ties: lower token first),
 * to scores / ids ([rows][k]).  rule_tokens is a DEVICE int32 array holding, in order,
 * n_eos EOS, n_suppress suppressed, n_begin begin-suppressed, n_bos forced-BOS and
 * n_forced_eos forced-EOS token ids.  1 <= k <= 16; lengths may be NULL only without
 * rule tokens.  Repetition penalty and n-gram bans (which read the history) are not
 * covered: their callers apply them before, on the logits.  scores and ids may be
 * device memory or pinned host memory (hipHostMalloc): the kernel stores straight into
 * either, so a caller that needs the result on the host synchronizes the stream and
 * reads it, with no copy launch.
 */
int vfl_logprob_topk(const void *logits, int64_t row_stride, int64_t rows, int vocab, int dtype,
                     const int64_t *lengths, const int32_t *rule_tokens, int min_length,
                     int max_length, int begin_index, int n_eos, int n_suppress, int n_begin,
                     int n_bos, int n_forced_eos, int log_softmax, int k, float *scores,
                     int64_t *ids, void *stream);

/* vfl_linear flags */
enum vfl_linear_flags {
  VFL_LINEAR_GELU = 1,     /* exact GELU after the bias (on the value rounded to the dtype) */
  VFL_LINEAR_X_PACKED = 2, /* x is a packed activation (layout below); x_stride ignored    */
  VFL_LINEAR_Y_PACKED = 4  /* y is written as a packed activation; y_stride ignored        */
};

/*
 * The decoder's projections for a decode step's rows: the fused q|k|v, the
 * self-attention output and the cross-attention query and output projections, and the
 * feed-forward block fc2(gelu(fc1(h))) (vflorence/models/bart.py:111,114,142,146 and
 * :192-201 -- nn.Linear in the reference, no vllm_cpu_attn counterpart):
 *   y[r][n] = act(sum_k x[r][k] * weight[n][k] + bias[n])     (bias may be NULL)
 * 16-bit x / weight / bias / y (dtype VFL_BFLOAT16 or VFL_FLOAT16), fp32 sums, rounded
 * once on the store (with VFL_LINEAR_GELU: rounded, then GELU in fp32, rounded again --
 * what a separate activation kernel computes).
 *
 * Packed layout (weights always; activations with the X/Y_PACKED flags): an [R][C]
 * array stored as 1024-byte blocks of 16 rows x 32 columns in the matrix cores' operand
 * order -- block (r, c), at element (r * C / 32 + c) * 512, holds row 16 r + l % 16,
 * columns 32 c + 8 (l / 16) .. +7 at element 8 l for l < 64 -- with R padded to a
 * multiple of 32: vfl_linear_packed_elems(R, C) elements.  vfl_pack_linear_weight
 * writes it for a weight (padding rows zero); a packed output leaves its padding rows
 * unwritten (they only reach output rows that are dropped).
 *
 * in_features a multiple of 256 (and out_features of 32 for a packed output); rows at
 * most 65535 * 32.  x and `packed` 16-byte aligned; an unpacked x has a row stride
 * (elements) that is a multiple of 8 and at least in_features.  Split-K over the 8
 * waves of a workgroup per 32 x 32 output tile: one memory round trip for the weight
 * when in_features <= 1024.
 */
int64_t vfl_linear_packed_elems(int rows, int cols);
int vfl_pack_linear_weight(const void *weight, int64_t weight_stride, int out_features,
                           int in_features, void *packed, int dtype, void *stream);
int vfl_linear(const void *x, int64_t x_stride, const void *packed_weight, const void *bias,
               void *y, int64_t y_stride, int64_t rows, int out_features, int in_features,
               int flags, int dtype, void *stream);

/*
 * Deferred LayerNorm across the decoder's projections (no vllm_cpu_attn counterpart:
 * BART's post-LN sublayers, h' = LN(h + y), vflorence/models/bart.py:259-261).
 *
 * vfl_linear_residual: a sublayer's output projection.  y becomes the pre-norm sum
 *   v[r][n] = rnd(rnd(sum_k x[r][k] W[n][k] + bias[n]) + h[r][n])
 * (rnd: rounding to the dtype, where the separate projection and residual + LayerNorm
 * kernels round) and y_stats[r][t] = (mean, sum of squared deviations) of v[r] over
 * features 32 t .. 32 t + 31.  h is `residual` itself when r_stats is NULL, else
 * LN(residual) under r_stats, r_gamma, r_beta, r_eps (an earlier call's v and stats).
 * out_features a multiple of 32; flags: VFL_LINEAR_X_PACKED only; y and residual 8-byte
 * aligned with row strides multiples of 4, r_gamma / r_beta 8-byte aligned; y_stats
 * [rows][out_features / 32] float pairs, not aliasing r_stats.
 *
 * vfl_linear_norm: a projection of h' = LN(v) given v and its statistics x_stats
 * ([rows][in_features / 32] pairs), with the LayerNorm folded into the weight:
 *   y[r][n] = act(rstd_r * (sum_k v[r][k] W'[n][k] - mean_r * u[n]) + folded_bias[n])
 * for packed_weight = the packed W' = rnd(W diag(gamma)), u[n] = sum_k W'[n][k] and
 * folded_bias = bias + W beta (fp32, in the caller's order), where the row's mean and
 * rstd combine its tiles: mean = sum_t m_t / T, M2 = sum_t M2_t + 32 sum_t (m_t - mean)^2,
 * rstd = 1 / sqrt(M2 / (32 T) + eps).  flags: VFL_LINEAR_GELU and VFL_LINEAR_Y_PACKED.
 *
 * vfl_layer_norm_apply: out = rnd((v - mean) * rstd * gamma + beta) per row from v's
 * statistics (dim a multiple of 32; 8-byte aligned operands, row strides multiples of 4).
 */
int vfl_linear_residual(const void *x, int64_t x_stride, const void *packed_weight,
                        const void *bias, const void *residual, int64_t r_stride,
                        const float *r_stats, const void *r_gamma, const void *r_beta,
                        float r_eps, void *y, int64_t y_stride, float *y_stats, int64_t rows,
                        int out_features, int in_features, int flags, int dtype, void *stream);
int vfl_linear_norm(const void *x, int64_t x_stride, const float *x_stats, float eps,
                    const void *packed_weight, const float *u, const float *folded_bias,
                    void *y, int64_t y_stride, int64_t rows, int out_features, int in_features,
                    int flags, int dtype, void *stream);
int vfl_layer_norm_apply(const void *v, int64_t v_stride, const float *v_stats,
                         const void *gamma, const void *beta, float eps, void *out,
                         int64_t out_stride, int64_t rows, int dim, int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VFLORENCE_AMD_H */
