/*
 * vfl_engine.h -- C ABI of the engine's native host core (CPU only, no HIP).
 *
 * Two objects:
 *
 *   vfl_pool    the paged KV block pool: per-block reference counts, a FIFO free list
 *               and the copy-on-write rule.  Replaces vflorence's BlockManager
 *               (vflorence/engine/block_manager.py:4-73) with the same observable
 *               behaviour: blocks leave the free list from the front and return to its
 *               back, a released table returns its blocks last block first, a fork
 *               shares every block of its parent, and a row about to write into a
 *               block that others still hold moves to a fresh copy -- except the last
 *               holder, which writes in place.
 *
 *   vfl_engine  the decode loop's host state: waiting and running hypotheses (token
 *               ids, block tables, cached-token counts, cumulative log-probs), request
 *               admission, the step's metadata written straight into the caller's
 *               (pinned) buffers, and the per-step greedy / beam-search updates.
 *               Replaces the per-step Python of Scheduler.schedule / postprocess
 *               (vflorence/engine/scheduler.py:35-127), the host half of
 *               ModelRunner._prepare (vflorence/engine/model_runner.py:273-341) and the
 *               candidate merge of ModelRunner._beam_search (model_runner.py:383-410).
 *
 * Conventions: functions return VFL_HOST_OK (0) or a negative VFL_HOST_E_* code, and
 * vfl_host_last_error() then holds a message for the calling thread.  Objects are not
 * thread-safe; one thread drives one engine (the reference's single in-flight step).
 */
#ifndef VFL_ENGINE_H
#define VFL_ENGINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum vfl_host_status {
  VFL_HOST_OK = 0,
  VFL_HOST_E_INVALID = -1, /* bad argument                                       */
  VFL_HOST_E_FULL = -2,    /* the block pool cannot cover the step (RuntimeError)  */
  VFL_HOST_E_STATE = -3    /* call out of order (e.g. update before schedule)      */
};

/* Message for the last failing call on this thread ("" if none). */
const char *vfl_host_last_error(void);

/* ------------------------------------------------------------------------------- */
/* vfl_pool                                                                          */
/* ------------------------------------------------------------------------------- */
typedef struct vfl_pool vfl_pool;

/* A pool of num_blocks blocks of block_size tokens, every block free (ids 0, 1, ...
 * in free-list order).  NULL on bad sizes. */
vfl_pool *vfl_pool_create(int32_t num_blocks, int32_t block_size);
void vfl_pool_destroy(vfl_pool *pool);
/* Every block free again, free list back in id order (after an aborted batch). */
void vfl_pool_reset(vfl_pool *pool);
int32_t vfl_pool_num_blocks(const vfl_pool *pool);
int32_t vfl_pool_num_free(const vfl_pool *pool);
/* Copies the num_blocks reference counts into out. */
void vfl_pool_refcounts(const vfl_pool *pool, int32_t *out);
/* Copies the free list, front first, into out (vfl_pool_num_free entries). */
void vfl_pool_free_list(const vfl_pool *pool, int32_t *out);

/*
 * Make the position `cached` of a row with block table `table[0..len)` writable
 * (BlockManager.ensure_capacity, block_manager.py:44-59).  Returns
 *   0  nothing to do (the block exists and this row is its only holder);
 *   1  the position starts a new block: *block is a fresh block to append;
 *   2  copy-on-write: the block at index cached / block_size is shared; *src is that
 *      block (its count drops by one), *block a fresh block that replaces it in the
 *      table, to be filled with a copy of *src before the write;
 * or VFL_HOST_E_FULL when no block is free (nothing changed).  The table itself is
 * not modified: the caller applies the append or the replacement.
 */
int vfl_pool_prepare_write(vfl_pool *pool, const int32_t *table, int32_t len, int32_t cached,
                           int32_t *block, int32_t *src);

/*
 * Blocks one pass of vfl_pool_prepare_write over `rows` rows would take
 * (BlockManager.required_new_blocks, block_manager.py:28-42): write_block[r] is the
 * block row r writes into, or -1 when its position starts a new block.  A shared
 * block costs one copy per writer except the last of its holders.
 */
int64_t vfl_pool_blocks_needed(const vfl_pool *pool, const int32_t *write_block, int32_t rows);

/* A fork: every block of table[0..len) gains a holder (BlockManager.fork). */
int vfl_pool_share(vfl_pool *pool, const int32_t *table, int32_t len);
/* A row leaves: its blocks lose a holder, last block first; blocks nobody holds go to
 * the back of the free list (BlockManager.deallocate). */
int vfl_pool_release(vfl_pool *pool, const int32_t *table, int32_t len);

/* ------------------------------------------------------------------------------- */
/* vfl_engine                                                                        */
/* ------------------------------------------------------------------------------- */
typedef struct vfl_engine vfl_engine;

/* An engine over its own pool of num_blocks blocks; at most max_num_seqs beams run
 * at once (admission counts each running request's num_beams). */
vfl_engine *vfl_engine_create(int32_t num_blocks, int32_t block_size, int32_t max_num_seqs);
void vfl_engine_destroy(vfl_engine *engine);
/* The engine's pool (borrowed; lives as long as the engine). */
vfl_pool *vfl_engine_pool(vfl_engine *engine);
/* Drops every waiting, running and finishing request and frees every block. */
void vfl_engine_reset(vfl_engine *engine);

/*
 * Queue a request (Scheduler.add of a fresh Sequence, sequence.py semantics): its one
 * hypothesis starts from the decoder prompt `prompt[0..n)`.  It finishes when its last
 * token is one of eos[0..n_eos) or it has generated max_tokens tokens; beam search
 * keeps num_beams hypotheses scored cum_logprob / max(generated, 1)^length_penalty.
 */
int vfl_engine_add_request(vfl_engine *engine, int64_t request_id, const int32_t *prompt,
                           int32_t n, int32_t num_beams, int32_t max_tokens,
                           const int32_t *eos, int32_t n_eos, double length_penalty,
                           int32_t early_stopping);

int32_t vfl_engine_num_waiting(const vfl_engine *engine);
int32_t vfl_engine_num_running(const vfl_engine *engine);
/* Requests with finished beam hypotheses but still running beams. */
int32_t vfl_engine_num_pending_beams(const vfl_engine *engine);

/*
 * Start a step (Scheduler.schedule, scheduler.py:35-58): admit waiting requests in
 * order while the running requests' beams plus the next request's fit max_num_seqs
 * (their ids go to admitted[0..*n_admitted), at most admitted_cap), check that the
 * pool covers the step (VFL_HOST_E_FULL otherwise: "KV cache is full"), then make
 * every running row's next position writable in row order.  *n_rows running rows
 * and *n_pairs copy-on-write pairs result.  On VFL_HOST_E_FULL nothing has changed:
 * the requests the call would have admitted are back at the head of the waiting
 * queue in their order and *n_admitted is 0.
 */
int vfl_engine_schedule(vfl_engine *engine, int64_t *admitted, int32_t admitted_cap,
                        int32_t *n_admitted, int32_t *n_rows, int32_t *n_pairs);

/*
 * The scheduled step's metadata (ModelRunner._prepare, model_runner.py:288-305), for
 * `padded` >= n_rows rows (rows past n_rows are padding: token 0 at position 0, slot
 * -1, context 0, length 1, an all-zero table row):
 *   input_ids[r]    the row's last token          positions[r]  its cached tokens
 *   slots[r]        table[pos / bs] * bs + pos % bs
 *   lengths[r]      the row's token count          context_lens[r]  pos + 1
 *   tables          [padded][table_width] block tables, zero-padded
 *   copy_src/dst    the step's copy-on-write pairs (n_pairs entries)
 *   row_requests    [n_rows] each row's request id
 * Row groups for the self-attention kernel: runs of rows of one request (a request's
 * beams are adjacent) cut every max_group rows.  When some group holds more than one
 * row, group_start gets the padded + 1 group starts (padding rows in groups of
 * max_group, then empty groups up to padded) and *grouped = 1; otherwise order gets the row
 * indices by descending context length, stable (longest first), and *grouped = 0.
 */
int vfl_engine_pack(const vfl_engine *engine, int32_t padded, int32_t table_width,
                    int32_t max_group, int64_t *input_ids, int64_t *positions, int64_t *slots,
                    int64_t *lengths, int64_t *copy_src, int64_t *copy_dst,
                    int32_t *context_lens, int32_t *order, int32_t *group_start,
                    int32_t *tables, int64_t *row_requests, int32_t *grouped);

/* Longest table and most tokens over the running rows (buffer sizing, history width). */
int32_t vfl_engine_max_table_len(const vfl_engine *engine);
int32_t vfl_engine_max_row_tokens(const vfl_engine *engine);

/* [n_rows][width] token histories, right-aligned and left-padded with -1 (the rules of
 * LogitsProcessor that read history); width >= vfl_engine_max_row_tokens. */
int vfl_engine_history(const vfl_engine *engine, int64_t *out, int32_t width);

/*
 * End a greedy step (Scheduler._postprocess_greedy, scheduler.py:69-79): every row's
 * cached count grows by one, row r appends tokens[r]; rows that finish leave in row
 * order (their blocks return to the pool) and their requests are reported through
 * vfl_engine_next_finished.
 */
int vfl_engine_greedy_update(vfl_engine *engine, const int64_t *tokens, int32_t rows);

/*
 * End a beam-search step (ModelRunner._beam_search + Scheduler._postprocess_beam,
 * model_runner.py:383-410, scheduler.py:81-127).  scores / ids: [rows][k] each row's
 * best k processed log-probs and their token ids, best first.  Per request, its rows'
 * candidates take score + (float) cum_logprob in float32, are sorted by that value,
 * best first and stably (row order, then each row's order), and the best
 * max(2, 1 + n_eos) * num_beams are walked: a candidate that ends its hypothesis
 * (EOS or max_tokens) joins the finished hypotheses if it ranks within num_beams, a
 * live one becomes a running child while fewer than num_beams are; finished
 * hypotheses keep the best num_beams by length-penalised score.  The request ends
 * when no child lives, or num_beams are finished and early stopping is set or the
 * worst finished score is at least the best child's; its best finished hypothesis is
 * reported.  Children share their parent's blocks; every parent leaves (its blocks
 * lose a holder) in row order.  The children run next, in request order.
 */
int vfl_engine_beam_update(vfl_engine *engine, const float *scores, const int64_t *ids,
                           int32_t rows, int32_t k);

/* Drops a request between steps (a caller's cancellation): its waiting or running
 * hypotheses leave in row order (their blocks lose a holder) and it is not reported as
 * finished.  Returns 1 if the request was known, 0 if not. */
int vfl_engine_abort_request(vfl_engine *engine, int64_t request_id);

/* Pops the next finished request: its id and completion tokens (tokens after the
 * decoder prompt).  Returns 1 if one was popped, 0 if none; VFL_HOST_E_INVALID if cap
 * is too small (nothing popped, *n holds the length needed). */
int vfl_engine_next_finished(vfl_engine *engine, int64_t *request_id, int32_t *tokens,
                             int32_t cap, int32_t *n);

/* One running row: request id, token count, cached tokens, cumulative log-prob and
 * block-table length; tokens / table copied when non-NULL (cap entries at most). */
int vfl_engine_row(const vfl_engine *engine, int32_t row, int64_t *request_id,
                   int32_t *n_tokens, int32_t *cached, double *cum_logprob, int32_t *table_len,
                   int32_t *tokens, int32_t *table, int32_t cap);

#ifdef __cplusplus
}
#endif

#endif /* VFL_ENGINE_H */
