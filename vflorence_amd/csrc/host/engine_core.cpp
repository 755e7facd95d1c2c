// Native host core of the decode engine (see include/vfl_engine.h): the paged KV block
// pool and the per-step host state of continuous batching with greedy or beam-search
// decoding.  Plain C++17; everything a step needs lives in flat vectors, so a step's
// host work is a few passes over the running rows instead of per-object Python calls.
#include "../../../include/vfl_engine.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <deque>
#include <limits>
#include <string>
#include <utility>
#include <vector>

namespace {

thread_local char g_error[512];

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace

// ---------------------------------------------------------------------------------
// Block pool: reference counts plus the free list as a ring (front = next block out).
// ---------------------------------------------------------------------------------
struct vfl_pool {
  int32_t block_size = 16;
  std::vector<int32_t> holders;  // per block: tables that list it
  std::vector<int32_t> ring;     // free blocks, ring[(head + i) % n] for i < count
  int64_t head = 0, count = 0;
  // scratch of blocks_needed: holders not yet accounted for, valid where stamp == epoch
  mutable std::vector<int32_t> left;
  mutable std::vector<uint32_t> stamp;
  mutable uint32_t epoch = 0;

  vfl_pool(int32_t n, int32_t bs) : block_size(bs), holders(n), ring(n), left(n), stamp(n) {
    reset();
  }

  int32_t size() const { return (int32_t)holders.size(); }

  void reset() {
    std::fill(holders.begin(), holders.end(), 0);
    for (int32_t i = 0; i < size(); ++i) ring[i] = i;
    head = 0;
    count = size();
  }

  bool take(int32_t *block) {
    if (count == 0) return false;
    *block = ring[head];
    head = (head + 1) % size();
    --count;
    holders[*block] = 1;
    return true;
  }

  void put_back(int32_t block) {
    ring[(head + count) % size()] = block;
    ++count;
  }

  void share(const int32_t *t, int32_t n) {
    for (int32_t i = 0; i < n; ++i) ++holders[t[i]];
  }

  void release(const int32_t *t, int32_t n) {
    for (int32_t i = n - 1; i >= 0; --i)
      if (--holders[t[i]] == 0) put_back(t[i]);
  }

  // 0 nothing, 1 append *block, 2 replace the shared *src by *block, -1 pool empty.
  int prepare_write(const int32_t *table, int32_t len, int32_t cached, int32_t *block,
                    int32_t *src) {
    const int32_t idx = cached / block_size;
    if (idx >= len) return take(block) ? 1 : -1;
    const int32_t b = table[idx];
    if (holders[b] == 1) return 0;
    if (!take(block)) return -1;
    --holders[b];
    *src = b;
    return 2;
  }

  int64_t blocks_needed(const int32_t *write_block, int32_t rows) const {
    if (++epoch == 0) {  // stamps wrapped: forget them all
      std::fill(stamp.begin(), stamp.end(), 0u);
      epoch = 1;
    }
    int64_t need = 0;
    for (int32_t r = 0; r < rows; ++r) {
      const int32_t b = write_block[r];
      if (b < 0) {
        ++need;
        continue;
      }
      if (stamp[b] != epoch) {
        stamp[b] = epoch;
        left[b] = holders[b];
      }
      if (left[b] > 1) {  // another holder writes later or keeps it: this one copies
        ++need;
        --left[b];
      }
    }
    return need;
  }
};

// ---------------------------------------------------------------------------------
// Engine state
// ---------------------------------------------------------------------------------
namespace {

struct Request {
  int64_t id = 0;
  int32_t num_beams = 1, max_tokens = 1, prompt_len = 1;
  std::vector<int32_t> eos;
  double length_penalty = 1.0;
  bool early_stopping = false;
  struct Done {
    std::vector<int32_t> tokens;
    double score;
  };
  std::vector<Done> finished;  // beam hypotheses that ended, best first
  bool is_eos(int32_t t) const { return std::find(eos.begin(), eos.end(), t) != eos.end(); }
  double score(double cum, int32_t generated) const {
    return cum / std::pow((double)std::max(generated, 1), length_penalty);
  }
};

struct Row {  // one running (or waiting) hypothesis
  int32_t req = 0;  // index into Engine::requests
  std::vector<int32_t> tokens;
  std::vector<int32_t> table;
  int32_t cached = 0;
  double cum = 0.0;
};

struct Finished {
  int64_t id;
  std::vector<int32_t> completion;
};

struct BeamCand {  // a continuation: cumulative log-prob, parent row, token
  float value;
  int32_t row;
  int32_t token;
};

}  // namespace

struct vfl_engine {
  vfl_pool pool;
  int32_t max_num_seqs;
  std::vector<Request> requests;  // slots; a finished request's slot is reused
  std::vector<int32_t> free_slots;
  std::deque<Row> waiting;
  std::vector<Row> running;
  std::vector<std::pair<int32_t, int32_t>> pairs;  // this step's copy-on-write pairs
  std::deque<Finished> done;
  bool scheduled = false;
  std::vector<uint32_t> req_stamp;
  uint32_t req_epoch = 0;
  // beam_update's working storage, kept across steps so that a step allocates nothing
  // once the batch has reached its size: candidates, the rows being built, and token
  // and table vectors (emptied, capacity kept) that the last step's parents left
  std::vector<BeamCand> cands;
  std::vector<std::pair<int32_t, BeamCand>> live;  // (parent row, candidate)
  std::vector<Row> next_rows;
  std::vector<std::vector<int32_t>> spare_tokens, spare_tables;
  std::vector<int32_t> handed;      // parent row -> index in next_rows of its first child
  std::vector<uint8_t> has_child;   // parent row -> a live child takes it

  // An emptied vector from `spares` (capacity kept), or a new one.
  static std::vector<int32_t> take_spare(std::vector<std::vector<int32_t>> &spares) {
    if (spares.empty()) return {};
    std::vector<int32_t> v = std::move(spares.back());
    spares.pop_back();
    return v;
  }
  // A row's storage back to the spares (at most one spare per row a batch can hold).
  void recycle(Row &r) {
    if (r.tokens.capacity() && (int32_t)spare_tokens.size() < max_num_seqs) {
      r.tokens.clear();
      spare_tokens.push_back(std::move(r.tokens));
    }
    if (r.table.capacity() && (int32_t)spare_tables.size() < max_num_seqs) {
      r.table.clear();
      spare_tables.push_back(std::move(r.table));
    }
  }

  vfl_engine(int32_t nb, int32_t bs, int32_t mns) : pool(nb, bs), max_num_seqs(mns) {}

  void reset() {
    requests.clear();
    free_slots.clear();
    waiting.clear();
    running.clear();
    pairs.clear();
    done.clear();
    pool.reset();
    scheduled = false;
  }

  int32_t new_slot() {
    if (!free_slots.empty()) {
      int32_t s = free_slots.back();
      free_slots.pop_back();
      return s;
    }
    requests.emplace_back();
    req_stamp.push_back(0);
    return (int32_t)requests.size() - 1;
  }

  void end_request(int32_t slot, std::vector<int32_t> &&tokens) {
    Request &q = requests[slot];
    Finished f{q.id, {}};
    f.completion.assign(tokens.begin() + std::min<size_t>(q.prompt_len, tokens.size()),
                        tokens.end());
    done.push_back(std::move(f));
    q.finished.clear();
    free_slots.push_back(slot);
  }

  // Distinct running requests' beams (admission counts a request once).
  int64_t running_beams() {
    if (++req_epoch == 0) {
      std::fill(req_stamp.begin(), req_stamp.end(), 0u);
      req_epoch = 1;
    }
    int64_t used = 0;
    for (const Row &r : running)
      if (req_stamp[r.req] != req_epoch) {
        req_stamp[r.req] = req_epoch;
        used += requests[r.req].num_beams;
      }
    return used;
  }
};

extern "C" {

const char *vfl_host_last_error(void) { return g_error; }

// ------------------------------- pool ---------------------------------------------
vfl_pool *vfl_pool_create(int32_t num_blocks, int32_t block_size) {
  clear_error();
  if (num_blocks <= 0 || block_size <= 0) {
    fail(VFL_HOST_E_INVALID, "pool: bad sizes (blocks %d, block_size %d)", num_blocks,
         block_size);
    return nullptr;
  }
  return new vfl_pool(num_blocks, block_size);
}

void vfl_pool_destroy(vfl_pool *pool) { delete pool; }
void vfl_pool_reset(vfl_pool *pool) { pool->reset(); }
int32_t vfl_pool_num_blocks(const vfl_pool *pool) { return pool->size(); }
int32_t vfl_pool_num_free(const vfl_pool *pool) { return (int32_t)pool->count; }

void vfl_pool_refcounts(const vfl_pool *pool, int32_t *out) {
  std::copy(pool->holders.begin(), pool->holders.end(), out);
}

void vfl_pool_free_list(const vfl_pool *pool, int32_t *out) {
  for (int64_t i = 0; i < pool->count; ++i) out[i] = pool->ring[(pool->head + i) % pool->size()];
}

static bool valid_table(const vfl_pool *pool, const int32_t *table, int32_t len) {
  if (len < 0 || (len > 0 && !table)) return false;
  for (int32_t i = 0; i < len; ++i)
    if (table[i] < 0 || table[i] >= pool->size()) return false;
  return true;
}

int vfl_pool_prepare_write(vfl_pool *pool, const int32_t *table, int32_t len, int32_t cached,
                           int32_t *block, int32_t *src) {
  clear_error();
  if (!block || !src || cached < 0 || !valid_table(pool, table, len))
    return fail(VFL_HOST_E_INVALID, "pool: bad table or position");
  const int st = pool->prepare_write(table, len, cached, block, src);
  if (st < 0) return fail(VFL_HOST_E_FULL, "KV cache is full; increase num_blocks");
  return st;
}

int64_t vfl_pool_blocks_needed(const vfl_pool *pool, const int32_t *write_block, int32_t rows) {
  clear_error();
  if (rows < 0 || (rows > 0 && !write_block))
    return fail(VFL_HOST_E_INVALID, "pool: bad rows");
  for (int32_t r = 0; r < rows; ++r)
    if (write_block[r] >= pool->size()) return fail(VFL_HOST_E_INVALID, "pool: bad block id");
  return pool->blocks_needed(write_block, rows);
}

int vfl_pool_share(vfl_pool *pool, const int32_t *table, int32_t len) {
  clear_error();
  if (!valid_table(pool, table, len)) return fail(VFL_HOST_E_INVALID, "pool: bad table");
  pool->share(table, len);
  return VFL_HOST_OK;
}

int vfl_pool_release(vfl_pool *pool, const int32_t *table, int32_t len) {
  clear_error();
  if (!valid_table(pool, table, len)) return fail(VFL_HOST_E_INVALID, "pool: bad table");
  for (int32_t i = 0; i < len; ++i)
    if (pool->holders[table[i]] <= 0)
      return fail(VFL_HOST_E_STATE, "pool: block %d released without a holder", table[i]);
  pool->release(table, len);
  return VFL_HOST_OK;
}

// ------------------------------- engine -------------------------------------------
vfl_engine *vfl_engine_create(int32_t num_blocks, int32_t block_size, int32_t max_num_seqs) {
  clear_error();
  if (num_blocks <= 0 || block_size <= 0 || max_num_seqs <= 0) {
    fail(VFL_HOST_E_INVALID, "engine: bad sizes (blocks %d, block_size %d, max_num_seqs %d)",
         num_blocks, block_size, max_num_seqs);
    return nullptr;
  }
  return new vfl_engine(num_blocks, block_size, max_num_seqs);
}

void vfl_engine_destroy(vfl_engine *engine) { delete engine; }
vfl_pool *vfl_engine_pool(vfl_engine *engine) { return &engine->pool; }
void vfl_engine_reset(vfl_engine *engine) { engine->reset(); }

int vfl_engine_add_request(vfl_engine *e, int64_t request_id, const int32_t *prompt, int32_t n,
                           int32_t num_beams, int32_t max_tokens, const int32_t *eos,
                           int32_t n_eos, double length_penalty, int32_t early_stopping) {
  clear_error();
  if (n <= 0 || !prompt || num_beams <= 0 || max_tokens <= 0 || n_eos < 0 ||
      (n_eos > 0 && !eos) || !std::isfinite(length_penalty))
    return fail(VFL_HOST_E_INVALID, "add_request: bad arguments");
  const int32_t slot = e->new_slot();
  Request &q = e->requests[slot];
  q.id = request_id;
  q.num_beams = num_beams;
  q.max_tokens = max_tokens;
  q.prompt_len = n;
  q.eos.assign(eos, eos + n_eos);
  q.length_penalty = length_penalty;
  q.early_stopping = early_stopping != 0;
  q.finished.clear();
  Row r;
  r.req = slot;
  r.tokens.assign(prompt, prompt + n);
  e->waiting.push_back(std::move(r));
  return VFL_HOST_OK;
}

int32_t vfl_engine_num_waiting(const vfl_engine *e) { return (int32_t)e->waiting.size(); }
int32_t vfl_engine_num_running(const vfl_engine *e) { return (int32_t)e->running.size(); }

int32_t vfl_engine_num_pending_beams(const vfl_engine *e) {
  int32_t n = 0;
  for (const Request &q : e->requests) n += !q.finished.empty();
  return n;
}

int vfl_engine_schedule(vfl_engine *e, int64_t *admitted, int32_t admitted_cap,
                        int32_t *n_admitted, int32_t *n_rows, int32_t *n_pairs) {
  clear_error();
  if (!n_admitted || !n_rows || !n_pairs || (admitted_cap > 0 && !admitted))
    return fail(VFL_HOST_E_INVALID, "schedule: null output");
  e->scheduled = false;
  e->pairs.clear();
  *n_admitted = 0;
  if (!e->waiting.empty()) {
    int64_t used = e->running_beams();
    while (!e->waiting.empty() &&
           used + e->requests[e->waiting.front().req].num_beams <= e->max_num_seqs) {
      if (*n_admitted >= admitted_cap)
        return fail(VFL_HOST_E_INVALID, "schedule: more than %d admissions", admitted_cap);
      admitted[(*n_admitted)++] = e->requests[e->waiting.front().req].id;
      used += e->requests[e->waiting.front().req].num_beams;
      e->running.push_back(std::move(e->waiting.front()));
      e->waiting.pop_front();
    }
  }
  vfl_pool &pool = e->pool;
  std::vector<int32_t> writes(e->running.size());
  for (size_t i = 0; i < e->running.size(); ++i) {
    const Row &r = e->running[i];
    const int32_t idx = r.cached / pool.block_size;
    writes[i] = idx < (int32_t)r.table.size() ? r.table[idx] : -1;
  }
  if (pool.blocks_needed(writes.data(), (int32_t)writes.size()) > pool.count) {
    // Nothing has touched the pool yet: put this call's admissions back at the head of
    // the waiting queue, in order, so a failed call leaves the engine as it found it.
    for (int32_t a = 0; a < *n_admitted; ++a) {
      e->waiting.push_front(std::move(e->running.back()));
      e->running.pop_back();
    }
    *n_admitted = 0;
    return fail(VFL_HOST_E_FULL, "KV cache is full; increase num_blocks");
  }
  for (Row &r : e->running) {
    int32_t block = -1, src = -1;
    const int st = pool.prepare_write(r.table.data(), (int32_t)r.table.size(), r.cached, &block,
                                      &src);
    if (st == 1) {
      r.table.push_back(block);
    } else if (st == 2) {
      r.table[r.cached / pool.block_size] = block;
      e->pairs.emplace_back(src, block);
    } else if (st < 0) {  // cannot happen after the check above
      return fail(VFL_HOST_E_FULL, "KV cache is full; increase num_blocks");
    }
  }
  *n_rows = (int32_t)e->running.size();
  *n_pairs = (int32_t)e->pairs.size();
  e->scheduled = true;
  return VFL_HOST_OK;
}

int32_t vfl_engine_max_table_len(const vfl_engine *e) {
  size_t m = 0;
  for (const Row &r : e->running) m = std::max(m, r.table.size());
  return (int32_t)m;
}

int32_t vfl_engine_max_row_tokens(const vfl_engine *e) {
  size_t m = 0;
  for (const Row &r : e->running) m = std::max(m, r.tokens.size());
  return (int32_t)m;
}

int vfl_engine_pack(const vfl_engine *e, int32_t padded, int32_t table_width, int32_t max_group,
                    int64_t *input_ids, int64_t *positions, int64_t *slots, int64_t *lengths,
                    int64_t *copy_src, int64_t *copy_dst, int32_t *context_lens, int32_t *order,
                    int32_t *group_start, int32_t *tables, int64_t *row_requests,
                    int32_t *grouped) {
  clear_error();
  if (!e->scheduled) return fail(VFL_HOST_E_STATE, "pack: no scheduled step");
  const int32_t n = (int32_t)e->running.size();
  if (padded < n || max_group < 1 || table_width < vfl_engine_max_table_len(e))
    return fail(VFL_HOST_E_INVALID, "pack: padded %d < rows %d, max_group %d or table width %d",
                padded, n, max_group, table_width);
  if (!input_ids || !positions || !slots || !lengths || !context_lens || !order ||
      !group_start || !tables || !row_requests || !grouped ||
      (!e->pairs.empty() && (!copy_src || !copy_dst)))
    return fail(VFL_HOST_E_INVALID, "pack: null buffer");
  const int32_t bs = e->pool.block_size;
  for (int32_t i = 0; i < n; ++i) {
    const Row &r = e->running[i];
    const int32_t pos = r.cached;
    int32_t *trow = tables + (int64_t)i * table_width;
    std::copy(r.table.begin(), r.table.end(), trow);
    std::fill(trow + r.table.size(), trow + table_width, 0);
    input_ids[i] = r.tokens.back();
    positions[i] = pos;
    slots[i] = (int64_t)r.table[pos / bs] * bs + pos % bs;
    lengths[i] = (int64_t)r.tokens.size();
    context_lens[i] = pos + 1;
    row_requests[i] = e->requests[r.req].id;
  }
  for (int32_t i = n; i < padded; ++i) {
    input_ids[i] = 0;
    positions[i] = 0;
    slots[i] = -1;
    lengths[i] = 1;
    context_lens[i] = 0;
    std::fill(tables + (int64_t)i * table_width, tables + (int64_t)(i + 1) * table_width, 0);
  }
  for (size_t p = 0; p < e->pairs.size(); ++p) {
    copy_src[p] = e->pairs[p].first;
    copy_dst[p] = e->pairs[p].second;
  }
  // runs of one request's rows, cut every max_group rows
  int32_t groups = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (i == 0 || e->running[i].req != e->running[i - 1].req ||
        i - group_start[groups - 1] >= max_group)
      group_start[groups++] = i;
  }
  if (groups < n) {  // some group holds several rows: beam groups
    // padding rows (empty contexts) in groups of max_group, so a launch sized for the
    // real groups plus a few covers them
    for (int32_t i = n; i < padded; i += max_group) group_start[groups++] = i;
    for (int32_t g = groups; g <= padded; ++g) group_start[g] = padded;
    *grouped = 1;
  } else {
    for (int32_t i = 0; i < padded; ++i) order[i] = i;
    std::stable_sort(order, order + padded, [&](int32_t a, int32_t b) {
      return context_lens[a] > context_lens[b];
    });
    *grouped = 0;
  }
  return VFL_HOST_OK;
}

int vfl_engine_history(const vfl_engine *e, int64_t *out, int32_t width) {
  clear_error();
  if (!out || width < vfl_engine_max_row_tokens(e))
    return fail(VFL_HOST_E_INVALID, "history: width %d too small", width);
  for (size_t i = 0; i < e->running.size(); ++i) {
    const std::vector<int32_t> &t = e->running[i].tokens;
    int64_t *row = out + (int64_t)i * width;
    const int32_t pad = width - (int32_t)t.size();
    std::fill(row, row + pad, -1);
    std::copy(t.begin(), t.end(), row + pad);
  }
  return VFL_HOST_OK;
}

int vfl_engine_greedy_update(vfl_engine *e, const int64_t *tokens, int32_t rows) {
  clear_error();
  if (!e->scheduled) return fail(VFL_HOST_E_STATE, "greedy_update: no scheduled step");
  if (rows != (int32_t)e->running.size() || (rows > 0 && !tokens))
    return fail(VFL_HOST_E_INVALID, "greedy_update: %d tokens for %zu rows", rows,
                e->running.size());
  e->scheduled = false;
  std::vector<Row> keep;
  keep.reserve(e->running.size());
  for (int32_t i = 0; i < rows; ++i) {
    Row &r = e->running[i];
    const Request &q = e->requests[r.req];
    r.cached += 1;
    r.tokens.push_back((int32_t)tokens[i]);
    const int32_t generated = (int32_t)r.tokens.size() - q.prompt_len;
    if (q.is_eos(r.tokens.back()) || generated >= q.max_tokens) {
      e->pool.release(r.table.data(), (int32_t)r.table.size());
      e->end_request(r.req, std::move(r.tokens));
    } else {
      keep.push_back(std::move(r));
    }
  }
  e->running.swap(keep);
  return VFL_HOST_OK;
}

int vfl_engine_beam_update(vfl_engine *e, const float *scores, const int64_t *ids, int32_t rows,
                           int32_t k) {
  clear_error();
  if (!e->scheduled) return fail(VFL_HOST_E_STATE, "beam_update: no scheduled step");
  if (rows != (int32_t)e->running.size() || k <= 0 || (rows > 0 && (!scores || !ids)))
    return fail(VFL_HOST_E_INVALID, "beam_update: [%d, %d] candidates for %zu rows", rows, k,
                e->running.size());
  e->scheduled = false;
  for (Row &r : e->running) r.cached += 1;

  using Cand = BeamCand;
  std::vector<Cand> &cands = e->cands;
  std::vector<Row> &next = e->next_rows;
  next.clear();
  next.reserve(e->running.size());
  std::vector<std::pair<int32_t, Cand>> &live = e->live;
  std::vector<int32_t> &handed = e->handed;
  handed.assign(rows, -1);
  std::vector<uint8_t> &has_child = e->has_child;
  has_child.assign(rows, 0);

  int32_t i = 0;
  while (i < rows) {  // a request's rows are adjacent
    const int32_t slot = e->running[i].req;
    int32_t j = i;
    while (j < rows && e->running[j].req == slot) ++j;
    Request &q = e->requests[slot];
    const int32_t nb = q.num_beams;
    const int32_t keep = std::max<int32_t>(2, 1 + (int32_t)q.eos.size()) * nb;
    // Best first, ties in row-major order (a stable sort).  When each row's list is best
    // first (the device top-k's order), the best `keep` come from merging the rows'
    // lists head by head, reading the scores in place (on a tie the lower row first);
    // otherwise every candidate goes through an insertion sort, with no temporary buffer.
    const int32_t nr = j - i;
    bool rows_sorted = nr <= 16;
    for (int32_t r = i; r < j && rows_sorted; ++r) {
      const float cum = (float)e->running[r].cum;
      const float *sr = scores + (int64_t)r * k;
      for (int32_t c = 1; c < k; ++c)
        if (!(sr[c - 1] + cum >= sr[c] + cum)) {
          rows_sorted = false;
          break;
        }
    }
    cands.clear();
    if (rows_sorted) {
      const int32_t take = (int32_t)std::min<int64_t>(keep, (int64_t)nr * k);
      int32_t at[16];
      float head[16], cumf[16];
      for (int32_t r = 0; r < nr; ++r) {
        at[r] = 0;
        cumf[r] = (float)e->running[i + r].cum;
        head[r] = scores[(int64_t)(i + r) * k] + cumf[r];
      }
      for (int32_t t = 0; t < take; ++t) {
        int32_t best = -1;
        for (int32_t r = 0; r < nr; ++r)
          if (at[r] < k && (best < 0 || head[r] > head[best])) best = r;
        const int64_t c = (int64_t)(i + best) * k + at[best];
        cands.push_back({head[best], i + best, (int32_t)ids[c]});
        if (++at[best] < k) head[best] = scores[c + 1] + cumf[best];
      }
    } else {
      for (int32_t r = i; r < j; ++r) {
        const float cum = (float)e->running[r].cum;
        for (int32_t c = 0; c < k; ++c)
          cands.push_back({scores[(int64_t)r * k + c] + cum, r, (int32_t)ids[(int64_t)r * k + c]});
      }
      for (size_t a = 1; a < cands.size(); ++a) {
        const Cand c = cands[a];
        size_t b = a;
        while (b > 0 && cands[b - 1].value < c.value) {
          cands[b] = cands[b - 1];
          --b;
        }
        cands[b] = c;
      }
      if ((int32_t)cands.size() > keep) cands.resize(keep);
    }

    live.clear();
    for (int32_t rank = 0; rank < (int32_t)cands.size(); ++rank) {
      if (rank >= nb && (int32_t)live.size() >= nb) break;
      const Cand &c = cands[rank];
      const Row &parent = e->running[c.row];
      const int32_t generated = (int32_t)parent.tokens.size() + 1 - q.prompt_len;
      if (q.is_eos(c.token) || generated >= q.max_tokens) {
        if (rank < nb) {
          Request::Done d;
          d.tokens = parent.tokens;
          d.tokens.push_back(c.token);
          d.score = q.score((double)c.value, generated);
          q.finished.push_back(std::move(d));
        }
      } else if ((int32_t)live.size() < nb) {
        live.emplace_back(c.row, c);
      }
    }
    std::stable_sort(q.finished.begin(), q.finished.end(),
                     [](const Request::Done &a, const Request::Done &b) {
                       return a.score > b.score;
                     });
    if ((int32_t)q.finished.size() > nb) q.finished.resize(nb);

    bool finish = live.empty();
    if (!finish && (int32_t)q.finished.size() >= nb) {
      if (q.early_stopping) {
        finish = true;
      } else {
        double best = -std::numeric_limits<double>::infinity();
        for (const auto &l : live) {
          const Row &parent = e->running[l.first];
          const int32_t generated = (int32_t)parent.tokens.size() + 1 - q.prompt_len;
          best = std::max(best, q.score((double)l.second.value, generated));
        }
        finish = q.finished.back().score >= best;
      }
    }
    if (finish) {
      // Unreachable: k >= 1, so the request's best candidate (rank 0 < num_beams) became
      // either a finished hypothesis or a live one, and a request that ends with live
      // candidates holds num_beams finished ones.  Kept as a guard, not a code path.
      if (q.finished.empty())
        return fail(VFL_HOST_E_STATE, "beam_update: request %lld ends with no hypothesis",
                    (long long)q.id);
      std::vector<int32_t> best = std::move(q.finished.front().tokens);
      e->end_request(slot, std::move(best));
    } else {
      // A parent's first live child takes over its table and its token list; later
      // children of the same parent share the table (one more holder per block), as
      // forking every child and then releasing every parent would leave them, and copy
      // the first child's tokens with their own last token -- into the token storage of
      // a parent with no live child where there is one (no allocation).
      for (const auto &l : live) has_child[l.first] = 1;
      int32_t spare = i;
      for (const auto &l : live) {
        const int32_t p = l.first;
        Row child;
        child.req = slot;
        child.cached = e->running[p].cached;
        child.cum = (double)l.second.value;
        if (handed[p] < 0) {
          child.tokens = std::move(e->running[p].tokens);
          e->running[p].tokens.clear();
          child.tokens.push_back(l.second.token);
          child.table = std::move(e->running[p].table);
          e->running[p].table.clear();
          handed[p] = (int32_t)next.size();
        } else {
          while (spare < j && has_child[spare]) ++spare;
          if (spare < j) {
            child.tokens = std::move(e->running[spare].tokens);
            e->running[spare].tokens.clear();
            ++spare;
          } else {
            child.tokens = vfl_engine::take_spare(e->spare_tokens);
          }
          const Row &first = next[handed[p]];
          child.tokens.assign(first.tokens.begin(), first.tokens.end());
          child.tokens.back() = l.second.token;
          child.table = vfl_engine::take_spare(e->spare_tables);
          child.table.assign(first.table.begin(), first.table.end());
          e->pool.share(child.table.data(), (int32_t)child.table.size());
        }
        next.push_back(std::move(child));
      }
    }
    i = j;
  }
  // every parent leaves, in row order (tables handed to a child are empty by now), and
  // leaves its storage for the next step's children
  for (Row &r : e->running) e->pool.release(r.table.data(), (int32_t)r.table.size());
  e->running.swap(next);
  for (Row &r : next) e->recycle(r);
  next.clear();
  return VFL_HOST_OK;
}

int vfl_engine_abort_request(vfl_engine *e, int64_t request_id) {
  clear_error();
  if (e->scheduled) return fail(VFL_HOST_E_STATE, "abort_request: inside a scheduled step");
  int32_t slot = -1;
  for (auto it = e->waiting.begin(); it != e->waiting.end(); ++it)
    if (e->requests[it->req].id == request_id) {
      slot = it->req;
      e->waiting.erase(it);
      break;
    }
  std::vector<Row> keep;
  keep.reserve(e->running.size());
  for (Row &r : e->running) {
    if (e->requests[r.req].id == request_id) {
      slot = r.req;
      e->pool.release(r.table.data(), (int32_t)r.table.size());
    } else {
      keep.push_back(std::move(r));
    }
  }
  e->running.swap(keep);
  if (slot < 0) return 0;
  e->requests[slot].finished.clear();
  e->free_slots.push_back(slot);
  return 1;
}

int vfl_engine_next_finished(vfl_engine *e, int64_t *request_id, int32_t *tokens, int32_t cap,
                             int32_t *n) {
  clear_error();
  if (e->done.empty()) return 0;
  const Finished &f = e->done.front();
  if (n) *n = (int32_t)f.completion.size();
  if (!request_id || (int32_t)f.completion.size() > cap || (!tokens && !f.completion.empty()))
    return fail(VFL_HOST_E_INVALID, "next_finished: %zu tokens do not fit %d",
                f.completion.size(), cap);
  *request_id = f.id;
  std::copy(f.completion.begin(), f.completion.end(), tokens);
  e->done.pop_front();
  return 1;
}

int vfl_engine_row(const vfl_engine *e, int32_t row, int64_t *request_id, int32_t *n_tokens,
                   int32_t *cached, double *cum_logprob, int32_t *table_len, int32_t *tokens,
                   int32_t *table, int32_t cap) {
  clear_error();
  if (row < 0 || row >= (int32_t)e->running.size())
    return fail(VFL_HOST_E_INVALID, "row %d of %zu", row, e->running.size());
  const Row &r = e->running[row];
  if (request_id) *request_id = e->requests[r.req].id;
  if (n_tokens) *n_tokens = (int32_t)r.tokens.size();
  if (cached) *cached = r.cached;
  if (cum_logprob) *cum_logprob = r.cum;
  if (table_len) *table_len = (int32_t)r.table.size();
  if (tokens) std::copy_n(r.tokens.begin(), std::min<size_t>(cap, r.tokens.size()), tokens);
  if (table) std::copy_n(r.table.begin(), std::min<size_t>(cap, r.table.size()), table);
  return VFL_HOST_OK;
}

}  // extern "C"
