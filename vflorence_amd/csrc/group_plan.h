// Group plans for decode self-attention over row groups whose rows keep their own
// block tables (the beams of a request), built on the host once per decode step and
// read by every layer's launch (decode_planned.h).
//
// Layout, int32 words:
//   [0]            slots in use (the kernel's workgroups of later slots exit)
//   [1 .. 3]       zero
//   slot s at PLAN_PREFIX + s * stride:
//     [0] first row   [1] rows   [2] entries   [3] blocks of the group's longest row
//     entry e at PLAN_HEADER + PLAN_ENTRY * e:
//       [0] block id
//       [1] copy << 31 | position << 16 | tokens << 8 | row mask (bit c: row first + c)
//           copy (set by fold_plan_copies): the entry is its one row's fork block, and
//           [0] holds the block copy-on-write fills it from.  The fused launch reads
//           that source, writes the whole block with the row's new token in it to the
//           row's slot block (its fork block, by the fused write's contract), and the
//           step needs no separate copy launch.  Only the fused launch can read such a
//           plan: the plain launch would read the source as the row's block.
// A slot's entries list, position by position, the distinct block ids the group's
// rows hold there (ids outside [0, num_blocks) left out), each once, with the rows
// that list it, in order of each id's first row: the blocks the shared kernel finds
// by walking the tables, in the order it finds them.  `tokens` (1..block_size) is how
// many of the block's tokens the longest of those rows attends to: the kernel reads
// no K or V past them.
// Plain C++ (no HIP): compiled into the attention library and the engine's host core.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace vfl {

constexpr int PLAN_PREFIX = 4;
constexpr int PLAN_MAX_ROWS = 8;        // rows per group
constexpr int PLAN_HEADER = 4;
constexpr int PLAN_ENTRY = 2;
constexpr int PLAN_MAX_POSITION = 32767;
constexpr uint32_t PLAN_COPY = 1u << 31;

// Words of one slot for groups of up to max_group rows and tables max_blocks wide:
// room for every row holding a distinct block at every position, rounded up to 16
// bytes.  0 when the sizes are out of range.
inline int64_t group_plan_stride(int max_group, int64_t max_blocks) {
  if (max_group < 1 || max_group > PLAN_MAX_ROWS || max_blocks < 0 ||
      max_blocks > PLAN_MAX_POSITION + 1)
    return 0;
  const int64_t words = PLAN_HEADER + (int64_t)PLAN_ENTRY * max_group * max_blocks;
  return (words + 3) / 4 * 4;
}

// Fill plan (PLAN_PREFIX + num_slots * stride words) for the groups of one step:
// slot s holds group order[s] (group s when order is null) for s < num_groups, the
// rest are empty.  Group g owns rows group_start[g] .. group_start[g+1]-1 of
// block_table (row stride bt_stride, max_blocks entries read per row) and seq_lens; a
// row reads its first min(ceil(len / block_size), max_blocks) blocks.
// Returns 0, or -1 with *why set (nothing is guaranteed about plan then).
inline int build_group_plan(const int32_t *block_table, int64_t bt_stride, int max_blocks,
                            const int32_t *seq_lens, int64_t num_rows,
                            const int32_t *group_start, const int32_t *order,
                            int64_t num_groups, int block_size, int64_t num_blocks,
                            int32_t *plan, int64_t num_slots, int64_t stride,
                            const char **why) {
  *why = nullptr;
  if (num_groups < 0 || num_groups > num_slots || num_rows < 0 || max_blocks < 0 ||
      max_blocks > PLAN_MAX_POSITION + 1 || block_size <= 0 || block_size > 255 ||
      stride < PLAN_HEADER ||
      stride % 4 != 0 || bt_stride < max_blocks) {
    *why = "bad sizes";
    return -1;
  }
  if (num_groups > 0 && (!block_table || !seq_lens || !group_start)) {
    *why = "null table, lengths or group starts";
    return -1;
  }
  const int64_t cap = (stride - PLAN_HEADER) / PLAN_ENTRY;
  plan[0] = (int32_t)num_groups;
  plan[1] = plan[2] = plan[3] = 0;
  for (int64_t s = 0; s < num_slots; ++s) {
    int32_t *rec = plan + PLAN_PREFIX + s * stride;
    rec[0] = rec[1] = rec[2] = rec[3] = 0;
    if (s >= num_groups) continue;
    const int64_t g = order ? order[s] : s;
    if (g < 0 || g >= num_groups) {
      *why = "group order entry out of range";
      return -1;
    }
    const int64_t r0 = group_start[g], r1 = group_start[g + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_rows || r1 - r0 > PLAN_MAX_ROWS) {
      *why = "group rows out of range (at most 8 rows per group)";
      return -1;
    }
    const int n = (int)(r1 - r0);
    int nblk[PLAN_MAX_ROWS];
    int64_t covered[PLAN_MAX_ROWS];  // tokens the row attends to: min(len, nblk * bs)
    int widest = 0;
    for (int c = 0; c < n; ++c) {
      const int64_t len = seq_lens[r0 + c];
      int64_t b = len > 0 ? (len + block_size - 1) / block_size : 0;
      if (b > max_blocks) b = max_blocks;
      nblk[c] = (int)b;
      covered[c] = len < b * block_size ? len : b * block_size;
      if (nblk[c] > widest) widest = nblk[c];
    }
    int64_t ne = 0;
    int32_t *ent = rec + PLAN_HEADER;
    for (int p = 0; p < widest; ++p) {
      const int64_t first = ne;
      for (int c = 0; c < n; ++c) {
        if (p >= nblk[c]) continue;
        const int32_t id = block_table[(r0 + c) * bt_stride + p];
        if (id < 0 || id >= num_blocks) continue;
        int64_t t = covered[c] - (int64_t)p * block_size;  // >= 1 since p < nblk[c]
        if (t > block_size) t = block_size;
        int64_t k = first;
        while (k < ne && ent[PLAN_ENTRY * k] != id) ++k;
        if (k < ne) {
          uint32_t w = (uint32_t)ent[PLAN_ENTRY * k + 1];
          const uint32_t had = (w >> 8) & 0xffu;
          if ((uint32_t)t > had) w = (w & ~0xff00u) | ((uint32_t)t << 8);
          ent[PLAN_ENTRY * k + 1] = (int32_t)(w | (1u << c));
        } else {
          if (ne >= cap) {
            *why = "a group has more distinct blocks than the plan stride holds";
            return -1;
          }
          ent[PLAN_ENTRY * ne] = id;
          ent[PLAN_ENTRY * ne + 1] =
              (int32_t)(((uint32_t)p << 16) | ((uint32_t)t << 8) | (1u << c));
          ++ne;
        }
      }
    }
    rec[0] = (int32_t)r0;
    rec[1] = n;
    rec[2] = (int32_t)ne;
    rec[3] = widest;
  }
  return 0;
}

// Slot descriptors of shared-table row groups (the beams of a request reading its
// encoder pages in cross-attention): slot s at s * stride, for s < num_groups the group
// group_order[s] (s when order is null): [first row, rows, length of the first row, 0,
// the first row's table row (max_blocks ids)]; later slots [0, 0, 0, 0].  The
// attention launch reads its group from its slot in one load level.
inline int64_t slot_descriptor_stride(int64_t max_blocks) {
  if (max_blocks < 0 || max_blocks > (int64_t)1 << 24) return 0;
  return (4 + max_blocks + 3) / 4 * 4;
}

inline int build_slot_descriptors(const int32_t *block_table, int64_t bt_stride, int max_blocks,
                                  const int32_t *seq_lens, int64_t num_rows,
                                  const int32_t *group_start, const int32_t *order,
                                  int64_t num_groups, int32_t *desc, int64_t num_slots,
                                  int64_t stride, const char **why) {
  *why = nullptr;
  if (num_groups < 0 || num_groups > num_slots || num_rows < 0 || max_blocks < 0 ||
      stride < slot_descriptor_stride(max_blocks) || stride % 4 != 0 || bt_stride < max_blocks) {
    *why = "bad sizes";
    return -1;
  }
  if (num_groups > 0 && (!block_table || !seq_lens || !group_start)) {
    *why = "null table, lengths or group starts";
    return -1;
  }
  for (int64_t s = 0; s < num_slots; ++s) {
    int32_t *rec = desc + s * stride;
    rec[0] = rec[1] = rec[2] = rec[3] = 0;
    if (s >= num_groups) continue;
    const int64_t g = order ? order[s] : s;
    if (g < 0 || g >= num_groups) {
      *why = "group order entry out of range";
      return -1;
    }
    const int64_t r0 = group_start[g], r1 = group_start[g + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_rows) {
      *why = "group rows out of range";
      return -1;
    }
    if (r1 == r0) continue;
    rec[0] = (int32_t)r0;
    rec[1] = (int32_t)(r1 - r0);
    rec[2] = seq_lens[r0];
    for (int b = 0; b < max_blocks; ++b) rec[4 + b] = block_table[r0 * bt_stride + b];
  }
  return 0;
}

// Destination block -> copy pair index, for fold_plan_copies: open addressing over a
// power-of-two table at least twice the pairs, kept per thread so that a call
// allocates only when a step brings more pairs than any before it.
struct CopyDestinations {
  std::vector<int64_t> key, pair;
  int64_t mask = 0;

  void reset(int64_t num_pairs) {
    int64_t cap = 16;
    while (cap < 2 * num_pairs) cap *= 2;
    if ((int64_t)key.size() < cap) {
      key.resize(cap);
      pair.resize(cap);
    }
    mask = cap - 1;
    std::fill(key.begin(), key.begin() + cap, -1);
  }
  int64_t slot_of(int64_t block) const {
    int64_t h = (int64_t)(((uint64_t)block * 0x9E3779B97F4A7C15ull) >> 20) & mask;
    while (key[h] != -1 && key[h] != block) h = (h + 1) & mask;
    return h;
  }
  // false when block is a destination already
  bool insert(int64_t block, int64_t i) {
    const int64_t h = slot_of(block);
    if (key[h] == block) return false;
    key[h] = block;
    pair[h] = i;
    return true;
  }
  int64_t find(int64_t block) const {  // the pair index, or -1
    if (block < 0) return -1;  // -1 marks a free table slot
    const int64_t h = slot_of(block);
    return key[h] == block ? pair[h] : -1;
  }
};

// Fold a step's copy-on-write pairs (src[i] -> dst[i]) into its plan (the used slots
// of build_group_plan's output): the entry holding block dst[i] gets the copy flag and
// src[i] in place of dst[i].  Each destination must be a block in
// [0, num_blocks) that exactly one entry of the plan holds, for one row, at that row's
// last position (the fresh block a fork writes into), one per row; sources in
// [0, num_blocks); no block both a destination and a source, no destination twice.  All
// pairs are checked before the plan changes: on -1 (with *why set) the plan is as it
// was and the caller copies the pairs itself.
inline int fold_plan_copies(int32_t *plan, int64_t num_slots, int64_t stride,
                            const int64_t *src, const int64_t *dst, int64_t num_pairs,
                            int64_t num_blocks, const char **why) {
  *why = nullptr;
  if (num_pairs < 0 || num_slots < 0 || stride < PLAN_HEADER || stride % 4 != 0 ||
      (num_pairs > 0 && (!src || !dst))) {
    *why = "bad sizes or null pairs";
    return -1;
  }
  if (num_pairs == 0) return 0;
  const int64_t used = plan[0];
  if (used < 0 || used > num_slots) {
    *why = "plan slot count out of range";
    return -1;
  }
  for (int64_t i = 0; i < num_pairs; ++i)
    if (src[i] < 0 || src[i] >= num_blocks || dst[i] < 0 || dst[i] >= num_blocks) {
      *why = "copy pair block out of range";
      return -1;
    }
  static thread_local CopyDestinations dests;
  dests.reset(num_pairs);
  for (int64_t i = 0; i < num_pairs; ++i)
    if (!dests.insert(dst[i], i)) {
      *why = "a block is the destination of two copies";
      return -1;
    }
  for (int64_t i = 0; i < num_pairs; ++i)
    if (dests.find(src[i]) >= 0) {
      *why = "a block is both a copy source and a destination";
      return -1;
    }
  static thread_local std::vector<int32_t *> where;  // each pair's destination entry
  where.assign(num_pairs, nullptr);
  // A bit per pool block marks the destinations, so the scan below tests most entries
  // with one bit instead of a hash probe (a 64 x 4-beam step's ~40 pairs over ~640
  // entries: 8.6 -> 5.2 us on one host core); the bits are cleared again on return.
  static thread_local std::vector<uint64_t> is_dst;
  if ((int64_t)is_dst.size() * 64 < num_blocks) is_dst.resize((size_t)((num_blocks + 63) / 64));
  for (int64_t i = 0; i < num_pairs; ++i) is_dst[(size_t)dst[i] >> 6] |= 1ull << (dst[i] & 63);
  struct ClearBits {
    const int64_t *d;
    int64_t n;
    ~ClearBits() {
      for (int64_t i = 0; i < n; ++i) is_dst[(size_t)d[i] >> 6] = 0;
    }
  } clear_bits{dst, num_pairs};
  for (int64_t s = 0; s < used; ++s) {
    int32_t *rec = plan + PLAN_PREFIX + s * stride;
    const int64_t ne = rec[2];
    if (ne < 0 || PLAN_HEADER + ne * PLAN_ENTRY > stride) {
      *why = "plan slot entry count out of range";
      return -1;
    }
    // each row's last position in the slot (a destination must be there: it is the block
    // the row's new token goes to, where the fused launch stores the copy), found once a
    // slot holds a destination
    int32_t last_pos[PLAN_MAX_ROWS];
    bool have_last = false;
    uint32_t taken = 0;  // rows of the slot that received a copy source
    for (int64_t e = 0; e < ne; ++e) {
      int32_t *ent = rec + PLAN_HEADER + PLAN_ENTRY * e;
      const int64_t id = ent[0];
      if (id < 0 || id >= num_blocks || !((is_dst[(size_t)id >> 6] >> (id & 63)) & 1u)) continue;
      const int64_t i = dests.find(id);
      if (i < 0) continue;
      const uint32_t rows = (uint32_t)ent[1] & 0xffu;
      if (where[i] != nullptr || rows == 0 || (rows & (rows - 1u)) != 0) {
        *why = "a copy destination is listed by several rows or entries";
        return -1;
      }
      const int c = __builtin_ctz(rows);
      if ((taken >> c) & 1u) {
        *why = "a row has two copy destinations";
        return -1;
      }
      if (!have_last) {
        for (int r = 0; r < PLAN_MAX_ROWS; ++r) last_pos[r] = -1;
        for (int64_t f = 0; f < ne; ++f) {
          const uint32_t meta = (uint32_t)rec[PLAN_HEADER + PLAN_ENTRY * f + 1];
          const int32_t pos = (int32_t)((meta >> 16) & 0x7fffu);
          for (uint32_t m = meta & 0xffu; m; m &= m - 1u) {
            const int r = __builtin_ctz(m);
            last_pos[r] = std::max(last_pos[r], pos);
          }
        }
        have_last = true;
      }
      if ((int32_t)(((uint32_t)ent[1] >> 16) & 0x7fffu) != last_pos[c]) {
        *why = "a copy destination is not its row's last block";
        return -1;
      }
      taken |= 1u << c;
      where[i] = ent;
    }
  }
  for (int64_t i = 0; i < num_pairs; ++i)
    if (where[i] == nullptr) {
      *why = "a copy destination is not a block of the plan";
      return -1;
    }
  for (int64_t i = 0; i < num_pairs; ++i) {
    where[i][0] = (int32_t)src[i];
    where[i][1] = (int32_t)((uint32_t)where[i][1] | PLAN_COPY);
  }
  return 0;
}

}  // namespace vfl
