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
//       [1] position << 16 | tokens << 8 | row mask (bit c: row first + c)
// A slot's entries list, position by position, the distinct block ids the group's
// rows hold there (ids outside [0, num_blocks) left out), each once, with the rows
// that list it, in order of each id's first row: the blocks the shared kernel finds
// by walking the tables, in the order it finds them.  `tokens` (1..block_size) is how
// many of the block's tokens the longest of those rows attends to: the kernel reads
// no K or V past them.
// Plain C++ (no HIP): compiled into the attention library and the engine's host core.
#pragma once

#include <stdint.h>

namespace vfl {

constexpr int PLAN_PREFIX = 4;
constexpr int PLAN_HEADER = 4;
constexpr int PLAN_ENTRY = 2;
constexpr int PLAN_MAX_ROWS = 8;        // rows per group
constexpr int PLAN_MAX_POSITION = 65535;

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

}  // namespace vfl
