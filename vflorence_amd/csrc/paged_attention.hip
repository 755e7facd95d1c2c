// Paged decode attention for gfx950: the entry points of include/vflorence_amd.h that
// run attention (metadata, group plans, attention with and without the fused KV write)
// and their dispatch to the kernels:
//   decode_valu.h     fp32 caches (VALU; any head size)
//   decode_mfma.h     16-bit caches, one row or a group sharing one table per workgroup
//   decode_shared.h   16-bit, beams keeping their own tables, walked in the launch
//   decode_planned.h  16-bit, beams keeping their own tables, from a host-built plan
// The beam-group, group-plan and fused-write kernels are built for head sizes 64 and
// 128 (BART, Florence-2); the reference's other head sizes run the one-row / shared-
// table kernels (attention_dims.hip) with the KV write as a separate launch.
#include "attention_dispatch.h"
#include "decode_planned.h"
#include "decode_valu.h"

namespace vfl {


// bf16 / fp16 caches: matrix-core kernel over the token-interleaved V layout; the tile
// columns hold up to 16 query rows per group, so one instantiation serves any G.
constexpr int MFMA_STAGE_BLOCKS = 2;
// Stage size of the own-tables group kernel (measured on MI355X, 64 x 4-beam decode
// steps: 3 and 4 blocks per stage were no faster and cost occupancy).
constexpr int SHARED_STAGE_BLOCKS = 2;

// Stage size of the planned group kernel: every wave requests this many blocks per
// round trip.  Measured on the 64 x 4-beam decode step (two passes each, one box): 4 / 5
// / 6 / 8 blocks ran the step in 0.5382 / 0.5361 / 0.5350 / 0.5354 ms; six needs 204
// VGPRs, still two waves per SIMD (all the launch's waves resident).
constexpr int PLANNED_STAGE_BLOCKS = 6;

template <int DT, int D, int NW>
static int launch_planned(const AttnArgs &a) {
  const dim3 grid((unsigned)xcd_grid(a.plan_slots, a.H));
  if (a.kvw.slots)
    paged_decode_planned_kernel<DT, D, NW, PLANNED_STAGE_BLOCKS, true>
        <<<grid, dim3(NW * 64), 0, a.stream>>>(
        (const uint16_t *)a.q, a.q_st, a.q_sh, a.q_vec, (const uint16_t *)a.kc,
        (const uint16_t *)a.vc, (uint16_t *)a.out, a.seq_lens, a.plan, a.plan_stride,
        a.plan_slots, a.max_blocks, a.num_rows, a.H, a.num_blocks, a.scale_log2, a.kvw);
  else
    paged_decode_planned_kernel<DT, D, NW, PLANNED_STAGE_BLOCKS, false>
        <<<grid, dim3(NW * 64), 0, a.stream>>>(
        (const uint16_t *)a.q, a.q_st, a.q_sh, a.q_vec, (const uint16_t *)a.kc,
        (const uint16_t *)a.vc, (uint16_t *)a.out, a.seq_lens, a.plan, a.plan_stride,
        a.plan_slots, a.max_blocks, a.num_rows, a.H, a.num_blocks, a.scale_log2, a.kvw);
  return launch_status("attention_with_kv_cache");
}

template <int DT, int D, int NW>
static int launch_mfma(const AttnArgs &a) {
  if (a.plan) return launch_planned<DT, D, NW>(a);
  const dim3 grid((unsigned)xcd_grid(a.num_groups, a.H));
  if (a.own_tables) {
    if (a.kvw.slots)
      paged_decode_shared_kernel<DT, D, NW, SHARED_STAGE_BLOCKS, true>
          <<<grid, dim3(NW * 64), 0, a.stream>>>(
          (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
          (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
          a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw);
    else
      paged_decode_shared_kernel<DT, D, NW, SHARED_STAGE_BLOCKS, false>
          <<<grid, dim3(NW * 64), 0, a.stream>>>(
          (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
          (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
          a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw);
    return launch_status("attention_with_kv_cache");
  }
  if (a.kvw.slots)
    paged_decode_mfma_kernel<DT, D, NW, MFMA_STAGE_BLOCKS, true, 0>
        <<<grid, dim3(NW * 64), 0, a.stream>>>(
        (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
        (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
        a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw);
  else
    paged_decode_mfma_kernel<DT, D, NW, MFMA_STAGE_BLOCKS, false, 0>
        <<<grid, dim3(NW * 64), 0, a.stream>>>(
        (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
        (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
        a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw, a.desc,
        a.desc_stride);
  return launch_status("attention_with_kv_cache");
}

template <int DT, int D>
static int mfma_waves(const AttnArgs &a, int nw) {
  switch (nw) {
    case 1: return launch_mfma<DT, D, 1>(a);
    case 2: return launch_mfma<DT, D, 2>(a);
    case 4: return launch_mfma<DT, D, 4>(a);
    default:
      // The merge buffer of 8 waves x head_dim 128 exceeds 64 KiB of LDS.
      if constexpr (D <= 64) return launch_mfma<DT, D, 8>(a);
      else return launch_mfma<DT, D, 4>(a);
  }
}

static int dispatch(const AttnArgs &a, int dtype, int head_dim, int gmax, int nw) {
  if (a.bs_shift != 0) return dispatch_block32(a, dtype, head_dim, gmax, nw);
  if (dtype == VFL_FLOAT32) {
    if (head_dim == 64) return valu_group<64>(a, gmax, nw);
    if (head_dim == 128) return valu_group<128>(a, gmax, nw);
  } else if (dtype == VFL_BFLOAT16) {
    if (head_dim == 64) return mfma_waves<VFL_BFLOAT16, 64>(a, nw);
    if (head_dim == 128) return mfma_waves<VFL_BFLOAT16, 128>(a, nw);
  } else {
    if (head_dim == 64) return mfma_waves<VFL_FLOAT16, 64>(a, nw);
    if (head_dim == 128) return mfma_waves<VFL_FLOAT16, 128>(a, nw);
  }
  return dispatch_other_head_dim(a, dtype, head_dim, gmax, nw);
}

static bool kernel_exists(int dtype, int block_size, int head_dim) {
  return (dtype == VFL_FLOAT32 || dtype == VFL_BFLOAT16 || dtype == VFL_FLOAT16) &&
         block_shift(block_size) >= 0 && head_dim_supported(head_dim);
}

constexpr int MAX_GROUP = 8;
constexpr int MAX_WAVES = 8;

// Waves per (group, head) workgroup.  Measured on MI355X (bf16, head_dim 64, K/V pages
// loaded non-temporally), 64 x 4-beam cross-attention (1024 workgroups) in the decode
// step: two / four / eight waves 34.9 / 29.5 / 30.6 us (four keeps all 1024 workgroups
// resident at once); 256 ragged self-attention rows (4096 workgroups) run within noise
// of each other with two, four or eight.  So four, and eight only below two workgroups
// per CU, where a workgroup's blocks need the extra waves.  Never more waves than
// blocks.
static int default_waves(int64_t num_groups, int num_heads, int64_t max_blocks) {
  const int64_t wgs = num_groups * num_heads;
  int nw = wgs >= 512 ? 4 : 8;
  while (nw > 1 && nw / 2 >= max_blocks) nw /= 2;
  return nw;
}

}  // namespace vfl

using namespace vfl;

extern "C" const char *vfl_get_isa(int dtype, int block_size, int head_dim) {
  return kernel_exists(dtype, block_size, head_dim) ? "gfx950" : nullptr;
}

extern "C" int vfl_get_scheduler_metadata(int64_t num_rows, int64_t num_groups, int num_heads,
                                          int head_dim, int block_size,
                                          int64_t max_blocks_per_seq, int max_group_size,
                                          int dtype, int waves_per_workgroup, int group_tables,
                                          vfl_sched_meta *meta) {
  clear_error();
  if (!meta) {
    set_error("get_scheduler_metadata: meta is NULL");
    return VFL_E_INVALID;
  }
  if (num_rows < 0 || num_groups < 0 || num_groups > num_rows || num_heads <= 0 ||
      num_heads > 65535 || max_blocks_per_seq < 0 || max_blocks_per_seq > (1 << 30)) {
    set_error("get_scheduler_metadata: bad sizes (rows %lld groups %lld heads %d blocks %lld)",
              (long long)num_rows, (long long)num_groups, num_heads,
              (long long)max_blocks_per_seq);
    return VFL_E_INVALID;
  }
  if (!kernel_exists(dtype, block_size, head_dim)) {
    set_error("get_scheduler_metadata: no kernel for dtype %d block_size %d head_dim %d", dtype,
              block_size, head_dim);
    return VFL_E_UNSUPPORTED;
  }
  if (max_group_size < 1 || max_group_size > MAX_GROUP) {
    set_error("get_scheduler_metadata: max_group_size %d outside [1, %d]", max_group_size,
              MAX_GROUP);
    return VFL_E_UNSUPPORTED;
  }
  if (group_tables != VFL_GROUP_SHARED_TABLE && group_tables != VFL_GROUP_OWN_TABLES) {
    set_error("get_scheduler_metadata: group_tables %d is not VFL_GROUP_SHARED_TABLE or "
              "VFL_GROUP_OWN_TABLES", group_tables);
    return VFL_E_INVALID;
  }
  int nw = waves_per_workgroup;
  if (nw == 0) nw = default_waves(num_groups, num_heads, max_blocks_per_seq);
  if (nw != 1 && nw != 2 && nw != 4 && nw != 8) {
    set_error("get_scheduler_metadata: waves_per_workgroup %d not in {0, 1, 2, 4, 8}", nw);
    return VFL_E_UNSUPPORTED;
  }
  if (xcd_grid(num_groups, num_heads) > 2147483647LL) {
    set_error("get_scheduler_metadata: too many groups x heads for one grid");
    return VFL_E_UNSUPPORTED;
  }
  meta->num_rows = num_rows;
  meta->num_groups = num_groups;
  meta->num_heads = num_heads;
  meta->head_dim = head_dim;
  meta->max_blocks_per_seq = (int32_t)max_blocks_per_seq;
  meta->waves_per_workgroup = nw;
  meta->max_group_size = max_group_size;
  meta->group_tables = group_tables;
  meta->group_plan = nullptr;
  meta->group_plan_stride = 0;
  meta->group_plan_slots = 0;
  return VFL_OK;
}

extern "C" int64_t vfl_group_plan_stride(int max_group_size, int64_t max_blocks_per_seq) {
  return group_plan_stride(max_group_size, max_blocks_per_seq);
}

extern "C" int vfl_build_group_plan(const int32_t *block_table, int64_t block_table_stride,
                                    int max_blocks_per_seq, const int32_t *seq_lens,
                                    int64_t num_rows, const int32_t *group_start,
                                    const int32_t *group_order, int64_t num_groups,
                                    int block_size, int64_t num_blocks, int32_t *plan,
                                    int64_t num_slots, int64_t stride) {
  clear_error();
  if (!plan) {
    set_error("build_group_plan: plan is NULL");
    return VFL_E_INVALID;
  }
  const char *why = nullptr;
  if (build_group_plan(block_table, block_table_stride, max_blocks_per_seq, seq_lens, num_rows,
                       group_start, group_order, num_groups, block_size, num_blocks, plan,
                       num_slots, stride, &why) != 0) {
    set_error("build_group_plan: %s", why);
    return VFL_E_INVALID;
  }
  return VFL_OK;
}

extern "C" int64_t vfl_slot_descriptor_stride(int64_t max_blocks_per_seq) {
  return slot_descriptor_stride(max_blocks_per_seq);
}

extern "C" int vfl_build_slot_descriptors(const int32_t *block_table, int64_t block_table_stride,
                                          int max_blocks_per_seq, const int32_t *seq_lens,
                                          int64_t num_rows, const int32_t *group_start,
                                          const int32_t *group_order, int64_t num_groups,
                                          int32_t *desc, int64_t num_slots, int64_t stride) {
  clear_error();
  if (!desc) {
    set_error("build_slot_descriptors: desc is NULL");
    return VFL_E_INVALID;
  }
  const char *why = nullptr;
  if (build_slot_descriptors(block_table, block_table_stride, max_blocks_per_seq, seq_lens,
                             num_rows, group_start, group_order, num_groups, desc, num_slots,
                             stride, &why) != 0) {
    set_error("build_slot_descriptors: %s", why);
    return VFL_E_INVALID;
  }
  return VFL_OK;
}

extern "C" int vfl_fold_plan_copies(int32_t *plan, int64_t num_slots, int64_t stride,
                                    const int64_t *src, const int64_t *dst, int64_t num_pairs,
                                    int64_t num_blocks) {
  clear_error();
  if (!plan) {
    set_error("fold_plan_copies: plan is NULL");
    return VFL_E_INVALID;
  }
  const char *why = nullptr;
  if (fold_plan_copies(plan, num_slots, stride, src, dst, num_pairs, num_blocks, &why) != 0) {
    set_error("fold_plan_copies: %s", why);
    return VFL_E_INVALID;
  }
  return VFL_OK;
}

// Shared argument checks and launch of both attention entry points.
static int attention_impl(const void *query, int64_t query_stride_token,
                          int64_t query_stride_head, const void *k_cache, const void *v_cache,
                          void *out, const int32_t *seq_lens, const int32_t *block_table,
                          int64_t block_table_stride, const int32_t *group_start,
                          const int32_t *group_order, int64_t num_rows, int64_t num_groups,
                          int num_heads, int head_dim, int block_size, int64_t num_blocks,
                          float scale, int dtype, const vfl_sched_meta *meta, void *stream,
                          const KvWrite &kvw, const char *who) {
  if (!meta) {
    set_error("%s: meta is NULL", who);
    return VFL_E_INVALID;
  }
  if (!kernel_exists(dtype, block_size, head_dim)) {
    set_error("%s: no kernel for dtype %d block_size %d head_dim %d", who, dtype, block_size,
              head_dim);
    return VFL_E_UNSUPPORTED;
  }
  if (num_rows < 0 || num_heads <= 0 || num_blocks < 0) {
    set_error("%s: bad sizes", who);
    return VFL_E_INVALID;
  }
  if (meta->num_rows != num_rows || meta->num_groups != num_groups ||
      meta->num_heads != num_heads || meta->head_dim != head_dim) {
    set_error("%s: metadata was made for rows %lld groups %lld heads %d head_dim %d, call has "
              "rows %lld groups %lld heads %d head_dim %d",
              who, (long long)meta->num_rows, (long long)meta->num_groups, meta->num_heads,
              meta->head_dim, (long long)num_rows, (long long)num_groups, num_heads, head_dim);
    return VFL_E_INVALID;
  }
  if (group_start == nullptr && num_groups != num_rows) {
    set_error("%s: without group_start, num_groups (%lld) must equal num_rows (%lld)", who,
              (long long)num_groups, (long long)num_rows);
    return VFL_E_INVALID;
  }
  if (num_groups < 0 || num_groups > num_rows || num_heads <= 0 || num_heads > 65535 ||
      xcd_grid(num_groups, num_heads) > 2147483647LL) {
    set_error("%s: num_groups %lld / num_heads %d out of range", who, (long long)num_groups,
              num_heads);
    return VFL_E_INVALID;
  }
  const int nw = meta->waves_per_workgroup;
  if (meta->max_group_size < 1 || meta->max_group_size > MAX_GROUP ||
      (nw != 1 && nw != 2 && nw != 4 && nw != 8) || meta->max_blocks_per_seq < 0 ||
      (meta->group_tables != VFL_GROUP_SHARED_TABLE &&
       meta->group_tables != VFL_GROUP_OWN_TABLES)) {
    set_error("%s: inconsistent metadata", who);
    return VFL_E_INVALID;
  }
  if (block_table_stride < meta->max_blocks_per_seq) {
    set_error("%s: block_table_stride %lld < max_blocks_per_seq %d", who,
              (long long)block_table_stride, meta->max_blocks_per_seq);
    return VFL_E_INVALID;
  }
  if (num_rows == 0 || num_groups == 0) return VFL_OK;
  if (!query || !k_cache || !v_cache || !out || !seq_lens || !block_table) {
    set_error("%s: null pointer argument", who);
    return VFL_E_INVALID;
  }
  if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) % 16 != 0) {
    set_error("%s: caches and out must be 16-byte aligned", who);
    return VFL_E_INVALID;
  }
  AttnArgs a;
  a.q = query;
  a.q_st = query_stride_token;
  a.q_sh = query_stride_head;
  a.kc = k_cache;
  a.vc = v_cache;
  a.out = out;
  a.seq_lens = seq_lens;
  a.bt = block_table;
  a.bt_stride = block_table_stride;
  a.max_blocks = meta->max_blocks_per_seq;
  a.group_start = group_start;
  a.group_order = group_order;
  a.num_rows = num_rows;
  a.num_groups = num_groups;
  a.H = num_heads;
  a.num_blocks = num_blocks;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.stream = (hipStream_t)stream;
  a.kvw = kvw;
  a.own_tables = group_start != nullptr && meta->group_tables == VFL_GROUP_OWN_TABLES;
  a.plan = nullptr;
  a.plan_stride = a.plan_slots = 0;
  a.q_vec = (uintptr_t)query % 16 == 0 && query_stride_token % 8 == 0 &&
            query_stride_head % 8 == 0;
  a.bs_shift = block_shift(block_size);
  // Kernels with own-table groups, plans and the fused write exist for 16-bit caches
  // of head size 64 and 128 in 16-token blocks.
  const bool full_set = dtype != VFL_FLOAT32 && head_dim_native(head_dim) && block_size == 16;
  if (meta->group_plan != nullptr && a.own_tables && full_set) {
    if ((uintptr_t)meta->group_plan % 16 != 0 || meta->group_plan_stride < PLAN_HEADER ||
        meta->group_plan_stride % 4 != 0 || meta->group_plan_slots < num_groups ||
        xcd_grid(meta->group_plan_slots, num_heads) > 2147483647LL ||
        meta->max_group_size > PLAN_MAX_ROWS) {
      set_error("%s: group plan of %lld slots x %lld words (16-byte aligned, stride a "
                "multiple of 4, at least num_groups %lld slots, groups of <= %d rows)",
                who, (long long)meta->group_plan_slots, (long long)meta->group_plan_stride,
                (long long)num_groups, PLAN_MAX_ROWS);
      return VFL_E_INVALID;
    }
    a.plan = meta->group_plan;
    a.plan_stride = meta->group_plan_stride;
    a.plan_slots = meta->group_plan_slots;
  }
  // Shared-table groups (cross-attention beams) with slot descriptors in group_plan.
  a.desc = nullptr;
  a.desc_stride = 0;
  if (meta->group_plan != nullptr && !a.own_tables && group_start != nullptr && full_set &&
      kvw.slots == nullptr) {
    if ((uintptr_t)meta->group_plan % 16 != 0 ||
        meta->group_plan_stride < slot_descriptor_stride(meta->max_blocks_per_seq) ||
        meta->group_plan_stride % 4 != 0 || meta->group_plan_slots < num_groups) {
      set_error("%s: slot descriptors of %lld slots x %lld words (16-byte aligned, stride at "
                "least %lld, at least num_groups %lld slots)",
                who, (long long)meta->group_plan_slots, (long long)meta->group_plan_stride,
                (long long)slot_descriptor_stride(meta->max_blocks_per_seq),
                (long long)num_groups);
      return VFL_E_INVALID;
    }
    a.desc = meta->group_plan;
    a.desc_stride = meta->group_plan_stride;
  }
  if (a.own_tables && !full_set) {
    // The VALU kernel and the one-row matrix-core kernel read one table per group; with
    // rows keeping their own tables every row is its own group instead (same results:
    // grouping is only a sharing of loads), in natural order.
    a.own_tables = false;
    a.group_start = nullptr;
    a.group_order = nullptr;
    a.num_groups = num_rows;
    return dispatch(a, dtype, head_dim, 1, nw);
  }
  return dispatch(a, dtype, head_dim, meta->max_group_size, nw);
}

extern "C" int vfl_attention_with_kv_cache(
    const void *query, int64_t query_stride_token, int64_t query_stride_head,
    const void *k_cache, const void *v_cache, void *out, const int32_t *seq_lens,
    const int32_t *block_table, int64_t block_table_stride, const int32_t *group_start,
    const int32_t *group_order, int64_t num_rows, int64_t num_groups, int num_heads,
    int head_dim, int block_size, int64_t num_blocks, float scale, int dtype,
    const vfl_sched_meta *meta, void *stream) {
  clear_error();
  const KvWrite none = {nullptr, 0, 0, nullptr, 0, 0, nullptr, false};
  return attention_impl(query, query_stride_token, query_stride_head, k_cache, v_cache, out,
                        seq_lens, block_table, block_table_stride, group_start, group_order,
                        num_rows, num_groups, num_heads, head_dim, block_size, num_blocks, scale,
                        dtype, meta, stream, none, "attention_with_kv_cache");
}

extern "C" int vfl_self_attention_with_kv_write(
    const void *query, int64_t query_stride_token, int64_t query_stride_head, const void *key,
    int64_t key_stride_token, int64_t key_stride_head, const void *value,
    int64_t value_stride_token, int64_t value_stride_head, const int64_t *slot_mapping,
    void *k_cache, void *v_cache, void *out, const int32_t *seq_lens,
    const int32_t *block_table, int64_t block_table_stride, const int32_t *group_start,
    const int32_t *group_order, int64_t num_rows, int64_t num_groups, int num_heads,
    int head_dim, int block_size, int64_t num_blocks, float scale, int dtype,
    const vfl_sched_meta *meta, void *stream) {
  clear_error();
  if (num_rows > 0 && (!key || !value || !slot_mapping)) {
    set_error("self_attention_with_kv_write: null key, value or slot_mapping");
    return VFL_E_INVALID;
  }
  if (group_start != nullptr && (meta == nullptr || meta->group_tables != VFL_GROUP_OWN_TABLES)) {
    set_error("self_attention_with_kv_write: row groups need metadata made with "
              "VFL_GROUP_OWN_TABLES (every row keeps its own block table)");
    return VFL_E_INVALID;
  }
  if (dtype == VFL_FLOAT32 || !head_dim_native(head_dim) || block_size != 16) {
    // No fused kernel for fp32, for head sizes other than 64 and 128, or for 32-token
    // blocks: the same two steps as the reference.
    int st = vfl_reshape_and_cache(key, value, key_stride_token, key_stride_head,
                                   value_stride_token, value_stride_head, k_cache, v_cache,
                                   slot_mapping, num_rows, num_heads, head_dim, block_size,
                                   num_blocks, dtype, stream);
    if (st != VFL_OK) return st;
    return vfl_attention_with_kv_cache(query, query_stride_token, query_stride_head, k_cache,
                                       v_cache, out, seq_lens, block_table, block_table_stride,
                                       group_start, group_order, num_rows, num_groups,
                                       num_heads, head_dim, block_size, num_blocks, scale, dtype,
                                       meta, stream);
  }
  const bool vec = (uintptr_t)key % 16 == 0 && key_stride_token % 8 == 0 &&
                   key_stride_head % 8 == 0 && (uintptr_t)value % 16 == 0 &&
                   value_stride_token % 8 == 0 && value_stride_head % 8 == 0;
  const KvWrite kvw = {(const uint16_t *)key, key_stride_token, key_stride_head,
                       (const uint16_t *)value, value_stride_token, value_stride_head,
                       slot_mapping, vec};
  if (num_rows == 0) return VFL_OK;
  return attention_impl(query, query_stride_token, query_stride_head, k_cache, v_cache, out,
                        seq_lens, block_table, block_table_stride, group_start, group_order,
                        num_rows, num_groups, num_heads, head_dim, block_size, num_blocks, scale,
                        dtype, meta, stream, kvw, "self_attention_with_kv_write");
}
