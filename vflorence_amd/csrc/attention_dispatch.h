// Launch arguments and kernel selection shared by the attention entry points
// (paged_attention.hip) and the instantiations for the reference's other head sizes
// (attention_dims.hip).
#pragma once

#include "decode_mfma.h"
#include "decode_valu.h"

namespace vfl {

struct AttnArgs {
  const void *q;
  int64_t q_st, q_sh;
  const void *kc, *vc;
  void *out;
  const int32_t *seq_lens, *bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t *group_start, *group_order;
  int64_t num_rows, num_groups;
  int H;
  int64_t num_blocks;
  float scale_log2;
  hipStream_t stream;
  KvWrite kvw;      // slots == nullptr: no fused KV write
  bool own_tables;  // groups whose rows keep their own tables (paged_decode_shared_kernel)
  const int32_t *plan;  // group plan (paged_decode_planned_kernel), or nullptr
  int64_t plan_stride, plan_slots;
  const int32_t *desc;  // slot descriptors of shared-table groups (decode_mfma.h), or nullptr
  int64_t desc_stride;
  bool q_vec;  // query rows 16-byte aligned
  int bs_shift;  // pool blocks of 16 << bs_shift tokens
};

// Head sizes the reference's attention op accepts (vflorence/layers/attention.py:6).
inline bool head_dim_supported(int d) {
  switch (d) {
    case 32: case 48: case 64: case 80: case 96: case 112: case 128:
    case 160: case 192: case 224: case 256: case 512:
      return true;
    default:
      return false;
  }
}

// Head sizes with every kernel built (beam groups with their own tables, the group
// plan, the fused KV write): BART's and Florence-2's 64, and 128.
inline bool head_dim_native(int d) { return d == 64 || d == 128; }


// fp32 caches: VALU kernel over the logical V layout, G query rows per group; pool
// blocks of 16 << SHIFT tokens.
template <int D, int G, int NW, int SHIFT = 0>
int launch_valu(const AttnArgs &a) {
  constexpr int DT = VFL_FLOAT32;
  using T = typename Elem<DT>::T;
  constexpr int BS = 16;
  const dim3 grid((unsigned)xcd_grid(a.num_groups, a.H));
  paged_decode_kernel<DT, D, BS, G, NW, stage_blocks<DT, D, G>(), stage_pipeline<G>(), SHIFT>
      <<<grid, dim3(NW * 64), 0, a.stream>>>(
      (const T *)a.q, a.q_st, a.q_sh, (const T *)a.kc, (const T *)a.vc, (T *)a.out, a.seq_lens,
      a.bt, a.bt_stride, a.max_blocks, a.group_start, a.group_order, a.num_rows, a.num_groups,
      a.H, a.num_blocks, a.scale_log2);
  return launch_status("attention_with_kv_cache");
}

template <int D, int G>
int valu_waves(const AttnArgs &a, int nw) {
  switch (nw) {
    case 1: return launch_valu<D, G, 1>(a);
    case 2: return launch_valu<D, G, 2>(a);
    case 4: return launch_valu<D, G, 4>(a);
    default: return launch_valu<D, G, 8>(a);
  }
}

template <int D>
int valu_group(const AttnArgs &a, int gmax, int nw) {
  if (gmax <= 1) return valu_waves<D, 1>(a, nw);
  if (gmax <= 2) return valu_waves<D, 2>(a, nw);
  if (gmax <= 4) return valu_waves<D, 4>(a, nw);
  return valu_waves<D, 8>(a, nw);
}

// bf16 / fp16 caches, one row or a group sharing one table per workgroup, no fused
// KV write: the matrix-core kernel of decode_mfma.h.
template <int DT, int D, int NW, int U, int SHIFT = 0>
int launch_mfma_rows(const AttnArgs &a) {
  const dim3 grid((unsigned)xcd_grid(a.num_groups, a.H));
  paged_decode_mfma_kernel<DT, D, NW, U, false, SHIFT><<<grid, dim3(NW * 64), 0, a.stream>>>(
      (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
      (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
      a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw, a.desc,
      a.desc_stride);
  return launch_status("attention_with_kv_cache");
}

// The reference's head sizes other than 64 and 128 (attention_dims.hip): one row or a
// shared-table group per workgroup, no fused KV write (the caller makes the separate
// write first) and no own-table groups (every row its own group).
int dispatch_other_head_dim(const AttnArgs &a, int dtype, int head_dim, int gmax, int nw);

// Pools of 32-token blocks (attention_block32.hip): every head size on the one-row /
// shared-table kernels, which read a block as two 16-token parts.
int dispatch_block32(const AttnArgs &a, int dtype, int head_dim, int gmax, int nw);

}  // namespace vfl
