// Paged decode attention for gfx950: one query row per sequence over ragged block
// tables of 16-token blocks, used for both the decoder self-attention (rows are
// sequences) and the cross-attention over encoder K/V (rows grouped by request,
// so a request's beams share one read of its pages).
//
// Work decomposition
//   grid = (partition, row group, head group); one wave per head, NW heads per
//   workgroup, so a workgroup reads NW adjacent 2 KiB head slices of each block.
//   A partition covers `part_blocks` consecutive blocks of the group's context.
//   Groups with one partition write the output directly; longer ones write fp32
//   partials (unnormalised accumulator, running max, running sum) that
//   paged_decode_reduce_kernel merges.
//
// Lane layout inside a wave (bf16, head_dim 64): a 16-byte load per lane covers
//   8 token rows x 64 dims (1 KiB, fully coalesced).  Lane = tok * LPT + c holds
//   dims [c*VEC, c*VEC+VEC) of token row `tok`.  Scores are summed over the LPT
//   lanes of a row with DPP; each of the TPL token rows keeps its own online
//   softmax state, merged across rows once at the end (no cross-row traffic in the
//   loop).
#include "common.h"

namespace vfl {

constexpr float NEG_INF = -__builtin_huge_valf();

template <int DT, int D, int BS, int G> struct DecodeState {
  static constexpr int VEC = Elem<DT>::VEC;
  float m[G];
  float l[G];
  float acc[G][VEC];
};

// Fold NT loaded token rows (K chunks kr, V chunks vr) into the running state of
// every live row of the group.  MASKED selects per-lane validity `valid[j]`.
template <int DT, int D, int G, int NT, bool MASKED>
__device__ __forceinline__ void consume(const uint4 (&qv)[G], const uint4 *kr, const uint4 *vr,
                                        const bool *valid, int nrows, float scale_log2,
                                        float (&m)[G], float (&l)[G],
                                        float (&acc)[G][Elem<DT>::VEC]) {
  constexpr int VEC = Elem<DT>::VEC;
  constexpr int LPT = D / VEC;
  float vf[NT][VEC];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    unpack16<DT>(vr[j], vf[j]);
    if constexpr (MASKED) {
      if (!valid[j]) {
#pragma unroll
        for (int d = 0; d < VEC; ++d) vf[j][d] = 0.f;
      }
    }
  }
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    if (gi >= nrows) break;
    float s[NT];
    float mx = m[gi];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      s[j] = group_sum<LPT>(dot16<DT>(qv[gi], kr[j])) * scale_log2;
      if constexpr (MASKED) s[j] = valid[j] ? s[j] : NEG_INF;
      mx = fmaxf(mx, s[j]);
    }
    const float ms = (mx == NEG_INF) ? 0.f : mx;
    const float corr = fast_exp2(m[gi] - ms);
    float lsum = l[gi] * corr;
#pragma unroll
    for (int d = 0; d < VEC; ++d) acc[gi][d] *= corr;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const float p = fast_exp2(s[j] - ms);
      lsum += p;
#pragma unroll
      for (int d = 0; d < VEC; ++d) acc[gi][d] = fmaf(p, vf[j][d], acc[gi][d]);
    }
    l[gi] = lsum;
    m[gi] = mx;
  }
}

template <int DT, int D, int BS, int G, int NW, int U>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t q_st, int64_t q_sh,
    const typename Elem<DT>::T *__restrict__ kc, const typename Elem<DT>::T *__restrict__ vc,
    typename Elem<DT>::T *__restrict__ out, float *__restrict__ ws_acc,
    float2 *__restrict__ ws_ml, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ bt, int64_t bt_stride, int max_blocks,
    const int32_t *__restrict__ group_start, int64_t num_rows, int H, int64_t num_blocks,
    int part_blocks, int max_parts, float scale_log2) {
  using T = typename Elem<DT>::T;
  constexpr int VEC = Elem<DT>::VEC;
  constexpr int LPT = D / VEC;   // lanes per token row
  constexpr int TPL = 64 / LPT;  // token rows per wave-wide load
  constexpr int NLD = BS / TPL;  // loads per block per head
  static_assert(D % VEC == 0 && 64 % LPT == 0 && BS % TPL == 0, "unsupported tile");

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.z * NW + wave;
  if (h >= H) return;
  const int g = blockIdx.y;
  const int p = blockIdx.x;
  int row0 = g, nrows = 1;
  if (group_start) {
    row0 = group_start[g];
    nrows = min(group_start[g + 1] - row0, G);
  }
  // A malformed group table must not send the kernel outside the rows it was given.
  if (row0 < 0 || row0 >= num_rows) return;
  nrows = (int)min((int64_t)nrows, num_rows - row0);
  if (nrows <= 0) return;
  const int L = seq_lens[row0];
  int nblk = L > 0 ? (L + BS - 1) / BS : 0;
  nblk = min(nblk, max_blocks);
  const int Lc = min(L, nblk * BS);
  const int tok = lane / LPT;
  const int c = lane % LPT;

  if (nblk == 0) {
    if (p == 0 && tok == 0) {
      const uint4 z = make_uint4(0, 0, 0, 0);
      for (int gi = 0; gi < nrows; ++gi)
        *reinterpret_cast<uint4 *>(out + ((int64_t)(row0 + gi) * H + h) * D + c * VEC) = z;
    }
    return;
  }
  const int b0 = p * part_blocks;
  if (b0 >= nblk) return;
  const int b1 = min(nblk, b0 + part_blocks);
  const int nparts = (nblk + part_blocks - 1) / part_blocks;

  uint4 qv[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    qv[gi] = make_uint4(0, 0, 0, 0);
    if (gi < nrows) qv[gi] = load16_unaligned<DT>(q + (row0 + gi) * q_st + h * q_sh + c * VEC);
  }
  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    m[gi] = NEG_INF;
    l[gi] = 0.f;
#pragma unroll
    for (int d = 0; d < VEC; ++d) acc[gi][d] = 0.f;
  }

  const int32_t *btrow = bt + (int64_t)row0 * bt_stride;
  const int64_t block_elems = (int64_t)H * BS * D;
  const int lane_off = h * BS * D + tok * D + c * VEC;

  int b = b0;
  // Fast path: U whole blocks per step, every token valid.
  const int bfull = min(b1, Lc / BS);
  for (; b + U <= bfull; b += U) {
    int ids[U];
    bool ok = true;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ids[u] = btrow[b + u];
      ok = ok && ids[u] >= 0 && ids[u] < num_blocks;
    }
    if (!ok) break;  // the masked loop below handles blocks with bad ids
    uint4 kr[U * NLD], vr[U * NLD];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const T *kb = kc + (int64_t)ids[u] * block_elems + lane_off;
      const T *vb = vc + (int64_t)ids[u] * block_elems + lane_off;
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        kr[u * NLD + i] = *reinterpret_cast<const uint4 *>(kb + i * TPL * D);
        vr[u * NLD + i] = *reinterpret_cast<const uint4 *>(vb + i * TPL * D);
      }
    }
    consume<DT, D, G, U * NLD, false>(qv, kr, vr, nullptr, nrows, scale_log2, m, l, acc);
  }
  // Remaining blocks one at a time, with token and block-id masking.
  for (; b < b1; ++b) {
    const int id = btrow[b];
    const bool ok = id >= 0 && id < num_blocks;
    uint4 kr[NLD], vr[NLD];
    bool valid[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      valid[i] = ok && (b * BS + i * TPL + tok) < Lc;
      kr[i] = make_uint4(0, 0, 0, 0);
      vr[i] = make_uint4(0, 0, 0, 0);
    }
    if (ok) {
      const T *kb = kc + (int64_t)id * block_elems + lane_off;
      const T *vb = vc + (int64_t)id * block_elems + lane_off;
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        kr[i] = *reinterpret_cast<const uint4 *>(kb + i * TPL * D);
        vr[i] = *reinterpret_cast<const uint4 *>(vb + i * TPL * D);
      }
    }
    consume<DT, D, G, NLD, true>(qv, kr, vr, valid, nrows, scale_log2, m, l, acc);
  }

  // Merge the TPL token-row states of each column c (lanes c, c+LPT, ...).
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    if (gi >= nrows) break;
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
      const float mo = __shfl_xor(m[gi], off, 64);
      const float lo = __shfl_xor(l[gi], off, 64);
      const float mx = fmaxf(m[gi], mo);
      const float ms = (mx == NEG_INF) ? 0.f : mx;
      const float wa = fast_exp2(m[gi] - ms);
      const float wb = fast_exp2(mo - ms);
      l[gi] = l[gi] * wa + lo * wb;
#pragma unroll
      for (int d = 0; d < VEC; ++d) {
        const float ao = __shfl_xor(acc[gi][d], off, 64);
        acc[gi][d] = acc[gi][d] * wa + ao * wb;
      }
      m[gi] = mx;
    }
  }

  if (tok != 0) return;
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    if (gi >= nrows) break;
    const int64_t rh = (int64_t)(row0 + gi) * H + h;
    if (nparts == 1) {
      const float inv = l[gi] > 0.f ? 1.f / l[gi] : 0.f;
      float o[VEC];
#pragma unroll
      for (int d = 0; d < VEC; ++d) o[d] = acc[gi][d] * inv;
      *reinterpret_cast<uint4 *>(out + rh * D + c * VEC) = pack16<DT>(o);
    } else {
      float *dst = ws_acc + (rh * max_parts + p) * D + c * VEC;
#pragma unroll
      for (int d = 0; d < VEC; d += 4)
        *reinterpret_cast<float4 *>(dst + d) =
            make_float4(acc[gi][d], acc[gi][d + 1], acc[gi][d + 2], acc[gi][d + 3]);
      if (c == 0) ws_ml[rh * max_parts + p] = make_float2(m[gi], l[gi]);
    }
  }
}

// Merge the partitions of every group that needed more than one.
template <int DT, int D, int BS, int G, int NW>
__global__ __launch_bounds__(NW * 64) void paged_decode_reduce_kernel(
    typename Elem<DT>::T *__restrict__ out, const float *__restrict__ ws_acc,
    const float2 *__restrict__ ws_ml, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ group_start, int64_t num_rows, int H, int max_blocks,
    int part_blocks, int max_parts) {
  using T = typename Elem<DT>::T;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * NW + wave;
  if (h >= H) return;
  const int g = blockIdx.x;
  int row0 = g, nrows = 1;
  if (group_start) {
    row0 = group_start[g];
    nrows = min(group_start[g + 1] - row0, G);
  }
  if (row0 < 0 || row0 >= num_rows) return;
  nrows = (int)min((int64_t)nrows, num_rows - row0);
  const int L = seq_lens[row0];
  int nblk = L > 0 ? (L + BS - 1) / BS : 0;
  nblk = min(nblk, max_blocks);
  const int nparts = (nblk + part_blocks - 1) / part_blocks;
  if (nparts <= 1) return;
  for (int gi = 0; gi < nrows; ++gi) {
    const int64_t rh = (int64_t)(row0 + gi) * H + h;
    const float2 *ml = ws_ml + rh * max_parts;
    float M = NEG_INF;
    for (int pp = 0; pp < nparts; ++pp) M = fmaxf(M, ml[pp].x);
    const float Ms = (M == NEG_INF) ? 0.f : M;
    float Ls = 0.f;
    float o[(D + 63) / 64];
#pragma unroll
    for (int k = 0; k < (D + 63) / 64; ++k) o[k] = 0.f;
    for (int pp = 0; pp < nparts; ++pp) {
      const float2 mlp = ml[pp];
      const float w = fast_exp2(mlp.x - Ms);
      Ls = fmaf(mlp.y, w, Ls);
      const float *a = ws_acc + (rh * max_parts + pp) * D;
#pragma unroll
      for (int k = 0; k < (D + 63) / 64; ++k) {
        const int d = lane + 64 * k;
        if (d < D) o[k] = fmaf(a[d], w, o[k]);
      }
    }
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
#pragma unroll
    for (int k = 0; k < (D + 63) / 64; ++k) {
      const int d = lane + 64 * k;
      if (d >= D) continue;
      const float v = o[k] * inv;
      if constexpr (DT == VFL_FLOAT32)
        out[rh * D + d] = v;
      else if constexpr (DT == VFL_BFLOAT16)
        out[rh * D + d] = (T)f32_to_bf16(v);
      else
        out[rh * D + d] = (T)f32_to_f16(v);
    }
  }
}

constexpr int NW_HEADS = 4;  // heads (waves) per workgroup
constexpr int UNROLL = 2;    // whole blocks per fast-path step

struct AttnArgs {
  const void *q;
  int64_t q_st, q_sh;
  const void *kc, *vc;
  void *out;
  float *ws_acc;
  float2 *ws_ml;
  const int32_t *seq_lens, *bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t *group_start;
  int64_t num_rows, num_groups;
  int H;
  int64_t num_blocks;
  int part_blocks, max_parts;
  float scale_log2;
  hipStream_t stream;
};

template <int DT, int D, int G>
static int launch_attention(const AttnArgs &a) {
  using T = typename Elem<DT>::T;
  constexpr int BS = 16;
  const dim3 block(NW_HEADS * 64);
  const unsigned hz = (unsigned)((a.H + NW_HEADS - 1) / NW_HEADS);
  const dim3 grid((unsigned)a.max_parts, (unsigned)a.num_groups, hz);
  paged_decode_kernel<DT, D, BS, G, NW_HEADS, UNROLL><<<grid, block, 0, a.stream>>>(
      (const T *)a.q, a.q_st, a.q_sh, (const T *)a.kc, (const T *)a.vc, (T *)a.out, a.ws_acc,
      a.ws_ml, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start, a.num_rows, a.H,
      a.num_blocks, a.part_blocks, a.max_parts, a.scale_log2);
  int st = launch_status("attention_with_kv_cache");
  if (st != VFL_OK || a.max_parts <= 1) return st;
  const dim3 rgrid((unsigned)a.num_groups, hz);
  paged_decode_reduce_kernel<DT, D, BS, G, NW_HEADS><<<rgrid, block, 0, a.stream>>>(
      (T *)a.out, a.ws_acc, a.ws_ml, a.seq_lens, a.group_start, a.num_rows, a.H, a.max_blocks,
      a.part_blocks, a.max_parts);
  return launch_status("attention_with_kv_cache (reduce)");
}

template <int DT, int D>
static int dispatch_group(const AttnArgs &a, int gmax) {
  if (gmax <= 1) return launch_attention<DT, D, 1>(a);
  if (gmax <= 2) return launch_attention<DT, D, 2>(a);
  if (gmax <= 4) return launch_attention<DT, D, 4>(a);
  return launch_attention<DT, D, 8>(a);
}

template <int DT>
static int dispatch_dim(const AttnArgs &a, int head_dim, int gmax) {
  switch (head_dim) {
    case 64: return dispatch_group<DT, 64>(a, gmax);
    case 128: return dispatch_group<DT, 128>(a, gmax);
    default: break;
  }
  set_error("attention_with_kv_cache: head_dim %d has no kernel (built: 64, 128)", head_dim);
  return VFL_E_UNSUPPORTED;
}

static bool kernel_exists(int dtype, int block_size, int head_dim) {
  return (dtype == VFL_FLOAT32 || dtype == VFL_BFLOAT16 || dtype == VFL_FLOAT16) &&
         block_size == 16 && (head_dim == 64 || head_dim == 128);
}

static size_t workspace_for(int64_t rows, int H, int D, int max_parts) {
  if (max_parts <= 1) return 0;
  const size_t parts = (size_t)rows * H * max_parts;
  size_t acc_bytes = parts * D * sizeof(float);
  acc_bytes = (acc_bytes + 255) & ~(size_t)255;
  return acc_bytes + parts * sizeof(float2);
}

constexpr int MAX_GROUP = 8;

}  // namespace vfl

using namespace vfl;

extern "C" const char *vfl_get_isa(int dtype, int block_size, int head_dim) {
  return kernel_exists(dtype, block_size, head_dim) ? "gfx950" : nullptr;
}

extern "C" int vfl_get_scheduler_metadata(int64_t num_rows, int64_t num_groups, int num_heads,
                                          int head_dim, int block_size,
                                          int64_t max_blocks_per_seq, int max_group_size,
                                          int dtype, int partition_blocks, vfl_sched_meta *meta) {
  clear_error();
  if (!meta) {
    set_error("get_scheduler_metadata: meta is NULL");
    return VFL_E_INVALID;
  }
  if (num_rows < 0 || num_groups < 0 || num_groups > num_rows || num_heads <= 0 ||
      max_blocks_per_seq < 0 || max_blocks_per_seq > (1 << 30) || partition_blocks < 0) {
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
  int pb = partition_blocks;
  if (pb == 0) pb = 16;
  const int64_t mb = max_blocks_per_seq > 0 ? max_blocks_per_seq : 1;
  const int64_t parts = (mb + pb - 1) / pb;
  if (parts > 65535 || num_groups > 65535) {
    set_error("get_scheduler_metadata: grid too large (%lld partitions, %lld groups)",
              (long long)parts, (long long)num_groups);
    return VFL_E_UNSUPPORTED;
  }
  meta->num_rows = num_rows;
  meta->num_heads = num_heads;
  meta->head_dim = head_dim;
  meta->max_blocks_per_seq = (int32_t)max_blocks_per_seq;
  meta->partition_blocks = pb;
  meta->max_partitions = (int32_t)parts;
  meta->max_group_size = max_group_size;
  meta->heads_per_workgroup = NW_HEADS;
  meta->workspace_bytes = workspace_for(num_rows, num_heads, head_dim, (int)parts);
  return VFL_OK;
}

extern "C" int vfl_attention_with_kv_cache(
    const void *query, int64_t query_stride_token, int64_t query_stride_head,
    const void *k_cache, const void *v_cache, void *out, const int32_t *seq_lens,
    const int32_t *block_table, int64_t block_table_stride, const int32_t *group_start,
    int64_t num_rows, int64_t num_groups, int num_heads, int head_dim, int block_size,
    int64_t num_blocks, float scale, int dtype, const vfl_sched_meta *meta, void *workspace,
    size_t workspace_bytes, void *stream) {
  clear_error();
  if (!meta) {
    set_error("attention_with_kv_cache: meta is NULL");
    return VFL_E_INVALID;
  }
  if (!kernel_exists(dtype, block_size, head_dim)) {
    set_error("attention_with_kv_cache: no kernel for dtype %d block_size %d head_dim %d", dtype,
              block_size, head_dim);
    return VFL_E_UNSUPPORTED;
  }
  if (num_rows < 0 || num_heads <= 0 || num_blocks < 0) {
    set_error("attention_with_kv_cache: bad sizes");
    return VFL_E_INVALID;
  }
  if (meta->num_rows != num_rows || meta->num_heads != num_heads ||
      meta->head_dim != head_dim) {
    set_error("attention_with_kv_cache: metadata was made for rows %lld heads %d head_dim %d, "
              "call has rows %lld heads %d head_dim %d",
              (long long)meta->num_rows, meta->num_heads, meta->head_dim, (long long)num_rows,
              num_heads, head_dim);
    return VFL_E_INVALID;
  }
  if (group_start == nullptr && num_groups != num_rows) {
    set_error("attention_with_kv_cache: without group_start, num_groups (%lld) must equal "
              "num_rows (%lld)",
              (long long)num_groups, (long long)num_rows);
    return VFL_E_INVALID;
  }
  if (num_groups < 0 || num_groups > num_rows || num_groups > 65535) {
    set_error("attention_with_kv_cache: num_groups %lld out of range", (long long)num_groups);
    return VFL_E_INVALID;
  }
  if (meta->partition_blocks <= 0 || meta->max_partitions < 1 ||
      (int64_t)meta->max_partitions * meta->partition_blocks < meta->max_blocks_per_seq ||
      meta->max_group_size < 1 || meta->max_group_size > MAX_GROUP) {
    set_error("attention_with_kv_cache: inconsistent metadata");
    return VFL_E_INVALID;
  }
  if (block_table_stride < meta->max_blocks_per_seq) {
    set_error("attention_with_kv_cache: block_table_stride %lld < max_blocks_per_seq %d",
              (long long)block_table_stride, meta->max_blocks_per_seq);
    return VFL_E_INVALID;
  }
  if (num_rows == 0) return VFL_OK;
  if (!query || !k_cache || !v_cache || !out || !seq_lens || !block_table) {
    set_error("attention_with_kv_cache: null pointer argument");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) % 16 != 0) {
    set_error("attention_with_kv_cache: caches and out must be 16-byte aligned");
    return VFL_E_INVALID;
  }
  const size_t need = workspace_for(num_rows, num_heads, head_dim, meta->max_partitions);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need ||
                   ((uintptr_t)workspace % 256) != 0)) {
    set_error("attention_with_kv_cache: workspace of %zu bytes (256-byte aligned) required, "
              "got %zu",
              need, workspace ? workspace_bytes : (size_t)0);
    return VFL_E_WORKSPACE;
  }
  AttnArgs a;
  a.q = query;
  a.q_st = query_stride_token;
  a.q_sh = query_stride_head;
  a.kc = k_cache;
  a.vc = v_cache;
  a.out = out;
  a.ws_acc = (float *)workspace;
  a.ws_ml = nullptr;
  if (need > 0) {
    size_t acc_bytes = (size_t)num_rows * num_heads * meta->max_partitions * head_dim * 4;
    acc_bytes = (acc_bytes + 255) & ~(size_t)255;
    a.ws_ml = (float2 *)((uint8_t *)workspace + acc_bytes);
  }
  a.seq_lens = seq_lens;
  a.bt = block_table;
  a.bt_stride = block_table_stride;
  a.max_blocks = meta->max_blocks_per_seq;
  a.group_start = group_start;
  a.num_rows = num_rows;
  a.num_groups = num_groups;
  a.H = num_heads;
  a.num_blocks = num_blocks;
  a.part_blocks = meta->partition_blocks;
  a.max_parts = meta->max_partitions;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.stream = (hipStream_t)stream;
  const int gmax = meta->max_group_size;
  switch (dtype) {
    case VFL_FLOAT32: return dispatch_dim<VFL_FLOAT32>(a, head_dim, gmax);
    case VFL_BFLOAT16: return dispatch_dim<VFL_BFLOAT16>(a, head_dim, gmax);
    default: return dispatch_dim<VFL_FLOAT16>(a, head_dim, gmax);
  }
}
