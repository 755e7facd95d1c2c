// Paged decode attention for gfx950: one query row per sequence over ragged block
// tables of 16-token blocks, used for both the decoder self-attention (rows are
// sequences) and the cross-attention over encoder K/V (rows grouped by request,
// so a request's beams share one read of its pages).
//
// Work decomposition
//   grid = (head, row group); the workgroup's NW waves split the group's context
//   into NW contiguous runs of blocks and merge their softmax states through LDS at
//   the end, so each (group, head) is one workgroup and one launch does the whole
//   op (no partial buffers, no second kernel).  An optional host-computed order
//   dispatches the longest groups first.
//
// Lane layout inside a wave (bf16, head_dim 64): a 16-byte load per lane covers
//   8 token rows x 64 dims (1 KiB, fully coalesced); a block's 2 KiB head slice is
//   two loads.  Lane = tok * LPT + c holds dims [c*VEC, c*VEC+VEC) of token row
//   `tok`.  Scores are summed over the LPT lanes of a row with DPP; each of the TPL
//   token rows keeps its own online-softmax state, merged across rows once at the
//   end (no cross-row traffic in the loop).
#include "common.h"
#include "decode_planned.h"

namespace vfl {

// Fold NT loaded token rows (K chunks kr, V chunks vr) into the running state of
// every live row of the group.  MASKED applies per-lane validity `valid[j]` (token
// past the context, or a block id outside the pool).
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
    float mb = NEG_INF_F;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      s[j] = group_sum<LPT>(dot16<DT>(qv[gi], kr[j])) * scale_log2;
      if constexpr (MASKED) s[j] = valid[j] ? s[j] : NEG_INF_F;
      mb = fmaxf(mb, s[j]);
    }
    // Wave-uniform branch: rescale only if some lane's block max ran away.
    if (__builtin_amdgcn_ballot_w64(mb > m[gi] + RESCALE_SLACK_LOG2) != 0) {
      const float mn = fmaxf(m[gi], mb);
      const float corr = (mn == NEG_INF_F) ? 1.f : fast_exp2(m[gi] - mn);
      l[gi] *= corr;
#pragma unroll
      for (int d = 0; d < VEC; ++d) acc[gi][d] *= corr;
      m[gi] = mn;
    }
    const float ms = (m[gi] == NEG_INF_F) ? 0.f : m[gi];
    float lsum = l[gi];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const float p = fast_exp2(s[j] - ms);
      lsum += p;
#pragma unroll
      for (int d = 0; d < VEC; ++d) acc[gi][d] = fmaf(p, vf[j][d], acc[gi][d]);
    }
    l[gi] = lsum;
  }
}

// Issue the loads of U consecutive blocks (one stage) into registers.  Block ids
// outside the pool load nothing and are marked invalid.
template <int DT, int D, int BS, int U>
__device__ __forceinline__ void load_stage(const typename Elem<DT>::T *__restrict__ kc,
                                           const typename Elem<DT>::T *__restrict__ vc,
                                           WaveBlockIds &ids, int b, int64_t block_elems,
                                           int lane_off, int64_t num_blocks, uint4 *kr,
                                           uint4 *vr, bool *ok) {
  constexpr int VEC = Elem<DT>::VEC;
  constexpr int TPL = 64 / (D / VEC);
  constexpr int NLD = BS / TPL;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int id = ids.get(b + u);
    ok[u] = id >= 0 && id < num_blocks;
    const int64_t base = (ok[u] ? (int64_t)id : 0) * block_elems + lane_off;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      kr[u * NLD + i] = make_uint4(0, 0, 0, 0);
      vr[u * NLD + i] = make_uint4(0, 0, 0, 0);
      if (ok[u]) {
        kr[u * NLD + i] = *reinterpret_cast<const uint4 *>(kc + base + i * TPL * D);
        vr[u * NLD + i] = *reinterpret_cast<const uint4 *>(vc + base + i * TPL * D);
      }
    }
  }
}

// Consume one stage of U whole blocks; a stage holding an invalid block id takes the
// masked path for its tokens.
template <int DT, int D, int BS, int G, int U>
__device__ __forceinline__ void consume_stage(const uint4 (&qv)[G], const uint4 *kr,
                                              const uint4 *vr, const bool *ok, int nrows,
                                              float scale_log2, float (&m)[G], float (&l)[G],
                                              float (&acc)[G][Elem<DT>::VEC]) {
  constexpr int VEC = Elem<DT>::VEC;
  constexpr int TPL = 64 / (D / VEC);
  constexpr int NLD = BS / TPL;
  bool all_ok = true;
#pragma unroll
  for (int u = 0; u < U; ++u) all_ok = all_ok && ok[u];
  if (all_ok) {
    consume<DT, D, G, U * NLD, false>(qv, kr, vr, nullptr, nrows, scale_log2, m, l, acc);
  } else {
    bool valid[U * NLD];
#pragma unroll
    for (int j = 0; j < U * NLD; ++j) valid[j] = ok[j / NLD];
    consume<DT, D, G, U * NLD, true>(qv, kr, vr, valid, nrows, scale_log2, m, l, acc);
  }
}

template <int DT> __device__ __forceinline__ typename Elem<DT>::T to_elem(float v) {
  if constexpr (DT == VFL_FLOAT32)
    return v;
  else if constexpr (DT == VFL_BFLOAT16)
    return (typename Elem<DT>::T)f32_to_bf16(v);
  else
    return (typename Elem<DT>::T)f32_to_f16(v);
}

template <int DT, int D, int BS, int G, int NW, int U, bool PIPE>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t q_st, int64_t q_sh,
    const typename Elem<DT>::T *__restrict__ kc, const typename Elem<DT>::T *__restrict__ vc,
    typename Elem<DT>::T *__restrict__ out, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ bt, int64_t bt_stride, int max_blocks,
    const int32_t *__restrict__ group_start, const int32_t *__restrict__ group_order,
    int64_t num_rows, int64_t num_groups, int H, int64_t num_blocks, float scale_log2) {
  using T = typename Elem<DT>::T;
  constexpr int VEC = Elem<DT>::VEC;
  constexpr int LPT = D / VEC;   // lanes per token row
  constexpr int TPL = 64 / LPT;  // token rows per wave-wide load
  constexpr int NLD = BS / TPL;  // loads per block per head
  static_assert(D % VEC == 0 && 64 % LPT == 0 && BS % TPL == 0, "unsupported tile");

  // Per-wave softmax states for the cross-wave merge.
  __shared__ float s_acc[NW > 1 ? NW : 1][G][D];
  __shared__ float s_ml[NW > 1 ? NW : 1][G][2];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // 1-D grid, head fastest: a group's heads are dispatched together.
  const int h = (int)(blockIdx.x % (unsigned)H);
  int g = (int)(blockIdx.x / (unsigned)H);
  if (group_order) g = group_order[g];
  // Workgroup-uniform exits only (before any barrier).
  if (g < 0 || g >= num_groups || h >= H) return;
  int row0 = g, nrows = 1;
  if (group_start) {
    row0 = group_start[g];
    nrows = min(group_start[g + 1] - row0, G);
  }
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
    for (int i = threadIdx.x; i < nrows * D; i += NW * 64) {
      const int gi = i / D, d = i % D;
      out[((int64_t)(row0 + gi) * H + h) * D + d] = to_elem<DT>(0.f);
    }
    return;
  }

  // This wave's run of blocks.
  const int chunk = (nblk + NW - 1) / NW;
  const int b0 = min(nblk, wave * chunk);
  const int b1 = min(nblk, b0 + chunk);

  uint4 qv[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    qv[gi] = make_uint4(0, 0, 0, 0);
    if (gi < nrows) qv[gi] = load16_unaligned<DT>(q + (row0 + gi) * q_st + h * q_sh + c * VEC);
  }
  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    m[gi] = NEG_INF_F;
    l[gi] = 0.f;
#pragma unroll
    for (int d = 0; d < VEC; ++d) acc[gi][d] = 0.f;
  }

  WaveBlockIds ids;
  ids.init(bt + (int64_t)row0 * bt_stride, b0, b1);
  const int64_t block_elems = (int64_t)H * BS * D;
  const int lane_off = h * BS * D + tok * D + c * VEC;

  // Whole blocks of this wave's run are consumed U at a time.  With PIPE the loads
  // of stage s+1 are issued before stage s is consumed (two register stages live),
  // so each wave keeps K/V in flight while it computes; without it, latency is hidden
  // by the other waves the smaller register footprint lets the CU hold.
  const int bfull = max(b0, min(b1, Lc / BS));
  const int stages = (bfull - b0) / U;
  int b = b0;
  if constexpr (PIPE) {
    if (stages > 0) {
      uint4 ka[U * NLD], va[U * NLD], kb[U * NLD], vb[U * NLD];
      bool oka[U], okb[U];
      load_stage<DT, D, BS, U>(kc, vc, ids, b, block_elems, lane_off, num_blocks, ka, va,
                               oka);
      for (int st = 0; st < stages; st += 2) {
        if (st + 1 < stages)
          load_stage<DT, D, BS, U>(kc, vc, ids, b + U, block_elems, lane_off, num_blocks, kb,
                                   vb, okb);
        consume_stage<DT, D, BS, G, U>(qv, ka, va, oka, nrows, scale_log2, m, l, acc);
        b += U;
        if (st + 1 >= stages) break;
        if (st + 2 < stages)
          load_stage<DT, D, BS, U>(kc, vc, ids, b + U, block_elems, lane_off, num_blocks, ka,
                                   va, oka);
        consume_stage<DT, D, BS, G, U>(qv, kb, vb, okb, nrows, scale_log2, m, l, acc);
        b += U;
      }
    }
  } else {
    for (int st = 0; st < stages; ++st, b += U) {
      uint4 kr[U * NLD], vr[U * NLD];
      bool ok[U];
      load_stage<DT, D, BS, U>(kc, vc, ids, b, block_elems, lane_off, num_blocks, kr, vr, ok);
      consume_stage<DT, D, BS, G, U>(qv, kr, vr, ok, nrows, scale_log2, m, l, acc);
    }
  }
  // Remaining blocks one at a time, with token and block-id masking.
  for (; b < b1; ++b) {
    uint4 kr[NLD], vr[NLD];
    bool ok[1];
    load_stage<DT, D, BS, 1>(kc, vc, ids, b, block_elems, lane_off, num_blocks, kr, vr, ok);
    bool valid[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) valid[i] = ok[0] && (b * BS + i * TPL + tok) < Lc;
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
      const float ms = (mx == NEG_INF_F) ? 0.f : mx;
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

  if constexpr (NW == 1) {
    if (tok != 0) return;
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      if (gi >= nrows) break;
      const float inv = l[gi] > 0.f ? 1.f / l[gi] : 0.f;
      float o[VEC];
#pragma unroll
      for (int d = 0; d < VEC; ++d) o[d] = acc[gi][d] * inv;
      *reinterpret_cast<uint4 *>(out + ((int64_t)(row0 + gi) * H + h) * D + c * VEC) =
          pack16<DT>(o);
    }
  } else {
    // Cross-wave merge through LDS.
    if (tok == 0) {
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        if (gi >= nrows) break;
#pragma unroll
        for (int d = 0; d < VEC; ++d) s_acc[wave][gi][c * VEC + d] = acc[gi][d];
        if (c == 0) {
          s_ml[wave][gi][0] = m[gi];
          s_ml[wave][gi][1] = l[gi];
        }
      }
    }
    lds_barrier();
    for (int i = threadIdx.x; i < nrows * D; i += NW * 64) {
      const int gi = i / D, d = i % D;
      float M = NEG_INF_F;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_ml[w][gi][0]);
      const float Ms = (M == NEG_INF_F) ? 0.f : M;
      float S = 0.f, o = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = fast_exp2(s_ml[w][gi][0] - Ms);
        S = fmaf(s_ml[w][gi][1], f, S);
        o = fmaf(s_acc[w][gi][d], f, o);
      }
      out[((int64_t)(row0 + gi) * H + h) * D + d] = to_elem<DT>(S > 0.f ? o / S : 0.f);
    }
  }
}

// Blocks per stage: about four 16-byte K loads (plus four V loads) per lane -- fewer
// when fp32 or head_dim 128 need more loads per block.
template <int DT, int D, int G> constexpr int stage_blocks() {
  constexpr int nld = 16 / (64 / (D / Elem<DT>::VEC));
  return nld >= 4 ? 1 : 4 / nld;
}
// Register pipelining (two live stages) measured slower than the occupancy the
// smaller footprint buys, for every beam count; kept as a kernel option.
template <int G> constexpr bool stage_pipeline() { return false; }

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
  bool q_vec;  // query rows 16-byte aligned
};

// fp32 caches: VALU kernel over the logical V layout, G query rows per group.
template <int D, int G, int NW>
static int launch_valu(const AttnArgs &a) {
  constexpr int DT = VFL_FLOAT32;
  using T = typename Elem<DT>::T;
  constexpr int BS = 16;
  const dim3 grid((unsigned)(a.num_groups * a.H));
  paged_decode_kernel<DT, D, BS, G, NW, stage_blocks<DT, D, G>(), stage_pipeline<G>()>
      <<<grid, dim3(NW * 64), 0, a.stream>>>(
      (const T *)a.q, a.q_st, a.q_sh, (const T *)a.kc, (const T *)a.vc, (T *)a.out, a.seq_lens,
      a.bt, a.bt_stride, a.max_blocks, a.group_start, a.group_order, a.num_rows, a.num_groups,
      a.H, a.num_blocks, a.scale_log2);
  return launch_status("attention_with_kv_cache");
}

template <int D, int G>
static int valu_waves(const AttnArgs &a, int nw) {
  switch (nw) {
    case 1: return launch_valu<D, G, 1>(a);
    case 2: return launch_valu<D, G, 2>(a);
    case 4: return launch_valu<D, G, 4>(a);
    default: return launch_valu<D, G, 8>(a);
  }
}

template <int D>
static int valu_group(const AttnArgs &a, int gmax, int nw) {
  if (gmax <= 1) return valu_waves<D, 1>(a, nw);
  if (gmax <= 2) return valu_waves<D, 2>(a, nw);
  if (gmax <= 4) return valu_waves<D, 4>(a, nw);
  return valu_waves<D, 8>(a, nw);
}

// bf16 / fp16 caches: matrix-core kernel over the token-interleaved V layout; the tile
// columns hold up to 16 query rows per group, so one instantiation serves any G.
constexpr int MFMA_STAGE_BLOCKS = 2;
// Stage size of the own-tables group kernel (measured on MI355X, 64 x 4-beam decode
// steps: 3 and 4 blocks per stage were no faster and cost occupancy).
constexpr int SHARED_STAGE_BLOCKS = 2;

// Stage size of the planned group kernel: every wave requests this many blocks per
// round trip.
constexpr int PLANNED_STAGE_BLOCKS = 4;

template <int DT, int D, int NW>
static int launch_planned(const AttnArgs &a) {
  const dim3 grid((unsigned)(a.plan_slots * a.H));
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
  const dim3 grid((unsigned)(a.num_groups * a.H));
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
    paged_decode_mfma_kernel<DT, D, NW, MFMA_STAGE_BLOCKS, true>
        <<<grid, dim3(NW * 64), 0, a.stream>>>(
        (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
        (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
        a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw);
  else
    paged_decode_mfma_kernel<DT, D, NW, MFMA_STAGE_BLOCKS, false>
        <<<grid, dim3(NW * 64), 0, a.stream>>>(
        (const uint16_t *)a.q, a.q_st, a.q_sh, (const uint16_t *)a.kc, (const uint16_t *)a.vc,
        (uint16_t *)a.out, a.seq_lens, a.bt, a.bt_stride, a.max_blocks, a.group_start,
        a.group_order, a.num_rows, a.num_groups, a.H, a.num_blocks, a.scale_log2, a.kvw);
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
  set_error("attention_with_kv_cache: head_dim %d has no kernel (built: 64, 128)", head_dim);
  return VFL_E_UNSUPPORTED;
}

static bool kernel_exists(int dtype, int block_size, int head_dim) {
  return (dtype == VFL_FLOAT32 || dtype == VFL_BFLOAT16 || dtype == VFL_FLOAT16) &&
         block_size == 16 && (head_dim == 64 || head_dim == 128);
}

constexpr int MAX_GROUP = 8;
constexpr int MAX_WAVES = 8;

// Waves per (group, head) workgroup.  Measured on MI355X (bf16, head_dim 64, K/V pages
// loaded non-temporally): 64 x 4-beam cross-attention (1024 workgroups) runs 30.3 us
// with eight waves, 32.8-33.6 with four, 36.1 with two; 256 ragged self-attention rows
// (4096 workgroups) run within noise of each other with two, four or eight (92.6-97.1
// us).  So eight below 2048 workgroups, four above.  Never more waves than blocks.
static int default_waves(int64_t num_groups, int num_heads, int64_t max_blocks) {
  const int64_t wgs = num_groups * num_heads;
  int nw = wgs >= 2048 ? 4 : 8;
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
  if (num_groups * num_heads > 2147483647LL) {
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
  if (num_groups < 0 || num_groups > num_rows || num_groups * num_heads > 2147483647LL ||
      num_heads > 65535) {
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
  if (meta->group_plan != nullptr && a.own_tables && dtype != VFL_FLOAT32) {
    if ((uintptr_t)meta->group_plan % 16 != 0 || meta->group_plan_stride < PLAN_HEADER ||
        meta->group_plan_stride % 4 != 0 || meta->group_plan_slots < num_groups ||
        meta->group_plan_slots * num_heads > 2147483647LL ||
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
  if (a.own_tables && dtype == VFL_FLOAT32) {
    // The VALU kernel reads one table per group; with rows keeping their own tables
    // every row is its own group instead (same results: grouping is only a sharing
    // of loads), in natural order.
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
  if (dtype == VFL_FLOAT32) {
    // The fp32 path has no fused kernel: the same two steps as the reference.
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
