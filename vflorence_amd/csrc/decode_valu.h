// Paged decode attention on the vector ALUs (fp32 caches; any head size that is a
// multiple of four), gfx950.  One query row per sequence over ragged block tables of
// 16-token blocks, for both the decoder self-attention (rows are sequences) and the
// cross-attention over encoder K/V (rows grouped by request, so a request's beams share
// one read of its pages).
//
// Work decomposition
//   grid = (head, row group); the workgroup's NW waves split the group's context
//   into NW contiguous runs of blocks and merge their softmax states through LDS at
//   the end, so each (group, head) is one workgroup and one launch does the whole
//   op (no partial buffers, no second kernel).  An optional host-computed order
//   dispatches the longest groups first.
//
// Lane layout inside a wave: a token row of the head is D / VEC 16-byte chunks.  LPT
//   lanes take one token row (the chunk count rounded up to a power of two, at most
//   64); lane = tok * LPT + c holds chunks c, c + LPT, ... (CPL of them, two only for
//   rows wider than 64 chunks), and lanes whose chunk lies past the row hold zeros.
//   A wave-wide load covers TPL = 64 / LPT token rows; for fp32 and head_dim 64 that is
//   4 rows x 256 bytes, fully coalesced.  Scores are summed over the LPT lanes of a row
//   with DPP; each of the TPL token rows keeps its own online-softmax state, merged
//   across rows once at the end (no cross-row traffic in the loop).
#pragma once

#include "common.h"

namespace vfl {

constexpr int pow2_ceil(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// The lane layout of head size D for element type DT (see the header comment).
template <int DT, int D> struct ValuLayout {
  static constexpr int VEC = Elem<DT>::VEC;
  static constexpr int NCHUNK = D / VEC;  // 16-byte chunks per token row
  static constexpr int LPT = pow2_ceil(NCHUNK) < 64 ? pow2_ceil(NCHUNK) : 64;
  static constexpr int CPL = (NCHUNK + LPT - 1) / LPT;  // chunks per lane
  static constexpr int TPL = 64 / LPT;                   // token rows per wave-wide load
  static_assert(D % VEC == 0, "head size must be a multiple of the 16-byte chunk");
  // The chunk (0 .. NCHUNK - 1) that lane column c holds in slot j, or -1.
  static __device__ __forceinline__ int chunk(int c, int j) {
    const int x = c + LPT * j;
    return x < NCHUNK ? x : -1;
  }
};

// Fold NT loaded token rows (K chunks kr, V chunks vr: CPL per row) into the running
// state of every live row of the group.  MASKED applies per-lane validity `valid[j]`
// (token past the context, or a block id outside the pool).
template <int DT, int D, int G, int NT, bool MASKED>
__device__ __forceinline__ void consume(const uint4 (&qv)[G][ValuLayout<DT, D>::CPL],
                                        const uint4 *kr, const uint4 *vr, const bool *valid,
                                        int nrows, float scale_log2, float (&m)[G],
                                        float (&l)[G],
                                        float (&acc)[G][ValuLayout<DT, D>::CPL * Elem<DT>::VEC]) {
  using Lay = ValuLayout<DT, D>;
  constexpr int VEC = Lay::VEC, CPL = Lay::CPL;
  float vf[NT][CPL * VEC];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
#pragma unroll
    for (int s = 0; s < CPL; ++s) unpack16<DT>(vr[j * CPL + s], &vf[j][s * VEC]);
    if constexpr (MASKED) {
      if (!valid[j]) {
#pragma unroll
        for (int d = 0; d < CPL * VEC; ++d) vf[j][d] = 0.f;
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
      float dot = dot16<DT>(qv[gi][0], kr[j * CPL]);
#pragma unroll
      for (int c = 1; c < CPL; ++c) dot += dot16<DT>(qv[gi][c], kr[j * CPL + c]);
      s[j] = group_sum<Lay::LPT>(dot) * scale_log2;
      if constexpr (MASKED) s[j] = valid[j] ? s[j] : NEG_INF_F;
      mb = fmaxf(mb, s[j]);
    }
    // Wave-uniform branch: rescale only if some lane's block max ran away.
    if (__builtin_amdgcn_ballot_w64(mb > m[gi] + RESCALE_SLACK_LOG2) != 0) {
      const float mn = fmaxf(m[gi], mb);
      const float corr = (mn == NEG_INF_F) ? 1.f : fast_exp2(m[gi] - mn);
      l[gi] *= corr;
#pragma unroll
      for (int d = 0; d < CPL * VEC; ++d) acc[gi][d] *= corr;
      m[gi] = mn;
    }
    const float ms = (m[gi] == NEG_INF_F) ? 0.f : m[gi];
    float lsum = l[gi];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const float p = fast_exp2(s[j] - ms);
      lsum += p;
#pragma unroll
      for (int d = 0; d < CPL * VEC; ++d) acc[gi][d] = fmaf(p, vf[j][d], acc[gi][d]);
    }
    l[gi] = lsum;
  }
}

// Issue the loads of U consecutive blocks (one stage) into registers.  Block ids
// outside the pool load nothing and are marked invalid; chunks past the row stay zero.
// b counts BS-token chunks; a pool block holds 1 << SHIFT of them (32-token blocks:
// two), chunk b being part b & mask of table entry b >> SHIFT.
template <int DT, int D, int BS, int U, int SHIFT>
__device__ __forceinline__ void load_stage(const typename Elem<DT>::T *__restrict__ kc,
                                           const typename Elem<DT>::T *__restrict__ vc,
                                           WaveBlockIds &ids, int b, int64_t block_elems,
                                           int lane_off, int c, int64_t num_blocks, uint4 *kr,
                                           uint4 *vr, bool *ok) {
  using Lay = ValuLayout<DT, D>;
  constexpr int VEC = Lay::VEC, CPL = Lay::CPL, TPL = Lay::TPL;
  constexpr int NLD = BS / TPL;
  constexpr int bs_shift = SHIFT, part_mask = (1 << SHIFT) - 1;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int id = ids.get((b + u) >> bs_shift);
    ok[u] = id >= 0 && id < num_blocks;
    const int64_t base = (ok[u] ? (int64_t)id : 0) * block_elems + lane_off +
                         ((b + u) & part_mask) * BS * D;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
#pragma unroll
      for (int s = 0; s < CPL; ++s) {
        const int x = (u * NLD + i) * CPL + s;
        const int ch = Lay::chunk(c, s);
        kr[x] = make_uint4(0, 0, 0, 0);
        vr[x] = make_uint4(0, 0, 0, 0);
        if (ok[u] && ch >= 0) {
          kr[x] = *reinterpret_cast<const uint4 *>(kc + base + i * TPL * D + ch * VEC);
          vr[x] = *reinterpret_cast<const uint4 *>(vc + base + i * TPL * D + ch * VEC);
        }
      }
    }
  }
}

// Consume one stage of U whole blocks; a stage holding an invalid block id takes the
// masked path for its tokens.
template <int DT, int D, int BS, int G, int U>
__device__ __forceinline__ void consume_stage(const uint4 (&qv)[G][ValuLayout<DT, D>::CPL],
                                              const uint4 *kr, const uint4 *vr, const bool *ok,
                                              int nrows, float scale_log2, float (&m)[G],
                                              float (&l)[G],
                                              float (&acc)[G][ValuLayout<DT, D>::CPL *
                                                              Elem<DT>::VEC]) {
  constexpr int NLD = BS / ValuLayout<DT, D>::TPL;
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

// SHIFT: pool blocks hold BS << SHIFT tokens (0, or 1 for the reference's 32-token
// blocks); the kernel walks BS-token parts of them.
template <int DT, int D, int BS, int G, int NW, int U, bool PIPE, int SHIFT>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t q_st, int64_t q_sh,
    const typename Elem<DT>::T *__restrict__ kc, const typename Elem<DT>::T *__restrict__ vc,
    typename Elem<DT>::T *__restrict__ out, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ bt, int64_t bt_stride, int max_blocks,
    const int32_t *__restrict__ group_start, const int32_t *__restrict__ group_order,
    int64_t num_rows, int64_t num_groups, int H, int64_t num_blocks, float scale_log2) {
  using Lay = ValuLayout<DT, D>;
  constexpr int bs_shift = SHIFT;
  constexpr int VEC = Lay::VEC, CPL = Lay::CPL, LPT = Lay::LPT, TPL = Lay::TPL;
  constexpr int NLD = BS / TPL;  // loads per block per head and chunk slot
  static_assert(64 % LPT == 0 && BS % TPL == 0, "unsupported tile");

  // Per-wave softmax states for the cross-wave merge.
  __shared__ float s_acc[NW > 1 ? NW : 1][G][D];
  __shared__ float s_ml[NW > 1 ? NW : 1][G][2];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // 1-D grid over (group position, head), a position's heads on one XCD.
  int64_t pos;
  int h;
  xcd_position(blockIdx.x, (unsigned)H, pos, h);
  if (pos >= num_groups) return;  // workgroup-uniform
  int g = (int)pos;
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
  int nblk = L > 0 ? (L + BS - 1) / BS : 0;  // BS-token chunks
  nblk = min(nblk, max_blocks << bs_shift);
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

  uint4 qv[G][CPL];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
#pragma unroll
    for (int s = 0; s < CPL; ++s) {
      qv[gi][s] = make_uint4(0, 0, 0, 0);
      const int ch = Lay::chunk(c, s);
      if (gi < nrows && ch >= 0)
        qv[gi][s] = load16_unaligned<DT>(q + (row0 + gi) * q_st + h * q_sh + ch * VEC);
    }
  }
  float m[G], l[G], acc[G][CPL * VEC];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    m[gi] = NEG_INF_F;
    l[gi] = 0.f;
#pragma unroll
    for (int d = 0; d < CPL * VEC; ++d) acc[gi][d] = 0.f;
  }

  WaveBlockIds ids;
  if constexpr (SHIFT == 0)
    ids.init(bt + (int64_t)row0 * bt_stride, b0, b1);
  else
    ids.init(bt + (int64_t)row0 * bt_stride, b0 >> SHIFT,
             b1 > b0 ? ((b1 - 1) >> SHIFT) + 1 : b0 >> SHIFT);
  const int64_t block_elems = (int64_t)H * (BS << bs_shift) * D;
  const int lane_off = h * (BS << bs_shift) * D + tok * D;

  // Whole blocks of this wave's run are consumed U at a time.  With PIPE the loads
  // of stage s+1 are issued before stage s is consumed (two register stages live),
  // so each wave keeps K/V in flight while it computes; without it, latency is hidden
  // by the other waves the smaller register footprint lets the CU hold.
  const int bfull = max(b0, min(b1, Lc / BS));
  const int stages = (bfull - b0) / U;
  int b = b0;
  constexpr int SLOTS = U * NLD * CPL;
  if constexpr (PIPE) {
    if (stages > 0) {
      uint4 ka[SLOTS], va[SLOTS], kb[SLOTS], vb[SLOTS];
      bool oka[U], okb[U];
      load_stage<DT, D, BS, U, SHIFT>(kc, vc, ids, b, block_elems, lane_off, c, num_blocks, ka, va,
                               oka);
      for (int st = 0; st < stages; st += 2) {
        if (st + 1 < stages)
          load_stage<DT, D, BS, U, SHIFT>(kc, vc, ids, b + U, block_elems, lane_off, c, num_blocks,
                                   kb, vb, okb);
        consume_stage<DT, D, BS, G, U>(qv, ka, va, oka, nrows, scale_log2, m, l, acc);
        b += U;
        if (st + 1 >= stages) break;
        if (st + 2 < stages)
          load_stage<DT, D, BS, U, SHIFT>(kc, vc, ids, b + U, block_elems, lane_off, c, num_blocks,
                                   ka, va, oka);
        consume_stage<DT, D, BS, G, U>(qv, kb, vb, okb, nrows, scale_log2, m, l, acc);
        b += U;
      }
    }
  } else {
    for (int st = 0; st < stages; ++st, b += U) {
      uint4 kr[SLOTS], vr[SLOTS];
      bool ok[U];
      load_stage<DT, D, BS, U, SHIFT>(kc, vc, ids, b, block_elems, lane_off, c, num_blocks, kr,
                                      vr, ok);
      consume_stage<DT, D, BS, G, U>(qv, kr, vr, ok, nrows, scale_log2, m, l, acc);
    }
  }
  // Remaining blocks one at a time, with token and block-id masking.
  for (; b < b1; ++b) {
    uint4 kr[NLD * CPL], vr[NLD * CPL];
    bool ok[1];
    load_stage<DT, D, BS, 1, SHIFT>(kc, vc, ids, b, block_elems, lane_off, c, num_blocks, kr, vr,
                                    ok);
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
      for (int d = 0; d < CPL * VEC; ++d) {
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
#pragma unroll
      for (int s = 0; s < CPL; ++s) {
        const int ch = Lay::chunk(c, s);
        if (ch < 0) continue;
        float o[VEC];
#pragma unroll
        for (int d = 0; d < VEC; ++d) o[d] = acc[gi][s * VEC + d] * inv;
        *reinterpret_cast<uint4 *>(out + ((int64_t)(row0 + gi) * H + h) * D + ch * VEC) =
            pack16<DT>(o);
      }
    }
  } else {
    // Cross-wave merge through LDS.
    if (tok == 0) {
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        if (gi >= nrows) break;
#pragma unroll
        for (int s = 0; s < CPL; ++s) {
          const int ch = Lay::chunk(c, s);
          if (ch < 0) continue;
#pragma unroll
          for (int d = 0; d < VEC; ++d) s_acc[wave][gi][ch * VEC + d] = acc[gi][s * VEC + d];
        }
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
// when fp32 or wide heads need more loads per block.
template <int DT, int D, int G> constexpr int stage_blocks() {
  using Lay = ValuLayout<DT, D>;
  constexpr int nld = (16 / Lay::TPL) * Lay::CPL;
  return nld >= 4 ? 1 : 4 / nld;
}
// Register pipelining (two live stages) measured slower than the occupancy the
// smaller footprint buys, for every beam count; kept as a kernel option.
template <int G> constexpr bool stage_pipeline() { return false; }

}  // namespace vfl
