// Paged decode attention for row groups driven by a group plan (bf16 / fp16 caches,
// gfx950): the beams of each request in decoder self-attention, as in
// decode_shared.h, with the walk over the block tables done once per decode step on
// the host instead of in every layer's launch.
//
// A group plan lists, for every row group, the distinct block ids its rows read and,
// for each, the logical position and the tile columns (rows) that list it there
// (group_plan.h builds it from the block tables).  The table walk of the shared
// kernel costs a dependent level of loads (table entries, then ballots to
// de-duplicate them) before the first K/V block can be requested, and runs in each of
// the step's 12 layers; here the workgroup reads its group's record -- header and
// entries in one level -- and requests K/V blocks right after.  The entries are
// dealt to the waves round robin, U per stage, so every wave issues U block loads
// per round trip whatever the positions' mix of shared and private blocks.
//
// Per block the arithmetic is mfma_consume_cols: a column attends to a block only
// where its row lists it, so every row sees exactly its own blocks.  The fused KV
// write substitutes a row's new token into the registers of the block holding its
// last position, as the shared kernel does.
#pragma once

#include "decode_shared.h"
#include "group_plan.h"

namespace vfl {

// One entry of the wave's current 64-entry window: lane e % 64 of `reg`.
struct PlanEntries {
  const int32_t *base;  // first entry of the group's record
  int count;            // entries the record holds (capacity-clamped)
  int chunk;            // window index of `cur`
  int2 cur, nxt;        // entries 64 * chunk + lane and 64 * (chunk + 1) + lane

  __device__ __forceinline__ int2 fetch(int c) const {
    const int e = 64 * c + (int)__lane_id();
    return e < count ? *reinterpret_cast<const int2 *>(base + PLAN_ENTRY * e) : make_int2(-1, 0);
  }
  __device__ __forceinline__ void init(const int32_t *b, int n) {
    base = b;
    count = n;
    chunk = 0;
    cur = fetch(0);
    nxt = make_int2(-1, 0);
    if (n > 64) nxt = fetch(1);
  }
  // Slide the window so that entry e (wave-uniform, never decreasing by more than the
  // window) lies in `cur` or `nxt`.
  __device__ __forceinline__ void advance(int e) {
    if ((e >> 6) > chunk) {
      cur = nxt;
      ++chunk;
      nxt = count > 64 * (chunk + 1) ? fetch(chunk + 1) : make_int2(-1, 0);
    }
  }
  // (id, copy << 31 | position << 16 | tokens << 8 | columns) of entry e, e in
  // [64 * chunk, 64 * chunk + 128).
  __device__ __forceinline__ int2 get(int e) const {
    const bool in_cur = (e >> 6) == chunk;
    const int lane = e & 63;
    const int x = in_cur ? __builtin_amdgcn_readlane(cur.x, lane) : __builtin_amdgcn_readlane(nxt.x, lane);
    const int y = in_cur ? __builtin_amdgcn_readlane(cur.y, lane) : __builtin_amdgcn_readlane(nxt.y, lane);
    return make_int2(x, y);
  }
};

// Launch: one workgroup per (plan slot, head).  A slot beyond plan[0] (the used
// slots) or with no rows exits, so a caller can size the grid for its largest step.
// The K/V block ids come from the plan; seq_lens, the query and the new token from
// the rows the slot names.  q_vec: query rows are 16-byte aligned (16-byte loads).
template <int DT, int D, int NW, int U, bool FUSE>
__global__ __launch_bounds__(NW * 64) void paged_decode_planned_kernel(
    const uint16_t *__restrict__ q, int64_t q_st, int64_t q_sh, bool q_vec, const uint16_t *kc,
    const uint16_t *vc, uint16_t *__restrict__ out, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ plan, int64_t plan_stride, int64_t num_slots, int max_blocks,
    int64_t num_rows, int H, int64_t num_blocks, float scale_log2, KvWrite kvw) {
  constexpr int BS = 16;
  constexpr int KCH = D / 32;
  static_assert(D % 32 == 0, "built for head sizes 64 and 128");
  constexpr int VCH = D / 16;
  constexpr int MAXG = 16;
  constexpr int NCH = D / 32;  // 16-byte chunks per lane of a new K or V row
  __shared__ float s_acc[NW > 1 ? NW : 1][D][MAXG + 1];
  __shared__ float s_ml[NW > 1 ? NW : 1][2][MAXG];
  __shared__ uint32_t s_written[NW > 1 ? NW : 1];
  // Each wave's copy of the group's new tokens, [row][K, V][dim]: written and read by
  // that wave only, so no barrier orders it.
  __shared__ __align__(16) uint16_t s_new[FUSE ? NW : 1][FUSE ? PLAN_MAX_ROWS : 1][2][D];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t slot;
  int h;
  xcd_position(blockIdx.x, (unsigned)H, slot, h);
  if (slot >= num_slots || h >= H) return;  // workgroup-uniform

  // Level 1: the used-slot count, the slot's header and its first entries, together.
  const int32_t *rec = plan + PLAN_PREFIX + slot * plan_stride;
  const int used = plan[0];
  const int4 hdr = *reinterpret_cast<const int4 *>(rec);
  const int cap = (int)min<int64_t>((plan_stride - PLAN_HEADER) / PLAN_ENTRY, 1 << 24);
  PlanEntries ents;
  ents.init(rec + PLAN_HEADER, max(0, min(hdr.z, cap)));
  if (slot >= used) return;
  const int row0 = hdr.x;
  if (row0 < 0 || row0 >= num_rows || hdr.y <= 0) return;
  const int nrows = (int)min<int64_t>(min(hdr.y, PLAN_MAX_ROWS), num_rows - row0);
  const int n_e = ents.count;
  const uint32_t row_bits = (1u << nrows) - 1u;

  const int col = lane & 15;  // this lane's row of the group (tile column)
  const int rg = lane >> 4;   // tokens 4*rg .. 4*rg+3 of a block
  const bool has_row = col < nrows;
  const int64_t row = row0 + col;

  // Level 2: the rows' lengths, slots, queries and new tokens, and the first stage's
  // blocks (below), all requested before any of them is waited for.
  const int L = has_row ? seq_lens[row] : 0;
  int64_t wslot = -1;
  if constexpr (FUSE) {
    wslot = has_row ? kvw.slots[row] : -1;
    if (wslot >= num_blocks * BS) wslot = -1;
  }
  uint4 qop[KCH];
#pragma unroll
  for (int kk = 0; kk < KCH; ++kk) {
    qop[kk] = make_uint4(0, 0, 0, 0);
    if (has_row) {
      const uint16_t *qp = q + row * q_st + h * q_sh + 32 * kk + 8 * rg;
      qop[kk] = q_vec ? *reinterpret_cast<const uint4 *>(qp) : load16_unaligned<DT>(qp);
    }
  }
  uint4 nk[NCH], nv[NCH];
  if constexpr (FUSE) {
    const uint16_t *ks = kvw.k + row * kvw.k_st + h * kvw.k_sh + (D / 4) * rg;
    const uint16_t *vs = kvw.v + row * kvw.v_st + h * kvw.v_sh + (D / 4) * rg;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      nk[i] = nv[i] = make_uint4(0, 0, 0, 0);
      if (has_row && wslot >= 0) {
        nk[i] = load_row16<DT>(ks + 8 * i, kvw.vec);
        nv[i] = load_row16<DT>(vs + 8 * i, kvw.vec);
      }
    }
  }

  const int64_t block_elems = (int64_t)H * BS * D;
  const int head_off = h * BS * D;
  const int k_lane = col * D + 8 * rg;
  const int v_lane = (rg * D + col) * 4;  // vtile_index(4 * rg, col, D)

  // Wave w takes entries w, w + NW, w + 2 NW, ...; a stage is U of them.  The first
  // stage's block loads go out before anything waits for the level-2 loads above.
  // A copy entry (fused launch only) names its copy source: all of it is read, and the
  // block goes whole, with the row's new token in it, to the row's slot block before it
  // is consumed.
  int e_id[U], e_pos[U];
  uint32_t e_cols[U];
  bool e_ok[U], e_copy[U];
  MfmaBlock<D> blk[U];
  auto load_stage = [&](int e0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = e0 + NW * u;
      e_id[u] = 0;
      e_pos[u] = 0;
      e_cols[u] = 0;
      e_ok[u] = false;
      e_copy[u] = false;
      int tokens = 0;
      if (e < n_e) {
        const int2 en = ents.get(e);
        e_pos[u] = (int)(((uint32_t)en.y >> 16) & 0x7fffu);
        tokens = (int)(((uint32_t)en.y >> 8) & 0xffu);
        e_cols[u] = (uint32_t)en.y & 0xffu & row_bits;
        e_ok[u] = en.x >= 0 && en.x < num_blocks && e_pos[u] < max_blocks && e_cols[u] != 0;
        e_id[u] = e_ok[u] ? en.x : 0;
        e_copy[u] = FUSE && e_ok[u] && ((uint32_t)en.y & PLAN_COPY);
        tokens = e_copy[u] ? BS : tokens;
      }
      // Only the K rows and V 4-token groups of tokens some listing row attends to
      // (masked tokens are never read, so the rest may stay zero); a copy reads all.
      const bool k_ok = e_ok[u] && col < tokens;
      const bool v_ok = e_ok[u] && 4 * rg < tokens;
      const int64_t base = (int64_t)e_id[u] * block_elems + head_off;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) {
        blk[u].k[kk] = make_uint4(0, 0, 0, 0);
        if (k_ok) blk[u].k[kk] = load_stream16(kc + base + k_lane + 32 * kk);
      }
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        blk[u].v[c] = make_uint2(0, 0);
        if (v_ok) blk[u].v[c] = load_stream8(vc + base + v_lane + 64 * c);
      }
    }
  };
  int e0 = wave;
  if (e0 < n_e) load_stage(e0);
  // the block of the row's slot, where a copy entry's block goes (after the first
  // stage's loads are out: it waits for the slot)
  const int wblk = wslot >= 0 ? (int)(wslot / BS) : 0;

  const int my_nblk = L > 0 ? min((L + BS - 1) / BS, max_blocks) : 0;
  const int Lc = min(L, my_nblk * BS);
  const int last = (FUSE && L >= 1 && (L - 1) / BS < my_nblk) ? (L - 1) / BS : -1;
  const int t_new = L >= 1 ? (L - 1) % BS : 0;
  uint32_t written = 0;  // columns whose new token this wave substituted (uniform)

  floatx4_t acc[VCH];
#pragma unroll
  for (int c = 0; c < VCH; ++c) acc[c] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float m = NEG_INF_F, l = 0.f;

  if constexpr (FUSE) {  // this wave's copy of every row's new token
    if (e0 < n_e && has_row) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        *reinterpret_cast<uint4 *>(&s_new[wave][col][0][(D / 4) * rg + 8 * i]) = nk[i];
        *reinterpret_cast<uint4 *>(&s_new[wave][col][1][(D / 4) * rg + 8 * i]) = nv[i];
      }
    }
  }

  while (e0 < n_e) {
    uint32_t sub[U];
    if constexpr (FUSE) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool mine = (e_cols[u] >> col) & 1u;
        // a copy entry names the source: its row's new token goes to the slot's block
        sub[u] = column_mask(e_ok[u] && mine && last == e_pos[u] &&
                             (e_copy[u] ? wslot >= 0 : (int64_t)e_id[u] * BS + t_new == wslot));
        written |= sub[u];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (e_ok[u]) {
        if constexpr (FUSE) {
          uint32_t todo = sub[u];
          while (todo) {
            const int c = __builtin_ctz(todo);
            todo &= todo - 1;
            const int tn = __builtin_amdgcn_readlane(t_new, c);
            if (col == tn) {
#pragma unroll
              for (int kk = 0; kk < KCH; ++kk)
                blk[u].k[kk] =
                    *reinterpret_cast<const uint4 *>(&s_new[wave][c][0][32 * kk + 8 * rg]);
            }
            uint32_t newv[VCH];
#pragma unroll
            for (int cc = 0; cc < VCH; ++cc) newv[cc] = s_new[wave][c][1][16 * cc + col];
            if (e_copy[u]) {
              // The copy-on-write of a fork's block, folded in: the source's tokens with
              // the row's new token, stored whole to the row's slot block before the
              // consume masks V past the context.
              store_new_token<D, false>(kc, vc, 0, block_elems, head_off, k_lane, v_lane,
                                        col, rg, tn, newv, blk[u]);
              store_block<D>(kc, vc, __builtin_amdgcn_readlane(wblk, c), block_elems, head_off,
                             k_lane, v_lane, blk[u]);
            } else {
              store_new_token<D>(kc, vc, e_id[u], block_elems, head_off, k_lane, v_lane, col,
                                 rg, tn, newv, blk[u]);
            }
          }
        }
        const bool mine = (e_cols[u] >> col) & 1u;
        const int ext = row_max16(mine ? Lc : 0);
        mfma_consume_cols<DT, D>(qop, blk[u], mine, e_pos[u] * BS, Lc, ext, rg, scale_log2, m,
                                 l, acc);
      }
    }
    e0 += NW * U;
    if (e0 < n_e) {
      ents.advance(e0);
      load_stage(e0);
    }
  }

  // Column totals of the running sums (the 4 row groups hold disjoint tokens).
  l = rows_sum4(l);
  uint32_t written_all = written;
  if constexpr (NW > 1) {
#pragma unroll
    for (int c = 0; c < VCH; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_acc[wave][16 * c + 4 * rg + j][col] = acc[c][j];
    if (rg == 0) {
      s_ml[wave][0][col] = m;
      s_ml[wave][1][col] = l;
    }
    if (lane == 0) s_written[wave] = written;
    lds_barrier();
#pragma unroll
    for (int w = 0; w < NW; ++w) written_all |= s_written[w];
  }

  if constexpr (FUSE) {
    // Slots no entry took (not at the row's last position, or that block id out of
    // range): written as given, without substitution, by wave 0.
    uint32_t todo = column_mask(has_row && wslot >= 0) & ~written_all;
    if (wave != 0) todo = 0;
    while (todo) {
      const int c = __builtin_ctz(todo);
      todo &= todo - 1;
      const int64_t ws = kvw.slots[row0 + c];
      const int64_t sb = ws / BS, so = ws % BS;
      const uint16_t *ks = kvw.k + (row0 + c) * kvw.k_st + h * kvw.k_sh;
      const uint16_t *vs = kvw.v + (row0 + c) * kvw.v_st + h * kvw.v_sh;
      uint16_t *kd = const_cast<uint16_t *>(kc) + ((sb * H + h) * BS + so) * D;
      uint16_t *vd = const_cast<uint16_t *>(vc) + (sb * H + h) * D * BS;
      for (int d = lane; d < D; d += 64) {
        kd[d] = ks[d];
        vd[vtile_index((int)so, d, D)] = vs[d];
      }
    }
  }

  if constexpr (NW == 1) {
    if (!has_row) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t *orow = out + (row * H + h) * D + 4 * rg;
#pragma unroll
    for (int c = 0; c < VCH; ++c) {
      const uint32_t a = Mfma<DT>::narrow2(acc[c][0] * inv, acc[c][1] * inv);
      const uint32_t bb = Mfma<DT>::narrow2(acc[c][2] * inv, acc[c][3] * inv);
      *reinterpret_cast<uint2 *>(orow + 16 * c) = make_uint2(a, bb);
    }
  } else {
    for (int i = threadIdx.x; i < nrows * D; i += NW * 64) {
      const int beam = i / D, d = i % D;
      float M = NEG_INF_F;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_ml[w][0][beam]);
      const float Ms = (M == NEG_INF_F) ? 0.f : M;
      float S = 0.f, o = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = fast_exp2(s_ml[w][0][beam] - Ms);
        S = fmaf(s_ml[w][1][beam], f, S);
        o = fmaf(s_acc[w][d][beam], f, o);
      }
      out[((int64_t)(row0 + beam) * H + h) * D + d] =
          (uint16_t)Mfma<DT>::narrow(S > 0.f ? o / S : 0.f);
    }
  }
}

}  // namespace vfl
