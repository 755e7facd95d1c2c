// Paged decode attention for row groups whose rows keep their own block tables
// (bf16 / fp16 caches, gfx950): the beams of a request in decoder self-attention.
//
// Beam search forks a hypothesis by sharing its parent's blocks
// (vflorence/engine/block_manager.py:61-65) and copies only the partial block a fork
// writes into (:44-59), so the beams of a request list the same physical blocks for
// their common prefix.  One workgroup takes a group of up to 16 rows and one head.
// At every logical block position it loads each distinct block id that the group's
// rows list there once and multiplies it against all the rows' queries, held in the
// 16 columns of the MFMA tiles (as the cross-attention kernel does for beams that
// share one encoder table).  A column whose row does not list that block at that
// position gets zero weight, so every row still attends to exactly its own blocks, in
// logical order; with one wave the result is bit-identical to the one-row kernel's.
//
// The grouping is a performance choice only: any partition of the rows gives the same
// results, and rows that share nothing just cost one block load per row and position,
// as in the one-row kernel.
#pragma once

#include "decode_mfma.h"

namespace vfl {

// Per-lane block ids of the lane's row (tile column) at a wave's positions
// first + stride * j, four per register: lane (col, rg) holds the id of step j = base + rg.
// Ids are fetched up to the table width without waiting for the row's length (the
// length masks them when read), and the next four while these are consumed, so no
// table load sits on the critical path.
struct GroupBlockIds {
  const int32_t *row;  // this lane's row of the block table, or nullptr
  int width;           // entries of a table row that may be read
  int first, stride;
  int base;  // step held by rg == 0 in `cur`
  int cur, nxt;

  __device__ __forceinline__ int fetch(int j) const {
    const int pos = first + stride * (j + (int)(__lane_id() >> 4));
    return (row != nullptr && pos < width) ? row[pos] : -1;
  }
  __device__ __forceinline__ void init(const int32_t *r, int w, int f, int s) {
    row = r;
    width = w;
    first = f;
    stride = s;
    base = 0;
    cur = fetch(0);
    nxt = fetch(4);
  }
  // The id this lane's row lists at the wave-uniform step j (j never decreases), or -1
  // past the row's nblk blocks.
  __device__ __forceinline__ int get(int j, int col, int nblk) {
    while (j - base >= 4) {
      cur = nxt;
      base += 4;
      nxt = fetch(base + 4);
    }
    const int id = __shfl(cur, col + 16 * (j - base), 64);
    return first + stride * j < nblk ? id : -1;
  }
};

// Tile-column mask of a per-lane predicate (lanes l and l + 16k hold the same column).
__device__ __forceinline__ uint32_t column_mask(bool pred) {
  return (uint32_t)__builtin_amdgcn_ballot_w64(pred) & 0xffffu;
}

// Maximum of a per-column value over the 16 columns (every lane gets it).
__device__ __forceinline__ int column_max(int x) {
  return row_max16(x);
}

// Fold one block into the lane's state for the columns that list it (`mine`).
// Lc: the lane column's context length; ext: the largest Lc among the columns that
// list the block -- V of tokens at or past it may be stale and is zeroed so that a zero
// weight never meets a NaN.  For a listing column this is the same arithmetic as
// mfma_consume; for the others every weight is zero and the state is unchanged.
template <int DT, int D>
__device__ __forceinline__ void mfma_consume_cols(const uint4 (&qop)[D / 32], MfmaBlock<D> &blk,
                                                  bool mine, int tok0, int Lc, int ext, int rg,
                                                  float scale_log2, float &m, float &l,
                                                  floatx4_t (&acc)[D / 16]) {
  using Ops = Mfma<DT>;
  floatx4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) s = Ops::qk(blk.k[kk], qop[kk], s);
  float sv[4];
  bool keep[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = tok0 + 4 * rg + j;
    keep[j] = t < ext;
    sv[j] = (mine && t < Lc) ? s[j] * scale_log2 : NEG_INF_F;
  }
  float mb = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mb = rows_max4(mb);
  // Each column moves its reference only when its own block max needs it, so a
  // column's arithmetic never depends on the other columns of the tile.
  const bool need = mb > m + RESCALE_SLACK_LOG2;
  if (__builtin_amdgcn_ballot_w64(need) != 0) {
    const float corr = need ? fast_exp2(m - mb) : 1.f;
    l *= corr;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) acc[c] *= corr;
    m = need ? mb : m;
  }
  const float ms = (m == NEG_INF_F) ? 0.f : m;
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p[j] = fast_exp2(sv[j] - ms);
    l += p[j];
  }
  uint2 phi, plo;
  split_weights<DT>(p, phi, plo);
  const uint32_t keep01 = (keep[0] ? 0xffffu : 0u) | (keep[1] ? 0xffff0000u : 0u);
  const uint32_t keep23 = (keep[2] ? 0xffffu : 0u) | (keep[3] ? 0xffff0000u : 0u);
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    blk.v[c].x &= keep01;
    blk.v[c].y &= keep23;
    acc[c] = Ops::pv(blk.v[c], phi, acc[c]);
    acc[c] = Ops::pv(blk.v[c], plo, acc[c]);
  }
}

// Store the new token from registers: its K row (already in blk.k) from the lanes
// holding it, and its V values patched into the whole 8-byte words of its 4-token group,
// so 16 lanes cover one full 128-byte line (no partial-line read-modify-write).  The
// other three tokens' bytes go back unchanged; no other workgroup touches this head's
// slice of a private block.  With STORE false only the registers are patched (the
// caller stores the whole block).
template <int D, bool STORE = true>
__device__ __forceinline__ void store_new_token(const uint16_t *kc, const uint16_t *vc, int id,
                                                int64_t block_elems, int head_off, int k_lane,
                                                int v_lane, int col, int rg, int t_new,
                                                const uint32_t (&newv)[D / 16],
                                                MfmaBlock<D> &blk) {
  constexpr bool store = STORE;
  uint16_t *tile_k = const_cast<uint16_t *>(kc) + (int64_t)id * block_elems + head_off;
  uint16_t *tile_v = const_cast<uint16_t *>(vc) + (int64_t)id * block_elems + head_off;
  if (store && col == t_new) {
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk)
      store_stream16(tile_k + k_lane + 32 * kk, blk.k[kk]);
  }
  if (rg == t_new / 4) {
    const bool upper = (t_new & 2) != 0;
    const int sh = 16 * (t_new & 1);
    const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const uint32_t x = (blk.v[c].x & keep) | (newv[c] << sh);
      const uint32_t y = (blk.v[c].y & keep) | (newv[c] << sh);
      blk.v[c].x = upper ? blk.v[c].x : x;
      blk.v[c].y = upper ? y : blk.v[c].y;
      if (store) store_stream8(tile_v + v_lane + 64 * c, blk.v[c]);
    }
  }
}

// Store a whole loaded block (this head's slice: every lane's K row chunks and V
// 4-token words) to block `id`: 16 tokens x D of K and of V, in the pools' layouts.
template <int D>
__device__ __forceinline__ void store_block(const uint16_t *kc, const uint16_t *vc, int id,
                                            int64_t block_elems, int head_off, int k_lane,
                                            int v_lane, const MfmaBlock<D> &blk) {
  uint16_t *tile_k = const_cast<uint16_t *>(kc) + (int64_t)id * block_elems + head_off;
  uint16_t *tile_v = const_cast<uint16_t *>(vc) + (int64_t)id * block_elems + head_off;
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk)
    store_stream16(tile_k + k_lane + 32 * kk, blk.k[kk]);
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
    store_stream8(tile_v + v_lane + 64 * c, blk.v[c]);
}

// 16 bytes of a new-token row (K or V of one head), 16-byte aligned when `vec`.
template <int DT>
__device__ __forceinline__ uint4 load_row16(const uint16_t *p, bool vec) {
  return vec ? *reinterpret_cast<const uint4 *>(p) : load16_unaligned<DT>(p);
}

// FUSE: also perform the KV slot write of every row of the group, under the contract
// of the one-row fused kernel: a row's slot is the cache position of its last context
// token, in a block no other row reads, or a slot no row of the call attends to.  The
// block holding a row's new token then appears in the row's column only; when that
// block is consumed the new token is substituted in registers and stored from there.
// The new tokens are loaded with the first table loads and parked in LDS by the wave
// that will substitute them, so their latency never sits in a stage.  A slot
// elsewhere is written without substitution after the row's blocks, by the wave that
// owns the row's last position.
//
// Launch: one workgroup per (group slot, head); a group slot with group_start[g] ==
// group_start[g + 1] is empty and exits, so a caller can pad the grid to a fixed size.
template <int DT, int D, int NW, int U, bool FUSE>
__global__ __launch_bounds__(NW * 64) void paged_decode_shared_kernel(
    const uint16_t *__restrict__ q, int64_t q_st, int64_t q_sh, const uint16_t *kc,
    const uint16_t *vc, uint16_t *__restrict__ out, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ bt, int64_t bt_stride, int max_blocks,
    const int32_t *__restrict__ group_start, const int32_t *__restrict__ group_order,
    int64_t num_rows, int64_t num_groups, int H, int64_t num_blocks, float scale_log2,
    KvWrite kvw) {
  constexpr int BS = 16;
  constexpr int KCH = D / 32;
  static_assert(D % 32 == 0, "built for head sizes 64 and 128");
  constexpr int VCH = D / 16;
  constexpr int MAXG = 16;
  __shared__ float s_acc[NW > 1 ? NW : 1][D][MAXG + 1];
  __shared__ float s_ml[NW > 1 ? NW : 1][2][MAXG];
  // New tokens of the group's rows, [row][K, V][dim]; a row's entry is written and read
  // only by the wave owning the row's last position.
  __shared__ __align__(16) uint16_t s_new[FUSE ? MAXG : 1][2][D];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t pos;
  int h;
  xcd_position(blockIdx.x, (unsigned)H, pos, h);
  if (pos >= num_groups) return;  // workgroup-uniform
  int g = (int)pos;
  if (group_order) g = group_order[g];
  if (g < 0 || g >= num_groups || h >= H) return;  // workgroup-uniform
  const int row0 = group_start[g];
  if (row0 < 0 || row0 >= num_rows) return;
  int nrows = min(group_start[g + 1] - row0, MAXG);
  nrows = (int)min((int64_t)nrows, num_rows - row0);
  if (nrows <= 0) return;

  const int col = lane & 15;  // this lane's row of the group (tile column)
  const int rg = lane >> 4;   // tokens 4*rg .. 4*rg+3 of a block
  const bool has_row = col < nrows;
  const int64_t row = row0 + col;

  // Issued together: the row's length, its slot, its first block ids, its query.
  GroupBlockIds ids;
  ids.init(has_row ? bt + row * bt_stride : nullptr, max_blocks, wave, NW);
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
    if (has_row) qop[kk] = load16_unaligned<DT>(q + row * q_st + h * q_sh + 32 * kk + 8 * rg);
  }
  // The row's new K and V (dims D/4 * rg ..), parked in LDS after the first stage's
  // loads are issued.
  constexpr int NCH = D / 32;  // 16-byte chunks per lane and per K or V row
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
  bool parked = false;

  const int my_nblk = L > 0 ? min((L + BS - 1) / BS, max_blocks) : 0;
  const int Lc = min(L, my_nblk * BS);
  const int nblk = __builtin_amdgcn_readfirstlane(column_max(my_nblk));
  // Fused KV write: the new token is position L-1 (block `last`, offset t_new); it is
  // substituted when the row's table puts that position at the slot.
  const int last = (FUSE && L >= 1 && (L - 1) / BS < my_nblk) ? (L - 1) / BS : -1;
  const int t_new = L >= 1 ? (L - 1) % BS : 0;
  bool written = false;

  floatx4_t acc[VCH];
#pragma unroll
  for (int c = 0; c < VCH; ++c) acc[c] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float m = NEG_INF_F, l = 0.f;

  // Wave w takes positions w, w + NW, w + 2 NW, ...: the positions after the beams
  // diverge hold the most distinct blocks, and interleaving spreads them over all waves.
  const int nsteps = nblk > wave ? (nblk - wave + NW - 1) / NW : 0;
  const int64_t block_elems = (int64_t)H * BS * D;
  const int head_off = h * BS * D;
  const int k_lane = col * D + 8 * rg;
  const int v_lane = (rg * D + col) * 4;  // vtile_index(4 * rg, col, D)

  // Entries (position, block id, columns listing it) in position order; within a
  // position, distinct ids in order of their first column.
  int step = 0;
  int myid = -1;
  uint32_t pending = 0;
  if (nsteps > 0) {
    myid = ids.get(0, col, my_nblk);
    pending = column_mask(myid >= 0 && myid < num_blocks);
  }
  while (true) {
    int e_pos[U], e_id[U];
    uint32_t e_cols[U];
    int n = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      while (pending == 0 && step < nsteps) {
        if (++step < nsteps) {
          myid = ids.get(step, col, my_nblk);
          pending = column_mask(myid >= 0 && myid < num_blocks);
        }
      }
      e_pos[u] = wave + NW * step;
      e_id[u] = 0;
      e_cols[u] = 0;
      if (pending != 0) {
        const int c = __builtin_ctz(pending);
        const int id = __builtin_amdgcn_readlane(myid, c);
        const uint32_t cols = column_mask(myid == id);
        pending &= ~cols;
        e_id[u] = id;
        e_cols[u] = cols;
        n = u + 1;
      }
    }
    if (n == 0) break;
    MfmaBlock<D> blk[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      mfma_load_block<DT, D>(kc, vc, e_id[u], u < n, block_elems, head_off, k_lane, v_lane,
                             blk[u]);
    uint32_t sub[U];
    if constexpr (FUSE) {
      if (!parked) {  // the owner of the row's last position parks its new token
        parked = true;
        if (last >= 0 && last % NW == wave) {
#pragma unroll
          for (int i = 0; i < NCH; ++i) {
            *reinterpret_cast<uint4 *>(&s_new[col][0][(D / 4) * rg + 8 * i]) = nk[i];
            *reinterpret_cast<uint4 *>(&s_new[col][1][(D / 4) * rg + 8 * i]) = nv[i];
          }
        }
      }
      // Rows whose new token goes into an entry of this stage (one per entry unless
      // the caller's contract is broken).
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool mine = (e_cols[u] >> col) & 1u;
        sub[u] = column_mask(u < n && mine && last == e_pos[u] &&
                             (int64_t)e_id[u] * BS + t_new == wslot);
        written = written || ((sub[u] >> col) & 1u);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u < n) {
        if constexpr (FUSE) {
          uint32_t todo = sub[u];
          while (todo) {
            const int c = __builtin_ctz(todo);
            todo &= todo - 1;
            const int tn = __builtin_amdgcn_readlane(t_new, c);
            if (col == tn) {
#pragma unroll
              for (int kk = 0; kk < KCH; ++kk)
                blk[u].k[kk] = *reinterpret_cast<const uint4 *>(&s_new[c][0][32 * kk + 8 * rg]);
            }
            uint32_t newv[VCH];
#pragma unroll
            for (int cc = 0; cc < VCH; ++cc) newv[cc] = s_new[c][1][16 * cc + col];
            store_new_token<D>(kc, vc, e_id[u], block_elems, head_off, k_lane, v_lane, col, rg,
                               tn, newv, blk[u]);
          }
        }
        const bool mine = (e_cols[u] >> col) & 1u;
        const int ext = column_max(mine ? Lc : 0);
        mfma_consume_cols<DT, D>(qop, blk[u], mine, e_pos[u] * BS, Lc, ext, rg, scale_log2, m,
                                 l, acc);
      }
    }
  }

  if constexpr (FUSE) {
    // Slots written without substitution (not at the row's last position, or that
    // position's block id out of range): by the wave owning the row's last position.
    const int owner = last >= 0 ? last % NW : 0;
    uint32_t todo = column_mask(wslot >= 0 && !written && owner == wave);
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

  if (nblk == 0) {
    if (wave == 0)
      for (int i = lane; i < nrows * D; i += 64)
        out[((int64_t)(row0 + i / D) * H + h) * D + i % D] = 0;
    return;
  }

  // Column totals of the running sums (the 4 row groups hold disjoint tokens).
  l = rows_sum4(l);

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
#pragma unroll
    for (int c = 0; c < VCH; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_acc[wave][16 * c + 4 * rg + j][col] = acc[c][j];
    if (rg == 0) {
      s_ml[wave][0][col] = m;
      s_ml[wave][1][col] = l;
    }
    lds_barrier();
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
