// Paged decode attention on the matrix cores (bf16 / fp16 caches), gfx950.
//
// Per 16-token block and head, with the G query rows of a group (the beams of a
// request; one row for self-attention) in the 16 columns of the MFMA tiles:
//
//   S[tok][beam]  = K_tile[tok][:] . Q[beam][:]      v_mfma_f32_16x16x32 (D/32 of them)
//   online softmax over tok, per beam column         (VALU, 4 scores per lane)
//   O^T[d][beam] += V^T_tile[d][tok] . P[tok][beam]  v_mfma_f32_16x16x16 (D/16 of them)
//
// The S output layout (lane l, register j -> row 4*(l/16)+j, column l%16) is exactly
// the B-operand layout of the second product, so the probabilities never leave the
// lane that computed them.  The second product takes 4 consecutive tokens of one dim
// per lane, which is why V pools of 16-bit type store each [block][head] slice with
// tokens interleaved in groups of four ([block_size/4][head_dim][4], vtile_index);
// K keeps the logical [block_size][head_dim] order.
// P is split into two 16-bit terms (p = hi + lo) so the weights keep ~16 mantissa
// bits; the extra products are cheap next to the HBM traffic.
//
// Register footprint is ~50-70 VGPRs, so a CU holds many waves and the kernel stays
// HBM-bound for any beam count up to 16.  Waves of a workgroup split the context
// and merge through LDS, as in the VALU kernel.
#pragma once

#include "common.h"
#include "mfma_ops.h"

namespace vfl {

// 32-wide K chunks of a head of size D (a multiple of 16): the last one is half empty
// when D is an odd multiple of 16, its dims past D zero in both the query and K operand.
template <int D> constexpr int k_chunks() { return (D + 31) / 32; }
// Whether lane row group rg's 8 dims of K chunk kk lie inside the head.
template <int D> __device__ __forceinline__ bool k_chunk_ok(int kk, int rg) {
  if constexpr (D % 32 == 0) return true;
  else return 32 * kk + 8 * rg < D;
}

// Loads of one block for this lane: k_chunks<D>() 16-byte K chunks (token `col`, dims
// 32*kk + 8*rg ..) and D/16 8-byte V chunks (dim 16*c + col, tokens 4*rg .. 4*rg+3).
template <int D> struct MfmaBlock {
  uint4 k[k_chunks<D>()];
  uint2 v[D / 16];
};

// The self-attention op's new token: its K/V rows and the slot they are written to.
// With it, the kernel writes the slot itself and feeds the new values straight into
// the last block instead of a separate scatter launch before the attention.
struct KvWrite {
  const uint16_t *k;
  int64_t k_st, k_sh;
  const uint16_t *v;
  int64_t v_st, v_sh;
  const int64_t *slots;
  bool vec;  // every K and V row is 16-byte aligned (16-byte loads)
};

// K/V pages are read once per decode step, so their loads are non-temporal: they stream
// through without displacing the metadata, queries and tables the step's next launches
// read from the caches.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 load_stream16(const uint16_t *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_stream8(const uint16_t *p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
  return make_uint2(v.x, v.y);
}
// The beam-group kernels' fused KV write stores non-temporally too.  Nothing in the
// launch reads them back, and a streamed line does not stay dirty in the XCD's L2, which
// the end of every launch writes back before the next one starts: on the 64 x 4-beam
// decode step the step ran 0.5113 -> 0.4924 ms with these stores streamed (write-through
// stores, sc0 sc1, ran it at 0.853 ms).  The one-row kernel below keeps ordinary stores:
// its write goes out after the first stage of a long launch, and streamed there the
// 256-sequence op ran 105.9 against 102.2 us.
__device__ __forceinline__ void store_stream16(uint16_t *p, uint4 v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t *>(p));
}
__device__ __forceinline__ void store_stream8(uint16_t *p, uint2 v) {
  __builtin_nontemporal_store(u32x2_t{v.x, v.y}, reinterpret_cast<u32x2_t *>(p));
}

// Load one block's K rows and V 4-token groups into MFMA operand order.  `tokens`
// (1..16) leaves the K rows and V groups of later tokens unread (zero): a partial last
// block then reads only its tokens, whose weights are all the masked consume uses.
template <int DT, int D>
__device__ __forceinline__ void mfma_load_block(const uint16_t *__restrict__ kc,
                                                const uint16_t *__restrict__ vc, int id, bool ok,
                                                int64_t block_elems, int head_off, int k_lane,
                                                int v_lane, MfmaBlock<D> &blk, int tokens = 16) {
  const int64_t base = (ok ? (int64_t)id : 0) * block_elems + head_off;
  const int rg = (int)(__lane_id() >> 4);
  const bool k_ok = ok && (int)(__lane_id() & 15) < tokens;
  const bool v_ok = ok && 4 * rg < tokens;
#pragma unroll
  for (int kk = 0; kk < k_chunks<D>(); ++kk) {
    blk.k[kk] = make_uint4(0, 0, 0, 0);
    if (k_ok && k_chunk_ok<D>(kk, rg)) blk.k[kk] = load_stream16(kc + base + k_lane + 32 * kk);
  }
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    blk.v[c] = make_uint2(0, 0);
    if (v_ok) blk.v[c] = load_stream8(vc + base + v_lane + 64 * c);
  }
}

// Fold one block into the lane's state.  tok0 is the block's first token index;
// MASKED handles tokens at or past Lc and invalid block ids (ok == false).
template <int DT, int D, bool MASKED>
__device__ __forceinline__ void mfma_consume(const uint4 (&qop)[k_chunks<D>()], MfmaBlock<D> &blk,
                                             bool ok, int tok0, int Lc, int rg,
                                             float scale_log2, float &m, float &l,
                                             floatx4_t (&acc)[D / 16]) {
  using Ops = Mfma<DT>;
  floatx4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < k_chunks<D>(); ++kk) s = Ops::qk(blk.k[kk], qop[kk], s);
  float sv[4];
  bool valid[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    valid[j] = true;
    if constexpr (MASKED) valid[j] = ok && (tok0 + 4 * rg + j) < Lc;
    sv[j] = valid[j] ? s[j] * scale_log2 : NEG_INF_F;
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
  if constexpr (MASKED) {
    // Stale or garbage V of masked tokens must not meet a zero weight (0 * NaN).
    const uint32_t keep01 = (valid[0] ? 0xffffu : 0u) | (valid[1] ? 0xffff0000u : 0u);
    const uint32_t keep23 = (valid[2] ? 0xffffu : 0u) | (valid[3] ? 0xffff0000u : 0u);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      blk.v[c].x &= keep01;
      blk.v[c].y &= keep23;
    }
  }
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    acc[c] = Ops::pv(blk.v[c], phi, acc[c]);
    acc[c] = Ops::pv(blk.v[c], plo, acc[c]);
  }
}

// Put the new token (K row chunks newk, V values newv) into the registers of its block
// and store it to the cache.  Lanes holding token t_new's K row (col == t_new) store
// their 16-byte chunks; lanes holding its 4-token V group (rg == t_new / 4) store the
// whole 8-byte word of each chunk, so 16 lanes cover one full 128-byte line and the
// write needs no read-modify-write below.  The other three tokens' bytes go back
// unchanged; no other workgroup touches this head's slice of a private block.
template <int D>
__device__ __forceinline__ void write_new_token(const uint16_t *kc, const uint16_t *vc, int id,
                                                int64_t block_elems, int head_off, int k_lane,
                                                int v_lane, int col, int rg, int t_new,
                                                const uint4 (&newk)[k_chunks<D>()],
                                                const uint32_t (&newv)[D / 16],
                                                MfmaBlock<D> &blk) {
  uint16_t *tile_k = const_cast<uint16_t *>(kc) + (int64_t)id * block_elems + head_off;
  uint16_t *tile_v = const_cast<uint16_t *>(vc) + (int64_t)id * block_elems + head_off;
  if (col == t_new) {
#pragma unroll
    for (int kk = 0; kk < k_chunks<D>(); ++kk) {
      if (!k_chunk_ok<D>(kk, rg)) continue;
      blk.k[kk] = newk[kk];
      *reinterpret_cast<uint4 *>(tile_k + k_lane + 32 * kk) = newk[kk];
    }
  }
  if (rg == t_new / 4) {
    // Selects, not a dynamically indexed reference, so the block stays in registers.
    const bool upper = (t_new & 2) != 0;
    const int sh = 16 * (t_new & 1);
    const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const uint32_t x = (blk.v[c].x & keep) | (newv[c] << sh);
      const uint32_t y = (blk.v[c].y & keep) | (newv[c] << sh);
      blk.v[c].x = upper ? blk.v[c].x : x;
      blk.v[c].y = upper ? y : blk.v[c].y;
      *reinterpret_cast<uint2 *>(tile_v + v_lane + 64 * c) = blk.v[c];
    }
  }
}

// FUSE: also perform the KV slot write of `kvw` (one row per group).  The caller
// guarantees that a row's slot, when it is the cache position of the row's last
// context token, lies in a block no other row reads; the write then needs no ordering
// against other workgroups.  A slot elsewhere is still written, without substitution.
// SHIFT: pool blocks hold 16 << SHIFT tokens (0, or 1 for the reference's 32-token
// blocks); the kernel walks 16-token chunks, chunk b being part b & mask of table entry
// b >> SHIFT (the same offset, 16 * D elements per part, in K and in the
// 4-token-interleaved V).
// desc (shared-table groups, no fused write): one descriptor per launch slot, at
// desc + slot * desc_stride: first row, rows, length, 0, then the group's table row.
// The workgroup then reads its group -- rows, length and first 64 block ids -- in one
// dependent load level instead of three (dispatch order, group start, then length and
// table); group_order, group_start, seq_lens and bt are not read.
template <int DT, int D, int NW, int U, bool FUSE, int SHIFT>
__global__ __launch_bounds__(NW * 64) void paged_decode_mfma_kernel(
    const uint16_t *__restrict__ q, int64_t q_st, int64_t q_sh, const uint16_t *kc,
    const uint16_t *vc, uint16_t *__restrict__ out, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ bt, int64_t bt_stride, int max_blocks,
    const int32_t *__restrict__ group_start, const int32_t *__restrict__ group_order,
    int64_t num_rows, int64_t num_groups, int H, int64_t num_blocks, float scale_log2,
    KvWrite kvw, const int32_t *__restrict__ desc = nullptr, int64_t desc_stride = 0) {
  constexpr int BS = 16;
  constexpr int bs_shift = SHIFT;
  static_assert(!FUSE || SHIFT == 0, "the fused KV write is built for 16-token blocks");
  constexpr int KCH = k_chunks<D>();
  constexpr int VCH = D / 16;
  constexpr int MAXG = 16;  // query rows per group held in the tile columns
  static_assert(D % 16 == 0, "head size must be a multiple of 16");
  // Cross-wave merge buffers: [wave][dim][beam] (+1 column of padding) and (m, l).
  __shared__ float s_acc[NW > 1 ? NW : 1][D][MAXG + 1];
  __shared__ float s_ml[NW > 1 ? NW : 1][2][MAXG];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t pos;
  int h;
  xcd_position(blockIdx.x, (unsigned)H, pos, h);
  if (pos >= num_groups || h >= H) return;  // workgroup-uniform
  int row0, nrows, L;
  WaveBlockIds ids;
  if (!FUSE && desc) {
    const int32_t *rec = desc + pos * desc_stride;
    const int4 hdr = *reinterpret_cast<const int4 *>(rec);
    ids.prefetch(rec + 4, max_blocks);
    row0 = hdr.x;
    nrows = min(hdr.y, MAXG);
    L = hdr.z;
    if (row0 < 0 || row0 >= num_rows) return;
    nrows = (int)min((int64_t)nrows, num_rows - row0);
    if (nrows <= 0) return;
  } else {
    int g = (int)pos;
    if (group_order) g = group_order[g];
    if (g < 0 || g >= num_groups) return;
    row0 = g;
    nrows = 1;
    if (group_start) {
      row0 = group_start[g];
      nrows = min(group_start[g + 1] - row0, MAXG);
    }
    if (row0 < 0 || row0 >= num_rows) return;
    nrows = (int)min((int64_t)nrows, num_rows - row0);
    if (nrows <= 0) return;
    ids.prefetch(bt + (int64_t)row0 * bt_stride, max_blocks);
    L = seq_lens[row0];
  }
  int nblk = L > 0 ? (L + BS - 1) / BS : 0;  // 16-token chunks
  nblk = min(nblk, max_blocks << bs_shift);
  const int Lc = min(L, nblk * BS);
  const int col = lane & 15;  // query row (beam) of this lane's tile column
  const int rg = lane >> 4;   // row group: tokens 4*rg .. 4*rg+3 of a block

  const int chunk = (nblk + NW - 1) / NW;
  const int b0 = min(nblk, wave * chunk);
  const int b1 = min(nblk, b0 + chunk);

  // Fused KV write: the new token is position L-1; `subst` when its slot is where
  // this row's table puts that position (the normal case).
  int64_t wslot = -1;
  int last = -1, t_new = 0;
  int32_t lid = -1;
  bool subst = false;
  if constexpr (FUSE) {
    wslot = kvw.slots[row0];
    if (wslot >= num_blocks * BS) wslot = -1;
    if (L >= 1 && (L - 1) / BS < nblk) {
      last = (L - 1) / BS;
      t_new = (L - 1) % BS;
      lid = bt[(int64_t)row0 * bt_stride + last];
      subst = wslot >= 0 && (int64_t)lid * BS + t_new == wslot;
    }
    // A slot the row does not attend to is written by wave 0 without substitution.
    if (wslot >= 0 && !subst && wave == 0) {
      const int64_t sb = wslot / BS, so = wslot % BS;
      const uint16_t *ks = kvw.k + row0 * kvw.k_st + h * kvw.k_sh;
      const uint16_t *vs = kvw.v + row0 * kvw.v_st + h * kvw.v_sh;
      uint16_t *kd = const_cast<uint16_t *>(kc) + ((sb * H + h) * BS + so) * D;
      uint16_t *vd = const_cast<uint16_t *>(vc) + (sb * H + h) * D * BS;
      for (int d = lane; d < D; d += 64) {
        kd[d] = ks[d];
        vd[vtile_index((int)so, d, D)] = vs[d];
      }
    }
  }

  if (nblk == 0) {
    for (int i = threadIdx.x; i < nrows * D; i += NW * 64)
      out[((int64_t)(row0 + i / D) * H + h) * D + i % D] = 0;
    return;
  }

  // Q^T operand: lane holds Q[beam col][32*kk + 8*rg .. +7]; zero for absent beams.
  uint4 qop[KCH];
#pragma unroll
  for (int kk = 0; kk < KCH; ++kk) {
    qop[kk] = make_uint4(0, 0, 0, 0);
    if (col < nrows && k_chunk_ok<D>(kk, rg))
      qop[kk] = load16_unaligned<DT>(q + (row0 + col) * q_st + h * q_sh + 32 * kk + 8 * rg);
  }
  floatx4_t acc[VCH];
#pragma unroll
  for (int c = 0; c < VCH; ++c) acc[c] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float m = NEG_INF_F, l = 0.f;

  ids.limit(b1 > b0 ? ((b1 - 1) >> SHIFT) + 1 : 0);
  constexpr int part_mask = (1 << SHIFT) - 1;
  const int64_t block_elems = (int64_t)H * (BS << bs_shift) * D;
  const int head_off = h * (BS << bs_shift) * D;
  const int k_lane = col * D + 8 * rg;
  const int v_lane = (rg * D + col) * 4;  // vtile_index(4 * rg, col, D)

  int bfull = max(b0, min(b1, Lc / BS));
  // The wave whose run ends with the new token's block loads that block and the new
  // K/V first and issues the slot write after its first stage, so the write's latency
  // hides behind the rest of the run; the block is still consumed last, in order, so
  // results are bit-identical to the separate write + attention.
  bool own_last = false;
  int b_stop = b1;
  MfmaBlock<D> lastblk;
  uint4 newk[KCH];
  uint32_t newv[VCH];
  if constexpr (FUSE) {
    own_last = subst && b0 <= last && last < b1;
    if (own_last) {
      b_stop = last;
      mfma_load_block<DT, D>(kc, vc, lid, true, block_elems, head_off, k_lane, v_lane, lastblk);
      const uint16_t *ks = kvw.k + row0 * kvw.k_st + h * kvw.k_sh;
      const uint16_t *vs = kvw.v + row0 * kvw.v_st + h * kvw.v_sh;
#pragma unroll
      for (int kk = 0; kk < KCH; ++kk) {
        newk[kk] = make_uint4(0, 0, 0, 0);
        if (k_chunk_ok<D>(kk, rg)) newk[kk] = load16_unaligned<DT>(ks + 32 * kk + 8 * rg);
      }
#pragma unroll
      for (int c = 0; c < VCH; ++c) newv[c] = vs[16 * c + col];
    }
  }
  bfull = min(bfull, max(b0, b_stop));
  int b = b0;
  for (; b + U <= bfull; b += U) {
    MfmaBlock<D> blk[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int id = ids.get((b + u) >> bs_shift);
      ok[u] = id >= 0 && id < num_blocks;
      mfma_load_block<DT, D>(kc, vc, id, ok[u], block_elems,
                             head_off + ((b + u) & part_mask) * BS * D, k_lane, v_lane, blk[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ok[u])
        mfma_consume<DT, D, false>(qop, blk[u], true, (b + u) * BS, Lc, rg, scale_log2, m, l,
                                   acc);
      else
        mfma_consume<DT, D, true>(qop, blk[u], false, (b + u) * BS, Lc, rg, scale_log2, m, l,
                                  acc);
    }
    if constexpr (FUSE) {
      if (own_last && b == b0)
        write_new_token<D>(kc, vc, lid, block_elems, head_off, k_lane, v_lane, col, rg, t_new,
                           newk, newv, lastblk);
    }
  }
  if constexpr (FUSE) {
    if (own_last && bfull - b0 < U)  // no whole stage ran: write now
      write_new_token<D>(kc, vc, lid, block_elems, head_off, k_lane, v_lane, col, rg, t_new,
                         newk, newv, lastblk);
  }
  for (; b < b_stop; ++b) {
    MfmaBlock<D> blk;
    const int id = ids.get(b >> bs_shift);
    const bool ok = id >= 0 && id < num_blocks;
    mfma_load_block<DT, D>(kc, vc, id, ok, block_elems, head_off + (b & part_mask) * BS * D,
                           k_lane, v_lane, blk, min(BS, Lc - b * BS));
    mfma_consume<DT, D, true>(qop, blk, ok, b * BS, Lc, rg, scale_log2, m, l, acc);
  }
  if constexpr (FUSE) {
    if (own_last)
      mfma_consume<DT, D, true>(qop, lastblk, true, last * BS, Lc, rg, scale_log2, m, l, acc);
  }

  // Column totals of the running sums (the 4 row groups hold disjoint tokens).
  l = rows_sum4(l);

  if constexpr (NW == 1) {
    if (col >= nrows) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t *orow = out + ((int64_t)(row0 + col) * H + h) * D + 4 * rg;
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
