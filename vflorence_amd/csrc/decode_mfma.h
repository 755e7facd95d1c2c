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
// lane that computed them.  The second product needs tokens contiguous for a fixed
// dim, which is why V pools of 16-bit type store each [block][head] slice transposed
// ([head_dim][block_size]); K keeps the logical [block_size][head_dim] order.
// P is split into two 16-bit terms (p = hi + lo) so the weights keep ~16 mantissa
// bits; the extra products are cheap next to the HBM traffic.
//
// Register footprint is ~50-70 VGPRs, so a CU holds many waves and the kernel stays
// HBM-bound for any beam count up to 16.  Waves of a workgroup split the context
// and merge through LDS, as in the VALU kernel.
#pragma once

#include "common.h"

namespace vfl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

template <int DT> struct Mfma;

template <> struct Mfma<VFL_BFLOAT16> {
  static __device__ __forceinline__ floatx4_t qk(const uint4 &k, const uint4 &q, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, k),
                                                   __builtin_bit_cast(bf16x8_t, q), c, 0, 0, 0);
  }
  static __device__ __forceinline__ floatx4_t pv(const uint2 &v, const uint2 &p, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, v),
                                                     __builtin_bit_cast(short4_t, p), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t narrow(float f) { return f32_to_bf16(f); }
  static __device__ __forceinline__ float widen(uint32_t h) { return __uint_as_float(h << 16); }
};

template <> struct Mfma<VFL_FLOAT16> {
  static __device__ __forceinline__ floatx4_t qk(const uint4 &k, const uint4 &q, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, k),
                                                  __builtin_bit_cast(half8_t, q), c, 0, 0, 0);
  }
  static __device__ __forceinline__ floatx4_t pv(const uint2 &v, const uint2 &p, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, v),
                                                 __builtin_bit_cast(half4_t, p), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t narrow(float f) { return f32_to_f16(f); }
  static __device__ __forceinline__ float widen(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
};

// Loads of one block for this lane: D/32 16-byte K chunks (token `col`, dims
// 32*kk + 8*rg ..) and D/16 8-byte V^T chunks (dim 16*c + col, tokens 4*rg ..).
template <int D> struct MfmaBlock {
  uint4 k[D / 32];
  uint2 v[D / 16];
};

template <int DT, int D>
__device__ __forceinline__ void mfma_load_block(const uint16_t *__restrict__ kc,
                                                const uint16_t *__restrict__ vc, int id, bool ok,
                                                int64_t block_elems, int head_off, int k_lane,
                                                int v_lane, MfmaBlock<D> &blk) {
  constexpr int BS = 16;
  const int64_t base = (ok ? (int64_t)id : 0) * block_elems + head_off;
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) {
    blk.k[kk] = make_uint4(0, 0, 0, 0);
    if (ok) blk.k[kk] = *reinterpret_cast<const uint4 *>(kc + base + k_lane + 32 * kk);
  }
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    blk.v[c] = make_uint2(0, 0);
    if (ok) blk.v[c] = *reinterpret_cast<const uint2 *>(vc + base + v_lane + 16 * c * BS);
  }
}

// Fold one block into the lane's state.  tok0 is the block's first token index;
// MASKED handles tokens at or past Lc and invalid block ids (ok == false).
template <int DT, int D, bool MASKED>
__device__ __forceinline__ void mfma_consume(const uint4 (&qop)[D / 32], MfmaBlock<D> &blk,
                                             bool ok, int tok0, int Lc, int rg,
                                             float scale_log2, float &m, float &l,
                                             floatx4_t (&acc)[D / 16]) {
  using Ops = Mfma<DT>;
  floatx4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) s = Ops::qk(blk.k[kk], qop[kk], s);
  float sv[4];
  bool valid[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    valid[j] = true;
    if constexpr (MASKED) valid[j] = ok && (tok0 + 4 * rg + j) < Lc;
    sv[j] = valid[j] ? s[j] * scale_log2 : NEG_INF_F;
  }
  float mb = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
  mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
  if (__builtin_amdgcn_ballot_w64(mb > m + RESCALE_SLACK_LOG2) != 0) {
    const float mn = fmaxf(m, mb);
    const float corr = (mn == NEG_INF_F) ? 1.f : fast_exp2(m - mn);
    l *= corr;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) acc[c] *= corr;
    m = mn;
  }
  const float ms = (m == NEG_INF_F) ? 0.f : m;
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p[j] = fast_exp2(sv[j] - ms);
    l += p[j];
  }
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hi[j] = Ops::narrow(p[j]);
    lo[j] = Ops::narrow(p[j] - Ops::widen(hi[j]));
  }
  const uint2 phi = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
  const uint2 plo = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
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

template <int DT, int D, int NW, int U>
__global__ __launch_bounds__(NW * 64) void paged_decode_mfma_kernel(
    const uint16_t *__restrict__ q, int64_t q_st, int64_t q_sh, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, uint16_t *__restrict__ out,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ bt, int64_t bt_stride,
    int max_blocks, const int32_t *__restrict__ group_start,
    const int32_t *__restrict__ group_order, int64_t num_rows, int64_t num_groups, int H,
    int64_t num_blocks, float scale_log2) {
  constexpr int BS = 16;
  constexpr int KCH = D / 32;
  constexpr int VCH = D / 16;
  constexpr int MAXG = 16;  // query rows per group held in the tile columns
  // Cross-wave merge buffers: [wave][dim][beam] (+1 column of padding) and (m, l).
  __shared__ float s_acc[NW > 1 ? NW : 1][D][MAXG + 1];
  __shared__ float s_ml[NW > 1 ? NW : 1][2][MAXG];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h = (int)(blockIdx.x % (unsigned)H);
  int g = (int)(blockIdx.x / (unsigned)H);
  if (group_order) g = group_order[g];
  if (g < 0 || g >= num_groups || h >= H) return;  // workgroup-uniform
  int row0 = g, nrows = 1;
  if (group_start) {
    row0 = group_start[g];
    nrows = min(group_start[g + 1] - row0, MAXG);
  }
  if (row0 < 0 || row0 >= num_rows) return;
  nrows = (int)min((int64_t)nrows, num_rows - row0);
  if (nrows <= 0) return;
  const int L = seq_lens[row0];
  int nblk = L > 0 ? (L + BS - 1) / BS : 0;
  nblk = min(nblk, max_blocks);
  const int Lc = min(L, nblk * BS);
  const int col = lane & 15;  // query row (beam) of this lane's tile column
  const int rg = lane >> 4;   // row group: tokens 4*rg .. 4*rg+3 of a block

  if (nblk == 0) {
    for (int i = threadIdx.x; i < nrows * D; i += NW * 64)
      out[((int64_t)(row0 + i / D) * H + h) * D + i % D] = 0;
    return;
  }
  const int chunk = (nblk + NW - 1) / NW;
  const int b0 = min(nblk, wave * chunk);
  const int b1 = min(nblk, b0 + chunk);

  // Q^T operand: lane holds Q[beam col][32*kk + 8*rg .. +7]; zero for absent beams.
  uint4 qop[KCH];
#pragma unroll
  for (int kk = 0; kk < KCH; ++kk) {
    qop[kk] = make_uint4(0, 0, 0, 0);
    if (col < nrows)
      qop[kk] = load16_unaligned<DT>(q + (row0 + col) * q_st + h * q_sh + 32 * kk + 8 * rg);
  }
  floatx4_t acc[VCH];
#pragma unroll
  for (int c = 0; c < VCH; ++c) acc[c] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float m = NEG_INF_F, l = 0.f;

  WaveBlockIds ids;
  ids.init(bt + (int64_t)row0 * bt_stride, b0, b1);
  const int64_t block_elems = (int64_t)H * BS * D;
  const int head_off = h * BS * D;
  const int k_lane = col * D + 8 * rg;
  const int v_lane = col * BS + 4 * rg;

  const int bfull = max(b0, min(b1, Lc / BS));
  int b = b0;
  for (; b + U <= bfull; b += U) {
    MfmaBlock<D> blk[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int id = ids.get(b + u);
      ok[u] = id >= 0 && id < num_blocks;
      mfma_load_block<DT, D>(kc, vc, id, ok[u], block_elems, head_off, k_lane, v_lane, blk[u]);
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
  }
  for (; b < b1; ++b) {
    MfmaBlock<D> blk;
    const int id = ids.get(b);
    const bool ok = id >= 0 && id < num_blocks;
    mfma_load_block<DT, D>(kc, vc, id, ok, block_elems, head_off, k_lane, v_lane, blk);
    mfma_consume<DT, D, true>(qop, blk, ok, b * BS, Lc, rg, scale_log2, m, l, acc);
  }

  // Column totals of the running sums (the 4 row groups hold disjoint tokens).
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);

  if constexpr (NW == 1) {
    if (col >= nrows) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t *orow = out + ((int64_t)(row0 + col) * H + h) * D + 4 * rg;
#pragma unroll
    for (int c = 0; c < VCH; ++c) {
      const uint32_t a = Mfma<DT>::narrow(acc[c][0] * inv) | (Mfma<DT>::narrow(acc[c][1] * inv) << 16);
      const uint32_t bb = Mfma<DT>::narrow(acc[c][2] * inv) | (Mfma<DT>::narrow(acc[c][3] * inv) << 16);
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
    __syncthreads();
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
