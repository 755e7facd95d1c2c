// Decode-step linear layers on the matrix cores (gfx950), 16-bit inputs and output,
// fp32 sums:
//
//   y[m][n] = sum_k x[m][k] * w[n][k] + bias[n]        (w: nn.Linear's [out, in])
//
// for the few hundred token rows of a decode step times the decoder's projection
// weights (vflorence/models/bart.py:111,114,142,146: the fused q|k|v, the attention
// output and the cross-attention query projections).  Each step streams every weight
// from HBM once (a decoder's weights exceed the last-level cache), so the time goes to
// memory round trips, not arithmetic: a GEMM that walks K in a loop pays one round
// trip per K step.  Here a workgroup owns a 32-feature x 32-token output tile and
// splits K over its 8 waves.  Each wave loads the operands of up to 4 K steps of 32 in
// one batch, so K <= 1024 costs one round trip; a longer K range is walked in batches
// of 2 steps with the next batch in flight while one is multiplied.  The waves' partial
// tiles are summed through LDS in the order of a 3-level tree (waves w and w + 4 first,
// then (s0 + s2) + (s1 + s3)) with three barriers, and four waves then add the bias and
// store one 16 x 16 quarter each.
//
// Operand order.  The product per 32-wide K step is mfma_f32_16x16x32 with A = 16
// weight rows (features) and B = 16 token rows, giving D[feature][token]; a lane's four
// D registers are four consecutive features of one token -- one 8-byte store.  Lane l
// holds row l % 16 and k = 8 (l / 16) .. +7 of both operands, so neighbouring lanes read
// rows 2 KB apart.  Loaded that way, every 16-byte chunk is a separate cache access.
// The operands are therefore brought in contiguously instead:
// - The weight is re-laid out once (vfl_pack_linear_weight) into 1 KB blocks of 16
//   rows x 32 k, each stored in lane order: block (r, c) holds, for lane l, row
//   16 r + l % 16 and k = 32 c + 8 (l / 16) .. +7 at byte 16 l.  One wave load is then
//   one contiguous KB.  Rows are padded with zeros to a multiple of 32.
// - Activation rows are read as 64-byte runs (lanes 4 i .. 4 i + 3 take row i) and
//   moved into operand order with ds_bpermute (lane l takes lane 4 (l % 16) + l / 16).
//   Activations that one call produces for another can skip that: the feed-forward
//   block (bart.py:192-201, fc2(gelu(fc1(h)))) runs fc1 with the exact GELU in its
//   epilogue and its output written in the packed layout (token rows as the weight's
//   rows), which fc2 then reads as one contiguous KB per wave load.
#include "common.h"
#include "mfma_ops.h"

namespace vfl {

constexpr int LIN_WAVES = 8;   // waves splitting K
constexpr int LIN_TILE = 32;   // features and tokens per workgroup
constexpr int LIN_BATCH = 4;   // K steps whose operands are loaded together
constexpr int LIN_PIPE_BATCH = 2;  // the same when two batches are in flight
constexpr int LIN_K_MULTIPLE = 32 * LIN_WAVES;
constexpr int LIN_BLOCK = 16 * 32;  // elements of one packed 16-row x 32-k weight block

__host__ __device__ constexpr int64_t packed_rows(int64_t out_features) {
  return (out_features + LIN_TILE - 1) / LIN_TILE * LIN_TILE;
}

// One thread per 16-byte chunk of the packed weight: chunk t is lane t % 64 of block
// t / 64 = (row block r, k block c).
__global__ __launch_bounds__(256) void pack_linear_weight_kernel(
    const uint16_t *__restrict__ w, int64_t ldw, int N, int K, uint16_t *__restrict__ packed,
    int64_t chunks) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= chunks) return;
  const int l = (int)(t & 63);
  const int64_t blk = t >> 6;
  const int ks = K / 32;
  const int64_t r = blk / ks;
  const int c = (int)(blk % ks);
  const int64_t row = 16 * r + (l & 15);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row < N) v = *reinterpret_cast<const uint4 *>(w + row * ldw + 32 * c + 8 * (l >> 4));
  *reinterpret_cast<uint4 *>(packed + t * 8) = v;
}

// Element offset of (row m, column k) in a packed [rows][K] array (weight or activation).
__device__ __forceinline__ int64_t packed_offset(int m, int k, int K) {
  return ((int64_t)(m / 16) * (K / 32) + k / 32) * LIN_BLOCK + (16 * ((k % 32) / 8) + m % 16) * 8 +
         k % 8;
}

// torch's exact GELU (x / 2 * (1 + erf(x / sqrt(2)))) in fp32 on a value already rounded to
// the element type, as the separate activation kernel would see it.
template <int DT> __device__ __forceinline__ float gelu_of_stored(float v) {
  const float x = Mfma<DT>::widen(Mfma<DT>::narrow(v));
  return x * 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
}

// Deferred LayerNorm across the decoder's projections.  BART's sublayers end in
// h' = LN(h + y) (post-LN, bart.py:259-261); a separate residual + LayerNorm launch per
// sublayer costs ~5 us in a decode step's graph, more than its bytes.  Instead:
// - the sublayer's output projection (LIN_RESIDUAL) stores the pre-norm sum
//   v = round(round(acc + bias) + h) -- the value the LayerNorm kernel normalizes -- and,
//   per row and 32-feature tile, the tile's mean and sum of squared deviations;
// - the projections that read h' (LIN_NORM_IN) multiply v itself, with LayerNorm's
//   weight folded into their packed weight (W' = W diag(gamma), rounded) and its bias
//   into theirs (b' = b + W beta), and finish in the epilogue:
//   y = rstd_r (acc - mean_r u[n]) + b'[n] with u[n] = sum_k W'[n][k];
// - the residual of the next sublayer is h' itself, normalized element by element in
//   that sublayer's output projection (or by vfl_layer_norm_apply).
// A row's mean and 1/std combine its T tiles: mean = sum_t m_t / T,
// M2 = sum_t M2_t + 32 sum_t (m_t - mean)^2, rstd = 1 / sqrt(M2 / (32 T) + eps).
constexpr int LIN_PLAIN = 0, LIN_NORM_IN = 1, LIN_RESIDUAL = 2;
constexpr int LIN_STAT_TILE = 32;   // features per statistics tile

struct LinNorm {
  const float2 *x_stats;  // LIN_NORM_IN: [rows][K / 32] of x
  const float *u, *fbias; // LIN_NORM_IN: [N] fp32
  float eps;
  bool vec4;              // LIN_NORM_IN: u and fbias 16-byte aligned
  const uint16_t *res;    // LIN_RESIDUAL: h, [rows][N] with row stride res_stride
  int64_t res_stride;
  const float2 *res_stats;  // null: h is plain; else h = LN(res) with these statistics
  const uint16_t *res_gamma, *res_beta;
  float res_eps;
  float2 *y_stats;        // LIN_RESIDUAL: [rows][N / 32] of the stored v
};

// The workgroup's 32 rows' means and 1/stds from their T tiles' (mean, M2) at
// st[row * T + t]: thread (row r = tid / 16, j = tid % 16) takes tiles j, j + 16, ...;
// the 16 threads of a row (one DPP row of a wave) combine them in a fixed order.
// Requested after the main loop, so the loads' latency overlaps the partial-tile
// reduction; results in s_ms[r] = (mean, rstd) before the reduction's last barrier.
struct RowStatLoads {
  float2 p[2];
  __device__ __forceinline__ void issue(const float2 *st, int T, int m0, int M) {
    const int r = (int)(threadIdx.x >> 4), j = (int)(threadIdx.x & 15);
    const float2 *row = st + (int64_t)min(m0 + r, M - 1) * T;
    p[0] = j < T ? row[j] : make_float2(0.f, 0.f);
    p[1] = j + 16 < T ? row[j + 16] : make_float2(0.f, 0.f);
  }
  __device__ __forceinline__ void finish(const float2 *st, int T, int m0, int M, float eps,
                                         float2 *s_ms) {
    const int r = (int)(threadIdx.x >> 4), j = (int)(threadIdx.x & 15);
    const float2 *row = st + (int64_t)min(m0 + r, M - 1) * T;
    float s = p[0].x + p[1].x;
    for (int t = j + 32; t < T; t += 16) s += row[t].x;
    const float mean = group_sum<16>(s) / (float)T;
    float m2 = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (j + 16 * i < T) {
        const float d = p[i].x - mean;
        m2 += p[i].y + (float)LIN_STAT_TILE * d * d;
      }
    }
    for (int t = j + 32; t < T; t += 16) {
      const float2 v = row[t];
      const float d = v.x - mean;
      m2 += v.y + (float)LIN_STAT_TILE * d * d;
    }
    m2 = group_sum<16>(m2);
    if (j == 0) s_ms[r] = make_float2(mean, rsqrtf(m2 / (float)(LIN_STAT_TILE * T) + eps));
  }
};

template <int DT> __device__ __forceinline__ float round_elem(float v) {
  return Mfma<DT>::widen(Mfma<DT>::narrow(v));
}

// LIN_RESIDUAL's epilogue inputs and epilogue.  Finishing wave w < 2 takes token
// quarter w and both feature quarters of the tile, so each lane holds 8 of a row's 32
// tile features (4 of each quarter: n0 + 16 f + 4 (lane / 16) .. +3) and the tile row's
// statistics need only the 4 lanes of the row (rows_sum4), no LDS exchange.
struct ResidualIn {
  float b[2][4], r[2][4], g[2][4], be[2][4];  // bias, residual (or its pre-norm sum), LN's
  uint2 raw[2];                               // the residual's 8 values as loaded
  // The residual itself, requested with the operands (its 4 registers are the only ones
  // held through the products).
  __device__ __forceinline__ void issue_residual(const LinNorm &nrm, int wv, int lane, int m0,
                                                 int n0, int M) {
    if (wv >= 2) return;
    const int64_t row = min(m0 + 16 * wv + (lane & 15), M - 1);
#pragma unroll
    for (int f = 0; f < 2; ++f)  // n + 3 < N: N is a multiple of 32
      raw[f] = *reinterpret_cast<const uint2 *>(nrm.res + row * nrm.res_stride + n0 + 16 * f +
                                                4 * (lane >> 4));
  }
  template <int DT>
  __device__ __forceinline__ void issue(const uint16_t *bias, const LinNorm &nrm, int wv,
                                        int lane, int n0) {
    if (wv >= 2) return;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int n = n0 + 16 * f + 4 * (lane >> 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[f][j] = bias ? Mfma<DT>::widen(bias[n + j]) : 0.f;
      unpack4<DT>(raw[f], r[f]);
      if (nrm.res_stats) {
        unpack4<DT>(*reinterpret_cast<const uint2 *>(nrm.res_gamma + n), g[f]);
        unpack4<DT>(*reinterpret_cast<const uint2 *>(nrm.res_beta + n), be[f]);
      }
    }
  }
  template <int DT> __device__ __forceinline__ static void unpack4(uint2 w, float (&o)[4]) {
    o[0] = Mfma<DT>::widen_lo(w.x);
    o[1] = Mfma<DT>::widen_hi(w.x);
    o[2] = Mfma<DT>::widen_lo(w.y);
    o[3] = Mfma<DT>::widen_hi(w.y);
  }
};

// The values are rounded where the separate projection store and LayerNorm kernel round
// them: y, the normalized residual, v.
template <int DT>
__device__ __forceinline__ void residual_epilogue(const floatx4_t *s_part, int wv, int lane,
                                                  int m0, int n0, int M, int N,
                                                  const ResidualIn &in, const float2 *s_ms,
                                                  uint16_t *y, int64_t ldy, const LinNorm &nrm) {
  constexpr int SUB = 4, TT = 2;
  if (wv >= TT) return;
  const int r = 16 * wv + (lane & 15);  // the workgroup's row
  const int m = m0 + r;
  float mean = 0.f, rstd = 1.f;
  if (nrm.res_stats) {
    mean = s_ms[r].x;
    rstd = s_ms[r].y;
  }
  float o[2][4];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int q = f * TT + wv;  // quarter (feature quarter f, token quarter wv)
    const floatx4_t v = (s_part[q * 64 + lane] + s_part[(2 * SUB + q) * 64 + lane]) +
                        (s_part[(SUB + q) * 64 + lane] + s_part[(3 * SUB + q) * 64 + lane]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float yj = round_elem<DT>(v[j] + in.b[f][j]);
      const float hj = nrm.res_stats
                           ? round_elem<DT>((in.r[f][j] - mean) * rstd * in.g[f][j] + in.be[f][j])
                           : in.r[f][j];
      o[f][j] = round_elem<DT>(yj + hj);
    }
  }
  // The tile row's mean over the lane's 8 values and the row's 4 lanes, then the sum of
  // squared deviations from it, in a fixed order.
  const float tmean =
      rows_sum4(((o[0][0] + o[0][1]) + (o[0][2] + o[0][3])) +
                ((o[1][0] + o[1][1]) + (o[1][2] + o[1][3]))) / (float)LIN_STAT_TILE;
  float dd = 0.f;
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = o[f][j] - tmean;
      dd = fmaf(d, d, dd);
    }
  const float m2 = rows_sum4(dd);
  if (m >= M) return;
#pragma unroll
  for (int f = 0; f < 2; ++f)
    *reinterpret_cast<uint2 *>(y + (int64_t)m * ldy + n0 + 16 * f + 4 * (lane >> 4)) =
        make_uint2(Mfma<DT>::narrow2(o[f][0], o[f][1]), Mfma<DT>::narrow2(o[f][2], o[f][3]));
  if (lane < 16)
    nrm.y_stats[(int64_t)m * (N / LIN_STAT_TILE) + n0 / LIN_STAT_TILE] = make_float2(tmean, m2);
}

// XP: x is packed (no ds_bpermute); GELU: exact GELU after the bias; YP: y is written
// packed (rows padded to 32; padding rows are left unwritten); PIPE: batches of
// LIN_PIPE_BATCH steps, double-buffered (for more than LIN_BATCH steps per wave);
// MODE: LIN_PLAIN, LIN_NORM_IN (x is a pre-norm sum, nrm.x_stats its statistics) or
// LIN_RESIDUAL (y = v and nrm.y_stats, as described above).
template <int DT, bool XP, bool GELU, bool YP, bool PIPE, int MODE>
__global__ __launch_bounds__(64 * LIN_WAVES) void decode_linear_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, const uint16_t *__restrict__ wp,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y, int64_t ldy, int M, int N,
    int K, bool vec_store, LinNorm nrm) {
  static_assert(MODE != LIN_RESIDUAL || (!GELU && !YP), "the residual epilogue stores v");
  static_assert(MODE != LIN_NORM_IN || !XP, "a pre-norm x is stored row by row");
  constexpr int FT = LIN_TILE / 16, TT = LIN_TILE / 16;
  constexpr int SUB = FT * TT;  // 16 x 16 quarters of the tile
  constexpr int B = PIPE ? LIN_PIPE_BATCH : LIN_BATCH;
  // Partial tiles of four waves, each in the MFMA result order (16 bytes per lane).
  __shared__ floatx4_t s_part[(LIN_WAVES / 2) * SUB * 64];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n0 = blockIdx.x * LIN_TILE, m0 = blockIdx.y * LIN_TILE;
  const int ks = K / 32;
  const int kq = K / LIN_WAVES;  // this wave's K range: [wv * kq, (wv + 1) * kq)
  const int kb = wv * kq;
  // byte address of the lane whose 64-byte run holds this lane's operand chunk
  const int src = 4 * (4 * (lane & 15) + (lane >> 4));

  // Packed weight blocks of this wave's first K step; activation runs (rows past M read
  // the last row; their results are dropped).
  const uint16_t *wblk[FT];
  const uint16_t *xrow[TT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
    wblk[f] = wp + ((int64_t)(n0 / 16 + f) * ks + kb / 32) * LIN_BLOCK + lane * 8;
#pragma unroll
  for (int t = 0; t < TT; ++t)
    xrow[t] = XP ? x + ((int64_t)(m0 / 16 + t) * ks + kb / 32) * LIN_BLOCK + lane * 8
                 : x + (int64_t)min(m0 + 16 * t + (lane >> 2), M - 1) * ldx + kb +
                       8 * (lane & 3);
  constexpr int XSTEP = XP ? LIN_BLOCK : 32;

  // Wave q < SUB finishes quarter q of the tile: features 16 (q / TT) + 4 (lane / 16) .. +3
  // of token 16 (q % TT) + lane % 16.  Its bias is requested now, with the operands, so
  // that no load is left for after the reduction.
  static_assert(SUB <= LIN_WAVES, "one quarter per finishing wave");
  const int qf = wv / TT, qt = wv % TT;
  const int qn = n0 + 16 * qf + 4 * (lane >> 4);
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (bias && wv < SUB && MODE == LIN_PLAIN) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bv[j] = qn + j < N ? Mfma<DT>::widen(bias[qn + j]) : 0.f;
  }
  // The epilogue inputs requested before the operands so that they have landed when
  // the products have (loads complete in order): the rows' tile statistics (two per
  // thread) and, for LIN_NORM_IN's finishing lanes (features qn .. qn + 3), u and b'.
  __shared__ float2 s_ms[MODE == LIN_PLAIN ? 1 : LIN_TILE];
  RowStatLoads rsl;
  const float2 *row_st = nullptr;
  int row_t = 0;
  float fa[4] = {0.f, 0.f, 0.f, 0.f}, fb[4] = {0.f, 0.f, 0.f, 0.f};  // LIN_NORM_IN: u, b'
  if constexpr (MODE == LIN_NORM_IN) {
    row_st = nrm.x_stats;
    row_t = K / LIN_STAT_TILE;
    if (wv < SUB) {
      if (qn + 3 < N && nrm.vec4) {  // one 16-byte load each
        const float4 a = *reinterpret_cast<const float4 *>(nrm.u + qn);
        const float4 b = *reinterpret_cast<const float4 *>(nrm.fbias + qn);
        fa[0] = a.x, fa[1] = a.y, fa[2] = a.z, fa[3] = a.w;
        fb[0] = b.x, fb[1] = b.y, fb[2] = b.z, fb[3] = b.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          fa[j] = qn + j < N ? nrm.u[qn + j] : 0.f;
          fb[j] = qn + j < N ? nrm.fbias[qn + j] : 0.f;
        }
      }
    }
  }
  if constexpr (MODE == LIN_RESIDUAL) {
    row_st = nrm.res_stats;  // null: a plain residual
    row_t = N / LIN_STAT_TILE;
  }
  if (MODE != LIN_PLAIN && row_st) rsl.issue(row_st, row_t, m0, M);
  // The residual too, for one batch of K steps (a 1024-deep output projection: 6.2
  // against 6.3 us); a longer, double-buffered K loop ran 0.1 us slower with it here.
  ResidualIn rin;
  if constexpr (MODE == LIN_RESIDUAL && !PIPE) rin.issue_residual(nrm, wv, lane, m0, n0, M);

  floatx4_t acc[FT][TT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[f][t] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  const int steps = kq / 32;
  auto load = [&](uint4 (&a)[B][FT], uint4 (&b)[B][TT], int s0) {
#pragma unroll
    for (int g = 0; g < B; ++g) {
      if (s0 + g < steps) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
          a[g][f] = *reinterpret_cast<const uint4 *>(wblk[f] + LIN_BLOCK * (s0 + g));
#pragma unroll
        for (int t = 0; t < TT; ++t)
          b[g][t] = *reinterpret_cast<const uint4 *>(xrow[t] + XSTEP * (s0 + g));
      }
    }
  };
  auto multiply = [&](uint4 (&a)[B][FT], uint4 (&b)[B][TT], int s0) {
#pragma unroll
    for (int g = 0; g < B; ++g) {
      if (s0 + g < steps) {
#pragma unroll
        for (int t = 0; t < TT && !XP; ++t) {
          b[g][t].x = __builtin_amdgcn_ds_bpermute(src, (int)b[g][t].x);
          b[g][t].y = __builtin_amdgcn_ds_bpermute(src, (int)b[g][t].y);
          b[g][t].z = __builtin_amdgcn_ds_bpermute(src, (int)b[g][t].z);
          b[g][t].w = __builtin_amdgcn_ds_bpermute(src, (int)b[g][t].w);
        }
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
          for (int t = 0; t < TT; ++t) acc[f][t] = Mfma<DT>::qk(a[g][f], b[g][t], acc[f][t]);
      }
    }
  };
  if constexpr (PIPE) {
    uint4 a0[B][FT], b0[B][TT], a1[B][FT], b1[B][TT];
    load(a0, b0, 0);
    for (int s0 = 0; s0 < steps; s0 += 2 * B) {
      if (s0 + B < steps) load(a1, b1, s0 + B);
      multiply(a0, b0, s0);
      if (s0 + 2 * B < steps) load(a0, b0, s0 + 2 * B);
      if (s0 + B < steps) multiply(a1, b1, s0 + B);
    }
  } else {
    for (int s0 = 0; s0 < steps; s0 += B) {
      uint4 a[B][FT], b[B][TT];
      load(a, b, s0);
      multiply(a, b, s0);
    }
  }

  // LIN_RESIDUAL's per-feature inputs, requested now so that they overlap the reduction
  // below (with them before the operands, a 1024-wide output projection ran 0.3 us
  // slower).
  if constexpr (MODE == LIN_RESIDUAL) {
    if constexpr (PIPE) rin.issue_residual(nrm, wv, lane, m0, n0, M);
    rin.issue<DT>(bias, nrm, wv, lane, n0);
  }

  // Sum the waves' partial tiles: waves 4..7 hand theirs to waves 0..3, which add and
  // publish the four sums.
  if (wv >= LIN_WAVES / 2) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int t = 0; t < TT; ++t)
        s_part[((wv - LIN_WAVES / 2) * SUB + f * TT + t) * 64 + lane] = acc[f][t];
  }
  __syncthreads();
  if (wv < LIN_WAVES / 2) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[f][t] += s_part[(wv * SUB + f * TT + t) * 64 + lane];
  }
  __syncthreads();
  if (wv < LIN_WAVES / 2) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int t = 0; t < TT; ++t) s_part[(wv * SUB + f * TT + t) * 64 + lane] = acc[f][t];
  }
  if (MODE != LIN_PLAIN && row_st)
    rsl.finish(row_st, row_t, m0, M, MODE == LIN_NORM_IN ? nrm.eps : nrm.res_eps, s_ms);
  __syncthreads();

  const int m = m0 + 16 * qt + (lane & 15);
  if constexpr (MODE == LIN_RESIDUAL) {
    residual_epilogue<DT>(s_part, wv, lane, m0, n0, M, N, rin, s_ms, y, ldy, nrm);
    return;
  }
  if (wv >= SUB) return;
  if (qn >= N || m >= M) return;
  const floatx4_t v = (s_part[wv * 64 + lane] + s_part[(2 * SUB + wv) * 64 + lane]) +
                      (s_part[(SUB + wv) * 64 + lane] + s_part[(3 * SUB + wv) * 64 + lane]);
  float mean = 0.f, rstd = 1.f;
  if constexpr (MODE == LIN_NORM_IN) {
    const float2 ms = s_ms[16 * qt + (lane & 15)];
    mean = ms.x;
    rstd = ms.y;
  }
  uint32_t h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float o = MODE == LIN_NORM_IN ? fmaf(fmaf(-mean, fa[j], v[j]), rstd, fb[j])
                                        : v[j] + bv[j];
    h[j] = Mfma<DT>::narrow(GELU ? gelu_of_stored<DT>(o) : o);
  }
  if constexpr (YP) {  // 4 consecutive columns of one row: 8 bytes of one lane's chunk
    *reinterpret_cast<uint2 *>(y + packed_offset(m, qn, N)) =
        make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    return;
  }
  uint16_t *dst = y + (int64_t)m * ldy + qn;
  if (vec_store && qn + 3 < N) {
    *reinterpret_cast<uint2 *>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (qn + j < N) dst[j] = (uint16_t)h[j];
  }
}

static int check_features(int out_features, int in_features, int dtype, const char *who) {
  if (dtype != VFL_BFLOAT16 && dtype != VFL_FLOAT16) {
    set_error("%s: dtype %d has no kernel (bf16 and fp16 only)", who, dtype);
    return VFL_E_UNSUPPORTED;
  }
  if (out_features <= 0 || in_features <= 0) {
    set_error("%s: bad sizes (out %d in %d)", who, out_features, in_features);
    return VFL_E_INVALID;
  }
  if (in_features % LIN_K_MULTIPLE != 0) {
    set_error("%s: in_features must be a multiple of %d (got %d)", who, LIN_K_MULTIPLE,
              in_features);
    return VFL_E_UNSUPPORTED;
  }
  return VFL_OK;
}

}  // namespace vfl

using namespace vfl;

extern "C" int64_t vfl_linear_packed_elems(int rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return packed_rows(rows) * cols;
}

extern "C" int vfl_pack_linear_weight(const void *weight, int64_t weight_stride,
                                      int out_features, int in_features, void *packed,
                                      int dtype, void *stream) {
  clear_error();
  int st = check_features(out_features, in_features, dtype, "pack_linear_weight");
  if (st != VFL_OK) return st;
  if (weight_stride < in_features) {
    set_error("pack_linear_weight: weight_stride %lld < in_features %d",
              (long long)weight_stride, in_features);
    return VFL_E_INVALID;
  }
  if (!weight || !packed) {
    set_error("pack_linear_weight: null pointer argument");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)weight | (uintptr_t)packed) % 16 != 0 || weight_stride % 8 != 0) {
    set_error("pack_linear_weight: weight and packed must be 16-byte aligned, the weight "
              "row stride a multiple of 8 elements");
    return VFL_E_INVALID;
  }
  const int64_t chunks = packed_rows(out_features) * in_features / 8;
  pack_linear_weight_kernel<<<dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                              (hipStream_t)stream>>>(
      (const uint16_t *)weight, weight_stride, out_features, in_features, (uint16_t *)packed,
      chunks);
  return launch_status("pack_linear_weight");
}

template <bool XP, bool GELU, bool YP, bool PIPE, int MODE>
static void launch_linear_dt(const dim3 &grid, hipStream_t s, int dtype, const void *x,
                             int64_t x_stride, const void *wp, const void *bias, void *y,
                             int64_t y_stride, int64_t rows, int out_features, int in_features,
                             bool vec_store, const LinNorm &nrm) {
  if (dtype == VFL_BFLOAT16)
    decode_linear_kernel<VFL_BFLOAT16, XP, GELU, YP, PIPE, MODE>
        <<<grid, dim3(64 * LIN_WAVES), 0, s>>>(
        (const uint16_t *)x, x_stride, (const uint16_t *)wp, (const uint16_t *)bias,
        (uint16_t *)y, y_stride, (int)rows, out_features, in_features, vec_store, nrm);
  else
    decode_linear_kernel<VFL_FLOAT16, XP, GELU, YP, PIPE, MODE>
        <<<grid, dim3(64 * LIN_WAVES), 0, s>>>(
        (const uint16_t *)x, x_stride, (const uint16_t *)wp, (const uint16_t *)bias,
        (uint16_t *)y, y_stride, (int)rows, out_features, in_features, vec_store, nrm);
}

// More K steps per wave than one batch holds: double-buffered batches.
template <bool XP, bool GELU, bool YP, int MODE = LIN_PLAIN>
static void launch_linear(const dim3 &grid, hipStream_t s, int dtype, const void *x,
                          int64_t x_stride, const void *wp, const void *bias, void *y,
                          int64_t y_stride, int64_t rows, int out_features, int in_features,
                          bool vec_store, const LinNorm &nrm = LinNorm{}) {
  if (in_features / LIN_WAVES / 32 > LIN_BATCH)
    launch_linear_dt<XP, GELU, YP, true, MODE>(grid, s, dtype, x, x_stride, wp, bias, y,
                                               y_stride, rows, out_features, in_features,
                                               vec_store, nrm);
  else
    launch_linear_dt<XP, GELU, YP, false, MODE>(grid, s, dtype, x, x_stride, wp, bias, y,
                                                y_stride, rows, out_features, in_features,
                                                vec_store, nrm);
}

extern "C" int vfl_linear(const void *x, int64_t x_stride, const void *packed_weight,
                          const void *bias, void *y, int64_t y_stride, int64_t rows,
                          int out_features, int in_features, int flags, int dtype,
                          void *stream) {
  clear_error();
  int st = check_features(out_features, in_features, dtype, "linear");
  if (st != VFL_OK) return st;
  if (rows < 0 || rows > 65535LL * LIN_TILE) {
    set_error("linear: rows must be in [0, %lld] (got %lld)", 65535LL * LIN_TILE,
              (long long)rows);
    return rows < 0 ? VFL_E_INVALID : VFL_E_UNSUPPORTED;
  }
  if (flags & ~(VFL_LINEAR_GELU | VFL_LINEAR_X_PACKED | VFL_LINEAR_Y_PACKED)) {
    set_error("linear: unknown flags 0x%x", flags);
    return VFL_E_INVALID;
  }
  const bool xp = flags & VFL_LINEAR_X_PACKED, yp = flags & VFL_LINEAR_Y_PACKED;
  if ((!xp && x_stride < in_features) || (!yp && y_stride < out_features)) {
    set_error("linear: row strides must cover the rows (x %lld y %lld)", (long long)x_stride,
              (long long)y_stride);
    return VFL_E_INVALID;
  }
  if (yp && out_features % LIN_TILE != 0) {
    set_error("linear: a packed output needs out_features a multiple of %d (got %d)", LIN_TILE,
              out_features);
    return VFL_E_UNSUPPORTED;
  }
  if (rows == 0) return VFL_OK;
  if (!x || !packed_weight || !y) {
    set_error("linear: null pointer argument");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)x | (uintptr_t)packed_weight) % 16 != 0 || (!xp && x_stride % 8 != 0) ||
      (uintptr_t)y % (yp ? 8 : 2) != 0 || (uintptr_t)bias % 2 != 0) {
    set_error("linear: x and the packed weight must be 16-byte aligned, the x row stride a "
              "multiple of 8 elements");
    return VFL_E_INVALID;
  }
  const bool vec_store = (uintptr_t)y % 8 == 0 && y_stride % 4 == 0;
  const dim3 grid((unsigned)(packed_rows(out_features) / LIN_TILE),
                  (unsigned)((rows + LIN_TILE - 1) / LIN_TILE));
  hipStream_t s = (hipStream_t)stream;
  const bool gelu = flags & VFL_LINEAR_GELU;
#define VFL_LIN(XP, G, YP)                                                                   \
  launch_linear<XP, G, YP>(grid, s, dtype, x, x_stride, packed_weight, bias, y, y_stride, rows, \
                           out_features, in_features, vec_store)
  if (!xp && !gelu && !yp)
    VFL_LIN(false, false, false);
  else if (!xp && gelu && yp)
    VFL_LIN(false, true, true);
  else if (xp && !gelu && !yp)
    VFL_LIN(true, false, false);
  else if (!xp && gelu && !yp)
    VFL_LIN(false, true, false);
  else if (!xp && !gelu && yp)
    VFL_LIN(false, false, true);
  else if (xp && gelu && !yp)
    VFL_LIN(true, true, false);
  else if (xp && !gelu && yp)
    VFL_LIN(true, false, true);
  else
    VFL_LIN(true, true, true);
#undef VFL_LIN
  return launch_status("linear");
}

namespace vfl {

// h = LN(v) from v's tile statistics (the last sublayer's output before the LM head):
// one wave per row, the row's tiles combined in a fixed order, then the LayerNorm
// kernel's expression per element.
template <int DT>
__global__ __launch_bounds__(128) void layer_norm_apply_kernel(
    const uint16_t *__restrict__ v, int64_t v_stride, const float2 *__restrict__ st,
    const uint16_t *__restrict__ gamma, const uint16_t *__restrict__ beta, float eps,
    uint16_t *__restrict__ out, int64_t out_stride, int64_t rows, int dim) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int T = dim / LIN_STAT_TILE;
  const float2 *rs = st + row * T;
  float s = 0.f;
  for (int t = lane; t < T; t += 64) s += rs[t].x;
  const float mean = group_sum<64>(s) / (float)T;
  float m2 = 0.f;
  for (int t = lane; t < T; t += 64) {
    const float2 p = rs[t];
    const float d = p.x - mean;
    m2 += p.y + (float)LIN_STAT_TILE * d * d;
  }
  const float rstd = rsqrtf(group_sum<64>(m2) / (float)dim + eps);
  for (int i = 4 * lane; i < dim; i += 256) {
    const uint2 a = *reinterpret_cast<const uint2 *>(v + row * v_stride + i);
    const uint2 g = *reinterpret_cast<const uint2 *>(gamma + i);
    const uint2 b = *reinterpret_cast<const uint2 *>(beta + i);
    const uint32_t aw[2] = {a.x, a.y}, gw[2] = {g.x, g.y}, bw[2] = {b.x, b.y};
    uint32_t o[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const float lo = (Mfma<DT>::widen_lo(aw[w]) - mean) * rstd * Mfma<DT>::widen_lo(gw[w]) +
                       Mfma<DT>::widen_lo(bw[w]);
      const float hi = (Mfma<DT>::widen_hi(aw[w]) - mean) * rstd * Mfma<DT>::widen_hi(gw[w]) +
                       Mfma<DT>::widen_hi(bw[w]);
      o[w] = Mfma<DT>::narrow2(lo, hi);
    }
    *reinterpret_cast<uint2 *>(out + row * out_stride + i) = make_uint2(o[0], o[1]);
  }
}

}  // namespace vfl

static int check_norm_rows(int64_t rows, const char *who) {
  if (rows < 0 || rows > 65535LL * LIN_TILE) {
    set_error("%s: rows must be in [0, %lld] (got %lld)", who, 65535LL * LIN_TILE,
              (long long)rows);
    return rows < 0 ? VFL_E_INVALID : VFL_E_UNSUPPORTED;
  }
  return VFL_OK;
}

extern "C" int vfl_linear_norm(const void *x, int64_t x_stride, const float *x_stats, float eps,
                               const void *packed_weight, const float *u,
                               const float *folded_bias, void *y, int64_t y_stride,
                               int64_t rows, int out_features, int in_features, int flags,
                               int dtype, void *stream) {
  clear_error();
  int st = check_features(out_features, in_features, dtype, "linear_norm");
  if (st == VFL_OK) st = check_norm_rows(rows, "linear_norm");
  if (st != VFL_OK) return st;
  if (flags & ~(VFL_LINEAR_GELU | VFL_LINEAR_Y_PACKED)) {
    set_error("linear_norm: flags 0x%x (GELU and Y_PACKED only: x is a pre-norm sum)", flags);
    return VFL_E_INVALID;
  }
  const bool yp = flags & VFL_LINEAR_Y_PACKED, gelu = flags & VFL_LINEAR_GELU;
  if (x_stride < in_features || (!yp && y_stride < out_features) || !(eps >= 0.f)) {
    set_error("linear_norm: row strides must cover the rows (x %lld y %lld), eps >= 0",
              (long long)x_stride, (long long)y_stride);
    return VFL_E_INVALID;
  }
  if (yp && out_features % LIN_TILE != 0) {
    set_error("linear_norm: a packed output needs out_features a multiple of %d (got %d)",
              LIN_TILE, out_features);
    return VFL_E_UNSUPPORTED;
  }
  if (rows == 0) return VFL_OK;
  if (!x || !x_stats || !packed_weight || !u || !folded_bias || !y) {
    set_error("linear_norm: null pointer argument");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)x | (uintptr_t)packed_weight) % 16 != 0 || x_stride % 8 != 0 ||
      (uintptr_t)x_stats % 8 != 0 || ((uintptr_t)u | (uintptr_t)folded_bias) % 4 != 0 ||
      (uintptr_t)y % (yp ? 8 : 2) != 0) {
    set_error("linear_norm: x and the packed weight must be 16-byte aligned, the x row stride "
              "a multiple of 8 elements, x_stats 8-byte and u / folded_bias 4-byte aligned");
    return VFL_E_INVALID;
  }
  LinNorm nrm{};
  nrm.x_stats = reinterpret_cast<const float2 *>(x_stats);
  nrm.u = u;
  nrm.fbias = folded_bias;
  nrm.eps = eps;
  nrm.vec4 = ((uintptr_t)u | (uintptr_t)folded_bias) % 16 == 0;
  const bool vec_store = (uintptr_t)y % 8 == 0 && y_stride % 4 == 0;
  const dim3 grid((unsigned)(packed_rows(out_features) / LIN_TILE),
                  (unsigned)((rows + LIN_TILE - 1) / LIN_TILE));
  hipStream_t s = (hipStream_t)stream;
#define VFL_LINN(G, YP)                                                                   \
  launch_linear<false, G, YP, LIN_NORM_IN>(grid, s, dtype, x, x_stride, packed_weight, nullptr, \
                                           y, y_stride, rows, out_features, in_features,     \
                                           vec_store, nrm)
  if (!gelu && !yp)
    VFL_LINN(false, false);
  else if (gelu && yp)
    VFL_LINN(true, true);
  else if (gelu)
    VFL_LINN(true, false);
  else
    VFL_LINN(false, true);
#undef VFL_LINN
  return launch_status("linear_norm");
}

extern "C" int vfl_linear_residual(const void *x, int64_t x_stride, const void *packed_weight,
                                   const void *bias, const void *residual, int64_t r_stride,
                                   const float *r_stats, const void *r_gamma,
                                   const void *r_beta, float r_eps, void *y, int64_t y_stride,
                                   float *y_stats, int64_t rows, int out_features,
                                   int in_features, int flags, int dtype, void *stream) {
  clear_error();
  int st = check_features(out_features, in_features, dtype, "linear_residual");
  if (st == VFL_OK) st = check_norm_rows(rows, "linear_residual");
  if (st != VFL_OK) return st;
  if (flags & ~VFL_LINEAR_X_PACKED) {
    set_error("linear_residual: flags 0x%x (X_PACKED only: y is the pre-norm sum)", flags);
    return VFL_E_INVALID;
  }
  const bool xp = flags & VFL_LINEAR_X_PACKED;
  if (out_features % LIN_STAT_TILE != 0) {
    set_error("linear_residual: out_features must be a multiple of %d (got %d)", LIN_STAT_TILE,
              out_features);
    return VFL_E_UNSUPPORTED;
  }
  if ((!xp && x_stride < in_features) || y_stride < out_features || r_stride < out_features ||
      (r_stats && !(r_eps >= 0.f))) {
    set_error("linear_residual: row strides must cover the rows (x %lld y %lld residual %lld)",
              (long long)x_stride, (long long)y_stride, (long long)r_stride);
    return VFL_E_INVALID;
  }
  if (rows == 0) return VFL_OK;
  if (!x || !packed_weight || !residual || !y || !y_stats ||
      (r_stats && (!r_gamma || !r_beta))) {
    set_error("linear_residual: null pointer argument");
    return VFL_E_INVALID;
  }
  if ((const void *)y_stats == (const void *)r_stats) {
    set_error("linear_residual: y_stats must not alias r_stats (every workgroup of a row "
              "reads the residual's statistics)");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)x | (uintptr_t)packed_weight) % 16 != 0 || (!xp && x_stride % 8 != 0) ||
      (uintptr_t)y % 8 != 0 || y_stride % 4 != 0 || (uintptr_t)bias % 2 != 0 ||
      (uintptr_t)residual % 8 != 0 || r_stride % 4 != 0 ||
      ((uintptr_t)y_stats | (uintptr_t)r_stats) % 8 != 0 ||
      ((uintptr_t)r_gamma | (uintptr_t)r_beta) % 8 != 0) {
    set_error("linear_residual: x and the packed weight must be 16-byte aligned (x row "
              "stride a multiple of 8 elements), y and the residual 8-byte aligned with row "
              "strides multiples of 4, gamma / beta and the statistics 8-byte aligned");
    return VFL_E_INVALID;
  }
  LinNorm nrm{};
  nrm.res = (const uint16_t *)residual;
  nrm.res_stride = r_stride;
  nrm.res_stats = reinterpret_cast<const float2 *>(r_stats);
  nrm.res_gamma = (const uint16_t *)r_gamma;
  nrm.res_beta = (const uint16_t *)r_beta;
  nrm.res_eps = r_eps;
  nrm.y_stats = reinterpret_cast<float2 *>(y_stats);
  const dim3 grid((unsigned)(out_features / LIN_TILE),
                  (unsigned)((rows + LIN_TILE - 1) / LIN_TILE));
  hipStream_t s = (hipStream_t)stream;
  if (xp)
    launch_linear<true, false, false, LIN_RESIDUAL>(grid, s, dtype, x, 0, packed_weight, bias, y,
                                                    y_stride, rows, out_features, in_features,
                                                    true, nrm);
  else
    launch_linear<false, false, false, LIN_RESIDUAL>(grid, s, dtype, x, x_stride, packed_weight,
                                                     bias, y, y_stride, rows, out_features,
                                                     in_features, true, nrm);
  return launch_status("linear_residual");
}

extern "C" int vfl_layer_norm_apply(const void *v, int64_t v_stride, const float *v_stats,
                                    const void *gamma, const void *beta, float eps, void *out,
                                    int64_t out_stride, int64_t rows, int dim, int dtype,
                                    void *stream) {
  clear_error();
  if (dtype != VFL_BFLOAT16 && dtype != VFL_FLOAT16) {
    set_error("layer_norm_apply: dtype %d has no kernel (bf16 and fp16 only)", dtype);
    return VFL_E_UNSUPPORTED;
  }
  if (rows < 0 || dim <= 0 || dim % LIN_STAT_TILE != 0 || v_stride < dim ||
      out_stride < dim || !(eps >= 0.f)) {
    set_error("layer_norm_apply: bad sizes (rows %lld dim %d, a multiple of %d; strides "
              "covering dim; eps >= 0)", (long long)rows, dim, LIN_STAT_TILE);
    return VFL_E_INVALID;
  }
  if (rows == 0) return VFL_OK;
  if (rows > 2LL * 2147483647LL) {
    set_error("layer_norm_apply: too many rows");
    return VFL_E_UNSUPPORTED;
  }
  if (!v || !v_stats || !gamma || !beta || !out) {
    set_error("layer_norm_apply: null pointer argument");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)v | (uintptr_t)out | (uintptr_t)gamma | (uintptr_t)beta |
       (uintptr_t)v_stats) % 8 != 0 || v_stride % 4 != 0 || out_stride % 4 != 0) {
    set_error("layer_norm_apply: v, out, gamma, beta and v_stats must be 8-byte aligned and "
              "the row strides multiples of 4 elements");
    return VFL_E_INVALID;
  }
  const dim3 grid((unsigned)((rows + 1) / 2));
  hipStream_t s = (hipStream_t)stream;
  const float2 *st = reinterpret_cast<const float2 *>(v_stats);
  if (dtype == VFL_BFLOAT16)
    layer_norm_apply_kernel<VFL_BFLOAT16><<<grid, dim3(128), 0, s>>>(
        (const uint16_t *)v, v_stride, st, (const uint16_t *)gamma, (const uint16_t *)beta, eps,
        (uint16_t *)out, out_stride, rows, dim);
  else
    layer_norm_apply_kernel<VFL_FLOAT16><<<grid, dim3(128), 0, s>>>(
        (const uint16_t *)v, v_stride, st, (const uint16_t *)gamma, (const uint16_t *)beta, eps,
        (uint16_t *)out, out_stride, rows, dim);
  return launch_status("layer_norm_apply");
}
