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

// XP: x is packed (no ds_bpermute); GELU: exact GELU after the bias; YP: y is written
// packed (rows padded to 32; padding rows are left unwritten); PIPE: batches of
// LIN_PIPE_BATCH steps, double-buffered (for more than LIN_BATCH steps per wave).
template <int DT, bool XP, bool GELU, bool YP, bool PIPE>
__global__ __launch_bounds__(64 * LIN_WAVES) void decode_linear_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, const uint16_t *__restrict__ wp,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y, int64_t ldy, int M, int N,
    int K, bool vec_store) {
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
  if (bias && wv < SUB) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bv[j] = qn + j < N ? Mfma<DT>::widen(bias[qn + j]) : 0.f;
  }

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
  __syncthreads();

  if (wv >= SUB) return;
  const int m = m0 + 16 * qt + (lane & 15);
  if (qn >= N || m >= M) return;
  const floatx4_t v = (s_part[wv * 64 + lane] + s_part[(2 * SUB + wv) * 64 + lane]) +
                      (s_part[(SUB + wv) * 64 + lane] + s_part[(3 * SUB + wv) * 64 + lane]);
  uint32_t h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float o = v[j] + bv[j];
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

template <bool XP, bool GELU, bool YP, bool PIPE>
static void launch_linear_dt(const dim3 &grid, hipStream_t s, int dtype, const void *x,
                             int64_t x_stride, const void *wp, const void *bias, void *y,
                             int64_t y_stride, int64_t rows, int out_features, int in_features,
                             bool vec_store) {
  if (dtype == VFL_BFLOAT16)
    decode_linear_kernel<VFL_BFLOAT16, XP, GELU, YP, PIPE><<<grid, dim3(64 * LIN_WAVES), 0, s>>>(
        (const uint16_t *)x, x_stride, (const uint16_t *)wp, (const uint16_t *)bias,
        (uint16_t *)y, y_stride, (int)rows, out_features, in_features, vec_store);
  else
    decode_linear_kernel<VFL_FLOAT16, XP, GELU, YP, PIPE><<<grid, dim3(64 * LIN_WAVES), 0, s>>>(
        (const uint16_t *)x, x_stride, (const uint16_t *)wp, (const uint16_t *)bias,
        (uint16_t *)y, y_stride, (int)rows, out_features, in_features, vec_store);
}

// More K steps per wave than one batch holds: double-buffered batches.
template <bool XP, bool GELU, bool YP>
static void launch_linear(const dim3 &grid, hipStream_t s, int dtype, const void *x,
                          int64_t x_stride, const void *wp, const void *bias, void *y,
                          int64_t y_stride, int64_t rows, int out_features, int in_features,
                          bool vec_store) {
  if (in_features / LIN_WAVES / 32 > LIN_BATCH)
    launch_linear_dt<XP, GELU, YP, true>(grid, s, dtype, x, x_stride, wp, bias, y, y_stride,
                                         rows, out_features, in_features, vec_store);
  else
    launch_linear_dt<XP, GELU, YP, false>(grid, s, dtype, x, x_stride, wp, bias, y, y_stride,
                                          rows, out_features, in_features, vec_store);
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
