// Decode-step linear layer on the matrix cores (gfx950), 16-bit inputs and output,
// fp32 sums:
//
//   y[m][n] = sum_k x[m][k] * w[n][k] + bias[n]        (w: nn.Linear's [out, in])
//
// for the few hundred token rows of a decode step times a weight of up to 1024 x 1024
// (the decoder's attention output and cross-attention query projections,
// vflorence/models/bart.py:114,142,146).  Each step streams the weight from HBM
// once (a decoder's weights exceed the last-level cache), so the time goes to
// memory round trips, not arithmetic: a GEMM that walks K in a loop pays one round
// trip per K step.  Here a workgroup
// owns a 32-feature x 32-token output tile and splits K over its 8 waves.  Each wave
// loads the operands of up to 4 K steps of 32 in one batch (16-byte chunks straight
// into the MFMA operand registers, no LDS staging), so K <= 1024 costs one round
// trip.  The waves' partial tiles are summed through LDS in a 3-level tree, and wave
// 0 adds the bias and stores.
//
// Product per 32-wide K step (mfma_f32_16x16x32): A = 16 weight rows (features),
// B = 16 token rows, D[feature][token]; a lane's four D registers are four consecutive
// features of one token -- one 8-byte store.
#include "common.h"
#include "mfma_ops.h"

namespace vfl {

constexpr int LIN_WAVES = 8;   // waves splitting K
constexpr int LIN_TILE = 32;   // features and tokens per workgroup
constexpr int LIN_BATCH = 4;   // K steps whose operands are loaded together
constexpr int LIN_K_MULTIPLE = 32 * LIN_WAVES;
constexpr int LIN_MAX_DIM = 1024;

template <int DT>
__global__ __launch_bounds__(64 * LIN_WAVES) void decode_linear_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, const uint16_t *__restrict__ w, int64_t ldw,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y, int64_t ldy, int M, int N,
    int K, bool vec_store) {
  constexpr int FT = LIN_TILE / 16, TT = LIN_TILE / 16;
  constexpr int ROW = LIN_TILE + 4;  // LDS floats per token row of a partial tile
  __shared__ float s_part[(LIN_WAVES / 2) * LIN_TILE * ROW];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n0 = blockIdx.x * LIN_TILE, m0 = blockIdx.y * LIN_TILE;
  const int kq = K / LIN_WAVES;  // this wave's K range: [wv * kq, (wv + 1) * kq)
  const int kb = wv * kq;
  const int col = lane & 15, chunk = 8 * (lane >> 4);

  // Operand rows; rows past M / N read the last row and their results are dropped.
  const uint16_t *wrow[FT];
  const uint16_t *xrow[TT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
    wrow[f] = w + (int64_t)min(n0 + 16 * f + col, N - 1) * ldw + kb + chunk;
#pragma unroll
  for (int t = 0; t < TT; ++t)
    xrow[t] = x + (int64_t)min(m0 + 16 * t + col, M - 1) * ldx + kb + chunk;

  floatx4_t acc[FT][TT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[f][t] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  const int steps = kq / 32;
  for (int s0 = 0; s0 < steps; s0 += LIN_BATCH) {
    uint4 a[LIN_BATCH][FT], b[LIN_BATCH][TT];
#pragma unroll
    for (int g = 0; g < LIN_BATCH; ++g) {
      if (s0 + g < steps) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
          a[g][f] = *reinterpret_cast<const uint4 *>(wrow[f] + 32 * (s0 + g));
#pragma unroll
        for (int t = 0; t < TT; ++t)
          b[g][t] = *reinterpret_cast<const uint4 *>(xrow[t] + 32 * (s0 + g));
      }
    }
#pragma unroll
    for (int g = 0; g < LIN_BATCH; ++g) {
      if (s0 + g < steps) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
          for (int t = 0; t < TT; ++t) acc[f][t] = Mfma<DT>::qk(a[g][f], b[g][t], acc[f][t]);
      }
    }
  }

  // Sum the waves' partial tiles: at each level the upper half writes, the lower half adds.
#pragma unroll
  for (int half = LIN_WAVES / 2; half >= 1; half /= 2) {
    if (wv >= half && wv < 2 * half) {
      float *slot = s_part + (wv - half) * LIN_TILE * ROW;
#pragma unroll
      for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int t = 0; t < TT; ++t)
          *reinterpret_cast<floatx4_t *>(slot + (16 * t + col) * ROW + 16 * f +
                                         4 * (lane >> 4)) = acc[f][t];
    }
    __syncthreads();
    if (wv < half) {
      const float *slot = s_part + wv * LIN_TILE * ROW;
#pragma unroll
      for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int t = 0; t < TT; ++t)
          acc[f][t] += *reinterpret_cast<const floatx4_t *>(slot + (16 * t + col) * ROW +
                                                             16 * f + 4 * (lane >> 4));
    }
    __syncthreads();
  }
  if (wv != 0) return;

#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int n = n0 + 16 * f + 4 * (lane >> 4);
    if (n >= N) continue;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = n + j < N ? Mfma<DT>::widen(bias[n + j]) : 0.f;
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int m = m0 + 16 * t + col;
      if (m >= M) continue;
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = Mfma<DT>::narrow(acc[f][t][j] + bv[j]);
      uint16_t *dst = y + (int64_t)m * ldy + n;
      if (vec_store && n + 3 < N) {
        *reinterpret_cast<uint2 *>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (n + j < N) dst[j] = (uint16_t)h[j];
      }
    }
  }
}

}  // namespace vfl

using namespace vfl;

extern "C" int vfl_linear(const void *x, int64_t x_stride, const void *weight,
                          int64_t weight_stride, const void *bias, void *y, int64_t y_stride,
                          int64_t rows, int out_features, int in_features, int dtype,
                          void *stream) {
  clear_error();
  if (dtype != VFL_BFLOAT16 && dtype != VFL_FLOAT16) {
    set_error("linear: dtype %d has no kernel (bf16 and fp16 only)", dtype);
    return VFL_E_UNSUPPORTED;
  }
  if (rows < 0 || out_features <= 0 || in_features <= 0) {
    set_error("linear: bad sizes (rows %lld out %d in %d)", (long long)rows, out_features,
              in_features);
    return VFL_E_INVALID;
  }
  if (in_features % LIN_K_MULTIPLE != 0 || in_features > LIN_MAX_DIM ||
      out_features > LIN_MAX_DIM) {
    set_error("linear: in_features must be a multiple of %d and both feature counts at most "
              "%d (got out %d in %d)",
              LIN_K_MULTIPLE, LIN_MAX_DIM, out_features, in_features);
    return VFL_E_UNSUPPORTED;
  }
  if (rows > 65535LL * LIN_TILE) {
    set_error("linear: at most %lld rows per call (got %lld)", 65535LL * LIN_TILE,
              (long long)rows);
    return VFL_E_UNSUPPORTED;
  }
  if (x_stride < in_features || weight_stride < in_features || y_stride < out_features) {
    set_error("linear: row strides must cover the rows (x %lld weight %lld y %lld)",
              (long long)x_stride, (long long)weight_stride, (long long)y_stride);
    return VFL_E_INVALID;
  }
  if (rows == 0) return VFL_OK;
  if (!x || !weight || !y) {
    set_error("linear: null pointer argument");
    return VFL_E_INVALID;
  }
  if (((uintptr_t)x | (uintptr_t)weight) % 16 != 0 || x_stride % 8 != 0 ||
      weight_stride % 8 != 0 || (uintptr_t)y % 2 != 0 || (uintptr_t)bias % 2 != 0) {
    set_error("linear: x and weight must be 16-byte aligned with row strides a multiple of "
              "8 elements");
    return VFL_E_INVALID;
  }
  const bool vec_store = (uintptr_t)y % 8 == 0 && y_stride % 4 == 0;
  const dim3 grid((unsigned)((out_features + LIN_TILE - 1) / LIN_TILE),
                  (unsigned)((rows + LIN_TILE - 1) / LIN_TILE));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == VFL_BFLOAT16)
    decode_linear_kernel<VFL_BFLOAT16><<<grid, dim3(64 * LIN_WAVES), 0, s>>>(
        (const uint16_t *)x, x_stride, (const uint16_t *)weight, weight_stride,
        (const uint16_t *)bias, (uint16_t *)y, y_stride, (int)rows, out_features, in_features,
        vec_store);
  else
    decode_linear_kernel<VFL_FLOAT16><<<grid, dim3(64 * LIN_WAVES), 0, s>>>(
        (const uint16_t *)x, x_stride, (const uint16_t *)weight, weight_stride,
        (const uint16_t *)bias, (uint16_t *)y, y_stride, (int)rows, out_features, in_features,
        vec_store);
  return launch_status("linear");
}
