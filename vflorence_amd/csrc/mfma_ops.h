// Matrix-core (MFMA) operand types and the two products the gfx950 kernels use, for
// 16-bit inputs with fp32 accumulation:
//
//   qk: v_mfma_f32_16x16x32  D[16][16] += A[16][32] . B[32][16]
//       A operand: lane l holds row l%16, columns 8*(l/16) .. +7 (one 16-byte chunk)
//       B operand: lane l holds rows 8*(l/16) .. +7 of column l%16 (one 16-byte chunk)
//       D: lane l, register j holds D[4*(l/16) + j][l%16]
//   pv: v_mfma_f32_16x16x16  the same with 4-element (8-byte) chunks, rows 4*(l/16) ..
#pragma once

#include "common.h"

namespace vfl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));

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
  // Round to nearest even on gfx950's packed conversion (v_cvt_pk_bf16_f32): the same
  // bits as f32_to_bf16 for every non-NaN value, in one instruction per pair.
  static __device__ __forceinline__ uint32_t narrow2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{a, b}, bf16x2_t));
  }
  static __device__ __forceinline__ uint32_t narrow(float f) { return narrow2(f, 0.f) & 0xffffu; }
  static __device__ __forceinline__ float widen(uint32_t h) { return __uint_as_float(h << 16); }
  // The two values of a packed pair, widened.
  static __device__ __forceinline__ float widen_lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float widen_hi(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
  }
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
  static __device__ __forceinline__ uint32_t narrow2(float a, float b) {
    return f32_to_f16(a) | (f32_to_f16(b) << 16);
  }
  static __device__ __forceinline__ float widen(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  static __device__ __forceinline__ float widen_lo(uint32_t w) { return widen(w & 0xffffu); }
  static __device__ __forceinline__ float widen_hi(uint32_t w) { return widen(w >> 16); }
};

// Softmax weights as two 16-bit terms, p = hi + lo, so they keep ~16 mantissa bits
// through the 16-bit PV product: hi and lo of four weights, packed in MFMA operand order.
template <int DT>
__device__ __forceinline__ void split_weights(const float (&p)[4], uint2 &hi, uint2 &lo) {
  using Ops = Mfma<DT>;
  hi = make_uint2(Ops::narrow2(p[0], p[1]), Ops::narrow2(p[2], p[3]));
  lo = make_uint2(Ops::narrow2(p[0] - Ops::widen_lo(hi.x), p[1] - Ops::widen_hi(hi.x)),
                  Ops::narrow2(p[2] - Ops::widen_lo(hi.y), p[3] - Ops::widen_hi(hi.y)));
}

}  // namespace vfl
