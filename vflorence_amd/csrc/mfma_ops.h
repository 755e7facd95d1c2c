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

}  // namespace vfl
