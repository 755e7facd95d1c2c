// Shared device helpers for the gfx950 decode-attention kernels: element traits,
// 16-byte vector moves, bf16/f16 dot products on the dot2 units, row-local DPP
// reductions and the C-ABI error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vflorence_amd.h"

namespace vfl {

// ---------------------------------------------------------------------------
// error reporting for the C ABI
// ---------------------------------------------------------------------------
void set_error(const char *fmt, ...);
void clear_error();
int launch_status(const char *what);

// ---------------------------------------------------------------------------
// element traits: every kernel moves data in 16-byte chunks (one dwordx4 per lane)
// ---------------------------------------------------------------------------
template <int DT> struct Elem;
template <> struct Elem<VFL_FLOAT32> {
  using T = float;
  static constexpr int VEC = 4;
};
template <> struct Elem<VFL_BFLOAT16> {
  using T = uint16_t;
  static constexpr int VEC = 8;
};
template <> struct Elem<VFL_FLOAT16> {
  using T = uint16_t;
  static constexpr int VEC = 8;
};

inline int elem_bytes(int dtype) { return dtype == VFL_FLOAT32 ? 4 : 2; }

// Tokens per KV block: 16 (this build's pools) or the 32 the reference uses on x86
// (vflorence/config.py:42); the attention kernels walk 16-token parts, 1 << shift per
// block.  Any other size has no kernel (-1): the 16-bit V layout interleaves tokens by
// four inside a block, so a size that is not a multiple of 16 would break the parts.
inline int block_shift(int block_size) {
  return block_size == 16 ? 0 : (block_size == 32 ? 1 : -1);
}

// Workgroup ids of the attention launches, one workgroup per (group position, head).
// MI355X deals a launch's workgroup ids to its 8 XCDs round robin (id % 8), each XCD
// with its own L2.  The ids are laid out so that all H heads of a group position run
// on one XCD: id = 8 (H (pos / 8) + h) + pos % 8.  The heads' slices of a block then
// come through one L2, and within an XCD its CUs still see positions p, p + 16, p + 32,
// ... (with 16 heads), the pattern the balanced dispatch order is built for.  Read-only
// probe of the cross-attention's pages: 26.9 against 27.6 us per layer with
// consecutive ids per group.  The grid covers positions rounded up to 8; the extra
// workgroups exit.
constexpr int XCDS = 8;
inline int64_t xcd_grid(int64_t positions, int H) {
  return (positions + XCDS - 1) / XCDS * XCDS * H;
}
__device__ __forceinline__ void xcd_position(unsigned id, unsigned H, int64_t &pos, int &h) {
  const unsigned j = id / XCDS;
  h = (int)(j % H);
  pos = (int64_t)XCDS * (j / H) + id % XCDS;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even; NaN becomes the canonical quiet NaN 0x7fc0
// (the same bits torch's float -> bfloat16 conversion produces).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// <q, k> over one 16-byte chunk, fp32 accumulation.
template <int DT> __device__ __forceinline__ float dot16(const uint4 &q, const uint4 &k);

template <> __device__ __forceinline__ float dot16<VFL_BFLOAT16>(const uint4 &q, const uint4 &k) {
  float s = 0.f;
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.x),
                                      __builtin_bit_cast(bf16x2_t, k.x), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.y),
                                      __builtin_bit_cast(bf16x2_t, k.y), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.z),
                                      __builtin_bit_cast(bf16x2_t, k.z), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.w),
                                      __builtin_bit_cast(bf16x2_t, k.w), s, false);
  return s;
}

template <> __device__ __forceinline__ float dot16<VFL_FLOAT16>(const uint4 &q, const uint4 &k) {
  float s = 0.f;
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.x), __builtin_bit_cast(f16x2_t, k.x), s,
                             false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.y), __builtin_bit_cast(f16x2_t, k.y), s,
                             false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.z), __builtin_bit_cast(f16x2_t, k.z), s,
                             false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.w), __builtin_bit_cast(f16x2_t, k.w), s,
                             false);
  return s;
}

template <> __device__ __forceinline__ float dot16<VFL_FLOAT32>(const uint4 &q, const uint4 &k) {
  float s = __uint_as_float(q.x) * __uint_as_float(k.x);
  s = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), s);
  s = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), s);
  s = fmaf(__uint_as_float(q.w), __uint_as_float(k.w), s);
  return s;
}

// Unpack one 16-byte chunk into VEC floats.
template <int DT> __device__ __forceinline__ void unpack16(const uint4 &v, float *f);

template <> __device__ __forceinline__ void unpack16<VFL_BFLOAT16>(const uint4 &v, float *f) {
  f[0] = bf16lo(v.x); f[1] = bf16hi(v.x);
  f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
  f[4] = bf16lo(v.z); f[5] = bf16hi(v.z);
  f[6] = bf16lo(v.w); f[7] = bf16hi(v.w);
}

template <> __device__ __forceinline__ void unpack16<VFL_FLOAT16>(const uint4 &v, float *f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f16x2_t h = __builtin_bit_cast(f16x2_t, w[i]);
    f[2 * i] = (float)h.x;
    f[2 * i + 1] = (float)h.y;
  }
}

template <> __device__ __forceinline__ void unpack16<VFL_FLOAT32>(const uint4 &v, float *f) {
  f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
  f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
}

// Pack VEC floats into one 16-byte chunk of element type DT (round to nearest even).
template <int DT> __device__ __forceinline__ uint4 pack16(const float *f);

template <> __device__ __forceinline__ uint4 pack16<VFL_BFLOAT16>(const float *f) {
  uint4 r;
  r.x = f32_to_bf16(f[0]) | (f32_to_bf16(f[1]) << 16);
  r.y = f32_to_bf16(f[2]) | (f32_to_bf16(f[3]) << 16);
  r.z = f32_to_bf16(f[4]) | (f32_to_bf16(f[5]) << 16);
  r.w = f32_to_bf16(f[6]) | (f32_to_bf16(f[7]) << 16);
  return r;
}

template <> __device__ __forceinline__ uint4 pack16<VFL_FLOAT16>(const float *f) {
  uint4 r;
  r.x = f32_to_f16(f[0]) | (f32_to_f16(f[1]) << 16);
  r.y = f32_to_f16(f[2]) | (f32_to_f16(f[3]) << 16);
  r.z = f32_to_f16(f[4]) | (f32_to_f16(f[5]) << 16);
  r.w = f32_to_f16(f[6]) | (f32_to_f16(f[7]) << 16);
  return r;
}

template <> __device__ __forceinline__ uint4 pack16<VFL_FLOAT32>(const float *f) {
  uint4 r;
  r.x = __float_as_uint(f[0]); r.y = __float_as_uint(f[1]);
  r.z = __float_as_uint(f[2]); r.w = __float_as_uint(f[3]);
  return r;
}

// Load 16 bytes from an address that may be only element-aligned.
template <int DT>
__device__ __forceinline__ uint4 load16_unaligned(const typename Elem<DT>::T *p) {
  if constexpr (DT == VFL_FLOAT32) {
    uint4 r;
    r.x = __float_as_uint(p[0]); r.y = __float_as_uint(p[1]);
    r.z = __float_as_uint(p[2]); r.w = __float_as_uint(p[3]);
    return r;
  } else {
    uint4 r;
    r.x = (uint32_t)p[0] | ((uint32_t)p[1] << 16);
    r.y = (uint32_t)p[2] | ((uint32_t)p[3] << 16);
    r.z = (uint32_t)p[4] | ((uint32_t)p[5] << 16);
    r.w = (uint32_t)p[6] | ((uint32_t)p[7] << 16);
    return r;
  }
}

template <int DT>
__device__ __forceinline__ void store16_unaligned(typename Elem<DT>::T *p, const uint4 &v) {
  if constexpr (DT == VFL_FLOAT32) {
    p[0] = __uint_as_float(v.x); p[1] = __uint_as_float(v.y);
    p[2] = __uint_as_float(v.z); p[3] = __uint_as_float(v.w);
  } else {
    p[0] = (uint16_t)v.x; p[1] = (uint16_t)(v.x >> 16);
    p[2] = (uint16_t)v.y; p[3] = (uint16_t)(v.y >> 16);
    p[4] = (uint16_t)v.z; p[5] = (uint16_t)(v.z >> 16);
    p[6] = (uint16_t)v.w; p[7] = (uint16_t)(v.w >> 16);
  }
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// Sum over aligned groups of N consecutive lanes (N = 1..64, power of two); every
// lane of a group ends with the group's sum.  Within a 16-lane row the partners come
// from DPP (no LDS traffic): after the quad sums, half-row mirroring pairs each
// quad with the other quad of its half-row, and row mirroring pairs the halves.
// Across rows, v_permlane16_swap pairs rows 0-1 and 2-3 and v_permlane32_swap the two
// halves (VALU moves too); each pair's lanes add the same two values, as lane l and
// lane l ^ 16 (l ^ 32) of an xor butterfly would.
template <int N> __device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<DPP_QUAD_XOR1>(x);
  if constexpr (N >= 4) x += dpp<DPP_QUAD_XOR2>(x);
  if constexpr (N >= 8) x += dpp<DPP_ROW_HALF_MIRROR>(x);
  if constexpr (N >= 16) x += dpp<DPP_ROW_MIRROR>(x);
  if constexpr (N >= 32) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  if constexpr (N >= 64) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  return x;
}

// Maximum over the 16 lanes of each row (every lane gets its row's maximum).
__device__ __forceinline__ int row_max16(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, DPP_QUAD_XOR1, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, DPP_QUAD_XOR2, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, DPP_ROW_HALF_MIRROR, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, DPP_ROW_MIRROR, 0xF, 0xF, false));
  return x;
}

// Across the four 16-lane rows, lane-wise: lanes l, l^16, l^32 and l^48 (the four row
// groups of one MFMA tile column) all end with the same value.  v_permlane16_swap
// pairs rows 0-1 and 2-3, v_permlane32_swap rows 0-2 and 1-3; both are VALU moves, no
// LDS round trip.  The sum is (r0 + r1) + (r2 + r3) on every lane, the order of an
// xor-16-then-xor-32 butterfly.
__device__ __forceinline__ float rows_max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float NEG_INF_F = -__builtin_huge_valf();

// Online-softmax maxima are lazy references: scores are exponentiated against the
// reference and it only moves (rescaling the accumulators) when a block max exceeds
// it by more than this many log2 units, so weights stay <= 2^8 and most blocks skip
// the rescale.  The final normalisation makes the result exact in exact arithmetic.
constexpr float RESCALE_SLACK_LOG2 = 8.0f;

// V pools of 16-bit element type hold every [block][head] slice with tokens grouped
// by four and interleaved: [block_size/4][head_dim][4].  The matrix-core kernel then
// reads 4 consecutive tokens of one dim as 8 bytes (its reduction operand), and one
// token's head_dim values lie 8 bytes apart in a 512-byte span, so writing a token
// touches few memory sectors.  fp32 pools keep the logical [block_size][head_dim].
inline bool v_tile_interleaved(int dtype) { return dtype != VFL_FLOAT32; }

// Element offset of (token t, dim d) inside an interleaved V tile of head size D.
__host__ __device__ __forceinline__ int vtile_index(int t, int d, int D) {
  return ((t >> 2) * D + d) * 4 + (t & 3);
}

// Workgroup barrier that orders LDS only: global stores issued before it (the fused
// KV write) stay in flight instead of being drained, as __syncthreads() would.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A wave's block ids, 64 at a time in one VGPR (lane i holds the id of block
// base + i), read back with readlane: no scalar load sits between one block's
// K/V loads and the next.
struct WaveBlockIds {
  const int32_t *row;
  int end, base, reg;

  __device__ __forceinline__ void fetch(int b) {
    base = b;
    const int lane = __lane_id();
    reg = (b + lane < end) ? row[b + lane] : -1;
  }
  __device__ __forceinline__ void init(const int32_t *r, int b0, int b1) {
    row = r;
    end = b1;
    fetch(b0);
  }
  // Ids 0..63 of a table row `width` entries wide, requested before the row's length
  // is known (one dependent load level less); limit() then bounds later fetches to the
  // row's blocks.
  __device__ __forceinline__ void prefetch(const int32_t *r, int width) {
    row = r;
    end = width;
    fetch(0);
  }
  __device__ __forceinline__ void limit(int b1) { end = b1; }
  // b is wave-uniform and b0 <= b < b1.
  __device__ __forceinline__ int get(int b) {
    if (b - base >= 64) fetch(b);
    return __builtin_amdgcn_readlane(reg, b - base);
  }
};

}  // namespace vfl
