// Decoder-step kernels around the attention path, for gfx950:
//
//   add_layer_norm_kernel  -- out = LayerNorm(x + residual) * weight + bias, one row per
//                             workgroup; the sum is rounded to the element type first
//                             (what a separate add kernel stores), statistics in fp32.
//   logprob_topk_kernel    -- per row: log-softmax of the logits, the generation rules
//                             (min length, forced BOS / EOS, suppressed tokens), and the
//                             k best (score, token) pairs, best first; one read of the
//                             logits.  With log_softmax off the scores are the processed
//                             logits themselves (greedy decoding's argmax at k = 1).
//
// Both are bandwidth-bound streams over [rows, dim] / [rows, vocab] in HBM.
#include <math.h>
#include <stdio.h>

#include "common.h"

namespace vfl {

// ---------------------------------------------------------------------------
// wave-wide reductions (64 lanes) on VALU lane moves: v_permlane32/16_swap across the
// 16-lane rows, DPP inside them.  __shfl_xor compiles to ds_bpermute, an LDS round trip
// per step; the top-k's selection loop makes dozens of these reductions per row (256 x
// 50265 bf16 logits, k = 8: 22.3-24.5 us per launch with ds_bpermute).
// ---------------------------------------------------------------------------
constexpr int DPP_QUAD_REVERSE = 0x1B;  // quad_perm [3,2,1,0]
constexpr int DPP_ROW_ROR8 = 0x128;     // row_ror:8: lane i of a row takes lane i ^ 8

template <int CTRL> __device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
// The value of lane l ^ M (M = 1, 2, 4, 8: inside a 16-lane row).  Lane l ^ 4 is the
// quad reversal followed by the half-row mirror: (l & ~3 | 3 - l % 4) mirrored in its
// 8 lanes is l ^ 4.
template <int M> __device__ __forceinline__ uint32_t lane_xor(uint32_t x) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "row-local partner");
  if constexpr (M == 1) return dpp_u<DPP_QUAD_XOR1>(x);
  else if constexpr (M == 2) return dpp_u<DPP_QUAD_XOR2>(x);
  else if constexpr (M == 4) return dpp_u<DPP_ROW_HALF_MIRROR>(dpp_u<DPP_QUAD_REVERSE>(x));
  else return dpp_u<DPP_ROW_ROR8>(x);
}
// Lane l's value and lane (l ^ 32)'s (P = 32), or l ^ 16's (P = 16), in some order: the
// swap pairs the two halves (rows 0-1 with 2-3), resp. rows 0 with 1 and 2 with 3.
template <int P> __device__ __forceinline__ void lane_pair(uint32_t x, uint32_t &a, uint32_t &b) {
  static_assert(P == 16 || P == 32, "cross-row partner");
  if constexpr (P == 32) {
    const auto s = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    a = s[0], b = s[1];
  } else {
    const auto s = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    a = s[0], b = s[1];
  }
}

// Sum over the 64 lanes, every lane getting it: the xor butterfly with offsets 32, 16,
// 8, 4, 2, 1, each step adding the partner's value to the lane's own (floating-point
// addition commutes, so the bits are those of the same butterfly on __shfl_xor).
__device__ __forceinline__ float wave_sum(float v) {
  uint32_t a, b;
  lane_pair<32>(__float_as_uint(v), a, b);
  v = __uint_as_float(a) + __uint_as_float(b);
  lane_pair<16>(__float_as_uint(v), a, b);
  v = __uint_as_float(a) + __uint_as_float(b);
  v += __uint_as_float(lane_xor<8>(__float_as_uint(v)));
  v += __uint_as_float(lane_xor<4>(__float_as_uint(v)));
  v += __uint_as_float(lane_xor<2>(__float_as_uint(v)));
  v += __uint_as_float(lane_xor<1>(__float_as_uint(v)));
  return v;
}

template <int DT> __device__ __forceinline__ void load4(const typename Elem<DT>::T *p, float v[4]);
template <> __device__ __forceinline__ void load4<VFL_FLOAT32>(const float *p, float v[4]) {
  const float4 u = *reinterpret_cast<const float4 *>(p);
  v[0] = u.x, v[1] = u.y, v[2] = u.z, v[3] = u.w;
}
template <> __device__ __forceinline__ void load4<VFL_BFLOAT16>(const uint16_t *p, float v[4]) {
  const uint2 u = *reinterpret_cast<const uint2 *>(p);
  v[0] = bf16lo(u.x), v[1] = bf16hi(u.x), v[2] = bf16lo(u.y), v[3] = bf16hi(u.y);
}
template <> __device__ __forceinline__ void load4<VFL_FLOAT16>(const uint16_t *p, float v[4]) {
  const uint2 u = *reinterpret_cast<const uint2 *>(p);
  const f16x2_t a = __builtin_bit_cast(f16x2_t, u.x), b = __builtin_bit_cast(f16x2_t, u.y);
  v[0] = (float)a.x, v[1] = (float)a.y, v[2] = (float)b.x, v[3] = (float)b.y;
}

template <int DT> __device__ __forceinline__ void store4(typename Elem<DT>::T *p, const float v[4]);
template <> __device__ __forceinline__ void store4<VFL_FLOAT32>(float *p, const float v[4]) {
  *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ void store4<VFL_BFLOAT16>(uint16_t *p, const float v[4]) {
  uint2 u;
  u.x = f32_to_bf16(v[0]) | (f32_to_bf16(v[1]) << 16);
  u.y = f32_to_bf16(v[2]) | (f32_to_bf16(v[3]) << 16);
  *reinterpret_cast<uint2 *>(p) = u;
}
template <> __device__ __forceinline__ void store4<VFL_FLOAT16>(uint16_t *p, const float v[4]) {
  uint2 u;
  u.x = f32_to_f16(v[0]) | (f32_to_f16(v[1]) << 16);
  u.y = f32_to_f16(v[2]) | (f32_to_f16(v[3]) << 16);
  *reinterpret_cast<uint2 *>(p) = u;
}

// The value a kernel that stores `v` in the element type would leave behind.
template <int DT> __device__ __forceinline__ float round_to_elem(float v);
template <> __device__ __forceinline__ float round_to_elem<VFL_FLOAT32>(float v) { return v; }
template <> __device__ __forceinline__ float round_to_elem<VFL_BFLOAT16>(float v) {
  return __uint_as_float(f32_to_bf16(v) << 16);
}
template <> __device__ __forceinline__ float round_to_elem<VFL_FLOAT16>(float v) {
  return (float)(_Float16)v;
}

// ---------------------------------------------------------------------------
// residual add + LayerNorm: one wave per row, statistics by wave shuffles (no
// workgroup barrier on the row's critical path)
// ---------------------------------------------------------------------------
// Rows (waves) per workgroup.  Measured over a 4-beam BART-large engine step (37 calls of
// 256 rows x 1024): 2 rows per workgroup 2.45 ms per step, 4 rows 2.47-2.48, 1 row 2.48.
constexpr int LN_ROWS = 2;

// Rows of x and residual taken from tables: row r reads x row x_rows[r] + x_offset and
// residual row r_rows[r] + r_offset, the residual row times r_scale rounded to the
// element type first when r_scale != 1 (what a scaled embedding lookup stores).  A row
// whose index falls outside its table comes out NaN.
struct RowGather {
  const int64_t *x_rows, *r_rows;
  int64_t x_offset, r_offset, x_count, r_count;
  float r_scale;
};

template <int DT, int NV, bool GATHER>  // NV: 4-element vectors per lane (dim <= 256 * NV)
__global__ __launch_bounds__(64 * LN_ROWS) void add_layer_norm_kernel(
    const typename Elem<DT>::T *x, int64_t x_stride, const typename Elem<DT>::T *residual,
    int64_t r_stride, const typename Elem<DT>::T *__restrict__ weight,
    const typename Elem<DT>::T *__restrict__ bias, typename Elem<DT>::T *out, int64_t out_stride,
    int64_t rows, int dim, float eps, RowGather g) {
  // out may alias x or residual: each lane reads its elements before the reductions
  // and writes the same elements after them.
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * LN_ROWS + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int nvec = dim >> 2;
  int64_t xr = row, rr = row;
  if constexpr (GATHER) {
    xr = g.x_rows[row] + g.x_offset;
    rr = g.r_rows[row] + g.r_offset;
    if (xr < 0 || xr >= g.x_count || rr < 0 || rr >= g.r_count) {  // wave-uniform
      for (int i = lane; i < nvec; i += 64) {
        const float nan4[4] = {NAN, NAN, NAN, NAN};
        store4<DT>(out + row * out_stride + i * 4, nan4);
      }
      return;
    }
  }
  float v[NV][4], w[NV][4], b[NV][4];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int vi = lane + 64 * k;
    if (vi < nvec) {
      float a[4], c[4];
      load4<DT>(x + xr * x_stride + vi * 4, a);
      load4<DT>(residual + rr * r_stride + vi * 4, c);
      load4<DT>(weight + vi * 4, w[k]);
      load4<DT>(bias + vi * 4, b[k]);
      if constexpr (GATHER) {
        if (g.r_scale != 1.f) {
#pragma unroll
          for (int e = 0; e < 4; ++e) c[e] = round_to_elem<DT>(c[e] * g.r_scale);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[k][e] = round_to_elem<DT>(a[e] + c[e]);
        sum += v[k][e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[k][e] = 0.f;
    }
  }
  const float mean = wave_sum(sum) / (float)dim;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (lane + 64 * k < nvec) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[k][e] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int vi = lane + 64 * k;
    if (vi < nvec) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (v[k][e] - mean) * rstd * w[k][e] + b[k][e];
      store4<DT>(out + row * out_stride + vi * 4, o);
    }
  }
}

template <int DT, bool GATHER>
static int launch_add_layer_norm(const void *x, int64_t xs, const void *r, int64_t rs,
                                 const void *w, const void *b, void *out, int64_t os, int64_t rows,
                                 int dim, float eps, const RowGather &g, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const int nvec = dim / 4;
  const dim3 grid((unsigned)((rows + LN_ROWS - 1) / LN_ROWS)), block(64 * LN_ROWS);
#define VFL_LN(NV)                                                                             \
  add_layer_norm_kernel<DT, NV, GATHER><<<grid, block, 0, stream>>>(                           \
      (const T *)x, xs, (const T *)r, rs, (const T *)w, (const T *)b, (T *)out, os, rows, dim, \
      eps, g)
  if (nvec <= 64)
    VFL_LN(1);
  else if (nvec <= 128)
    VFL_LN(2);
  else if (nvec <= 256)
    VFL_LN(4);
  else if (nvec <= 512)
    VFL_LN(8);
  else
    VFL_LN(16);
#undef VFL_LN
  return launch_status(GATHER ? "embed_layer_norm" : "add_layer_norm");
}

// ---------------------------------------------------------------------------
// log-softmax + generation rules + per-row top-k
// ---------------------------------------------------------------------------
constexpr int TK_MAX_RULE_TOKENS = 256;

// (score, token) order: higher score first, then lower token id, then lower lane.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  return a > b || (a == b && ia < ib);
}

// Insert (v, t) into a descending list of K entries if it beats the last one.
template <int K> __device__ __forceinline__ void insert(float (&val)[K], int (&tok)[K], float v, int t) {
  if (!better(v, t, val[K - 1], tok[K - 1])) return;
  val[K - 1] = v, tok[K - 1] = t;
#pragma unroll
  for (int j = K - 1; j > 0; --j) {
    if (better(val[j], tok[j], val[j - 1], tok[j - 1])) {
      const float fv = val[j];
      val[j] = val[j - 1], val[j - 1] = fv;
      const int ft = tok[j];
      tok[j] = tok[j - 1], tok[j - 1] = ft;
    }
  }
}

// Pop the head of a descending list (the tail refills with an empty entry).
template <int K> __device__ __forceinline__ void pop_head(float (&val)[K], int (&tok)[K]) {
#pragma unroll
  for (int j = 0; j + 1 < K; ++j) val[j] = val[j + 1], tok[j] = tok[j + 1];
  val[K - 1] = -INFINITY, tok[K - 1] = INT32_MAX;
}

// (bv, bt, bl) becomes the better of itself and (ov, ot, ol): higher score, then lower
// token, then lower lane -- a strict order over the lanes' triples.
__device__ __forceinline__ void take_better(float &bv, int &bt, int &bl, float ov, int ot, int ol) {
  if (better(ov, ot, bv, bt) || (ov == bv && ot == bt && ol < bl)) bv = ov, bt = ot, bl = ol;
}
template <int P> __device__ __forceinline__ void best_across(float &v, int &t, int &l) {
  uint32_t v0, v1, t0, t1, l0, l1;
  lane_pair<P>(__float_as_uint(v), v0, v1);
  lane_pair<P>((uint32_t)t, t0, t1);
  lane_pair<P>((uint32_t)l, l0, l1);
  v = __uint_as_float(v0), t = (int)t0, l = (int)l0;
  take_better(v, t, l, __uint_as_float(v1), (int)t1, (int)l1);
}
template <int M> __device__ __forceinline__ void best_within(float &v, int &t, int &l) {
  take_better(v, t, l, __uint_as_float(lane_xor<M>(__float_as_uint(v))),
              (int)lane_xor<M>((uint32_t)t), (int)lane_xor<M>((uint32_t)l));
}

// Wave-wide best (score, token) among every lane's head; ties by lane.  The best of a
// strict order does not depend on how the butterfly pairs the lanes.
__device__ __forceinline__ void wave_best(float v, int t, float &bv, int &bt, int &blane) {
  int l = threadIdx.x & 63;
  best_within<1>(v, t, l);
  best_within<2>(v, t, l);
  best_within<4>(v, t, l);
  best_within<8>(v, t, l);
  best_across<16>(v, t, l);
  best_across<32>(v, t, l);
  bv = v, bt = t, blane = l;
}

struct TopkRules {
  int32_t min_length, max_length, begin_index;
  int32_t n_eos, n_suppress, n_begin, n_bos, n_feos;
};

__device__ __forceinline__ bool in_list(const int *list, int n, int t) {
  for (int i = 0; i < n; ++i)
    if (list[i] == t) return true;
  return false;
}

template <int DT> __device__ __forceinline__ float elem_to_f32(typename Elem<DT>::T v) {
  if constexpr (DT == VFL_FLOAT32) return v;
  else if constexpr (DT == VFL_BFLOAT16) return __uint_as_float((uint32_t)v << 16);
  else return (float)__builtin_bit_cast(_Float16, v);
}

// Element j of a 16-byte vector as fp32 (j a compile-time constant after unrolling).
template <int DT> __device__ __forceinline__ float vec_elem(const uint4 &u, int j) {
  if constexpr (DT == VFL_FLOAT32) {
    const uint32_t w = j == 0 ? u.x : j == 1 ? u.y : j == 2 ? u.z : u.w;
    return __uint_as_float(w);
  } else {
    const uint32_t w = (j >> 1) == 0 ? u.x : (j >> 1) == 1 ? u.y : (j >> 1) == 2 ? u.z : u.w;
    const uint32_t h = (j & 1) ? (w >> 16) : (w & 0xffffu);
    if constexpr (DT == VFL_BFLOAT16) return __uint_as_float(h << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
}

// Wave-wide maximum.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __uint_as_float(lane_xor<1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(lane_xor<2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(lane_xor<4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(lane_xor<8>(__float_as_uint(v))));
  uint32_t a, b;
  lane_pair<16>(__float_as_uint(v), a, b);
  v = fmaxf(__uint_as_float(a), __uint_as_float(b));
  lane_pair<32>(__float_as_uint(v), a, b);
  return fmaxf(__uint_as_float(a), __uint_as_float(b));
}

// Row top-k in two reads of the row (the second mostly from L2):
//   1. each thread's largest allowed value, and the row maximum for the normaliser;
//      the k-th largest of the per-thread maxima, tau, bounds the row's k-th value
//      from below (k threads hold a value >= tau);
//   2. the sum of exp(x - max), and every allowed value >= tau appended to an LDS list
//      (a handful per row);
//   3. one wave picks the k best of that list.
// Rows with a forced token, fewer than k allowed finite values, or more than CAP
// values tied at the threshold take a third read that keeps per-lane k-best lists.
template <int DT, int K, int NT>
__global__ __launch_bounds__(NT, 2) void logprob_topk_kernel(
    const typename Elem<DT>::T *__restrict__ logits, int64_t stride, int vocab,
    const int64_t *__restrict__ lengths, const int32_t *__restrict__ rule_tokens, TopkRules rules,
    int log_softmax, int k_out, float *__restrict__ out_scores, int64_t *__restrict__ out_ids) {
  using T = typename Elem<DT>::T;
  constexpr int NWAVE = NT / 64;
  constexpr int VE = 16 / sizeof(T);  // elements per 16-byte load
  constexpr int CAP = 512;            // threshold candidates kept in LDS
  constexpr int LPL = CAP / 64;       // candidates per lane in the final pick
  constexpr int TPL = NT / 64;        // per-thread maxima per lane when finding tau
  __shared__ int s_ban[TK_MAX_RULE_TOKENS];
  __shared__ int s_force[TK_MAX_RULE_TOKENS];
  __shared__ float s_tmax[NT];
  __shared__ float s_cv[CAP];
  __shared__ int s_ct[CAP];
  __shared__ float s_val[NWAVE][K];
  __shared__ int s_tok[NWAVE][K];
  __shared__ float s_red[NWAVE];
  __shared__ int s_nban, s_nforce, s_count;
  __shared__ float s_tau;

  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T *x = logits + row * stride;

  // The row's active rules, in the processors' order: min-length bans EOS; forced BOS
  // (length 1) and forced EOS (length max_length - 1) replace every score; suppressed
  // tokens and, at begin_index, the begin-suppressed tokens are banned afterwards.
  if (threadIdx.x == 0) {
    const int64_t len = lengths ? lengths[row] : 0;
    const int *eos = rule_tokens, *sup = eos + rules.n_eos, *beg = sup + rules.n_suppress;
    const int *bos = beg + rules.n_begin, *feos = bos + rules.n_bos;
    int nf = 0, nb = 0;
    if (rules.n_feos && len == rules.max_length - 1) {
      for (int i = 0; i < rules.n_feos; ++i) s_force[nf++] = feos[i];
    } else if (rules.n_bos && len == 1) {
      for (int i = 0; i < rules.n_bos; ++i) s_force[nf++] = bos[i];
    }
    if (nf == 0 && len < rules.min_length)
      for (int i = 0; i < rules.n_eos; ++i) s_ban[nb++] = eos[i];
    for (int i = 0; i < rules.n_suppress; ++i) s_ban[nb++] = sup[i];
    if (len == rules.begin_index)
      for (int i = 0; i < rules.n_begin; ++i) s_ban[nb++] = beg[i];
    s_nban = nb, s_nforce = nf, s_count = 0;
  }
  __syncthreads();
  const int nban = s_nban, nforce = s_nforce;

  // The row in 16-byte loads: scalar elements up to the first aligned address, the
  // aligned body RD loads per thread in flight at a time, then the scalar tail.  Every
  // thread visits its tokens in increasing order.
  constexpr int RD = 8;
  const int head = min(vocab, (int)(((16 - ((uintptr_t)x & 15)) & 15) / sizeof(T)));
  const int nvec = (vocab - head) / VE;
  const uint4 *xv = reinterpret_cast<const uint4 *>(x + head);
  auto scan = [&](auto &&visit) {
    if ((int)threadIdx.x < head) visit(elem_to_f32<DT>(x[threadIdx.x]), (int)threadIdx.x);
    for (int i = threadIdx.x; i < nvec; i += RD * NT) {
      uint4 u[RD];
#pragma unroll
      for (int r = 0; r < RD; ++r)
        if (i + r * NT < nvec) u[r] = xv[i + r * NT];
#pragma unroll
      for (int r = 0; r < RD; ++r) {
        if (i + r * NT < nvec) {
#pragma unroll
          for (int j = 0; j < VE; ++j) visit(vec_elem<DT>(u[r], j), head + (i + r * NT) * VE + j);
        }
      }
    }
    for (int t = head + nvec * VE + threadIdx.x; t < vocab; t += NT)
      visit(elem_to_f32<DT>(x[t]), t);
  };

  float mx = 0.f, lse = 0.f;
  if (nforce == 0) {
    // 1: row maximum and each thread's largest value (bans are applied to the few
    // candidates of step 3, so the scans stay branch-free)
    float rawmax = -INFINITY;
    scan([&](float v, int) { rawmax = fmaxf(rawmax, v); });
    s_tmax[threadIdx.x] = rawmax;
    rawmax = wave_max(rawmax);
    if (lane == 0) s_red[wave] = rawmax;
    __syncthreads();
    mx = s_red[0];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) mx = fmaxf(mx, s_red[w]);
    if (wave == 0) {
      // tau: the (K + nban)-th largest per-thread maximum (with multiplicity).  At least
      // K + nban values are >= tau and at most nban of them are banned, so the row's
      // K-th allowed value is >= tau too.
      float c[TPL];
      int ci[TPL];
#pragma unroll
      for (int i = 0; i < TPL; ++i) c[i] = -INFINITY, ci[i] = INT32_MAX;
#pragma unroll
      for (int i = 0; i < TPL; ++i) insert<TPL>(c, ci, s_tmax[lane * TPL + i], lane * TPL + i);
      float tau = -INFINITY;
      const int need = min(K + nban, NT);
      for (int r = 0; r < need; ++r) {
        float bv;
        int bt, bl;
        wave_best(c[0], ci[0], bv, bt, bl);
        if (lane == bl) pop_head<TPL>(c, ci);
        tau = bv;
      }
      if (lane == 0) s_tau = (K + nban <= NT) ? tau : -INFINITY;
    }
    __syncthreads();
    const float tau = s_tau;
    const float pick = tau == -INFINITY ? INFINITY : tau;  // no shortcut without a bound
    // 2: normaliser sum and every value at or above tau.  The terms are exp2 of the
    // log2e-scaled differences (the hardware exponential: 256 x 50265 logits in 23.4
    // against 26.9 us with expf, selections identical, scores within 1e-6).
    constexpr float LOG2E_F = 1.4426950408889634f;
    float sum = 0.f;
    scan([&](float v, int t) {
      if (log_softmax && v != -INFINITY) sum += fast_exp2((v - mx) * LOG2E_F);
      if (v >= pick) {
        const int slot = atomicAdd(&s_count, 1);
        if (slot < CAP) s_cv[slot] = v, s_ct[slot] = t;
      }
    });
    if (log_softmax) {
      sum = wave_sum(sum);
      __syncthreads();  // s_red is reused
      if (lane == 0) s_red[wave] = sum;
    }
    __syncthreads();
    if (log_softmax) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < NWAVE; ++w) tot += s_red[w];
      lse = logf(tot);
    }
    const int count = s_count;
    if (tau != -INFINITY && count <= CAP) {
      // 3: the K best allowed candidates
      if (wave != 0) return;
      float cv[LPL];
      int ct[LPL];
#pragma unroll
      for (int i = 0; i < LPL; ++i) cv[i] = -INFINITY, ct[i] = INT32_MAX;
      for (int i = 0; i < LPL; ++i) {
        const int c = lane + 64 * i;
        if (c < count && !in_list(s_ban, nban, s_ct[c])) insert<LPL>(cv, ct, s_cv[c], s_ct[c]);
      }
      for (int r = 0; r < k_out; ++r) {
        float bv;
        int bt, bl;
        wave_best(cv[0], ct[0], bv, bt, bl);
        if (lane == bl) pop_head<LPL>(cv, ct);
        if (lane == 0) {
          out_scores[row * k_out + r] = log_softmax ? (bv - mx) - lse : bv;
          out_ids[row * k_out + r] = bt;
        }
      }
      return;
    }
  }

  // Per-lane k-best lists over the whole row (forced rows and the rare fallbacks).
  float val[K];
  int tok[K];
#pragma unroll
  for (int j = 0; j < K; ++j) val[j] = -INFINITY, tok[j] = INT32_MAX;
  // a plain element loop: these rows are rare, and the code stays small
#pragma nounroll
  for (int t = threadIdx.x; t < vocab; t += NT) {
    const float v = elem_to_f32<DT>(x[t]);
    if (nforce) {
      const float f = (in_list(s_force, nforce, t) && !in_list(s_ban, nban, t)) ? 0.f : -INFINITY;
      insert<K>(val, tok, f, t);
    } else if (better(v, t, val[K - 1], tok[K - 1])) {
      insert<K>(val, tok, in_list(s_ban, nban, t) ? -INFINITY : v, t);
    }
  }
  for (int r = 0; r < K; ++r) {
    float bv;
    int bt, bl;
    wave_best(val[0], tok[0], bv, bt, bl);
    if (lane == bl) pop_head<K>(val, tok);
    if (lane == 0) s_val[wave][r] = bv, s_tok[wave][r] = bt;
  }
  __syncthreads();
  if (wave != 0) return;
  constexpr int CPL = (NWAVE * K + 63) / 64;
  float cv[CPL];
  int ct[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) cv[i] = -INFINITY, ct[i] = INT32_MAX;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < NWAVE * K) insert<CPL>(cv, ct, s_val[c / K][c % K], s_tok[c / K][c % K]);
  }
  for (int r = 0; r < k_out; ++r) {
    float bv;
    int bt, bl;
    wave_best(cv[0], ct[0], bv, bt, bl);
    if (lane == bl) pop_head<CPL>(cv, ct);
    if (lane == 0) {
      // processed log-prob: (x - max) - log(sum exp(x - max)); forced tokens score 0
      float outv = bv;
      if (log_softmax && !nforce && bv != -INFINITY) outv = (bv - mx) - lse;
      out_scores[row * k_out + r] = outv;
      out_ids[row * k_out + r] = bt;
    }
  }
}

template <int DT>
static int launch_topk(const void *logits, int64_t stride, int64_t rows, int vocab,
                       const int64_t *lengths, const int32_t *rule_tokens, const TopkRules &rules,
                       int log_softmax, int k, float *scores, int64_t *ids, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const dim3 grid((unsigned)rows);
  // 8 waves per row; each lane's list lives in registers (k <= 16 keeps it there)
#define VFL_TK(KK, NT)                                                                         \
  logprob_topk_kernel<DT, KK, NT><<<grid, dim3(NT), 0, stream>>>(                              \
      (const T *)logits, stride, vocab, lengths, rule_tokens, rules, log_softmax, k, scores, ids)
  if (k <= 1)
    VFL_TK(1, 512);
  else if (k <= 8)
    VFL_TK(8, 512);
  else
    VFL_TK(16, 512);
#undef VFL_TK
  return launch_status("logprob_topk");
}

}  // namespace vfl

using namespace vfl;

static bool aligned(const void *p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// Shared argument checks of the residual + LayerNorm entry points.
static int check_layer_norm(const char *who, int64_t rows, int dim, int dtype, const void *x,
                            int64_t x_stride, const void *residual, int64_t residual_stride,
                            const void *weight, const void *bias, const void *out,
                            int64_t out_stride) {
  if (dtype != VFL_FLOAT32 && dtype != VFL_BFLOAT16 && dtype != VFL_FLOAT16) {
    set_error("%s: unsupported dtype code %d", who, dtype);
    return VFL_E_INVALID;
  }
  if (rows < 0 || rows > 2147483647LL || dim <= 0 || dim % 4 || dim > 4096) {
    set_error("%s: dim %d must be a positive multiple of 4 up to 4096 (rows %lld)", who, dim,
              (long long)rows);
    return VFL_E_INVALID;
  }
  if (!x || !residual || !weight || !bias || !out) {
    set_error("%s: null pointer argument", who);
    return VFL_E_INVALID;
  }
  const int vb = 4 * elem_bytes(dtype);
  if (x_stride % 4 || residual_stride % 4 || out_stride % 4 || !aligned(x, vb) ||
      !aligned(residual, vb) || !aligned(weight, vb) || !aligned(bias, vb) || !aligned(out, vb) ||
      x_stride < dim || residual_stride < dim || out_stride < dim) {
    set_error("%s: rows must be %d-byte aligned with strides that are multiples of 4 "
              "elements and at least dim",
              who, vb);
    return VFL_E_INVALID;
  }
  return VFL_OK;
}

template <bool GATHER>
static int launch_layer_norm(int dtype, const void *x, int64_t xs, const void *r, int64_t rs,
                             const void *w, const void *b, void *out, int64_t os, int64_t rows,
                             int dim, float eps, const RowGather &g, hipStream_t s) {
  if (dtype == VFL_FLOAT32)
    return launch_add_layer_norm<VFL_FLOAT32, GATHER>(x, xs, r, rs, w, b, out, os, rows, dim,
                                                      eps, g, s);
  if (dtype == VFL_BFLOAT16)
    return launch_add_layer_norm<VFL_BFLOAT16, GATHER>(x, xs, r, rs, w, b, out, os, rows, dim,
                                                       eps, g, s);
  return launch_add_layer_norm<VFL_FLOAT16, GATHER>(x, xs, r, rs, w, b, out, os, rows, dim, eps,
                                                    g, s);
}

extern "C" int vfl_add_layer_norm(const void *x, int64_t x_stride, const void *residual,
                                  int64_t residual_stride, const void *weight, const void *bias,
                                  void *out, int64_t out_stride, int64_t rows, int dim, float eps,
                                  int dtype, void *stream) {
  clear_error();
  const int st = check_layer_norm("add_layer_norm", rows, dim, dtype, x, x_stride, residual,
                                  residual_stride, weight, bias, out, out_stride);
  if (st != VFL_OK) return st;
  if (rows == 0) return VFL_OK;
  return launch_layer_norm<false>(dtype, x, x_stride, residual, residual_stride, weight, bias,
                                  out, out_stride, rows, dim, eps, RowGather{},
                                  (hipStream_t)stream);
}

extern "C" int vfl_embed_layer_norm(const int64_t *ids, const int64_t *positions, int64_t rows,
                                    const void *token_table, int64_t token_rows,
                                    int64_t token_stride, float token_scale,
                                    const void *position_table, int64_t position_rows,
                                    int64_t position_stride, int64_t position_offset,
                                    const void *weight, const void *bias, void *out,
                                    int64_t out_stride, int dim, float eps, int dtype,
                                    void *stream) {
  clear_error();
  const int st = check_layer_norm("embed_layer_norm", rows, dim, dtype, position_table,
                                  position_stride, token_table, token_stride, weight, bias, out,
                                  out_stride);
  if (st != VFL_OK) return st;
  if (!ids || !positions || token_rows <= 0 || position_rows <= 0) {
    set_error("embed_layer_norm: null index array or empty table (token rows %lld, position "
              "rows %lld)",
              (long long)token_rows, (long long)position_rows);
    return VFL_E_INVALID;
  }
  if (rows == 0) return VFL_OK;
  // x: the position rows, residual: the (scaled) token rows -- the operand order of
  // add_layer_norm(position embedding, token embedding)
  const RowGather g{positions, ids, position_offset, 0, position_rows, token_rows, token_scale};
  return launch_layer_norm<true>(dtype, position_table, position_stride, token_table,
                                 token_stride, weight, bias, out, out_stride, rows, dim, eps, g,
                                 (hipStream_t)stream);
}

extern "C" int vfl_logprob_topk(const void *logits, int64_t row_stride, int64_t rows, int vocab,
                                int dtype, const int64_t *lengths, const int32_t *rule_tokens,
                                int min_length, int max_length, int begin_index, int n_eos,
                                int n_suppress, int n_begin, int n_bos, int n_forced_eos,
                                int log_softmax, int k, float *scores, int64_t *ids,
                                void *stream) {
  clear_error();
  if (dtype != VFL_FLOAT32 && dtype != VFL_BFLOAT16 && dtype != VFL_FLOAT16) {
    set_error("logprob_topk: unsupported dtype code %d", dtype);
    return VFL_E_INVALID;
  }
  if (rows < 0 || rows > 2147483647LL || vocab <= 0 || row_stride < vocab || k < 1 || k > 16 ||
      k > vocab) {
    set_error("logprob_topk: need 1 <= k <= min(16, vocab) and row_stride >= vocab (k %d, vocab "
              "%d, stride %lld)",
              k, vocab, (long long)row_stride);
    return VFL_E_INVALID;
  }
  const int counts[5] = {n_eos, n_suppress, n_begin, n_bos, n_forced_eos};
  int total = 0;
  for (int c : counts) {
    if (c < 0) {
      set_error("logprob_topk: negative rule-token count");
      return VFL_E_INVALID;
    }
    total += c;
  }
  if (n_eos + n_suppress + n_begin > TK_MAX_RULE_TOKENS || n_bos > TK_MAX_RULE_TOKENS ||
      n_forced_eos > TK_MAX_RULE_TOKENS) {
    set_error("logprob_topk: at most %d banned and %d forced tokens", TK_MAX_RULE_TOKENS,
              TK_MAX_RULE_TOKENS);
    return VFL_E_INVALID;
  }
  if (!logits || !scores || !ids || (total && !rule_tokens)) {
    set_error("logprob_topk: null pointer argument");
    return VFL_E_INVALID;
  }
  if (!lengths && total) {
    set_error("logprob_topk: the rules need per-row lengths");
    return VFL_E_INVALID;
  }
  if (rows == 0) return VFL_OK;
  TopkRules r{min_length, max_length, begin_index, n_eos, n_suppress, n_begin, n_bos,
              n_forced_eos};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == VFL_FLOAT32)
    return launch_topk<VFL_FLOAT32>(logits, row_stride, rows, vocab, lengths, rule_tokens, r,
                                    log_softmax, k, scores, ids, s);
  if (dtype == VFL_BFLOAT16)
    return launch_topk<VFL_BFLOAT16>(logits, row_stride, rows, vocab, lengths, rule_tokens, r,
                                     log_softmax, k, scores, ids, s);
  return launch_topk<VFL_FLOAT16>(logits, row_stride, rows, vocab, lengths, rule_tokens, r,
                                  log_softmax, k, scores, ids, s);
}
