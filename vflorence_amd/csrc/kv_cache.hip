// KV-cache data movement on gfx950: the slot_mapping scatter that writes new K/V
// rows into the paged pools, and the batched copy-on-write block copy.  Both are
// bit-exact byte moves; every lane moves 16-byte chunks so a wave covers 1 KiB per
// instruction.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "common.h"

namespace vfl {

static thread_local char g_error[512];

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int launch_status(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return VFL_E_LAUNCH;
  }
  return VFL_OK;
}

// Whether tokens t .. t+3 (all < T) take slots s .. s+3 in order, s = slots[t] a
// multiple of 4: one whole 4-token group of a block.
__device__ __forceinline__ bool fills_group(const int64_t *slots, int64_t t, int64_t T,
                                            int64_t num_slots) {
  if (t < 0 || t + 3 >= T) return false;
  const int64_t s = slots[t];
  return s >= 0 && s % 4 == 0 && s + 3 < num_slots && slots[t + 1] == s + 1 &&
         slots[t + 2] == s + 2 && slots[t + 3] == s + 3;
}

// ---------------------------------------------------------------------------
// reshape_and_cache: one thread per 16-byte chunk of a (token, head) row.
// ---------------------------------------------------------------------------
// VT: the V pool stores each [block][head] slice with tokens interleaved in groups of
// four (16-bit pools, vtile_index: [token/4][dim][token%4]).  Tokens whose slots fill
// a 4-token group in order (every group of a prompt's encoder tokens but a ragged last
// one) are written by the thread of the group's first token: its 8 dims of the 4 tokens
// are 64 contiguous bytes, so a group's threads write its whole run for the head in
// full 128-byte lines, and the group's other threads skip V.  Any other token
// (scattered slots, a ragged group) writes its own V element by element.
// whole_words: the V pool is 16-byte aligned (the group's stores are then aligned).
template <int DT, bool ALIGNED, bool VT>
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(
    const typename Elem<DT>::T *__restrict__ key, const typename Elem<DT>::T *__restrict__ value,
    int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh, typename Elem<DT>::T *__restrict__ kc,
    typename Elem<DT>::T *__restrict__ vc, const int64_t *__restrict__ slots, int64_t num_tokens,
    int num_heads, int chunks_per_row, int block_size, int64_t num_slots, bool whole_words) {
  using T = typename Elem<DT>::T;
  constexpr int VEC = Elem<DT>::VEC;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = num_tokens * num_heads * chunks_per_row;
  if (idx >= total) return;
  const int c = (int)(idx % chunks_per_row);
  const int64_t row = idx / chunks_per_row;
  const int h = (int)(row % num_heads);
  const int64_t t = row / num_heads;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / block_size;
  const int off = (int)(slot % block_size);
  const int head_dim = chunks_per_row * VEC;
  const int64_t dst = ((blk * num_heads + h) * block_size + off) * head_dim + c * VEC;
  const T *ks = key + t * k_st + h * k_sh + c * VEC;
  const T *vs = value + t * v_st + h * v_sh + c * VEC;
  static_assert(!VT || DT != VFL_FLOAT32, "interleaved V tiles are 16-bit");
  auto load = [](const T *p) {
    if constexpr (ALIGNED) return *reinterpret_cast<const uint4 *>(p);
    else return load16_unaligned<DT>(p);
  };
  const uint4 kv = load(ks);
  if constexpr (ALIGNED) *reinterpret_cast<uint4 *>(kc + dst) = kv;
  else store16_unaligned<DT>(kc + dst, kv);
  if constexpr (!VT) {
    const uint4 vv = load(vs);
    if constexpr (ALIGNED) *reinterpret_cast<uint4 *>(vc + dst) = vv;
    else store16_unaligned<DT>(vc + dst, vv);
  } else {
    T *vt = vc + (blk * num_heads + h) * (int64_t)head_dim * block_size;
    if (whole_words && off % 4 == 0 && fills_group(slots, t, num_tokens, num_slots)) {
      // tokens t .. t+3, dims 8c .. 8c+7: word q of token j holds dims 8c+2q, 8c+2q+1
      uint4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = load(vs + j * v_st);
      uint4 *run = reinterpret_cast<uint4 *>(vt + vtile_index(off, c * VEC, head_dim));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t a = (&v[0].x)[q], b = (&v[1].x)[q], e = (&v[2].x)[q], f = (&v[3].x)[q];
        run[q] = make_uint4((a & 0xffffu) | (b << 16), (e & 0xffffu) | (f << 16),
                            (a >> 16) | (b & 0xffff0000u), (e >> 16) | (f & 0xffff0000u));
      }
      return;
    }
    const int k = off % 4;
    if (whole_words && k != 0 && t >= k && slots[t - k] == slot - k &&
        fills_group(slots, t - k, num_tokens, num_slots))
      return;  // written by the group's first token
    const uint4 vv = load(vs);
    const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      vt[vtile_index(off, c * VEC + e, head_dim)] = (T)(w[e / 2] >> (16 * (e & 1)));
  }
}

template <int DT>
static void launch_reshape(bool aligned, const void *key, const void *value, int64_t k_st,
                           int64_t k_sh, int64_t v_st, int64_t v_sh, void *kc, void *vc,
                           const int64_t *slots, int64_t T, int H, int D, int BS,
                           int64_t num_blocks, hipStream_t stream) {
  using E = typename Elem<DT>::T;
  const int cpr = D / Elem<DT>::VEC;
  const int64_t total = T * H * cpr;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  constexpr bool VT = DT != VFL_FLOAT32;  // v_tile_interleaved(DT)
  const bool whole_words = (uintptr_t)vc % 16 == 0;
  if (aligned)
    reshape_and_cache_kernel<DT, true, VT><<<dim3((unsigned)blocks), dim3(threads), 0, stream>>>(
        (const E *)key, (const E *)value, k_st, k_sh, v_st, v_sh, (E *)kc, (E *)vc, slots, T, H,
        cpr, BS, num_blocks * BS, whole_words);
  else
    reshape_and_cache_kernel<DT, false, VT><<<dim3((unsigned)blocks), dim3(threads), 0, stream>>>(
        (const E *)key, (const E *)value, k_st, k_sh, v_st, v_sh, (E *)kc, (E *)vc, slots, T, H,
        cpr, BS, num_blocks * BS, whole_words);
}

// ---------------------------------------------------------------------------
// copy_blocks: one workgroup per (8 KiB chunk of a block, pair, cache).  Each
// thread moves CPT 16-byte chunks, issuing all loads before the stores.  Measured on
// MI355X over a 4-beam decode's copy pairs (~48 pairs x 24 pools of 32 KiB blocks):
// 8 KiB per workgroup runs 16 us per step, 16 KiB 18 us, 32 KiB 26 us -- more and
// smaller workgroups keep more of the copy in flight.  The source blocks are read
// once, so their loads are non-temporal (they do not displace the step's re-read
// data from the caches); at 115 pairs x 24 pools (181 MB moved) that took a launch
// from 38.8 to 32.4 us (0.58 -> 0.70 of 8 TB/s).  Two, four or eight chunks per thread
// (fewer threads) ran 33.2-33.5 us with non-temporal loads and 44.9-67.5 us without;
// non-temporal stores as well ran 35.4 us.
// mode 0: src -> dst; mode 1: src -> staging; mode 2: staging -> dst.
// ---------------------------------------------------------------------------
constexpr int COPY_THREADS = 512;
constexpr int COPY_CPT = 1;
constexpr int64_t COPY_BYTES_PER_WG = (int64_t)COPY_THREADS * COPY_CPT * 16;

typedef uint32_t copy_u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 copy_load_stream(const uint4 *p) {
  const copy_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const copy_u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__global__ __launch_bounds__(COPY_THREADS) void copy_blocks_kernel(
    void *const *__restrict__ caches, const int64_t *__restrict__ src,
    const int64_t *__restrict__ dst, int64_t num_pairs, int64_t block_bytes, int64_t num_blocks,
    int mode, uint8_t *__restrict__ staging) {
  const int64_t p = blockIdx.y;
  const int c = blockIdx.z;
  const int64_t s = src[p], d = dst[p];
  if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) return;
  uint8_t *base = (uint8_t *)caches[c];
  const uint8_t *from;
  uint8_t *to;
  if (mode == 0) {
    from = base + s * block_bytes;
    to = base + d * block_bytes;
  } else if (mode == 1) {
    from = base + s * block_bytes;
    to = staging + ((int64_t)c * num_pairs + p) * block_bytes;
  } else {
    from = staging + ((int64_t)c * num_pairs + p) * block_bytes;
    to = base + d * block_bytes;
  }
  const int64_t chunk0 = (int64_t)blockIdx.x * COPY_BYTES_PER_WG / 16 + threadIdx.x;
  const int64_t nchunks = block_bytes / 16;
  uint4 v[COPY_CPT];
#pragma unroll
  for (int i = 0; i < COPY_CPT; ++i) {
    const int64_t ch = chunk0 + (int64_t)i * COPY_THREADS;
    if (ch < nchunks) v[i] = copy_load_stream(reinterpret_cast<const uint4 *>(from) + ch);
  }
#pragma unroll
  for (int i = 0; i < COPY_CPT; ++i) {
    const int64_t ch = chunk0 + (int64_t)i * COPY_THREADS;
    if (ch < nchunks) reinterpret_cast<uint4 *>(to)[ch] = v[i];
  }
}

// ---------------------------------------------------------------------------
// Library-held staging for vfl_copy_blocks_noalloc: one array per GPU, in the code
// object's device memory, so the entry point never allocates.  Host code must not pass
// the array's name to a kernel (it is a host-side stand-in there); the device address
// of each GPU's copy is looked up once per device with hipGetSymbolAddress.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[VFL_NOALLOC_STAGING_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mutex;
static void *g_scratch_ptr[MAX_DEVICES];

// Device address of the current device's scratch array (looked up on the first call on
// that device); nullptr with the error set on failure.
static void *device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    set_error("copy_blocks_noalloc: no current HIP device (device %d)", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      set_error("copy_blocks_noalloc: hipGetSymbolAddress on device %d failed: %s", dev,
                hipGetErrorString(err));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace vfl

using namespace vfl;

extern "C" const char *vfl_last_error(void) { return g_error; }

extern "C" int vfl_version(void) { return 100; }

static bool supported_dtype(int dtype) {
  return dtype == VFL_FLOAT32 || dtype == VFL_BFLOAT16 || dtype == VFL_FLOAT16;
}

extern "C" int vfl_reshape_and_cache(const void *key, const void *value,
                                     int64_t key_stride_token, int64_t key_stride_head,
                                     int64_t value_stride_token, int64_t value_stride_head,
                                     void *k_cache, void *v_cache, const int64_t *slot_mapping,
                                     int64_t num_tokens, int num_heads, int head_dim,
                                     int block_size, int64_t num_blocks, int dtype,
                                     void *stream) {
  clear_error();
  if (!supported_dtype(dtype)) {
    set_error("reshape_and_cache: unsupported dtype code %d", dtype);
    return VFL_E_INVALID;
  }
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0) {
    set_error("reshape_and_cache: bad sizes (tokens %lld heads %d head_dim %d block_size %d "
              "blocks %lld)",
              (long long)num_tokens, num_heads, head_dim, block_size, (long long)num_blocks);
    return VFL_E_INVALID;
  }
  const int vec = 16 / elem_bytes(dtype);
  if (head_dim % vec != 0) {
    set_error("reshape_and_cache: head_dim %d must be a multiple of %d", head_dim, vec);
    return VFL_E_UNSUPPORTED;
  }
  // Only pools that an attention kernel reads are written (16- and 32-token blocks): the
  // 16-bit V layout interleaves tokens by four inside a block, so a block size that is
  // not a multiple of 4 would place V outside its block-head slice.
  if (block_shift(block_size) < 0) {
    set_error("reshape_and_cache: block_size %d has no attention kernel (supported: 16, 32)",
              block_size);
    return VFL_E_UNSUPPORTED;
  }
  if (num_tokens == 0) return VFL_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) {
    set_error("reshape_and_cache: null pointer argument");
    return VFL_E_INVALID;
  }
  // 16-byte vector path when every source and destination chunk is 16-byte aligned.
  const uintptr_t align_bits = (uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache |
                               (uintptr_t)v_cache;
  const bool aligned = (align_bits % 16 == 0) && (key_stride_token % vec == 0) &&
                       (key_stride_head % vec == 0) && (value_stride_token % vec == 0) &&
                       (value_stride_head % vec == 0);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case VFL_FLOAT32:
      launch_reshape<VFL_FLOAT32>(aligned, key, value, key_stride_token, key_stride_head,
                                  value_stride_token, value_stride_head, k_cache, v_cache,
                                  slot_mapping, num_tokens, num_heads, head_dim, block_size,
                                  num_blocks, s);
      break;
    case VFL_BFLOAT16:
      launch_reshape<VFL_BFLOAT16>(aligned, key, value, key_stride_token, key_stride_head,
                                   value_stride_token, value_stride_head, k_cache, v_cache,
                                   slot_mapping, num_tokens, num_heads, head_dim, block_size,
                                   num_blocks, s);
      break;
    default:
      launch_reshape<VFL_FLOAT16>(aligned, key, value, key_stride_token, key_stride_head,
                                  value_stride_token, value_stride_head, k_cache, v_cache,
                                  slot_mapping, num_tokens, num_heads, head_dim, block_size,
                                  num_blocks, s);
      break;
  }
  return launch_status("reshape_and_cache");
}

// Host checks shared by both copy entry points; VFL_OK when there is work to launch, 1
// when there is nothing to do.
static int check_copy_args(const char *who, void *const *caches, int num_caches,
                           const int64_t *src, const int64_t *dst, int64_t num_pairs,
                           int64_t block_bytes) {
  if (num_caches < 0 || num_pairs < 0 || block_bytes <= 0 || block_bytes % 16 != 0) {
    set_error("%s: bad sizes (caches %d pairs %lld block_bytes %lld)", who, num_caches,
              (long long)num_pairs, (long long)block_bytes);
    return VFL_E_INVALID;
  }
  if (num_caches == 0 || num_pairs == 0) return 1;
  if (!caches || !src || !dst) {
    set_error("%s: null pointer argument", who);
    return VFL_E_INVALID;
  }
  if (num_pairs > 65535 || num_caches > 65535) {
    set_error("%s: at most 65535 pairs and 65535 caches per call (got %lld, %d)", who,
              (long long)num_pairs, num_caches);
    return VFL_E_INVALID;
  }
  return VFL_OK;
}

// The copy itself: one direct pass, or gather into `staging` then scatter from it.
static int launch_copy(void *const *caches, int num_caches, const int64_t *src,
                       const int64_t *dst, int64_t num_pairs, int64_t block_bytes,
                       int64_t num_blocks, uint8_t *staging, hipStream_t s, const char *who) {
  const unsigned gx = (unsigned)((block_bytes + COPY_BYTES_PER_WG - 1) / COPY_BYTES_PER_WG);
  const dim3 grid(gx, (unsigned)num_pairs, (unsigned)num_caches);
  if (!staging) {
    copy_blocks_kernel<<<grid, COPY_THREADS, 0, s>>>(caches, src, dst, num_pairs, block_bytes,
                                                     num_blocks, 0, nullptr);
  } else {
    copy_blocks_kernel<<<grid, COPY_THREADS, 0, s>>>(caches, src, dst, num_pairs, block_bytes,
                                                     num_blocks, 1, staging);
    int st = launch_status(who);
    if (st != VFL_OK) return st;
    copy_blocks_kernel<<<grid, COPY_THREADS, 0, s>>>(caches, src, dst, num_pairs, block_bytes,
                                                     num_blocks, 2, staging);
  }
  return launch_status(who);
}

extern "C" int vfl_copy_blocks_noalloc(void *const *caches, int num_caches, const int64_t *src,
                                       const int64_t *dst, int64_t num_pairs,
                                       int64_t block_bytes, int64_t num_blocks, int staged,
                                       void *stream) {
  clear_error();
  int st = check_copy_args("copy_blocks_noalloc", caches, num_caches, src, dst, num_pairs,
                           block_bytes);
  if (st != VFL_OK) return st == 1 ? VFL_OK : st;
  uint8_t *staging = nullptr;
  if (staged) {
    const int64_t need = (int64_t)num_caches * num_pairs * block_bytes;
    if (need > (int64_t)VFL_NOALLOC_STAGING_BYTES) {
      set_error("copy_blocks_noalloc: staging %lld bytes (%d caches x %lld pairs x %lld) "
                "exceeds the library's %lld-byte buffer",
                (long long)need, num_caches, (long long)num_pairs, (long long)block_bytes,
                (long long)VFL_NOALLOC_STAGING_BYTES);
      return VFL_E_INVALID;
    }
    staging = (uint8_t *)device_scratch();
    if (!staging) return VFL_E_LAUNCH;
  }
  return launch_copy(caches, num_caches, src, dst, num_pairs, block_bytes, num_blocks, staging,
                     (hipStream_t)stream, "copy_blocks_noalloc");
}

extern "C" int vfl_copy_blocks(void *const *caches, int num_caches, const int64_t *src,
                               const int64_t *dst, int64_t num_pairs, int64_t block_bytes,
                               int64_t num_blocks, void *staging, void *stream) {
  clear_error();
  int st = check_copy_args("copy_blocks", caches, num_caches, src, dst, num_pairs, block_bytes);
  if (st != VFL_OK) return st == 1 ? VFL_OK : st;
  if (staging && ((uintptr_t)staging % 16) != 0) {
    set_error("copy_blocks: staging buffer must be 16-byte aligned");
    return VFL_E_INVALID;
  }
  return launch_copy(caches, num_caches, src, dst, num_pairs, block_bytes, num_blocks,
                     (uint8_t *)staging, (hipStream_t)stream, "copy_blocks");
}

